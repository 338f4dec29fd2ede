"""bench.py's counter-measured figures (roofline.traffic and roofline.valu) are constants taken from the rocprofv3
summaries under profiles/; this checks them against those summaries' own tables, so that a re-measured profile and
the bench line cannot drift apart.  CPU only."""
import os
import re
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def counter_rows(path):
    """kernel -> list of (read GB, write GB, SQ_INSTS_VALU M) from a profile's per-dispatch counter table"""
    rows = {}
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 6 and cells[0].startswith("k_") and re.fullmatch(r"[0-9.]+", cells[3] or "x"):
            rows.setdefault(cells[0], []).append((float(cells[3]), float(cells[4]), float(cells[5])))
    return rows


def test_hmult_constants_match_the_profile():
    sys.path.insert(0, REPO)
    import bench
    path = os.path.join(REPO, "profiles", "hmult_config2_kernels.md")
    rows = counter_rows(path)
    # the dominant launch: T's forward NTT, pass A over 2,944 limbs plus the pass B that ends in the combine
    a = [r for r in rows["k_ntt_fwd_a"] if abs(r[0] - 1.545) < 0.05]
    b = rows["k_ntt_fwd_b_mdr<3, true>"][0]
    assert len(a) == 1
    traffic = (a[0][0] + a[0][1] + b[0] + b[1]) * 1e9
    valu = (a[0][2] + b[2]) * 1e6
    meas = bench.MEASURED[("hmult", "ntt_fwd_mdr")]
    assert abs(meas["traffic"] - traffic) / traffic < 0.01
    assert abs(meas["valu_insts"] - valu) / valu < 0.01
    # the ModUp NTT: both passes over the 4,608 extension limbs
    fa = [r for r in rows["k_ntt_fwd_a"] if abs(r[0] - 2.418) < 0.05][0]
    fb = rows["k_ntt_fwd_b"][0]
    meas = bench.MEASURED[("hmult", "ntt_fwd_2pass")]
    assert abs(meas["traffic"] - (fa[0] + fa[1] + fb[0] + fb[1]) * 1e9) / meas["traffic"] < 0.01
    assert abs(meas["valu_insts"] - (fa[2] + fb[2]) * 1e6) / meas["valu_insts"] < 0.01
    # and the summary row the profile quotes for it
    text = open(path).read()
    m = re.search(r"\| T NTT \+ combine \(A \+ B_mdr\) \| [0-9.]+ \| [0-9.]+ \| \*\*([0-9.]+)\*\* \| [0-9.]+ \| "
                  r"\*\*([0-9.]+)\*\* \|", text)
    assert m and abs(float(m.group(1)) * 1e9 - traffic) / traffic < 0.002
    assert abs(float(m.group(2)) * 1e6 - valu) / valu < 0.002


def test_ntt_constants_match_the_profile():
    sys.path.insert(0, REPO)
    import bench
    rows = counter_rows(os.path.join(REPO, "profiles", "ntt_config1_kernel_trace.md"))
    for name, (p1, p2) in {"ntt_fwd_2pass": ("k_ntt_fwd_a", "k_ntt_fwd_b"),
                           "ntt_inv_2pass": ("k_ntt_inv_b", "k_ntt_inv_a")}.items():
        r1, r2 = rows[p1][0], rows[p2][0]
        meas = bench.MEASURED[("ntt", name)]
        traffic = (r1[0] + r1[1] + r2[0] + r2[1]) * 1e9
        assert abs(meas["traffic"] - traffic) / traffic < 0.01, name
        valu = (r1[2] + r2[2]) * 1e6
        assert abs(meas["valu_insts"] - valu) / valu < 0.01, name
