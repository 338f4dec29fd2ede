"""bench.py's counter-measured figures (roofline.traffic, kernel_io.traffic and kernel_io.valu) and its stream rates are
constants taken from the rocprofv3 and stream summaries under profiles/; this checks them against those summaries' own
tables, so that a re-measured profile and the bench line cannot drift apart.  CPU only."""
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
    b = rows["k_ntt_fwd_b_mdr<3, true, false>"][0]
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


def counter_rows_with_dispatches(path):
    """(kernel, dispatches, read GB, write GB) for every row of a profile's per-dispatch counter table"""
    out = []
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 6 and cells[0].startswith("k_") and re.fullmatch(r"[0-9.]+", cells[3] or "x"):
            out.append((cells[0], int(cells[2]), float(cells[3]), float(cells[4])))
    return out


def test_hmult_step_traffic_is_the_sum_over_every_dispatch():
    """roofline.traffic of config 2 = the counter-measured bytes of one HMult step summed over all its dispatches (the
    profiled run holds 5 steps: 1 warmup, 3 timed, 1 profiled)"""
    sys.path.insert(0, REPO)
    import bench
    rows = counter_rows_with_dispatches(os.path.join(REPO, "profiles", "hmult_config2_kernels.md"))
    per_step = sum((r + w) * n for (_, n, r, w) in rows) / 5 * 1e9
    meas = bench.MEASURED[("hmult", "step")]["traffic"]
    assert abs(meas - per_step) / per_step < 0.01
    # against the SURVEY 8(d) unit: the step moves about 3x the algorithmic bytes
    ratio = meas / (bench.N_PAIRS * bench.HMULT_UNIT_BYTES)
    assert 2.0 < ratio < 4.0


def test_ntt_step_traffic_is_forward_plus_inverse():
    sys.path.insert(0, REPO)
    import bench
    step = bench.MEASURED[("ntt", "step")]["traffic"]
    assert abs(step - bench.MEASURED[("ntt", "ntt_fwd_2pass")]["traffic"] -
               bench.MEASURED[("ntt", "ntt_inv_2pass")]["traffic"]) < 1e6


def test_stream_constants_are_the_profile_maxima():
    """the "achievable" denominators are the best read-only and nontemporal-copy rates of the committed stream table"""
    sys.path.insert(0, REPO)
    import bench
    reads, copies = [], []
    for line in open(os.path.join(REPO, "profiles", "hbm_stream.md")):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and all(re.fullmatch(r"[0-9.]+", c) for c in cells):
            reads.append(float(cells[3]))
            copies.append(float(cells[4]))
    assert len(reads) >= 20
    assert bench.STREAM_READ_GBS == max(reads)
    assert bench.STREAM_COPY_GBS == max(copies)
    assert bench.achievable(0.0) == bench.STREAM_READ_GBS and bench.achievable(0.5) == bench.STREAM_COPY_GBS


def test_unit_constants_follow_the_limb_counts():
    """SURVEY 8(d)'s per-op units as limb counts (one limb = 2^16 x 8 B)"""
    sys.path.insert(0, REPO)
    import bench
    assert bench.HMULT_UNIT_BYTES == (96 + 192 + 46) * bench.LIMB_BYTES
    assert bench.HMULT_EVK_AMORTISED_BYTES == (96 + 3 + 46) * bench.LIMB_BYTES
    assert bench.KS_UNIT_BYTES == (24 + 192 + 48) * bench.LIMB_BYTES
    limbs, per_dir = bench.ntt_bytes()
    assert limbs == 3072 and per_dir == 3_246_391_296


def test_step_roofline_fields():
    sys.path.insert(0, REPO)
    import bench
    r = bench.step_roofline("hmult", 64 * bench.HMULT_UNIT_BYTES, 7.6452, 46 / 334, "x")
    assert abs(r["achieved"] - 64 * bench.HMULT_UNIT_BYTES / 7.6452e-3 / 1e9) < 0.1
    assert r["frac"] == round(r["achieved"] / 8000.0, 4)
    assert r["achievable"] == bench.STREAM_COPY_GBS
    assert r["traffic"] == bench.MEASURED[("hmult", "step")]["traffic"]
    assert 2.0 < r["traffic_over_algorithmic"] < 4.0


def step_total(path):
    """(read GB, write GB) of the '**step total**' row of a profile's counter table"""
    for line in open(path):
        cells = [c.strip().strip("*") for c in line.strip().strip("|").split("|")]
        if cells and cells[0] == "step total":
            return float(cells[3]), float(cells[4])
    raise AssertionError(f"no step total row in {path}")


def test_pcmm_and_bootstrap_step_traffic_match_their_profiles():
    sys.path.insert(0, REPO)
    import bench
    for workload, name in (("pcmm", "pcmm_config3_kernel_trace.md"), ("bootstrap", "bootstrap_config4_kernel_trace.md")):
        path = os.path.join(REPO, "profiles", name)
        r, w = step_total(path)
        meas = bench.MEASURED[(workload, "step")]
        assert meas["source"] == "profiles/" + name
        assert abs(meas["traffic"] - (r + w) * 1e9) / meas["traffic"] < 0.002, workload
    # the PCMM MAC row: read + write of its one dispatch
    rows = {}
    for line in open(os.path.join(REPO, "profiles", "pcmm_config3_kernel_trace.md")):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == "k_bsgs_mac" and re.fullmatch(r"[0-9.]+", cells[3]):
            rows["mac"] = float(cells[3]) + float(cells[4])
    assert abs(bench.MEASURED[("pcmm", "bsgs_mac")]["traffic"] - rows["mac"] * 1e9) < 2e6


def test_decode_step_traffic_matches_the_phase_table():
    """config 5's roofline.traffic: the '**step**' row of the phase table (read GB + write GB)"""
    sys.path.insert(0, REPO)
    import bench
    path = os.path.join(REPO, "profiles", "decode_config5_kernel_trace.md")
    for line in open(path):
        cells = [c.strip().strip("*") for c in line.strip().strip("|").split("|")]
        if cells and cells[0] == "step" and len(cells) >= 6:
            r, w = float(cells[4]), float(cells[5])
            break
    else:
        raise AssertionError("no step row")
    meas = bench.MEASURED[("decode", "step")]
    assert meas["source"] == "profiles/decode_config5_kernel_trace.md"
    assert abs(meas["traffic"] - (r + w) * 1e9) / meas["traffic"] < 0.001
