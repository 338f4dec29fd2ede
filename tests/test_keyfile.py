"""Seeded key part files (the reference's evalrot.partNNN.seeded.bin, hpc_gpu_port/seeded_keys.hpp:44-51) through
the C ABI.  CPU: the header reader against files written from the specification (tests/keypart_util.py), and its
refusals.  GPU: a key loaded from such a file is b from the file and a = the ChaCha20 expansion of its seed (the
oracle's sampler, pinned by RFC 8439 vectors in test_oracle); the engine's writer produces the specification's bytes
for a generated key, and reading them back gives the key word for word.

Ciphertext files (the serve protocol's req.N.t / resp.N.t; the engine's own flat layout, declared in
include/ckks_engine.h): the header reader against files written from that layout, its refusals, and on the GPU
save == the layout's bytes, load == the saved words, refusals of another chain and of words >= q."""
import struct

import numpy as np
import pytest

from engine_loader import load_ckks
from keypart_util import TAG_SKEY, part_bytes

N16 = 16
MOD16 = [97, 193, 257, 353, 449]  # any values: the header reader does not check the chain


def _write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def _small_records(n_keys, num_part_q=2, T=5, seed=1):
    rng = np.random.default_rng(seed)
    return [(int(2 * rng.integers(1, 1000) + 1), bytes(rng.integers(0, 256, 32, dtype=np.uint8)),
             rng.integers(0, 97, (num_part_q, T, N16), dtype=np.uint64)) for _ in range(n_keys)]


def test_header_and_indices_round_trip(tmp_path):
    ckks = load_ckks()
    recs = _small_records(3)
    path = _write(tmp_path, "p.bin", part_bytes(N16, MOD16, 3, 2, 2, 2, "rot-tag", recs))
    h = ckks.seeded_part_header(path)
    assert (h["version"], h["expander"], h["N"], h["size_q"], h["size_p"]) == (1, 1, N16, 3, 2)
    assert (h["num_part_q"], h["num_per_part_q"], h["count"], h["key_tag"]) == (2, 2, 3, "rot-tag")
    assert h["moduli"] == MOD16
    assert ckks.seeded_part_indices(path) == [r[0] for r in recs]


def test_empty_part(tmp_path):
    ckks = load_ckks()
    path = _write(tmp_path, "e.bin", part_bytes(N16, MOD16, 3, 2, 2, 2, "t", []))
    assert ckks.seeded_part_header(path)["count"] == 0
    assert ckks.seeded_part_indices(path) == []


@pytest.mark.parametrize("kind", ["magic", "version", "expander", "truncated", "count", "tag", "count_overflow",
                                  "digits"])
def test_header_refusals(tmp_path, kind):
    ckks = load_ckks()
    recs = _small_records(2)
    kw = {}
    if kind == "magic":
        kw["magic"] = b"FSSMSKY2"
    if kind == "version":
        kw["version"] = 2
    if kind == "expander":
        kw["expander"] = 7
    if kind == "count":
        kw["count"] = 3  # one record more than the file holds
    if kind == "count_overflow":
        # the largest count: the size check divides instead of multiplying, so no count can wrap the product
        kw["count"] = 0xFFFFFFFF
    num_part_q = 2
    if kind == "digits":
        num_part_q = 1 << 20  # more digits than limbs
    data = part_bytes(N16, MOD16, 3, 2, num_part_q, 2, "x" * 5000 if kind == "tag" else "t", recs, **kw)
    if kind == "truncated":
        data = data[:-8]
    path = _write(tmp_path, "bad.bin", data)
    with pytest.raises(ckks.CkksError):
        ckks.seeded_part_header(path)


def test_missing_file(tmp_path):
    ckks = load_ckks()
    with pytest.raises(ckks.CkksError):
        ckks.seeded_part_header(str(tmp_path / "nope.bin"))


def ct_bytes(n, level, scale, moduli, words, magic=b"FSSMCTX1", version=1, n_polys=2):
    """a ciphertext file from the layout: magic, u32 version, N, level, n_polys, f64 scale, u64 moduli[level],
    u64 words[2][level][N], little-endian"""
    head = magic + struct.pack("<4Id", version, n, level, n_polys, scale)
    return head + struct.pack(f"<{level}Q", *moduli[:level]) + np.asarray(words, dtype="<u8").tobytes()


def test_ct_file_info(tmp_path):
    ckks = load_ckks()
    w = np.arange(2 * 3 * N16, dtype=np.uint64).reshape(2, 3, N16) % 97
    path = _write(tmp_path, "c.bin", ct_bytes(N16, 3, 2.0 ** 40, MOD16, w))
    assert ckks.ct_file_info(path) == {"N": N16, "level": 3, "scale": 2.0 ** 40}


@pytest.mark.parametrize("kind", ["magic", "version", "polys", "scale", "truncated", "longer", "ring"])
def test_ct_file_refusals(tmp_path, kind):
    ckks = load_ckks()
    w = np.zeros((2, 3, N16), dtype=np.uint64)
    args = dict(n=N16, level=3, scale=2.0 ** 40, moduli=MOD16, words=w)
    if kind == "magic":
        args["magic"] = b"FSSMCTX2"
    elif kind == "version":
        args["version"] = 2
    elif kind == "polys":
        args["n_polys"] = 3
    elif kind == "scale":
        args["scale"] = 0.0
    elif kind == "ring":
        args["n"] = 24
    data = ct_bytes(**args)
    if kind == "truncated":
        data = data[:-8]
    elif kind == "longer":
        data = data + b"\0" * 8
    path = _write(tmp_path, "bad.bin", data)
    with pytest.raises(ckks.CkksError):
        ckks.ct_file_info(path)


# ---------------------------------------------------------------- GPU
N = 1 << 16


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


@pytest.fixture(scope="module")
def ctx(ckks):
    return ckks.Context(num_q=4, num_p=2, dnum=2, q_bits=54, p_bits=60)


@pytest.mark.gpu
def test_load_from_specification_file(tmp_path, ckks, ctx, oracle):
    """b from the file, a expanded from the seed (nonce {digit, limb, "SKEY"}) -- against the oracle's sampler"""
    T, D = ctx.L + ctx.K, ctx.dnum
    q = np.array(ctx.moduli[:T], dtype=np.uint64)
    rng = np.random.default_rng(7)
    recs = []
    for r in range(2):
        b = rng.integers(0, 2**63, (D, T, N), dtype=np.uint64) % q[None, :, None]
        recs.append((ckks.rotation_index(r + 1), bytes(rng.integers(0, 256, 32, dtype=np.uint8)), b))
    path = _write(tmp_path, "k.bin", part_bytes(N, ctx.moduli[:T], ctx.L, ctx.K, D, (ctx.L + D - 1) // D, "auto",
                                                 recs))
    buf = ckks.DeviceBuffer(D * 2 * T * N * 8)
    for r, (g, seed, b) in enumerate(recs):
        assert ctx.seeded_part_load_key(path, r, buf.ptr) == g
        got = buf.download((D, 2, T, N))
        assert np.array_equal(got[:, 0], b)
        for d in range(D):
            for i in range(T):
                assert np.array_equal(got[d, 1, i], oracle.fill_uniform(seed, d, i, TAG_SKEY, ctx.moduli[i], N)), (d, i)


@pytest.mark.gpu
def test_write_matches_specification_and_reloads(tmp_path, ckks, ctx):
    T, D = ctx.L + ctx.K, ctx.dnum
    sk = ctx.secret(b"K" * 32, 64)
    seeds = [bytes([11 + i]) * 32 for i in range(2)]
    gs = [ckks.rotation_index(1), ckks.rotation_index(-5)]
    keys = []
    for i, g in enumerate(gs):
        k = ckks.DeviceBuffer(D * 2 * T * N * 8)
        ctx.keygen_automorphism(sk, g, seeds[i], bytes([40 + i]) * 32, k.ptr)
        keys.append(k)
    path = str(tmp_path / "w.bin")
    ctx.seeded_part_write(path, "mytag", gs, seeds, [k.ptr for k in keys])
    words = [k.download((D, 2, T, N)) for k in keys]
    want = part_bytes(N, ctx.moduli[:T], ctx.L, ctx.K, D, (ctx.L + D - 1) // D, "mytag",
                      [(g, s, w[:, 0]) for g, s, w in zip(gs, seeds, words)])
    assert open(path, "rb").read() == want
    back = ckks.DeviceBuffer(D * 2 * T * N * 8)
    for r in range(2):
        assert ctx.seeded_part_load_key(path, r, back.ptr) == gs[r]
        assert np.array_equal(back.download((D, 2, T, N)), words[r]), r


@pytest.mark.gpu
def test_load_refuses_another_context(tmp_path, ckks, ctx):
    T, D = ctx.L + ctx.K, ctx.dnum
    other = list(ctx.moduli[:T])
    other[1] = other[2]
    b = np.zeros((D, T, N), dtype=np.uint64)
    path = _write(tmp_path, "o.bin", part_bytes(N, other, ctx.L, ctx.K, D, (ctx.L + D - 1) // D, "t",
                                                 [(5, b"\0" * 32, b)]))
    buf = ckks.DeviceBuffer(D * 2 * T * N * 8)
    with pytest.raises(ckks.CkksError):
        ctx.seeded_part_load_key(path, 0, buf.ptr)
    path2 = _write(tmp_path, "o2.bin", part_bytes(N, ctx.moduli[:T], ctx.L, ctx.K, D + 1, 1, "t",
                                                  [(5, b"\0" * 32, np.zeros((D + 1, T, N), np.uint64))]))
    with pytest.raises(ckks.CkksError):
        ctx.seeded_part_load_key(path2, 0, buf.ptr)


@pytest.mark.gpu
def test_ct_save_matches_layout_and_reloads(tmp_path, ckks, ctx):
    lv = 3
    q = np.array(ctx.moduli[:lv], dtype=np.uint64)
    rng = np.random.default_rng(21)
    w = rng.integers(0, 2**63, (2, lv, N), dtype=np.uint64) % q[None, :, None]
    buf = ckks.DeviceBuffer(2 * ctx.L * N * 8)
    buf.upload(w)
    path = str(tmp_path / "ct.bin")
    ctx.ct_save(path, buf.ptr, lv, 2.0 ** 45)
    assert open(path, "rb").read() == ct_bytes(N, lv, 2.0 ** 45, ctx.moduli, w)
    back = ckks.DeviceBuffer(2 * ctx.L * N * 8)
    assert ctx.ct_load(path, back.ptr, ctx.L) == (lv, 2.0 ** 45)
    assert np.array_equal(back.download((2, lv, N)), w)
    with pytest.raises(ckks.CkksError):          # more limbs than the destination holds
        ctx.ct_load(path, back.ptr, lv - 1)
    bad = w.copy()
    bad[1, 2, 77] = q[2]                          # a word >= its prime
    p2 = _write(tmp_path, "ge.bin", ct_bytes(N, lv, 2.0 ** 45, ctx.moduli, bad))
    with pytest.raises(ckks.CkksError):
        ctx.ct_load(p2, back.ptr, ctx.L)
    other = list(ctx.moduli)
    other[0] = other[1]
    p3 = _write(tmp_path, "oc.bin", ct_bytes(N, lv, 2.0 ** 45, other, w))
    with pytest.raises(ckks.CkksError):
        ctx.ct_load(p3, back.ptr, ctx.L)


@pytest.mark.gpu
def test_rotation_keys_load_follows_the_dev_sidecar(tmp_path, ckks, ctx):
    """LoadContext's rotation keys (gpu_real_model.cu:1436-1529, FIDESlib's upload of the key of each rotation the
    .dev sidecar lists): keys generated on the device and written into two seeded parts; the sidecar lists a subset
    of their rotations, out of order, one of them as the other sign of a half-slot rotation; each loaded buffer holds
    its rotation's key word for word; a rotation with no key in the parts is refused"""
    T, D = ctx.L + ctx.K, ctx.dnum
    sk = ctx.secret(b"R" * 32, 64)
    steps = [1, 2, -3, 7, N // 4]
    words = {}
    parts = []
    for p, chunk in enumerate((steps[:3], steps[3:])):
        gs, seeds, bufs = [], [], []
        for i, s in enumerate(chunk):
            g = ckks.rotation_index(s)
            seed = bytes([60 + 10 * p + i]) * 32
            k = ckks.DeviceBuffer(D * 2 * T * N * 8)
            ctx.keygen_automorphism(sk, g, seed, bytes([90 + 10 * p + i]) * 32, k.ptr)
            gs.append(g)
            seeds.append(seed)
            bufs.append(k)
            words[s] = k.download((D, 2, T, N))
        path = str(tmp_path / f"evalrot.part{p:03d}.seeded.bin")
        ctx.seeded_part_write(path, "rot", gs, seeds, [b.ptr for b in bufs])
        parts.append(path)
    listed = [7, -3, -(N // 4), 1]
    dev = str(tmp_path / "cryptocontext.bin.dev")
    ckks.dev_sidecar_write(dev, listed, [N // 2])
    out = [ckks.DeviceBuffer(D * 2 * T * N * 8) for _ in listed]
    ctx.rotation_keys_load(dev, parts, [b.ptr for b in out])
    for s, b in zip(listed, out):
        want = words[s if s in words else -s]
        assert np.array_equal(b.download((D, 2, T, N)), want), s
    with pytest.raises(ckks.CkksError, match="buffers"):
        ctx.rotation_keys_load(dev, parts, [b.ptr for b in out[:2]])
    ckks.dev_sidecar_write(dev, [1, 5], [])
    with pytest.raises(ckks.CkksError, match="no key for rotation 5"):
        ctx.rotation_keys_load(dev, parts, [b.ptr for b in out[:2]])
