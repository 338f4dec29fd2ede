"""Hoisted rotations, plaintext operators and the BSGS diagonal matvec on the GPU.

- bit-exact: hoisted rotations == individual rotations == oracle rotations; the BSGS composition against
  the oracle composition of the same stages (hoisted baby rotations, ct x pt MAC, giant rotations summed in Q_l P,
  one ModDown, rescale) at small shapes;
- decrypted: the full config-3 product (768 x 768 weights N(0, 1/768), u uniform in [-1, 1], 28 baby and
  28 giant steps, L = 16) against the float64 matvec, relErrRms <= 1e-6.
"""
import numpy as np
import pytest

from engine_loader import load_ckks
from pcmm_util import bsgs_diagonals, replicate, steps

pytestmark = pytest.mark.gpu

L, K, DNUM = 24, 8, 3
N = 1 << 16
SCALE = 2.0**50


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


@pytest.fixture(scope="module")
def ctx(ckks):
    return ckks.Context(num_q=L, num_p=K, dnum=DNUM, q_bits=54, p_bits=60, scale=SCALE)


@pytest.fixture(scope="module")
def octx(oracle, ctx):
    return oracle.Ctx(16, ctx.moduli, L, K, DNUM)


def residues(moduli, shape_prefix, prime_idx, seed):
    rng = np.random.default_rng(seed)
    q = np.array([moduli[i] for i in prime_idx], dtype=np.uint64)
    x = rng.integers(0, 2**63, tuple(shape_prefix) + (len(prime_idx), N), dtype=np.uint64)
    return x % q.reshape((1,) * len(shape_prefix) + (-1, 1))


def modq(x, moduli, l):
    q = np.array(moduli[:l], dtype=object).reshape(-1, 1)
    return (x % q).astype(np.uint64)


def test_mul_add_plain(ckks, ctx):
    l, B = 3, 2
    ct = residues(ctx.moduli, (B, 2), list(range(l)), 1)
    pt = residues(ctx.moduli, (), list(range(l)), 2)
    dct, dpt = ckks.DeviceBuffer.from_array(ct), ckks.DeviceBuffer.from_array(pt)
    out = ckks.DeviceBuffer(ct.nbytes)
    ctx.eval_mult_plain(dct.ptr, B, l, dpt.ptr, out.ptr)
    got = out.download(ct.shape)
    for b in range(B):
        for p in range(2):
            assert np.array_equal(got[b, p], modq(ct[b, p].astype(object) * pt.astype(object), ctx.moduli, l))
    ctx.eval_add_plain(dct.ptr, B, l, dpt.ptr, out.ptr)
    got = out.download(ct.shape)
    for b in range(B):
        assert np.array_equal(got[b, 0], modq(ct[b, 0].astype(object) + pt.astype(object), ctx.moduli, l))
        assert np.array_equal(got[b, 1], ct[b, 1])


def test_hoisted_and_batched_rotations_bit_exact(ckks, ctx, octx):
    l = 7
    st = [1, 2, 5, -3]
    evks = [residues(ctx.moduli, (DNUM, 2), list(range(L + K)), 100 + i) for i in range(len(st))]
    devks = [ckks.DeviceBuffer.from_array(e) for e in evks]
    ct = residues(ctx.moduli, (2,), list(range(l)), 3)
    dct = ckks.DeviceBuffer.from_array(ct)
    out = ckks.DeviceBuffer(len(st) * ct.nbytes)
    ctx.eval_rotate_hoisted(dct.ptr, l, st, [d.ptr for d in devks], out.ptr)
    hoisted = out.download((len(st), 2, l, N))
    for i, s in enumerate(st):
        assert np.array_equal(hoisted[i], octx.rotate(ct, l, octx.rot_index(s), evks[i])), s
    # many ciphertexts, one key each
    cts = residues(ctx.moduli, (len(st), 2), list(range(l)), 4)
    dcts = ckks.DeviceBuffer.from_array(cts)
    ctx.eval_rotate_many(dcts.ptr, l, st, [d.ptr for d in devks], out.ptr)
    many = out.download((len(st), 2, l, N))
    for i, s in enumerate(st):
        assert np.array_equal(many[i], octx.rotate(cts[i], l, octx.rot_index(s), evks[i])), s


@pytest.mark.parametrize("bs,n_diag", [(4, 10), (4, 4), (2, 9)])
def test_bsgs_composition_bit_exact(ckks, ctx, octx, bs, n_diag):
    """ckks_linear_transform_bsgs against the oracle composed from its stages: babies rotated (hoisted, each with its
    own ModDown), the ct x pt MAC over Q_l, then the giant sums rotated in Q_l P and brought down once --
    T = (P v0_0, P v0_1) + sum_{g >= 1} Auto_g(<ModUp(v_g.c1), evk_g> + (P v_g.c0, 0)), ModDown(T), rescale.
    Shapes: 3 giants with a short last one, a single giant (no rotation), 5 giants of 2 babies."""
    l = 5
    ng = -(-n_diag // bs)
    babies_st, giants_st = list(range(1, bs)), [g * bs for g in range(1, ng)]
    bevk = [residues(ctx.moduli, (DNUM, 2), list(range(L + K)), 200 + i) for i in range(len(babies_st))]
    gevk = [residues(ctx.moduli, (DNUM, 2), list(range(L + K)), 300 + i) for i in range(len(giants_st))]
    dbe = [ckks.DeviceBuffer.from_array(e) for e in bevk]
    dge = [ckks.DeviceBuffer.from_array(e) for e in gevk]
    ct = residues(ctx.moduli, (2,), list(range(l)), 5)
    diags = residues(ctx.moduli, (n_diag,), list(range(l)), 6)
    dct, dd = ckks.DeviceBuffer.from_array(ct), ckks.DeviceBuffer.from_array(diags)
    out = ckks.DeviceBuffer(2 * (l - 1) * N * 8)
    ctx.linear_transform_bsgs(dct.ptr, l, dd.ptr, n_diag, bs, [d.ptr for d in dbe], [d.ptr for d in dge], out.ptr)
    # oracle composition
    babies = [ct] + [octx.rotate(ct, l, octx.rot_index(s), bevk[i]) for i, s in enumerate(babies_st)]
    q = np.array(ctx.moduli[:l], dtype=object).reshape(1, -1, 1)
    pmap = list(range(l)) + list(range(L, L + K))
    E = l + K
    qe = np.array([ctx.moduli[i] for i in pmap], dtype=object).reshape(1, -1, 1)
    P = 1
    for k in range(K):
        P *= ctx.moduli[L + k]
    pq = np.array([P % ctx.moduli[i] for i in range(l)], dtype=object).reshape(-1, 1)
    T = np.zeros((2, E, N), dtype=object)
    for g in range(ng):
        acc = np.zeros((2, l, N), dtype=object)
        for j in range(bs):
            k = g * bs + j
            if k < n_diag:
                acc += babies[j].astype(object) * diags[k].astype(object)[None]
        v = (acc % q).astype(np.uint64)
        if g == 0:
            T[:, :l] += v.astype(object) * pq[None]
        else:
            x = octx.ks_inner(octx.modup(v[1], l), l, gevk[g - 1]).astype(object)
            x[0, :l] += v[0].astype(object) * pq
            x = (x % qe).astype(np.uint64)
            T += octx.automorph_eval(x, octx.rot_index(giants_st[g - 1])).astype(object)
    T = (T % qe).astype(np.uint64)
    want = octx.rescale(np.stack([octx.moddown(T[p], l) for p in range(2)]), l)
    assert np.array_equal(out.download((2, l - 1, N)), want)


@pytest.mark.timeout(600)
def test_pcmm_config3_decrypts(ckks, ctx):
    """768 x 768 weights N(0, 1/768), BSGS 28 x 28, ciphertext at L = 16 (config 3)."""
    d, bs, l = 768, 28, 16
    rng = np.random.default_rng(2024)
    W = rng.normal(0.0, np.sqrt(1.0 / d), (d, d))
    u = rng.uniform(-1.0, 1.0, d)
    sk = ctx.secret(b"P" * 32, 192)
    bst, gst = steps(d, bs)
    kb = DNUM * 2 * (L + K) * N * 8
    bkeys = [ckks.DeviceBuffer(kb) for _ in bst]
    gkeys = [ckks.DeviceBuffer(kb) for _ in gst]
    for i, s in enumerate(bst):
        ctx.keygen_automorphism(sk, ckks.rotation_index(s), bytes([1, i]) * 16, bytes([2, i]) * 16, bkeys[i].ptr)
    for i, s in enumerate(gst):
        ctx.keygen_automorphism(sk, ckks.rotation_index(s), bytes([3, i]) * 16, bytes([4, i]) * 16, gkeys[i].ptr)
    diags = bsgs_diagonals(W, bs)
    dd = ckks.DeviceBuffer(d * l * N * 8)
    for k in range(d):
        ctx.encode(diags[k], l, SCALE, dd.ptr + k * l * N * 8)
    pt = ckks.DeviceBuffer(l * N * 8)
    ct = ckks.DeviceBuffer(2 * l * N * 8)
    ctx.encode(replicate(u), l, SCALE, pt.ptr)
    ctx.encrypt(sk, pt.ptr, l, b"U" * 32, 0, ct.ptr)
    out = ckks.DeviceBuffer(2 * (l - 1) * N * 8)
    ctx.linear_transform_bsgs(ct.ptr, l, dd.ptr, d, bs, [k.ptr for k in bkeys], [k.ptr for k in gkeys], out.ptr)
    scale = SCALE * SCALE / ctx.moduli[l - 1]
    got = ctx.decrypt(sk, out.ptr, l - 1, scale)[:d]
    want = W @ u
    err = float(np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2)))
    assert err < 1e-6, err
