"""GPU parity of hybrid key switching, rescale, HMult+relin(+rescale), automorphism, rotation and add
against the CPU oracle, through the C ABI.  BASELINE config-2 parameters: N = 2^16, L = 24 x 54-bit,
K = 8 x 60-bit, dnum = 3.  Bar: bit-exact words.  Keys and ciphertexts are seeded uniform residues
(every integer stage is a deterministic function of its input words, so random words exercise it
fully; decryption-level checks with real keys are in test_gpu_ckks.py).
"""
import numpy as np
import pytest

from engine_loader import load_ckks

pytestmark = pytest.mark.gpu

L, K, DNUM = 24, 8, 3
N = 1 << 16


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


@pytest.fixture(scope="module")
def ctx(ckks):
    return ckks.Context(num_q=L, num_p=K, dnum=DNUM, q_bits=54, p_bits=60)


@pytest.fixture(scope="module")
def octx(oracle, ctx):
    return oracle.Ctx(16, ctx.moduli, L, K, DNUM)


def residues(moduli, shape_prefix, prime_idx, seed):
    rng = np.random.default_rng(seed)
    q = np.array([moduli[i] for i in prime_idx], dtype=np.uint64)
    x = rng.integers(0, 2**63, tuple(shape_prefix) + (len(prime_idx), N), dtype=np.uint64)
    return x % q.reshape((1,) * len(shape_prefix) + (-1, 1))


@pytest.fixture(scope="module")
def evk(ctx):
    return residues(ctx.moduli, (DNUM, 2), list(range(L + K)), seed=77)


@pytest.fixture(scope="module")
def d_evk(ckks, evk):
    return ckks.DeviceBuffer.from_array(evk)


def ext_primes(l):
    return list(range(l)) + [L + k for k in range(K)]


def test_modup_inner_moddown_stagewise(ckks, ctx, octx, evk, d_evk):
    B, l = 2, 24
    D, E = ctx.num_digits(l), l + K
    x = residues(ctx.moduli, (B,), list(range(l)), seed=1)
    dx = ckks.DeviceBuffer.from_array(x)
    dext = ckks.DeviceBuffer(B * D * E * N * 8)
    ctx.modup(dx.ptr, B, l, dext.ptr)
    ext = dext.download((B, D, E, N))
    for b in range(B):
        assert np.array_equal(ext[b], octx.modup(x[b], l)), b
    dacc = ckks.DeviceBuffer(B * 2 * E * N * 8)
    ctx.ks_inner(dext.ptr, B, l, d_evk.ptr, dacc.ptr)
    acc = dacc.download((B, 2, E, N))
    for b in range(B):
        assert np.array_equal(acc[b], octx.ks_inner(ext[b], l, evk)), b
    dout = ckks.DeviceBuffer(B * 2 * l * N * 8)
    ctx.moddown(dacc.ptr, 2 * B, l, dout.ptr)
    out = dout.download((B, 2, l, N))
    for b in range(B):
        for p in range(2):
            assert np.array_equal(out[b, p], octx.moddown(acc[b, p], l)), (b, p)


@pytest.mark.parametrize("l", [24, 13, 8, 1])
def test_keyswitch_levels(ckks, ctx, octx, evk, d_evk, l):
    """every digit count (3, 2, 1) and a ragged last digit (13 = 8 + 5)"""
    x = residues(ctx.moduli, (1,), list(range(l)), seed=10 + l)
    dx = ckks.DeviceBuffer.from_array(x)
    dout = ckks.DeviceBuffer(2 * l * N * 8)
    ctx.keyswitch(dx.ptr, 1, l, d_evk.ptr, dout.ptr)
    assert np.array_equal(dout.download((2, l, N)), octx.keyswitch(x[0], l, evk))


@pytest.mark.parametrize("l", [24, 11, 2])
def test_rescale(ckks, ctx, octx, l):
    x = residues(ctx.moduli, (3,), list(range(l)), seed=20 + l)
    dx = ckks.DeviceBuffer.from_array(x)
    dout = ckks.DeviceBuffer(3 * (l - 1) * N * 8)
    ctx.rescale(dx.ptr, 3, l, dout.ptr)
    assert np.array_equal(dout.download((3, l - 1, N)), octx.rescale(x, l))
    # the input is not modified
    assert np.array_equal(dx.download(x.shape), x)


def test_rescale_edge_values(ckks, ctx, octx):
    """last limb at 0, q/2, q/2 + 1 and q - 1: both sides of the centered-lift threshold"""
    l = 4
    x = residues(ctx.moduli, (1,), list(range(l)), seed=5)
    ql = ctx.moduli[l - 1]
    coef = np.zeros(N, dtype=np.uint64)
    coef[:4] = [0, ql // 2, ql // 2 + 1, ql - 1]
    coef[4:] = (np.arange(N - 4, dtype=np.uint64) * np.uint64(7919)) % np.uint64(ql)
    x[0, l - 1] = octx.ntt_fwd(coef[None], [l - 1])[0]
    dx = ckks.DeviceBuffer.from_array(x)
    dout = ckks.DeviceBuffer((l - 1) * N * 8)
    ctx.rescale(dx.ptr, 1, l, dout.ptr)
    assert np.array_equal(dout.download((1, l - 1, N)), octx.rescale(x, l))


def test_eval_mult_rescale_batch(ckks, ctx, octx, evk, d_evk):
    B, l = 2, 24
    a = residues(ctx.moduli, (B, 2), list(range(l)), seed=31)
    b = residues(ctx.moduli, (B, 2), list(range(l)), seed=32)
    da, db = ckks.DeviceBuffer.from_array(a), ckks.DeviceBuffer.from_array(b)
    dout = ckks.DeviceBuffer(B * 2 * (l - 1) * N * 8)
    ctx.eval_mult_rescale(da.ptr, db.ptr, B, l, d_evk.ptr, dout.ptr)
    out = dout.download((B, 2, l - 1, N))
    for i in range(B):
        assert np.array_equal(out[i], octx.hmult_relin_rescale(a[i], b[i], l, evk)), i


@pytest.mark.timeout(300)
def test_eval_mult_rescale_config2_full_batch(ckks, ctx, octx, evk, d_evk):
    """the shape bench.py times: 64 pairs at l = 24 in one call (launch grids 16 x 1472 for T's NTT with the combine,
    256 x 64 for the ModUp BConvs); the first and last pair and 2 seeded ones in between word for word against the
    oracle, every output word reduced"""
    B, l = 64, 24
    a = residues(ctx.moduli, (B, 2), list(range(l)), seed=35)
    b = residues(ctx.moduli, (B, 2), list(range(l)), seed=36)
    da, db = ckks.DeviceBuffer.from_array(a), ckks.DeviceBuffer.from_array(b)
    dout = ckks.DeviceBuffer(B * 2 * (l - 1) * N * 8)
    ctx.eval_mult_rescale(da.ptr, db.ptr, B, l, d_evk.ptr, dout.ptr)
    out = dout.download((B, 2, l - 1, N))
    q = np.array(ctx.moduli[:l - 1], dtype=np.uint64)
    assert bool((out < q[None, None, :, None]).all())
    rng = np.random.default_rng(37)
    for i in [0, B - 1] + sorted(rng.choice(np.arange(1, B - 1), 2, replace=False).tolist()):
        assert np.array_equal(out[i], octx.hmult_relin_rescale(a[i], b[i], l, evk)), i


@pytest.mark.parametrize("alias", ["a", "b"])
def test_eval_mult_rescale_in_place(ckks, ctx, octx, evk, d_evk, alias):
    """The output written over an input (the product's d0 / d1 then take the tensor kernel's round trip, since the
    ModDown combine would read the inputs while writing the output)."""
    B, l = 2, 7
    a = residues(ctx.moduli, (B, 2), list(range(l)), seed=33)
    b = residues(ctx.moduli, (B, 2), list(range(l)), seed=34)
    da, db = ckks.DeviceBuffer.from_array(a), ckks.DeviceBuffer.from_array(b)
    dst = da if alias == "a" else db
    ctx.eval_mult_rescale(da.ptr, db.ptr, B, l, d_evk.ptr, dst.ptr)
    out = dst.download((B, 2, l - 1, N))
    for i in range(B):
        assert np.array_equal(out[i], octx.hmult_relin_rescale(a[i], b[i], l, evk)), i


def test_relin_and_keyswitch_fused_ntt_mode(ckks, ctx, octx, evk, d_evk):
    """The other NTT schedule (mode 1: one limb per workgroup) takes the unfused combines (k_mdr_combine_ks with the
    product's inputs, k_ks_sub_list and k_sub_scale after the NTT, the stored inner products, the separate lift) in
    place of the NTT passes that end in or begin with them: same words."""
    B, l = 2, 9
    a = residues(ctx.moduli, (B, 2), list(range(l)), seed=35)
    b = residues(ctx.moduli, (B, 2), list(range(l)), seed=36)
    x = residues(ctx.moduli, (1,), list(range(l)), seed=37)
    ct = residues(ctx.moduli, (2, 2), list(range(l)), seed=38)
    da, db, dx, dct = (ckks.DeviceBuffer.from_array(v) for v in (a, b, x, ct))
    dout = ckks.DeviceBuffer(B * 2 * (l - 1) * N * 8)
    dks = ckks.DeviceBuffer(2 * l * N * 8)
    drot = ckks.DeviceBuffer(ct.nbytes)
    dres = ckks.DeviceBuffer(3 * (l - 1) * N * 8)
    ctx.set_ntt_mode(1)
    try:
        ctx.eval_mult_rescale(da.ptr, db.ptr, B, l, d_evk.ptr, dout.ptr)
        ctx.keyswitch(dx.ptr, 1, l, d_evk.ptr, dks.ptr)
        ctx.eval_rotate(dct.ptr, 2, l, 5, d_evk.ptr, drot.ptr)
        ctx.rescale(da.ptr, 3, l, dres.ptr)
    finally:
        ctx.set_ntt_mode(0)
    out = dout.download((B, 2, l - 1, N))
    for i in range(B):
        assert np.array_equal(out[i], octx.hmult_relin_rescale(a[i], b[i], l, evk)), i
    assert np.array_equal(dks.download((2, l, N)), octx.keyswitch(x[0], l, evk))
    rot = drot.download(ct.shape)
    for i in range(2):
        assert np.array_equal(rot[i], octx.rotate(ct[i], l, octx.rot_index(5), evk)), i
    assert np.array_equal(dres.download((3, l - 1, N)), octx.rescale(a.reshape(-1, l, N)[:3], l))


def test_eval_mult_no_rescale(ckks, ctx, octx, evk, d_evk):
    l = 9
    a = residues(ctx.moduli, (1, 2), list(range(l)), seed=41)
    b = residues(ctx.moduli, (1, 2), list(range(l)), seed=42)
    da, db = ckks.DeviceBuffer.from_array(a), ckks.DeviceBuffer.from_array(b)
    dout = ckks.DeviceBuffer(2 * l * N * 8)
    ctx.eval_mult(da.ptr, db.ptr, 1, l, d_evk.ptr, dout.ptr)
    d = octx.tensor(a[0], b[0], l)
    ks = octx.keyswitch(d[2], l, evk)
    q = np.array(ctx.moduli[:l], dtype=np.uint64)[:, None]
    want = np.stack([(d[p].astype(object) + ks[p].astype(object)) % q.astype(object) for p in range(2)]).astype(np.uint64)
    assert np.array_equal(dout.download((2, l, N)), want)


@pytest.mark.parametrize("step", [1, 3, -7, 1024])
def test_automorphism(ckks, ctx, octx, step):
    l = 3
    g = ckks.rotation_index(step)
    assert g == octx.rot_index(step)
    x = residues(ctx.moduli, (2,), list(range(l)), seed=50 + abs(step))
    dx = ckks.DeviceBuffer.from_array(x)
    dout = ckks.DeviceBuffer(x.nbytes)
    ctx.automorphism(dx.ptr, 2, l, g, dout.ptr)
    out = dout.download(x.shape)
    for p in range(2):
        assert np.array_equal(out[p], octx.automorph_eval(x[p], g))
    # conjugation index 2N - 1
    ctx.automorphism(dx.ptr, 2, l, 2 * N - 1, dout.ptr)
    assert np.array_equal(dout.download(x.shape)[1], octx.automorph_eval(x[1], 2 * N - 1))


@pytest.mark.parametrize("step", [5, -3])
def test_eval_rotate(ckks, ctx, octx, evk, d_evk, step):
    l = 16
    ct = residues(ctx.moduli, (2, 2), list(range(l)), seed=60 + step)
    dct = ckks.DeviceBuffer.from_array(ct)
    dout = ckks.DeviceBuffer(ct.nbytes)
    ctx.eval_rotate(dct.ptr, 2, l, step, d_evk.ptr, dout.ptr)
    out = dout.download(ct.shape)
    g = octx.rot_index(step)
    for i in range(2):
        assert np.array_equal(out[i], octx.rotate(ct[i], l, g, evk)), i


def test_rotation_lists_out_of_place_and_in_place(ckks, ctx, octx, evk, d_evk):
    """The list rotations (many, hoisted, automorphism with key switch), whose automorphism the key-switch combine
    applies as it stores, against the oracle's rotations -- out of place, and in place, where the output overlaps
    the ciphertext whose c0 the combine adds (the combine then writes a workspace and a permutation pass follows)."""
    l = 12
    cts = residues(ctx.moduli, (2, 2), list(range(l)), seed=91)
    g1, g3, gc = octx.rot_index(1), octx.rot_index(-3), 2 * N - 1
    r01 = octx.rotate(cts[0], l, g1, evk)
    r03 = octx.rotate(cts[0], l, g3, evk)
    r13 = octx.rotate(cts[1], l, g3, evk)
    r0c = octx.rotate(cts[0], l, gc, evk)
    keys = [d_evk.ptr, d_evk.ptr]
    dct = ckks.DeviceBuffer.from_array(cts)
    dout = ckks.DeviceBuffer(cts.nbytes)
    ctx.eval_rotate_many(dct.ptr, l, [1, -3], keys, dout.ptr)
    out = dout.download(cts.shape)
    assert np.array_equal(out[0], r01) and np.array_equal(out[1], r13)
    ctx.eval_rotate_hoisted(dct.ptr, l, [1, -3], keys, dout.ptr)
    out = dout.download(cts.shape)
    assert np.array_equal(out[0], r01) and np.array_equal(out[1], r03)
    ctx.eval_automorphism_ks(dct.ptr, 1, l, gc, d_evk.ptr, dout.ptr)
    assert np.array_equal(dout.download(cts[0].shape), r0c)
    # in place: the hoisted rotations' outputs over the ciphertext itself, the conjugation of ciphertext 0 over itself
    dbuf = ckks.DeviceBuffer.from_array(cts)
    ctx.eval_rotate_hoisted(dbuf.ptr, l, [1, -3], keys, dbuf.ptr)
    out = dbuf.download(cts.shape)
    assert np.array_equal(out[0], r01) and np.array_equal(out[1], r03)
    dbuf = ckks.DeviceBuffer.from_array(cts)
    ctx.eval_automorphism_ks(dbuf.ptr, 1, l, gc, d_evk.ptr, dbuf.ptr)
    out = dbuf.download(cts.shape)
    assert np.array_equal(out[0], r0c) and np.array_equal(out[1], cts[1])


def test_eval_add(ckks, ctx):
    l = 5
    x = residues(ctx.moduli, (4,), list(range(l)), seed=70)
    y = residues(ctx.moduli, (4,), list(range(l)), seed=71)
    dx, dy = ckks.DeviceBuffer.from_array(x), ckks.DeviceBuffer.from_array(y)
    dout = ckks.DeviceBuffer(x.nbytes)
    ctx.eval_add(dx.ptr, dy.ptr, 4, l, dout.ptr)
    q = np.array(ctx.moduli[:l], dtype=np.uint64)[None, :, None]
    want = ((x.astype(object) + y.astype(object)) % q.astype(object)).astype(np.uint64)
    assert np.array_equal(dout.download(x.shape), want)


def test_error_paths(ckks, ctx):
    """bad levels and aliasing are refused with a status code, nothing is launched"""
    lib = ckks.load()
    assert lib.ckks_rescale(ctx.h, 1, 2, 1, 2, None) != 0
    assert b"alias" in lib.ckks_last_error() or b"level" in lib.ckks_last_error()
    assert lib.ckks_keyswitch(ctx.h, 1, 1, L + 1, 1, 1, None) == 1
    assert b"level" in lib.ckks_last_error()
    assert lib.ckks_eval_rotate(ctx.h, 8, 1, 4, 1, 8, 8, None) == 1


def test_four_digit_key_switch(ckks, oracle):
    """Four digits (L = 32, dnum = 4): the 4-digit instances of the kernels that form the evk inner products inside
    the NTT passes (relinearization with rescale, key switch, rotation) against the oracle."""
    L4, K4, D4 = 32, 8, 4
    c4 = ckks.Context(num_q=L4, num_p=K4, dnum=D4, q_bits=54, p_bits=60)
    o4 = oracle.Ctx(16, c4.moduli, L4, K4, D4)
    l = L4
    assert c4.num_digits(l) == 4
    ev = residues(c4.moduli, (D4, 2), list(range(L4 + K4)), seed=91)
    dev = ckks.DeviceBuffer.from_array(ev)
    a = residues(c4.moduli, (1, 2), list(range(l)), seed=92)
    b = residues(c4.moduli, (1, 2), list(range(l)), seed=93)
    x = residues(c4.moduli, (1,), list(range(l)), seed=94)
    da, db, dx = (ckks.DeviceBuffer.from_array(v) for v in (a, b, x))
    dout = ckks.DeviceBuffer(2 * (l - 1) * N * 8)
    c4.eval_mult_rescale(da.ptr, db.ptr, 1, l, dev.ptr, dout.ptr)
    assert np.array_equal(dout.download((2, l - 1, N)), o4.hmult_relin_rescale(a[0], b[0], l, ev))
    dks = ckks.DeviceBuffer(2 * l * N * 8)
    c4.keyswitch(dx.ptr, 1, l, dev.ptr, dks.ptr)
    assert np.array_equal(dks.download((2, l, N)), o4.keyswitch(x[0], l, ev))
    drot = ckks.DeviceBuffer(a.nbytes)
    c4.eval_rotate(da.ptr, 1, l, 3, dev.ptr, drot.ptr)
    assert np.array_equal(drot.download(a.shape)[0], o4.rotate(a[0], l, o4.rot_index(3), ev))
    c4.close()


def test_rotate_sum_of_64_rotations(ckks, oracle):
    """ckks_eval_rotate_sum at its limit of 64 rotations (steps 1..64, each with its own key), on a small chain so
    that the 64 keys stay small: ct + sum_s Rot_s(ct) with one ModUp and one ModDown, against the oracle composed
    from its stages -- ModDown((P c0, P c1) + sum_s Auto_s(<ModUp(c1), evk_s> + (P c0, 0))) per poly"""
    Ls, Ks, Ds = 2, 1, 2
    cs = ckks.Context(num_q=Ls, num_p=Ks, dnum=Ds, q_bits=54, p_bits=60)
    os_ = oracle.Ctx(16, cs.moduli, Ls, Ks, Ds)
    l, E = Ls, Ls + Ks
    steps = list(range(1, 65))
    ev = {s: residues(cs.moduli, (Ds, 2), list(range(Ls + Ks)), seed=500 + s) for s in steps}
    dk = {s: ckks.DeviceBuffer.from_array(e) for s, e in ev.items()}
    x = residues(cs.moduli, (1, 2), list(range(l)), seed=95)
    dx = ckks.DeviceBuffer.from_array(x)
    out = ckks.DeviceBuffer(x.nbytes)
    cs.eval_rotate_sum(dx.ptr, 1, l, steps, [dk[s].ptr for s in steps], out.ptr)
    qe = np.array(list(cs.moduli[:l]) + list(cs.moduli[Ls:Ls + Ks]), dtype=object).reshape(-1, 1)
    P = cs.moduli[Ls]
    pq = np.array([P % q for q in cs.moduli[:l]], dtype=object).reshape(-1, 1)
    c = x[0]
    T = np.zeros((2, E, N), dtype=object)
    T[0, :l] = c[0].astype(object) * pq % qe[:l]
    T[1, :l] = c[1].astype(object) * pq % qe[:l]
    ext = os_.modup(c[1], l)
    for s in steps:
        acc = os_.ks_inner(ext, l, ev[s]).astype(object)
        acc[0, :l] += c[0].astype(object) * pq % qe[:l]
        T += os_.automorph_eval((acc % qe[None]).astype(np.uint64), os_.rot_index(s)).astype(object)
    T = (T % qe[None]).astype(np.uint64)
    want = np.stack([os_.moddown(T[p], l) for p in range(2)])
    assert np.array_equal(out.download(x.shape)[0], want)
    # 65 rotations are refused
    with pytest.raises(RuntimeError):
        cs.eval_rotate_sum(dx.ptr, 1, l, steps + [65], [dk[1].ptr] * 65, out.ptr)
    cs.close()
