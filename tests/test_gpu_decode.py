"""Config 5 on the GPU: the decode-step entry points bit-exact against the oracle composed from its
stages, the config-5 chain's bootstrapping precision, and the encrypted decode step against the float64
reference model (relErrRms <= 1e-3, the north star's bar for the full step).

Chain (fhe-ssm_amd/decode_step.py): q0 50-bit, 28 scaling primes within 2^-12 of 2^40 (chosen so that the
FLEXIBLE scales stay at 2^40), 3 x 60-bit CoeffToSlot primes, P 7 x 60-bit, dnum 4 (so K = 7 < alpha = 8:
P only has to exceed each digit's product).
"""
import numpy as np
import pytest

from engine_loader import load_ckks, load_module

pytestmark = pytest.mark.gpu

N = 1 << 16
SLOTS = N // 2
LOG_REP = 5


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


@pytest.fixture(scope="module")
def DS():
    return load_module("decode_step")


@pytest.fixture(scope="module")
def M():
    return load_module("rwkv_model")


@pytest.fixture(scope="module")
def ctx5(ckks, DS):
    c = ckks.Context(num_q=32, num_p=7, dnum=4, scale=2.0**40, moduli=DS.config5_moduli(ckks))
    c.set_moddown_exact(True)
    return c


@pytest.fixture(scope="module")
def octx5(oracle, ctx5):
    return oracle.Ctx(16, ctx5.moduli, ctx5.L, ctx5.K, ctx5.dnum, moddown_exact=True)


@pytest.mark.parametrize("exact", [False, True])
def test_moddown_keyswitch_bit_exact(ckks, oracle, ctx5, exact):
    """ModDown and the full key switch in both rounding modes against the oracle (config-5 chain, K < alpha)"""
    L, K, D = ctx5.L, ctx5.K, ctx5.dnum
    oc = oracle.Ctx(16, ctx5.moduli, L, K, D, moddown_exact=exact)
    ctx5.set_moddown_exact(exact)
    try:
        l = 13
        x = residues(ctx5.moduli, (2,), list(range(l)) + [L + k for k in range(K)], 41)
        dx = ckks.DeviceBuffer.from_array(x)
        out = ckks.DeviceBuffer(2 * l * N * 8)
        ctx5.moddown(dx.ptr, 2, l, out.ptr)
        got = out.download((2, l, N))
        for p in range(2):
            assert np.array_equal(got[p], oc.moddown(x[p], l)), p
        evk = residues(ctx5.moduli, (D, 2), list(range(L + K)), 42)
        devk = ckks.DeviceBuffer.from_array(evk)
        y = residues(ctx5.moduli, (1,), list(range(l)), 43)
        dy = ckks.DeviceBuffer.from_array(y)
        ctx5.keyswitch(dy.ptr, 1, l, devk.ptr, out.ptr)
        assert np.array_equal(out.download((2, l, N)), oc.keyswitch(y[0], l, evk))
    finally:
        ctx5.set_moddown_exact(True)


def residues(moduli, shape_prefix, prime_idx, seed):
    rng = np.random.default_rng(seed)
    q = np.array([moduli[i] for i in prime_idx], dtype=np.uint64)
    x = rng.integers(0, 2**63, tuple(shape_prefix) + (len(prime_idx), N), dtype=np.uint64)
    return x % q.reshape((1,) * len(shape_prefix) + (-1, 1))


def qcol(ctx, l):
    return np.array(ctx.moduli[:l], dtype=object).reshape(-1, 1)


def expand(comp):
    """compressed periodic plaintext [..., l, N/32] -> evaluation form [..., l, N]"""
    return np.repeat(comp, 1 << LOG_REP, axis=-1)


def test_chain(ctx5):
    m = ctx5.moduli
    assert m[0].bit_length() == 50 and all(abs(q / 2.0**40 - 1) < 2.0**-12 for q in m[1:29])
    assert all(q.bit_length() == 60 for q in m[29:]) and len(set(m)) == 39
    assert all(q % (1 << 17) == 1 for q in m)
    # the FLEXIBLE scales from 2^40 at the CoeffToSlot levels down to level 1 stay within 2^+-0.001 of 2^40
    S = 2.0**40
    for l in range(29, 1, -1):
        S = S * S / m[l - 1]
        assert abs(np.log2(S) - 40) < 1e-3, l


def test_mult_sum_bit_exact(ckks, ctx5, octx5):
    """relin(sum_j a_j (x) b_j) + rescale == the oracle's tensors summed, key-switched, rescaled"""
    l, B, npr = 9, 2, 3
    L, K, D = ctx5.L, ctx5.K, ctx5.dnum
    evk = residues(ctx5.moduli, (D, 2), list(range(L + K)), 5)
    devk = ckks.DeviceBuffer.from_array(evk)
    cts = residues(ctx5.moduli, (B, npr, 2, 2), list(range(l)), 6)  # [b][j][a/b][poly]
    dc = ckks.DeviceBuffer.from_array(cts)
    ctw = 2 * l * N * 8

    def ptr(b, j, w):
        return dc.ptr + ((b * npr + j) * 2 + w) * ctw

    out = ckks.DeviceBuffer(B * 2 * (l - 1) * N * 8)
    ctx5.eval_mult_sum([[(ptr(b, j, 0), ptr(b, j, 1)) for j in range(npr)] for b in range(B)], l, devk.ptr, out.ptr)
    got = out.download((B, 2, l - 1, N))
    q = qcol(ctx5, l)
    for b in range(B):
        acc = None
        for j in range(npr):
            d = octx5.tensor(cts[b, j, 0], cts[b, j, 1], l).astype(object)
            acc = d if acc is None else acc + d
        acc = (acc % q[None]).astype(np.uint64)
        ks = octx5.keyswitch(acc[2], l, evk).astype(object)
        rel = ((acc[:2].astype(object) + ks) % q[None]).astype(np.uint64)
        assert np.array_equal(got[b], octx5.rescale(rel, l)), b
    # one product: the same as EvalMult + rescale
    out1 = ckks.DeviceBuffer(2 * (l - 1) * N * 8)
    ctx5.eval_mult_sum([[(ptr(0, 0, 0), ptr(0, 0, 1))]], l, devk.ptr, out1.ptr)
    ref = ckks.DeviceBuffer(2 * (l - 1) * N * 8)
    ctx5.eval_mult_rescale(ptr(0, 0, 0), ptr(0, 0, 1), 1, l, devk.ptr, ref.ptr)
    assert np.array_equal(out1.download((2, l - 1, N)), ref.download((2, l - 1, N)))


def test_mult_plain_compressed_bit_exact(ckks, ctx5):
    l, B = 4, 2
    ct = residues(ctx5.moduli, (B, 2), list(range(l)), 7)
    comp = residues(ctx5.moduli, (), list(range(l)), 8)[:, : N >> LOG_REP]
    dct, dp = ckks.DeviceBuffer.from_array(ct), ckks.DeviceBuffer.from_array(np.ascontiguousarray(comp))
    out = ckks.DeviceBuffer(ct.nbytes)
    ctx5.eval_mult_plain_ex(dct.ptr, B, l, dp.ptr, LOG_REP, out.ptr)
    full = expand(comp)
    q = qcol(ctx5, l)
    want = ((ct.astype(object) * full.astype(object)[None, None]) % q[None, None]).astype(np.uint64)
    assert np.array_equal(out.download(ct.shape), want)


def test_encode_periodic_decrypts(ckks, ctx5, M):
    """a 1024-periodic plaintext multiplied into an encryption of x decrypts to x (.) periodic vector"""
    l = 6
    sk = ctx5.secret(b"Q" * 32, 192)
    rng = np.random.default_rng(9)
    x = rng.uniform(-1, 1, SLOTS)
    p = rng.uniform(-1, 1, M.DPAD)
    S = 2.0**40
    pt = ckks.DeviceBuffer(l * N * 8)
    ct = ckks.DeviceBuffer(2 * l * N * 8)
    ctx5.encode(x, l, S, pt.ptr)
    ctx5.encrypt(sk, pt.ptr, l, b"x" * 32, 0, ct.ptr)
    comp = ckks.DeviceBuffer(l * (N >> LOG_REP) * 8)
    ctx5.encode_periodic(p[None], l, S, comp.ptr)
    out = ckks.DeviceBuffer(2 * l * N * 8)
    ctx5.eval_mult_plain_ex(ct.ptr, 1, l, comp.ptr, LOG_REP, out.ptr)
    got = ctx5.decrypt(sk, out.ptr, l, S * S)
    assert np.max(np.abs(got - x * np.tile(p, SLOTS // M.DPAD))) < 1e-6


def test_rotate_masked_bit_exact(ckks, ctx5, octx5):
    l, n, n_sets = 5, 3, 2
    L, K, D = ctx5.L, ctx5.K, ctx5.dnum
    lo, hi = [0, 1, 5], [0, -63, -59]
    steps = sorted(set(lo + hi) - {0})
    evk = {s: residues(ctx5.moduli, (D, 2), list(range(L + K)), 100 + i) for i, s in enumerate(steps)}
    dk = {s: ckks.DeviceBuffer.from_array(e) for s, e in evk.items()}
    ct = residues(ctx5.moduli, (2,), list(range(l)), 11)
    comp = residues(ctx5.moduli, (n_sets, n, 2), list(range(l)), 12)[..., : N >> LOG_REP]
    dct, dp = ckks.DeviceBuffer.from_array(ct), ckks.DeviceBuffer.from_array(np.ascontiguousarray(comp))
    out = ckks.DeviceBuffer(n_sets * n * 2 * (l - 1) * N * 8)
    ctx5.eval_rotate_masked(dct.ptr, l, lo, [dk[s].ptr if s else None for s in lo], hi,
                            [dk[s].ptr if s else None for s in hi], n_sets, dp.ptr, LOG_REP, out.ptr)
    got = out.download((n_sets, n, 2, l - 1, N))
    q = qcol(ctx5, l)

    def rot(s):
        return ct if s == 0 else octx5.rotate(ct, l, octx5.rot_index(s), evk[s])

    for s in range(n_sets):
        for t in range(n):
            acc = rot(lo[t]).astype(object) * expand(comp[s, t, 0]).astype(object)[None] + \
                rot(hi[t]).astype(object) * expand(comp[s, t, 1]).astype(object)[None]
            want = octx5.rescale((acc % q[None]).astype(np.uint64), l)
            assert np.array_equal(got[s, t], want), (s, t)


@pytest.mark.parametrize("gst,rescale", [([0, 3, -3], True), ([3, 0, -3], False), ([3, -3], True)])
def test_linear_transform_multi_bit_exact(ckks, ctx5, octx5, gst, rescale):
    """2 inputs sharing babies {0, 1, 2}, 2 outputs sharing the babies, compressed diagonals, with and without the
    rescale, the identity giant first, in the middle or absent: against the oracle composition -- babies rotated
    (each with its own ModDown), the MAC over Q_l, then each output's giant sums rotated in Q_l P and brought down
    once: T = (P v_{g0}) + sum_{g != g0} Auto_g(<ModUp(v_g.c1), evk_g> + (P v_g.c0, 0)), ModDown(T) (then rescale)"""
    l, n_in, n_out = 4, 2, 2
    L, K, D = ctx5.L, ctx5.K, ctx5.dnum
    bst = [0, 1, 2]
    nb, ng = len(bst), len(gst)
    steps = [1, 2, 3, -3]
    evk = {s: residues(ctx5.moduli, (D, 2), list(range(L + K)), 200 + i) for i, s in enumerate(steps)}
    dk = {s: ckks.DeviceBuffer.from_array(e) for s, e in evk.items()}
    xs = residues(ctx5.moduli, (n_in, 2), list(range(l)), 21)
    diags = residues(ctx5.moduli, (n_out, ng, n_in * nb), list(range(l)), 22)[..., : N >> LOG_REP]
    dx, dd = ckks.DeviceBuffer.from_array(xs), ckks.DeviceBuffer.from_array(np.ascontiguousarray(diags))
    lo = l - 1 if rescale else l
    out = ckks.DeviceBuffer(n_out * 2 * lo * N * 8)
    ctw = 2 * l * N * 8
    ctx5.linear_transform_multi([dx.ptr + i * ctw for i in range(n_in)], l, dd.ptr, LOG_REP, bst,
                                [dk[s].ptr if s else None for s in bst], gst,
                                [dk[s].ptr if s else None for s in gst], n_out, rescale, out.ptr)
    got = out.download((n_out, 2, lo, N))
    q = qcol(ctx5, l)
    pmap = list(range(l)) + list(range(L, L + K))
    E = l + K
    qe = np.array([ctx5.moduli[i] for i in pmap], dtype=object).reshape(-1, 1)
    P = 1
    for k in range(K):
        P *= ctx5.moduli[L + k]
    pq = np.array([P % ctx5.moduli[i] for i in range(l)], dtype=object).reshape(-1, 1)

    def rot(c, s):
        return c if s == 0 else octx5.rotate(c, l, octx5.rot_index(s), evk[s])

    babies = [rot(xs[i], s) for i in range(n_in) for s in bst]
    for o in range(n_out):
        T = np.zeros((2, E, N), dtype=object)
        for g in range(ng):
            acc = sum(babies[j].astype(object) * expand(diags[o, g, j]).astype(object)[None] for j in range(n_in * nb))
            v = (acc % q[None]).astype(np.uint64)
            if gst[g] == 0:
                T[:, :l] += v.astype(object) * pq[None]
                continue
            x = octx5.ks_inner(octx5.modup(v[1], l), l, evk[gst[g]]).astype(object)
            x[0, :l] += v[0].astype(object) * pq
            x = (x % qe[None]).astype(np.uint64)
            T += octx5.automorph_eval(x, octx5.rot_index(gst[g])).astype(object)
        T = (T % qe[None]).astype(np.uint64)
        want = np.stack([octx5.moddown(T[p], l) for p in range(2)])
        if rescale:
            want = octx5.rescale(want, l)
        assert np.array_equal(got[o], want), o


@pytest.mark.parametrize("gst", [[0, 3, -3], [3, 0, -3], [2, 3, -3]])
def test_linear_transform_hoisted_bit_exact(ckks, ctx5, octx5, gst):
    """Double-hoisted BSGS (the bootstrap's CoeffToSlot / SlotToCoeff form) against the oracle composed from its
    stages: babies rotated in Q_l P without a ModDown, diagonals over Q_l P, one ModDown per giant inner sum,
    giant rotations summed in Q_l P, ModDown then rescale.  A giant's inner sum S = (S0, S1) brings only S1 down to
    Q_l (the key switch needs it there); the rotation in Q_l P is Auto(<ModUp(ModDown(S1)), evk> + (S0, 0)), and the
    identity giant's S is added as it is.  2 inputs, 2 outputs, babies {0, 1, 2}; giants with the identity first, in
    the middle, or absent."""
    l, n_in, n_out = 5, 2, 2
    L, K, D = ctx5.L, ctx5.K, ctx5.dnum
    bst = [0, 1, 2]
    nb, ng = len(bst), len(gst)
    steps = [1, 2, 3, -3]
    pmap = list(range(l)) + list(range(L, L + K))
    E = l + K
    evk = {s: residues(ctx5.moduli, (D, 2), list(range(L + K)), 300 + i) for i, s in enumerate(steps)}
    dk = {s: ckks.DeviceBuffer.from_array(e) for s, e in evk.items()}
    xs = residues(ctx5.moduli, (n_in, 2), list(range(l)), 31)
    diags = residues(ctx5.moduli, (n_out, ng, n_in * nb), pmap, 32)
    dx, dd = ckks.DeviceBuffer.from_array(xs), ckks.DeviceBuffer.from_array(diags)
    out = ckks.DeviceBuffer(n_out * 2 * (l - 1) * N * 8)
    ctw = 2 * l * N * 8
    ctx5.linear_transform_hoisted([dx.ptr + i * ctw for i in range(n_in)], l, dd.ptr, bst,
                                  [dk[s].ptr if s else None for s in bst], gst,
                                  [dk[s].ptr if s else None for s in gst], n_out, out.ptr)
    got = out.download((n_out, 2, l - 1, N))
    qe = np.array([ctx5.moduli[i] for i in pmap], dtype=object).reshape(-1, 1)
    P = 1
    for k in range(K):
        P *= ctx5.moduli[L + k]
    pq = np.array([P % ctx5.moduli[i] for i in range(l)], dtype=object).reshape(-1, 1)

    def lift(c, both):
        """(P c0, P c1) (both) or (P c0, 0) on the Q limbs, zero on the P limbs: [2][E][N] objects"""
        r = np.zeros((2, E, N), dtype=object)
        r[0, :l] = c[0].astype(object) * pq % qe[:l]
        if both:
            r[1, :l] = c[1].astype(object) * pq % qe[:l]
        return r

    def rot_qp(c, s):
        """rotation by s kept in Q_l P: Auto(<ModUp(c1), evk> + (P c0, 0)), or (P c0, P c1) for s = 0"""
        if s == 0:
            return lift(c, True)
        acc = octx5.ks_inner(octx5.modup(c[1], l), l, evk[s]).astype(object)
        v = ((acc + lift(c, False)) % qe[None]).astype(np.uint64)
        return octx5.automorph_eval(v, octx5.rot_index(s)).astype(object)

    def giant_qp(S, s):
        """a giant rotation of an inner sum S over Q_l P: Auto(<ModUp(ModDown(S1)), evk> + (S0, 0))"""
        acc = octx5.ks_inner(octx5.modup(octx5.moddown(S[1], l), l), l, evk[s]).astype(object)
        acc[0] += S[0].astype(object)
        v = (acc % qe[None]).astype(np.uint64)
        return octx5.automorph_eval(v, octx5.rot_index(s)).astype(object)

    babies = [rot_qp(xs[i], s) for i in range(n_in) for s in bst]
    g0 = gst.index(0) if 0 in gst else -1
    for o in range(n_out):
        T = np.zeros((2, E, N), dtype=object)
        for g in range(ng):
            S = sum(babies[j] * diags[o, g, j].astype(object)[None] for j in range(n_in * nb))
            S = (S % qe[None]).astype(np.uint64)
            T += S.astype(object) if g == g0 else giant_qp(S, gst[g])
        T = (T % qe[None]).astype(np.uint64)
        want = octx5.rescale(np.stack([octx5.moddown(T[p], l) for p in range(2)]), l)
        assert np.array_equal(got[o], want), o


def test_rotate_sum_bit_exact(ckks, ctx5, octx5):
    """ckks_eval_rotate_sum (a rotate-and-add window hoisted over one ModUp and one ModDown) against the oracle
    composed from its stages: ModDown( (P c0, P c1) + sum_s Auto_s(<ModUp(c1), evk_s> + (P c0, 0)) ) per poly, for a
    batch of 2 ciphertexts, in place and out of place; and a window of one step"""
    l, B = 5, 2
    L, K, D = ctx5.L, ctx5.K, ctx5.dnum
    steps = [1, 2, -3, 7]
    E = l + K
    pmap = list(range(l)) + list(range(L, L + K))
    evk = {s: residues(ctx5.moduli, (D, 2), list(range(L + K)), 400 + i) for i, s in enumerate(steps)}
    dk = {s: ckks.DeviceBuffer.from_array(e) for s, e in evk.items()}
    xs = residues(ctx5.moduli, (B, 2), list(range(l)), 41)
    qe = np.array([ctx5.moduli[i] for i in pmap], dtype=object).reshape(-1, 1)
    P = 1
    for k in range(K):
        P *= ctx5.moduli[L + k]
    pq = np.array([P % ctx5.moduli[i] for i in range(l)], dtype=object).reshape(-1, 1)

    def want(c, st):
        T = np.zeros((2, E, N), dtype=object)
        T[0, :l] = c[0].astype(object) * pq % qe[:l]
        T[1, :l] = c[1].astype(object) * pq % qe[:l]
        ext = octx5.modup(c[1], l)
        for s in st:
            acc = octx5.ks_inner(ext, l, evk[s]).astype(object)
            acc[0, :l] += c[0].astype(object) * pq % qe[:l]
            v = (acc % qe[None]).astype(np.uint64)
            T += octx5.automorph_eval(v, octx5.rot_index(s)).astype(object)
        T = (T % qe[None]).astype(np.uint64)
        return np.stack([octx5.moddown(T[p], l) for p in range(2)])

    for st in (steps, [-3]):
        dx = ckks.DeviceBuffer.from_array(xs)
        out = ckks.DeviceBuffer(B * 2 * l * N * 8)
        ctx5.eval_rotate_sum(dx.ptr, B, l, st, [dk[s].ptr for s in st], out.ptr)
        got = out.download((B, 2, l, N))
        for b in range(B):
            assert np.array_equal(got[b], want(xs[b], st)), (st, b)
        # in place
        ctx5.eval_rotate_sum(dx.ptr, B, l, st, [dk[s].ptr for s in st], dx.ptr)
        assert np.array_equal(dx.download((B, 2, l, N)), got), st
    # refusals: no steps, the identity, a missing key
    dx = ckks.DeviceBuffer.from_array(xs)
    for st, keys in (([], []), ([0], [dk[1].ptr]), ([1], [None])):
        with pytest.raises(RuntimeError):
            ctx5.eval_rotate_sum(dx.ptr, B, l, st, keys, dx.ptr)


def test_rotate_sum_decrypts_to_the_window_sum(engine, DS):
    """an encrypted rotate-and-add window (the norms' lane sum: windows 1..31, 32..480 by 32, 512) decrypts to the
    sums over 1,024 consecutive slots, within the key-switching noise"""
    be, sk = engine
    rng = np.random.default_rng(77)
    z = rng.uniform(-1, 1, SLOTS)
    ct = be.encrypt(sk, z, 10)
    s = ct
    for w in DS.M.NORM_UP:
        s = be.rotate_sum(s, w)
    got = be.decrypt(sk, s)
    want = sum(np.roll(z, -k) for k in range(1024))
    assert np.abs(got - want).max() < 1e-4 * np.abs(want).max()


@pytest.fixture(scope="module")
def engine(ckks, DS):
    be, sk = DS.build_engine(ckks)
    return be, sk


@pytest.mark.timeout(900)
def test_config5_chain_bootstrap(engine):
    """sparse-secret encapsulation (h' = 32), K = 14, Chebyshev 59, 2 double angles on the config-5 chain:
    level 17 out, precision bar 11 bits"""
    be, sk = engine
    assert be.top_level == 17
    rng = np.random.default_rng(31)
    z = rng.uniform(-1, 1, SLOTS)
    ct = be.encrypt(sk, z, 3)
    out = be.bootstrap(ct, "state")
    got = be.decrypt(sk, out)
    err = np.abs(got - z)
    bits = -np.log2(err.max())
    print(f"config-5 chain bootstrap: {bits:.2f} bits (max {err.max():.3e}, rms {np.sqrt(np.mean(err**2)):.3e})")
    assert bits > 11.0


@pytest.mark.timeout(900)
def test_bootstrap_many_matches_single(engine):
    """the batched bootstrap is the single-ciphertext bootstrap word for word, for every item of the batch (4
    items: the linear transforms' MAC then takes 4 instances per workgroup, 2 at the two-input level)"""
    be, sk = engine
    boot, ins = be.boots["state"]
    keys = be.boot_keys["state"]
    rng = np.random.default_rng(33)
    B = 4
    cts = [be.at_scale(be.encrypt(sk, rng.uniform(-1, 1, SLOTS), 3, seed=bytes([b]) * 32), 1, ins) for b in range(B)]
    batch = be._new(B, 1, ins)
    for b in range(B):
        be.ctx.eval_lincomb(1, [cts[b].ptr()], [1], [1.0], None, ins, 0.0, 1, True, batch.ptr(b))
    out = be._new(B, be.top_level, be.S(be.top_level))
    boot.run_many(batch.ptr(), B, be.relin, be.conj_key, keys, out.ptr())
    words = out.buf.download((B, 2, be.top_level, N))
    for b in range(B):
        one = be._new(1, be.top_level, be.S(be.top_level))
        boot.run(cts[b].ptr(), be.relin, be.conj_key, keys, one.ptr())
        assert np.array_equal(one.buf.download((2, be.top_level, N)), words[b]), b


@pytest.mark.timeout(900)
def test_decode_step_one_layer(engine, DS, M):
    """one layer, two tokens with the state carried: decrypted output against the float64 model"""
    from oracle import rwkv_ref as ref
    be, sk = engine
    W = M.make_weights(5, n_layers=1)
    step = DS.DecodeStep(be, W)
    st = ref.init_state(32, 1)
    for s in range(2):
        x = M.embed_tokens(np.arange(32) + 100 * s)
        out = step(be.encrypt(sk, M.pack_lanes(x), be.top_level, seed=bytes([s]) * 32))
        xo, _ = ref.step(x, st, W)
        got = M.unpack_lanes(be.decrypt(sk, out).real)
        err = np.sqrt(np.mean((got - xo) ** 2)) / np.sqrt(np.mean(xo ** 2))
        print(f"token {s}: relErrRms {err:.3e}, bootstraps so far {step.stats['bootstraps']}")
        assert err < 1e-3, err


@pytest.mark.timeout(900)
def test_native_decoder_matches_python_plan(engine, DS, M):
    """the C++ driver (libfhe_ssm_decode.so) issues the same engine calls as the Python plan: two layers (the second
    with the value residual toward the first's value), two tokens with the state carried, output ciphertexts equal
    word for word, same level, scale and bootstrap count"""
    ND = load_module("native_decode")
    be, sk = engine
    W = M.make_weights(5, n_layers=2)
    py = DS.DecodeStep(be, W)
    nat = ND.from_backend(be, 2)
    nat.set_weights(W)
    for s in range(2):
        x = M.embed_tokens(np.arange(32) + 100 * s)
        ct = be.encrypt(sk, M.pack_lanes(x), be.top_level, seed=bytes([7, s]) * 16)
        want = py(ct)
        out, lv, sc = nat.step(ct.ptr(), ct.level, ct.scale)
        assert (lv, sc) == (want.level, want.scale), (lv, sc, want.level, want.scale)
        got = out.download((2, lv, N))
        assert np.array_equal(got, want.buf.download((2, lv, N))), s
        print(f"token {s}: native == python plan at level {lv}")
    assert nat.bootstraps == py.stats["bootstraps"] == 2 * 2 * 28
    nat.close()


@pytest.mark.timeout(900)
def test_native_decoder_store_file(engine, M, tmp_path):
    """the matvec coefficients a decoder encoded, saved to a store file and loaded by a fresh decoder with the same
    weights: its first step (no matvec encoded) gives the first decoder's output word for word; a decoder with other
    weights refuses the file (its stamp names them)"""
    ND = load_module("native_decode")
    be, sk = engine
    W = M.make_weights(5, n_layers=1)
    x = be.encrypt(sk, M.pack_lanes(M.embed_tokens(np.arange(32) + 3)), be.top_level, seed=bytes([9, 1]) * 16)
    a = ND.from_backend(be, 1)
    a.set_weights(W)
    out_a, lv, sc = a.step(x.ptr(), x.level, x.scale)
    path = str(tmp_path / "matvec.store")
    n = a.store_save(path)
    assert n >= 4  # the layer's tm, wo, ck, cv
    assert ND.store_read_stamp(path).startswith("fhe-ssm-amd-matvec-coeffs-v1|ring=65536|dpad=1024")
    b = ND.from_backend(be, 1)
    b.set_weights(W)
    assert b.store_load(path) == n
    out_b, lv_b, sc_b = b.step(x.ptr(), x.level, x.scale)
    assert (lv_b, sc_b) == (lv, sc)
    assert np.array_equal(out_b.download((2, lv, N)), out_a.download((2, lv, N)))
    c = ND.from_backend(be, 1)
    c.set_weights(M.make_weights(6, n_layers=1))
    with pytest.raises(RuntimeError, match="different configuration"):
        c.store_load(path)
    for d in (a, b, c):
        d.close()


@pytest.mark.timeout(900)
def test_native_decoder_serves_a_directory(engine, M, tmp_path):
    """the serve-directory protocol with the decode step as its handler (one layer): a stateful session -- two
    tokens with the reset marker, a two-token request whose second file is bad (it fails after one step; the carried
    state must be the one from before it), one more token, then a reset request -- and a request in another layout;
    every response file equals the direct steps' output word for word (cold start, carried state, reset)"""
    import os
    import threading
    ND = load_module("native_decode")
    SC = load_module("serve_client")
    be, sk = engine
    W = M.make_weights(5, n_layers=1)
    nat = ND.from_backend(be, 1)
    nat.set_weights(W)
    top = be.top_level
    xs = [be.encrypt(sk, M.pack_lanes(M.embed_tokens(np.arange(32) + 100 * s)), top, seed=bytes([8, s]) * 16)
          for s in range(3)]
    d = str(tmp_path)
    box = {}
    log = open(os.path.join(d, "server.jsonl"), "w")

    def run():
        box["rep"] = nat.serve(d, timeout_sec=600, stateful=True, log_fd=log.fileno(), poll_ms=20)
    th = threading.Thread(target=run, daemon=True)
    th.start()

    def writer(cts):
        return lambda t, path: be.ctx.ct_save(path, cts[t].ptr(), cts[t].level, cts[t].scale)
    def half_bad(t, path):
        # token 0 is good (a whole step runs on it), token 1 is not a ciphertext file: the request fails part way
        if t == 0:
            return writer(xs[2:])(0, path)
        with open(path, "wb") as f:
            f.write(b"not a ciphertext")
    SC.submit(d, 0, writer(xs[:2]), 2, SC.request_meta(2, 32, top), reset=True)
    r0 = SC.wait(d, 0, timeout=600, alive=th.is_alive)
    SC.submit(d, 1, half_bad, 2, SC.request_meta(2, 32, top))
    with pytest.raises(SC.ServeError):
        SC.wait(d, 1, timeout=600, alive=th.is_alive)
    # the failed request left the carried state as request 0 did: request 2 continues from there
    SC.submit(d, 2, writer(xs[2:]), 1, SC.request_meta(1, 32, top))
    r1 = SC.wait(d, 2, timeout=600, alive=th.is_alive)
    SC.submit(d, 3, writer(xs[2:]), 1, SC.request_meta(1, 32, top), reset=True)
    r2 = SC.wait(d, 3, timeout=600, alive=th.is_alive)
    SC.submit(d, 4, writer(xs[:1]), 1, SC.request_meta(1, 32, top, pack_tokens=2))
    with pytest.raises(SC.ServeError):
        SC.wait(d, 4, timeout=600, alive=th.is_alive)
    SC.stop(d)
    th.join(timeout=120)
    log.close()
    assert not th.is_alive()
    assert box["rep"] == {"served": 5, "failed": 2, "next_req": 5, "exit_reason": "stop"}, box
    # the same tokens as direct steps
    want = []
    nat.reset()
    for s in range(3):
        o, lv, sc = nat.step(xs[s].ptr(), top, xs[s].scale)
        want.append((o.download((2, lv, N)), lv, sc))
    nat.reset()
    o, lv, sc = nat.step(xs[2].ptr(), top, xs[2].scale)
    want.append((o.download((2, lv, N)), lv, sc))
    ckks = load_ckks()
    for (prefix, t), (w, lv, sc) in zip([(r0, 0), (r0, 1), (r1, 0), (r2, 0)], want):
        path = f"{prefix}.{t}"
        assert ckks.ct_file_info(path) == {"N": N, "level": lv, "scale": sc}
        buf = ckks.DeviceBuffer(2 * lv * N * 8)
        assert be.ctx.ct_load(path, buf.ptr, lv) == (lv, sc)
        assert np.array_equal(buf.download((2, lv, N)), w), path
    m0 = SC.response_meta(d, 0)
    assert (m0["count"], m0["tokensReal"], m0["lanes"], m0["level"], m0["ringDim"]) == (2, 2, 32, want[0][1], N)
    print(f"served 4 requests; responses == direct steps at level {want[0][1]}")
    nat.close()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("driver", ["python", "native"])
def test_decode_step_full_config5(engine, DS, M, driver):
    """the full config-5 step: 12 layers, two tokens (cold start, then the carried state); decrypted output
    and the client's vocabulary logits against the float64 model, relErrRms <= 1e-3 -- through the Python plan and
    through the C++ driver that bench.py times (libfhe_ssm_decode.so)"""
    from oracle import rwkv_ref as ref
    be, sk = engine
    W = M.make_weights(9, n_layers=12)
    if driver == "native":
        nat = load_module("native_decode").from_backend(be, 12)
        nat.set_weights(W)

        def step(ct):
            out, lv, sc = nat.step(ct.ptr(), ct.level, ct.scale)
            return DS.HECt(out, 1, lv, sc)
        n_boot = lambda: nat.bootstraps
    else:
        step = DS.DecodeStep(be, W)
        n_boot = lambda: step.stats["bootstraps"]
    st = ref.init_state(32, 12)
    head = M.head_matrix(W, rows=4096)
    for s in range(2):
        x = M.embed_tokens(np.arange(32) * 3 + 1000 * s)
        out = step(be.encrypt(sk, M.pack_lanes(x), be.top_level, seed=bytes([9, s]) * 16))
        xo, _ = ref.step(x, st, W)
        got = M.unpack_lanes(be.decrypt(sk, out).real)
        err = np.sqrt(np.mean((got - xo) ** 2)) / np.sqrt(np.mean(xo ** 2))
        lg, lg_ref = got @ head.T, xo @ head.T
        lerr = np.sqrt(np.mean((lg - lg_ref) ** 2)) / np.sqrt(np.mean(lg_ref ** 2))
        print(f"{driver} token {s}: relErrRms {err:.3e}, logits (4096-row slice) {lerr:.3e}")
        assert err < 1e-3 and lerr < 1e-3, (err, lerr)
    assert n_boot() == 2 * 12 * 28
    if driver == "native":
        nat.close()
