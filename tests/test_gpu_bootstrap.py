"""Full-slot CKKS bootstrapping on the GPU, through the C ABI.

Chain: q0 60-bit, 22 x 50-bit scaling primes, 3 x 60-bit CoeffToSlot primes on top, 8 x 60-bit special
primes, dnum 3; secret ternary with Hamming weight 192; input a level-1 ciphertext (the q0 limb only) of
uniform slots in [-1, 1] at scale 2^55 (the reference's FirstModSize = ScalingModSize + 5 rule,
gpu_real_model.cu:1153-1154).

Config 4 as stated: EvalMod = Chebyshev degree 59 + 2 double-angle steps.  The level-1 input is switched to a sparse
h' = 32 secret before ModRaise and back to the h = 192 secret at the top level (sparse-secret encapsulation), so the
raised message is m + q0 I with I the rounded sum of 33 uniforms on [-1/2, 1/2] per coefficient: K = 14, with a
Chernoff failure bound of 1.2e-15 per bootstrap (tests/test_boot_params.py).  The labelled variant keeps the dense
secret throughout: I is a sum of 193 uniforms, K = 32 (bound 1.9e-9), 3 double-angle steps.  Precision is
-log2 max|error| over all 32768 slots; the bar written here is 14 bits.
"""
import numpy as np
import pytest

from engine_loader import load_ckks, load_module

pytestmark = pytest.mark.gpu

N = 1 << 16
SLOTS = N // 2


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


def _exact(ctx):
    ctx.set_moddown_exact(True)
    return ctx


def _config4_ctx(ckks):
    big = ckks.gen_primes(60, 12)
    return ckks.Context(num_q=26, num_p=8, dnum=3, scale=2.0**50,
                        moduli=big[:1] + ckks.gen_primes(50, 22) + big[1:4] + big[4:])


# (context factory, K, Chebyshev degree, double angles, top scale, input scale, sparse Hamming weight or 0)
CHAINS = {
    "config4": (_config4_ctx, 14.0, 59, 2, 2.0**55, 2.0**55, 32),
    "config4_dense_r3": (_config4_ctx, 32.0, 59, 3, 2.0**55, 2.0**55, 0),
    "config5": (lambda ckks: _exact(ckks.Context(num_q=32, num_p=7, dnum=4, scale=2.0**40,
                                                 moduli=load_module("decode_step").config5_moduli(ckks))),
                32.0, 59, 3, 2.0**52, 2.0**48, 0),
}


@pytest.fixture(scope="module", params=sorted(CHAINS))
def chain(request, ckks):
    make, K, deg, r, top, ins, hs = CHAINS[request.param]
    return make(ckks), K, deg, r, top, ins, hs


class BootKeys:
    """relinearization, conjugation and rotation keys of a plan under sk, and (hs > 0) the sparse-secret
    encapsulation keys sk -> sparse (on q0 and P only) and back, set on the plan"""

    def __init__(self, ckks, ctx, bt, sk, tag: int, hs: int = 0):
        L, K, D = ctx.L, ctx.K, ctx.dnum
        kb = D * 2 * (L + K) * N * 8
        self.relin = ckks.DeviceBuffer(kb)
        ctx.keygen_relin(sk, b"r" * 32, b"s" * 32, self.relin.ptr)
        self.conj = ckks.DeviceBuffer(kb)
        ctx.keygen_automorphism(sk, 2 * N - 1, b"c" * 32, b"d" * 32, self.conj.ptr)
        self.keys, self.bufs = {}, []
        for i, s in enumerate(bt.steps):
            b = ckks.DeviceBuffer(kb)
            ctx.keygen_automorphism(sk, ckks.rotation_index(s), bytes([tag, i % 256]) * 16,
                                    bytes([tag + 1, i % 256]) * 16, b.ptr)
            self.keys[s] = b.ptr
            self.bufs.append(b)
        self.sparse = None
        if hs:
            self.sparse = ctx.secret(bytes([tag + 2]) * 32, hs)
            self.to_sparse = ckks.DeviceBuffer(kb)
            ctx.keygen_switch(sk, self.sparse, b"t" * 32, b"u" * 32, self.to_sparse.ptr, q_limbs=1)
            self.from_sparse = ckks.DeviceBuffer(kb)
            ctx.keygen_switch(self.sparse, sk, b"v" * 32, b"w" * 32, self.from_sparse.ptr)
            bt.set_sparse_keys(self.to_sparse.ptr, self.from_sparse.ptr)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("form", ["config4", "config4_dense_r3"])
def test_bootstrap_config4_precision(ckks, form):
    """config 4 as stated (sparse-secret encapsulation, K = 14, 2 double angles) and the dense 3-double-angle
    variant: the bootstrapped ciphertext decrypts to the level-1 input's slots to 14 bits or better"""
    make, Kr, deg, r, top, ins, hs = CHAINS[form]
    ctx = make(ckks)
    L = ctx.L
    bt = ckks.Bootstrap(ctx, K=Kr, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins)
    # CoeffToSlot 3 levels, Chebyshev 59 (6 levels + the scaling), r double angles, SlotToCoeff 3 levels
    assert bt.out_level == L - 13 - r, bt.out_level
    sk = ctx.secret(b"B" * 32, 192)
    bk = BootKeys(ckks, ctx, bt, sk, 5, hs)
    rng = np.random.default_rng(44)
    z = rng.uniform(-1.0, 1.0, SLOTS)
    pt = ckks.DeviceBuffer(1 * N * 8)
    ct = ckks.DeviceBuffer(2 * 1 * N * 8)
    ctx.encode(z, 1, ins, pt.ptr)
    ctx.encrypt(sk, pt.ptr, 1, b"e" * 32, 0, ct.ptr)
    # the level-1 input decrypts to z
    assert np.max(np.abs(ctx.decrypt(sk, ct.ptr, 1, ins) - z)) < 1e-9
    out = ckks.DeviceBuffer(2 * bt.out_level * N * 8)
    bt.run(ct.ptr, bk.relin.ptr, bk.conj.ptr, bk.keys, out.ptr)
    got = ctx.decrypt(sk, out.ptr, bt.out_level, bt.scale(bt.out_level), SLOTS, complex_out=True)
    err = np.abs(got - z)
    bits = -np.log2(err.max())
    print(f"{form} bootstrap precision: {bits:.2f} bits (max err {err.max():.3e}, mean {err.mean():.3e}), "
          f"output level {bt.out_level}")
    assert bits > 14.0, bits


def _bitrev(n):
    b = n.bit_length() - 1
    r = np.zeros(n, dtype=np.int64)
    for i in range(n):
        r[i] = int(format(i, f"0{b}b")[::-1], 2)
    return r


@pytest.mark.timeout(900)
def test_bootstrap_stagewise(ckks, oracle, chain):
    """Each stage against its mathematical expectation, computed from the secret and the input words:
    ModRaise decrypts to m + q0 I exactly; CoeffToSlot (its last level split into real and imaginary parts,
    stage 2 their recombination Re + i Im) to the bit-reversed coefficients (m'_k + i m'_{k+n})/(q0 K);
    stage 3 to their real and imaginary parts; EvalMod to sin(2 pi K t); the recombination to their sum.
    With sparse-secret encapsulation, m' is formed from the level-1 ciphertext switched to the sparse secret
    (the same key switch the bootstrap runs, through ckks_keyswitch) and the sparse secret's coefficients, and
    |I| must stay within K."""
    ctx, Kr, deg, r, top, ins, hs = chain
    L = ctx.L
    bt = ckks.Bootstrap(ctx, K=Kr, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins)
    sk = ctx.secret(b"T" * 32, 192)
    bk = BootKeys(ckks, ctx, bt, sk, 7, hs)
    rng = np.random.default_rng(45)
    z = rng.uniform(-1.0, 1.0, SLOTS)
    pt = ckks.DeviceBuffer(N * 8)
    ct = ckks.DeviceBuffer(2 * N * 8)
    ctx.encode(z, 1, ins, pt.ptr)
    ctx.encrypt(sk, pt.ptr, 1, b"f" * 32, 0, ct.ptr)
    q0 = ctx.moduli[0]
    octx = oracle.Ctx(16, [q0], 1, 0, 1)
    cw = ct.download((2, 1, N))
    s_raise = sk
    if hs:
        ks = ckks.DeviceBuffer(2 * N * 8)
        ctx.keyswitch(ct.ptr + N * 8, 1, 1, bk.to_sparse.ptr, ks.ptr)
        kw = ks.download((2, 1, N))
        cw = np.stack([(cw[0].astype(object) + kw[0].astype(object)) % q0, kw[1].astype(object)]).astype(np.uint64)
        s_raise = bk.sparse
    c = octx.ntt_inv(cw[:, 0:1, :].reshape(2, 1, N), [0]).reshape(2, N).astype(object)
    c = np.where(c > q0 // 2, c - q0, c)
    s = s_raise.coeffs().astype(np.int64)
    assert int(np.count_nonzero(s)) == (hs or 192)
    conv = np.zeros(N, dtype=object)
    for j in np.nonzero(s)[0]:
        sh = np.concatenate([-c[1][N - j:], c[1][:N - j]]) if j else c[1].copy()
        conv += int(s[j]) * sh
    mp = c[0] + conv  # m' = [c0] + [c1] s over the integers
    m = np.array([int(x) % q0 for x in mp], dtype=object)
    m = np.where(m > q0 // 2, m - q0, m)
    I = (mp - m) // q0
    max_i = max(abs(int(x)) for x in I)
    print("max |I| =", max_i)
    assert max_i <= Kr - 1
    out = ckks.DeviceBuffer(2 * 2 * L * N * 8)
    keys = (bk.relin.ptr, bk.conj.ptr, bk.keys)
    # stage 1: ModRaise
    lvl = bt.run_stage(ct.ptr, *keys, 1, out.ptr)
    assert lvl == L
    dec = ctx.decrypt_coeffs(sk, out.ptr, lvl)
    mpf = mp.astype(np.float64)
    e1 = np.max(np.abs(dec - mpf)) / np.max(np.abs(mpf))
    print("stage 1 rel err", e1)
    assert e1 < 1e-12
    # expected slot vectors
    n = SLOTS
    wprime = (mpf[:n] + 1j * mpf[n:]) / (q0 * Kr)
    v = wprime[_bitrev(n)]
    stages = {2: [v], 3: [v.real, v.imag], 4: [np.sin(2 * np.pi * Kr * v.real), np.sin(2 * np.pi * Kr * v.imag)]}
    stages[5] = [stages[4][0] + 1j * stages[4][1]]
    for st_ in (2, 3, 4, 5):
        lvl = bt.run_stage(ct.ptr, *keys, st_, out.ptr)
        for b, want in enumerate(stages[st_]):
            got = ctx.decrypt(sk, out.ptr + b * 2 * lvl * N * 8, lvl, bt.scale(lvl), SLOTS, complex_out=True)
            err = np.max(np.abs(got - want))
            print(f"stage {st_} part {b} level {lvl}: max err {err:.3e} (max |want| {np.max(np.abs(want)):.3e})")
            assert err < 1e-3 * max(1.0, np.max(np.abs(want))), (st_, b, err)


@pytest.mark.timeout(900)
def test_shared_plan_matches_a_plan_of_its_own(ckks):
    """a plan sharing another's diagonals (ckks_bootstrap_setup_shared, input scale 8x smaller: EvalMod's output
    times 8 before SlotToCoeff) bootstraps to the same message as a plan built for that input scale, to their own
    precision; destroying the base plan first leaves the shared one working"""
    make, K, deg, r, top, ins, _ = CHAINS["config4_dense_r3"]
    ctx = make(ckks)
    base = ckks.Bootstrap(ctx, K=K, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins * 8)
    shared = ckks.Bootstrap(ctx, in_scale=ins, share=base)
    own = ckks.Bootstrap(ctx, K=K, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins)
    assert shared.steps == own.steps and shared.out_level == own.out_level
    with pytest.raises(ckks.CkksError):
        ckks.Bootstrap(ctx, in_scale=ins * 3, share=shared)   # 8 ins / (3 ins) is not an integer
    sk = ctx.secret(b"Q" * 32, 192)
    bk = BootKeys(ckks, ctx, own, sk, 9)
    rng = np.random.default_rng(46)
    z = rng.uniform(-1.0, 1.0, SLOTS)
    pt = ckks.DeviceBuffer(N * 8)
    ct = ckks.DeviceBuffer(2 * N * 8)
    ctx.encode(z, 1, ins, pt.ptr)
    ctx.encrypt(sk, pt.ptr, 1, b"g" * 32, 0, ct.ptr)
    base.close()
    outs = {}
    for name, bt in (("shared", shared), ("own", own)):
        out = ckks.DeviceBuffer(2 * bt.out_level * N * 8)
        bt.run(ct.ptr, bk.relin.ptr, bk.conj.ptr, bk.keys, out.ptr)
        outs[name] = ctx.decrypt(sk, out.ptr, bt.out_level, bt.scale(bt.out_level), SLOTS, complex_out=True)
        bits = -np.log2(np.max(np.abs(outs[name] - z)))
        print(f"{name} plan: {bits:.2f} bits")
        assert bits > 14.0, (name, bits)


@pytest.mark.timeout(900)
def test_bootstrap_words_equal_across_ntt_modes(ckks):
    """The two-pass NTT's fused combines (a scalar combination formed inside its rescale's combine, the Chebyshev
    doubling 2 T^2 - 1 applied by the relinearization's ModDown combine, the key-switch combines) against the fused-NTT
    mode, which runs each of those steps as a kernel of its own (lincomb then rescale, ModDown then an integer
    lincomb): a config-4 bootstrap and a five-term scalar combination come out word for word equal"""
    make, Kr, deg, r, top, ins, hs = CHAINS["config4"]
    ctx = make(ckks)
    bt = ckks.Bootstrap(ctx, K=Kr, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins)
    sk = ctx.secret(b"M" * 32, 192)
    bk = BootKeys(ckks, ctx, bt, sk, 9, hs)
    rng = np.random.default_rng(47)
    z = rng.uniform(-1.0, 1.0, SLOTS)
    pt = ckks.DeviceBuffer(N * 8)
    ct = ckks.DeviceBuffer(2 * N * 8)
    ctx.encode(z, 1, ins, pt.ptr)
    ctx.encrypt(sk, pt.ptr, 1, b"g" * 32, 0, ct.ptr)
    B, lt = 2, 17
    terms = []
    for lv in (20, 21, 22, 23, 24):
        t = ckks.DeviceBuffer(B * 2 * lv * N * 8)
        q = np.array(ctx.moduli[:lv], dtype=np.uint64)[None, None, :, None]
        t.upload(rng.integers(0, 2**62, (B, 2, lv, N), dtype=np.uint64) % q)
        terms.append((t, lv))
    scales = [ctx.scale * (1 + 0.001 * t) for t in range(5)]
    words = {}
    try:
        for mode in (0, 1):
            ctx.set_ntt_mode(mode)
            out = ckks.DeviceBuffer(2 * bt.out_level * N * 8)
            bt.run(ct.ptr, bk.relin.ptr, bk.conj.ptr, bk.keys, out.ptr)
            lc = ckks.DeviceBuffer(B * 2 * lt * N * 8)
            ctx.eval_lincomb(B, [t.ptr for t, _ in terms], [lv for _, lv in terms], [0.3, -1.7, 2.5, 0.01, -0.6],
                             scales, ctx.scale, 0.25, lt, False, lc.ptr)
            words[mode] = (out.download((2, bt.out_level, N)), lc.download((B, 2, lt, N)))
    finally:
        ctx.set_ntt_mode(0)
    assert np.array_equal(words[0][0], words[1][0])
    assert np.array_equal(words[0][1], words[1][1])
    got = ctx.decrypt(sk, ct.ptr, 1, ins)
    assert np.max(np.abs(got - z)) < 1e-9
