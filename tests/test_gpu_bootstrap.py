"""Full-slot CKKS bootstrapping on the GPU, through the C ABI.

Chain: q0 60-bit, 22 x 50-bit scaling primes, 3 x 60-bit CoeffToSlot primes on top, 8 x 60-bit special
primes, dnum 3; secret ternary with Hamming weight 192; input a level-1 ciphertext (the q0 limb only) of
uniform slots in [-1, 1] at scale 2^55 (the reference's FirstModSize = ScalingModSize + 5 rule,
gpu_real_model.cu:1153-1154).  EvalMod: Chebyshev degree 59, 3 double-angle steps, K = 32: the raised message is
m + q0 I with I the rounded sum of 193 uniforms on [-1/2, 1/2] per coefficient, and the Chernoff bound
P(S >= t) <= min_l exp(-l t) (sinh(l/2) / (l/2))^193 at t = 31.5, times 2 x 2^16 coefficients, puts a failure
(|I + m/q0| beyond K) below 1.9e-9 per bootstrap (tests/test_boot_params.py checks the figure on the CPU).  Precision is -log2 max|error| over all 32768 slots; the bar written here is 14 bits.
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


@pytest.fixture(scope="module")
def boot_ctx(ckks):
    big = ckks.gen_primes(60, 12)
    qs = ckks.gen_primes(50, 22)
    return ckks.Context(num_q=26, num_p=8, dnum=3, scale=2.0**50, moduli=big[:1] + qs + big[1:4] + big[4:])


def _exact(ctx):
    ctx.set_moddown_exact(True)
    return ctx


# (context factory, K, Chebyshev degree, double angles, top scale, input scale)
CHAINS = {
    "config4": (lambda ckks: ckks.Context(num_q=26, num_p=8, dnum=3, scale=2.0**50,
                                          moduli=ckks.gen_primes(60, 1) + ckks.gen_primes(50, 22) +
                                          ckks.gen_primes(60, 12)[1:4] + ckks.gen_primes(60, 12)[4:]),
                32.0, 59, 3, 2.0**55, 2.0**55),
    "config5": (lambda ckks: _exact(ckks.Context(num_q=32, num_p=7, dnum=4, scale=2.0**40,
                                                 moduli=load_module("decode_step").config5_moduli(ckks))),
                32.0, 59, 3, 2.0**52, 2.0**48),
}


@pytest.fixture(scope="module", params=sorted(CHAINS))
def chain(request, ckks):
    make, K, deg, r, top, ins = CHAINS[request.param]
    return make(ckks), K, deg, r, top, ins


@pytest.mark.timeout(900)
def test_bootstrap_config4_precision(ckks, boot_ctx):
    ctx = boot_ctx
    L, K, D = ctx.L, ctx.K, ctx.dnum
    bt = ckks.Bootstrap(ctx, K=32.0, cheb_degree=59, double_angles=3, top_scale=2.0**55, in_scale=2.0**55)
    assert bt.out_level == L - 16
    sk = ctx.secret(b"B" * 32, 192)
    kb = D * 2 * (L + K) * N * 8
    relin = ckks.DeviceBuffer(kb)
    ctx.keygen_relin(sk, b"r" * 32, b"s" * 32, relin.ptr)
    conj = ckks.DeviceBuffer(kb)
    ctx.keygen_automorphism(sk, 2 * N - 1, b"c" * 32, b"d" * 32, conj.ptr)
    keys = {}
    bufs = []
    for i, s in enumerate(bt.steps):
        b = ckks.DeviceBuffer(kb)
        ctx.keygen_automorphism(sk, ckks.rotation_index(s), bytes([5, i % 256]) * 16, bytes([6, i % 256]) * 16, b.ptr)
        keys[s] = b.ptr
        bufs.append(b)
    rng = np.random.default_rng(44)
    z = rng.uniform(-1.0, 1.0, SLOTS)
    pt = ckks.DeviceBuffer(1 * N * 8)
    ct = ckks.DeviceBuffer(2 * 1 * N * 8)
    ctx.encode(z, 1, 2.0**55, pt.ptr)
    ctx.encrypt(sk, pt.ptr, 1, b"e" * 32, 0, ct.ptr)
    # the level-1 input decrypts to z
    assert np.max(np.abs(ctx.decrypt(sk, ct.ptr, 1, 2.0**55) - z)) < 1e-9
    out = ckks.DeviceBuffer(2 * bt.out_level * N * 8)
    bt.run(ct.ptr, relin.ptr, conj.ptr, keys, out.ptr)
    got = ctx.decrypt(sk, out.ptr, bt.out_level, bt.scale(bt.out_level), SLOTS, complex_out=True)
    err = np.abs(got - z)
    bits = -np.log2(err.max())
    print(f"bootstrap precision: {bits:.2f} bits (max err {err.max():.3e}, mean {err.mean():.3e})")
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
    stage 3 to their real and imaginary parts; EvalMod to sin(2 pi K t); the recombination to their sum."""
    ctx, Kr, deg, r, top, ins = chain
    L, K, D = ctx.L, ctx.K, ctx.dnum
    bt = ckks.Bootstrap(ctx, K=Kr, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins)
    sk = ctx.secret(b"T" * 32, 192)
    kb = D * 2 * (L + K) * N * 8
    relin = ckks.DeviceBuffer(kb)
    ctx.keygen_relin(sk, b"r" * 32, b"s" * 32, relin.ptr)
    conj = ckks.DeviceBuffer(kb)
    ctx.keygen_automorphism(sk, 2 * N - 1, b"c" * 32, b"d" * 32, conj.ptr)
    keys, bufs = {}, []
    for i, s in enumerate(bt.steps):
        b = ckks.DeviceBuffer(kb)
        ctx.keygen_automorphism(sk, ckks.rotation_index(s), bytes([7, i % 256]) * 16, bytes([8, i % 256]) * 16, b.ptr)
        keys[s] = b.ptr
        bufs.append(b)
    rng = np.random.default_rng(45)
    z = rng.uniform(-1.0, 1.0, SLOTS)
    pt = ckks.DeviceBuffer(N * 8)
    ct = ckks.DeviceBuffer(2 * N * 8)
    ctx.encode(z, 1, ins, pt.ptr)
    ctx.encrypt(sk, pt.ptr, 1, b"f" * 32, 0, ct.ptr)
    q0 = ctx.moduli[0]
    octx = oracle.Ctx(16, [q0], 1, 0, 1)
    cw = ct.download((2, 1, N))
    c = octx.ntt_inv(cw[:, 0:1, :].reshape(2, 1, N), [0]).reshape(2, N).astype(object)
    c = np.where(c > q0 // 2, c - q0, c)
    s = sk.coeffs().astype(np.int64)
    conv = np.zeros(N, dtype=object)
    for j in np.nonzero(s)[0]:
        sh = np.concatenate([-c[1][N - j:], c[1][:N - j]]) if j else c[1].copy()
        conv += int(s[j]) * sh
    mp = c[0] + conv  # m' = [c0] + [c1] s over the integers
    m = np.array([int(x) % q0 for x in mp], dtype=object)
    m = np.where(m > q0 // 2, m - q0, m)
    I = (mp - m) // q0
    print("max |I| =", max(abs(int(x)) for x in I))
    out = ckks.DeviceBuffer(2 * 2 * L * N * 8)
    # stage 1: ModRaise
    lvl = bt.run_stage(ct.ptr, relin.ptr, conj.ptr, keys, 1, out.ptr)
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
        lvl = bt.run_stage(ct.ptr, relin.ptr, conj.ptr, keys, st_, out.ptr)
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
    make, K, deg, r, top, ins = CHAINS["config4"]
    ctx = make(ckks)
    L, Kp, D = ctx.L, ctx.K, ctx.dnum
    base = ckks.Bootstrap(ctx, K=K, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins * 8)
    shared = ckks.Bootstrap(ctx, in_scale=ins, share=base)
    own = ckks.Bootstrap(ctx, K=K, cheb_degree=deg, double_angles=r, top_scale=top, in_scale=ins)
    assert shared.steps == own.steps and shared.out_level == own.out_level
    with pytest.raises(ckks.CkksError):
        ckks.Bootstrap(ctx, in_scale=ins * 3, share=shared)   # 8 ins / (3 ins) is not an integer
    sk = ctx.secret(b"Q" * 32, 192)
    kb = D * 2 * (L + Kp) * N * 8
    relin = ckks.DeviceBuffer(kb)
    ctx.keygen_relin(sk, b"r" * 32, b"s" * 32, relin.ptr)
    conj = ckks.DeviceBuffer(kb)
    ctx.keygen_automorphism(sk, 2 * N - 1, b"c" * 32, b"d" * 32, conj.ptr)
    keys, bufs = {}, []
    for i, s in enumerate(own.steps):
        b = ckks.DeviceBuffer(kb)
        ctx.keygen_automorphism(sk, ckks.rotation_index(s), bytes([9, i % 256]) * 16, bytes([10, i % 256]) * 16, b.ptr)
        keys[s] = b.ptr
        bufs.append(b)
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
        bt.run(ct.ptr, relin.ptr, conj.ptr, keys, out.ptr)
        outs[name] = ctx.decrypt(sk, out.ptr, bt.out_level, bt.scale(bt.out_level), SLOTS, complex_out=True)
        bits = -np.log2(np.max(np.abs(outs[name] - z)))
        print(f"{name} plan: {bits:.2f} bits")
        assert bits > 14.0, (name, bits)
