"""GPU parity of the batched NTT/INTT against the CPU oracle, through the C ABI.

Bar: bit-exact words.  Sizes: oracle-checked batches of a few hundred limbs, plus the full config-1
shape (64 ct x 2 polys x 24 limbs) checked on a seeded sample of limbs and by the size-independent
round trip INTT(NTT(x)) = x over every limb.
"""
import numpy as np
import pytest

from engine_loader import load_ckks

pytestmark = pytest.mark.gpu

L, K = 24, 8


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


@pytest.fixture(scope="module")
def ctx(ckks):
    return ckks.Context(num_q=L, num_p=K, dnum=3, q_bits=54, p_bits=60)


@pytest.fixture(scope="module")
def octx(oracle, ctx):
    return oracle.Ctx(16, ctx.moduli, L, K, 3)


@pytest.fixture
def ntt_mode(ctx, request):
    """sets the context's NTT schedule for one test and restores the default (0, two passes, the one bench.py
    times) afterwards, whatever the test does"""
    ctx.set_ntt_mode(request.param)
    yield request.param
    ctx.set_ntt_mode(0)


def rand_polys(moduli, n_polys, prime_idx, seed):
    rng = np.random.default_rng(seed)
    q = np.array([moduli[i] for i in prime_idx], dtype=np.uint64)
    return (rng.integers(0, 2**63, (n_polys, len(prime_idx), 1 << 16), dtype=np.uint64) % q[None, :, None])


def test_context_matches_oracle_parameters(oracle, ctx, octx):
    q = oracle.gen_primes(54, L, 2**17)
    p = oracle.gen_primes(60, K, 2**17, exclude=q)
    assert ctx.moduli == q + p
    assert ctx.roots == octx.psi


@pytest.mark.parametrize("ntt_mode", [0, 1], indirect=True)
@pytest.mark.parametrize("prime_idx", [list(range(24)), list(range(24, 32)), [3, 31, 0, 17, 24]])
def test_ntt_forward_inverse_bit_exact(ckks, ctx, octx, ntt_mode, prime_idx):
    x = rand_polys(ctx.moduli, 3, prime_idx, seed=len(prime_idx) + ntt_mode)
    buf = ckks.DeviceBuffer.from_array(x)
    ctx.ntt_forward(buf.ptr, 3, prime_idx)
    X = buf.download(x.shape)
    want = octx.ntt_fwd(x, prime_idx)
    assert np.array_equal(X, want)
    ctx.ntt_inverse(buf.ptr, 3, prime_idx)
    assert np.array_equal(buf.download(x.shape), x)
    # inverse on its own vs the oracle inverse of random (bit-reversed-order) data
    y = rand_polys(ctx.moduli, 3, prime_idx, seed=99)
    buf.upload(y)
    ctx.ntt_inverse(buf.ptr, 3, prime_idx)
    assert np.array_equal(buf.download(y.shape), octx.ntt_inv(y, prime_idx))


@pytest.mark.parametrize("ntt_mode", [0, 1], indirect=True)
def test_ntt_edge_values(ckks, ctx, octx, ntt_mode):
    """all-zero, all q-1 and delta limbs (extremes of the lazy-reduction ranges)"""
    pi = [0, 23, 24, 31]
    x = np.zeros((3, 4, 1 << 16), dtype=np.uint64)
    for j, p in enumerate(pi):
        x[1, j, :] = ctx.moduli[p] - 1
        x[2, j, 1] = 1
    buf = ckks.DeviceBuffer.from_array(x)
    ctx.ntt_forward(buf.ptr, 3, pi)
    assert np.array_equal(buf.download(x.shape), octx.ntt_fwd(x, pi))
    ctx.ntt_inverse(buf.ptr, 3, pi)
    assert np.array_equal(buf.download(x.shape), x)


@pytest.mark.parametrize("ntt_mode", [0, 1], indirect=True)
def test_ntt_config1_full_shape(ckks, ctx, octx, ntt_mode):
    """64 ciphertexts x 2 polys x 24 limbs (the shape bench.py times, in both schedules): sampled limbs vs the
    oracle, forward and inverse each on their own, and the round trip on all limbs."""
    n_polys = 128
    prime_idx = list(range(L))
    rng = np.random.default_rng(2024)
    q = np.array(ctx.moduli[:L], dtype=np.uint64)
    x = rng.integers(0, 2**63, (n_polys, L, 1 << 16), dtype=np.uint64) % q[None, :, None]
    buf = ckks.DeviceBuffer.from_array(x)
    ctx.ntt_forward(buf.ptr, n_polys, prime_idx)
    X = buf.download(x.shape)
    for p, l in zip(rng.integers(0, n_polys, 24), rng.permutation(L)):
        assert np.array_equal(X[p, l], octx.ntt_fwd(x[p, l][None], [l])[0]), (p, l)
    assert bool((X < q[None, :, None]).all())
    ctx.ntt_inverse(buf.ptr, n_polys, prime_idx)
    assert np.array_equal(buf.download(x.shape), x)
    # the inverse on its own: random bit-reversed-order input, sampled limbs vs the oracle inverse
    buf.upload(X[::-1].copy())
    ctx.ntt_inverse(buf.ptr, n_polys, prime_idx)
    Y = buf.download(x.shape)
    for p, l in zip(rng.integers(0, n_polys, 24), rng.permutation(L)):
        assert np.array_equal(Y[p, l], octx.ntt_inv(X[n_polys - 1 - p, l][None], [l])[0]), (p, l)


def test_ntt_prime_sizes(ckks, oracle):
    """every prime size the engine meets (20..60 bits): below 2^56 the forward transform takes the unreduced
    butterflies and the final quotient-estimate reduction, from 2^56 the reduced ones; random and edge limbs
    (all q-1, a delta) vs the oracle, and the round trip"""
    moduli = []
    for bits in (20, 30, 40, 50, 54, 55):
        moduli += ckks.gen_primes(bits, 1, moduli)
    p_mod = []
    for bits in (56, 57, 60):
        p_mod += ckks.gen_primes(bits, 1, moduli + p_mod)
    ctx = ckks.Context(num_q=len(moduli), num_p=len(p_mod), dnum=2, moduli=moduli + p_mod)
    allm = moduli + p_mod
    octx = oracle.Ctx(16, allm, len(moduli), len(p_mod), 2)
    pi = list(range(len(allm)))
    x = rand_polys(allm, 3, pi, seed=31)
    for j, p in enumerate(pi):
        x[1, j, :] = allm[p] - 1
        x[2, j, :] = 0
        x[2, j, 1] = 1
    buf = ckks.DeviceBuffer.from_array(x)
    ctx.ntt_forward(buf.ptr, 3, pi)
    assert np.array_equal(buf.download(x.shape), octx.ntt_fwd(x, pi))
    ctx.ntt_inverse(buf.ptr, 3, pi)
    assert np.array_equal(buf.download(x.shape), x)
