"""The encoders (ckks_encode, ckks_encode_periodic) at word level, through the C ABI, on the config-5 chain.

- Dense encode vs the oracle: the plaintext is brought back to coefficients with the oracle's inverse NTT (pinned
  bit-exact), every limb must hold the residues of one integer polynomial X (CRT of limbs 0 and 1 checked against
  every other limb), X must be sparse at the stride a replicated vector implies, divisible by 2^log_approx, and
  X / 2^log_approx must be the oracle's round_rule (hpc_gpu_port/periodic_encode.hpp:199-236) of the oracle's
  independent float coefficients (numpy FFT).  The float parts of the two sides differ by rounding only: a
  coefficient whose exact value lies within TOL of a half-integer may round either way, every other must match
  exactly, and none may be off by more than 1.
- Periodic == dense, word for word (the reference's periodic_encode_test.cpp:1-13 check): the compressed plaintext
  expanded by comp[k >> log_rep] equals the dense encoding of the same period, over several periods and levels,
  real and complex, including a vector large enough to need approxFactor.
"""
import numpy as np
import pytest

from engine_loader import load_ckks, load_module

pytestmark = pytest.mark.gpu

N = 1 << 16
SLOTS = N // 2
TOL = 1e-3  # coefficients within TOL of a half-integer may round either way (float paths differ in the last bits)


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


@pytest.fixture(scope="module")
def ctx5(ckks):
    DS = load_module("decode_step")
    return ckks.Context(num_q=32, num_p=7, dnum=4, scale=2.0**40, moduli=DS.config5_moduli(ckks))


@pytest.fixture(scope="module")
def octx5(oracle, ctx5):
    return oracle.Ctx(16, ctx5.moduli, ctx5.L, ctx5.K, ctx5.dnum)


def coefficients(octx, ctx, words, l):
    """eval-form plaintext [l][N] -> the signed integer coefficients X (CRT of limbs 0, 1), checked on every limb"""
    coef = octx.ntt_inv(words, list(range(l)))
    q0, q1 = ctx.moduli[0], ctx.moduli[1]
    Q = q0 * q1
    inv = pow(q0, -1, q1)
    r0 = coef[0].astype(object)
    r1 = coef[1].astype(object)
    X = r0 + q0 * (((r1 - r0) * inv) % q1)
    X = np.where(X > Q // 2, X - Q, X)
    for i in range(2, l):
        assert np.array_equal(coef[i].astype(object), X % ctx.moduli[i]), f"limb {i} is not the same polynomial"
    return X


def check_against_rule(oracle, X, z, scale, rep):
    """X (the engine's integer polynomial) against round_rule(slot_coeffs(z)): exact structure (sparse at the stride,
    a multiple of 2^log_approx with the rule's log_approx), and the rounded values equal except where float noise
    may decide.  The noise bound 2^-54 scale / 2^log_approx covers both float paths (a radix-2 FFT of N terms of
    size ~scale: its outputs carry ~sqrt(log2 N) ulp of scale sqrt(N), divided by N); below 0.05 every coefficient
    farther than max(TOL, noise) from a half-integer must match exactly."""
    m = oracle.slot_coeffs(z, scale)
    want, a = oracle.round_rule(m)
    assert not np.any(X[np.arange(N) % rep != 0]), "not sparse at the replication stride"
    Xs = X[::rep]
    assert all(int(x) % (1 << a) == 0 for x in Xs), "not a multiple of 2^log_approx"
    got = np.array([int(x) >> a for x in Xs], dtype=object)
    diff = (got - want.astype(object)).astype(np.float64)
    noise = 2.0**-54 * scale / 2.0**a
    if noise < 0.05:
        v = m / 2.0**a
        near_half = np.abs(np.abs(v - np.trunc(v)) - 0.5) < max(TOL, noise)
        assert np.all(np.abs(diff) <= 1)
        assert np.all(diff[~near_half] == 0), (np.count_nonzero(diff[~near_half]), a)
    else:
        assert np.all(np.abs(diff) <= noise + 1), (np.max(np.abs(diff)), noise)
    return a


@pytest.mark.parametrize("n_slots,cplx,scale,l", [
    (SLOTS, False, 2.0**40, 6), (SLOTS, True, 2.0**45, 12), (1024, False, 2.0**40, 20), (1024, True, 2.0**40, 3),
    (64, False, 2.0**45, 8), (SLOTS, False, 2.0**70, 4), (1024, True, 2.0**75, 5)])
def test_dense_encode_matches_rule(ckks, oracle, ctx5, octx5, n_slots, cplx, scale, l):
    rng = np.random.default_rng(n_slots + l)
    z = rng.uniform(-1, 1, n_slots) + (1j * rng.uniform(-1, 1, n_slots) if cplx else 0)
    pt = ckks.DeviceBuffer(l * N * 8)
    ctx5.encode(z, l, scale, pt.ptr)
    X = coefficients(octx5, ctx5, pt.download((l, N)), l)
    a = check_against_rule(oracle, X, z, scale, N // (2 * n_slots))
    assert (a > 0) == (scale > 2.0**60), a


@pytest.mark.parametrize("period,cplx,scale,l", [
    (1024, False, 2.0**40, 6), (1024, True, 2.0**40, 21), (2048, False, 2.0**52, 32), (64, True, 2.0**40, 9),
    (2, False, 2.0**40, 4), (1024, False, 2.0**72, 7)])
def test_periodic_equals_dense_word_for_word(ckks, ctx5, period, cplx, scale, l):
    rng = np.random.default_rng(period * 7 + l)
    n_vec = 3
    z = rng.uniform(-1, 1, (n_vec, period)) + (1j * rng.uniform(-1, 1, (n_vec, period)) if cplx else 0)
    Np = 2 * period
    log_rep = (N // Np).bit_length() - 1
    comp = ckks.DeviceBuffer(n_vec * l * Np * 8)
    ctx5.encode_periodic(z, l, scale, comp.ptr)
    c = comp.download((n_vec, l, Np))
    pt = ckks.DeviceBuffer(l * N * 8)
    for n in range(n_vec):
        ctx5.encode(z[n], l, scale, pt.ptr)
        dense = pt.download((l, N))
        expanded = c[n][:, np.arange(N) >> log_rep]
        assert np.array_equal(expanded, dense), (period, l, n)


def test_periodic_matches_rule(ckks, oracle, ctx5, octx5):
    """the small-ring GPU encoder (k_encode_small) on its own against the oracle: expanded, then as above"""
    period, l, scale = 1024, 10, 2.0**40
    rng = np.random.default_rng(77)
    z = rng.uniform(-1, 1, (2, period))
    Np = 2 * period
    log_rep = (N // Np).bit_length() - 1
    comp = ckks.DeviceBuffer(2 * l * Np * 8)
    ctx5.encode_periodic(z, l, scale, comp.ptr)
    c = comp.download((2, l, Np))
    for n in range(2):
        X = coefficients(octx5, ctx5, np.ascontiguousarray(c[n][:, np.arange(N) >> log_rep]), l)
        check_against_rule(oracle, X, z[n], scale, N // Np)


def test_encode_refuses_too_small_scale(ckks, ctx5):
    pt = ckks.DeviceBuffer(4 * N * 8)
    with pytest.raises(ckks.CkksError):
        ctx5.encode(np.full(SLOTS, 1e-3), 4, 1.0, pt.ptr)
    comp = ckks.DeviceBuffer(4 * 2048 * 8)
    with pytest.raises(ckks.CkksError):
        ctx5.encode_periodic(np.full((1, 1024), 1e-3), 4, 1.0, comp.ptr)


@pytest.mark.parametrize("period,scale", [(1024, 2.0**40), (2048, 2.0**52), (1024, 2.0**72)])
def test_coefficient_store_expands_to_the_encoder_words(ckks, ctx5, period, scale):
    """ckks_encode_periodic_coeffs + ckks_expand_periodic (a plaintext store kept as 2 period int64 per vector,
    expanded when applied) == ckks_encode_periodic word for word, at several levels from one coefficient set,
    including a scale that needs approxFactor (2^72)"""
    rng = np.random.default_rng(period + int(np.log2(scale)))
    n_vec = 5
    z = rng.uniform(-1, 1, (n_vec, period))
    Np = 2 * period
    dc = ckks.DeviceBuffer(n_vec * Np * 8)
    dl = ckks.DeviceBuffer(n_vec * 4)
    ctx5.encode_periodic_coeffs(z, scale, dc.ptr, dl.ptr)
    la = dl.download((n_vec,), np.int32)
    assert np.all(la == 0) == (scale < 2.0**60), la
    for l in (3, 17, 32):
        want = ckks.DeviceBuffer(n_vec * l * Np * 8)
        ctx5.encode_periodic(z, l, scale, want.ptr)
        got = ckks.DeviceBuffer(n_vec * l * Np * 8)
        ctx5.expand_periodic(dc.ptr, dl.ptr, n_vec, period, l, got.ptr)
        assert np.array_equal(got.download((n_vec, l, Np)), want.download((n_vec, l, Np))), l
