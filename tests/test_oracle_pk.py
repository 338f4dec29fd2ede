"""Pins for the oracle's public key and public-key encryption (harness/boot_overflow_probe.cpp:22,132-142,
PKEBase::KeyGenInternal: b = ns*e - a*s over the key's basis Q*P, elements {b, a}, ns = 1 for CKKS).

The checks are properties the formulas fix, not a second copy of them: b + a*s is exactly the rounded Gaussian of
the seed (a small polynomial, found by CRT with Python integers); the public key is a secret-key encryption of zero
(b + a*s small over every limb of Q*P); a public-key ciphertext decrypts to its plaintext with an error bounded by
the ModDown rounding (|v e + e0 + e1 s| / P is far below one, so the error is the approximate ModDown's u (< K)
times the secret plus one); a key with the sign of a*s flipped (the mistake a restatement could make) fails that
bound by orders of magnitude.
"""
from functools import reduce

import numpy as np
import pytest


def crt_centered(res, mods):
    M = reduce(lambda a, b: a * b, mods, 1)
    x = 0
    for r, m in zip(res, mods):
        Mi = M // m
        x += int(r) * Mi * pow(Mi, -1, m)
    x %= M
    return x - M if x > M // 2 else x


@pytest.fixture(scope="module")
def small(oracle):
    """logN = 10, L = 5 Q limbs (40-bit), K = 2 P limbs (50-bit), dnum = 3"""
    logN = 10
    qs = oracle.gen_primes(40, 5, 2 << logN)
    ps = oracle.gen_primes(50, 2, 2 << logN, exclude=qs)
    return oracle.Ctx(logN, qs + ps, 5, 2, 3)


def secret(oracle, ctx, h=32):
    s = np.zeros(ctx.N, dtype=np.int8)
    s[:] = oracle_ternary(oracle, ctx.N, h)
    return s, ctx.small_to_eval(s, list(range(ctx.L + ctx.K)))


def oracle_ternary(oracle, N, h):
    rng = np.random.default_rng(3)
    s = np.zeros(N, dtype=np.int8)
    pos = rng.choice(N, h, replace=False)
    s[pos] = rng.choice([-1, 1], h)
    return s


def decrypt_coeffs(ctx, ct, s_eval, l):
    """c0 + c1 s over the first l Q limbs, back to coefficients, centered by CRT (Python integers)"""
    d = np.zeros((l, ctx.N), dtype=np.uint64)
    for i in range(l):
        q = ctx.q[i]
        prod = (ct[1, i].astype(object) * s_eval[i].astype(object)) % q
        d[i] = ((ct[0, i].astype(object) + prod) % q).astype(np.uint64)
    c = ctx.ntt_inv(d[None], list(range(l)))[0]
    return np.array([crt_centered([c[i][k] for i in range(l)], ctx.q[:l]) for k in range(ctx.N)], dtype=object)


def test_public_key_is_an_encryption_of_its_gaussian(oracle, small):
    s, se = secret(oracle, small)
    pk = small.pk_gen(se, b"pk-seed".ljust(32, b"\0"), b"pk-eseed".ljust(32, b"\0"))
    T = small.L + small.K
    # b + a s over every limb of Q*P, back to coefficients: the seed's rounded Gaussian, exactly
    z = np.zeros((T, small.N), dtype=np.uint64)
    for i in range(T):
        q = small.q[i]
        z[i] = ((pk[0, i].astype(object) + (pk[1, i].astype(object) * se[i].astype(object)) % q) % q).astype(np.uint64)
    zc = small.ntt_inv(z[None], list(range(T)))[0]
    e = oracle.sample_gauss2(b"pk-eseed".ljust(32, b"\0"), 0, 0, small.N, 3.19)
    for k in range(0, small.N, 7):
        assert crt_centered([zc[i][k] for i in range(T)], small.q[:T]) == int(e[k])
    assert np.abs(e).max() < 7 * 3.19 and np.abs(e).max() > 0
    # a is uniform over each limb (not a copy of b or of zero)
    assert all(len(np.unique(pk[1, i])) > small.N // 2 for i in range(T))


@pytest.mark.parametrize("l", [5, 3])
def test_public_key_encryption_decrypts(oracle, small, l):
    s, se = secret(oracle, small)
    pk = small.pk_gen(se, b"pk-seed".ljust(32, b"\0"), b"pk-eseed".ljust(32, b"\0"))
    rng = np.random.default_rng(l)
    mc = rng.integers(-2**30, 2**30, small.N)
    m = np.stack([np.array([int(v) % small.q[i] for v in mc], dtype=np.uint64) for i in range(l)])
    m = small.ntt_fwd(m[None], list(range(l)))[0]
    ct = small.pk_encrypt(pk, m, l, b"enc-seed".ljust(32, b"\0"), 7)
    got = decrypt_coeffs(small, ct, se, l)
    err = np.array([int(g) - int(w) for g, w in zip(got, mc)])
    h = int(np.abs(s).sum())
    assert np.abs(err).max() <= small.K * (h + 1) + 1, np.abs(err).max()
    # two encryptions of the same plaintext differ (fresh v, e0, e1 per index) but both decrypt
    ct2 = small.pk_encrypt(pk, m, l, b"enc-seed".ljust(32, b"\0"), 8)
    assert not np.array_equal(ct, ct2)


def test_a_sign_mistake_in_the_key_fails_decryption(oracle, small):
    """planted mistake: b = e + a s instead of e - a s"""
    s, se = secret(oracle, small)
    pk = small.pk_gen(se, b"pk-seed".ljust(32, b"\0"), b"pk-eseed".ljust(32, b"\0"))
    T = small.L + small.K
    bad = pk.copy()
    for i in range(T):
        q = small.q[i]
        two_as = (2 * (pk[1, i].astype(object) * se[i].astype(object))) % q
        bad[0, i] = ((pk[0, i].astype(object) + two_as) % q).astype(np.uint64)
    l = 5
    m = np.zeros((l, small.N), dtype=np.uint64)
    ct = small.pk_encrypt(bad, m, l, b"enc-seed".ljust(32, b"\0"), 1)
    err = decrypt_coeffs(small, ct, se, l)
    assert max(abs(int(x)) for x in err) > 10**6
