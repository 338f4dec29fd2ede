"""CPU check of the quotient estimate that ends the unreduced forward NTT (ntt.hip reduce_open, constants from
context.cpp make_prime_info): for v < 72 q, k' = hi32(floor(v / 2^s) * M) with s = max(0, bits(q) - 25) and
M = floor(2^(32+s) / q) must be floor(v / q) or one less, so that v - k' q lies in [0, 2q).  Checked at the
multiples of q and their neighbours (where an over-estimate would show first) for primes of 20..55 bits, and
on random v."""
import numpy as np
import pytest

from engine_loader import load_ckks


def estimate(v, q):
    bits = q.bit_length()
    s = max(0, bits - 25)
    M = (1 << (32 + s)) // q
    t = (v >> s) & 0xFFFFFFFF
    assert t == v >> s, "floor(v / 2^s) must fit 32 bits"
    return (t * M) >> 32


@pytest.mark.parametrize("bits", [20, 25, 26, 30, 40, 50, 54, 55])
def test_quotient_estimate_is_floor_or_one_less(bits):
    ckks = load_ckks()
    q = ckks.gen_primes(bits, 1)[0]
    assert q < 1 << 56
    rng = np.random.default_rng(bits)
    vs = []
    for k in range(72):
        vs += [k * q, k * q + 1, k * q + q // 2, k * q + q - 1]
    vs += [int(r) for r in rng.integers(0, 72, 2000)]
    vs = [v if v < 72 * q else v % (72 * q) for v in vs]
    vs += [int(rng.integers(0, 72 * q)) if 72 * q < 2**63 else 0 for _ in range(2000)]
    for v in vs:
        k = v // q
        ke = estimate(v, q)
        assert ke in (k - 1, k), (q, v, k, ke)
        assert 0 <= v - ke * q < 2 * q


def test_estimate_would_fail_without_the_floor_margin():
    """a planted mistake: rounding M up instead of down over-estimates the quotient just below a multiple of q"""
    q = load_ckks().gen_primes(54, 1)[0]
    s = q.bit_length() - 25
    M_up = -(-(1 << (32 + s)) // q)
    bad = [v for k in range(1, 72) for v in (k * q - 1,) if ((v >> s) * M_up) >> 32 > v // q]
    assert bad, "the round-up variant should over-estimate somewhere"
