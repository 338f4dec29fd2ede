"""Pins the oracle's encoding pieces (oracle/oracle.py: slot_coeffs, round_rule), the checkers of the engine's
encoders in tests/test_gpu_encode.py.

round_rule restates hpc_gpu_port/periodic_encode.hpp:199-225 (OpenFHE CKKSPackedEncoding::Encode): the checks are
hand-computed cases of that rule -- plain llround below 2^61 (halves away from zero), the approxFactor exponent at
and past the 61-bit boundary, the refusal of a too small scaling factor.  slot_coeffs (an independent numpy-FFT
path) is pinned by the definition of the canonical embedding: evaluating its polynomial at the slot points
zeta'^(5^j) by brute force returns scale z_j, and a replicated vector is the same polynomial in X^rep."""
import numpy as np
import pytest

from oracle import oracle as o


def test_round_plain_llround():
    m = np.array([0.0, 2.5, -2.5, 3.49, -3.51, 2.0**60 + 2048.0, -(2.0**61) + 4096.0])
    c, a = o.round_rule(m)
    assert a == 0
    assert c.tolist() == [0, 3, -3, 3, -4, 2**60 + 2048, -(2**61) + 4096]


def test_round_all_zero():
    c, a = o.round_rule(np.zeros(8))
    assert a == 0 and not c.any()


@pytest.mark.parametrize("top,want_a", [(2.0**61, 0), (2.0**61 * (1 + 2.0**-20), 1), (2.0**62, 1),
                                        (2.0**62 * (1 + 2.0**-20), 2), (2.0**70, 9), (-(2.0**75), 14),
                                        (2.0**61 + 2.0**10, 0)])
def test_round_approx_factor(top, want_a):
    """logc = ceil(log2 max |m|) in double precision; 61 bits kept, the rest divided out (and multiplied back mod q
    per limb).  2^61 + 2^10 keeps logc = 61: its double log2 rounds to exactly 61, as in the reference's rule."""
    m = np.array([top, 3.0 * 2.0**40, -7.0])
    c, a = o.round_rule(m)
    assert a == want_a
    assert c[0] == int(top) // 2**a if top > 0 else -(int(-top) // 2**a)
    assert c[1] == round(3 * 2**40 / 2**a)


@pytest.mark.parametrize("vals", [[0.5, -0.25], [1e-3], [0.5]])
def test_round_refuses_too_small_scale(vals):
    with pytest.raises(ValueError):
        o.round_rule(np.array(vals))


def test_round_accepts_just_above_half():
    c, a = o.round_rule(np.array([0.75, 0.1]))
    assert (c.tolist(), a) == ([1, 0], 0)


def test_llround_large_integral():
    v = np.array([2.0**52 + 1, -(2.0**52 + 1), 2.0**53 + 2, 0.5, -0.5, 1.5])
    assert o.llround(v).tolist() == [2**52 + 1, -(2**52 + 1), 2**53 + 2, 1, -1, 2]


@pytest.mark.parametrize("slots", [2, 8, 64])
def test_slot_coeffs_evaluates_to_slots(slots):
    rng = np.random.default_rng(slots)
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    scale = 2.0**20
    m = o.slot_coeffs(z, scale)
    Np = 2 * slots
    for j in range(slots):
        x = np.exp(1j * np.pi * pow(5, j, 2 * Np) / Np)
        val = np.sum(m * x ** np.arange(Np))
        assert abs(val - scale * z[j]) < 1e-6 * scale, j


def test_slot_coeffs_replicated_is_sparse():
    rng = np.random.default_rng(3)
    z = rng.uniform(-1, 1, 16)
    small = o.slot_coeffs(z, 2.0**30)
    big = o.slot_coeffs(np.tile(z, 8), 2.0**30)
    assert np.allclose(big[::8], small, atol=1e-3)
    mask = np.ones(len(big), bool)
    mask[::8] = False
    assert np.max(np.abs(big[mask])) < 1e-3
