"""Pins for the oracle's scalar layer: primes, roots of unity, ChaCha20, seeded samplers.

Golden data: tests/golden/chain_moduli.json (the reference's n32 / n32a4 chains,
results/estimator-speedrun-port-20261103/chain_moduli.jsonl:1-2) and RFC 8439 known answers.
"""
import json
import os

import numpy as np
import pytest
import sympy

from conftest import GOLDEN


def test_reference_chain_moduli_are_ntt_primes(oracle):
    rows = json.load(open(os.path.join(GOLDEN, "chain_moduli.json")))["rows"]
    assert rows
    for r in rows:
        two_n = 2 * r["n"]
        for q in r["q"] + r["p"]:
            assert oracle.is_prime(q)
            assert (q - 1) % two_n == 0
        # neighbours of the chain: the test must also reject (a one-sided test would pin nothing)
        for q in r["q"][:8]:
            for d in (2, 4, 6, two_n):
                assert oracle.is_prime(q + d) == sympy.isprime(q + d)


def test_is_prime_matches_sympy():
    from oracle import oracle as o
    rng = np.random.default_rng(1)
    xs = [int(x) for x in rng.integers(1, 2**62, size=300, dtype=np.uint64)]
    xs += [2**61 - 1, 2**59 - 55, 3215031751, 3825123056546413051, 318665857834031151167461 % 2**64]
    for x in xs:
        assert o.is_prime(x) == sympy.isprime(x), x


@pytest.mark.parametrize("bits,count,m", [(20, 6, 2**5), (30, 5, 2**11), (54, 4, 2**17), (60, 3, 2**17)])
def test_gen_primes_are_the_largest_below_2_pow_bits(oracle, bits, count, m):
    ps = oracle.gen_primes(bits, count, m)
    assert len(ps) == count
    assert all(p < 2**bits and (p - 1) % m == 0 and sympy.isprime(p) for p in ps)
    assert ps == sorted(ps, reverse=True)
    # no NTT prime was skipped: every candidate 1 mod m between consecutive outputs is composite
    top = 2**bits - (2**bits % m) + 1
    if top >= 2**bits:
        top -= m
    cands = range(top, ps[-1] - 1, -m)
    assert [c for c in cands if sympy.isprime(c)] == ps


def test_gen_primes_exclude(oracle):
    a = oracle.gen_primes(54, 3, 2**17)
    b = oracle.gen_primes(54, 2, 2**17, exclude=a[:1])
    assert b == a[1:3]


@pytest.mark.parametrize("q,m", [(257, 16), (7681, 512), (12289, 2048), (65537, 256)])
def test_min_root_is_minimal_primitive_root(oracle, q, m):
    brute = [x for x in range(2, q) if pow(x, m // 2, q) == q - 1]
    assert oracle.min_root(q, m) == min(brute)


# RFC 8439 section 2.3.2: key 00..1f, nonce 000000090000004a00000000, counter 1
RFC_232_OUT = bytes.fromhex(
    "10f1e7e4d13b5915500fdd1fa32071c4c7d1f4c733c068030422aa9ac3d46c4e"
    "d2826446079faa0914c2d705d98b02a2b5129cd1de164eb9cbd083e8a2503c4e")
# RFC 8439 appendix A.1 test vector #1: zero key, zero nonce, counter 0
RFC_A1_OUT = bytes.fromhex(
    "76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"
    "da41597c5157488d7724e03fb8d84a376a43b8f41518a11cc387b669b2ee6586")


def test_chacha20_rfc8439_known_answers(oracle):
    key = np.frombuffer(bytes(range(32)), dtype="<u4")
    nonce = np.frombuffer(bytes.fromhex("000000090000004a00000000"), dtype="<u4")
    out = oracle.chacha20_block(key, 1, nonce)
    assert out.astype("<u4").tobytes() == RFC_232_OUT
    out0 = oracle.chacha20_block(np.zeros(8, np.uint32), 0, np.zeros(3, np.uint32))
    assert out0.astype("<u4").tobytes() == RFC_A1_OUT


def test_seeded_uniform_stream_layout(oracle):
    """seeded_keys.hpp:28-43: key = seed LE words, nonce {digit, limb, SKEY}, blocks -> LE uint64
    words, rejection below 2^64 - (2^64 mod q).  Here q is chosen so rejection actually fires."""
    seed = bytes(range(100, 132))
    q = (1 << 63) + 1  # 2^64 mod q = 2^63 - 1 -> about half the words are rejected
    got = oracle.fill_uniform(seed, 2, 5, oracle.SKEY_TAG, q, 40)
    key = np.frombuffer(seed, dtype="<u4")
    nonce = np.array([2, 5, oracle.SKEY_TAG], dtype=np.uint32)
    words = []
    for ctr in range(64):
        blk = oracle.chacha20_block(key, ctr, nonce).astype("<u4").tobytes()
        words += list(np.frombuffer(blk, dtype="<u8"))
    lim = 2**64 - (2**64 % q)
    acc = [int(w) % q for w in words if int(w) < lim][:40]
    assert [int(x) for x in got] == acc
    assert len([w for w in words[:60] if int(w) >= lim]) > 5


def test_seeded_uniform_is_uniform_and_reproducible(oracle):
    q = oracle.gen_primes(54, 1, 2**17)[0]
    a = oracle.fill_uniform(b"\x07" * 32, 0, 3, oracle.SKEY_TAG, q, 1 << 15)
    b = oracle.fill_uniform(b"\x07" * 32, 0, 3, oracle.SKEY_TAG, q, 1 << 15)
    c = oracle.fill_uniform(b"\x07" * 32, 0, 4, oracle.SKEY_TAG, q, 1 << 15)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert int(a.max()) < q
    mean = float(np.mean(a.astype(np.float64))) / q
    assert abs(mean - 0.5) < 0.01


def test_ternary_secret_weight_and_support(oracle):
    s = oracle.sample_ternary(b"\x01" * 32, 1 << 16, 192)
    assert int(np.count_nonzero(s)) == 192
    assert set(np.unique(s).tolist()) <= {-1, 0, 1}
    assert 60 < int((s == 1).sum()) < 132


def test_gaussian_noise_moments(oracle):
    e = oracle.sample_gauss(b"\x02" * 32, 0, 1 << 16, 3.19)
    sd = float(np.std(e.astype(np.float64)))
    assert abs(sd - np.sqrt(3.19**2 + 1 / 12)) < 0.05
    assert abs(float(np.mean(e))) < 0.05
    assert int(np.abs(e).max()) < 40
