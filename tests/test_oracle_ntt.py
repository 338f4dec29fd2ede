"""Pins for the oracle NTT/INTT (OpenFHE order, hpc_gpu_port/periodic_encode.hpp:150-160,240-260).

Closed form: A[k] = sum_j a_j psi^((2*brev(k)+1)*j) mod q (bit-reversed output), brute force
O(N^2) at small N; inverse = identity; NTT(a)*NTT(b) = NTT(a (x) b) for the negacyclic product,
checked against a schoolbook product in Python integers.
"""
import numpy as np
import pytest


def brev(v, bits):
    return int(format(v, f"0{bits}b")[::-1], 2) if bits else 0


def mk_ctx(oracle, logN, nq=2, bits=30):
    qs = oracle.gen_primes(bits, nq, 2 << logN)
    return oracle.Ctx(logN, qs, nq, 0, 1), qs


@pytest.mark.parametrize("logN", [4, 6, 8])
def test_ntt_closed_form(oracle, logN):
    ctx, qs = mk_ctx(oracle, logN)
    N = 1 << logN
    rng = np.random.default_rng(logN)
    for pi, q in enumerate(qs):
        a = [int(x) for x in rng.integers(0, q, N, dtype=np.uint64)]
        got = ctx.ntt_fwd(np.array([a], dtype=np.uint64), [pi])[0]
        psi = ctx.psi[pi]
        assert pow(psi, N, q) == q - 1
        for k in range(N):
            e = 2 * brev(k, logN) + 1
            want = sum(a[j] * pow(psi, e * j, q) for j in range(N)) % q
            assert int(got[k]) == want


def test_ntt_tables_follow_openfhe_layout(oracle):
    ctx, qs = mk_ctx(oracle, 6)
    t, tp, it, itp = ctx.tables(0)
    q, psi = qs[0], ctx.psi[0]
    for i in range(64):
        assert int(t[brev(i, 6)]) == pow(psi, i, q)
        assert int(it[brev(i, 6)]) == pow(psi, -i, q)
        assert int(tp[i]) == (int(t[i]) << 64) // q


def negacyclic(a, b, q):
    N = len(a)
    c = [0] * N
    for i in range(N):
        if a[i] == 0:
            continue
        for j in range(N):
            k = i + j
            if k < N:
                c[k] += a[i] * b[j]
            else:
                c[k - N] -= a[i] * b[j]
    return [x % q for x in c]


@pytest.mark.parametrize("logN,bits", [(6, 54), (9, 60), (10, 54)])
def test_ntt_convolution_theorem(oracle, logN, bits):
    ctx, qs = mk_ctx(oracle, logN, nq=1, bits=bits)
    q, N = qs[0], 1 << logN
    rng = np.random.default_rng(7)
    a = rng.integers(0, q, N, dtype=np.uint64)
    b = rng.integers(0, q, N, dtype=np.uint64)
    A = ctx.ntt_fwd(a[None], [0])[0]
    B = ctx.ntt_fwd(b[None], [0])[0]
    C = np.array([(int(x) * int(y)) % q for x, y in zip(A, B)], dtype=np.uint64)
    c = ctx.ntt_inv(C[None], [0])[0]
    assert [int(x) for x in c] == negacyclic([int(x) for x in a], [int(x) for x in b], q)


def test_ntt_roundtrip_full_size(oracle):
    """N = 2^16, the BASELINE ring, 54-bit and 60-bit primes; also linearity."""
    qs = oracle.gen_primes(54, 2, 2**17) + oracle.gen_primes(60, 1, 2**17)
    ctx = oracle.Ctx(16, qs, 2, 1, 1)
    rng = np.random.default_rng(3)
    x = np.stack([rng.integers(0, q, 1 << 16, dtype=np.uint64) for q in qs])
    y = np.stack([rng.integers(0, q, 1 << 16, dtype=np.uint64) for q in qs])
    X = ctx.ntt_fwd(x, [0, 1, 2])
    assert not np.array_equal(X, x)
    assert np.array_equal(ctx.ntt_inv(X, [0, 1, 2]), x)
    Y = ctx.ntt_fwd(y, [0, 1, 2])
    qv = np.array(qs, dtype=object)[:, None]
    S = ((x.astype(object) + y.astype(object)) % qv).astype(np.uint64)
    assert np.array_equal(ctx.ntt_fwd(S, [0, 1, 2]), ((X.astype(object) + Y.astype(object)) % qv).astype(np.uint64))
    # delta function: NTT(X^1) at slot k = psi^(2 brev(k) + 1)
    d = np.zeros((1, 1 << 16), dtype=np.uint64)
    d[0, 1] = 1
    D = ctx.ntt_fwd(d, [2])[0]
    for k in (0, 1, 12345, 65535):
        assert int(D[k]) == pow(ctx.psi[2], 2 * brev(k, 16) + 1, qs[2])
