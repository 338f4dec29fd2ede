"""The bootstrapping parameters' failure bound, on the CPU.

ModRaise turns the level-1 message m into m + q0 I, I = round(S) per coefficient with S the sum of c0 / q0 and the
192 terms +-c1_j / q0 of c1 s: 193 independent uniforms on [-1/2, 1/2] (c0, c1 uniform mod q0, the secret of Hamming
weight 192).  EvalMod is exact only while |I + m/q0| <= K, so a bootstrap fails when some |S| reaches K - 1/2.  The
Chernoff bound P(S >= t) <= exp(-l t) E[e^(l U)]^193, E[e^(l U)] = sinh(l/2) / (l/2), holds for every l > 0 (the
minimum over a grid is still a bound); times two signs and 2^16 coefficients it bounds the failure rate of one
bootstrap.  bench.py's config-4 K must keep it below 1e-6; the K = 22 of the earlier parameters did not.

With sparse-secret encapsulation (config 4 as stated) the raised ciphertext is the level-1 input switched to a sparse
secret of Hamming weight h', so S is a sum of h' + 1 uniforms: K = 14 at h' = 32.
"""
import math
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def failure_bound(K: float, n_terms: int = 193, n_coeffs: int = 1 << 16) -> float:
    t = K - 0.5
    log_best = 0.0
    for i in range(1, 4000):
        lam = i * 0.005
        log_best = min(log_best, -lam * t + n_terms * math.log(math.sinh(lam / 2) / (lam / 2)))
    return 2 * n_coeffs * math.exp(log_best)


def test_config4_k_fails_less_than_once_per_million_bootstraps():
    sys.path.insert(0, REPO)
    import bench
    sparse = bench.BOOT_FORMS["sparse_r2"]
    assert sparse["sparse_h"] == bench.BOOT_SPARSE_H == 32 and sparse["K"] == bench.BOOT_K
    assert sparse["r"] == 2 and sparse["deg"] == 59           # Chebyshev 59 + 2 double angles
    assert failure_bound(bench.BOOT_K, bench.BOOT_SPARSE_H + 1) < 2e-15
    assert failure_bound(bench.BOOT_K - 2, bench.BOOT_SPARSE_H + 1) > 1e-8   # K = 12 would be marginal
    dense = bench.BOOT_FORMS["dense_r3"]
    assert dense["sparse_h"] == 0
    assert failure_bound(dense["K"]) < 2e-9
    assert failure_bound(22.0) > 1e-2          # the earlier K: a failure every few dozen bootstraps by this bound
    assert failure_bound(bench.BOOT_K) > 0.5   # K = 14 without the encapsulation: certain failure


def test_bound_against_exact_small_case():
    """the same bound for 3 uniforms against the Irwin-Hall tail it must dominate: P(S >= 1) = 1/48"""
    t, n = 1.0, 3
    exact = (1.5 - t) ** 3 / 6          # P(U1 + U2 + U3 >= 1) on [-1/2, 1/2]^3: the corner simplex
    assert abs(exact - 1 / 48) < 1e-15
    best = min(math.exp(-l * t + n * math.log(math.sinh(l / 2) / (l / 2))) for l in [i * 0.01 for i in range(1, 3000)])
    assert exact <= best < 20 * exact
