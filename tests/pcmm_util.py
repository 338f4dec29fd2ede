"""Plaintext side of the BSGS diagonal matrix-vector product, as the reference
builds it (hpc_gpu_port/gpu_real_model.cu:2767-2823; algebra checked in harness/cpu_real_model.cpp:270-318):

  y = sum_g rot_{g*bs}( sum_j d'_{g*bs+j} (.) rot_j(x) ),   d'_k[row + g*bs] = W[row][(row + k) mod d]

The rotation modulus equals the matrix dimension d.  d = 768 does not divide the 32768 slots, so the input
is replicated with period d over all slots (x[i] = u[i mod d]); every slot a product reads,
row + g*bs + j <= 767 + 27*28 + 27, lies before the end of the slot vector, so outputs 0..d-1 are exact.
"""
import numpy as np

SLOTS = 1 << 15


def replicate(u: np.ndarray, slots: int = SLOTS) -> np.ndarray:
    d = len(u)
    return u[np.arange(slots) % d]


def bsgs_diagonals(W: np.ndarray, bs: int, slots: int = SLOTS) -> np.ndarray:
    """[d][slots] pre-rotated diagonals, diagonal k = g*bs + j at row k."""
    d = W.shape[0]
    assert W.shape == (d, d)
    rows = np.arange(d)
    out = np.zeros((d, slots))
    for k in range(d):
        g = k // bs
        out[k, rows + g * bs] = W[rows, (rows + k) % d]
    return out


def steps(d: int, bs: int):
    ng = -(-d // bs)
    return list(range(1, bs)), [g * bs for g in range(1, ng)]
