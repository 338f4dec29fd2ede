"""ctypes + numpy front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker.  The product (the HIP library under fhe-ssm_amd/) never imports it.

Conventions followed (reference file:line) are listed in ckks_oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
MAX_PRIMES = 80
SKEY_TAG = 0x59454B53  # "SKEY" little-endian, seeded_keys.hpp:30-33

_u64p = ctypes.POINTER(ctypes.c_uint64)
_u32p = ctypes.POINTER(ctypes.c_uint32)


class _Ctx(ctypes.Structure):
    _fields_ = [
        ("N", ctypes.c_uint32), ("logN", ctypes.c_uint32),
        ("L", ctypes.c_uint32), ("K", ctypes.c_uint32),
        ("dnum", ctypes.c_uint32), ("alpha", ctypes.c_uint32),
        ("q", ctypes.c_uint64 * MAX_PRIMES),
        ("psi", ctypes.c_uint64 * MAX_PRIMES),
        ("ninv", ctypes.c_uint64 * MAX_PRIMES),
        ("tab", _u64p), ("tabp", _u64p), ("itab", _u64p), ("itabp", _u64p),
        ("moddown_exact", ctypes.c_uint32),
    ]


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.POINTER(_Ctx)
        u64, u32, vp = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p
        sig = {
            "or_mulmod": (u64, [u64, u64, u64]),
            "or_powmod": (u64, [u64, u64, u64]),
            "or_invmod": (u64, [u64, u64]),
            "or_is_prime": (ctypes.c_int, [u64]),
            "or_bitrev": (u32, [u32, u32]),
            "or_gen_primes": (u32, [u32, u32, u64, vp, u32, vp]),
            "or_min_root": (u64, [u64, u64]),
            "or_ctx_init": (ctypes.c_int, [P, u32, vp, u32, u32, u32]),
            "or_ctx_free": (None, [P]),
            "or_ntt_fwd": (None, [P, u32, vp]),
            "or_ntt_inv": (None, [P, u32, vp]),
            "or_ntt_fwd_batch": (None, [P, vp, u32, u32, vp]),
            "or_ntt_inv_batch": (None, [P, vp, u32, u32, vp]),
            "or_bconv": (None, [P, vp, u32, vp, vp, u32, vp]),
            "or_bconv_centered": (None, [P, vp, u32, vp, vp, u32, vp]),
            "or_tensor": (None, [P, vp, vp, u32, vp]),
            "or_num_digits": (u32, [P, u32]),
            "or_modup": (None, [P, vp, u32, vp]),
            "or_ks_inner": (None, [P, vp, u32, vp, vp]),
            "or_moddown": (None, [P, vp, u32, vp]),
            "or_keyswitch": (None, [P, vp, u32, vp, vp]),
            "or_rescale": (None, [P, vp, u32, u32, vp]),
            "or_hmult_relin_rescale": (None, [P, vp, vp, u32, vp, vp]),
            "or_hmult_relin_rescale_batch": (None, [P, vp, vp, u32, u32, vp, vp]),
            "or_set_threads": (None, [ctypes.c_int]),
            "or_max_threads": (ctypes.c_int, []),
            "or_automorph_coef": (None, [P, vp, u32, vp, u32, vp]),
            "or_automorph_eval": (None, [P, vp, u32, u32, vp]),
            "or_rot_index": (u32, [P, ctypes.c_int64]),
            "or_rotate": (None, [P, vp, u32, u32, vp, vp]),
            "or_chacha20_block": (None, [vp, u32, vp, vp]),
            "or_fill_uniform": (None, [vp, u32, u32, u32, u64, vp, ctypes.c_size_t]),
            "or_sample_ternary": (None, [vp, u32, u32, vp]),
            "or_sample_gauss": (None, [vp, u32, u32, ctypes.c_double, vp]),
            "or_small_to_eval_i8": (None, [P, vp, u32, vp, vp]),
            "or_small_to_eval_i32": (None, [P, vp, u32, vp, vp]),
            "or_ksk_gen": (None, [P, vp, vp, vp, vp, ctypes.c_double, vp]),
            "or_sample_gauss2": (None, [vp, u32, u32, u32, ctypes.c_double, vp]),
            "or_pk_gen": (None, [P, vp, vp, vp, ctypes.c_double, vp]),
            "or_pk_encrypt": (None, [P, vp, vp, u32, vp, u32, ctypes.c_double, vp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _u32(xs) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(xs, dtype=np.uint32))


def gen_primes(bits: int, count: int, m: int, exclude=()) -> list[int]:
    out = np.zeros(count, dtype=np.uint64)
    ex = np.ascontiguousarray(np.asarray(list(exclude) or [0], dtype=np.uint64))
    n = lib().or_gen_primes(bits, count, m, _p(ex), len(exclude), _p(out))
    return [int(x) for x in out[:n]]


def is_prime(n: int) -> bool:
    return bool(lib().or_is_prime(n))


def min_root(q: int, m: int) -> int:
    return int(lib().or_min_root(q, m))


def chacha20_block(key_words, counter: int, nonce_words) -> np.ndarray:
    k = _u32(key_words)
    n = _u32(nonce_words)
    out = np.zeros(16, dtype=np.uint32)
    lib().or_chacha20_block(_p(k), counter, _p(n), _p(out))
    return out


def fill_uniform(seed: bytes, w0: int, w1: int, tag: int, q: int, n: int) -> np.ndarray:
    s = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
    out = np.zeros(n, dtype=np.uint64)
    lib().or_fill_uniform(_p(s), w0, w1, tag, q, _p(out), n)
    return out


def sample_ternary(seed: bytes, N: int, h: int) -> np.ndarray:
    s = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
    out = np.zeros(N, dtype=np.int8)
    lib().or_sample_ternary(_p(s), N, h, _p(out))
    return out


def sample_gauss(seed: bytes, stream: int, N: int, sigma: float) -> np.ndarray:
    s = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
    out = np.zeros(N, dtype=np.int32)
    lib().or_sample_gauss(_p(s), stream, N, sigma, _p(out))
    return out


def sample_gauss2(seed: bytes, w0: int, w1: int, N: int, sigma: float) -> np.ndarray:
    s = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
    out = np.zeros(N, dtype=np.int32)
    lib().or_sample_gauss2(_p(s), w0, w1, N, sigma, _p(out))
    return out


class Ctx:
    """Oracle context: moduli = Q chain (L) followed by P (K), dnum digits."""

    def __init__(self, logN: int, moduli, L: int, K: int, dnum: int, moddown_exact: bool = False):
        self._c = _Ctx()
        m = np.ascontiguousarray(np.asarray(moduli, dtype=np.uint64))
        rc = lib().or_ctx_init(ctypes.byref(self._c), logN, _p(m), L, K, dnum)
        if rc != 0:
            raise ValueError(f"or_ctx_init failed: {rc}")
        self._c.moddown_exact = 1 if moddown_exact else 0
        self.logN, self.N, self.L, self.K, self.dnum = logN, 1 << logN, L, K, dnum
        self.alpha = self._c.alpha
        self.q = [int(x) for x in m]
        self.psi = [int(self._c.psi[i]) for i in range(L + K)]

    def __del__(self):
        try:
            lib().or_ctx_free(ctypes.byref(self._c))
        except Exception:
            pass

    @property
    def ref(self):
        return ctypes.byref(self._c)

    def tables(self, pi: int):
        N = self.N
        t = np.ctypeslib.as_array(self._c.tab, shape=((self.L + self.K) * N,))[pi * N:(pi + 1) * N].copy()
        tp = np.ctypeslib.as_array(self._c.tabp, shape=((self.L + self.K) * N,))[pi * N:(pi + 1) * N].copy()
        it = np.ctypeslib.as_array(self._c.itab, shape=((self.L + self.K) * N,))[pi * N:(pi + 1) * N].copy()
        itp = np.ctypeslib.as_array(self._c.itabp, shape=((self.L + self.K) * N,))[pi * N:(pi + 1) * N].copy()
        return t, tp, it, itp

    # --- transforms ---------------------------------------------------------------------------
    def ntt_fwd(self, data: np.ndarray, prime_idx) -> np.ndarray:
        """data [..., n_limbs, N] uint64 (copied); limb l uses prime prime_idx[l]."""
        a = np.ascontiguousarray(data, dtype=np.uint64).copy()
        nl = a.shape[-2]
        pi = _u32(prime_idx)
        assert len(pi) == nl
        lib().or_ntt_fwd_batch(self.ref, _p(a), a.size // (nl * self.N), nl, _p(pi))
        return a

    def ntt_inv(self, data: np.ndarray, prime_idx) -> np.ndarray:
        a = np.ascontiguousarray(data, dtype=np.uint64).copy()
        nl = a.shape[-2]
        pi = _u32(prime_idx)
        lib().or_ntt_inv_batch(self.ref, _p(a), a.size // (nl * self.N), nl, _p(pi))
        return a

    def bconv(self, x: np.ndarray, in_idx, out_idx) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.uint64)
        ii, oo = _u32(in_idx), _u32(out_idx)
        out = np.zeros((len(oo), self.N), dtype=np.uint64)
        lib().or_bconv(self.ref, _p(x), len(ii), _p(ii), _p(out), len(oo), _p(oo))
        return out

    def bconv_centered(self, x: np.ndarray, in_idx, out_idx) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.uint64)
        ii, oo = _u32(in_idx), _u32(out_idx)
        out = np.zeros((len(oo), self.N), dtype=np.uint64)
        lib().or_bconv_centered(self.ref, _p(x), len(ii), _p(ii), _p(out), len(oo), _p(oo))
        return out

    def tensor(self, a, b, l):
        a = np.ascontiguousarray(a, dtype=np.uint64)
        b = np.ascontiguousarray(b, dtype=np.uint64)
        d = np.zeros((3, l, self.N), dtype=np.uint64)
        lib().or_tensor(self.ref, _p(a), _p(b), l, _p(d))
        return d

    def num_digits(self, l: int) -> int:
        return int(lib().or_num_digits(self.ref, l))

    def modup(self, x, l):
        x = np.ascontiguousarray(x, dtype=np.uint64)
        D = self.num_digits(l)
        ext = np.zeros((D, l + self.K, self.N), dtype=np.uint64)
        lib().or_modup(self.ref, _p(x), l, _p(ext))
        return ext

    def ks_inner(self, ext, l, evk):
        ext = np.ascontiguousarray(ext, dtype=np.uint64)
        evk = np.ascontiguousarray(evk, dtype=np.uint64)
        acc = np.zeros((2, l + self.K, self.N), dtype=np.uint64)
        lib().or_ks_inner(self.ref, _p(ext), l, _p(evk), _p(acc))
        return acc

    def moddown(self, x, l):
        x = np.ascontiguousarray(x, dtype=np.uint64)
        out = np.zeros((l, self.N), dtype=np.uint64)
        lib().or_moddown(self.ref, _p(x), l, _p(out))
        return out

    def keyswitch(self, x, l, evk):
        x = np.ascontiguousarray(x, dtype=np.uint64)
        evk = np.ascontiguousarray(evk, dtype=np.uint64)
        out = np.zeros((2, l, self.N), dtype=np.uint64)
        lib().or_keyswitch(self.ref, _p(x), l, _p(evk), _p(out))
        return out

    def rescale(self, x, l):
        x = np.ascontiguousarray(x, dtype=np.uint64)
        npoly = x.size // (l * self.N)
        out = np.zeros((npoly, l - 1, self.N), dtype=np.uint64)
        lib().or_rescale(self.ref, _p(x), npoly, l, _p(out))
        return out

    def hmult_relin_rescale(self, a, b, l, evk):
        a = np.ascontiguousarray(a, dtype=np.uint64)
        b = np.ascontiguousarray(b, dtype=np.uint64)
        evk = np.ascontiguousarray(evk, dtype=np.uint64)
        out = np.zeros((2, l - 1, self.N), dtype=np.uint64)
        lib().or_hmult_relin_rescale(self.ref, _p(a), _p(b), l, _p(evk), _p(out))
        return out

    def hmult_relin_rescale_batch(self, a, b, l, evk):
        """a, b [n][2][l][N] -> [n][2][l-1][N], the pairs spread over the OpenMP threads (set_threads)"""
        a = np.ascontiguousarray(a, dtype=np.uint64)
        b = np.ascontiguousarray(b, dtype=np.uint64)
        evk = np.ascontiguousarray(evk, dtype=np.uint64)
        n = a.shape[0]
        out = np.zeros((n, 2, l - 1, self.N), dtype=np.uint64)
        lib().or_hmult_relin_rescale_batch(self.ref, _p(a), _p(b), n, l, _p(evk), _p(out))
        return out

    def automorph_coef(self, x, prime_idx, g):
        x = np.ascontiguousarray(x, dtype=np.uint64)
        pi = _u32(prime_idx)
        out = np.zeros_like(x)
        lib().or_automorph_coef(self.ref, _p(x), len(pi), _p(pi), g, _p(out))
        return out

    def automorph_eval(self, x, g):
        x = np.ascontiguousarray(x, dtype=np.uint64)
        nl = x.size // self.N
        out = np.zeros_like(x)
        lib().or_automorph_eval(self.ref, _p(x), nl, g, _p(out))
        return out

    def rot_index(self, k: int) -> int:
        return int(lib().or_rot_index(self.ref, k))

    def rotate(self, ct, l, g, evk):
        ct = np.ascontiguousarray(ct, dtype=np.uint64)
        evk = np.ascontiguousarray(evk, dtype=np.uint64)
        out = np.zeros((2, l, self.N), dtype=np.uint64)
        lib().or_rotate(self.ref, _p(ct), l, g, _p(evk), _p(out))
        return out

    def small_to_eval(self, s: np.ndarray, prime_idx) -> np.ndarray:
        pi = _u32(prime_idx)
        out = np.zeros((len(pi), self.N), dtype=np.uint64)
        if s.dtype == np.int8:
            lib().or_small_to_eval_i8(self.ref, _p(np.ascontiguousarray(s)), len(pi), _p(pi), _p(out))
        else:
            e = np.ascontiguousarray(s, dtype=np.int32)
            lib().or_small_to_eval_i32(self.ref, _p(e), len(pi), _p(pi), _p(out))
        return out

    def pk_gen(self, s_eval, seed: bytes, eseed: bytes, sigma: float = 3.19):
        """public key [2][L+K][N]: b = e - a s over Q*P (s_eval: the secret over all L+K limbs)"""
        T = self.L + self.K
        se = np.ascontiguousarray(s_eval, dtype=np.uint64)
        sd = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
        es = np.frombuffer(bytes(eseed), dtype=np.uint8).copy()
        pk = np.zeros((2, T, self.N), dtype=np.uint64)
        lib().or_pk_gen(self.ref, _p(se), _p(sd), _p(es), sigma, _p(pk))
        return pk

    def pk_encrypt(self, pk, m, l: int, seed: bytes, index: int, sigma: float = 3.19):
        """public-key encryption of the plaintext m [l][N] at level l -> [2][l][N]"""
        pk = np.ascontiguousarray(pk, dtype=np.uint64)
        m = np.ascontiguousarray(m, dtype=np.uint64)
        sd = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
        ct = np.zeros((2, l, self.N), dtype=np.uint64)
        lib().or_pk_encrypt(self.ref, _p(pk), _p(m), l, _p(sd), index, sigma, _p(ct))
        return ct

    def ksk_gen(self, s_old_eval, s_new: np.ndarray, seed: bytes, eseed: bytes, sigma: float = 3.19):
        so = np.ascontiguousarray(s_old_eval, dtype=np.uint64)
        sn = np.ascontiguousarray(s_new, dtype=np.int8)
        sd = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
        es = np.frombuffer(bytes(eseed), dtype=np.uint8).copy()
        T = self.L + self.K
        evk = np.zeros((self.dnum, 2, T, self.N), dtype=np.uint64)
        lib().or_ksk_gen(self.ref, _p(so), _p(sn), _p(sd), _p(es), sigma, _p(evk))
        return evk


# ---------------------------------------------------------------- CKKS encoding (float part + the reference's rule)
def slot_coeffs(z, scale: float) -> np.ndarray:
    """Unrounded coefficients m[0..Np) of the polynomial of the ring of degree Np = 2 len(z) whose slot j (evaluation
    at zeta'^(5^j), zeta' = exp(i pi / Np)) is scale z_j:  m_k = (2 scale / Np) Re( sum_j z_j zeta'^(-5^j k) ).
    Computed with numpy's FFT over the odd exponents 5^j = 2t + 1 (mod 2 Np): an independent float path, not the
    engine's radix-2 transform."""
    z = np.asarray(z, dtype=np.complex128)
    slots = len(z)
    Np = 2 * slots
    M = 2 * Np
    t = np.empty(slots, dtype=np.int64)
    e = 1
    for j in range(slots):
        t[j] = (e - 1) // 2
        e = e * 5 % M
    w = np.zeros(Np, dtype=np.complex128)
    w[t] = z
    F = np.fft.fft(w)  # sum_t w_t exp(-2 pi i t k / Np)
    k = np.arange(Np)
    return (2.0 * scale / Np) * (np.exp(-1j * np.pi * k / Np) * F).real


MAX_BITS_IN_WORD = 61
MAX_BIT_VALUE = float((1 << 63) - (1 << 9) - 1)


def llround(v: np.ndarray) -> np.ndarray:
    """C llround: nearest integer, halves away from zero (|v| >= 2^52 is already integral)"""
    v = np.asarray(v, dtype=np.float64)
    a = np.abs(v)
    r = np.where(a >= 2.0**52, a, np.floor(a + 0.5))
    return (np.sign(v) * r).astype(np.int64)


def round_rule(m):
    """The rounding of encoded coefficients, hpc_gpu_port/periodic_encode.hpp:199-225 (OpenFHE
    CKKSPackedEncoding::Encode): logc = max ceil(log2 |m_k|) over the nonzero m_k (0 if none); logc < 0 is refused
    (too small a scaling factor); log_approx = max(logc - 61, 0); coef = llround(m / 2^log_approx), refused above
    2^63 - 2^9 - 1.  Returns (coef int64 array, log_approx).  The residues of the plaintext are then
    coef * 2^log_approx mod q (periodic_encode.hpp:228-236)."""
    m = np.asarray(m, dtype=np.float64)
    if not np.all(np.isfinite(m)):
        raise ValueError("non-finite coefficient")
    nz = m[m != 0.0]
    logc = int(np.max(np.ceil(np.log2(np.abs(nz))))) if nz.size else 0
    if logc < 0:
        raise ValueError("scaling factor too small")
    log_approx = max(logc - MAX_BITS_IN_WORD, 0)
    v = m / 2.0**log_approx
    if np.any(np.abs(v) > MAX_BIT_VALUE):
        raise ValueError("coefficient overflow")
    return llround(v), log_approx


def set_threads(n: int) -> int:
    """OpenMP threads of the oracle's batch forms (n < 1: all processors); returns the count now in effect"""
    lib().or_set_threads(int(n))
    return int(lib().or_max_threads())
