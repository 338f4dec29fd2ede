"""ctypes front end of libckks_hip.so (the C ABI in include/ckks_engine.h).

This is the Python side of the drop-in boundary: plain pointers and sizes go through; device memory
is either allocated through the ABI (DeviceBuffer) or comes from torch tensors (data_ptr()).
There is no CPU fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libckks_hip.so")

CKKS_OK = 0

_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_int = ctypes.c_int


class Params(ctypes.Structure):
    _fields_ = [("log_n", _u32), ("num_q", _u32), ("num_p", _u32), ("dnum", _u32),
                ("q_bits", _u32), ("p_bits", _u32), ("scale", ctypes.c_double), ("device", _int)]


class SeededPartHeader(ctypes.Structure):
    """ckks_seeded_part_header: the header of a seeded key part file"""
    _fields_ = [("version", _u32), ("expander", _u32), ("ring_dim", _u32), ("size_q", _u32), ("size_p", _u32),
                ("num_part_q", _u32), ("num_per_part_q", _u32), ("count", _u32), ("key_tag", ctypes.c_char * 256),
                ("moduli", _u64 * 128)]


class DevSidecarInfo(ctypes.Structure):
    """ckks_dev_sidecar: the flags and counts of a FIDESlib .dev sidecar"""
    _fields_ = [("n_devices", _u32), ("devices", _u32 * 64), ("auto_load_ciphertexts", ctypes.c_int32),
                ("auto_load_plaintexts", ctypes.c_int32), ("key_dist", ctypes.c_int32), ("n_rotations", _u32),
                ("n_boot_slots", _u32)]


# name -> (restype, argtypes); the exported C ABI (kept in step with include/ckks_engine.h)
SIGNATURES = {
    "ckks_profile_phase": (_int, [_vp, ctypes.c_char_p, _vp]),
    "ckks_profile_phase_markers": (_int, [_vp, _int]),
    "ckks_profile_phase_id": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32)]),
    "ckks_profile_phase_query": (_int, [_vp, _u32, ctypes.c_char_p, _u32, ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_int32)]),
    "ckks_dev_sidecar_read": (_int, [ctypes.c_char_p, _vp, _vp, _u32, _vp, _u32]),
    "ckks_dev_sidecar_write": (_int, [ctypes.c_char_p, _vp, _u32, _vp, _u32]),
    "ckks_rotation_keys_resolve": (_int, [ctypes.c_char_p, _vp, _u32, _vp, _vp, _vp, _u32, ctypes.POINTER(_u32)]),
    "ckks_rotation_keys_load": (_int, [_vp, ctypes.c_char_p, _vp, _u32, _vp, _u32]),
    "ckks_last_error": (ctypes.c_char_p, []),
    "ckks_context_create": (_int, [ctypes.POINTER(Params), ctypes.POINTER(_vp)]),
    "ckks_context_create_from_moduli": (_int, [_u32, _vp, _u32, _vp, _u32, _u32, ctypes.c_double, _int,
                                               ctypes.POINTER(_vp)]),
    "ckks_context_destroy": (None, [_vp]),
    "ckks_context_info": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "ckks_context_moduli": (_int, [_vp, _vp, _u32]),
    "ckks_context_roots": (_int, [_vp, _vp, _u32]),
    "ckks_set_ntt_mode": (_int, [_vp, _int]),
    "ckks_buffer_alloc": (_int, [ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "ckks_buffer_free": (_int, [_vp]),
    "ckks_memcpy_h2d": (_int, [_vp, _vp, ctypes.c_size_t]),
    "ckks_memcpy_d2h": (_int, [_vp, _vp, ctypes.c_size_t]),
    "ckks_device_sync": (_int, []),
    "ckks_ntt_forward": (_int, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "ckks_ntt_inverse": (_int, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "ckks_modup": (_int, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "ckks_ks_inner": (_int, [_vp, _vp, _u32, _u32, _vp, _vp, _vp]),
    "ckks_moddown": (_int, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "ckks_keyswitch": (_int, [_vp, _vp, _u32, _u32, _vp, _vp, _vp]),
    "ckks_rescale": (_int, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "ckks_eval_mult": (_int, [_vp, _vp, _vp, _u32, _u32, _vp, _vp, _vp]),
    "ckks_eval_mult_rescale": (_int, [_vp, _vp, _vp, _u32, _u32, _vp, _vp, _vp]),
    "ckks_eval_mult_rescale_noalloc": (_int, [_vp, _vp, _vp, _u32, _u32, _vp, _vp, _vp]),
    "ckks_eval_add": (_int, [_vp, _vp, _vp, _u32, _u32, _vp, _vp]),
    "ckks_rotation_index": (_u32, [ctypes.c_int64]),
    "ckks_automorphism": (_int, [_vp, _vp, _u32, _u32, _u32, _vp, _vp]),
    "ckks_eval_rotate": (_int, [_vp, _vp, _u32, _u32, ctypes.c_int64, _vp, _vp, _vp]),
    "ckks_eval_mult_plain": (_int, [_vp, _vp, _u32, _u32, _vp, _int, _vp, _vp]),
    "ckks_eval_add_plain": (_int, [_vp, _vp, _u32, _u32, _vp, _int, _vp, _vp]),
    "ckks_eval_rotate_hoisted": (_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp]),
    "ckks_eval_rotate_many": (_int, [_vp, _vp, _u32, _u32, _vp, _vp, _vp, _vp]),
    "ckks_eval_rotate_sum": (_int, [_vp, _vp, _u32, _u32, _vp, _u32, _vp, _vp, _vp]),
    "ckks_linear_transform_bsgs": (_int, [_vp, _vp, _u32, _vp, _u32, _u32, _vp, _vp, _vp, _vp]),
    "ckks_gen_primes": (_int, [_u32, _u32, _vp, _u32, _vp]),
    "ckks_encode_periodic": (_int, [_vp, _vp, _vp, _u32, _u32, _u32, ctypes.c_double, _vp]),
    "ckks_eval_mult_plain_ex": (_int, [_vp, _vp, _u32, _u32, _vp, _int, _u32, _vp, _vp]),
    "ckks_linear_transform_general": (_int, [_vp, _vp, _u32, _vp, _u32, _u32, _vp, _vp, _u32, _vp, _vp, _vp, _vp]),
    "ckks_linear_transform_multi": (_int, [_vp, _vp, _u32, _u32, _vp, _u32, _u32, _vp, _vp, _u32, _vp, _vp, _u32,
                                           _int, _vp, _vp]),
    "ckks_linear_transform_hoisted": (_int, [_vp, _vp, _u32, _u32, _vp, _u32, _vp, _vp, _u32, _vp, _vp, _u32, _vp,
                                             _vp]),
    "ckks_eval_mult_sum": (_int, [_vp, _vp, _u32, _u32, _u32, _vp, _int, _vp, _vp]),
    "ckks_eval_rotate_masked": (_int, [_vp, _vp, _u32, _u32, _vp, _vp, _vp, _vp, _u32, _vp, _u32, _vp, _vp]),
    "ckks_eval_automorphism_ks": (_int, [_vp, _vp, _u32, _u32, _u32, _vp, _vp, _vp]),
    "ckks_eval_mul_i": (_int, [_vp, _vp, _u32, _u32, _int, _vp, _vp]),
    "ckks_eval_lincomb": (_int, [_vp, _u32, _u32, _vp, _vp, _vp, _vp, ctypes.c_double, ctypes.c_double, _u32, _int,
                                 _vp, _vp]),
    "ckks_bootstrap_setup_shared": (_int, [_vp, _vp, ctypes.c_double, ctypes.POINTER(_vp)]),
    "ckks_bootstrap_setup": (_int, [_vp, ctypes.c_double, _u32, _u32, ctypes.c_double, ctypes.c_double,
                                    ctypes.POINTER(_vp)]),
    "ckks_bootstrap_destroy": (None, [_vp]),
    "ckks_bootstrap_steps": (_int, [_vp, _vp, _u32, ctypes.POINTER(_u32)]),
    "ckks_bootstrap_out_level": (_u32, [_vp]),
    "ckks_bootstrap_scale": (ctypes.c_double, [_vp, _u32]),
    "ckks_eval_bootstrap": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _vp]),
    "ckks_eval_bootstrap_stage": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _vp, ctypes.POINTER(_u32)]),
    "ckks_decrypt_coeffs": (_int, [_vp, _vp, _vp, _u32, _vp]),
    "ckks_secret_generate": (_int, [_vp, _vp, _u32, ctypes.POINTER(_vp)]),
    "ckks_secret_destroy": (None, [_vp]),
    "ckks_secret_coeffs": (_int, [_vp, _vp, _u32]),
    "ckks_keygen_relin": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "ckks_keygen_automorphism": (_int, [_vp, _vp, _u32, _vp, _vp, _vp]),
    "ckks_seeded_part_read_header": (_int, [ctypes.c_char_p, ctypes.POINTER(SeededPartHeader)]),
    "ckks_seeded_part_indices": (_int, [ctypes.c_char_p, _vp, _u32, ctypes.POINTER(_u32)]),
    "ckks_seeded_part_load_key": (_int, [_vp, ctypes.c_char_p, _u32, ctypes.POINTER(_u32), _vp]),
    "ckks_seeded_part_write": (_int, [_vp, ctypes.c_char_p, ctypes.c_char_p, _u32, _vp, _vp, _vp]),
    "ckks_ct_file_info": (_int, [ctypes.c_char_p, ctypes.POINTER(_u32), ctypes.POINTER(_u32),
                                 ctypes.POINTER(ctypes.c_double)]),
    "ckks_ct_save": (_int, [_vp, ctypes.c_char_p, _vp, _u32, ctypes.c_double]),
    "ckks_ct_load": (_int, [_vp, ctypes.c_char_p, _u32, _vp, ctypes.POINTER(_u32), ctypes.POINTER(ctypes.c_double)]),
    "ckks_host_alloc": (_int, [ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "ckks_host_free": (_int, [_vp]),
    "ckks_side_copy": (_int, [_vp, _vp, _vp, ctypes.c_size_t, _vp, ctypes.POINTER(ctypes.c_uint64)]),
    "ckks_side_wait": (_int, [_vp, ctypes.c_uint64, _vp]),
    "ckks_side_sync": (_int, [_vp]),
    "ckks_encode_periodic_coeffs": (_int, [_vp, _vp, _vp, _u32, _u32, ctypes.c_double, _vp, _vp]),
    "ckks_expand_periodic": (_int, [_vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp]),
    "ckks_encode": (_int, [_vp, _vp, _vp, _u32, _u32, ctypes.c_double, _vp]),
    "ckks_encrypt": (_int, [_vp, _vp, _vp, _u32, _vp, _u32, _vp]),
    "ckks_keygen_public": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "ckks_encrypt_public": (_int, [_vp, _vp, _vp, _u32, _vp, _u32, _vp]),
    "ckks_decrypt_decode": (_int, [_vp, _vp, _vp, _u32, ctypes.c_double, _vp, _vp, _u32]),
    "ckks_context_counters": (_int, [_vp, _vp, _int]),
    "ckks_context_memory": (_int, [_vp, _vp, _u32]),
    "ckks_set_moddown_exact": (_int, [_vp, _int]),
    "ckks_keygen_switch": (_int, [_vp, _vp, _vp, _vp, _vp, _u32, _vp]),
    "ckks_bootstrap_set_sparse_keys": (_int, [_vp, _vp, _vp]),
    "ckks_eval_bootstrap_many": (_int, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _vp, _vp]),
    "ckks_profile_enable": (_int, [_vp, _int]),
    "ckks_profile_reset": (_int, [_vp]),
    "ckks_profile_query": (_int, [_vp, _u32, ctypes.c_char_p, _u32, _vp, _vp, _vp]),
}


class CkksError(RuntimeError):
    pass


_lib = None


def load(path: str = LIB_PATH):
    """Load the engine library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise CkksError(f"{path} is missing: build it with __graft_entry__.build() (make -C fhe-ssm_amd)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != CKKS_OK:
        raise CkksError(f"ckks error {rc}: {load().ckks_last_error().decode()}")


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_vp)


class DeviceBuffer:
    """A device allocation made through the ABI."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _vp()
        check(load().ckks_buffer_alloc(self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(load().ckks_memcpy_h2d(self.ptr, _ptr(a), a.nbytes))

    def download(self, shape, dtype=np.uint64) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(load().ckks_memcpy_d2h(_ptr(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(load().ckks_buffer_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync() -> None:
    check(load().ckks_device_sync())


class Context:
    """Engine context (moduli, NTT tables and key-switch constants resident on the device)."""

    def __init__(self, num_q: int = 24, num_p: int = 8, dnum: int = 3, q_bits: int = 54, p_bits: int = 60,
                 scale: float = 2.0**50, device: int = 0, log_n: int = 16, moduli=None):
        lib = load()
        h = _vp()
        if moduli is None:
            p = Params(log_n, num_q, num_p, dnum, q_bits, p_bits, scale, device)
            check(lib.ckks_context_create(ctypes.byref(p), ctypes.byref(h)))
        else:
            q = np.ascontiguousarray(np.asarray(moduli[:num_q], dtype=np.uint64))
            pp = np.ascontiguousarray(np.asarray(list(moduli[num_q:num_q + num_p]) or [0], dtype=np.uint64))
            check(lib.ckks_context_create_from_moduli(log_n, _ptr(q), num_q, _ptr(pp), num_p, dnum, scale, device,
                                                      ctypes.byref(h)))
        self.h = h.value
        n, L, K, D = _u32(), _u32(), _u32(), _u32()
        check(lib.ckks_context_info(self.h, ctypes.byref(n), ctypes.byref(L), ctypes.byref(K), ctypes.byref(D)))
        self.N, self.L, self.K, self.dnum = n.value, L.value, K.value, D.value
        self.scale = scale
        m = np.zeros(self.L + self.K, dtype=np.uint64)
        check(lib.ckks_context_moduli(self.h, _ptr(m), len(m)))
        self.moduli = [int(x) for x in m]
        r = np.zeros(self.L + self.K, dtype=np.uint64)
        check(lib.ckks_context_roots(self.h, _ptr(r), len(r)))
        self.roots = [int(x) for x in r]

    def close(self) -> None:
        if self.h:
            load().ckks_context_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_ntt_mode(self, mode: int) -> None:
        check(load().ckks_set_ntt_mode(self.h, mode))

    # raw stages on device pointers -------------------------------------------------------------
    def ntt_forward(self, d_ptr: int, n_polys: int, prime_idx, stream=None) -> None:
        pi = np.ascontiguousarray(np.asarray(prime_idx, dtype=np.uint32))
        check(load().ckks_ntt_forward(self.h, d_ptr, n_polys, len(pi), _ptr(pi), stream))

    def ntt_inverse(self, d_ptr: int, n_polys: int, prime_idx, stream=None) -> None:
        pi = np.ascontiguousarray(np.asarray(prime_idx, dtype=np.uint32))
        check(load().ckks_ntt_inverse(self.h, d_ptr, n_polys, len(pi), _ptr(pi), stream))

    def num_digits(self, level: int) -> int:
        alpha = -(-self.L // self.dnum)
        return -(-level // alpha)

    def modup(self, d_x, batch, level, d_ext, stream=None):
        check(load().ckks_modup(self.h, d_x, batch, level, d_ext, stream))

    def ks_inner(self, d_ext, batch, level, d_evk, d_acc, stream=None):
        check(load().ckks_ks_inner(self.h, d_ext, batch, level, d_evk, d_acc, stream))

    def moddown(self, d_x, n_polys, level, d_out, stream=None):
        check(load().ckks_moddown(self.h, d_x, n_polys, level, d_out, stream))

    def keyswitch(self, d_x, batch, level, d_evk, d_out, stream=None):
        check(load().ckks_keyswitch(self.h, d_x, batch, level, d_evk, d_out, stream))

    def rescale(self, d_in, n_polys, level, d_out, stream=None):
        check(load().ckks_rescale(self.h, d_in, n_polys, level, d_out, stream))

    def eval_mult(self, d_a, d_b, batch, level, d_evk, d_out, stream=None):
        check(load().ckks_eval_mult(self.h, d_a, d_b, batch, level, d_evk, d_out, stream))

    def eval_mult_rescale(self, d_a, d_b, batch, level, d_evk, d_out, stream=None):
        check(load().ckks_eval_mult_rescale(self.h, d_a, d_b, batch, level, d_evk, d_out, stream))

    def eval_mult_rescale_noalloc(self, d_a, d_b, batch, level, d_evk, d_out, stream=None):
        check(load().ckks_eval_mult_rescale_noalloc(self.h, d_a, d_b, batch, level, d_evk, d_out, stream))

    def eval_add(self, d_x, d_y, n_polys, level, d_out, stream=None):
        check(load().ckks_eval_add(self.h, d_x, d_y, n_polys, level, d_out, stream))

    def automorphism(self, d_in, n_polys, level, g, d_out, stream=None):
        check(load().ckks_automorphism(self.h, d_in, n_polys, level, g, d_out, stream))

    def eval_rotate(self, d_ct, batch, level, step, d_evk, d_out, stream=None):
        check(load().ckks_eval_rotate(self.h, d_ct, batch, level, step, d_evk, d_out, stream))


    def eval_mult_plain(self, d_ct, batch, level, d_pt, d_out, pt_shared=True, stream=None):
        check(load().ckks_eval_mult_plain(self.h, d_ct, batch, level, d_pt, 1 if pt_shared else 0, d_out, stream))

    def eval_add_plain(self, d_ct, batch, level, d_pt, d_out, pt_shared=True, stream=None):
        check(load().ckks_eval_add_plain(self.h, d_ct, batch, level, d_pt, 1 if pt_shared else 0, d_out, stream))

    def eval_rotate_hoisted(self, d_ct, level, steps, d_evks, d_out, stream=None):
        st = np.ascontiguousarray(np.asarray(steps, dtype=np.int64))
        keys = _ptr_array(d_evks)
        check(load().ckks_eval_rotate_hoisted(self.h, d_ct, level, _ptr(st), len(st), keys, d_out, stream))

    def eval_rotate_sum(self, d_ct, batch, level, steps, d_evks, d_out, stream=None):
        """out = ct + sum_i Rot_{steps[i]}(ct), the rotations hoisted over one ModUp and one ModDown"""
        st = np.ascontiguousarray(np.asarray(steps, dtype=np.int64))
        keys = _ptr_array(d_evks)
        check(load().ckks_eval_rotate_sum(self.h, d_ct, batch, level, _ptr(st), len(st), keys, d_out, stream))

    def eval_rotate_many(self, d_cts, level, steps, d_evks, d_out, stream=None):
        st = np.ascontiguousarray(np.asarray(steps, dtype=np.int64))
        keys = _ptr_array(d_evks)
        check(load().ckks_eval_rotate_many(self.h, d_cts, len(st), level, _ptr(st), keys, d_out, stream))

    def linear_transform_bsgs(self, d_ct, level, d_diags, n_diag, baby_steps, baby_evks, giant_evks, d_out,
                              stream=None):
        check(load().ckks_linear_transform_bsgs(self.h, d_ct, level, d_diags, n_diag, baby_steps,
                                                _ptr_array(baby_evks), _ptr_array(giant_evks), d_out, stream))

    def encode_periodic(self, values, level: int, scale: float, d_out) -> None:
        """values [n][period] (real or complex); out [n][level][2 period] compressed periodic plaintexts"""
        v = np.atleast_2d(np.asarray(values))
        re = np.ascontiguousarray(v.real, dtype=np.float64)
        im = np.ascontiguousarray(v.imag, dtype=np.float64) if np.iscomplexobj(v) else None
        check(load().ckks_encode_periodic(self.h, _ptr(re), _ptr(im) if im is not None else None, v.shape[0],
                                          v.shape[1], level, scale, d_out))

    def encode_periodic_coeffs(self, values, scale: float, d_coef, d_log_approx) -> None:
        """the host half of encode_periodic: d_coef [n][2 period] int64, d_log_approx [n] int32 (any level)"""
        v = np.atleast_2d(np.asarray(values))
        re = np.ascontiguousarray(v.real, dtype=np.float64)
        im = np.ascontiguousarray(v.imag, dtype=np.float64) if np.iscomplexobj(v) else None
        check(load().ckks_encode_periodic_coeffs(self.h, _ptr(re), _ptr(im) if im is not None else None, v.shape[0],
                                                 v.shape[1], scale, d_coef, d_log_approx))

    def expand_periodic(self, d_coef, d_log_approx, n_vectors: int, period: int, level: int, d_out,
                        stream=None) -> None:
        """the device half: d_out [n][level][2 period], the words encode_periodic writes"""
        check(load().ckks_expand_periodic(self.h, d_coef, d_log_approx, n_vectors, period, level, d_out, stream))

    def eval_mult_plain_ex(self, d_ct, batch, level, d_pt, log_rep, d_out, pt_shared=True, stream=None):
        check(load().ckks_eval_mult_plain_ex(self.h, d_ct, batch, level, d_pt, 1 if pt_shared else 0, log_rep,
                                             d_out, stream))

    def linear_transform_general(self, d_ct, level, d_diags, log_rep, baby_steps, baby_evks, giant_steps,
                                 giant_evks, d_out, stream=None):
        bs = np.ascontiguousarray(np.asarray(baby_steps, dtype=np.int64))
        gs = np.ascontiguousarray(np.asarray(giant_steps, dtype=np.int64))
        check(load().ckks_linear_transform_general(self.h, d_ct, level, d_diags, log_rep, len(bs), _ptr(bs),
                                                   _ptr_array([k or 0 for k in baby_evks]), len(gs), _ptr(gs),
                                                   _ptr_array([k or 0 for k in giant_evks]), d_out, stream))

    def linear_transform_multi(self, inputs, level, d_diags, log_rep, baby_steps, baby_evks, giant_steps,
                               giant_evks, n_out, rescale, d_out, stream=None):
        bs = np.ascontiguousarray(np.asarray(baby_steps, dtype=np.int64))
        gs = np.ascontiguousarray(np.asarray(giant_steps, dtype=np.int64))
        check(load().ckks_linear_transform_multi(self.h, _ptr_array(inputs), len(inputs), level, d_diags, log_rep,
                                                 len(bs), _ptr(bs), _ptr_array([k or 0 for k in baby_evks]), len(gs),
                                                 _ptr(gs), _ptr_array([k or 0 for k in giant_evks]), n_out,
                                                 1 if rescale else 0, d_out, stream))

    def linear_transform_hoisted(self, inputs, level, d_diags, baby_steps, baby_evks, giant_steps, giant_evks,
                                 n_out, d_out, stream=None):
        """double-hoisted BSGS with the rescale; d_diags over the primes of Q_level then P"""
        bs = np.ascontiguousarray(np.asarray(baby_steps, dtype=np.int64))
        gs = np.ascontiguousarray(np.asarray(giant_steps, dtype=np.int64))
        check(load().ckks_linear_transform_hoisted(self.h, _ptr_array(inputs), len(inputs), level, d_diags, len(bs),
                                                   _ptr(bs), _ptr_array([k or 0 for k in baby_evks]), len(gs),
                                                   _ptr(gs), _ptr_array([k or 0 for k in giant_evks]), n_out, d_out,
                                                   stream))

    def eval_mult_sum(self, pairs, level, d_evk, d_out, rescale=True, stream=None):
        """pairs: [batch][n_products] of (a, b) device pointers"""
        batch, npr = len(pairs), len(pairs[0])
        flat = [p for item in pairs for ab in item for p in ab]
        assert len(flat) == batch * npr * 2
        check(load().ckks_eval_mult_sum(self.h, _ptr_array(flat), npr, batch, level, d_evk, 1 if rescale else 0,
                                        d_out, stream))

    def eval_rotate_masked(self, d_ct, level, steps_lo, evks_lo, steps_hi, evks_hi, n_sets, d_pts, log_rep, d_out,
                           stream=None):
        lo = np.ascontiguousarray(np.asarray(steps_lo, dtype=np.int64))
        hi = np.ascontiguousarray(np.asarray(steps_hi, dtype=np.int64))
        check(load().ckks_eval_rotate_masked(self.h, d_ct, level, len(lo), _ptr(lo),
                                             _ptr_array([k or 0 for k in evks_lo]), _ptr(hi),
                                             _ptr_array([k or 0 for k in evks_hi]), n_sets, d_pts, log_rep, d_out,
                                             stream))

    def eval_automorphism_ks(self, d_ct, batch, level, g, d_evk, d_out, stream=None):
        check(load().ckks_eval_automorphism_ks(self.h, d_ct, batch, level, g, d_evk, d_out, stream))

    def eval_mul_i(self, d_in, n_polys, level, sign, d_out, stream=None):
        check(load().ckks_eval_mul_i(self.h, d_in, n_polys, level, sign, d_out, stream))

    def eval_lincomb(self, batch, terms, levels, coeffs, scales_in, scale_out, add_const, target_level, integer,
                     d_out, stream=None):
        lv = np.ascontiguousarray(np.asarray(levels, dtype=np.uint32))
        cf = np.ascontiguousarray(np.asarray(coeffs, dtype=np.float64))
        si = np.ascontiguousarray(np.asarray(scales_in if scales_in is not None else [1.0] * len(terms),
                                             dtype=np.float64))
        check(load().ckks_eval_lincomb(self.h, batch, len(terms), _ptr_array(terms), _ptr(lv), _ptr(cf), _ptr(si),
                                       scale_out, add_const, target_level, 1 if integer else 0, d_out, stream))

    # client side ------------------------------------------------------------------------------
    def secret(self, seed: bytes, hamming_weight: int = 192) -> "Secret":
        return Secret(self, seed, hamming_weight)

    def keygen_relin(self, sk, seed: bytes, eseed: bytes, d_evk) -> None:
        check(load().ckks_keygen_relin(self.h, sk.h, _seed(seed), _seed(eseed), d_evk))

    def keygen_switch(self, sk_from, sk_to, seed: bytes, eseed: bytes, d_evk, q_limbs: int = 0) -> None:
        check(load().ckks_keygen_switch(self.h, sk_from.h, sk_to.h, _seed(seed), _seed(eseed), q_limbs, d_evk))

    def keygen_automorphism(self, sk, g: int, seed: bytes, eseed: bytes, d_evk) -> None:
        check(load().ckks_keygen_automorphism(self.h, sk.h, g, _seed(seed), _seed(eseed), d_evk))

    def seeded_part_load_key(self, path: str, record: int, d_evk) -> int:
        """key `record` of a seeded part file into d_evk; returns its automorphism index"""
        idx = _u32(0)
        check(load().ckks_seeded_part_load_key(self.h, path.encode(), record, ctypes.byref(idx), d_evk))
        return int(idx.value)

    def rotation_keys_load(self, dev_path: str, part_paths, d_evks) -> None:
        """LoadContext's rotation keys: the key of each rotation the .dev sidecar lists, from the seeded part files,
        into d_evks (one device buffer per listed rotation, in the sidecar's order)"""
        check(load().ckks_rotation_keys_load(self.h, dev_path.encode(), _str_array(part_paths), len(part_paths),
                                             _ptr_array(list(d_evks)), len(d_evks)))

    def seeded_part_write(self, path: str, key_tag: str, indices, seeds, d_evks) -> None:
        ix = np.ascontiguousarray(np.asarray(indices, dtype=np.uint32))
        sd = np.frombuffer(b"".join(bytes(x) for x in seeds), dtype=np.uint8).copy()
        assert sd.size == 32 * len(ix) and len(d_evks) == len(ix)
        check(load().ckks_seeded_part_write(self.h, path.encode(), key_tag.encode(), len(ix), _ptr(ix) if len(ix) else None,
                                            _ptr(sd) if len(ix) else None, _ptr_array(d_evks)))

    def ct_save(self, path: str, d_ct, level: int, scale: float) -> None:
        """a ciphertext [2][level][N] into a ciphertext file (the serve protocol's req.N.t / resp.N.t)"""
        check(load().ckks_ct_save(self.h, path.encode(), d_ct, level, scale))

    def ct_load(self, path: str, d_ct, cap_level: int):
        """a ciphertext file into d_ct (room for cap_level limbs); returns (level, scale)"""
        lv, sc = _u32(0), ctypes.c_double()
        check(load().ckks_ct_load(self.h, path.encode(), cap_level, d_ct, ctypes.byref(lv), ctypes.byref(sc)))
        return int(lv.value), float(sc.value)

    def encode(self, values, level: int, scale: float, d_pt) -> None:
        v = np.asarray(values)
        re = np.ascontiguousarray(v.real, dtype=np.float64)
        im = np.ascontiguousarray(v.imag, dtype=np.float64) if np.iscomplexobj(v) else None
        check(load().ckks_encode(self.h, _ptr(re), _ptr(im) if im is not None else None, len(re), level, scale,
                                 d_pt))

    def encrypt(self, sk, d_pt, level: int, seed: bytes, index: int, d_ct) -> None:
        check(load().ckks_encrypt(self.h, sk.h, d_pt, level, _seed(seed), index, d_ct))

    def keygen_public(self, sk, seed: bytes, eseed: bytes, d_pk) -> None:
        """public key [2][L+K][N] over Q*P: b = e - a s"""
        check(load().ckks_keygen_public(self.h, sk.h, _seed(seed), _seed(eseed), d_pk))

    def encrypt_public(self, d_pk, d_pt, level: int, seed: bytes, index: int, d_ct) -> None:
        check(load().ckks_encrypt_public(self.h, d_pk, d_pt, level, _seed(seed), index, d_ct))

    def decrypt(self, sk, d_ct, level: int, scale: float, n_slots: int = 1 << 15, complex_out: bool = False):
        re = np.zeros(n_slots, dtype=np.float64)
        im = np.zeros(n_slots, dtype=np.float64)
        check(load().ckks_decrypt_decode(self.h, sk.h, d_ct, level, scale, _ptr(re), _ptr(im), n_slots))
        return re + 1j * im if complex_out else re

    def decrypt_coeffs(self, sk, d_ct, level: int) -> np.ndarray:
        out = np.zeros(self.N, dtype=np.float64)
        check(load().ckks_decrypt_coeffs(self.h, sk.h, d_ct, level, _ptr(out)))
        return out

    def memory(self) -> dict:
        """device bytes the context holds itself: constant tables, key-switching workspaces, bootstrapping pool, and
        the library's static scratch for the allocation-free entry point (one per GPU, shared by its contexts)"""
        v = np.zeros(4, dtype=np.uint64)
        check(load().ckks_context_memory(self.h, _ptr(v), 4))
        return {"tables": int(v[0]), "workspaces": int(v[1]), "bootstrap_pool": int(v[2]),
                "noalloc_scratch_per_gpu": int(v[3])}

    # profiling ---------------------------------------------------------------------------------
    def profile(self, on: bool) -> None:
        check(load().ckks_profile_enable(self.h, 1 if on else 0))

    def profile_reset(self) -> None:
        check(load().ckks_profile_reset(self.h))

    def set_moddown_exact(self, exact: bool) -> None:
        check(load().ckks_set_moddown_exact(self.h, 1 if exact else 0))

    def key_switches(self, reset: bool = False) -> int:
        n = ctypes.c_uint64()
        check(load().ckks_context_counters(self.h, ctypes.byref(n), 1 if reset else 0))
        return n.value

    def profile_phase(self, phase: str, stream=None) -> None:
        """label the launches that follow (see ckks_profile_phase)"""
        check(load().ckks_profile_phase(self.h, phase.encode(), stream))

    def profile_phase_markers(self, on: bool) -> None:
        check(load().ckks_profile_phase_markers(self.h, 1 if on else 0))

    def profile_phase_id(self, phase: str) -> int:
        """the marker id of a phase label (-1 if it was never set with markers on)"""
        mid = ctypes.c_int32()
        check(load().ckks_profile_phase_id(self.h, phase.encode(), ctypes.byref(mid)))
        return int(mid.value)

    def profile_phase_report(self) -> dict:
        """{phase label: (launches, total_ms, total_algorithmic_bytes, marker id)}"""
        out = {}
        i = 0
        name = ctypes.create_string_buffer(64)
        while True:
            n, ms, by, mid = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_int32()
            rc = load().ckks_profile_phase_query(self.h, i, name, 64, ctypes.byref(n), ctypes.byref(ms),
                                                 ctypes.byref(by), ctypes.byref(mid))
            if rc != CKKS_OK:
                break
            out[name.value.decode()] = (n.value, ms.value, by.value, mid.value)
            i += 1
        return out

    def profile_report(self) -> dict:
        """{kernel name: (launches, total_ms, total_algorithmic_bytes)}"""
        out = {}
        i = 0
        name = ctypes.create_string_buffer(64)
        while True:
            n, ms, by = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double()
            rc = load().ckks_profile_query(self.h, i, name, 64, ctypes.byref(n), ctypes.byref(ms), ctypes.byref(by))
            if rc != CKKS_OK:
                break
            out[name.value.decode()] = (n.value, ms.value, by.value)
            i += 1
        return out


def _ptr_array(ptrs):
    ptrs = list(ptrs)
    if not ptrs:
        return None
    arr = (_vp * len(ptrs))(*ptrs)
    return ctypes.cast(arr, _vp)


def seeded_part_header(path: str) -> dict:
    """the header of a seeded key part file (host only: no context, no device)"""
    h = SeededPartHeader()
    check(load().ckks_seeded_part_read_header(path.encode(), ctypes.byref(h)))
    n = h.size_q + h.size_p
    return {"version": h.version, "expander": h.expander, "N": h.ring_dim, "size_q": h.size_q, "size_p": h.size_p,
            "num_part_q": h.num_part_q, "num_per_part_q": h.num_per_part_q, "count": h.count,
            "key_tag": h.key_tag.decode(), "moduli": [int(h.moduli[i]) for i in range(n)]}


def _str_array(strs):
    arr = (ctypes.c_char_p * max(1, len(strs)))(*[x.encode() for x in strs])
    return ctypes.cast(arr, _vp)


def dev_sidecar_read(path: str) -> dict:
    """a FIDESlib .dev sidecar (host only): devices, flags, rotation amounts and bootstrap slot counts"""
    info = DevSidecarInfo()
    check(load().ckks_dev_sidecar_read(path.encode(), ctypes.byref(info), None, 0, None, 0))
    rots = np.zeros(max(1, info.n_rotations), dtype=np.int32)
    slots = np.zeros(max(1, info.n_boot_slots), dtype=np.uint32)
    check(load().ckks_dev_sidecar_read(path.encode(), ctypes.byref(info), _ptr(rots), info.n_rotations, _ptr(slots),
                                       info.n_boot_slots))
    return {"devices": [int(info.devices[i]) for i in range(info.n_devices)],
            "AutoLoadCiphertexts": int(info.auto_load_ciphertexts), "AutoLoadPlaintexts": int(info.auto_load_plaintexts),
            "KeyDist": int(info.key_dist), "RotationIndexes": [int(x) for x in rots[: info.n_rotations]],
            "BootstrapSlots": [int(x) for x in slots[: info.n_boot_slots]]}


def dev_sidecar_write(path: str, rotations, boot_slots) -> None:
    """the reference client's cryptocontext.bin.dev for these rotation amounts and bootstrap slot counts"""
    r = np.ascontiguousarray(np.asarray(list(rotations), dtype=np.int32))
    b = np.ascontiguousarray(np.asarray(list(boot_slots), dtype=np.uint32))
    check(load().ckks_dev_sidecar_write(path.encode(), _ptr(r) if len(r) else None, len(r),
                                        _ptr(b) if len(b) else None, len(b)))


def rotation_keys_resolve(dev_path: str, part_paths) -> list:
    """(part, record, automorphism index) holding the key of each rotation the sidecar lists (host only)"""
    n = _u32(0)
    check(load().ckks_rotation_keys_resolve(dev_path.encode(), _str_array(part_paths), len(part_paths), None, None,
                                            None, 0, ctypes.byref(n)))
    cap = n.value
    p, r, g = (np.zeros(max(1, cap), dtype=np.uint32) for _ in range(3))
    check(load().ckks_rotation_keys_resolve(dev_path.encode(), _str_array(part_paths), len(part_paths), _ptr(p), _ptr(r),
                                            _ptr(g), cap, ctypes.byref(n)))
    return [(int(p[i]), int(r[i]), int(g[i])) for i in range(n.value)]


def ct_file_info(path: str) -> dict:
    """the header of a ciphertext file (host only: no context, no device)"""
    n, lv, sc = _u32(0), _u32(0), ctypes.c_double()
    check(load().ckks_ct_file_info(path.encode(), ctypes.byref(n), ctypes.byref(lv), ctypes.byref(sc)))
    return {"N": int(n.value), "level": int(lv.value), "scale": float(sc.value)}


def seeded_part_indices(path: str) -> list:
    count = _u32(0)
    check(load().ckks_seeded_part_indices(path.encode(), None, 0, ctypes.byref(count)))
    out = np.zeros(max(1, count.value), dtype=np.uint32)
    check(load().ckks_seeded_part_indices(path.encode(), _ptr(out), count.value, ctypes.byref(count)))
    return [int(x) for x in out[: count.value]]


def _seed(seed: bytes):
    b = bytes(seed)
    assert len(b) == 32
    return ctypes.c_char_p(b)


class Secret:
    def __init__(self, ctx: Context, seed: bytes, hamming_weight: int):
        h = _vp()
        check(load().ckks_secret_generate(ctx.h, _seed(seed), hamming_weight, ctypes.byref(h)))
        self.h = h.value
        self.ctx = ctx

    def coeffs(self) -> np.ndarray:
        out = np.zeros(1 << 16, dtype=np.int8)
        check(load().ckks_secret_coeffs(self.h, _ptr(out), len(out)))
        return out

    def close(self):
        if self.h:
            load().ckks_secret_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rotation_index(step: int) -> int:
    return int(load().ckks_rotation_index(step))


def gen_primes(bits: int, count: int, skip=()) -> list:
    sk = np.ascontiguousarray(np.asarray(list(skip) or [0], dtype=np.uint64))
    out = np.zeros(count, dtype=np.uint64)
    check(load().ckks_gen_primes(bits, count, _ptr(sk), len(skip), _ptr(out)))
    return [int(x) for x in out]


class Bootstrap:
    """EvalBootstrapSetup: plan (CtS/StC diagonals, Chebyshev coefficients) resident on the device."""

    def __init__(self, ctx: Context, K: float = 22.0, cheb_degree: int = 59, double_angles: int = 2,
                 top_scale: float = 2.0**50, in_scale: float = 2.0**50, share=None):
        """share: another Bootstrap of this context whose diagonals this plan uses (its in_scale an integer
        multiple of this one's; K, degree, double angles and top scale are then the other plan's)"""
        h = _vp()
        if share is not None:
            check(load().ckks_bootstrap_setup_shared(ctx.h, share.h, in_scale, ctypes.byref(h)))
        else:
            check(load().ckks_bootstrap_setup(ctx.h, K, cheb_degree, double_angles, top_scale, in_scale,
                                              ctypes.byref(h)))
        self.h = h.value
        self.ctx = ctx
        n = _u32()
        check(load().ckks_bootstrap_steps(self.h, None, 0, ctypes.byref(n)))
        st = np.zeros(max(1, n.value), dtype=np.int64)
        check(load().ckks_bootstrap_steps(self.h, _ptr(st), len(st), ctypes.byref(n)))
        self.steps = [int(x) for x in st[:n.value]]
        self.out_level = int(load().ckks_bootstrap_out_level(self.h))

    def scale(self, level: int) -> float:
        return float(load().ckks_bootstrap_scale(self.h, level))

    def set_sparse_keys(self, d_to_sparse, d_from_sparse) -> None:
        check(load().ckks_bootstrap_set_sparse_keys(self.h, d_to_sparse, d_from_sparse))

    def run(self, d_ct_in, d_relin, d_conj, keys: dict, d_out, stream=None):
        steps = np.ascontiguousarray(np.asarray(list(keys.keys()), dtype=np.int64))
        check(load().ckks_eval_bootstrap(self.ctx.h, self.h, d_ct_in, d_relin, d_conj, _ptr(steps), _ptr_array(
            list(keys.values())), len(steps), d_out, stream))

    def run_many(self, d_ct_in, batch, d_relin, d_conj, keys: dict, d_out, stream=None):
        steps = np.ascontiguousarray(np.asarray(list(keys.keys()), dtype=np.int64))
        check(load().ckks_eval_bootstrap_many(self.ctx.h, self.h, d_ct_in, batch, d_relin, d_conj, _ptr(steps),
                                              _ptr_array(list(keys.values())), len(steps), d_out, stream))

    def run_stage(self, d_ct_in, d_relin, d_conj, keys: dict, stage: int, d_out) -> int:
        steps = np.ascontiguousarray(np.asarray(list(keys.keys()), dtype=np.int64))
        lvl = _u32()
        check(load().ckks_eval_bootstrap_stage(self.ctx.h, self.h, d_ct_in, d_relin, d_conj, _ptr(steps), _ptr_array(
            list(keys.values())), len(steps), stage, d_out, ctypes.byref(lvl)))
        return lvl.value

    def close(self):
        if self.h:
            load().ckks_bootstrap_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
