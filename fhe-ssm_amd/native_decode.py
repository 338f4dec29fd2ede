"""ctypes front end of libfhe_ssm_decode.so (include/fhe_ssm_decode.h): the config-5 decode step's native driver.

The driver is C++ over the engine's C ABI; this module only hands it the context, the refresh plans, the keys
and the weights, and calls one step at a time -- or hands it a directory to serve (the reference's --serve DIR
protocol, the loop in host/serve.cpp).  There is no Python fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfhe_ssm_decode.so")

_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_int = ctypes.c_int


class Refresh(ctypes.Structure):
    _fields_ = [("plan", _vp), ("in_scale", ctypes.c_double)]


class ServeOpts(ctypes.Structure):
    """fhe_ssm_serve_opts"""
    _fields_ = [("timeout_sec", _u32), ("poll_ms", _u32), ("stateful", ctypes.c_int32), ("log_fd", ctypes.c_int32),
                ("first_req", _u32)]


class ServeReport(ctypes.Structure):
    """fhe_ssm_serve_report"""
    _fields_ = [("served", _u32), ("failed", _u32), ("next_req", _u32), ("exit_reason", ctypes.c_int32)]


# int handler(void* user, uint32_t req, const char* req_prefix, const char* resp_prefix, const char* meta_json,
#             int32_t reset, char* err, size_t err_cap)
ServeHandler = ctypes.CFUNCTYPE(_int, _vp, _u32, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int32,
                                _vp, ctypes.c_size_t)


SIGNATURES = {
    "fhe_ssm_last_error": (ctypes.c_char_p, []),
    "fhe_ssm_decoder_create": (_int, [_vp, _u32, Refresh, Refresh, Refresh, _vp, _vp, _vp, _vp, _u32,
                                      ctypes.POINTER(_vp)]),
    "fhe_ssm_decoder_destroy": (None, [_vp]),
    "fhe_ssm_rotation_steps": (_int, [_vp, _u32, ctypes.POINTER(_u32)]),
    "fhe_ssm_decoder_set_weight": (_int, [_vp, ctypes.c_char_p, ctypes.c_int32, _vp, ctypes.c_size_t]),
    "fhe_ssm_decoder_step": (_int, [_vp, _vp, _u32, ctypes.c_double, _vp, ctypes.POINTER(_u32),
                                    ctypes.POINTER(ctypes.c_double)]),
    "fhe_ssm_decoder_stats": (_int, [_vp, ctypes.POINTER(ctypes.c_uint64)]),
    "fhe_ssm_decoder_reset": (_int, [_vp]),
    "fhe_ssm_serve_dir": (_int, [ctypes.c_char_p, ctypes.POINTER(ServeOpts), ServeHandler, _vp,
                                 ctypes.POINTER(ServeReport)]),
    "fhe_ssm_decoder_serve": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ServeOpts), ctypes.POINTER(ServeReport)]),
    "fhe_ssm_meta_int": (ctypes.c_longlong, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_longlong]),
    "fhe_ssm_decoder_memory": (_int, [_vp, _vp, _u32]),
    "fhe_ssm_client_encrypt_rows": (_int, [_vp, _vp, ctypes.c_char_p, _u32, _u32, _u32, _u32, _u32,
                                           ctypes.c_double, _vp]),
    "fhe_ssm_client_decrypt_logits": (_int, [_vp, _vp, ctypes.c_char_p, _vp, _u32, _u32, _u32]),
    "fhe_ssm_store_create": (_int, [ctypes.POINTER(_vp)]),
    "fhe_ssm_store_destroy": (None, [_vp]),
    "fhe_ssm_store_put": (_int, [_vp, _vp, _vp, _u64]),
    "fhe_ssm_store_count": (_int, [_vp, ctypes.POINTER(_u64)]),
    "fhe_ssm_store_entry": (_int, [_vp, _u64, _vp, ctypes.POINTER(_u64)]),
    "fhe_ssm_store_get": (_int, [_vp, _vp, _vp, _u64, ctypes.POINTER(_u64)]),
    "fhe_ssm_store_save": (_int, [_vp, ctypes.c_char_p, ctypes.c_char_p]),
    "fhe_ssm_store_load": (_int, [_vp, ctypes.c_char_p, ctypes.c_char_p, _u32, _u32, ctypes.POINTER(_u64)]),
    "fhe_ssm_store_read_stamp": (_int, [ctypes.c_char_p, _vp, _u64, ctypes.POINTER(_u64)]),
    "fhe_ssm_store_append": (_int, [ctypes.c_char_p, _vp, _vp, _u64]),
    "fhe_ssm_store_load_journal": (_int, [_vp, ctypes.c_char_p, _u32, _u32, ctypes.POINTER(_u64),
                                          ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "fhe_ssm_decoder_store_save": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
    "fhe_ssm_decoder_store_load": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
}

LAYER_WEIGHTS = ("g1", "g2", "k_k", "mu_r", "mu_k", "mu_v", "mu_w", "mu_a", "mu_g", "mu_c", "W_r", "W_k", "W_v",
                 "W_w", "W_a", "W_g", "W_o", "W_ck", "W_cv", "p_n1", "p_n2", "p_w", "p_a", "p_g", "p_h",
                 "W_vg", "k_a", "r_k", "ln_w", "ln_b", "p_v", "p_kn", "p_gn")
MODEL_WEIGHTS = ("g_o", "p_o")

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"fhe_ssm error {rc}: {load().fhe_ssm_last_error().decode()}")


def rotation_steps() -> list:
    n = _u32()
    check(load().fhe_ssm_rotation_steps(None, 0, ctypes.byref(n)))
    buf = (ctypes.c_int64 * n.value)()
    check(load().fhe_ssm_rotation_steps(buf, n.value, ctypes.byref(n)))
    return list(buf)


class NativeDecoder:
    """The decode step in C++.  boots: refresh kind ("state", "inc_tm", "inc_cm") -> (ckks.Bootstrap, in_scale);
    keys: rotation step -> device pointer of its automorphism key (every layer step and every plan step)."""

    def __init__(self, ckks, ctx, n_layers: int, boots: dict, d_relin: int, d_conj: int, keys: dict):
        self.ckks, self.ctx, self.n_layers = ckks, ctx, n_layers
        steps = np.ascontiguousarray(np.asarray(sorted(keys), dtype=np.int64))
        ptrs = (_vp * len(steps))(*[keys[int(s)] for s in steps])
        ref = {k: Refresh(boots[k][0].h, float(boots[k][1])) for k in ("state", "inc_tm", "inc_cm")}
        h = _vp()
        check(load().fhe_ssm_decoder_create(ctx.h, n_layers, ref["state"], ref["inc_tm"], ref["inc_cm"], d_relin,
                                            d_conj, steps.ctypes.data, ptrs, len(steps), ctypes.byref(h)))
        self.h = h.value
        self._keep = (boots, steps, ptrs)

    def set_weights(self, W: dict) -> None:
        """W in the layout of rwkv_model.make_weights (first n_layers layers)"""
        for li in range(self.n_layers):
            for name in LAYER_WEIGHTS:
                self._set(name, li, W["layers"][li][name])
        for name in MODEL_WEIGHTS:
            self._set(name, -1, W[name])

    def _set(self, name: str, layer: int, arr) -> None:
        a = np.ascontiguousarray(np.asarray(arr, dtype=np.float64)).reshape(-1)
        check(load().fhe_ssm_decoder_set_weight(self.h, name.encode(), layer, a.ctypes.data, a.size))

    def step(self, d_x: int, level: int, scale: float):
        """one decode step; returns (DeviceBuffer [2][level][N] holding the output, its level, its scale)"""
        out = self.ckks.DeviceBuffer(2 * level * (1 << 16) * 8)
        lv, sc = _u32(), ctypes.c_double()
        check(load().fhe_ssm_decoder_step(self.h, d_x, level, scale, out.ptr, ctypes.byref(lv), ctypes.byref(sc)))
        return out, lv.value, sc.value

    def reset(self) -> None:
        """drop the carried state: the next step starts cold"""
        check(load().fhe_ssm_decoder_reset(self.h))

    def store_save(self, path: str) -> int:
        """write the matvecs encoded so far to a store file; returns their number"""
        n = _u64()
        check(load().fhe_ssm_decoder_store_save(self.h, path.encode(), ctypes.byref(n)))
        return n.value

    def store_load(self, path: str) -> int:
        """take the matvecs from a store file (stamp-checked) instead of encoding them; before the first step"""
        n = _u64()
        check(load().fhe_ssm_decoder_store_load(self.h, path.encode(), ctypes.byref(n)))
        return n.value

    def memory(self) -> dict:
        """bytes the decoder holds: elementwise plaintexts, diagonal staging/expansion buffers, ciphertext pool (all
        it has allocated), carried state (part of the pool) on the device; the previous state's copy and the matvec
        coefficients in pinned host memory"""
        v = np.zeros(6, dtype=np.uint64)
        check(load().fhe_ssm_decoder_memory(self.h, v.ctypes.data, 6))
        return {"plaintexts": int(v[0]), "diagonal_buffers": int(v[1]), "ciphertext_pool": int(v[2]),
                "carried_state": int(v[3]), "host_state_copy": int(v[4]), "host_matvec_store": int(v[5])}

    def serve(self, directory: str, timeout_sec: int = 3600, stateful: bool = True, log_fd: int = -1,
              poll_ms: int = 200, first_req: int = 0) -> dict:
        """the serve-directory protocol with this decoder's step as the handler, until `stop` or idle timeout"""
        opts = ServeOpts(timeout_sec, poll_ms, 1 if stateful else 0, log_fd, first_req)
        rep = ServeReport()
        check(load().fhe_ssm_decoder_serve(self.h, directory.encode(), ctypes.byref(opts), ctypes.byref(rep)))
        return _report(rep)

    @property
    def bootstraps(self) -> int:
        n = ctypes.c_uint64()
        check(load().fhe_ssm_decoder_stats(self.h, ctypes.byref(n)))
        return n.value

    def close(self) -> None:
        if self.h:
            load().fhe_ssm_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _report(rep: ServeReport) -> dict:
    return {"served": rep.served, "failed": rep.failed, "next_req": rep.next_req,
            "exit_reason": "stop" if rep.exit_reason == 0 else "idleTimeout"}


def serve_dir(directory: str, handler, timeout_sec: int = 3600, stateful: bool = True, log_fd: int = -1,
              poll_ms: int = 200, first_req: int = 0) -> dict:
    """the serve-directory protocol loop (host only) with a Python handler
    handler(req, req_prefix, resp_prefix, meta: dict, reset: bool) -> None; an exception answers resp.N.error"""

    def cb(user, req, req_prefix, resp_prefix, meta_json, reset, err, err_cap):
        try:
            handler(int(req), req_prefix.decode(), resp_prefix.decode(), json.loads(meta_json.decode()), bool(reset))
            return 0
        except Exception as e:  # reported through the protocol's error marker and log line
            msg = (type(e).__name__ + ": " + str(e)).encode()[: max(0, err_cap - 1)] + b"\0"
            ctypes.memmove(err, msg, len(msg))
            return 1

    fn = ServeHandler(cb)
    opts = ServeOpts(timeout_sec, poll_ms, 1 if stateful else 0, log_fd, first_req)
    rep = ServeReport()
    check(load().fhe_ssm_serve_dir(directory.encode(), ctypes.byref(opts), fn, None, ctypes.byref(rep)))
    return _report(rep)


def meta_int(text: str, key: str, dflt: int = -1) -> int:
    return int(load().fhe_ssm_meta_int(text.encode(), key.encode(), dflt))


def from_backend(be, n_layers: int) -> NativeDecoder:
    """A native decoder over the same context, plans and keys as a decode_step.HEBackend."""
    return NativeDecoder(be.ckks, be.ctx, n_layers, be.boots, be.relin, be.conj_key, be.keys)


def client_encrypt_rows(ctx, d_pk: int, rows_path: str, tokens: int, lanes: int, d: int, dpad: int, level: int,
                        scale: float, seed: bytes) -> None:
    """the reference driver's --enc-in: rows_path (lanes x tokens x d float64, lane-major) -> rows_path.ct.<t> and
    rows_path.ct.meta, encrypted under the public key d_pk"""
    sd = (ctypes.c_uint8 * 32).from_buffer_copy(bytes(seed).ljust(32, b"\0")[:32])
    check(load().fhe_ssm_client_encrypt_rows(ctx.h, d_pk, rows_path.encode(), tokens, lanes, d, dpad, level, scale,
                                             sd))


def client_decrypt_logits(ctx, sk, in_prefix: str, head: np.ndarray, dpad: int) -> None:
    """the reference driver's --dec-out: in_prefix.meta + in_prefix.<t> -> in_prefix.logits.f64 (tokens x lanes rows
    of vocab float64) with head (vocab x d) applied to each lane's decrypted channels"""
    head = np.ascontiguousarray(head, dtype=np.float64)
    check(load().fhe_ssm_client_decrypt_logits(ctx.h, sk.h, in_prefix.encode(), head.ctypes.data, head.shape[0],
                                               head.shape[1], dpad))


# ---- the store file (base + journal), host only ---------------------------------------------------------------------
def _key7(key) -> np.ndarray:
    k = np.ascontiguousarray(np.asarray(key, dtype=np.int32))
    if k.shape != (7,):
        raise ValueError("a store key has 7 fields (layer, op, chunk, rowOff, diag, half, lvl)")
    return k


class Store:
    """An in-memory store of (7-field key -> uint64 words) entries, read from and written to the store file format."""

    def __init__(self):
        h = _vp()
        check(load().fhe_ssm_store_create(ctypes.byref(h)))
        self.h = h.value

    def put(self, key, words) -> None:
        k = _key7(key)
        w = np.ascontiguousarray(np.asarray(words, dtype=np.uint64))
        check(load().fhe_ssm_store_put(self.h, k.ctypes.data, w.ctypes.data if w.size else None, w.size))

    def __len__(self) -> int:
        n = _u64()
        check(load().fhe_ssm_store_count(self.h, ctypes.byref(n)))
        return n.value

    def keys(self) -> list:
        out = []
        for i in range(len(self)):
            k = np.zeros(7, dtype=np.int32)
            n = _u64()
            check(load().fhe_ssm_store_entry(self.h, i, k.ctypes.data, ctypes.byref(n)))
            out.append(tuple(int(x) for x in k))
        return out

    def get(self, key) -> np.ndarray:
        k = _key7(key)
        n = _u64()
        check(load().fhe_ssm_store_get(self.h, k.ctypes.data, None, 0, ctypes.byref(n)))
        w = np.zeros(n.value, dtype=np.uint64)
        check(load().fhe_ssm_store_get(self.h, k.ctypes.data, w.ctypes.data if w.size else None, w.size,
                                       ctypes.byref(n)))
        return w

    def save(self, path: str, stamp: str) -> None:
        check(load().fhe_ssm_store_save(self.h, path.encode(), stamp.encode()))

    def load(self, path: str, stamp=None, depth: int = 0, comp_cw: int = 0) -> int:
        n = _u64()
        check(load().fhe_ssm_store_load(self.h, path.encode(), stamp.encode() if stamp is not None else None, depth,
                                        comp_cw, ctypes.byref(n)))
        return n.value

    def load_journal(self, journal_path: str, depth: int = 0, comp_cw: int = 0) -> dict:
        g, d, b = _u64(), _u64(), _u64()
        check(load().fhe_ssm_store_load_journal(self.h, journal_path.encode(), depth, comp_cw, ctypes.byref(g),
                                                ctypes.byref(d), ctypes.byref(b)))
        return {"good": g.value, "duplicates": d.value, "dropped_bytes": b.value}

    def close(self) -> None:
        if self.h:
            load().fhe_ssm_store_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def store_append(journal_path: str, key, words) -> None:
    """one self-checksummed record appended to a store journal"""
    k = _key7(key)
    w = np.ascontiguousarray(np.asarray(words, dtype=np.uint64))
    check(load().fhe_ssm_store_append(journal_path.encode(), k.ctypes.data, w.ctypes.data if w.size else None, w.size))


def store_read_stamp(path: str) -> str:
    n = _u64()
    check(load().fhe_ssm_store_read_stamp(path.encode(), None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(n.value + 1)
    check(load().fhe_ssm_store_read_stamp(path.encode(), ctypes.cast(buf, _vp), n.value + 1, ctypes.byref(n)))
    return buf.value.decode()
