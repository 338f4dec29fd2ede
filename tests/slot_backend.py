"""Slot-vector simulator of the decode-step backend (test infrastructure).

Runs the encrypted driver's plan (fhe-ssm_amd/decode_step.py) on plain complex slot vectors: every primitive
does to the 32768 slot values what the engine does to the encrypted ones (rotations are np.roll, plaintext
products are slot-wise products, bootstrapping is the identity), with the same level bookkeeping.  It checks
the packing algebra (diagonals and their pre-rotation, masks, the WKV diagonal layout, the state packing)
against the float64 reference model without any encryption noise.
"""
from __future__ import annotations

import numpy as np

from engine_loader import load_module

M = load_module("rwkv_model")
DS = load_module("decode_step")

SLOTS = 1 << 15


class SimCt:
    __slots__ = ("v", "level", "scale")

    def __init__(self, v, level, scale=1.0):
        self.v = np.asarray(v, dtype=np.complex128).reshape(-1, SLOTS)
        self.level, self.scale = level, scale

    @property
    def B(self):
        return self.v.shape[0]


class SimPt:
    def __init__(self, vecs, level):
        self.vecs, self.level = vecs, level


def tile(vec1024):
    return np.tile(vec1024, SLOTS // len(vec1024))


class SlotBackend(DS.Backend):
    def __init__(self, top_level=16):
        self.top_level = top_level
        self.log = []

    def S(self, level):
        return 1.0

    def _check(self, *cts, level=None):
        for c in cts:
            assert c.level >= 1, "level exhausted"
            if level is not None:
                assert c.level == level, (c.level, level)

    # client
    def encrypt(self, sk, slots, level, seed=None, index=0):
        return SimCt(slots, level)

    def decrypt(self, sk, ct, b=0):
        return ct.v[b].copy()

    # plaintexts
    def encode_periodic(self, vecs, level):
        return SimPt(np.asarray(vecs).reshape(-1, M.DPAD), level)

    def encode_matvec(self, diags, level):
        nb = M.MV_SPAN // diags.shape[1]
        return {"d": diags, "level": level, "n_out": diags.shape[0], "ng": diags.shape[1], "nb": nb,
                "n_in": diags.shape[2] // nb}

    # bookkeeping
    def zeros(self, B, level):
        return SimCt(np.zeros((B, SLOTS)), level)

    def item(self, a, i):
        return SimCt(a.v[i], a.level, a.scale)

    def slice(self, a, i0, i1):
        return SimCt(a.v[i0:i1], a.level, a.scale)

    def concat(self, parts):
        assert len({(p.level, p.scale) for p in parts}) == 1
        return SimCt(np.concatenate([p.v for p in parts]), parts[0].level, parts[0].scale)

    def halve(self, a):
        return SimCt(a.v / 2, a.level, a.scale * 2)

    # primitives
    def _adjust(self, a, lt, coeff=1.0, const=0.0):
        assert a.level >= lt + 1 and lt >= 1, (a.level, lt)
        return SimCt(coeff * a.v + const, lt)

    def at_neg(self, a, lt):
        return self._adjust(a, lt, -1.0)

    def _lin_scalar(self, terms, coeffs, const, lt):
        assert lt >= 1 and all(t.level >= lt + 1 for t in terms)
        return SimCt(sum(c * t.v for c, t in zip(coeffs, terms)) + const, lt)

    def _lin_int(self, terms, coeffs):
        lv, sc = terms[0].level, terms[0].scale
        assert all(t.level == lv and t.scale == sc for t in terms)
        return SimCt(sum(c * t.v for c, t in zip(coeffs, terms)), lv, sc)

    def _mult_sum(self, pairs, level):
        assert level >= 2
        out = np.zeros((len(pairs), SLOTS), dtype=np.complex128)
        sc = None
        for b, item in enumerate(pairs):
            for (a, i, c, j) in item:
                self._check(a, c, level=level)
                s = a.scale * c.scale
                assert sc is None or sc == s
                sc = s
                out[b] += a.v[i] * c.v[j]
        return SimCt(out, level - 1, sc)

    def rotate(self, a, k):
        return SimCt(np.roll(a.v, -k, axis=1), a.level, a.scale)

    def rotate_sum(self, a, steps):
        return SimCt(a.v + sum(np.roll(a.v, -k, axis=1) for k in steps), a.level, a.scale)

    def mul_pt(self, a, pt):
        assert pt.level == a.level and pt.vecs.shape[0] == 1 and a.level >= 2
        return SimCt(a.v * tile(pt.vecs[0])[None, :], a.level - 1, a.scale)

    def rotate_masked(self, a, pts, n_sets):
        assert a.B == 1 and pts.level == a.level and a.level >= 2
        T = M.WKV_T
        m = pts.vecs.reshape(n_sets, T, 2, M.DPAD)
        out = np.zeros((n_sets * T, SLOTS), dtype=np.complex128)
        for t in range(T):
            lo = np.roll(a.v[0], -M.WKV_LO[t])
            hi = np.roll(a.v[0], -M.WKV_HI[t])
            for s in range(n_sets):
                out[s * T + t] = tile(m[s, t, 0]) * lo + tile(m[s, t, 1]) * hi
        return SimCt(out, a.level - 1, a.scale)

    def matvec(self, inputs, h):
        lv = inputs[0].level
        assert all(x.level == lv and x.B == 1 for x in inputs) and h["level"] == lv and lv >= 2
        assert len(inputs) == h["n_in"]
        d = h["d"]
        babies = [np.roll(x.v[0], -b) for x in inputs for b in M.mv_babies(h["nb"])]
        out = np.zeros((h["n_out"], SLOTS), dtype=np.complex128)
        for o in range(h["n_out"]):
            for gi, G in enumerate(M.mv_giants(h["nb"])):
                acc = np.zeros(SLOTS, dtype=np.complex128)
                for j, bv in enumerate(babies):
                    if np.any(d[o, gi, j]):
                        acc += tile(d[o, gi, j]) * bv
                out[o] += np.roll(acc, -G)
        return SimCt(out, lv - 1, inputs[0].scale)

    def mul_i(self, a, sign):
        return SimCt(1j * sign * a.v, a.level, a.scale)

    def conj(self, a):
        return SimCt(np.conj(a.v), a.level, a.scale)

    def bootstrap(self, a, kind="state"):
        assert a.level >= 2
        self.log.append(("bootstrap", kind, a.B, a.level))
        return SimCt(a.v, self.top_level)
