"""The config-5 encrypted decode step: the caller that drives the engine's C ABI the way the reference's
served step drives FIDESlib (hpc_gpu_port/gpu_real_model.cu:4674-5300: per layer rmsnorm, token shift,
matvecBatch with shared babies, scan, gate, output projection, residual, channel mix; refresh/boot policy
:2535-2599).  The model itself is described in rwkv_model.py.

The step is written against a small backend interface (Backend below): the level/scale rules live here,
the primitives in the backend.  HEBackend runs them on the GPU through ckks.py; the tests also run the same
plan on a slot-vector simulator to check the packing algebra without encryption.

Level rules (OpenFHE FLEXIBLEAUTO semantics, gpu_real_model.cu:1156): every ciphertext at level l carries
the canonical scale S(l) of the bootstrapping plan (S(l-1) = S(l)^2 / q_{l-1}), except transiently the
unpacked state (2 S(l)).  An operand above the level of its partner is brought down by a scalar
multiplication that lands on the canonical scale (one rescale); products then land on S(l-1).
Plaintexts applied at level l are encoded at scale S(l), which keeps the product canonical.

Refresh policy: the residual stream x never leaves the top level.  Each block's increment (o from the time
mix, f from the channel mix) comes out at a low level, is bootstrapped on its own and added to x there, so
x itself is never bootstrapped: the sine of EvalMod shrinks large coefficients slightly (a coherent
relative error ~(2 pi m / q0)^2 / 6), and the increments are ~5-100x smaller than x.  Each increment kind
has its own bootstrapping plan whose input scale suits its magnitude (more signal over EvalMod's noise).
The carried WKV state is bootstrapped once per layer: its 64 diagonal ciphertexts are packed 4 -> 3 into the
lanes' unused channels (768..1023), the 48 packed two per complex ciphertext, and unpacked with one conjugation
and three masked rotations.  The WKV readout y and the per-head bonus coefficient are bootstrapped together
mid-mix: the per-head GroupNorm of y needs more levels than the scan leaves.  28 bootstraps per layer.
"""
from __future__ import annotations

import numpy as np

import rwkv_model as M


class Backend:
    """Level/scale rules over backend primitives.  Ciphertext handles expose .B (batch), .level, .scale."""

    # -- primitives a backend provides ------------------------------------------------------------
    def S(self, level):  # canonical scale
        raise NotImplementedError

    def _adjust(self, a, lt, coeff=1.0, const=0.0):  # scalar mode: a at level >= lt + 1 -> lt, canonical
        raise NotImplementedError

    def _lin_scalar(self, terms, coeffs, const, lt):
        raise NotImplementedError

    def _lin_int(self, terms, coeffs):  # same level and scale, integer coefficients, no level
        raise NotImplementedError

    def _mult_sum(self, pairs, level):  # pairs[b] = [(ct, idx, ct, idx), ...], all operands at level
        raise NotImplementedError

    # -- rules -------------------------------------------------------------------------------------
    def at(self, a, lt):
        """a at level lt with the canonical scale"""
        if a.level == lt and self._canonical(a):
            return a
        if a.level < lt + 1:
            raise ValueError(f"cannot bring a level-{a.level} ciphertext to level {lt}")
        return self._adjust(a, lt)

    def _canonical(self, a):
        return abs(a.scale / self.S(a.level) - 1.0) < 1e-9

    def add(self, a, b, sign=1):
        m = min(a.level, b.level)
        a2, b2 = self._align_pair(a, b, m)
        return self._lin_int([a2, b2], [1, sign])

    def _align_pair(self, a, b, m):
        a2 = a if (a.level == m and (self._canonical(a) or b.level == m)) else self.at(a, m)
        b2 = b if (b.level == m and (self._canonical(b) or a.level == m)) else self.at(b, m)
        if abs(a2.scale / b2.scale - 1.0) > 1e-9:
            # same level, different scales: both go down one level onto the canonical scale
            a2, b2 = self.at(a2, m - 1), self.at(b2, m - 1)
        return a2, b2

    def lin(self, terms, coeffs, const=0.0, lt=None):
        """sum_t c_t x_t + const, scalar coefficients: one level below the lowest term (or lt)"""
        lo = min(t.level for t in terms)
        lt = lo - 1 if lt is None else lt
        return self._lin_scalar(terms, coeffs, const, lt)

    def mul(self, a, b):
        """a (.) b with relinearization and rescale; a batch of 1 broadcasts against a batch"""
        B = max(a.B, b.B)
        m = min(a.level, b.level)
        a2 = self.at(a, m) if a.level > m else a
        b2 = self.at(b, m) if b.level > m else b
        pairs = [[(a2, i % a2.B, b2, i % b2.B)] for i in range(B)]
        return self._mult_sum(pairs, m)

    def mult_sum(self, pairs):
        """pairs[b] = [(ct, idx, ct, idx), ...] summed then relinearized and rescaled; operands are brought
        to the lowest level among them first"""
        m = min(min(p[0].level, p[2].level) for item in pairs for p in item)
        cache = {}

        def lower(c):
            key = id(c)
            if key not in cache:
                cache[key] = c if (c.level == m and self._canonical(c)) else self.at(c, m)
            return cache[key]

        pairs2 = [[(lower(a), i, lower(b), j) for (a, i, b, j) in item] for item in pairs]
        return self._mult_sum(pairs2, m)

    def poly3(self, z, c):
        """c0 + c1 z + c2 z^2 + c3 z^3 in depth 2 (z^2 (c3 z + c2) + (c1 z + c0))"""
        m = z.level
        z2 = self.mul(z, z)
        u = self.lin([z], [c[3]], c[2], lt=m - 1)
        t = self.mul(z2, u)
        v = self.lin([z], [c[1]], c[0], lt=m - 2)
        return self.add(t, v)


class DecodeStep:
    """One encrypted decode step over all layers; the WKV state and token-shift carries persist between
    calls (the reference's stateful serve loop, gpu_real_model.cu:4674-4720)."""

    def __init__(self, be: Backend, weights: dict, n_layers: int | None = None):
        self.be = be
        self.W = weights
        self.n_layers = len(weights["layers"]) if n_layers is None else n_layers
        self.pt = {}        # (name, level) -> backend plaintext handle
        self.state = None   # per layer: {"D": [(ct batch, index) of D_t] * 64, "xp_t": ct, "xp_c": ct}
        self.stats = {"bootstraps": 0}

    # -- plaintexts (encoded on first use at the level they are applied) ----------------------------
    def _vec_pt(self, name, level, vecs):
        key = (name, level)
        if key not in self.pt:
            self.pt[key] = self.be.encode_periodic(np.asarray(vecs, dtype=np.float64).reshape(-1, M.DPAD), level)
        return self.pt[key]

    def _mv_pt(self, name, level, blocks_fn):
        key = (name, level)
        if key not in self.pt:
            blocks = blocks_fn()
            self.pt[key] = self.be.encode_matvec(M.matvec_diagonals(blocks), level)
        return self.pt[key]

    # -- blocks --------------------------------------------------------------------------------------
    def _norm(self, x, pcoef, tag):
        """x * p(mean(x^2)) per lane"""
        be = self.be
        s = be.mul(x, x)
        for w in M.NORM_UP:
            s = be.rotate_sum(s, w)
        s = be.mul_pt(s, self._vec_pt("lane_start", s.level, M.lane_start_mask(1.0 / M.D)))
        for w in M.NORM_DOWN:
            s = be.rotate_sum(s, w)
        n = be.poly3(s, pcoef)
        return be.mul(x, n)

    def _boot(self, x, kind):
        self.stats["bootstraps"] += x.B
        return self.be.bootstrap(x, kind)

    def _head_sum(self, x, scale):
        """every head's sum of x (times scale), broadcast over the head's 64 channels: a rotate-and-add window of 64
        (slot h*64 of a lane then holds head h's sum), mask the head starts (times scale), broadcast back"""
        be = self.be
        s = x
        for w in M.HEAD_UP:
            s = be.rotate_sum(s, w)
        s = be.mul_pt(s, self._vec_pt(f"head_start{scale!r}", s.level, M.head_start_mask(scale)))
        for w in M.HEAD_DOWN:
            s = be.rotate_sum(s, w)
        return s

    def _time_mix(self, li, x, st, v0):
        """the time-mix increment o (x + o is the layer's residual) and the first layer's value v0 (the value
        residual of the later layers mixes toward it)"""
        be, L = self.be, self.W["layers"][li]
        xn = self._norm(x, L["p_n1"], "n1")
        xp = st["xp_t"]
        lv = min(xn.level, xp.level)
        first = v0 is None

        def tm_blocks():
            def mix(Wm, mu):
                return [Wm * (L["g1"] * (1 - mu))[None, :], Wm * (L["g1"] * mu)[None, :]]
            out = [mix(L["W_" + m], L["mu_" + m]) for m in M.MIX_NAMES]
            out.append(mix(L["W_k"] * L["k_k"][:, None], L["mu_k"]))      # kk = k_k (.) k
            if not first:
                out.append(mix(L["W_vg"], L["mu_v"]))                    # the value gate's argument
            return out

        proj = be.matvec([be.at(xn, lv), be.at(xp, lv)], self._mv_pt(f"tm{li}", lv, tm_blocks))
        r, k, v, zw, za, zg, kk = (be.item(proj, i) for i in range(7))
        w = be.poly3(zw, L["p_w"])
        a = be.poly3(za, L["p_a"])
        g = be.poly3(zg, L["p_g"])
        if first:
            v0 = v
        else:  # value residual: v + (v0 - v) p_v(W_vg u_v)
            gate = be.poly3(be.item(proj, 7), L["p_v"])
            v = be.add(v, be.mul(be.add(v0, v, -1), gate))
        # the per-head L2 norm of kk enters only the removal term, as its square:
        # (S kh)(kh a)^T = n^2 (S kk)(kk a)^T with kh = n kk, n = p_kn(|kk_h|^2)
        nk = be.poly3(self._head_sum(be.mul(kk, kk), 1.0), L["p_kn"])
        n2 = be.mul(nk, nk)
        masks = M.wkv_masks()
        # k's masked rotations: rot64_t(kk) = rot64_t(k) k_k, and the key update k' = k (1 - k_a) + (k a) k_a
        KX = be.rotate_masked(k, self._vec_pt(f"mask_k{li}", k.level, np.concatenate(
            [M.wkv_masks(L["k_k"]), M.wkv_masks(1 - L["k_a"])])), 2)
        KK_t, K1_t = be.slice(KX, 0, 64), be.slice(KX, 64, 128)
        ka = be.mul(k, a)
        KB = be.rotate_masked(ka, self._vec_pt(f"mask_ka{li}", ka.level, np.concatenate(
            [M.wkv_masks(L["k_k"]), M.wkv_masks(L["k_a"])])), 2)
        B_t, K2_t = be.slice(KB, 0, 64), be.slice(KB, 64, 128)
        R_t = be.rotate_masked(r, self._vec_pt("mask", r.level, masks), 1)
        W_t = be.rotate_masked(w, self._vec_pt("mask", w.level, masks), 1)
        D = st["D"]  # (batch, index) of D_t
        T = M.WKV_T
        sa = be.mult_sum([[(D[t][0], D[t][1], KK_t, t) for t in range(T)]])
        nsa = be.mul(be.at_neg(sa, n2.level), n2)
        Dn = be.mult_sum([[(D[t][0], D[t][1], W_t, t), (nsa, 0, B_t, t), (v, 0, K1_t, t), (v, 0, K2_t, t)]
                          for t in range(T)])
        y = be.mult_sum([[(Dn, t, R_t, t) for t in range(T)]])
        # the bonus coefficient per head: sum of r k' r_k = (r k) (1 - k_a) r_k + (r ka) k_a r_k
        rk = be.add(be.mul_pt(be.mul(r, k), self._vec_pt(f"rk1_{li}", r.level - 1, M.periodic((1 - L["k_a"]) * L["r_k"]))),
                    be.mul_pt(be.mul(r, ka), self._vec_pt(f"rk2_{li}", ka.level - 1, M.periodic(L["k_a"] * L["r_k"]))))
        sb = self._head_sum(rk, 1.0)
        # y and the bonus coefficient are bootstrapped together (GroupNorm needs more levels than are left)
        m = min(y.level, sb.level)
        yb = self._boot(be.concat([be.at(y, m), be.at(sb, m)]), "state")
        Y, SB = be.item(yb, 0), be.item(yb, 1)
        # GroupNorm per head: mean and mean of squares from one batch of rotations, var = E[y^2] - mean^2
        mom = self._head_sum(be.concat([be.at(Y, Y.level - 1), be.mul(Y, Y)]), 1.0 / M.HS)
        mu, ey2 = be.item(mom, 0), be.item(mom, 1)
        var = be.add(ey2, be.mul(mu, mu), -1)
        yn = be.mul(be.add(Y, mu, -1), be.poly3(var, L["p_gn"]))
        yl = be.mul_pt(yn, self._vec_pt(f"ln_w{li}", yn.level, M.periodic(L["ln_w"])))
        y3 = be.add(yl, be.mul(SB, v))
        # (y3 + ln_b) g: ln_b enters as ln_b (.) g
        yg = be.add(be.mul(y3, g), be.mul_pt(g, self._vec_pt(f"ln_b{li}", g.level, M.periodic(L["ln_b"]))))
        o = be.matvec([yg], self._mv_pt(f"wo{li}", yg.level, lambda: [[L["W_o"]]]))
        st["xp_t"] = xn
        st["Dn"] = Dn
        return o, v0

    def _channel_mix(self, li, x, st):
        """the channel-mix increment f"""
        be, L = self.be, self.W["layers"][li]
        xn2 = self._norm(x, L["p_n2"], "n2")
        xp = st["xp_c"]
        lv = min(xn2.level, xp.level)

        def ck_blocks():
            a = (L["g2"] * (1 - L["mu_c"]))[None, :]
            b = (L["g2"] * L["mu_c"])[None, :]
            return [[L["W_ck"][o * M.D:(o + 1) * M.D] * a, L["W_ck"][o * M.D:(o + 1) * M.D] * b] for o in range(4)]

        hs = be.matvec([be.at(xn2, lv), be.at(xp, lv)], self._mv_pt(f"ck{li}", lv, ck_blocks))
        h = be.poly3(hs, L["p_h"])
        f = be.matvec([be.item(h, i) for i in range(4)],
                      self._mv_pt(f"cv{li}", h.level, lambda: [[L["W_cv"][:, i * M.D:(i + 1) * M.D] for i in range(4)]]))
        st["xp_c"] = xn2
        return f

    def _refresh_state(self, st):
        """bootstrap the new state once: the 64 diagonals packed 4 -> 3 into the lanes' unused channels, the 48
        packed two per complex ciphertext (Q_j + i Q'_j), 24 bootstraps, unpacked with one conjugation and three
        masked rotations"""
        be = self.be
        Dn = st.pop("Dn")
        q = M.WKV_T // 4
        quarter = [be.slice(Dn, k * q, (k + 1) * q) for k in range(4)]
        # pieces of the fourth quarter into the gaps of the first three
        packed3 = []
        for p, g in enumerate(M.GAP_SHIFT):
            m = self._vec_pt(f"gap_in{p}", quarter[3].level, M.channel_range_mask(256 * p, 256 * (p + 1)))
            packed3.append(be.add(quarter[p], be.rotate(be.mul_pt(quarter[3], m), -g)))
        A, B, C = packed3
        h = q // 2
        pk = be.concat([be.add(A, be.mul_i(B, 1)),
                        be.add(be.slice(C, 0, h), be.mul_i(be.slice(C, h, q), 1))])
        self.stats["bootstraps"] += pk.B
        P = be.bootstrap(pk, "state")
        Cj = be.conj(P)
        re2 = be.halve(be.add(P, Cj))                   # 2 Re: A, C[0:8]; declared at twice the scale
        im2 = be.halve(be.mul_i(be.add(Cj, P, -1), 1))  # i (conj - P) = 2 Im: B, C[8:16]
        A2, B2 = be.slice(re2, 0, q), be.slice(im2, 0, q)
        C2 = be.concat([be.slice(re2, q, q + h), be.slice(im2, q, q + h)])
        # the fourth quarter back out of the gaps
        terms = []
        for p, (src, g) in enumerate(zip((A2, B2, C2), M.GAP_SHIFT)):
            m = self._vec_pt(f"gap_out{p}", src.level, M.channel_range_mask(256 * p, 256 * (p + 1)))
            terms.append(be.mul_pt(be.rotate(src, g), m))
        D4 = be._lin_int(terms, [1, 1, 1])
        st["D"] = [(A2, t) for t in range(q)] + [(B2, t) for t in range(q)] + [(C2, t) for t in range(q)] + \
                  [(D4, t) for t in range(q)]

    def state_diagonals(self, li):
        """(ciphertext batch, index) of D_t, t = 0..63, for layer li"""
        return self.state[li]["D"]

    def cold_state(self):
        be = self.be
        lt = be.top_level
        out = []
        for _ in range(self.n_layers):
            z = be.zeros(M.WKV_T, lt)
            out.append({"D": [(z, t) for t in range(M.WKV_T)], "xp_t": be.zeros(1, lt), "xp_c": be.zeros(1, lt)})
        return out

    def __call__(self, x):
        """x: ciphertext of the lanes' embeddings; returns the ciphertext of the output-normed hidden state"""
        if self.state is None:
            self.state = self.cold_state()
        be = self.be
        v0 = None
        for li in range(self.n_layers):
            st = self.state[li]
            o, v0 = self._time_mix(li, x, st, v0)
            x = be.add(x, self._boot(o, "inc_tm"))
            self._refresh_state(st)
            x = be.add(x, self._boot(self._channel_mix(li, x, st), "inc_cm"))
        xo = self._norm(x, self.W["p_o"], "out")
        return self.be.mul_pt(xo, self._vec_pt("g_o", xo.level, M.periodic(self.W["g_o"])))


# ======================================================================================== GPU backend
class HECt:
    """a batch of B ciphertexts [B][2][level][N] in a pooled device buffer (or a view into another's)"""
    __slots__ = ("buf", "off", "B", "level", "scale", "_pool", "base")

    def __init__(self, buf, B, level, scale, off=0, pool=None, base=None):
        self.buf, self.B, self.level, self.scale, self.off, self._pool = buf, B, level, scale, off, pool
        self.base = base  # a view keeps the ciphertext it points into alive

    def ptr(self, b=0):
        return self.buf.ptr + self.off + b * 2 * self.level * HEBackend.N * 8

    @property
    def nbytes(self):
        return self.B * 2 * self.level * HEBackend.N * 8

    def __del__(self):
        if self._pool is not None:
            self._pool.put(self.buf)


class _Pool:
    """free lists of device buffers by size (a decode step allocates the same shapes every layer)"""

    def __init__(self, ckks):
        self.ckks = ckks
        self.free = {}

    def get(self, nbytes):
        lst = self.free.get(nbytes)
        if lst:
            return lst.pop()
        return self.ckks.DeviceBuffer(nbytes)

    def put(self, buf):
        self.free.setdefault(buf.nbytes, []).append(buf)


class HEBackend(Backend):
    """Decode-step primitives on the GPU engine (through ckks.py and the C ABI)."""
    N = 1 << 16

    def __init__(self, ckks, ctx, boots: dict, relin, conj, keys: dict):
        """boots: refresh kind -> (bootstrapping plan, its input scale); kind "state" must be present"""
        self.ckks, self.ctx, self.boots = ckks, ctx, boots
        boot = boots["state"][0]
        self.relin, self.conj_key, self.keys = relin, conj, keys
        self.top_level = boot.out_level
        self.pool = _Pool(ckks)
        self._S = {l: boot.scale(l) for l in range(1, boot.out_level + 1)}
        self.moduli = ctx.moduli
        self.boot_batch = 16  # ciphertexts per batched bootstrap (bounds its workspace)
        self.boot_keys = {k: {s: keys[s] for s in b.steps} for k, (b, _) in boots.items()}

    def S(self, level):
        return self._S[level]

    def _new(self, B, level, scale):
        return HECt(self.pool.get(B * 2 * level * self.N * 8), B, level, scale, pool=self.pool)

    # -- client side ---------------------------------------------------------------------------------
    def encrypt(self, sk, slots, level, seed=b"x" * 32, index=0):
        pt = self.ckks.DeviceBuffer(level * self.N * 8)
        self.ctx.encode(slots, level, self.S(level), pt.ptr)
        ct = self._new(1, level, self.S(level))
        self.ctx.encrypt(sk, pt.ptr, level, seed, index, ct.ptr())
        return ct

    def decrypt(self, sk, ct, b=0):
        return self.ctx.decrypt(sk, ct.ptr(b), ct.level, ct.scale, 1 << 15, complex_out=True)

    # -- plaintexts ----------------------------------------------------------------------------------
    def encode_periodic(self, vecs, level):
        vecs = np.atleast_2d(vecs)
        n = vecs.shape[0]
        buf = self.ckks.DeviceBuffer(n * level * (self.N >> M.LOG_REP) * 8)
        self.ctx.encode_periodic(vecs, level, self.S(level), buf.ptr)
        return buf

    def encode_matvec(self, diags, level):
        n_out, ng, nbt = diags.shape[:3]
        flat = diags.reshape(-1, M.DPAD)
        buf = self.ckks.DeviceBuffer(flat.shape[0] * level * (self.N >> M.LOG_REP) * 8)
        step = 4096
        per = level * (self.N >> M.LOG_REP) * 8
        for s in range(0, flat.shape[0], step):
            chunk = flat[s:s + step]
            self.ctx.encode_periodic(chunk, level, self.S(level), buf.ptr + s * per)
        nb = M.MV_SPAN // ng
        return {"buf": buf, "n_out": n_out, "ng": ng, "nb": nb, "n_in": nbt // nb}

    # -- ciphertext bookkeeping ----------------------------------------------------------------------
    def zeros(self, B, level):
        ct = self._new(B, level, self.S(level))
        ct.buf.upload(np.zeros(ct.nbytes // 8, dtype=np.uint64))
        return ct

    def item(self, a, i):
        return HECt(a.buf, 1, a.level, a.scale, off=a.off + i * 2 * a.level * self.N * 8, base=a)

    def slice(self, a, i0, i1):
        return HECt(a.buf, i1 - i0, a.level, a.scale, off=a.off + i0 * 2 * a.level * self.N * 8, base=a)

    def concat(self, parts):
        """the parts side by side in one batch (same level; scales equal to 1e-9, the rule add() applies)"""
        lv, sc = parts[0].level, parts[0].scale
        out = self._new(sum(p.B for p in parts), lv, sc)
        o = 0
        for p in parts:
            assert p.level == lv and abs(p.scale / sc - 1.0) < 1e-9
            self.ctx.eval_lincomb(p.B, [p.ptr()], [lv], [1.0], None, sc, 0.0, lv, True, out.ptr(o))
            o += p.B
        return out

    def halve(self, a):
        """the same ciphertext declared at twice the scale (the value halves): no arithmetic"""
        a.scale *= 2.0
        return a

    # -- primitives ----------------------------------------------------------------------------------
    def _adjust(self, a, lt, coeff=1.0, const=0.0):
        out = self._new(a.B, lt, self.S(lt))
        self.ctx.eval_lincomb(a.B, [a.ptr()], [a.level], [coeff], [a.scale], self.S(lt), const, lt, False,
                              out.ptr())
        return out

    def at_neg(self, a, lt):
        return self._adjust(a, lt, -1.0)

    def _lin_scalar(self, terms, coeffs, const, lt):
        B = terms[0].B
        out = self._new(B, lt, self.S(lt))
        self.ctx.eval_lincomb(B, [t.ptr() for t in terms], [t.level for t in terms], list(coeffs),
                              [t.scale for t in terms], self.S(lt), const, lt, False, out.ptr())
        return out

    def _lin_int(self, terms, coeffs):
        B, lv, sc = terms[0].B, terms[0].level, terms[0].scale
        out = self._new(B, lv, sc)
        self.ctx.eval_lincomb(B, [t.ptr() for t in terms], [lv] * len(terms), [float(c) for c in coeffs], None, sc,
                              0.0, lv, True, out.ptr())
        return out

    def _mult_sum(self, pairs, level):
        B = len(pairs)
        a0, _, b0, _ = pairs[0][0]
        scale = a0.scale * b0.scale / self.moduli[level - 1]
        out = self._new(B, level - 1, scale)
        ptrs = [[(a.ptr(i), b.ptr(j)) for (a, i, b, j) in item] for item in pairs]
        self.ctx.eval_mult_sum(ptrs, level, self.relin, out.ptr(), rescale=True)
        return out

    def rotate(self, a, k):
        out = self._new(a.B, a.level, a.scale)
        self.ctx.eval_rotate(a.ptr(), a.B, a.level, k, self.keys[k], out.ptr())
        return out

    def rotate_sum(self, a, steps):
        out = self._new(a.B, a.level, a.scale)
        self.ctx.eval_rotate_sum(a.ptr(), a.B, a.level, steps, [self.keys[k] for k in steps], out.ptr())
        return out

    def mul_pt(self, a, pt):
        tmp = self._new(a.B, a.level, a.scale)
        self.ctx.eval_mult_plain_ex(a.ptr(), a.B, a.level, pt.ptr, M.LOG_REP, tmp.ptr(), pt_shared=True)
        out = self._new(a.B, a.level - 1, a.scale * self.S(a.level) / self.moduli[a.level - 1])
        self.ctx.rescale(tmp.ptr(), 2 * a.B, a.level, out.ptr())
        return out

    def rotate_masked(self, a, pts, n_sets):
        assert a.B == 1
        T = M.WKV_T
        out = self._new(n_sets * T, a.level - 1, a.scale * self.S(a.level) / self.moduli[a.level - 1])
        self.ctx.eval_rotate_masked(a.ptr(), a.level, M.WKV_LO, [self.keys.get(s) for s in M.WKV_LO], M.WKV_HI,
                                    [self.keys.get(s) for s in M.WKV_HI], n_sets, pts.ptr, M.LOG_REP, out.ptr())
        return out

    def matvec(self, inputs, h):
        lv = inputs[0].level
        assert all(x.level == lv and x.B == 1 for x in inputs) and len(inputs) == h["n_in"]
        out = self._new(h["n_out"], lv - 1, inputs[0].scale * self.S(lv) / self.moduli[lv - 1])
        bs, gs = M.mv_babies(h["nb"]), M.mv_giants(h["nb"])
        self.ctx.linear_transform_multi([x.ptr() for x in inputs], lv, h["buf"].ptr, M.LOG_REP, bs,
                                        [self.keys.get(s) for s in bs], gs, [self.keys.get(s) for s in gs],
                                        h["n_out"], True, out.ptr())
        return out

    def mul_i(self, a, sign):
        out = self._new(a.B, a.level, a.scale)
        self.ctx.eval_mul_i(a.ptr(), 2 * a.B, a.level, sign, out.ptr())
        return out

    def conj(self, a):
        out = self._new(a.B, a.level, a.scale)
        self.ctx.eval_automorphism_ks(a.ptr(), a.B, a.level, 2 * self.N - 1, self.conj_key, out.ptr())
        return out

    def bootstrap(self, a, kind="state"):
        boot, in_scale = self.boots.get(kind, self.boots["state"])
        keys = self.boot_keys.get(kind, self.boot_keys["state"])
        lo = self.at_scale(a, 1, in_scale)
        out = self._new(a.B, self.top_level, self.S(self.top_level))
        # passes of equal size (24 -> 12 + 12): one buffer shape in the bootstrap's pool
        n_pass = -(-a.B // self.boot_batch)
        per = -(-a.B // n_pass)
        for b0 in range(0, a.B, per):
            nb = min(per, a.B - b0)
            boot.run_many(lo.ptr(b0), nb, self.relin, self.conj_key, keys, out.ptr(b0))
        return out

    def at_scale(self, a, lt, scale):
        out = self._new(a.B, lt, scale)
        self.ctx.eval_lincomb(a.B, [a.ptr()], [a.level], [1.0], [a.scale], scale, 0.0, lt, False, out.ptr())
        return out


# ======================================================================================== set-up
def _is_prime(n: int) -> bool:
    """deterministic Miller-Rabin for n < 2^64"""
    if n < 2:
        return False
    small = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37)
    for p in small:
        if n % p == 0:
            return n == p
    d, r = n - 1, 0
    while d % 2 == 0:
        d //= 2
        r += 1
    for a in small:
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(r - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def _nearest_ntt_prime(target: float, used: set, two_n: int = 1 << 17) -> int:
    """the prime q = 1 mod 2N nearest to target that is not in used"""
    k0 = int(round((target - 1) / two_n))
    for d in range(0, 1 << 20):
        for k in ((k0 + d, k0 - d) if d else (k0,)):
            q = k * two_n + 1
            if q > 1 and q not in used and _is_prime(q):
                return q
    raise ValueError("no prime found")


def config5_moduli(ckks, log_scale: int = 40, n_scaling: int = 28):
    """The config-5 chain: q0 50-bit, 28 scaling primes near 2^40, 3 x 60-bit CoeffToSlot primes on top;
    P = 7 x 60-bit (1783 bits in all; the reference's n32 chains have 1730-1759, tests/golden/chain_moduli.json).

    The scaling primes are chosen top-down so that the FLEXIBLE scales S(l-1) = S(l)^2 / q_{l-1}, which
    double any deviation at every level, stay at 2^40: q_{l-1} is the NTT prime nearest S(l)^2 / 2^40
    (OpenFHE picks its FLEXIBLE moduli on alternating sides of 2^p for the same reason)."""
    big = ckks.gen_primes(60, 10)
    q0 = ckks.gen_primes(50, 1)
    used = set(big) | set(q0)
    target = 2.0**log_scale
    S = target
    scaling = []
    for _ in range(n_scaling):  # q_28 first (under the CoeffToSlot primes), down to q_1
        q = _nearest_ntt_prime(S * S / target, used)
        used.add(q)
        scaling.append(q)
        S = S * S / q
    return q0 + scaling[::-1] + big[:3] + big[3:]


def build_engine(ckks, secret_seed=b"S" * 32, n_keys_seed=7, steps=None, cheb_degree=39, double_angles=2):
    """Context, bootstrapping plan, secret and every key the decode step uses; returns (backend, secret)."""
    ctx = ckks.Context(num_q=32, num_p=7, dnum=4, scale=2.0**40, moduli=config5_moduli(ckks))
    ctx.set_moddown_exact(True)  # unbiased key-switch rounding: the 2^40 chain bootstraps to ~13 bits with it
    # sparse-secret encapsulation (h' = 32): |I| <= ~8 sigma = 8 sqrt(33/12) ~ 13, so K = 14 (EvalMod's noise
    # grows as K^2).  Degree 47 with two double angles approximates sin(2 pi K t) to ~2e-11 -- far below the
    # noise -- in the depth of degree 59, with 14 instead of 16 products per ciphertext (degree 31 with three
    # double angles would save more products but costs one more level).  One plan per refresh kind, differing
    # only in the input scale: the state and the channel-mix increment (|f| <= ~0.6)
    # enter at q0 (m/q0 stays ~1e-3 per coefficient), the time-mix increment (|o| <= ~0.05) at 8 q0: more signal
    # over EvalMod's noise.
    # The two input scales share one set of CoeffToSlot / SlotToCoeff diagonals (~9 GB each): the 2^50 plan is the
    # 2^53 plan with EvalMod's output multiplied by 8 before SlotToCoeff.
    base = ckks.Bootstrap(ctx, K=14.0, cheb_degree=cheb_degree, double_angles=double_angles, top_scale=2.0**52,
                          in_scale=2.0**53)
    low = ckks.Bootstrap(ctx, in_scale=2.0**50, share=base)
    plans = {"state": (low, 2.0**50), "inc_cm": (low, 2.0**50), "inc_tm": (base, 2.0**53)}
    sk = ctx.secret(secret_seed, 192)
    sk_sparse = ctx.secret(bytes(reversed(secret_seed)), 32)
    kb = ctx.dnum * 2 * (ctx.L + ctx.K) * ctx.N * 8
    to_sparse = ckks.DeviceBuffer(kb)
    ctx.keygen_switch(sk, sk_sparse, b"t" * 32, b"u" * 32, to_sparse.ptr, q_limbs=1)
    from_sparse = ckks.DeviceBuffer(kb)
    ctx.keygen_switch(sk_sparse, sk, b"v" * 32, b"w" * 32, from_sparse.ptr)
    for b, _ in plans.values():
        b.set_sparse_keys(to_sparse.ptr, from_sparse.ptr)
    relin = ckks.DeviceBuffer(kb)
    ctx.keygen_relin(sk, b"r" * 32, b"s" * 32, relin.ptr)
    conj = ckks.DeviceBuffer(kb)
    ctx.keygen_automorphism(sk, 2 * ctx.N - 1, b"c" * 32, b"d" * 32, conj.ptr)
    want = sorted(set(M.rotation_steps() if steps is None else steps) |
                  set(s for b, _ in plans.values() for s in b.steps))
    keys, bufs = {}, []
    for i, s in enumerate(want):
        b = ckks.DeviceBuffer(kb)
        tag = i.to_bytes(2, "little")
        ctx.keygen_automorphism(sk, ckks.rotation_index(s), bytes([n_keys_seed]) + tag + b"k" * 29,
                                bytes([n_keys_seed]) + tag + b"e" * 29, b.ptr)
        keys[s] = b.ptr
        bufs.append(b)
    be = HEBackend(ckks, ctx, plans, relin.ptr, conj.ptr, keys)
    be._owned = (relin, conj, bufs, to_sparse, from_sparse, sk_sparse)  # keep the keys alive with the backend
    return be, sk
