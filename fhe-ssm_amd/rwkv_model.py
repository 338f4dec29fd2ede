"""Shape, weights and slot layout of the config-5 decode step: an RWKV-7-0.1B-shaped polynomial recurrent
model evaluated on 32 conversation lanes packed in the slots of one N = 2^16 ciphertext.

Shape (RWKV-7 0.1B): 12 layers, d_model 768, 12 heads of size 64, channel-mix width 3072, vocabulary 65536.
Every nonlinearity is a degree-3 polynomial p(z) = c0 + c1 z + c2 z^2 + c3 z^3 with seeded coefficients in
[-0.5, 0.5]; weights are random-init (seeded).  Per layer and lane (x in R^768, carried state S_h in
R^{64x64} per head, xp_t, xp_c in R^768):

  time mix      n  = p_n1(mean(x^2));  xn = x n                       (RMSNorm: rsqrt -> p_n1)
                u_m = g1 (1 - mu_m) xn + g1 mu_m xp_t,  m in {r, k, v, w, a, g}      (token shift)
                r, k, v = W_r u_r, W_k u_k, W_v u_v
                w, a, g = p_w(W_w u_w), p_a(W_a u_a), p_g(W_g u_g)    (decay, in-context rate, gate)
                v <- v + (v0 - v) p_v(W_vg u_v)   in layers > 0, v0 = layer 0's v      (value residual)
                kk = k k_k;  k <- k (1 + (a - 1) k_a)                  (removal key, key update)
                kh_h = kk_h p_kn(|kk_h|^2)                             (per-head L2 norm: 1/|kk| -> p_kn)
                S_h <- S_h diag(w_h) - (S_h kh_h)(kh_h a_h)^T + v_h k_h^T    (WKV-7 state update)
                y_h = S_h r_h
                y_h <- (y_h - mean(y_h)) p_gn(var(y_h)) ln_w_h + ln_b_h   (per-head GroupNorm: rsqrt -> p_gn)
                y_h <- y_h + (sum_i r_i k_i r_k,i)_h v_h                (bonus)
                x <- x + W_o (y g);  xp_t <- xn
  channel mix   xn2 = x p_n2(mean(x^2));  u = g2 (1 - mu_c) xn2 + g2 mu_c xp_c
                x <- x + W_cv p_h(W_ck u);  xp_c <- xn2
  output        xo = g_o x p_o(mean(x^2));  logits = W_head xo     (the head runs on the client)

This is RWKV-7's time mixing step for step (results/vector-d-20261104/raw/rwkv_v7_numpy.py:13-44); its LoRA pairs
for w, a, g and the value gate are dense 768 x 768 maps here, its sigmoid/exp/tanh and the norms' inverse square
roots degree-3 polynomials.  The reference's served FHE driver (gpu_real_model.cu:4674-5300) runs the same sequence
of norms, token shift, projections, scan, gate, output projection and channel mix.

Slot layout (lane-major, gpu_real_model.cu:483-519): slot lane * 1024 + c holds channel c < 768 of lane
lane; channels 768..1023 are zero.  Every plaintext that is the same for all lanes is 1024-periodic and
stored compressed (N / 32 words per limb).
"""
from __future__ import annotations

import numpy as np

N_LAYERS = 12
D = 768
DPAD = 1024
HEADS = 12
HS = 64
FF = 3072
VOCAB = 65536
LANES = 32
SLOTS = 1 << 15
LOG_REP = 5  # 1024-periodic plaintexts: N / 2^5 words per limb

MIX_NAMES = ("r", "k", "v", "w", "a", "g")


def _poly_coeffs(rng):
    return rng.uniform(-0.5, 0.5, 4)


def make_weights(seed: int = 5, n_layers: int = N_LAYERS, vocab: int = VOCAB) -> dict:
    """Seeded random-init weights.  The scales keep every activation O(1) over the 12 layers (the
    bootstrapped values must stay well inside the EvalMod range)."""
    rng = np.random.default_rng(seed)
    layers = []
    for _ in range(n_layers):
        L = {}
        L["g1"] = 1.0 + 0.1 * rng.standard_normal(D)
        L["g2"] = 1.0 + 0.1 * rng.standard_normal(D)
        for m in MIX_NAMES:
            L["mu_" + m] = rng.uniform(0.0, 1.0, D)
        L["mu_c"] = rng.uniform(0.0, 1.0, D)
        for m in ("r", "k", "v"):
            L["W_" + m] = rng.standard_normal((D, D)) / np.sqrt(D)
        for m in ("w", "a", "g"):
            L["W_" + m] = 0.5 * rng.standard_normal((D, D)) / np.sqrt(D)
        L["W_o"] = 0.5 * rng.standard_normal((D, D)) / np.sqrt(D)
        L["k_k"] = rng.uniform(0.05, 0.15, D)
        L["W_ck"] = 0.5 * rng.standard_normal((FF, D)) / np.sqrt(D)
        L["W_cv"] = 0.5 * rng.standard_normal((D, FF)) / np.sqrt(FF)
        for p in ("p_n1", "p_n2", "p_w", "p_a", "p_g", "p_h"):
            L[p] = _poly_coeffs(rng)
        # the rest of RWKV-7's time mixing: the value gate (a dense map, like w, a, g), the key update, the per-head
        # L2 norm of kk, the per-head GroupNorm of y and the bonus term
        L["W_vg"] = 0.5 * rng.standard_normal((D, D)) / np.sqrt(D)
        L["k_a"] = rng.uniform(0.0, 0.5, D)
        L["r_k"] = 0.05 * rng.standard_normal(D)
        L["ln_w"] = 1.0 + 0.1 * rng.standard_normal(D)
        L["ln_b"] = 0.02 * rng.standard_normal(D)
        for p in ("p_v", "p_kn", "p_gn"):
            L[p] = _poly_coeffs(rng)
        layers.append(L)
    out = {"layers": layers, "g_o": 1.0 + 0.1 * rng.standard_normal(D), "p_o": _poly_coeffs(rng)}
    out["emb_scale"] = 1.0
    out["head_seed"] = int(rng.integers(0, 2**31))
    out["vocab"] = vocab
    return out


def head_matrix(weights: dict, rows: int | None = None) -> np.ndarray:
    """The vocabulary head [vocab][768] (N(0, 1/768)), generated from its seed (rows: a prefix)."""
    rng = np.random.default_rng(weights["head_seed"])
    n = weights["vocab"] if rows is None else rows
    return rng.standard_normal((n, D)) / np.sqrt(D)


def embed_tokens(tokens, seed: int = 11) -> np.ndarray:
    """Client-side embedding of one token per lane: [lanes][768], entries N(0, 1) / 2."""
    rng = np.random.default_rng([seed] + [int(t) for t in tokens])
    return 0.5 * rng.standard_normal((len(tokens), D))


# ---------------------------------------------------------------- slot layout
def pack_lanes(X: np.ndarray) -> np.ndarray:
    """[lanes][<=1024] -> [32768] slots (lane-major, zero padded)."""
    X = np.atleast_2d(X)
    out = np.zeros((LANES, DPAD), dtype=X.dtype)
    out[: X.shape[0], : X.shape[1]] = X
    return out.reshape(-1)


def unpack_lanes(v: np.ndarray, width: int = D) -> np.ndarray:
    return np.asarray(v).reshape(LANES, DPAD)[:, :width]


def periodic(vec: np.ndarray) -> np.ndarray:
    """A per-channel vector (<= 1024 entries) as its 1024-period (zero padded)."""
    out = np.zeros(DPAD, dtype=np.asarray(vec).dtype)
    out[: len(vec)] = vec
    return out


# ---------------------------------------------------------------- BSGS diagonals (signed rotations)
# y[i] = sum_j M[i][j] x[j] inside each lane with i, j < 768: rotation r = j - i in (-768, 768), never leaving
# the lane.  r = G + b with babies b in [0, nb) and giants G = nb g, g in [-768/nb, 768/nb).  A matvec with at least
# as many outputs as inputs takes nb = 64 (24 giant rotations per output instead of 48: a giant costs a key switch
# per output, a hoisted baby about half of one per input), otherwise nb = 32.
MV_SPAN = 1536


def mv_nb(n_in: int, n_out: int) -> int:
    return 64 if n_out >= n_in else 32


def mv_babies(nb: int) -> tuple:
    return tuple(range(nb))


def mv_giants(nb: int) -> tuple:
    return tuple(nb * g for g in range(-(MV_SPAN // 2) // nb, (MV_SPAN // 2) // nb))


def matvec_diagonals(blocks) -> np.ndarray:
    """blocks[o][i]: 768 x 768 matrices (output block o, input block i; None = zero).
    Returns [n_out][n_giant][n_in * nb][1024] (nb = mv_nb(n_in, n_out)): the 1024-periodic diagonal for giant g,
    input i, baby b, pre-rotated by -G_g (gpu_real_model.cu:2767-2823's pre-rotation,
    harness/cpu_real_model.cpp:270-318)."""
    n_out, n_in = len(blocks), len(blocks[0])
    nb = mv_nb(n_in, n_out)
    giants = mv_giants(nb)
    out = np.zeros((n_out, len(giants), n_in * nb, DPAD))
    rows = np.arange(D)
    for o in range(n_out):
        for i in range(n_in):
            M = blocks[o][i]
            if M is None:
                continue
            for gi, G in enumerate(giants):
                for b in range(nb):
                    r = G + b
                    cols = rows + r
                    ok = (cols >= 0) & (cols < D)
                    d = np.zeros(DPAD)
                    d[rows[ok]] = M[rows[ok], cols[ok]]
                    # pre-rotation by -G of a 1024-periodic vector: d'[p] = d[(p - G) mod 1024]
                    out[o, gi, i * nb + b] = np.roll(d, G)
    return out


# ---------------------------------------------------------------- WKV diagonal layout
# D_t[lane*1024 + h*64 + i] = S_h[i][(i + t) mod 64], t = 0..63 (one ciphertext per t, all heads and lanes).
# rot64_t(x) (cyclic rotation by t inside every 64-block) = m_lo,t (.) Rot_t(x) + m_hi,t (.) Rot_{t-64}(x).
WKV_T = HS
WKV_LO = tuple(range(WKV_T))
WKV_HI = (0,) + tuple(t - HS for t in range(1, WKV_T))


def wkv_masks(extra: np.ndarray | None = None) -> np.ndarray:
    """[64][2][1024]: the lo/hi masks of rot64_t, optionally times rot64_t(extra) (a per-channel vector folded
    into the same plaintext)."""
    i = np.arange(DPAD) % HS
    valid = np.arange(DPAD) < D
    out = np.zeros((WKV_T, 2, DPAD))
    e = periodic(extra) if extra is not None else None
    for t in range(WKV_T):
        lo = valid & (i + t < HS)
        hi = valid & (i + t >= HS) if t else np.zeros(DPAD, dtype=bool)
        out[t, 0] = lo
        out[t, 1] = hi
        if e is not None:
            src = (np.arange(DPAD) // HS) * HS + (i + t) % HS
            out[t, :] *= np.where(valid, e[np.minimum(src, DPAD - 1)], 0.0)[None, :]
    return out


def state_to_diag(S: np.ndarray) -> np.ndarray:
    """[lanes][12][64][64] -> [64][32768] diagonal-layout slot vectors."""
    lanes = S.shape[0]
    out = np.zeros((WKV_T, LANES, DPAD))
    i = np.arange(HS)
    for t in range(WKV_T):
        vals = S[:, :, i, (i + t) % HS]  # [lanes][12][64]
        out[t, :lanes, :D] = vals.reshape(lanes, D)
    return out.reshape(WKV_T, -1)


def diag_to_state(Dg: np.ndarray, lanes: int = LANES) -> np.ndarray:
    S = np.zeros((lanes, HEADS, HS, HS))
    i = np.arange(HS)
    Dg = np.asarray(Dg).reshape(WKV_T, LANES, DPAD)
    for t in range(WKV_T):
        S[:, :, i, (i + t) % HS] = Dg[t, :lanes, :D].reshape(lanes, HEADS, HS)
    return S


# ---------------------------------------------------------------- norms
# The lane and head sums are rotate-and-add windows (the reference's red = EvalAdd(red, rot(red, p)) loops,
# gpu_real_model.cu:3524,3540), each window one hoisted rotation sum s + sum_k Rot_k(s) over a set of steps (one
# ModUp and one ModDown for the whole set).  Slot lane*1024 gets the lane's sum from windows of 32 (steps 1..31), then
# 16 x 32 (steps 32, 64, .., 480), then 2 x 512; the broadcast of the masked sum runs the same windows downwards.
# Every step is one the matvecs or the WKV scan already hold a key for.
NORM_UP = (tuple(range(1, 32)), tuple(range(32, 512, 32)), (512,))
NORM_DOWN = tuple(tuple(-k for k in w) for w in NORM_UP)


HEAD_UP = (tuple(range(1, 64)),)  # slot h*64 of a lane gets head h's sum
HEAD_DOWN = (tuple(-k for k in HEAD_UP[0]),)  # broadcast the masked sums over their heads


def head_start_mask(scale: float = 1.0) -> np.ndarray:
    """scale at channel h*64 of every head h < 12, else 0"""
    m = np.zeros(DPAD)
    m[0:D:HS] = scale
    return m


def lane_start_mask(scale: float = 1.0) -> np.ndarray:
    m = np.zeros(DPAD)
    m[0] = scale
    return m


# ---------------------------------------------------------------- gap packing of the state
# Channels 768..1023 of every lane are unused (a quarter of the slots).  Before the state is bootstrapped, the
# 64 diagonal ciphertexts are packed 4 -> 3: piece p (channels 256p .. 256p + 255) of D_{48+j} is moved into the gap
# of D_{16p+j} by a rotation of -(768 - 256p); after the bootstrap it is moved back by +(768 - 256p) and masked.
# The gaps of D_0..D_47 then hold those pieces: every use of D_t multiplies it by a masked rotation (zero on the
# gap), so they never reach a valid channel.
GAP_SHIFT = (768, 512, 256)  # piece p of the fourth quarter lives in the gap of quarter p, shifted by GAP_SHIFT[p]


def channel_range_mask(lo: int, hi: int) -> np.ndarray:
    """1 on channels lo .. hi-1 of every lane, else 0"""
    m = np.zeros(DPAD)
    m[lo:hi] = 1.0
    return m


def rotation_steps() -> list:
    """Every rotation step the decode step uses (keys to generate)."""
    s = set(WKV_LO) | set(WKV_HI)
    for w in NORM_UP + NORM_DOWN + HEAD_UP + HEAD_DOWN:
        s |= set(w)
    for nb in (32, 64):
        s |= set(mv_babies(nb)) | set(mv_giants(nb))
    s |= set(GAP_SHIFT) | set(-g for g in GAP_SHIFT)
    s.discard(0)
    return sorted(s)
