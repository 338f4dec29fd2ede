"""Float64 plaintext restatement of the config-5 decode step (test infrastructure, like the rest of oracle/:
tests and bench.py's CPU baseline use it as the checker; the product path never imports it).

It evaluates the model described in fhe-ssm_amd/rwkv_model.py in its natural matrix form (per-head 64 x 64
states, dense products), independent of the slot layout, diagonals and rotations the encrypted driver
uses.  The pieces of the RWKV-7 time mixing are separate functions so that each can be checked on its own
(results/vector-d-20261104/raw/rwkv_v7_numpy.py is the RWKV-7 step they restate, line numbers below):

  token_shift     u = (1 - mu) x + mu x_prev (times a gain g): `x + m * (last_x - x)` (:20)
  value_residual  v + (v0 - v) gate: `v += (v0 - v) * sigmoid(...)` (:26-30), the gate a polynomial here
  k_update        k (1 + (a - 1) k_a): `k += k * (a-1) * k_a` (:33)
  head_l2norm     kk p(|kk_h|^2) per head: `kk /= max(norm(kk), 1e-12)` per head (:36-37), 1/|kk| a polynomial of
                  the squared norm here
  wkv_update      S <- S diag(w) - (S kh)(kh a)^T + v k^T per head:
                  `S = S * w.mT - S @ kk * (kk*a).mT + v * k.mT` (:39)
  wkv_readout     y = S r per head: `y = S @ r` (:40)
  group_norm      (y_h - mean(y_h)) p(var(y_h)) ln_w + ln_b per head: `group_norm(y, ln_w, ln_b)` (:9,42), the inverse
                  square root a polynomial here
  bonus           y + (sum_i r_i k_i r_k,i)_h v_h: `y += ((r * k * r_k).sum(axis=1,keepdims=1) * v)` (:43)

Here S is [lanes][heads][64][64] with S[i][j] the entry of row i (value index) and column j (key index), as
the reference's per-head S of shape (HEAD_SIZE, HEAD_SIZE) with v (HEAD_SIZE, 1) times k.mT.  The model
differs from RWKV-7 where rwkv_model.py says (polynomial nonlinearities, dense maps for the LoRA pairs).
gpu_real_model.cu:4674-5300 sequences the same stages.
"""
from __future__ import annotations

import numpy as np

D, HEADS, HS, FF = 768, 12, 64, 3072


def poly(c, z):
    return c[0] + z * (c[1] + z * (c[2] + z * c[3]))


def init_state(lanes: int, n_layers: int):
    return [{"S": np.zeros((lanes, HEADS, HS, HS)), "xp_t": np.zeros((lanes, D)), "xp_c": np.zeros((lanes, D))}
            for _ in range(n_layers)]


def token_shift(x, x_prev, mu, gain):
    """gain ((1 - mu) x + mu x_prev), elementwise over channels"""
    return x * (gain * (1 - mu)) + x_prev * (gain * mu)


def heads(z):
    """[lanes][768] -> [lanes][12][64]"""
    return z.reshape(z.shape[0], HEADS, HS)


def value_residual(v, v0, gate):
    """v + (v0 - v) gate: the value mixed toward the first layer's value"""
    return v + (v0 - v) * gate


def k_update(k, a, k_a):
    """k (1 + (a - 1) k_a), elementwise"""
    return k + k * (a - 1) * k_a


def head_l2norm(kk, pcoef):
    """kk_h p(|kk_h|^2) for every head h of every lane: [lanes][768] -> [lanes][768]"""
    kh = heads(kk)
    z = np.sum(kh * kh, axis=2, keepdims=True)
    return (kh * poly(pcoef, z)).reshape(kk.shape)


def wkv_update(S, w, kh, a, v, k):
    """S [lanes][heads][64][64]; w, kh, a, v, k [lanes][heads][64] -> the new S:
    S diag(w) - (S kh)(kh * a)^T + v k^T (each head on its own)"""
    sa = np.einsum("lhij,lhj->lhi", S, kh)
    return S * w[:, :, None, :] - sa[:, :, :, None] * (kh * a)[:, :, None, :] + v[:, :, :, None] * k[:, :, None, :]


def wkv_readout(S, r):
    """y = S r per head: [lanes][heads][64]"""
    return np.einsum("lhij,lhj->lhi", S, r)


def group_norm(y, pcoef, ln_w, ln_b):
    """per head: (y_h - mean(y_h)) p(var(y_h)), then ln_w y + ln_b over the channels: [lanes][768]"""
    yh = heads(y)
    mu = np.mean(yh, axis=2, keepdims=True)
    yc = yh - mu
    var = np.mean(yc * yc, axis=2, keepdims=True)
    return (yc * poly(pcoef, var)).reshape(y.shape) * ln_w + ln_b


def bonus(y, r, k, r_k, v):
    """y + (sum_i r_i k_i r_k,i over each head) v_h"""
    s = np.sum(heads(r * k * r_k), axis=2, keepdims=True)
    return y + (s * heads(v)).reshape(y.shape)


def layer(x, st, L, v0=None):
    """one layer for all lanes: x [lanes][768]; st is updated in place; v0 the first layer's value (None in the
    first layer, which sets it); returns (the new x, v0)"""
    lanes = x.shape[0]
    n = poly(L["p_n1"], np.mean(x * x, axis=1))
    xn = x * n[:, None]
    u = {m: token_shift(xn, st["xp_t"], L["mu_" + m], L["g1"]) for m in ("r", "k", "v", "w", "a", "g")}
    r = u["r"] @ L["W_r"].T
    k = u["k"] @ L["W_k"].T
    v = u["v"] @ L["W_v"].T
    w = poly(L["p_w"], u["w"] @ L["W_w"].T)
    a = poly(L["p_a"], u["a"] @ L["W_a"].T)
    g = poly(L["p_g"], u["g"] @ L["W_g"].T)
    if v0 is None:
        v0 = v
    else:
        v = value_residual(v, v0, poly(L["p_v"], u["v"] @ L["W_vg"].T))
    kk = k * L["k_k"]
    k = k_update(k, a, L["k_a"])
    kh = head_l2norm(kk, L["p_kn"])
    S = wkv_update(st["S"], heads(w), heads(kh), heads(a), heads(v), heads(k))
    y = wkv_readout(S, heads(r)).reshape(lanes, D)
    y = bonus(group_norm(y, L["p_gn"], L["ln_w"], L["ln_b"]), r, k, L["r_k"], v)
    st["S"] = S
    st["xp_t"] = xn
    x = x + (y * g) @ L["W_o"].T
    n2 = poly(L["p_n2"], np.mean(x * x, axis=1))
    xn2 = x * n2[:, None]
    uc = token_shift(xn2, st["xp_c"], L["mu_c"], L["g2"])
    h = poly(L["p_h"], uc @ L["W_ck"].T)
    st["xp_c"] = xn2
    return x + h @ L["W_cv"].T, v0


def step(x, state, W, n_layers=None):
    """one decode step: returns (xo [lanes][768] after the output norm, per-layer activations)"""
    n_layers = len(W["layers"]) if n_layers is None else n_layers
    acts = []
    v0 = None
    for li in range(n_layers):
        x, v0 = layer(x, state[li], W["layers"][li], v0)
        acts.append(x.copy())
    xo = x * poly(W["p_o"], np.mean(x * x, axis=1))[:, None] * W["g_o"]
    return xo, acts
