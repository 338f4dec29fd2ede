"""Float64 plaintext restatement of the config-5 decode step (test infrastructure, like the rest of oracle/:
tests and bench.py's CPU baseline use it as the checker; the product path never imports it).

It evaluates the model described in fhe-ssm_amd/rwkv_model.py in its natural matrix form (per-head 64 x 64
states, dense products), independent of the slot layout, diagonals and rotations the encrypted driver
uses.  The WKV-7 update and readout follow the RWKV-7 recurrence S <- S diag(w) - (S kh)(kh a)^T + v k^T,
y = S r (the model the reference's served step runs; gpu_real_model.cu:4674-5300 sequences the same
stages).
"""
from __future__ import annotations

import numpy as np

D, HEADS, HS, FF = 768, 12, 64, 3072


def poly(c, z):
    return c[0] + z * (c[1] + z * (c[2] + z * c[3]))


def init_state(lanes: int, n_layers: int):
    return [{"S": np.zeros((lanes, HEADS, HS, HS)), "xp_t": np.zeros((lanes, D)), "xp_c": np.zeros((lanes, D))}
            for _ in range(n_layers)]


def layer(x, st, L):
    """one layer for all lanes: x [lanes][768]; st is updated in place; returns the new x"""
    lanes = x.shape[0]
    n = poly(L["p_n1"], np.mean(x * x, axis=1))
    xn = x * n[:, None]
    u = {m: xn * (L["g1"] * (1 - L["mu_" + m])) + st["xp_t"] * (L["g1"] * L["mu_" + m])
         for m in ("r", "k", "v", "w", "a", "g")}
    r = u["r"] @ L["W_r"].T
    k = u["k"] @ L["W_k"].T
    v = u["v"] @ L["W_v"].T
    w = poly(L["p_w"], u["w"] @ L["W_w"].T)
    a = poly(L["p_a"], u["a"] @ L["W_a"].T)
    g = poly(L["p_g"], u["g"] @ L["W_g"].T)
    kh = k * L["eta"]
    hv = lambda z: z.reshape(lanes, HEADS, HS)
    S = st["S"]
    sa = np.einsum("lhij,lhj->lhi", S, hv(kh))
    S = S * hv(w)[:, :, None, :] - sa[:, :, :, None] * hv(kh * a)[:, :, None, :] \
        + hv(v)[:, :, :, None] * hv(k)[:, :, None, :]
    y = np.einsum("lhij,lhj->lhi", S, hv(r)).reshape(lanes, D)
    st["S"] = S
    st["xp_t"] = xn
    x = x + (y * g) @ L["W_o"].T
    n2 = poly(L["p_n2"], np.mean(x * x, axis=1))
    xn2 = x * n2[:, None]
    uc = xn2 * (L["g2"] * (1 - L["mu_c"])) + st["xp_c"] * (L["g2"] * L["mu_c"])
    h = poly(L["p_h"], uc @ L["W_ck"].T)
    st["xp_c"] = xn2
    return x + h @ L["W_cv"].T


def step(x, state, W, n_layers=None):
    """one decode step: returns (xo [lanes][768] after the output norm, per-layer activations)"""
    n_layers = len(W["layers"]) if n_layers is None else n_layers
    acts = []
    for li in range(n_layers):
        x = layer(x, state[li], W["layers"][li])
        acts.append(x.copy())
    xo = x * poly(W["p_o"], np.mean(x * x, axis=1))[:, None] * W["g_o"]
    return xo, acts
