"""Pins oracle/rwkv_ref.py, the float64 checker of config 5, by closed forms the RWKV-7 recurrence fixes
(results/vector-d-20261104/raw/rwkv_v7_numpy.py:20,39-40 is the recurrence it restates):

  - from S = 0 one update gives S = v k^T, and the readout y = v (k . r);
  - with w = 1 and a = 0 the state after T steps is sum_t v_t k_t^T;
  - with w = 1, a = 1, v = 0 and |kh| = 1 the removal term projects kh out of S (S' kh = 0, S' u = S u for u
    orthogonal to kh);
  - with a = 0 and v = 0 the decay scales column j (key index) by w_j;
  - the token shift is (1 - mu) x + mu x_prev;
  - a layer with identity projections and constant polynomials has a closed-form output over two steps, which
    pins which projection feeds which slot of the recurrence and where the token shift reads its carry.

Each check is run against planted mistakes (a transposed outer product, a sign flip of the removal, the decay
on the wrong index, a transposed readout, a swapped token shift): every mutant must fail at least one check.
"""
import numpy as np
import pytest

from oracle import rwkv_ref as ref

HS = ref.HS


def rand(rng, *shape):
    return rng.standard_normal(shape)


# ---------------------------------------------------------------- the checks, parametrised by the functions
def check_first_step(upd, rd, rng):
    v, k, r = rand(rng, 2, 3, HS), rand(rng, 2, 3, HS), rand(rng, 2, 3, HS)
    w, kh, a = rand(rng, 2, 3, HS), rand(rng, 2, 3, HS), rand(rng, 2, 3, HS)
    S = upd(np.zeros((2, 3, HS, HS)), w, kh, a, v, k)
    want = np.einsum("lhi,lhj->lhij", v, k)
    y = rd(S, r)
    return np.allclose(S, want, atol=1e-12) and np.allclose(y, v * np.sum(k * r, axis=2, keepdims=True), atol=1e-12)


def check_accumulation(upd, rd, rng):
    T = 5
    S = np.zeros((1, 2, HS, HS))
    want = np.zeros_like(S)
    for _ in range(T):
        v, k, kh = rand(rng, 1, 2, HS), rand(rng, 1, 2, HS), rand(rng, 1, 2, HS)
        S = upd(S, np.ones((1, 2, HS)), kh, np.zeros((1, 2, HS)), v, k)
        want += np.einsum("lhi,lhj->lhij", v, k)
    r = rand(rng, 1, 2, HS)
    return np.allclose(S, want, atol=1e-11) and np.allclose(rd(S, r), np.einsum("lhij,lhj->lhi", want, r), atol=1e-10)


def check_removal_projects(upd, rd, rng):
    S = rand(rng, 1, 2, HS, HS)
    kh = rand(rng, 1, 2, HS)
    kh /= np.linalg.norm(kh, axis=2, keepdims=True)
    S2 = upd(S, np.ones((1, 2, HS)), kh, np.ones((1, 2, HS)), np.zeros((1, 2, HS)), rand(rng, 1, 2, HS))
    u = rand(rng, 1, 2, HS)
    u -= np.sum(u * kh, axis=2, keepdims=True) * kh  # u orthogonal to kh
    return (np.allclose(rd(S2, kh), 0, atol=1e-11)
            and np.allclose(rd(S2, u), np.einsum("lhij,lhj->lhi", S, u), atol=1e-11))


def check_decay(upd, rd, rng):
    S = rand(rng, 1, 2, HS, HS)
    w = rng.uniform(0.1, 0.9, (1, 2, HS))
    S2 = upd(S, w, rand(rng, 1, 2, HS), np.zeros((1, 2, HS)), np.zeros((1, 2, HS)), rand(rng, 1, 2, HS))
    return np.allclose(S2, S * w[:, :, None, :], atol=1e-13)


def check_token_shift(ts, rng):
    x, xp, g = rand(rng, 3, 768), rand(rng, 3, 768), rand(rng, 768)
    mu = rng.uniform(0, 1, 768)
    return (np.allclose(ts(x, xp, np.zeros(768), g), g * x) and np.allclose(ts(x, xp, np.ones(768), g), g * xp)
            and np.allclose(ts(x, xp, mu, g), g * ((1 - mu) * x + mu * xp), atol=1e-13))


WKV_CHECKS = [check_first_step, check_accumulation, check_removal_projects, check_decay]


@pytest.mark.parametrize("check", WKV_CHECKS, ids=lambda c: c.__name__)
def test_wkv_closed_forms(check):
    assert check(ref.wkv_update, ref.wkv_readout, np.random.default_rng(WKV_CHECKS.index(check) + 1))


def test_token_shift_closed_form():
    assert check_token_shift(ref.token_shift, np.random.default_rng(3))


# ---------------------------------------------------------------- planted mistakes must fail
def _upd_transposed_outer(S, w, kh, a, v, k):
    sa = np.einsum("lhij,lhj->lhi", S, kh)
    return S * w[:, :, None, :] - sa[:, :, :, None] * (kh * a)[:, :, None, :] + k[:, :, :, None] * v[:, :, None, :]


def _upd_removal_sign(S, w, kh, a, v, k):
    sa = np.einsum("lhij,lhj->lhi", S, kh)
    return S * w[:, :, None, :] + sa[:, :, :, None] * (kh * a)[:, :, None, :] + v[:, :, :, None] * k[:, :, None, :]


def _upd_decay_rows(S, w, kh, a, v, k):
    sa = np.einsum("lhij,lhj->lhi", S, kh)
    return S * w[:, :, :, None] - sa[:, :, :, None] * (kh * a)[:, :, None, :] + v[:, :, :, None] * k[:, :, None, :]


def _upd_removal_transposed(S, w, kh, a, v, k):
    sa = np.einsum("lhji,lhj->lhi", S, kh)
    return S * w[:, :, None, :] - sa[:, :, :, None] * (kh * a)[:, :, None, :] + v[:, :, :, None] * k[:, :, None, :]


def _rd_transposed(S, r):
    return np.einsum("lhji,lhj->lhi", S, r)


@pytest.mark.parametrize("upd,rd", [
    (_upd_transposed_outer, ref.wkv_readout),
    (_upd_removal_sign, ref.wkv_readout),
    (_upd_decay_rows, ref.wkv_readout),
    (_upd_removal_transposed, ref.wkv_readout),
    (ref.wkv_update, _rd_transposed),
], ids=["outer-transposed", "removal-sign", "decay-rows", "removal-transposed", "readout-transposed"])
def test_wkv_mutants_fail(upd, rd):
    rng = np.random.default_rng(7)
    assert not all(c(upd, rd, rng) for c in WKV_CHECKS)


def test_token_shift_mutant_fails():
    assert not check_token_shift(lambda x, xp, mu, g: x * (g * mu) + xp * (g * (1 - mu)), np.random.default_rng(4))


# ---------------------------------------------------------------- one layer's wiring, closed form over two steps
def _identity_layer():
    D, FF = ref.D, ref.FF
    one, zero = np.array([1.0, 0, 0, 0]), np.zeros(4)
    L = {"p_n1": one, "p_n2": one, "p_w": one, "p_a": zero, "p_g": one, "p_h": np.array([0.0, 1, 0, 0]),
         "g1": np.ones(D), "g2": np.full(D, 2.0), "eta": np.full(D, 0.3)}
    for m in ("r", "v", "w", "a", "g"):
        L["mu_" + m] = np.zeros(D)
    L["mu_k"] = np.ones(D)  # k reads the previous step's normalised input only
    L["mu_c"] = np.full(D, 0.25)
    for m in ("r", "k", "v", "o"):
        L["W_" + m] = np.eye(D)
    for m in ("w", "a", "g"):
        L["W_" + m] = np.zeros((D, D))
    L["W_ck"] = np.vstack([np.eye(D), np.zeros((FF - D, D))])
    L["W_cv"] = np.hstack([np.eye(D), np.zeros((D, FF - D))])
    return L


def test_layer_wiring_closed_form():
    """r = v = x_t, k = x_{t-1} (mu_k = 1, the carry), w = 1, a = 0, g = 1:
    S_1 = x_1 x_0^T (x_0 = 0, so S_1 = 0), S_2 = x_2 x_1^T, y_2 = x_2 (x_1 . x_2) per head; the channel mix
    with h = W_ck u, W_cv = [I 0] adds g2 ((1 - mu_c) x' + mu_c xp_c) with xp_c the previous step's x'."""
    rng = np.random.default_rng(11)
    L = _identity_layer()
    st = ref.init_state(3, 1)[0]
    x1, x2 = 0.3 * rand(rng, 3, ref.D), 0.3 * rand(rng, 3, ref.D)
    out1 = ref.layer(x1, st, L)
    # step 1: k = xp_t = 0, so S stays 0 and y = 0; x' = x1; channel mix adds 2 * 0.75 * x1
    assert np.allclose(out1, x1 + 1.5 * x1, atol=1e-13)
    assert np.allclose(st["S"], 0) and np.allclose(st["xp_t"], x1) and np.allclose(st["xp_c"], x1)
    out2 = ref.layer(x2, st, L)
    h1, h2 = x1.reshape(3, 12, 64), x2.reshape(3, 12, 64)
    y = (h2 * np.sum(h1 * h2, axis=2, keepdims=True)).reshape(3, ref.D)
    xm = x2 + y
    assert np.allclose(st["S"], np.einsum("lhi,lhj->lhij", h2, h1), atol=1e-13)
    assert np.allclose(out2, xm + 2.0 * (0.75 * xm + 0.25 * x1), atol=1e-12)


def test_output_norm_closed_form():
    rng = np.random.default_rng(12)
    L = _identity_layer()
    W = {"layers": [L], "p_o": np.array([0.0, 1, 0, 0]), "g_o": rng.uniform(0.5, 1.5, ref.D)}
    x = 0.3 * rand(rng, 2, ref.D)
    xo, acts = ref.step(x, ref.init_state(2, 1), W)
    xl = acts[0]
    assert np.allclose(xl, 2.5 * x, atol=1e-13)
    assert np.allclose(xo, xl * np.mean(xl * xl, axis=1, keepdims=True) * W["g_o"], atol=1e-13)
