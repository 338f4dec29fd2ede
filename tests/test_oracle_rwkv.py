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

The rest of RWKV-7's time mixing (rwkv_v7_numpy.py:26-30,32-33,36-37,42-43), each by closed forms and a planted
mistake that must fail them:
  - value residual v + (v0 - v) gate: gate 0 keeps v, gate 1 gives v0 (mutant: the difference reversed);
  - key update k (1 + (a - 1) k_a): a = 1 or k_a = 0 keep k, k_a = 1 gives k a (mutant: the k term dropped);
  - per-head L2 norm kk p(|kk_h|^2): on heads of unit norm it is kk p(1); p(z) = z gives kk |kk_h|^2 per head
    (mutant: the norm over the whole lane);
  - GroupNorm: a head-constant y gives ln_b; p = 1, ln_w = 1, ln_b = 0 gives y minus its head mean; p(z) = z gives
    (y - mean) var per head (mutants: the mean over the whole lane, ln_b multiplied);
  - bonus y + (sum r k r_k)_h v_h: with unit vectors it picks one head's coefficient (mutants: the sum over the lane,
    no sum at all);
  - the first layer's value reaches the later layers' residual (mutant: each layer mixing toward its own value).
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
         "g1": np.ones(D), "g2": np.full(D, 2.0), "k_k": np.full(D, 0.3), "k_a": np.zeros(D), "p_kn": one,
         "p_gn": one, "ln_w": np.ones(D), "ln_b": np.zeros(D), "r_k": np.zeros(D), "p_v": zero}
    for m in ("r", "v", "w", "a", "g"):
        L["mu_" + m] = np.zeros(D)
    L["mu_k"] = np.ones(D)  # k reads the previous step's normalised input only
    L["mu_c"] = np.full(D, 0.25)
    for m in ("r", "k", "v", "o"):
        L["W_" + m] = np.eye(D)
    for m in ("w", "a", "g", "vg"):
        L["W_" + m] = np.zeros((D, D))
    L["W_ck"] = np.vstack([np.eye(D), np.zeros((FF - D, D))])
    L["W_cv"] = np.hstack([np.eye(D), np.zeros((D, FF - D))])
    return L


def test_layer_wiring_closed_form():
    """r = v = x_t, k = x_{t-1} (mu_k = 1, the carry), w = 1, a = 0, g = 1, k_a = 0, GroupNorm with p = 1,
    ln_w = 1, ln_b = 0 (y minus its head mean), no bonus: S_1 = x_1 x_0^T (x_0 = 0, so S_1 = 0), S_2 = x_2 x_1^T,
    y_2 = x_2 (x_1 . x_2) per head, centered per head; the channel mix with h = W_ck u, W_cv = [I 0] adds
    g2 ((1 - mu_c) x' + mu_c xp_c) with xp_c the previous step's x'."""
    rng = np.random.default_rng(11)
    L = _identity_layer()
    st = ref.init_state(3, 1)[0]
    x1, x2 = 0.3 * rand(rng, 3, ref.D), 0.3 * rand(rng, 3, ref.D)
    out1, v0 = ref.layer(x1, st, L)
    assert np.allclose(v0, x1)  # the first layer's value: v = x (W_v = I, mu_v = 0, p_n1 = 1)
    # step 1: k = xp_t = 0, so S stays 0 and y = 0; x' = x1; channel mix adds 2 * 0.75 * x1
    assert np.allclose(out1, x1 + 1.5 * x1, atol=1e-13)
    assert np.allclose(st["S"], 0) and np.allclose(st["xp_t"], x1) and np.allclose(st["xp_c"], x1)
    out2, _ = ref.layer(x2, st, L)
    h1, h2 = x1.reshape(3, 12, 64), x2.reshape(3, 12, 64)
    yh = h2 * np.sum(h1 * h2, axis=2, keepdims=True)
    y = (yh - yh.mean(axis=2, keepdims=True)).reshape(3, ref.D)
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


# ---------------------------------------------------------------- the rest of RWKV-7's time mixing
def check_value_residual(f, rng):
    v, v0 = rand(rng, 2, 768), rand(rng, 2, 768)
    g = rng.uniform(0, 1, (2, 768))
    return (np.allclose(f(v, v0, np.zeros_like(v)), v) and np.allclose(f(v, v0, np.ones_like(v)), v0)
            and np.allclose(f(v, v0, g), (1 - g) * v + g * v0, atol=1e-14))


def check_k_update(f, rng):
    k, a, ka = rand(rng, 2, 768), rand(rng, 2, 768), rng.uniform(0, 1, 768)
    return (np.allclose(f(k, np.ones_like(a), ka), k) and np.allclose(f(k, a, np.zeros(768)), k)
            and np.allclose(f(k, a, np.ones(768)), k * a, atol=1e-14))


def check_head_l2norm(f, rng):
    kk = rand(rng, 2, 768)
    unit = (kk.reshape(2, 12, 64) / np.linalg.norm(kk.reshape(2, 12, 64), axis=2, keepdims=True)).reshape(2, 768)
    c = rng.uniform(-0.5, 0.5, 4)
    n2 = np.repeat(np.sum(kk.reshape(2, 12, 64) ** 2, axis=2), 64, axis=1)
    return (np.allclose(f(unit, c), unit * np.sum(c), atol=1e-13)
            and np.allclose(f(kk, np.array([0.0, 1, 0, 0])), kk * n2, atol=1e-12))


def check_group_norm(f, rng):
    y = rand(rng, 2, 768)
    w, b = rng.uniform(0.5, 1.5, 768), rand(rng, 768)
    const = np.repeat(rand(rng, 2, 12), 64, axis=1)
    yh = y.reshape(2, 12, 64)
    yc = yh - yh.mean(axis=2, keepdims=True)
    var = np.mean(yc ** 2, axis=2, keepdims=True)
    one = np.array([1.0, 0, 0, 0])
    return (np.allclose(f(const, rng.uniform(-1, 1, 4), w, b), np.broadcast_to(b, (2, 768)), atol=1e-13)
            and np.allclose(f(y, one, np.ones(768), np.zeros(768)), yc.reshape(2, 768), atol=1e-13)
            and np.allclose(f(y, np.array([0.0, 1, 0, 0]), w, b), (yc * var).reshape(2, 768) * w + b, atol=1e-12))


def check_bonus(f, rng):
    y, v = rand(rng, 1, 768), rand(rng, 1, 768)
    r, k, rk = np.zeros((1, 768)), np.zeros((1, 768)), np.zeros(768)
    r[0, 64 * 3 + 5], k[0, 64 * 3 + 5], rk[64 * 3 + 5] = 2.0, 3.0, 0.5   # one channel of head 3
    want = y.copy()
    want[0, 192:256] += 3.0 * v[0, 192:256]
    r2, k2, rk2 = rand(rng, 1, 768), rand(rng, 1, 768), rand(rng, 768)
    s = np.sum((r2 * k2 * rk2).reshape(1, 12, 64), axis=2, keepdims=True)
    return (np.allclose(f(y, r, k, rk, v), want, atol=1e-14)
            and np.allclose(f(y, r2, k2, rk2, v), y + (s * v.reshape(1, 12, 64)).reshape(1, 768), atol=1e-12))


def test_time_mix_parts_closed_forms():
    rng = np.random.default_rng(21)
    assert check_value_residual(ref.value_residual, rng)
    assert check_k_update(ref.k_update, rng)
    assert check_head_l2norm(ref.head_l2norm, rng)
    assert check_group_norm(ref.group_norm, rng)
    assert check_bonus(ref.bonus, rng)


def _l2norm_per_lane(kk, c):
    return kk * ref.poly(c, np.sum(kk * kk, axis=1, keepdims=True))


def _gn_per_lane(y, c, w, b):
    yc = y - y.mean(axis=1, keepdims=True)
    return yc * ref.poly(c, np.mean(yc * yc, axis=1, keepdims=True)) * w + b


def _gn_bias_multiplied(y, c, w, b):
    return ref.group_norm(y, c, w, np.zeros_like(b)) * (1 + b)


def _bonus_per_lane(y, r, k, rk, v):
    return y + np.sum(r * k * rk, axis=1, keepdims=True) * v


def _bonus_unsummed(y, r, k, rk, v):
    return y + r * k * rk * v


@pytest.mark.parametrize("check,mutant", [
    (check_value_residual, lambda v, v0, g: v + (v - v0) * g),
    (check_k_update, lambda k, a, ka: k * (a - 1) * ka),
    (check_head_l2norm, _l2norm_per_lane),
    (check_group_norm, _gn_per_lane),
    (check_group_norm, _gn_bias_multiplied),
    (check_bonus, _bonus_per_lane),
    (check_bonus, _bonus_unsummed),
], ids=["residual-reversed", "k-term-dropped", "l2norm-per-lane", "groupnorm-per-lane", "ln-bias-multiplied",
        "bonus-per-lane", "bonus-unsummed"])
def test_time_mix_part_mutants_fail(check, mutant):
    assert not check(mutant, np.random.default_rng(22))


def _two_layers():
    L0 = _identity_layer()
    L1 = _identity_layer()
    L1["mu_k"] = np.zeros(ref.D)          # k reads the layer's own input
    L1["W_v"] = np.zeros((ref.D, ref.D))  # the layer's own value is 0 ...
    L1["p_v"] = np.array([1.0, 0, 0, 0])  # ... and the gate 1: its value is the first layer's
    return {"layers": [L0, L1], "p_o": np.array([1.0, 0, 0, 0]), "g_o": np.ones(ref.D)}


def test_first_layer_value_reaches_the_second():
    """layer 0 (k from the carry: S stays 0, y = 0) leaves x' = 2.5 x and its value v0 = x; layer 1 (value 0, gate 1)
    updates its state from S = 0 with v0 and its own k = its input: S_1 = x (2.5 x)^T per head"""
    rng = np.random.default_rng(23)
    W = _two_layers()
    x = 0.3 * rand(rng, 2, ref.D)
    st = ref.init_state(2, 2)
    ref.step(x, st, W)
    h = x.reshape(2, 12, 64)
    assert np.allclose(st[1]["S"], np.einsum("lhi,lhj->lhij", h, 2.5 * h), atol=1e-13)


def test_own_value_mutant_fails():
    """the same run with each layer mixing toward its own value (v0 reset per layer) gives S_1 = 0"""
    rng = np.random.default_rng(23)
    W = _two_layers()
    x = 0.3 * rand(rng, 2, ref.D)
    st = ref.init_state(2, 2)
    x1, _ = ref.layer(x, st[0], W["layers"][0])
    ref.layer(x1, st[1], W["layers"][1], None)   # the mutant: no v0 passed on
    h = x.reshape(2, 12, 64)
    assert not np.allclose(st[1]["S"], np.einsum("lhi,lhj->lhij", h, 2.5 * h), atol=1e-13)
