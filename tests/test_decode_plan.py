"""The config-5 decode step's plan on the slot-vector simulator (CPU): the encrypted driver
(fhe-ssm_amd/decode_step.py) with every primitive applied to plain slot values must reproduce the float64
reference model (oracle/rwkv_ref.py), which is written in matrix form without slots, diagonals or
rotations.  This pins the packing algebra: BSGS diagonals and their pre-rotation, the lane-sum and
broadcast of the norms, the WKV diagonal layout and its masked block rotations, the state packing (4 -> 3 into the
unused channels, then two per complex ciphertext) and unpacking, and the token-shift carries across steps."""
import numpy as np
import pytest

from slot_backend import DS, M, SlotBackend
from oracle import rwkv_ref as ref


def test_wkv_layout_roundtrip():
    rng = np.random.default_rng(1)
    S = rng.standard_normal((32, 12, 64, 64))
    Dg = M.state_to_diag(S)
    assert Dg.shape == (64, 1 << 15)
    assert np.array_equal(M.diag_to_state(Dg), S)


def test_masked_block_rotation():
    """m_lo,t (.) Rot_t(x) + m_hi,t (.) Rot_{t-64}(x) is the cyclic rotation by t inside each 64-block"""
    rng = np.random.default_rng(2)
    x = M.pack_lanes(rng.standard_normal((32, 768)))
    masks = M.wkv_masks()
    for t in (0, 1, 17, 63):
        got = np.tile(masks[t, 0], 32) * np.roll(x, -M.WKV_LO[t]) + np.tile(masks[t, 1], 32) * np.roll(x, -M.WKV_HI[t])
        blocks = x.reshape(32, 16, 64)
        want = np.roll(blocks, -t, axis=2).reshape(-1)
        want.reshape(32, 1024)[:, 768:] = 0
        assert np.allclose(got, want, atol=0), t


@pytest.mark.parametrize("n_in,n_out", [(1, 1), (2, 1), (1, 3)])
def test_matvec_diagonals(n_in, n_out):
    """the BSGS sum over the diagonals is the block matvec, for both baby/giant splits (nb = 64 when n_out >= n_in)"""
    rng = np.random.default_rng(3)
    A = rng.standard_normal((n_out, n_in, 768, 768))
    d = M.matvec_diagonals([[A[o, i] for i in range(n_in)] for o in range(n_out)])
    nb = M.mv_nb(n_in, n_out)
    assert d.shape == (n_out, M.MV_SPAN // nb, n_in * nb, M.DPAD) and nb == (64 if n_out >= n_in else 32)
    x = rng.standard_normal((n_in, 32, 768))
    xs = [M.pack_lanes(x[i]) for i in range(n_in)]
    for o in range(n_out):
        y = np.zeros(1 << 15)
        for gi, G in enumerate(M.mv_giants(nb)):
            acc = sum(np.tile(d[o, gi, i * nb + b], 32) * np.roll(xs[i], -b) for i in range(n_in) for b in range(nb))
            y += np.roll(acc, -G)
        want = sum(x[i] @ A[o, i].T for i in range(n_in))
        assert np.allclose(M.unpack_lanes(y), want, atol=1e-9)
        assert np.all(y.reshape(32, 1024)[:, 768:] == 0)


@pytest.mark.timeout(300)
def test_decode_step_plan_matches_reference():
    """two layers (the second mixes its value toward the first's), two tokens with the state carried"""
    W = M.make_weights(5, n_layers=2)
    be = SlotBackend(17)
    step = DS.DecodeStep(be, W)
    st = ref.init_state(32, 2)
    for s in range(2):
        x = M.embed_tokens(np.arange(32) + 100 * s)
        out = step(be.encrypt(None, M.pack_lanes(x), 17))
        xo, _ = ref.step(x, st, W)
        got = M.unpack_lanes(be.decrypt(None, out))
        assert np.max(np.abs(got - xo)) < 1e-12
        assert np.max(np.abs(be.decrypt(None, out).reshape(32, 1024)[:, 768:])) == 0
        for li in range(2):
            Dg = np.stack([ct.v[i].real for ct, i in step.state_diagonals(li)])
            assert np.allclose(M.diag_to_state(Dg), st[li]["S"], atol=1e-14)
    # per layer and step: y with its bonus coefficient, the two increments and the 24 packed state ciphertexts;
    # the residual stays on top
    assert step.stats["bootstraps"] == 2 * 2 * 28
    assert [e[1] for e in be.log[:4]] == ["state", "inc_tm", "state", "inc_cm"]
    assert out.level == 11


def test_head_sum_and_masks():
    """the per-head sums the L2 norm, GroupNorm and bonus use: rotate-and-add by 1 .. 32 within each lane, the
    head-start mask, broadcast back; the gap channels stay zero"""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((32, 768))
    be = SlotBackend(17)
    step = DS.DecodeStep(be, M.make_weights(5, n_layers=1))
    got = M.unpack_lanes(be.decrypt(None, step._head_sum(be.encrypt(None, M.pack_lanes(x), 17), 0.5)))
    want = np.repeat(0.5 * x.reshape(32, 12, 64).sum(axis=2), 64, axis=1)
    assert np.allclose(got.real, want, atol=1e-12)
