"""The client's file steps through the C ABI (fhe_ssm_client_encrypt_rows / fhe_ssm_client_decrypt_logits: the
reference driver's --enc-in and --dec-out, hpc_gpu_port/gpu_real_model.cu:2345-2533) at config-2 parameters.

- enc-in, word level: token t's file holds exactly ckks_encode + ckks_encrypt_public (seed, index t) of the slot
  vector the reference builds from lane-major rows (slot rep*dpad + i = lane (rep mod lanes) channel i, every
  replica, :2378-2395); the public-key encryption itself is pinned bit-exact against the oracle in test_gpu_pk.py.
- enc-in, decrypted: the slots decrypt to the rows (relErrRms < 1e-7 at 2^40 over all slots; every replica
  checked), so a transposed or mis-strided layout fails even where the word check would agree with itself.
- meta: the reference's keys in its order (writeCtMeta, :2333-2340).
- dec-out: the logits file is tokens x lanes rows of head @ (lane's channels), token-major, lane-minor
  (:2468-2522), within 1e-5 relative of the float64 product of the plaintext rows; a meta whose layout differs is
  refused.
"""
import json
import os

import numpy as np
import pytest

from engine_loader import load_ckks, load_module

pytestmark = pytest.mark.gpu

L, K, DNUM = 24, 8, 3
N = 1 << 16
SLOTS = N // 2
SCALE = 2.0**40
SEED = b"client-files-seed".ljust(32, b"\0")


@pytest.fixture(scope="module")
def setup():
    ckks = load_ckks()
    ND = load_module("native_decode")
    ctx = ckks.Context(num_q=L, num_p=K, dnum=DNUM, q_bits=54, p_bits=60, scale=SCALE)
    sk = ctx.secret(b"client-files-secret".ljust(32, b"\0"), 192)
    d_pk = ckks.DeviceBuffer(2 * (L + K) * N * 8)
    ctx.keygen_public(sk, b"pk".ljust(32, b"\0"), b"pk-e".ljust(32, b"\0"), d_pk.ptr)
    return ckks, ND, ctx, sk, d_pk


def expected_slots(rows, t, lanes, d, dpad):
    sv = np.zeros(SLOTS)
    for rep in range(SLOTS // dpad):
        sv[rep * dpad:rep * dpad + d] = rows[rep % lanes, t]
    return sv


@pytest.mark.parametrize("lanes,d,dpad,level", [(3, 40, 64, 12), (1, 64, 64, 24)])
def test_encrypt_rows_files(setup, tmp_path, lanes, d, dpad, level):
    ckks, ND, ctx, sk, d_pk = setup
    tokens = 2
    rng = np.random.default_rng(lanes * 100 + d)
    rows = rng.uniform(-1, 1, (lanes, tokens, d))
    path = str(tmp_path / "rows.f64")
    rows.astype("<f8").tofile(path)
    ND.client_encrypt_rows(ctx, d_pk.ptr, path, tokens, lanes, d, dpad, level, SCALE, SEED)

    meta = open(path + ".ct.meta").read()
    assert list(json.loads(meta)) == ["count", "packTokens", "tokensReal", "dpad", "interleave", "lanes", "ringDim",
                                      "level"]
    assert json.loads(meta) == {"count": tokens, "packTokens": 1, "tokensReal": tokens, "dpad": dpad,
                                "interleave": 0, "lanes": lanes, "ringDim": N, "level": level}

    d_ct = ckks.DeviceBuffer(2 * L * N * 8)
    d_pt = ckks.DeviceBuffer(level * N * 8)
    d_want = ckks.DeviceBuffer(2 * level * N * 8)
    for t in range(tokens):
        got_level, got_scale = ctx.ct_load(f"{path}.ct.{t}", d_ct.ptr, L)
        assert got_level == level and got_scale == SCALE
        sv = expected_slots(rows, t, lanes, d, dpad)
        ctx.encode(sv, level, SCALE, d_pt.ptr)
        ctx.encrypt_public(d_pk.ptr, d_pt.ptr, level, SEED, t, d_want.ptr)
        assert np.array_equal(d_ct.download((2, level, N)), d_want.download((2, level, N))), f"token {t}"
        # every slot against the layout rule; padding channels decrypt to zero.  The public-key ciphertext's
        # error is the ModDown rounding (u0 + u1 s, 0 <= u < K): not centred, so it gathers in the few slots whose
        # roots lie near 1 (|sum_k zeta^k| ~ 2N/pi); the max bound (K h + K + 1) N / scale covers every slot.
        dec = ctx.decrypt(sk, d_ct.ptr, level, SCALE)
        assert np.sqrt(np.mean((dec - sv) ** 2)) < 1e-7 * np.sqrt(np.mean(sv ** 2)), t
        assert np.abs(dec - sv).max() < (K * 192 + K + 1) * N / SCALE, t
        for rep in (0, 1, lanes, SLOTS // dpad - 1):
            assert np.abs(dec[rep * dpad:rep * dpad + d] - rows[rep % lanes, t]).max() < 1e-5, (t, rep)


def test_decrypt_logits_file(setup, tmp_path):
    ckks, ND, ctx, sk, d_pk = setup
    lanes, tokens, d, dpad, vocab, level = 4, 3, 48, 64, 50, 6
    rng = np.random.default_rng(7)
    rows = rng.uniform(-1, 1, (lanes, tokens, d))
    head = rng.normal(0, 0.2, (vocab, d))
    path = str(tmp_path / "rows.f64")
    rows.astype("<f8").tofile(path)
    ND.client_encrypt_rows(ctx, d_pk.ptr, path, tokens, lanes, d, dpad, level, SCALE, SEED)
    ND.client_decrypt_logits(ctx, sk, path + ".ct", head, dpad)
    got = np.fromfile(path + ".ct.logits.f64", dtype="<f8")
    assert got.size == tokens * lanes * vocab
    got = got.reshape(tokens, lanes, vocab)
    want = np.einsum("vd,ltd->tlv", head, rows)
    rel = np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2))
    assert rel < 1e-5, rel

    # a meta whose dpad differs from the caller's is the reference's "layout mismatch"
    with pytest.raises(RuntimeError, match="layout mismatch"):
        ND.client_decrypt_logits(ctx, sk, path + ".ct", head, 2 * dpad)


def test_encrypt_rows_refuses_a_short_file(setup, tmp_path):
    ckks, ND, ctx, sk, d_pk = setup
    path = str(tmp_path / "short.f64")
    np.zeros(2 * 3 * 10 - 1).astype("<f8").tofile(path)
    with pytest.raises(RuntimeError, match="short file"):
        ND.client_encrypt_rows(ctx, d_pk.ptr, path, 3, 2, 10, 16, 4, SCALE, SEED)
    assert not os.path.exists(path + ".ct.meta")
