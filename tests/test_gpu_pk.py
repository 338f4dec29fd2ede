"""GPU parity of the public key and public-key encryption (ckks_keygen_public / ckks_encrypt_public) against the
oracle restatement (oracle/ckks_oracle.c or_pk_gen / or_pk_encrypt, pinned in tests/test_oracle_pk.py), through the
C ABI, at config-2 parameters (N = 2^16, L = 24 x 54-bit, K = 8 x 60-bit, dnum = 3, h = 192).  Bar: bit-exact words
for the key and for ciphertexts at two levels; the ciphertexts decrypt to their slots (relErrRms < 1e-7 at 2^40)."""
import numpy as np
import pytest

from engine_loader import load_ckks

pytestmark = pytest.mark.gpu

L, K, DNUM = 24, 8, 3
N = 1 << 16
SEED = b"pk-gpu-seed".ljust(32, b"\0")
ESEED = b"pk-gpu-eseed".ljust(32, b"\0")


@pytest.fixture(scope="module")
def setup(oracle):
    ckks = load_ckks()
    ctx = ckks.Context(num_q=L, num_p=K, dnum=DNUM, q_bits=54, p_bits=60, scale=2.0**40)
    sk = ctx.secret(b"pk-secret".ljust(32, b"\0"), 192)
    octx = oracle.Ctx(16, ctx.moduli, L, K, DNUM)
    s_eval = octx.small_to_eval(sk.coeffs().astype(np.int8), list(range(L + K)))
    d_pk = ckks.DeviceBuffer(2 * (L + K) * N * 8)
    ctx.keygen_public(sk, SEED, ESEED, d_pk.ptr)
    return ckks, ctx, sk, octx, s_eval, d_pk


def test_public_key_bit_exact(setup):
    ckks, ctx, sk, octx, s_eval, d_pk = setup
    want = octx.pk_gen(s_eval, SEED, ESEED)
    assert np.array_equal(d_pk.download((2, L + K, N)), want)


@pytest.mark.parametrize("level", [24, 9])
def test_public_key_encryption_bit_exact_and_decrypts(setup, level):
    ckks, ctx, sk, octx, s_eval, d_pk = setup
    rng = np.random.default_rng(level)
    z = rng.uniform(-1, 1, N // 2)
    d_pt = ckks.DeviceBuffer(level * N * 8)
    ctx.encode(z, level, 2.0**40, d_pt.ptr)
    d_ct = ckks.DeviceBuffer(2 * level * N * 8)
    ctx.encrypt_public(d_pk.ptr, d_pt.ptr, level, b"pk-enc".ljust(32, b"\0"), 5, d_ct.ptr)
    pk = d_pk.download((2, L + K, N))
    want = octx.pk_encrypt(pk, d_pt.download((level, N)), level, b"pk-enc".ljust(32, b"\0"), 5)
    assert np.array_equal(d_ct.download((2, level, N)), want)
    got = ctx.decrypt(sk, d_ct.ptr, level, 2.0**40)
    rel = float(np.sqrt(np.mean((got - z) ** 2)) / np.sqrt(np.mean(z ** 2)))
    assert rel < 1e-7, rel
