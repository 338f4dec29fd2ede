"""GPU test of the allocation-free entry point ckks_eval_mult_rescale_noalloc, through the C ABI: on two calls in
a row, the second with a smaller input, its output words equal those of ckks_eval_mult_rescale (the allocating
entry point it mirrors) on the same inputs; a call does not take device memory; a shape whose workspace exceeds
the scratch is refused with CKKS_EINVAL and leaves the output untouched.  Inputs are seeded uniform residues (the
HMult + relinearize + rescale words are a deterministic function of the input words).  Config-2 parameters:
N = 2^16, L = 24 x 54-bit, K = 8 x 60-bit, dnum = 3."""
import numpy as np
import pytest

from engine_loader import load_ckks

pytestmark = pytest.mark.gpu

L, K, DNUM = 24, 8, 3
N = 1 << 16


def residues(moduli, shape_prefix, prime_idx, seed):
    rng = np.random.default_rng(seed)
    q = np.array([moduli[i] for i in prime_idx], dtype=np.uint64)
    x = rng.integers(0, 2**63, tuple(shape_prefix) + (len(prime_idx), N), dtype=np.uint64)
    return x % q.reshape((1,) * len(shape_prefix) + (-1, 1))


def hip_runtime_path():
    """the HIP runtime the engine library itself linked: the libamdhip64 object mapped into this process once the
    engine is loaded (whatever its soname on this ROCm)"""
    load_ckks().load()
    with open("/proc/self/maps") as f:
        for line in f:
            path = line.split()[-1]
            if "libamdhip64.so" in path.rsplit("/", 1)[-1]:
                return path
    raise RuntimeError("the engine library is loaded but no libamdhip64 is mapped")


def free_device_bytes():
    """hipMemGetInfo of the HIP runtime the engine library itself links (already loaded with it)"""
    import ctypes
    hip = ctypes.CDLL(hip_runtime_path())
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_hmult_equals_the_allocating_entry_point():
    ckks = load_ckks()
    # a fresh context: none of the call's tables are in its caches yet, so the first calls build them in scratch
    ctx = ckks.Context(num_q=L, num_p=K, dnum=DNUM, q_bits=54, p_bits=60)
    d_evk = ckks.DeviceBuffer.from_array(residues(ctx.moduli, (DNUM, 2), list(range(L + K)), seed=11))
    for call, (B, l) in enumerate([(1, 24), (1, 13)]):
        print(f"noalloc call {call}: batch {B}, level {l}", flush=True)
        da = ckks.DeviceBuffer.from_array(residues(ctx.moduli, (B, 2), list(range(l)), seed=100 + call))
        db = ckks.DeviceBuffer.from_array(residues(ctx.moduli, (B, 2), list(range(l)), seed=200 + call))
        shape = (B, 2, l - 1, N)
        out_na = ckks.DeviceBuffer(B * 2 * (l - 1) * N * 8)
        out_ref = ckks.DeviceBuffer(B * 2 * (l - 1) * N * 8)
        ckks.sync()
        free0 = free_device_bytes()
        ctx.eval_mult_rescale_noalloc(da.ptr, db.ptr, B, l, d_evk.ptr, out_na.ptr)
        ckks.sync()
        free1 = free_device_bytes()
        got = out_na.download(shape)
        # the allocating path's workspace alone would be >= 70 MiB at these shapes
        assert free0 - free1 < (32 << 20), f"call {call} took {(free0 - free1) >> 20} MiB of device memory"
        ctx.eval_mult_rescale(da.ptr, db.ptr, B, l, d_evk.ptr, out_ref.ptr)
        want = out_ref.download(shape)
        assert np.array_equal(got, want), f"call {call}: words differ"
        # and once more now that the allocating call has filled the context's caches
        ctx.eval_mult_rescale_noalloc(da.ptr, db.ptr, B, l, d_evk.ptr, out_na.ptr)
        assert np.array_equal(out_na.download(shape), want), f"call {call} (warm caches): words differ"
        for buf in (da, db, out_na, out_ref):
            buf.free()


def test_noalloc_refuses_a_workspace_beyond_its_scratch():
    ckks = load_ckks()
    ctx = ckks.Context(num_q=L, num_p=K, dnum=DNUM, q_bits=54, p_bits=60)
    B, l = 2, 24  # 2 x 280 limbs of 512 KiB: beyond 159 MiB
    d_evk = ckks.DeviceBuffer.from_array(residues(ctx.moduli, (DNUM, 2), list(range(L + K)), seed=12))
    da = ckks.DeviceBuffer.from_array(residues(ctx.moduli, (B, 2), list(range(l)), seed=5))
    out = ckks.DeviceBuffer(B * 2 * (l - 1) * N * 8)
    out.upload(np.zeros((B, 2, l - 1, N), dtype=np.uint64))
    with pytest.raises(ckks.CkksError, match="scratch|workspace"):
        ctx.eval_mult_rescale_noalloc(da.ptr, da.ptr, B, l, d_evk.ptr, out.ptr)
    assert not out.download((B, 2, l - 1, N)).any()
    # a fitting call right after the refusal still works and matches the allocating path
    ref = ckks.DeviceBuffer(2 * (l - 1) * N * 8)
    ctx.eval_mult_rescale_noalloc(da.ptr, da.ptr, 1, l, d_evk.ptr, out.ptr)
    ctx.eval_mult_rescale(da.ptr, da.ptr, 1, l, d_evk.ptr, ref.ptr)
    assert np.array_equal(out.download((1, 2, l - 1, N)), ref.download((1, 2, l - 1, N)))
