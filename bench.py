#!/usr/bin/env python3
"""Benchmark of the MI355X RNS-CKKS hot path; prints ONE JSON line.

Workloads (inputs seeded and resident in HBM before the timed region):
  hmult  config 2 (default): CKKS HMult + relinearize + rescale on 64 ciphertext pairs, N=2^16,
         L=24 x 54-bit + K=8 x 60-bit, hybrid key switching dnum=3; ternary secret h=192, Gaussian
         errors sigma=3.19, slots uniform in [-1,1] at scale 2^50.  One step = one batched
         EvalMult+Rescale over the 64 pairs.  value = HMult+relin ops/s.
  ntt    config 1: forward then inverse NTT over 64 ct x 2 polys x 24 limbs.  value = algorithmic GB/s.
  pcmm   config 3: 768x768 plaintext matrix x one ciphertext (L=16) by BSGS 28 x 28.  value = ms.
  bootstrap  config 4: full-slot bootstrap of a level-1 ciphertext (scale 2^55 under a 60-bit q0).  value = ms;
         precision in bits.
  decode config 5: one encrypted decode step of the RWKV-7-0.1B-shaped model (12 layers, 32 lanes, state
         carried, bootstrapped once per layer).  value = s/step; decrypted output and logits checked
         against the float64 model.
The default run also reports the config-1, -3, -4 and -5 figures beside the config-2 metric.

Roofline: `roofline` is the step-level figure of SURVEY 8(d): the unit's algorithmic bytes times the units
one timed engine call processes (config 2: 175,112,192 B x 64 pairs), over the call's mean time by HIP events
on its stream, against the MI355X HBM peak (8 TB/s) and against the stream rate measured on the box
(profiles/hbm_stream.md); `traffic` is the step's counter-measured HBM bytes summed over all its dispatches.
`kernel_io` is the dominant launch of one profiled step (the engine records HIP events on its launch stream
around every kernel, ckks_profile_*): its own I/O bytes (intermediates included) over its mean launch time.
cpu_baseline: this repository's C oracle (an OpenFHE-convention restatement, not OpenFHE, which needs
the network to build) timed on the host over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes
import gc
import json
import os
import shutil
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tests"))

HBM_PEAK_GBS = 8000.0
N = 1 << 16
LIMB_BYTES = N * 8
TWIDDLE_BYTES_PER_PRIME = N * 16  # (w, w') pairs

L2, K2, DNUM2 = 24, 8, 3
N_PAIRS = 64


def seed_bytes(tag: str, seed: int) -> bytes:
    b = (tag.encode() + seed.to_bytes(8, "little")) * 4
    return b[:32]


def timed_steps(torch, stream, step, steps, warmup):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(steps):
        step()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return wall, per


# Achievable HBM bandwidth on the box, measured by the stream kernels of fhe-ssm_amd/microbench/copy_bw.hip (8 GiB
# read-only nontemporal stream; 4 GiB nontemporal copy, read + write bytes; the output is in profiles/hbm_stream.md).
# A rate whose bytes are at least 10% writes is divided by the copy figure, a read-dominated one by the read figure.
STREAM_READ_GBS = 7167.4
STREAM_COPY_GBS = 5498.6
STREAM_SOURCE = "profiles/hbm_stream.md"
# engine launches whose bytes are >= 90% reads (plaintext diagonals, keys and extensions streamed, few outputs)
READ_DOMINATED = {"bsgs_mac", "bsgs_mac_periodic", "bsgs_dh_mac", "qp_rot_sum"}


def achievable(write_share: float) -> float:
    return STREAM_READ_GBS if write_share < 0.1 else STREAM_COPY_GBS


# Counter-measured figures from rocprofv3 --pmc passes over the same bench command (one pass per counter group; the
# summaries and commands are in profiles/):
#   traffic: HBM bytes, read = 2 x FETCH_SIZE KiB, write = WRITE_SIZE KiB (the scaling a copy kernel of known size
#            reads off the two counters); for ("workload", "step") summed over every dispatch of one step;
#   valu:    wave64 VALU instructions issued (SQ_INSTS_VALU, all waves of the launch).
# A kernel "launch" is one engine call (both kernels of a two-pass NTT).  Measured, not computed: re-measure when the
# kernel or the workload changes.
MEASURED = {
    ("hmult", "step"): {"traffic": 33.103e9, "source": "profiles/hmult_config2_kernels.md"},
    ("hmult", "ntt_fwd_mdr"): {"traffic": 10.905e9, "valu_insts": 879.5e6, "source": "profiles/hmult_config2_kernels.md"},
    ("hmult", "ntt_fwd_2pass"): {"traffic": 9.700e9, "valu_insts": 776.7e6, "source": "profiles/hmult_config2_kernels.md"},
    ("ntt", "step"): {"traffic": 12.940e9, "source": "profiles/ntt_config1_kernel_trace.md"},
    ("pcmm", "step"): {"traffic": 18.373e9, "source": "profiles/pcmm_config3_kernel_trace.md"},
    ("pcmm", "bsgs_mac"): {"traffic": 7.382e9, "source": "profiles/pcmm_config3_kernel_trace.md"},
    ("bootstrap", "step"): {"traffic": 53.876e9, "source": "profiles/bootstrap_config4_kernel_trace.md"},
    ("decode", "step"): {"traffic": 21302.8e9, "source": "profiles/decode_config5_kernel_trace.md"},
    ("ntt", "ntt_fwd_2pass"): {"traffic": 6.470e9, "valu_insts": 480.5e6, "source": "profiles/ntt_config1_kernel_trace.md"},
    ("ntt", "ntt_inv_2pass"): {"traffic": 6.470e9, "valu_insts": 482.3e6, "source": "profiles/ntt_config1_kernel_trace.md"},
}
# int-VALU issue peak: 256 CUs x 4 SIMDs, one wave64 VALU instruction per SIMD every 4 cycles (16 lanes) at the
# 2.4 GHz peak engine clock
VALU_PEAK_GINSTS = 1024 * 2.4 / 4
# the rate v_mad_u64_u32 sustains on the box (fhe-ssm_amd/microbench/valu_rate.hip: 4.94 cycles per wave64
# instruction at the 2.4 GHz clock; profiles/valu_rates.md)
VALU_MAD_GINSTS = 1024 * 2.4 / 4.94


def step_roofline(workload: str, alg_bytes: float, step_ms: float, write_share: float, scope: str) -> dict:
    """The step-level HBM roofline: SURVEY 8(d)'s algorithmic bytes for one timed step (the unit times the units one
    engine call processes) over the step's HIP-event time, against the data-sheet peak and the measured stream rate;
    traffic = the counter-measured HBM bytes of one step summed over all its dispatches."""
    ach = alg_bytes / (step_ms * 1e-3) / 1e9
    stream = achievable(write_share)
    meas = MEASURED.get((workload, "step"), {})
    out = {"bound": "hbm", "scope": scope, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": meas.get("traffic"),
           "algorithmic_bytes_per_step": int(round(alg_bytes)), "step_ms": round(step_ms, 4),
           "achievable": stream, "frac_of_achievable": round(ach / stream, 4), "achievable_source": STREAM_SOURCE}
    if meas:
        out["traffic_over_algorithmic"] = round(meas["traffic"] / alg_bytes, 3)
        out["traffic_GBps"] = round(meas["traffic"] / (step_ms * 1e-3) / 1e9, 1)
        out["traffic_source"] = meas["source"]
    return out


def kernel_io(rep: dict, workload: str = ""):
    """The dominant engine launch of one profiled step by time: its own I/O bytes (every array it reads or writes,
    intermediates included, each once) over its mean launch time (HIP events on the launch stream)."""
    name, (n, ms, by) = max(rep.items(), key=lambda kv: kv[1][1])
    rate = by / (ms * 1e-3) / 1e9
    stream = STREAM_READ_GBS if name in READ_DOMINATED else STREAM_COPY_GBS
    meas = MEASURED.get((workload, name), {})
    out = {"kernel": name, "achieved": round(rate, 1), "unit": "GB/s", "frac": round(rate / HBM_PEAK_GBS, 4),
           "achievable": stream, "frac_of_achievable": round(rate / stream, 4), "traffic": meas.get("traffic"),
           "launches_in_profiled_step": n, "mean_launch_ms": round(ms / n, 4), "io_bytes_per_launch": round(by / n)}
    if meas.get("valu_insts"):
        g = meas["valu_insts"] / (ms / n * 1e-3) / 1e9
        out["valu"] = {"achieved": round(g, 1), "peak": VALU_PEAK_GINSTS, "unit": "G wave64 VALU inst/s",
                       "frac": round(g / VALU_PEAK_GINSTS, 4), "insts_per_launch": meas["valu_insts"],
                       "frac_of_measured_mad_rate": round(g / VALU_MAD_GINSTS, 4)}
    if meas:
        out["counters_source"] = meas["source"]
    return out


def kernel_table(rep: dict):
    return {k: {"launches": n, "total_ms": round(ms, 4), "GBps": round(by / (ms * 1e-3) / 1e9, 1)}
            for k, (n, ms, by) in sorted(rep.items(), key=lambda kv: -kv[1][1])}


def profile_bytes(rep: dict) -> float:
    """the engine's algorithmic (own-I/O) bytes summed over every launch of a profiled step"""
    return float(sum(by for (_, _, by) in rep.values()))


# ----------------------------------------------------------------------------------------- config 2
def bench_hmult(ckks, torch, steps, warmup, seed):
    ctx = ckks.Context(num_q=L2, num_p=K2, dnum=DNUM2, q_bits=54, p_bits=60, scale=2.0**50)
    scale = 2.0**50
    sk = ctx.secret(seed_bytes("secret", seed), 192)
    T = L2 + K2
    dev = torch.device("cuda:0")
    evk = torch.empty((DNUM2, 2, T, N), dtype=torch.int64, device=dev)
    ctx.keygen_relin(sk, seed_bytes("relin-a", seed), seed_bytes("relin-e", seed), evk.data_ptr())
    A = torch.empty((N_PAIRS, 2, L2, N), dtype=torch.int64, device=dev)
    B = torch.empty_like(A)
    OUT = torch.empty((N_PAIRS, 2, L2 - 1, N), dtype=torch.int64, device=dev)
    pt = torch.empty((L2, N), dtype=torch.int64, device=dev)
    rng = np.random.default_rng(seed)
    msgs = {}
    ct_bytes = 2 * L2 * N * 8
    for i in range(2 * N_PAIRS):
        z = rng.uniform(-1.0, 1.0, N // 2)
        if i in (0, N_PAIRS, 1, N_PAIRS + 1):
            msgs[i] = z
        ctx.encode(z, L2, scale, pt.data_ptr())
        dst = (A if i < N_PAIRS else B)
        ctx.encrypt(sk, pt.data_ptr(), L2, seed_bytes("enc", seed), i,
                    dst.data_ptr() + (i % N_PAIRS) * ct_bytes)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)

    def step():
        ctx.eval_mult_rescale(A.data_ptr(), B.data_ptr(), N_PAIRS, L2, evk.data_ptr(), OUT.data_ptr(), sh)

    wall, per = timed_steps(torch, stream, step, steps, warmup)
    step_ms = wall * 1e3 / steps
    # decrypted check of the timed outputs: product of the inputs, scale Delta^2 / q_{L-1}
    out_scale = scale * scale / ctx.moduli[L2 - 1]
    errs = []
    for i in (0, 1):
        got = ctx.decrypt(sk, OUT.data_ptr() + i * 2 * (L2 - 1) * N * 8, L2 - 1, out_scale)
        want = msgs[i] * msgs[N_PAIRS + i]
        errs.append(float(np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2))))
    rel_err = max(errs)
    if not rel_err < 1e-6:
        raise SystemExit(f"HMult output does not decrypt to the product (relErrRms {rel_err:.3e}): invalid")
    # one profiled step: per-kernel HIP events on the launch stream
    ctx.profile_reset()
    ctx.profile(True)
    step()
    torch.cuda.synchronize()
    ctx.profile(False)
    rep = ctx.profile_report()
    ctx.profile_reset()
    ops = N_PAIRS / (step_ms * 1e-3)
    res = {
        "metric": "HMult+relin ops/s at N=2^16",
        "value": round(ops, 1),
        "unit": "ops/s",
        "ms_per_step": round(step_ms, 4),
        "dtype": "u64",
        "config": {"workload": "config2: HMult+relin+rescale, 64 ciphertext pairs, N=2^16, L=24x54-bit + "
                               "K=8x60-bit, dnum=3, h=192, sigma=3.19, scale 2^50",
                   "batch": N_PAIRS, "level_in": L2, "ntt_mode": "two-pass", "seed": seed,
                   "step_ms_min": round(min(per), 4), "step_ms_max": round(max(per), 4)},
        "check": {"decrypted_relErrRms_max": rel_err, "ciphertexts_checked": 2},
        "kernels": kernel_table(rep),
        "roofline": step_roofline("hmult", N_PAIRS * HMULT_UNIT_BYTES, step_ms, 46 / 334,
                                  "step: one ckks_eval_mult_rescale call over 64 pairs; SURVEY 8(d) config-2 unit "
                                  "175,112,192 B per op (inputs 96 + evk 192 + output 46 limbs) x 64"),
        "kernel_io": kernel_io(rep, "hmult"),
        "ks_stage": ks_stage(rep, step_ms),
    }
    res["roofline"]["evk_amortised"] = step_roofline(
        "", N_PAIRS * HMULT_EVK_AMORTISED_BYTES, step_ms, 46 / 145,
        "the same step with the evk counted once per 64 ops: 76,021,760 B per op")
    return res


# SURVEY 8(d) config-2 units per op: HMult+relin+rescale (inputs 96 + evk 192 + output 46 limbs), the same with the
# evk amortised over the batch (96 + 3 + 46 limbs), and the key-switching unit (d2 24 + evk 192 + output 48 limbs)
HMULT_UNIT_BYTES = 175_112_192
HMULT_EVK_AMORTISED_BYTES = 76_021_760
KS_UNIT_BYTES = 138_412_032


def ks_stage(rep: dict, step_ms: float):
    """the key-switching part of the timed HMult step (every kernel but the tensor product; the rescale is fused into
    the ModDown) against the key-switching unit: its time is the timed step's scaled by the key-switching kernels'
    share of the profiled step's kernel time (per-kernel events make a profiled step longer than a timed one)"""
    ks_ms_prof = sum(v[1] for k, v in rep.items() if k != "tensor")
    all_ms_prof = sum(v[1] for v in rep.values())
    ms = step_ms * ks_ms_prof / all_ms_prof
    gbs = N_PAIRS * KS_UNIT_BYTES / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 4), "share_of_step": round(ks_ms_prof / all_ms_prof, 4),
            "algorithmic_bytes": N_PAIRS * KS_UNIT_BYTES, "achieved": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "frac_of_achievable": round(gbs / STREAM_COPY_GBS, 4),
            "kernels": sorted(k for k in rep if k != "tensor")}


def host_cpu():
    """the host's processor model and logical CPU count (recorded beside every CPU figure)"""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "nproc": os.cpu_count() or 1}


def host_threads():
    """threads for an all-core leg: the job's CPU share where the environment states one (OMP_NUM_THREADS), else
    every processor"""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "")))
    except ValueError:
        return os.cpu_count() or 1


def cpu_baseline_hmult(seed, budget_s=10.0):
    """Oracle HMult+relin+rescale on real-shaped random words of the config-2 context: one thread, then every host
    thread with one pair per thread (OpenMP over the pairs)."""
    from oracle import oracle as o
    qs = o.gen_primes(54, L2, 2 * N)
    ps = o.gen_primes(60, K2, 2 * N, exclude=qs)
    octx = o.Ctx(16, qs + ps, L2, K2, DNUM2)
    rng = np.random.default_rng(seed)
    q = np.array(qs, dtype=np.uint64)[:, None]
    T = L2 + K2
    qp = np.array(qs + ps, dtype=np.uint64)[:, None]
    evk = (rng.integers(0, 2**63, (DNUM2, 2, T, N), dtype=np.uint64) % qp[None, None])
    pair = lambda n: rng.integers(0, 2**63, (n, 2, L2, N), dtype=np.uint64) % q[None, None]
    done, el = 0, 0.0  # the time of the HMult calls only (input generation left out)
    while el < budget_s and done < 4:
        a, b = pair(1), pair(1)
        t = time.perf_counter()
        octx.hmult_relin_rescale(a[0], b[0], L2, evk)
        el += time.perf_counter() - t
        done += 1
    single = done / el
    threads = o.set_threads(host_threads())
    n = 2 * threads
    a, b = pair(n), pair(n)
    t = time.perf_counter()
    octx.hmult_relin_rescale_batch(a, b, L2, evk)
    el_all = time.perf_counter() - t
    o.set_threads(0)
    cpu = host_cpu()
    return {"value": round(n / el_all, 4), "unit": "ops/s", "cores": threads, "kind": "port",
            "sample": f"{n} HMult+relin+rescale of config-2 pairs over {threads} threads ({el_all:.1f} s), C oracle, "
                      f"one pair per thread",
            "single_thread": {"value": round(single, 4), "unit": "ops/s", "cores": 1,
                              "sample": f"{done} pairs one after another ({el:.1f} s)"},
            "cpu_model": cpu["model"], "nproc": cpu["nproc"]}


# ----------------------------------------------------------------------------------------- config 3
def bench_pcmm(ckks, torch, steps_n, warmup, seed):
    """768 x 768 plaintext weights N(0, 1/768) times one ciphertext at L=16, BSGS 28 baby x 28 giant."""
    from pcmm_util import bsgs_diagonals, replicate, steps
    d, bs, l = 768, 28, 16
    ctx = ckks.Context(num_q=L2, num_p=K2, dnum=DNUM2, q_bits=54, p_bits=60, scale=2.0**50)
    scale = 2.0**50
    sk = ctx.secret(seed_bytes("pcmm-secret", seed), 192)
    dev = torch.device("cuda:0")
    bst, gst = steps(d, bs)
    T = L2 + K2
    keys = torch.empty((len(bst) + len(gst), DNUM2, 2, T, N), dtype=torch.int64, device=dev)
    kb = DNUM2 * 2 * T * N * 8
    for i, s_ in enumerate(bst + gst):
        ctx.keygen_automorphism(sk, ckks.rotation_index(s_), seed_bytes(f"rk{i}a", seed), seed_bytes(f"rk{i}e", seed),
                                keys.data_ptr() + i * kb)
    bptr = [keys.data_ptr() + i * kb for i in range(len(bst))]
    gptr = [keys.data_ptr() + (len(bst) + i) * kb for i in range(len(gst))]
    rng = np.random.default_rng(seed)
    W = rng.normal(0.0, np.sqrt(1.0 / d), (d, d))
    u = rng.uniform(-1.0, 1.0, d)
    diags = bsgs_diagonals(W, bs)
    D = torch.empty((d, l, N), dtype=torch.int64, device=dev)
    for k in range(d):
        ctx.encode(diags[k], l, scale, D.data_ptr() + k * l * N * 8)
    del diags
    pt = torch.empty((l, N), dtype=torch.int64, device=dev)
    ct = torch.empty((2, l, N), dtype=torch.int64, device=dev)
    out = torch.empty((2, l - 1, N), dtype=torch.int64, device=dev)
    ctx.encode(replicate(u), l, scale, pt.data_ptr())
    ctx.encrypt(sk, pt.data_ptr(), l, seed_bytes("pcmm-enc", seed), 0, ct.data_ptr())
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)

    def step():
        ctx.linear_transform_bsgs(ct.data_ptr(), l, D.data_ptr(), d, bs, bptr, gptr, out.data_ptr(), sh)

    wall, per = timed_steps(torch, stream, step, steps_n, warmup)
    got = ctx.decrypt(sk, out.data_ptr(), l - 1, scale * scale / ctx.moduli[l - 1])[:d]
    want = W @ u
    rel = float(np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2)))
    ctx.profile_reset()
    ctx.profile(True)
    step()
    torch.cuda.synchronize()
    ctx.profile(False)
    rep = ctx.profile_report()
    ctx.profile_reset()
    ms = wall * 1e3 / steps_n
    # algorithmic bytes: the SURVEY 8(d) config-3 unit with this BSGS's key count (27 baby + 27 giant keys of
    # 96 limbs -- the identity baby and giant steps need none -- not the unit's 56): keys + 768 x 16 plaintext limbs
    # + ct in/out 62 limbs
    alg = ((len(bst) + len(gst)) * 96 + d * l + 62) * LIMB_BYTES
    return {"ms_per_pcmm": round(ms, 4), "relErrRms_vs_fp64": rel,
            "kernels": kernel_table(rep), "kernel_io": kernel_io(rep, "pcmm"),
            "roofline": step_roofline("pcmm", alg, ms, 30 / (alg / LIMB_BYTES),
                                      f"step: one ckks_linear_transform_bsgs call; SURVEY 8(d) config-3 unit with "
                                      f"{len(bst) + len(gst)} keys: keys + 768 x 16 diagonal limbs + ct in/out"),
            "workload": "config3: 768x768 fp64 weights N(0,1/768) x 1 ct at L=16, BSGS 28 baby x 28 giant, "
                        "period-768 replicated layout"}


# ----------------------------------------------------------------------------------------- config 4
# Config-4 bootstrapping parameters, as BASELINE states them: EvalMod = Chebyshev degree 59 + 2 double-angle steps.
# The input's scale follows the reference's parameter rule FirstModSize = min(60, ScalingModSize + 5)
# (hpc_gpu_port/gpu_real_model.cu:1153-1154): q0 of 60 bits over a 2^55 message, so EvalMod's signal
# sin(2 pi m / q0) stands 2^5 below q0.  The input's secret is the dense h = 192 ternary secret; before ModRaise the
# level-1 ciphertext is switched to a sparse h' = 32 secret and the raised one back to the dense secret at the top
# level (sparse-secret encapsulation, Bossuat-Troncoso-Pastoriza-Hubaux, ePrint 2022/024), so the raised message's
# integer part I is the rounded sum of 33 uniforms on [-1/2, 1/2] per coefficient (c0 and 32 secret terms): the
# Chernoff bound puts P(some |I| > K - 1/2) at 1.2e-15 per bootstrap for K = 14 (tests/test_boot_params.py), and
# with two double angles the degree-59 interpolant covers cos(2 pi (K t - 1/4) / 4) over |K t| <= 14.
BOOT_SPARSE_H = 32
BOOT_K, BOOT_DEG, BOOT_R, BOOT_TOP, BOOT_IN = 14.0, 59, 2, 2.0**55, 2.0**55
# The labelled variant: the dense secret throughout (no encapsulation), so I is a sum of 193 uniforms and K = 32
# (Chernoff bound 1.9e-9 per bootstrap); three double angles keep the degree-59 interpolant of
# cos(2 pi (K t - 1/4) / 8) far below the noise.
BOOT_DENSE = {"K": 32.0, "deg": 59, "r": 3, "top": 2.0**55, "in": 2.0**55}
BOOT_FORMS = {
    "sparse_r2": {"K": BOOT_K, "deg": BOOT_DEG, "r": BOOT_R, "top": BOOT_TOP, "in": BOOT_IN, "sparse_h": BOOT_SPARSE_H},
    "dense_r3": dict(BOOT_DENSE, sparse_h=0),
}


def bootstrap_context(ckks):
    """q0 60-bit, 22 x 50-bit, 3 x 60-bit CoeffToSlot primes on top; 8 x 60-bit special primes; dnum 3."""
    big = ckks.gen_primes(60, 12)
    qs = ckks.gen_primes(50, 22)
    return ckks.Context(num_q=26, num_p=8, dnum=3, scale=2.0**50, moduli=big[:1] + qs + big[1:4] + big[4:])


def bench_bootstrap(ckks, torch, steps_n, warmup, seed, form="sparse_r2", stage_errors=True):
    f = BOOT_FORMS[form]
    ctx = bootstrap_context(ckks)
    L, K, D = ctx.L, ctx.K, ctx.dnum
    bt = ckks.Bootstrap(ctx, K=f["K"], cheb_degree=f["deg"], double_angles=f["r"], top_scale=f["top"],
                        in_scale=f["in"])
    sk = ctx.secret(seed_bytes("boot-secret", seed), 192)
    dev = torch.device("cuda:0")
    kb = D * 2 * (L + K) * N * 8
    nk = len(bt.steps) + 4
    keys = torch.empty((nk, kb // 8), dtype=torch.int64, device=dev)
    kp = [keys.data_ptr() + i * kb for i in range(nk)]
    ctx.keygen_relin(sk, seed_bytes("boot-ra", seed), seed_bytes("boot-re", seed), kp[0])
    ctx.keygen_automorphism(sk, 2 * N - 1, seed_bytes("boot-ca", seed), seed_bytes("boot-ce", seed), kp[1])
    sk_sparse = None
    if f["sparse_h"]:
        sk_sparse = ctx.secret(seed_bytes("boot-sparse", seed), f["sparse_h"])
        ctx.keygen_switch(sk, sk_sparse, seed_bytes("boot-ta", seed), seed_bytes("boot-te", seed), kp[2], q_limbs=1)
        ctx.keygen_switch(sk_sparse, sk, seed_bytes("boot-fa", seed), seed_bytes("boot-fe", seed), kp[3])
        bt.set_sparse_keys(kp[2], kp[3])
    rot = {}
    for i, s_ in enumerate(bt.steps):
        ctx.keygen_automorphism(sk, ckks.rotation_index(s_), seed_bytes(f"bk{i}a", seed), seed_bytes(f"bk{i}e", seed),
                                kp[4 + i])
        rot[s_] = kp[4 + i]
    rng = np.random.default_rng(seed)
    z = rng.uniform(-1.0, 1.0, N // 2)
    pt = torch.empty((1, N), dtype=torch.int64, device=dev)
    ct = torch.empty((2, 1, N), dtype=torch.int64, device=dev)
    out = torch.empty((2, bt.out_level, N), dtype=torch.int64, device=dev)
    ctx.encode(z, 1, f["in"], pt.data_ptr())
    ctx.encrypt(sk, pt.data_ptr(), 1, seed_bytes("boot-enc", seed), 0, ct.data_ptr())
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)

    def step():
        bt.run(ct.data_ptr(), kp[0], kp[1], rot, out.data_ptr(), sh)

    wall, per = timed_steps(torch, stream, step, steps_n, warmup)
    got = ctx.decrypt(sk, out.data_ptr(), bt.out_level, bt.scale(bt.out_level), N // 2, complex_out=True)
    bits = float(-np.log2(np.max(np.abs(got - z))))
    stages = bootstrap_stage_errors(ckks, ctx, bt, f["K"], sk, ct, kp, rot, got, z) if stage_errors else None
    ctx.profile_reset()
    ctx.profile(True)
    step()
    torch.cuda.synchronize()
    ctx.profile(False)
    rep = ctx.profile_report()
    ctx.profile_reset()
    ms = wall * 1e3 / steps_n
    if f["sparse_h"]:
        em = (f"EvalMod Chebyshev {f['deg']} + {f['r']} double-angle (sparse-secret encapsulation h'={f['sparse_h']}, "
              f"K={f['K']:g}, P(|I| > K) < 1.3e-15 per bootstrap)")
    else:
        em = (f"EvalMod Chebyshev {f['deg']} + {f['r']} double-angle (dense secret throughout, K={f['K']:g}, "
              f"P(|I| > K) < 1.9e-9 per bootstrap)")
    del sk_sparse
    return {"ms_per_bootstrap": round(ms, 3), "precision_bits": round(bits, 2),
            "levels_in_out": [1, bt.out_level], "rotation_keys": len(bt.steps), "stage_errors": stages,
            "form": form, "kernels": kernel_table(rep), "kernel_io": kernel_io(rep, "bootstrap"),
            "roofline": step_roofline("bootstrap" if form == "sparse_r2" else "", profile_bytes(rep), ms, 0.5,
                                      "step: one ckks_eval_bootstrap call; SURVEY 8(d) config-4 unit: the sum of its "
                                      "launches' algorithmic bytes (each launch's inputs, keys, diagonals and outputs "
                                      "once)"),
            "workload": "config4: full-slot bootstrap N=2^16, 32768 slots, level-1 input at scale 2^55 (q0 60 bits), "
                        f"secret h=192, CtS 3 levels, {em}, StC 3 levels; chain q0 60 + 22x50 + 3x60 bits, P 8x60, "
                        "dnum 3"}


def bootstrap_stage_errors(ckks, ctx, bt, Kr, sk, ct, kp, rot, got, z):
    """Error budget of one bootstrap, stage by stage (the engine stops after a stage on request): ModRaise decrypts
    to m' = m + q0 I; after CoeffToSlot the slots hold t = (m'_k + i m'_{k+n}) / (q0 K), bit-reversed; EvalMod gives
    sin(2 pi K t) per real part; SlotToCoeff gives z.  Each figure is the max error over the slots in the units of
    that stage's signal, beside the signal's max (EvalMod's signal is ~2 pi m / q0: its absolute error, times
    q0 / (2 pi scale_in), is the output's)."""
    import torch
    n = N // 2
    L = ctx.L
    buf = torch.empty((2, 2, L, N), dtype=torch.int64, device="cuda:0")
    lvl = bt.run_stage(ct.data_ptr(), kp[0], kp[1], rot, 1, buf.data_ptr())
    mp = ctx.decrypt_coeffs(sk, buf.data_ptr(), lvl)
    rev = np.zeros(n, dtype=np.int64)
    b = n.bit_length() - 1
    for i in range(n):
        rev[i] = int(format(i, f"0{b}b")[::-1], 2)
    t = ((mp[:n] + 1j * mp[n:]) / (ctx.moduli[0] * Kr))[rev]
    res = {}
    lvl = bt.run_stage(ct.data_ptr(), kp[0], kp[1], rot, 2, buf.data_ptr())
    dec = ctx.decrypt(sk, buf.data_ptr(), lvl, bt.scale(lvl), n, complex_out=True)
    res["coeff_to_slot"] = {"max_err": float(np.max(np.abs(dec - t))), "signal_max": float(np.max(np.abs(t))),
                            "level": lvl}
    lvl = bt.run_stage(ct.data_ptr(), kp[0], kp[1], rot, 4, buf.data_ptr())
    errs, sig = [], []
    for part, want in enumerate((np.sin(2 * np.pi * Kr * t.real), np.sin(2 * np.pi * Kr * t.imag))):
        dec = ctx.decrypt(sk, buf.data_ptr() + part * 2 * lvl * N * 8, lvl, bt.scale(lvl), n, complex_out=True)
        errs.append(float(np.max(np.abs(dec - want))))
        sig.append(float(np.max(np.abs(want))))
    res["eval_mod"] = {"max_err": max(errs), "signal_max": max(sig), "level": lvl}
    res["slot_to_coeff"] = {"max_err": float(np.max(np.abs(got - z))), "signal_max": float(np.max(np.abs(z))),
                            "level": bt.out_level}
    return res


# ----------------------------------------------------------------------------------------- config 5
DECODE_LANES = 32


def phase_table(ph: dict, step_ms: float):
    """the profiled step by phase label (the engine's per-launch events): launches, event time, the share of the
    step's event time scaled to the timed step, algorithmic bytes, and each label's marker-kernel id"""
    tot = sum(v[1] for v in ph.values()) or 1.0
    return {k: {"launches": n, "event_ms": round(ms, 3), "share": round(ms / tot, 4),
                "ms_in_timed_step": round(step_ms * ms / tot, 2), "algorithmic_GB": round(by / 1e9, 3),
                "marker_id": mid}
            for k, (n, ms, by, mid) in sorted(ph.items(), key=lambda kv: -kv[1][1])}


def bench_decode(ckks, torch, steps_n, warmup, seed, n_layers=12, driver="native", serve_requests=0,
                 phase_markers=False):
    """Config 5: one encrypted decode step of the RWKV-7-0.1B-shaped polynomial model (12 layers, 32 lanes in
    the slots, state carried across steps, state bootstrapped once per layer).  The client side (token
    embedding + encryption before the step, decryption + the 768 x 65536 vocabulary head after it) is
    outside the timed region and reported separately.  driver: "native" runs the C++ driver
    (libfhe_ssm_decode.so), "python" the same plan in decode_step.py (identical engine calls and words)."""
    from engine_loader import load_module
    DS = load_module("decode_step")
    M = load_module("rwkv_model")
    free0, total0 = torch.cuda.mem_get_info()
    mem_before = total0 - free0  # what the process held on the device before config 5's setup
    t0 = time.perf_counter()
    be, sk = DS.build_engine(ckks)
    t_keys = time.perf_counter() - t0
    log = lambda msg: print(f"[decode] {msg}", file=sys.stderr, flush=True)
    log(f"keys ready in {t_keys:.1f} s ({len(be.keys)} rotation keys)")
    W = M.make_weights(seed + 4, n_layers)
    if driver == "native":
        ND = load_module("native_decode")
        nat = ND.from_backend(be, n_layers)
        nat.set_weights(W)

        def step(ct):
            out, lv, sc = nat.step(ct.ptr(), ct.level, ct.scale)
            return DS.HECt(out, 1, lv, sc)

        n_boot = lambda: nat.bootstraps
    else:
        py = DS.DecodeStep(be, W)
        step = py
        n_boot = lambda: py.stats["bootstraps"]
    ctx = be.ctx
    if phase_markers:  # an empty marker kernel at every change of phase label, for splitting a trace by phase
        ctx.profile_phase_markers(True)
    tokens = lambda i: (np.arange(DECODE_LANES) * 7919 + 131 * i + seed) % M.VOCAB

    def client_in(i):
        x = M.embed_tokens(tokens(i), seed=seed)
        return x, be.encrypt(sk, M.pack_lanes(x), be.top_level, seed=seed_bytes(f"dec{i}", seed))

    xs, outs, times, ks = [], [], [], []
    t_enc0 = time.perf_counter()
    for i in range(warmup):  # the first step also encodes every plaintext (weights, masks) on first use
        x, ct = client_in(i)
        xs.append(x)
        outs.append(step(ct))
        torch.cuda.synchronize()
        log(f"warmup step {i} done at {time.perf_counter() - t_enc0:.1f} s")
    t_warm = time.perf_counter() - t_enc0
    free_b, total_b = torch.cuda.mem_get_info()
    for i in range(warmup, warmup + steps_n):
        x, ct = client_in(i)
        xs.append(x)
        torch.cuda.synchronize()
        ctx.key_switches(reset=True)
        t = time.perf_counter()
        outs.append(step(ct))
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t)
        ks.append(ctx.key_switches())
        log(f"timed step {i}: {times[-1]:.2f} s, {ks[-1]} key switches")
    # client side of the last step: decrypt, vocabulary head on the plaintext
    t = time.perf_counter()
    xo = M.unpack_lanes(be.decrypt(sk, outs[-1]).real)
    head = M.head_matrix(W)
    logits = xo @ head.T
    t_client = time.perf_counter() - t
    # one profiled step for the kernel table (state keeps carrying)
    x, ct = client_in(warmup + steps_n)
    xs.append(x)
    ctx.profile_reset()
    ctx.profile(True)
    outs.append(step(ct))
    torch.cuda.synchronize()
    ctx.profile(False)
    rep = ctx.profile_report()
    phases = ctx.profile_phase_report()
    marker_ids = {k: ctx.profile_phase_id(k) for k in ("step", "idle", "state_backup")} if phase_markers else {}
    ctx.profile_reset()
    s_per_step = sum(times) / len(times)
    free_b2, _ = torch.cuda.mem_get_info()
    mem = {"device_gb_after_timed_steps": round((total_b - free_b2) / 1e9, 1),
           "device_gb_in_use_before_setup": round(mem_before / 1e9, 1)}
    if driver == "native":
        mem["decoder_gb"] = {k: round(v / 1e9, 2) for k, v in nat.memory().items()}
    mem["context_gb"] = {k: round(v / 1e9, 2) for k, v in ctx.memory().items()}
    mem["keys_gb"] = round((len(be.keys) + 4) * ctx.dnum * 2 * (ctx.L + ctx.K) * N * 8 / 1e9, 1)
    serve = None
    if serve_requests and driver == "native":
        serve = bench_serve(torch, be, nat, client_in, warmup + steps_n + 1, serve_requests, log)
        serve["step_s"] = round(s_per_step, 3)
        serve["overhead_ms_per_request"] = round((serve["request_s"] - s_per_step) * 1e3, 1)
    return {"s_per_step": round(s_per_step, 3), "serve": serve, "key_switches_per_step": int(np.mean(ks)),
            "bootstraps_per_step": n_boot() // (warmup + steps_n + 1), "driver": driver,
            "setup_s": {"keys": round(t_keys, 1), "first_steps_with_plaintext_encoding": round(t_warm, 1)},
            "device_memory_in_use_gb_after_warmup": round((total_b - free_b) / 1e9, 1), "memory": mem,
            "client_s": {"decrypt_and_vocab_head": round(t_client, 3)},
            "kernels": kernel_table(rep), "kernel_io": kernel_io(rep, "decode"),
            "phases": phase_table(phases, s_per_step * 1e3), "phase_marker_ids": marker_ids,
            "roofline": step_roofline("decode", profile_bytes(rep), s_per_step * 1e3, 0.5,
                                      "step: one decode step of the native driver; SURVEY 8(d) config-5 unit: the sum "
                                      "of its launches' algorithmic bytes (each launch's inputs, keys, diagonals and "
                                      "outputs once)"),
            "_check": {"xs": xs, "outs": outs, "logits": logits, "logits_step": warmup + steps_n - 1, "W": W,
                       "be": be, "sk": sk, "M": M, "n_steps": warmup + steps_n + 1},
            "workload": f"config5: RWKV-7-0.1B-shaped decode step, {n_layers} layers, d=768, 12 heads x 64, "
                        f"degree-3 polynomial nonlinearities (seeded coefficients in [-0.5, 0.5]), 32 lanes in "
                        f"the slots of one N=2^16 ciphertext, WKV state carried and bootstrapped once per layer; "
                        f"chain q0 50 + 28 x 40 + 3 x 60 bits, P 7 x 60, dnum 4; sparse-secret bootstrapping"}


def bench_serve(torch, be, nat, client_in, i0, n_req, log):
    """The serve-directory protocol around the same decoder (state carried on): n_req one-token requests, each
    timed from the client writing its ciphertext file to the answer being complete (resp.N.done present,
    req.N.ready gone).  Both ends poll every 20 ms here (the reference's server polls every 200 ms)."""
    import tempfile
    import threading
    from engine_loader import load_module
    SC = load_module("serve_client")
    d = tempfile.mkdtemp(prefix="fhe_serve_")
    box = {}
    th = threading.Thread(target=lambda: box.update(rep=nat.serve(d, timeout_sec=600, stateful=True, poll_ms=20)),
                          daemon=True)
    th.start()
    times = []
    for n in range(n_req):
        _, ct = client_in(i0 + n)
        torch.cuda.synchronize()
        t = time.perf_counter()
        SC.submit(d, n, lambda k, path: be.ctx.ct_save(path, ct.ptr(), ct.level, ct.scale), 1,
                  SC.request_meta(1, DECODE_LANES, be.top_level))
        resp = SC.wait(d, n, timeout=600, poll=0.02, alive=th.is_alive)
        times.append(time.perf_counter() - t)
        log(f"serve request {n}: {times[-1]:.2f} s ({os.path.getsize(resp + '.0') / 2**20:.1f} MiB response)")
    SC.stop(d)
    th.join(timeout=60)
    in_mib = 2 * be.top_level * (1 << 16) * 8 / 2**20
    shutil.rmtree(d, ignore_errors=True)
    return {"requests": n_req, "request_s": round(sum(times) / len(times), 3), "poll_ms": 20,
            "request_file_MiB": round(in_mib, 1), "served": box.get("rep", {}).get("served")}


def cpu_baseline_decode(res, seed, budget_s=15.0):
    """The oracle's key switch (ModUp + inner product + ModDown) at level 10 of the config-5 chain, single
    thread, times the step's key-switch count: a lower bound for the step on the CPU (NTT-only, elementwise
    and encoding work left out).  The same leg checks the decrypted step against the float64 model."""
    from oracle import oracle as o
    from oracle import rwkv_ref as ref
    chk = res["_check"]
    be = chk["be"]
    ctx = be.ctx
    oc = o.Ctx(16, ctx.moduli, ctx.L, ctx.K, ctx.dnum, moddown_exact=True)
    rng = np.random.default_rng(seed)
    l = 10
    q = np.array(ctx.moduli[:l], dtype=np.uint64)[:, None]
    x = rng.integers(0, 2**62, (l, N), dtype=np.uint64) % q
    qall = np.array(ctx.moduli, dtype=np.uint64)[None, None, :, None]
    evk = rng.integers(0, 2**62, (ctx.dnum, 2, ctx.L + ctx.K, N), dtype=np.uint64) % qall[0]
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n == 0:
        oc.keyswitch(x, l, evk)
        n += 1
    per_ks = (time.perf_counter() - t0) / n
    # accuracy of every decrypted step against the float64 model (state carried identically)
    M = chk["M"]
    st = ref.init_state(DECODE_LANES, len(chk["W"]["layers"]))
    errs = []
    head = M.head_matrix(chk["W"])
    for i in range(chk["n_steps"]):
        xo_ref, _ = ref.step(chk["xs"][i], st, chk["W"])
        got = M.unpack_lanes(be.decrypt(chk["sk"], chk["outs"][i]).real)
        errs.append(float(np.sqrt(np.mean((got - xo_ref) ** 2)) / np.sqrt(np.mean(xo_ref ** 2))))
        if i == chk["logits_step"]:
            lg_ref = xo_ref @ head.T
    lg_err = float(np.sqrt(np.mean((chk["logits"] - lg_ref) ** 2)) / np.sqrt(np.mean(lg_ref ** 2)))
    est = per_ks * res["key_switches_per_step"]
    return {"value": round(est, 1), "unit": "s/step", "cores": 1, "kind": "port",
            "sample": f"{n} oracle key switches (level 10, config-5 chain, one thread) at {per_ks:.3f} s each x "
                      f"{res['key_switches_per_step']} key switches per step; a lower bound (leaves out the "
                      f"NTT-only and elementwise work)"}, {"relErrRms_per_step": [round(e, 6) for e in errs],
                                                          "logits_relErrRms_last_step": round(lg_err, 6)}


# ----------------------------------------------------------------------------------------- config 1
def ntt_bytes():
    limbs = 2 * N_PAIRS * L2
    return limbs, limbs * 2 * LIMB_BYTES + L2 * TWIDDLE_BYTES_PER_PRIME


def bench_ntt(ckks, torch, steps, warmup, seed):
    limbs, bytes_dir = ntt_bytes()
    n_polys = 2 * N_PAIRS
    ctx = ckks.Context(num_q=L2, num_p=K2, dnum=DNUM2, q_bits=54, p_bits=60)
    prime_idx = list(range(L2))
    rng = np.random.default_rng(seed)
    q = np.array(ctx.moduli[:L2], dtype=np.uint64)
    host = rng.integers(0, 2**63, (n_polys, L2, N), dtype=np.uint64) % q[None, :, None]
    data = torch.from_numpy(host.view(np.int64)).to("cuda:0")
    first = host[0, 0].copy()
    del host
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    ptr = data.data_ptr()

    def step():
        ctx.ntt_forward(ptr, n_polys, prime_idx, sh)
        ctx.ntt_inverse(ptr, n_polys, prime_idx, sh)

    wall, _ = timed_steps(torch, stream, step, steps, warmup)
    if not np.array_equal(data[0, 0].cpu().numpy().view(np.uint64), first):
        raise SystemExit("NTT round trip changed the data: results invalid")
    ctx.profile_reset()
    ctx.profile(True)
    step()
    torch.cuda.synchronize()
    ctx.profile(False)
    rep = ctx.profile_report()
    step_ms = wall * 1e3 / steps
    return {
        "metric": "NTT HBM GB/s (algorithmic bytes, forward+inverse, N=2^16)",
        "value": round(2 * bytes_dir / (step_ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(step_ms, 4),
        "dtype": "u64",
        "config": {"workload": "config1: fwd+inv negacyclic NTT, N=2^16, 64 ct x 2 polys x L=24 54-bit limbs",
                   "limbs_per_direction": limbs, "algorithmic_bytes_per_direction": bytes_dir,
                   "ntt_mode": "two-pass", "seed": seed},
        "kernels": kernel_table(rep),
        "roofline": step_roofline("ntt", 2 * bytes_dir, step_ms, 0.5,
                                  "step: one forward + one inverse ckks_ntt call over the 3,072 limbs; SURVEY 8(d) "
                                  "config-1 unit 3,246,391,296 B per direction x 2"),
        "kernel_io": kernel_io(rep, "ntt"),
    }


def cpu_baseline_ntt(seed, budget_s=6.0):
    """Oracle forward + inverse NTT over config-1 limbs: every host thread (OpenMP over the limbs), then one."""
    from oracle import oracle as o
    limbs_total, bytes_dir = ntt_bytes()
    qs = o.gen_primes(54, L2, 2 * N)
    octx = o.Ctx(16, qs, L2, 0, 1)
    rng = np.random.default_rng(seed)
    q = np.array(qs, dtype=np.uint64)
    x = rng.integers(0, 2**63, (2, L2, N), dtype=np.uint64) % q[None, :, None]

    def leg(threads):
        got = o.set_threads(threads)
        done, t0 = 0, time.perf_counter()
        while True:
            y = octx.ntt_fwd(x, list(range(L2)))
            octx.ntt_inv(y, list(range(L2)))
            done += 2 * L2
            el = time.perf_counter() - t0
            if el > budget_s or done >= limbs_total:
                break
        return got, done, el, done * 2 * (bytes_dir / limbs_total) / el / 1e9

    cores, done, el, gbs = leg(host_threads())
    _, done1, el1, gbs1 = leg(1)
    o.set_threads(0)
    cpu = host_cpu()
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{done} limbs fwd+inv of the config-1 batch ({el:.1f} s), C oracle with OpenMP over limbs",
            "single_thread": {"value": round(gbs1, 3), "unit": "GB/s", "cores": 1,
                              "sample": f"{done1} limbs fwd+inv ({el1:.1f} s)"},
            "cpu_model": cpu["model"], "nproc": cpu["nproc"]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="hmult", choices=["hmult", "ntt", "pcmm", "bootstrap", "decode"])
    ap.add_argument("--layers", type=int, default=12, help="decode workload: layers (12 = config 5)")
    ap.add_argument("--serve-requests", type=int, default=0,
                    help="decode workload: also time this many one-token requests through the serve protocol")
    ap.add_argument("--decode-driver", default="native", choices=["native", "python"],
                    help="decode workload: the C++ driver (default) or the same plan in Python")
    ap.add_argument("--phase-markers", action="store_true",
                    help="decode workload: enqueue an empty marker kernel at every change of phase label (for "
                         "splitting a rocprofv3 trace or counter pass by phase; the phase table is always reported)")
    ap.add_argument("--boot-form", default="sparse_r2", choices=sorted(BOOT_FORMS),
                    help="bootstrap workload: config 4 as stated (sparse_r2: sparse-secret encapsulation, K = 14, "
                         "2 double angles) or the dense-secret variant (dense_r3: K = 32, 3 double angles)")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ntt-line", action="store_true", help="skip the config-1 NTT figure in the hmult run")
    ap.add_argument("--no-pcmm-line", action="store_true", help="skip the config-3 PCMM figure in the hmult run")
    ap.add_argument("--no-boot-line", action="store_true", help="skip the config-4 bootstrap figure in the hmult run")
    ap.add_argument("--no-decode-line", action="store_true", help="skip the config-5 decode figure in the hmult run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is a design note, "
                                   "not an implemented path", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from engine_loader import load_ckks
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    ckks = load_ckks()
    if args.workload == "hmult":
        res = bench_hmult(ckks, torch, args.steps, args.warmup, args.seed)
        extra = {}
        if not args.no_ntt_line:
            n = bench_ntt(ckks, torch, max(3, args.steps // 2), 1, args.seed)
            extra["ntt_config1"] = {"GBps": n["value"], "ms_per_step": n["ms_per_step"],
                                    "roofline": n["roofline"], "kernel_io": n["kernel_io"]}
        if not args.no_pcmm_line:
            p = bench_pcmm(ckks, torch, max(3, args.steps // 2), 1, args.seed)
            extra["pcmm_config3"] = {k: p[k] for k in ("ms_per_pcmm", "relErrRms_vs_fp64", "roofline", "kernel_io")}
        if not args.no_boot_line:
            b = bench_bootstrap(ckks, torch, max(2, args.steps // 4), 1, args.seed)
            extra["bootstrap_config4"] = {k: b[k] for k in ("ms_per_bootstrap", "precision_bits", "levels_in_out",
                                                             "stage_errors", "roofline", "kernel_io", "workload")}
            v = bench_bootstrap(ckks, torch, max(2, args.steps // 4), 1, args.seed, form="dense_r3",
                                stage_errors=False)
            extra["bootstrap_config4_variant_dense_r3"] = {k: v[k] for k in ("ms_per_bootstrap", "precision_bits",
                                                                              "levels_in_out", "workload")}
        if not args.no_decode_line:
            # the earlier workloads' contexts, keys and buffers go before config 5 (and torch's cache returns their
            # tensors' memory, so the decode line's device figures are config 5's own)
            gc.collect()
            torch.cuda.empty_cache()
            d = bench_decode(ckks, torch, 2, 1, args.seed, driver=args.decode_driver)  # mean of 2 timed steps
            line = {"s_per_step": d["s_per_step"], "metric": "s/step for 32-lane decode (config 5)",
                    "roofline": d["roofline"], "kernel_io": d["kernel_io"], "phases": d["phases"]}
            line.update({k: d[k] for k in ("key_switches_per_step", "bootstraps_per_step", "setup_s", "client_s",
                                           "device_memory_in_use_gb_after_warmup", "memory", "driver")})
            if not args.no_cpu_baseline:
                line["cpu_baseline"], acc = cpu_baseline_decode(d, args.seed)
                line.update(acc)
            extra["decode_config5"] = line
            del d
        cpu = None if args.no_cpu_baseline else cpu_baseline_hmult(args.seed)
    elif args.workload == "decode":
        d = bench_decode(ckks, torch, args.steps, args.warmup, args.seed, args.layers, args.decode_driver,
                         args.serve_requests, args.phase_markers)
        res = {"metric": "s/step for 32-lane decode (config 5)", "value": d["s_per_step"], "unit": "s/step",
               "ms_per_step": round(d["s_per_step"] * 1e3, 1), "dtype": "u64",
               "config": {"workload": d["workload"], "lanes": DECODE_LANES, "layers": args.layers},
               "kernels": d["kernels"], "roofline": d["roofline"], "kernel_io": d["kernel_io"],
               "phases": d["phases"], "phase_marker_ids": d["phase_marker_ids"],
               "check": {k: d[k] for k in ("key_switches_per_step", "bootstraps_per_step", "setup_s", "client_s",
                                           "device_memory_in_use_gb_after_warmup", "memory", "driver")}}
        if d["serve"]:
            res["check"]["serve"] = d["serve"]
        extra = {}
        cpu = None
        if not args.no_cpu_baseline:
            cpu, acc = cpu_baseline_decode(d, args.seed)
            res["check"].update(acc)
    elif args.workload == "bootstrap":
        b = bench_bootstrap(ckks, torch, args.steps, args.warmup, args.seed, form=args.boot_form)
        res = {"metric": "bootstrap ms (full-slot, N=2^16)", "value": b["ms_per_bootstrap"], "unit": "ms",
               "ms_per_step": b["ms_per_bootstrap"], "dtype": "u64", "config": {"workload": b["workload"]},
               "kernels": b["kernels"], "roofline": b["roofline"], "kernel_io": b["kernel_io"],
               "check": {"precision_bits": b["precision_bits"], "levels_in_out": b["levels_in_out"],
                         "stage_errors": b["stage_errors"]}}
        extra, cpu = {}, None
    elif args.workload == "pcmm":
        p = bench_pcmm(ckks, torch, args.steps, args.warmup, args.seed)
        res = {"metric": "PCMM ms (768x768 BSGS, N=2^16, L=16)", "value": p["ms_per_pcmm"], "unit": "ms",
               "ms_per_step": p["ms_per_pcmm"], "dtype": "u64", "config": {"workload": p["workload"]},
               "kernels": p["kernels"], "roofline": p["roofline"], "kernel_io": p["kernel_io"],
               "check": {"relErrRms_vs_fp64": p["relErrRms_vs_fp64"]}}
        extra, cpu = {}, None
    else:
        res = bench_ntt(ckks, torch, args.steps, args.warmup, args.seed)
        extra = {}
        cpu = None if args.no_cpu_baseline else cpu_baseline_ntt(args.seed)
    out = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
           "higher_is_better": res["unit"] not in ("ms", "s/step"), "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"],
           "data": "synthetic (seeded)", "config": res["config"], "roofline": res["roofline"],
           "kernel_io": res["kernel_io"], "kernels": res["kernels"]}
    if "check" in res:
        out["check"] = res["check"]
    if "ks_stage" in res:
        out["ks_stage"] = res["ks_stage"]
    for k in ("phases", "phase_marker_ids"):
        if k in res:
            out[k] = res[k]
    out.update(extra)
    if cpu is not None:
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
