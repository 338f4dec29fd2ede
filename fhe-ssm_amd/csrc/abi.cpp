// abi.cpp -- the extern "C" entry points declared in include/ckks_engine.h.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <exception>
#include <string>

#include <map>

#include "bootstrap.hpp"
#include "ckks_engine.h"
#include "client.hpp"
#include "engine.hpp"
#include "keyfile.hpp"
#include "ops.hpp"

namespace fhe {
std::vector<uint64_t> ntt_primes(uint32_t bits, uint32_t count, uint64_t m, const std::vector<uint64_t>& skip);
void context_init(Context& c, const std::vector<uint64_t>& q, const std::vector<uint64_t>& p, uint32_t dnum,
                  double scale, int device);
void context_release(Context& c);
}  // namespace fhe

struct ckks_context {
    fhe::Context c;
};

struct ckks_bootstrap {
    fhe::BootPlan* p;
    const ckks_context* owner;
};

struct ckks_secret {
    fhe::Secret* s;
    const ckks_context* owner;
};

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(CKKS_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr)                                \
    do {                                             \
        hipError_t _e = (expr);                      \
        if (_e != hipSuccess) return hip_fail(_e, #expr); \
    } while (0)

template <class F>
int guarded(F&& f) {
    try {
        return f();
    } catch (const std::invalid_argument& e) {
        return fail(CKKS_EINVAL, e.what());
    } catch (const std::bad_alloc&) {
        return fail(CKKS_ENOMEM, "host allocation failed");
    } catch (const std::exception& e) {
        return fail(CKKS_EHIP, e.what());
    }
}

int check_limbs(const ckks_context* ctx, uint32_t n_limbs, const uint32_t* prime_idx) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (n_limbs == 0 || n_limbs > fhe::kMaxPmap) return fail(CKKS_EINVAL, "n_limbs must be in [1, 96]");
    if (!prime_idx) return fail(CKKS_EINVAL, "null prime_idx");
    for (uint32_t i = 0; i < n_limbs; i++)
        if (prime_idx[i] >= ctx->c.L + ctx->c.K) return fail(CKKS_EINVAL, "prime index out of range");
    return CKKS_OK;
}

int ntt_entry(ckks_context* ctx, uint64_t* d, uint32_t n_polys, uint32_t n_limbs, const uint32_t* prime_idx,
              void* stream, bool inverse) {
    if (int rc = check_limbs(ctx, n_limbs, prime_idx)) return rc;
    if (!d) return fail(CKKS_EINVAL, "null data");
    if (n_polys == 0) return CKKS_OK;
    const uint64_t jobs = (uint64_t)n_polys * n_limbs;
    if (jobs > 0x7fffffffull) return fail(CKKS_EINVAL, "too many limbs");
    fhe::JobSpec js{};
    js.jobs = nullptr;
    js.n_polys = n_polys;
    js.period = n_limbs;
    for (uint32_t i = 0; i < n_limbs; i++) js.pmap[i] = (uint8_t)prime_idx[i];
    HIP_TRY(fhe::launch_ntt(ctx->c, d, js, (uint32_t)jobs, inverse, ctx->c.ntt_mode, (hipStream_t)stream));
    return CKKS_OK;
}

int check_ctx_level(const ckks_context* ctx, uint32_t level, bool need_p) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (level == 0 || level > ctx->c.L) return fail(CKKS_EINVAL, "level out of range [1, L]");
    if (need_p && ctx->c.K == 0) return fail(CKKS_EINVAL, "context has no special primes");
    return CKKS_OK;
}

}  // namespace

extern "C" {

const char* ckks_last_error(void) { return g_err.c_str(); }

int ckks_context_create(const ckks_params* p, ckks_context** out) {
    if (!p || !out) return fail(CKKS_EINVAL, "null argument");
    if (p->log_n != fhe::kLogN) return fail(CKKS_ENOTSUP, "this build supports log_n = 16 only");
    if (p->q_bits < 20 || p->q_bits > 60 || p->p_bits < 20 || p->p_bits > 60)
        return fail(CKKS_EINVAL, "prime sizes must be in [20, 60] bits");
    return guarded([&] {
        const uint64_t m = 2ull * fhe::kN;
        auto q = fhe::ntt_primes(p->q_bits, p->num_q, m, {});
        auto pp = fhe::ntt_primes(p->p_bits, p->num_p, m, q);
        auto* ctx = new ckks_context();
        try {
            fhe::context_init(ctx->c, q, pp, p->dnum, p->scale, p->device);
        } catch (...) {
            fhe::context_release(ctx->c);
            delete ctx;
            throw;
        }
        *out = ctx;
        return CKKS_OK;
    });
}

int ckks_context_create_from_moduli(uint32_t log_n, const uint64_t* q, uint32_t num_q, const uint64_t* p,
                                    uint32_t num_p, uint32_t dnum, double scale, int device, ckks_context** out) {
    if (!out || !q || (num_p && !p)) return fail(CKKS_EINVAL, "null argument");
    if (log_n != fhe::kLogN) return fail(CKKS_ENOTSUP, "this build supports log_n = 16 only");
    return guarded([&] {
        auto* ctx = new ckks_context();
        try {
            fhe::context_init(ctx->c, std::vector<uint64_t>(q, q + num_q), std::vector<uint64_t>(p, p + num_p), dnum,
                              scale, device);
        } catch (...) {
            fhe::context_release(ctx->c);
            delete ctx;
            throw;
        }
        *out = ctx;
        return CKKS_OK;
    });
}

void ckks_context_destroy(ckks_context* ctx) {
    if (!ctx) return;
    fhe::context_release(ctx->c);
    delete ctx;
}

int ckks_context_info(const ckks_context* ctx, uint32_t* n, uint32_t* num_q, uint32_t* num_p, uint32_t* dnum) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (n) *n = fhe::kN;
    if (num_q) *num_q = ctx->c.L;
    if (num_p) *num_p = ctx->c.K;
    if (dnum) *dnum = ctx->c.dnum;
    return CKKS_OK;
}

int ckks_context_moduli(const ckks_context* ctx, uint64_t* out, uint32_t cap) {
    if (!ctx || !out) return fail(CKKS_EINVAL, "null argument");
    if (cap < ctx->c.moduli.size()) return fail(CKKS_EINVAL, "buffer too small");
    std::memcpy(out, ctx->c.moduli.data(), ctx->c.moduli.size() * 8);
    return CKKS_OK;
}

int ckks_context_roots(const ckks_context* ctx, uint64_t* out, uint32_t cap) {
    if (!ctx || !out) return fail(CKKS_EINVAL, "null argument");
    if (cap < ctx->c.psi.size()) return fail(CKKS_EINVAL, "buffer too small");
    std::memcpy(out, ctx->c.psi.data(), ctx->c.psi.size() * 8);
    return CKKS_OK;
}

int ckks_set_ntt_mode(ckks_context* ctx, int mode) {
    if (!ctx || (mode != 0 && mode != 1)) return fail(CKKS_EINVAL, "mode must be 0 or 1");
    ctx->c.ntt_mode = mode ? fhe::NttMode::Fused : fhe::NttMode::TwoPass;
    return CKKS_OK;
}

int ckks_set_moddown_exact(ckks_context* ctx, int exact) {
    if (!ctx || (exact != 0 && exact != 1)) return fail(CKKS_EINVAL, "exact must be 0 or 1");
    ctx->c.moddown_exact = exact != 0;
    return CKKS_OK;
}

int ckks_buffer_alloc(size_t bytes, void** d_out) {
    if (!d_out) return fail(CKKS_EINVAL, "null argument");
    HIP_TRY(hipMalloc(d_out, bytes ? bytes : 1));
    return CKKS_OK;
}

int ckks_buffer_free(void* d) {
    HIP_TRY(hipFree(d));
    return CKKS_OK;
}

int ckks_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes) {
    HIP_TRY(hipMemcpy(d_dst, h_src, bytes, hipMemcpyHostToDevice));
    return CKKS_OK;
}

int ckks_host_alloc(size_t bytes, void** h_out) {
    if (!h_out) return fail(CKKS_EINVAL, "null argument");
    *h_out = nullptr;
    HIP_TRY(hipHostMalloc(h_out, bytes ? bytes : 1, hipHostMallocDefault));
    return CKKS_OK;
}

int ckks_host_free(void* h) {
    if (h) HIP_TRY(hipHostFree(h));
    return CKKS_OK;
}

int ckks_side_copy(ckks_context* ctx, void* dst, const void* src, size_t bytes, void* stream, uint64_t* ticket) {
    if (!ctx || !dst || !src || !ticket) return fail(CKKS_EINVAL, "null argument");
    fhe::Context& c = ctx->c;
    // copies to host memory on their own side stream: a step's run of state copies out does not hold up the
    // prefetches into device memory queued behind it
    // the destination is host memory unless the runtime reports device memory: pinned host memory reports
    // hipMemoryTypeHost, pageable host memory fails the query or reports hipMemoryTypeUnregistered
    hipPointerAttribute_t at{};
    bool to_host = true;
    if (hipPointerGetAttributes(&at, dst) == hipSuccess)
        to_host = at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeManaged && at.type != hipMemoryTypeArray;
    else
        (void)hipGetLastError();
    hipStream_t& side = to_host ? c.side_out : c.side;
    if (!side) HIP_TRY(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
    // after the work enqueued so far on stream
    hipEvent_t after = nullptr, done = nullptr;
    HIP_TRY(hipEventCreateWithFlags(&after, hipEventDisableTiming));
    hipError_t e = hipEventRecord(after, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(side, after, 0);
    if (e == hipSuccess) e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, side);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(done, side);
    c.side_after.push_back(after);  // destroyed at the next ckks_side_sync, once the side stream has drained
    if (e != hipSuccess) {
        if (done) (void)hipEventDestroy(done);
        return fail(CKKS_EHIP, std::string("side copy: ") + hipGetErrorString(e));
    }
    *ticket = ++c.side_next;
    c.side_ev[*ticket] = done;
    return CKKS_OK;
}

int ckks_side_wait(ckks_context* ctx, uint64_t ticket, void* stream) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    auto it = ctx->c.side_ev.find(ticket);
    if (it == ctx->c.side_ev.end()) return CKKS_OK;  // already synchronized (ckks_side_sync)
    HIP_TRY(hipStreamWaitEvent((hipStream_t)stream, it->second, 0));
    return CKKS_OK;
}

int ckks_side_sync(ckks_context* ctx) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    fhe::Context& c = ctx->c;
    if (c.side) HIP_TRY(hipStreamSynchronize(c.side));
    if (c.side_out) HIP_TRY(hipStreamSynchronize(c.side_out));
    for (auto& kv : c.side_ev) (void)hipEventDestroy(kv.second);
    c.side_ev.clear();
    for (auto ev : c.side_after) (void)hipEventDestroy(ev);
    c.side_after.clear();
    return CKKS_OK;
}

int ckks_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes) {
    HIP_TRY(hipMemcpy(h_dst, d_src, bytes, hipMemcpyDeviceToHost));
    return CKKS_OK;
}

int ckks_device_sync(void) {
    HIP_TRY(hipDeviceSynchronize());
    return CKKS_OK;
}

int ckks_ntt_forward(ckks_context* ctx, uint64_t* d_data, uint32_t n_polys, uint32_t n_limbs,
                     const uint32_t* prime_idx, void* stream) {
    return ntt_entry(ctx, d_data, n_polys, n_limbs, prime_idx, stream, false);
}

int ckks_ntt_inverse(ckks_context* ctx, uint64_t* d_data, uint32_t n_polys, uint32_t n_limbs,
                     const uint32_t* prime_idx, void* stream) {
    return ntt_entry(ctx, d_data, n_polys, n_limbs, prime_idx, stream, true);
}

int ckks_modup(ckks_context* ctx, const uint64_t* d_x, uint32_t batch, uint32_t level, uint64_t* d_ext,
               void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_x || !d_ext) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::modup(ctx->c, d_x, d_ext, batch, level, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_ks_inner(ckks_context* ctx, const uint64_t* d_ext, uint32_t batch, uint32_t level, const uint64_t* d_evk,
                  uint64_t* d_acc, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ext || !d_evk || !d_acc) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::ks_inner(ctx->c, d_ext, d_evk, d_acc, batch, level, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_moddown(ckks_context* ctx, uint64_t* d_x, uint32_t n_polys, uint32_t level, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_x || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!n_polys) return CKKS_OK;
    return guarded([&] {
        fhe::moddown_inplace(ctx->c, d_x, n_polys, level, nullptr, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_keyswitch(ckks_context* ctx, const uint64_t* d_x, uint32_t batch, uint32_t level, const uint64_t* d_evk,
                   uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_x || !d_evk || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::keyswitch(ctx->c, d_x, batch, level, d_evk, nullptr, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_rescale(ckks_context* ctx, const uint64_t* d_in, uint32_t n_polys, uint32_t level, uint64_t* d_out,
                 void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (level < 2) return fail(CKKS_EINVAL, "rescale needs level >= 2");
    if (!d_in || !d_out || d_in == d_out) return fail(CKKS_EINVAL, "null or aliased buffer");
    if (!n_polys) return CKKS_OK;
    return guarded([&] {
        fhe::rescale(ctx->c, d_in, n_polys, level, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_mult(ckks_context* ctx, const uint64_t* d_a, const uint64_t* d_b, uint32_t batch, uint32_t level,
                   const uint64_t* d_evk, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_a || !d_b || !d_evk || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::hmult(ctx->c, d_a, d_b, batch, level, d_evk, d_out, false, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_mult_rescale(ckks_context* ctx, const uint64_t* d_a, const uint64_t* d_b, uint32_t batch,
                           uint32_t level, const uint64_t* d_evk, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (level < 2) return fail(CKKS_EINVAL, "rescale needs level >= 2");
    if (!d_a || !d_b || !d_evk || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::hmult(ctx->c, d_a, d_b, batch, level, d_evk, d_out, true, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_mult_rescale_noalloc(ckks_context* ctx, const uint64_t* d_a, const uint64_t* d_b, uint32_t batch,
                                   uint32_t level, const uint64_t* d_evk, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (level < 2) return fail(CKKS_EINVAL, "rescale needs level >= 2");
    if (!d_a || !d_b || !d_evk || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::hmult_rescale_noalloc(ctx->c, d_a, d_b, batch, level, d_evk, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_add(ckks_context* ctx, const uint64_t* d_x, const uint64_t* d_y, uint32_t n_polys, uint32_t level,
                  uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_x || !d_y || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!n_polys) return CKKS_OK;
    return guarded([&] {
        fhe::add(ctx->c, d_x, d_y, d_out, n_polys, level, (hipStream_t)stream);
        return CKKS_OK;
    });
}

uint32_t ckks_rotation_index(int64_t step) { return fhe::rotation_index(step); }

int ckks_eval_mult_plain(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, const uint64_t* d_pt,
                         int pt_shared, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_ct || !d_pt || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::mul_plain(ctx->c, d_ct, batch, level, d_pt, pt_shared != 0, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_add_plain(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, const uint64_t* d_pt,
                        int pt_shared, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_ct || !d_pt || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::add_plain(ctx->c, d_ct, batch, level, d_pt, pt_shared != 0, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_rotate_hoisted(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, const int64_t* steps,
                             uint32_t n, const uint64_t* const* d_evks, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ct || !steps || !d_evks || !d_out) return fail(CKKS_EINVAL, "null argument");
    for (uint32_t i = 0; i < n; i++)
        if (!d_evks[i]) return fail(CKKS_EINVAL, "null key");
    if (!n) return CKKS_OK;
    return guarded([&] {
        fhe::rotate_hoisted(ctx->c, d_ct, level, steps, n, d_evks, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_rotate_sum(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, const int64_t* steps,
                         uint32_t n, const uint64_t* const* d_evks, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ct || !steps || !d_evks || !d_out) return fail(CKKS_EINVAL, "null argument");
    if (n == 0 || n > 64) return fail(CKKS_EINVAL, "1..64 rotations per sum");
    for (uint32_t i = 0; i < n; i++) {
        if (!d_evks[i]) return fail(CKKS_EINVAL, "null key");
        if (fhe::rotation_index(steps[i]) == 1) return fail(CKKS_EINVAL, "a step of the identity (no key switch)");
    }
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::rotate_sum(ctx->c, d_ct, batch, level, steps, n, d_evks, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_rotate_many(ckks_context* ctx, const uint64_t* d_cts, uint32_t n, uint32_t level, const int64_t* steps,
                          const uint64_t* const* d_evks, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_cts || !steps || !d_evks || !d_out || d_cts == d_out) return fail(CKKS_EINVAL, "null or aliased argument");
    for (uint32_t i = 0; i < n; i++)
        if (!d_evks[i]) return fail(CKKS_EINVAL, "null key");
    if (!n) return CKKS_OK;
    return guarded([&] {
        fhe::rotate_list(ctx->c, d_cts, n, level, steps, d_evks, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_linear_transform_bsgs(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, const uint64_t* d_diags,
                               uint32_t n_diag, uint32_t baby_steps, const uint64_t* const* d_baby_evks,
                               const uint64_t* const* d_giant_evks, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ct || !d_diags || !d_out || n_diag == 0 || baby_steps == 0) return fail(CKKS_EINVAL, "bad argument");
    const uint32_t ng = (n_diag + baby_steps - 1) / baby_steps;
    if (baby_steps > 1 && !d_baby_evks) return fail(CKKS_EINVAL, "null baby keys");
    if (ng > 1 && !d_giant_evks) return fail(CKKS_EINVAL, "null giant keys");
    for (uint32_t i = 0; i + 1 < baby_steps; i++)
        if (!d_baby_evks[i]) return fail(CKKS_EINVAL, "null baby key");
    for (uint32_t i = 0; i + 1 < ng; i++)
        if (!d_giant_evks[i]) return fail(CKKS_EINVAL, "null giant key");
    return guarded([&] {
        fhe::bsgs_matvec(ctx->c, d_ct, level, d_diags, n_diag, baby_steps, d_baby_evks, d_giant_evks, d_out,
                         (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_automorphism(ckks_context* ctx, const uint64_t* d_in, uint32_t n_polys, uint32_t level, uint32_t g,
                      uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_in || !d_out || d_in == d_out) return fail(CKKS_EINVAL, "null or aliased buffer");
    if (!n_polys) return CKKS_OK;
    return guarded([&] {
        fhe::automorph(ctx->c, d_in, d_out, n_polys, level, g, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_rotate(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, int64_t step,
                     const uint64_t* d_evk, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ct || !d_evk || !d_out || d_ct == d_out) return fail(CKKS_EINVAL, "null or aliased buffer");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::rotate(ctx->c, d_ct, batch, level, fhe::rotation_index(step), d_evk, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_secret_generate(ckks_context* ctx, const uint8_t* seed32, uint32_t hamming_weight, ckks_secret** out) {
    if (!ctx || !seed32 || !out) return fail(CKKS_EINVAL, "null argument");
    if (hamming_weight == 0 || hamming_weight > fhe::kN) return fail(CKKS_EINVAL, "hamming weight out of range");
    return guarded([&] {
        auto* sk = new ckks_secret{nullptr, ctx};
        try {
            sk->s = fhe::secret_create(ctx->c, seed32, hamming_weight);
        } catch (...) {
            delete sk;
            throw;
        }
        *out = sk;
        return CKKS_OK;
    });
}

void ckks_secret_destroy(ckks_secret* sk) {
    if (!sk) return;
    fhe::secret_destroy(sk->s);
    delete sk;
}

int ckks_secret_coeffs(const ckks_secret* sk, int8_t* out, uint32_t n) {
    if (!sk || !out) return fail(CKKS_EINVAL, "null argument");
    if (n < fhe::kN) return fail(CKKS_EINVAL, "buffer too small");
    std::memcpy(out, sk->s->coeffs.data(), fhe::kN);
    return CKKS_OK;
}

static int check_secret(const ckks_context* ctx, const ckks_secret* sk) {
    if (!ctx || !sk) return fail(CKKS_EINVAL, "null context or secret");
    if (sk->owner != ctx) return fail(CKKS_EINVAL, "secret belongs to another context");
    return CKKS_OK;
}

int ckks_keygen_relin(ckks_context* ctx, const ckks_secret* sk, const uint8_t* seed32, const uint8_t* eseed32,
                      uint64_t* d_evk) {
    if (int rc = check_secret(ctx, sk)) return rc;
    if (!seed32 || !eseed32 || !d_evk) return fail(CKKS_EINVAL, "null argument");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "context has no special primes");
    return guarded([&] {
        fhe::keygen_relin(ctx->c, *sk->s, seed32, eseed32, 3.19, d_evk);
        return CKKS_OK;
    });
}

int ckks_keygen_automorphism(ckks_context* ctx, const ckks_secret* sk, uint32_t g, const uint8_t* seed32,
                             const uint8_t* eseed32, uint64_t* d_evk) {
    if (int rc = check_secret(ctx, sk)) return rc;
    if (!seed32 || !eseed32 || !d_evk) return fail(CKKS_EINVAL, "null argument");
    if ((g & 1) == 0 || g >= 2 * fhe::kN) return fail(CKKS_EINVAL, "automorphism index must be odd and < 2N");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "context has no special primes");
    return guarded([&] {
        fhe::keygen_automorphism(ctx->c, *sk->s, g, seed32, eseed32, 3.19, d_evk);
        return CKKS_OK;
    });
}

int ckks_seeded_part_read_header(const char* path, ckks_seeded_part_header* out) {
    if (!path || !out) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        const fhe::SeededPartHeader h = fhe::read_seeded_part_header(path);
        if (h.key_tag.size() >= sizeof(out->key_tag)) return fail(CKKS_EINVAL, "seeded part: key tag too long");
        if (h.moduli.size() > sizeof(out->moduli) / sizeof(out->moduli[0]))
            return fail(CKKS_EINVAL, "seeded part: more moduli than the header struct holds");
        std::memset(out, 0, sizeof(*out));
        out->version = h.version;
        out->expander = h.expander;
        out->ring_dim = h.N;
        out->size_q = h.size_q;
        out->size_p = h.size_p;
        out->num_part_q = h.num_part_q;
        out->num_per_part_q = h.num_per_part_q;
        out->count = h.count;
        std::memcpy(out->key_tag, h.key_tag.data(), h.key_tag.size());
        for (size_t i = 0; i < h.moduli.size(); i++) out->moduli[i] = h.moduli[i];
        return CKKS_OK;
    });
}

int ckks_seeded_part_indices(const char* path, uint32_t* indices, uint32_t cap, uint32_t* count) {
    if (!path || !count || (cap && !indices)) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        const std::vector<uint32_t> idx = fhe::seeded_part_indices(path);
        *count = (uint32_t)idx.size();
        for (size_t i = 0; i < idx.size() && i < cap; i++) indices[i] = idx[i];
        return CKKS_OK;
    });
}

int ckks_seeded_part_load_key(ckks_context* ctx, const char* path, uint32_t record, uint32_t* index, uint64_t* d_evk) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (!path || !d_evk) return fail(CKKS_EINVAL, "null argument");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "context has no special primes");
    return guarded([&] {
        fhe::load_seeded_part_key(ctx->c, path, record, index, d_evk);
        return CKKS_OK;
    });
}

int ckks_seeded_part_write(ckks_context* ctx, const char* path, const char* key_tag, uint32_t n_keys,
                           const uint32_t* indices, const uint8_t* seeds, const uint64_t* const* d_evks) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (!path || !key_tag || (n_keys && (!indices || !seeds || !d_evks))) return fail(CKKS_EINVAL, "null argument");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "context has no special primes");
    for (uint32_t i = 0; i < n_keys; i++) {
        if (!d_evks[i]) return fail(CKKS_EINVAL, "null key");
        if ((indices[i] & 1) == 0 || indices[i] >= 2 * fhe::kN)
            return fail(CKKS_EINVAL, "automorphism index must be odd and < 2N");
    }
    return guarded([&] {
        fhe::write_seeded_part(ctx->c, path, key_tag, n_keys, indices, seeds, d_evks);
        return CKKS_OK;
    });
}

int ckks_dev_sidecar_read(const char* path, ckks_dev_sidecar* info, int32_t* rotations, uint32_t rot_cap,
                          uint32_t* boot_slots, uint32_t slot_cap) {
    if (!path || !info || (rot_cap && !rotations) || (slot_cap && !boot_slots)) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        const fhe::DevSidecar s = fhe::read_dev_sidecar(path);
        std::memset(info, 0, sizeof(*info));
        if (s.devices.size() > sizeof(info->devices) / sizeof(info->devices[0]))
            return fail(CKKS_EINVAL, "dev sidecar: more devices than the struct holds");
        info->n_devices = (uint32_t)s.devices.size();
        for (size_t i = 0; i < s.devices.size(); i++) info->devices[i] = s.devices[i];
        info->auto_load_ciphertexts = s.auto_load_ciphertexts;
        info->auto_load_plaintexts = s.auto_load_plaintexts;
        info->key_dist = s.key_dist;
        info->n_rotations = (uint32_t)s.rotations.size();
        info->n_boot_slots = (uint32_t)s.boot_slots.size();
        for (size_t i = 0; i < s.rotations.size() && i < rot_cap; i++) rotations[i] = s.rotations[i];
        for (size_t i = 0; i < s.boot_slots.size() && i < slot_cap; i++) boot_slots[i] = s.boot_slots[i];
        return CKKS_OK;
    });
}

int ckks_dev_sidecar_write(const char* path, const int32_t* rotations, uint32_t n_rotations, const uint32_t* boot_slots,
                           uint32_t n_boot_slots) {
    if (!path || (n_rotations && !rotations) || (n_boot_slots && !boot_slots)) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        fhe::DevSidecar s;
        s.rotations.assign(rotations, rotations + n_rotations);
        s.boot_slots.assign(boot_slots, boot_slots + n_boot_slots);
        fhe::write_dev_sidecar(path, s);
        return CKKS_OK;
    });
}

static std::vector<std::string> path_list(const char* const* paths, uint32_t n) {
    std::vector<std::string> v;
    for (uint32_t i = 0; i < n; i++) {
        if (!paths[i]) throw std::invalid_argument("null part path");
        v.emplace_back(paths[i]);
    }
    return v;
}

int ckks_rotation_keys_resolve(const char* dev_path, const char* const* part_paths, uint32_t n_parts,
                               uint32_t* part_of, uint32_t* record_of, uint32_t* index_of, uint32_t cap, uint32_t* n) {
    if (!dev_path || !part_paths || !n || (cap && (!part_of || !record_of || !index_of)))
        return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        const fhe::DevSidecar s = fhe::read_dev_sidecar(dev_path);
        const auto loc = fhe::resolve_rotation_keys(s.rotations, path_list(part_paths, n_parts));
        *n = (uint32_t)loc.size();
        for (size_t i = 0; i < loc.size() && i < cap; i++) {
            part_of[i] = loc[i].part;
            record_of[i] = loc[i].record;
            index_of[i] = loc[i].index;
        }
        return CKKS_OK;
    });
}

int ckks_rotation_keys_load(ckks_context* ctx, const char* dev_path, const char* const* part_paths, uint32_t n_parts,
                            uint64_t* const* d_evks, uint32_t n_keys) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (!dev_path || !part_paths || (n_keys && !d_evks)) return fail(CKKS_EINVAL, "null argument");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "context has no special primes");
    for (uint32_t i = 0; i < n_keys; i++)
        if (!d_evks[i]) return fail(CKKS_EINVAL, "null key buffer");
    return guarded([&] {
        fhe::load_rotation_keys(ctx->c, dev_path, path_list(part_paths, n_parts), d_evks, n_keys);
        return CKKS_OK;
    });
}

int ckks_ct_file_info(const char* path, uint32_t* ring_dim, uint32_t* level, double* scale) {
    if (!path || !ring_dim || !level || !scale) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        const fhe::CtFileHeader h = fhe::read_ct_header(path);
        *ring_dim = h.N;
        *level = h.level;
        *scale = h.scale;
        return CKKS_OK;
    });
}

int ckks_ct_save(ckks_context* ctx, const char* path, const uint64_t* d_ct, uint32_t level, double scale) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (!path || !d_ct) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        fhe::save_ct(ctx->c, path, d_ct, level, scale);
        return CKKS_OK;
    });
}

int ckks_ct_load(ckks_context* ctx, const char* path, uint32_t cap_level, uint64_t* d_ct, uint32_t* level,
                 double* scale) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (!path || !d_ct || !level || !scale) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        fhe::load_ct(ctx->c, path, cap_level, d_ct, level, scale);
        return CKKS_OK;
    });
}

int ckks_keygen_switch(ckks_context* ctx, const ckks_secret* sk_from, const ckks_secret* sk_to,
                       const uint8_t* seed32, const uint8_t* eseed32, uint32_t q_limbs, uint64_t* d_evk) {
    if (int rc = check_secret(ctx, sk_from)) return rc;
    if (int rc = check_secret(ctx, sk_to)) return rc;
    if (!seed32 || !eseed32 || !d_evk) return fail(CKKS_EINVAL, "null argument");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "context has no special primes");
    if (q_limbs > ctx->c.L) return fail(CKKS_EINVAL, "q_limbs exceeds the chain");
    return guarded([&] {
        fhe::keygen_switch_secret(ctx->c, *sk_from->s, *sk_to->s, seed32, eseed32, 3.19, q_limbs, d_evk);
        return CKKS_OK;
    });
}

int ckks_bootstrap_set_sparse_keys(ckks_bootstrap* bt, const uint64_t* d_to_sparse, const uint64_t* d_from_sparse) {
    if (!bt || (!d_to_sparse) != (!d_from_sparse)) return fail(CKKS_EINVAL, "both keys or neither");
    bt->p->sse_to = d_to_sparse;
    bt->p->sse_from = d_from_sparse;
    return CKKS_OK;
}

int ckks_encode(ckks_context* ctx, const double* re, const double* im, uint32_t n_slots, uint32_t level, double scale,
                uint64_t* d_pt) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_pt || (!re && !im)) return fail(CKKS_EINVAL, "null argument");
    if (!(scale > 0)) return fail(CKKS_EINVAL, "scale must be positive");
    return guarded([&] {
        fhe::encode(ctx->c, re, im, n_slots, level, scale, d_pt);
        return CKKS_OK;
    });
}

int ckks_encrypt(ckks_context* ctx, const ckks_secret* sk, const uint64_t* d_pt, uint32_t level, const uint8_t* seed32,
                 uint32_t index, uint64_t* d_ct) {
    if (int rc = check_secret(ctx, sk)) return rc;
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_pt || !seed32 || !d_ct) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        fhe::encrypt(ctx->c, *sk->s, d_pt, level, seed32, index, d_ct);
        return CKKS_OK;
    });
}

int ckks_keygen_public(ckks_context* ctx, const ckks_secret* sk, const uint8_t* seed32, const uint8_t* eseed32,
                       uint64_t* d_pk) {
    if (int rc = check_secret(ctx, sk)) return rc;
    if (!seed32 || !eseed32 || !d_pk) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        fhe::keygen_public(ctx->c, *sk->s, seed32, eseed32, 3.19, d_pk);
        return CKKS_OK;
    });
}

int ckks_encrypt_public(ckks_context* ctx, const uint64_t* d_pk, const uint64_t* d_pt, uint32_t level,
                        const uint8_t* seed32, uint32_t index, uint64_t* d_ct) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_pk || !d_pt || !seed32 || !d_ct) return fail(CKKS_EINVAL, "null argument");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "public-key encryption needs special primes (the key is over Q*P)");
    return guarded([&] {
        fhe::encrypt_public(ctx->c, d_pk, d_pt, level, seed32, index, d_ct);
        return CKKS_OK;
    });
}

int ckks_decrypt_decode(ckks_context* ctx, const ckks_secret* sk, const uint64_t* d_ct, uint32_t level, double scale,
                        double* re, double* im, uint32_t n_slots) {
    if (int rc = check_secret(ctx, sk)) return rc;
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_ct || (!re && !im)) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        fhe::decrypt_decode(ctx->c, *sk->s, d_ct, level, scale, re, im, n_slots);
        return CKKS_OK;
    });
}

int ckks_encode_periodic(ckks_context* ctx, const double* re, const double* im, uint32_t n_vectors, uint32_t period,
                         uint32_t level, double scale, uint64_t* d_out) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_out || (!re && !im)) return fail(CKKS_EINVAL, "null argument");
    if (!(scale > 0)) return fail(CKKS_EINVAL, "scale must be positive");
    if (!n_vectors) return CKKS_OK;
    return guarded([&] {
        fhe::encode_periodic(ctx->c, re, im, n_vectors, period, level, scale, d_out);
        return CKKS_OK;
    });
}

int ckks_encode_periodic_coeffs(ckks_context* ctx, const double* re, const double* im, uint32_t n_vectors,
                                uint32_t period, double scale, int64_t* d_coef, int32_t* d_log_approx) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (!d_coef || !d_log_approx || (!re && !im)) return fail(CKKS_EINVAL, "null argument");
    if (!(scale > 0)) return fail(CKKS_EINVAL, "scale must be positive");
    if (!n_vectors) return CKKS_OK;
    return guarded([&] {
        fhe::encode_periodic_coeffs(ctx->c, re, im, n_vectors, period, scale, d_coef, d_log_approx);
        return CKKS_OK;
    });
}

int ckks_expand_periodic(ckks_context* ctx, const int64_t* d_coef, const int32_t* d_log_approx, uint32_t n_vectors,
                         uint32_t period, uint32_t level, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_coef || !d_log_approx || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (!n_vectors) return CKKS_OK;
    if (n_vectors > 0x7fffffffu) return fail(CKKS_EINVAL, "too many vectors");
    return guarded([&] {
        fhe::expand_periodic(ctx->c, d_coef, d_log_approx, n_vectors, period, level, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_mult_plain_ex(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level,
                            const uint64_t* d_pt, int pt_shared, uint32_t log_rep, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_ct || !d_pt || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (log_rep > 6) return fail(CKKS_EINVAL, "log_rep must be <= 6");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::mul_plain(ctx->c, d_ct, batch, level, d_pt, pt_shared != 0, d_out, (hipStream_t)stream, log_rep);
        return CKKS_OK;
    });
}

int ckks_linear_transform_general(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, const uint64_t* d_diags,
                                  uint32_t log_rep, uint32_t n_baby, const int64_t* baby_steps,
                                  const uint64_t* const* d_baby_evks, uint32_t n_giant, const int64_t* giant_steps,
                                  const uint64_t* const* d_giant_evks, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ct || !d_diags || !d_out || !baby_steps || !giant_steps || !d_baby_evks || !d_giant_evks)
        return fail(CKKS_EINVAL, "null argument");
    if (n_baby == 0 || n_baby > 32 || n_giant == 0 || n_giant > 64 || log_rep > 6)
        return fail(CKKS_EINVAL, "bad BSGS shape");
    for (uint32_t i = 0; i < n_baby; i++)
        if (baby_steps[i] && !d_baby_evks[i]) return fail(CKKS_EINVAL, "null baby key");
    for (uint32_t i = 0; i < n_giant; i++)
        if (giant_steps[i] && !d_giant_evks[i]) return fail(CKKS_EINVAL, "null giant key");
    return guarded([&] {
        fhe::bsgs_general(ctx->c, d_ct, level, d_diags, n_baby, baby_steps, d_baby_evks, n_giant, giant_steps,
                          d_giant_evks, d_out, (hipStream_t)stream, log_rep);
        return CKKS_OK;
    });
}

int ckks_linear_transform_multi(ckks_context* ctx, const uint64_t* const* d_in, uint32_t n_in, uint32_t level,
                                const uint64_t* d_diags, uint32_t log_rep, uint32_t n_baby, const int64_t* baby_steps,
                                const uint64_t* const* d_baby_evks, uint32_t n_giant, const int64_t* giant_steps,
                                const uint64_t* const* d_giant_evks, uint32_t n_out, int rescale, uint64_t* d_out,
                                void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_in || !d_diags || !d_out || !baby_steps || !giant_steps || !d_baby_evks || !d_giant_evks)
        return fail(CKKS_EINVAL, "null argument");
    if (n_in == 0 || n_out == 0 || n_baby == 0 || n_in * n_baby > 256 || n_giant == 0 || n_giant > 64 || log_rep > 6)
        return fail(CKKS_EINVAL, "bad BSGS shape");
    if (rescale && level < 2) return fail(CKKS_EINVAL, "rescale needs level >= 2");
    for (uint32_t i = 0; i < n_in; i++)
        if (!d_in[i]) return fail(CKKS_EINVAL, "null input");
    for (uint32_t i = 0; i < n_baby; i++)
        if (baby_steps[i] && !d_baby_evks[i]) return fail(CKKS_EINVAL, "null baby key");
    for (uint32_t i = 0; i < n_giant; i++)
        if (giant_steps[i] && !d_giant_evks[i]) return fail(CKKS_EINVAL, "null giant key");
    return guarded([&] {
        fhe::bsgs_multi(ctx->c, d_in, n_in, level, d_diags, n_baby, baby_steps, d_baby_evks, n_giant, giant_steps,
                        d_giant_evks, n_out, rescale != 0, d_out, (hipStream_t)stream, log_rep);
        return CKKS_OK;
    });
}

int ckks_linear_transform_hoisted(ckks_context* ctx, const uint64_t* const* d_in, uint32_t n_in, uint32_t level,
                                  const uint64_t* d_diags, uint32_t n_baby, const int64_t* baby_steps,
                                  const uint64_t* const* d_baby_evks, uint32_t n_giant, const int64_t* giant_steps,
                                  const uint64_t* const* d_giant_evks, uint32_t n_out, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_in || !d_diags || !d_out || !baby_steps || !giant_steps || !d_baby_evks || !d_giant_evks)
        return fail(CKKS_EINVAL, "null argument");
    if (n_in == 0 || n_out == 0 || n_baby == 0 || n_baby > 32 || n_in * n_baby > 64 || n_giant == 0 ||
        n_giant > 64)
        return fail(CKKS_EINVAL, "bad BSGS shape");
    if (level < 2) return fail(CKKS_EINVAL, "rescale needs level >= 2");
    if (ctx->c.K == 0) return fail(CKKS_EINVAL, "the extended basis needs special primes");
    for (uint32_t i = 0; i < n_in; i++)
        if (!d_in[i]) return fail(CKKS_EINVAL, "null input");
    for (uint32_t i = 0; i < n_baby; i++)
        if (baby_steps[i] && !d_baby_evks[i]) return fail(CKKS_EINVAL, "null baby key");
    uint32_t n_zero = 0;
    for (uint32_t i = 0; i < n_giant; i++) {
        if (giant_steps[i] && !d_giant_evks[i]) return fail(CKKS_EINVAL, "null giant key");
        n_zero += giant_steps[i] == 0 ? 1 : 0;
    }
    if (n_zero > 1) return fail(CKKS_EINVAL, "at most one giant step 0");
    return guarded([&] {
        fhe::bsgs_dh_batch(ctx->c, d_in, 1, n_in, level, d_diags, n_baby, baby_steps, d_baby_evks, n_giant,
                           giant_steps, d_giant_evks, n_out, d_out, (hipStream_t)stream, false);
        return CKKS_OK;
    });
}

int ckks_eval_mult_sum(ckks_context* ctx, const uint64_t* const* d_pairs, uint32_t n_products, uint32_t batch,
                       uint32_t level, const uint64_t* d_evk, int rescale, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_pairs || !d_evk || !d_out) return fail(CKKS_EINVAL, "null argument");
    if (n_products == 0 || n_products > 64) return fail(CKKS_EINVAL, "1..64 products per output");
    if (rescale && level < 2) return fail(CKKS_EINVAL, "rescale needs level >= 2");
    for (size_t j = 0; j < (size_t)batch * n_products * 2; j++)
        if (!d_pairs[j]) return fail(CKKS_EINVAL, "null operand");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::hmult_sum(ctx->c, d_pairs, n_products, batch, level, d_evk, d_out, rescale != 0, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_rotate_masked(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, uint32_t n,
                            const int64_t* steps_lo, const uint64_t* const* d_evks_lo, const int64_t* steps_hi,
                            const uint64_t* const* d_evks_hi, uint32_t n_sets, const uint64_t* d_pts,
                            uint32_t log_rep, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ct || !steps_lo || !steps_hi || !d_evks_lo || !d_evks_hi || !d_pts || !d_out)
        return fail(CKKS_EINVAL, "null argument");
    if (level < 2) return fail(CKKS_EINVAL, "the masked pairs are rescaled: level >= 2");
    if (n == 0 || n_sets == 0 || log_rep > 6) return fail(CKKS_EINVAL, "bad shape");
    for (uint32_t i = 0; i < n; i++)
        if ((steps_lo[i] && !d_evks_lo[i]) || (steps_hi[i] && !d_evks_hi[i])) return fail(CKKS_EINVAL, "null key");
    return guarded([&] {
        fhe::rotate_masked(ctx->c, d_ct, level, n, steps_lo, d_evks_lo, steps_hi, d_evks_hi, n_sets, d_pts, log_rep,
                           d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_automorphism_ks(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, uint32_t g,
                              const uint64_t* d_evk, uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, true)) return rc;
    if (!d_ct || !d_evk || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if ((g & 1) == 0 || g >= 2u * (1u << 16)) return fail(CKKS_EINVAL, "automorphism index must be odd and < 2N");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        std::vector<uint32_t> gs(batch, g);
        std::vector<const uint64_t*> ks(batch, d_evk);
        fhe::automorph_ks_list(ctx->c, d_ct, batch, level, gs.data(), ks.data(), d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_mul_i(ckks_context* ctx, const uint64_t* d_in, uint32_t n_polys, uint32_t level, int sign,
                    uint64_t* d_out, void* stream) {
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_in || !d_out) return fail(CKKS_EINVAL, "null buffer");
    if (sign != 1 && sign != -1) return fail(CKKS_EINVAL, "sign must be +1 or -1");
    if (!n_polys) return CKKS_OK;
    return guarded([&] {
        fhe::mul_i(ctx->c, d_in, n_polys, level, sign, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_lincomb(ckks_context* ctx, uint32_t batch, uint32_t n_terms, const uint64_t* const* d_terms,
                      const uint32_t* levels, const double* coeffs, const double* scales_in, double scale_out,
                      double add_const, uint32_t target_level, int integer_mode, uint64_t* d_out, void* stream) {
    if (!ctx || !d_terms || !levels || !coeffs || !d_out || (!integer_mode && !scales_in))
        return fail(CKKS_EINVAL, "null argument");
    for (uint32_t t = 0; t < n_terms; t++)
        if (!d_terms[t]) return fail(CKKS_EINVAL, "null term");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::lincomb(ctx->c, batch, n_terms, d_terms, levels, coeffs, scales_in, scale_out, add_const, target_level,
                     integer_mode != 0, d_out, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_gen_primes(uint32_t bits, uint32_t count, const uint64_t* skip, uint32_t n_skip, uint64_t* out) {
    if (!out || (n_skip && !skip)) return fail(CKKS_EINVAL, "null argument");
    if (bits < 20 || bits > 60) return fail(CKKS_EINVAL, "bits must be in [20, 60]");
    return guarded([&] {
        auto v = fhe::ntt_primes(bits, count, 2ull * fhe::kN, std::vector<uint64_t>(skip, skip + n_skip));
        std::memcpy(out, v.data(), v.size() * 8);
        return CKKS_OK;
    });
}

int ckks_bootstrap_setup(ckks_context* ctx, double K, uint32_t cheb_degree, uint32_t double_angles, double top_scale,
                         double in_scale, ckks_bootstrap** out) {
    if (!ctx || !out) return fail(CKKS_EINVAL, "null argument");
    if (!(K >= 1) || !(top_scale > 0) || !(in_scale > 0) || double_angles > 6)
        return fail(CKKS_EINVAL, "bad bootstrap parameters");
    return guarded([&] {
        auto* bt = new ckks_bootstrap{nullptr, ctx};
        try {
            bt->p = fhe::bootstrap_plan(ctx->c, K, (int)cheb_degree, (int)double_angles, top_scale, in_scale);
        } catch (...) {
            delete bt;
            throw;
        }
        *out = bt;
        return CKKS_OK;
    });
}

int ckks_bootstrap_setup_shared(ckks_context* ctx, const ckks_bootstrap* base, double in_scale, ckks_bootstrap** out) {
    if (!ctx || !base || !out) return fail(CKKS_EINVAL, "null argument");
    if (base->owner != ctx) return fail(CKKS_EINVAL, "the base plan belongs to another context");
    if (!(in_scale > 0)) return fail(CKKS_EINVAL, "bad bootstrap parameters");
    return guarded([&] {
        auto* bt = new ckks_bootstrap{nullptr, ctx};
        try {
            bt->p = fhe::bootstrap_plan_shared(*base->p, in_scale);
        } catch (...) {
            delete bt;
            throw;
        }
        *out = bt;
        return CKKS_OK;
    });
}

void ckks_bootstrap_destroy(ckks_bootstrap* bt) {
    if (!bt) return;
    fhe::bootstrap_plan_destroy(bt->p);
    delete bt;
}

int ckks_bootstrap_steps(const ckks_bootstrap* bt, int64_t* steps, uint32_t cap, uint32_t* n) {
    if (!bt || !n) return fail(CKKS_EINVAL, "null argument");
    *n = (uint32_t)bt->p->steps.size();
    if (steps) {
        if (cap < *n) return fail(CKKS_EINVAL, "buffer too small");
        std::memcpy(steps, bt->p->steps.data(), *n * 8);
    }
    return CKKS_OK;
}

uint32_t ckks_bootstrap_out_level(const ckks_bootstrap* bt) { return bt ? bt->p->l_out : 0; }

double ckks_bootstrap_scale(const ckks_bootstrap* bt, uint32_t level) {
    if (!bt || level == 0 || level >= bt->p->S.size()) return 0.0;
    return (double)bt->p->S[level];
}

int ckks_eval_bootstrap(ckks_context* ctx, const ckks_bootstrap* bt, const uint64_t* d_ct_in, const uint64_t* d_relin,
                        const uint64_t* d_conj, const int64_t* steps, const uint64_t* const* d_evks, uint32_t n_keys,
                        uint64_t* d_out, void* stream) {
    if (!ctx || !bt || bt->owner != ctx) return fail(CKKS_EINVAL, "null context or plan of another context");
    if (!d_ct_in || !d_relin || !d_conj || !d_out || (n_keys && (!steps || !d_evks)))
        return fail(CKKS_EINVAL, "null argument");
    for (uint32_t i = 0; i < n_keys; i++)
        if (!d_evks[i]) return fail(CKKS_EINVAL, "null key");
    return guarded([&] {
        fhe::bootstrap(ctx->c, *bt->p, d_ct_in, 1, d_relin, d_conj, steps, d_evks, n_keys, d_out,
                       (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_bootstrap_many(ckks_context* ctx, const ckks_bootstrap* bt, const uint64_t* d_ct_in, uint32_t batch,
                             const uint64_t* d_relin, const uint64_t* d_conj, const int64_t* steps,
                             const uint64_t* const* d_evks, uint32_t n_keys, uint64_t* d_out, void* stream) {
    if (!ctx || !bt || bt->owner != ctx) return fail(CKKS_EINVAL, "null context or plan of another context");
    if (!d_ct_in || !d_relin || !d_conj || !d_out || (n_keys && (!steps || !d_evks)))
        return fail(CKKS_EINVAL, "null argument");
    if (batch > 64) return fail(CKKS_EINVAL, "at most 64 ciphertexts per call");
    for (uint32_t i = 0; i < n_keys; i++)
        if (!d_evks[i]) return fail(CKKS_EINVAL, "null key");
    if (!batch) return CKKS_OK;
    return guarded([&] {
        fhe::bootstrap(ctx->c, *bt->p, d_ct_in, batch, d_relin, d_conj, steps, d_evks, n_keys, d_out,
                       (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_eval_bootstrap_stage(ckks_context* ctx, const ckks_bootstrap* bt, const uint64_t* d_ct_in,
                              const uint64_t* d_relin, const uint64_t* d_conj, const int64_t* steps,
                              const uint64_t* const* d_evks, uint32_t n_keys, uint32_t stage, uint64_t* d_out,
                              uint32_t* level) {
    if (!ctx || !bt || bt->owner != ctx || !level) return fail(CKKS_EINVAL, "bad argument");
    if (!d_ct_in || !d_relin || !d_conj || !d_out || (n_keys && (!steps || !d_evks)))
        return fail(CKKS_EINVAL, "null argument");
    if (stage < 1 || stage > 6) return fail(CKKS_EINVAL, "stage must be in [1, 6]");
    return guarded([&] {
        *level = fhe::bootstrap(ctx->c, *bt->p, d_ct_in, 1, d_relin, d_conj, steps, d_evks, n_keys, d_out, nullptr,
                                stage);
        return CKKS_OK;
    });
}

int ckks_decrypt_coeffs(ckks_context* ctx, const ckks_secret* sk, const uint64_t* d_ct, uint32_t level, double* out) {
    if (int rc = check_secret(ctx, sk)) return rc;
    if (int rc = check_ctx_level(ctx, level, false)) return rc;
    if (!d_ct || !out) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        fhe::decrypt_coeffs(ctx->c, *sk->s, d_ct, level, out);
        return CKKS_OK;
    });
}

int ckks_profile_enable(ckks_context* ctx, int on) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    ctx->c.prof_on = on != 0;
    return CKKS_OK;
}

int ckks_profile_phase(ckks_context* ctx, const char* phase, void* stream) {
    if (!ctx || !phase) return fail(CKKS_EINVAL, "null argument");
    return guarded([&] {
        (void)fhe::set_phase(ctx->c, phase, (hipStream_t)stream);
        return CKKS_OK;
    });
}

int ckks_profile_phase_markers(ckks_context* ctx, int on) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    ctx->c.phase_marks = on != 0;
    return CKKS_OK;
}

int ckks_profile_phase_query(ckks_context* ctx, uint32_t idx, char* name, uint32_t name_cap, uint64_t* launches,
                             double* total_ms, double* total_bytes, int32_t* marker_id) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    std::vector<std::string> order;
    std::map<std::string, std::tuple<uint64_t, double, double>> agg;
    for (auto& r : ctx->c.prof) {
        HIP_TRY(hipEventSynchronize(r.e1));
        float ms = 0;
        HIP_TRY(hipEventElapsedTime(&ms, r.e0, r.e1));
        auto it = agg.find(r.phase);
        if (it == agg.end()) {
            order.push_back(r.phase);
            it = agg.emplace(r.phase, std::make_tuple(0ull, 0.0, 0.0)).first;
        }
        std::get<0>(it->second) += 1;
        std::get<1>(it->second) += ms;
        std::get<2>(it->second) += r.bytes;
    }
    if (idx >= order.size()) return fail(CKKS_EINVAL, "no such phase entry");
    const std::string& ph = order[idx];
    if (name && name_cap) {
        std::strncpy(name, ph.c_str(), name_cap - 1);
        name[name_cap - 1] = '\0';
    }
    if (launches) *launches = std::get<0>(agg[ph]);
    if (total_ms) *total_ms = std::get<1>(agg[ph]);
    if (total_bytes) *total_bytes = std::get<2>(agg[ph]);
    if (marker_id) {
        auto it = ctx->c.phase_ids.find(ph);
        *marker_id = it == ctx->c.phase_ids.end() ? -1 : (int32_t)it->second;
    }
    return CKKS_OK;
}

int ckks_profile_phase_id(const ckks_context* ctx, const char* phase, int32_t* marker_id) {
    if (!ctx || !phase || !marker_id) return fail(CKKS_EINVAL, "null argument");
    auto it = ctx->c.phase_ids.find(phase);
    *marker_id = it == ctx->c.phase_ids.end() ? -1 : (int32_t)it->second;
    return CKKS_OK;
}

int ckks_profile_reset(ckks_context* ctx) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    fhe::prof_clear(ctx->c);
    return CKKS_OK;
}

int ckks_context_counters(ckks_context* ctx, uint64_t* key_switches, int reset) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (key_switches) *key_switches = ctx->c.n_keyswitch;
    if (reset) ctx->c.n_keyswitch = 0;
    return CKKS_OK;
}

int ckks_context_memory(const ckks_context* ctx, uint64_t* bytes, uint32_t n) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    if (!bytes && n) return fail(CKKS_EINVAL, "null argument");
    const fhe::Context& c = ctx->c;
    const uint64_t T = c.L + c.K;
    uint64_t v[4] = {0, 0, 0, 0};
    v[0] = 4 * T * fhe::kN * sizeof(fhe::TwPair) + T * sizeof(fhe::PrimeInfo);
    for (auto& kv : c.small_ntt) v[0] += T * kv.first * sizeof(fhe::TwPair);
    for (auto& s : c.scratch) v[1] += s.second;
    for (auto& kv : c.buf_pool) v[2] += kv.first * kv.second.size();
    // the allocation-free entry point's static scratch: held on every GPU the library has run on, whether or not
    // that entry point is called, and shared by all contexts on that GPU (counted once per context here)
    v[3] = fhe::kScratchBytes;
    for (uint32_t i = 0; i < n && i < 4; i++) bytes[i] = v[i];
    return CKKS_OK;
}

int ckks_profile_query(ckks_context* ctx, uint32_t idx, char* name, uint32_t name_cap, uint64_t* launches,
                       double* total_ms, double* total_bytes) {
    if (!ctx) return fail(CKKS_EINVAL, "null context");
    std::vector<std::string> order;
    std::map<std::string, std::tuple<uint64_t, double, double>> agg;
    for (auto& r : ctx->c.prof) {
        HIP_TRY(hipEventSynchronize(r.e1));
        float ms = 0;
        HIP_TRY(hipEventElapsedTime(&ms, r.e0, r.e1));
        auto it = agg.find(r.name);
        if (it == agg.end()) {
            order.push_back(r.name);
            agg[r.name] = std::make_tuple(1ull, (double)ms, r.bytes);
        } else {
            std::get<0>(it->second) += 1;
            std::get<1>(it->second) += ms;
            std::get<2>(it->second) += r.bytes;
        }
    }
    if (idx >= order.size()) return fail(CKKS_EINVAL, "no such profile entry");
    const auto& a = agg[order[idx]];
    if (name && name_cap) {
        std::strncpy(name, order[idx].c_str(), name_cap - 1);
        name[name_cap - 1] = 0;
    }
    if (launches) *launches = std::get<0>(a);
    if (total_ms) *total_ms = std::get<1>(a);
    if (total_bytes) *total_bytes = std::get<2>(a);
    return CKKS_OK;
}

}  // extern "C"
