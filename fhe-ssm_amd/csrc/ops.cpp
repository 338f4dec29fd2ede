// ops.cpp -- composition of the hot path out of the kernels: hybrid key switching (ModUp -> evk
// inner product -> ModDown), rescale, HMult + relinearize + rescale, rotation.  Host code only: it
// builds the per-level plans (BConv constant tables, NTT job lists), owns the workspace and issues
// the launches on one stream.
//
// Semantics follow OpenFHE's HYBRID key switching and CKKS rescale as the reference uses them
// (FIDESlib/OpenFHE calls of hpc_gpu_port/gpu_real_model.cu; key layout seeded_keys.hpp:216-256;
// centered lift harness/boot_overflow_probe.cpp:93-94): at level l the Q limbs 0..l-1 split into
// digits of alpha = ceil(L/dnum) limbs, digit d = [d*alpha, min((d+1)*alpha, l)); each digit is
// brought to coefficients, switched by the approximate CRT (no correction of the overflow
// multiple of the digit modulus) to every other limb of Q_l * P, and taken back to evaluation form.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

#include "engine.hpp"
#include "ops.hpp"

namespace fhe {

uint64_t mulmod_h(uint64_t a, uint64_t b, uint64_t q);
uint64_t invmod_h(uint64_t a, uint64_t q);
uint8_t* arena_take(Arena& a, size_t bytes);

hipError_t launch_tensor(const Context& ctx, const uint64_t* a, const uint64_t* b, uint64_t* d01, uint64_t* d2,
                         uint32_t B, uint32_t l, uint64_t* d2e, uint64_t d2e_bstride, const uint32_t* ext_off,
                         hipStream_t st, uint32_t t0 = 0);
hipError_t launch_bconv(const Context& ctx, const BConvPlan& plan, const uint64_t* in, uint64_t in_bstride,
                        const uint32_t* in_off, uint64_t* out, uint64_t out_bstride, const uint32_t* out_off,
                        uint32_t B, hipStream_t st);
hipError_t launch_ks_inner(const Context& ctx, const uint64_t* ext, const uint64_t* evk, uint64_t* acc, uint32_t B,
                           uint32_t l, hipStream_t st, uint32_t t0 = 0);
hipError_t launch_bconv_mdr(const Context& ctx, const BConvPlan& plan, const uint64_t* in, uint64_t in_bstride,
                            const uint32_t* in_off, uint64_t* T, uint32_t n_polys, const uint64_t* xlast,
                            uint64_t xlast_pstride, const uint64_t* addc, TwPair pinv_last, hipStream_t st);
hipError_t launch_mdr_combine(const Context& ctx, const uint64_t* x, uint64_t x_pstride, const uint64_t* add,
                              uint64_t add_pstride, const uint64_t* T, uint64_t* out, uint32_t n_polys, uint32_t l,
                              const TwPair* pinv, const TwPair* qlinv, hipStream_t st);
hipError_t launch_mdr_combine_ks(const Context& ctx, const uint64_t* ext, const uint64_t* evk, const uint64_t* add,
                                 uint64_t add_pstride, const uint64_t* T, uint64_t* out, uint32_t B, uint32_t l,
                                 const TwPair* pinv, const TwPair* qlinv, hipStream_t st,
                                 const uint64_t* ta = nullptr, const uint64_t* tb = nullptr);
hipError_t launch_ntt_fwd_ksl(const Context& ctx, uint64_t* y, const uint64_t* const* ext, const uint64_t* const* evk,
                              const uint64_t* add, uint64_t add_stride, uint32_t add_group, uint64_t* out, uint32_t n,
                              uint32_t l, hipStream_t st, const uint32_t* gidx = nullptr);
hipError_t launch_ntt_inv_ksl(const Context& ctx, uint64_t* acc, const JobSpec& js, uint32_t n_jobs,
                              const uint64_t* const* ext, const uint64_t* const* evk, uint32_t n, uint32_t D,
                              uint32_t E, hipStream_t st);
hipError_t launch_ntt_inv_ks(const Context& ctx, uint64_t* acc, const JobSpec& js, uint32_t n_jobs,
                             const uint64_t* ext, const uint64_t* evk, uint32_t D, uint32_t E, hipStream_t st);
hipError_t launch_ntt_fwd_sub(const Context& ctx, uint64_t* y, const uint64_t* x, uint64_t x_pstride,
                              const uint64_t* add, uint64_t add_pstride, uint32_t add_div, uint32_t add_group,
                              uint64_t* out, uint64_t out_pstride, uint32_t n_polys, uint32_t l, const TwPair* s,
                              hipStream_t st, const uint64_t* lift = nullptr, uint64_t lift_pstride = 0,
                              uint64_t lift_q = 0);
hipError_t launch_ntt_fwd_lsub(const Context& ctx, uint64_t* y, uint32_t n_terms, const uint64_t* const* x,
                               const uint32_t* stride, const uint64_t* C, const uint64_t* add, uint64_t* out,
                               uint64_t out_pstride, uint32_t n_polys, uint32_t l, const TwPair* s, hipStream_t st,
                               const uint64_t* lift, uint64_t lift_pstride, uint64_t lift_q);
hipError_t launch_ntt_fwd_mdr(const Context& ctx, uint64_t* T, uint32_t B, uint32_t l, const uint64_t* ext,
                              const uint64_t* evk, const uint64_t* ta, const uint64_t* tb, const uint64_t* add,
                              uint64_t add_pstride, uint64_t* out, const TwPair* pmod, const TwPair* cfin,
                              hipStream_t st, const int64_t* post = nullptr, bool own_from_inputs = false);
hipError_t launch_sub_scale(const Context& ctx, const uint64_t* x, uint64_t x_pstride, const uint64_t* y,
                            uint64_t y_pstride, const uint64_t* add, uint64_t add_pstride, uint32_t add_div,
                            uint64_t* out, uint64_t out_pstride, uint32_t n_polys, uint32_t l, const TwPair* s,
                            hipStream_t st, uint32_t add_group = 0);
hipError_t launch_lift_centered(const Context& ctx, const uint64_t* last, uint64_t last_pstride, uint64_t* tmp,
                                uint32_t n_polys, uint32_t n_out, uint64_t ql, hipStream_t st);
hipError_t launch_add(const Context& ctx, const uint64_t* x, const uint64_t* y, uint64_t* out, uint32_t n_polys,
                      uint32_t l, hipStream_t st);
hipError_t launch_automorph(const uint64_t* in, uint64_t* out, uint32_t n_polys, uint32_t l, uint32_t g,
                            hipStream_t st);
hipError_t launch_ks_inner_list(const Context& ctx, const uint64_t* const* ext, const uint64_t* const* evk,
                                uint64_t* acc, uint32_t n, uint32_t l, hipStream_t st, uint32_t t0 = 0);
hipError_t launch_ks_sub_list(const Context& ctx, const uint64_t* const* ext, const uint64_t* const* evk,
                              const uint64_t* conv, const uint64_t* add, uint64_t add_stride, uint32_t add_group,
                              uint64_t* out, uint32_t n, uint32_t l, const TwPair* pinv, hipStream_t st);
hipError_t launch_automorph_list(const Context& ctx, const uint64_t* in, uint64_t* out, uint32_t n, uint32_t l,
                                 const uint32_t* g, hipStream_t st);
hipError_t launch_bsgs_mac(const Context& ctx, const uint64_t* const* baby, const uint64_t* diag, uint64_t* out,
                           uint32_t nb, uint32_t n_diag, uint32_t ng, uint32_t l, uint32_t log_rep, hipStream_t st,
                           uint32_t l_q = 0, uint32_t n_inst = 1, uint64_t inst_stride = 0, uint64_t out_stride = 0);
hipError_t launch_bsgs_dh_mac(const Context& ctx, const uint64_t* ext, uint64_t ext_stride, const uint64_t* src,
                              uint64_t src_stride, const uint64_t* const* keys, const uint32_t* g, uint32_t n_inst,
                              uint32_t n_in, uint32_t nb, const uint64_t* diag, uint32_t n_diag, uint32_t n_out,
                              uint32_t ngp, int32_t g0, uint32_t l, const TwPair* pmod, uint64_t* out,
                              uint64_t* id_out, uint64_t id_inst_stride, uint64_t id_stride, uint32_t chain_delta,
                              hipStream_t st);
hipError_t launch_qp_rot_sum(const Context& ctx, const uint64_t* ext, uint64_t ext_stride, const uint64_t* src,
                             uint64_t src_stride, const uint64_t* const* keys, const uint32_t* g, uint32_t n_out,
                             uint32_t nt, uint32_t A, uint32_t M, uint32_t l, uint64_t* dst, hipStream_t st,
                             uint32_t R = 1, uint32_t c_off = 0, uint64_t s_lo = 0, bool accumulate = false,
                             const TwPair* src_pmod = nullptr, const uint64_t* id_src = nullptr,
                             uint64_t id_stride = 0);
hipError_t launch_mul_plain(const Context& ctx, const uint64_t* ct, const uint64_t* pt, uint64_t* out, uint32_t B,
                            uint32_t l, uint64_t pt_bstride, uint32_t log_rep, hipStream_t st);
hipError_t launch_add_plain(const Context& ctx, const uint64_t* ct, const uint64_t* pt, uint64_t* out, uint32_t B,
                            uint32_t l, uint64_t pt_bstride, hipStream_t st);
hipError_t launch_lincomb(const Context& ctx, uint64_t* out, uint32_t B, uint32_t l_out, uint32_t n_terms,
                          const uint64_t* const* x, const uint32_t* stride, const uint64_t* C, const uint64_t* add,
                          hipStream_t st, uint32_t i0 = 0);
hipError_t launch_mul_i(const Context& ctx, const uint64_t* in, uint64_t* out, uint32_t n_polys, uint32_t l, int sign,
                        hipStream_t st);
hipError_t launch_pair_mac(const Context& ctx, const uint64_t* R, const uint64_t* pt, uint64_t* out, uint32_t n_sets,
                           uint32_t n, uint32_t l, uint32_t log_rep, hipStream_t st);
hipError_t launch_gather(const Context& ctx, const uint64_t* const* src, uint32_t n, uint64_t words, uint64_t* dst,
                         hipStream_t st);
hipError_t launch_tensor_sum(const Context& ctx, const uint64_t* const* d_tab, uint32_t np, uint64_t* d01,
                             uint64_t* d2, uint32_t B, uint32_t l, uint64_t* d2e, uint64_t d2e_bstride,
                             const uint32_t* ext_off, hipStream_t st);
hipError_t launch_sum_list(const Context& ctx, const uint64_t* const* in, uint32_t n, uint64_t* out, uint32_t n_polys,
                           uint32_t l, hipStream_t st);

namespace {

constexpr size_t W = kN;  // words per limb

#define HIPX(expr)                                                                      \
    do {                                                                                \
        hipError_t _e = (expr);                                                         \
        if (_e != hipSuccess)                                                           \
            throw std::runtime_error(std::string(#expr) + ": " + hipGetErrorString(_e)); \
    } while (0)

uint64_t shoup_companion(uint64_t w, uint64_t q) { return (uint64_t)(((unsigned __int128)w << 64) / q); }

// regular JobSpec over a dense [n_polys][period][N] buffer whose limb t uses prime pmap[t]
JobSpec regular_jobs(uint32_t n_polys, const std::vector<uint32_t>& pmap) {
    JobSpec js{};
    js.jobs = nullptr;
    js.n_polys = n_polys;
    js.period = (uint32_t)pmap.size();
    for (size_t i = 0; i < pmap.size(); i++) js.pmap[i] = (uint8_t)pmap[i];
    return js;
}

// explicit job list, stored once per key; ordered prime-major (jobs sharing a twiddle table adjacent)
JobSpec cached_jobs(Context& ctx, const std::string& key, std::vector<Job> jobs) {
    auto it = ctx.job_cache.find(key);
    if (it == ctx.job_cache.end() && ctx.arena) {
        // allocation-free call: the list goes into the arena for this call only
        std::stable_sort(jobs.begin(), jobs.end(), [](const Job& a, const Job& b) { return a.prime < b.prime; });
        uint32_t distinct = 0;
        for (size_t i = 0; i < jobs.size(); i++) distinct += (i == 0 || jobs[i].prime != jobs[i - 1].prime) ? 1 : 0;
        Job* d = (Job*)arena_take(*ctx.arena, std::max<size_t>(1, jobs.size()) * sizeof(Job));
        HIPX(arena_put(d, jobs.data(), jobs.size() * sizeof(Job), ctx.arena->st));
        JobSpec js{};
        js.jobs = d;
        js.n_primes = distinct;
        return js;
    }
    if (it == ctx.job_cache.end()) {
        std::stable_sort(jobs.begin(), jobs.end(), [](const Job& a, const Job& b) { return a.prime < b.prime; });
        uint32_t distinct = 0;
        for (size_t i = 0; i < jobs.size(); i++) distinct += (i == 0 || jobs[i].prime != jobs[i - 1].prime) ? 1 : 0;
        Job* d = nullptr;
        HIPX(hipMalloc(&d, std::max<size_t>(1, jobs.size()) * sizeof(Job)));
        HIPX(hipMemcpy(d, jobs.data(), jobs.size() * sizeof(Job), hipMemcpyHostToDevice));
        it = ctx.job_cache.emplace(key, std::make_pair(d, distinct)).first;
    }
    JobSpec js{};
    js.jobs = it->second.first;
    js.n_primes = it->second.second;
    return js;
}

}  // namespace

// ------------------------------------------------------------------ workspace
// bump allocation from the arena of an allocation-free call (256-byte aligned); refuses what does not fit
uint8_t* arena_take(Arena& a, size_t bytes) {
    const size_t off = (a.used + 255) & ~(size_t)255;
    if (off > a.cap || bytes > a.cap - off)
        throw std::invalid_argument("the call needs more device scratch than the allocation-free entry point's " +
                                    std::to_string(a.cap >> 20) + " MiB");
    a.used = off + bytes;
    return a.base + off;
}

void* ws_get(Context& ctx, uint32_t slot, size_t bytes) {
    if (ctx.arena) {
        Arena& a = *ctx.arena;
        if (slot >= kArenaSlots) throw std::logic_error("workspace slot out of range");
        // a slot asked for again with more bytes gets a new region (as a regrown workspace buffer would)
        if (a.slot_bytes[slot] < bytes) {
            a.slot_off[slot] = (size_t)(arena_take(a, bytes) - a.base);
            a.slot_bytes[slot] = bytes;
        }
        return a.base + a.slot_off[slot];
    }
    if (ctx.scratch.size() <= slot) ctx.scratch.resize(slot + 1, {nullptr, 0});
    auto& s = ctx.scratch[slot];
    if (s.second < bytes) {
        if (s.first) HIPX(hipFree(s.first));
        s.first = nullptr;
        s.second = 0;
        HIPX(hipMalloc(&s.first, bytes));
        s.second = bytes;
    }
    return s.first;
}

// ------------------------------------------------------------------ pinned table ring
// The next ring slot, waiting (rarely) for the kernel that last read it; allocates the ring on first use.
uint32_t ring_acquire(Context& ctx) {
    if (!ctx.ring_host) {
        HIPX(hipHostMalloc((void**)&ctx.ring_host, Context::kRingSlots * Context::kRingSlotBytes,
                           hipHostMallocDefault));
        HIPX(hipMalloc((void**)&ctx.ring_dev, Context::kRingSlots * Context::kRingSlotBytes));
        for (auto& e : ctx.ring_ev) HIPX(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    const uint32_t slot = ctx.ring_next;
    ctx.ring_next = (ctx.ring_next + 1) % Context::kRingSlots;
    if (ctx.ring_used[slot]) HIPX(hipEventSynchronize(ctx.ring_ev[slot]));
    return slot;
}

// marks the slot busy until the work enqueued on st so far (the copy and the kernel reading it) completes
void ring_release(Context& ctx, uint32_t slot, hipStream_t st) {
    HIPX(hipEventRecord(ctx.ring_ev[slot], st));
    ctx.ring_used[slot] = true;
}

// ------------------------------------------------------------------ BConv plans
// Montgomery reduction of the output sums is exact when every sum stays below p_j 2^64: a sum is at most
// p_j (sum_i q_i) plus the centered correction (below 16 p_j)
static bool bconv_mont(const Context& ctx, const std::vector<uint32_t>& in_idx) {
    unsigned __int128 s = 16;
    for (auto i : in_idx) s += ctx.moduli[i];
    return s < ((unsigned __int128)1 << 64);
}

const BConvPlan& bconv_plan(Context& ctx, const std::vector<uint32_t>& in_idx, const std::vector<uint32_t>& out_idx,
                            bool centered, const std::vector<uint64_t>& col_scale) {
    if (!col_scale.empty() && col_scale.size() != out_idx.size())
        throw std::invalid_argument("one column scale per BConv output");
    std::string key = centered ? "c" : "b";
    for (auto i : in_idx) key += ":" + std::to_string(i);
    key += ">";
    for (auto j : out_idx) key += ":" + std::to_string(j);
    if (!col_scale.empty()) {
        key += "*";
        for (auto f : col_scale) key += ":" + std::to_string(f);
    }
    auto it = ctx.bconv_cache.find(key);
    if (it != ctx.bconv_cache.end()) return it->second;
    BConvPlan p;
    if (ctx.arena) {
        // allocation-free call: the table (host copy computed once per context) goes into the arena
        auto ht = ctx.bconv_host.find(key);
        if (ht != ctx.bconv_host.end()) {
            p.n_in = (uint32_t)in_idx.size();
            p.n_out = (uint32_t)out_idx.size();
            p.in_idx = in_idx;
            p.out_idx = out_idx;
            p.centered = centered;
            p.mont = bconv_mont(ctx, in_idx);
            p.d_tab = (uint64_t*)arena_take(*ctx.arena, ht->second.size() * 8);
            HIPX(arena_put(p.d_tab, ht->second.data(), ht->second.size() * 8, ctx.arena->st));
            ctx.arena->plans.push_back(std::move(p));
            return ctx.arena->plans.back();
        }
    }
    p.n_in = (uint32_t)in_idx.size();
    p.n_out = (uint32_t)out_idx.size();
    p.in_idx = in_idx;
    p.out_idx = out_idx;
    p.centered = centered;
    p.mont = bconv_mont(ctx, in_idx);
    // R = 2^64 mod p_j: the Montgomery form of a table column
    auto to_mont = [&](uint64_t v, uint64_t pj) {
        return p.mont ? (uint64_t)(((unsigned __int128)v << 64) % pj) : v;
    };
    std::vector<uint64_t> tab(2 * p.n_in + (size_t)p.n_in * p.n_out + (centered ? 2 * p.n_in + p.n_out : 0));
    for (uint32_t i = 0; i < p.n_in; i++) {
        const uint64_t qi = ctx.moduli[in_idx[i]];
        uint64_t prod = 1;
        for (uint32_t k = 0; k < p.n_in; k++)
            if (k != i) prod = mulmod_h(prod, ctx.moduli[in_idx[k]] % qi, qi);
        const uint64_t inv = invmod_h(prod, qi);
        tab[2 * i] = inv;
        tab[2 * i + 1] = shoup_companion(inv, qi);
        for (uint32_t j = 0; j < p.n_out; j++) {
            const uint64_t pj = ctx.moduli[out_idx[j]];
            uint64_t m = 1;
            for (uint32_t k = 0; k < p.n_in; k++)
                if (k != i) m = mulmod_h(m, ctx.moduli[in_idx[k]] % pj, pj);
            const uint64_t v = to_mont(col_scale.empty() ? m : mulmod_h(m, col_scale[j], pj), pj);
            tab[2 * p.n_in + (size_t)i * p.n_out + j] = ((v >> 30) << 32) | (v & 0x3FFFFFFFull);  // pack30
        }
    }
    if (centered) {
        uint64_t* cfix = tab.data() + 2 * p.n_in + (size_t)p.n_in * p.n_out;
        for (uint32_t i = 0; i < p.n_in; i++) {
            const unsigned __int128 c = (~(unsigned __int128)0) / ctx.moduli[in_idx[i]];  // floor(2^128 / q_i)
            cfix[2 * i] = (uint64_t)c;
            cfix[2 * i + 1] = (uint64_t)(c >> 64);
        }
        for (uint32_t j = 0; j < p.n_out; j++) {
            const uint64_t pj = ctx.moduli[out_idx[j]];
            uint64_t m = 1;
            for (uint32_t k = 0; k < p.n_in; k++) m = mulmod_h(m, ctx.moduli[in_idx[k]] % pj, pj);
            cfix[2 * p.n_in + j] = to_mont(col_scale.empty() ? m : mulmod_h(m, col_scale[j], pj), pj);
        }
    }
    if (ctx.arena) {
        p.d_tab = (uint64_t*)arena_take(*ctx.arena, tab.size() * 8);
        HIPX(arena_put(p.d_tab, tab.data(), tab.size() * 8, ctx.arena->st));
        ctx.bconv_host.emplace(key, std::move(tab));
        ctx.arena->plans.push_back(std::move(p));
        return ctx.arena->plans.back();
    }
    HIPX(hipMalloc(&p.d_tab, tab.size() * 8));
    HIPX(hipMemcpy(p.d_tab, tab.data(), tab.size() * 8, hipMemcpyHostToDevice));
    return ctx.bconv_cache.emplace(key, std::move(p)).first->second;
}

// ------------------------------------------------------------------ level geometry
uint32_t num_digits(const Context& ctx, uint32_t l) { return (l + ctx.alpha - 1) / ctx.alpha; }

// P mod q (P the product of the special primes)
static uint64_t p_mod(const Context& ctx, uint64_t q) {
    uint64_t P = 1;
    for (uint32_t k = 0; k < ctx.K; k++) P = mulmod_h(P, ctx.moduli[ctx.L + k] % q, q);
    return P;
}

// the per-limb constant tables of the context (each computed once; a call reads the first l entries)
static const std::vector<TwPair>& pinv_tab(Context& ctx) {
    if (ctx.tab_pinv.empty()) {
        for (uint32_t i = 0; i < ctx.L; i++) {
            const uint64_t q = ctx.moduli[i], v = invmod_h(p_mod(ctx, q), q);
            ctx.tab_pinv.push_back(TwPair{v, shoup_companion(v, q)});
        }
    }
    return ctx.tab_pinv;
}

static const std::vector<TwPair>& pmodr_tab(Context& ctx) {
    if (ctx.tab_pmodr.empty()) {
        for (uint32_t i = 0; i < ctx.L; i++) {
            const uint64_t q = ctx.moduli[i];
            const uint64_t rinv = invmod_h((uint64_t)(((unsigned __int128)1 << 64) % q), q);
            const uint64_t v = mulmod_h(p_mod(ctx, q), rinv, q);
            ctx.tab_pmodr.push_back(TwPair{v, shoup_companion(v, q)});
        }
    }
    return ctx.tab_pmodr;
}

static const std::vector<TwPair>& pmod_tab(Context& ctx) {
    if (ctx.tab_pmod.empty()) {
        for (uint32_t i = 0; i < ctx.L; i++) {
            const uint64_t q = ctx.moduli[i], v = p_mod(ctx, q);
            ctx.tab_pmod.push_back(TwPair{v, shoup_companion(v, q)});
        }
    }
    return ctx.tab_pmod;
}

// an integer (|v| < 2^120, carried as long double) reduced mod q
static uint64_t residue_of(long double v, uint64_t q) {
    const bool neg = v < 0;
    const unsigned __int128 x = (unsigned __int128)(neg ? -v : v);
    const uint64_t r = (uint64_t)(x % q);
    return neg ? (r ? q - r : 0) : r;
}

static const std::vector<TwPair>& qinv_row(Context& ctx, uint32_t j) {
    auto it = ctx.tab_qinv.find(j);
    if (it != ctx.tab_qinv.end()) return it->second;
    std::vector<TwPair> row(j);
    const uint64_t qj = ctx.moduli[j];
    for (uint32_t i = 0; i < j; i++) {
        const uint64_t q = ctx.moduli[i], v = invmod_h(qj % q, q);
        row[i] = TwPair{v, shoup_companion(v, q)};
    }
    return ctx.tab_qinv.emplace(j, std::move(row)).first->second;
}

static uint32_t ext_prime(const Context& ctx, uint32_t l, uint32_t t) { return t < l ? t : ctx.L + (t - l); }

static void check_level(const Context& ctx, uint32_t l) {
    if (l == 0 || l > ctx.L) throw std::invalid_argument("level (limb count) out of range");
    if (num_digits(ctx, l) > 8) throw std::invalid_argument("more than 8 digits");
}

// ------------------------------------------------------------------ ModUp
// x2c: [B][l][N] coefficient form (INTT already applied) of the polynomial to extend;
// ext: [B][D][E][N].  Fills every limb but the digits' own (neither read nor written here: the caller stores them in
// evaluation form, or their consumer forms them).
void modup_from_coef(Context& ctx, const uint64_t* x2c, uint64_t* ext, uint32_t B, uint32_t l, hipStream_t st) {
    const uint32_t D = num_digits(ctx, l), E = l + ctx.K, al = ctx.alpha;
    std::vector<Job> jobs;
    for (uint32_t d = 0; d < D; d++) {
        const uint32_t lo = d * al, hi = std::min(lo + al, l);
        std::vector<uint32_t> in_idx, in_off, out_idx, out_off;
        for (uint32_t i = lo; i < hi; i++) {
            in_idx.push_back(i);
            in_off.push_back(i);
        }
        for (uint32_t t = 0; t < E; t++) {
            if (t >= lo && t < hi) continue;
            out_idx.push_back(ext_prime(ctx, l, t));
            out_off.push_back(t);
        }
        const BConvPlan& plan = bconv_plan(ctx, in_idx, out_idx);
        HIPX(launch_bconv(ctx, plan, x2c, (uint64_t)l * W, in_off.data(), ext + (size_t)d * E * W,
                          (uint64_t)D * E * W, out_off.data(), B, st));
        for (uint32_t b = 0; b < B; b++)
            for (uint32_t j = 0; j < out_off.size(); j++)
                jobs.push_back(Job{(b * D + d) * E + out_off[j], out_idx[j]});
    }
    const JobSpec js = cached_jobs(ctx, "modup:" + std::to_string(B) + ":" + std::to_string(l), std::move(jobs));
    const uint32_t n_jobs = B * D * (E) - B * l;  // every limb of every digit except the digit's own
    HIPX(launch_ntt(ctx, ext, js, n_jobs, false, ctx.ntt_mode, st));
}

// x: [B] polys of l limbs, x_bstride words apart (0: l * N), evaluation form -> ext [B][D][E][N] evaluation
// form.  x is only read: the inverse NTT reads x, writes the coefficient-form copy it works on (so a ciphertext's
// c1 is extended in place, no extraction) and, in its first pass, copies x's limbs into their digits' own limbs of
// ext.
void modup(Context& ctx, const uint64_t* x, uint64_t* ext, uint32_t B, uint32_t l, hipStream_t st,
           uint64_t x_bstride) {
    check_level(ctx, l);
    const uint32_t D = num_digits(ctx, l), E = l + ctx.K, al = ctx.alpha;
    if (x_bstride == 0) x_bstride = (uint64_t)l * W;
    if (x_bstride % W) throw std::invalid_argument("ModUp input stride must be whole limbs");
    uint64_t* xc = (uint64_t*)ws_get(ctx, WS_X2C, (size_t)B * l * W * 8);
    std::vector<uint32_t> pm(l);
    for (uint32_t t = 0; t < l; t++) pm[t] = t;
    JobSpec js = regular_jobs(B, pm);
    js.src = x;
    js.src_period = (uint32_t)(x_bstride / W);
    js.copy = ext;
    js.copy_pstride = (uint64_t)D * E * W;
    js.copy_alpha = al;
    js.copy_E = E;
    HIPX(launch_ntt(ctx, xc, js, B * l, true, ctx.ntt_mode, st));
    modup_from_coef(ctx, xc, ext, B, l, st);
}

// ------------------------------------------------------------------ inner product
void ks_inner(Context& ctx, const uint64_t* ext, const uint64_t* evk, uint64_t* acc, uint32_t B, uint32_t l,
              hipStream_t st) {
    check_level(ctx, l);
    HIPX(launch_ks_inner(ctx, ext, evk, acc, B, l, st));
}

// ------------------------------------------------------------------ ModDown
// x: [n_polys][E][N] evaluation form over Q_l * P (P limbs are overwritten: they are transformed to
// coefficients in place).  out: [n_polys][l][N] = (x_Q - BConv_{P->Q}(x_P)) * P^-1 (+ add).
void moddown_inplace(Context& ctx, uint64_t* x, uint32_t n_polys, uint32_t l, const uint64_t* add, uint64_t* out,
                     hipStream_t st, uint32_t add_div, int64_t add_pstride, uint32_t add_group, uint32_t x_plimbs) {
    check_level(ctx, l);
    const uint32_t E = l + ctx.K, K = ctx.K;
    if (K == 0) throw std::invalid_argument("ModDown needs special primes");
    const uint32_t xs = x_plimbs ? x_plimbs : E;  // limbs between the polys of x
    if (xs < E) throw std::invalid_argument("ModDown: poly stride below the extended limb count");
    std::vector<Job> jobs;
    for (uint32_t pc = 0; pc < n_polys; pc++)
        for (uint32_t k = 0; k < K; k++) jobs.push_back(Job{pc * xs + l + k, ctx.L + k});
    const JobSpec js = cached_jobs(ctx, "mdP:" + std::to_string(n_polys) + ":" + std::to_string(l) + ":" +
                                            std::to_string(xs),
                                   std::move(jobs));
    HIPX(launch_ntt(ctx, x, js, n_polys * K, true, ctx.ntt_mode, st));
    std::vector<uint32_t> in_idx, in_off, out_idx, out_off;
    for (uint32_t k = 0; k < K; k++) {
        in_idx.push_back(ctx.L + k);
        in_off.push_back(l + k);
    }
    for (uint32_t i = 0; i < l; i++) {
        out_idx.push_back(i);
        out_off.push_back(i);
    }
    const BConvPlan& plan = bconv_plan(ctx, in_idx, out_idx, ctx.moddown_exact);
    uint64_t* conv = (uint64_t*)ws_get(ctx, WS_CONV, (size_t)n_polys * l * W * 8);
    HIPX(launch_bconv(ctx, plan, x, (uint64_t)xs * W, in_off.data(), conv, (uint64_t)l * W, out_off.data(), n_polys,
                      st));
    const std::vector<TwPair> pinv(pinv_tab(ctx).begin(), pinv_tab(ctx).begin() + l);
    const uint64_t aps = add_pstride < 0 ? (uint64_t)add_div * l * W : (uint64_t)add_pstride;
    if (ctx.ntt_mode == NttMode::TwoPass) {
        // the forward NTT of conv ends in the combine (conv is never stored in evaluation form)
        HIPX(launch_ntt_fwd_sub(ctx, conv, x, (uint64_t)xs * W, add, aps, add_div, add_group, out, (uint64_t)l * W,
                                n_polys, l, pinv.data(), st));
        return;
    }
    HIPX(launch_ntt(ctx, conv, regular_jobs(n_polys, out_idx), n_polys * l, false, ctx.ntt_mode, st));
    HIPX(launch_sub_scale(ctx, x, (uint64_t)xs * W, conv, (uint64_t)l * W, add, aps, add_div, out, (uint64_t)l * W,
                          n_polys, l, pinv.data(), st, add_group));
}

// ModDown fused with the rescale that follows it (the same words as moddown_inplace + rescale, one forward
// NTT of l-1 limbs fewer): x [n_polys][E][N] evaluation form over Q_l * P (its P limbs and limb l-1 are
// transformed in place), add [n_polys][l][N] (or null) -> out [n_polys][l-1][N].  The BConv writes
// T_i = conv_i P^-1 + lift(z)_i directly (P^-1 folded into its table).  With ext/evk given (a relinearization,
// n_polys = 2B), x holds only limbs l-1.. of the evk inner product (k_ks_inner from t0 = l-1) and the combine
// forms limbs 0..l-2 itself from ext and evk.
void moddown_rescale(Context& ctx, uint64_t* x, uint32_t n_polys, uint32_t l, const uint64_t* add, uint64_t* out,
                     hipStream_t st, const uint64_t* ext, const uint64_t* evk, const uint64_t* ta,
                     const uint64_t* tb, bool x_from_ext, const Affine* aff, bool own_from_inputs) {
    if (aff && !ext) throw std::invalid_argument("an affine output needs a relinearization");
    if (own_from_inputs && (!ext || !ta || ctx.ntt_mode != NttMode::TwoPass || num_digits(ctx, l) > 4))
        throw std::logic_error("own-digit words from the inputs need the fused two-pass combine");
    check_level(ctx, l);
    if (l < 2) throw std::invalid_argument("rescale needs l >= 2");
    const uint32_t E = l + ctx.K, K = ctx.K;
    if (K == 0) throw std::invalid_argument("ModDown needs special primes");
    // P limbs and limb l-1 of x to coefficients, in place
    std::vector<Job> jobs;
    for (uint32_t pc = 0; pc < n_polys; pc++) {
        jobs.push_back(Job{pc * E + l - 1, l - 1});
        for (uint32_t k = 0; k < K; k++) jobs.push_back(Job{pc * E + l + k, ctx.L + k});
    }
    const JobSpec js = cached_jobs(ctx, "mdrP:" + std::to_string(n_polys) + ":" + std::to_string(l), std::move(jobs));
    if (x_from_ext)  // those limbs of x are the evk inner product, formed by the transform's first pass
        HIPX(launch_ntt_inv_ks(ctx, x, js, n_polys * (K + 1), ext, evk, num_digits(ctx, l), E, st));
    else
        HIPX(launch_ntt(ctx, x, js, n_polys * (K + 1), true, ctx.ntt_mode, st));
    // limb l-1 of the addend to coefficients (a copy: the addend is the caller's)
    uint64_t* addc = nullptr;
    if (add) {
        addc = (uint64_t*)ws_get(ctx, WS_LAST, (size_t)n_polys * W * 8);
        JobSpec ja = regular_jobs(n_polys, {l - 1});
        ja.src = add + (size_t)(l - 1) * W;
        ja.src_period = l;
        HIPX(launch_ntt(ctx, addc, ja, n_polys, true, ctx.ntt_mode, st));
    }
    const std::vector<TwPair>& ptab = pinv_tab(ctx);
    const std::vector<TwPair>& qrow = qinv_row(ctx, l - 1);
    std::vector<TwPair> pinv(ptab.begin(), ptab.begin() + l), qlinv(l);
    std::vector<uint64_t> col(l);
    for (uint32_t i = 0; i < l; i++) {
        col[i] = i + 1 < l ? pinv[i].w : 1;  // columns 0..l-2 carry P^-1; the dropped limb's column stays plain
        qlinv[i] = i + 1 < l ? qrow[i] : TwPair{0, 0};
    }
    std::vector<uint32_t> in_idx, in_off, out_idx;
    for (uint32_t k = 0; k < K; k++) {
        in_idx.push_back(ctx.L + k);
        in_off.push_back(l + k);
    }
    for (uint32_t i = 0; i < l; i++) out_idx.push_back(i);
    const BConvPlan& plan = bconv_plan(ctx, in_idx, out_idx, ctx.moddown_exact, col);
    uint64_t* T = (uint64_t*)ws_get(ctx, WS_RTMP, (size_t)n_polys * (l - 1) * W * 8);
    const uint64_t xps = (uint64_t)E * W;
    HIPX(launch_bconv_mdr(ctx, plan, x, xps, in_off.data(), T, n_polys, x + (size_t)(l - 1) * W, xps, addc,
                          pinv[l - 1], st));
    std::vector<uint32_t> pm(l - 1);
    for (uint32_t i = 0; i + 1 < l; i++) pm[i] = i;
    // a relinearization: T's forward NTT finishes with the combine in its second pass (the addend formed from the
    // product's inputs, or read), so T is never stored in evaluation form
    const uint32_t D = num_digits(ctx, l);
    if (ext && ctx.ntt_mode == NttMode::TwoPass && D <= 4) {
        // the combine reduces one 128-bit sum by REDC and scales it by R P^-1 q_{l-1}^-1 (R = 2^64)
        // (times the affine factor: the combine's one Shoup product scales the word by it)
        std::vector<TwPair> cfin(l - 1);
        for (uint32_t i = 0; i + 1 < l; i++) {
            const uint64_t q = ctx.moduli[i];
            uint64_t v = mulmod_h(mulmod_h(pinv[i].w, qlinv[i].w, q), ctx.primes[i].r_mod, q);
            if (aff) v = mulmod_h(v, residue_of((long double)aff->factor, q), q);
            cfin[i] = TwPair{v, shoup_companion(v, q)};
        }
        HIPX(launch_ntt_fwd_mdr(ctx, T, n_polys / 2, l, ext, evk, ta, tb, ta ? nullptr : add, (uint64_t)l * W, out,
                                pmod_tab(ctx).data(), cfin.data(), st, aff ? &aff->post : nullptr, own_from_inputs));
        return;
    }
    HIPX(launch_ntt(ctx, T, regular_jobs(n_polys, pm), n_polys * (l - 1), false, ctx.ntt_mode, st));
    if (ext && ta)  // the addend formed from the product's inputs (add holds limb l-1 only, read above)
        HIPX(launch_mdr_combine_ks(ctx, ext, evk, nullptr, 0, T, out, n_polys / 2, l, pinv.data(), qlinv.data(), st,
                                   ta, tb));
    else if (ext)
        HIPX(launch_mdr_combine_ks(ctx, ext, evk, add, (uint64_t)l * W, T, out, n_polys / 2, l, pinv.data(),
                                   qlinv.data(), st));
    else
        HIPX(launch_mdr_combine(ctx, x, xps, add, (uint64_t)l * W, T, out, n_polys, l, pinv.data(), qlinv.data(),
                                st));
    if (aff) {  // the affine map as an integer combination over the output, in place
        const uint32_t lo = l - 1, B = n_polys / 2;
        std::vector<uint64_t> C(lo), pa(lo);
        for (uint32_t i = 0; i < lo; i++) {
            C[i] = residue_of((long double)aff->factor, ctx.moduli[i]);
            pa[i] = residue_of((long double)aff->post, ctx.moduli[i]);
        }
        const uint64_t* xs[1] = {out};
        const uint32_t stride[1] = {lo};
        HIPX(launch_lincomb(ctx, out, B, lo, 1, xs, stride, C.data(), aff->post ? pa.data() : nullptr, st));
    }
}

// Key switch of a list of n <= 64 items (item c: extended digits ext[c] [D][E][N], key evk[c]) with its ModDown:
// out [n][2][l][N] = ((sum_d ext_c[d] evk_c[d])_Q - BConv_{P->Q}(.._P)) P^-1, plus the addend's poly 0 (the
// ciphertext at add + (c / add_group) * add_stride) on poly 0.  The inner product of the P limbs is formed by their
// inverse NTT's first pass (stored first under the fused NTT mode); the combine, at the end of the converted part's
// forward NTT, forms the Q limbs' itself; P^-1 rides in the BConv table.  Same words as k_ks_inner_list +
// moddown_inplace.  gidx (optional): item c's output is then mapped by X -> X^gidx[c] (a rotation's automorphism),
// applied by the combine as it stores.
void ks_moddown_list(Context& ctx, const uint64_t* const* ext, const uint64_t* const* evk, uint32_t n, uint32_t l,
                     const uint64_t* add, uint64_t add_stride, uint32_t add_group, uint64_t* out, hipStream_t st,
                     const uint32_t* gidx = nullptr) {
    check_level(ctx, l);
    const uint32_t E = l + ctx.K, K = ctx.K;
    if (K == 0) throw std::invalid_argument("ModDown needs special primes");
    uint64_t* acc = (uint64_t*)ws_get(ctx, WS_ACC, (size_t)n * 2 * E * W * 8);
    const bool fused = ctx.ntt_mode == NttMode::TwoPass && num_digits(ctx, l) <= 4;
    std::vector<Job> jobs;
    for (uint32_t pc = 0; pc < 2 * n; pc++)
        for (uint32_t k = 0; k < K; k++) jobs.push_back(Job{pc * E + l + k, ctx.L + k});
    const JobSpec js = cached_jobs(ctx, "mdP:" + std::to_string(2 * n) + ":" + std::to_string(l), std::move(jobs));
    if (fused) {
        // the P limbs' inner products are formed by their inverse NTT's first pass
        ctx.n_keyswitch += n;
        HIPX(launch_ntt_inv_ksl(ctx, acc, js, 2 * n * K, ext, evk, n, num_digits(ctx, l), E, st));
    } else {
        HIPX(launch_ks_inner_list(ctx, ext, evk, acc, n, l, st, l));
        HIPX(launch_ntt(ctx, acc, js, 2 * n * K, true, ctx.ntt_mode, st));
    }
    std::vector<uint32_t> in_idx, in_off, out_idx;
    for (uint32_t k = 0; k < K; k++) {
        in_idx.push_back(ctx.L + k);
        in_off.push_back(l + k);
    }
    const std::vector<TwPair> pinv(pinv_tab(ctx).begin(), pinv_tab(ctx).begin() + l);
    std::vector<uint64_t> col(l);
    for (uint32_t i = 0; i < l; i++) {
        out_idx.push_back(i);
        col[i] = pinv[i].w;
    }
    const BConvPlan& plan = bconv_plan(ctx, in_idx, out_idx, ctx.moddown_exact, col);
    uint64_t* conv = (uint64_t*)ws_get(ctx, WS_CONV, (size_t)2 * n * l * W * 8);
    HIPX(launch_bconv(ctx, plan, acc, (uint64_t)E * W, in_off.data(), conv, (uint64_t)l * W, out_idx.data(), 2 * n,
                      st));
    // the combine applies the automorphisms as it stores, unless out overlaps the addends' polys 0 (a permuted store
    // may land on words another workgroup has still to read): then the key switch goes to a workspace first
    const uint64_t* add_end = add ? add + (size_t)((n - 1) / std::max(add_group, 1u)) * add_stride + (size_t)l * W : nullptr;
    const bool add_overlap = add && out < add_end && add < out + (size_t)n * 2 * l * W;
    uint64_t* ks = gidx && (!fused || add_overlap) ? (uint64_t*)ws_get(ctx, WS_RELIN, (size_t)n * 2 * l * W * 8) : out;
    if (fused) {
        // the forward NTT of conv ends in the combine (conv never stored in evaluation form)
        HIPX(launch_ntt_fwd_ksl(ctx, conv, ext, evk, add, add_stride, add_group, ks, n, l, st,
                                ks == out ? gidx : nullptr));
    } else {
        HIPX(launch_ntt(ctx, conv, regular_jobs(2 * n, out_idx), 2 * n * l, false, ctx.ntt_mode, st));
        HIPX(launch_ks_sub_list(ctx, ext, evk, conv, add, add_stride, add_group, ks, n, l, pinv.data(), st));
    }
    if (gidx && ks != out) HIPX(launch_automorph_list(ctx, ks, out, n, l, gidx, st));
}

// ------------------------------------------------------------------ key switch
// x: [B][l][N] eval; evk [dnum][2][L+K][N]; out2: [B][2][l][N] (+= add [B][2][l][N] if given)
// x_bstride: words between the B input polys (0: l * N)
void keyswitch(Context& ctx, const uint64_t* x, uint32_t B, uint32_t l, const uint64_t* evk, const uint64_t* add,
               uint64_t* out2, hipStream_t st, uint32_t add_div, uint64_t x_bstride) {
    check_level(ctx, l);
    const uint32_t D = num_digits(ctx, l), E = l + ctx.K;
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)B * D * E * W * 8);
    uint64_t* acc = (uint64_t*)ws_get(ctx, WS_ACC, (size_t)B * 2 * E * W * 8);
    modup(ctx, x, ext, B, l, st, x_bstride);
    if (ctx.ntt_mode == NttMode::TwoPass && D <= 4 && B <= 64 && (!add || add_div == 2)) {
        // as a key-switch list with one key (up to 64 items): the inner products are formed by the ModDown's NTTs
        // (the addend, when given, is a ciphertext batch whose c0 goes on poly 0)
        std::vector<const uint64_t*> pe(B), pk(B, evk);
        for (uint32_t c = 0; c < B; c++) pe[c] = ext + (size_t)c * D * E * W;
        ks_moddown_list(ctx, pe.data(), pk.data(), B, l, add, add ? (uint64_t)2 * l * W : 0, 1, out2, st);
        return;
    }
    HIPX(launch_ks_inner(ctx, ext, evk, acc, B, l, st));
    moddown_inplace(ctx, acc, 2 * B, l, add, out2, st, add_div);
}

// ------------------------------------------------------------------ rescale
// in: [n_polys][l][N] eval -> out: [n_polys][l-1][N] eval.  in may equal neither out nor workspace.
void rescale(Context& ctx, const uint64_t* in, uint32_t n_polys, uint32_t l, uint64_t* out, hipStream_t st) {
    if (l < 2 || l > ctx.L) throw std::invalid_argument("rescale needs 2 <= l <= L");
    uint64_t* last = (uint64_t*)ws_get(ctx, WS_LAST, (size_t)n_polys * W * 8);
    uint64_t* tmp = (uint64_t*)ws_get(ctx, WS_RTMP, (size_t)n_polys * (l - 1) * W * 8);
    // the dropped limb of every poly to coefficients, read in place
    JobSpec jl = regular_jobs(n_polys, {l - 1});
    jl.src = in + (size_t)(l - 1) * W;
    jl.src_period = l;
    HIPX(launch_ntt(ctx, last, jl, n_polys, true, ctx.ntt_mode, st));
    const std::vector<TwPair>& s = qinv_row(ctx, l - 1);  // q_{l-1}^-1 mod q_i, i < l-1
    const uint64_t ql = ctx.moduli[l - 1];
    if (ctx.ntt_mode == NttMode::TwoPass) {
        // the lift happens in the forward NTT's first pass, and its second pass ends in the combine:
        // out = (in - NTT(lift(last))) q_{l-1}^-1
        HIPX(launch_ntt_fwd_sub(ctx, tmp, in, (uint64_t)l * W, nullptr, 0, 1, 0, out, (uint64_t)(l - 1) * W, n_polys,
                                l - 1, s.data(), st, last, W, ql));
        return;
    }
    HIPX(launch_lift_centered(ctx, last, W, tmp, n_polys, l - 1, ql, st));
    std::vector<uint32_t> pm(l - 1);
    for (uint32_t i = 0; i + 1 < l; i++) pm[i] = i;
    HIPX(launch_ntt(ctx, tmp, regular_jobs(n_polys, pm), n_polys * (l - 1), false, ctx.ntt_mode, st));
    HIPX(launch_sub_scale(ctx, in, (uint64_t)l * W, tmp, (uint64_t)(l - 1) * W, nullptr, 0, 1, out,
                          (uint64_t)(l - 1) * W, n_polys, l - 1, s.data(), st));
}

// Rescaled linear combination of ciphertext batches: out [B][2][lo-1][N] = rescale(sum_t C_t x_t + add) with the
// combination formed at lo limbs (term t read in place, stride[t] >= lo limbs per poly; add on poly 0).  C [n_terms][lo]
// and add [lo] (or null) reduced mod q_i.  The same words as a lincomb launch into a buffer and its rescale: under the
// two-pass NTT the combination is never stored -- its dropped limb alone is formed for the inverse NTT, and the other
// limbs are formed by the rescale's combine (k_ntt_fwd_b_lsub) from the terms.
void rescale_lincomb(Context& ctx, uint32_t B, uint32_t lo, uint32_t n_terms, const uint64_t* const* x,
                     const uint32_t* stride, const uint64_t* C, const uint64_t* add, uint64_t* out, hipStream_t st) {
    if (lo < 2 || lo > ctx.L) throw std::invalid_argument("rescale needs 2 <= l <= L");
    const uint32_t n_polys = 2 * B, lt = lo - 1;
    if (ctx.ntt_mode != NttMode::TwoPass || lt > 32 || n_terms > 8) {
        uint64_t* tmp = (uint64_t*)ws_get(ctx, WS_LIN, (size_t)n_polys * lo * W * 8);
        HIPX(launch_lincomb(ctx, tmp, B, lo, n_terms, x, stride, C, add, st));
        rescale(ctx, tmp, n_polys, lo, out, st);
        return;
    }
    // the dropped limb lo-1 of the combination, then to coefficients
    uint64_t* last_in = (uint64_t*)ws_get(ctx, WS_LIN, (size_t)n_polys * W * 8);
    std::vector<uint64_t> Cl(n_terms);
    for (uint32_t t = 0; t < n_terms; t++) Cl[t] = C[(size_t)t * lo + lt];
    HIPX(launch_lincomb(ctx, last_in, B, 1, n_terms, x, stride, Cl.data(), add ? add + lt : nullptr, st, lt));
    uint64_t* last = (uint64_t*)ws_get(ctx, WS_LAST, (size_t)n_polys * W * 8);
    JobSpec jl = regular_jobs(n_polys, {lt});
    jl.src = last_in;
    jl.src_period = 1;
    HIPX(launch_ntt(ctx, last, jl, n_polys, true, ctx.ntt_mode, st));
    // limbs 0..lo-2: (x - NTT(lift(last))) q_{lo-1}^-1 with x formed from the terms
    uint64_t* y = (uint64_t*)ws_get(ctx, WS_RTMP, (size_t)n_polys * lt * W * 8);
    std::vector<uint64_t> Ck((size_t)n_terms * lt);
    for (uint32_t t = 0; t < n_terms; t++)
        for (uint32_t i = 0; i < lt; i++) Ck[(size_t)t * lt + i] = C[(size_t)t * lo + i];
    const std::vector<TwPair>& s = qinv_row(ctx, lt);
    HIPX(launch_ntt_fwd_lsub(ctx, y, n_terms, x, stride, Ck.data(), add, out, (uint64_t)lt * W, n_polys, lt, s.data(),
                             st, last, W, ctx.moduli[lt]));
}

// ------------------------------------------------------------------ HMult + relinearize (+ rescale)
// a, b: [B][2][l][N] eval -> out: [B][2][l-1][N] (rescaled) or [B][2][l][N] (do_rescale = false)
// relinearization (+ rescale) after the tensor step: d01 [B][2][l][N], d2 in x2c (evaluation form) and in
// each digit's own limbs of ext
// ta, tb: the product's inputs when the tensor kernel wrote d0 and d1 for limb l-1 only (with the rescale)
// x2c_coef: x2c already holds d2 in coefficient form (the inverse NTT formed it from the inputs)
// own_from_inputs: ext's own-digit limbs hold d2 at limb l-1 only (the ModDown combine forms the others from ta, tb)
static void relin_tail(Context& ctx, uint64_t* d01, uint64_t* x2c, uint64_t* ext, uint32_t B, uint32_t l,
                       const uint64_t* evk, uint64_t* out, bool do_rescale, hipStream_t st,
                       const uint64_t* ta = nullptr, const uint64_t* tb = nullptr, bool x2c_coef = false,
                       const Affine* aff = nullptr, bool own_from_inputs = false) {
    if (aff && !do_rescale) throw std::invalid_argument("an affine output needs the rescale");
    const uint32_t E = l + ctx.K;
    uint64_t* acc = (uint64_t*)ws_get(ctx, WS_ACC, (size_t)B * 2 * E * W * 8);
    std::vector<uint32_t> pm(l);
    for (uint32_t i = 0; i < l; i++) pm[i] = i;
    if (!x2c_coef) HIPX(launch_ntt(ctx, x2c, regular_jobs(B, pm), B * l, true, ctx.ntt_mode, st));
    modup_from_coef(ctx, x2c, ext, B, l, st);
    if (!do_rescale) {
        HIPX(launch_ks_inner(ctx, ext, evk, acc, B, l, st));
        moddown_inplace(ctx, acc, 2 * B, l, d01, out, st, 1);
        return;
    }
    // inner product of limb l-1 and the P limbs only, formed by their inverse NTT's first pass (or stored first, under
    // the fused NTT mode or more than 4 digits); the combine forms limbs 0..l-2
    if (ctx.ntt_mode == NttMode::TwoPass && num_digits(ctx, l) <= 4) {
        ctx.n_keyswitch += B;
        moddown_rescale(ctx, acc, 2 * B, l, d01, out, st, ext, evk, ta, tb, true, aff, own_from_inputs);
        return;
    }
    if (own_from_inputs) throw std::logic_error("own-digit words from the inputs need the fused two-pass combine");
    HIPX(launch_ks_inner(ctx, ext, evk, acc, B, l, st, l - 1));
    moddown_rescale(ctx, acc, 2 * B, l, d01, out, st, ext, evk, ta, tb, false, aff);
}

void hmult(Context& ctx, const uint64_t* a, const uint64_t* b, uint32_t B, uint32_t l, const uint64_t* evk,
           uint64_t* out, bool do_rescale, hipStream_t st, const Affine* aff) {
    check_level(ctx, l);
    const uint32_t D = num_digits(ctx, l), E = l + ctx.K;
    uint64_t* d01 = (uint64_t*)ws_get(ctx, WS_D01, (size_t)B * 2 * l * W * 8);
    uint64_t* x2c = (uint64_t*)ws_get(ctx, WS_X2C, (size_t)B * l * W * 8);
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)B * D * E * W * 8);
    // d2 = a1 b1 is formed by the inverse NTT's first pass as it reads a1 and b1: it writes the product, in
    // evaluation form, straight into each digit's own limbs of the extension buffer and transforms it into x2c.  The
    // tensor kernel writes d0 and d1 only; with the rescale, only their limb l-1: the ModDown combine forms limbs
    // 0..l-2 from a and b (two limbs read per product instead of d0 and d1 written and read back) -- unless the
    // output overlaps an input, since the combine would then read a and b while writing.
    auto overlaps = [&](const uint64_t* x) {
        const uint64_t *xe = x + (size_t)B * 2 * l * W, *oe = out + (size_t)B * 2 * (l - (do_rescale ? 1 : 0)) * W;
        return out < xe && x < oe;
    };
    const bool from_inputs = do_rescale && !overlaps(a) && !overlaps(b);
    // with the fused two-pass combine, the digits' own limbs of d2 below l-1 are not stored either: the combine forms
    // them as a1 b1 from the inputs it reads for d0 and d1 (limb l-1's is read by the P part's inner product)
    const bool own = from_inputs && ctx.ntt_mode == NttMode::TwoPass && D <= 4;
    HIPX(launch_tensor(ctx, a, b, d01, nullptr, B, l, nullptr, 0, nullptr, st, from_inputs ? l - 1 : 0));
    std::vector<uint32_t> pm(l);
    for (uint32_t t = 0; t < l; t++) pm[t] = t;
    JobSpec js = regular_jobs(B, pm);
    js.src = a + (size_t)l * W;  // poly 1 of each ciphertext
    js.src2 = b + (size_t)l * W;
    js.src_period = 2 * l;
    js.copy = ext;
    js.copy_pstride = (uint64_t)D * E * W;
    js.copy_alpha = ctx.alpha;
    js.copy_E = E;
    js.copy_from = own ? l - 1 : 0;
    HIPX(launch_ntt(ctx, x2c, js, B * l, true, ctx.ntt_mode, st));
    if (from_inputs)
        relin_tail(ctx, d01, x2c, ext, B, l, evk, out, true, st, a, b, true, aff, own);
    else
        relin_tail(ctx, d01, x2c, ext, B, l, evk, out, do_rescale, st, nullptr, nullptr, true, aff);
}

// Device workspace of hmult with the rescale (bytes): d01 2Bl, d2 Bl, extension B D E, inner product 2B E,
// the addend's dropped limb 2B and the rescale's T 2B (l-1) limbs
size_t hmult_rescale_scratch_bytes(const Context& ctx, uint32_t B, uint32_t l) {
    const size_t D = num_digits(ctx, l), E = l + ctx.K;
    const size_t limbs = (size_t)B * (2 * l + l + D * E + 2 * E + 2 + 2 * (l - 1));
    return limbs * W * 8;
}

// hmult + rescale with every workspace buffer and per-call table in the device scratch: no device allocation.
// Same kernels, launches and words as hmult(..., true, ...).
void hmult_rescale_noalloc(Context& ctx, const uint64_t* a, const uint64_t* b, uint32_t B, uint32_t l,
                           const uint64_t* evk, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    if (l < 2) throw std::invalid_argument("rescale needs l >= 2");
    uint8_t* base = scratch_ptr(ctx.device);
    if (!base) throw std::runtime_error("device scratch not initialised for this context's device");
    const size_t need = hmult_rescale_scratch_bytes(ctx, B, l);
    if (need > kScratchBytes - kScratchTableBytes)
        throw std::invalid_argument("batch " + std::to_string(B) + " at level " + std::to_string(l) + " needs " +
                                    std::to_string(need >> 20) + " MiB of workspace; the allocation-free entry "
                                    "point has " + std::to_string((kScratchBytes - kScratchTableBytes) >> 20) +
                                    " MiB (use ckks_eval_mult_rescale, or a smaller batch)");
    Arena ar;
    ar.base = base;
    ar.cap = kScratchBytes;
    ar.st = st;
    struct Reset {
        Context& c;
        ~Reset() { c.arena = nullptr; }
    } reset{ctx};
    ctx.arena = &ar;
    hmult(ctx, a, b, B, l, evk, out, true, st);
}

// out[c] = relin( sum_j a[c][j] (x) b[c][j] ) (+ rescale): one key switch per batch item for np products.
// pairs: [B][np][2] ciphertext pointers, each [2][l][N].
void hmult_sum(Context& ctx, const uint64_t* const* pairs, uint32_t np, uint32_t B, uint32_t l, const uint64_t* evk,
               uint64_t* out, bool do_rescale, hipStream_t st) {
    check_level(ctx, l);
    if (np == 0 || np > 64) throw std::invalid_argument("1..64 products per item");
    const uint32_t D = num_digits(ctx, l), E = l + ctx.K;
    uint64_t* d01 = (uint64_t*)ws_get(ctx, WS_D01, (size_t)B * 2 * l * W * 8);
    uint64_t* x2c = (uint64_t*)ws_get(ctx, WS_X2C, (size_t)B * l * W * 8);
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)B * D * E * W * 8);
    const size_t tab_bytes = (size_t)B * np * 2 * sizeof(void*);
    std::vector<uint32_t> ext_off(l);
    for (uint32_t t = 0; t < l; t++) ext_off[t] = (t / ctx.alpha) * E + t;
    if (tab_bytes <= Context::kRingSlotBytes) {
        // staged through the pinned ring: the copy is asynchronous and the caller's array may go at once
        const uint32_t slot = ring_acquire(ctx);
        uint8_t* h = ctx.ring_host + (size_t)slot * Context::kRingSlotBytes;
        auto* d_tab = (const uint64_t**)(ctx.ring_dev + (size_t)slot * Context::kRingSlotBytes);
        std::memcpy(h, pairs, tab_bytes);
        HIPX(hipMemcpyAsync(d_tab, h, tab_bytes, hipMemcpyHostToDevice, st));
        HIPX(launch_tensor_sum(ctx, d_tab, np, d01, x2c, B, l, ext, (uint64_t)D * E * W, ext_off.data(), st));
        ring_release(ctx, slot, st);
    } else {
        auto* d_tab = (const uint64_t**)ws_get(ctx, WS_PTAB, tab_bytes);
        HIPX(hipMemcpyAsync(d_tab, pairs, tab_bytes, hipMemcpyHostToDevice, st));
        HIPX(launch_tensor_sum(ctx, d_tab, np, d01, x2c, B, l, ext, (uint64_t)D * E * W, ext_off.data(), st));
        // the pointer table must outlive the copy: the caller's array may be freed on return
        HIPX(hipStreamSynchronize(st));
    }
    relin_tail(ctx, d01, x2c, ext, B, l, evk, out, do_rescale, st);
}

// ------------------------------------------------------------------ rotation
// ct: [B][2][l][N] -> out [B][2][l][N]: KS of c1 under evk_g, add c0, then X -> X^g on both polys
void rotate(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, uint32_t g, const uint64_t* evk, uint64_t* out,
            hipStream_t st) {
    check_level(ctx, l);
    if ((g & 1) == 0 || g >= 2 * kN) throw std::invalid_argument("automorphism index must be odd and < 2N");
    // a key-switch list with one key and one index: the combine applies the automorphism as it stores
    const std::vector<uint32_t> gv(B, g);
    const std::vector<const uint64_t*> kv(B, evk);
    automorph_ks_list(ctx, ct, B, l, gv.data(), kv.data(), out, st);
}

uint32_t rotation_index(int64_t k) {
    const uint64_t M = 2ull * kN, ord = kN / 2;  // 5 has order N/2 in (Z/2N)^*
    int64_t e = k % (int64_t)ord;
    if (e < 0) e += (int64_t)ord;
    uint64_t r = 1, b = 5;
    for (uint64_t x = (uint64_t)e; x; x >>= 1) {
        if (x & 1) r = r * b % M;
        b = b * b % M;
    }
    return (uint32_t)r;
}

// out = ct + sum_j Rot_{steps[j]}(ct) for each of B ciphertexts [B][2][l][N] (a rotate-and-add window, e.g. a sum
// over a lane's slots): the n rotations share one ModUp of c1 and are summed in Q_l P -- sum_j Auto_j(<ext, evk_j> +
// (P c0, 0)) + P ct (k_qp_rot_sum) -- before a single ModDown, so a sum of n rotations costs one key switch's ModUp and
// ModDown plus n inner products.  The words differ from n separate rotations only in the key-switching rounding (one
// ModDown instead of n).
void rotate_sum(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, const int64_t* steps, uint32_t n,
                const uint64_t* const* evk, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    if (n == 0 || n > 64) throw std::invalid_argument("1..64 rotations per sum");
    if (B == 0) return;
    const uint32_t E = l + ctx.K, D = num_digits(ctx, l);
    const size_t ctw = (size_t)2 * l * W, exw = (size_t)D * E * W;
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)B * exw * 8);
    uint64_t* T = (uint64_t*)ws_get(ctx, WS_GROT, (size_t)B * 2 * E * W * 8);
    modup(ctx, ct + (size_t)l * W, ext, B, l, st, ctw);  // the c1 polys, read in place
    std::vector<uint32_t> g(n);
    for (uint32_t j = 0; j < n; j++) g[j] = rotation_index(steps[j]);
    for (uint32_t c = 0; c < B; c++)
        // one output, n terms all reading ciphertext c's extension and c0 (strides 0), its identity term P ct
        HIPX(launch_qp_rot_sum(ctx, ext + c * exw, 0, ct + c * ctw, 0, evk, g.data(), 1, n, 1, 0, l, T, st, 1, c, 0,
                               false, pmod_tab(ctx).data(), ct + c * ctw, 0));
    moddown_inplace(ctx, T, 2 * B, l, nullptr, out, st);
}

// n ciphertexts [n][2][l][N], each rotated by its own step with its own key -> out [n][2][l][N]
void rotate_list(Context& ctx, const uint64_t* cts, uint32_t n, uint32_t l, const int64_t* steps,
                 const uint64_t* const* evk, uint64_t* out, hipStream_t st) {
    std::vector<uint32_t> g(n);
    for (uint32_t c = 0; c < n; c++) g[c] = rotation_index(steps[c]);
    automorph_ks_list(ctx, cts, n, l, g.data(), evk, out, st);
}

// n ciphertexts, ciphertext c mapped by X -> X^g[c] with the key of g[c] (KS of c1, add c0, permute)
void automorph_ks_list(Context& ctx, const uint64_t* cts, uint32_t n, uint32_t l, const uint32_t* gidx,
                       const uint64_t* const* evk, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    if (n == 0) return;
    if (n > 64) {  // in chunks of 64 (the list kernels take 64 pointers)
        for (uint32_t c0 = 0; c0 < n; c0 += 64)
            automorph_ks_list(ctx, cts + (size_t)c0 * 2 * l * W, std::min(64u, n - c0), l, gidx + c0, evk + c0,
                              out + (size_t)c0 * 2 * l * W, st);
        return;
    }
    const uint32_t D = num_digits(ctx, l), E = l + ctx.K;
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)n * D * E * W * 8);
    modup(ctx, cts + (size_t)l * W, ext, n, l, st, (uint64_t)2 * l * W);  // the c1 polys, read in place
    std::vector<const uint64_t*> ep(n);
    for (uint32_t c = 0; c < n; c++) {
        ep[c] = ext + (size_t)c * D * E * W;
        if ((gidx[c] & 1) == 0 || gidx[c] >= 2 * kN) throw std::invalid_argument("automorphism index must be odd < 2N");
    }
    ks_moddown_list(ctx, ep.data(), evk, n, l, cts, (uint64_t)2 * l * W, 1, out, st, gidx);
}

// one ciphertext [2][l][N] rotated by n steps with one shared ModUp -> out [n][2][l][N]
void rotate_hoisted(Context& ctx, const uint64_t* ct, uint32_t l, const int64_t* steps, uint32_t n,
                    const uint64_t* const* evk, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    if (n == 0) return;
    const uint32_t E = l + ctx.K;
    const uint32_t D = num_digits(ctx, l);
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)D * E * W * 8);
    modup(ctx, ct + (size_t)l * W, ext, 1, l, st);
    rotate_hoisted_ext(ctx, ct, ext, l, steps, n, evk, out, st);
}

// the rotations of a hoisted set from its ModUp output ext ([D][E][N] of c1), in chunks of 64
void rotate_hoisted_ext(Context& ctx, const uint64_t* ct, const uint64_t* ext, uint32_t l, const int64_t* steps,
                        uint32_t n, const uint64_t* const* evk, uint64_t* out, hipStream_t st) {
    if (n > 64) {
        for (uint32_t c0 = 0; c0 < n; c0 += 64)
            rotate_hoisted_ext(ctx, ct, ext, l, steps + c0, std::min(64u, n - c0), evk + c0,
                               out + (size_t)c0 * 2 * l * W, st);
        return;
    }
    std::vector<const uint64_t*> ep(n, ext);
    std::vector<uint32_t> g(n);
    for (uint32_t c = 0; c < n; c++) g[c] = rotation_index(steps[c]);
    // c0 (the same for every rotation) is the ModDown addend of poly 0 of each output
    ks_moddown_list(ctx, ep.data(), evk, n, l, ct, 0, 1, out, st, g.data());
}

// n_ct ciphertexts [n_ct][2][l][N], each rotated by the same n steps over one ModUp of its own:
// out [n_ct][n][2][l][N].  The inner products of up to 64 (ciphertext, step) pairs run as one list.
void rotate_hoisted_multi(Context& ctx, const uint64_t* cts, uint32_t n_ct, uint32_t l, const int64_t* steps,
                          uint32_t n, const uint64_t* const* evk, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    if (n_ct == 0 || n == 0) return;
    const size_t ctw = (size_t)2 * l * W;
    if (n_ct == 1 || n > 64) {
        for (uint32_t c = 0; c < n_ct; c++) rotate_hoisted(ctx, cts + c * ctw, l, steps, n, evk, out + c * n * ctw, st);
        return;
    }
    const uint32_t E = l + ctx.K, D = num_digits(ctx, l);
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)n_ct * D * E * W * 8);
    modup(ctx, cts + (size_t)l * W, ext, n_ct, l, st, ctw);  // the c1 polys, read in place
    std::vector<uint32_t> g(n);
    for (uint32_t s = 0; s < n; s++) g[s] = rotation_index(steps[s]);
    const uint32_t per = 64 / n;  // ciphertexts per list (a list starts at a ciphertext boundary)
    for (uint32_t c0 = 0; c0 < n_ct; c0 += per) {
        const uint32_t nc = std::min(per, n_ct - c0), m = nc * n;
        std::vector<const uint64_t*> ep(m), kp(m);
        std::vector<uint32_t> gm(m);
        for (uint32_t j = 0; j < m; j++) {
            ep[j] = ext + (size_t)(c0 + j / n) * D * E * W;
            kp[j] = evk[j % n];
            gm[j] = g[j % n];
        }
        // c0 of ciphertext c is the addend of poly 0 of its n outputs
        ks_moddown_list(ctx, ep.data(), kp.data(), m, l, cts + (size_t)c0 * ctw, ctw, n, out + (size_t)c0 * n * ctw,
                        st, gm.data());
    }
}

void mul_plain(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, const uint64_t* pt, bool pt_shared,
               uint64_t* out, hipStream_t st, uint32_t log_rep) {
    check_level(ctx, l);
    HIPX(launch_mul_plain(ctx, ct, pt, out, B, l, pt_shared ? 0 : (uint64_t)l * (W >> log_rep), log_rep, st));
}

void add_plain(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, const uint64_t* pt, bool pt_shared,
               uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    HIPX(launch_add_plain(ctx, ct, pt, out, B, l, pt_shared ? 0 : (uint64_t)l * W, st));
}

// Baby-step giant-step diagonal matrix-vector product (gpu_real_model.cu:2767-2823):
// y = rescale( sum_g rot_{g*bs}( sum_j diag'_{g*bs+j} (.) rot_j(u) ) ), diagonals pre-rotated by -g*bs.
// Babies rot_1..rot_{bs-1} share one ModUp (hoisted).  The giant rotations share one ModDown: each rotating giant
// sum v_g's c1 is extended (one ModUp over all of them), and sum_g Auto_g(<ext_g, evk_g> + (P c0_g, 0)) + P v_0 is
// formed in Q_l P by one kernel (the key switches' inner products at the automorphisms' source words, the P
// scaling of the Q_l sums on the fly), then brought down and rescaled together: ng - 1 ModDowns fewer than rotating
// each giant on its own.  The words differ from the per-giant form's only by the key-switching rounding (one
// ModDown's instead of the sum of ng - 1).
void bsgs_matvec(Context& ctx, const uint64_t* ct, uint32_t l, const uint64_t* diags, uint32_t n_diag, uint32_t bs,
                 const uint64_t* const* baby_evk, const uint64_t* const* giant_evk, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    if (l < 2) throw std::invalid_argument("matvec consumes a level: needs l >= 2");
    if (bs == 0 || bs > 32) throw std::invalid_argument("baby steps must be in [1, 32]");
    const uint32_t ng = (n_diag + bs - 1) / bs;
    if (ng == 0 || ng > 65) throw std::invalid_argument("giant steps must be in [1, 65]");
    const size_t ctw = (size_t)2 * l * W;
    uint64_t* baby = (uint64_t*)ws_get(ctx, WS_BABY, (size_t)bs * ctw * 8);
    uint64_t* v = (uint64_t*)ws_get(ctx, WS_GIANT, (size_t)ng * ctw * 8);
    HIPX(hipMemcpyAsync(baby, ct, ctw * 8, hipMemcpyDeviceToDevice, st));
    if (bs > 1) {
        std::vector<int64_t> steps(bs - 1);
        for (uint32_t j = 1; j < bs; j++) steps[j - 1] = j;
        rotate_hoisted(ctx, ct, l, steps.data(), bs - 1, baby_evk, baby + ctw, st);
    }
    std::vector<const uint64_t*> bp(bs);
    for (uint32_t j = 0; j < bs; j++) bp[j] = baby + (size_t)j * ctw;
    HIPX(launch_bsgs_mac(ctx, bp.data(), diags, v, bs, n_diag, ng, l, 0, st));
    if (ng == 1) {
        rescale(ctx, v, 2, l, out, st);
        return;
    }
    const uint32_t ngr = ng - 1, E = l + ctx.K, D = num_digits(ctx, l);
    const size_t exw = (size_t)D * E * W;
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)ngr * exw * 8);
    uint64_t* T = (uint64_t*)ws_get(ctx, WS_GROT, (size_t)2 * E * W * 8);
    modup(ctx, v + ctw + (size_t)l * W, ext, ngr, l, st, ctw);  // the c1 halves of v_1 .. v_{ng-1}, read in place
    std::vector<const uint64_t*> keys(ngr);
    std::vector<uint32_t> g(ngr);
    for (uint32_t j = 0; j < ngr; j++) {
        keys[j] = giant_evk[j];
        g[j] = rotation_index((int64_t)(j + 1) * bs);
    }
    HIPX(launch_qp_rot_sum(ctx, ext, exw, v + ctw, ctw, keys.data(), g.data(), 1, ngr, 1, ngr, l, T, st, 1, 0, 0,
                           false, pmod_tab(ctx).data(), v, 0));
    moddown_rescale(ctx, T, 2, l, nullptr, out, st);
}

// General BSGS linear transform on one ciphertext [2][l][N]:
//   y = sum_g Rot_{G[g]}( sum_b diag[g*nb + b] (.) Rot_{Bs[b]}(x) )   (no rescale; out [2][l][N])
// A step of 0 is the identity (no key).  Baby rotations share one ModUp; giant rotations run as one batch.
// General BSGS with n_in inputs sharing the baby steps and n_out outputs sharing the babies, over n_inst
// independent instances that share the diagonals:
//   out_{s,o} = sum_g Rot_{G_g}( sum_{i, b} diag[o][g][i nb + b] (.) Rot_{B_b}(in_{s,i}) )   (+ rescale)
// Step 0 is the identity (no key).  diags: [n_out][ng][n_in nb][l][N >> log_rep], term (g, i, b) pre-rotated
// by -G_g.  in: [n_inst][n_in] pointers; out: [n_inst][n_out] (by_output: [n_out][n_inst]) ciphertexts.
// Each input's babies share one ModUp; all giant rotations of all outputs and instances run as one list.
void bsgs_multi_batch(Context& ctx, const uint64_t* const* in, uint32_t n_inst, uint32_t n_in, uint32_t l,
                      const uint64_t* diags, uint32_t nb, const int64_t* bsteps, const uint64_t* const* bevk,
                      uint32_t ng, const int64_t* gsteps, const uint64_t* const* gevk, uint32_t n_out,
                      bool do_rescale, uint64_t* out, hipStream_t st, uint32_t log_rep, bool by_output) {
    check_level(ctx, l);
    if (nb == 0 || n_in == 0 || n_out == 0 || ng == 0 || ng > 64 || n_inst == 0)
        throw std::invalid_argument("bad BSGS shape");
    if (do_rescale && l < 2) throw std::invalid_argument("rescale needs l >= 2");
    const size_t ctw = (size_t)2 * l * W;
    const uint32_t nbt = n_in * nb, n_x = n_inst * n_in;
    uint64_t* v = (uint64_t*)ws_get(ctx, WS_GIANT, (size_t)n_inst * n_out * ng * ctw * 8);
    // the inputs side by side (the hoisted rotations take one strided batch)
    uint64_t* X = (uint64_t*)ws_get(ctx, WS_BINP, (size_t)n_x * ctw * 8);
    HIPX(launch_gather(ctx, in, n_x, ctw, X, st));
    std::vector<int64_t> rs;
    std::vector<const uint64_t*> rk;
    std::vector<int32_t> ridx(nb, -1);  // baby b -> its rotation among rs, or -1 (identity: the input itself)
    for (uint32_t b = 0; b < nb; b++)
        if (bsteps[b] != 0) {
            ridx[b] = (int32_t)rs.size();
            rs.push_back(bsteps[b]);
            rk.push_back(bevk[b]);
        }
    const uint32_t nr = (uint32_t)rs.size();
    uint64_t* tmp = nullptr;
    if (nr) {
        tmp = (uint64_t*)ws_get(ctx, WS_SUM, (size_t)n_x * nr * ctw * 8);
        rotate_hoisted_multi(ctx, X, n_x, l, rs.data(), nr, rk.data(), tmp, st);
    }
    // babies [i nb + b] of instance s, read where they are (no packing copies)
    std::vector<const uint64_t*> bp(nbt);
    for (uint32_t s = 0; s < n_inst; s++) {
        for (uint32_t i = 0; i < n_in; i++)
            for (uint32_t b = 0; b < nb; b++) {
                const size_t x = (size_t)s * n_in + i;
                bp[i * nb + b] = ridx[b] < 0 ? X + x * ctw : tmp + (x * nr + (uint32_t)ridx[b]) * ctw;
            }
        HIPX(launch_bsgs_mac(ctx, bp.data(), diags, v + (size_t)s * n_out * ng * ctw, nbt, nbt * n_out * ng,
                             n_out * ng, l, log_rep, st));
    }
    // the giant rotations share one ModDown per output: the rotating giant sums of every instance and output, packed
    // contiguously, have their c1 extended (in chunks of outputs whose extensions fit a bounded buffer), and each
    // output's sum_g Auto_g(<ext_g, evk_g> + (P c0_g, 0)) + P v_{g0} is formed in Q_l P by one kernel, placed at the
    // output's slot; one ModDown (with the rescale) brings all outputs down
    const uint32_t n_o = n_inst * n_out;
    std::vector<const uint64_t*> gk;
    std::vector<uint32_t> gidx;
    int32_t g0 = -1;
    for (uint32_t g = 0; g < ng; g++) {
        if (gsteps[g] == 0) {
            if (g0 >= 0) throw std::invalid_argument("BSGS: at most one giant step 0");
            g0 = (int32_t)g;
            continue;
        }
        gk.push_back(gevk[g]);
        gidx.push_back(rotation_index(gsteps[g]));
    }
    const uint32_t ngr = (uint32_t)gk.size();
    const auto slot_of = [&](uint32_t c) {  // output c = s n_out + o -> its place in out
        return by_output ? (size_t)(c % n_out) * n_inst + c / n_out : (size_t)c;
    };
    if (ngr == 0) {  // the identity giant only: its sums are the outputs
        uint64_t* dst = do_rescale ? (uint64_t*)ws_get(ctx, WS_LIN, (size_t)n_o * ctw * 8) : out;
        for (uint32_t c = 0; c < n_o; c++) {
            const uint64_t* term = v + ((size_t)c * ng + (uint32_t)g0) * ctw;
            HIPX(launch_sum_list(ctx, &term, 1, dst + slot_of(c) * ctw, 2, l, st));
        }
        if (do_rescale) rescale(ctx, dst, 2 * n_o, l, out, st);
        return;
    }
    const uint32_t E = l + ctx.K, D = num_digits(ctx, l);
    const size_t exw = (size_t)D * E * W, cte = (size_t)2 * E * W;
    uint64_t* packed = (uint64_t*)ws_get(ctx, WS_SUM, (size_t)n_o * ngr * ctw * 8);
    {
        std::vector<const uint64_t*> src;
        src.reserve((size_t)n_o * ngr);
        for (uint32_t c = 0; c < n_o; c++)
            for (uint32_t g = 0; g < ng; g++)
                if ((int32_t)g != g0) src.push_back(v + ((size_t)c * ng + g) * ctw);
        HIPX(launch_gather(ctx, src.data(), (uint32_t)src.size(), ctw, packed, st));
    }
    uint64_t* T = (uint64_t*)ws_get(ctx, WS_GROT, (size_t)n_o * cte * 8);
    const uint32_t chunk = std::max<uint32_t>(1, 32 / ngr);
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)std::min(chunk, n_o) * ngr * exw * 8);
    const TwPair* pm = pmod_tab(ctx).data();
    for (uint32_t o0 = 0; o0 < n_o; o0 += chunk) {
        const uint32_t m = std::min(chunk, n_o - o0);
        const uint64_t* src = packed + (size_t)o0 * ngr * ctw;
        modup(ctx, src + (size_t)l * W, ext, m * ngr, l, st, ctw);
        const uint64_t* id = g0 >= 0 ? v + ((size_t)o0 * ng + (uint32_t)g0) * ctw : nullptr;
        if (by_output)
            HIPX(launch_qp_rot_sum(ctx, ext, exw, src, ctw, gk.data(), gidx.data(), m, ngr, 1, ngr, l, T, st, n_out, o0,
                                   (uint64_t)n_inst * cte, false, pm, id, (uint64_t)ng * ctw));
        else
            HIPX(launch_qp_rot_sum(ctx, ext, exw, src, ctw, gk.data(), gidx.data(), m, ngr, 1, ngr, l,
                                   T + (size_t)o0 * cte, st, 1, 0, 0, false, pm, id, (uint64_t)ng * ctw));
    }
    if (do_rescale)
        moddown_rescale(ctx, T, 2 * n_o, l, nullptr, out, st);
    else
        moddown_inplace(ctx, T, 2 * n_o, l, nullptr, out, st);
}

// Double-hoisted BSGS (the same transform as bsgs_multi_batch with do_rescale, over n_inst instances that share
// the diagonals; Bossuat, Mouchet, Troncoso-Pastoriza, Hubaux, EUROCRYPT 2021, the hoisted linear transform):
// the baby rotations stay in the extended basis Q_l * P (no ModDown: (P c0 + ks0, ks1) under Auto_b), the
// diagonals -- encoded over Q_l * P, diags [n_out][ng][n_in nb][l + K][N] -- multiply them there, each giant's
// inner sum is brought down once, rotated by the giant step again without its ModDown, and the giant sums are
// brought down and rescaled together: ng + 1 ModDowns per output instead of (nb - 1) + ng.
// out [n_inst][n_out][2][l-1][N] (by_output: [n_out][n_inst]).  The babies are formed inside the MAC kernel
// (k_bsgs_dh_mac: key switch and automorphism in LDS, never stored); the giants' key switches, automorphisms and
// sum run as one kernel (k_qp_rot_sum).  nb <= 32, n_in nb <= 64.
void bsgs_dh_batch(Context& ctx, const uint64_t* const* in, uint32_t n_inst, uint32_t n_in, uint32_t l,
                   const uint64_t* diags_qp, uint32_t nb, const int64_t* bsteps, const uint64_t* const* bevk,
                   uint32_t ng, const int64_t* gsteps, const uint64_t* const* gevk, uint32_t n_out, uint64_t* out,
                   hipStream_t st, bool by_output) {
    check_level(ctx, l);
    if (nb == 0 || nb > 32 || n_in * nb > 64 || n_in == 0 || n_out == 0 || ng == 0 || ng > 64 || n_inst == 0 ||
        l < 2)
        throw std::invalid_argument("bad BSGS shape");
    const uint32_t E = l + ctx.K, D = num_digits(ctx, l);
    const size_t ctw = (size_t)2 * l * W, cte = (size_t)2 * E * W, exw = (size_t)D * E * W;
    const uint32_t nbt = n_in * nb, n_x = n_inst * n_in, n_o = n_inst * n_out;
    // P R^-1 mod q_t (R = 2^64; the double-hoisted MAC keeps its babies R^-1-scaled)
    const std::vector<TwPair>& pmod = pmodr_tab(ctx);
    // the inputs side by side (read in place when they already are), their c1 extended once
    const uint64_t* X = in[0];
    for (uint32_t x = 1; x < n_x; x++)
        if (in[x] != in[0] + x * ctw) X = nullptr;
    if (!X) {
        uint64_t* Xg = (uint64_t*)ws_get(ctx, WS_BINP, (size_t)n_x * ctw * 8);
        HIPX(launch_gather(ctx, in, n_x, ctw, Xg, st));
        X = Xg;
    }
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT2, (size_t)n_x * exw * 8);
    modup(ctx, X + (size_t)l * W, ext, n_x, l, st, ctw);
    // giant sums T [n_o][2][E][N] in Q_l P (by_output: output o of instance s at slot o n_inst + s).  The MAC forms
    // the babies itself (never stored) and writes the inner sum of the identity giant step (if any) straight into T;
    // the other inner sums, S [n_inst][n_out][ngr][2][E][N], go down to Q_l once (the giant rotation needs c1 in
    // Q_l) and come back rotated in Q_l P, added to T.
    int32_t g0 = -1;
    std::vector<const uint64_t*> rk;
    std::vector<uint32_t> rg;
    for (uint32_t g = 0; g < ng; g++) {
        if (gsteps[g] == 0) {
            if (g0 >= 0) throw std::invalid_argument("double-hoisted BSGS: at most one giant step 0");
            g0 = (int32_t)g;
            continue;
        }
        rk.push_back(gevk[g]);
        rg.push_back(rotation_index(gsteps[g]));
    }
    const uint32_t ngr = (uint32_t)rk.size();
    uint64_t* T = (uint64_t*)ws_get(ctx, WS_GROT, (size_t)n_o * cte * 8);
    uint64_t* S = ngr ? (uint64_t*)ws_get(ctx, WS_GIANT, (size_t)n_o * ngr * cte * 8) : nullptr;
    {
        std::vector<uint32_t> g(nb);
        for (uint32_t b = 0; b < nb; b++) g[b] = bsteps[b] ? rotation_index(bsteps[b]) : 1;
        const uint64_t id_inst = by_output ? cte : (uint64_t)n_out * cte, id_o = by_output ? (uint64_t)n_inst * cte : cte;
        // baby steps b delta (delta > 0) let the MAC order its tiles along the rotation chains
        int64_t delta = nb > 1 ? bsteps[1] : 0;
        for (uint32_t b = 0; b < nb; b++)
            if (bsteps[b] != (int64_t)b * delta) delta = 0;
        if (delta < 0 || delta >= (int64_t)(kN / 2) || (delta & (delta - 1))) delta = 0;  // a power of two
        HIPX(launch_bsgs_dh_mac(ctx, ext, exw, X, ctw, bevk, g.data(), n_inst, n_in, nb, diags_qp, nbt * n_out * ng,
                                n_out, ng, g0, l, pmod.data(), S, T, id_inst, id_o, (uint32_t)delta, st));
    }
    if (ngr) {
        // only the c1 halves come down (the key switch needs c1 in Q_l); the c0 halves join the rotations in Q_l P as
        // they are: S0 = P SQ0 + [S0]_P, and the final ModDown divides that remainder by P
        uint64_t* SQ1 = (uint64_t*)ws_get(ctx, WS_SUM, (size_t)n_o * ngr * l * W * 8);
        moddown_inplace(ctx, S + (size_t)E * W, n_o * ngr, l, nullptr, SQ1, st, 1, -1, 0, 2 * E);
        // outputs in chunks whose extensions fit a bounded buffer
        const uint32_t chunk = std::max<uint32_t>(1, 32 / ngr);
        uint64_t* ext2 = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)std::min(chunk, n_o) * ngr * exw * 8);
        const bool acc = g0 >= 0;
        for (uint32_t o0 = 0; o0 < n_o; o0 += chunk) {
            const uint32_t m = std::min(chunk, n_o - o0);
            modup(ctx, SQ1 + (size_t)o0 * ngr * l * W, ext2, m * ngr, l, st);
            const uint64_t* src = S + (size_t)o0 * ngr * cte;
            if (by_output)
                HIPX(launch_qp_rot_sum(ctx, ext2, exw, src, cte, rk.data(), rg.data(), m, ngr, 1, ngr, l, T, st, n_out,
                                       o0, (uint64_t)n_inst * cte, acc));
            else
                HIPX(launch_qp_rot_sum(ctx, ext2, exw, src, cte, rk.data(), rg.data(), m, ngr, 1, ngr, l,
                                       T + (size_t)o0 * cte, st, 1, 0, 0, acc));
        }
    }
    // one ModDown for the giant sums, fused with the rescale
    moddown_rescale(ctx, T, 2 * n_o, l, nullptr, out, st);
}

void bsgs_multi(Context& ctx, const uint64_t* const* in, uint32_t n_in, uint32_t l, const uint64_t* diags,
                uint32_t nb, const int64_t* bsteps, const uint64_t* const* bevk, uint32_t ng, const int64_t* gsteps,
                const uint64_t* const* gevk, uint32_t n_out, bool do_rescale, uint64_t* out, hipStream_t st,
                uint32_t log_rep) {
    bsgs_multi_batch(ctx, in, 1, n_in, l, diags, nb, bsteps, bevk, ng, gsteps, gevk, n_out, do_rescale, out, st,
                     log_rep, false);
}

void bsgs_general(Context& ctx, const uint64_t* ct, uint32_t l, const uint64_t* diags, uint32_t nb,
                  const int64_t* bsteps, const uint64_t* const* bevk, uint32_t ng, const int64_t* gsteps,
                  const uint64_t* const* gevk, uint64_t* out, hipStream_t st, uint32_t log_rep) {
    bsgs_multi(ctx, &ct, 1, l, diags, nb, bsteps, bevk, ng, gsteps, gevk, 1, false, out, st, log_rep);
}

// Masked rotation pairs of one ciphertext (cyclic rotations inside blocks, assembled from two plain ones):
//   out[s][t] = rescale( pt[s][t][0] (.) Rot_{lo_t}(ct) + pt[s][t][1] (.) Rot_{hi_t}(ct) )
// all 2n rotations hoisted over one ModUp; pt [n_sets][n][2][l][N >> log_rep]; out [n_sets][n][2][l-1][N].
void rotate_masked(Context& ctx, const uint64_t* ct, uint32_t l, uint32_t n, const int64_t* lo,
                   const uint64_t* const* lo_evk, const int64_t* hi, const uint64_t* const* hi_evk, uint32_t n_sets,
                   const uint64_t* pts, uint32_t log_rep, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    if (l < 2 || n == 0 || n_sets == 0) throw std::invalid_argument("bad masked rotation shape");
    const size_t ctw = (size_t)2 * l * W;
    uint64_t* R = (uint64_t*)ws_get(ctx, WS_BABY, (size_t)2 * n * ctw * 8);
    std::vector<int64_t> steps(lo, lo + n);
    steps.insert(steps.end(), hi, hi + n);
    std::vector<const uint64_t*> keys(lo_evk, lo_evk + n);
    keys.insert(keys.end(), hi_evk, hi_evk + n);
    // a zero step is the identity (a copy); each run of non-zero steps rotates straight into place over one
    // shared ModUp of c1
    const uint32_t E = l + ctx.K, D = num_digits(ctx, l);
    uint64_t* ext = (uint64_t*)ws_get(ctx, WS_EXT, (size_t)D * E * W * 8);
    modup(ctx, ct + (size_t)l * W, ext, 1, l, st);
    for (uint32_t j = 0; j < 2 * n;) {
        if (steps[j] == 0) {
            HIPX(hipMemcpyAsync(R + j * ctw, ct, ctw * 8, hipMemcpyDeviceToDevice, st));
            j++;
            continue;
        }
        uint32_t e = j;
        while (e < 2 * n && steps[e] != 0) e++;
        rotate_hoisted_ext(ctx, ct, ext, l, steps.data() + j, e - j, keys.data() + j, R + j * ctw, st);
        j = e;
    }
    uint64_t* m = (uint64_t*)ws_get(ctx, WS_LIN, (size_t)n_sets * n * ctw * 8);
    HIPX(launch_pair_mac(ctx, R, pts, m, n_sets, n, l, log_rep, st));
    rescale(ctx, m, 2 * n_sets * n, l, out, st);
}

void mul_i(Context& ctx, const uint64_t* x, uint32_t n_polys, uint32_t l, int sign, uint64_t* out, hipStream_t st) {
    check_level(ctx, l);
    HIPX(launch_mul_i(ctx, x, out, n_polys, l, sign, st));
}

// Linear combination of ciphertext batches [B][2][l_t][N] (term t at level levels[t], scale scales_in[t]):
//  integer mode: sum_t round(c_t) x_t + round(a * scale_out) at level lt (every term at lt), no rescale;
//  scalar mode:  every term read at lt + 1 limbs, multiplied by round(c_t scale_out q_lt / scales_in[t]),
//                round(a scale_out) q_lt added, then rescaled to lt: the result has scale scale_out.
void lincomb(Context& ctx, uint32_t B, uint32_t n_terms, const uint64_t* const* x, const uint32_t* levels,
             const double* coeffs, const double* scales_in, double scale_out, double add_const, uint32_t lt,
             bool integer_mode, uint64_t* out, hipStream_t st) {
    if (n_terms == 0 || n_terms > 8) throw std::invalid_argument("1..8 terms");
    if (lt == 0 || lt > ctx.L) throw std::invalid_argument("target level out of range");
    const uint32_t lo = integer_mode ? lt : lt + 1;
    if (lo > ctx.L || lo > 40) throw std::invalid_argument("target level too high");
    for (uint32_t t = 0; t < n_terms; t++) {
        if (integer_mode ? levels[t] != lt : levels[t] < lo) throw std::invalid_argument("term level");
    }
    std::vector<uint64_t> C((size_t)n_terms * lo), add(lo);
    const long double qlt = (long double)ctx.moduli[integer_mode ? 0 : lt];
    for (uint32_t t = 0; t < n_terms; t++) {
        const long double c = integer_mode ? std::roundl((long double)coeffs[t])
                                           : std::roundl((long double)coeffs[t] * scale_out * qlt / scales_in[t]);
        for (uint32_t i = 0; i < lo; i++) C[(size_t)t * lo + i] = residue_of(c, ctx.moduli[i]);
    }
    const long double a = std::roundl((long double)add_const * scale_out);
    for (uint32_t i = 0; i < lo; i++) {
        const uint64_t qi = ctx.moduli[i];
        add[i] = integer_mode ? residue_of(a, qi) : mulmod_h(residue_of(a, qi), ctx.moduli[lt] % qi, qi);
    }
    std::vector<uint32_t> stride(levels, levels + n_terms);
    if (integer_mode) {
        HIPX(launch_lincomb(ctx, out, B, lo, n_terms, x, stride.data(), C.data(), add_const != 0.0 ? add.data() : nullptr,
                            st));
        return;
    }
    rescale_lincomb(ctx, B, lo, n_terms, x, stride.data(), C.data(), add_const != 0.0 ? add.data() : nullptr, out, st);
}

void add(Context& ctx, const uint64_t* x, const uint64_t* y, uint64_t* out, uint32_t n_polys, uint32_t l,
         hipStream_t st) {
    if (l == 0 || l > ctx.L) throw std::invalid_argument("level out of range");
    HIPX(launch_add(ctx, x, y, out, n_polys, l, st));
}

void automorph(Context& ctx, const uint64_t* in, uint64_t* out, uint32_t n_polys, uint32_t l, uint32_t g,
               hipStream_t st) {
    (void)ctx;
    if ((g & 1) == 0 || g >= 2 * kN) throw std::invalid_argument("automorphism index must be odd and < 2N");
    HIPX(launch_automorph(in, out, n_polys, l, g, st));
}

}  // namespace fhe
