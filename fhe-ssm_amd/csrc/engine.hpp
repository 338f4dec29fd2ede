// engine.hpp -- internal types of the MI355X RNS-CKKS engine (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <deque>
#include <map>
#include <string>
#include <vector>

namespace fhe {

constexpr uint32_t kLogN = 16;
constexpr uint32_t kN = 1u << kLogN;
constexpr uint32_t kMaxPrimes = 96;
constexpr uint32_t kMaxPmap = 96;

struct TwPair {
    uint64_t w, wp;  // twiddle and its Shoup companion floor(w * 2^64 / q)
};

struct PrimeInfo {
    uint64_t q;
    uint64_t ninv, ninv_p;      // N^-1 mod q and Shoup companion
    uint64_t w1ninv, w1ninv_p;  // inverse-table entry 1 (psi^-N/2) times N^-1: the last inverse stage
    uint64_t mu_hi, mu_lo;      // floor(2^128 / q)
    // quotient estimate of a value v < 128 q: hi32(floor(v / 2^red_shift) * red_mul) is floor(v / q) or one less,
    // with red_shift = max(0, bits(q) - 25), red_mul = floor(2^(32 + red_shift) / q)
    uint32_t red_shift, red_mul;
    uint64_t mont_ninv;  // -q^-1 mod 2^64 (Montgomery reduction of a 128-bit sum, R = 2^64)
    uint64_t r_mod, r_mod_p;  // R = 2^64 mod q and its Shoup companion (takes an R^-1-scaled value back to plain)
    // Q primes: P mod q (P the product of the special primes), and R P^-1 mod q with its Shoup companion (a ModDown
    // combine that reduces one 128-bit sum by REDC scales it by these); 0 for the special primes
    uint64_t pmod, rpinv, rpinv_p;
};

// One limb to transform: offset (in units of N words) from the base pointer, and its prime index.
struct Job {
    uint32_t off, prime;
};

// Either an explicit device job list, or a dense [n_polys][period][N] buffer whose limb l uses
// prime pmap[l] (enumerated prime-major).  Inverse transforms of a dense buffer may read their input from
// another buffer (src: limb l of poly p at src + (p * src_period + l) * N) and write the dense buffer: the
// copy that an in-place transform of someone else's data would need is folded into the first pass.
struct JobSpec {
    const Job* jobs;
    uint32_t n_polys, period;
    uint32_t n_primes;  // distinct primes among the jobs (host-side byte accounting only)
    const uint64_t* src;  // out-of-place input (dense specs, inverse only), or null
    uint32_t src_period;  // limbs between polys of src
    uint8_t pmap[kMaxPmap];
    // With src (two-pass mode only): src2, if set, makes the input the product src * src2 mod q, both factors read
    // at src's layout; copy, if set, receives the input (or that product) as read, before the transform: limb l of
    // poly p at copy + p * copy_pstride + ((l / copy_alpha) * copy_E + l) * N -- a ModUp extension buffer's
    // digit-own limbs.  Only limbs l >= copy_from are copied (0: all).
    const uint64_t* src2;
    uint64_t* copy;
    uint64_t copy_pstride;
    uint32_t copy_alpha, copy_E, copy_from;
    // Forward dense specs (two-pass mode only): lift, if set, is read in place of the buffer -- the input of limb l of
    // poly p is the centered lift of lift[p * lift_pstride + k] (a residue mod lift_q, above lift_q / 2 standing for
    // a negative value) into limb l's prime: a rescale's dropped limb spread over the kept ones.
    const uint64_t* lift;
    uint64_t lift_pstride, lift_q;
};

enum class NttMode { TwoPass = 0, Fused = 1 };

// Precomputed constants for one approximate CRT switch (BConv) from `n_in` source limbs to `n_out`
// target limbs: y_i = [x_i * qhat_inv_i]_{q_i};  out_j = sum_i y_i * qhat_mod[i][j] mod p_j.
struct BConvPlan {
    uint32_t n_in = 0, n_out = 0;
    bool centered = false;  // exact (centered) conversion: table also holds floor(2^128/q_i) and prod mod p_j
    // the output sums are reduced by Montgomery's REDC (R = 2^64) instead of Barrett: the table's qhat_mod (and
    // prod mod p_j) columns then hold their values times R mod p_j.  Taken when sum_i q_i + 16 < 2^64, which keeps
    // every sum below p_j R (REDC's input bound).
    bool mont = false;
    std::vector<uint32_t> in_idx, out_idx;  // prime indices
    uint64_t* d_tab = nullptr;  // [n_in] (qhat_inv, companion) pairs, then [n_in][n_out] qhat_mod split into 30-bit
                                // halves ((v >> 30) << 32 | v mod 2^30)
};

// Device memory lent to one call of the allocation-free entry point: the library's static scratch (scratch.hip).
// Workspace slots and the call's own device tables (NTT job lists, BConv constants not yet in the context's caches)
// are carved from it in request order; the tables are written into it by a kernel from its arguments (arena_put),
// on the call's stream.  Nothing is allocated on the device.
constexpr size_t kScratchBytes = (size_t)160 << 20;    // the scratch's size on each GPU
constexpr size_t kScratchTableBytes = (size_t)1 << 20;  // the part kept for the call's tables
constexpr uint32_t kArenaSlots = 32;

struct Arena {
    uint8_t* base = nullptr;
    size_t cap = 0, used = 0;
    hipStream_t st = nullptr;
    size_t slot_off[kArenaSlots] = {}, slot_bytes[kArenaSlots] = {};
    std::deque<BConvPlan> plans;  // the call's BConv plans whose tables live in the arena
};

// One profiled launch: HIP events recorded on the launch stream around the kernel, plus the
// algorithmic bytes that launch must move (inputs read once, outputs written once, shared tables once).
struct ProfRec {
    std::string name;
    double bytes;
    hipEvent_t e0, e1;
    std::string phase;  // the caller's phase label when the launch was issued (set_phase)
};

struct Context {
    int device = 0;
    uint32_t L = 0, K = 0, dnum = 0, alpha = 0;
    double scale = 0.0;
    std::vector<uint64_t> moduli;  // Q chain then P
    std::vector<uint64_t> psi;
    std::vector<PrimeInfo> primes;
    TwPair* d_tw = nullptr;   // [L+K][N] forward table (brev order)
    TwPair* d_itw = nullptr;  // [L+K][N] inverse table (brev order)
    // the NTT pass-B copies of d_tw / d_itw: the same pairs, the entries of pass B's strided stages (forward stages
    // 13..15, inverse stages with t = 1, 2, 4) stored per 256-word block as [k][lane] (see ntt.hip)
    TwPair* d_twb = nullptr;
    TwPair* d_itwb = nullptr;
    PrimeInfo* d_primes = nullptr;
    NttMode ntt_mode = NttMode::TwoPass;
    // cached device job lists keyed by a shape string (list, distinct primes in it)
    std::map<std::string, std::pair<Job*, uint32_t>> job_cache;
    std::map<std::string, BConvPlan> bconv_cache;
    // per-limb constants of the Q chain with their Shoup companions, computed on first use: P^-1 mod q_i,
    // P R^-1 mod q_i (R = 2^64), P mod q_i, and by j the row q_j^-1 mod q_i (i < j)
    std::vector<TwPair> tab_pinv, tab_pmodr, tab_pmod;
    std::map<uint32_t, std::vector<TwPair>> tab_qinv;
    // growable scratch
    std::vector<std::pair<void*, size_t>> scratch;
    // device tables [L+K][N'] of the small-ring NTTs used by periodic encoding, by ring size N'
    std::map<uint32_t, TwPair*> small_ntt;
    // free device buffers by size, reused across bootstrapping calls (a call needs tens of buffers of
    // B x 2 x L limbs; allocating them per call costs more than the smaller kernels it runs)
    std::map<size_t, std::vector<uint64_t*>> buf_pool;
    // ring of pinned host + device slots for per-call tables (pointer lists) copied asynchronously; a slot is
    // reused once the event recorded after the kernel that read it has completed
    static constexpr uint32_t kRingSlots = 16;
    static constexpr size_t kRingSlotBytes = 64 * 1024;
    uint8_t* ring_host = nullptr;
    uint8_t* ring_dev = nullptr;
    hipEvent_t ring_ev[kRingSlots] = {};
    bool ring_used[kRingSlots] = {};
    uint32_t ring_next = 0;
    // side streams for copies that overlap the work (created on first use, non-blocking, default priority): copies to
    // host memory on side_out, every other copy on side (so that a long run of copies out never delays a copy in);
    // the events of the copies issued on them, by ticket
    hipStream_t side = nullptr;
    hipStream_t side_out = nullptr;
    uint64_t side_next = 0;
    std::map<uint64_t, hipEvent_t> side_ev;
    std::vector<hipEvent_t> side_after;  // the events the side copies waited on
    // per-launch profiling (off by default)
    bool prof_on = false;
    mutable std::vector<ProfRec> prof;
    // phase attribution: the label every profiled launch records; with phase_marks, each change of label also
    // enqueues an empty marker kernel (k_phase_mark, phase_ids[label] + 1 workgroups) so that a kernel trace or a
    // counter pass can be split by phase
    std::string prof_phase;
    bool phase_marks = false;
    std::map<std::string, uint32_t> phase_ids;
    // key switches issued (evk inner products, one per ciphertext), always counted
    mutable uint64_t n_keyswitch = 0;
    // ModDown rounding: false = approximate P -> Q conversion (OpenFHE ApproxModDown, floor(x/P) - u with
    // u in [0, K)); true = exact round(x / P) (centered conversion)
    bool moddown_exact = false;
    // set only for the duration of an allocation-free call (workspace and new tables then come from it)
    Arena* arena = nullptr;
    // host copies of the BConv tables built during allocation-free calls (computed once, uploaded per call)
    std::map<std::string, std::vector<uint64_t>> bconv_host;
};

// Profiling helpers: no-ops unless ctx.prof_on.
int prof_begin(const Context& ctx, const char* name, double bytes, hipStream_t st);
// the phase label of the launches that follow (the marker kernel, if phase_marks, on st); returns the previous label
std::string set_phase(Context& ctx, const std::string& phase, hipStream_t st);
hipError_t launch_phase_mark(uint32_t id, hipStream_t st);
void prof_end(const Context& ctx, int idx, hipStream_t st);
void prof_clear(const Context& ctx);

// the scratch of the allocation-free entry point: its device address resolved once per device (with that device
// current), then looked up; arena_put writes host words into device memory by a kernel, without staging
hipError_t scratch_init(int device);
uint8_t* scratch_ptr(int device);
hipError_t arena_put(void* dst, const void* src, size_t bytes, hipStream_t st);

hipError_t launch_ntt(const Context& ctx, uint64_t* data, const JobSpec& js, uint32_t n_jobs, bool inverse,
                      NttMode mode, hipStream_t st);

}  // namespace fhe
