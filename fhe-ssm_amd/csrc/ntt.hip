// ntt.hip -- batched negacyclic NTT / INTT at N = 2^16 for gfx950.
//
// Semantics are OpenFHE's (restated in hpc_gpu_port/periodic_encode.hpp:240-260): forward is the
// Cooley-Tukey network over the table Table[brev(i)] = psi^i, natural order in, bit-reversed order
// out; inverse is the Gentleman-Sande network over the psi^-1 table, bit-reversed in, natural out,
// times N^-1.  The kernels run exactly that butterfly network, so the words they write are the
// words the CPU loop writes.
//
// Decomposition: N = 256 x 256.  The 16 stages split into two passes of 8:
//   pass A  (forward stages 0..7 / inverse stages 8..15): butterflies of stride >= 256.  Element j =
//           c + 256 r; for a fixed column c the 256 rows are an independent 8-stage problem whose
//           twiddles depend only on r.  A tile = 16 adjacent columns x 256 rows (32 KiB), so every
//           global access is a run of 16 consecutive words (128 B) per row.
//   pass B  (forward stages 8..15 / inverse 0..7): butterflies of stride < 256 inside each
//           contiguous 256-word block.  A tile = 16 blocks.
// Inside a tile each of 256 threads holds 16 words in registers and performs 4 stages (a radix-16
// step) between two LDS exchanges.  Values stay lazily reduced (Harvey): [0, 8q) forward, [0, 4q)
// inverse, with the twiddle product from shoup_lazy4; N^-1 is folded into the last inverse stage.  Forward
// transforms of primes below 2^56 skip the per-butterfly reduction altogether (fwd_bfly<true>: the bound grows by
// 4q a stage, to < 72q) and reduce once at the end with a quotient estimate (reduce_open).
//
// Launch layout: a "job" is one limb (offset in units of N words + prime index).  Jobs are
// enumerated prime-major so that concurrently running workgroups share one prime's twiddle table
// (1 MiB) in L2.  Either both passes run as separate kernels (grid 16 x jobs, 256 threads), or the
// fused kernel runs one limb per 512-thread workgroup (2 tiles at a time, passes separated by a
// workgroup barrier; the intermediate stays in L2/MALL instead of making a second HBM round trip).
//
// The key-switching steps around the transforms are folded into their first and last passes, so that the
// elementwise data they would store and reload never makes the round trip: an inverse first pass may form its input
// (a product of two limbs, an evk inner product) and copy it into a ModUp buffer; a forward first pass may lift a
// rescale's dropped limb; a forward last pass may end in a ModDown / rescale / key-switch combine (k_ntt_fwd_b_mdr,
// k_ntt_fwd_b_sub, k_ntt_fwd_b_ksl) instead of storing the transform.
#include <algorithm>
#include <set>
#include <type_traits>

#include "engine.hpp"
#include "ks_device.hpp"
#include "modarith.hpp"
#include "ntt_device.hpp"

namespace fhe {

namespace {

constexpr int kTileThreads = 256;
constexpr int kLdsWords = 16 * 272;  // one tile, padded to 17 words per 16 (both passes: no bank conflicts)

__device__ __forceinline__ void job_of(const JobSpec& js, uint32_t u, uint32_t& off, uint32_t& prime) {
    if (js.jobs) {
        const Job j = js.jobs[u];
        off = j.off;
        prime = j.prime;
    } else {
        // prime-major enumeration of a dense [polys][period][N] buffer.  The prime index is read as the aligned
        // 32-bit word holding it (a scalar load: the data loads need not wait for a vector byte load)
        const uint32_t l = uni_div(u, js.n_polys), p = u - l * js.n_polys;
        off = p * js.period + l;
        const uint32_t w = reinterpret_cast<const uint32_t*>(js.pmap)[l >> 2];
        prime = (w >> (8 * (l & 3))) & 0xFFu;
    }
}

// where job u reads its input: the buffer itself, or the out-of-place source of a dense spec
__device__ __forceinline__ const uint64_t* job_src(const JobSpec& js, uint32_t u, const uint64_t* data, uint32_t off) {
    if (js.src && !js.jobs) {
        const uint32_t l = uni_div(u, js.n_polys), p = u - l * js.n_polys;
        return js.src + ((size_t)p * js.src_period + l) * kN;
    }
    return data + (size_t)off * kN;
}

// a dense spec's second input factor and the copy destination of its input, for job u (null when unused)
struct JobIn {
    const uint64_t* in2;
    uint64_t* cpy;
};

__device__ __forceinline__ JobIn job_in(const JobSpec& js, uint32_t u) {
    JobIn r{nullptr, nullptr};
    const uint32_t l = uni_div(u, js.n_polys), p = u - l * js.n_polys;
    if (js.src2) r.in2 = js.src2 + ((size_t)p * js.src_period + l) * kN;
    if (js.copy && l >= js.copy_from)
        r.cpy = js.copy + p * js.copy_pstride + ((size_t)(l / js.copy_alpha) * js.copy_E + l) * kN;
    return r;
}

// Inverse (Gentleman-Sande) butterfly, values kept in [0, 4q).
__device__ __forceinline__ void gs_bfly(uint64_t& X, uint64_t& Y, const TwPair& w, uint64_t q4, uint64_t nq) {
    const uint64_t s = csub_s(X + Y, q4);
    const uint64_t d = X + q4 - Y;
    X = s;
    Y = shoup_lazy4(d, w.w, w.wp, nq);
}

// Inverse butterflies for primes below 2^55, the sum left unreduced.  A radix-16 group is 4 GS stages over a
// thread's 16 values, stage s pairing k and k + 2^s.  Before stage s every value below E q has a bound that depends
// on k's low s bits only: 4 q if bit s-1 is set (it was a stage's Shoup product), else twice its bound before stage
// s-1 (it was a sum of two values of the same bound).  Entered below 32 q, the group leaves value 0 below 512 q
// (< 2^64 with q < 2^55: no sum wraps) and every other value below 32 q; value 0 alone is brought back below 32 q
// with four conditional subtracts, so every group (and both passes) can be entered below 32 q.  The difference
// X - Y is lifted by Y's bound, X + c_Y - Y, a multiple of q; the Shoup product takes any 64-bit input.
constexpr uint64_t kGsOpenMaxQ = 1ull << 55;

struct GsBounds {
    uint8_t lg[5][16];  // log2 of the bound (units of q) of value k before stage s (s = 4: after the group)
};
constexpr GsBounds make_gs_bounds() {
    GsBounds g{};
    uint32_t b[16] = {};
    for (int k = 0; k < 16; k++) b[k] = 32;
    for (int s = 0; s <= 4; s++) {
        for (int k = 0; k < 16; k++) {
            uint8_t l = 0;
            while ((1u << l) < b[k]) l++;
            g.lg[s][k] = l;
        }
        if (s == 4) break;
        for (int k = 0; k < 16; k++)
            if (!(k & (1 << s))) {
                b[k] += b[k + (1 << s)];
                b[k + (1 << s)] = 4;
            }
    }
    return g;
}
constexpr GsBounds kGs = make_gs_bounds();
constexpr bool gs_bounds_ok() {
    // value 0 leaves a group below 512 q, every other value below 32 q; no stage's X + Y reaches 512 q
    for (int k = 1; k < 16; k++)
        if (kGs.lg[4][k] > 5) return false;
    for (int s = 0; s < 4; s++)
        for (int k = 0; k < 16; k++)
            if (!(k & (1 << s)) && (1u << kGs.lg[s][k]) + (1u << kGs.lg[s][k + (1 << s)]) > 512) return false;
    return kGs.lg[4][0] == 9;
}
static_assert(gs_bounds_ok(), "GS group bounds");

// stage s of a group on the pair (X = value k, Y = value k + 2^s)
template <bool kOpen>
__device__ __forceinline__ void gs_step(uint64_t& X, uint64_t& Y, const TwPair& w, uint64_t q, int s, int k,
                                        uint64_t q4, uint64_t nq) {
    if (kOpen) {
        const uint64_t d = X + (q << kGs.lg[s][k + (1 << s)]) - Y;
        X = X + Y;
        Y = shoup_lazy4(d, w.w, w.wp, nq);
    } else {
        gs_bfly(X, Y, w, q4, nq);
    }
}

// end of an open group: value 0 from below 512 q to below 32 q
template <bool kOpen>
__device__ __forceinline__ void gs_group_end(uint64_t* x, uint64_t q) {
    if (kOpen) {
        x[0] = csub_s(x[0], q << 8);
        x[0] = csub_s(x[0], q << 7);
        x[0] = csub_s(x[0], q << 6);
        x[0] = csub_s(x[0], q << 5);
    }
}

// ---------------------------------------------------------------- forward pass A (strided columns)
// tile: columns [16*tile, 16*tile + 16).  g: thread id within the 256-thread group.
// lift (optional): the words are read from there and lifted (centered, from residues mod lq) into this prime
template <bool kOpen, bool kLift = false>
__device__ __forceinline__ void fwd_a_tile(uint64_t* __restrict__ a, const TwPair* __restrict__ tw, uint64_t q,
                                           int tile, int g, uint64_t* lds, const uint64_t* lift = nullptr,
                                           uint64_t lq = 0, const Barrett br = Barrett{}) {
    const uint64_t q4 = q << 2, nq = 0 - q;
    const int cl = g & 15, rg = g >> 4;
    const int col = tile * 16 + cl;
    uint64_t x[16];
    if (kLift) {
#pragma unroll
        for (int k = 0; k < 16; k++) x[k] = __builtin_nontemporal_load(&lift[col + 256 * (rg + 16 * k)]);
        if (lq <= 2 * q) {
            // v > lq/2 stands for v - lq = v + dl (mod q), dl = -lq mod q: the sum is below 3q, a valid input (this
            // pass takes words below 8q), so no reduction
            const uint64_t lm = lq >= q ? lq - q : lq, dl = lm ? q - lm : 0;
#pragma unroll
            for (int k = 0; k < 16; k++) x[k] += x[k] > (lq >> 1) ? dl : 0;
        } else {
#pragma unroll
            for (int k = 0; k < 16; k++) x[k] = lift_centered(x[k], lq, br);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) x[k] = __builtin_nontemporal_load(&a[col + 256 * (rg + 16 * k)]);
    }
    // stages 0..3: rows r = rg + 16k, pairs differ in bit (3-s) of k; twiddle (1<<s) + (k >> (4-s))
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int h = 8 >> s;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            fwd_bfly<kOpen>(x[k], x[k + h], tw[(1 << s) + (k >> (4 - s))], q4, nq);
        }
    }
#pragma unroll
    for (int k = 0; k < 16; k++) lds[(rg + 16 * k) * 17 + cl] = x[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = lds[(16 * rg + k) * 17 + cl];
    // stages 4..7: rows r = 16 rg + k, pairs differ in bit (7-s) of r; twiddle (1<<s) + (r >> (8-s))
#pragma unroll
    for (int s = 4; s < 8; s++) {
        const int h = 128 >> s;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            fwd_bfly<kOpen>(x[k], x[k + h], tw[(1 << s) + ((16 * rg + k) >> (8 - s))], q4, nq);
        }
    }
#pragma unroll
    for (int k = 0; k < 16; k++) __builtin_nontemporal_store(x[k], &a[col + 256 * (16 * rg + k)]);
}

// ---------------------------------------------------------------- forward pass B (256-word blocks)
// Epi: what becomes of the transformed tile, held transposed in LDS (word rl + 16 k of block b at L[rl + 17 k]) --
// StoreLimb (the default): stored over the limb; otherwise first = epi.begin(b, rl) before the final reduction and
// exchange (loads that do not depend on the tile), then epi.end(first, L, b, rl).
struct StoreLimb {
    struct First {};
};

template <bool kOpen, class Epi = StoreLimb>
__device__ __forceinline__ void fwd_b_tile(uint64_t* __restrict__ a, const TwPair* __restrict__ tw, const PrimeInfo& P,
                                           int tile, int g, uint64_t* lds, const Epi& epi = Epi{}) {
    const uint64_t q = P.q;
    const uint64_t q4 = q << 2, nq = 0 - q;
    const int bl = g >> 4, rl = g & 15;
    const int b = tile * 16 + bl;  // block index within the limb
    uint64_t* blk = a + 256 * b;
    uint64_t* L = lds + bl * 272;
    uint64_t x[16];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = __builtin_nontemporal_load(&blk[rl + 16 * k]);
    // stages 8+s, s = 0..3: r = rl + 16k; twiddle 2^(8+s) + b 2^s + (k >> (4-s)), which pass B's table stores at
    // 2^(8+s) + (k >> (4-s)) 256 + b (the four blocks of a wave read adjacent pairs).  All 15 are requested with the
    // data (left to the compiler, each stage's loads were issued just before its butterflies, one exposed L2 round
    // trip per stage); their registers are free again for the later stages' twiddles below.
    TwPair tw03[15];
#pragma unroll
    for (int s = 0, n = 0; s < 4; s++)
#pragma unroll
        for (int j = 0; j < (1 << s); j++, n++) tw03[n] = tw[(256 << s) + (j << 8) + b];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int h = 8 >> s;
        const int base = (1 << s) - 1;  // stage s's first entry in tw03
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            fwd_bfly<kOpen>(x[k], x[k + h], tw03[base + (k >> (4 - s))], q4, nq);
        }
    }
    // stages 8+s, s = 4..7: r = 16 rl + k; twiddle 2^(8+s) + b 2^s + (r >> (8-s)) = ... + rl 2^(s-4) + (k >> (8-s)).
    // Pass B's table (twb) stores each block's 2^s entries of these stages as [k >> (8-s)][rl], so the 16 lanes of a
    // block read 16 consecutive pairs per load instead of 16 pairs 2^(s-4) apart (one cache line per lane).
    // A thread uses 2^(s-4) of them per stage.  Stages 4..6 (7 pairs) are loaded before the LDS exchange and stage 7
    // (8 pairs) right after it, so their latency overlaps the exchange and the earlier stages (the LDS tile already
    // limits the kernel to 4 waves per SIMD, which leaves room for the registers).
    TwPair tw4[7], tw7[8];
#pragma unroll
    for (int s = 4, n = 0; s < 7; s++)
#pragma unroll
        for (int i = 0; i < (1 << (s - 4)); i++, n++) tw4[n] = tw[(256 << s) + (b << s) + (i << 4) + rl];
    // LDS word index of r: r + (r >> 4)
#pragma unroll
    for (int k = 0; k < 16; k++) L[rl + 17 * k] = x[k];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) tw7[i] = tw[(256 << 7) + (b << 7) + (i << 4) + rl];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = L[17 * rl + k];
#pragma unroll
    for (int s = 4; s < 8; s++) {
        const int h = 128 >> s;
        const int base = (1 << (s - 4)) - 1;  // stage s's first entry in tw4
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            const int i = k >> (8 - s);
            fwd_bfly<kOpen>(x[k], x[k + h], s < 7 ? tw4[base + i] : tw7[i], q4, nq);
        }
    }
    // canonical [0, q), then transpose through LDS for coalesced stores (direct 16-byte stores of each
    // thread's contiguous run measured slower)
    // (an epilogue's first loads are issued here, ahead of the reduction and the exchange)
    typename Epi::First first{};
    if constexpr (!std::is_same<Epi, StoreLimb>::value) first = epi.begin(b, rl);
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = kOpen ? reduce_open(x[k], q, nq, P.red_shift, P.red_mul) : canon8(x[k], q);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) L[17 * rl + k] = x[k];
    __syncthreads();
    if constexpr (std::is_same<Epi, StoreLimb>::value) {
#pragma unroll
        for (int k = 0; k < 16; k++) __builtin_nontemporal_store(L[rl + 17 * k], &blk[rl + 16 * k]);
    } else {
        epi.end(first, L, b, rl);
    }
}

// ---------------------------------------------------------------- inverse pass B (256-word blocks)
// GS stages with t = 2^u, u = 0..7: m = 2^(15-u), twiddle m + (j >> (u+1)), j = 256 b + r.
// in: the limb read (a itself, or the out-of-place source).  kProd: the input is in * in2 mod q (q < 2^60, both
// factors canonical, so the product's high word is below q).  ji.cpy (optional): the input words, as read or formed,
// are also stored there.
// kD > 0: the input is the evk inner product sum_d in[d xs] * ks.e[d es] of a key switch (KsIn), kD digits.
struct KsIn {
    const uint64_t* e;  // the job's evk limb of digit 0 (digit d at e + d es)
    size_t xs, es;      // digit strides of the extension (in) and of the key, in words
};

template <bool kOpen, bool kProd, int kD = 0>
__device__ __forceinline__ void inv_b_tile(uint64_t* a, const uint64_t* in, JobIn ji, const PrimeInfo& P,
                                           const TwPair* __restrict__ tw, int tile, int g, uint64_t* lds,
                                           const KsIn ks = KsIn{}) {
    const uint64_t q = P.q;
    const uint64_t q4 = q << 2, nq = 0 - q;
    const int bl = g >> 4, rl = g & 15;
    const int b = tile * 16 + bl;
    uint64_t* blk = a + 256 * b;
    const uint64_t* src = in + 256 * b;
    uint64_t* L = lds + bl * 272;
    uint64_t x[16];
    if constexpr (kD > 0) {
        // two words at a time, all their digit loads issued before the products (sums of kD <= 4 products of
        // residues below q < 2^60: the high word stays below q)
        const Barrett br{q, P.mu_hi, P.mu_lo};
        const uint64_t* e = ks.e + 256 * b;
#pragma unroll
        for (int k0 = 0; k0 < 16; k0 += 2) {
            uint64_t xv[2][kD], ev[2][kD];
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int d = 0; d < kD; d++) {
                    xv[j][d] = src[d * ks.xs + rl + 16 * (k0 + j)];
                    ev[j][d] = e[d * ks.es + rl + 16 * (k0 + j)];
                }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                Acc s;
#pragma unroll
                for (int d = 0; d < kD; d++) s.add(xv[j][d], ev[j][d]);
                const U128 v = s.get();
                L[rl + 17 * (k0 + j)] = reduce128(v.hi, v.lo, br);
            }
        }
    } else if (kProd || ji.cpy) {
#pragma unroll
        for (int k = 0; k < 16; k++) x[k] = __builtin_nontemporal_load(&src[rl + 16 * k]);
        if (kProd) {
            const uint64_t* src2 = ji.in2 + 256 * b;
            const Barrett br{q, P.mu_hi, P.mu_lo};
#pragma unroll
            for (int k = 0; k < 16; k++) {
                Acc s;
                s.add(x[k], __builtin_nontemporal_load(&src2[rl + 16 * k]));
                const U128 v = s.get();
                x[k] = reduce128(v.hi, v.lo, br);
            }
        }
        if (ji.cpy) {
#pragma unroll
            for (int k = 0; k < 16; k++) __builtin_nontemporal_store(x[k], &ji.cpy[256 * b + rl + 16 * k]);
        }
#pragma unroll
        for (int k = 0; k < 16; k++) L[rl + 17 * k] = x[k];
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) L[rl + 17 * k] = __builtin_nontemporal_load(&src[rl + 16 * k]);
    }
    // u = 0..3: r = 16 rl + k, pairs differ in bit u of k; twiddle ... + (r >> (u+1)) = ... + rl 2^(3-u) + (k >> (u+1)),
    // stored by pass B's table (twb) as [k >> (u+1)][rl] within each block (consecutive pairs for a block's lanes).
    // A thread uses 2^(3-u) of them per stage; all 15 are loaded before the LDS exchange so that their latency
    // overlaps it (the LDS tile limits the kernel to 4 waves per SIMD; the registers are free)
    TwPair tw01[15];
#pragma unroll
    for (int u = 0, n = 0; u < 4; u++)
#pragma unroll
        for (int i = 0; i < (8 >> u); i++, n++) tw01[n] = tw[(32768 >> u) + (b << (7 - u)) + (i << 4) + rl];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = L[17 * rl + k];
    // u = 4..7 (after the second exchange): r = rl + 16k, pairs differ in bit (u-4) of k; r >> (u+1) = k >> (u-3);
    // pass B's table stores twiddle 2^(15-u) + b 2^(7-u) + j at 2^(15-u) + j 256 + b (the four blocks of a wave read
    // adjacent pairs).  All 15 are loaded once u = 0, 1 have freed their registers.
    TwPair tw45[15];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int h = 1 << u;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            const int i = k >> (u + 1);
            gs_step<kOpen>(x[k], x[k + h], tw01[16 - (16 >> u) + i], q, u, k, q4, nq);
        }
        if (u == 1) {
#pragma unroll
            for (int v = 4, n = 0; v < 8; v++)
#pragma unroll
                for (int j = 0; j < (8 >> (v - 4)); j++, n++) tw45[n] = tw[(32768 >> v) + b + (j << 8)];
        }
    }
    gs_group_end<kOpen>(x, q);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) L[17 * rl + k] = x[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = L[rl + 17 * k];
#pragma unroll
    for (int u = 4; u < 8; u++) {
        const int h = 1 << (u - 4);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            const int j = k >> (u - 3);
            gs_step<kOpen>(x[k], x[k + h], tw45[16 - (16 >> (u - 4)) + j], q, u - 4, k, q4, nq);
        }
    }
    gs_group_end<kOpen>(x, q);  // the intermediate is stored below 32 q (below 4 q when not open)
#pragma unroll
    for (int k = 0; k < 16; k++) __builtin_nontemporal_store(x[k], &blk[rl + 16 * k]);
}

// ---------------------------------------------------------------- inverse pass A (strided columns)
// GS stages with t = 2^(8+u), u = 0..7: m = 2^(7-u), twiddle m + (r >> (u+1)); then * N^-1.
template <bool kOpen>
__device__ __forceinline__ void inv_a_tile(uint64_t* __restrict__ a, const TwPair* __restrict__ tw, uint64_t q,
                                           TwPair ninv, TwPair w1ninv, int tile, int g, uint64_t* lds) {
    const uint64_t q4 = q << 2, nq = 0 - q;
    const int cl = g & 15, rg = g >> 4;
    const int col = tile * 16 + cl;
    uint64_t x[16];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = __builtin_nontemporal_load(&a[col + 256 * (16 * rg + k)]);
    // u = 0..3: r = 16 rg + k, pairs differ in bit u of k; twiddle (128 >> u) + rg 2^(3-u) + (k >> (u+1)).  Those of
    // u = 0, 1 (12 pairs) are requested with the data, not just before their butterflies
    TwPair twa[12];
#pragma unroll
    for (int u = 0, n = 0; u < 2; u++)
#pragma unroll
        for (int i = 0; i < (8 >> u); i++, n++) twa[n] = tw[(128 >> u) + (rg << (3 - u)) + i];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int h = 1 << u;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            const int i = k >> (u + 1);
            gs_step<kOpen>(x[k], x[k + h], u < 2 ? twa[(u ? 8 : 0) + i] : tw[(128 >> u) + (rg << (3 - u)) + i], q, u,
                           k, q4, nq);
        }
    }
    gs_group_end<kOpen>(x, q);
#pragma unroll
    for (int k = 0; k < 16; k++) lds[(16 * rg + k) * 17 + cl] = x[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = lds[(rg + 16 * k) * 17 + cl];
    // u = 4..6: r = rg + 16k, pairs differ in bit (u-4) of k; r >> (u+1) = k >> (u-3)
#pragma unroll
    for (int u = 4; u < 7; u++) {
        const int h = 1 << (u - 4);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k & h) continue;
            gs_step<kOpen>(x[k], x[k + h], tw[(128 >> u) + (k >> (u - 3))], q, u - 4, k, q4, nq);
        }
    }
    // u = 7 (m = 1, stride N/2) with N^-1 folded in: X' = (X + Y) N^-1, Y' = (X - Y) w_1 N^-1.  Open: the three
    // stages above leave value k + 8 below 2^lg[3][k+8] q and X + Y below 512 q.
    // X' without a multiply by N^-1: q = 1 + c 2^16 (q = 1 mod 2N), so N^-1 = q - c and, with v = a 2^16 + b (b < 2^16),
    // v N^-1 = -v c = -a (q - 1) - b c = a - b c (mod q).  a + q - b c lies in (a, a + q] with b c < q and
    // a = v / 2^16 < q / 128, so below 2q: one conditional subtract to [0, q), where the Shoup product by N^-1 took
    // twelve instructions and left [0, 4q).
    const uint64_t cn = q - ninv.w;  // c = (q - 1) / 2^16
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint64_t X = x[k], Y = x[k + 8];
        const uint64_t v = X + Y;
        x[k] = (v >> 16) + q - (uint64_t)((uint32_t)v & 0xFFFFu) * cn;
        x[k + 8] = shoup_lazy4(X + (kOpen ? q << kGs.lg[3][k + 8] : q4) - Y, w1ninv.w, w1ninv.wp, nq);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) __builtin_nontemporal_store(csub_s(x[k], q), &a[col + 256 * (rg + 16 * k)]);
#pragma unroll
    for (int k = 8; k < 16; k++) {
        const uint64_t v = csub_s(x[k], q << 1);
        __builtin_nontemporal_store(csub_s(v, q), &a[col + 256 * (rg + 16 * k)]);
    }
}

// ---------------------------------------------------------------- kernels
__global__ __launch_bounds__(kTileThreads) void k_ntt_fwd_a(uint64_t* data, JobSpec js, const TwPair* tw_all,
                                                           const PrimeInfo* primes) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const uint64_t q = primes[prime].q;
    uint64_t* a = data + (size_t)off * kN;
    const TwPair* tw = tw_all + (size_t)prime * kN;
    if (js.lift && !js.jobs) {
        const uint32_t p = blockIdx.y - uni_div(blockIdx.y, js.n_polys) * js.n_polys;
        const uint64_t* src = js.lift + p * js.lift_pstride;
        if (q < kOpenMaxQ)
            fwd_a_tile<true, true>(a, tw, q, blockIdx.x, threadIdx.x, lds, src, js.lift_q, barrett_of(primes[prime]));
        else
            fwd_a_tile<false, true>(a, tw, q, blockIdx.x, threadIdx.x, lds, src, js.lift_q, barrett_of(primes[prime]));
    } else if (q < kOpenMaxQ) {
        fwd_a_tile<true>(a, tw, q, blockIdx.x, threadIdx.x, lds);
    } else {
        fwd_a_tile<false>(a, tw, q, blockIdx.x, threadIdx.x, lds);
    }
}

__global__ __launch_bounds__(kTileThreads) void k_ntt_fwd_b(uint64_t* data, JobSpec js, const TwPair* tw_all,
                                                           const PrimeInfo* primes) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const PrimeInfo& P = primes[prime];
    if (P.q < kOpenMaxQ)
        fwd_b_tile<true>(data + (size_t)off * kN, tw_all + (size_t)prime * kN, P, blockIdx.x, threadIdx.x, lds);
    else
        fwd_b_tile<false>(data + (size_t)off * kN, tw_all + (size_t)prime * kN, P, blockIdx.x, threadIdx.x, lds);
}

__global__ __launch_bounds__(kTileThreads) void k_ntt_inv_b(uint64_t* data, JobSpec js, const TwPair* tw_all,
                                                           const PrimeInfo* primes) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const PrimeInfo& P = primes[prime];
    uint64_t* a = data + (size_t)off * kN;
    const uint64_t* in = job_src(js, blockIdx.y, data, off);
    const TwPair* tw = tw_all + (size_t)prime * kN;
    const JobIn ji = js.jobs ? JobIn{nullptr, nullptr} : job_in(js, blockIdx.y);
    if (ji.in2) {
        if (P.q < kGsOpenMaxQ)
            inv_b_tile<true, true>(a, in, ji, P, tw, blockIdx.x, threadIdx.x, lds);
        else
            inv_b_tile<false, true>(a, in, ji, P, tw, blockIdx.x, threadIdx.x, lds);
    } else if (P.q < kGsOpenMaxQ) {
        inv_b_tile<true, false>(a, in, ji, P, tw, blockIdx.x, threadIdx.x, lds);
    } else {
        inv_b_tile<false, false>(a, in, ji, P, tw, blockIdx.x, threadIdx.x, lds);
    }
}

// The first inverse pass over a job list of ModDown limbs (off = pc E + t of an accumulator [n_polys][E][N]) whose
// input is the evk inner product of a key switch of ciphertext pc / 2, poly pc % 2, formed here from the extension
// [B][kD][E][N] and the key [dnum][2][T][N] (in place of a separate inner-product launch and its stores).
struct KsJobArgs {
    const uint64_t* ext;
    const uint64_t* evk;
    uint32_t E, T;
};

template <int kD>
__global__ __launch_bounds__(kTileThreads) void k_ntt_inv_b_ks(uint64_t* data, JobSpec js, const TwPair* tw_all,
                                                              const PrimeInfo* primes, KsJobArgs ka) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const uint32_t pc = off / ka.E, t = off - pc * ka.E, c = pc >> 1, p = pc & 1;
    const PrimeInfo& P = primes[prime];
    const uint64_t* xin = ka.ext + ((size_t)c * kD * ka.E + t) * kN;
    const KsIn ks{ka.evk + ((size_t)p * ka.T + prime) * kN, (size_t)ka.E * kN, 2 * (size_t)ka.T * kN};
    uint64_t* a = data + (size_t)off * kN;
    const TwPair* tw = tw_all + (size_t)prime * kN;
    const JobIn none{nullptr, nullptr};
    if (P.q < kGsOpenMaxQ)
        inv_b_tile<true, false, kD>(a, xin, none, P, tw, blockIdx.x, threadIdx.x, lds, ks);
    else
        inv_b_tile<false, false, kD>(a, xin, none, P, tw, blockIdx.x, threadIdx.x, lds, ks);
}

// k_ntt_inv_b_ks over a key-switch list: item c = pc / 2 has its own extension [kD][E][N] and key
struct KslJobArgs {
    ListPtrs ext, evk;
    uint32_t E, T;
};

template <int kD>
__global__ __launch_bounds__(kTileThreads) void k_ntt_inv_b_ksl(uint64_t* data, JobSpec js, const TwPair* tw_all,
                                                               const PrimeInfo* primes, KslJobArgs ka) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const uint32_t pc = off / ka.E, t = off - pc * ka.E, c = pc >> 1, p = pc & 1;
    const PrimeInfo& P = primes[prime];
    const uint64_t* xin = ka.ext.p[c] + (size_t)t * kN;
    const KsIn ks{ka.evk.p[c] + ((size_t)p * ka.T + prime) * kN, (size_t)ka.E * kN, 2 * (size_t)ka.T * kN};
    uint64_t* a = data + (size_t)off * kN;
    const TwPair* tw = tw_all + (size_t)prime * kN;
    const JobIn none{nullptr, nullptr};
    if (P.q < kGsOpenMaxQ)
        inv_b_tile<true, false, kD>(a, xin, none, P, tw, blockIdx.x, threadIdx.x, lds, ks);
    else
        inv_b_tile<false, false, kD>(a, xin, none, P, tw, blockIdx.x, threadIdx.x, lds, ks);
}

__global__ __launch_bounds__(kTileThreads) void k_ntt_inv_a(uint64_t* data, JobSpec js, const TwPair* tw_all,
                                                           const PrimeInfo* primes) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const PrimeInfo& P = primes[prime];
    if (P.q < kGsOpenMaxQ)
        inv_a_tile<true>(data + (size_t)off * kN, tw_all + (size_t)prime * kN, P.q, TwPair{P.ninv, P.ninv_p},
                         TwPair{P.w1ninv, P.w1ninv_p}, blockIdx.x, threadIdx.x, lds);
    else
        inv_a_tile<false>(data + (size_t)off * kN, tw_all + (size_t)prime * kN, P.q, TwPair{P.ninv, P.ninv_p},
                          TwPair{P.w1ninv, P.w1ninv_p}, blockIdx.x, threadIdx.x, lds);
}

// ---------------------------------------------------------------- forward pass B that finishes a ModDown
// The forward NTT of a relinearization's ModDown term T ([2B][l-1] limbs, poly 2c + p of ciphertext c) ends with the
// combine instead of a store of T: for each word of limb i,
//   out[2c+p][i] = (x_p P^-1 + add_p - T_p) q_{l-1}^-1,  x_p = sum_d ext[c][d][i] evk[d][p][i]  (the evk inner product),
// add_0 = d0 = a0 b0 and add_1 = d1 = a0 b1 + a1 b0 formed from the product's inputs a, b [B][2][l][N], or read from
// an addend [2B][..][N].  The same words as the NTT followed by k_mdr_combine_ks, without T's store and
// reload.  With the inputs given, the extension's own-digit limbs 0..l-2 are not read (their producer need not store
// them): the word of digit i / own_alpha at limb i, d2 = a1 b1 mod q_i, is formed here from the inputs the combine
// reads anyway.  A workgroup is two 256-thread groups, one per poly of ciphertext c, each transforming the same tile of its
// poly's limb i into an LDS tile of its own; then every thread finishes 8 words of the tile for both polys, so the
// ext digits and the inputs are read once for the two.
struct MdrFuse {
    const uint64_t* ext;  // [B][D][E][N]
    const uint64_t* evk;  // [dnum][2][T][N]
    const uint64_t* ta;   // [B][2][l][N] or null
    const uint64_t* tb;
    const uint64_t* add;  // [2B] polys add_pstride words apart, or null
    uint64_t* out;        // [2B][l-1][N]
    uint64_t add_pstride;
    uint32_t B, l, E, T;
    int64_t post;       // with has_post: added (mod q_i) to every poly 0 word of the output
    uint32_t has_post;
    uint32_t own_alpha;  // with ta/tb: the digit size (limb i's own digit is i / own_alpha; its word is a1 b1)
    TwPair pmod[kMaxPmap];  // P mod q_i
    TwPair cfin[kMaxPmap];  // R P^-1 q_{l-1}^-1 mod q_i (R = 2^64), times the caller's factor
};

// a word at a byte offset from a wave-uniform base (the global_load form with a scalar base and a 32-bit offset)
__device__ __forceinline__ uint64_t ld_at(const uint64_t* base, uint32_t byte_off) {
    return *reinterpret_cast<const uint64_t*>(reinterpret_cast<const char*>(base) + byte_off);
}
__device__ __forceinline__ uint64_t ld_at_nt(const uint64_t* base, uint32_t byte_off) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(reinterpret_cast<const char*>(base) + byte_off));
}

// The combine of one thread's words (lane rl of block blk, words rl + 16 k for k = 8g .. 8g+7), after the transform.
// kTa: the addends are formed from the product's inputs (else read from the addend).  Every pointer and constant is
// derived from the kernel arguments and the job when needed, so that nothing of it is held in registers across the
// transform.  Each word's loads are issued before the previous word's arithmetic (the first word's before the
// transform's last exchange).
template <int kD, bool kTa, bool kPost>
struct MdrEpi {
    struct First {
        uint64_t xv[kD], e0[kD], e1[kD], u0, u1, u2, u3;
    };
    const MdrFuse& f;
    const PrimeInfo& P;
    uint32_t i, c, g;  // limb, ciphertext, the thread's group (= the poly whose tile it transformed)
    uint32_t dn;       // kTa: the digit whose word is formed from the inputs (limb i's own), workgroup-uniform

    __device__ __forceinline__ void load(First& B, int blk, int rl, int k) const {
        const uint32_t bo = (256 * blk + rl + 16 * k) * 8;  // byte offset of the word within a limb
        const size_t li = (size_t)i * kN, xs = (size_t)f.E * kN, es = (size_t)f.T * kN, pw = (size_t)f.l * kN;
        const uint64_t* x = f.ext + (size_t)c * kD * f.E * kN + li;
        const uint64_t* e = f.evk + li;
        if (kTa) {
            // the kD - 1 stored digits in slots 0..kD-2 (slot j holds digit j + (j >= dn), a scalar index), the own
            // digit's key in slot kD-1 (its word is formed from the inputs)
#pragma unroll
            for (int j = 0; j + 1 < kD; j++) {
                const uint32_t d = (uint32_t)j + ((uint32_t)j >= dn ? 1u : 0u);
                B.xv[j] = ld_at(x + d * xs, bo);
                B.e0[j] = ld_at(e + (2 * d) * es, bo);
                B.e1[j] = ld_at(e + (2 * d + 1) * es, bo);
            }
            B.e0[kD - 1] = ld_at(e + (2 * dn) * es, bo);
            B.e1[kD - 1] = ld_at(e + (2 * dn + 1) * es, bo);
        } else {
#pragma unroll
            for (int d = 0; d < kD; d++) {
                B.xv[d] = ld_at(x + d * xs, bo);
                B.e0[d] = ld_at(e + (2 * d) * es, bo);
                B.e1[d] = ld_at(e + (2 * d + 1) * es, bo);
            }
        }
        if (kTa) {
            const uint64_t* a = f.ta + (size_t)c * 2 * pw + li;
            const uint64_t* b = f.tb + (size_t)c * 2 * pw + li;
            B.u0 = ld_at_nt(a, bo);       // a0
            B.u1 = ld_at_nt(a + pw, bo);  // a1
            B.u2 = ld_at_nt(b, bo);       // b0
            B.u3 = ld_at_nt(b + pw, bo);  // b1
        } else {
            B.u0 = ld_at_nt(f.add + 2 * c * f.add_pstride + li, bo);
            B.u1 = ld_at_nt(f.add + (2 * c + 1) * f.add_pstride + li, bo);
        }
    }

    __device__ __forceinline__ First begin(int blk, int rl) const {
        First B;
        load(B, blk, rl, 8 * g);
        return B;
    }

    // L: this group's tile; the tiles of polys 0 and 1 are adjacent (kLdsWords apart)
    // out_p = (x_p P^-1 + d_p - T_p) q_{l-1}^-1 as one 128-bit sum per poly, A_p = x_p + P d_p + P (q - T_p) (P a0 and
    // P a1 formed first, so that d_p's products enter the sum already times P), then REDC(A_p) R P^-1 q_{l-1}^-1: one
    // Montgomery reduction and one Shoup product per word instead of four Barrett reductions, two products by
    // constants and the modular adds between them.  A_p is at most kD + 3 <= 7 products, one factor below 2q and the
    // rest below q < 2^60: A_p < 7 q^2 < q R (REDC's input bound), and the accumulator's cross-product sum (below
    // 2^61.6 a term) stays below 2^64.
    __device__ __forceinline__ void end(First cur, const uint64_t* L, int blk, int rl) const {
        const uint64_t* L0 = L - g * kLdsWords;
        const uint64_t* L1 = L0 + kLdsWords;
        const size_t po = (size_t)(f.l - 1) * kN;
        uint64_t* out0 = f.out + 2 * c * po + (size_t)i * kN;
        uint64_t* out1 = out0 + po;
        const uint64_t q = P.q, ninv = P.mont_ninv;
        const TwPair pm = f.pmod[i], cf = f.cfin[i];
        uint64_t post = 0;  // f.post mod q_i
        if (kPost) {
            const uint64_t m = reduce128(0, f.post >= 0 ? (uint64_t)f.post : 0 - (uint64_t)f.post, Barrett{q, P.mu_hi, P.mu_lo});
            post = (f.post < 0 && m) ? q - m : m;
        }
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const int k = 8 * g + kk;
            // with the inputs: the own digit's word a1 b1 (slot kD-1), formed before the next word's loads are
            // issued (their registers and the product's are not live together)
            if (kTa) cur.xv[kD - 1] = mul_mod(cur.u1, cur.u3, Barrett{q, P.mu_hi, P.mu_lo});
            First nxt;
            if (kk < 7) load(nxt, blk, rl, k + 1);
            Acc s0, s1;
#pragma unroll
            for (int d = 0; d < kD; d++) {
                s0.add(cur.xv[d], cur.e0[d]);
                s1.add(cur.xv[d], cur.e1[d]);
            }
            if (kTa) {
                const uint64_t pa0 = shoup(cur.u0, pm.w, pm.wp, q), pa1 = shoup(cur.u1, pm.w, pm.wp, q);
                s0.add(pa0, cur.u2);                     // P a0 b0
                s1.add(pa0, cur.u3);                     // P a0 b1
                s1.add(pa1, cur.u2);                     // P a1 b0
                s0.add(q - L0[rl + 17 * k], pm.w);       // P (q - T0)
                s1.add(q - L1[rl + 17 * k], pm.w);
            } else {
                s0.add(cur.u0 + q - L0[rl + 17 * k], pm.w);  // P (add0 + q - T0)
                s1.add(cur.u1 + q - L1[rl + 17 * k], pm.w);
            }
            // the Shoup product takes any word below 2^64 to [0, q): the REDC's [0, 2q) needs no subtraction first
            uint64_t v0 = shoup(s0.redc_lazy(q, ninv), cf.w, cf.wp, q);
            const uint64_t v1 = shoup(s1.redc_lazy(q, ninv), cf.w, cf.wp, q);
            if (kPost) v0 = add_mod(v0, post, q);
            const uint32_t bo = (256 * blk + rl + 16 * k) * 8;
            __builtin_nontemporal_store(v0, reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(out0) + bo));
            __builtin_nontemporal_store(v1, reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(out1) + bo));
            if (kk < 7) cur = nxt;
        }
    }
};

// grid (16 tiles, B (l-1) jobs), 512 threads; job v = i B + c (limb-major: a limb's evk is shared by the batch)
template <int kD, bool kTa, bool kPost>
__global__ __launch_bounds__(2 * kTileThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_ntt_fwd_b_mdr(
    uint64_t* T, const TwPair* tw_all, const PrimeInfo* primes, MdrFuse f) {
    __shared__ uint64_t lds[2 * kLdsWords];
    const uint32_t i = uni_div(blockIdx.y, f.B), c = blockIdx.y - i * f.B;
    const uint32_t g = threadIdx.x >> 8, t = threadIdx.x & 255;
    const PrimeInfo& P = primes[i];
    const uint32_t dn = kTa ? uni_div(i, f.own_alpha) : (uint32_t)kD;
    const MdrEpi<kD, kTa, kPost> epi{f, P, i, c, g, dn};
    uint64_t* a = T + ((size_t)(2 * c + g) * (f.l - 1) + i) * kN;
    const TwPair* tw = tw_all + (size_t)i * kN;
    if (P.q < kOpenMaxQ)
        fwd_b_tile<true>(a, tw, P, blockIdx.x, t, lds + g * kLdsWords, epi);
    else
        fwd_b_tile<false>(a, tw, P, blockIdx.x, t, lds + g * kLdsWords, epi);
}

template <int kD>
void launch_b_mdr(dim3 grid, dim3 block, hipStream_t st, uint64_t* T, const TwPair* twb, const PrimeInfo* primes,
                  const MdrFuse& f) {
    // the poly-0 constant (an affine output) is a separate instance: the plain relinearization pays nothing for it
    if (f.ta && f.has_post)
        hipLaunchKernelGGL((k_ntt_fwd_b_mdr<kD, true, true>), grid, block, 0, st, T, twb, primes, f);
    else if (f.ta)
        hipLaunchKernelGGL((k_ntt_fwd_b_mdr<kD, true, false>), grid, block, 0, st, T, twb, primes, f);
    else if (f.has_post)
        hipLaunchKernelGGL((k_ntt_fwd_b_mdr<kD, false, true>), grid, block, 0, st, T, twb, primes, f);
    else
        hipLaunchKernelGGL((k_ntt_fwd_b_mdr<kD, false, false>), grid, block, 0, st, T, twb, primes, f);
}

// ---------------------------------------------------------------- forward pass B that finishes a key-switch list
// The forward NTT of a key-switch list's converted P part y ([2n][l] limbs, poly 2c + p of item c, dense) ends with the
// combine of k_ks_sub_list instead of a store of y: for each word of limb i,
//   out[c][p][i] = x_p P^-1 - y_p (+ the addend's poly 0 on p = 0),  x_p = sum_d ext_c[d][i] evk_c[d][p][i],
// with per-item extensions and keys.  Workgroups as k_ntt_fwd_b_mdr: one 256-thread half per poly, then every thread
// finishes 8 words of the tile for both polys.
struct KslFuse {
    ListPtrs ext, evk;    // item c: [D][E][N] and [dnum][2][T][N]
    const uint64_t* add;  // the addend ciphertexts [2][l][N] (poly 0 used), (c / add_group) add_stride apart, or null
    uint64_t* out;        // [n][2][l][N]
    uint64_t add_stride;
    uint32_t n, l, E, T, add_group;
    // auto_on: item c's output is mapped by X -> X^g_c (a rotation), ginv[c] = g_c^-1 mod 2N: the word formed at
    // index s is stored at the index whose source s is (see KslEpi::end)
    uint32_t auto_on;
    uint32_t ginv[kMaxList];
};

template <int kD>
struct KslEpi {
    struct First {
        uint64_t xv[kD], e0[kD], e1[kD], u0;
    };
    const KslFuse& f;
    const PrimeInfo& P;
    uint32_t i, c, g;  // limb, item, the thread's group (= the poly whose tile it transformed)

    __device__ __forceinline__ void load(First& B, int blk, int rl, int k) const {
        const uint32_t bo = (256 * blk + rl + 16 * k) * 8;
        const size_t li = (size_t)i * kN, xs = (size_t)f.E * kN, es = (size_t)f.T * kN;
        const uint64_t* x = f.ext.p[c] + li;
        const uint64_t* e = f.evk.p[c] + li;
#pragma unroll
        for (int d = 0; d < kD; d++) {
            B.xv[d] = ld_at(x + d * xs, bo);
            B.e0[d] = ld_at(e + (2 * d) * es, bo);
            B.e1[d] = ld_at(e + (2 * d + 1) * es, bo);
        }
        if (f.add) B.u0 = ld_at(f.add + (size_t)(c / f.add_group) * f.add_stride + li, bo);
    }

    __device__ __forceinline__ First begin(int blk, int rl) const {
        First B;
        load(B, blk, rl, 8 * g);
        return B;
    }

    // L: this group's tile; the tiles of polys 0 and 1 are adjacent (kLdsWords apart)
    __device__ __forceinline__ void end(First cur, const uint64_t* L, int blk, int rl) const {
        const uint64_t* L0 = L - g * kLdsWords;
        const uint64_t* L1 = L0 + kLdsWords;
        const size_t pw = (size_t)f.l * kN;
        uint64_t* out0 = f.out + 2 * c * pw + (size_t)i * kN;
        uint64_t* out1 = out0 + pw;
        const uint64_t q = P.q, ninv = P.mont_ninv, pm = P.pmod;
        const TwPair rp{P.rpinv, P.rpinv_p};
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const int k = 8 * g + kk;
            First nxt;
            if (kk < 7) load(nxt, blk, rl, k + 1);
            // x_p P^-1 - conv_p (+ c0 on poly 0) as one 128-bit sum per poly, A_p = x_p + P (q - conv_p [+ c0]),
            // finished by REDC(A_p) R P^-1: at most kD + 1 <= 5 products, one factor below 2q, the others below
            // q < 2^60, so A_p < 6 q^2 < q R and the accumulator's cross-product sum stays below 2^64
            Acc s0, s1;
#pragma unroll
            for (int d = 0; d < kD; d++) {
                s0.add(cur.xv[d], cur.e0[d]);
                s1.add(cur.xv[d], cur.e1[d]);
            }
            s0.add((f.add ? cur.u0 : 0) + q - L0[rl + 17 * k], pm);
            s1.add(q - L1[rl + 17 * k], pm);
            const uint64_t v0 = shoup(s0.redc_lazy(q, ninv), rp.w, rp.wp, q);
            const uint64_t v1 = shoup(s1.redc_lazy(q, ninv), rp.w, rp.wp, q);
            const uint32_t w = 256 * blk + rl + 16 * k;
            if (f.auto_on) {
                // the automorphism: out[k'] = v[src(k')] with src(k') = brev((g (2 brev(k') + 1) mod 2N - 1) / 2), so
                // word w goes to k' = brev((g^-1 (2 brev(w) + 1) mod 2N - 1) / 2).  That index lies in one 256-word
                // block for all w of a block (the low 8 bits of an exponent r' = g r + (g - 1) / 2 depend on those of
                // r only), so a block's stores fill one output block: ordinary stores, which the L2 merges
                const uint32_t r = __brev(w) >> (32 - kLogN);
                const uint32_t e = (f.ginv[c] * (2u * r + 1u)) & (2u * kN - 1u);
                const uint32_t dst = __brev((e - 1u) >> 1) >> (32 - kLogN);
                out0[dst] = v0;
                out1[dst] = v1;
            } else {
                const uint32_t bo = w * 8;
                __builtin_nontemporal_store(v0, reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(out0) + bo));
                __builtin_nontemporal_store(v1, reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(out1) + bo));
            }
            if (kk < 7) cur = nxt;
        }
    }
};

// grid (16 tiles, n l jobs), 512 threads; job v = i n + c (limb-major: a limb's tiles of all items on one XCD)
template <int kD>
__global__ __launch_bounds__(2 * kTileThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_ntt_fwd_b_ksl(
    uint64_t* y, const TwPair* tw_all, const PrimeInfo* primes, KslFuse f) {
    __shared__ uint64_t lds[2 * kLdsWords];
    const uint32_t i = uni_div(blockIdx.y, f.n), c = blockIdx.y - i * f.n;
    const uint32_t g = threadIdx.x >> 8, t = threadIdx.x & 255;
    const PrimeInfo& P = primes[i];
    const KslEpi<kD> epi{f, P, i, c, g};
    uint64_t* a = y + ((size_t)(2 * c + g) * f.l + i) * kN;
    const TwPair* tw = tw_all + (size_t)i * kN;
    if (P.q < kOpenMaxQ)
        fwd_b_tile<true>(a, tw, P, blockIdx.x, t, lds + g * kLdsWords, epi);
    else
        fwd_b_tile<false>(a, tw, P, blockIdx.x, t, lds + g * kLdsWords, epi);
}

// ---------------------------------------------------------------- forward pass B that finishes a plain ModDown
// The forward NTT of a ModDown's converted P part y ([n_polys][l] limbs, dense) ends with the combine of k_sub_scale
// instead of a store of y: out[pc][i] = (x[pc][i] - y[pc][i]) s_i (+ the addend for polys pc % add_div == 0, read at
// (pc / add_group) add_pstride).  The same words as the NTT followed by k_sub_scale, without y's store and reload.
struct SubEpi {
    struct First {
        uint64_t xv[4];
    };
    // the pointers and constants are derived when needed (nothing of them held in registers across the transform)
    const CombineArgs& ca;
    const uint64_t* xb;    // x
    const uint64_t* addb;  // the addend, or null
    uint64_t* outb;        // out
    const PrimeInfo& P;
    uint32_t i, pc;

    __device__ __forceinline__ const uint64_t* xp() const { return xb + pc * ca.x_pstride + (size_t)i * kN; }

    __device__ __forceinline__ First begin(int blk, int rl) const {
        First B;
        const uint32_t bo = (256 * blk + rl) * 8;
        const uint64_t* x = xp();
#pragma unroll
        for (int k = 0; k < 4; k++) B.xv[k] = ld_at_nt(x, bo + 128 * k);
        return B;
    }

    // words in two halves of 8, each half's x words (but the 4 loaded ahead) and addends requested together
    __device__ __forceinline__ void end(First cur, const uint64_t* L, int blk, int rl) const {
        const uint32_t bo = (256 * blk + rl) * 8;
        const uint64_t* x = xp();
        const uint64_t* add =
            addb && pc % ca.add_div == 0 ? addb + (pc / ca.add_group) * ca.add_pstride + (size_t)i * kN : nullptr;
        uint64_t* out = outb + pc * ca.out_pstride + (size_t)i * kN;
        const uint64_t q = P.q;
        const TwPair s = ca.s[i];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint64_t xv[8], av[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                xv[k] = (h == 0 && k < 4) ? cur.xv[k] : ld_at_nt(x, bo + 128 * (8 * h + k));
            if (add) {
#pragma unroll
                for (int k = 0; k < 8; k++) av[k] = ld_at(add, bo + 128 * (8 * h + k));
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int kk = 8 * h + k;
                uint64_t v = shoup(sub_mod(xv[k], L[rl + 17 * kk], q), s.w, s.wp, q);
                if (add) v = add_mod(v, av[k], q);
                __builtin_nontemporal_store(v,
                                            reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(out) + bo + 128 * kk));
            }
        }
    }
};

__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_ntt_fwd_b_sub(uint64_t* y, JobSpec js, const TwPair* tw_all,
                                                               const PrimeInfo* primes, CombineArgs ca,
                                                               const uint64_t* x, const uint64_t* add,
                                                               uint64_t* out) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const uint32_t i = uni_div(blockIdx.y, js.n_polys), pc = blockIdx.y - i * js.n_polys;
    const PrimeInfo& P = primes[prime];
    const SubEpi epi{ca, x, add, out, P, i, pc};
    uint64_t* a = y + (size_t)off * kN;
    const TwPair* tw = tw_all + (size_t)prime * kN;
    if (P.q < kOpenMaxQ)
        fwd_b_tile<true>(a, tw, P, blockIdx.x, threadIdx.x, lds, epi);
    else
        fwd_b_tile<false>(a, tw, P, blockIdx.x, threadIdx.x, lds, epi);
}

// ---------------------------------------------------------------- forward pass B that finishes a scalar combination
// A rescaled linear combination: out[pc][i] = (x[pc][i] - y[pc][i]) s_i with x = sum_t C_t,i x_t + add_i (add on
// polys 0 only) formed here from the terms, word for word as k_lincomb forms it (the sum of the products by C R mod
// q_i reduced by one REDC, then the addend), instead of being stored by a lincomb launch and read back.
constexpr int kLsubTerms = 8;
constexpr int kLsubLimbs = 32;

struct LinSubArgs {
    const uint64_t* x[kLsubTerms];  // term t: [n_polys][stride_t][N], limbs 0 .. l-1 read
    uint32_t stride[kLsubTerms];
    uint32_t n_terms, l, has_add;
    uint64_t out_pstride;
    uint64_t C[kLsubTerms][kLsubLimbs];  // C_t,i R mod q_i
    uint64_t add[kLsubLimbs];
    TwPair s[kLsubLimbs];
};

// the workgroup's share of LinSubArgs (limb i of poly pc), read out of the kernel arguments once
struct LinSubEpi {
    struct First {};
    const uint64_t* xt[kLsubTerms];  // term t's limb i of poly pc
    uint64_t c[kLsubTerms];          // C_t,i R mod q_i
    uint64_t addv;                   // add_i on polys 0, else 0
    TwPair s;
    uint64_t* out;                   // out's limb i of poly pc
    uint64_t q, mont_ninv;
    uint32_t n;

    __device__ __forceinline__ First begin(int, int) const { return First{}; }

    // kG words at a time, every term's words requested together before their products
    static constexpr int kG = 2;
    __device__ __forceinline__ void end(First, const uint64_t* L, int blk, int rl) const {
        const uint32_t bo = (256 * blk + rl) * 8;
#pragma unroll
        for (int h = 0; h < 16 / kG; h++) {
            uint64_t v[kLsubTerms][kG];
#pragma unroll
            for (int t = 0; t < kLsubTerms; t++)
                if (t < (int)n) {
#pragma unroll
                    for (int k = 0; k < kG; k++) v[t][k] = ld_at_nt(xt[t], bo + 128 * (kG * h + k));
                }
#pragma unroll
            for (int k = 0; k < kG; k++) {
                Acc acc;
#pragma unroll
                for (int t = 0; t < kLsubTerms; t++)
                    if (t < (int)n) acc.add(v[t][k], c[t]);
                const uint64_t x = add_mod(acc.redc(q, mont_ninv), addv, q);
                const int kk = kG * h + k;
                const uint64_t r = shoup(sub_mod(x, L[rl + 17 * kk], q), s.w, s.wp, q);
                __builtin_nontemporal_store(r, reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(out) + bo + 128 * kk));
            }
        }
    }
};

__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_ntt_fwd_b_lsub(
    uint64_t* y, JobSpec js, const TwPair* tw_all, const PrimeInfo* primes, LinSubArgs la, uint64_t* out) {
    __shared__ uint64_t lds[kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.y, off, prime);
    const uint32_t i = uni_div(blockIdx.y, js.n_polys), pc = blockIdx.y - i * js.n_polys;
    const PrimeInfo& P = primes[prime];
    LinSubEpi epi;
#pragma unroll
    for (int t = 0; t < kLsubTerms; t++) {
        epi.xt[t] = la.x[t] + ((size_t)pc * la.stride[t] + i) * kN;
        epi.c[t] = la.C[t][i];
    }
    epi.addv = la.has_add && (pc & 1) == 0 ? la.add[i] : 0;
    epi.s = la.s[i];
    epi.out = out + pc * la.out_pstride + (size_t)i * kN;
    epi.q = P.q;
    epi.mont_ninv = P.mont_ninv;
    epi.n = la.n_terms;
    uint64_t* a = y + (size_t)off * kN;
    const TwPair* tw = tw_all + (size_t)prime * kN;
    if (P.q < kOpenMaxQ)
        fwd_b_tile<true>(a, tw, P, blockIdx.x, threadIdx.x, lds, epi);
    else
        fwd_b_tile<false>(a, tw, P, blockIdx.x, threadIdx.x, lds, epi);
}

// Fused: one limb per workgroup of 4 x 256 threads; each 256-thread group owns one LDS tile.
constexpr int kFusedGroups = 2;

__global__ __launch_bounds__(kTileThreads* kFusedGroups) void k_ntt_fwd_fused(uint64_t* data, JobSpec js,
                                                                              const TwPair* tw_all,
                                                                              const TwPair* twb_all,
                                                                              const PrimeInfo* primes) {
    __shared__ uint64_t lds[kFusedGroups * kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.x, off, prime);
    uint64_t* a = data + (size_t)off * kN;
    const TwPair* tw = tw_all + (size_t)prime * kN;
    const uint64_t q = primes[prime].q;
    const int grp = threadIdx.x >> 8, g = threadIdx.x & 255;
    uint64_t* L = lds + grp * kLdsWords;
    for (int t = grp; t < 16; t += kFusedGroups) {
        fwd_a_tile<false>(a, tw, q, t, g, L);
        __syncthreads();
    }
    for (int t = grp; t < 16; t += kFusedGroups) {
        fwd_b_tile<false>(a, twb_all + (size_t)prime * kN, primes[prime], t, g, L);
        __syncthreads();
    }
}

__global__ __launch_bounds__(kTileThreads* kFusedGroups) void k_ntt_inv_fused(uint64_t* data, JobSpec js,
                                                                              const TwPair* tw_all,
                                                                              const TwPair* twb_all,
                                                                              const PrimeInfo* primes) {
    __shared__ uint64_t lds[kFusedGroups * kLdsWords];
    uint32_t off, prime;
    job_of(js, blockIdx.x, off, prime);
    uint64_t* a = data + (size_t)off * kN;
    const TwPair* tw = tw_all + (size_t)prime * kN;
    const PrimeInfo& P = primes[prime];
    const int grp = threadIdx.x >> 8, g = threadIdx.x & 255;
    uint64_t* L = lds + grp * kLdsWords;
    const uint64_t* in = job_src(js, blockIdx.x, data, off);
    for (int t = grp; t < 16; t += kFusedGroups) {
        inv_b_tile<false, false>(a, in, JobIn{nullptr, nullptr}, P, twb_all + (size_t)prime * kN, t, g, L);
        __syncthreads();
    }
    for (int t = grp; t < 16; t += kFusedGroups) {
        inv_a_tile<false>(a, tw, P.q, TwPair{P.ninv, P.ninv_p}, TwPair{P.w1ninv, P.w1ninv_p}, t, g, L);
        __syncthreads();
    }
}

}  // namespace

hipError_t launch_ntt_kernels(const Context& ctx, uint64_t* data, const JobSpec& js, uint32_t n_jobs, bool inverse,
                              NttMode mode, const TwPair* tw, const TwPair* twb, hipStream_t st);

hipError_t launch_ntt(const Context& ctx, uint64_t* data, const JobSpec& js_in, uint32_t n_jobs, bool inverse,
                      NttMode mode, hipStream_t st) {
    if (n_jobs == 0) return hipSuccess;
    JobSpec js = js_in;
    if (!js.jobs && js.n_primes == 0) {
        bool seen[kMaxPrimes] = {};
        for (uint32_t i = 0; i < js.period; i++) {
            js.n_primes += seen[js.pmap[i]] ? 0 : 1;
            seen[js.pmap[i]] = true;
        }
    }
    if (js.src2 || js.copy) {
        // product / copy of the input: dense inverse specs with an out-of-place source, two-pass kernels only
        if (js.jobs || !js.src || !inverse || (js.copy && (js.copy_alpha == 0 || js.copy_E == 0)))
            return hipErrorInvalidValue;
        for (uint32_t i = 0; i < js.period; i++)
            if (js.src2 && ctx.moduli[js.pmap[i]] >= (1ull << 60)) return hipErrorInvalidValue;
        mode = NttMode::TwoPass;
    }
    if (js.lift) {
        // a lifted input: dense forward specs, two-pass kernels only
        if (js.jobs || inverse) return hipErrorInvalidValue;
        mode = NttMode::TwoPass;
    }
    const TwPair* tw = inverse ? ctx.d_itw : ctx.d_tw;
    const TwPair* twb = inverse ? ctx.d_itwb : ctx.d_twb;
    // algorithmic bytes: every limb read and written once (plus the second factor read and the copy written), each
    // prime's table (w, w') read once
    const double streams = 2.0 + (js.src2 ? 1.0 : 0.0);
    const double copied = js.copy ? (double)n_jobs - (double)js.n_polys * std::min(js.copy_from, js.period) : 0.0;
    const double bytes = ((double)n_jobs * streams + copied) * kN * 8 + (double)js.n_primes * kN * sizeof(TwPair);
    const char* name = mode == NttMode::Fused ? (inverse ? "ntt_inv_fused" : "ntt_fwd_fused")
                                              : (inverse ? "ntt_inv_2pass" : "ntt_fwd_2pass");
    const int pi = prof_begin(ctx, name, bytes, st);
    hipError_t err = launch_ntt_kernels(ctx, data, js, n_jobs, inverse, mode, tw, twb, st);
    prof_end(ctx, pi, st);
    return err;
}

// launch_ntt_inv_ks for a key-switch list of n items (item c: extension ext[c] [D][E][N], key evk[c])
hipError_t launch_ntt_inv_ksl(const Context& ctx, uint64_t* acc, const JobSpec& js, uint32_t n_jobs,
                              const uint64_t* const* ext, const uint64_t* const* evk, uint32_t n, uint32_t D,
                              uint32_t E, hipStream_t st) {
    if (!js.jobs || D < 1 || D > 4 || n_jobs == 0 || n == 0 || n > (uint32_t)kMaxList) return hipErrorInvalidValue;
    KslJobArgs ka{};
    for (uint32_t c = 0; c < n; c++) {
        ka.ext.p[c] = ext[c];
        ka.evk.p[c] = evk[c];
    }
    ka.E = E;
    ka.T = ctx.L + ctx.K;
    // algorithmic bytes: per job the limb written, read back by the second pass and written again; per distinct
    // extension and per distinct key D limbs for each of an item's jobs (items of a hoisted list share an extension,
    // items of a batch a key); the tables
    std::set<const uint64_t*> de(ext, ext + n), dk(evk, evk + n);
    const double per_item = (double)n_jobs / n;
    const double bytes = ((double)n_jobs * 3 + ((double)de.size() + (double)dk.size()) * per_item * D) * kN * 8 +
                         (double)js.n_primes * kN * sizeof(TwPair);
    const int pi = prof_begin(ctx, "ntt_inv_ks", bytes, st);
    const dim3 grid(16, n_jobs), block(kTileThreads);
    switch (D) {
        case 1: hipLaunchKernelGGL(k_ntt_inv_b_ksl<1>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
        case 2: hipLaunchKernelGGL(k_ntt_inv_b_ksl<2>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
        case 3: hipLaunchKernelGGL(k_ntt_inv_b_ksl<3>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
        default: hipLaunchKernelGGL(k_ntt_inv_b_ksl<4>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
    }
    hipLaunchKernelGGL(k_ntt_inv_a, grid, block, 0, st, acc, js, ctx.d_itw, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// Forward NTT of a key-switch list's converted P part y [2n][l][N] (coefficients, limb i over prime i; dense) whose
// pass B ends in k_ks_sub_list's combine: out [n][2][l][N] = x P^-1 - NTT(y) (+ the addend's poly 0), x the evk inner
// product of item c's extension and key.  gidx (optional): item c's output mapped by X -> X^gidx[c] (odd, < 2N) as it
// is stored -- a rotation's automorphism, no separate permutation pass.  y is left holding the first pass's
// intermediate.  Digit counts 1..4 and Q primes below 2^60 (others: hipErrorInvalidValue, the caller runs the NTT and
// k_ks_sub_list).
hipError_t launch_ntt_fwd_ksl(const Context& ctx, uint64_t* y, const uint64_t* const* ext, const uint64_t* const* evk,
                              const uint64_t* add, uint64_t add_stride, uint32_t add_group, uint64_t* out, uint32_t n,
                              uint32_t l, hipStream_t st, const uint32_t* gidx) {
    const uint32_t D = (l + ctx.alpha - 1) / ctx.alpha, E = l + ctx.K;
    if (l == 0 || l > kMaxPmap || n == 0 || n > (uint32_t)kMaxList || D < 1 || D > 4 || add_group == 0)
        return hipErrorInvalidValue;
    for (uint32_t i = 0; i < l; i++)
        if (ctx.moduli[i] >= (1ull << 60)) return hipErrorInvalidValue;  // the combine's sum bound
    JobSpec js{};
    js.n_polys = 2 * n;
    js.period = l;
    js.n_primes = l;
    for (uint32_t i = 0; i < l; i++) js.pmap[i] = (uint8_t)i;
    KslFuse f{};
    uint32_t distinct_ext = 0;
    for (uint32_t c = 0; c < n; c++) {
        f.ext.p[c] = ext[c];
        f.evk.p[c] = evk[c];
        distinct_ext += (c == 0 || ext[c] != ext[c - 1]) ? 1 : 0;
    }
    f.add = add;
    f.out = out;
    f.add_stride = add_stride;
    f.n = n;
    f.l = l;
    f.E = E;
    f.T = ctx.L + ctx.K;
    f.add_group = add_group;
    if (gidx) {
        f.auto_on = 1;
        for (uint32_t c = 0; c < n; c++) {
            if ((gidx[c] & 1u) == 0 || gidx[c] >= 2 * kN) return hipErrorInvalidValue;
            // g^-1 mod 2N by Newton's iteration (g odd: x = g is correct to 3 bits, each step doubles them)
            uint32_t x = gidx[c];
            for (int it = 0; it < 4; it++) x *= 2u - gidx[c] * x;
            f.ginv[c] = x & (2 * kN - 1);
        }
    }
    const uint32_t n_jobs = 2 * n * l;
    // algorithmic bytes: y read and written by pass A, read by pass B; ext limbs once per distinct ext, the keys and
    // out per item, addend polys once per group; tables
    const double limbs = (double)n_jobs * 3 + ((double)distinct_ext * D + (double)n * (2.0 * D + 2) +
                                               (add ? (double)(n + add_group - 1) / add_group : 0.0)) * l;
    const int pi = prof_begin(ctx, "ntt_fwd_ksl", limbs * kN * 8 + (double)l * kN * sizeof(TwPair), st);
    hipLaunchKernelGGL(k_ntt_fwd_a, dim3(16, n_jobs), dim3(kTileThreads), 0, st, y, js, ctx.d_tw, ctx.d_primes);
    const dim3 grid(16, n * l), block(2 * kTileThreads);
    switch (D) {
        case 1: hipLaunchKernelGGL(k_ntt_fwd_b_ksl<1>, grid, block, 0, st, y, ctx.d_twb, ctx.d_primes, f); break;
        case 2: hipLaunchKernelGGL(k_ntt_fwd_b_ksl<2>, grid, block, 0, st, y, ctx.d_twb, ctx.d_primes, f); break;
        case 3: hipLaunchKernelGGL(k_ntt_fwd_b_ksl<3>, grid, block, 0, st, y, ctx.d_twb, ctx.d_primes, f); break;
        default: hipLaunchKernelGGL(k_ntt_fwd_b_ksl<4>, grid, block, 0, st, y, ctx.d_twb, ctx.d_primes, f); break;
    }
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// Inverse NTT of a job list over an accumulator [n_polys][E][N] (off = pc E + t) whose input, limb t of poly pc, is
// the evk inner product sum_d ext[pc / 2][d][t] evk[d][pc % 2][prime] (the inner product a key switch would store
// there first).  Digit counts 1..4 (others: hipErrorInvalidValue, the caller stores the inner product first).
hipError_t launch_ntt_inv_ks(const Context& ctx, uint64_t* acc, const JobSpec& js, uint32_t n_jobs,
                             const uint64_t* ext, const uint64_t* evk, uint32_t D, uint32_t E, hipStream_t st) {
    if (!js.jobs || D < 1 || D > 4 || n_jobs == 0) return hipErrorInvalidValue;
    const KsJobArgs ka{ext, evk, E, ctx.L + ctx.K};
    // algorithmic bytes: per job D extension limbs read, the limb written, read back by the second pass and written
    // again; the key shared by the batch once: D limbs for each distinct (poly half, prime) of the jobs; the tables
    const double key_limbs = std::min<double>(n_jobs, 2.0 * js.n_primes) * D;
    const double bytes = ((double)n_jobs * (D + 3.0) + key_limbs) * kN * 8 + (double)js.n_primes * kN * sizeof(TwPair);
    const int pi = prof_begin(ctx, "ntt_inv_ks", bytes, st);
    const dim3 grid(16, n_jobs), block(kTileThreads);
    switch (D) {
        case 1: hipLaunchKernelGGL(k_ntt_inv_b_ks<1>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
        case 2: hipLaunchKernelGGL(k_ntt_inv_b_ks<2>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
        case 3: hipLaunchKernelGGL(k_ntt_inv_b_ks<3>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
        default: hipLaunchKernelGGL(k_ntt_inv_b_ks<4>, grid, block, 0, st, acc, js, ctx.d_itwb, ctx.d_primes, ka); break;
    }
    hipLaunchKernelGGL(k_ntt_inv_a, grid, block, 0, st, acc, js, ctx.d_itw, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// The rescale of a linear combination (see LinSubEpi): y [n_polys][l][N] receives the forward NTT of the lift of
// the combination's dropped limb (lift: its coefficients, one limb per poly lift_pstride words apart, residues mod
// lift_q); out [n_polys][..][N] (out_pstride words between polys) = (x - y) s with x formed from the terms.
// C [n_terms][l] and add [l] (or null) are the combination's constants reduced mod q_i; s [l].
hipError_t launch_ntt_fwd_lsub(const Context& ctx, uint64_t* y, uint32_t n_terms, const uint64_t* const* x,
                               const uint32_t* stride, const uint64_t* C, const uint64_t* add, uint64_t* out,
                               uint64_t out_pstride, uint32_t n_polys, uint32_t l, const TwPair* s, hipStream_t st,
                               const uint64_t* lift, uint64_t lift_pstride, uint64_t lift_q) {
    if (l == 0 || l > (uint32_t)kLsubLimbs || n_polys == 0 || n_terms == 0 || n_terms > (uint32_t)kLsubTerms)
        return hipErrorInvalidValue;
    JobSpec js{};
    js.n_polys = n_polys;
    js.period = l;
    js.n_primes = l;
    for (uint32_t i = 0; i < l; i++) js.pmap[i] = (uint8_t)i;
    js.lift = lift;
    js.lift_pstride = lift_pstride;
    js.lift_q = lift_q;
    LinSubArgs la{};
    la.n_terms = n_terms;
    la.l = l;
    la.has_add = add ? 1 : 0;
    la.out_pstride = out_pstride;
    for (uint32_t t = 0; t < n_terms; t++) {
        if (stride[t] < l) return hipErrorInvalidValue;
        la.x[t] = x[t];
        la.stride[t] = stride[t];
        for (uint32_t i = 0; i < l; i++) {
            // C R mod q_i (REDC of the sum gives the combination), a Shoup product by the context's R mod q_i
            const PrimeInfo& pr = ctx.primes[i];
            const uint64_t c = C[(size_t)t * l + i] % pr.q;
            const uint64_t h = (uint64_t)(((unsigned __int128)c * pr.r_mod_p) >> 64);
            const uint64_t v = c * pr.r_mod - h * pr.q;
            la.C[t][i] = v >= pr.q ? v - pr.q : v;
        }
    }
    for (uint32_t i = 0; i < l; i++) {
        la.add[i] = add ? add[i] : 0;
        la.s[i] = s[i];
    }
    const uint32_t n_jobs = n_polys * l;
    // algorithmic bytes: the lift source once per poly, y written by pass A and read by pass B, the terms read, out
    // written; tables
    const double bytes = ((double)n_polys + 2.0 * n_jobs + (double)n_jobs * n_terms + n_jobs) * kN * 8 +
                         (double)l * kN * sizeof(TwPair);
    const int pi = prof_begin(ctx, "ntt_fwd_lsub", bytes, st);
    const dim3 grid(16, n_jobs), block(kTileThreads);
    hipLaunchKernelGGL(k_ntt_fwd_a, grid, block, 0, st, y, js, ctx.d_tw, ctx.d_primes);
    hipLaunchKernelGGL(k_ntt_fwd_b_lsub, grid, block, 0, st, y, js, ctx.d_twb, ctx.d_primes, la, out);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// Forward NTT of a ModDown's converted P part y [n_polys][l][N] (coefficients, limb i over prime i; dense) whose pass
// B ends in k_sub_scale's combine: out[pc][i] = (x[pc][i] - NTT(y)[pc][i]) s_i (+ the addend).  y is left holding
// the first pass's intermediate.  Same argument meaning as launch_sub_scale.  lift (optional): y's input is instead
// formed by the first pass from one limb per poly (JobSpec.lift).
hipError_t launch_ntt_fwd_sub(const Context& ctx, uint64_t* y, const uint64_t* x, uint64_t x_pstride,
                              const uint64_t* add, uint64_t add_pstride, uint32_t add_div, uint32_t add_group,
                              uint64_t* out, uint64_t out_pstride, uint32_t n_polys, uint32_t l, const TwPair* s,
                              hipStream_t st, const uint64_t* lift, uint64_t lift_pstride, uint64_t lift_q) {
    if (l == 0 || l > kMaxPmap || n_polys == 0) return hipErrorInvalidValue;
    JobSpec js{};
    js.n_polys = n_polys;
    js.period = l;
    js.n_primes = l;
    for (uint32_t i = 0; i < l; i++) js.pmap[i] = (uint8_t)i;
    js.lift = lift;
    js.lift_pstride = lift_pstride;
    js.lift_q = lift_q;
    CombineArgs ca{};
    ca.l = l;
    ca.add_div = add_div ? add_div : 1;
    ca.add_group = add_group ? add_group : ca.add_div;
    ca.x_pstride = x_pstride;
    ca.y_pstride = (uint64_t)l * kN;
    ca.out_pstride = out_pstride;
    ca.add_pstride = add_pstride;
    for (uint32_t i = 0; i < l; i++) ca.s[i] = s[i];
    const uint32_t n_jobs = n_polys * l;
    // algorithmic bytes: y read (or the lift source, once per poly) and written by pass A, read by pass B; x read,
    // out written; the addends; tables
    const double n_add = add ? (double)n_polys / ca.add_div : 0.0;
    const double reads_a = lift ? (double)n_polys : (double)n_jobs;
    const double bytes = ((double)n_jobs * 4 + reads_a + n_add * l) * kN * 8 + (double)l * kN * sizeof(TwPair);
    const int pi = prof_begin(ctx, "ntt_fwd_sub", bytes, st);
    const dim3 grid(16, n_jobs), block(kTileThreads);
    hipLaunchKernelGGL(k_ntt_fwd_a, grid, block, 0, st, y, js, ctx.d_tw, ctx.d_primes);
    hipLaunchKernelGGL(k_ntt_fwd_b_sub, grid, block, 0, st, y, js, ctx.d_twb, ctx.d_primes, ca, x, add, out);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// Forward NTT of a relinearization's ModDown term T [2B][l-1][N] (coefficients, limb i over prime i) whose pass B
// ends in the combine (k_ntt_fwd_b_mdr): out [2B][l-1][N] = (x P^-1 + add - NTT(T)) q_{l-1}^-1 with x the evk inner
// product of ext [B][D][E][N] and evk, add from ta/tb (the product's inputs) or add.  pmod[i] = P mod q_i and
// cfin[i] = R P^-1 q_{l-1}^-1 mod q_i (R = 2^64), with Shoup companions, for limbs i < l-1 (primes below 2^60).  T is
// left holding the first pass's intermediate.  Digit counts 1..4 (others: hipErrorInvalidValue, the caller runs the
// two kernels).  own_from_inputs (required with ta, tb, and only then): ext's own-digit limbs 0..l-2 are not read;
// each is d2 = a1 b1, formed from the inputs.
hipError_t launch_ntt_fwd_mdr(const Context& ctx, uint64_t* T, uint32_t B, uint32_t l, const uint64_t* ext,
                              const uint64_t* evk, const uint64_t* ta, const uint64_t* tb, const uint64_t* add,
                              uint64_t add_pstride, uint64_t* out, const TwPair* pmod, const TwPair* cfin,
                              hipStream_t st, const int64_t* post, bool own_from_inputs) {
    const uint32_t D = (l + ctx.alpha - 1) / ctx.alpha, E = l + ctx.K;
    if (l < 2 || l > kMaxPmap || B == 0 || D < 1 || D > 4 || (ta && (!tb || add)) || (!ta && !add) ||
        own_from_inputs != (ta != nullptr) || ctx.alpha == 0)
        return hipErrorInvalidValue;
    JobSpec js{};
    js.n_polys = 2 * B;
    js.period = l - 1;
    js.n_primes = l - 1;
    for (uint32_t i = 0; i + 1 < l; i++) js.pmap[i] = (uint8_t)i;
    MdrFuse f{};
    f.ext = ext;
    f.evk = evk;
    f.ta = ta;
    f.tb = tb;
    f.add = add;
    f.add_pstride = add_pstride;
    f.out = out;
    f.B = B;
    f.l = l;
    f.E = E;
    f.T = ctx.L + ctx.K;
    f.has_post = post ? 1 : 0;
    f.post = post ? *post : 0;
    f.own_alpha = own_from_inputs ? ctx.alpha : 0;
    for (uint32_t i = 0; i + 1 < l; i++) {
        if (ctx.moduli[i] >= (1ull << 60)) return hipErrorInvalidValue;  // the combine's sum bound
        f.pmod[i] = pmod[i];
        f.cfin[i] = cfin[i];
    }
    const uint32_t n_jobs = 2 * B * (l - 1);
    // algorithmic bytes: T read and written by pass A, read by pass B; per ciphertext and limb D ext limbs (D - 1
    // when the own digit's word is formed from the inputs), the 4 product inputs or 2 addend limbs, 2 outputs; the
    // level's evk limbs and the twiddle tables once
    const double n_ext = own_from_inputs ? D - 1.0 : (double)D;
    const double limbs = (double)n_jobs * 3 + (double)B * (l - 1) * (n_ext + (ta ? 4 : add ? 2 : 0) + 2) +
                         2.0 * D * (l - 1);
    const int pi = prof_begin(ctx, "ntt_fwd_mdr", limbs * kN * 8 + (double)(l - 1) * kN * sizeof(TwPair), st);
    hipLaunchKernelGGL(k_ntt_fwd_a, dim3(16, n_jobs), dim3(kTileThreads), 0, st, T, js, ctx.d_tw, ctx.d_primes);
    const dim3 grid(16, B * (l - 1)), block(2 * kTileThreads);
    switch (D) {
        case 1: launch_b_mdr<1>(grid, block, st, T, ctx.d_twb, ctx.d_primes, f); break;
        case 2: launch_b_mdr<2>(grid, block, st, T, ctx.d_twb, ctx.d_primes, f); break;
        case 3: launch_b_mdr<3>(grid, block, st, T, ctx.d_twb, ctx.d_primes, f); break;
        default: launch_b_mdr<4>(grid, block, st, T, ctx.d_twb, ctx.d_primes, f); break;
    }
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_ntt_kernels(const Context& ctx, uint64_t* data, const JobSpec& js, uint32_t n_jobs, bool inverse,
                              NttMode mode, const TwPair* tw, const TwPair* twb, hipStream_t st) {
    if (mode == NttMode::Fused) {
        if (inverse)
            hipLaunchKernelGGL(k_ntt_inv_fused, dim3(n_jobs), dim3(kTileThreads * kFusedGroups), 0, st, data, js, tw,
                               twb, ctx.d_primes);
        else
            hipLaunchKernelGGL(k_ntt_fwd_fused, dim3(n_jobs), dim3(kTileThreads * kFusedGroups), 0, st, data, js, tw,
                               twb, ctx.d_primes);
        return hipGetLastError();
    }
    // pass B reads pass B's table (the same pairs, its last four stages' entries reordered per block)
    const dim3 grid(16, n_jobs), block(kTileThreads);
    if (inverse) {
        hipLaunchKernelGGL(k_ntt_inv_b, grid, block, 0, st, data, js, twb, ctx.d_primes);
        hipLaunchKernelGGL(k_ntt_inv_a, grid, block, 0, st, data, js, tw, ctx.d_primes);
    } else {
        hipLaunchKernelGGL(k_ntt_fwd_a, grid, block, 0, st, data, js, tw, ctx.d_primes);
        hipLaunchKernelGGL(k_ntt_fwd_b, grid, block, 0, st, data, js, twb, ctx.d_primes);
    }
    return hipGetLastError();
}

}  // namespace fhe
