// rns.hip -- limb-wise kernels of the RNS-CKKS core: tensor product, approximate CRT basis
// conversion (BConv, the heart of ModUp / ModDown), the key-switch inner product, the ModDown and
// rescale combines, the centered lift of rescale, additions and the evaluation-form automorphism.
//
// All of these are HBM-streaming elementwise kernels: one thread per coefficient index k, limbs
// walked in registers, residues canonical in [0, q) on every store (but the BConv's, which only forward NTTs read:
// see there).  Products that are not by a per-limb constant accumulate in 128 bits and reduce once (Barrett, mu =
// floor(2^128 / q), or Montgomery's REDC against R-scaled constants); products by a per-limb constant use Shoup with a
// precomputed companion.
#include <algorithm>

#include "engine.hpp"
#include "ks_device.hpp"
#include "modarith.hpp"

namespace fhe {

namespace {

// ------------------------------------------------------------------ tensor product
// a, b: [B][2][l][N]; d01: [B][2][l][N] (d0, d1); d2: [B][l][N]; d2e (optional): second copy of d2
// scattered into the ModUp extension buffer: limb t of ciphertext c goes to d2e + c*d2e_bstride +
// ext_off[t]*N.
// Limbs t0..l-1 only (grid y = l - t0).  d2 null: d0 and d1 alone (the relinearization's inverse NTT then forms d2
// from a1 and b1 as it reads them, and a relinearization with its rescale forms d0 and d1 of limbs 0..l-2 in the
// ModDown combine, so it asks for limb l-1 only).
struct TensorArgs {
    uint32_t l, B, t0;
    uint64_t* d2e;
    uint64_t d2e_bstride;
    uint32_t ext_off[kMaxPmap];
};

__global__ __launch_bounds__(256) void k_tensor(const uint64_t* __restrict__ a, const uint64_t* __restrict__ b,
                                                uint64_t* __restrict__ d01, uint64_t* __restrict__ d2,
                                                TensorArgs ta, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t t = ta.t0 + blockIdx.y, c = blockIdx.z;
    const Barrett br = barrett_of(primes[t]);
    const size_t P = (size_t)ta.l * kN;
    const size_t o = (size_t)c * 2 * P + (size_t)t * kN + k;
    const uint64_t a0 = a[o], a1 = a[o + P], b0 = b[o], b1 = b[o + P];
    Acc s0, s1;
    s0.add(a0, b0);
    s1.add(a0, b1);
    s1.add(a1, b0);
    // outputs streamed (nontemporal): each is read once, by a later kernel
    __builtin_nontemporal_store(reduce_u128(s0.get(), br), &d01[o]);
    __builtin_nontemporal_store(reduce_u128(s1.get(), br), &d01[o + P]);
    if (!d2) return;
    Acc s2;
    s2.add(a1, b1);
    const uint64_t v2 = reduce_u128(s2.get(), br);
    __builtin_nontemporal_store(v2, &d2[(size_t)c * P + (size_t)t * kN + k]);
    if (ta.d2e) __builtin_nontemporal_store(v2, &ta.d2e[c * ta.d2e_bstride + (size_t)ta.ext_off[t] * kN + k]);
}

// Sum of np tensor products per batch item: tab[(c np + j) 2 + 0/1] point at ciphertexts [2][l][N];
// d01/d2 as in k_tensor.  The 128-bit sums hold up to 2 np products below 2^120: np <= 64.
__global__ __launch_bounds__(256) void k_tensor_sum(const uint64_t* const* __restrict__ tab, uint32_t np,
                                                    uint64_t* __restrict__ d01, uint64_t* __restrict__ d2,
                                                    TensorArgs ta, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t t = blockIdx.y, c = blockIdx.z;
    const Barrett br = barrett_of(primes[t]);
    const size_t P = (size_t)ta.l * kN, w = (size_t)t * kN + k;
    Acc s0, s1, s2;
    // 4 products at a time (s1 takes two terms per product: a fold every 4), their 16 words requested together
    for (uint32_t j0 = 0; j0 < np; j0 += 4) {
        uint64_t a0[4], a1[4], b0[4], b1[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (j0 + u < np) {
                const uint64_t* a = tab[((size_t)c * np + j0 + u) * 2];
                const uint64_t* b = tab[((size_t)c * np + j0 + u) * 2 + 1];
                a0[u] = a[w];
                a1[u] = a[P + w];
                b0[u] = b[w];
                b1[u] = b[P + w];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (j0 + u < np) {
                s0.add(a0[u], b0[u]);
                s1.add(a0[u], b1[u]);
                s1.add(a1[u], b0[u]);
                s2.add(a1[u], b1[u]);
            }
        }
        s0.fold();
        s1.fold();
        s2.fold();
    }
    const size_t o = (size_t)c * 2 * P + w;
    d01[o] = reduce_u128(s0.get(), br);
    d01[o + P] = reduce_u128(s1.get(), br);
    const uint64_t v2 = reduce_u128(s2.get(), br);
    d2[(size_t)c * P + w] = v2;
    if (ta.d2e) ta.d2e[c * ta.d2e_bstride + (size_t)ta.ext_off[t] * kN + k] = v2;
}

// ------------------------------------------------------------------ BConv
// out_j[k] = sum_i [x_i[k] * qhinv_i]_{q_i} * qhmod[i][j]  mod p_j
// in  : batch c -> in + c*in_bstride, source limb i at off(in_desc[i])*N, prime prime(in_desc[i])
// out : batch c -> out + c*out_bstride, target limb j at off(out_desc[j])*N, prime prime(out_desc[j])
// tab : [n_in] TwPair (qhinv, companion) followed by [n_in][n_out] uint64 qhmod
// Every BConv output is the input of a forward NTT, which takes words below 8q and stores canonical residues: the
// Montgomery-reduced instances leave their outputs in [0, 2q) (redc_lazy), skipping the final conditional
// subtraction; the ModDown+rescale instance adds the rescale's lift to that, below q (lift_centered) or below 3q (the
// fast lift), so its outputs stay below 5q.  The bounds, in units of the output prime q:
constexpr uint32_t kRedcLazyBound = 2;    // redc_lazy: [0, 2q)
constexpr uint32_t kFastLiftBound = 3;    // z + [z > q_{l-1}/2] dl with z < q_{l-1} <= 2q and dl < q: [0, 3q)
constexpr uint32_t kNttFwdInputBound = 8; // the forward NTT's first stage takes words below 8q (fwd_a_tile, ct_bfly)
static_assert(kRedcLazyBound + kFastLiftBound <= kNttFwdInputBound,
              "a BConv output must stay below the forward NTT's input bound");
// A limb descriptor is one dword, offset | prime << 16: the output loop indexes it with a wave-uniform j, which
// a scalar load serves (byte or half-word arrays would be read with vector loads, one round trip per output).
constexpr int kMaxBconvIn = 16;
constexpr int kMaxBconvOut = 80;

struct BConvArgs {
    uint32_t n_in, n_out;
    uint32_t centered;  // subtract u * (prod of input primes) with u = round(sum_i y_i / q_i)
    uint32_t mont;      // the table's columns are in Montgomery form: reduce the sums by REDC
    uint64_t in_bstride, out_bstride;
    uint32_t in_desc[kMaxBconvIn];
    uint32_t out_desc[kMaxBconvOut];
};

__device__ __forceinline__ uint32_t desc_off(uint32_t d) { return d & 0xFFFFu; }
__device__ __forceinline__ uint32_t desc_prime(uint32_t d) { return d >> 16; }

// Extra inputs of the ModDown BConv fused with the rescale that follows (k_bconv<NIN, true, ..>).  The plan's last
// output column is the dropped limb l-1 (plain table); every other column j has P^-1 mod q_j folded into its
// table, so the column sums are conv_j P^-1 directly.  Per coefficient the kernel forms
//   z = addc + (x_{l-1} - conv_{l-1}) P^-1  (mod q_{l-1}, x_{l-1} and addc in coefficient form)
// and writes T_j = conv_j P^-1 + [z]_{q_j} (centered lift) for j < l-1.
struct MdrBconvArgs {
    const uint64_t* xlast;  // limb l-1 of each input poly, coefficient form, poly stride xlast_pstride
    uint64_t xlast_pstride;
    const uint64_t* addc;   // [n_polys][N] coefficient form of the addend's limb l-1, or null
    TwPair pinv_last;       // P^-1 mod q_{l-1}
    // fast_lift (set when q_{l-1} <= 2 q_j for every output j): the lift of z into q_j is z + [z > q_{l-1} / 2] dl[j]
    // with dl[j] = -q_{l-1} mod q_j, below 3 q_j -- no reduction; added to the Montgomery sum's [0, 2q_j), T_j stays
    // below 5 q_j (the forward NTT that reads T takes words below 8q: kNttFwdInputBound)
    uint32_t fast_lift;
    uint64_t dl[kMaxBconvOut];
};

// NIN = number of input limbs (a template parameter: the term loops unroll without run-time guards).  The table's
// q-hat constants are stored pre-split into 30-bit halves (pack30), the y_i are split once, and every term is three
// multiply-adds into carry-free sums (Acc30k; inputs taken in chunks of at most 8).
// kMode: 0 = the plan's flags read at run time; 1 = Montgomery-reduced, not centered; 2 = Montgomery-reduced and
// centered (the flags known at compile time: no per-output tests of them).
template <int NIN, bool kMdr, int kMode>
__global__ __launch_bounds__(256) void k_bconv(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                               BConvArgs ba, const uint64_t* __restrict__ tab,
                                               const PrimeInfo* __restrict__ primes, MdrBconvArgs mb) {
    const bool centered = kMode == 0 ? ba.centered != 0 : kMode == 2, mont = kMode == 0 ? ba.mont != 0 : true;
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t c = blockIdx.y;
    const uint64_t* src = in + c * ba.in_bstride + k;
    uint64_t* dst = out + c * ba.out_bstride + k;
    const TwPair* qhinv = reinterpret_cast<const TwPair*>(tab);
    const uint64_t* qhmod = tab + 2 * ba.n_in;  // [n_in][n_out], pack30 form
    uint64_t y[NIN];
    uint32_t y0[NIN], y1[NIN], ys[NIN];
#pragma unroll
    for (int i = 0; i < NIN; i++) {
        const uint64_t q = primes[desc_prime(ba.in_desc[i])].q;
        y[i] = shoup(__builtin_nontemporal_load(&src[(size_t)desc_off(ba.in_desc[i]) * kN]), qhinv[i].w, qhinv[i].wp,
                     q);
        y0[i] = (uint32_t)y[i] & 0x3FFFFFFFu;
        y1[i] = (uint32_t)(y[i] >> 30);
        ys[i] = y0[i] + y1[i];
    }
    // centered form (exact ModDown): u = round(sum_i y_i / q_i) from the 128-bit fixed-point sum of
    // floor(y_i * floor(2^128 / q_i) / 2^64); the table then holds [n_in] (lo, hi) words of floor(2^128 / q_i)
    // and [n_out] (prod of the input primes) mod p_j
    uint64_t u = 0;
    const uint64_t* cfix = qhmod + (size_t)ba.n_in * ba.n_out;
    const uint64_t* pmod = cfix + 2 * ba.n_in;
    if (centered) {
        U128 F{0, 0};
#pragma unroll
        for (int i = 0; i < NIN; i++) {
            mac128(F, y[i], cfix[2 * i + 1]);
            const uint64_t h = mulhi64(y[i], cfix[2 * i]);
            F.lo += h;
            F.hi += (F.lo < h) ? 1 : 0;
        }
        const uint64_t lo = F.lo + (1ull << 63);
        u = F.hi + (lo < F.lo ? 1 : 0);
    }
    // column sums of outputs j and j2 (= j when only one is wanted), before the final reduction
    auto sums = [&](uint32_t j, uint32_t j2, U128& r, U128& r2) {
        Acc30k a, b;
#pragma unroll
        for (int i = 0; i < (NIN < 8 ? NIN : 8); i++) {
            a.add(y0[i], y1[i], ys[i], qhmod[(size_t)i * ba.n_out + j]);
            b.add(y0[i], y1[i], ys[i], qhmod[(size_t)i * ba.n_out + j2]);
        }
        r = a.get();
        r2 = b.get();
        if constexpr (NIN > 8) {
            Acc30k a2, b2;
#pragma unroll
            for (int i = 8; i < NIN; i++) {
                a2.add(y0[i], y1[i], ys[i], qhmod[(size_t)i * ba.n_out + j]);
                b2.add(y0[i], y1[i], ys[i], qhmod[(size_t)i * ba.n_out + j2]);
            }
            const U128 s = a2.get(), s2 = b2.get();
            r.lo += s.lo;
            r.hi += s.hi + (r.lo < s.lo ? 1u : 0u);
            r2.lo += s2.lo;
            r2.hi += s2.hi + (r2.lo < s2.lo ? 1u : 0u);
        }
    };
    // the centered correction: acc - u * pmod_j, kept non-negative by adding 16 p_j (u <= n_in <= 16)
    auto correct = [&](U128& acc, uint32_t j, const Barrett& br) {
        if (centered) {
            const uint64_t t = 16 * br.q - u * pmod[j];
            acc.lo += t;
            acc.hi += (acc.lo < t) ? 1 : 0;
        }
    };
    uint32_t n_main = ba.n_out;
    uint64_t z = 0, ql = 0;
    bool zneg = false;  // z stands for z - q_{l-1}
    if constexpr (kMdr) {
        n_main = ba.n_out - 1;
        U128 acc, unused;
        sums(n_main, n_main, acc, unused);
        const PrimeInfo& pl = primes[desc_prime(ba.out_desc[n_main])];
        const Barrett bl = barrett_of(pl);
        correct(acc, n_main, bl);
        const uint64_t conv = mont ? redc(acc, pl.q, pl.mont_ninv) : reduce_u128(acc, bl);
        ql = bl.q;
        z = shoup(sub_mod(mb.xlast[c * mb.xlast_pstride + k], conv, ql), mb.pinv_last.w, mb.pinv_last.wp, ql);
        if (mb.addc) z = add_mod(z, mb.addc[(size_t)c * kN + k], ql);
        zneg = z > (ql >> 1);
    }
    auto finish = [&](U128 acc, uint32_t j) {
        const uint32_t dj = ba.out_desc[j];
        const PrimeInfo& pj = primes[desc_prime(dj)];
        const Barrett br = barrett_of(pj);
        correct(acc, j, br);
        uint64_t v;
        if (mont) {
            // left in [0, 2q) (plus the lift: [0, 3q) with lift_centered, [0, 5q) with the fast lift): the consumer
            // is a forward NTT (inputs below 8q)
            v = redc_lazy(acc, pj.q, pj.mont_ninv);
            if constexpr (kMdr) v += mb.fast_lift ? z + (zneg ? mb.dl[j] : 0) : lift_centered(z, ql, br);
        } else {
            if constexpr (kMdr) {
                const uint64_t r = lift_centered(z, ql, br);
                acc.lo += r;
                acc.hi += (acc.lo < r) ? 1u : 0u;
            }
            v = reduce_u128(acc, br);
        }
        // streamed: read once, by the next NTT (nontemporal, so the L2 keeps what is reused)
        __builtin_nontemporal_store(v, &dst[(size_t)desc_off(dj) * kN]);
    };
    // Montgomery-reduced, not centered, at most 8 inputs (the ModUp and ModDown instances): each output's REDC is
    // taken from its three Karatsuba sums directly (Acc30k::redc_lazy, the same word as through the 128-bit sum)
    constexpr bool kFast = kMode == 1 && NIN <= 8;
    auto terms = [&](uint32_t j, uint32_t j2, Acc30k& a, Acc30k& b) {
#pragma unroll
        for (int i = 0; i < (NIN < 8 ? NIN : 8); i++) {
            a.add(y0[i], y1[i], ys[i], qhmod[(size_t)i * ba.n_out + j]);
            b.add(y0[i], y1[i], ys[i], qhmod[(size_t)i * ba.n_out + j2]);
        }
    };
    auto finish_fast = [&](const Acc30k& a, uint32_t j) {
        const uint32_t dj = ba.out_desc[j];
        const PrimeInfo& pj = primes[desc_prime(dj)];
        // [0, 2q) (with the lift, as in finish)
        uint64_t v = a.redc_lazy(pj.q, pj.mont_ninv);
        if constexpr (kMdr) v += mb.fast_lift ? z + (zneg ? mb.dl[j] : 0) : lift_centered(z, ql, barrett_of(pj));
        __builtin_nontemporal_store(v, &dst[(size_t)desc_off(dj) * kN]);
    };
    // the outputs of this workgroup's share (grid z splits them when the batch is too small to fill the GPU), two
    // per iteration: independent accumulation chains for the scheduler to interleave
    const uint32_t share = ((n_main + gridDim.z - 1) / gridDim.z + 1) & ~1u;
    const uint32_t j_end = min(n_main, (blockIdx.z + 1) * share);
    uint32_t j = blockIdx.z * share;
    for (; j + 1 < j_end; j += 2) {
        if constexpr (kFast) {
            Acc30k a, b;
            terms(j, j + 1, a, b);
            finish_fast(a, j);
            finish_fast(b, j + 1);
        } else {
            U128 r, r2;
            sums(j, j + 1, r, r2);
            finish(r, j);
            finish(r2, j + 1);
        }
    }
    if (j < j_end) {
        if constexpr (kFast) {
            Acc30k a, b;
            terms(j, j, a, b);
            finish_fast(a, j);
        } else {
            U128 r, unused;
            sums(j, j, r, unused);
            finish(r, j);
        }
    }
}

// grid z of a ModUp BConv launch: with fewer than 8 workgroups of 256 coefficients per CU the outputs are split over
// z (each share at least 4 outputs; every share converts its inputs itself).  The ModDown instance is not split: each
// share would form the dropped limb's conversion and lift again, and measured slower.
static uint32_t bconv_split(uint32_t n_polys, uint32_t n_out) {
    const uint32_t wg = (kN / 256) * n_polys, want = 2048;
    if (wg >= want) return 1;
    return std::max(1u, std::min((want + wg - 1) / wg, n_out / 4));
}

// k_bconv instance for a run-time input count (1..kMaxBconvIn)
template <bool kMdr, int kMode>
static void (*bconv_kernel_m(uint32_t n_in))(const uint64_t*, uint64_t*, BConvArgs, const uint64_t*,
                                             const PrimeInfo*, MdrBconvArgs) {
    switch (n_in) {
        case 1: return k_bconv<1, kMdr, kMode>;
        case 2: return k_bconv<2, kMdr, kMode>;
        case 3: return k_bconv<3, kMdr, kMode>;
        case 4: return k_bconv<4, kMdr, kMode>;
        case 5: return k_bconv<5, kMdr, kMode>;
        case 6: return k_bconv<6, kMdr, kMode>;
        case 7: return k_bconv<7, kMdr, kMode>;
        case 8: return k_bconv<8, kMdr, kMode>;
        case 9: return k_bconv<9, kMdr, kMode>;
        case 10: return k_bconv<10, kMdr, kMode>;
        case 11: return k_bconv<11, kMdr, kMode>;
        case 12: return k_bconv<12, kMdr, kMode>;
        case 13: return k_bconv<13, kMdr, kMode>;
        case 14: return k_bconv<14, kMdr, kMode>;
        case 15: return k_bconv<15, kMdr, kMode>;
        case 16: return k_bconv<16, kMdr, kMode>;
        default: return nullptr;
    }
}

template <bool kMdr>
static void (*bconv_kernel(const BConvPlan& plan))(const uint64_t*, uint64_t*, BConvArgs, const uint64_t*,
                                                   const PrimeInfo*, MdrBconvArgs) {
    if (plan.mont) return plan.centered ? bconv_kernel_m<kMdr, 2>(plan.n_in) : bconv_kernel_m<kMdr, 1>(plan.n_in);
    return bconv_kernel_m<kMdr, 0>(plan.n_in);
}

// ------------------------------------------------------------------ key-switch inner product
// acc[c][0][t] = sum_d ext[c][d][t] * evk[d][0][prime(t)],  acc[c][1][t] = ... * evk[d][1][prime(t)]
// One thread per (c, k, t), the ciphertext index fastest in the grid: the workgroups that read one evk tile run
// back to back, so each XCD fetches the tile once into its L2 and every load of a thread is independent.


__global__ __launch_bounds__(256) void k_ks_inner(const uint64_t* __restrict__ ext, const uint64_t* __restrict__ evk,
                                                  uint64_t* __restrict__ acc, InnerArgs ia,
                                                  const PrimeInfo* __restrict__ primes) {
    const uint32_t c = blockIdx.x, k = blockIdx.y * 256 + threadIdx.x;
    const uint32_t t = ia.t0 + blockIdx.z;
    const uint32_t p = ia.prime_of[t];
    const Barrett br = barrett_of(primes[p]);
    const uint64_t* x = ext + (size_t)c * ia.D * ia.E * kN + (size_t)t * kN + k;
    const uint64_t* e = evk + (size_t)p * kN + k;
    Acc s0, s1;  // at most kMaxDigits = 8 terms: no intermediate fold
    ks_dot<true>(x, (size_t)ia.E * kN, e, (size_t)ia.T * kN, ia.D, s0, s1);  // ext: one ciphertext's, read once
    uint64_t* o = acc + (size_t)c * 2 * ia.E * kN + (size_t)t * kN + k;
    __builtin_nontemporal_store(reduce_u128(s0.get(), br), &o[0]);
    __builtin_nontemporal_store(reduce_u128(s1.get(), br), &o[(size_t)ia.E * kN]);
}

// ------------------------------------------------------------------ ModDown / rescale combines
// out[c][p][i] = (x[c][p][i] - y[c][p][i]) * s_i  (+ add[c][p][i])  mod q_i,   s_i per-limb constant
// The addend, if any, is applied to the polys pc with pc % add_div == 0, read at add + (pc / add_div) *
// add_pstride (add_div = 2 adds c0 of a ciphertext batch to poly 0 of each output ciphertext only).
__global__ __launch_bounds__(256) void k_sub_scale(const uint64_t* __restrict__ x, const uint64_t* __restrict__ y,
                                                   const uint64_t* __restrict__ add, uint64_t* __restrict__ out,
                                                   CombineArgs ca, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;  // pc = poly index over the batch
    const uint64_t q = primes[i].q;
    const size_t li = (size_t)i * kN + k;
    // x, y and out are streamed (nontemporal); the addend may be shared by several polys and is read normally
    const uint64_t d = sub_mod(__builtin_nontemporal_load(&x[pc * ca.x_pstride + li]),
                               __builtin_nontemporal_load(&y[pc * ca.y_pstride + li]), q);
    uint64_t v = shoup(d, ca.s[i].w, ca.s[i].wp, q);
    if (add && pc % ca.add_div == 0) v = add_mod(v, add[(pc / ca.add_group) * ca.add_pstride + li], q);
    __builtin_nontemporal_store(v, &out[pc * ca.out_pstride + li]);
}

// centered lift of the dropped limb (coefficient form) into limbs 0..l-2:
// tmp[pc][i][k] = v > ql/2 ? v - ql (mod q_i) : v (mod q_i)
__global__ __launch_bounds__(256) void k_lift_centered(const uint64_t* __restrict__ last, uint64_t last_pstride,
                                                       uint64_t* __restrict__ tmp, uint32_t n_out, uint64_t ql,
                                                       const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;
    __builtin_nontemporal_store(lift_centered(last[pc * last_pstride + k], ql, barrett_of(primes[i])),
                                &tmp[((size_t)pc * n_out + i) * kN + k]);
}

// ------------------------------------------------------------------ elementwise helpers
// out = x + y mod q over [n_polys][l][N] (limb i uses prime i)
__global__ __launch_bounds__(256) void k_add(const uint64_t* __restrict__ x, const uint64_t* __restrict__ y,
                                             uint64_t* __restrict__ out, uint32_t l,
                                             const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;
    const size_t o = ((size_t)pc * l + i) * kN + k;
    out[o] = add_mod(x[o], y[o], primes[i].q);
}

// evaluation-form automorphism X -> X^g on [n_polys][l][N]: out[k] = in[src(k)],
// src(k) = brev(((g (2 brev(k) + 1)) mod 2N - 1) / 2)
__global__ __launch_bounds__(256) void k_automorph(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                   uint32_t g) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const size_t base = ((size_t)blockIdx.z * gridDim.y + blockIdx.y) * kN;
    const uint32_t e = (uint32_t)(((uint64_t)g * (2u * (__brev(k) >> (32 - kLogN)) + 1u)) & (2u * kN - 1u));
    const uint32_t src = __brev((e - 1u) >> 1) >> (32 - kLogN);
    __builtin_nontemporal_store(__builtin_nontemporal_load(&in[base + src]), &out[base + k]);
}

// ------------------------------------------------------------------ list forms (one key per item)
// acc[c][0/1][t] = sum_d ext_c[d][t] * evk_c[d][0/1][prime(t)] with per-item ext and evk pointers
// (hoisted rotations share one ext; giant-step rotations have one ext each).

// XCD-aware order of a list kernel's one-dimensional grid: workgroups go to the 8 XCDs round-robin (wg mod 8), so
// the m items of one (coefficient tile, limb) tile are given the ids xcd + 8 (blk m + item), all on one XCD: the
// tile's shared ext and evk words are fetched into that XCD's L2 once for all items.  The grid has m * n_tiles
// workgroups (n_tiles a multiple of 8).
struct ListTile {
    uint32_t item, kt, limb;
};

// tiles_per_limb coefficient tiles per limb (kN / 256 for 256-thread tiles)
__device__ __forceinline__ ListTile list_tile(uint32_t m, uint32_t tiles_per_limb = kN / 256) {
    const uint32_t n = blockIdx.x, q = n >> 3, qm = uni_div(q, m);
    const uint32_t tile = qm * 8 + (n & 7);
    return ListTile{q - qm * m, tile % tiles_per_limb, tile / tiles_per_limb};
}

__global__ __launch_bounds__(256) void k_ks_inner_list(ListPtrs ext, ListPtrs evk, uint64_t* __restrict__ acc,
                                                       InnerArgs ia, const PrimeInfo* __restrict__ primes) {
    const ListTile lt = list_tile(ia.B);
    const uint32_t c = lt.item, k = lt.kt * 256 + threadIdx.x;
    const uint32_t t = ia.t0 + lt.limb;
    const uint32_t p = ia.prime_of[t];
    const Barrett br = barrett_of(primes[p]);
    const uint64_t* x = ext.p[c] + (size_t)t * kN + k;
    const uint64_t* e = evk.p[c] + (size_t)p * kN + k;
    Acc s0, s1;  // at most kMaxDigits = 8 terms
    ks_dot(x, (size_t)ia.E * kN, e, (size_t)ia.T * kN, ia.D, s0, s1);
    uint64_t* o = acc + (size_t)c * 2 * ia.E * kN + (size_t)t * kN + k;
    __builtin_nontemporal_store(reduce_u128(s0.get(), br), &o[0]);
    __builtin_nontemporal_store(reduce_u128(s1.get(), br), &o[(size_t)ia.E * kN]);
}

// ModDown combine of a key-switch list with the evk inner product of the Q limbs formed on the fly:
//   out[c][p][i] = x P^-1 - conv[c][p][i]  (+ the addend's poly 0 for p = 0),  x = sum_d ext_c[d][i] evk_c[d][p][i]
// conv [n][2][l][N] is the evaluation form of the P -> Q BConv with P^-1 folded into its table; item c's addend
// is the ciphertext at add + (c / add_group) * add_stride.  Grid: item fastest (hoisted items share ext).
struct PinvArgs {
    TwPair pinv[kMaxPmap];  // P^-1 mod q_i
};

__global__ __launch_bounds__(256) void k_ks_sub_list(ListPtrs ext, ListPtrs evk, const uint64_t* __restrict__ conv,
                                                     const uint64_t* __restrict__ add, uint64_t add_stride,
                                                     uint32_t add_group, uint64_t* __restrict__ out, uint32_t l,
                                                     InnerArgs ia, PinvArgs pa, const PrimeInfo* __restrict__ primes) {
    const ListTile lt = list_tile(ia.B);
    const uint32_t c = lt.item, k = lt.kt * 256 + threadIdx.x, i = lt.limb;
    const Barrett br = barrett_of(primes[i]);
    const uint64_t q = br.q;
    const size_t li = (size_t)i * kN + k;
    const uint64_t* x = ext.p[c] + li;
    const uint64_t* e = evk.p[c] + li;
    Acc s0, s1;
    ks_dot(x, (size_t)ia.E * kN, e, (size_t)ia.T * kN, ia.D, s0, s1);
    const size_t pw = (size_t)l * kN;  // words per poly of conv and out
    const uint64_t* cv = conv + (size_t)c * 2 * pw + li;
    uint64_t* o = out + (size_t)c * 2 * pw + li;
    uint64_t v0 = sub_mod(shoup(reduce_u128(s0.get(), br), pa.pinv[i].w, pa.pinv[i].wp, q),
                          __builtin_nontemporal_load(&cv[0]), q);
    if (add) v0 = add_mod(v0, add[(size_t)(c / add_group) * add_stride + li], q);
    __builtin_nontemporal_store(v0, &o[0]);
    __builtin_nontemporal_store(sub_mod(shoup(reduce_u128(s1.get(), br), pa.pinv[i].w, pa.pinv[i].wp, q),
                                        __builtin_nontemporal_load(&cv[pw]), q),
                                &o[pw]);
}

// ---------------------------------------------------------------- ModDown fused with the following rescale
// The relinearized y_i = add_i + (x_i - NTT(conv_i)) P^-1 and its rescale out_i = (y_i - NTT(lift(z))_i) q_l^-1
// (z the dropped limb l-1 of y in coefficient form) combine, by linearity of the NTT mod q_i, into
//   out_i = (add_i + x_i P^-1 - NTT(T_i)) q_l^-1,  T_i = conv_i P^-1 + lift(z)_i,
//   z = INTT(add_{l-1}) + (INTT(x_{l-1}) - conv_{l-1}) P^-1   (mod q_{l-1}):
// the same words with one forward NTT of l-1 limbs instead of two (l for conv, l-1 for the lift).  The BConv
// writes T directly (k_bconv<NIN, true, ..>); in a relinearization the evk inner product of limbs 0..l-2 is formed inside
// the combine and never stored (the forward NTT of T ends in that combine, k_ntt_fwd_b_mdr in ntt.hip; under the fused
// NTT mode k_mdr_combine_ks follows the NTT).

// out_i = (add_i + x_i P^-1 - T_i) q_{l-1}^-1 in evaluation form, i < l-1
__global__ __launch_bounds__(256) void k_mdr_combine(const uint64_t* __restrict__ x, const uint64_t* __restrict__ add,
                                                     const uint64_t* __restrict__ T, uint64_t* __restrict__ out,
                                                     MdrArgs ma, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x, i = blockIdx.y, pc = blockIdx.z;
    const uint64_t q = primes[i].q;
    const size_t li = (size_t)i * kN + k;
    uint64_t v = shoup(x[pc * ma.x_pstride + li], ma.pinv[i].w, ma.pinv[i].wp, q);
    if (add) v = add_mod(v, add[pc * ma.add_pstride + li], q);
    v = sub_mod(v, T[(size_t)pc * (ma.l - 1) * kN + li], q);
    out[(size_t)pc * (ma.l - 1) * kN + li] = shoup(v, ma.qlinv[i].w, ma.qlinv[i].wp, q);
}

// k_mdr_combine for the relinearization of a batch, x formed on the fly: x[c][p][i] = sum_d ext[c][d][i] *
// evk[d][p][i] (the same sums k_ks_inner would store), then out[c][p][i] = (add + x P^-1 - T) q_{l-1}^-1 for both
// polys p of ciphertext c.  Grid as k_ks_inner: the ciphertext index fastest.
// ta, tb (optional, in place of add): the inputs [B][2][l][N] of the product being relinearized; the addend of
// poly 0 is then d0 = a0 b0 and of poly 1 d1 = a0 b1 + a1 b0, formed here instead of read from the tensor kernel.
__global__ __launch_bounds__(256) void k_mdr_combine_ks(const uint64_t* __restrict__ ext,
                                                        const uint64_t* __restrict__ evk,
                                                        const uint64_t* __restrict__ add,
                                                        const uint64_t* __restrict__ T, uint64_t* __restrict__ out,
                                                        InnerArgs ia, MdrArgs ma, const uint64_t* __restrict__ ta,
                                                        const uint64_t* __restrict__ tb,
                                                        const PrimeInfo* __restrict__ primes) {
    const uint32_t c = blockIdx.x, k = blockIdx.y * 256 + threadIdx.x, i = blockIdx.z;
    const Barrett br = barrett_of(primes[i]);
    const uint64_t q = br.q;
    const size_t po = (size_t)(ma.l - 1) * kN, li = (size_t)i * kN + k;
    const uint64_t* x = ext + (size_t)c * ia.D * ia.E * kN + li;
    const uint64_t* e = evk + li;
    Acc s0, s1;  // at most kMaxDigits = 8 terms: no intermediate fold
    // ext, the addend, T and out are each touched once (nontemporal); the key is shared by the batch
    ks_dot<true>(x, (size_t)ia.E * kN, e, (size_t)ia.T * kN, ia.D, s0, s1);
    const uint64_t xs[2] = {reduce_u128(s0.get(), br), reduce_u128(s1.get(), br)};
    uint64_t dt[2] = {0, 0};
    if (ta) {
        const size_t pw = (size_t)ma.l * kN, o = (size_t)c * 2 * pw + li;
        const uint64_t a0 = __builtin_nontemporal_load(&ta[o]), a1 = __builtin_nontemporal_load(&ta[o + pw]);
        const uint64_t b0 = __builtin_nontemporal_load(&tb[o]), b1 = __builtin_nontemporal_load(&tb[o + pw]);
        Acc u0, u1;
        u0.add(a0, b0);
        u1.add(a0, b1);
        u1.add(a1, b0);
        dt[0] = reduce_u128(u0.get(), br);
        dt[1] = reduce_u128(u1.get(), br);
    }
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const size_t pc = 2 * (size_t)c + p;
        uint64_t v = shoup(xs[p], ma.pinv[i].w, ma.pinv[i].wp, q);
        if (ta) v = add_mod(v, dt[p], q);
        if (add) v = add_mod(v, __builtin_nontemporal_load(&add[pc * ma.add_pstride + li]), q);
        v = sub_mod(v, __builtin_nontemporal_load(&T[pc * po + li]), q);
        __builtin_nontemporal_store(shoup(v, ma.qlinv[i].w, ma.qlinv[i].wp, q), &out[pc * po + li]);
    }
}

// dst[c] = src[c] for up to 64 items of `words` words each (gathers scattered ciphertexts into one batch)
__global__ __launch_bounds__(256) void k_gather(ListPtrs src, uint64_t* __restrict__ dst, uint64_t words) {
    const uint32_t c = blockIdx.y;
    const uint64_t* s = src.p[c];
    uint64_t* d = dst + (size_t)c * words;
    for (uint64_t w = (uint64_t)blockIdx.x * 256 + threadIdx.x; w < words; w += (uint64_t)gridDim.x * 256) d[w] = s[w];
}

// per-ciphertext automorphism index: [n][2][l][N], ciphertext c uses g[c]
struct AutoList {
    uint32_t g[kMaxList];
};

__global__ __launch_bounds__(256) void k_automorph_list(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                        uint32_t l, AutoList al) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;  // pc = 2 c + poly
    const uint32_t g = al.g[pc >> 1];
    const size_t base = ((size_t)pc * l + i) * kN;
    const uint32_t e = (uint32_t)(((uint64_t)g * (2u * (__brev(k) >> (32 - kLogN)) + 1u)) & (2u * kN - 1u));
    const uint32_t src = __brev((e - 1u) >> 1) >> (32 - kLogN);
    __builtin_nontemporal_store(__builtin_nontemporal_load(&in[base + src]), &out[base + k]);
}

// Giant rotations kept in the extended basis Q_l * P, summed per output (double-hoisted BSGS).  Each term's input is a
// giant inner sum S_x = (S0, S1) over Q_l * P encrypting P m; its c1 came down to Q_l once (SQ1 = ModDown(S1)) and
// was extended again (ext_x).  Output c ([2][E][N] at dst + c 2 E N) is the sum over its nt terms j of
//   Auto_g( <ext_x, evk>_0 + S0_x,  <ext_x, evk>_1 )     (a key-switched term: S0 = P SQ0 + r with r = [S0]_P, so
//                                                         this encrypts P Auto_g(m) plus r, which the final ModDown
//                                                         divides by P -- S0 itself needs no ModDown)
//   Auto_g( S0_x, S1_x )                                 (an identity term, evk null)
// with x = (c / A) M + j the term's input (its ModUp extension [D][E][N] at ext + x ext_stride, S_x [2][E][N] at
// src + x src_stride) and key index c % A + j (evk, g).  Output c goes to dst + (u / R) s_hi + (u % R) s_lo,
// u = c + c_off (R = 1, s_hi = 2 E N: contiguous); accumulate adds to it.  The evk inner product is formed at the
// automorphism's source word, so nothing is stored between the key switch and the automorphism; the source words
// of a wave's 64 consecutive outputs are a permutation of one aligned 64-word block (the automorphism multiplies
// the bit-reversed index by an odd g), so the gathers stay coalesced.
// Q_l sources (src_q): the terms' inner sums are ciphertexts over Q_l (a single-hoisted BSGS's giant sums), taken
// into Q_l * P as (P c0, P c1) -- P c mod q_t by the Shoup pair pmod[t], zero on the P limbs -- so that their giant
// rotations share one ModDown.  id_src (any mode; Q_l only with src_q): one more identity term per output c, read
// at id_src + c id_stride (a giant step 0 kept out of the packed terms).
struct QpRotArgs {
    uint32_t l, E, L, D, T, nt, A, M;
    uint32_t n_out, R, c_off, accumulate;
    uint64_t ext_stride, src_stride, s_hi, s_lo;
    uint32_t src_q;
    uint64_t src_poly;  // words between a source's c0 and c1 (E N, or l N with src_q)
    const uint64_t* id_src;
    uint64_t id_stride;
    const uint64_t* evk[kMaxList];
    uint32_t g[kMaxList];
    TwPair pmod[kMaxPmap];  // P mod q_t, t < l (src_q)
};

__global__ __launch_bounds__(256) void k_qp_rot_sum(const uint64_t* __restrict__ ext,
                                                    const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                                    QpRotArgs a, const PrimeInfo* __restrict__ primes) {
    const ListTile lt = list_tile(a.n_out);  // outputs of one tile on one XCD: their ext and evk words meet in L2
    const uint32_t k = lt.kt * 256 + threadIdx.x;
    const uint32_t t = lt.limb, c = lt.item;
    const uint32_t pi = t < a.l ? t : a.L + (t - a.l);
    const Barrett br = barrett_of(primes[pi]);
    const uint64_t q = br.q;
    // a Q_l source has no words on the P limbs (P c = 0 there); on a Q limb its words are scaled by P mod q_t
    const bool src_here = !a.src_q || t < a.l;
    const TwPair pm = a.src_q && t < a.l ? a.pmod[t] : TwPair{0, 0};
    auto src_word = [&](const uint64_t* p) -> uint64_t {
        if (!src_here) return 0;
        return a.src_q ? shoup(p[0], pm.w, pm.wp, q) : p[0];
    };
    uint64_t v0 = 0, v1 = 0;
    for (uint32_t j = 0; j < a.nt; j++) {
        const uint32_t cA = uni_div(c, a.A);
        const uint32_t x = cA * a.M + j, kk = c - cA * a.A + j;
        const uint32_t g = a.g[kk];
        const uint32_t e = (uint32_t)(((uint64_t)g * (2u * (__brev(k) >> (32 - kLogN)) + 1u)) & (2u * kN - 1u));
        const uint32_t sw = __brev((e - 1u) >> 1) >> (32 - kLogN);
        const uint64_t* sx = src + (size_t)x * a.src_stride + (size_t)t * kN + sw;
        const uint64_t* ek = a.evk[kk];
        if (ek) {
            const uint64_t* xe = ext + (size_t)x * a.ext_stride + (size_t)t * kN + sw;
            const uint64_t* ep = ek + (size_t)pi * kN + sw;
            Acc s0, s1;  // at most kMaxDigits = 8 terms
            ks_dot(xe, (size_t)a.E * kN, ep, (size_t)a.T * kN, a.D, s0, s1);
            v0 = add_mod(v0, add_mod(reduce_u128(s0.get(), br), src_word(sx), q), q);
            v1 = add_mod(v1, reduce_u128(s1.get(), br), q);
        } else {
            v0 = add_mod(v0, src_word(sx), q);
            v1 = add_mod(v1, src_word(sx + a.src_poly), q);
        }
    }
    if (a.id_src) {  // the identity term of output c (no automorphism)
        const uint64_t* ix = a.id_src + (size_t)c * a.id_stride + (size_t)t * kN + k;
        v0 = add_mod(v0, src_word(ix), q);
        v1 = add_mod(v1, src_word(ix + a.src_poly), q);
    }
    const uint32_t u = c + a.c_off, uR = uni_div(u, a.R);
    uint64_t* o = dst + (size_t)uR * a.s_hi + (size_t)(u - uR * a.R) * a.s_lo + (size_t)t * kN + k;
    if (a.accumulate) {
        v0 = add_mod(v0, o[0], q);
        v1 = add_mod(v1, o[(size_t)a.E * kN], q);
    }
    __builtin_nontemporal_store(v0, &o[0]);
    __builtin_nontemporal_store(v1, &o[(size_t)a.E * kN]);
}

// BSGS multiply-accumulate: babies [nb][2][l][N], diagonals [n_diag][l][N] (diagonal g*nb + j pairs with
// baby j), out [ng][2][l][N]: out_g = sum_j baby_j (.) diag_{g*nb+j}.
// A workgroup owns 64 coefficients of one limb: it stages those words of every baby in LDS once, then its
// 4 wave-rows take the giant steps g = row, row + 4, ...; every diagonal word is read exactly once and each
// wave reads 64 consecutive words (512 B) per diagonal.
constexpr int kMaxBaby = 64;
constexpr int kMacCoef = 64;  // one wave64 per MAC row
constexpr int kMacRows = 8;

// The giant sums of a BSGS MAC from babies staged in LDS (sb: word kk of baby j, poly p at (2 j + p) kMacCoef + kk):
// out_g = sum_j baby_j (.) diag[g nb_total + j0 + j] for g < ng (out [ng][2][P], diagonals Pd words apart, this
// thread's word at dk in a diagonal and off in an output poly).  Diagonals past n_diag (a short last giant step) are
// zero; acc != 0 adds to what out holds.  A wave row takes two giant steps at a time: four independent accumulation
// chains per thread, and every baby word read from LDS feeds two products.
// Destinations of the giant sums: sum G goes to out + G 2 P, or, with g0 >= 0 (an identity giant step), writing
// G = o ngp + g: sum (o, g0) to id_out + o id_stride and the others to out + (o (ngp - 1) + g - [g > g0]) 2 P.
struct GiantMap {
    uint32_t ngp;
    int32_t g0;
    uint64_t* id_out;
    uint64_t id_stride;
};

__device__ __forceinline__ void mac_giants(const uint64_t* sb, const uint64_t* __restrict__ diag,
                                           uint64_t* __restrict__ out, uint32_t nb, uint32_t nb_total, uint32_t j0,
                                           uint32_t ng, uint32_t n_diag, size_t P, size_t Pd, size_t dk, size_t off,
                                           uint32_t acc, const Barrett& br, uint32_t kk, uint32_t row,
                                           const GiantMap& gm = GiantMap{1, -1, nullptr, 0}) {
    auto count = [&](uint32_t g) {
        const int64_t rem = (int64_t)n_diag - (int64_t)g * nb_total - j0;
        return rem <= 0 ? 0u : (uint32_t)min<int64_t>(rem, nb);
    };
    auto store = [&](uint32_t g, Acc& a0, Acc& a1) {
        uint64_t* o = out + (size_t)g * 2 * P + off;
        if (gm.g0 >= 0) {
            const uint32_t oi = g / gm.ngp, gi = g - oi * gm.ngp;
            if (gi == (uint32_t)gm.g0)
                o = gm.id_out + (size_t)oi * gm.id_stride + off;
            else
                o = out + ((size_t)oi * (gm.ngp - 1) + gi - (gi > (uint32_t)gm.g0 ? 1 : 0)) * 2 * P + off;
        }
        uint64_t r0 = reduce_u128(a0.get(), br), r1 = reduce_u128(a1.get(), br);
        if (acc) {
            r0 = add_mod(r0, o[0], br.q);
            r1 = add_mod(r1, o[P], br.q);
        }
        __builtin_nontemporal_store(r0, &o[0]);
        __builtin_nontemporal_store(r1, &o[P]);
    };
    for (uint32_t g = row; g < ng; g += 2 * kMacRows) {
        const uint32_t g2 = g + kMacRows;
        const uint32_t jn1 = count(g), jn2 = g2 < ng ? count(g2) : 0u;  // jn2 <= jn1
        const uint64_t* d1 = diag + ((size_t)g * nb_total + j0) * Pd + dk;
        const uint64_t* d2 = diag + ((size_t)g2 * nb_total + j0) * Pd + dk;
        Acc a0, a1, b0, b1;
        // 8 babies at a time: their diagonal words are all requested before the first product waits
        for (uint32_t j0 = 0; j0 < jn2; j0 += 8) {
            uint64_t m1[8], m2[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (j0 + u < jn2) {
                    m1[u] = d1[(size_t)(j0 + u) * Pd];
                    m2[u] = d2[(size_t)(j0 + u) * Pd];
                }
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (j0 + u < jn2) {
                    const uint32_t j = j0 + u;
                    const uint64_t x0 = sb[(2 * j) * kMacCoef + kk], x1 = sb[(2 * j + 1) * kMacCoef + kk];
                    a0.add(x0, m1[u]);
                    a1.add(x1, m1[u]);
                    b0.add(x0, m2[u]);
                    b1.add(x1, m2[u]);
                }
            }
            a0.fold();
            a1.fold();
            b0.fold();
            b1.fold();
        }
        for (uint32_t j0 = jn2; j0 < jn1; j0 += 8) {
            uint64_t m1[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (j0 + u < jn1) m1[u] = d1[(size_t)(j0 + u) * Pd];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (j0 + u < jn1) {
                    const uint32_t j = j0 + u;
                    a0.add(sb[(2 * j) * kMacCoef + kk], m1[u]);
                    a1.add(sb[(2 * j + 1) * kMacCoef + kk], m1[u]);
                }
            }
            a0.fold();
            a1.fold();
        }
        store(g, a0, a1);
        if (g2 < ng) store(g2, b0, b1);
    }
}

// log_rep > 0: the diagonals are compressed periodic plaintexts, [n_diag][l][N >> log_rep], whose
// evaluation-form word k is comp[k >> log_rep] (the reference's store expansion, gpu_real_model.cu:145-155).
// Babies j0 .. j0 + nb - 1 of a list of nb_total are taken, each a ciphertext [2][l][N] anywhere in memory (baby.p,
// so the rotated babies are read where the rotations wrote them; diagonal g * nb_total + j, zero from n_diag on);
// acc != 0 adds the result to what out holds (the MAC over more babies than fit in LDS runs in baby chunks).
// n_inst instances share the diagonals: instance s takes its babies at baby.p[j] + s inst_stride and writes
// out + s out_stride; the instances of one (coefficient tile, limb) run on one XCD (list_tile), so each diagonal
// word is fetched from HBM once for all of them.
__global__ __launch_bounds__(kMacCoef* kMacRows) void k_bsgs_mac(ListPtrs baby,
                                                                  const uint64_t* __restrict__ diag,
                                                                  uint64_t* __restrict__ out, uint32_t nb,
                                                                  uint32_t nb_total, uint32_t j0, uint32_t ng,
                                                                  uint32_t n_diag, uint32_t l, uint32_t log_rep,
                                                                  uint32_t acc, uint32_t l_q, uint32_t Lp,
                                                                  uint32_t n_inst, uint64_t inst_stride,
                                                                  uint64_t out_stride,
                                                                  const PrimeInfo* __restrict__ primes) {
    extern __shared__ uint64_t sb[];
    const ListTile lt = list_tile(n_inst, kN / kMacCoef);
    // a row is one wave (kMacCoef = 64 lanes): its index, and every baby / giant index derived from it, is wave-uniform
    // and lives in scalar registers (left to the compiler, the per-baby division and addressing ran on the VALU)
    const uint32_t kk = threadIdx.x & (kMacCoef - 1), row = __builtin_amdgcn_readfirstlane(threadIdx.x / kMacCoef);
    const uint32_t k = lt.kt * kMacCoef + kk;
    const uint32_t i = lt.limb;  // limb; limbs from l_q on are P limbs (prime Lp + i - l_q)
    const Barrett br = barrett_of(primes[i < l_q ? i : Lp + (i - l_q)]);
    const size_t P = (size_t)l * kN, off = (size_t)i * kN + k;
    const size_t so = (size_t)lt.item * inst_stride;
    out += (size_t)lt.item * out_stride;
    for (uint32_t jp = row; jp < 2 * nb; jp += kMacRows) {  // jp = 2 j + poly; baby j of this chunk at baby.p[j]
        const uint32_t j = jp >> 1, p = jp & 1;
        sb[jp * kMacCoef + kk] = baby.p[j][so + p * P + off];
    }
    __syncthreads();
    mac_giants(sb, diag, out, nb, nb_total, j0, ng, n_diag, P, (size_t)l * (kN >> log_rep),
               (size_t)i * (kN >> log_rep) + (k >> log_rep), off, acc, br, kk, row);
}

// Double-hoisted BSGS MAC: the babies are formed in LDS from the inputs' ModUp extensions and never stored.  Over
// Q_l * P (E limbs), baby j = i nb + b of instance s is the rotation of input x = s n_in + i by baby step b kept in
// the extended basis (see k_qp_rot_sum): Auto_b(<ext_x, evk_b> + (P c0_x, 0)), or (P c0_x, P c1_x) for b's
// identity step; then the giant sums sum_j baby_j (.) diag[G nbt + j] as in k_bsgs_mac (diagonals [n_diag][E][N],
// shared by the instances, whose workgroups of one tile run on one XCD), G = o ngp + g.  The sums of the identity
// giant step g0 need no rotation: they go to id_out (where the giant rotations are later added), the others to
// out_s [n_out][ngp - 1][2][E][N] (all ngp when g0 < 0).
constexpr int kMaxDhBaby = 32;

// Coefficient tile order for rotations by multiples of delta slots.  Tile kt (64 consecutive evaluation words) is the
// odd residue u = 2 brev10(kt) + 1 mod 2048, and the automorphism X -> X^g maps it onto the tile of g u mod 2048
// (the words stay in their aligned 64-word block, permuted).  With the babies' g_b = 5^(b delta), tile u reads the
// blocks u 5^(b delta): ordering the tiles along the chains u0 5^(delta m) makes consecutive tiles read nearly the same
// blocks (15 of 16 for 16 babies), so a baby input's words come from L2 instead of HBM.  The odd residues are
// +-5^a (a < 512); the chains are the cosets +-5^a <5^delta>, a < min(delta, 512).  Position pos in [0, 1024) of the
// order -> tile kt; delta = 0 keeps kt = pos.
__device__ __forceinline__ uint32_t chain_tile(uint32_t pos, uint32_t delta) {
    if (delta == 0) return pos;
    const uint32_t d = delta >= 512 ? 512u : delta;         // 5 has order 512 mod 2048
    const uint32_t len = 512u / d;                           // chain length
    const uint32_t c = pos / len, m = pos - c * len;
    const uint32_t per_sign = 512u / len;                    // chains per sign (= d)
    const uint32_t neg = c / per_sign, a = c - neg * per_sign;
    uint32_t e = (a + (uint32_t)(((uint64_t)delta * m) & 511u)) & 511u;
    uint32_t u = 1, b = 5;
    for (; e; e >>= 1) {
        if (e & 1) u = (u * b) & 2047u;
        b = (b * b) & 2047u;
    }
    if (neg) u = (2048u - u) & 2047u;
    return __brev((u - 1u) >> 1) >> 22;                      // brev10((u - 1) / 2)
}

struct DhMacArgs {
    uint32_t l, E, L, D, T;          // Q limbs, extended limbs, first P prime, digits, evk limbs per poly
    uint32_t n_in, nb, ng, n_diag, n_inst;
    uint32_t ngp;                     // giant steps per output (ng = n_out ngp)
    int32_t g0;                       // the identity giant step (or -1): its sums go to id_out
    uint32_t chain_delta;             // baby steps b chain_delta (0: not an arithmetic progression)
    uint64_t ext_stride, src_stride;  // per input x
    uint64_t out_stride;              // per instance
    uint64_t* id_out;
    uint64_t id_inst_stride, id_stride;  // id_out: per instance, per output
    const uint64_t* evk[kMaxDhBaby];  // per baby step (null: the identity)
    uint32_t g[kMaxDhBaby];
    // P R^-1 mod q_t, t < l (R = 2^64): the babies are kept R^-1-scaled -- their inner products are Montgomery-reduced
    // (one REDC each instead of a Barrett reduction) -- and each giant sum is scaled back by R (PrimeInfo.r_mod)
    TwPair pmod[kMaxPmap];
};

// ND: the digit count (a template parameter, so that a baby's extension and key loads are all issued before the
// first product waits on them).
template <int ND>
__global__ __launch_bounds__(kMacCoef* kMacRows) void k_bsgs_dh_mac(const uint64_t* __restrict__ ext,
                                                                     const uint64_t* __restrict__ src,
                                                                     const uint64_t* __restrict__ diag,
                                                                     uint64_t* __restrict__ out, DhMacArgs a,
                                                                     const PrimeInfo* __restrict__ primes) {
    extern __shared__ uint64_t sb[];
    // XCD x (workgroups x mod 8) takes one contiguous run of the (limb, chain-ordered tile) sequence; the instances of
    // a tile follow each other on it (they share the tile's keys and diagonals)
    const uint32_t xcd = blockIdx.x & 7, qi = blockIdx.x >> 3;
    const uint32_t qn = uni_div(qi, a.n_inst);
    const uint32_t s = qi - qn * a.n_inst, seq = xcd * (a.E * (kN / kMacCoef) / 8) + qn;
    const uint32_t t = seq / (kN / kMacCoef);
    // a row is one wave (kMacCoef = 64 lanes): its index, and every baby / giant index derived from it, is wave-uniform
    // and lives in scalar registers (left to the compiler, the per-baby division and addressing ran on the VALU)
    const uint32_t kk = threadIdx.x & (kMacCoef - 1), row = __builtin_amdgcn_readfirstlane(threadIdx.x / kMacCoef);
    const uint32_t k = chain_tile(seq % (kN / kMacCoef), a.chain_delta) * kMacCoef + kk;
    const bool qlimb = t < a.l;
    const uint32_t pi = qlimb ? t : a.L + (t - a.l);
    const Barrett br = barrett_of(primes[pi]);
    const uint64_t q = br.q, ninv = primes[pi].mont_ninv;
    const uint32_t nbt = a.n_in * a.nb;
    for (uint32_t j = row; j < nbt; j += kMacRows) {
        const uint32_t i = j / a.nb, b = j - i * a.nb, x = s * a.n_in + i;
        const uint32_t g = a.g[b];
        const uint32_t e = (uint32_t)(((uint64_t)g * (2u * (__brev(k) >> (32 - kLogN)) + 1u)) & (2u * kN - 1u));
        const uint32_t sw = __brev((e - 1u) >> 1) >> (32 - kLogN);
        const uint64_t* sx = src + (size_t)x * a.src_stride + (size_t)t * kN + sw;
        const uint64_t* ek = a.evk[b];
        uint64_t v0 = 0, v1 = 0;
        if (ek) {
            const uint64_t* xe = ext + (size_t)x * a.ext_stride + (size_t)t * kN + sw;
            const uint64_t* ep = ek + (size_t)pi * kN + sw;
            uint64_t xv[ND], e0[ND], e1[ND];
#pragma unroll
            for (int d = 0; d < ND; d++) {
                xv[d] = xe[(size_t)d * a.E * kN];
                e0[d] = ep[((size_t)d * 2 + 0) * a.T * kN];
                e1[d] = ep[((size_t)d * 2 + 1) * a.T * kN];
            }
            const uint64_t c0 = qlimb ? sx[0] : 0;
            Acc s0, s1;  // at most kMaxDigits = 8 terms
#pragma unroll
            for (int d = 0; d < ND; d++) {
                s0.add(xv[d], e0[d]);
                s1.add(xv[d], e1[d]);
            }
            // P c0 joins the poly-0 sum (P mod q_t times c0: the REDC below takes the whole sum to R^-1 scale, the
            // baby's form), instead of a Shoup product by P R^-1 and a modular add after it.  REDC: sums of at most
            // 9 products of residues below q < 2^60 stay below q 2^64; the accumulator folds its cross sums first
            // when 8 terms are already in
            if (qlimb) {
                if (ND >= 8) s0.fold();
                s0.add(c0, primes[pi].pmod);
            }
            v0 = s0.redc(q, ninv);
            v1 = s1.redc(q, ninv);
        } else if (qlimb) {
            v0 = shoup(sx[0], a.pmod[t].w, a.pmod[t].wp, q);
            v1 = shoup(sx[(size_t)a.l * kN], a.pmod[t].w, a.pmod[t].wp, q);
        }
        sb[(2 * j) * kMacCoef + kk] = v0;
        sb[(2 * j + 1) * kMacCoef + kk] = v1;
    }
    __syncthreads();
    // giant sums: with fewer giants than rows, each giant's babies are split over kMacRows / ng rows (slices) whose
    // partial sums meet in LDS, so every row works
    const size_t P = (size_t)a.E * kN, off = (size_t)t * kN + k;
    const uint32_t slices = a.ng < (uint32_t)kMacRows ? kMacRows / a.ng : 1u;
    uint64_t* part = sb + (size_t)2 * nbt * kMacCoef;  // [kMacRows][2][kMacCoef]
    out += (size_t)s * a.out_stride;
    uint64_t* id_out = a.g0 >= 0 ? a.id_out + (size_t)s * a.id_inst_stride : nullptr;
    auto dest = [&](uint32_t G) {
        if (a.g0 < 0) return out + (size_t)G * 2 * P + off;
        const uint32_t oi = G / a.ngp, gi = G - oi * a.ngp;
        if (gi == (uint32_t)a.g0) return id_out + (size_t)oi * a.id_stride + off;
        return out + ((size_t)oi * (a.ngp - 1) + gi - (gi > (uint32_t)a.g0 ? 1 : 0)) * 2 * P + off;
    };
    const uint32_t per = (nbt + slices - 1) / slices;
    for (uint32_t G0 = 0; G0 < a.ng; G0 += kMacRows / slices) {
        const uint32_t G = G0 + row % (kMacRows / slices), sl = row / (kMacRows / slices);
        uint64_t r0 = 0, r1 = 0;
        if (G < a.ng) {
            const uint32_t j_lo = sl * per, j_hi = min(nbt, j_lo + per);
            const int64_t rem = (int64_t)a.n_diag - (int64_t)G * nbt;  // diagonals past n_diag are zero
            const uint32_t j_end = rem <= 0 ? 0u : min<uint32_t>(j_hi, (uint32_t)min<int64_t>(rem, nbt));
            const uint64_t* d = diag + (size_t)G * nbt * P + off;
            Acc s0, s1;
            // 8 babies at a time: their diagonal words are all requested before the first product waits
            for (uint32_t j0 = j_lo; j0 < j_end; j0 += 8) {
                uint64_t m[8];
#pragma unroll
                for (int u = 0; u < 8; u++) m[u] = j0 + u < j_end ? d[(size_t)(j0 + u) * P] : 0;
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    if (j0 + u < j_end) {
                        const uint32_t j = j0 + u;
                        s0.add(sb[(2 * j) * kMacCoef + kk], m[u]);
                        s1.add(sb[(2 * j + 1) * kMacCoef + kk], m[u]);
                    }
                }
                s0.fold();
                s1.fold();
            }
            r0 = reduce_u128(s0.get(), br);
            r1 = reduce_u128(s1.get(), br);
        }
        if (slices > 1) {
            part[(2 * row) * kMacCoef + kk] = r0;
            part[(2 * row + 1) * kMacCoef + kk] = r1;
            __syncthreads();
            if (sl == 0 && G < a.ng) {
                for (uint32_t o = 1; o < slices; o++) {
                    const uint32_t rr = row + o * (kMacRows / slices);
                    r0 = add_mod(r0, part[(2 * rr) * kMacCoef + kk], q);
                    r1 = add_mod(r1, part[(2 * rr + 1) * kMacCoef + kk], q);
                }
            }
            __syncthreads();
        }
        if (sl == 0 && G < a.ng) {
            // the babies' R^-1 taken back out
            const uint64_t rm = primes[pi].r_mod, rmp = primes[pi].r_mod_p;
            uint64_t* o = dest(G);
            __builtin_nontemporal_store(shoup(r0, rm, rmp, q), &o[0]);
            __builtin_nontemporal_store(shoup(r1, rm, rmp, q), &o[P]);
        }
    }
}

// Masked pairs: out[s][t] = pt[s][t][0] (.) R[t] + pt[s][t][1] (.) R[n + t] on both polys, with
// R [2n][2][l][N] and pt [n_sets][n][2][l][N >> log_rep] compressed periodic plaintexts.
__global__ __launch_bounds__(256) void k_pair_mac(const uint64_t* __restrict__ R, const uint64_t* __restrict__ pt,
                                                  uint64_t* __restrict__ out, uint32_t n, uint32_t l,
                                                  uint32_t log_rep, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, z = blockIdx.z;  // z = (s n + t) 2 + poly
    const uint32_t poly = z & 1, st = z >> 1, t = st % n;
    const Barrett br = barrett_of(primes[i]);
    const size_t P = (size_t)l * kN, Pc = (size_t)l * (kN >> log_rep);
    const size_t w = (size_t)poly * P + (size_t)i * kN + k;
    const uint64_t* p = pt + (size_t)st * 2 * Pc + (size_t)i * (kN >> log_rep) + (k >> log_rep);
    Acc s;
    s.add(R[(size_t)t * 2 * P + w], p[0]);
    s.add(R[(size_t)(n + t) * 2 * P + w], p[Pc]);
    out[(size_t)st * 2 * P + w] = reduce_u128(s.get(), br);
}

// ct (.) pt on both polys: ct [B][2][l][N], pt [B or 1][l][N >> log_rep] (pt_bstride 0 = shared plaintext;
// log_rep > 0 = compressed periodic plaintext, word k of the evaluation form is comp[k >> log_rep])
__global__ __launch_bounds__(256) void k_mul_plain(const uint64_t* __restrict__ ct, const uint64_t* __restrict__ pt,
                                                   uint64_t* __restrict__ out, uint32_t l, uint64_t pt_bstride,
                                                   uint32_t log_rep, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;
    const Barrett br = barrett_of(primes[i]);
    const size_t o = ((size_t)pc * l + i) * kN + k;
    const uint64_t m = pt[(size_t)(pc >> 1) * pt_bstride + (size_t)i * (kN >> log_rep) + (k >> log_rep)];
    out[o] = mul_mod(ct[o], m, br);
}

// c0 + pt: ct [B][2][l][N]; out gets (c0 + m, c1)
__global__ __launch_bounds__(256) void k_add_plain(const uint64_t* __restrict__ ct, const uint64_t* __restrict__ pt,
                                                   uint64_t* __restrict__ out, uint32_t l, uint64_t pt_bstride,
                                                   const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;
    const size_t o = ((size_t)pc * l + i) * kN + k;
    uint64_t v = ct[o];
    if ((pc & 1) == 0) v = add_mod(v, pt[(size_t)(pc >> 1) * pt_bstride + (size_t)i * kN + k], primes[i].q);
    out[o] = v;
}

// out = sum of n inputs, each [n_polys][l][N]
__global__ __launch_bounds__(256) void k_sum_list(ListPtrs in, uint32_t n, uint64_t* __restrict__ out, uint32_t l,
                                                  const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;
    const uint64_t q = primes[i].q;
    const size_t o = ((size_t)pc * l + i) * kN + k;
    uint64_t acc = 0;
    for (uint32_t j0 = 0; j0 < n; j0 += 8) {  // 8 words requested together
        uint64_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j0 + u < n) v[u] = in.p[j0 + u][o];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j0 + u < n) acc = add_mod(acc, v[u], q);
    }
    out[o] = acc;
}

// Integer linear combination over ciphertext batches:
//   out[c][p][i] = sum_t C[t][i] * x_t[c][p][i]  (+ add[i] on poly 0)   mod q_i,   i < l_out
// Term t reads ciphertext c at x_t + c * 2 * stride_t * N (stride_t = the term's own limb count, so a term
// at a higher level is read without copying; only its first l_out limbs are used).
constexpr int kMaxTerms = 8;
constexpr int kMaxLcLimbs = 40;

struct LinArgs {
    const uint64_t* x[kMaxTerms];
    uint32_t stride[kMaxTerms];
    uint32_t n_terms, l_out, has_add;
    uint32_t i0;  // limbs i0 .. i0 + l_out - 1 are formed (out holds l_out limbs per poly; C and add are per out limb)
    uint64_t C[kMaxTerms][kMaxLcLimbs];
    uint64_t add[kMaxLcLimbs];
};

__global__ __launch_bounds__(256) void k_lincomb(uint64_t* __restrict__ out, LinArgs la,
                                                 const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t j = blockIdx.y, i = la.i0 + j, pc = blockIdx.z;  // out limb j is limb i; pc = 2 c + poly
    const uint32_t c = pc >> 1, p = pc & 1;
    const Barrett br = barrett_of(primes[i]);
    Acc acc;  // at most kMaxTerms = 8 terms
    uint64_t v[kMaxTerms];  // every term's word requested before the first product waits
#pragma unroll
    for (int t = 0; t < kMaxTerms; t++)
        if (t < (int)la.n_terms) v[t] = la.x[t][((size_t)(2 * c + p) * la.stride[t] + i) * kN + k];
#pragma unroll
    for (int t = 0; t < kMaxTerms; t++)
        if (t < (int)la.n_terms) acc.add(v[t], la.C[t][j]);
    // the coefficients carry a factor R = 2^64 (C R mod q_i), so the REDC of the sum is the combination itself;
    // at most 8 products of residues below q < 2^60 keep the sum below q R
    uint64_t r = acc.redc(br.q, primes[i].mont_ninv);
    if (la.has_add && p == 0) r = add_mod(r, la.add[j], br.q);
    __builtin_nontemporal_store(r, &out[((size_t)pc * la.l_out + j) * kN + k]);
}

// multiply by X^(N/2) (slot-wise by +-i): evaluation slot k holds a(psi^(2 brev(k)+1)); X^(N/2) there is
// psi^(N/2 (2 brev(k)+1)) = +iq for k < N/2 and -iq for k >= N/2 (iq = psi^(N/2) = forward-table entry 1).
// sign = 1 multiplies by X^(N/2), sign = -1 by -X^(N/2).
__global__ __launch_bounds__(256) void k_mul_i(const uint64_t* __restrict__ in, uint64_t* __restrict__ out, uint32_t l,
                                               int sign, const TwPair* __restrict__ tw_all,
                                               const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y, pc = blockIdx.z;
    const uint64_t q = primes[i].q;
    const TwPair w = tw_all[(size_t)i * kN + 1];
    const size_t o = ((size_t)pc * l + i) * kN + k;
    uint64_t v = shoup(in[o], w.w, w.wp, q);
    const bool neg = (k >= kN / 2) != (sign < 0);
    out[o] = (neg && v) ? q - v : v;
}

}  // namespace

// ------------------------------------------------------------------ launchers
hipError_t launch_tensor(const Context& ctx, const uint64_t* a, const uint64_t* b, uint64_t* d01, uint64_t* d2,
                         uint32_t B, uint32_t l, uint64_t* d2e, uint64_t d2e_bstride, const uint32_t* ext_off,
                         hipStream_t st, uint32_t t0) {
    if (t0 >= l || (d2e && !d2)) return hipErrorInvalidValue;
    TensorArgs ta{};
    ta.l = l;
    ta.B = B;
    ta.t0 = t0;
    ta.d2e = d2e;
    ta.d2e_bstride = d2e_bstride;
    if (d2e)
        for (uint32_t t = 0; t < l; t++) ta.ext_off[t] = ext_off[t];
    // per limb: inputs read, d0 and d1 written, d2 (and its copy) written
    const double per = 4.0 + 2.0 + (d2 ? 1.0 : 0.0) + (d2e ? 1.0 : 0.0);
    const int pi = prof_begin(ctx, "tensor", (double)B * (l - t0) * per * kN * 8, st);
    hipLaunchKernelGGL(k_tensor, dim3(kN / 256, l - t0, B), dim3(256), 0, st, a, b, d01, d2, ta, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

static BConvArgs bconv_args(const BConvPlan& plan, uint64_t in_bstride, const uint32_t* in_off, uint64_t out_bstride,
                            const uint32_t* out_off, uint32_t n_written) {
    BConvArgs ba{};
    ba.n_in = plan.n_in;
    ba.n_out = plan.n_out;
    ba.centered = plan.centered ? 1 : 0;
    ba.mont = plan.mont ? 1 : 0;
    ba.in_bstride = in_bstride;
    ba.out_bstride = out_bstride;
    for (uint32_t i = 0; i < plan.n_in; i++) ba.in_desc[i] = (in_off[i] & 0xFFFFu) | ((uint32_t)plan.in_idx[i] << 16);
    for (uint32_t j = 0; j < plan.n_out; j++)
        ba.out_desc[j] = ((j < n_written ? out_off[j] : 0u) & 0xFFFFu) | ((uint32_t)plan.out_idx[j] << 16);
    return ba;
}

hipError_t launch_bconv(const Context& ctx, const BConvPlan& plan, const uint64_t* in, uint64_t in_bstride,
                        const uint32_t* in_off, uint64_t* out, uint64_t out_bstride, const uint32_t* out_off,
                        uint32_t B, hipStream_t st) {
    if (plan.n_in == 0 || plan.n_in > (uint32_t)kMaxBconvIn || plan.n_out > (uint32_t)kMaxBconvOut)
        return hipErrorInvalidValue;
    const BConvArgs ba = bconv_args(plan, in_bstride, in_off, out_bstride, out_off, plan.n_out);
    const int pi = prof_begin(ctx, "bconv", (double)B * (plan.n_in + plan.n_out) * kN * 8, st);
    hipLaunchKernelGGL(bconv_kernel<false>(plan), dim3(kN / 256, B, bconv_split(B, plan.n_out)), dim3(256), 0, st,
                       in, out, ba, plan.d_tab, ctx.d_primes, MdrBconvArgs{});
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// ModDown BConv fused with the rescale's lift (plan from bconv_plan with the P^-1 column scaling, outputs
// 0..l-1 with l-1 last): in [n_polys] polys of stride in_bstride holding the P limbs (coefficient form) at
// in_off; xlast = limb l-1 of the same polys (coefficient form); T [n_polys][l-1][N].
hipError_t launch_bconv_mdr(const Context& ctx, const BConvPlan& plan, const uint64_t* in, uint64_t in_bstride,
                            const uint32_t* in_off, uint64_t* T, uint32_t n_polys, const uint64_t* xlast,
                            uint64_t xlast_pstride, const uint64_t* addc, TwPair pinv_last, hipStream_t st) {
    if (plan.n_in == 0 || plan.n_in > (uint32_t)kMaxBconvIn || plan.n_out > (uint32_t)kMaxBconvOut || plan.n_out < 2)
        return hipErrorInvalidValue;
    const uint32_t l = plan.n_out;
    std::vector<uint32_t> out_off(l - 1);
    for (uint32_t j = 0; j + 1 < l; j++) out_off[j] = j;
    const BConvArgs ba = bconv_args(plan, in_bstride, in_off, (uint64_t)(l - 1) * kN, out_off.data(), l - 1);
    MdrBconvArgs mb{};
    mb.xlast = xlast;
    mb.xlast_pstride = xlast_pstride;
    mb.addc = addc;
    mb.pinv_last = pinv_last;
    const uint64_t ql = ctx.moduli[plan.out_idx[l - 1]];
    mb.fast_lift = 1;
    for (uint32_t j = 0; j + 1 < l; j++) {
        const uint64_t qj = ctx.moduli[plan.out_idx[j]];
        if (ql > 2 * qj) mb.fast_lift = 0;  // the fast lift's [0, 3q_j) needs q_{l-1} <= 2 q_j
        mb.dl[j] = (qj - ql % qj) % qj;
        // the NTT's 8q input bound must hold in 64 bits too: 5 q_j < 2^64
        if (qj > (~0ull) / kNttFwdInputBound) return hipErrorInvalidValue;
    }
    // P limbs + limb l-1 (+ the addend's) read, l-1 limbs written
    const double bytes = (double)n_polys * (plan.n_in + 1 + (addc ? 1 : 0) + (l - 1)) * kN * 8;
    const int pi = prof_begin(ctx, "bconv_mdr", bytes, st);
    hipLaunchKernelGGL(bconv_kernel<true>(plan), dim3(kN / 256, n_polys), dim3(256), 0, st, in, T, ba, plan.d_tab,
                       ctx.d_primes, mb);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

static InnerArgs inner_args(const Context& ctx, uint32_t l, uint32_t B) {
    InnerArgs ia{};
    ia.E = l + ctx.K;
    ia.D = (l + ctx.alpha - 1) / ctx.alpha;
    ia.T = ctx.L + ctx.K;
    ia.B = B;
    for (uint32_t t = 0; t < ia.E && t < kMaxPmap; t++) ia.prime_of[t] = (uint8_t)(t < l ? t : ctx.L + (t - l));
    return ia;
}

// evk inner product of the extended limbs t0..E-1 (t0 > 0 when the combine forms the others itself)
hipError_t launch_ks_inner(const Context& ctx, const uint64_t* ext, const uint64_t* evk, uint64_t* acc, uint32_t B,
                           uint32_t l, hipStream_t st, uint32_t t0) {
    ctx.n_keyswitch += B;
    InnerArgs ia = inner_args(ctx, l, B);
    if (ia.D > (uint32_t)kMaxDigits || ia.E > kMaxPmap || t0 >= ia.E) return hipErrorInvalidValue;
    ia.t0 = t0;
    const uint32_t nt = ia.E - t0;
    // ext read once per ciphertext, acc written once, the evk limbs of the level read once
    const double bytes = ((double)B * (ia.D * nt + 2 * nt) + 2.0 * ia.D * nt) * kN * 8;
    const int pi = prof_begin(ctx, "ks_inner", bytes, st);
    hipLaunchKernelGGL(k_ks_inner, dim3(B, kN / 256, nt), dim3(256), 0, st, ext, evk, acc, ia, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_sub_scale(const Context& ctx, const uint64_t* x, uint64_t x_pstride, const uint64_t* y,
                            uint64_t y_pstride, const uint64_t* add, uint64_t add_pstride, uint32_t add_div,
                            uint64_t* out, uint64_t out_pstride, uint32_t n_polys, uint32_t l, const TwPair* s,
                            hipStream_t st, uint32_t add_group) {
    CombineArgs ca{};
    ca.l = l;
    ca.add_div = add_div ? add_div : 1;
    ca.add_group = add_group ? add_group : ca.add_div;
    ca.x_pstride = x_pstride;
    ca.y_pstride = y_pstride;
    ca.out_pstride = out_pstride;
    ca.add_pstride = add_pstride;
    for (uint32_t i = 0; i < l; i++) ca.s[i] = s[i];
    const double n_add = add ? (double)n_polys / ca.add_div : 0.0;
    const int pi = prof_begin(ctx, "sub_scale", ((double)n_polys * 3 + n_add) * l * kN * 8, st);
    hipLaunchKernelGGL(k_sub_scale, dim3(kN / 256, l, n_polys), dim3(256), 0, st, x, y, add, out, ca, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_lift_centered(const Context& ctx, const uint64_t* last, uint64_t last_pstride, uint64_t* tmp,
                                uint32_t n_polys, uint32_t n_out, uint64_t ql, hipStream_t st) {
    const int pi = prof_begin(ctx, "lift_centered", (double)n_polys * (1 + n_out) * kN * 8, st);
    hipLaunchKernelGGL(k_lift_centered, dim3(kN / 256, n_out, n_polys), dim3(256), 0, st, last, last_pstride, tmp,
                       n_out, ql, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_add(const Context& ctx, const uint64_t* x, const uint64_t* y, uint64_t* out, uint32_t n_polys,
                      uint32_t l, hipStream_t st) {
    const int pi = prof_begin(ctx, "add", (double)n_polys * l * 3 * kN * 8, st);
    hipLaunchKernelGGL(k_add, dim3(kN / 256, l, n_polys), dim3(256), 0, st, x, y, out, l, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_ks_inner_list(const Context& ctx, const uint64_t* const* ext, const uint64_t* const* evk,
                                uint64_t* acc, uint32_t n, uint32_t l, hipStream_t st, uint32_t t0) {
    ctx.n_keyswitch += n;
    InnerArgs ia = inner_args(ctx, l, n);
    if (ia.D > (uint32_t)kMaxDigits || ia.E > kMaxPmap || n > (uint32_t)kMaxList || t0 >= ia.E)
        return hipErrorInvalidValue;
    ia.t0 = t0;
    const uint32_t nt = ia.E - t0;
    ListPtrs pe{}, pk{};
    uint32_t distinct_ext = 0;
    for (uint32_t c = 0; c < n; c++) {
        pe.p[c] = ext[c];
        pk.p[c] = evk[c];
        distinct_ext += (c == 0 || ext[c] != ext[c - 1]) ? 1 : 0;
    }
    const double bytes = ((double)distinct_ext * ia.D * nt + (double)n * (2 * ia.D * nt + 2 * nt)) * kN * 8;
    const int pi = prof_begin(ctx, "ks_inner_list", bytes, st);
    hipLaunchKernelGGL(k_ks_inner_list, dim3(n * (kN / 256) * nt), dim3(256), 0, st, pe, pk, acc, ia, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// out [n][2][l][N] = ModDown combine of a key-switch list (k_ks_sub_list); conv [n][2][l][N] evaluation form
hipError_t launch_ks_sub_list(const Context& ctx, const uint64_t* const* ext, const uint64_t* const* evk,
                              const uint64_t* conv, const uint64_t* add, uint64_t add_stride, uint32_t add_group,
                              uint64_t* out, uint32_t n, uint32_t l, const TwPair* pinv, hipStream_t st) {
    InnerArgs ia = inner_args(ctx, l, n);
    if (ia.D > (uint32_t)kMaxDigits || ia.E > kMaxPmap || n > (uint32_t)kMaxList || add_group == 0)
        return hipErrorInvalidValue;
    ListPtrs pe{}, pk{};
    uint32_t distinct_ext = 0;
    for (uint32_t c = 0; c < n; c++) {
        pe.p[c] = ext[c];
        pk.p[c] = evk[c];
        distinct_ext += (c == 0 || ext[c] != ext[c - 1]) ? 1 : 0;
    }
    PinvArgs pa{};
    for (uint32_t i = 0; i < l; i++) pa.pinv[i] = pinv[i];
    // ext limbs (once per distinct ext), evk, conv and out per item, addend polys once per group
    const double bytes = ((double)distinct_ext * ia.D + (double)n * (2 * ia.D + 4) +
                          (add ? (double)(n + add_group - 1) / add_group : 0.0)) * l * kN * 8;
    const int pi = prof_begin(ctx, "ks_sub_list", bytes, st);
    hipLaunchKernelGGL(k_ks_sub_list, dim3(n * (kN / 256) * l), dim3(256), 0, st, pe, pk, conv, add, add_stride,
                       add_group, out, l, ia, pa, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_automorph_list(const Context& ctx, const uint64_t* in, uint64_t* out, uint32_t n, uint32_t l,
                                 const uint32_t* g, hipStream_t st) {
    if (n > (uint32_t)kMaxList) return hipErrorInvalidValue;
    AutoList al{};
    for (uint32_t c = 0; c < n; c++) al.g[c] = g[c];
    const int pi = prof_begin(ctx, "automorph", (double)n * 2 * l * 2 * kN * 8, st);
    hipLaunchKernelGGL(k_automorph_list, dim3(kN / 256, l, 2 * n), dim3(256), 0, st, in, out, l, al);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// l limbs per poly; with l_q < l the limbs from l_q on are the P limbs (an extended-basis MAC)
hipError_t launch_bsgs_mac(const Context& ctx, const uint64_t* const* baby, const uint64_t* diag, uint64_t* out,
                           uint32_t nb, uint32_t n_diag, uint32_t ng, uint32_t l, uint32_t log_rep, hipStream_t st,
                           uint32_t l_q, uint32_t n_inst, uint64_t inst_stride, uint64_t out_stride) {
    if (l_q == 0 || l_q > l) l_q = l;
    if (nb == 0 || log_rep > 6 || n_diag > nb * ng || n_inst == 0 || n_inst > 4096) return hipErrorInvalidValue;
    const double bytes =
        ((double)n_inst * (nb * 2 * l + ng * 2 * l) + (double)n_diag * l / (1u << log_rep)) * kN * 8;
    const int pi = prof_begin(ctx, log_rep ? "bsgs_mac_periodic" : "bsgs_mac", bytes, st);
    for (uint32_t j0 = 0; j0 < nb; j0 += kMaxBaby) {
        const uint32_t nbc = std::min<uint32_t>(kMaxBaby, nb - j0);
        ListPtrs bp{};
        for (uint32_t j = 0; j < nbc; j++) bp.p[j] = baby[j0 + j];
        hipLaunchKernelGGL(k_bsgs_mac, dim3(n_inst * (kN / kMacCoef) * l), dim3(kMacCoef * kMacRows),
                           (size_t)nbc * 2 * kMacCoef * 8, st, bp, diag, out, nbc, nb, j0, ng, n_diag, l, log_rep,
                           j0 ? 1u : 0u, l_q, ctx.L, n_inst, inst_stride, out_stride, ctx.d_primes);
    }
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// babies b < nb (keys[b] null: identity; g[b] its automorphism) of n_in inputs per instance, n_inst instances:
// ext [n_inst n_in] extensions ext_stride apart, src the inputs src_stride apart; n_out outputs of ngp giant sums
// each, the identity giant g0's (g0 >= 0) to id_out + s id_inst_stride + o id_stride, the others to out
// [n_inst][n_out][ngp or ngp - 1][2][E][N]
hipError_t launch_bsgs_dh_mac(const Context& ctx, const uint64_t* ext, uint64_t ext_stride, const uint64_t* src,
                              uint64_t src_stride, const uint64_t* const* keys, const uint32_t* g, uint32_t n_inst,
                              uint32_t n_in, uint32_t nb, const uint64_t* diag, uint32_t n_diag, uint32_t n_out,
                              uint32_t ngp, int32_t g0, uint32_t l, const TwPair* pmod, uint64_t* out,
                              uint64_t* id_out, uint64_t id_inst_stride, uint64_t id_stride, uint32_t chain_delta,
                              hipStream_t st) {
    const uint32_t ng = n_out * ngp;
    const uint32_t E = l + ctx.K, D = (l + ctx.alpha - 1) / ctx.alpha;
    if (n_inst == 0 || n_inst > 4096 || nb == 0 || nb > (uint32_t)kMaxDhBaby || n_in * nb > (uint32_t)kMaxBaby ||
        n_diag > n_in * nb * ng || E > kMaxPmap || D > (uint32_t)kMaxDigits || g0 >= (int32_t)ngp ||
        (g0 >= 0 && !id_out))
        return hipErrorInvalidValue;
    DhMacArgs a{};
    a.l = l;
    a.E = E;
    a.L = ctx.L;
    a.D = D;
    a.T = ctx.L + ctx.K;
    a.n_in = n_in;
    a.nb = nb;
    a.ng = ng;
    a.n_diag = n_diag;
    a.n_inst = n_inst;
    a.ext_stride = ext_stride;
    a.src_stride = src_stride;
    a.ngp = ngp;
    a.g0 = g0;
    a.chain_delta = chain_delta;
    a.out_stride = (uint64_t)n_out * (g0 >= 0 ? ngp - 1 : ngp) * 2 * E * kN;
    a.id_out = id_out;
    a.id_inst_stride = id_inst_stride;
    a.id_stride = id_stride;
    uint32_t n_ks = 0;
    for (uint32_t b = 0; b < nb; b++) {
        a.evk[b] = keys[b];
        a.g[b] = g[b];
        n_ks += keys[b] ? 1 : 0;
    }
    for (uint32_t t = 0; t < l; t++) a.pmod[t] = pmod[t];
    // the babies' inner products are not counted as key switches: they have neither a ModUp nor a ModDown of their own
    // algorithmic bytes, every array once per launch: each input's extension (if a baby is key-switched) and its c0
    // (and c1, if a baby is the identity), the keys and the diagonals, the giant sums written.  (Each baby re-reads
    // its input's words through another automorphism, and each instance re-reads the keys and diagonals of a tile:
    // those re-reads are served by L2 and are not counted.)
    const double by = (double)n_inst * n_in * ((n_ks ? (double)D * E : 0.0) + (n_ks < nb ? 2.0 : 1.0) * l) +
                      (double)n_ks * 2 * D * E + (double)n_diag * E + (double)n_inst * ng * 2 * E;
    const int pi = prof_begin(ctx, "bsgs_dh_mac", by * kN * 8, st);
    using MacKernel = void (*)(const uint64_t*, const uint64_t*, const uint64_t*, uint64_t*, DhMacArgs,
                               const PrimeInfo*);
    static constexpr MacKernel kByDigits[kMaxDigits] = {k_bsgs_dh_mac<1>, k_bsgs_dh_mac<2>, k_bsgs_dh_mac<3>,
                                                        k_bsgs_dh_mac<4>, k_bsgs_dh_mac<5>, k_bsgs_dh_mac<6>,
                                                        k_bsgs_dh_mac<7>, k_bsgs_dh_mac<8>};
    hipLaunchKernelGGL(kByDigits[D - 1], dim3(n_inst * (kN / kMacCoef) * E), dim3(kMacCoef * kMacRows),
                       ((size_t)n_in * nb + kMacRows) * 2 * kMacCoef * 8, st, ext, src, diag, out, a, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// the phase marker: no work; phase id + 1 workgroups of 64 threads make it recognizable in a trace or counter pass
__global__ __launch_bounds__(64) void k_phase_mark(uint32_t) {}

hipError_t launch_phase_mark(uint32_t id, hipStream_t st) {
    hipLaunchKernelGGL(k_phase_mark, dim3(id + 1), dim3(64), 0, st, id);
    return hipGetLastError();
}

hipError_t launch_pair_mac(const Context& ctx, const uint64_t* R, const uint64_t* pt, uint64_t* out, uint32_t n_sets,
                           uint32_t n, uint32_t l, uint32_t log_rep, hipStream_t st) {
    if (log_rep > 6 || n == 0) return hipErrorInvalidValue;
    const double bytes = ((double)2 * n * 2 * l + (double)n_sets * n * 2 * l / (1u << log_rep) +
                          (double)n_sets * n * 2 * l) * kN * 8;
    const int pi = prof_begin(ctx, "pair_mac", bytes, st);
    hipLaunchKernelGGL(k_pair_mac, dim3(kN / 256, l, n_sets * n * 2), dim3(256), 0, st, R, pt, out, n, l, log_rep,
                       ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

static MdrArgs mdr_args(uint32_t l, uint64_t x_pstride, uint64_t add_pstride, const TwPair* pinv,
                        const TwPair* qlinv) {
    MdrArgs ma{};
    ma.l = l;
    ma.x_pstride = x_pstride;
    ma.add_pstride = add_pstride;
    for (uint32_t i = 0; i < l; i++) {
        ma.pinv[i] = pinv[i];
        ma.qlinv[i] = qlinv[i];
    }
    return ma;
}

hipError_t launch_mdr_combine(const Context& ctx, const uint64_t* x, uint64_t x_pstride, const uint64_t* add,
                              uint64_t add_pstride, const uint64_t* T, uint64_t* out, uint32_t n_polys, uint32_t l,
                              const TwPair* pinv, const TwPair* qlinv, hipStream_t st) {
    if (l < 2 || l > (uint32_t)kMaxPmap) return hipErrorInvalidValue;
    const MdrArgs ma = mdr_args(l, x_pstride, add ? add_pstride : 0, pinv, qlinv);
    const int pi = prof_begin(ctx, "mdr_combine", (double)n_polys * (l - 1) * (add ? 4 : 3) * kN * 8, st);
    hipLaunchKernelGGL(k_mdr_combine, dim3(kN / 256, l - 1, n_polys), dim3(256), 0, st, x, add, T, out, ma,
                       ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// the same combine for a relinearization of B ciphertexts (polys 2c, 2c+1), the evk inner product of limbs
// 0..l-2 formed in the kernel from ext [B][D][E][N] and evk [dnum][2][L+K][N]
hipError_t launch_mdr_combine_ks(const Context& ctx, const uint64_t* ext, const uint64_t* evk, const uint64_t* add,
                                 uint64_t add_pstride, const uint64_t* T, uint64_t* out, uint32_t B, uint32_t l,
                                 const TwPair* pinv, const TwPair* qlinv, hipStream_t st, const uint64_t* ta,
                                 const uint64_t* tb) {
    if (l < 2 || l > (uint32_t)kMaxPmap || (ta && (!tb || add))) return hipErrorInvalidValue;
    const InnerArgs ia = inner_args(ctx, l, B);
    if (ia.D > (uint32_t)kMaxDigits || ia.E > kMaxPmap) return hipErrorInvalidValue;
    const MdrArgs ma = mdr_args(l, 0, add ? add_pstride : 0, pinv, qlinv);
    // per ciphertext: D ext limbs, 2 T, 2 add (or the 4 product inputs), 2 out; the level's evk limbs once
    const double bytes =
        ((double)B * (ia.D + 2 + (add ? 2 : 0) + (ta ? 4 : 0) + 2) + 2.0 * ia.D) * (l - 1) * kN * 8;
    const int pi = prof_begin(ctx, "mdr_combine_ks", bytes, st);
    hipLaunchKernelGGL(k_mdr_combine_ks, dim3(B, kN / 256, l - 1), dim3(256), 0, st, ext, evk, add, T, out, ia, ma,
                       ta, tb, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

// n_out outputs of nt terms each (see k_qp_rot_sum; src: the terms' inner sums over Q_l * P, or over Q_l when
// src_pmod (P mod q_t, t < l) is given); keys[i] / steps g[i], i < A + nt - 1 <= 64 (null key: identity term);
// id_src: one more identity term per output c at id_src + c id_stride (or null); output c at
// dst + (u / R) 2 E N + (u % R) s_lo, u = c + c_off; accumulate adds to it
hipError_t launch_qp_rot_sum(const Context& ctx, const uint64_t* ext, uint64_t ext_stride, const uint64_t* src,
                             uint64_t src_stride, const uint64_t* const* keys, const uint32_t* g, uint32_t n_out,
                             uint32_t nt, uint32_t A, uint32_t M, uint32_t l, uint64_t* dst,
                             hipStream_t st, uint32_t R, uint32_t c_off, uint64_t s_lo, bool accumulate,
                             const TwPair* src_pmod, const uint64_t* id_src, uint64_t id_stride) {
    const uint32_t E = l + ctx.K;
    if (n_out == 0 || nt == 0 || A == 0 || A + nt - 1 > (uint32_t)kMaxList || E > kMaxPmap || n_out > 4096)
        return hipErrorInvalidValue;
    const uint32_t D = (l + ctx.alpha - 1) / ctx.alpha;
    if (D > (uint32_t)kMaxDigits) return hipErrorInvalidValue;
    QpRotArgs a{};
    a.l = l;
    a.E = E;
    a.L = ctx.L;
    a.D = D;
    a.T = ctx.L + ctx.K;
    a.nt = nt;
    a.A = A;
    a.M = M;
    a.ext_stride = ext_stride;
    a.src_stride = src_stride;
    a.n_out = n_out;
    a.accumulate = accumulate ? 1 : 0;
    a.R = R ? R : 1;
    a.c_off = c_off;
    a.s_hi = (uint64_t)2 * E * kN;
    a.s_lo = s_lo;
    a.src_q = src_pmod ? 1 : 0;
    a.src_poly = (uint64_t)(src_pmod ? l : E) * kN;
    a.id_src = id_src;
    a.id_stride = id_stride;
    if (src_pmod)
        for (uint32_t t = 0; t < l; t++) a.pmod[t] = src_pmod[t];
    uint32_t n_ks = 0, n_keys = 0;
    for (uint32_t i = 0; i < A + nt - 1; i++) {
        a.evk[i] = keys[i];
        a.g[i] = g[i];
        n_keys += keys[i] ? 1 : 0;
    }
    for (uint32_t c = 0; c < A; c++)
        for (uint32_t j = 0; j < nt; j++) n_ks += keys[c + j] ? 1 : 0;
    // algorithmic bytes, every array once per launch: per key-switched term its extension D E and c0 (Es limbs of the
    // source) -- once for all terms when they share one input (ext_stride 0: a hoisted sum of one ciphertext's
    // rotations) --, per identity term both source polys; the distinct keys (2 D E each) once; the outputs 2 E
    const double Es = src_pmod ? l : E;
    const double terms = (double)n_out / A;
    const double ks_in = ext_stride == 0 ? (n_ks ? 1.0 : 0.0) : (double)n_ks;
    const double by = (ks_in * ((double)D * E + Es) + ((double)A * nt - n_ks) * 2.0 * Es) * terms +
                      (id_src ? (double)n_out * 2.0 * Es : 0.0) + (double)n_keys * 2 * D * E + (double)n_out * 2 * E;
    // key switches: one per term with an extension of its own; a hoisted sum over one extension is one (its ModUp and
    // ModDown), its other terms inner products only
    ctx.n_keyswitch += (uint64_t)ks_in * (uint64_t)(n_out / A);
    const int pi = prof_begin(ctx, "qp_rot_sum", by * kN * 8, st);
    hipLaunchKernelGGL(k_qp_rot_sum, dim3(n_out * (kN / 256) * E), dim3(256), 0, st, ext, src, dst, a, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_gather(const Context& ctx, const uint64_t* const* src, uint32_t n, uint64_t words, uint64_t* dst,
                         hipStream_t st) {
    for (uint32_t c0 = 0; c0 < n; c0 += kMaxList) {
        const uint32_t m = std::min<uint32_t>(kMaxList, n - c0);
        ListPtrs lp{};
        for (uint32_t j = 0; j < m; j++) lp.p[j] = src[c0 + j];
        const uint32_t bx = (uint32_t)std::min<uint64_t>((words + 255) / 256, 1024);
        hipLaunchKernelGGL(k_gather, dim3(bx, m), dim3(256), 0, st, lp, dst + (size_t)c0 * words, words);
    }
    return hipGetLastError();
}

hipError_t launch_tensor_sum(const Context& ctx, const uint64_t* const* d_tab, uint32_t np, uint64_t* d01,
                             uint64_t* d2, uint32_t B, uint32_t l, uint64_t* d2e, uint64_t d2e_bstride,
                             const uint32_t* ext_off, hipStream_t st) {
    if (np == 0 || np > 64) return hipErrorInvalidValue;
    TensorArgs ta{};
    ta.l = l;
    ta.B = B;
    ta.d2e = d2e;
    ta.d2e_bstride = d2e_bstride;
    if (d2e)
        for (uint32_t t = 0; t < l; t++) ta.ext_off[t] = ext_off[t];
    const int pi = prof_begin(ctx, "tensor_sum", (double)B * l * (4.0 * np + 3 + (d2e ? 1 : 0)) * kN * 8, st);
    hipLaunchKernelGGL(k_tensor_sum, dim3(kN / 256, l, B), dim3(256), 0, st, d_tab, np, d01, d2, ta, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_mul_plain(const Context& ctx, const uint64_t* ct, const uint64_t* pt, uint64_t* out, uint32_t B,
                            uint32_t l, uint64_t pt_bstride, uint32_t log_rep, hipStream_t st) {
    const int pi = prof_begin(ctx, "mul_plain",
                              ((double)B * 4 * l + (pt_bstride ? B : 1) * (double)l / (1u << log_rep)) * kN * 8, st);
    hipLaunchKernelGGL(k_mul_plain, dim3(kN / 256, l, 2 * B), dim3(256), 0, st, ct, pt, out, l, pt_bstride, log_rep,
                       ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_add_plain(const Context& ctx, const uint64_t* ct, const uint64_t* pt, uint64_t* out, uint32_t B,
                            uint32_t l, uint64_t pt_bstride, hipStream_t st) {
    hipLaunchKernelGGL(k_add_plain, dim3(kN / 256, l, 2 * B), dim3(256), 0, st, ct, pt, out, l, pt_bstride,
                       ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_sum_list(const Context& ctx, const uint64_t* const* in, uint32_t n, uint64_t* out, uint32_t n_polys,
                           uint32_t l, hipStream_t st) {
    if (n == 0 || n > (uint32_t)kMaxList) return hipErrorInvalidValue;
    ListPtrs lp{};
    for (uint32_t j = 0; j < n; j++) lp.p[j] = in[j];
    const int pi = prof_begin(ctx, "sum_list", (double)(n + 1) * n_polys * l * kN * 8, st);
    hipLaunchKernelGGL(k_sum_list, dim3(kN / 256, l, n_polys), dim3(256), 0, st, lp, n, out, l, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_lincomb(const Context& ctx, uint64_t* out, uint32_t B, uint32_t l_out, uint32_t n_terms,
                          const uint64_t* const* x, const uint32_t* stride, const uint64_t* C /*[n_terms][l_out]*/,
                          const uint64_t* add /*[l_out] or null*/, hipStream_t st, uint32_t i0) {
    if (n_terms == 0 || n_terms > (uint32_t)kMaxTerms || l_out > (uint32_t)kMaxLcLimbs) return hipErrorInvalidValue;
    for (uint32_t t = 0; t < n_terms; t++)
        if (i0 + l_out > stride[t]) return hipErrorInvalidValue;
    LinArgs la{};
    la.n_terms = n_terms;
    la.l_out = l_out;
    la.i0 = i0;
    la.has_add = add ? 1 : 0;
    for (uint32_t t = 0; t < n_terms; t++) {
        la.x[t] = x[t];
        la.stride[t] = stride[t];
        for (uint32_t i = 0; i < l_out; i++) {
            // C R mod q_i (k_lincomb reduces by REDC), a Shoup product by the context's R mod q_i
            const PrimeInfo& pr = ctx.primes[i0 + i];
            const uint64_t c = C[(size_t)t * l_out + i] % pr.q;
            const uint64_t h = (uint64_t)(((unsigned __int128)c * pr.r_mod_p) >> 64);
            const uint64_t v = c * pr.r_mod - h * pr.q;
            la.C[t][i] = v >= pr.q ? v - pr.q : v;
        }
    }
    if (add)
        for (uint32_t i = 0; i < l_out; i++) la.add[i] = add[i];
    const int pi = prof_begin(ctx, "lincomb", (double)B * 2 * l_out * (n_terms + 1) * kN * 8, st);
    hipLaunchKernelGGL(k_lincomb, dim3(kN / 256, l_out, 2 * B), dim3(256), 0, st, out, la, ctx.d_primes);
    prof_end(ctx, pi, st);
    return hipGetLastError();
}

hipError_t launch_mul_i(const Context& ctx, const uint64_t* in, uint64_t* out, uint32_t n_polys, uint32_t l, int sign,
                        hipStream_t st) {
    hipLaunchKernelGGL(k_mul_i, dim3(kN / 256, l, n_polys), dim3(256), 0, st, in, out, l, sign, ctx.d_tw,
                       ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_automorph(const uint64_t* in, uint64_t* out, uint32_t n_polys, uint32_t l, uint32_t g,
                            hipStream_t st) {
    hipLaunchKernelGGL(k_automorph, dim3(kN / 256, l, n_polys), dim3(256), 0, st, in, out, g);
    return hipGetLastError();
}

}  // namespace fhe
