// ks_device.hpp -- device helpers and launch arguments shared by the key-switch kernels (rns.hip) and the NTT
// kernels that finish a ModDown in their last pass (ntt.hip).
#pragma once
#include "engine.hpp"
#include "modarith.hpp"

namespace fhe {

__device__ __forceinline__ Barrett barrett_of(const PrimeInfo& p) { return Barrett{p.q, p.mu_hi, p.mu_lo}; }

__device__ __forceinline__ uint64_t reduce_u128(const U128& x, const Barrett& b) {
    // hi may exceed q when several products were summed; fold it once (hi < 2^6 q in our uses)
    uint64_t hi = x.hi;
    if (hi >= b.q) hi = hi % b.q;
    return reduce128(hi, x.lo, b);
}

// centered residue of v in [0, ql) modulo q: v > ql/2 stands for v - ql (harness/boot_overflow_probe.cpp:93-94)
__device__ __forceinline__ uint64_t lift_centered(uint64_t v, uint64_t ql, const Barrett& br) {
    const uint64_t q = br.q;
    if (v > (ql >> 1)) {
        const uint64_t neg = ql - v;  // value is -neg
        const uint64_t m = neg >= q ? reduce128(0, neg, br) : neg;
        return m ? q - m : 0;
    }
    return v >= q ? reduce128(0, v, br) : v;
}

constexpr int kMaxDigits = 8;

// The evk inner product of one extended word over D <= kMaxDigits digits: s0 += sum_d x[d xs] e[2d es],
// s1 += sum_d x[d xs] e[(2d+1) es].  Every digit's loads are issued before the first product waits on them (a
// load-multiply loop per digit makes each digit a separate round trip to memory).
// kStreamX: the extension words are read once (no other item shares them): nontemporal loads.
template <bool kStreamX = false>
__device__ __forceinline__ void ks_dot(const uint64_t* __restrict__ x, size_t xs, const uint64_t* __restrict__ e,
                                       size_t es, uint32_t D, Acc& s0, Acc& s1) {
    uint64_t xv[kMaxDigits], e0[kMaxDigits], e1[kMaxDigits];
#pragma unroll
    for (int d = 0; d < kMaxDigits; d++) {
        if (d < (int)D) {
            xv[d] = kStreamX ? __builtin_nontemporal_load(&x[(size_t)d * xs]) : x[(size_t)d * xs];
            e0[d] = e[((size_t)d * 2 + 0) * es];
            e1[d] = e[((size_t)d * 2 + 1) * es];
        }
    }
#pragma unroll
    for (int d = 0; d < kMaxDigits; d++) {
        if (d < (int)D) {
            s0.add(xv[d], e0[d]);
            s1.add(xv[d], e1[d]);
        }
    }
}

// per-item pointers of a list launch (up to kMaxList items)
constexpr int kMaxList = 64;

struct ListPtrs {
    const uint64_t* p[kMaxList];
};

struct InnerArgs {
    uint32_t D, E, T, B;
    uint32_t t0;  // first extended limb computed (k_ks_inner: limbs t0..E-1)
    uint8_t prime_of[kMaxPmap];
};

struct MdrArgs {
    uint32_t l;           // limbs before the rescale
    uint64_t x_pstride;   // words between polys of x ([E][N] each)
    uint64_t add_pstride; // words between polys of add (0: no addend)
    TwPair pinv[kMaxPmap];   // P^-1 mod q_i
    TwPair qlinv[kMaxPmap];  // q_{l-1}^-1 mod q_i
};

// ModDown combine: out = (x - y) s_i (+ the addend), over [n_polys][l][N] (k_sub_scale and the forward NTT that ends
// in it)
struct CombineArgs {
    uint32_t l;                 // limbs per poly of out/y/add
    uint32_t add_div, add_group;  // polys pc % add_div == 0 get addend (pc / add_group) * add_pstride
    uint64_t x_pstride;         // words between polys of x (x may carry extra limbs, e.g. P limbs)
    uint64_t y_pstride, out_pstride, add_pstride;
    TwPair s[kMaxPmap];
};

}  // namespace fhe
