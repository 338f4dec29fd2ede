// modarith.hpp -- 64-bit modular arithmetic for gfx950 built from 32-bit VALU multiplies.
//
// Moduli are NTT primes q < 2^62 (54-bit Q limbs, 60-bit P limbs).  Residues live in uint64.
// Lazy (Harvey) reduction: NTT butterflies keep values in [0, 2q) / [0, 4q) between stages and
// reduce to [0, q) once at the end, so every value a kernel writes is canonical and results are
// bit-identical to any other correct reduction order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fhe {

// high 64 bits of a 64x64 product
__device__ __forceinline__ uint64_t mulhi64(uint64_t a, uint64_t b) { return __umul64hi(a, b); }

// Shoup multiply by a constant w with companion wp = floor(w * 2^64 / q): result in [0, 2q) for any
// x < 2^64 (w < q).  Same companion as hpc_gpu_port/periodic_encode.hpp:115-120.
__device__ __forceinline__ uint64_t shoup_lazy(uint64_t x, uint64_t w, uint64_t wp, uint64_t q) {
    const uint64_t hi = mulhi64(x, wp);
    return x * w - hi * q;
}

__device__ __forceinline__ uint64_t csub(uint64_t x, uint64_t q) { return x >= q ? x - q : x; }

// Shoup multiply from 32-bit pieces, for q < 2^61 and any x < 2^64; result in [0, 4q).
// The quotient H'' = x1*p1 + hi(x1*p0) + hi(x0*p1) drops the low partial product and the carries of the
// middle terms, so H - 2 <= H'' <= H (H = floor(x * wp / 2^64), for which x*w - H*q lies in [0, 2q)).
// The remainder is accumulated with nq = 2^64 - q so that every step is a multiply-add mod 2^64:
// 2 mul_hi + 2 mad_u64 + 4 mul_lo + 1 mad_u64 + adds.
__device__ __forceinline__ uint64_t shoup_lazy4(uint64_t x, uint64_t w, uint64_t wp, uint64_t nq) {
    const uint32_t x0 = (uint32_t)x, x1 = (uint32_t)(x >> 32);
    const uint32_t p0 = (uint32_t)wp, p1 = (uint32_t)(wp >> 32);
    const uint64_t h = (uint64_t)x1 * p1 + ((uint64_t)__umulhi(x1, p0) + __umulhi(x0, p1));
    const uint32_t h0 = (uint32_t)h, h1 = (uint32_t)(h >> 32);
    const uint32_t w0 = (uint32_t)w, w1 = (uint32_t)(w >> 32);
    const uint32_t n0 = (uint32_t)nq, n1 = (uint32_t)(nq >> 32);
    const uint64_t t = (uint64_t)x0 * w0 + (uint64_t)h0 * n0;
    const uint32_t c1 = x1 * w0 + x0 * w1, c2 = h1 * n0 + h0 * n1;
    // the high word as one 32-bit add of three terms (left to the compiler, this became 64-bit adds and moves)
    uint32_t hi;
    asm("v_add3_u32 %0, %1, %2, %3" : "=v"(hi) : "v"((uint32_t)(t >> 32)), "v"(c1), "v"(c2));
    return ((uint64_t)hi << 32) | (uint32_t)t;
}

// x in [0, 2c) -> [0, c): x - c, or x when the subtraction borrows (x < c).  Written as the four instructions it
// needs (subtract with borrow out, then two selects on the borrow): the C form costs a separate 64-bit compare.
__device__ __forceinline__ uint64_t csub_s(uint64_t x, uint64_t c) {
    uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
    uint32_t dlo, dhi;
    asm(
        "v_sub_co_u32 %0, vcc, %2, %4\n\t"
        "v_subb_co_u32 %1, vcc, %3, %5, vcc\n\t"
        "v_cndmask_b32 %0, %0, %2, vcc\n\t"
        "v_cndmask_b32 %1, %1, %3, vcc"
        : "=&v"(dlo), "=&v"(dhi)
        : "v"(lo), "v"(hi), "v"((uint32_t)c), "v"((uint32_t)(c >> 32))
        : "vcc");
    return ((uint64_t)dhi << 32) | dlo;
}

__device__ __forceinline__ uint64_t shoup(uint64_t x, uint64_t w, uint64_t wp, uint64_t q) {
    return csub(shoup_lazy(x, w, wp, q), q);
}

__device__ __forceinline__ uint64_t add_mod(uint64_t a, uint64_t b, uint64_t q) { return csub(a + b, q); }
__device__ __forceinline__ uint64_t sub_mod(uint64_t a, uint64_t b, uint64_t q) { return a >= b ? a - b : a + q - b; }

// Barrett reduction of a 128-bit value (hi:lo) with hi < q, using mu = floor(2^128 / q) split as
// (mu_hi, mu_lo).  Result in [0, q).
struct Barrett {
    uint64_t q, mu_hi, mu_lo;
};

__device__ __forceinline__ uint64_t reduce128(uint64_t hi, uint64_t lo, const Barrett& b) {
    // Quotient estimate qt = hi*mu_hi + floor(hi*mu_lo / 2^64) + floor(lo*mu_hi / 2^64): it drops lo*mu_lo / 2^128
    // and two fractional parts (< 3 in all) from x*mu / 2^128, which itself is at most 1 below x / q.  So
    // floor(x / q) - 3 <= qt <= floor(x / q) and the remainder x - qt*q lies in [0, 4q) (q < 2^62).
    const uint64_t q = b.q;
    const uint64_t t1 = mulhi64(lo, b.mu_hi);
    const uint64_t t2 = mulhi64(hi, b.mu_lo);
    const uint64_t qt = hi * b.mu_hi + t1 + t2;
    const uint64_t r = csub_s(lo - qt * q, q << 1);
    return csub_s(r, q);
}

__device__ __forceinline__ uint64_t mul_mod(uint64_t a, uint64_t b, const Barrett& br) {
    return reduce128(mulhi64(a, b), a * b, br);
}

// 128-bit accumulator
struct U128 {
    uint64_t lo, hi;
};

__device__ __forceinline__ void mac128(U128& acc, uint64_t a, uint64_t b) {
    const uint64_t lo = a * b;
    const uint64_t hi = mulhi64(a, b);
    const uint64_t nlo = acc.lo + lo;
    acc.hi += hi + (nlo < lo ? 1 : 0);
    acc.lo = nlo;
}

// a workgroup-uniform quotient (both operands uniform): the division by a kernel argument runs on the VALU (there is
// no scalar divide), so its result is taken back into a scalar register -- the addresses and constants derived from
// it then stay scalar instead of occupying (and, across a transform, spilling) vector registers
__device__ __forceinline__ uint32_t uni_div(uint32_t a, uint32_t b) { return __builtin_amdgcn_readfirstlane(a / b); }

// Lazy 128-bit multiply-accumulate for operands below 2^60 (every modulus of this engine is): the four 32 x 32
// partial products go to separate 64-bit sums -- the low products to lo, the two cross products (< 2^60 each) to
// m, the high product (< 2^56) straight into hi -- so a term costs four v_mad_u64_u32 and a carry, against ~30
// instructions for a full 64 x 64 -> 128 product per term.  The carry out of lo is the carry-out the multiply-add
// itself reports (its scalar destination), counted in c and added to hi at the fold; in C it had been a 64-bit
// compare, a select, a zero extension and a 64-bit add per term.
// m takes at most 8 terms (< 2^61 each) between folds: call fold() at least every 8 add()s.
struct Acc {
    uint64_t lo, hi, m;
    uint32_t c;  // carries out of lo since the last fold
    __device__ __forceinline__ Acc() : lo(0), hi(0), m(0), c(0) {}
    __device__ __forceinline__ void add(uint64_t a, uint64_t b) {
        const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32);
        const uint32_t b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
        uint64_t carry;  // the low product's carry-out (a scalar register pair)
        asm("v_mad_u64_u32 %0, %4, %5, %7, %0\n\t"   // lo += a0 b0, carry out
            "v_mad_u64_u32 %1, vcc, %6, %8, %1\n\t"  // hi += a1 b1
            "v_mad_u64_u32 %2, vcc, %5, %8, %2\n\t"  // m += a0 b1
            "v_mad_u64_u32 %2, vcc, %6, %7, %2\n\t"  // m += a1 b0
            "v_addc_co_u32_e64 %3, vcc, 0, %3, %4"     // c += carry
            : "+v"(lo), "+v"(hi), "+v"(m), "+v"(c), "=&s"(carry)
            : "v"(a0), "v"(a1), "v"(b0), "v"(b1)
            : "vcc");
    }
    __device__ __forceinline__ void fold() {
        const uint64_t s = m << 32;
        lo += s;
        hi += (m >> 32) + (lo < s ? 1u : 0u) + c;
        m = 0;
        c = 0;
    }
    __device__ __forceinline__ U128 get() {
        fold();
        return U128{lo, hi};
    }
    // Montgomery's REDC (R = 2^64) of the sum, lazily: [0, 2q), the same value as redc_lazy(get(), q, ninv).  The
    // fold's carries run through VCC from one add into the next: the low word's high half is lo_h + m_lo (carry c1),
    // the high word hi + m_hi + c1 + c; then (T + m' q) / R = high + hi(m' q) + [low != 0], m' = low (-q^-1) mod R.
    // Requires the sum below q R, as redc_lazy does.
    __device__ __forceinline__ uint64_t redc_lazy(uint64_t q, uint64_t ninv) const {
        uint32_t lh, hl, hh;
        asm("v_add_co_u32 %0, vcc, %3, %5\n\t"
            "v_addc_co_u32 %1, vcc, %4, %6, vcc\n\t"
            "v_addc_co_u32_e64 %2, vcc, %7, 0, vcc\n\t"
            "v_add_co_u32 %1, vcc, %1, %8\n\t"
            "v_addc_co_u32_e64 %2, vcc, %2, 0, vcc"
            : "=&v"(lh), "=&v"(hl), "=&v"(hh)
            : "v"((uint32_t)(lo >> 32)), "v"((uint32_t)hi), "v"((uint32_t)m), "v"((uint32_t)(m >> 32)),
              "v"((uint32_t)(hi >> 32)), "v"(c)
            : "vcc");
        const uint32_t ll = (uint32_t)lo;
        const uint64_t mm = (((uint64_t)lh << 32) | ll) * ninv;
        const uint64_t hq = mulhi64(mm, q);
        uint32_t rl, rh, nz;
        asm("v_or_b32 %2, %3, %4\n\t"
            "v_cmp_ne_u32 vcc, 0, %2\n\t"
            "v_addc_co_u32 %0, vcc, %5, %7, vcc\n\t"
            "v_addc_co_u32 %1, vcc, %6, %8, vcc"
            : "=&v"(rl), "=&v"(rh), "=&v"(nz)
            : "v"(ll), "v"(lh), "v"(hl), "v"(hh), "v"((uint32_t)hq), "v"((uint32_t)(hq >> 32))
            : "vcc");
        return ((uint64_t)rh << 32) | rl;
    }
    // the canonical REDC: [0, q)
    __device__ __forceinline__ uint64_t redc(uint64_t q, uint64_t ninv) const { return csub_s(redc_lazy(q, ninv), q); }
};

// Multiply-accumulate over 30-bit halves, for sums of at most 8 products of operands below 2^60: with
// a = a1 2^30 + a0 and b = b1 2^30 + b0 (all halves < 2^30), s0 += a0 b0, s1 += a0 b1 + a1 b0, s2 += a1 b1 are
// each one v_mad_u64_u32 and cannot overflow (16 terms below 2^60 in s1), so a term costs exactly four
// multiply-adds with no carry handling.  The constant operand comes packed as (b1 << 32) | b0 (pack30 on the host).
struct Acc30 {
    uint64_t s0, s1, s2;
    __device__ __forceinline__ Acc30() : s0(0), s1(0), s2(0) {}
    __device__ __forceinline__ void add(uint32_t a0, uint32_t a1, uint64_t bp) {
        const uint32_t b0 = (uint32_t)bp, b1 = (uint32_t)(bp >> 32);
        s0 += (uint64_t)a0 * b0;
        s1 += (uint64_t)a0 * b1;
        s1 += (uint64_t)a1 * b0;
        s2 += (uint64_t)a1 * b1;
    }
    // the sum as 128 bits: s0 + s1 2^30 + s2 2^60
    __device__ __forceinline__ U128 get() const { return combine30(s0, s1, s2); }
    __device__ __forceinline__ static U128 combine30(uint64_t s0, uint64_t s1, uint64_t s2) {
        const uint64_t m = s1 << 30, t = s2 << 60;
        uint64_t lo = s0 + m;
        uint64_t hi = (s1 >> 34) + (s2 >> 4) + (lo < m ? 1u : 0u);
        lo += t;
        hi += (lo < t) ? 1u : 0u;
        return U128{lo, hi};
    }
};

// Montgomery's REDC with R = 2^64: x < q R -> x R^-1 mod q in [0, q) (redc_lazy: in [0, 2q)).  m = x_lo (-q^-1)
// mod 2^64 makes x + m q a multiple of R; its low word sums to R exactly when x_lo != 0, so (x + m q) / R = x_hi +
// hi(m q) + [x_lo != 0], below 2q.
__device__ __forceinline__ uint64_t redc_lazy(const U128& x, uint64_t q, uint64_t ninv) {
    const uint64_t m = x.lo * ninv;
    return x.hi + mulhi64(m, q) + (x.lo != 0 ? 1u : 0u);
}
__device__ __forceinline__ uint64_t redc(const U128& x, uint64_t q, uint64_t ninv) {
    return csub_s(redc_lazy(x, q, ninv), q);
}

// Acc30 with three multiply-adds a term (Karatsuba): s0 += a0 b0, s2 += a1 b1 and sm += (a0 + a1)(b0 + b1) mod 2^64;
// the middle sum is s1 = sm - s0 - s2 mod 2^64, exact because the true s1 is below 2^64 (the Acc30 bound).  The
// caller passes a0 + a1 (< 2^31) with the halves; b0 + b1 of a wave-uniform constant is a scalar add.
struct Acc30k {
    uint64_t s0, s2, sm;
    __device__ __forceinline__ Acc30k() : s0(0), s2(0), sm(0) {}
    __device__ __forceinline__ void add(uint32_t a0, uint32_t a1, uint32_t as, uint64_t bp) {
        const uint32_t b0 = (uint32_t)bp, b1 = (uint32_t)(bp >> 32);
        s0 += (uint64_t)a0 * b0;
        s2 += (uint64_t)a1 * b1;
        sm += (uint64_t)as * (b0 + b1);
    }
    __device__ __forceinline__ U128 get() const { return Acc30::combine30(s0, sm - s0 - s2, s2); }
    // redc_lazy(get(), q, ninv) without the 128-bit sum in between: T = s0 + s1 2^30 + s2 2^60 (s1 = sm - s0 - s2)
    // has low word lo = s0 + (s1 << 30) + (s2 << 60) and high word (s2 >> 4) + (s1 >> 34) + the two carries of lo;
    // the carries go from one add straight into the next through VCC (in C each became a compare, a select, a zero
    // extension and a 64-bit add).  REDC: (T + m q) / 2^64 = hi + hi(m q) + [lo != 0], m = lo (-q^-1) mod 2^64.
    __device__ __forceinline__ uint64_t redc_lazy(uint64_t q, uint64_t ninv) const {
        const uint64_t s1 = sm - s0 - s2;
        const uint64_t sh = s1 << 30, h0 = s2 >> 4;
        const uint32_t s1h = (uint32_t)(s1 >> 34), t = (uint32_t)s2 << 28;  // s2 2^60 touches the high word only
        uint32_t lol, loh, hl, hh, a_hi;
        asm("v_add_co_u32 %0, vcc, %5, %7\n\t"           // s0 + (s1 << 30): low word
            "v_addc_co_u32 %4, vcc, %6, %8, vcc\n\t"     // its high word, carry c1
            "v_addc_co_u32 %2, vcc, %9, %11, vcc\n\t"    // (s2 >> 4) + (s1 >> 34) + c1
            "v_addc_co_u32_e64 %3, vcc, %10, 0, vcc\n\t"
            "v_add_co_u32 %1, vcc, %4, %12\n\t"          // + (s2 << 60): high word only, carry c2
            "v_addc_co_u32_e64 %2, vcc, %2, 0, vcc\n\t"  // + c2
            "v_addc_co_u32_e64 %3, vcc, %3, 0, vcc"
            : "=&v"(lol), "=&v"(loh), "=&v"(hl), "=&v"(hh), "=&v"(a_hi)
            : "v"((uint32_t)s0), "v"((uint32_t)(s0 >> 32)), "v"((uint32_t)sh), "v"((uint32_t)(sh >> 32)),
              "v"((uint32_t)h0), "v"((uint32_t)(h0 >> 32)), "v"(s1h), "v"(t)
            : "vcc");
        const uint64_t m = (((uint64_t)loh << 32) | lol) * ninv;
        const uint64_t hq = mulhi64(m, q);
        uint32_t rl, rh, nz;
        asm("v_or_b32 %2, %3, %4\n\t"
            "v_cmp_ne_u32 vcc, 0, %2\n\t"                // [lo != 0]
            "v_addc_co_u32 %0, vcc, %5, %7, vcc\n\t"
            "v_addc_co_u32 %1, vcc, %6, %8, vcc"
            : "=&v"(rl), "=&v"(rh), "=&v"(nz)
            : "v"(lol), "v"(loh), "v"(hl), "v"(hh), "v"((uint32_t)hq), "v"((uint32_t)(hq >> 32))
            : "vcc");
        return ((uint64_t)rh << 32) | rl;
    }
};

}  // namespace fhe
