// ntt_device.hpp -- the NTT butterflies and final reductions shared by the limb NTT (ntt.hip) and the small-ring
// encoder of periodic plaintexts (client.hip).
#pragma once
#include "engine.hpp"
#include "modarith.hpp"

namespace fhe {

// Forward (Cooley-Tukey) butterfly, values kept in [0, 8q) (q < 2^60): X is brought to [0, 4q), the
// twiddle product is in [0, 4q), so X + T and X - T + 4q stay in [0, 8q).
__device__ __forceinline__ void ct_bfly(uint64_t& X, uint64_t& Y, const TwPair& w, uint64_t q4, uint64_t nq) {
    const uint64_t x = csub_s(X, q4);
    const uint64_t t = shoup_lazy4(Y, w.w, w.wp, nq);
    X = x + t;
    Y = x + q4 - t;
}

// Forward butterfly for primes below 2^56, X left unreduced: the twiddle product is in [0, 4q) whatever Y is, so
// every stage adds at most 4q to the bound (inputs below 8q leave the 16 stages below 72q < 2^63) and the values
// are brought to [0, q) once, at the end (reduce_open).  Saves the four instructions of the conditional subtract.
constexpr uint64_t kOpenMaxQ = 1ull << 56;

template <bool kOpen>
__device__ __forceinline__ void fwd_bfly(uint64_t& X, uint64_t& Y, const TwPair& w, uint64_t q4, uint64_t nq) {
    if (kOpen) {
        const uint64_t x = X;
        const uint64_t t = shoup_lazy4(Y, w.w, w.wp, nq);
        X = x + t;
        Y = x + q4 - t;
    } else {
        ct_bfly(X, Y, w, q4, nq);
    }
}

// v < 128 q -> [0, q): k = hi32(floor(v / 2^s) M), M = floor(2^(32+s) / q), is floor(v/q) or one less (the
// truncations lose less than 2^-24 + v / 2^(32+s) < 0.6), so v - k q lies in [0, 2q); one conditional subtract.
__device__ __forceinline__ uint64_t reduce_open(uint64_t v, uint64_t q, uint64_t nq, uint32_t s, uint32_t M) {
    const uint32_t k = __umulhi((uint32_t)(v >> s), M);
    uint64_t r = (uint64_t)k * (uint32_t)nq + v;               // v + k nq (mod 2^64), nq = 2^64 - q
    r += (uint64_t)(k * (uint32_t)(nq >> 32)) << 32;
    return csub_s(r, q);
}

// [0, 8q) -> [0, q)
__device__ __forceinline__ uint64_t canon8(uint64_t v, uint64_t q) {
    v = csub_s(v, q << 2);
    v = csub_s(v, q << 1);
    return csub_s(v, q);
}

}  // namespace fhe
