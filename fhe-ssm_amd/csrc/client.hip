// client.hip -- limb kernels of the client-side operations (key generation, encryption, decryption):
// small signed polynomials to RNS limbs, the key-switching-key formula, secret-key encryption and
// the decryption inner product.  Not on the evaluation hot path; used to produce seeded keys and
// ciphertexts on the device and to read results back.
#include <vector>

#include "engine.hpp"
#include "modarith.hpp"
#include "ntt_device.hpp"

namespace fhe {

namespace {

__device__ __forceinline__ Barrett barrett_c(const PrimeInfo& p) { return Barrett{p.q, p.mu_hi, p.mu_lo}; }

// residue of a signed coefficient (|c| <= 2^63): c mod q, or q - (|c| mod q) for c < 0 (0 when q divides |c|);
// |c| mod q by one Barrett reduction
__device__ __forceinline__ uint64_t small_residue(int64_t c, const Barrett& br) {
    const uint64_t m = reduce128(0, c >= 0 ? (uint64_t)c : 0 - (uint64_t)c, br);
    return (c < 0 && m) ? br.q - m : m;
}

// 2^e mod q (square and multiply)
__device__ __forceinline__ uint64_t pow2_mod(uint32_t e, const Barrett& br) {
    uint64_t r = 1 % br.q, b = 2 % br.q;
    for (; e; e >>= 1) {
        if (e & 1) r = mul_mod(r, b, br);
        b = mul_mod(b, b, br);
    }
    return r;
}

// out[pc][l][k] = coef[pc][k] 2^log_approx mod q_{pmap[l]} (signed coefficients; log_approx > 0 only for plaintexts
// whose coefficients were divided by 2^log_approx before rounding)
struct PmapArgs {
    uint32_t n_limbs;
    uint32_t log_approx;
    uint8_t pmap[kMaxPmap];
};

__global__ __launch_bounds__(256) void k_small_to_rns(const int64_t* __restrict__ coef, uint64_t* __restrict__ out,
                                                      PmapArgs pa, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t l = blockIdx.y, pc = blockIdx.z;
    const PrimeInfo& P = primes[pa.pmap[l]];
    const Barrett br = barrett_c(P);
    uint64_t r = small_residue(coef[(size_t)pc * kN + k], br);
    if (pa.log_approx) r = mul_mod(r, pow2_mod(pa.log_approx, br), br);
    out[((size_t)pc * pa.n_limbs + l) * kN + k] = r;
}

// key-switching key of one digit over Q*P (T limbs, limb i uses prime i):
// b[i] = -a[i] * s_new[i] + e[i] + (digit limb ? pmod_i * s_old[i] : 0)
struct KskArgs {
    uint32_t lo, hi;     // Q limbs of this digit
    TwPair pmod[kMaxPmap];
};

__global__ __launch_bounds__(256) void k_ksk_b(const uint64_t* __restrict__ a, const uint64_t* __restrict__ s_new,
                                               const uint64_t* __restrict__ e, const uint64_t* __restrict__ s_old,
                                               uint64_t* __restrict__ b, KskArgs ka,
                                               const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y;
    const size_t o = (size_t)i * kN + k;
    const Barrett br = barrett_c(primes[i]);
    const uint64_t q = br.q;
    const uint64_t as = mul_mod(a[o], s_new[o], br);
    uint64_t v = sub_mod(e[o], as, q);
    if (i >= ka.lo && i < ka.hi) v = add_mod(v, shoup(s_old[o], ka.pmod[i].w, ka.pmod[i].wp, q), q);
    b[o] = v;
}

// secret-key encryption of l limbs: c0 = m + e - a*s, c1 = a  (ct layout [2][l][N])
__global__ __launch_bounds__(256) void k_encrypt(const uint64_t* __restrict__ m, const uint64_t* __restrict__ e,
                                                 const uint64_t* __restrict__ a, const uint64_t* __restrict__ s,
                                                 uint64_t* __restrict__ ct, uint32_t l,
                                                 const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y;
    const size_t o = (size_t)i * kN + k;
    const Barrett br = barrett_c(primes[i]);
    const uint64_t as = mul_mod(a[o], s[o], br);
    ct[o] = sub_mod(add_mod(m[o], e[o], br.q), as, br.q);
    ct[(size_t)l * kN + o] = a[o];
}

// public-key encryption before its ModDown: x[p][t] = pk[p][prime t] * v[t] + e[p][t] over the E limbs of Q_l * P
// (limb t uses prime pmap[t]; pk [2][L+K][N], v [E][N], e [2][E][N], x [2][E][N])
__global__ __launch_bounds__(256) void k_pk_mac(const uint64_t* __restrict__ pk, const uint64_t* __restrict__ v,
                                                const uint64_t* __restrict__ e, uint64_t* __restrict__ x, PmapArgs pa,
                                                uint32_t T, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t t = blockIdx.y, p = blockIdx.z;
    const uint32_t pi = pa.pmap[t];
    const Barrett br = barrett_c(primes[pi]);
    const size_t o = (size_t)t * kN + k, oe = ((size_t)p * pa.n_limbs + t) * kN + k;
    x[oe] = add_mod(mul_mod(pk[((size_t)p * T + pi) * kN + k], v[o], br), e[oe], br.q);
}

// decryption inner product: out = c0 + c1 * s over l limbs
__global__ __launch_bounds__(256) void k_decrypt(const uint64_t* __restrict__ ct, const uint64_t* __restrict__ s,
                                                 uint64_t* __restrict__ out, uint32_t l,
                                                 const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y;
    const size_t o = (size_t)i * kN + k;
    const Barrett br = barrett_c(primes[i]);
    out[o] = add_mod(ct[o], mul_mod(ct[(size_t)l * kN + o], s[o], br), br.q);
}

// elementwise product over [l][N] (limb i uses prime i)
__global__ __launch_bounds__(256) void k_mul(const uint64_t* __restrict__ x, const uint64_t* __restrict__ y,
                                             uint64_t* __restrict__ out, const PrimeInfo* __restrict__ primes) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t i = blockIdx.y;
    const size_t o = (size_t)i * kN + k;
    out[o] = mul_mod(x[o], y[o], barrett_c(primes[i]));
}

}  // namespace

// Periodic-plaintext encoder: vector n, limb i -> the N'-point negacyclic NTT (root psi^(N/N'), output in
// bit-reversed order) of the small polynomial coef[n] 2^log_approx[n] mod q_i.  One workgroup per (n, i), the limb
// in LDS (N' words of dynamic shared memory).  The Cooley-Tukey network of the table tab (stage s uses
// Table[2^s + group]) runs up to three stages per LDS round: a thread takes the 2^R words of a unit through R stages
// in registers, so N' = 2^11 takes four barriers.  Values stay lazily reduced (below 8q with ct_bfly; for primes below
// 2^56 unreduced, below q + 4q L <= 49q at N' = 2^12) and are brought to [0, q) once before the store, so the words
// are those of any exact evaluation of the network.
constexpr int kMaxSmallN = 4096;

// stages s .. s+R-1 of the network over a (N' = 2^lg words).  At stage s (2^s groups of 2t words, t = N' / 2^(s+1)) a
// unit is the 2^R words j + k d, k < 2^R, d = 2t / 2^R, j = grp 2t + r (r < d): they stay inside one group for the R
// stages, and at stage s + i word k belongs to group grp 2^i + (k >> (R - i)) and pairs with word k + 2^(R-1-i).
template <int R, bool kOpen>
__device__ __forceinline__ void encode_small_round(uint64_t* a, uint32_t Np, uint32_t lg, uint32_t s,
                                                   const TwPair* __restrict__ tw, uint64_t q4, uint64_t nq) {
    constexpr int U = 1 << R;
    const uint32_t lt = lg - s - 1, sub = lt + 1 - R, d = 1u << sub;
    for (uint32_t u = threadIdx.x; u < (Np >> R); u += 256) {
        const uint32_t grp = u >> sub, j = (grp << (lt + 1)) + (u & (d - 1));
        TwPair w[U - 1];  // the unit's twiddles, stage by stage, requested with its words
#pragma unroll
        for (int i = 0, n = 0; i < R; i++)
#pragma unroll
            for (int g = 0; g < (1 << i); g++, n++) w[n] = tw[((1u << s) << i) + (grp << i) + g];
        uint64_t x[U];
#pragma unroll
        for (int k = 0; k < U; k++) x[k] = a[j + k * d];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int hh = U >> (i + 1);
#pragma unroll
            for (int k = 0; k < U; k++) {
                if (k & hh) continue;
                fwd_bfly<kOpen>(x[k], x[k + hh], w[(1 << i) - 1 + (k >> (R - i))], q4, nq);
            }
        }
#pragma unroll
        for (int k = 0; k < U; k++) a[j + k * d] = x[k];
    }
    __syncthreads();
}

template <bool kOpen>
__device__ __forceinline__ void encode_small_ntt(uint64_t* a, uint32_t Np, const TwPair* __restrict__ tw,
                                                 const PrimeInfo& P) {
    const uint64_t q = P.q, q4 = q << 2, nq = 0 - q;
    const uint32_t lg = 31 - __builtin_clz(Np);
    uint32_t s = 0;
    for (; s + 3 <= lg; s += 3) encode_small_round<3, kOpen>(a, Np, lg, s, tw, q4, nq);
    if (lg - s == 2) encode_small_round<2, kOpen>(a, Np, lg, s, tw, q4, nq);
    if (lg - s == 1) encode_small_round<1, kOpen>(a, Np, lg, s, tw, q4, nq);
}

__global__ __launch_bounds__(256) void k_encode_small(const int64_t* __restrict__ coef,
                                                      const int32_t* __restrict__ log_approx,
                                                      uint64_t* __restrict__ out, uint32_t Np, uint32_t l,
                                                      const TwPair* __restrict__ tab,
                                                      const PrimeInfo* __restrict__ primes) {
    extern __shared__ uint64_t a[];  // Np words
    const uint32_t n = blockIdx.x, i = blockIdx.y;
    const PrimeInfo& P = primes[i];
    const uint64_t q = P.q;
    const int64_t* c = coef + (size_t)n * Np;
    const uint32_t la = (uint32_t)log_approx[n];
    const Barrett br = barrett_c(P);
    const uint64_t f = la == 0 ? 1 : la < 64 ? reduce128(0, 1ull << la, br) : pow2_mod(la, br);
    for (uint32_t k = threadIdx.x; k < Np; k += 256) {
        const uint64_t r = small_residue(c[k], br);
        a[k] = la ? mul_mod(r, f, br) : r;
    }
    __syncthreads();
    const TwPair* tw = tab + (size_t)i * Np;
    const bool open = q < kOpenMaxQ;
    if (open)
        encode_small_ntt<true>(a, Np, tw, P);
    else
        encode_small_ntt<false>(a, Np, tw, P);
    uint64_t* o = out + ((size_t)n * l + i) * Np;
    for (uint32_t k = threadIdx.x; k < Np; k += 256)
        o[k] = open ? reduce_open(a[k], q, 0 - q, P.red_shift, P.red_mul) : canon8(a[k], q);
}

hipError_t launch_encode_small(const Context& ctx, const int64_t* coef, const int32_t* log_approx, uint64_t* out,
                               uint32_t n_vec, uint32_t Np, uint32_t l, const TwPair* tab, hipStream_t st) {
    if (Np > (uint32_t)kMaxSmallN || Np < 2 || (Np & (Np - 1))) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_encode_small, dim3(n_vec, l), dim3(256), (size_t)Np * 8, st, coef, log_approx, out, Np, l, tab,
                       ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_small_to_rns(const Context& ctx, const int64_t* coef, uint64_t* out, uint32_t n_polys,
                               const std::vector<uint32_t>& pmap, uint32_t log_approx, hipStream_t st) {
    if (pmap.size() > kMaxPmap) return hipErrorInvalidValue;
    PmapArgs pa{};
    pa.n_limbs = (uint32_t)pmap.size();
    pa.log_approx = log_approx;
    for (size_t i = 0; i < pmap.size(); i++) pa.pmap[i] = (uint8_t)pmap[i];
    hipLaunchKernelGGL(k_small_to_rns, dim3(kN / 256, pa.n_limbs, n_polys), dim3(256), 0, st, coef, out, pa,
                       ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_ksk_b(const Context& ctx, const uint64_t* a, const uint64_t* s_new, const uint64_t* e,
                        const uint64_t* s_old, uint64_t* b, uint32_t lo, uint32_t hi, const TwPair* pmod,
                        hipStream_t st) {
    KskArgs ka{};
    ka.lo = lo;
    ka.hi = hi;
    const uint32_t T = ctx.L + ctx.K;
    for (uint32_t i = 0; i < T; i++) ka.pmod[i] = pmod[i];
    hipLaunchKernelGGL(k_ksk_b, dim3(kN / 256, T), dim3(256), 0, st, a, s_new, e, s_old, b, ka, ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_encrypt(const Context& ctx, const uint64_t* m, const uint64_t* e, const uint64_t* a,
                          const uint64_t* s, uint64_t* ct, uint32_t l, hipStream_t st) {
    hipLaunchKernelGGL(k_encrypt, dim3(kN / 256, l), dim3(256), 0, st, m, e, a, s, ct, l, ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_pk_mac(const Context& ctx, const uint64_t* pk, const uint64_t* v, const uint64_t* e, uint64_t* x,
                         const std::vector<uint32_t>& pmap, hipStream_t st) {
    if (pmap.empty() || pmap.size() > kMaxPmap) return hipErrorInvalidValue;
    PmapArgs pa{};
    pa.n_limbs = (uint32_t)pmap.size();
    for (size_t i = 0; i < pmap.size(); i++) pa.pmap[i] = (uint8_t)pmap[i];
    hipLaunchKernelGGL(k_pk_mac, dim3(kN / 256, pa.n_limbs, 2), dim3(256), 0, st, pk, v, e, x, pa, ctx.L + ctx.K,
                       ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_decrypt(const Context& ctx, const uint64_t* ct, const uint64_t* s, uint64_t* out, uint32_t l,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_decrypt, dim3(kN / 256, l), dim3(256), 0, st, ct, s, out, l, ctx.d_primes);
    return hipGetLastError();
}

hipError_t launch_mul(const Context& ctx, const uint64_t* x, const uint64_t* y, uint64_t* out, uint32_t l,
                      hipStream_t st) {
    hipLaunchKernelGGL(k_mul, dim3(kN / 256, l), dim3(256), 0, st, x, y, out, ctx.d_primes);
    return hipGetLastError();
}

}  // namespace fhe
