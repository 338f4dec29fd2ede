// client.hip -- limb kernels of the client-side operations (key generation, encryption, decryption):
// small signed polynomials to RNS limbs, the key-switching-key formula, secret-key encryption and
// the decryption inner product.  Not on the evaluation hot path; used to produce seeded keys and
// ciphertexts on the device and to read results back.
#include <vector>

#include "engine.hpp"
#include "modarith.hpp"

namespace fhe {

namespace {

__device__ __forceinline__ Barrett barrett_c(const PrimeInfo& p) { return Barrett{p.q, p.mu_hi, p.mu_lo}; }

// residue of a signed coefficient: c mod q, or q - (|c| mod q) for c < 0 (0 when q divides |c|)
__device__ __forceinline__ uint64_t signed_residue(int64_t c, uint64_t q) {
    if (c >= 0) return (uint64_t)c % q;
    const uint64_t m = (uint64_t)(-(c + 1)) % q;  // -(c+1) >= 0 even for INT64_MIN
    return (m + 1 == q) ? 0 : q - 1 - m;
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
    uint64_t r = signed_residue(coef[(size_t)pc * kN + k], P.q);
    if (pa.log_approx) {
        const Barrett br = barrett_c(P);
        r = mul_mod(r, pow2_mod(pa.log_approx, br), br);
    }
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
// in LDS.
constexpr int kMaxSmallN = 4096;

__global__ __launch_bounds__(256) void k_encode_small(const int64_t* __restrict__ coef,
                                                      const int32_t* __restrict__ log_approx,
                                                      uint64_t* __restrict__ out, uint32_t Np, uint32_t l,
                                                      const TwPair* __restrict__ tab,
                                                      const PrimeInfo* __restrict__ primes) {
    __shared__ uint64_t a[kMaxSmallN];
    const uint32_t n = blockIdx.x, i = blockIdx.y;
    const uint64_t q = primes[i].q;
    const int64_t* c = coef + (size_t)n * Np;
    const uint32_t la = (uint32_t)log_approx[n];
    const Barrett br = barrett_c(primes[i]);
    const uint64_t f = la ? pow2_mod(la, br) : 1;
    for (uint32_t k = threadIdx.x; k < Np; k += 256) {
        const uint64_t r = signed_residue(c[k], q);
        a[k] = la ? mul_mod(r, f, br) : r;
    }
    __syncthreads();
    const TwPair* tw = tab + (size_t)i * Np;
    for (uint32_t m = 1, t = Np >> 1; m < Np; m <<= 1, t >>= 1) {
        for (uint32_t b = threadIdx.x; b < Np / 2; b += 256) {
            const uint32_t grp = b / t, lo = grp * 2 * t + (b - grp * t);
            const TwPair w = tw[m + grp];
            const uint64_t x = shoup(a[lo + t], w.w, w.wp, q);
            const uint64_t u = a[lo];
            a[lo] = add_mod(u, x, q);
            a[lo + t] = sub_mod(u, x, q);
        }
        __syncthreads();
    }
    uint64_t* o = out + ((size_t)n * l + i) * Np;
    for (uint32_t k = threadIdx.x; k < Np; k += 256) o[k] = a[k];
}

hipError_t launch_encode_small(const Context& ctx, const int64_t* coef, const int32_t* log_approx, uint64_t* out,
                               uint32_t n_vec, uint32_t Np, uint32_t l, const TwPair* tab, hipStream_t st) {
    if (Np > (uint32_t)kMaxSmallN || Np < 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_encode_small, dim3(n_vec, l), dim3(256), 0, st, coef, log_approx, out, Np, l, tab,
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
