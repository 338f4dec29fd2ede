// client.cpp -- client-side operations: seeded sampling (ChaCha20 expander of
// hpc_gpu_port/seeded_keys.hpp:28-43), key-switching-key generation (seeded_keys.hpp:216-256),
// CKKS encode/decode (special FFT, slot j <-> evaluation at zeta^(5^j), zeta = exp(i pi / N)),
// secret-key encryption and decryption.  Host code; the limb arithmetic runs in client.hip kernels.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <complex>
#include <cstring>
#include <stdexcept>
#include <string>
#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "client.hpp"
#include "engine.hpp"
#include "ops.hpp"

namespace fhe {

uint64_t mulmod_h(uint64_t a, uint64_t b, uint64_t q);
uint64_t powmod_h(uint64_t a, uint64_t e, uint64_t q);
uint64_t invmod_h(uint64_t a, uint64_t q);
hipError_t launch_ntt(const Context& ctx, uint64_t* data, const JobSpec& js, uint32_t n_jobs, bool inverse,
                      NttMode mode, hipStream_t st);
hipError_t launch_small_to_rns(const Context& ctx, const int64_t* coef, uint64_t* out, uint32_t n_polys,
                               const std::vector<uint32_t>& pmap, uint32_t log_approx, hipStream_t st);
hipError_t launch_ksk_b(const Context& ctx, const uint64_t* a, const uint64_t* s_new, const uint64_t* e,
                        const uint64_t* s_old, uint64_t* b, uint32_t lo, uint32_t hi, const TwPair* pmod,
                        hipStream_t st);
hipError_t launch_encrypt(const Context& ctx, const uint64_t* m, const uint64_t* e, const uint64_t* a,
                          const uint64_t* s, uint64_t* ct, uint32_t l, hipStream_t st);
hipError_t launch_decrypt(const Context& ctx, const uint64_t* ct, const uint64_t* s, uint64_t* out, uint32_t l,
                          hipStream_t st);
hipError_t launch_encode_small(const Context& ctx, const int64_t* coef, const int32_t* log_approx, uint64_t* out,
                               uint32_t n_vec, uint32_t Np, uint32_t l, const TwPair* tab, hipStream_t st);
hipError_t launch_mul(const Context& ctx, const uint64_t* x, const uint64_t* y, uint64_t* out, uint32_t l,
                      hipStream_t st);
hipError_t launch_pk_mac(const Context& ctx, const uint64_t* pk, const uint64_t* v, const uint64_t* e, uint64_t* x,
                         const std::vector<uint32_t>& pmap, hipStream_t st);

namespace {

#define HIPC(expr)                                                                      \
    do {                                                                                \
        hipError_t _e = (expr);                                                         \
        if (_e != hipSuccess)                                                           \
            throw std::runtime_error(std::string(#expr) + ": " + hipGetErrorString(_e)); \
    } while (0)

constexpr uint32_t kTagKey = 0x59454b53u;   // "SKEY" (seeded_keys.hpp:32)
constexpr uint32_t kTagSecret = 0x52434553u;  // "SECR"
constexpr uint32_t kTagGauss = 0x53554147u;   // "GAUS"
constexpr uint32_t kTagCtA = 0x41585443u;     // "CTXA"
constexpr uint32_t kTagPkA = 0x59454b50u;     // "PKEY"
constexpr uint32_t kTagEncV = 0x56434e45u;    // "ENCV"

// ---------------------------------------------------------------- ChaCha20 (RFC 8439)
inline uint32_t rotl(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

void chacha_block(const uint32_t key[8], uint32_t counter, const uint32_t nonce[3], uint32_t out[16]) {
    const uint32_t init[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, key[0], key[1],
                               key[2],      key[3],      key[4],      key[5],      key[6], key[7],
                               counter,     nonce[0],    nonce[1],    nonce[2]};
    uint32_t x[16];
    std::memcpy(x, init, sizeof(x));
    auto qr = [&](int a, int b, int c, int d) {
        x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 16);
        x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 12);
        x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 8);
        x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 7);
    };
    for (int r = 0; r < 10; r++) {
        qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);
        qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + init[i];
}

class Stream {
public:
    Stream(const uint8_t seed[32], uint32_t w0, uint32_t w1, uint32_t tag) {
        for (int k = 0; k < 8; k++)
            key_[k] = (uint32_t)seed[4 * k] | ((uint32_t)seed[4 * k + 1] << 8) | ((uint32_t)seed[4 * k + 2] << 16) |
                      ((uint32_t)seed[4 * k + 3] << 24);
        nonce_[0] = w0;
        nonce_[1] = w1;
        nonce_[2] = tag;
    }
    uint64_t next() {
        if (pos_ == 8) {
            chacha_block(key_, ctr_++, nonce_, w_);
            pos_ = 0;
        }
        const uint64_t v = (uint64_t)w_[2 * pos_] | ((uint64_t)w_[2 * pos_ + 1] << 32);
        pos_++;
        return v;
    }

private:
    uint32_t key_[8], nonce_[3], w_[16], ctr_ = 0;
    int pos_ = 8;
};

void fill_uniform(const uint8_t seed[32], uint32_t w0, uint32_t w1, uint32_t tag, uint64_t q, uint64_t* out,
                  size_t n) {
    Stream s(seed, w0, w1, tag);
    const uint64_t r = (0 - q) % q, lim = 0 - r;
    for (size_t k = 0; k < n; k++) {
        uint64_t w = s.next();
        while (r != 0 && w >= lim) w = s.next();
        out[k] = w % q;
    }
}

void gauss(const uint8_t seed[32], uint32_t w0, uint32_t w1, double sigma, int64_t* e) {
    Stream s(seed, w0, w1, kTagGauss);
    const double two53 = 9007199254740992.0;
    for (uint32_t k = 0; k < kN; k++) {
        const double u1 = ((double)(s.next() >> 11) + 1.0) / two53;
        const double u2 = (double)(s.next() >> 11) / two53;
        const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
        e[k] = (int64_t)std::llround(sigma * z);
    }
}

// device upload + conversion of signed coefficient polys to the given limbs, evaluation form
struct DevBuf {
    void* p = nullptr;
    explicit DevBuf(size_t bytes) { HIPC(hipMalloc(&p, bytes)); }
    ~DevBuf() { (void)hipFree(p); }
    template <class T>
    T* as() const { return (T*)p; }
};

// signed coefficients (times 2^log_approx) -> residues of the limbs pmap -> NTT
void coeffs_to_eval(Context& ctx, const int64_t* h_coef, uint32_t n_polys, const std::vector<uint32_t>& pmap,
                    uint64_t* d_out, hipStream_t st, uint32_t log_approx = 0) {
    DevBuf dc((size_t)n_polys * kN * 8);
    HIPC(hipMemcpy(dc.p, h_coef, (size_t)n_polys * kN * 8, hipMemcpyHostToDevice));
    HIPC(launch_small_to_rns(ctx, dc.as<int64_t>(), d_out, n_polys, pmap, log_approx, st));
    JobSpec js{};
    js.n_polys = n_polys;
    js.period = (uint32_t)pmap.size();
    for (size_t i = 0; i < pmap.size(); i++) js.pmap[i] = (uint8_t)pmap[i];
    HIPC(launch_ntt(ctx, d_out, js, n_polys * (uint32_t)pmap.size(), false, ctx.ntt_mode, st));
    HIPC(hipStreamSynchronize(st));
}

std::vector<uint32_t> iota(uint32_t n) {
    std::vector<uint32_t> v(n);
    for (uint32_t i = 0; i < n; i++) v[i] = i;
    return v;
}

// ---------------------------------------------------------------- FFT (radix 2, in place)
void fft(std::vector<std::complex<double>>& a, int sign) {
    const size_t n = a.size();
    for (size_t i = 1, j = 0; i < n; i++) {
        size_t bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) std::swap(a[i], a[j]);
    }
    for (size_t len = 2; len <= n; len <<= 1) {
        const size_t h = len / 2;
        std::vector<std::complex<double>> w(h);
        for (size_t k = 0; k < h; k++) {
            const double ang = sign * 2.0 * M_PI * (double)k / (double)len;
            w[k] = std::complex<double>(std::cos(ang), std::sin(ang));
        }
        for (size_t i = 0; i < n; i += len)
            for (size_t k = 0; k < h; k++) {
                const auto u = a[i + k], v = a[i + k + h] * w[k];
                a[i + k] = u + v;
                a[i + k + h] = u - v;
            }
    }
}

// The real coefficients m[0..Np) of the polynomial of the ring of degree Np = 2 slots whose slot j (evaluation at
// zeta'^(5^j), zeta' = exp(i pi / Np)) is scale * (re[j] + i im[j]): the inverse special FFT, unrounded.
void slot_coeffs(const double* re, const double* im, uint32_t slots, double scale, double* m) {
    const uint32_t Np = 2 * slots;
    const uint64_t M = 2ull * Np;
    std::vector<std::complex<double>> v(Np, 0.0);
    uint64_t e = 1;
    for (uint32_t j = 0; j < slots; j++) {
        const std::complex<double> z(re ? re[j] : 0.0, im ? im[j] : 0.0);
        v[(e - 1) / 2] = z * scale;
        v[(M - e - 1) / 2] = std::conj(z) * scale;
        e = e * 5 % M;
    }
    fft(v, -1);  // sum_t v_t w^(-tk)
    for (uint32_t k = 0; k < Np; k++) {
        const double ang = -M_PI * (double)k / (double)Np;  // zeta'^-k
        m[k] = (v[k] * std::complex<double>(std::cos(ang), std::sin(ang))).real() / (double)Np;
    }
}

// t index (evaluation point zeta^(2t+1)) of slot j and of its conjugate
void slot_points(std::vector<uint32_t>& t_of, std::vector<uint32_t>& tc_of) {
    const uint64_t M = 2ull * kN;
    t_of.resize(kN / 2);
    tc_of.resize(kN / 2);
    uint64_t e = 1;
    for (uint32_t j = 0; j < kN / 2; j++) {
        t_of[j] = (uint32_t)((e - 1) / 2);
        tc_of[j] = (uint32_t)((M - e - 1) / 2);
        e = e * 5 % M;
    }
}

}  // namespace

// The rounding rule of encoded coefficients (OpenFHE CKKSPackedEncoding::Encode, restated in
// hpc_gpu_port/periodic_encode.hpp:199-236): logc = the largest ceil(log2 |m_k|) over the nonzero scaled coefficients
// (0 when all are zero; a negative logc -- every coefficient below 1/2 -- is refused as a too small scaling
// factor); coefficients wider than MAX_BITS_IN_WORD = 61 bits are divided by approxFactor = 2^(logc - 61) before
// llround (a quotient above 2^63 - 2^9 - 1 is refused), and the residues are multiplied back by 2^(logc - 61) mod q
// per limb.  Returns log2(approxFactor).
int32_t round_coeffs(const double* m, uint32_t n, int64_t* coef) {
    int32_t logc = INT32_MIN;
    for (uint32_t k = 0; k < n; k++) {
        if (!std::isfinite(m[k])) throw std::invalid_argument("encode: non-finite value");
        if (m[k] != 0.0) logc = std::max(logc, (int32_t)std::ceil(std::log2(std::fabs(m[k]))));
    }
    if (logc == INT32_MIN) logc = 0;
    if (logc < 0) throw std::invalid_argument("encode: scaling factor too small (every coefficient is below 1/2)");
    constexpr int32_t kMaxBitsInWord = 61;
    const int32_t log_approx = logc > kMaxBitsInWord ? logc - kMaxBitsInWord : 0;
    const double approx = std::ldexp(1.0, log_approx);
    const double max_v = (double)(int64_t)((1ull << 63) - (1ull << 9) - 1);
    for (uint32_t k = 0; k < n; k++) {
        const double v = m[k] / approx;
        if (std::fabs(v) > max_v) throw std::invalid_argument("encode: coefficient overflows after approxFactor");
        coef[k] = (int64_t)std::llround(v);
    }
    return log_approx;
}

// ---------------------------------------------------------------- public (C++) API used by abi.cpp
void sample_ternary(const uint8_t seed[32], uint32_t h, int8_t* s) {
    Stream st(seed, 0, 0, kTagSecret);
    std::memset(s, 0, kN);
    for (uint32_t i = 0; i < h && i < kN; i++) {
        for (;;) {
            const uint64_t w = st.next();
            const uint32_t p = (uint32_t)(w & (kN - 1));
            if (s[p]) continue;
            s[p] = (w >> 63) ? -1 : 1;
            break;
        }
    }
}

Secret* secret_create(Context& ctx, const uint8_t seed[32], uint32_t h) {
    auto* sk = new Secret();
    sk->coeffs.resize(kN);
    sample_ternary(seed, h, sk->coeffs.data());
    const uint32_t T = ctx.L + ctx.K;
    try {
        HIPC(hipMalloc(&sk->d_eval, (size_t)T * kN * 8));
        std::vector<int64_t> c(sk->coeffs.begin(), sk->coeffs.end());
        coeffs_to_eval(ctx, c.data(), 1, iota(T), sk->d_eval, nullptr);
    } catch (...) {
        secret_destroy(sk);
        throw;
    }
    return sk;
}

void secret_destroy(Secret* sk) {
    if (!sk) return;
    (void)hipFree(sk->d_eval);
    delete sk;
}

// Key-switching key from s_old (device, evaluation form, Q limbs [L][N]) to s_new (signed coefficients).
// f(0) .. f(n-1) over up to 16 host threads (the limbs of a key are independent streams)
template <class F>
static void parallel_for(uint32_t n, F f) {
    const uint32_t nt = std::min<uint32_t>(n, std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
    std::vector<std::thread> th;
    std::atomic<uint32_t> next{0};
    for (uint32_t t = 0; t < nt; t++)
        th.emplace_back([&] {
            for (uint32_t i; (i = next.fetch_add(1)) < n;) f(i);
        });
    for (auto& x : th) x.join();
}

void keygen_switch(Context& ctx, const uint64_t* d_s_old, const int8_t* s_new, const uint8_t seed[32],
                   const uint8_t eseed[32], double sigma, uint64_t* d_evk) {
    const uint32_t T = ctx.L + ctx.K;
    DevBuf dsn((size_t)T * kN * 8), de((size_t)T * kN * 8);
    std::vector<int64_t> c(s_new, s_new + kN);
    coeffs_to_eval(ctx, c.data(), 1, iota(T), dsn.as<uint64_t>(), nullptr);
    std::vector<TwPair> pmod(T);
    for (uint32_t i = 0; i < T; i++) {
        const uint64_t q = ctx.moduli[i];
        uint64_t P = 1;
        for (uint32_t k = 0; k < ctx.K; k++) P = mulmod_h(P, ctx.moduli[ctx.L + k] % q, q);
        pmod[i] = TwPair{P, (uint64_t)(((unsigned __int128)P << 64) / q)};
    }
    std::vector<uint64_t> a((size_t)T * kN);
    std::vector<int64_t> e(kN);
    for (uint32_t d = 0; d < ctx.dnum; d++) {
        uint64_t* b_d = d_evk + ((size_t)d * 2 + 0) * T * kN;
        uint64_t* a_d = d_evk + ((size_t)d * 2 + 1) * T * kN;
        parallel_for(T, [&](uint32_t i) {
            fill_uniform(seed, d, i, kTagKey, ctx.moduli[i], a.data() + (size_t)i * kN, kN);
        });
        HIPC(hipMemcpy(a_d, a.data(), a.size() * 8, hipMemcpyHostToDevice));
        gauss(eseed, d, 0, sigma, e.data());
        coeffs_to_eval(ctx, e.data(), 1, iota(T), de.as<uint64_t>(), nullptr);
        const uint32_t lo = d * ctx.alpha, hi = std::min(lo + ctx.alpha, ctx.L);
        HIPC(launch_ksk_b(ctx, a_d, dsn.as<uint64_t>(), de.as<uint64_t>(), d_s_old, b_d, lo, hi, pmod.data(), nullptr));
    }
    HIPC(hipDeviceSynchronize());
}

// the a-halves of a key-switching key [dnum][2][L+K][N] (poly 1 of every digit) from its seed, as keygen_switch
// draws them (seeded_keys.hpp:28-43: nonce {digit, limb, "SKEY"})
void expand_key_a(Context& ctx, const uint8_t seed[32], uint64_t* d_evk) {
    const uint32_t T = ctx.L + ctx.K;
    std::vector<uint64_t> a((size_t)T * kN);
    for (uint32_t d = 0; d < ctx.dnum; d++) {
        parallel_for(T, [&](uint32_t i) {
            fill_uniform(seed, d, i, kTagKey, ctx.moduli[i], a.data() + (size_t)i * kN, kN);
        });
        HIPC(hipMemcpy(d_evk + ((size_t)d * 2 + 1) * T * kN, a.data(), a.size() * 8, hipMemcpyHostToDevice));
    }
}

// switching key from sk_from to sk_to; q_limbs > 0 keeps only Q limbs [0, q_limbs) (and P), zeroing the rest:
// a key to a sparse secret is then published at the small modulus q_0..q_{q_limbs-1} P only
void keygen_switch_secret(Context& ctx, const Secret& from, const Secret& to, const uint8_t seed[32],
                          const uint8_t eseed[32], double sigma, uint32_t q_limbs, uint64_t* d_evk) {
    keygen_switch(ctx, from.d_eval, to.coeffs.data(), seed, eseed, sigma, d_evk);
    if (q_limbs == 0 || q_limbs >= ctx.L) return;
    const uint32_t T = ctx.L + ctx.K;
    for (uint32_t dp = 0; dp < 2 * ctx.dnum; dp++)
        HIPC(hipMemset(d_evk + ((size_t)dp * T + q_limbs) * kN, 0, (size_t)(ctx.L - q_limbs) * kN * 8));
    HIPC(hipDeviceSynchronize());
}

void keygen_relin(Context& ctx, const Secret& sk, const uint8_t seed[32], const uint8_t eseed[32], double sigma,
                  uint64_t* d_evk) {
    DevBuf s2((size_t)ctx.L * kN * 8);
    HIPC(launch_mul(ctx, sk.d_eval, sk.d_eval, s2.as<uint64_t>(), ctx.L, nullptr));
    keygen_switch(ctx, s2.as<uint64_t>(), sk.coeffs.data(), seed, eseed, sigma, d_evk);
}

// EvalAutomorphismKeyGen: switch from s to tau_{g^-1}(s) (seeded_keys.hpp:159-168)
void keygen_automorphism(Context& ctx, const Secret& sk, uint32_t g, const uint8_t seed[32], const uint8_t eseed[32],
                         double sigma, uint64_t* d_evk) {
    const uint64_t M = 2ull * kN;
    // g^-1 mod 2N: the order of g in (Z/2N)^* divides N/2, so g^(N/2 - 1) = g^-1
    uint64_t gi = 1, base = g % M;
    for (uint64_t e = kN / 2 - 1; e; e >>= 1) {
        if (e & 1) gi = gi * base % M;
        base = base * base % M;
    }
    std::vector<int8_t> sp(kN, 0);
    for (uint32_t j = 0; j < kN; j++) {
        const uint64_t e = (uint64_t)j * gi % M;
        if (e < kN) sp[e] = (int8_t)(sp[e] + sk.coeffs[j]);
        else sp[e - kN] = (int8_t)(sp[e - kN] - sk.coeffs[j]);
    }
    keygen_switch(ctx, sk.d_eval, sp.data(), seed, eseed, sigma, d_evk);
}

// values (re, im may be null) of n_slots slots, replicated to N/2 when n_slots divides N/2
void encode(Context& ctx, const double* re, const double* im, uint32_t n_slots, uint32_t l, double scale,
            uint64_t* d_pt) {
    encode_primes(ctx, re, im, n_slots, iota(l), scale, d_pt);
}

// the same plaintext over the primes pmap (limb t of the output is mod prime pmap[t]).  A vector of n_slots < N/2
// (replicated over the N/2 slots) is sparsely packed as OpenFHE packs a batch smaller than N/2: the coefficients
// are those of the ring of degree 2 n_slots, placed at stride N / (2 n_slots) -- the same polynomial the full
// special FFT of the replicated vector describes, computed from one period.
void encode_primes(Context& ctx, const double* re, const double* im, uint32_t n_slots,
                   const std::vector<uint32_t>& pmap, double scale, uint64_t* d_pt) {
    if (n_slots == 0 || (kN / 2) % n_slots != 0) throw std::invalid_argument("n_slots must divide N/2");
    const uint32_t Np = 2 * n_slots, rep = kN / Np;
    std::vector<double> m(Np);
    slot_coeffs(re, im, n_slots, scale, m.data());
    std::vector<int64_t> small(Np), coef(kN, 0);
    const int32_t log_approx = round_coeffs(m.data(), Np, small.data());
    for (uint32_t k = 0; k < Np; k++) coef[(size_t)k * rep] = small[k];
    coeffs_to_eval(ctx, coef.data(), 1, pmap, d_pt, nullptr, (uint32_t)log_approx);
}

// the N'-point table Table[brev(j)] = psi'^j, psi' = psi^(N/N'), per prime of the chain (made on first use)
static const TwPair* small_table(Context& ctx, uint32_t Np) {
    auto it = ctx.small_ntt.find(Np);
    if (it == ctx.small_ntt.end()) {
        uint32_t logNp = 0;
        while ((1u << logNp) < Np) logNp++;
        const uint32_t rep = kN / Np, T = ctx.L + ctx.K;
        std::vector<TwPair> tabs((size_t)T * Np);
        for (uint32_t i = 0; i < T; i++) {
            const uint64_t q = ctx.moduli[i];
            const uint64_t psi_p = powmod_h(ctx.psi[i], rep, q);
            uint64_t x = 1;
            for (uint32_t j = 0; j < Np; j++) {
                uint32_t r = 0;
                for (uint32_t t = 0, v = j; t < logNp; t++, v >>= 1) r = (r << 1) | (v & 1);
                tabs[(size_t)i * Np + r] = TwPair{x, (uint64_t)(((unsigned __int128)x << 64) / q)};
                x = mulmod_h(x, psi_p, q);
            }
        }
        TwPair* d = nullptr;
        HIPC(hipMalloc(&d, tabs.size() * sizeof(TwPair)));
        HIPC(hipMemcpy(d, tabs.data(), tabs.size() * sizeof(TwPair), hipMemcpyHostToDevice));
        it = ctx.small_ntt.emplace(Np, d).first;
    }
    return it->second;
}

static void check_period(uint32_t P) {
    if (P < 2 || (P & (P - 1)) || P > 2048) throw std::invalid_argument("period must be a power of two in [2, 2048]");
}

// Periodic plaintexts (hpc_gpu_port/periodic_encode.hpp:179-260).  A slot vector of period P (replicated REP = N/(2P) times) is the encoding of a polynomial in
// X^REP, i.e. of one period in the ring of degree N' = 2P.  Its evaluation form, in the bit-reversed order of the
// N-point NTT, has word k equal to word k >> log2(REP) of the N'-point NTT (root psi^REP) of that small polynomial,
// so only N' words per limb are stored.  The special FFT and rounding run on the host (over threads): their result,
// the small polynomial's integer coefficients (and each vector's approxFactor exponent), is independent of the
// level and N' words per vector in all; the residues and the N'-point NTTs of any number of limbs follow on the GPU.
// d_coef [n_vec][N'] int64, d_log_approx [n_vec] int32 (device memory, or pinned host memory).
void encode_periodic_coeffs(Context& ctx, const double* re, const double* im, uint32_t n_vec, uint32_t P,
                            double scale, int64_t* d_coef, int32_t* d_log_approx) {
    (void)ctx;
    check_period(P);
    const uint32_t Np = 2 * P;
    std::vector<int64_t> coef((size_t)n_vec * Np);
    std::vector<int32_t> log_approx(n_vec, 0);
    std::vector<std::string> errs(n_vec);
    parallel_for(n_vec, [&](uint32_t n) {
        std::vector<double> m(Np);
        slot_coeffs(re ? re + (size_t)n * P : nullptr, im ? im + (size_t)n * P : nullptr, P, scale, m.data());
        try {
            log_approx[n] = round_coeffs(m.data(), Np, coef.data() + (size_t)n * Np);
        } catch (const std::exception& e) {
            errs[n] = e.what();
        }
    });
    for (const auto& e : errs)
        if (!e.empty()) throw std::invalid_argument(e);
    // device or pinned host destinations
    HIPC(hipMemcpy(d_coef, coef.data(), coef.size() * 8, hipMemcpyDefault));
    HIPC(hipMemcpy(d_log_approx, log_approx.data(), log_approx.size() * 4, hipMemcpyDefault));
}

// the device half: coefficients -> [n_vec][l][N'] evaluation-form limbs, enqueued on st
void expand_periodic(Context& ctx, const int64_t* d_coef, const int32_t* d_log_approx, uint32_t n_vec, uint32_t P,
                     uint32_t l, uint64_t* d_out, hipStream_t st) {
    check_period(P);
    const TwPair* tab = small_table(ctx, 2 * P);
    HIPC(launch_encode_small(ctx, d_coef, d_log_approx, d_out, n_vec, 2 * P, l, tab, st));
}

// both halves: out [n_vec][l][N']
void encode_periodic(Context& ctx, const double* re, const double* im, uint32_t n_vec, uint32_t P, uint32_t l,
                     double scale, uint64_t* d_out) {
    check_period(P);
    DevBuf dc((size_t)n_vec * 2 * P * 8), dl((size_t)n_vec * 4);
    encode_periodic_coeffs(ctx, re, im, n_vec, P, scale, dc.as<int64_t>(), dl.as<int32_t>());
    expand_periodic(ctx, dc.as<int64_t>(), dl.as<int32_t>(), n_vec, P, l, d_out, nullptr);
    HIPC(hipDeviceSynchronize());
}

void encrypt(Context& ctx, const Secret& sk, const uint64_t* d_pt, uint32_t l, const uint8_t seed[32],
             uint32_t index, uint64_t* d_ct) {
    DevBuf da((size_t)l * kN * 8), de((size_t)l * kN * 8);
    std::vector<uint64_t> a((size_t)l * kN);
    for (uint32_t i = 0; i < l; i++) fill_uniform(seed, index, i, kTagCtA, ctx.moduli[i], a.data() + (size_t)i * kN, kN);
    HIPC(hipMemcpy(da.p, a.data(), a.size() * 8, hipMemcpyHostToDevice));
    std::vector<int64_t> e(kN);
    gauss(seed, index, 1, 3.19, e.data());
    coeffs_to_eval(ctx, e.data(), 1, iota(l), de.as<uint64_t>(), nullptr);
    HIPC(launch_encrypt(ctx, d_pt, de.as<uint64_t>(), da.as<uint64_t>(), sk.d_eval, d_ct, l, nullptr));
    HIPC(hipDeviceSynchronize());
}

// Public key over Q*P (PKEBase::KeyGenInternal, harness/boot_overflow_probe.cpp:22,139): b = e - a s, a uniform
// (ChaCha20 "PKEY" stream, nonce {0, limb}), e rounded Gaussian (stream {0, 0} of eseed): the secret-key
// encryption of zero over all L+K limbs.  d_pk [2][L+K][N].
void keygen_public(Context& ctx, const Secret& sk, const uint8_t seed[32], const uint8_t eseed[32], double sigma,
                   uint64_t* d_pk) {
    const uint32_t T = ctx.L + ctx.K;
    DevBuf da((size_t)T * kN * 8), de((size_t)T * kN * 8), dz((size_t)T * kN * 8);
    std::vector<uint64_t> a((size_t)T * kN);
    parallel_for(T, [&](uint32_t i) { fill_uniform(seed, 0, i, kTagPkA, ctx.moduli[i], a.data() + (size_t)i * kN, kN); });
    HIPC(hipMemcpy(da.p, a.data(), a.size() * 8, hipMemcpyHostToDevice));
    std::vector<int64_t> e(kN);
    gauss(eseed, 0, 0, sigma, e.data());
    coeffs_to_eval(ctx, e.data(), 1, iota(T), de.as<uint64_t>(), nullptr);
    HIPC(hipMemset(dz.p, 0, (size_t)T * kN * 8));
    HIPC(launch_encrypt(ctx, de.as<uint64_t>(), dz.as<uint64_t>(), da.as<uint64_t>(), sk.d_eval, d_pk, T, nullptr));
    HIPC(hipDeviceSynchronize());
}

// Public-key encryption at level l (PKEBase::EncryptZeroCore with the key over Q*P, then ApproxModDown to Q_l):
// x = (b v + e0, a v + e1) over Q_l * P with v uniform ternary ("ENCV" stream {index, 0}, words mod 3: 0, 1, 2 ->
// 0, 1, -1) and e0, e1 rounded Gaussians (streams {index, 2}, {index, 3}); ct = (ModDown(x0) + m, ModDown(x1)).
void encrypt_public(Context& ctx, const uint64_t* d_pk, const uint64_t* d_pt, uint32_t l, const uint8_t seed[32],
                    uint32_t index, uint64_t* d_ct) {
    const uint32_t E = l + ctx.K;
    if (ctx.K == 0) throw std::invalid_argument("public-key encryption needs special primes (the key is over Q*P)");
    std::vector<uint32_t> pm(E);
    for (uint32_t t = 0; t < E; t++) pm[t] = t < l ? t : ctx.L + (t - l);
    std::vector<int64_t> c(3 * (size_t)kN);
    std::vector<uint64_t> u(kN);
    fill_uniform(seed, index, 0, kTagEncV, 3, u.data(), kN);
    for (uint32_t k = 0; k < kN; k++) c[k] = u[k] == 2 ? -1 : (int64_t)u[k];
    gauss(seed, index, 2, 3.19, c.data() + kN);
    gauss(seed, index, 3, 3.19, c.data() + 2 * (size_t)kN);
    DevBuf dv((size_t)3 * E * kN * 8), dx((size_t)2 * E * kN * 8);
    coeffs_to_eval(ctx, c.data(), 3, pm, dv.as<uint64_t>(), nullptr);  // [3][E][N]: v, e0, e1
    uint64_t* v = dv.as<uint64_t>();
    HIPC(launch_pk_mac(ctx, d_pk, v, v + (size_t)E * kN, dx.as<uint64_t>(), pm, nullptr));
    moddown_inplace(ctx, dx.as<uint64_t>(), 2, l, d_pt, d_ct, nullptr, 2);
    HIPC(hipDeviceSynchronize());
}

// decrypt (c0 + c1 s) to centered coefficients (CRT of the first two limbs, |m| < q0 q1 / 2), as doubles
void decrypt_coeffs(Context& ctx, const Secret& sk, const uint64_t* d_ct, uint32_t l, double* out) {
    DevBuf dm((size_t)l * kN * 8);
    HIPC(launch_decrypt(ctx, d_ct, sk.d_eval, dm.as<uint64_t>(), l, nullptr));
    const uint32_t nl = l >= 2 ? 2 : 1;
    JobSpec js{};
    js.n_polys = 1;
    js.period = nl;
    for (uint32_t i = 0; i < nl; i++) js.pmap[i] = (uint8_t)i;
    HIPC(launch_ntt(ctx, dm.as<uint64_t>(), js, nl, true, ctx.ntt_mode, nullptr));
    std::vector<uint64_t> limbs((size_t)nl * kN);
    HIPC(hipMemcpy(limbs.data(), dm.p, limbs.size() * 8, hipMemcpyDeviceToHost));
    const uint64_t q0 = ctx.moduli[0];
    for (uint32_t k = 0; k < kN; k++) {
        if (nl == 1) {
            const uint64_t x = limbs[k];
            out[k] = x > q0 / 2 ? -(double)(q0 - x) : (double)x;
        } else {
            const uint64_t q1 = ctx.moduli[1];
            const uint64_t x0 = limbs[k], x1 = limbs[kN + k];
            const uint64_t d = mulmod_h((x1 + q1 - x0 % q1) % q1, invmod_h(q0 % q1, q1), q1);
            const unsigned __int128 Q = (unsigned __int128)q0 * q1;
            const unsigned __int128 x = (unsigned __int128)d * q0 + x0;
            out[k] = x > Q / 2 ? -(double)(Q - x) : (double)x;
        }
    }
}

// decrypt (c0 + c1 s), to coefficients, CRT of the first two limbs (|m| < q0 q1 / 2), decode
void decrypt_decode(Context& ctx, const Secret& sk, const uint64_t* d_ct, uint32_t l, double scale, double* re,
                    double* im, uint32_t n_slots) {
    if (n_slots == 0 || n_slots > kN / 2) throw std::invalid_argument("n_slots must be in [1, N/2]");
    DevBuf dm((size_t)l * kN * 8);
    HIPC(launch_decrypt(ctx, d_ct, sk.d_eval, dm.as<uint64_t>(), l, nullptr));
    const uint32_t nl = l >= 2 ? 2 : 1;
    JobSpec js{};
    js.n_polys = 1;
    js.period = nl;
    for (uint32_t i = 0; i < nl; i++) js.pmap[i] = (uint8_t)i;
    HIPC(launch_ntt(ctx, dm.as<uint64_t>(), js, nl, true, ctx.ntt_mode, nullptr));
    std::vector<uint64_t> limbs((size_t)nl * kN);
    HIPC(hipMemcpy(limbs.data(), dm.p, limbs.size() * 8, hipMemcpyDeviceToHost));
    const uint64_t q0 = ctx.moduli[0];
    std::vector<std::complex<double>> v(kN);
    for (uint32_t k = 0; k < kN; k++) {
        double m;
        if (nl == 1) {
            const uint64_t x = limbs[k];
            m = x > q0 / 2 ? -(double)(q0 - x) : (double)x;
        } else {
            const uint64_t q1 = ctx.moduli[1];
            const uint64_t x0 = limbs[k], x1 = limbs[kN + k];
            const uint64_t q0inv = invmod_h(q0 % q1, q1);
            const uint64_t d = mulmod_h((x1 + q1 - x0 % q1) % q1, q0inv, q1);
            const unsigned __int128 Q = (unsigned __int128)q0 * q1;
            const unsigned __int128 x = (unsigned __int128)d * q0 + x0;
            m = x > Q / 2 ? -(double)(Q - x) : (double)x;
        }
        const double ang = M_PI * (double)k / (double)kN;  // zeta^k
        v[k] = std::complex<double>(m * std::cos(ang), m * std::sin(ang));
    }
    fft(v, +1);
    std::vector<uint32_t> t_of, tc_of;
    slot_points(t_of, tc_of);
    for (uint32_t j = 0; j < n_slots; j++) {
        const auto z = v[t_of[j]] / scale;
        if (re) re[j] = z.real();
        if (im) im[j] = z.imag();
    }
}

}  // namespace fhe
