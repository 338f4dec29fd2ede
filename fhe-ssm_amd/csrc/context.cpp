// context.cpp -- parameter generation (prime chain, roots, NTT tables) and device upload.
#include <hip/hip_runtime.h>

#include <cstring>
#include <stdexcept>
#include <string>

#include "ckks_engine.h"
#include "engine.hpp"

namespace fhe {

using u128 = unsigned __int128;

uint64_t mulmod_h(uint64_t a, uint64_t b, uint64_t q) { return (uint64_t)((u128)a * b % q); }

uint64_t powmod_h(uint64_t a, uint64_t e, uint64_t q) {
    uint64_t r = 1 % q;
    a %= q;
    for (; e; e >>= 1) {
        if (e & 1) r = mulmod_h(r, a, q);
        a = mulmod_h(a, a, q);
    }
    return r;
}

uint64_t invmod_h(uint64_t a, uint64_t q) { return powmod_h(a, q - 2, q); }

bool is_prime_h(uint64_t n) {
    static const uint64_t bases[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
    if (n < 2) return false;
    for (uint64_t b : bases) {
        if (n == b) return true;
        if (n % b == 0) return false;
    }
    uint64_t d = n - 1;
    int r = 0;
    while (!(d & 1)) d >>= 1, r++;
    for (uint64_t b : bases) {
        uint64_t x = powmod_h(b, d, n);
        if (x == 1 || x == n - 1) continue;
        bool composite = true;
        for (int i = 1; i < r && composite; i++) {
            x = mulmod_h(x, x, n);
            if (x == n - 1) composite = false;
        }
        if (composite) return false;
    }
    return true;
}

// largest primes below 2^bits with p = 1 mod m, excluding `skip`
std::vector<uint64_t> ntt_primes(uint32_t bits, uint32_t count, uint64_t m, const std::vector<uint64_t>& skip) {
    std::vector<uint64_t> out;
    const uint64_t top = 1ull << bits;
    uint64_t c = top - (top % m) + 1;
    if (c >= top) c -= m;
    for (; out.size() < count && c > m; c -= m) {
        bool excluded = false;
        for (uint64_t s : skip) excluded |= (s == c);
        if (!excluded && is_prime_h(c)) out.push_back(c);
    }
    if (out.size() != count) throw std::runtime_error("not enough NTT primes below 2^" + std::to_string(bits));
    return out;
}

// smallest primitive m-th root of unity mod q (m a power of two)
uint64_t min_root_h(uint64_t q, uint64_t m) {
    uint64_t psi = 0;
    for (uint64_t g = 2; g < q && !psi; g++) {
        const uint64_t x = powmod_h(g, (q - 1) / m, q);
        if (powmod_h(x, m / 2, q) == q - 1) psi = x;
    }
    if (!psi) throw std::runtime_error("no primitive root");
    uint64_t best = psi, cur = psi;
    const uint64_t sq = mulmod_h(psi, psi, q);
    for (uint64_t j = 1; j < m / 2; j++) {
        cur = mulmod_h(cur, sq, q);
        if (cur < best) best = cur;
    }
    return best;
}

static uint32_t brev(uint32_t v, uint32_t bits) {
    uint32_t r = 0;
    for (uint32_t b = 0; b < bits; b++, v >>= 1) r = (r << 1) | (v & 1);
    return r;
}

static uint64_t shoup_companion(uint64_t w, uint64_t q) { return (uint64_t)(((u128)w << 64) / q); }

PrimeInfo make_prime_info(uint64_t q, uint64_t itab1) {
    PrimeInfo p{};
    p.q = q;
    p.ninv = invmod_h(kN % q, q);
    // the last inverse NTT stage multiplies by N^-1 as a - b c with c = q - N^-1 = (q - 1) / N (q = 1 mod 2N)
    if ((q - 1) % (2 * (uint64_t)kN) != 0 || p.ninv != q - (q - 1) / kN)
        throw std::invalid_argument("modulus is not 1 mod 2N");
    p.ninv_p = shoup_companion(p.ninv, q);
    p.w1ninv = mulmod_h(itab1, p.ninv, q);
    p.w1ninv_p = shoup_companion(p.w1ninv, q);
    // mu = floor(2^128 / q) = floor((2^128 - 1) / q) for q not a power of two
    const u128 mu = ~(u128)0 / q;
    p.mu_hi = (uint64_t)(mu >> 64);
    p.mu_lo = (uint64_t)mu;
    const uint32_t bits = 64 - (uint32_t)__builtin_clzll(q);
    p.red_shift = bits > 25 ? bits - 25 : 0;
    p.red_mul = (uint32_t)(((u128)1 << (32 + p.red_shift)) / q);
    // q^-1 mod 2^64 by Newton's iteration (q odd: x = q is correct to 3 bits, each step doubles them)
    uint64_t x = q;
    for (int i = 0; i < 5; i++) x *= 2 - q * x;
    p.mont_ninv = 0 - x;
    p.r_mod = (uint64_t)(((u128)1 << 64) % q);
    p.r_mod_p = shoup_companion(p.r_mod, q);
    return p;
}

void context_init(Context& c, const std::vector<uint64_t>& q, const std::vector<uint64_t>& p, uint32_t dnum,
                  double scale, int device) {
    if (q.empty() || dnum == 0 || dnum > q.size()) throw std::invalid_argument("bad num_q / dnum");
    if (q.size() + p.size() > kMaxPrimes) throw std::invalid_argument("too many primes");
    c.device = device;
    c.L = (uint32_t)q.size();
    c.K = (uint32_t)p.size();
    c.dnum = dnum;
    c.alpha = (c.L + dnum - 1) / dnum;
    c.scale = scale;
    c.moduli = q;
    c.moduli.insert(c.moduli.end(), p.begin(), p.end());
    const uint32_t T = c.L + c.K;
    for (uint64_t m : c.moduli)
        if (m >= (1ull << 60) || (m - 1) % (2ull * kN) != 0 || !is_prime_h(m))
            throw std::invalid_argument("modulus is not an NTT prime below 2^60: " + std::to_string(m));
    std::vector<TwPair> tw((size_t)T * kN), itw((size_t)T * kN);
    c.psi.resize(T);
    c.primes.resize(T);
    for (uint32_t i = 0; i < T; i++) {
        const uint64_t m = c.moduli[i];
        const uint64_t psi = min_root_h(m, 2ull * kN), psiinv = invmod_h(psi, m);
        c.psi[i] = psi;
        uint64_t x = 1, y = 1;
        TwPair* t = tw.data() + (size_t)i * kN;
        TwPair* it = itw.data() + (size_t)i * kN;
        for (uint32_t j = 0; j < kN; j++) {
            const uint32_t r = brev(j, kLogN);
            t[r] = TwPair{x, shoup_companion(x, m)};
            it[r] = TwPair{y, shoup_companion(y, m)};
            x = mulmod_h(x, psi, m);
            y = mulmod_h(y, psiinv, m);
        }
        c.primes[i] = make_prime_info(m, it[1].w);
    }
    for (uint32_t i = 0; i < c.L; i++) {
        PrimeInfo& pi = c.primes[i];
        uint64_t pm = 1;
        for (uint32_t k = 0; k < c.K; k++) pm = mulmod_h(pm, c.moduli[c.L + k] % pi.q, pi.q);
        pi.pmod = pm;
        pi.rpinv = mulmod_h(pi.r_mod, invmod_h(pm, pi.q), pi.q);
        pi.rpinv_p = shoup_companion(pi.rpinv, pi.q);
    }
    if (hipSetDevice(device) != hipSuccess) throw std::runtime_error("hipSetDevice failed");
    // the allocation-free entry point's scratch on this device: its address resolved once, with the device current
    if (scratch_init(device) != hipSuccess) throw std::runtime_error("device scratch address lookup failed");
    auto up = [](void** d, const void* h, size_t bytes) {
        if (hipMalloc(d, bytes) != hipSuccess) throw std::runtime_error("hipMalloc failed");
        if (hipMemcpy(*d, h, bytes, hipMemcpyHostToDevice) != hipSuccess) throw std::runtime_error("hipMemcpy failed");
    };
    up((void**)&c.d_tw, tw.data(), tw.size() * sizeof(TwPair));
    up((void**)&c.d_itw, itw.data(), itw.size() * sizeof(TwPair));
    // pass B's tables: within each block of 16 * 2^m entries of a strided stage, entry rl 2^m + kk moves to kk 16 + rl
    // (forward stages 8 + s, s = 5..7, m = s - 4, blocks of 2^s at 2^(8+s) + b 2^s; inverse t = 2^u, u = 0..2,
    // m = 3 - u, blocks of 2^(7-u) at 2^(15-u) + b 2^(7-u))
    std::vector<TwPair> twb(tw), itwb(itw);
    for (uint32_t i = 0; i < T; i++) {
        const size_t base = (size_t)i * kN;
        for (uint32_t m = 1; m <= 3; m++) {
            const size_t f0 = (size_t)1 << (12 + m), i0 = (size_t)1 << (12 + m);  // forward s = 4 + m; inverse u = 3 - m
            const uint32_t bs = 16u << m;
            for (uint32_t b = 0; b < 256; b++)
                for (uint32_t rl = 0; rl < 16; rl++)
                    for (uint32_t kk = 0; kk < (1u << m); kk++) {
                        twb[base + f0 + (size_t)b * bs + kk * 16 + rl] = tw[base + f0 + (size_t)b * bs + (rl << m) + kk];
                        itwb[base + i0 + (size_t)b * bs + kk * 16 + rl] =
                            itw[base + i0 + (size_t)b * bs + (rl << m) + kk];
                    }
        }
    }
    // and the broadcast stages (forward s = 1..3, inverse u = 4..6): entry b 2^s + j of a region moves to j 256 + b
    for (uint32_t i = 0; i < T; i++) {
        const size_t base = (size_t)i * kN;
        for (uint32_t s = 1; s <= 3; s++) {
            const size_t r0 = (size_t)256 << s;  // forward stage 8 + s; the inverse u = 7 - s has the same region
            for (uint32_t b = 0; b < 256; b++)
                for (uint32_t j = 0; j < (1u << s); j++) {
                    twb[base + r0 + (size_t)j * 256 + b] = tw[base + r0 + ((size_t)b << s) + j];
                    itwb[base + r0 + (size_t)j * 256 + b] = itw[base + r0 + ((size_t)b << s) + j];
                }
        }
    }
    up((void**)&c.d_twb, twb.data(), twb.size() * sizeof(TwPair));
    up((void**)&c.d_itwb, itwb.data(), itwb.size() * sizeof(TwPair));
    up((void**)&c.d_primes, c.primes.data(), c.primes.size() * sizeof(PrimeInfo));
}

std::string set_phase(Context& ctx, const std::string& phase, hipStream_t st) {
    std::string old = ctx.prof_phase;
    if (phase == old) return old;
    ctx.prof_phase = phase;
    if (ctx.phase_marks && !ctx.arena) {
        auto it = ctx.phase_ids.find(phase);
        if (it == ctx.phase_ids.end()) it = ctx.phase_ids.emplace(phase, (uint32_t)ctx.phase_ids.size()).first;
        (void)launch_phase_mark(it->second, st);
    }
    return old;
}

int prof_begin(const Context& ctx, const char* name, double bytes, hipStream_t st) {
    if (!ctx.prof_on || ctx.arena) return -1;  // no events are created inside an allocation-free call
    ProfRec r{name, bytes, nullptr, nullptr, ctx.prof_phase};
    if (hipEventCreate(&r.e0) != hipSuccess || hipEventCreate(&r.e1) != hipSuccess) return -1;
    if (hipEventRecord(r.e0, st) != hipSuccess) return -1;
    ctx.prof.push_back(r);
    return (int)ctx.prof.size() - 1;
}

void prof_end(const Context& ctx, int idx, hipStream_t st) {
    if (idx < 0 || idx >= (int)ctx.prof.size()) return;
    (void)hipEventRecord(ctx.prof[idx].e1, st);
}

void prof_clear(const Context& ctx) {
    for (auto& r : ctx.prof) {
        (void)hipEventDestroy(r.e0);
        (void)hipEventDestroy(r.e1);
    }
    ctx.prof.clear();
}

void context_release(Context& c) {
    (void)hipFree(c.d_tw);
    (void)hipFree(c.d_itw);
    (void)hipFree(c.d_twb);
    (void)hipFree(c.d_itwb);
    (void)hipFree(c.d_primes);
    for (auto& kv : c.job_cache) (void)hipFree(kv.second.first);
    prof_clear(c);
    for (auto& kv : c.bconv_cache) (void)hipFree(kv.second.d_tab);
    for (auto& s : c.scratch) (void)hipFree(s.first);
    for (auto& kv : c.small_ntt) (void)hipFree(kv.second);
    c.small_ntt.clear();
    for (auto& kv : c.buf_pool)
        for (auto* p : kv.second) (void)hipFree(p);
    c.buf_pool.clear();
    if (c.ring_host) (void)hipHostFree(c.ring_host);
    if (c.ring_dev) (void)hipFree(c.ring_dev);
    for (auto& e : c.ring_ev)
        if (e) (void)hipEventDestroy(e);
    c.ring_host = c.ring_dev = nullptr;
    if (c.side) (void)hipStreamSynchronize(c.side);
    if (c.side_out) (void)hipStreamSynchronize(c.side_out);
    for (auto& kv : c.side_ev) (void)hipEventDestroy(kv.second);
    c.side_ev.clear();
    for (auto ev : c.side_after) (void)hipEventDestroy(ev);
    c.side_after.clear();
    if (c.side) (void)hipStreamDestroy(c.side);
    if (c.side_out) (void)hipStreamDestroy(c.side_out);
    c.side = nullptr;
    c.side_out = nullptr;
    c.job_cache.clear();
    c.bconv_cache.clear();
    c.scratch.clear();
    c.d_tw = c.d_itw = c.d_twb = c.d_itwb = nullptr;
    c.d_primes = nullptr;
}

}  // namespace fhe
