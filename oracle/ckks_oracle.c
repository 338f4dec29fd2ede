/*
 * ckks_oracle.c -- CPU restatement of the RNS-CKKS integer core.  TEST INFRASTRUCTURE ONLY:
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the
 * product never links it.  Every function cites the reference file:line whose convention it follows
 * (the header lists them); how each is pinned is stated in ckks_oracle.h.
 */
#include "ckks_oracle.h"

#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

/* ------------------------------------------------------------------ scalar arithmetic */

uint64_t or_mulmod(uint64_t a, uint64_t b, uint64_t q) { return (uint64_t)(((u128)a * b) % q); }

uint64_t or_powmod(uint64_t a, uint64_t e, uint64_t q) {
    uint64_t r = 1 % q;
    a %= q;
    while (e) {
        if (e & 1) r = or_mulmod(r, a, q);
        a = or_mulmod(a, a, q);
        e >>= 1;
    }
    return r;
}

/* q prime: a^(q-2) */
uint64_t or_invmod(uint64_t a, uint64_t q) { return or_powmod(a, q - 2, q); }

/* Deterministic Miller-Rabin for n < 2^64 (bases = first 12 primes). */
int or_is_prime(uint64_t n) {
    static const uint64_t bases[12] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
    if (n < 2) return 0;
    for (int i = 0; i < 12; i++) {
        if (n == bases[i]) return 1;
        if (n % bases[i] == 0) return 0;
    }
    uint64_t d = n - 1;
    int r = 0;
    while ((d & 1) == 0) { d >>= 1; r++; }
    for (int i = 0; i < 12; i++) {
        uint64_t x = or_powmod(bases[i], d, n);
        if (x == 1 || x == n - 1) continue;
        int comp = 1;
        for (int k = 1; k < r; k++) {
            x = or_mulmod(x, x, n);
            if (x == n - 1) { comp = 0; break; }
        }
        if (comp) return 0;
    }
    return 1;
}

uint32_t or_bitrev(uint32_t v, uint32_t bits) {
    uint32_t r = 0;
    for (uint32_t b = 0; b < bits; b++) { r = (r << 1) | (v & 1u); v >>= 1; }
    return r;
}

uint32_t or_gen_primes(uint32_t bits, uint32_t count, uint64_t m, const uint64_t* exclude,
                       uint32_t n_exclude, uint64_t* out) {
    /* largest candidate below 2^bits that is 1 mod m, then step down by m */
    uint64_t top = (bits >= 64) ? ~0ull : (1ull << bits);
    uint64_t cand = top - (top % m) + 1;
    if (cand >= top) cand -= m;
    uint32_t found = 0;
    while (found < count && cand > m) {
        int skip = 0;
        for (uint32_t i = 0; i < n_exclude; i++) if (exclude[i] == cand) skip = 1;
        if (!skip && or_is_prime(cand)) out[found++] = cand;
        cand -= m;
    }
    return found;
}

/* m = 2^k.  A primitive m-th root is g^((q-1)/m) for any quadratic non-residue-rich element g whose
 * image has order exactly m; we scan g = 2,3,... for one, then take the minimum over all odd powers
 * (every primitive m-th root is psi^j for odd j).  The minimum makes the choice independent of g. */
uint64_t or_min_root(uint64_t q, uint64_t m) {
    uint64_t psi = 0;
    for (uint64_t g = 2; g < q; g++) {
        uint64_t x = or_powmod(g, (q - 1) / m, q);
        if (or_powmod(x, m / 2, q) == q - 1) { psi = x; break; }
    }
    if (!psi) return 0;
    uint64_t best = psi, sq = or_mulmod(psi, psi, q), cur = psi;
    for (uint64_t j = 1; j < m / 2; j++) {  /* cur = psi^(2j+1) */
        cur = or_mulmod(cur, sq, q);
        if (cur < best) best = cur;
    }
    return best;
}

/* ------------------------------------------------------------------ context */

int or_ctx_init(or_ctx* c, uint32_t logN, const uint64_t* moduli, uint32_t L, uint32_t K, uint32_t dnum) {
    memset(c, 0, sizeof(*c));
    if (L + K > OR_MAX_PRIMES || L == 0 || dnum == 0) return -1;
    c->logN = logN;
    c->N = 1u << logN;
    c->L = L;
    c->K = K;
    c->dnum = dnum;
    c->alpha = (L + dnum - 1) / dnum;
    const uint32_t N = c->N, T = L + K;
    c->tab = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)T * N);
    c->tabp = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)T * N);
    c->itab = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)T * N);
    c->itabp = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)T * N);
    if (!c->tab || !c->tabp || !c->itab || !c->itabp) return -2;
    for (uint32_t p = 0; p < T; p++) {
        const uint64_t q = moduli[p];
        if ((q - 1) % (2ull * N) != 0 || q >= (1ull << 62)) return -3;
        c->q[p] = q;
        c->psi[p] = or_min_root(q, 2ull * N);
        if (!c->psi[p]) return -4;
        c->ninv[p] = or_invmod(N, q);
        /* periodic_encode.hpp:150-160: Table[brev(i)] = psi^i; Shoup w' = floor(w * 2^64 / q) */
        const uint64_t psiinv = or_invmod(c->psi[p], q);
        uint64_t x = 1, y = 1;
        uint64_t* t = c->tab + (size_t)p * N;
        uint64_t* tp = c->tabp + (size_t)p * N;
        uint64_t* it = c->itab + (size_t)p * N;
        uint64_t* itp = c->itabp + (size_t)p * N;
        for (uint32_t i = 0; i < N; i++) {
            const uint32_t ir = or_bitrev(i, logN);
            t[ir] = x;
            tp[ir] = (uint64_t)(((u128)x << 64) / q);
            it[ir] = y;
            itp[ir] = (uint64_t)(((u128)y << 64) / q);
            x = or_mulmod(x, c->psi[p], q);
            y = or_mulmod(y, psiinv, q);
        }
    }
    return 0;
}

void or_ctx_free(or_ctx* c) {
    free(c->tab);
    free(c->tabp);
    free(c->itab);
    free(c->itabp);
    c->tab = c->tabp = c->itab = c->itabp = NULL;
}

/* ------------------------------------------------------------------ NTT */

/* periodic_encode.hpp:115-120 */
static inline uint64_t mul_shoup(uint64_t x, uint64_t w, uint64_t wp, uint64_t q) {
    const uint64_t hi = (uint64_t)(((u128)x * wp) >> 64);
    uint64_t r = x * w - hi * q;
    return r >= q ? r - q : r;
}

/* periodic_encode.hpp:240-260 (OpenFHE ForwardTransformToBitReverse): natural in, bit-reversed out */
void or_ntt_fwd(const or_ctx* c, uint32_t pi, uint64_t* a) {
    const uint64_t q = c->q[pi];
    const uint64_t* tab = c->tab + (size_t)pi * c->N;
    const uint64_t* tabp = c->tabp + (size_t)pi * c->N;
    const uint32_t n = c->N;
    for (uint32_t m = 1, t = n >> 1; m < n; m <<= 1, t >>= 1) {
        for (uint32_t i = 0; i < m; ++i) {
            const uint32_t j1 = i * (t << 1), j2 = j1 + t;
            const uint64_t w = tab[m + i], wp = tabp[m + i];
            for (uint32_t lo = j1; lo < j2; ++lo) {
                const uint32_t hi = lo + t;
                const uint64_t x = mul_shoup(a[hi], w, wp, q);
                const uint64_t lv = a[lo];
                uint64_t hv = lv + x;
                if (hv >= q) hv -= q;
                const uint64_t lw = lv >= x ? lv - x : lv + q - x;
                a[lo] = hv;
                a[hi] = lw;
            }
        }
    }
}

/* OpenFHE InverseTransformFromBitReverse: Gentleman-Sande over the bit-reversed psi^-1 table,
 * bit-reversed in, natural out, then * N^{-1}. */
void or_ntt_inv(const or_ctx* c, uint32_t pi, uint64_t* a) {
    const uint64_t q = c->q[pi];
    const uint64_t* tab = c->itab + (size_t)pi * c->N;
    const uint64_t* tabp = c->itabp + (size_t)pi * c->N;
    const uint32_t n = c->N;
    for (uint32_t m = n >> 1, t = 1; m >= 1; m >>= 1, t <<= 1) {
        for (uint32_t i = 0; i < m; ++i) {
            const uint32_t j1 = i * (t << 1), j2 = j1 + t;
            const uint64_t w = tab[m + i], wp = tabp[m + i];
            for (uint32_t lo = j1; lo < j2; ++lo) {
                const uint32_t hi = lo + t;
                const uint64_t lv = a[lo], hv = a[hi];
                uint64_t s = lv + hv;
                if (s >= q) s -= q;
                const uint64_t d = lv >= hv ? lv - hv : lv + q - hv;
                a[lo] = s;
                a[hi] = mul_shoup(d, w, wp, q);
            }
        }
    }
    const uint64_t ni = c->ninv[pi];
    for (uint32_t j = 0; j < n; j++) a[j] = or_mulmod(a[j], ni, q);
}

/* batch forms: limbs are independent; OpenMP spreads them over OMP_NUM_THREADS host threads */
void or_ntt_fwd_batch(const or_ctx* c, uint64_t* data, uint32_t n_polys, uint32_t n_limbs, const uint32_t* prime_idx) {
    const long total = (long)n_polys * n_limbs;
#pragma omp parallel for schedule(static)
    for (long u = 0; u < total; u++)
        or_ntt_fwd(c, prime_idx[u % n_limbs], data + (size_t)u * c->N);
}

void or_ntt_inv_batch(const or_ctx* c, uint64_t* data, uint32_t n_polys, uint32_t n_limbs, const uint32_t* prime_idx) {
    const long total = (long)n_polys * n_limbs;
#pragma omp parallel for schedule(static)
    for (long u = 0; u < total; u++)
        or_ntt_inv(c, prime_idx[u % n_limbs], data + (size_t)u * c->N);
}

/* ------------------------------------------------------------------ basis conversion */

void or_bconv(const or_ctx* c, const uint64_t* in, uint32_t n_in, const uint32_t* in_idx,
              uint64_t* out, uint32_t n_out, const uint32_t* out_idx) {
    const uint32_t N = c->N;
    uint64_t* qhinv = (uint64_t*)malloc(sizeof(uint64_t) * n_in);
    uint64_t* qhmod = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)n_in * n_out);
    for (uint32_t i = 0; i < n_in; i++) {
        const uint64_t qi = c->q[in_idx[i]];
        uint64_t prod = 1;
        for (uint32_t k = 0; k < n_in; k++)
            if (k != i) prod = or_mulmod(prod, c->q[in_idx[k]] % qi, qi);
        qhinv[i] = or_invmod(prod, qi);
        for (uint32_t j = 0; j < n_out; j++) {
            const uint64_t pj = c->q[out_idx[j]];
            uint64_t pm = 1;
            for (uint32_t k = 0; k < n_in; k++)
                if (k != i) pm = or_mulmod(pm, c->q[in_idx[k]] % pj, pj);
            qhmod[(size_t)i * n_out + j] = pm;
        }
    }
    uint64_t* y = (uint64_t*)malloc(sizeof(uint64_t) * n_in);
    for (uint32_t k = 0; k < N; k++) {
        for (uint32_t i = 0; i < n_in; i++)
            y[i] = or_mulmod(in[(size_t)i * N + k], qhinv[i], c->q[in_idx[i]]);
        for (uint32_t j = 0; j < n_out; j++) {
            const uint64_t pj = c->q[out_idx[j]];
            uint64_t acc = 0;
            for (uint32_t i = 0; i < n_in; i++) {
                acc += or_mulmod(y[i] % pj, qhmod[(size_t)i * n_out + j], pj);
                if (acc >= pj) acc -= pj;
            }
            out[(size_t)j * N + k] = acc;
        }
    }
    free(y);
    free(qhinv);
    free(qhmod);
}

/* Exact (centered) conversion for ModDown.  The approximate conversion above returns x_P + u P with
 * u in [0, n_in) (u = floor(sum_i y_i / p_i)); ModDown then computes floor(x / P) - u, an error that is
 * biased (mean ~n_in / 2 per coefficient, multiplied by the secret in decryption).  Taking
 * u = round(sum_i y_i / p_i) instead makes the conversion the centered representative of x mod P and
 * ModDown exactly round(x / P) (the floating-point-corrected base conversion of Halevi, Polyakov and
 * Shoup, ePrint 2018/117, here in 128-bit fixed point so that CPU and GPU agree word for word). */
void or_bconv_centered(const or_ctx* c, const uint64_t* in, uint32_t n_in, const uint32_t* in_idx,
                       uint64_t* out, uint32_t n_out, const uint32_t* out_idx) {
    typedef unsigned __int128 u128;
    const uint32_t N = c->N;
    or_bconv(c, in, n_in, in_idx, out, n_out, out_idx);
    u128* cfix = (u128*)malloc(sizeof(u128) * n_in);
    uint64_t* qhinv = (uint64_t*)malloc(sizeof(uint64_t) * n_in);
    uint64_t* pmod = (uint64_t*)malloc(sizeof(uint64_t) * n_out);
    for (uint32_t i = 0; i < n_in; i++) {
        const uint64_t qi = c->q[in_idx[i]];
        uint64_t prod = 1;
        for (uint32_t k = 0; k < n_in; k++)
            if (k != i) prod = or_mulmod(prod, c->q[in_idx[k]] % qi, qi);
        qhinv[i] = or_invmod(prod, qi);
        cfix[i] = (~(u128)0) / qi; /* floor(2^128 / q_i): q_i is odd */
    }
    for (uint32_t j = 0; j < n_out; j++) {
        const uint64_t pj = c->q[out_idx[j]];
        uint64_t m = 1;
        for (uint32_t k = 0; k < n_in; k++) m = or_mulmod(m, c->q[in_idx[k]] % pj, pj);
        pmod[j] = m;
    }
    for (uint32_t k = 0; k < N; k++) {
        u128 F = 0;
        for (uint32_t i = 0; i < n_in; i++) {
            const uint64_t y = or_mulmod(in[(size_t)i * N + k], qhinv[i], c->q[in_idx[i]]);
            const uint64_t clo = (uint64_t)cfix[i], chi = (uint64_t)(cfix[i] >> 64);
            F += (u128)y * chi + (uint64_t)(((u128)y * clo) >> 64);
        }
        const uint64_t u = (uint64_t)((F + ((u128)1 << 63)) >> 64);
        for (uint32_t j = 0; j < n_out; j++) {
            const uint64_t pj = c->q[out_idx[j]];
            const uint64_t t = or_mulmod(u % pj, pmod[j], pj);
            uint64_t* o = out + (size_t)j * N + k;
            *o = *o >= t ? *o - t : *o + pj - t;
        }
    }
    free(cfix);
    free(qhinv);
    free(pmod);
}

/* ------------------------------------------------------------------ elementwise */

void or_tensor(const or_ctx* c, const uint64_t* a, const uint64_t* b, uint32_t l, uint64_t* d) {
    const size_t N = c->N, P = (size_t)l * N;
    for (uint32_t t = 0; t < l; t++) {
        const uint64_t q = c->q[t];
        for (size_t k = 0; k < N; k++) {
            const size_t o = (size_t)t * N + k;
            const uint64_t a0 = a[o], a1 = a[P + o], b0 = b[o], b1 = b[P + o];
            d[o] = or_mulmod(a0, b0, q);
            d[P + o] = (or_mulmod(a0, b1, q) + or_mulmod(a1, b0, q)) % q;
            d[2 * P + o] = or_mulmod(a1, b1, q);
        }
    }
}

/* ------------------------------------------------------------------ hybrid key switching */

uint32_t or_num_digits(const or_ctx* c, uint32_t l) { return (l + c->alpha - 1) / c->alpha; }

/* prime index of extended limb t at level l */
static inline uint32_t ext_prime(const or_ctx* c, uint32_t l, uint32_t t) { return t < l ? t : c->L + (t - l); }

void or_modup(const or_ctx* c, const uint64_t* x, uint32_t l, uint64_t* ext) {
    const uint32_t N = c->N, E = l + c->K, D = or_num_digits(c, l);
    uint32_t in_idx[OR_MAX_PRIMES], out_idx[OR_MAX_PRIMES], out_pos[OR_MAX_PRIMES];
    uint64_t* coef = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)c->alpha * N);
    uint64_t* conv = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)E * N);
    for (uint32_t d = 0; d < D; d++) {
        const uint32_t lo = d * c->alpha, hi = (lo + c->alpha < l) ? lo + c->alpha : l, n_in = hi - lo;
        uint64_t* dst = ext + (size_t)d * E * N;
        for (uint32_t i = 0; i < n_in; i++) {
            in_idx[i] = lo + i;
            memcpy(coef + (size_t)i * N, x + (size_t)(lo + i) * N, sizeof(uint64_t) * N);
            or_ntt_inv(c, lo + i, coef + (size_t)i * N);
            memcpy(dst + (size_t)(lo + i) * N, x + (size_t)(lo + i) * N, sizeof(uint64_t) * N);
        }
        uint32_t n_out = 0;
        for (uint32_t t = 0; t < E; t++) {
            if (t >= lo && t < hi) continue;
            out_idx[n_out] = ext_prime(c, l, t);
            out_pos[n_out] = t;
            n_out++;
        }
        or_bconv(c, coef, n_in, in_idx, conv, n_out, out_idx);
        for (uint32_t j = 0; j < n_out; j++) {
            or_ntt_fwd(c, out_idx[j], conv + (size_t)j * N);
            memcpy(dst + (size_t)out_pos[j] * N, conv + (size_t)j * N, sizeof(uint64_t) * N);
        }
    }
    free(coef);
    free(conv);
}

void or_ks_inner(const or_ctx* c, const uint64_t* ext, uint32_t l, const uint64_t* evk, uint64_t* acc) {
    const uint32_t N = c->N, E = l + c->K, D = or_num_digits(c, l), T = c->L + c->K;
    for (uint32_t t = 0; t < E; t++) {
        const uint32_t pi = ext_prime(c, l, t);
        const uint64_t q = c->q[pi];
        for (uint32_t k = 0; k < N; k++) {
            uint64_t s0 = 0, s1 = 0;
            for (uint32_t d = 0; d < D; d++) {
                const uint64_t x = ext[((size_t)d * E + t) * N + k];
                const uint64_t b = evk[(((size_t)d * 2 + 0) * T + pi) * N + k];
                const uint64_t a = evk[(((size_t)d * 2 + 1) * T + pi) * N + k];
                s0 = (s0 + or_mulmod(x, b, q)) % q;
                s1 = (s1 + or_mulmod(x, a, q)) % q;
            }
            acc[((size_t)0 * E + t) * N + k] = s0;
            acc[((size_t)1 * E + t) * N + k] = s1;
        }
    }
}

void or_moddown(const or_ctx* c, const uint64_t* x, uint32_t l, uint64_t* out) {
    const uint32_t N = c->N, K = c->K;
    uint32_t in_idx[OR_MAX_PRIMES], out_idx[OR_MAX_PRIMES];
    uint64_t* coef = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)K * N);
    uint64_t* conv = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)l * N);
    for (uint32_t k = 0; k < K; k++) {
        in_idx[k] = c->L + k;
        memcpy(coef + (size_t)k * N, x + (size_t)(l + k) * N, sizeof(uint64_t) * N);
        or_ntt_inv(c, c->L + k, coef + (size_t)k * N);
    }
    for (uint32_t i = 0; i < l; i++) out_idx[i] = i;
    if (c->moddown_exact)
        or_bconv_centered(c, coef, K, in_idx, conv, l, out_idx);
    else
        or_bconv(c, coef, K, in_idx, conv, l, out_idx);
    for (uint32_t i = 0; i < l; i++) {
        const uint64_t q = c->q[i];
        uint64_t pinv = 1;
        for (uint32_t k = 0; k < K; k++) pinv = or_mulmod(pinv, c->q[c->L + k] % q, q);
        pinv = or_invmod(pinv, q);
        uint64_t* cv = conv + (size_t)i * N;
        or_ntt_fwd(c, i, cv);
        for (uint32_t k = 0; k < N; k++) {
            const uint64_t v = x[(size_t)i * N + k];
            const uint64_t d = v >= cv[k] ? v - cv[k] : v + q - cv[k];
            out[(size_t)i * N + k] = or_mulmod(d, pinv, q);
        }
    }
    free(coef);
    free(conv);
}

void or_keyswitch(const or_ctx* c, const uint64_t* x, uint32_t l, const uint64_t* evk, uint64_t* out2) {
    const uint32_t N = c->N, E = l + c->K, D = or_num_digits(c, l);
    uint64_t* ext = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)D * E * N);
    uint64_t* acc = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)2 * E * N);
    or_modup(c, x, l, ext);
    or_ks_inner(c, ext, l, evk, acc);
    or_moddown(c, acc, l, out2);
    or_moddown(c, acc + (size_t)E * N, l, out2 + (size_t)l * N);
    free(ext);
    free(acc);
}

/* ------------------------------------------------------------------ rescale */

/* OpenFHE DropLastElementAndScale: last limb to coefficients, centered lift (v > q_l>>1 => v - q_l,
 * boot_overflow_probe.cpp:93-94) into every remaining q_i, back to eval, (c_i - t_i) * q_l^{-1}. */
void or_rescale(const or_ctx* c, const uint64_t* in, uint32_t n_polys, uint32_t l, uint64_t* out) {
    const uint32_t N = c->N;
    const uint64_t ql = c->q[l - 1];
    uint64_t* last = (uint64_t*)malloc(sizeof(uint64_t) * N);
    uint64_t* t = (uint64_t*)malloc(sizeof(uint64_t) * N);
    for (uint32_t p = 0; p < n_polys; p++) {
        memcpy(last, in + ((size_t)p * l + (l - 1)) * N, sizeof(uint64_t) * N);
        or_ntt_inv(c, l - 1, last);
        for (uint32_t i = 0; i + 1 < l; i++) {
            const uint64_t q = c->q[i];
            for (uint32_t k = 0; k < N; k++) {
                const uint64_t v = last[k];
                t[k] = (v > (ql >> 1)) ? (q - ((ql - v) % q)) % q : v % q;
            }
            or_ntt_fwd(c, i, t);
            const uint64_t qlinv = or_invmod(ql % q, q);
            const uint64_t* src = in + ((size_t)p * l + i) * N;
            uint64_t* dst = out + ((size_t)p * (l - 1) + i) * N;
            for (uint32_t k = 0; k < N; k++) {
                const uint64_t d = src[k] >= t[k] ? src[k] - t[k] : src[k] + q - t[k];
                dst[k] = or_mulmod(d, qlinv, q);
            }
        }
    }
    free(last);
    free(t);
}

void or_hmult_relin_rescale(const or_ctx* c, const uint64_t* a, const uint64_t* b, uint32_t l,
                            const uint64_t* evk, uint64_t* out) {
    const size_t N = c->N, P = (size_t)l * N;
    uint64_t* d = (uint64_t*)malloc(sizeof(uint64_t) * 3 * P);
    uint64_t* ks = (uint64_t*)malloc(sizeof(uint64_t) * 2 * P);
    or_tensor(c, a, b, l, d);
    or_keyswitch(c, d + 2 * P, l, evk, ks);
    for (uint32_t pp = 0; pp < 2; pp++)
        for (uint32_t t = 0; t < l; t++) {
            const uint64_t q = c->q[t];
            for (size_t k = 0; k < N; k++) {
                const size_t o = pp * P + (size_t)t * N + k;
                uint64_t v = d[o] + ks[o];
                if (v >= q) v -= q;
                d[o] = v;
            }
        }
    or_rescale(c, d, 2, l, out);
    free(d);
    free(ks);
}

/* n_pairs independent HMult+relin+rescale calls spread over the host threads (one pair per thread at a time; the
 * per-pair work itself stays scalar).  a, b [n_pairs][2][l][N], out [n_pairs][2][l-1][N].  For the timed CPU
 * baseline's all-core leg. */
void or_hmult_relin_rescale_batch(const or_ctx* c, const uint64_t* a, const uint64_t* b, uint32_t n_pairs,
                                  uint32_t l, const uint64_t* evk, uint64_t* out) {
    const size_t in_words = (size_t)2 * l * c->N, out_words = (size_t)2 * (l - 1) * c->N;
#pragma omp parallel for schedule(dynamic, 1)
    for (long p = 0; p < (long)n_pairs; p++)
        or_hmult_relin_rescale(c, a + (size_t)p * in_words, b + (size_t)p * in_words, l, evk,
                               out + (size_t)p * out_words);
}

/* host threads of the OpenMP batch forms (n < 1: the runtime's default) and the count now in effect */
void or_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : omp_get_num_procs());
#else
    (void)n;
#endif
}

int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ automorphism */

uint32_t or_rot_index(const or_ctx* c, int64_t k) {
    const uint64_t M = 2ull * c->N, ord = c->N / 2;   /* order of 5 in (Z/2N)^* */
    int64_t e = k % (int64_t)ord;
    if (e < 0) e += (int64_t)ord;
    return (uint32_t)or_powmod(5, (uint64_t)e, M);
}

void or_automorph_coef(const or_ctx* c, const uint64_t* in, uint32_t n_limbs, const uint32_t* prime_idx,
                       uint32_t g, uint64_t* out) {
    const uint32_t N = c->N;
    const uint64_t M = 2ull * N;
    for (uint32_t l = 0; l < n_limbs; l++) {
        const uint64_t q = c->q[prime_idx[l]];
        const uint64_t* src = in + (size_t)l * N;
        uint64_t* dst = out + (size_t)l * N;
        for (uint32_t j = 0; j < N; j++) {
            const uint64_t e = ((uint64_t)j * g) % M;
            if (e < N) dst[e] = src[j];
            else dst[e - N] = src[j] ? q - src[j] : 0;
        }
    }
}

/* Slot k of the bit-reversed NTT holds a(psi^(2*brev(k)+1)); a(X^g) at that point is a at
 * psi^(g*(2*brev(k)+1)), i.e. slot brev(((g*(2*brev(k)+1)) mod 2N - 1)/2). */
void or_automorph_eval(const or_ctx* c, const uint64_t* in, uint32_t n_limbs, uint32_t g, uint64_t* out) {
    const uint32_t N = c->N, lg = c->logN;
    const uint64_t M = 2ull * N;
    for (uint32_t k = 0; k < N; k++) {
        const uint64_t e = (2ull * or_bitrev(k, lg) + 1) * g % M;
        const uint32_t src = or_bitrev((uint32_t)((e - 1) / 2), lg);
        for (uint32_t l = 0; l < n_limbs; l++) out[(size_t)l * N + k] = in[(size_t)l * N + src];
    }
}

void or_rotate(const or_ctx* c, const uint64_t* ct, uint32_t l, uint32_t g, const uint64_t* evk, uint64_t* out) {
    const size_t N = c->N, P = (size_t)l * N;
    uint64_t* ks = (uint64_t*)malloc(sizeof(uint64_t) * 2 * P);
    or_keyswitch(c, ct + P, l, evk, ks);
    for (uint32_t t = 0; t < l; t++) {
        const uint64_t q = c->q[t];
        for (size_t k = 0; k < N; k++) {
            const size_t o = (size_t)t * N + k;
            uint64_t v = ks[o] + ct[o];
            if (v >= q) v -= q;
            ks[o] = v;
        }
    }
    or_automorph_eval(c, ks, l, g, out);
    or_automorph_eval(c, ks + P, l, g, out + P);
    free(ks);
}

/* ------------------------------------------------------------------ ChaCha20 + seeded sampling */

static inline uint32_t rotl32(uint32_t v, int s) { return (v << s) | (v >> (32 - s)); }
#define OR_QR(a, b, c, d)                \
    a += b; d ^= a; d = rotl32(d, 16);   \
    c += d; b ^= c; b = rotl32(b, 12);   \
    a += b; d ^= a; d = rotl32(d, 8);    \
    c += d; b ^= c; b = rotl32(b, 7);

/* RFC 8439 section 2.3; seeded_keys.hpp:81-105 */
void or_chacha20_block(const uint32_t key[8], uint32_t counter, const uint32_t nonce[3], uint32_t out[16]) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, key[0], key[1], key[2], key[3],
                      key[4], key[5], key[6], key[7], counter, nonce[0], nonce[1], nonce[2]};
    uint32_t x[16];
    memcpy(x, s, sizeof(s));
    for (int r = 0; r < 10; r++) {
        OR_QR(x[0], x[4], x[8], x[12]);
        OR_QR(x[1], x[5], x[9], x[13]);
        OR_QR(x[2], x[6], x[10], x[14]);
        OR_QR(x[3], x[7], x[11], x[15]);
        OR_QR(x[0], x[5], x[10], x[15]);
        OR_QR(x[1], x[6], x[11], x[12]);
        OR_QR(x[2], x[7], x[8], x[13]);
        OR_QR(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

typedef struct {
    uint32_t key[8], nonce[3], w[16], counter;
    int pos;
} or_stream;

static void stream_init(or_stream* s, const uint8_t seed[32], uint32_t w0, uint32_t w1, uint32_t tag) {
    for (int k = 0; k < 8; k++)
        s->key[k] = (uint32_t)seed[4 * k] | ((uint32_t)seed[4 * k + 1] << 8) | ((uint32_t)seed[4 * k + 2] << 16) |
                    ((uint32_t)seed[4 * k + 3] << 24);
    s->nonce[0] = w0;
    s->nonce[1] = w1;
    s->nonce[2] = tag;
    s->counter = 0;
    s->pos = 8;
}

/* seeded_keys.hpp:114-122: little-endian uint64 words of consecutive blocks */
static uint64_t stream_next(or_stream* s) {
    if (s->pos == 8) {
        or_chacha20_block(s->key, s->counter++, s->nonce, s->w);
        s->pos = 0;
    }
    const uint64_t v = (uint64_t)s->w[2 * s->pos] | ((uint64_t)s->w[2 * s->pos + 1] << 32);
    s->pos++;
    return v;
}

/* seeded_keys.hpp:129-137: rejection below lim = 2^64 - (2^64 mod q), accept w mod q */
void or_fill_uniform(const uint8_t seed[32], uint32_t word0, uint32_t word1, uint32_t tag, uint64_t q,
                     uint64_t* out, size_t n) {
    or_stream s;
    stream_init(&s, seed, word0, word1, tag);
    const uint64_t r = (0 - q) % q, lim = 0 - r;
    for (size_t k = 0; k < n; k++) {
        uint64_t w = stream_next(&s);
        while (r != 0 && w >= lim) w = stream_next(&s);
        out[k] = w % q;
    }
}

/* Ternary secret, Hamming weight h: positions from the "SECR" stream (w & (N-1), redrawn while
 * occupied), sign = top bit of the same word. */
void or_sample_ternary(const uint8_t seed[32], uint32_t N, uint32_t h, int8_t* s) {
    or_stream st;
    stream_init(&st, seed, 0, 0, 0x52434553u);
    memset(s, 0, N);
    for (uint32_t i = 0; i < h && i < N; i++) {
        for (;;) {
            const uint64_t w = stream_next(&st);
            const uint32_t p = (uint32_t)(w & (N - 1));
            if (s[p]) continue;
            s[p] = (w >> 63) ? -1 : 1;
            break;
        }
    }
}

/* Rounded Gaussian: Box-Muller on two 53-bit uniforms from the "GAUS" stream (nonce words w0, w1). */
void or_sample_gauss2(const uint8_t seed[32], uint32_t w0, uint32_t w1, uint32_t N, double sigma, int32_t* e) {
    or_stream st;
    stream_init(&st, seed, w0, w1, 0x53554147u);
    const double two53 = 9007199254740992.0;
    for (uint32_t k = 0; k < N; k++) {
        const double u1 = ((double)(stream_next(&st) >> 11) + 1.0) / two53;
        const double u2 = (double)(stream_next(&st) >> 11) / two53;
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        e[k] = (int32_t)llround(sigma * z);
    }
}

void or_sample_gauss(const uint8_t seed[32], uint32_t stream, uint32_t N, double sigma, int32_t* e) {
    or_sample_gauss2(seed, stream, 0, N, sigma, e);
}

void or_small_to_eval_i8(const or_ctx* c, const int8_t* s, uint32_t n_limbs, const uint32_t* prime_idx, uint64_t* out) {
    for (uint32_t l = 0; l < n_limbs; l++) {
        const uint64_t q = c->q[prime_idx[l]];
        uint64_t* d = out + (size_t)l * c->N;
        for (uint32_t k = 0; k < c->N; k++) d[k] = s[k] >= 0 ? (uint64_t)s[k] : q - (uint64_t)(-s[k]);
        or_ntt_fwd(c, prime_idx[l], d);
    }
}

void or_small_to_eval_i32(const or_ctx* c, const int32_t* e, uint32_t n_limbs, const uint32_t* prime_idx, uint64_t* out) {
    for (uint32_t l = 0; l < n_limbs; l++) {
        const uint64_t q = c->q[prime_idx[l]];
        uint64_t* d = out + (size_t)l * c->N;
        for (uint32_t k = 0; k < c->N; k++) d[k] = e[k] >= 0 ? (uint64_t)e[k] % q : q - ((uint64_t)(-(int64_t)e[k]) % q);
        or_ntt_fwd(c, prime_idx[l], d);
    }
}

/* seeded_keys.hpp:216-256: b_j = -a_j * s_new_ext + e_j + [Q limbs of digit j] PModq_i * s_old_i */
void or_ksk_gen(const or_ctx* c, const uint64_t* s_old_eval, const int8_t* s_new, const uint8_t seed[32],
                const uint8_t eseed[32], double sigma, uint64_t* evk) {
    const uint32_t N = c->N, T = c->L + c->K;
    uint32_t idx[OR_MAX_PRIMES];
    for (uint32_t i = 0; i < T; i++) idx[i] = i;
    uint64_t* sn = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)T * N);
    uint64_t* ee = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)T * N);
    int32_t* e = (int32_t*)malloc(sizeof(int32_t) * N);
    or_small_to_eval_i8(c, s_new, T, idx, sn);
    for (uint32_t d = 0; d < c->dnum; d++) {
        uint64_t* b = evk + ((size_t)d * 2 + 0) * T * N;
        uint64_t* a = evk + ((size_t)d * 2 + 1) * T * N;
        for (uint32_t i = 0; i < T; i++) or_fill_uniform(seed, d, i, 0x59454b53u, c->q[i], a + (size_t)i * N, N);
        or_sample_gauss(eseed, d, N, sigma, e);
        or_small_to_eval_i32(c, e, T, idx, ee);
        const uint32_t lo = d * c->alpha, hi = (lo + c->alpha < c->L) ? lo + c->alpha : c->L;
        for (uint32_t i = 0; i < T; i++) {
            const uint64_t q = c->q[i];
            uint64_t pmod = 1;
            for (uint32_t k = 0; k < c->K; k++) pmod = or_mulmod(pmod, c->q[c->L + k] % q, q);
            for (uint32_t k = 0; k < N; k++) {
                const size_t o = (size_t)i * N + k;
                uint64_t v = (q - or_mulmod(a[o], sn[o], q)) % q;
                v = (v + ee[o]) % q;
                if (i >= lo && i < hi) v = (v + or_mulmod(pmod, s_old_eval[o], q)) % q;
                b[o] = v;
            }
        }
    }
    free(sn);
    free(ee);
    free(e);
}

/* Public key over Q*P: pk = (b, a) with b = e - a*s (noise scale 1), as PKEBase::KeyGenInternal builds it
 * (harness/boot_overflow_probe.cpp:22,139: b = ns*e - a*s, elements {b, a}; the key over paramsPK, which may hold
 * more towers than Q, :132-:142).  a_i = or_fill_uniform(seed, 0, i, "PKEY"), e = or_sample_gauss2(eseed, 0, 0). */
void or_pk_gen(const or_ctx* c, const uint64_t* s_eval, const uint8_t seed[32], const uint8_t eseed[32],
               double sigma, uint64_t* pk) {
    const uint32_t N = c->N, T = c->L + c->K;
    uint32_t idx[OR_MAX_PRIMES];
    for (uint32_t i = 0; i < T; i++) idx[i] = i;
    uint64_t* b = pk;
    uint64_t* a = pk + (size_t)T * N;
    int32_t* e = (int32_t*)malloc(sizeof(int32_t) * N);
    or_sample_gauss2(eseed, 0, 0, N, sigma, e);
    or_small_to_eval_i32(c, e, T, idx, b);
    for (uint32_t i = 0; i < T; i++) {
        const uint64_t q = c->q[i];
        or_fill_uniform(seed, 0, i, 0x59454b50u, q, a + (size_t)i * N, N);
        for (uint32_t k = 0; k < N; k++) {
            const size_t o = (size_t)i * N + k;
            b[o] = (b[o] + q - or_mulmod(a[o], s_eval[o], q)) % q;
        }
    }
    free(e);
}

/* Public-key encryption at level l: the key's Q_l and P limbs, x0 = b v + e0, x1 = a v + e1 over Q_l*P, then
 * ApproxModDown of both to Q_l and the plaintext added to the first: ct = (ModDown(x0) + m, ModDown(x1)).  v is
 * uniform ternary (or_fill_uniform(seed, index, 0, "ENCV", 3): 0, 1, 2 -> 0, 1, -1), e0 and e1 Gaussian streams
 * (index, 2) and (index, 3) of the seed.  pk [2][L+K][N], m [l][N], ct [2][l][N]. */
void or_pk_encrypt(const or_ctx* c, const uint64_t* pk, const uint64_t* m, uint32_t l, const uint8_t seed[32],
                   uint32_t index, double sigma, uint64_t* ct) {
    const uint32_t N = c->N, T = c->L + c->K, E = l + c->K;
    uint32_t idx[OR_MAX_PRIMES];
    for (uint32_t t = 0; t < E; t++) idx[t] = t < l ? t : c->L + (t - l);
    uint64_t* u = (uint64_t*)malloc(sizeof(uint64_t) * N);
    int8_t* v = (int8_t*)malloc(N);
    int32_t* e = (int32_t*)malloc(sizeof(int32_t) * N);
    uint64_t* ve = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)E * N);
    uint64_t* ee = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)E * N);
    uint64_t* x = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)E * N);
    or_fill_uniform(seed, index, 0, 0x56434e45u, 3, u, N);
    for (uint32_t k = 0; k < N; k++) v[k] = u[k] == 2 ? -1 : (int8_t)u[k];
    or_small_to_eval_i8(c, v, E, idx, ve);
    for (uint32_t p = 0; p < 2; p++) {
        or_sample_gauss2(seed, index, 2 + p, N, sigma, e);
        or_small_to_eval_i32(c, e, E, idx, ee);
        for (uint32_t t = 0; t < E; t++) {
            const uint64_t q = c->q[idx[t]];
            const uint64_t* key = pk + ((size_t)p * T + idx[t]) * N;
            for (uint32_t k = 0; k < N; k++) {
                const size_t o = (size_t)t * N + k;
                x[o] = (or_mulmod(key[k], ve[o], q) + ee[o]) % q;
            }
        }
        uint64_t* out = ct + (size_t)p * l * N;
        or_moddown(c, x, l, out);
        if (p == 0)
            for (uint32_t i = 0; i < l; i++)
                for (uint32_t k = 0; k < N; k++) {
                    const size_t o = (size_t)i * N + k;
                    out[o] = (out[o] + m[o]) % c->q[i];
                }
    }
    free(u);
    free(v);
    free(e);
    free(ve);
    free(ee);
    free(x);
}
