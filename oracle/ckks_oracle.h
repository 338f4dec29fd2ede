/*
 * ckks_oracle.h -- CPU restatement of the RNS-CKKS integer core (TEST INFRASTRUCTURE ONLY).
 *
 * This is the checker, never the product: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Plain C99 + unsigned __int128, scalar, one thread per call.
 *
 * It restates, function by function, the OpenFHE 1.5.1 conventions that the reference spells out
 * in its own host code (the arithmetic itself lives in OpenFHE/FIDESlib, which are not in the
 * reference tree):
 *   NTT order + Shoup  : hpc_gpu_port/periodic_encode.hpp:102-120 (Shoup), :150-160 (root table
 *                        Table[brev(i)] = psi^i), :240-260 (ForwardTransformToBitReverse loop)
 *   centered lift      : harness/boot_overflow_probe.cpp:8-9,93-94 (SwitchModulus: v > q>>1 => v-q)
 *   key-switch key     : hpc_gpu_port/seeded_keys.hpp:216-256 (b_j = -a_j*s'_ext + e_j
 *                        + [digit j] PModq_i * s_i), extendToQP :170-193
 *   ChaCha20 expander  : hpc_gpu_port/seeded_keys.hpp:28-43 (normative), :81-134
 *   automorphism index : hpc_gpu_port/gpu_real_model.cu:1337-1360 (5^k mod 2N), conjugate 2N-1
 *   public key         : harness/boot_overflow_probe.cpp:22,139 ({b = e - a*s, a}; dec = b + a*s)
 *
 * How each function is pinned (tests/test_oracle_*.py): brute-force O(N^2) negacyclic DFT and
 * schoolbook products, CRT reconstruction with Python big integers (BConv/ModUp/ModDown/rescale
 * identities), RFC 8439 ChaCha20 known-answer vectors, the reference's chain_moduli.jsonl and
 * contract_r17.json fixtures, and decryption noise bounds (key switching).  Functions whose exact
 * bits only OpenFHE itself could confirm (its prime-chain choice, its RootOfUnity choice, its PRNG
 * streams) follow a documented convention of this repo and are "parity unpinned" against OpenFHE.
 */
#ifndef CKKS_ORACLE_H
#define CKKS_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_MAX_PRIMES 80

typedef struct {
    uint32_t N, logN;
    uint32_t L, K;          /* Q limbs (chain order), P limbs (special primes) */
    uint32_t dnum, alpha;   /* digits, limbs per digit = ceil(L/dnum) */
    uint64_t q[OR_MAX_PRIMES];     /* moduli: q[0..L) = Q chain, q[L..L+K) = P */
    uint64_t psi[OR_MAX_PRIMES];   /* primitive 2N-th root per modulus */
    uint64_t ninv[OR_MAX_PRIMES];  /* N^{-1} mod q */
    uint64_t *tab, *tabp;          /* [L+K][N] forward table (brev order) + Shoup companions */
    uint64_t *itab, *itabp;        /* [L+K][N] inverse table (brev order) + Shoup companions */
    uint32_t moddown_exact;        /* 0: approximate P->Q conversion (OpenFHE ApproxModDown); 1: exact rounding */
} or_ctx;

/* ---- scalar modular arithmetic ---- */
uint64_t or_mulmod(uint64_t a, uint64_t b, uint64_t q);
uint64_t or_powmod(uint64_t a, uint64_t e, uint64_t q);
uint64_t or_invmod(uint64_t a, uint64_t q);
int      or_is_prime(uint64_t n);
uint32_t or_bitrev(uint32_t v, uint32_t bits);

/* Largest `count` primes below 2^bits with p = 1 (mod m), skipping `exclude`; returns count found. */
uint32_t or_gen_primes(uint32_t bits, uint32_t count, uint64_t m, const uint64_t* exclude,
                       uint32_t n_exclude, uint64_t* out);
/* Smallest primitive m-th root of unity mod q (m a power of two, q = 1 mod m). */
uint64_t or_min_root(uint64_t q, uint64_t m);

/* ---- context ---- */
int  or_ctx_init(or_ctx* c, uint32_t logN, const uint64_t* moduli, uint32_t L, uint32_t K, uint32_t dnum);
void or_ctx_free(or_ctx* c);

/* ---- NTT (one limb; prime index pi into the context) ---- */
void or_ntt_fwd(const or_ctx* c, uint32_t pi, uint64_t* a);
void or_ntt_inv(const or_ctx* c, uint32_t pi, uint64_t* a);
/* batch: data [n_polys][n_limbs][N], limb l of every poly uses prime prime_idx[l] */
void or_ntt_fwd_batch(const or_ctx* c, uint64_t* data, uint32_t n_polys, uint32_t n_limbs, const uint32_t* prime_idx);
void or_ntt_inv_batch(const or_ctx* c, uint64_t* data, uint32_t n_polys, uint32_t n_limbs, const uint32_t* prime_idx);

/* ---- approximate CRT basis conversion (coefficient form) ----
 * in [n_in][N] with moduli q[in_idx[i]], out [n_out][N] with moduli q[out_idx[j]]:
 * out_j = sum_i [x_i * Qhat_i^{-1}]_{q_i} * (Qhat_i mod p_j) mod p_j,  Qhat_i = prod_{k!=i} q_k. */
void or_bconv(const or_ctx* c, const uint64_t* in, uint32_t n_in, const uint32_t* in_idx,
              uint64_t* out, uint32_t n_out, const uint32_t* out_idx);

/* ---- elementwise ---- */
void or_tensor(const or_ctx* c, const uint64_t* a, const uint64_t* b, uint32_t l, uint64_t* d);  /* a,b [2][l][N] -> d [3][l][N] */

/* ---- hybrid key switching at level l (l active Q limbs; evk over all L+K limbs) ----
 * extended layout: [digits][l+K][N] where limb index t < l is Q limb t and t >= l is P limb t-l. */
uint32_t or_num_digits(const or_ctx* c, uint32_t l);
void or_modup(const or_ctx* c, const uint64_t* x, uint32_t l, uint64_t* ext);                       /* x eval [l][N] */
void or_ks_inner(const or_ctx* c, const uint64_t* ext, uint32_t l, const uint64_t* evk, uint64_t* acc); /* evk [dnum][2][L+K][N]; acc [2][l+K][N] */
void or_moddown(const or_ctx* c, const uint64_t* x, uint32_t l, uint64_t* out);
/* basis conversion returning the centered representative: sum_i y_i Qhat_i - u Q with u = round(sum_i y_i / q_i),
 * u from the 128-bit fixed-point sum of floor(y_i * floor(2^128 / q_i) / 2^64) */
void or_bconv_centered(const or_ctx* c, const uint64_t* in, uint32_t n_in, const uint32_t* in_idx,
                       uint64_t* out, uint32_t n_out, const uint32_t* out_idx);                     /* x eval [l+K][N] -> out eval [l][N] */
void or_keyswitch(const or_ctx* c, const uint64_t* x, uint32_t l, const uint64_t* evk, uint64_t* out2); /* out2 [2][l][N] */

/* ---- rescale: in eval [n_polys][l][N] -> out eval [n_polys][l-1][N] ---- */
void or_rescale(const or_ctx* c, const uint64_t* in, uint32_t n_polys, uint32_t l, uint64_t* out);

/* ---- HMult + relinearize + rescale of one pair at level l: a,b [2][l][N] -> out [2][l-1][N] ---- */
void or_hmult_relin_rescale(const or_ctx* c, const uint64_t* a, const uint64_t* b, uint32_t l,
                            const uint64_t* evk, uint64_t* out);
void or_hmult_relin_rescale_batch(const or_ctx* c, const uint64_t* a, const uint64_t* b, uint32_t n_pairs,
                                  uint32_t l, const uint64_t* evk, uint64_t* out);
void or_set_threads(int n);   /* OpenMP threads of the batch forms (n < 1: all processors) */
int or_max_threads(void);

/* ---- automorphism X -> X^g (g odd) ----
 * coefficient form: out[(j*g) mod N] = +-in[j] (negated when (j*g) mod 2N >= N)
 * evaluation form (bit-reversed NTT order): pure permutation of slots. */
void or_automorph_coef(const or_ctx* c, const uint64_t* in, uint32_t n_limbs, const uint32_t* prime_idx,
                       uint32_t g, uint64_t* out);
void or_automorph_eval(const or_ctx* c, const uint64_t* in, uint32_t n_limbs, uint32_t g, uint64_t* out);
uint32_t or_rot_index(const or_ctx* c, int64_t k);   /* 5^k mod 2N (negative k via the group order) */

/* ---- rotation (EvalRotate) of a ciphertext [2][l][N] with key evk_g over Q.P ----
 * KS of c1 under evk_g, add c0, then apply X -> X^g to both polys. */
void or_rotate(const or_ctx* c, const uint64_t* ct, uint32_t l, uint32_t g, const uint64_t* evk, uint64_t* out);

/* ---- ChaCha20 (RFC 8439) + the seeded uniform expander ---- */
void or_chacha20_block(const uint32_t key[8], uint32_t counter, const uint32_t nonce[3], uint32_t out[16]);
void or_fill_uniform(const uint8_t seed[32], uint32_t word0, uint32_t word1, uint32_t tag, uint64_t q,
                     uint64_t* out, size_t n);

/* ---- seeded secret / noise (this repo's convention) ---- */
void or_sample_ternary(const uint8_t seed[32], uint32_t N, uint32_t h, int8_t* s);   /* Hamming weight h */
void or_sample_gauss(const uint8_t seed[32], uint32_t stream, uint32_t N, double sigma, int32_t* e);
void or_sample_gauss2(const uint8_t seed[32], uint32_t w0, uint32_t w1, uint32_t N, double sigma, int32_t* e);

/* small signed poly -> eval form limbs for the given primes */
void or_small_to_eval_i8(const or_ctx* c, const int8_t* s, uint32_t n_limbs, const uint32_t* prime_idx, uint64_t* out);
void or_small_to_eval_i32(const or_ctx* c, const int32_t* e, uint32_t n_limbs, const uint32_t* prime_idx, uint64_t* out);

/* ---- key-switching key: switch from s_old (eval, Q limbs [L][N]) to s_new (signed coeffs) ----
 * evk [dnum][2][L+K][N]: evk[j][0] = b_j, evk[j][1] = a_j.
 * a_j: or_fill_uniform(seed, j, limb, 0x59454b53 "SKEY"), e_j: or_sample_gauss(eseed, stream j). */
void or_ksk_gen(const or_ctx* c, const uint64_t* s_old_eval, const int8_t* s_new, const uint8_t seed[32],
                const uint8_t eseed[32], double sigma, uint64_t* evk);

/* ---- public key (b = e - a s over Q*P) and public-key encryption at level l (ModDown from Q_l*P) ----
 * pk [2][L+K][N]; ct [2][l][N] = (ModDown(b v + e0) + m, ModDown(a v + e1)) */
void or_pk_gen(const or_ctx* c, const uint64_t* s_eval, const uint8_t seed[32], const uint8_t eseed[32],
               double sigma, uint64_t* pk);
void or_pk_encrypt(const or_ctx* c, const uint64_t* pk, const uint64_t* m, uint32_t l, const uint8_t seed[32],
                   uint32_t index, double sigma, uint64_t* ct);

#ifdef __cplusplus
}
#endif
#endif
