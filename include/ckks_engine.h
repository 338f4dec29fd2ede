/*
 * ckks_engine.h -- C ABI of the MI355X-native RNS-CKKS evaluation engine (libckks_hip.so).
 *
 * What it replaces.  The reference evaluates its encrypted recurrent step through FIDESlib's
 * OpenFHE-compatible C++ class API, fideslib::CryptoContext<DCRTPoly> (hpc_gpu_port/gpu_real_model.cu:66,185);
 * every EvalMult / RescaleInPlace / EvalRotate / EvalAdd / EvalBootstrap call of the driver goes there.
 * This header is the drop-in boundary for that path: plain C, opaque handles, raw device pointers and
 * sizes, status codes instead of exceptions (the reference's exceptions surface as JSON `fatal` lines,
 * gpu_real_model.cu:924-928; here every entry point returns an int and ckks_last_error() explains).
 *
 * Data layout (kept from the reference, gpu_real_model.cu:1762-1790 and seeded_keys.hpp:216-256):
 *   - a polynomial is a list of limbs, each limb N = 2^16 contiguous uint64 residues in [0, q);
 *   - evaluation form uses OpenFHE's bit-reversed NTT order (periodic_encode.hpp:240-260);
 *   - limb index = global prime index in chain order: 0..L-1 the Q chain, L..L+K-1 the special primes P;
 *     limbs are dropped from the end (level l keeps Q limbs 0..l-1);
 *   - a ciphertext batch is uint64[B][2][l][N] (B ciphertexts, polys c0,c1, l limbs);
 *   - a key-switching key is uint64[dnum][2][L+K][N]: [j][0] = b_j, [j][1] = a_j, EVALUATION form
 *     (EvalKeyRelinImpl{A[dnum], B[dnum]} of OpenFHE).
 *
 * Threading: one host thread per context issues all work; entry points are not re-entrant per
 * context (the reference's FIDESlib usage has the same rule, gpu_real_model.cu:3017-3024).
 * Streams: every compute entry point takes a hipStream_t (as void*); NULL is the null stream.
 * Device pointers may come from ckks_buffer_alloc or from any HIP allocator (e.g. torch tensors).
 */
#ifndef CKKS_ENGINE_H
#define CKKS_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define CKKS_OK 0
#define CKKS_EINVAL 1   /* bad argument / shape / level */
#define CKKS_EHIP 2     /* HIP runtime error (message in ckks_last_error) */
#define CKKS_ENOMEM 3
#define CKKS_ENOTSUP 4

typedef struct ckks_context ckks_context;

typedef struct {
    uint32_t log_n;     /* ring dimension log2; this build supports 16 */
    uint32_t num_q;     /* L: Q-chain limbs (multiplicative depth + 1) */
    uint32_t num_p;     /* K: special primes for hybrid key switching */
    uint32_t dnum;      /* digits of the hybrid key switch */
    uint32_t q_bits;    /* bit size of the Q primes (largest primes below 2^q_bits, = 1 mod 2N) */
    uint32_t p_bits;    /* bit size of the P primes */
    double scale;       /* CKKS scaling factor Delta */
    int device;         /* HIP device ordinal */
} ckks_params;

/* Last error message of the calling thread ("" when none). */
const char* ckks_last_error(void);

/* ---- context -------------------------------------------------------------------------------
 * Replaces GenCryptoContext + the device upload of FIDESlib's LoadContext (gpu_real_model.cu:1138-1164,
 * 1530).  Moduli: the largest primes below 2^q_bits (then 2^p_bits, skipping Q primes) with
 * q = 1 mod 2N; root of unity per prime: the smallest primitive 2N-th root. */
int ckks_context_create(const ckks_params* params, ckks_context** out);
/* Same, with the moduli given explicitly (Q chain order, then P). */
int ckks_context_create_from_moduli(uint32_t log_n, const uint64_t* q, uint32_t num_q, const uint64_t* p,
                                    uint32_t num_p, uint32_t dnum, double scale, int device, ckks_context** out);
void ckks_context_destroy(ckks_context* ctx);
int ckks_context_info(const ckks_context* ctx, uint32_t* n, uint32_t* num_q, uint32_t* num_p, uint32_t* dnum);
/* moduli (num_q + num_p) and the primitive 2N-th roots used by the NTT, chain order */
int ckks_context_moduli(const ckks_context* ctx, uint64_t* out, uint32_t cap);
int ckks_context_roots(const ckks_context* ctx, uint64_t* out, uint32_t cap);
/* NTT schedule: 0 = two kernels (pass A, pass B; default), 1 = fused one-limb-per-workgroup */
int ckks_set_ntt_mode(ckks_context* ctx, int mode);
/* ckks_set_moddown_exact: ModDown rounding.  0 (default): OpenFHE's ApproxModDown, floor(x / P) - u with
 * u in [0, K) from the approximate P -> Q conversion (a bias of ~K/2 per coefficient, multiplied by the
 * secret on decryption: it costs ~10 bits of bootstrapping precision at a 2^40 scale).  1: exact
 * round(x / P): the conversion subtracts round(sum_i y_i / p_i) P, computed in 128-bit fixed point
 * (Halevi-Polyakov-Shoup's corrected base conversion). */
int ckks_set_moddown_exact(ckks_context* ctx, int exact);

/* ---- device memory helpers (plain HIP; any HIP allocation works with the compute calls) ---- */
int ckks_buffer_alloc(size_t bytes, void** d_out);
int ckks_buffer_free(void* d);
int ckks_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes);
int ckks_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes);
/* Pinned host memory, and copies on a side stream of the context that overlap the work on the caller's stream (no
 * counterpart in the reference; for a caller that keeps copies of device data on the host while it computes):
 * ckks_side_copy   copies bytes (any direction) once the work enqueued so far on stream is done; returns a ticket.
 *                  Copies to host memory (pinned or pageable: any destination the runtime does not report as device
 *                  memory) run on one side stream, all others on another: copies of one kind complete in issue order,
 *                  copies of different kinds are not ordered against each other (wait on the ticket).  A copy from or
 *                  to pageable host memory is not asynchronous to the host.
 * ckks_side_wait   makes stream wait (without blocking the host) until the copy of ticket is done
 * ckks_side_sync   blocks the host until every side copy is done and forgets the tickets; each side copy holds two
 *                  events until the next ckks_side_sync, so a caller that issues side copies in a loop (the decode
 *                  driver: once per step) calls it periodically to release them */
int ckks_host_alloc(size_t bytes, void** h_out);
int ckks_host_free(void* h);
int ckks_side_copy(ckks_context* ctx, void* dst, const void* src, size_t bytes, void* stream, uint64_t* ticket);
int ckks_side_wait(ckks_context* ctx, uint64_t ticket, void* stream);
int ckks_side_sync(ckks_context* ctx);
int ckks_device_sync(void);

/* ---- raw stages (the hot path; all buffers device-resident, limb-major) ----------------------
 * NTT over a dense buffer uint64[n_polys][n_limbs][N]; limb l of every poly uses prime prime_idx[l]
 * (host array, n_limbs <= 96).  Forward: natural -> bit-reversed (OpenFHE
 * ForwardTransformToBitReverse, periodic_encode.hpp:240-260); inverse: bit-reversed -> natural, * N^-1.
 * Inputs must be canonical residues in [0, q); outputs are canonical. In place. */
int ckks_ntt_forward(ckks_context* ctx, uint64_t* d_data, uint32_t n_polys, uint32_t n_limbs,
                     const uint32_t* prime_idx, void* stream);
int ckks_ntt_inverse(ckks_context* ctx, uint64_t* d_data, uint32_t n_polys, uint32_t n_limbs,
                     const uint32_t* prime_idx, void* stream);

/* ---- hybrid key switching (OpenFHE HYBRID, restated by FIDESlib's modup_ksk_moddown; the reference
 * reaches it through every EvalMult / EvalRotate, gpu_real_model.cu:2762-2765,4627) ----------------
 * Level l = number of active Q limbs.  D = ceil(l / alpha) digits, alpha = ceil(L / dnum); E = l + K.
 * Extended layout [B][D][E][N]: limb t < l is Q limb t, t >= l is P limb t - l; evaluation form.
 * ckks_modup      x [B][l][N] eval -> ext [B][D][E][N] eval
 * ckks_ks_inner   ext, evk [dnum][2][L+K][N] -> acc [B][2][E][N]: acc[.][0] = sum_d ext_d * b_d, [1] with a_d
 * ckks_moddown    x [n_polys][E][N] eval -> out [n_polys][l][N] = (x_Q - BConv_{P->Q}(x_P)) * P^-1;
 *                 the P limbs of x are used as scratch (overwritten)
 * ckks_keyswitch  x [B][l][N] -> out [B][2][l][N] (ModUp, inner product, ModDown of both polys) */
int ckks_modup(ckks_context* ctx, const uint64_t* d_x, uint32_t batch, uint32_t level, uint64_t* d_ext, void* stream);
int ckks_ks_inner(ckks_context* ctx, const uint64_t* d_ext, uint32_t batch, uint32_t level, const uint64_t* d_evk,
                  uint64_t* d_acc, void* stream);
int ckks_moddown(ckks_context* ctx, uint64_t* d_x, uint32_t n_polys, uint32_t level, uint64_t* d_out, void* stream);
int ckks_keyswitch(ckks_context* ctx, const uint64_t* d_x, uint32_t batch, uint32_t level, const uint64_t* d_evk,
                   uint64_t* d_out, void* stream);

/* ---- evaluation operators (CryptoContext API mirror; ciphertexts are batches [B][2][l][N]) ---------
 * ckks_rescale             RescaleInPlace: [n_polys][l][N] -> [n_polys][l-1][N] (drop the last limb,
 *                          centered lift, * q_{l-1}^-1), in != out
 * ckks_eval_mult           EvalMult(ct, ct) with relinearization: a, b -> out [B][2][l][N]
 * ckks_eval_mult_rescale   EvalMult + RescaleInPlace fused: a, b -> out [B][2][l-1][N] (out may overlap a or b)
 * ckks_eval_add            EvalAdd(ct, ct): elementwise over [n_polys][l][N]
 * ckks_rotation_index      automorphism index of rotation step k: 5^k mod 2N (gpu_real_model.cu:1337-1360)
 * ckks_automorphism        X -> X^g on [n_polys][l][N] evaluation form (a slot permutation), in != out
 * ckks_eval_rotate         EvalRotate(ct, k) with the key of g = ckks_rotation_index(k):
 *                          KS of c1, add c0, then X -> X^g on both polys; in != out */
int ckks_rescale(ckks_context* ctx, const uint64_t* d_in, uint32_t n_polys, uint32_t level, uint64_t* d_out,
                 void* stream);
int ckks_eval_mult(ckks_context* ctx, const uint64_t* d_a, const uint64_t* d_b, uint32_t batch, uint32_t level,
                   const uint64_t* d_evk, uint64_t* d_out, void* stream);
int ckks_eval_mult_rescale(ckks_context* ctx, const uint64_t* d_a, const uint64_t* d_b, uint32_t batch,
                           uint32_t level, const uint64_t* d_evk, uint64_t* d_out, void* stream);
int ckks_eval_add(ckks_context* ctx, const uint64_t* d_x, const uint64_t* d_y, uint32_t n_polys, uint32_t level,
                  uint64_t* d_out, void* stream);

/* ckks_eval_mult_rescale_noalloc: ckks_eval_mult_rescale (same arguments, kernels and output words) that allocates
 * no device memory.  It has no counterpart in the reference: it is for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its workspace and per-call tables
 * live in a static device array of 160 MiB per GPU that the library holds until the process ends; a call whose
 * workspace, B * (3l + D(l+K) + 2(l+K) + 2(l-1) + 2) limbs of 512 KiB (D = ceil(l / alpha)), exceeds 159 MiB is
 * refused with CKKS_EINVAL (config 2's shape, L=24 K=8 dnum=3, takes one pair per call).  Every call on one GPU
 * shares that array: calls that overlap on one GPU (other streams, other host threads) race. */
int ckks_eval_mult_rescale_noalloc(ckks_context* ctx, const uint64_t* d_a, const uint64_t* d_b, uint32_t batch,
                                   uint32_t level, const uint64_t* d_evk, uint64_t* d_out, void* stream);
uint32_t ckks_rotation_index(int64_t step);
int ckks_automorphism(ckks_context* ctx, const uint64_t* d_in, uint32_t n_polys, uint32_t level, uint32_t g,
                      uint64_t* d_out, void* stream);
int ckks_eval_rotate(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, int64_t step,
                     const uint64_t* d_evk, uint64_t* d_out, void* stream);

/* ---- plaintext operators, hoisted rotations, BSGS linear transform -----------------------------
 * ckks_eval_mult_plain   EvalMult(ct, pt): both polys (.) pt; pt [l][N] shared by the batch (pt_shared = 1)
 *                        or [B][l][N]; no rescale (gpu_real_model.cu:3316-3334 multiplies then rescales once)
 * ckks_eval_add_plain    EvalAdd(ct, pt): c0 + pt
 * ckks_eval_rotate_hoisted  EvalFastRotation: one ciphertext rotated by steps[0..n) (n <= 64) with one shared
 *                        ModUp of c1; key i = the automorphism key of rotation steps[i]; out [n][2][l][N]
 * ckks_eval_rotate_many  n ciphertexts [n][2][l][N], ciphertext i rotated by steps[i] with key i (n <= 64)
 * ckks_eval_rotate_sum  out = ct + sum_i Rot_{steps[i]}(ct) for each of batch ciphertexts [B][2][l][N] (1 <= n <= 64,
 *                        no identity step): the rotate-and-add loops of the reference's lane sums
 *                        (gpu_real_model.cu:3524,3540: red = EvalAdd(red, rot(red, p))) as windows, the n rotations
 *                        hoisted over one ModUp of c1 and summed over Q_l P before one ModDown; key i = the
 *                        automorphism key of steps[i]; out may be ct.  Equal to the loop of single rotations up to
 *                        the key-switching rounding (one ModDown instead of n)
 * ckks_linear_transform_bsgs  the reference's baby-step giant-step diagonal matvec (gpu_real_model.cu:2767-2823):
 *                        out = Rescale( sum_g Rot_{g*bs}( sum_j diag[g*bs + j] (.) Rot_j(ct) ) ), diag [n_diag][l][N]
 *                        encoded plaintexts already pre-rotated by -g*bs; baby keys for steps 1..bs-1, giant keys
 *                        for steps bs, 2bs, ...; out [2][l-1][N] */
int ckks_eval_mult_plain(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, const uint64_t* d_pt,
                         int pt_shared, uint64_t* d_out, void* stream);
int ckks_eval_add_plain(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, const uint64_t* d_pt,
                        int pt_shared, uint64_t* d_out, void* stream);
int ckks_eval_rotate_hoisted(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, const int64_t* steps,
                             uint32_t n, const uint64_t* const* d_evks, uint64_t* d_out, void* stream);
int ckks_eval_rotate_many(ckks_context* ctx, const uint64_t* d_cts, uint32_t n, uint32_t level, const int64_t* steps,
                          const uint64_t* const* d_evks, uint64_t* d_out, void* stream);
int ckks_eval_rotate_sum(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, const int64_t* steps,
                         uint32_t n, const uint64_t* const* d_evks, uint64_t* d_out, void* stream);
int ckks_linear_transform_bsgs(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, const uint64_t* d_diags,
                               uint32_t n_diag, uint32_t baby_steps, const uint64_t* const* d_baby_evks,
                               const uint64_t* const* d_giant_evks, uint64_t* d_out, void* stream);

/* ---- periodic plaintexts, general transforms, linear combinations (decode-step support) ----------
 * ckks_encode_periodic      n_vectors slot vectors of period `period` (a power of two; replicated over the N/2
 *                           slots) encoded in the compressed form of hpc_gpu_port/periodic_encode.hpp:179-260:
 *                           out [n][l][2 period]; the evaluation form of limb i is comp[i][k >> log2(N/(2 period))]
 *                           (the expansion of gpu_real_model.cu:145-155)
 * ckks_eval_mult_plain_ex   ct (.) pt with pt [l][N >> log_rep] (log_rep = 0: full plaintext)
 * ckks_linear_transform_general  y = sum_g Rot_{G_g}( sum_b diag[g n_baby + b] (.) Rot_{B_b}(ct) ) with explicit
 *                           baby and giant steps (0 = identity, no key), diagonals compressed by log_rep, term
 *                           (g, b) pre-rotated by -G_g; no rescale; out [2][l][N]
 * ckks_linear_transform_multi  n_in inputs share the baby steps, n_out outputs share the babies:
 *                           out_o = sum_g Rot_{G_g}( sum_{i,b} diag[o][g][i n_baby + b] (.) Rot_{B_b}(in_i) ),
 *                           diags [n_out][n_giant][n_in n_baby][l][N >> log_rep]; rescale != 0 rescales each
 *                           output (matvecBatchImpl with shared babies, gpu_real_model.cu:2902-3424)
 * ckks_eval_mult_sum        out[c] = relin( sum_j a[c][j] (x) b[c][j] ) (+ rescale): one key switch for up to 64
 *                           products; d_pairs [batch][n_products][2] pointers to ciphertexts [2][l][N]
 * ckks_eval_rotate_masked   out[s][t] = rescale( pt[s][t][0] (.) Rot_{lo_t}(ct) + pt[s][t][1] (.) Rot_{hi_t}(ct) ),
 *                           all 2n rotations hoisted over one ModUp; pt [n_sets][n][2][l][N >> log_rep] (cyclic
 *                           rotations inside slot blocks built from two plain rotations and complementary masks)
 * ckks_eval_automorphism_ks X -> X^g with the key of g on a batch (g = 2N - 1: EvalConjugate)
 * ckks_eval_mul_i           multiply every slot by i (sign 1) or -i (sign -1): exact, no level
 * ckks_eval_lincomb         integer mode: sum_t round(c_t) x_t + round(add_const scale_out), all terms at
 *                           target_level, no rescale; scalar mode: terms at any level >= target_level + 1 (read
 *                           without copying), each scaled so the result has scale scale_out after one rescale
 *                           to target_level (FLEXIBLE scaling, gpu_real_model.cu:1156). Terms are batches
 *                           [batch][2][l_t][N]; at most 8 terms. */
int ckks_encode_periodic(ckks_context* ctx, const double* re, const double* im, uint32_t n_vectors, uint32_t period,
                         uint32_t level, double scale, uint64_t* d_out);
/* ckks_encode_periodic in two halves, so that a store of plaintexts can be kept in a level-independent form of
 * 2 period words per vector and expanded to its limbs when it is applied (the reference keeps its compressed store
 * on the host and streams it into a device pool, gpu_real_model.cu:1660-1706,3085-3285):
 * ckks_encode_periodic_coeffs  the host half: special FFT, rounding (with the approxFactor rule): d_coef
 *                              [n][2 period] int64 and d_log_approx [n] int32, device or pinned host memory
 * ckks_expand_periodic         the device half, enqueued on stream: d_out [n][level][2 period], the words
 *                              ckks_encode_periodic writes */
int ckks_encode_periodic_coeffs(ckks_context* ctx, const double* re, const double* im, uint32_t n_vectors,
                                uint32_t period, double scale, int64_t* d_coef, int32_t* d_log_approx);
int ckks_expand_periodic(ckks_context* ctx, const int64_t* d_coef, const int32_t* d_log_approx, uint32_t n_vectors,
                         uint32_t period, uint32_t level, uint64_t* d_out, void* stream);
int ckks_eval_mult_plain_ex(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level,
                            const uint64_t* d_pt, int pt_shared, uint32_t log_rep, uint64_t* d_out, void* stream);
int ckks_linear_transform_general(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, const uint64_t* d_diags,
                                  uint32_t log_rep, uint32_t n_baby, const int64_t* baby_steps,
                                  const uint64_t* const* d_baby_evks, uint32_t n_giant, const int64_t* giant_steps,
                                  const uint64_t* const* d_giant_evks, uint64_t* d_out, void* stream);
int ckks_linear_transform_multi(ckks_context* ctx, const uint64_t* const* d_in, uint32_t n_in, uint32_t level,
                                const uint64_t* d_diags, uint32_t log_rep, uint32_t n_baby, const int64_t* baby_steps,
                                const uint64_t* const* d_baby_evks, uint32_t n_giant, const int64_t* giant_steps,
                                const uint64_t* const* d_giant_evks, uint32_t n_out, int rescale, uint64_t* d_out,
                                void* stream);
/* ckks_linear_transform_hoisted  the BSGS linear transform of EvalBootstrap's CoeffToSlot / SlotToCoeff
 *                           (gpu_real_model.cu:2544; FIDESlib's hoisted transform, an external dependency) in its
 *                           double-hoisted form: the sum of ckks_linear_transform_multi with the rescale, but the
 *                           babies stay in the extended basis Q_l P (no ModDown), the diagonals multiply them there,
 *                           each giant's inner sum is brought down once, the giant rotations are summed in Q_l P and
 *                           one ModDown, fused with the rescale, ends it.  diags [n_out][n_giant][n_in n_baby][l+K][N]
 *                           over the primes of Q_l then P (uncompressed); out [n_out][2][l-1][N]; n_baby <= 32,
 *                           n_in n_baby <= 64, n_giant <= 64, at most one giant step 0.  The giants' inner sums bring
 *                           only their c1 down to Q_l; their c0 enter the rotations over Q_l P as they are.  Decrypts like
 *                           ckks_linear_transform_multi's output up to the key-switching rounding (different words). */
int ckks_linear_transform_hoisted(ckks_context* ctx, const uint64_t* const* d_in, uint32_t n_in, uint32_t level,
                                  const uint64_t* d_diags, uint32_t n_baby, const int64_t* baby_steps,
                                  const uint64_t* const* d_baby_evks, uint32_t n_giant, const int64_t* giant_steps,
                                  const uint64_t* const* d_giant_evks, uint32_t n_out, uint64_t* d_out, void* stream);
int ckks_eval_mult_sum(ckks_context* ctx, const uint64_t* const* d_pairs, uint32_t n_products, uint32_t batch,
                       uint32_t level, const uint64_t* d_evk, int rescale, uint64_t* d_out, void* stream);
int ckks_eval_rotate_masked(ckks_context* ctx, const uint64_t* d_ct, uint32_t level, uint32_t n,
                            const int64_t* steps_lo, const uint64_t* const* d_evks_lo, const int64_t* steps_hi,
                            const uint64_t* const* d_evks_hi, uint32_t n_sets, const uint64_t* d_pts,
                            uint32_t log_rep, uint64_t* d_out, void* stream);
int ckks_eval_automorphism_ks(ckks_context* ctx, const uint64_t* d_ct, uint32_t batch, uint32_t level, uint32_t g,
                              const uint64_t* d_evk, uint64_t* d_out, void* stream);
int ckks_eval_mul_i(ckks_context* ctx, const uint64_t* d_in, uint32_t n_polys, uint32_t level, int sign,
                    uint64_t* d_out, void* stream);
int ckks_eval_lincomb(ckks_context* ctx, uint32_t batch, uint32_t n_terms, const uint64_t* const* d_terms,
                      const uint32_t* levels, const double* coeffs, const double* scales_in, double scale_out,
                      double add_const, uint32_t target_level, int integer_mode, uint64_t* d_out, void* stream);

/* ---- bootstrapping (EvalBootstrapSetup / EvalBootstrapKeyGen / EvalBootstrap, gpu_real_model.cu:1335-1336,
 * 1444,2544) ------------------------------------------------------------------------------------------
 * Full-slot (N/2 slots) CKKS bootstrap: ModRaise (centered q0 limb), CoeffToSlot (3 BSGS levels), EvalMod
 * (Chebyshev interpolant of degree cheb_degree of a scaled cosine on [-1, 1], evaluated by Chebyshev
 * division, then double_angles double-angle steps; K bounds |I| of the raised message m + q0 I), SlotToCoeff
 * (3 BSGS levels).  Consumes 3 + 7 + double_angles + 3 levels: the input is the q0 limb [2][1][N] of a
 * ciphertext whose message has scale in_scale; the output has ckks_bootstrap_out_level() limbs and scale
 * S(l): CoeffToSlot runs at S(l) = top_scale on l = L, L-1, L-2 (the top three Q primes should be the
 * largest; top_scale well above the context's scale keeps its noise, which EvalMod amplifies by 2 pi K,
 * small); its last level lands on S(L-3) = the context's scale (ckks_params.scale), then
 * S(l-1) = S(l)^2 / q_{l-1} (the FLEXIBLE chain; the scaling primes must keep it near that scale).
 * in_scale may exceed the context's scale: EvalMod's signal grows with in_scale / q0.  Keys: the relinearization key, the conjugation key
 * (automorphism 2N-1) and one automorphism key per rotation step of ckks_bootstrap_steps(). */
typedef struct ckks_bootstrap ckks_bootstrap;
int ckks_gen_primes(uint32_t bits, uint32_t count, const uint64_t* skip, uint32_t n_skip, uint64_t* out);
int ckks_bootstrap_setup(ckks_context* ctx, double K, uint32_t cheb_degree, uint32_t double_angles, double top_scale,
                         double in_scale, ckks_bootstrap** out);
void ckks_bootstrap_destroy(ckks_bootstrap* bt);
/* ckks_bootstrap_setup_shared: a plan for inputs of scale in_scale that shares every CoeffToSlot / SlotToCoeff
 * diagonal of base (no counterpart in the reference, whose EvalBootstrapSetup makes one plan per context; for a
 * caller that bootstraps inputs of several scales).  base's input scale / in_scale must be an integer f >= 1:
 * EvalMod's output is multiplied by f in the recombination before SlotToCoeff, which is what base's SlotToCoeff
 * constant q0 / (2 pi in_scale) would have applied.  Either plan may be destroyed first.  Sparse-secret keys are
 * copied from base at this call (set them on base first, or on the shared plan after). */
int ckks_bootstrap_setup_shared(ckks_context* ctx, const ckks_bootstrap* base, double in_scale, ckks_bootstrap** out);
/* ckks_bootstrap_set_sparse_keys: sparse-secret encapsulation (Bossuat, Troncoso-Pastoriza, Hubaux, ePrint
 * 2022/024): the level-1 input is switched to a sparse secret s' (key s -> s', q_limbs = 1) before ModRaise and
 * the raised ciphertext back to s (key s' -> s), so that |I| is bounded by the sparse weight: K drops from
 * ~8 sqrt(h/12) to ~8 sqrt(h'/12), and EvalMod's noise (~K^2) with it.  The keys stay owned by the caller. */
int ckks_bootstrap_set_sparse_keys(ckks_bootstrap* bt, const uint64_t* d_to_sparse, const uint64_t* d_from_sparse);
int ckks_bootstrap_steps(const ckks_bootstrap* bt, int64_t* steps, uint32_t cap, uint32_t* n);
uint32_t ckks_bootstrap_out_level(const ckks_bootstrap* bt);
double ckks_bootstrap_scale(const ckks_bootstrap* bt, uint32_t level);
int ckks_eval_bootstrap(ckks_context* ctx, const ckks_bootstrap* bt, const uint64_t* d_ct_in, const uint64_t* d_relin,
                        const uint64_t* d_conj, const int64_t* steps, const uint64_t* const* d_evks, uint32_t n_keys,
                        uint64_t* d_out, void* stream);
/* ckks_eval_bootstrap_many: batch independent level-1 ciphertexts [batch][2][1][N] -> [batch][2][l_out][N] in
 * one pass (every kernel over the whole batch; keys and diagonals read once per pass); batch <= 64 */
int ckks_eval_bootstrap_many(ckks_context* ctx, const ckks_bootstrap* bt, const uint64_t* d_ct_in, uint32_t batch,
                             const uint64_t* d_relin, const uint64_t* d_conj, const int64_t* steps,
                             const uint64_t* const* d_evks, uint32_t n_keys, uint64_t* d_out, void* stream);
/* stage-wise form for testing: stops after stage 1 ModRaise, 2 CoeffToSlot, 3 split (two ciphertexts),
 * 4 EvalMod (two ciphertexts), 5 recombination, 6 the full bootstrap; writes that ciphertext (batch) to d_out
 * (sized for the top level) and its level to *level.  Synchronous on the null stream. */
int ckks_eval_bootstrap_stage(ckks_context* ctx, const ckks_bootstrap* bt, const uint64_t* d_ct_in,
                              const uint64_t* d_relin, const uint64_t* d_conj, const int64_t* steps,
                              const uint64_t* const* d_evks, uint32_t n_keys, uint32_t stage, uint64_t* d_out,
                              uint32_t* level);

/* ---- client side: keys, encoding, encryption (CryptoContext KeyGen / EvalMultKeyGen /
 * EvalRotateKeyGen / MakeCKKSPackedPlaintext / Encrypt / Decrypt, gpu_real_model.cu:1293-1336,1577-1589,
 * 2202-2221).  Not on the evaluation hot path; used to make seeded inputs and read results.
 * Sampling is seeded and deterministic: the uniform a_j of a key-switching key follow the ChaCha20
 * expander of hpc_gpu_port/seeded_keys.hpp:28-43 (nonce {digit, limb, "SKEY"}); the secret (ternary,
 * fixed Hamming weight) and the rounded-Gaussian errors use the same expander with this library's tags.
 * Encoding: slot j <-> evaluation at zeta^(5^j), zeta = exp(i pi / N); n_slots must divide N/2 (the
 * vector is replicated); encrypt is secret-key encryption (c0 = m + e - a s, c1 = a). */
typedef struct ckks_secret ckks_secret;
int ckks_secret_generate(ckks_context* ctx, const uint8_t* seed32, uint32_t hamming_weight, ckks_secret** out);
void ckks_secret_destroy(ckks_secret* sk);
int ckks_secret_coeffs(const ckks_secret* sk, int8_t* out, uint32_t n);
/* evk [dnum][2][L+K][N]; relinearization key: s^2 -> s; automorphism key of index g: s -> tau_{g^-1}(s) */
int ckks_keygen_relin(ckks_context* ctx, const ckks_secret* sk, const uint8_t* seed32, const uint8_t* eseed32,
                      uint64_t* d_evk);
/* ckks_keygen_switch: key switching from sk_from to sk_to (EvalKeySwitchGen); q_limbs > 0 publishes only Q
 * limbs [0, q_limbs) and P (zeros elsewhere): the key to a sparse secret must live at a small modulus. */
int ckks_keygen_switch(ckks_context* ctx, const ckks_secret* sk_from, const ckks_secret* sk_to,
                       const uint8_t* seed32, const uint8_t* eseed32, uint32_t q_limbs, uint64_t* d_evk);
int ckks_keygen_automorphism(ckks_context* ctx, const ckks_secret* sk, uint32_t g, const uint8_t* seed32,
                             const uint8_t* eseed32, uint64_t* d_evk);

/* ---- seeded key parts (the reference's evalrot.partNNN.seeded.bin, hpc_gpu_port/seeded_keys.hpp:44-51; written by
 * writeSeededPart :302-334, read by readSeededPartHeader :338-360 and expandSeededKeys :374-415) ----------------
 * A part file holds `count` automorphism keys as (index, 32-byte seed, b-halves); each key's a-halves are the
 * ChaCha20 expansion of its seed (seeded_keys.hpp:28-43), so a loaded key equals the written one word for word.
 * ckks_seeded_part_read_header  the header (host only, no context): format and truncation errors are CKKS_EINVAL
 * ckks_seeded_part_indices      the automorphism index of each record (up to cap of them)
 * ckks_seeded_part_load_key     record -> d_evk [dnum][2][L+K][N]; the file's N, chain, special primes and digit
 *                               partition must be the context's (the loader's refusal of another context's parts)
 * ckks_seeded_part_write        n keys of this context into one part file: indices, seeds [n][32] (the seed each
 *                               key's a-halves were drawn from, the seed32 of ckks_keygen_automorphism), device keys */
typedef struct ckks_seeded_part_header {
    uint32_t version, expander, ring_dim, size_q, size_p, num_part_q, num_per_part_q, count;
    char key_tag[256]; /* NUL-terminated (longer tags are refused) */
    uint64_t moduli[128]; /* size_q + size_p of them */
} ckks_seeded_part_header;
int ckks_seeded_part_read_header(const char* path, ckks_seeded_part_header* out);
int ckks_seeded_part_indices(const char* path, uint32_t* indices, uint32_t cap, uint32_t* count);
int ckks_seeded_part_load_key(ckks_context* ctx, const char* path, uint32_t record, uint32_t* index, uint64_t* d_evk);
int ckks_seeded_part_write(ckks_context* ctx, const char* path, const char* key_tag, uint32_t n_keys,
                           const uint32_t* indices, const uint8_t* seeds, const uint64_t* const* d_evks);

/* ---- the FIDESlib .dev sidecar (cryptocontext.bin.dev: written by the reference client's writeDevSidecar,
 * hpc_gpu_port/mac_fhe_client.cpp:178-194; read by FIDESlib's LoadContext, which uploads the key of every listed
 * rotation from the key map gpu_real_model.cu:1436-1529 fills) -----------------------------------------------------
 * Six text lines: "1 { 0 }" (devices), "AutoLoadCiphertexts: 1", "AutoLoadPlaintexts: 0", "RotationIndexes: { ... }"
 * (rotation AMOUNTS, EvalRotate steps), "KeyDist: 1", "BootstrapSlots: { ... }" (slot counts); no binary content.
 * ckks_dev_sidecar_read       (host only) flags and counts into info, up to rot_cap rotation amounts and slot_cap
 *                             slot counts in file order; a malformed file is CKKS_EINVAL naming the line and reason
 * ckks_dev_sidecar_write      (host only) the reference writer's file: device 0, AutoLoadCiphertexts 1,
 *                             AutoLoadPlaintexts 0, KeyDist 1, the rotation amounts and slot counts as given
 * ckks_rotation_keys_resolve  (host only) for each rotation the sidecar lists (in its order): the part file (index
 *                             into part_paths), the record and the automorphism index 5^k mod 2N of its key; a
 *                             rotation whose key no part holds is CKKS_EINVAL (FIDESlib aborts on it: map::at)
 * ckks_rotation_keys_load     LoadContext's rotation keys: the key of each listed rotation, from the parts, into
 *                             d_evks[i] [dnum][2][L+K][N]; n_keys must be the sidecar's rotation count */
typedef struct ckks_dev_sidecar {
    uint32_t n_devices;
    uint32_t devices[64];
    int32_t auto_load_ciphertexts, auto_load_plaintexts, key_dist;
    uint32_t n_rotations, n_boot_slots;
} ckks_dev_sidecar;
int ckks_dev_sidecar_read(const char* path, ckks_dev_sidecar* info, int32_t* rotations, uint32_t rot_cap,
                          uint32_t* boot_slots, uint32_t slot_cap);
int ckks_dev_sidecar_write(const char* path, const int32_t* rotations, uint32_t n_rotations, const uint32_t* boot_slots,
                           uint32_t n_boot_slots);
int ckks_rotation_keys_resolve(const char* dev_path, const char* const* part_paths, uint32_t n_parts,
                               uint32_t* part_of, uint32_t* record_of, uint32_t* index_of, uint32_t cap, uint32_t* n);
int ckks_rotation_keys_load(ckks_context* ctx, const char* dev_path, const char* const* part_paths, uint32_t n_parts,
                            uint64_t* const* d_evks, uint32_t n_keys);

/* ---- ciphertext files (the payload of the serve-directory protocol's req.N.t / resp.N.t; the reference serializes
 * OpenFHE-cereal ciphertexts there, hpc_gpu_port/gpu_real_model.cu:2303-2324, a format only OpenFHE reads) ------
 * Layout (little-endian): char[8] "FSSMCTX1"; u32 version = 1; u32 N; u32 level; u32 n_polys = 2; f64 scale;
 * u64 moduli[level]; u64 words[2][level][N] (evaluation form, canonical residues).
 * ckks_ct_file_info  the header (host only, no context); format and size errors are CKKS_EINVAL
 * ckks_ct_save       d_ct [2][level][N] of this context into a file
 * ckks_ct_load       a file into d_ct (room for cap_level limbs); its ring, moduli and words must be this
 *                    context's (every word below its prime) */
int ckks_ct_file_info(const char* path, uint32_t* ring_dim, uint32_t* level, double* scale);
int ckks_ct_save(ckks_context* ctx, const char* path, const uint64_t* d_ct, uint32_t level, double scale);
int ckks_ct_load(ckks_context* ctx, const char* path, uint32_t cap_level, uint64_t* d_ct, uint32_t* level,
                 double* scale);

int ckks_encode(ckks_context* ctx, const double* re, const double* im, uint32_t n_slots, uint32_t level, double scale,
                uint64_t* d_pt);
int ckks_encrypt(ckks_context* ctx, const ckks_secret* sk, const uint64_t* d_pt, uint32_t level, const uint8_t* seed32,
                 uint32_t index, uint64_t* d_ct);
/* public key (PKEBase::KeyGenInternal, harness/boot_overflow_probe.cpp:22,132-142: b = ns*e - a*s over the
 * key's basis, elements {b, a}; ns = 1): d_pk [2][L+K][N] over Q*P, b = e - a s.  ckks_encrypt_public encrypts
 * with it at any level as the client's Encrypt(publicKey, pt) does (gpu_real_model.cu:2202-2221 encCh; the
 * client holds no secret, mac_fhe_client.cpp:570-609): ct = (ModDown(b v + e0) + m, ModDown(a v + e1)), v uniform
 * ternary, e0/e1 Gaussian, all from seed32 and index; needs special primes. */
int ckks_keygen_public(ckks_context* ctx, const ckks_secret* sk, const uint8_t* seed32, const uint8_t* eseed32,
                       uint64_t* d_pk);
int ckks_encrypt_public(ckks_context* ctx, const uint64_t* d_pk, const uint64_t* d_pt, uint32_t level,
                        const uint8_t* seed32, uint32_t index, uint64_t* d_ct);
int ckks_decrypt_decode(ckks_context* ctx, const ckks_secret* sk, const uint64_t* d_ct, uint32_t level, double scale,
                        double* re, double* im, uint32_t n_slots);
/* decryption to the N centered coefficients (CRT of the first two limbs) as doubles */
int ckks_decrypt_coeffs(ckks_context* ctx, const ckks_secret* sk, const uint64_t* d_ct, uint32_t level, double* out);

/* ---- per-launch profiling (HIP events on the launch stream) ------------------------------------
 * enable: start recording every kernel launch (name, algorithmic bytes, start/stop events);
 * query: aggregated per kernel name, idx = 0..; returns CKKS_EINVAL past the last name.
 * Waits for the recorded events. */
/* ckks_context_counters: key switches issued since the last reset (one per ciphertext key-switched) */
int ckks_context_counters(ckks_context* ctx, uint64_t* key_switches, int reset);
/* ckks_context_memory: device bytes the context holds itself (no counterpart in the reference; for memory
 * accounting): bytes[0] constant tables (twiddles, small-ring tables, prime data), bytes[1] the growable
 * key-switching workspaces, bytes[2] the bootstrapping buffer pool (free buffers kept for the next call),
 * bytes[3] the static scratch of ckks_eval_mult_rescale_noalloc (a 160 MiB device array the library holds on each
 * GPU it runs on whether or not that entry point is called, shared by every context on the GPU).
 * Fills min(n, 4) entries. */
int ckks_context_memory(const ckks_context* ctx, uint64_t* bytes, uint32_t n);
int ckks_profile_enable(ckks_context* ctx, int on);
/* phase attribution (no counterpart in the reference; for measurement): ckks_profile_phase labels the launches that
 * follow (every profiled launch records the label; the bootstrap labels its own stages boot_modraise,
 * boot_coeff_to_slot, boot_eval_mod, boot_slot_to_coeff and restores the caller's label); with
 * ckks_profile_phase_markers on, each change of label also enqueues on stream an empty kernel k_phase_mark of
 * id + 1 workgroups (id: the label's marker id, in order of first use), so that a trace or a counter pass of the
 * kernels can be split by phase.  ckks_profile_phase_query aggregates the profiled launches by label. */
int ckks_profile_phase(ckks_context* ctx, const char* phase, void* stream);
int ckks_profile_phase_markers(ckks_context* ctx, int on);
int ckks_profile_phase_query(ckks_context* ctx, uint32_t idx, char* name, uint32_t name_cap, uint64_t* launches,
                             double* total_ms, double* total_bytes, int32_t* marker_id);
/* the marker id of a label (-1: never set while markers were on) */
int ckks_profile_phase_id(const ckks_context* ctx, const char* phase, int32_t* marker_id);
int ckks_profile_reset(ckks_context* ctx);
int ckks_profile_query(ckks_context* ctx, uint32_t idx, char* name, uint32_t name_cap, uint64_t* launches,
                       double* total_ms, double* total_bytes);

#ifdef __cplusplus
}
#endif
#endif
