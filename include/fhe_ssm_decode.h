/* fhe_ssm_decode.h -- the config-5 encrypted decode step as a native driver over ckks_engine.h.
 *
 * This is the caller side of the hot path: the per-layer loop of the reference's served FHE step
 * (hpc_gpu_port/gpu_real_model.cu:4674-5300 -- RMSNorm, token shift, matvecBatch with shared babies, WKV scan,
 * gate, output projection, residual, channel mix; refresh/bootstrap policy :2535-2599), written against the
 * engine's C ABI only.  The model is RWKV-7-0.1B-shaped (12 layers, d = 768, 12 heads x 64, channel-mix width
 * 3072) with every nonlinearity a degree-3 polynomial; 32 conversation lanes share the slots of one N = 2^16
 * ciphertext (slot lane*1024 + channel).  The WKV state and both token-shift carries live inside the decoder
 * and persist across steps.
 *
 * Level rules (OpenFHE FLEXIBLEAUTO, gpu_real_model.cu:1156): a ciphertext at level l carries the canonical
 * scale S(l) of the state's bootstrapping plan; operands above their partner's level are brought down by one
 * scalar multiplication that lands on S(l).  Refresh policy: the residual stream stays at the top level; the
 * time-mix and channel-mix increments are bootstrapped on their own (their own plans and input scales) and
 * added back; the WKV state is bootstrapped once per layer, packed two per ciphertext (D_t + i D_{t+32}).
 *
 * Every function returns 0 or a CKKS_* status code; fhe_ssm_last_error() gives the message.  A decoder is
 * used from one host thread; all device work goes to the null stream in call order.
 */
#ifndef FHE_SSM_DECODE_H
#define FHE_SSM_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "ckks_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fhe_ssm_decoder fhe_ssm_decoder;

/* One refresh kind: its bootstrapping plan and the scale its input is brought to before ModRaise. */
typedef struct {
    const ckks_bootstrap* plan;
    double in_scale;
} fhe_ssm_refresh;

const char* fhe_ssm_last_error(void);

/* Replaces the driver's LoadContext + key loading (gpu_real_model.cu:1436-1530).  relin, conj (automorphism
 * 2N - 1) and one automorphism key per rotation step: every step of fhe_ssm_rotation_steps() and of the three
 * plans' ckks_bootstrap_steps().  Keys stay owned by the caller and must outlive the decoder. */
int fhe_ssm_decoder_create(ckks_context* ctx, uint32_t n_layers, fhe_ssm_refresh state, fhe_ssm_refresh inc_tm,
                           fhe_ssm_refresh inc_cm, const uint64_t* d_relin, const uint64_t* d_conj,
                           const int64_t* steps, const uint64_t* const* d_evks, uint32_t n_keys,
                           fhe_ssm_decoder** out);
void fhe_ssm_decoder_destroy(fhe_ssm_decoder* dec);

/* The rotation steps the layer loop itself uses (matvec babies/giants, WKV block rotations, norm sums);
 * n_steps receives the count (at most cap written). */
int fhe_ssm_rotation_steps(int64_t* steps, uint32_t cap, uint32_t* n_steps);

/* Weights, float64 row-major, per layer (0..n_layers-1) or model-wide (layer = -1):
 *   per layer  g1, g2, k_k, k_a, r_k, ln_w, ln_b, mu_r, mu_k, mu_v, mu_w, mu_a, mu_g, mu_c  [768]
 *              W_r, W_k, W_v, W_w, W_a, W_g, W_vg, W_o  [768][768];  W_ck [3072][768];  W_cv [768][3072]
 *              p_n1, p_n2, p_w, p_a, p_g, p_v, p_kn, p_gn, p_h  [4]  (polynomial c0 + c1 z + c2 z^2 + c3 z^3)
 *              (W_vg and p_v, the value gate, are read in layers > 0 only; layer 0 sets the value they mix toward)
 *   model      g_o [768], p_o [4]
 * count must match.  All must be set before the first step; plaintexts are encoded on first use. */
int fhe_ssm_decoder_set_weight(fhe_ssm_decoder* dec, const char* name, int32_t layer, const double* data,
                               size_t count);

/* One decode step.  d_x: the lanes' embeddings [2][level][N] at level = the state plan's output level with
 * scale S(level).  d_out receives the output-normed hidden state [2][*out_level][N] (sized for the input
 * level), its scale in *out_scale. */
int fhe_ssm_decoder_step(fhe_ssm_decoder* dec, const uint64_t* d_x, uint32_t level, double scale, uint64_t* d_out,
                         uint32_t* out_level, double* out_scale);

/* ciphertexts bootstrapped so far (28 per layer per step) */
int fhe_ssm_decoder_stats(const fhe_ssm_decoder* dec, uint64_t* bootstraps);

/* Drop the carried state (WKV state and both token-shift carries of every layer): the next step starts cold, as
 * the first one did.  The serve loop's req.N.reset / stateless request (gpu_real_model.cu:4461-4465). */
int fhe_ssm_decoder_reset(fhe_ssm_decoder* dec);
/* Bytes the decoder holds (no counterpart in the reference; for memory accounting): device bytes[0] the elementwise
 * plaintexts, bytes[1] the buffers the matvec diagonals are staged and expanded in, bytes[2] the ciphertext pool
 * (every buffer it has allocated, in use or free), bytes[3] the carried state (part of bytes[2]); pinned host
 * bytes[4] the copy of the previous state a step puts back if it fails, bytes[5] the matvec diagonals'
 * coefficients.  Fills min(n, 6) entries. */
int fhe_ssm_decoder_memory(const fhe_ssm_decoder* dec, uint64_t* bytes, uint32_t n);

/* ---- the compressed plaintext store file (the reference's --store-file with its append journal,
 * gpu_real_model.cu:1887-2141) ---------------------------------------------------------------------------------
 * Base file: "FHESSMSTORE1" and 4 zero bytes, u64 stamp length (1..4096), the stamp, u64 entry count (<= 10^8), per
 * entry 7 int32 key fields (layer, op, chunk, rowOff, diag, half, lvl), u64 word count and the words (u64), then an
 * FNV-1a hash over 64-bit words (offset basis 1469598103934665603, prime 1099511628211) of every entry's key fields
 * (each the u64 of its uint32), word count and words.  Written
 * whole through PATH.tmp and a rename.  Journal (conventionally PATH.journal): appended records of key fields, word
 * count, words and the FNV of that record; on load a record cut short or failing its hash ends the journal and the
 * file is truncated to the good prefix (a process killed mid-append loses that record only).  Length rule (depth > 0,
 * the reference's check): an entry's lvl lies in [0, depth] and it holds 0 (dead) or (depth + 1 - lvl) comp_cw words,
 * the limbs of a compressed plaintext (comp_cw = N / REP words per limb; such an entry is a plaintext
 * ckks_eval_mult_plain_ex takes with log_rep = log2 REP).  depth = 0: no length rule.
 * fhe_ssm_store_load refuses a bad magic, a stamp other than `stamp` (null: any), a truncated file, a broken rule, a
 * key already present and a checksum mismatch; entries are listed in key order. */
typedef struct fhe_ssm_store fhe_ssm_store;
int fhe_ssm_store_create(fhe_ssm_store** st);
void fhe_ssm_store_destroy(fhe_ssm_store* st);
int fhe_ssm_store_put(fhe_ssm_store* st, const int32_t* key7, const uint64_t* words, uint64_t n_words);
int fhe_ssm_store_count(const fhe_ssm_store* st, uint64_t* n);
int fhe_ssm_store_entry(const fhe_ssm_store* st, uint64_t i, int32_t* key7, uint64_t* n_words);
/* words may be null (the length only); cap: words the buffer holds */
int fhe_ssm_store_get(const fhe_ssm_store* st, const int32_t* key7, uint64_t* words, uint64_t cap, uint64_t* n_words);
int fhe_ssm_store_save(const fhe_ssm_store* st, const char* path, const char* stamp);
int fhe_ssm_store_load(fhe_ssm_store* st, const char* path, const char* stamp, uint32_t depth, uint32_t comp_cw,
                       uint64_t* n_loaded);
/* the stamp of a store file (*len bytes; stamp, if given, receives it NUL-terminated, cap >= *len + 1) */
int fhe_ssm_store_read_stamp(const char* path, char* stamp, uint64_t cap, uint64_t* len);
int fhe_ssm_store_append(const char* journal_path, const int32_t* key7, const uint64_t* words, uint64_t n_words);
/* good: records added; duplicates: records whose key was present (skipped); dropped_bytes: the torn tail removed */
int fhe_ssm_store_load_journal(fhe_ssm_store* st, const char* journal_path, uint32_t depth, uint32_t comp_cw,
                               uint64_t* good, uint64_t* duplicates, uint64_t* dropped_bytes);

/* The decoder's matvec store in a store file: fhe_ssm_decoder_store_save writes every matvec encoded so far (one
 * entry each: key (layer, op 1 tm / 2 wo / 3 ck / 4 cv, n_out, n_in, n_diag, nb, level), the small-ring coefficients
 * of its 1024-periodic diagonals and their approxFactor exponents as words); fhe_ssm_decoder_store_load, before the
 * first step, takes them from the file instead of encoding them.  The stamp names the ring, the slot layout, the
 * context's moduli, the plan's scales and every weight: a file made for anything else is refused. */
int fhe_ssm_decoder_store_save(fhe_ssm_decoder* dec, const char* path, uint64_t* n_entries);
int fhe_ssm_decoder_store_load(fhe_ssm_decoder* dec, const char* path, uint64_t* n_entries);

/* ---- the serve-directory protocol (the reference's persistent --serve DIR loop, gpu_real_model.cu:4363-4483 and
 * :5525-5576; its client is ml-eval/fhe_client.py:1394-1492) -------------------------------------------------
 * Inside dir, request N: the client writes req.N.0 .. req.N.<count-1> (ciphertext files, ckks_ct_save's layout),
 * req.N.meta -- one-line JSON {"count","packTokens","tokensReal","dpad","interleave","lanes","ringDim","level"}
 * with integer values -- optionally req.N.reset, and req.N.ready last.  The server answers with resp.N.<t>,
 * resp.N.meta and then resp.N.done (resp.N.error on failure), and only then removes the request's files, the
 * ready marker last.  While waiting it keeps serve.status ({"nextReq","served","pid","stateful","storeFile"})
 * current.  It returns on a file named `stop` or after timeout_sec idle seconds. */
typedef struct {
    uint32_t timeout_sec; /* idle seconds with no request before returning */
    uint32_t poll_ms;     /* 0: 200 */
    int32_t stateful;     /* 0: every request starts from a cold state; 1: the state carries across requests */
    int32_t log_fd;       /* JSON log lines (waiting, request, stateReset, badRequest, served, exit) go here; -1: none */
    uint32_t first_req;   /* the first request index (0 for a fresh client session) */
} fhe_ssm_serve_opts;

typedef struct {
    uint32_t served;      /* requests answered (done or error) */
    uint32_t failed;      /* of those, answered with resp.N.error (bad meta included) */
    uint32_t next_req;    /* the index the server was waiting for when it returned */
    int32_t exit_reason;  /* 0: stop file; 1: idle timeout */
} fhe_ssm_serve_report;

/* A request's computation: read req_prefix.<t> for t < count (count and the rest in meta_json), write
 * resp_prefix.<t> and resp_prefix.meta; reset: drop the carried state first.  Returns 0, or nonzero with a
 * message in err (err_cap bytes). */
typedef int (*fhe_ssm_serve_handler)(void* user, uint32_t req, const char* req_prefix, const char* resp_prefix,
                                     const char* meta_json, int32_t reset, char* err, size_t err_cap);

/* The protocol loop over any handler (host only; no device work of its own). */
int fhe_ssm_serve_dir(const char* dir, const fhe_ssm_serve_opts* opts, fhe_ssm_serve_handler handler, void* user,
                      fhe_ssm_serve_report* report);

/* The protocol loop with the decode step as its handler: every request holds count = tokensReal ciphertexts, one
 * token of up to 32 lanes each (packTokens 1, dpad 1024, ringDim 65536, at the state plan's output level), run as
 * consecutive steps; resp.N.<t> is step t's output.  A meta that does not describe this layout is answered with
 * resp.N.error. */
int fhe_ssm_decoder_serve(fhe_ssm_decoder* dec, const char* dir, const fhe_ssm_serve_opts* opts,
                          fhe_ssm_serve_report* report);

/* ---- the client's file steps (the reference driver's --enc-in and --dec-out, gpu_real_model.cu:2345-2533; the
 * client invokes them per tick, ml-eval/fhe_client.py:1312-1328) --------------------------------------------------
 * fhe_ssm_client_encrypt_rows   reads rows_path: lanes x tokens x d float64 little-endian rows, lane-major (lane r's
 *   tokens rows first, fhe_client.py:206-238); token t's ciphertext holds slot rep*dpad + i = lane (rep mod lanes)
 *   channel i for every rep < (N/2)/dpad (gpu_real_model.cu:2378-2395), encoded at level with scale and encrypted
 *   under the public key d_pk (ckks_encrypt_public, seed32 and index t); writes rows_path.ct.<t> (ckks_ct_save
 *   layout) and rows_path.ct.meta {"count","packTokens":1,"tokensReal","dpad","interleave":0,"lanes","ringDim",
 *   "level"} (writeCtMeta, :2333-2340; the reference writes level 0, this engine the ciphertexts' level).  A file
 *   shorter than the rows is refused (CKKS_EINVAL), as the reference's "short file" fatal.
 * fhe_ssm_client_decrypt_logits reads in_prefix.meta and in_prefix.<t> for t < tokensReal, decrypts each, and
 *   writes in_prefix.logits.f64: tokensReal * lanes rows (token-major, lane-minor) of vocab float64, row = head
 *   (vocab x d, row-major) times the lane's first d channels (slot lane*dpad + j) (:2468-2522).  A meta whose
 *   ringDim, dpad, interleave or packTokens differs is refused (the reference's "layout mismatch"). */
int fhe_ssm_client_encrypt_rows(ckks_context* ctx, const uint64_t* d_pk, const char* rows_path, uint32_t tokens,
                                uint32_t lanes, uint32_t d, uint32_t dpad, uint32_t level, double scale,
                                const uint8_t* seed32);
int fhe_ssm_client_decrypt_logits(ckks_context* ctx, const ckks_secret* sk, const char* in_prefix,
                                  const double* head, uint32_t vocab, uint32_t d, uint32_t dpad);

/* An integer value of a meta sidecar's one-line JSON (the reference's metaInt, gpu_real_model.cu:2327-2331); dflt
 * when the key is absent. */
long long fhe_ssm_meta_int(const char* text, const char* key, long long dflt);

#ifdef __cplusplus
}
#endif

#endif /* FHE_SSM_DECODE_H */
