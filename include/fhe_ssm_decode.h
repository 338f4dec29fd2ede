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
 *   per layer  g1, g2, eta, mu_r, mu_k, mu_v, mu_w, mu_a, mu_g, mu_c  [768]
 *              W_r, W_k, W_v, W_w, W_a, W_g, W_o  [768][768];  W_ck [3072][768];  W_cv [768][3072]
 *              p_n1, p_n2, p_w, p_a, p_g, p_h  [4]  (polynomial c0 + c1 z + c2 z^2 + c3 z^3)
 *   model      g_o [768], p_o [4]
 * count must match.  All must be set before the first step; plaintexts are encoded on first use. */
int fhe_ssm_decoder_set_weight(fhe_ssm_decoder* dec, const char* name, int32_t layer, const double* data,
                               size_t count);

/* One decode step.  d_x: the lanes' embeddings [2][level][N] at level = the state plan's output level with
 * scale S(level).  d_out receives the output-normed hidden state [2][*out_level][N] (sized for the input
 * level), its scale in *out_scale. */
int fhe_ssm_decoder_step(fhe_ssm_decoder* dec, const uint64_t* d_x, uint32_t level, double scale, uint64_t* d_out,
                         uint32_t* out_level, double* out_scale);

/* ciphertexts bootstrapped so far (26 per layer per step) */
int fhe_ssm_decoder_stats(const fhe_ssm_decoder* dec, uint64_t* bootstraps);

#ifdef __cplusplus
}
#endif

#endif /* FHE_SSM_DECODE_H */
