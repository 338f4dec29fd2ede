// ops.hpp -- host-side composition of the hot path (see ops.cpp).
#pragma once
#include "engine.hpp"

namespace fhe {

// workspace slots (grown on demand, owned by the context)
enum WsSlot : uint32_t {
    WS_X2C = 0,
    WS_EXT,
    WS_ACC,
    WS_CONV,
    WS_LAST,
    WS_RTMP,
    WS_D01,
    WS_RELIN,
    WS_C1,
    WS_BABY,
    WS_GIANT,
    WS_GROT,
    WS_SUM,
    WS_LIN,
    WS_PTAB,
    WS_BINP,
    WS_RTMP2,
    WS_EXT2,  // a second ModUp extension (double-hoisted BSGS: the inputs' while the giants' is in use)
    WS_COUNT
};

void* ws_get(Context& ctx, uint32_t slot, size_t bytes);
uint32_t ring_acquire(Context& ctx);
void ring_release(Context& ctx, uint32_t slot, hipStream_t st);
// col_scale (optional, one factor per output): every table column j (and its centered correction) is multiplied
// by col_scale[j] mod p_j, so output j comes out as conv_j * col_scale[j]
const BConvPlan& bconv_plan(Context& ctx, const std::vector<uint32_t>& in_idx, const std::vector<uint32_t>& out_idx,
                            bool centered = false, const std::vector<uint64_t>& col_scale = {});
uint32_t num_digits(const Context& ctx, uint32_t l);

// x_bstride: words between the B input polys (0: l * N; 2 l N reads the c1 of a ciphertext batch in place)
void modup(Context& ctx, const uint64_t* x, uint64_t* ext, uint32_t B, uint32_t l, hipStream_t st,
           uint64_t x_bstride = 0);
void ks_inner(Context& ctx, const uint64_t* ext, const uint64_t* evk, uint64_t* acc, uint32_t B, uint32_t l,
              hipStream_t st);
// add (optional): applied to output polys pc with pc % add_div == 0, at add + (pc / add_div) * add_div * l * N
// add_pstride < 0: add_div * l * N (the addend is a ciphertext batch); 0: one addend for every poly
// add_group (0 = add_div): polys pc with pc % add_div == 0 take the addend at (pc / add_group) * add_pstride
// x_plimbs (0 = E): limbs between consecutive polys of x (2E takes every other poly of a QP ciphertext batch)
void moddown_inplace(Context& ctx, uint64_t* x, uint32_t n_polys, uint32_t l, const uint64_t* add, uint64_t* out,
                     hipStream_t st, uint32_t add_div = 1, int64_t add_pstride = -1, uint32_t add_group = 0,
                     uint32_t x_plimbs = 0);
// ta, tb (with ext): the inputs [B][2][l][N] of the product being relinearized; add then holds d0 and d1 at limb
// l-1 only and the combine forms the other limbs' d0 = a0 b0, d1 = a0 b1 + a1 b0 itself
// x_from_ext (with ext and evk): limb l-1 and the P limbs of x are not read but formed as the evk inner product by
// their inverse NTT (x receives them)
// An integer affine map applied to a rescaled product as it is formed: out = factor * out + post (post on poly 0
// only; both reduced mod q_i).  The words are those of the product followed by an integer linear combination.
struct Affine {
    int64_t factor;
    int64_t post;
};
// aff (optional, a relinearization with ext only): the output is factor * out + post (Affine)
// own_from_inputs (with ta, tb, two-pass NTT mode, at most 4 digits): ext holds no own-digit words below limb l-1 (the
// combine forms them as a1 b1)
void moddown_rescale(Context& ctx, uint64_t* x, uint32_t n_polys, uint32_t l, const uint64_t* add, uint64_t* out,
                     hipStream_t st, const uint64_t* ext = nullptr, const uint64_t* evk = nullptr,
                     const uint64_t* ta = nullptr, const uint64_t* tb = nullptr, bool x_from_ext = false,
                     const Affine* aff = nullptr, bool own_from_inputs = false);
void keyswitch(Context& ctx, const uint64_t* x, uint32_t B, uint32_t l, const uint64_t* evk, const uint64_t* add,
               uint64_t* out2, hipStream_t st, uint32_t add_div = 1, uint64_t x_bstride = 0);
void rescale(Context& ctx, const uint64_t* in, uint32_t n_polys, uint32_t l, uint64_t* out, hipStream_t st);
// out [B][2][lo-1][N] = rescale(sum_t C_t x_t + add): C [n_terms][lo], add [lo] or null (reduced mod q_i), term t read
// at stride[t] limbs per poly; the combination is not stored under the two-pass NTT
void rescale_lincomb(Context& ctx, uint32_t B, uint32_t lo, uint32_t n_terms, const uint64_t* const* x,
                     const uint32_t* stride, const uint64_t* C, const uint64_t* add, uint64_t* out, hipStream_t st);
// aff (with do_rescale only): the rescaled product becomes factor * product + post (Affine)
void hmult(Context& ctx, const uint64_t* a, const uint64_t* b, uint32_t B, uint32_t l, const uint64_t* evk,
           uint64_t* out, bool do_rescale, hipStream_t st, const Affine* aff = nullptr);
// hmult with the rescale, workspace and tables in the device scratch (no allocation); refuses shapes whose
// workspace exceeds it
size_t hmult_rescale_scratch_bytes(const Context& ctx, uint32_t B, uint32_t l);
void hmult_rescale_noalloc(Context& ctx, const uint64_t* a, const uint64_t* b, uint32_t B, uint32_t l,
                           const uint64_t* evk, uint64_t* out, hipStream_t st);
void rotate(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, uint32_t g, const uint64_t* evk, uint64_t* out,
            hipStream_t st);
void add(Context& ctx, const uint64_t* x, const uint64_t* y, uint64_t* out, uint32_t n_polys, uint32_t l,
         hipStream_t st);
uint32_t rotation_index(int64_t k);
void rotate_sum(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, const int64_t* steps, uint32_t n,
                const uint64_t* const* evk, uint64_t* out, hipStream_t st);
void rotate_list(Context& ctx, const uint64_t* cts, uint32_t n, uint32_t l, const int64_t* steps,
                 const uint64_t* const* evk, uint64_t* out, hipStream_t st);
void automorph_ks_list(Context& ctx, const uint64_t* cts, uint32_t n, uint32_t l, const uint32_t* gidx,
                       const uint64_t* const* evk, uint64_t* out, hipStream_t st);
void bsgs_general(Context& ctx, const uint64_t* ct, uint32_t l, const uint64_t* diags, uint32_t nb,
                  const int64_t* bsteps, const uint64_t* const* bevk, uint32_t ng, const int64_t* gsteps,
                  const uint64_t* const* gevk, uint64_t* out, hipStream_t st, uint32_t log_rep = 0);
void rotate_hoisted(Context& ctx, const uint64_t* ct, uint32_t l, const int64_t* steps, uint32_t n,
                    const uint64_t* const* evk, uint64_t* out, hipStream_t st);
void rotate_hoisted_ext(Context& ctx, const uint64_t* ct, const uint64_t* ext, uint32_t l, const int64_t* steps,
                        uint32_t n, const uint64_t* const* evk, uint64_t* out, hipStream_t st);
void rotate_hoisted_multi(Context& ctx, const uint64_t* cts, uint32_t n_ct, uint32_t l, const int64_t* steps,
                          uint32_t n, const uint64_t* const* evk, uint64_t* out, hipStream_t st);
void bsgs_multi_batch(Context& ctx, const uint64_t* const* in, uint32_t n_inst, uint32_t n_in, uint32_t l,
                      const uint64_t* diags, uint32_t nb, const int64_t* bsteps, const uint64_t* const* bevk,
                      uint32_t ng, const int64_t* gsteps, const uint64_t* const* gevk, uint32_t n_out,
                      bool do_rescale, uint64_t* out, hipStream_t st, uint32_t log_rep, bool by_output);
// double-hoisted bsgs_multi_batch with the rescale: diags_qp [n_out][ng][n_in nb][l + K][N] over Q_l * P
void bsgs_dh_batch(Context& ctx, const uint64_t* const* in, uint32_t n_inst, uint32_t n_in, uint32_t l,
                   const uint64_t* diags_qp, uint32_t nb, const int64_t* bsteps, const uint64_t* const* bevk,
                   uint32_t ng, const int64_t* gsteps, const uint64_t* const* gevk, uint32_t n_out, uint64_t* out,
                   hipStream_t st, bool by_output);
void hmult_sum(Context& ctx, const uint64_t* const* pairs, uint32_t np, uint32_t B, uint32_t l, const uint64_t* evk,
               uint64_t* out, bool do_rescale, hipStream_t st);
void bsgs_multi(Context& ctx, const uint64_t* const* in, uint32_t n_in, uint32_t l, const uint64_t* diags,
                uint32_t nb, const int64_t* bsteps, const uint64_t* const* bevk, uint32_t ng, const int64_t* gsteps,
                const uint64_t* const* gevk, uint32_t n_out, bool do_rescale, uint64_t* out, hipStream_t st,
                uint32_t log_rep);
void rotate_masked(Context& ctx, const uint64_t* ct, uint32_t l, uint32_t n, const int64_t* lo,
                   const uint64_t* const* lo_evk, const int64_t* hi, const uint64_t* const* hi_evk, uint32_t n_sets,
                   const uint64_t* pts, uint32_t log_rep, uint64_t* out, hipStream_t st);
void mul_i(Context& ctx, const uint64_t* x, uint32_t n_polys, uint32_t l, int sign, uint64_t* out, hipStream_t st);
void mul_plain(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, const uint64_t* pt, bool pt_shared,
               uint64_t* out, hipStream_t st, uint32_t log_rep = 0);
void add_plain(Context& ctx, const uint64_t* ct, uint32_t B, uint32_t l, const uint64_t* pt, bool pt_shared,
               uint64_t* out, hipStream_t st);
void bsgs_matvec(Context& ctx, const uint64_t* ct, uint32_t l, const uint64_t* diags, uint32_t n_diag, uint32_t bs,
                 const uint64_t* const* baby_evk, const uint64_t* const* giant_evk, uint64_t* out, hipStream_t st);
void lincomb(Context& ctx, uint32_t B, uint32_t n_terms, const uint64_t* const* x, const uint32_t* levels,
             const double* coeffs, const double* scales_in, double scale_out, double add_const, uint32_t lt,
             bool integer_mode, uint64_t* out, hipStream_t st);
void automorph(Context& ctx, const uint64_t* in, uint64_t* out, uint32_t n_polys, uint32_t l, uint32_t g,
               hipStream_t st);

}  // namespace fhe
