// bootstrap.hpp -- CKKS bootstrapping plan and evaluation (see bootstrap.cpp).
#pragma once
#include <stdint.h>

#include <memory>
#include <vector>

#include "engine.hpp"

namespace fhe {

// one BSGS level of CoeffToSlot or SlotToCoeff: applied at l limbs, then rescaled
struct BootLevel {
    uint32_t l = 0, nb = 0, ng = 0;
    uint32_t n_in = 1, n_out = 1;  // the last CoeffToSlot level: inputs (y, conj y), outputs (2 Re, 2 Im)
    std::vector<int64_t> bsteps, gsteps;
    // [n_out][ng][n_in nb][l + K][N] over the primes of Q_l * P (the levels run double-hoisted), term (g, b)
    // pre-rotated by -gsteps[g]
    uint64_t* d_diags = nullptr;
};

struct BootPlan {
    double K = 0;
    int deg = 0, r = 0;
    double in_scale = 0;
    std::vector<long double> S;  // S[l]: scale of a ciphertext with l limbs
    std::vector<double> cheb;
    std::vector<BootLevel> cts, stc;
    std::vector<int64_t> steps;  // rotation steps whose keys evaluation needs (plus the conjugation key)
    uint32_t l_out = 0;
    // sparse-secret encapsulation (not owned): keys s -> s' (sparse, on q0 and P) and s' -> s
    const uint64_t* sse_to = nullptr;
    const uint64_t* sse_from = nullptr;
    // the CoeffToSlot / SlotToCoeff diagonals are shared by the plans made from one (bootstrap_plan_shared): the
    // last holder frees them
    std::shared_ptr<void> diags_owner;
    // integer factor applied to EvalMod's output in the recombination before SlotToCoeff: a plan made for a
    // smaller input scale reuses another's SlotToCoeff diagonals (whose constant is q0 / (2 pi in_scale))
    uint64_t stc_factor = 1;
};

BootPlan* bootstrap_plan(Context& ctx, double K, int deg, int r, double top_scale, double in_scale);
// a plan for input scale in_scale sharing every diagonal of base: base.in_scale / in_scale must be an integer
BootPlan* bootstrap_plan_shared(const BootPlan& base, double in_scale);
void bootstrap_plan_destroy(BootPlan* P);
uint32_t bootstrap(Context& ctx, const BootPlan& P, const uint64_t* ct_in, uint32_t B, const uint64_t* relin,
                   const uint64_t* conj_evk, const int64_t* steps, const uint64_t* const* evks, uint32_t n_keys,
                   uint64_t* out, hipStream_t st, uint32_t stop_stage = 0);

}  // namespace fhe
