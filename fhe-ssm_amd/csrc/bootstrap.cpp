// bootstrap.cpp -- full-slot CKKS bootstrapping (EvalBootstrap, gpu_real_model.cu:2544; setup
// EvalBootstrapSetup(levelBudget, {0,0}, slots), :1335,1444) composed from the engine's kernels.
//
//   ModRaise   the q0 limb of the input, read CENTERED (v > q0>>1 => v - q0, harness/boot_overflow_probe.cpp:5-13),
//              re-embedded in every limb of Q: the message becomes m + q0*I (I a small integer polynomial)
//   CoeffToSlot  3 BSGS levels of the inverse special FFT (15 radix-2 layers grouped 5 per level), scaled
//              so the slots hold t = (I + m/q0)/K in bit-reversed order; the factor 1/2 prepares the split
//   split      conj by X -> X^(2N-1): Re = ct + conj(ct), Im = -i (ct - conj(ct)) -- two real-slot ciphertexts
//   EvalMod    Chebyshev interpolant (degree deg) of cos(2 pi (K t - 1/4) / 2^r) on [-1, 1], evaluated by
//              Chebyshev division over T_8, T_16, T_32 with baby steps T_1..T_8, then r double-angle steps
//              c <- 2c^2 - 1, giving sin(2 pi K t) = sin(2 pi m/q0)
//   recombine  Re + i Im
//   SlotToCoeff 3 BSGS levels of the forward special FFT scaled by q0 / (2 pi Delta_in)
//
// Scales follow the FLEXIBLE rule: a ciphertext with l limbs has scale S(l), S(L) = Delta_top,
// S(l-1) = S(l)^2 / q_{l-1}; a plaintext or scalar applied at level l is encoded at S(l), so every product
// followed by a rescale lands exactly on S(l-1).  Level alignment of a term is one scalar multiplication.
#include <hip/hip_runtime.h>

#include <cmath>
#include <complex>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "bootstrap.hpp"
#include "client.hpp"
#include "engine.hpp"
#include "ops.hpp"

namespace fhe {

uint64_t mulmod_h(uint64_t a, uint64_t b, uint64_t q);
hipError_t launch_ntt(const Context& ctx, uint64_t* data, const JobSpec& js, uint32_t n_jobs, bool inverse,
                      NttMode mode, hipStream_t st);
hipError_t launch_lift_centered(const Context& ctx, const uint64_t* last, uint64_t last_pstride, uint64_t* tmp,
                                uint32_t n_polys, uint32_t n_out, uint64_t ql, hipStream_t st);
hipError_t launch_lincomb(const Context& ctx, uint64_t* out, uint32_t B, uint32_t l_out, uint32_t n_terms,
                          const uint64_t* const* x, const uint32_t* stride, const uint64_t* C, const uint64_t* add,
                          hipStream_t st, uint32_t i0 = 0);
hipError_t launch_mul_i(const Context& ctx, const uint64_t* in, uint64_t* out, uint32_t n_polys, uint32_t l, int sign,
                        hipStream_t st);

namespace {

#define HIPB(expr)                                                                      \
    do {                                                                                \
        hipError_t _e = (expr);                                                         \
        if (_e != hipSuccess)                                                           \
            throw std::runtime_error(std::string(#expr) + ": " + hipGetErrorString(_e)); \
    } while (0)

using cd = std::complex<double>;
constexpr uint32_t kSlots = kN / 2;
constexpr size_t W = kN;

// ------------------------------------------------------------------ special FFT layers
// Forward layer s (len = 2^s) on a bit-reversed slot vector, as {rotation offset: diagonal}:
// p in the first half of its block:  out[p] = x[p] + w x[p + len/2]
// p in the second half:              out[p] = x[p - len/2] - w x[p]
// w = exp(2 pi i ((5^j mod 4 len) (2N / 4 len)) / 2N), j = p mod len/2.  The inverse layer undoes it.
using Diags = std::map<long, std::vector<cd>>;

std::vector<uint64_t> rot_group() {
    std::vector<uint64_t> g(kSlots);
    uint64_t e = 1;
    for (uint32_t j = 0; j < kSlots; j++) {
        g[j] = e;
        e = e * 5 % (2ull * kN);
    }
    return g;
}

Diags fft_layer(uint32_t s, bool inverse, const std::vector<uint64_t>& rg) {
    const uint32_t len = 1u << s, h = len / 2;
    const uint64_t lenq = 4ull * len, M = 2ull * kN;
    std::vector<cd> a(kSlots), b(kSlots), c(kSlots);
    for (uint32_t p = 0; p < kSlots; p++) {
        const uint32_t j = p % len;
        const uint32_t jj = j < h ? j : j - h;
        const double ang = 2.0 * M_PI * (double)((rg[jj] % lenq) * (M / lenq)) / (double)M;
        const cd w(std::cos(ang), std::sin(ang));
        if (j < h) {
            a[p] = inverse ? 0.5 : 1.0;
            b[p] = inverse ? cd(0.5) : w;
        } else {
            a[p] = inverse ? -0.5 / w : -w;
            c[p] = inverse ? 0.5 / w : cd(1.0);
        }
    }
    Diags d;
    d[0] = std::move(a);
    d[(long)h] = std::move(b);
    d[-(long)h] = std::move(c);
    return d;
}

// (L o R): R applied first; rot_a(diag(v) rot_b x) = diag(v shifted by a) rot_{a+b} x
Diags compose(const Diags& Lf, const Diags& Rf) {
    Diags out;
    for (auto& [a, da] : Lf)
        for (auto& [b, db] : Rf) {
            auto& o = out[a + b];
            if (o.empty()) o.assign(kSlots, 0.0);
            for (uint32_t p = 0; p < kSlots; p++) {
                const uint32_t src = (uint32_t)(((long)p + a) % (long)kSlots + kSlots) % kSlots;
                o[p] += da[p] * db[src];
            }
        }
    return out;
}

// Chebyshev interpolant of f on [-1, 1]: c_j = 2/n sum_k f(x_k) cos(pi j (k + 1/2)/n), c_0 halved
std::vector<double> chebyshev_coeffs(int deg, double K, int r) {
    const int n = deg + 1;
    std::vector<double> fk(n), c(n);
    for (int k = 0; k < n; k++) {
        const double x = std::cos(M_PI * (k + 0.5) / n);
        fk[k] = std::cos(2.0 * M_PI * (K * x - 0.25) / std::ldexp(1.0, r));
    }
    for (int j = 0; j < n; j++) {
        double s = 0;
        for (int k = 0; k < n; k++) s += fk[k] * std::cos(M_PI * j * (k + 0.5) / n);
        c[j] = 2.0 / n * s;
    }
    c[0] *= 0.5;
    return c;
}

// signed integer (as long double, |v| < 2^120) reduced mod q
uint64_t mod_signed(long double v, uint64_t q) {
    const bool neg = v < 0;
    long double a = neg ? -v : v;
    const unsigned __int128 x = (unsigned __int128)a;
    const uint64_t r = (uint64_t)(x % q);
    return neg ? (r ? q - r : 0) : r;
}

}  // namespace

// ------------------------------------------------------------------ plan
// the device diagonals of a plan's levels, freed with the last plan that shares them
struct DiagStore {
    std::vector<uint64_t*> d;
    ~DiagStore() {
        for (auto* p : d) (void)hipFree(p);
    }
};

BootPlan* bootstrap_plan(Context& ctx, double K, int deg, int r, double top_scale, double in_scale) {
    if (ctx.K == 0) throw std::invalid_argument("bootstrapping needs special primes");
    if (deg < 8 || deg > 63) throw std::invalid_argument("Chebyshev degree must be in [8, 63]");
    const uint32_t L = ctx.L;
    // levels: CtS 3 + Chebyshev 7 + double angle r + StC 3, plus one limb left
    const uint32_t need = 3 + 7 + (uint32_t)r + 3 + 1;
    if (L < need + 1) throw std::invalid_argument("chain too short for bootstrapping: need " + std::to_string(need + 1));
    auto* P = new BootPlan();
    P->K = K;
    P->deg = deg;
    P->r = r;
    P->in_scale = in_scale;
    // CoeffToSlot runs at top_scale on limbs L, L-1, L-2 (these primes should be the largest of the chain:
    // the raised message is ~q0 K, and the absolute rounding and key-switching noise of these levels,
    // amplified by 2 pi K in EvalMod, is what limits the precision, so top_scale should be well above the
    // chain's scale).  Level l's diagonals are encoded at q_{l-1} S(l-1) / S(l): the first two keep the
    // scale, the last lands on the context's scale at L-3.  From L-3 on the FLEXIBLE rule
    // S(l-1) = S(l)^2 / q_{l-1} applies (the chain's scaling primes are chosen for it).  in_scale, the
    // input's scale, is independent of it: EvalMod's signal is sin(2 pi m / q0), so in_scale close to q0
    // (as OpenFHE's q0 ~ 2 Delta) keeps the signal well above EvalMod's noise.
    P->S.assign(L + 1, 0.0L);
    for (uint32_t l = L; l >= L - 2; l--) P->S[l] = top_scale;
    P->S[L - 3] = ctx.scale;
    for (uint32_t l = L - 3; l >= 2; l--) P->S[l - 1] = P->S[l] * P->S[l] / (long double)ctx.moduli[l - 1];
    P->cheb = chebyshev_coeffs(deg, K, r);
    const auto rg = rot_group();
    const double q0 = (double)ctx.moduli[0];
    // groups of 5 layers: CtS applies layers 15..11, 10..6, 5..1 (inverse); StC 1..5, 6..10, 11..15
    auto build_group = [&](int s_lo, int s_hi, bool inverse, double scale_c) {
        Diags D;
        D[0] = std::vector<cd>(kSlots, cd(scale_c));
        if (inverse)
            for (int s = s_hi; s >= s_lo; s--) D = compose(fft_layer(s, true, rg), D);
        else
            for (int s = s_lo; s <= s_hi; s++) D = compose(fft_layer(s, false, rg), D);
        return D;
    };
    // split: the level also separates real and imaginary parts.  With y its input, x = T(y) its output and
    // conj commuting with rotations, 2 Re x = x + conj x = sum_g Rot_G(sum_b d (.) Rot_b(y) + conj(d) (.)
    // Rot_b(conj y)) and 2 Im x = -i (x - conj x): one two-input, two-output BSGS over (y, conj y), whose
    // conjugation key switch runs at this level's (high) scale instead of at the EvalMod scale.
    auto add_level = [&](std::vector<BootLevel>& dst, const Diags& D, int s_lo, uint32_t l, double pt_scale,
                         bool split) {
        const long delta = 1L << (s_lo - 1);
        // The level's diagonals sit at offsets k delta, |k| <= 31.  When the slot count n is at most 63 delta,
        // offsets k and k - n / delta are the same rotation: those diagonals are summed, leaving n / delta of them
        // at k in [0, n / delta).  Otherwise k is taken in [-32, 32).  Babies are b delta (b < nb, b = 0 the
        // identity), giants (lo + g nb) delta, one of them 0.
        const long n_rot = (long)kSlots / delta;
        const bool wrap = n_rot <= 63;
        const long lo = wrap ? 0 : -32, span = wrap ? n_rot : 64;
        BootLevel bl;
        bl.l = l;
        bl.nb = (uint32_t)std::min<long>(16, span);
        bl.ng = (uint32_t)(span / bl.nb);
        bl.n_in = bl.n_out = split ? 2 : 1;
        for (uint32_t b = 0; b < bl.nb; b++) bl.bsteps.push_back((int64_t)b * delta);
        for (uint32_t g = 0; g < bl.ng; g++) bl.gsteps.push_back((lo + (int64_t)g * bl.nb) * delta);
        // the levels run double-hoisted: their diagonals are encoded over Q_l * P
        std::vector<uint32_t> pmap;
        for (uint32_t i = 0; i < l; i++) pmap.push_back(i);
        for (uint32_t k = 0; k < ctx.K; k++) pmap.push_back(ctx.L + k);
        const size_t E = pmap.size();
        const size_t n_terms = (size_t)bl.n_out * bl.ng * bl.n_in * bl.nb;
        HIPB(hipMalloc(&bl.d_diags, n_terms * E * W * 8));
        HIPB(hipMemset(bl.d_diags, 0, n_terms * E * W * 8));
        std::vector<double> re(kSlots), im(kSlots);
        auto put = [&](uint32_t o, uint32_t g, uint32_t j, const std::vector<cd>& v) {
            for (uint32_t s = 0; s < kSlots; s++) {
                re[s] = v[s].real();
                im[s] = v[s].imag();
            }
            const size_t t = ((size_t)o * bl.ng + g) * bl.n_in * bl.nb + j;
            encode_primes(ctx, re.data(), im.data(), kSlots, pmap, pt_scale, bl.d_diags + t * E * W);
        };
        std::map<long, std::vector<cd>> folded;  // k - lo -> diagonal
        for (auto& [off, d] : D) {
            if (off % delta) throw std::logic_error("unexpected diagonal offset");
            long k = off / delta;
            if (k < -31 || k > 31) throw std::logic_error("diagonal offset out of range");
            if (wrap) k = ((k % n_rot) + n_rot) % n_rot;
            auto& f = folded[k - lo];
            if (f.empty()) f.assign(kSlots, cd(0.0));
            for (uint32_t s = 0; s < kSlots; s++) f[s] += d[s];
        }
        // a diagonal that holds only the float residue of exact cancellations (below 1e-12 of the level's largest
        // entry) is zero: encoding it would refuse it (every coefficient below 1/2) or waste a baby-giant term
        double dmax = 0.0;
        for (auto& kv : folded)
            for (auto& v : kv.second) dmax = std::max(dmax, std::abs(v));
        std::vector<cd> dr(kSlots), tmp(kSlots);
        for (auto& [kp, d] : folded) {
            bool nz = false;
            for (auto& v : d) nz |= std::abs(v) > 1e-12 * dmax;
            if (!nz) continue;
            const uint32_t g = (uint32_t)(kp / bl.nb), b = (uint32_t)(kp % bl.nb);
            const long G = bl.gsteps[g];
            // term (g, b) is pre-rotated by -G: d'[s] = d[(s - G) mod n]
            for (uint32_t s = 0; s < kSlots; s++)
                dr[s] = d[(uint32_t)((((long)s - G) % (long)kSlots + kSlots) % kSlots)];
            if (!split) {
                put(0, g, b, dr);
                continue;
            }
            const cd I(0.0, 1.0);
            for (uint32_t s = 0; s < kSlots; s++) tmp[s] = std::conj(dr[s]);
            put(0, g, b, dr);
            put(0, g, bl.nb + b, tmp);
            for (uint32_t s = 0; s < kSlots; s++) tmp[s] = -I * dr[s];
            put(1, g, b, tmp);
            for (uint32_t s = 0; s < kSlots; s++) tmp[s] = I * std::conj(dr[s]);
            put(1, g, bl.nb + b, tmp);
        }
        dst.push_back(std::move(bl));
    };
    try {
        const double c_cts = (double)(P->S[L] / (q0 * K)) * 0.5;
        const auto qd = [&](uint32_t l) { return (double)((long double)ctx.moduli[l - 1] * P->S[l - 1] / P->S[l]); };
        add_level(P->cts, build_group(11, 15, true, c_cts), 11, L, qd(L), false);
        add_level(P->cts, build_group(6, 10, true, 1.0), 6, L - 1, qd(L - 1), false);
        add_level(P->cts, build_group(1, 5, true, 1.0), 1, L - 2, qd(L - 2), true);
        const uint32_t l_stc = L - 3 - 7 - (uint32_t)r;
        const double c_stc = q0 / (2.0 * M_PI * in_scale);
        add_level(P->stc, build_group(1, 5, false, c_stc), 1, l_stc, (double)P->S[l_stc], false);
        add_level(P->stc, build_group(6, 10, false, 1.0), 6, l_stc - 1, (double)P->S[l_stc - 1], false);
        add_level(P->stc, build_group(11, 15, false, 1.0), 11, l_stc - 2, (double)P->S[l_stc - 2], false);
        P->l_out = l_stc - 3;
    } catch (...) {
        bootstrap_plan_destroy(P);
        throw;
    }
    // the diagonals' owner: frees them when the last plan sharing them goes
    auto store = std::make_shared<DiagStore>();
    for (auto* lv : {&P->cts, &P->stc})
        for (auto& bl : *lv) store->d.push_back(bl.d_diags);
    P->diags_owner = store;
    std::map<int64_t, int> seen;
    for (auto* lv : {&P->cts, &P->stc})
        for (auto& bl : *lv) {
            for (auto s : bl.bsteps)
                if (s) seen[s] = 1;
            for (auto s : bl.gsteps)
                if (s) seen[s] = 1;
        }
    for (auto& kv : seen) P->steps.push_back(kv.first);
    return P;
}

BootPlan* bootstrap_plan_shared(const BootPlan& base, double in_scale) {
    const double f = base.in_scale / in_scale;
    if (!(f >= 1.0) || f > 1e15 || f != std::floor(f))
        throw std::invalid_argument("a shared plan's input scale must divide the base plan's by an integer");
    auto* P = new BootPlan(base);  // the level descriptors, scales and coefficients; the diagonals are shared
    P->in_scale = in_scale;
    P->stc_factor = base.stc_factor * (uint64_t)f;
    return P;
}

void bootstrap_plan_destroy(BootPlan* P) {
    if (!P) return;
    if (!P->diags_owner)  // a plan whose construction failed before its diagonals were handed to an owner
        for (auto* lv : {&P->cts, &P->stc})
            for (auto& bl : *lv) (void)hipFree(bl.d_diags);
    delete P;
}

// ------------------------------------------------------------------ evaluation
namespace {

// a batch of B ciphertexts [B][2][l][N] in a buffer sized for the top level
struct HCt {
    uint64_t* d = nullptr;
    uint32_t l = 0;
};

class Eval {
public:
    Eval(Context& ctx, const BootPlan& P, uint32_t B, const uint64_t* relin, hipStream_t st)
        : ctx_(ctx), P_(P), B_(B), relin_(relin), st_(st) {}
    ~Eval() {  // every buffer goes back to the context's pool for the next call
        auto& pool = ctx_.buf_pool[bytes()];
        for (auto* p : all_) pool.push_back(p);
    }

    size_t bytes() const { return (size_t)B_ * 2 * ctx_.L * W * 8; }

    HCt get(uint32_t l) {
        uint64_t* p;
        if (!free_.empty()) {
            p = free_.back();
            free_.pop_back();
        } else {
            auto& pool = ctx_.buf_pool[bytes()];
            if (!pool.empty()) {
                p = pool.back();
                pool.pop_back();
            } else {
                HIPB(hipMalloc(&p, bytes()));
            }
            all_.push_back(p);
        }
        return HCt{p, l};
    }
    void put(HCt& c) {
        if (c.d) free_.push_back(c.d);
        c.d = nullptr;
    }

    // integer combination sum_t k_t x_t (all at level l, small integer k_t), no rescale
    HCt int_comb(const std::vector<std::pair<HCt, long>>& terms, double add_const = 0.0) {
        const uint32_t l = terms[0].first.l;
        std::vector<const uint64_t*> x;
        std::vector<uint32_t> stride;
        std::vector<uint64_t> C;
        for (auto& t : terms) {
            if (t.first.l != l) throw std::logic_error("int_comb: level mismatch");
            x.push_back(t.first.d);
            stride.push_back(t.first.l);
        }
        C.resize(terms.size() * l);
        for (size_t t = 0; t < terms.size(); t++)
            for (uint32_t i = 0; i < l; i++) C[t * l + i] = mod_signed((long double)terms[t].second, ctx_.moduli[i]);
        std::vector<uint64_t> add(l);
        const long double a = std::roundl((long double)add_const * P_.S[l]);
        for (uint32_t i = 0; i < l; i++) add[i] = mod_signed(a, ctx_.moduli[i]);
        HCt out = get(l);
        HIPB(launch_lincomb(ctx_, out.d, B_, l, (uint32_t)x.size(), x.data(), stride.data(), C.data(),
                            add_const != 0.0 ? add.data() : nullptr, st_));
        return out;
    }

    // real-coefficient combination sum_t c_t x_t + a, landing at level lt = min level - 1 (one rescale)
    HCt scal_comb(const std::vector<std::pair<HCt, double>>& terms, double add_const, uint32_t lt) {
        std::vector<const uint64_t*> x;
        std::vector<uint32_t> stride;
        for (auto& t : terms) {
            if (t.first.l < lt + 1) throw std::logic_error("scal_comb: term below target");
            x.push_back(t.first.d);
            stride.push_back(t.first.l);
        }
        const uint32_t lo = lt + 1;  // limbs before the rescale
        const long double qlt = (long double)ctx_.moduli[lt];
        std::vector<uint64_t> C(terms.size() * lo), add(lo);
        for (size_t t = 0; t < terms.size(); t++) {
            const long double c =
                std::roundl((long double)terms[t].second * P_.S[lt] * qlt / P_.S[terms[t].first.l]);
            for (uint32_t i = 0; i < lo; i++) C[t * lo + i] = mod_signed(c, ctx_.moduli[i]);
        }
        // round(a S(lt)) * q_lt, reduced exactly per limb
        const long double a = std::roundl((long double)add_const * P_.S[lt]);
        for (uint32_t i = 0; i < lo; i++) {
            const uint64_t qi = ctx_.moduli[i];
            add[i] = mulmod_h(mod_signed(a, qi), ctx_.moduli[lt] % qi, qi);
        }
        HCt out = get(lt);
        rescale_lincomb(ctx_, B_, lo, (uint32_t)x.size(), x.data(), stride.data(), C.data(),
                        add_const != 0.0 ? add.data() : nullptr, out.d, st_);
        return out;
    }

    HCt adjust(const HCt& a, uint32_t lt) {
        if (a.l == lt) return copy(a);
        return scal_comb({{a, 1.0}}, 0.0, lt);
    }

    HCt copy(const HCt& a) {
        HCt o = get(a.l);
        HIPB(hipMemcpyAsync(o.d, a.d, (size_t)B_ * 2 * a.l * W * 8, hipMemcpyDeviceToDevice, st_));
        return o;
    }

    // factor * a b + add_const (the constant at the product's scale), relinearized and rescaled, a and b at one level:
    // the affine map is applied by the product's ModDown combine (the words of mult followed by int_comb)
    HCt mult_affine(const HCt& a, const HCt& b, long factor, double add_const) {
        if (a.l != b.l) throw std::logic_error("mult_affine: level mismatch");
        const long double post = std::roundl((long double)add_const * P_.S[a.l - 1]);
        if (!(std::fabs(post) < 0x1p62L)) {
            HCt sq = mult(a, b);
            HCt r = int_comb({{sq, factor}}, add_const);
            put(sq);
            return r;
        }
        const Affine aff{factor, (int64_t)post};
        HCt out = get(a.l - 1);
        hmult(ctx_, a.d, b.d, B_, a.l, relin_, out.d, true, st_, &aff);
        return out;
    }

    // product of two batches (levels aligned first), relinearized and rescaled
    HCt mult(const HCt& a, const HCt& b) {
        const uint32_t l = std::min(a.l, b.l);
        HCt aa = a.l == l ? HCt{a.d, l} : adjust(a, l);
        HCt bb = b.l == l ? HCt{b.d, l} : adjust(b, l);
        HCt out = get(l - 1);
        hmult(ctx_, aa.d, bb.d, B_, l, relin_, out.d, true, st_);
        if (aa.d != a.d) put(aa);
        if (bb.d != b.d) put(bb);
        return out;
    }

    // Chebyshev series sum_j c_j T_j(x) for x at level l0
    HCt chebyshev(const HCt& x, const std::vector<double>& c) {
        std::map<int, HCt> T;
        // T_j brought down to level l, made once and kept while the T_j live (the same T_j is needed at the same
        // lower level more than once: the words are those of a fresh adjust)
        std::map<std::pair<int, uint32_t>, HCt> Tat;
        auto at = [&](int j, uint32_t l) -> HCt {
            if (T[j].l == l) return T[j];
            auto it = Tat.find({j, l});
            if (it == Tat.end()) it = Tat.emplace(std::make_pair(j, l), adjust(T[j], l)).first;
            return it->second;
        };
        T[1] = copy(x);
        auto t2 = [&](int j) { return mult_affine(T[j], T[j], 2, -1.0); };  // T_{2j} = 2 T_j^2 - 1
        auto tsum = [&](int a, int b) {  // T_{a+b} = 2 T_a T_b - T_{a-b}, a > b
            const uint32_t l = std::min(T[a].l, T[b].l);
            HCt pr = mult(at(a, l), at(b, l));
            HCt r = int_comb({{pr, 2}, {at(a - b, pr.l), -1}});
            put(pr);
            return r;
        };
        T[2] = t2(1);
        T[3] = tsum(2, 1);
        T[4] = t2(2);
        T[5] = tsum(3, 2);
        T[6] = t2(3);
        T[7] = tsum(4, 3);
        T[8] = t2(4);
        int deg = (int)c.size() - 1;
        while (deg > 0 && c[deg] == 0.0) deg--;
        for (int n = 16; n <= deg; n *= 2) T[n] = t2(n / 2);  // the giant steps the division below uses
        for (auto& kv : Tat) put(kv.second);  // the products above are done with their level copies
        Tat.clear();
        // want: the level the caller consumes the result at (a leaf lands there directly when that is below its own
        // level, instead of being adjusted down by a second rescale afterwards)
        std::function<HCt(const std::vector<double>&, uint32_t)> rec = [&](const std::vector<double>& a,
                                                                            uint32_t want) -> HCt {
            int degp = (int)a.size() - 1;
            while (degp > 0 && a[degp] == 0.0) degp--;
            if (degp < 8) {
                // leaf: sum_{j<8} a_j T_j, all brought to one level by the scalar combination
                uint32_t lt = 1000;
                std::vector<std::pair<HCt, double>> terms;
                for (int j = 1; j <= degp; j++) {
                    terms.push_back({T[j], a[j]});
                    lt = std::min(lt, T[j].l - 1);
                }
                if (terms.empty()) terms.push_back({T[1], 0.0}), lt = T[1].l - 1;
                if (want >= 1) lt = std::min(lt, want);
                return scal_comb(terms, a[0], lt);
            }
            int n = 8;
            while (2 * n <= degp) n *= 2;
            // p = q T_n + r (Chebyshev division, deg p < 2n)
            std::vector<double> q(degp - n + 1, 0.0), rr(n, 0.0);
            for (int j = 0; j <= degp; j++) {
                if (j < n) rr[j] += a[j];
                else if (j == n) q[0] += a[j];
                else {
                    q[j - n] += 2 * a[j];
                    rr[2 * n - j] -= a[j];
                }
            }
            HCt hq = rec(q, T[n].l);  // multiplied by T_n at T_n's level
            const uint32_t lm = std::min(hq.l, T[n].l);
            HCt hqa = hq.l == lm ? hq : adjust(hq, lm);
            HCt prod = mult(hqa, at(n, lm));
            if (hqa.d != hq.d) put(hqa);
            put(hq);
            HCt hr = rec(rr, prod.l);  // added to the product at its level
            const uint32_t l = std::min(prod.l, hr.l);
            HCt pa = prod.l == l ? prod : adjust(prod, l);
            HCt ra = hr.l == l ? hr : adjust(hr, l);
            HCt out = int_comb({{pa, 1}, {ra, 1}});
            if (pa.d != prod.d) put(pa);
            if (ra.d != hr.d) put(ra);
            put(prod);
            put(hr);
            return out;
        };
        HCt res = rec(c, 0);  // the series at its own level
        for (auto& kv : Tat) put(kv.second);
        for (auto& kv : T) put(kv.second);
        return res;
    }

private:
    Context& ctx_;
    const BootPlan& P_;
    uint32_t B_;
    const uint64_t* relin_;
    hipStream_t st_;
    std::vector<uint64_t*> free_, all_;
};

}  // namespace

// ct_in: [2][1][N] (the q0 limb), message scale P.in_scale.  out: [2][P.l_out][N], scale S(l_out).
// B independent ciphertexts in one pass: every kernel runs over the whole batch and reads each key and
// plaintext diagonal once per pass.  ct_in: [B][2][1][N]; out: [B][2][l_out][N].
// stop_stage (testing): 1 after ModRaise, 2 after CoeffToSlot (Re + i Im), 3 after the split ([Re][B], [Im][B]),
// 4 after EvalMod (same layout), 5 after the recombination, 0 or 6 the full bootstrap.  Returns the level.
uint32_t bootstrap(Context& ctx, const BootPlan& P, const uint64_t* ct_in, uint32_t B, const uint64_t* relin,
                   const uint64_t* conj_evk, const int64_t* steps, const uint64_t* const* evks, uint32_t n_keys,
                   uint64_t* out, hipStream_t st, uint32_t stop_stage) {
    if (B == 0) return P.l_out;
    // the stages' phase labels (profiling), the caller's label put back on every way out
    struct PhaseGuard {
        Context& c;
        hipStream_t s;
        std::string old;
        ~PhaseGuard() { (void)set_phase(c, old, s); }
    } phase_guard{ctx, st, ctx.prof_phase};
    (void)set_phase(ctx, "boot_modraise", st);
    // stream-ordered like every call on a context: the pooled buffers go back for reuse by later work on st
    auto emit = [&](const uint64_t* src, uint32_t n, uint32_t l) {
        HIPB(hipMemcpyAsync(out, src, (size_t)n * 2 * l * W * 8, hipMemcpyDeviceToDevice, st));
        return l;
    };
    const uint32_t L = ctx.L;
    std::map<int64_t, const uint64_t*> key;
    for (uint32_t i = 0; i < n_keys; i++) key[steps[i]] = evks[i];
    for (auto s : P.steps)
        if (!key.count(s)) throw std::invalid_argument("missing rotation key for step " + std::to_string(s));
    Eval ev1(ctx, P, B, relin, st), ev2(ctx, P, 2 * B, relin, st);
    // ---- ModRaise: centered q0 limb -> all L limbs
    HCt raised = ev1.get(L);
    {
        uint64_t* last = raised.d;  // staging: the two q0 limbs, then lifted in place of the output
        HCt stage = ev1.get(1);
        if (P.sse_to) {
            // sparse-secret encapsulation: switch the q0 ciphertexts to the sparse secret, so that the raised
            // message m + q0 I has a small I (K bounds it), then switch back at the top level below
            keyswitch(ctx, ct_in + W, B, 1, P.sse_to, ct_in, stage.d, st, 2, 2 * W);  // c1 read in place
        } else {
            HIPB(hipMemcpyAsync(stage.d, ct_in, (size_t)B * 2 * W * 8, hipMemcpyDeviceToDevice, st));
        }
        JobSpec js{};
        js.n_polys = 2 * B;
        js.period = 1;
        js.pmap[0] = 0;
        HIPB(launch_ntt(ctx, stage.d, js, 2 * B, true, ctx.ntt_mode, st));
        HIPB(launch_lift_centered(ctx, stage.d, W, last, 2 * B, L, ctx.moduli[0], st));
        JobSpec jl{};
        jl.n_polys = 2 * B;
        jl.period = L;
        for (uint32_t i = 0; i < L; i++) jl.pmap[i] = (uint8_t)i;
        HIPB(launch_ntt(ctx, raised.d, jl, 2 * B * L, false, ctx.ntt_mode, st));
        ev1.put(stage);
        if (P.sse_from) {
            HCt back = ev1.get(L);
            keyswitch(ctx, raised.d + (size_t)L * W, B, L, P.sse_from, raised.d, back.d, st, 2, (uint64_t)2 * L * W);
            ev1.put(raised);
            raised = back;
        }
    }
    if (stop_stage == 1) return emit(raised.d, B, L);
    (void)set_phase(ctx, "boot_coeff_to_slot", st);
    // ---- CoeffToSlot: one BSGS level per call over the batch (diagonals and keys shared), then rescale
    auto keys_of = [&](const BootLevel& bl, std::vector<const uint64_t*>& bk, std::vector<const uint64_t*>& gk) {
        for (auto s : bl.bsteps) bk.push_back(s ? key[s] : nullptr);
        for (auto s : bl.gsteps) gk.push_back(s ? key[s] : nullptr);
    };
    auto apply_level = [&](Eval& ev, const HCt& in, const BootLevel& bl) {
        if (in.l != bl.l) throw std::logic_error("linear transform level mismatch");
        std::vector<const uint64_t*> bk, gk, ins(B);
        keys_of(bl, bk, gk);
        for (uint32_t b = 0; b < B; b++) ins[b] = in.d + (size_t)b * 2 * bl.l * W;
        HCt o = ev.get(bl.l - 1);
        bsgs_dh_batch(ctx, ins.data(), B, 1, bl.l, bl.d_diags, bl.nb, bl.bsteps.data(), bk.data(), bl.ng,
                      bl.gsteps.data(), gk.data(), 1, o.d, st, false);
        return o;
    };
    HCt x = raised;
    for (size_t i = 0; i + 1 < P.cts.size(); i++) {
        HCt y = apply_level(ev1, x, P.cts[i]);
        ev1.put(x);
        x = y;
    }
    // ---- last CoeffToSlot level with the split into real parts folded in: [2 Re t][B] then [2 Im t][B] as
    // one batch of 2B (the 1/2 is in the first level's constant)
    const BootLevel& bs = P.cts.back();
    if (x.l != bs.l || bs.n_in != 2 || bs.n_out != 2) throw std::logic_error("split level mismatch");
    const uint32_t lm = bs.l - 1;
    HCt pair = ev2.get(lm);
    {
        HCt cj = ev1.get(bs.l);
        std::vector<uint32_t> g(B, 2 * kN - 1);
        std::vector<const uint64_t*> ck(B, conj_evk);
        automorph_ks_list(ctx, x.d, B, bs.l, g.data(), ck.data(), cj.d, st);
        std::vector<const uint64_t*> bk, gk, ins(2 * B);
        keys_of(bs, bk, gk);
        for (uint32_t b = 0; b < B; b++) {
            ins[2 * b] = x.d + (size_t)b * 2 * bs.l * W;
            ins[2 * b + 1] = cj.d + (size_t)b * 2 * bs.l * W;
        }
        bsgs_dh_batch(ctx, ins.data(), B, 2, bs.l, bs.d_diags, bs.nb, bs.bsteps.data(), bk.data(), bs.ng,
                      bs.gsteps.data(), gk.data(), 2, pair.d, st, true);
        ev1.put(cj);
        ev1.put(x);
    }
    // f (Re[b] + i Im[b]) over the batch (pair holds the Re block then the Im block), f a small integer
    auto recombine = [&](const HCt& re_im, uint32_t l, uint64_t f) {
        const size_t half = (size_t)B * 2 * l * W;
        HCt im = ev1.get(l), z = ev1.get(l);
        HIPB(launch_mul_i(ctx, re_im.d + half, im.d, 2 * B, l, 1, st));
        const uint64_t* xs[2] = {re_im.d, im.d};
        const uint32_t strides[2] = {l, l};
        std::vector<uint64_t> C(2 * l);
        for (uint32_t t = 0; t < 2; t++)
            for (uint32_t i = 0; i < l; i++) C[(size_t)t * l + i] = f % ctx.moduli[i];
        HIPB(launch_lincomb(ctx, z.d, B, l, 2, xs, strides, C.data(), nullptr, st));
        ev1.put(im);
        return z;
    };
    if (stop_stage == 2) {  // the CoeffToSlot output itself: Re + i Im
        HCt z = recombine(pair, lm, 1);
        return emit(z.d, B, lm);
    }
    if (stop_stage == 3) return emit(pair.d, 2 * B, pair.l);
    // ---- EvalMod on both halves of every ciphertext
    (void)set_phase(ctx, "boot_eval_mod", st);
    HCt y = ev2.chebyshev(pair, P.cheb);
    ev2.put(pair);
    for (int k = 0; k < P.r; k++) {  // double angle: 2 y^2 - 1
        HCt z = ev2.mult_affine(y, y, 2, -1.0);
        ev2.put(y);
        y = z;
    }
    if (stop_stage == 4) return emit(y.d, 2 * B, y.l);
    // ---- recombine Re + i Im at the StC input level
    (void)set_phase(ctx, "boot_slot_to_coeff", st);
    const uint32_t ls = P.stc[0].l;
    HCt ya = y.l == ls ? y : ev2.adjust(y, ls);
    if (ya.d != y.d) ev2.put(y);
    HCt z = recombine(ya, ls, P.stc_factor);  // a shared plan's SlotToCoeff constant times its integer factor
    ev2.put(ya);
    if (stop_stage == 5) return emit(z.d, B, z.l);
    // ---- SlotToCoeff
    for (auto& bl : P.stc) {
        HCt w = apply_level(ev1, z, bl);
        ev1.put(z);
        z = w;
    }
    const uint32_t lo = emit(z.d, B, z.l);
    ev1.put(z);
    return lo;
}

}  // namespace fhe
