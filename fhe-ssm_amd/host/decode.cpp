// decode.cpp -- the config-5 encrypted decode step, driven through the engine's C ABI (ckks_engine.h).
//
// The caller side of the hot path: the per-layer loop of the reference's served step
// (hpc_gpu_port/gpu_real_model.cu:4674-5300) -- per layer RMSNorm, token shift, matvecBatch with shared babies
// (:2902-3424), WKV scan, gate, output projection, residual, channel mix -- with the refresh policy of :2535-2599
// re-decided for this engine (increments and the packed state are bootstrapped, the residual stream never is).
// Host code only: every device operation is one ckks_* call; this file owns the level/scale bookkeeping, the
// plaintext store and the model's slot layout.
//
// Model (RWKV-7-0.1B shape, every nonlinearity a degree-3 polynomial), per layer and lane:
//   time mix      xn = x p_n1(mean(x^2));  u_m = g1 (1 - mu_m) xn + g1 mu_m xp_t  (m in r, k, v, w, a, g)
//                 r, k, v = W u;  w, a, g = p(W u);  kh = k eta
//                 S_h <- S_h diag(w_h) - (S_h kh_h)(kh_h a_h)^T + v_h k_h^T;  y_h = S_h r_h
//                 x <- x + W_o (y g);  xp_t <- xn
//   channel mix   xn2 = x p_n2(mean(x^2));  x <- x + W_cv p_h(W_ck (g2 (1 - mu_c) xn2 + g2 mu_c xp_c));  xp_c <- xn2
//   output        g_o x p_o(mean(x^2))
// Slots: lane-major, slot lane*1024 + channel (channels >= 768 zero); plaintexts that are the same for every
// lane are 1024-periodic and stored compressed (N/32 words per limb).  WKV state in diagonal layout, one
// ciphertext per t: D_t[lane*1024 + h*64 + i] = S_h[i][(i + t) mod 64].
#include "fhe_ssm_decode.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

namespace {

constexpr uint32_t kN = 1u << 16;
constexpr int D = 768, DPAD = 1024, HS = 64, FF = 3072, WKV_T = 64;
constexpr uint32_t LOG_REP = 5;  // 1024-periodic plaintexts: N / 2^5 words per limb
// matvec BSGS: rotation r = G + b in (-768, 768) with babies b in [0, nb) and giants G = nb g, g in [-768/nb, 768/nb);
// nb = 64 when a matvec has at least as many outputs as inputs (half the giant rotations, each a key switch per
// output), else 32
constexpr int MV_SPAN = 1536;
int mv_nb(size_t n_in, size_t n_out) { return n_out >= n_in ? 64 : 32; }
// ciphertexts per batched bootstrap: its buffer pool and workspaces grow with it (the config-5 step's 24 state
// ciphertexts in passes of 8 instead of 12: -7 GB of device memory at no measurable cost in time; of 6: -3 GB more
// for +1% of the step)
constexpr uint32_t kBootBatch = 6;

thread_local std::string g_err;

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void ck(int rc, const char* what) {
    if (rc != CKKS_OK) throw Error(rc, std::string(what) + ": " + ckks_last_error());
}

// the store file's calls report through this library's own message
void ck_store(int rc, const char* what) {
    if (rc != CKKS_OK) throw Error(rc, std::string(what) + ": " + g_err);
}

// ------------------------------------------------------------------ device buffers
// Free lists of device buffers by size: a decode step allocates the same shapes in every layer.
class Pool {
   public:
    ~Pool() {
        for (auto& kv : free_)
            for (auto* p : kv.second) ckks_buffer_free(p);
    }
    uint64_t* get(size_t bytes) {
        auto& l = free_[bytes];
        if (!l.empty()) {
            uint64_t* p = l.back();
            l.pop_back();
            return p;
        }
        void* p = nullptr;
        ck(ckks_buffer_alloc(bytes, &p), "ckks_buffer_alloc");
        total_ += bytes;
        return (uint64_t*)p;
    }
    void put(uint64_t* p, size_t bytes) { free_[bytes].push_back(p); }
    size_t total() const { return total_; }  // every buffer allocated, in use or free

   private:
    std::map<size_t, std::vector<uint64_t*>> free_;
    size_t total_ = 0;
};

struct Buf {
    uint64_t* d;
    size_t bytes;
    Pool* pool;  // null: not pooled (plaintexts, freed directly)
    bool own;    // false: the caller's memory, never freed here
    Buf(uint64_t* d_, size_t bytes_, Pool* pool_, bool own_ = true) : d(d_), bytes(bytes_), pool(pool_), own(own_) {}
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    ~Buf() {
        if (!own) return;
        if (pool)
            pool->put(d, bytes);
        else
            ckks_buffer_free(d);
    }
};

// a batch of B ciphertexts [B][2][level][N] in a pooled buffer, or a view into another batch's buffer
struct Ct {
    std::shared_ptr<Buf> buf;
    size_t off = 0;  // words
    uint32_t B = 0, level = 0;
    double scale = 0.0;
    uint64_t* ptr(uint32_t b = 0) const { return buf->d + off + (size_t)b * 2 * level * kN; }
};

using Pair = std::tuple<const Ct*, uint32_t, const Ct*, uint32_t>;  // (a, item of a, b, item of b)

// pinned host memory, freed on scope exit
struct HostBuf {
    void* p = nullptr;
    size_t bytes = 0;
    explicit HostBuf(size_t b) : bytes(b) { ck(ckks_host_alloc(b, &p), "ckks_host_alloc"); }
    ~HostBuf() { (void)ckks_host_free(p); }
    HostBuf(const HostBuf&) = delete;
    HostBuf& operator=(const HostBuf&) = delete;
};

// A matvec's 1024-periodic diagonals, stored in pinned host memory as their small-ring integer coefficients
// (2048 int64 per diagonal and one int32 approxFactor exponent, whatever the level: ~1/level of the expanded
// plaintexts) and expanded to the level's limbs each time the matvec is applied (the reference likewise keeps its
// compressed store on the host and streams it to the device, gpu_real_model.cu:1660-1706,3085-3285).
struct Matvec {
    std::shared_ptr<HostBuf> coef;  // [n_diag][2 DPAD] int64, then [n_diag] int32
    uint32_t n_diag = 0, level = 0;
    uint32_t n_out = 0, n_in = 0, nb = 0;
};

// ------------------------------------------------------------------ the engine side (primitives + level rules)
class Engine {
   public:
    Engine(ckks_context* ctx, fhe_ssm_refresh state, fhe_ssm_refresh inc_tm, fhe_ssm_refresh inc_cm,
           const uint64_t* relin, const uint64_t* conj, const int64_t* steps, const uint64_t* const* evks,
           uint32_t n_keys)
        : ctx_(ctx), relin_(relin), conj_(conj) {
        uint32_t n = 0, nq = 0, np = 0, dnum = 0;
        ck(ckks_context_info(ctx, &n, &nq, &np, &dnum), "ckks_context_info");
        if (n != kN) throw Error(CKKS_EINVAL, "the decoder needs N = 2^16");
        moduli_.resize(nq + np);
        ck(ckks_context_moduli(ctx, moduli_.data(), nq + np), "ckks_context_moduli");
        if (!state.plan || !inc_tm.plan || !inc_cm.plan) throw Error(CKKS_EINVAL, "missing bootstrapping plan");
        top_ = ckks_bootstrap_out_level(state.plan);
        S_.assign(top_ + 1, 0.0);
        for (uint32_t l = 1; l <= top_; l++) S_[l] = ckks_bootstrap_scale(state.plan, l);
        for (uint32_t i = 0; i < n_keys; i++) keys_[steps[i]] = evks[i];
        boots_["state"] = state;
        boots_["inc_tm"] = inc_tm;
        boots_["inc_cm"] = inc_cm;
        for (auto& kv : boots_) {
            if (ckks_bootstrap_out_level(kv.second.plan) != top_)
                throw Error(CKKS_EINVAL, "every refresh plan must end at the state plan's level");
            uint32_t ns = 0;
            std::vector<int64_t> st(256);
            ck(ckks_bootstrap_steps(kv.second.plan, st.data(), (uint32_t)st.size(), &ns), "ckks_bootstrap_steps");
            st.resize(ns);
            auto& bk = boot_keys_[kv.first];
            for (auto s : st) {
                if (!keys_.count(s)) throw Error(CKKS_EINVAL, "missing rotation key for step " + std::to_string(s));
                bk.first.push_back(s);
                bk.second.push_back(keys_[s]);
            }
        }
    }

    uint32_t top_level() const { return top_; }
    ckks_context* ctx() const { return ctx_; }
    // the phase label of the engine launches that follow (profiling attribution; see ckks_profile_phase); returns
    // the previous one
    std::string set_phase(const std::string& p) {
        std::string old = phase_;
        if (p != phase_) {
            (void)ckks_profile_phase(ctx_, p.c_str(), nullptr);
            phase_ = p;
        }
        return old;
    }
    double S(uint32_t l) const { return S_.at(l); }
    const uint64_t* key(int64_t s) const {
        if (s == 0) return nullptr;
        auto it = keys_.find(s);
        if (it == keys_.end()) throw Error(CKKS_EINVAL, "missing rotation key for step " + std::to_string(s));
        return it->second;
    }

    Ct fresh(uint32_t B, uint32_t level, double scale) {
        const size_t bytes = (size_t)B * 2 * level * kN * 8;
        Ct c;
        c.buf = std::make_shared<Buf>(pool_.get(bytes), bytes, &pool_);
        c.B = B;
        c.level = level;
        c.scale = scale;
        return c;
    }
    // a ciphertext batch in the caller's memory (read or written in place, never freed)
    static Ct borrowed(const uint64_t* d, uint32_t B, uint32_t level, double scale) {
        Ct c;
        c.buf = std::make_shared<Buf>(const_cast<uint64_t*>(d), (size_t)B * 2 * level * kN * 8, nullptr, false);
        c.B = B;
        c.level = level;
        c.scale = scale;
        return c;
    }
    // dst <- a word for word (an integer combination with coefficient 1)
    void copy_to(const Ct& a, const Ct& dst) { lincomb(a.B, {&a}, {1.0}, false, a.scale, 0.0, a.level, true, dst); }
    Ct item(const Ct& a, uint32_t i) const { return slice(a, i, i + 1); }
    Ct slice(const Ct& a, uint32_t i0, uint32_t i1) const {
        Ct c = a;
        c.off = a.off + (size_t)i0 * 2 * a.level * kN;
        c.B = i1 - i0;
        return c;
    }
    Ct zeros(uint32_t B, uint32_t level) {
        Ct c = fresh(B, level, S(level));
        std::vector<uint64_t> z((size_t)B * 2 * level * kN, 0);
        ck(ckks_memcpy_h2d(c.ptr(), z.data(), z.size() * 8), "ckks_memcpy_h2d");
        return c;
    }

    // -- level rules --------------------------------------------------------------------------------
    bool canonical(const Ct& a) const { return std::fabs(a.scale / S(a.level) - 1.0) < 1e-9; }

    Ct at(const Ct& a, uint32_t lt) {  // a at level lt with the canonical scale
        if (a.level == lt && canonical(a)) return a;
        if (a.level < lt + 1)
            throw Error(CKKS_EINVAL, "cannot bring a level-" + std::to_string(a.level) + " ciphertext to level " +
                                         std::to_string(lt));
        return adjust(a, lt, 1.0, 0.0);
    }
    Ct at_neg(const Ct& a, uint32_t lt) { return adjust(a, lt, -1.0, 0.0); }
    Ct at_scale(const Ct& a, uint32_t lt, double scale) {
        Ct out = fresh(a.B, lt, scale);
        lincomb(a.B, {&a}, {1.0}, true, scale, 0.0, lt, false, out);
        return out;
    }

    Ct add(const Ct& a, const Ct& b, int sign = 1) {
        const uint32_t m = std::min(a.level, b.level);
        Ct a2 = (a.level == m && (canonical(a) || b.level == m)) ? a : at(a, m);
        Ct b2 = (b.level == m && (canonical(b) || a.level == m)) ? b : at(b, m);
        if (std::fabs(a2.scale / b2.scale - 1.0) > 1e-9) {
            // same level, different scales: both go down one level onto the canonical scale
            a2 = at(a2, m - 1);
            b2 = at(b2, m - 1);
        }
        return lin_int({&a2, &b2}, {1.0, (double)sign});
    }

    // sum_t c_t x_t + const with scalar coefficients, landing one level below the lowest term (or at lt)
    Ct lin(const std::vector<const Ct*>& terms, const std::vector<double>& coeffs, double cst, int lt = -1) {
        uint32_t lo = terms[0]->level;
        for (auto* t : terms) lo = std::min(lo, t->level);
        const uint32_t target = lt < 0 ? lo - 1 : (uint32_t)lt;
        Ct out = fresh(terms[0]->B, target, S(target));
        lincomb(terms[0]->B, terms, coeffs, true, S(target), cst, target, false, out);
        return out;
    }

    Ct lin_int(const std::vector<const Ct*>& terms, const std::vector<double>& coeffs) {
        const Ct& t0 = *terms[0];
        Ct out = fresh(t0.B, t0.level, t0.scale);
        lincomb(t0.B, terms, coeffs, false, t0.scale, 0.0, t0.level, true, out);
        return out;
    }

    Ct concat(const std::vector<Ct>& parts) {
        const uint32_t lv = parts[0].level;
        const double sc = parts[0].scale;
        uint32_t B = 0;
        for (auto& p : parts) B += p.B;
        Ct out = fresh(B, lv, sc);
        uint32_t o = 0;
        for (auto& p : parts) {
            // same level; scales equal to 1e-9 (the rule add() applies)
            if (p.level != lv || std::fabs(p.scale / sc - 1.0) > 1e-9)
                throw Error(CKKS_EINVAL, "concat of unlike ciphertexts");
            Ct dst = slice(out, o, o + p.B);
            lincomb(p.B, {&p}, {1.0}, false, sc, 0.0, lv, true, dst);
            o += p.B;
        }
        return out;
    }

    Ct mul(const Ct& a, const Ct& b) {  // a (.) b, relinearized and rescaled; a batch of 1 broadcasts
        const uint32_t B = std::max(a.B, b.B), m = std::min(a.level, b.level);
        Ct a2 = a.level > m ? at(a, m) : a;
        Ct b2 = b.level > m ? at(b, m) : b;
        std::vector<std::vector<Pair>> pairs(B);
        for (uint32_t i = 0; i < B; i++) pairs[i] = {Pair{&a2, i % a2.B, &b2, i % b2.B}};
        return mult_sum_at(pairs, m);
    }

    // pairs[b] = products summed before one relinearization and rescale; operands go to their lowest level
    Ct mult_sum(const std::vector<std::vector<Pair>>& pairs) {
        uint32_t m = UINT32_MAX;
        for (auto& item : pairs)
            for (auto& p : item) m = std::min({m, std::get<0>(p)->level, std::get<2>(p)->level});
        std::map<const Ct*, Ct> lowered;
        auto lower = [&](const Ct* c) -> const Ct* {
            auto it = lowered.find(c);
            if (it == lowered.end())
                it = lowered.emplace(c, (c->level == m && canonical(*c)) ? *c : at(*c, m)).first;
            return &it->second;
        };
        std::vector<std::vector<Pair>> p2(pairs.size());
        for (size_t b = 0; b < pairs.size(); b++)
            for (auto& p : pairs[b])
                p2[b].push_back(Pair{lower(std::get<0>(p)), std::get<1>(p), lower(std::get<2>(p)), std::get<3>(p)});
        return mult_sum_at(p2, m);
    }

    Ct poly3(const Ct& z, const std::vector<double>& c) {  // c0 + c1 z + c2 z^2 + c3 z^3 in depth 2
        const uint32_t m = z.level;
        Ct z2 = mul(z, z);
        Ct u = lin({&z}, {c[3]}, c[2], (int)m - 1);
        Ct t = mul(z2, u);
        Ct v = lin({&z}, {c[1]}, c[0], (int)m - 2);
        return add(t, v);
    }

    // -- operators ------------------------------------------------------------------------------------
    Ct rotate(const Ct& a, int64_t k) {
        Ct out = fresh(a.B, a.level, a.scale);
        ck(ckks_eval_rotate(ctx_, a.ptr(), a.B, a.level, k, key(k), out.ptr(), nullptr), "ckks_eval_rotate");
        return out;
    }

    // a + sum_k Rot_k(a) over the window's steps, hoisted (one ModUp, one ModDown)
    Ct rotate_sum(const Ct& a, const std::vector<int64_t>& steps) {
        Ct out = fresh(a.B, a.level, a.scale);
        std::vector<const uint64_t*> keys;
        for (auto k : steps) keys.push_back(key(k));
        ck(ckks_eval_rotate_sum(ctx_, a.ptr(), a.B, a.level, steps.data(), (uint32_t)steps.size(), keys.data(),
                                out.ptr(), nullptr),
           "ckks_eval_rotate_sum");
        return out;
    }

    Ct mul_pt(const Ct& a, const Buf& pt) {  // a (.) compressed periodic plaintext (encoded at S(a.level)), rescaled
        Ct tmp = fresh(a.B, a.level, a.scale);
        ck(ckks_eval_mult_plain_ex(ctx_, a.ptr(), a.B, a.level, pt.d, 1, LOG_REP, tmp.ptr(), nullptr),
           "ckks_eval_mult_plain_ex");
        Ct out = fresh(a.B, a.level - 1, a.scale * S(a.level) / (double)moduli_[a.level - 1]);
        ck(ckks_rescale(ctx_, tmp.ptr(), 2 * a.B, a.level, out.ptr(), nullptr), "ckks_rescale");
        return out;
    }

    // the 64 cyclic block rotations rot64_t(a), t = 0..63, each masked by n_sets plaintext pairs
    Ct rotate_masked(const Ct& a, const Buf& pts, uint32_t n_sets) {
        if (a.B != 1) throw Error(CKKS_EINVAL, "rotate_masked takes one ciphertext");
        std::vector<int64_t> lo(WKV_T), hi(WKV_T);
        std::vector<const uint64_t*> klo(WKV_T), khi(WKV_T);
        for (int t = 0; t < WKV_T; t++) {
            lo[t] = t;
            hi[t] = t ? t - HS : 0;
            klo[t] = key(lo[t]);
            khi[t] = key(hi[t]);
        }
        Ct out = fresh(n_sets * WKV_T, a.level - 1, a.scale * S(a.level) / (double)moduli_[a.level - 1]);
        ck(ckks_eval_rotate_masked(ctx_, a.ptr(), a.level, WKV_T, lo.data(), klo.data(), hi.data(), khi.data(),
                                   n_sets, pts.d, LOG_REP, out.ptr(), nullptr),
           "ckks_eval_rotate_masked");
        return out;
    }

    Ct matvec(const std::vector<Ct>& inputs, const Matvec& h) {
        const std::string prev = set_phase("matvec");  // (an exception leaves the label: only profiling reads it)
        Ct out = matvec_(inputs, h);
        set_phase(prev);
        return out;
    }
    Ct matvec_(const std::vector<Ct>& inputs, const Matvec& h) {
        const uint32_t lv = inputs[0].level;
        if (inputs.size() != h.n_in) throw Error(CKKS_EINVAL, "matvec input count");
        std::vector<const uint64_t*> in;
        for (auto& x : inputs) {
            if (x.level != lv || x.B != 1) throw Error(CKKS_EINVAL, "matvec inputs must be single, same level");
            in.push_back(x.ptr());
        }
        const int nb = (int)h.nb, ng = MV_SPAN / nb, g0 = -(MV_SPAN / 2) / nb;
        std::vector<int64_t> bs(nb), gs(ng);
        std::vector<const uint64_t*> kb(nb), kg(ng);
        for (int b = 0; b < nb; b++) {
            bs[b] = b;
            kb[b] = key(b);
        }
        for (int g = 0; g < ng; g++) {
            gs[g] = (int64_t)nb * (g0 + g);
            kg[g] = key(gs[g]);
        }
        if (h.level != lv) throw Error(CKKS_EINVAL, "matvec diagonals encoded for another level");
        Ct out = fresh(h.n_out, lv - 1, inputs[0].scale * S(lv) / (double)moduli_[lv - 1]);
        ck(ckks_linear_transform_multi(ctx_, in.data(), h.n_in, lv, expand(h), LOG_REP, nb, bs.data(), kb.data(), ng,
                                       gs.data(), kg.data(), h.n_out, 1, out.ptr(), nullptr),
           "ckks_linear_transform_multi");
        return out;
    }

    // A matvec's diagonals expanded to its level's limbs in one buffer shared by every matvec (grown to the
    // largest): the work is stream-ordered, so the previous matvec has read it before the next expansion writes.
    // The coefficients come from one of two device staging buffers: the matvecs of a step run in the same order
    // every step, so while one is applied the next one's coefficients are copied from the host into the other
    // buffer on the engine's side stream (the copy starts once the work already enqueued -- this expansion and
    // every earlier read of that buffer -- is done).
    void begin_step() { mv_pos_ = 0; }

    const uint64_t* expand(const Matvec& h) {
        if (mv_pos_ < mv_order_.size() && mv_order_[mv_pos_] != &h) mv_order_.resize(mv_pos_);  // another order
        if (mv_pos_ == mv_order_.size()) mv_order_.push_back(&h);
        mv_pos_++;
        // this matvec's coefficients on the device: prefetched, or copied now
        int s = stage_[0].holds == &h ? 0 : stage_[1].holds == &h ? 1 : -1;
        if (s < 0) {
            s = stage_[0].holds ? 1 : 0;
            stage_in(s, h);
        }
        ck(ckks_side_wait(ctx_, stage_[s].ticket, nullptr), "ckks_side_wait");
        const size_t bytes = (size_t)h.n_diag * h.level * (kN >> LOG_REP) * 8;
        if (!diag_ || diag_->bytes < bytes) {
            diag_.reset();
            void* p = nullptr;
            ck(ckks_buffer_alloc(bytes, &p), "ckks_buffer_alloc");
            diag_ = std::make_shared<Buf>((uint64_t*)p, bytes, nullptr);
        }
        const int64_t* c = reinterpret_cast<const int64_t*>(stage_[s].buf->d);
        const int32_t* la = reinterpret_cast<const int32_t*>(c + (size_t)h.n_diag * (kN >> LOG_REP));
        ck(ckks_expand_periodic(ctx_, c, la, h.n_diag, DPAD, h.level, diag_->d, nullptr), "ckks_expand_periodic");
        stage_[s].holds = nullptr;  // consumed: the buffer may take the matvec after next
        // the next matvec of the recorded order (the first one of the next step after the last)
        if (mv_order_.size() > 1) {
            const Matvec* nx = mv_order_[mv_pos_ < mv_order_.size() ? mv_pos_ : 0];
            if (nx != &h) stage_in(1 - s, *nx);
        }
        return diag_->d;
    }

   private:
    // copy h's coefficients into staging buffer s on the side stream
    void stage_in(int s, const Matvec& h) {
        auto& st = stage_[s];
        if (!st.buf || st.buf->bytes < h.coef->bytes) {
            if (st.buf) ck(ckks_side_sync(ctx_), "ckks_side_sync");  // no copy may still write the old buffer
            st.buf.reset();
            void* p = nullptr;
            ck(ckks_buffer_alloc(h.coef->bytes, &p), "ckks_buffer_alloc");
            st.buf = std::make_shared<Buf>((uint64_t*)p, h.coef->bytes, nullptr);
        }
        ck(ckks_side_copy(ctx_, st.buf->d, h.coef->p, h.coef->bytes, nullptr, &st.ticket), "ckks_side_copy");
        st.holds = &h;
    }

   public:

    Ct mul_i(const Ct& a, int sign) {
        Ct out = fresh(a.B, a.level, a.scale);
        ck(ckks_eval_mul_i(ctx_, a.ptr(), 2 * a.B, a.level, sign, out.ptr(), nullptr), "ckks_eval_mul_i");
        return out;
    }

    Ct conj(const Ct& a) {
        Ct out = fresh(a.B, a.level, a.scale);
        ck(ckks_eval_automorphism_ks(ctx_, a.ptr(), a.B, a.level, 2 * kN - 1, conj_, out.ptr(), nullptr),
           "ckks_eval_automorphism_ks");
        return out;
    }

    Ct bootstrap(const Ct& a, const std::string& kind) {
        const fhe_ssm_refresh& r = boots_.at(kind);
        const auto& bk = boot_keys_.at(kind);
        const std::string prev = set_phase("boot_prep");  // the bootstrap labels its own stages
        Ct lo = at_scale(a, 1, r.in_scale);
        Ct out = fresh(a.B, top_, S(top_));
        // passes of equal size (24 -> 12 + 12): one buffer shape in the bootstrap's pool
        const uint32_t n_pass = (a.B + kBootBatch - 1) / kBootBatch, per = (a.B + n_pass - 1) / n_pass;
        for (uint32_t b0 = 0; b0 < a.B; b0 += per) {
            const uint32_t nb = std::min(per, a.B - b0);
            ck(ckks_eval_bootstrap_many(ctx_, r.plan, lo.ptr(b0), nb, relin_, conj_, bk.first.data(),
                                        bk.second.data(), (uint32_t)bk.first.size(), out.ptr(b0), nullptr),
               "ckks_eval_bootstrap_many");
        }
        set_phase(prev);
        return out;
    }

    // -- plaintexts -----------------------------------------------------------------------------------
    // the coefficient form of 1024-periodic vectors at level's scale, in pinned host memory: [n][2 DPAD] int64,
    // then [n] int32
    std::shared_ptr<HostBuf> encode_coeffs(const std::vector<double>& vecs, uint32_t level, uint32_t* n_out) {
        const uint32_t n = (uint32_t)(vecs.size() / DPAD);
        const size_t per = (size_t)(kN >> LOG_REP) * 8;
        auto buf = std::make_shared<HostBuf>(n * (per + 4));
        int64_t* c = (int64_t*)buf->p;
        int32_t* la = (int32_t*)(c + (size_t)n * (kN >> LOG_REP));
        for (uint32_t s = 0; s < n; s += 4096) {  // in chunks (bounds the encoder's host staging)
            const uint32_t m = std::min<uint32_t>(4096, n - s);
            ck(ckks_encode_periodic_coeffs(ctx_, vecs.data() + (size_t)s * DPAD, nullptr, m, DPAD, S(level),
                                           c + (size_t)s * (kN >> LOG_REP), la + s),
               "ckks_encode_periodic_coeffs");
        }
        *n_out = n;
        return buf;
    }

    std::shared_ptr<Buf> encode_periodic(const std::vector<double>& vecs, uint32_t level) {
        const uint32_t n = (uint32_t)(vecs.size() / DPAD);
        const size_t per = (size_t)level * (kN >> LOG_REP) * 8;
        void* p = nullptr;
        ck(ckks_buffer_alloc(n * per, &p), "ckks_buffer_alloc");
        auto buf = std::make_shared<Buf>((uint64_t*)p, n * per, nullptr);
        // in chunks (bounds the encoder's host staging)
        for (uint32_t s = 0; s < n; s += 4096) {
            const uint32_t m = std::min<uint32_t>(4096, n - s);
            ck(ckks_encode_periodic(ctx_, vecs.data() + (size_t)s * DPAD, nullptr, m, DPAD, level, S(level),
                                    (uint64_t*)((uint8_t*)p + s * per)),
               "ckks_encode_periodic");
        }
        return buf;
    }

   private:
    void lincomb(uint32_t B, const std::vector<const Ct*>& terms, const std::vector<double>& coeffs, bool scaled,
                 double scale_out, double cst, uint32_t lt, bool integer, const Ct& out) {
        std::vector<const uint64_t*> ptrs;
        std::vector<uint32_t> levels;
        std::vector<double> scales;
        for (auto* t : terms) {
            ptrs.push_back(t->ptr());
            levels.push_back(t->level);
            scales.push_back(scaled ? t->scale : 1.0);
        }
        ck(ckks_eval_lincomb(ctx_, B, (uint32_t)terms.size(), ptrs.data(), levels.data(), coeffs.data(),
                             scales.data(), scale_out, cst, lt, integer ? 1 : 0, out.ptr(), nullptr),
           "ckks_eval_lincomb");
    }

    Ct adjust(const Ct& a, uint32_t lt, double coeff, double cst) {
        Ct out = fresh(a.B, lt, S(lt));
        lincomb(a.B, {&a}, {coeff}, true, S(lt), cst, lt, false, out);
        return out;
    }

    Ct mult_sum_at(const std::vector<std::vector<Pair>>& pairs, uint32_t level) {
        const uint32_t B = (uint32_t)pairs.size(), np = (uint32_t)pairs[0].size();
        const Ct& a0 = *std::get<0>(pairs[0][0]);
        const Ct& b0 = *std::get<2>(pairs[0][0]);
        Ct out = fresh(B, level - 1, a0.scale * b0.scale / (double)moduli_[level - 1]);
        std::vector<const uint64_t*> flat;
        for (auto& item : pairs) {
            if (item.size() != np) throw Error(CKKS_EINVAL, "every item needs the same number of products");
            for (auto& p : item) {
                flat.push_back(std::get<0>(p)->ptr(std::get<1>(p)));
                flat.push_back(std::get<2>(p)->ptr(std::get<3>(p)));
            }
        }
        ck(ckks_eval_mult_sum(ctx_, flat.data(), np, B, level, relin_, 1, out.ptr(), nullptr), "ckks_eval_mult_sum");
        return out;
    }

    ckks_context* ctx_;
    std::string phase_;
    const uint64_t *relin_, *conj_;
    std::vector<uint64_t> moduli_;
    uint32_t top_ = 0;
    std::vector<double> S_;
    std::map<int64_t, const uint64_t*> keys_;
    std::map<std::string, fhe_ssm_refresh> boots_;
    std::map<std::string, std::pair<std::vector<int64_t>, std::vector<const uint64_t*>>> boot_keys_;
    Pool pool_;
    std::shared_ptr<Buf> diag_;  // expanded matvec diagonals (see expand)
    struct Stage {
        std::shared_ptr<Buf> buf;
        const Matvec* holds = nullptr;  // whose coefficients the buffer holds (or is receiving)
        uint64_t ticket = 0;
    } stage_[2];
    std::vector<const Matvec*> mv_order_;  // the matvecs of a step, in order (recorded as they run)
    size_t mv_pos_ = 0;

   public:
    size_t pool_bytes() const { return pool_.total(); }
    size_t diag_bytes() const {
        return (diag_ ? diag_->bytes : 0) + (stage_[0].buf ? stage_[0].buf->bytes : 0) +
               (stage_[1].buf ? stage_[1].buf->bytes : 0);
    }
    std::shared_ptr<Buf> alloc(size_t bytes) { return std::make_shared<Buf>(pool_.get(bytes), bytes, &pool_); }
};

// a phase label for the launches of a scope, the enclosing label put back at its end
struct PhaseScope {
    Engine* e;
    std::string old;
    PhaseScope(Engine* eng, const char* p) : e(eng), old(eng->set_phase(p)) {}
    ~PhaseScope() { e->set_phase(old); }
    PhaseScope(const PhaseScope&) = delete;
    PhaseScope& operator=(const PhaseScope&) = delete;
};

// ------------------------------------------------------------------ slot-layout tables
// A 768 x 768 block of a matvec: element (row, col), or absent (zero).
using Block = std::function<double(int, int)>;

// [n_out][ng giants][n_in * nb][1024] (nb = mv_nb(n_in, n_out), ng = 1536 / nb): the 1024-periodic diagonal
// r = G + b of every block (giant G = nb g, baby b), pre-rotated by -G (gpu_real_model.cu:2767-2823,
// harness/cpu_real_model.cpp:270-318): d[row] = M[row][row + r] for 0 <= row + r < 768, then d'[p] = d[(p - G) mod 1024].
std::vector<double> matvec_diagonals(const std::vector<std::vector<Block>>& blocks) {
    const size_t n_out = blocks.size(), n_in = blocks[0].size();
    const int nb = mv_nb(n_in, n_out), ng = MV_SPAN / nb, g0 = -(MV_SPAN / 2) / nb;
    std::vector<double> out(n_out * ng * n_in * nb * DPAD, 0.0);
    std::vector<double> d(DPAD);
    for (size_t o = 0; o < n_out; o++)
        for (size_t i = 0; i < n_in; i++) {
            const Block& M = blocks[o][i];
            if (!M) continue;
            for (int gi = 0; gi < ng; gi++) {
                const int G = nb * (g0 + gi);
                for (int b = 0; b < nb; b++) {
                    const int r = G + b;
                    std::fill(d.begin(), d.end(), 0.0);
                    for (int row = 0; row < D; row++) {
                        const int col = row + r;
                        if (col >= 0 && col < D) d[row] = M(row, col);
                    }
                    double* dst = out.data() + (((o * ng + gi) * n_in + i) * nb + b) * DPAD;
                    for (int p = 0; p < DPAD; p++) dst[p] = d[(((p - G) % DPAD) + DPAD) % DPAD];
                }
            }
        }
    return out;
}

// [64][2][1024]: the lo / hi masks of rot64_t (rot64_t(x) = m_lo (.) Rot_t(x) + m_hi (.) Rot_{t-64}(x)), optionally
// times rot64_t(extra) (a per-channel vector folded into the same plaintext)
std::vector<double> wkv_masks(const double* extra) {
    std::vector<double> out((size_t)WKV_T * 2 * DPAD, 0.0);
    for (int t = 0; t < WKV_T; t++)
        for (int p = 0; p < DPAD; p++) {
            const int i = p % HS;
            const bool valid = p < D;
            const double lo = (valid && i + t < HS) ? 1.0 : 0.0;
            const double hi = (t && valid && i + t >= HS) ? 1.0 : 0.0;
            double f = 1.0;
            if (extra) {
                const int src = (p / HS) * HS + (i + t) % HS;
                const int s = std::min(src, DPAD - 1);
                f = valid ? (s < D ? extra[s] : 0.0) : 0.0;
            }
            out[((size_t)t * 2 + 0) * DPAD + p] = extra ? lo * f : lo;
            out[((size_t)t * 2 + 1) * DPAD + p] = extra ? hi * f : hi;
        }
    return out;
}

// channels 768..1023 of every lane are unused: piece p (channels 256p .. 256p + 255) of the fourth quarter of the
// state diagonals is carried in the gap of quarter p, shifted by kGapShift[p]
constexpr int kGapShift[3] = {768, 512, 256};

std::vector<double> channel_range_mask(int lo, int hi) {
    std::vector<double> m(DPAD, 0.0);
    for (int c = lo; c < hi; c++) m[c] = 1.0;
    return m;
}

// The lane and head sums as rotate-and-add windows (the reference's red = EvalAdd(red, rot(red, p)) loops,
// gpu_real_model.cu:3524,3540), each one hoisted rotation sum: a lane's 1,024 slots as windows of 32 (steps 1..31),
// 16 x 32 (32 .. 480) and 2 x 512; a head's 64 slots as one window of 64.  dir = -1: the same windows downwards (the
// broadcast of a masked sum).  The same windows as rwkv_model.NORM_UP / HEAD_UP, so both drivers give the same words.
std::vector<std::vector<int64_t>> norm_windows(int dir) {
    std::vector<std::vector<int64_t>> w(3);
    for (int k = 1; k < 32; k++) w[0].push_back(dir * k);
    for (int k = 32; k < 512; k += 32) w[1].push_back(dir * k);
    w[2].push_back(dir * 512);
    return w;
}

std::vector<int64_t> head_window(int dir) {
    std::vector<int64_t> w;
    for (int k = 1; k < HS; k++) w.push_back(dir * k);
    return w;
}

std::vector<int64_t> layer_rotation_steps() {
    std::vector<int64_t> s;
    for (int nb : {32, 64}) {
        for (int b = 0; b < nb; b++) s.push_back(b);
        for (int g = -(MV_SPAN / 2) / nb; g < (MV_SPAN / 2) / nb; g++) s.push_back((int64_t)nb * g);
    }
    for (int t = 1; t < WKV_T; t++) {
        s.push_back(t);       // rot64_t: Rot_t on the lanes' low part
        s.push_back(t - HS);  // and Rot_{t-64} on the wrapped part
    }
    for (const auto& w : norm_windows(1))
        for (auto k : w) s.push_back(k);
    for (const auto& w : norm_windows(-1))
        for (auto k : w) s.push_back(k);
    for (auto k : head_window(1)) s.push_back(k);
    for (auto k : head_window(-1)) s.push_back(k);
    for (int g : kGapShift) {
        s.push_back(g);
        s.push_back(-g);
    }
    std::map<int64_t, bool> u;
    for (auto x : s)
        if (x) u[x] = true;
    std::vector<int64_t> out;
    for (auto& kv : u) out.push_back(kv.first);
    return out;
}

// ------------------------------------------------------------------ weights
struct LayerW {
    std::map<std::string, std::vector<double>> v;
    const std::vector<double>& operator[](const std::string& k) const {
        auto it = v.find(k);
        if (it == v.end()) throw Error(CKKS_EINVAL, "weight " + k + " not set");
        return it->second;
    }
};

size_t weight_count(const std::string& n) {
    static const std::map<std::string, size_t> sizes = {
        {"g1", D},     {"g2", D},     {"k_k", D},    {"mu_r", D},       {"mu_k", D},       {"mu_v", D},
        {"mu_w", D},   {"mu_a", D},   {"mu_g", D},   {"mu_c", D},       {"W_r", D * D},    {"W_k", D * D},
        {"W_v", D * D}, {"W_w", D * D}, {"W_a", D * D}, {"W_g", D * D}, {"W_o", D * D},    {"W_ck", FF * D},
        {"W_cv", D * FF}, {"p_n1", 4}, {"p_n2", 4},   {"p_w", 4},        {"p_a", 4},        {"p_g", 4},
        {"p_h", 4},    {"W_vg", D * D}, {"k_a", D},   {"r_k", D},        {"ln_w", D},       {"ln_b", D},
        {"p_v", 4},    {"p_kn", 4},   {"p_gn", 4}};
    auto it = sizes.find(n);
    return it == sizes.end() ? 0 : it->second;
}

// ------------------------------------------------------------------ the step
// The carried state of one layer.  D_t (t = 0..63) is item Didx[t].second of the batch Dseg[Didx[t].first]: after a
// refresh the diagonals live in four batches (the gap-packed quarters), at first in one batch of zeros.
struct LayerState {
    std::vector<Ct> Dseg;
    std::vector<std::pair<uint32_t, uint32_t>> Didx;
    Ct xp_t, xp_c, Dn;
};


class Decoder {
   public:
    Decoder(Engine* be, uint32_t n_layers) : be_(be), layers_(n_layers) {}
    ~Decoder() {
        (void)ckks_side_sync(be_->ctx());
        for (auto& c : saved_.copies) (void)ckks_host_free(c.first);
        for (auto& kv : host_free_)
            for (void* p : kv.second) (void)ckks_host_free(p);
    }
    Decoder(const Decoder&) = delete;
    Decoder& operator=(const Decoder&) = delete;

    void set_weight(const std::string& name, int32_t layer, const double* data, size_t count) {
        size_t want = 0;
        if (layer < 0)
            want = name == "g_o" ? D : name == "p_o" ? 4 : 0;
        else
            want = weight_count(name);
        if (want == 0) throw Error(CKKS_EINVAL, "unknown weight " + name);
        if (count != want) throw Error(CKKS_EINVAL, "weight " + name + ": " + std::to_string(want) + " values");
        if (layer >= (int32_t)layers_.size()) throw Error(CKKS_EINVAL, "layer out of range");
        // plaintexts and matvec diagonals are encoded from the weights on first use and cached by name and level
        if (!pt_.empty() || !mv_.empty())
            throw Error(CKKS_EINVAL, "weights are fixed once a step has encoded them (set every weight before the "
                                     "first step)");
        auto& dst = layer < 0 ? model_.v[name] : layers_[layer].v[name];
        dst.assign(data, data + count);
    }

    // ---- the matvec coefficient store in a store file (the reference's --store-file, gpu_real_model.cu:1887-2141)
    // One entry per matvec: key (layer, op, n_out, n_in, n_diag, nb, level) with op 1 tm, 2 wo, 3 ck, 4 cv (its
    // 1024-periodic diagonals' small-ring coefficients [n_diag][2048] int64 and their [n_diag] int32 approxFactor
    // exponents, as 64-bit words).  The stamp names what the coefficients depend on -- ring, slot layout, the
    // context's moduli, the plan's scale table, every weight -- so a store made for another model or chain is refused.
    static constexpr const char* kMvOps[5] = {"", "tm", "wo", "ck", "cv"};

    std::string store_stamp() const {
        auto fnv = [](uint64_t h, uint64_t v) { return (h ^ v) * 1099511628211ULL; };
        auto dbits = [](double d) {
            uint64_t u;
            std::memcpy(&u, &d, 8);
            return u;
        };
        uint32_t n = 0, nq = 0, np = 0, dnum = 0;
        ck(ckks_context_info(be_->ctx(), &n, &nq, &np, &dnum), "ckks_context_info");
        std::vector<uint64_t> mod(2 * (nq + np));
        ck(ckks_context_moduli(be_->ctx(), mod.data(), (uint32_t)mod.size()), "ckks_context_moduli");
        uint64_t qh = 1469598103934665603ULL, sh = qh, wh = qh;
        for (uint32_t i = 0; i < nq + np; i++) qh = fnv(qh, mod[i]);
        for (uint32_t l = 1; l <= be_->top_level(); l++) sh = fnv(sh, dbits(be_->S(l)));
        auto mix_w = [&](const LayerW& w, int32_t layer) {
            for (const auto& kv : w.v) {
                wh = fnv(wh, (uint64_t)(uint32_t)layer);
                for (unsigned char ch : kv.first) wh = fnv(wh, ch);
                for (double d : kv.second) wh = fnv(wh, dbits(d));
            }
        };
        for (size_t li = 0; li < layers_.size(); li++) mix_w(layers_[li], (int32_t)li);
        mix_w(model_, -1);
        std::ostringstream st;
        st << "fhe-ssm-amd-matvec-coeffs-v1|ring=" << n << "|dpad=" << DPAD << "|logRep=" << LOG_REP
           << "|layers=" << layers_.size() << "|nq=" << nq << "|qhash=" << qh << "|scaleHash=" << sh
           << "|weightHash=" << wh;
        return st.str();
    }

    uint64_t store_save(const char* path) {
        fhe_ssm_store* st = nullptr;
        ck_store(fhe_ssm_store_create(&st), "fhe_ssm_store_create");
        std::unique_ptr<fhe_ssm_store, void (*)(fhe_ssm_store*)> hold(st, fhe_ssm_store_destroy);
        for (const auto& kv : mv_) {
            const std::string& name = kv.first.first;
            int op = 0;
            for (int o = 1; o < 5; o++)
                if (name.compare(0, 2, kMvOps[o]) == 0) op = o;
            if (op == 0) throw Error(CKKS_EINVAL, "store: unknown matvec " + name);
            const Matvec& m = kv.second;
            const int32_t key[7] = {std::stoi(name.substr(2)), op, (int32_t)m.n_out, (int32_t)m.n_in,
                                    (int32_t)m.n_diag, (int32_t)m.nb, (int32_t)m.level};
            std::vector<uint64_t> w((m.coef->bytes + 7) / 8, 0);
            std::memcpy(w.data(), m.coef->p, m.coef->bytes);
            ck_store(fhe_ssm_store_put(st, key, w.data(), w.size()), "fhe_ssm_store_put");
        }
        ck_store(fhe_ssm_store_save(st, path, store_stamp().c_str()), "fhe_ssm_store_save");
        return mv_.size();
    }

    // the matvecs of a store file (stamp checked) in place of encoding them on first use
    uint64_t store_load(const char* path) {
        if (!mv_.empty()) throw Error(CKKS_EINVAL, "store: the matvecs are already encoded (load before the first step)");
        fhe_ssm_store* st = nullptr;
        ck_store(fhe_ssm_store_create(&st), "fhe_ssm_store_create");
        std::unique_ptr<fhe_ssm_store, void (*)(fhe_ssm_store*)> hold(st, fhe_ssm_store_destroy);
        uint64_t n = 0;
        ck_store(fhe_ssm_store_load(st, path, store_stamp().c_str(), 0, 0, &n), "fhe_ssm_store_load");
        std::map<std::pair<std::string, uint32_t>, Matvec> got;
        for (uint64_t i = 0; i < n; i++) {
            int32_t key[7];
            uint64_t len = 0;
            ck_store(fhe_ssm_store_entry(st, i, key, &len), "fhe_ssm_store_entry");
            if (key[1] < 1 || key[1] > 4 || key[0] < 0 || key[0] >= (int32_t)layers_.size() || key[4] <= 0 ||
                key[6] <= 0 || (uint32_t)key[6] > be_->top_level())
                throw Error(CKKS_EINVAL, "store: entry " + std::to_string(i) + " is not a matvec of this model");
            Matvec m;
            m.n_out = (uint32_t)key[2];
            m.n_in = (uint32_t)key[3];
            m.n_diag = (uint32_t)key[4];
            m.nb = (uint32_t)key[5];
            m.level = (uint32_t)key[6];
            const size_t bytes = (size_t)m.n_diag * ((kN >> LOG_REP) * 8 + 4);
            if (len != (bytes + 7) / 8) throw Error(CKKS_EINVAL, "store: entry " + std::to_string(i) + " length");
            m.coef = std::make_shared<HostBuf>(bytes);
            std::vector<uint64_t> w(len);
            ck_store(fhe_ssm_store_get(st, key, w.data(), len, &len), "fhe_ssm_store_get");
            std::memcpy(m.coef->p, w.data(), bytes);
            got.emplace(std::make_pair(std::string(kMvOps[key[1]]) + std::to_string(key[0]), m.level), std::move(m));
        }
        mv_ = std::move(got);
        return n;
    }

    // One step over the carried state.  The step works on a copy of the state (handles: the ciphertexts are shared,
    // never written in place) and commits it only once every layer has succeeded, so a step that throws leaves the
    // state of the previous step in place (the reference commits its carry after the whole pass,
    // gpu_real_model.cu:5284-5286).  The previous state is not kept on the device meanwhile: at the start of the
    // step it is copied to pinned host memory on the engine's side stream (the copies overlap the first layer), and
    // each layer's old state is released once its new state exists and its copy has landed; a step that throws
    // puts the saved state back.  The device holds one state instead of two.
    Ct step(const Ct& x_in) {
        const bool own = !saved_.active;  // a backup held by the caller (a multi-token request) is kept
        be_->set_phase("step");           // a step's launches start after this label's marker
        be_->set_phase("state_backup");
        if (own) backup();
        be_->begin_step();
        try {
            std::vector<LayerState> work = state_.empty() ? cold_state() : state_;
            Ct x = x_in;
            Ct v0;  // the first layer's value (the later layers' value residual mixes toward it)
            for (uint32_t li = 0; li < layers_.size(); li++) {
                LayerState& st = work[li];
                be_->set_phase("elementwise");
                Ct o = time_mix(li, x, st, v0);
                x = be_->add(x, boot(o, "inc_tm"));
                refresh_state(st);
                Ct f = channel_mix(li, x, st);
                x = be_->add(x, boot(f, "inc_cm"));
                {
                    PhaseScope ps(be_, "state_backup");
                    release_layer(li);
                }
            }
            be_->set_phase("elementwise");
            Ct xo = norm(x, model_["p_o"]);
            std::vector<double> go(DPAD, 0.0);
            std::copy(model_["g_o"].begin(), model_["g_o"].end(), go.begin());
            Ct out = be_->mul_pt(xo, *vec_pt("g_o", xo.level, [&] { return go; }));
            be_->set_phase("idle");           // what the caller enqueues next is not the step's
            state_ = std::move(work);
            if (own) drop_backup();
            reserve_backup();
            return out;
        } catch (...) {
            be_->set_phase("idle");
            if (own) {
                restore_backup();
                drop_backup();
            }
            throw;
        }
    }

    // A backup the caller holds across several steps (a multi-token request is all or nothing): taken now, kept
    // until release_held, put back by restore_held.
    void hold_backup() {
        if (saved_.active) drop_backup();
        backup();
    }
    void restore_held() {
        if (!saved_.active) return;
        restore_backup();
        drop_backup();
    }
    void release_held() {
        if (saved_.active) drop_backup();
    }

    uint64_t bootstraps() const { return n_boot_; }
    // the next step starts cold (zero WKV state and token-shift carries), as the first one does
    void reset() {
        wait_backup();
        state_.clear();
    }
    // device bytes: the plaintext store, and the carried state (each buffer counted once)
    size_t store_bytes() const {  // device: the elementwise plaintexts
        size_t b = 0;
        for (auto& kv : pt_) b += kv.second->bytes;
        return b;
    }
    size_t store_host_bytes() const {  // pinned host: the matvec coefficients
        size_t b = 0;
        for (auto& kv : mv_) b += kv.second.coef->bytes;
        return b;
    }
    size_t state_bytes() const {
        std::set<const Buf*> seen;
        size_t b = 0;
        auto add = [&](const Ct& c) {
            if (c.buf && seen.insert(c.buf.get()).second) b += c.buf->bytes;
        };
        for (auto& st : state_) {
            for (auto& c : st.Dseg) add(c);
            add(st.xp_t);
            add(st.xp_c);
            add(st.Dn);
        }
        return b;
    }
    size_t backup_host_bytes() const {
        size_t b = 0;
        for (auto& kv : host_free_) b += kv.first * kv.second.size();
        for (auto& c : saved_.copies) b += c.second;
        return b;
    }

   private:
    // plaintexts, encoded on first use at the level they are applied
    std::shared_ptr<Buf> vec_pt(const std::string& name, uint32_t level,
                                const std::function<std::vector<double>()>& vecs) {
        auto key = std::make_pair(name, level);
        auto it = pt_.find(key);
        if (it == pt_.end()) it = pt_.emplace(key, be_->encode_periodic(vecs(), level)).first;
        return it->second;
    }

    const Matvec& mv_pt(const std::string& name, uint32_t level,
                        const std::function<std::vector<std::vector<Block>>()>& blocks_fn) {
        auto key = std::make_pair(name, level);
        auto it = mv_.find(key);
        if (it == mv_.end()) {
            const auto blocks = blocks_fn();
            Matvec m;
            m.n_out = (uint32_t)blocks.size();
            m.n_in = (uint32_t)blocks[0].size();
            m.nb = (uint32_t)mv_nb(m.n_in, m.n_out);
            m.level = level;
            m.coef = be_->encode_coeffs(matvec_diagonals(blocks), level, &m.n_diag);
            it = mv_.emplace(key, std::move(m)).first;
        }
        return it->second;
    }

    Ct boot(const Ct& x, const char* kind) {
        n_boot_ += x.B;
        return be_->bootstrap(x, kind);
    }

    // x * p(mean(x^2)) per lane: rotate-and-add windows to the lane start, mask (times 1/768), broadcast back
    Ct norm(const Ct& x, const std::vector<double>& pcoef) {
        PhaseScope ps(be_, "norm");
        Ct s = be_->mul(x, x);
        for (const auto& w : norm_windows(1)) s = be_->rotate_sum(s, w);
        s = be_->mul_pt(s, *vec_pt("lane_start", s.level, [] {
            std::vector<double> m(DPAD, 0.0);
            m[0] = 1.0 / D;
            return m;
        }));
        for (const auto& w : norm_windows(-1)) s = be_->rotate_sum(s, w);
        Ct n = be_->poly3(s, pcoef);
        return be_->mul(x, n);
    }

    // every head's sum of x (times scale), broadcast over the head's 64 channels: a rotate-and-add window of 64 (slot
    // h*64 of a lane then holds head h's sum), mask the head starts (times scale), broadcast back
    Ct head_sum(const Ct& x, double scale) {
        PhaseScope ps(be_, "head_sum");
        Ct s = be_->rotate_sum(x, head_window(1));
        char tag[48];
        std::snprintf(tag, sizeof(tag), "head_start%.17g", scale);
        s = be_->mul_pt(s, *vec_pt(tag, s.level, [scale] {
            std::vector<double> m(DPAD, 0.0);
            for (int c = 0; c < D; c += HS) m[c] = scale;
            return m;
        }));
        return be_->rotate_sum(s, head_window(-1));
    }

    static std::vector<double> periodic_of(const std::vector<double>& v) {
        std::vector<double> p(DPAD, 0.0);
        std::copy(v.begin(), v.end(), p.begin());
        return p;
    }

    // the time-mix increment o; v0: the first layer's value (set by layer 0, read by the later layers)
    Ct time_mix(uint32_t li, const Ct& x, LayerState& st, Ct& v0) {
        const LayerW& L = layers_[li];
        const std::string tag = std::to_string(li);
        const bool first = li == 0;
        Ct xn = norm(x, L["p_n1"]);
        const uint32_t lv = std::min(xn.level, st.xp_t.level);
        static const char* mix[6] = {"r", "k", "v", "w", "a", "g"};
        const Matvec& tm = mv_pt("tm" + tag, lv, [&] {
            std::vector<std::vector<Block>> out;
            const auto& g1 = L["g1"];
            // the token-shift pair of one projection: row scale rs (or none) times W, columns times g1 (1 - mu), g1 mu
            auto add = [&](const std::vector<double>& W, const std::vector<double>& mu, const std::vector<double>* rs) {
                auto a = std::make_shared<std::vector<double>>(D), b = std::make_shared<std::vector<double>>(D);
                for (int c = 0; c < D; c++) {
                    (*a)[c] = g1[c] * (1.0 - mu[c]);
                    (*b)[c] = g1[c] * mu[c];
                }
                const double* w = W.data();
                const double* r = rs ? rs->data() : nullptr;
                out.push_back({[w, a, r](int i, int c) { return (r ? r[i] : 1.0) * w[(size_t)i * D + c] * (*a)[c]; },
                               [w, b, r](int i, int c) { return (r ? r[i] : 1.0) * w[(size_t)i * D + c] * (*b)[c]; }});
            };
            for (auto* m : mix) add(L[std::string("W_") + m], L[std::string("mu_") + m], nullptr);
            add(L["W_k"], L["mu_k"], &L["k_k"]);       // kk = k_k (.) k
            if (!first) add(L["W_vg"], L["mu_v"], nullptr);  // the value gate's argument
            return out;
        });
        Ct proj = be_->matvec({be_->at(xn, lv), be_->at(st.xp_t, lv)}, tm);
        Ct r = be_->item(proj, 0), k = be_->item(proj, 1), v = be_->item(proj, 2), kk = be_->item(proj, 6);
        Ct w = be_->poly3(be_->item(proj, 3), L["p_w"]);
        Ct a = be_->poly3(be_->item(proj, 4), L["p_a"]);
        Ct g = be_->poly3(be_->item(proj, 5), L["p_g"]);
        if (first) {
            v0 = v;
        } else {  // value residual: v + (v0 - v) p_v(W_vg u_v)
            Ct gate = be_->poly3(be_->item(proj, 7), L["p_v"]);
            Ct dv = be_->add(v0, v, -1);
            Ct mix_v = be_->mul(dv, gate);
            v = be_->add(v, mix_v);
        }
        // the per-head L2 norm of kk enters only the removal term, as its square:
        // (S kh)(kh a)^T = n^2 (S kk)(kk a)^T with kh = n kk, n = p_kn(|kk_h|^2)
        Ct kk2 = be_->mul(kk, kk);
        Ct zk = head_sum(kk2, 1.0);
        Ct nk = be_->poly3(zk, L["p_kn"]);
        Ct n2 = be_->mul(nk, nk);
        const std::vector<double>& kkw = L["k_k"];
        const std::vector<double>& kaw = L["k_a"];
        std::vector<double> one_minus_ka(D);
        for (int c = 0; c < D; c++) one_minus_ka[c] = 1.0 - kaw[c];
        auto masks2 = [](const double* e1, const double* e2) {
            auto m = wkv_masks(e1), m2 = wkv_masks(e2);
            m.insert(m.end(), m2.begin(), m2.end());
            return m;
        };
        be_->set_phase("wkv");
        // k's masked rotations: rot64_t(kk) = rot64_t(k) k_k, and the key update k' = k (1 - k_a) + (k a) k_a
        Ct KX = be_->rotate_masked(k, *vec_pt("mask_k" + tag, k.level,
                                               [&] { return masks2(kkw.data(), one_minus_ka.data()); }), 2);
        Ct KK_t = be_->slice(KX, 0, WKV_T), K1_t = be_->slice(KX, WKV_T, 2 * WKV_T);
        Ct ka = be_->mul(k, a);
        Ct KB = be_->rotate_masked(ka, *vec_pt("mask_ka" + tag, ka.level,
                                                [&] { return masks2(kkw.data(), kaw.data()); }), 2);
        Ct B_t = be_->slice(KB, 0, WKV_T), K2_t = be_->slice(KB, WKV_T, 2 * WKV_T);
        auto masks = [] { return wkv_masks(nullptr); };
        Ct R_t = be_->rotate_masked(r, *vec_pt("mask", r.level, masks), 1);
        Ct W_t = be_->rotate_masked(w, *vec_pt("mask", w.level, masks), 1);
        auto Dt = [&](uint32_t t) { return &st.Dseg[st.Didx[t].first]; };
        std::vector<std::vector<Pair>> p1(1);
        for (uint32_t t = 0; t < WKV_T; t++) p1[0].push_back(Pair{Dt(t), st.Didx[t].second, &KK_t, t});
        Ct sa = be_->mult_sum(p1);
        Ct nsa0 = be_->at_neg(sa, n2.level);
        Ct nsa = be_->mul(nsa0, n2);
        std::vector<std::vector<Pair>> p2(WKV_T);
        for (uint32_t t = 0; t < WKV_T; t++)
            p2[t] = {Pair{Dt(t), st.Didx[t].second, &W_t, t}, Pair{&nsa, 0, &B_t, t}, Pair{&v, 0, &K1_t, t},
                     Pair{&v, 0, &K2_t, t}};
        Ct Dn = be_->mult_sum(p2);
        std::vector<std::vector<Pair>> p3(1);
        for (uint32_t t = 0; t < WKV_T; t++) p3[0].push_back(Pair{&Dn, t, &R_t, t});
        Ct y = be_->mult_sum(p3);
        be_->set_phase("elementwise");
        // the bonus coefficient per head: sum of r k' r_k = (r k) (1 - k_a) r_k + (r ka) k_a r_k
        const std::vector<double>& rkw = L["r_k"];
        Ct rk1p = be_->mul(r, k);
        Ct rk1 = be_->mul_pt(rk1p, *vec_pt("rk1_" + tag, rk1p.level, [&] {
            std::vector<double> m(DPAD, 0.0);
            for (int c = 0; c < D; c++) m[c] = (1.0 - kaw[c]) * rkw[c];
            return m;
        }));
        Ct rk2p = be_->mul(r, ka);
        Ct rk2 = be_->mul_pt(rk2p, *vec_pt("rk2_" + tag, rk2p.level, [&] {
            std::vector<double> m(DPAD, 0.0);
            for (int c = 0; c < D; c++) m[c] = kaw[c] * rkw[c];
            return m;
        }));
        Ct rk = be_->add(rk1, rk2);
        Ct sb = head_sum(rk, 1.0);
        // y and the bonus coefficient are bootstrapped together (GroupNorm needs more levels than are left)
        const uint32_t m = std::min(y.level, sb.level);
        Ct ya = be_->at(y, m), sba = be_->at(sb, m);
        Ct yb = boot(be_->concat({ya, sba}), "state");
        Ct Y = be_->item(yb, 0), SB = be_->item(yb, 1);
        // GroupNorm per head: mean and mean of squares from one batch of rotations, var = E[y^2] - mean^2
        Ct Ylow = be_->at(Y, Y.level - 1);
        Ct Y2 = be_->mul(Y, Y);
        Ct mom = head_sum(be_->concat({Ylow, Y2}), 1.0 / HS);
        Ct mu = be_->item(mom, 0), ey2 = be_->item(mom, 1);
        Ct mu2 = be_->mul(mu, mu);
        Ct var = be_->add(ey2, mu2, -1);
        Ct yc = be_->add(Y, mu, -1);
        Ct pg = be_->poly3(var, L["p_gn"]);
        Ct yn = be_->mul(yc, pg);
        Ct yl = be_->mul_pt(yn, *vec_pt("ln_w" + tag, yn.level, [&] { return periodic_of(L["ln_w"]); }));
        Ct bon = be_->mul(SB, v);
        Ct y3 = be_->add(yl, bon);
        // (y3 + ln_b) g: ln_b enters as ln_b (.) g
        Ct y3g = be_->mul(y3, g);
        Ct bg = be_->mul_pt(g, *vec_pt("ln_b" + tag, g.level, [&] { return periodic_of(L["ln_b"]); }));
        Ct yg = be_->add(y3g, bg);
        const double* wo = L["W_o"].data();
        Ct o = be_->matvec({yg}, mv_pt("wo" + tag, yg.level, [wo] {
            return std::vector<std::vector<Block>>{{[wo](int r, int c) { return wo[(size_t)r * D + c]; }}};
        }));
        st.xp_t = xn;
        st.Dn = Dn;
        return o;
    }

    Ct channel_mix(uint32_t li, const Ct& x, LayerState& st) {
        const LayerW& L = layers_[li];
        Ct xn2 = norm(x, L["p_n2"]);
        const uint32_t lv = std::min(xn2.level, st.xp_c.level);
        const Matvec& ck_mv = mv_pt("ck" + std::to_string(li), lv, [&] {
            const auto& g2 = L["g2"];
            const auto& mu = L["mu_c"];
            auto a = std::make_shared<std::vector<double>>(D), b = std::make_shared<std::vector<double>>(D);
            for (int c = 0; c < D; c++) {
                (*a)[c] = g2[c] * (1.0 - mu[c]);
                (*b)[c] = g2[c] * mu[c];
            }
            const double* w = L["W_ck"].data();
            std::vector<std::vector<Block>> out;
            for (int o = 0; o < 4; o++) {
                const double* wo = w + (size_t)o * D * D;
                out.push_back({[wo, a](int r, int c) { return wo[(size_t)r * D + c] * (*a)[c]; },
                               [wo, b](int r, int c) { return wo[(size_t)r * D + c] * (*b)[c]; }});
            }
            return out;
        });
        Ct hs = be_->matvec({be_->at(xn2, lv), be_->at(st.xp_c, lv)}, ck_mv);
        Ct h = be_->poly3(hs, L["p_h"]);
        const double* wcv = L["W_cv"].data();
        const Matvec& cv = mv_pt("cv" + std::to_string(li), h.level, [wcv] {
            std::vector<Block> row;
            for (int i = 0; i < 4; i++)
                row.push_back([wcv, i](int r, int c) { return wcv[(size_t)r * FF + (size_t)i * D + c]; });
            return std::vector<std::vector<Block>>{row};
        });
        std::vector<Ct> hin;
        for (uint32_t i = 0; i < 4; i++) hin.push_back(be_->item(h, i));
        Ct f = be_->matvec(hin, cv);
        st.xp_c = xn2;
        return f;
    }

    // bootstrap the new state once: the 64 diagonals packed 4 -> 3 into the lanes' unused channels, the 48 packed
    // two per complex ciphertext, 24 bootstraps, unpacked with one conjugation and three masked rotations
    void refresh_state(LayerState& st) {
        PhaseScope ps(be_, "state_pack");
        Ct Dn = st.Dn;
        st.Dn = Ct{};
        const uint32_t q = WKV_T / 4, h = q / 2;
        Ct quarter[4];
        for (uint32_t k = 0; k < 4; k++) quarter[k] = be_->slice(Dn, k * q, (k + 1) * q);
        Ct packed3[3];
        for (int p = 0; p < 3; p++) {
            auto m = vec_pt("gap_in" + std::to_string(p), quarter[3].level,
                            [p] { return channel_range_mask(256 * p, 256 * (p + 1)); });
            packed3[p] = be_->add(quarter[p], be_->rotate(be_->mul_pt(quarter[3], *m), -kGapShift[p]));
        }
        const Ct &A = packed3[0], &B = packed3[1], &C = packed3[2];
        Ct pk = be_->concat({be_->add(A, be_->mul_i(B, 1)),
                             be_->add(be_->slice(C, 0, h), be_->mul_i(be_->slice(C, h, q), 1))});
        n_boot_ += pk.B;
        Ct P = be_->bootstrap(pk, "state");
        be_->set_phase("state_unpack");
        Ct Cj = be_->conj(P);
        Ct re2 = be_->add(P, Cj);                     // 2 Re: A, C[0:8]
        Ct im2 = be_->mul_i(be_->add(Cj, P, -1), 1);  // i (conj - P) = 2 Im: B, C[8:16]
        re2.scale *= 2.0;  // the sums hold 2 D_t: the same words declared at twice the scale
        im2.scale *= 2.0;
        Ct A2 = be_->slice(re2, 0, q), B2 = be_->slice(im2, 0, q);
        Ct C2 = be_->concat({be_->slice(re2, q, q + h), be_->slice(im2, q, q + h)});
        const Ct* src[3] = {&A2, &B2, &C2};
        std::vector<Ct> terms;
        for (int p = 0; p < 3; p++) {
            auto m = vec_pt("gap_out" + std::to_string(p), src[p]->level,
                            [p] { return channel_range_mask(256 * p, 256 * (p + 1)); });
            terms.push_back(be_->mul_pt(be_->rotate(*src[p], kGapShift[p]), *m));
        }
        Ct D4 = be_->lin_int({&terms[0], &terms[1], &terms[2]}, {1.0, 1.0, 1.0});
        st.Dseg = {A2, B2, C2, D4};
        st.Didx.clear();
        for (uint32_t k = 0; k < 4; k++)
            for (uint32_t t = 0; t < q; t++) st.Didx.push_back({k, t});
    }

    // -- the host copy of the carried state ------------------------------------------------------------------
    template <class F>
    static void for_each_ct(LayerState& st, F&& f) {
        for (auto& c : st.Dseg) f(c);
        f(st.xp_t);
        f(st.xp_c);
        f(st.Dn);
    }

    void* host_get(size_t bytes) {
        auto& l = host_free_[bytes];
        if (!l.empty()) {
            void* p = l.back();
            l.pop_back();
            return p;
        }
        void* p = nullptr;
        ck(ckks_host_alloc(bytes, &p), "ckks_host_alloc");
        return p;
    }

    // pinned host buffers for the next step's copy of the state, allocated now (after the step that made the state)
    // rather than inside the next step
    void reserve_backup() {
        std::map<size_t, size_t> need;
        std::set<const Buf*> seen;
        for (auto& st : state_)
            for_each_ct(st, [&](Ct& c) {
                if (c.buf && seen.insert(c.buf.get()).second) need[c.buf->bytes]++;
            });
        for (auto& kv : need) {
            auto& l = host_free_[kv.first];
            while (l.size() < kv.second) {
                void* p = nullptr;
                ck(ckks_host_alloc(kv.first, &p), "ckks_host_alloc");
                l.push_back(p);
            }
        }
    }

    // every buffer of the state copied to the host on the side stream (after the work enqueued so far)
    void backup() {
        saved_ = Saved{};
        saved_.active = true;
        saved_.meta = state_;
        std::map<const Buf*, int> index;
        for (auto& st : saved_.meta) {
            std::vector<int> ids;
            uint64_t ticket = 0;
            for_each_ct(st, [&](Ct& c) {
                if (!c.buf) {
                    ids.push_back(-1);
                    return;
                }
                auto it = index.find(c.buf.get());
                if (it == index.end()) {
                    void* h = host_get(c.buf->bytes);
                    saved_.copies.emplace_back(h, c.buf->bytes);
                    ck(ckks_side_copy(be_->ctx(), h, c.buf->d, c.buf->bytes, nullptr, &ticket), "ckks_side_copy");
                    it = index.emplace(c.buf.get(), (int)saved_.copies.size() - 1).first;
                }
                ids.push_back(it->second);
                c.buf.reset();  // the metadata only: the device buffer is not held by the copy
            });
            saved_.ids.push_back(std::move(ids));
            saved_.ticket.push_back(ticket);
        }
    }

    // layer li's previous state is no longer needed on the device: once its copy has landed (the wait is ordered
    // on the work stream, before any reuse of the released buffers), let it go
    void release_layer(uint32_t li) {
        if (li >= state_.size()) return;
        if (saved_.active && li < saved_.ticket.size() && saved_.ticket[li])
            ck(ckks_side_wait(be_->ctx(), saved_.ticket[li], nullptr), "ckks_side_wait");
        if (saved_.active) {
            // every copy up to this layer's last one has landed: the buffers shared with later layers stay held
            state_[li] = LayerState{};
        }
    }

    // the device must not reuse a buffer still being copied
    void wait_backup() {
        if (!saved_.active) return;
        for (auto t : saved_.ticket)
            if (t) ck(ckks_side_wait(be_->ctx(), t, nullptr), "ckks_side_wait");
    }

    void restore_backup() {
        ck(ckks_side_sync(be_->ctx()), "ckks_side_sync");
        std::vector<std::shared_ptr<Buf>> bufs(saved_.copies.size());
        for (size_t i = 0; i < bufs.size(); i++) {
            bufs[i] = be_->alloc(saved_.copies[i].second);
            ck(ckks_memcpy_h2d(bufs[i]->d, saved_.copies[i].first, saved_.copies[i].second), "ckks_memcpy_h2d");
        }
        std::vector<LayerState> st = saved_.meta;
        for (size_t li = 0; li < st.size(); li++) {
            size_t j = 0;
            for_each_ct(st[li], [&](Ct& c) {
                const int id = saved_.ids[li][j++];
                if (id >= 0) c.buf = bufs[id];
            });
        }
        state_ = std::move(st);
    }

    void drop_backup() {
        wait_backup();
        ck(ckks_side_sync(be_->ctx()), "ckks_side_sync");  // the host buffers go back to the free lists
        for (auto& c : saved_.copies) host_free_[c.second].push_back(c.first);
        saved_ = Saved{};
    }

    std::vector<LayerState> cold_state() {
        const uint32_t lt = be_->top_level();
        std::vector<LayerState> state(layers_.size());
        for (auto& st : state) {
            st.Dseg = {be_->zeros(WKV_T, lt)};
            st.Didx.clear();
            for (uint32_t t = 0; t < (uint32_t)WKV_T; t++) st.Didx.push_back({0, t});
            st.xp_t = be_->zeros(1, lt);
            st.xp_c = be_->zeros(1, lt);
        }
        return state;
    }

    Engine* be_;
    std::vector<LayerW> layers_;
    LayerW model_;
    std::vector<LayerState> state_;
    // the previous state on the host while a step (or a held request) may still need to put it back
    struct Saved {
        bool active = false;
        std::vector<LayerState> meta;             // the state's ciphertexts without their buffers
        std::vector<std::vector<int>> ids;        // per layer, per ciphertext (for_each_ct order): its copy, or -1
        std::vector<std::pair<void*, size_t>> copies;  // pinned host buffer, bytes
        std::vector<uint64_t> ticket;             // per layer: the side copy of its last new buffer (0: none)
    } saved_;
    std::map<size_t, std::vector<void*>> host_free_;  // pinned host buffers kept for the next backup
    std::map<std::pair<std::string, uint32_t>, std::shared_ptr<Buf>> pt_;
    std::map<std::pair<std::string, uint32_t>, Matvec> mv_;
    uint64_t n_boot_ = 0;
};

template <class F>
int guarded(F&& f) {
    try {
        f();
        g_err.clear();
        return CKKS_OK;
    } catch (const Error& e) {
        g_err = e.what();
        return e.code;
    } catch (const std::bad_alloc&) {
        g_err = "out of host memory";
        return CKKS_ENOMEM;
    } catch (const std::exception& e) {
        g_err = e.what();
        return CKKS_EINVAL;
    }
}

}  // namespace

struct fhe_ssm_decoder {
    std::unique_ptr<Engine> be;
    std::unique_ptr<Decoder> dec;
};

// the library's last-error message, set from the other translation units of the library (host/serve.cpp)
namespace fhe_ssm_detail {
void set_error(const std::string& m) { g_err = m; }
}  // namespace fhe_ssm_detail

namespace {

// the decode step as the serve protocol's handler: one token (up to 32 lanes) per ciphertext file, run as
// consecutive steps over the carried state; the response meta stamps the request's lanes and count
// (gpu_real_model.cu:2332-2339, writeCtMeta)
struct ServeState {
    fhe_ssm_decoder* dec;
    uint64_t* d_in;
};

void serve_tokens(ServeState* sv, const char* req_prefix, const char* resp_prefix, long long count, long long tokens,
                  long long lanes, bool reset);

int serve_step(void* user, uint32_t, const char* req_prefix, const char* resp_prefix, const char* meta, int32_t reset,
               char* err, size_t err_cap) {
    auto* sv = static_cast<ServeState*>(user);
    const int rc = guarded([&] {
        Engine& be = *sv->dec->be;
        const uint32_t top = be.top_level();
        auto mi = [&](const char* k, long long dflt) { return fhe_ssm_meta_int(meta, k, dflt); };
        const long long count = mi("count", -1), tokens = mi("tokensReal", -1), lanes = mi("lanes", 1);
        if (count != tokens) throw Error(CKKS_EINVAL, "one token per ciphertext: count must equal tokensReal");
        if (mi("packTokens", -1) != 1 || mi("dpad", -1) != DPAD || mi("ringDim", -1) != (long long)kN ||
            mi("interleave", 0) != 0)
            throw Error(CKKS_EINVAL, "request layout is not this decoder's (packTokens 1, dpad 1024, ringDim 65536, "
                                     "interleave 0)");
        if (lanes < 1 || lanes > (long long)(kN / 2 / DPAD)) throw Error(CKKS_EINVAL, "lanes must be in [1, 32]");
        if (mi("level", -1) != (long long)top)
            throw Error(CKKS_EINVAL, "request level must be the state plan's output level " + std::to_string(top));
        // a request is all or nothing: on any failure the carried state is the one from before the request
        // (reset included), as in the reference, which commits its carry only after the whole pass
        // (gpu_real_model.cu:5284-5286)
        Decoder& dec = *sv->dec->dec;
        dec.hold_backup();  // the state from before the request, on the host until the request is done
        try {
            serve_tokens(sv, req_prefix, resp_prefix, count, tokens, lanes, reset != 0);
        } catch (...) {
            dec.restore_held();
            throw;
        }
        dec.release_held();
    });
    if (rc != CKKS_OK && err && err_cap) std::snprintf(err, err_cap, "%s", g_err.c_str());
    return rc;
}

void serve_tokens(ServeState* sv, const char* req_prefix, const char* resp_prefix, long long count, long long tokens,
                  long long lanes, bool reset) {
    Engine& be = *sv->dec->be;
    const uint32_t top = be.top_level();
    if (reset) sv->dec->dec->reset();
    uint32_t out_level = 0;
    for (long long t = 0; t < count; t++) {
        const std::string in = std::string(req_prefix) + "." + std::to_string(t);
        uint32_t lvl = 0;
        double sc = 0.0;
        ck(ckks_ct_load(be.ctx(), in.c_str(), top, sv->d_in, &lvl, &sc), "ckks_ct_load");
        if (lvl != top) throw Error(CKKS_EINVAL, in + ": not at the state plan's output level");
        if (std::fabs(sc / be.S(top) - 1.0) > 1e-9) throw Error(CKKS_EINVAL, in + ": scale is not S(level)");
        Ct y = sv->dec->dec->step(Engine::borrowed(sv->d_in, 1, top, sc));
        const std::string out = std::string(resp_prefix) + "." + std::to_string(t);
        ck(ckks_ct_save(be.ctx(), out.c_str(), y.ptr(), y.level, y.scale), "ckks_ct_save");
        out_level = y.level;
    }
    FILE* f = std::fopen((std::string(resp_prefix) + ".meta").c_str(), "w");
    if (!f) throw Error(CKKS_EINVAL, "cannot write the response meta");
    std::fprintf(f,
                 "{\"count\":%lld,\"packTokens\":1,\"tokensReal\":%lld,\"dpad\":%d,\"interleave\":0,"
                 "\"lanes\":%lld,\"ringDim\":%u,\"level\":%u}\n",
                 count, tokens, DPAD, lanes, kN, out_level);
    if (std::fclose(f) != 0) throw Error(CKKS_EINVAL, "cannot write the response meta");
}

}  // namespace

extern "C" {

const char* fhe_ssm_last_error(void) { return g_err.c_str(); }

int fhe_ssm_rotation_steps(int64_t* steps, uint32_t cap, uint32_t* n_steps) {
    return guarded([&] {
        const auto s = layer_rotation_steps();
        if (!n_steps) throw Error(CKKS_EINVAL, "n_steps is null");
        *n_steps = (uint32_t)s.size();
        for (uint32_t i = 0; i < s.size() && i < cap && steps; i++) steps[i] = s[i];
    });
}

int fhe_ssm_decoder_create(ckks_context* ctx, uint32_t n_layers, fhe_ssm_refresh state, fhe_ssm_refresh inc_tm,
                           fhe_ssm_refresh inc_cm, const uint64_t* d_relin, const uint64_t* d_conj,
                           const int64_t* steps, const uint64_t* const* d_evks, uint32_t n_keys,
                           fhe_ssm_decoder** out) {
    return guarded([&] {
        if (!ctx || !out || !d_relin || !d_conj || (n_keys && (!steps || !d_evks)) || n_layers == 0)
            throw Error(CKKS_EINVAL, "null argument or no layers");
        auto d = std::make_unique<fhe_ssm_decoder>();
        d->be = std::make_unique<Engine>(ctx, state, inc_tm, inc_cm, d_relin, d_conj, steps, d_evks, n_keys);
        for (auto s : layer_rotation_steps()) d->be->key(s);  // every layer-loop key present
        d->dec = std::make_unique<Decoder>(d->be.get(), n_layers);
        *out = d.release();
    });
}

void fhe_ssm_decoder_destroy(fhe_ssm_decoder* dec) {
    if (!dec) return;
    dec->dec.reset();  // ciphertexts and plaintexts go back before the pool is released
    dec->be.reset();
    delete dec;
}

int fhe_ssm_decoder_set_weight(fhe_ssm_decoder* dec, const char* name, int32_t layer, const double* data,
                               size_t count) {
    return guarded([&] {
        if (!dec || !name || !data) throw Error(CKKS_EINVAL, "null argument");
        dec->dec->set_weight(name, layer, data, count);
    });
}

int fhe_ssm_decoder_store_save(fhe_ssm_decoder* dec, const char* path, uint64_t* n_entries) {
    return guarded([&] {
        if (!dec || !path) throw Error(CKKS_EINVAL, "null argument");
        const uint64_t n = dec->dec->store_save(path);
        if (n_entries) *n_entries = n;
    });
}

int fhe_ssm_decoder_store_load(fhe_ssm_decoder* dec, const char* path, uint64_t* n_entries) {
    return guarded([&] {
        if (!dec || !path) throw Error(CKKS_EINVAL, "null argument");
        const uint64_t n = dec->dec->store_load(path);
        if (n_entries) *n_entries = n;
    });
}

int fhe_ssm_decoder_step(fhe_ssm_decoder* dec, const uint64_t* d_x, uint32_t level, double scale, uint64_t* d_out,
                         uint32_t* out_level, double* out_scale) {
    return guarded([&] {
        if (!dec || !d_x || !d_out || !out_level || !out_scale) throw Error(CKKS_EINVAL, "null argument");
        Engine& be = *dec->be;
        if (level != be.top_level()) throw Error(CKKS_EINVAL, "the input must be at the plan's output level");
        // the step reads its input in place and never writes it
        Ct y = dec->dec->step(Engine::borrowed(d_x, 1, level, scale));
        be.copy_to(y, Engine::borrowed(d_out, 1, y.level, y.scale));
        *out_level = y.level;
        *out_scale = y.scale;
    });
}

int fhe_ssm_decoder_reset(fhe_ssm_decoder* dec) {
    return guarded([&] {
        if (!dec) throw Error(CKKS_EINVAL, "null argument");
        dec->dec->reset();
    });
}

int fhe_ssm_decoder_serve(fhe_ssm_decoder* dec, const char* dir, const fhe_ssm_serve_opts* opts,
                          fhe_ssm_serve_report* report) {
    ServeState sv{dec, nullptr};
    int rc = guarded([&] {
        if (!dec || !dir || !opts || !report) throw Error(CKKS_EINVAL, "null argument");
        void* p = nullptr;
        ck(ckks_buffer_alloc((size_t)2 * dec->be->top_level() * kN * 8, &p), "ckks_buffer_alloc");
        sv.d_in = static_cast<uint64_t*>(p);
    });
    if (rc != CKKS_OK) return rc;
    rc = fhe_ssm_serve_dir(dir, opts, serve_step, &sv, report);  // sets the error message itself
    ckks_buffer_free(sv.d_in);
    if (rc == CKKS_OK) g_err.clear();
    return rc;
}

int fhe_ssm_decoder_memory(const fhe_ssm_decoder* dec, uint64_t* bytes, uint32_t n) {
    return guarded([&] {
        if (!dec || (!bytes && n)) throw Error(CKKS_EINVAL, "null argument");
        const uint64_t v[6] = {dec->dec->store_bytes(), dec->be->diag_bytes(), dec->be->pool_bytes(),
                               dec->dec->state_bytes(), dec->dec->backup_host_bytes(), dec->dec->store_host_bytes()};
        for (uint32_t i = 0; i < n && i < 6; i++) bytes[i] = v[i];
    });
}

int fhe_ssm_decoder_stats(const fhe_ssm_decoder* dec, uint64_t* bootstraps) {
    return guarded([&] {
        if (!dec || !bootstraps) throw Error(CKKS_EINVAL, "null argument");
        *bootstraps = dec->dec->bootstraps();
    });
}

}  // extern "C"
