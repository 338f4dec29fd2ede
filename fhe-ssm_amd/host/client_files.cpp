// client_files.cpp -- the client's file steps of the reference driver, over the engine's C ABI only:
//   --enc-in ROWS   (hpc_gpu_port/gpu_real_model.cu:2345-2433): T x d float64 rows -> ROWS.ct.<t> + ROWS.ct.meta
//   --dec-out RESP  (:2435-2533): RESP.meta + RESP.<t> -> decrypt -> plaintext vocabulary head -> RESP.logits.f64
// Rows are raw little-endian float64; with lanes > 1 they are lane-major (lane r's T rows first, the layout
// ml-eval/fhe_client.py:206-238 writes), and token t's ciphertext holds slot rep * dpad + i = lane (rep mod lanes)
// channel i for every replica rep < slots / dpad (:2378-2395).  Logits are tokensReal * lanes rows of vocab float64,
// token-major and lane-minor (row tok * lanes + lane, :2468-2480), each the head matrix times the lane's first d
// channels.  The ciphertext files are this engine's (ckks_ct_save); encryption uses the public key, as the reference's
// client does (it holds no secret at that step).
#include <sys/stat.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "fhe_ssm_decode.h"

namespace fhe_ssm_detail {
void set_error(const std::string& m);  // host/decode.cpp
}  // namespace fhe_ssm_detail

namespace {

constexpr uint32_t kN = 1u << 16, kSlots = kN / 2;

struct Fail {
    int code;
    std::string msg;
};

void ck(int rc, const char* what) {
    if (rc != CKKS_OK) throw Fail{rc, std::string(what) + ": " + ckks_last_error()};
}

template <class F>
int guarded(F&& f) {
    try {
        f();
        return CKKS_OK;
    } catch (const Fail& e) {
        fhe_ssm_detail::set_error(e.msg);
        return e.code;
    } catch (const std::bad_alloc&) {
        fhe_ssm_detail::set_error("out of host memory");
        return CKKS_ENOMEM;
    } catch (const std::exception& e) {
        fhe_ssm_detail::set_error(e.what());
        return CKKS_EINVAL;
    }
}

// a device buffer through the engine's allocator, freed on scope exit
struct DevBuf {
    void* p = nullptr;
    explicit DevBuf(size_t bytes) { ck(ckks_buffer_alloc(bytes, &p), "ckks_buffer_alloc"); }
    ~DevBuf() { ckks_buffer_free(p); }
    uint64_t* u() const { return static_cast<uint64_t*>(p); }
};

long long file_bytes(const std::string& path) {
    struct stat st;
    return ::stat(path.c_str(), &st) == 0 ? (long long)st.st_size : -1;
}

std::string read_text(const std::string& path) {
    std::ifstream f(path);
    if (!f) throw Fail{CKKS_EINVAL, "missing ct meta: " + path};
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

}  // namespace

extern "C" {

int fhe_ssm_client_encrypt_rows(ckks_context* ctx, const uint64_t* d_pk, const char* rows_path, uint32_t tokens,
                                uint32_t lanes, uint32_t d, uint32_t dpad, uint32_t level, double scale,
                                const uint8_t* seed32) {
    return guarded([&] {
        if (!ctx || !d_pk || !rows_path || !seed32) throw Fail{CKKS_EINVAL, "enc-in: null argument"};
        if (tokens < 1 || lanes < 1 || d < 1 || dpad < d || kSlots % dpad != 0)
            throw Fail{CKKS_EINVAL, "enc-in: tokens, lanes >= 1 and d <= dpad with dpad dividing N/2"};
        const uint32_t rep = kSlots / dpad;
        if (lanes > rep) throw Fail{CKKS_EINVAL, "enc-in: client-lanes > REP (slots / dpad)"};
        const long long need = (long long)lanes * tokens * d * (long long)sizeof(double);
        const long long have = file_bytes(rows_path);
        if (have < 0) throw Fail{CKKS_EINVAL, std::string("enc-in: cannot open ") + rows_path};
        if (have < need)
            throw Fail{CKKS_EINVAL, "enc-in: short file (" + std::to_string(have) + " bytes, need " +
                                        std::to_string(need) + ")"};
        std::vector<double> rows((size_t)need / sizeof(double));
        {
            std::ifstream f(rows_path, std::ios::binary);
            f.read(reinterpret_cast<char*>(rows.data()), need);
            if (!f) throw Fail{CKKS_EINVAL, std::string("enc-in: read failed: ") + rows_path};
        }
        const std::string prefix = std::string(rows_path) + ".ct";
        DevBuf pt((size_t)level * kN * 8), ct((size_t)2 * level * kN * 8);
        std::vector<double> sv(kSlots);
        for (uint32_t t = 0; t < tokens; t++) {
            std::fill(sv.begin(), sv.end(), 0.0);
            for (uint32_t r = 0; r < rep; r++) {
                const double* row = rows.data() + ((size_t)(r % lanes) * tokens + t) * d;
                std::copy(row, row + d, sv.begin() + (size_t)r * dpad);
            }
            ck(ckks_encode(ctx, sv.data(), nullptr, kSlots, level, scale, pt.u()), "ckks_encode");
            ck(ckks_encrypt_public(ctx, d_pk, pt.u(), level, seed32, t, ct.u()), "ckks_encrypt_public");
            ck(ckks_ct_save(ctx, (prefix + "." + std::to_string(t)).c_str(), ct.u(), level, scale), "ckks_ct_save");
        }
        FILE* f = std::fopen((prefix + ".meta").c_str(), "w");
        if (!f) throw Fail{CKKS_EINVAL, "enc-in: cannot write " + prefix + ".meta"};
        std::fprintf(f,
                     "{\"count\":%u,\"packTokens\":1,\"tokensReal\":%u,\"dpad\":%u,\"interleave\":0,\"lanes\":%u,"
                     "\"ringDim\":%u,\"level\":%u}\n",
                     tokens, tokens, dpad, lanes, kN, level);
        if (std::fclose(f) != 0) throw Fail{CKKS_EINVAL, "enc-in: cannot write " + prefix + ".meta"};
    });
}

int fhe_ssm_client_decrypt_logits(ckks_context* ctx, const ckks_secret* sk, const char* in_prefix,
                                  const double* head, uint32_t vocab, uint32_t d, uint32_t dpad) {
    return guarded([&] {
        if (!ctx || !sk || !in_prefix || !head) throw Fail{CKKS_EINVAL, "dec-out: null argument"};
        if (vocab < 1 || d < 1 || dpad < d || kSlots % dpad != 0)
            throw Fail{CKKS_EINVAL, "dec-out: vocab >= 1 and d <= dpad with dpad dividing N/2"};
        const std::string prefix(in_prefix);
        const std::string meta = read_text(prefix + ".meta");
        const long long count = fhe_ssm_meta_int(meta.c_str(), "count", -1);
        const long long tokens = fhe_ssm_meta_int(meta.c_str(), "tokensReal", -1);
        const long long lanes = std::max(1LL, fhe_ssm_meta_int(meta.c_str(), "lanes", 1));
        if (count <= 0 || tokens <= 0 || tokens > count)
            throw Fail{CKKS_EINVAL, "dec-out: bad meta (count " + std::to_string(count) + ", tokensReal " +
                                        std::to_string(tokens) + ")"};
        if (fhe_ssm_meta_int(meta.c_str(), "ringDim", 0) != (long long)kN ||
            fhe_ssm_meta_int(meta.c_str(), "dpad", 0) != (long long)dpad ||
            fhe_ssm_meta_int(meta.c_str(), "interleave", -1) != 0 ||
            fhe_ssm_meta_int(meta.c_str(), "packTokens", 1) != 1)
            throw Fail{CKKS_EINVAL, "dec-out: layout mismatch (ringDim 65536, the same dpad, interleave 0, packTokens 1)"};
        if ((long long)lanes * dpad > kSlots) throw Fail{CKKS_EINVAL, "dec-out: lanes * dpad exceeds the slots"};
        std::vector<double> logits((size_t)tokens * lanes * vocab);
        std::vector<double> re(kSlots), im(kSlots);
        std::unique_ptr<DevBuf> ct;
        uint32_t cap = 0;
        for (long long t = 0; t < tokens; t++) {
            const std::string path = prefix + "." + std::to_string(t);
            uint32_t ring = 0, level = 0;
            double scale = 0.0;
            ck(ckks_ct_file_info(path.c_str(), &ring, &level, &scale), "ckks_ct_file_info");
            if (level > cap || !ct) {
                ct.reset();
                ct.reset(new DevBuf((size_t)2 * std::max(level, 1u) * kN * 8));
                cap = std::max(level, 1u);
            }
            ck(ckks_ct_load(ctx, path.c_str(), cap, ct->u(), &level, &scale), "ckks_ct_load");
            ck(ckks_decrypt_decode(ctx, sk, ct->u(), level, scale, re.data(), im.data(), kSlots), "ckks_decrypt_decode");
            // logits of every lane: head (vocab x d) times the lane's first d channels, rows split over host threads
            const uint32_t nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
            std::vector<std::thread> th;
            for (uint32_t w = 0; w < nt; w++)
                th.emplace_back([&, w] {
                    for (uint32_t r = w; r < vocab; r += nt) {
                        const double* hr = head + (size_t)r * d;
                        for (long long lane = 0; lane < lanes; lane++) {
                            const double* hid = re.data() + (size_t)lane * dpad;
                            double s = 0.0;
                            for (uint32_t j = 0; j < d; j++) s += hr[j] * hid[j];
                            logits[((size_t)t * lanes + lane) * vocab + r] = s;
                        }
                    }
                });
            for (auto& x : th) x.join();
        }
        const std::string out = prefix + ".logits.f64";
        std::ofstream lf(out, std::ios::binary);
        lf.write(reinterpret_cast<const char*>(logits.data()), (std::streamsize)(logits.size() * sizeof(double)));
        if (!lf.good()) throw Fail{CKKS_EINVAL, "dec-out: write failed: " + out};
    });
}

}  // extern "C"
