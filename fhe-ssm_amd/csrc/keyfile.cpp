// keyfile.cpp -- seeded key-switching-key part files (the reference's "evalrot.partNNN.seeded.bin",
// hpc_gpu_port/seeded_keys.hpp:44-51), read and written on the host.
//
// Layout (all integers little-endian): char[8] "FSSMSKY1"; u32 version = 1; u32 expander = 1; u32 N; u32 sizeQ;
// u32 sizeP; u32 numPartQ; u32 numPerPartQ; u32 count; u32 keyTagLen; keyTag bytes; u64 moduli[sizeQ + sizeP];
// then per key: u32 automorphism index; u8 seed[32]; u64 b[numPartQ][sizeQ + sizeP][N] (evaluation form).
// A key's a-halves are not stored: they are the ChaCha20 expansion of the seed (nonce {digit, limb, "SKEY"},
// seeded_keys.hpp:28-43), the same expander this engine's key generation uses, so a loaded key is the key that
// was written word for word.  In device memory a key is [dnum][2][L + K][N] with b_d at poly 0 and a_d at poly 1.
//
// Ciphertext files carry the serve-directory protocol's payload (req.N.t / resp.N.t).  The reference writes
// OpenFHE-cereal ciphertexts there (gpu_real_model.cu:2303-2324, Serial::SerializeToFile), a format only OpenFHE
// reads; this engine's layout is flat: char[8] "FSSMCTX1"; u32 version = 1; u32 N; u32 level; u32 n_polys = 2;
// f64 scale; u64 moduli[level] (the chain's first `level` primes); u64 words[2][level][N] (evaluation form).
//
// The FIDESlib ".dev" sidecar (cryptocontext.bin.dev, hpc_gpu_port/mac_fhe_client.cpp:178-194) is read and written
// here too, with the loader that puts the key of every rotation it lists on the device (FIDESlib's LoadContext
// uploads GetRotationKeySwitchKey(pk, step) for each listed step, gpu_real_model.cu:1436-1529 fills its key map).
#include <hip/hip_runtime.h>

#include <climits>
#include <iterator>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "client.hpp"
#include "engine.hpp"
#include "keyfile.hpp"

namespace fhe {

namespace {

#define HIPC(expr)                                                                      \
    do {                                                                                \
        hipError_t _e = (expr);                                                         \
        if (_e != hipSuccess) throw std::runtime_error(std::string(#expr) + ": " + hipGetErrorString(_e)); \
    } while (0)

constexpr char kMagic[8] = {'F', 'S', 'S', 'M', 'S', 'K', 'Y', '1'};
constexpr uint32_t kVersion = 1, kExpander = 1;
constexpr char kCtMagic[8] = {'F', 'S', 'S', 'M', 'C', 'T', 'X', '1'};

uint32_t get32(std::istream& is, const char* what) {
    uint8_t b[4];
    if (!is.read((char*)b, 4)) throw std::invalid_argument(std::string("seeded part: short ") + what);
    return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
}

uint64_t get64(std::istream& is, const char* what) {
    uint8_t b[8];
    if (!is.read((char*)b, 8)) throw std::invalid_argument(std::string("seeded part: short ") + what);
    uint64_t v = 0;
    for (int i = 0; i < 8; i++) v |= (uint64_t)b[i] << (8 * i);
    return v;
}

void put32(std::ostream& os, uint32_t v) {
    const uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    os.write((const char*)b, 4);
}

void put64(std::ostream& os, uint64_t v) {
    uint8_t b[8];
    for (int i = 0; i < 8; i++) b[i] = (uint8_t)(v >> (8 * i));
    os.write((const char*)b, 8);
}

uint64_t record_bytes(const SeededPartHeader& h) {
    return 4 + 32 + (uint64_t)h.num_part_q * (h.size_q + h.size_p) * h.N * 8;
}

// the file's layout must be this context's: ring, chain, special primes and digit partition
void check_layout(const Context& ctx, const SeededPartHeader& h) {
    if (h.N != kN || h.size_q != ctx.L || h.size_p != ctx.K || h.num_part_q != ctx.dnum ||
        h.num_per_part_q != ctx.alpha)
        throw std::invalid_argument("seeded part: minted for another context (N, chain or digits differ)");
    for (uint32_t i = 0; i < ctx.L + ctx.K; i++)
        if (h.moduli[i] != ctx.moduli[i]) throw std::invalid_argument("seeded part: modulus chain differs");
}

}  // namespace

SeededPartHeader read_seeded_part_header(const std::string& path) {
    std::ifstream is(path, std::ios::binary);
    if (!is.good()) throw std::invalid_argument("seeded part: cannot open " + path);
    char magic[8];
    if (!is.read(magic, 8) || std::memcmp(magic, kMagic, 8) != 0) throw std::invalid_argument("seeded part: bad magic");
    SeededPartHeader h;
    h.version = get32(is, "header");
    h.expander = get32(is, "header");
    if (h.version != kVersion || h.expander != kExpander)
        throw std::invalid_argument("seeded part: unsupported version or expander");
    h.N = get32(is, "header");
    h.size_q = get32(is, "header");
    h.size_p = get32(is, "header");
    h.num_part_q = get32(is, "header");
    h.num_per_part_q = get32(is, "header");
    h.count = get32(is, "header");
    const uint32_t tag_len = get32(is, "header");
    if (tag_len > 4096) throw std::invalid_argument("seeded part: key tag too long");
    // bounds that keep record_bytes below 2^48 (N <= 2^17, at most 4096 limbs, at most one digit per limb)
    if (h.N == 0 || (h.N & (h.N - 1)) || h.N > (1u << 17) || h.size_q + h.size_p > 4096 || h.num_part_q == 0 ||
        h.num_part_q > h.size_q + h.size_p)
        throw std::invalid_argument("seeded part: implausible layout");
    h.key_tag.assign(tag_len, '\0');
    if (tag_len && !is.read(&h.key_tag[0], tag_len)) throw std::invalid_argument("seeded part: short key tag");
    h.moduli.resize(h.size_q + h.size_p);
    for (auto& m : h.moduli) m = get64(is, "moduli");
    h.header_bytes = 8 + 4 * 9 + tag_len + 8 * (uint64_t)h.moduli.size();
    // every record present
    is.seekg(0, std::ios::end);
    const uint64_t size = (uint64_t)is.tellg();
    // count records must fit (compared by division: count * record_bytes could overflow for a crafted header)
    if (size < h.header_bytes || (size - h.header_bytes) / record_bytes(h) < h.count)
        throw std::invalid_argument("seeded part: file shorter than its key count");
    return h;
}

std::vector<uint32_t> seeded_part_indices(const std::string& path) {
    const SeededPartHeader h = read_seeded_part_header(path);
    std::ifstream is(path, std::ios::binary);
    std::vector<uint32_t> idx(h.count);
    for (uint32_t r = 0; r < h.count; r++) {
        is.seekg((std::streamoff)(h.header_bytes + (uint64_t)r * record_bytes(h)));
        idx[r] = get32(is, "key record");
    }
    return idx;
}

void load_seeded_part_key(Context& ctx, const std::string& path, uint32_t record, uint32_t* index, uint64_t* d_evk) {
    const SeededPartHeader h = read_seeded_part_header(path);
    check_layout(ctx, h);
    if (record >= h.count) throw std::invalid_argument("seeded part: record index past the key count");
    std::ifstream is(path, std::ios::binary);
    is.seekg((std::streamoff)(h.header_bytes + (uint64_t)record * record_bytes(h)));
    const uint32_t g = get32(is, "key record");
    uint8_t seed[32];
    if (!is.read((char*)seed, 32)) throw std::invalid_argument("seeded part: short seed");
    const uint32_t T = ctx.L + ctx.K;
    std::vector<uint64_t> b((size_t)T * kN);
    for (uint32_t d = 0; d < ctx.dnum; d++) {
        if (!is.read((char*)b.data(), (std::streamsize)(b.size() * 8)))
            throw std::invalid_argument("seeded part: short b words");
        // every word below its modulus: the key-switch accumulators rely on operands below 2^60
        for (uint32_t i = 0; i < T; i++) {
            const uint64_t q = ctx.moduli[i];
            const uint64_t* bi = b.data() + (size_t)i * kN;
            uint64_t bad = 0;
            for (uint32_t k = 0; k < kN; k++) bad |= (uint64_t)(bi[k] >= q);
            if (bad) throw std::invalid_argument("seeded part: b word >= q");
        }
        HIPC(hipMemcpy(d_evk + (size_t)d * 2 * T * kN, b.data(), b.size() * 8, hipMemcpyHostToDevice));
    }
    expand_key_a(ctx, seed, d_evk);
    if (index) *index = g;
}

void write_seeded_part(Context& ctx, const std::string& path, const std::string& key_tag, uint32_t n,
                       const uint32_t* indices, const uint8_t* seeds, const uint64_t* const* d_evks) {
    if (key_tag.empty() || key_tag.size() > 4096) throw std::invalid_argument("seeded part: key tag length");
    std::ofstream os(path, std::ios::binary | std::ios::trunc);
    if (!os.good()) throw std::invalid_argument("seeded part: cannot create " + path);
    const uint32_t T = ctx.L + ctx.K;
    os.write(kMagic, 8);
    put32(os, kVersion);
    put32(os, kExpander);
    put32(os, kN);
    put32(os, ctx.L);
    put32(os, ctx.K);
    put32(os, ctx.dnum);
    put32(os, ctx.alpha);
    put32(os, n);
    put32(os, (uint32_t)key_tag.size());
    os.write(key_tag.data(), (std::streamsize)key_tag.size());
    for (uint32_t i = 0; i < T; i++) put64(os, ctx.moduli[i]);
    std::vector<uint64_t> b((size_t)T * kN);
    for (uint32_t r = 0; r < n; r++) {
        put32(os, indices[r]);
        os.write((const char*)(seeds + 32 * (size_t)r), 32);
        for (uint32_t d = 0; d < ctx.dnum; d++) {
            HIPC(hipMemcpy(b.data(), d_evks[r] + (size_t)d * 2 * T * kN, b.size() * 8, hipMemcpyDeviceToHost));
            os.write((const char*)b.data(), (std::streamsize)(b.size() * 8));
        }
    }
    os.flush();
    if (!os.good()) throw std::invalid_argument("seeded part: write failed: " + path);
}

CtFileHeader read_ct_header(const std::string& path) {
    std::ifstream is(path, std::ios::binary);
    if (!is.good()) throw std::invalid_argument("ciphertext file: cannot open " + path);
    char magic[8];
    if (!is.read(magic, 8) || std::memcmp(magic, kCtMagic, 8) != 0)
        throw std::invalid_argument("ciphertext file: bad magic");
    if (get32(is, "header") != kVersion) throw std::invalid_argument("ciphertext file: unsupported version");
    CtFileHeader h;
    h.N = get32(is, "header");
    h.level = get32(is, "header");
    h.n_polys = get32(is, "header");
    const uint64_t sb = get64(is, "header");
    std::memcpy(&h.scale, &sb, 8);
    if (h.N == 0 || (h.N & (h.N - 1)) || h.level == 0 || h.level > 4096 || h.n_polys != 2 || !(h.scale > 0.0))
        throw std::invalid_argument("ciphertext file: implausible header");
    h.moduli.resize(h.level);
    for (auto& m : h.moduli) m = get64(is, "moduli");
    h.header_bytes = 8 + 4 * 4 + 8 + 8 * (uint64_t)h.level;
    is.seekg(0, std::ios::end);
    if ((uint64_t)is.tellg() != h.header_bytes + (uint64_t)h.n_polys * h.level * h.N * 8)
        throw std::invalid_argument("ciphertext file: size does not match its header");
    return h;
}

void load_ct(Context& ctx, const std::string& path, uint32_t cap_level, uint64_t* d_ct, uint32_t* level,
             double* scale) {
    const CtFileHeader h = read_ct_header(path);
    if (h.N != kN) throw std::invalid_argument("ciphertext file: another ring dimension");
    if (h.level > ctx.L) throw std::invalid_argument("ciphertext file: more limbs than the chain");
    for (uint32_t i = 0; i < h.level; i++)
        if (h.moduli[i] != ctx.moduli[i]) throw std::invalid_argument("ciphertext file: modulus chain differs");
    if (h.level > cap_level) throw std::invalid_argument("ciphertext file: level above what the buffer holds");
    std::ifstream is(path, std::ios::binary);
    is.seekg((std::streamoff)h.header_bytes);
    std::vector<uint64_t> w((size_t)h.n_polys * h.level * kN);
    if (!is.read((char*)w.data(), (std::streamsize)(w.size() * 8)))
        throw std::invalid_argument("ciphertext file: short words");
    for (uint32_t p = 0; p < h.n_polys; p++)
        for (uint32_t i = 0; i < h.level; i++) {
            const uint64_t* row = w.data() + ((size_t)p * h.level + i) * kN;
            for (uint32_t k = 0; k < kN; k++)
                if (row[k] >= ctx.moduli[i]) throw std::invalid_argument("ciphertext file: word >= q");
        }
    HIPC(hipMemcpy(d_ct, w.data(), w.size() * 8, hipMemcpyHostToDevice));
    *level = h.level;
    *scale = h.scale;
}

void save_ct(Context& ctx, const std::string& path, const uint64_t* d_ct, uint32_t level, double scale) {
    if (level == 0 || level > ctx.L) throw std::invalid_argument("ciphertext file: level outside the chain");
    if (!(scale > 0.0)) throw std::invalid_argument("ciphertext file: scale must be positive");
    std::vector<uint64_t> w((size_t)2 * level * kN);
    HIPC(hipMemcpy(w.data(), d_ct, w.size() * 8, hipMemcpyDeviceToHost));
    std::ofstream os(path, std::ios::binary | std::ios::trunc);
    if (!os.good()) throw std::invalid_argument("ciphertext file: cannot create " + path);
    os.write(kCtMagic, 8);
    put32(os, kVersion);
    put32(os, kN);
    put32(os, level);
    put32(os, 2);
    uint64_t sb;
    std::memcpy(&sb, &scale, 8);
    put64(os, sb);
    for (uint32_t i = 0; i < level; i++) put64(os, ctx.moduli[i]);
    os.write((const char*)w.data(), (std::streamsize)(w.size() * 8));
    os.flush();
    if (!os.good()) throw std::invalid_argument("ciphertext file: write failed: " + path);
}

// ------------------------------------------------------------------ the FIDESlib .dev sidecar
// Six lines, as writeDevSidecar writes them (hpc_gpu_port/mac_fhe_client.cpp:183-194):
//   "<n> { <device> ... }"                 the device list ("1 { 0 }": one GPU, device 0)
//   "AutoLoadCiphertexts: <int>"
//   "AutoLoadPlaintexts: <int>"
//   "RotationIndexes: { <step> ... }"      rotation amounts, each followed by one space ("{ }" when empty)
//   "KeyDist: <int>"
//   "BootstrapSlots: { <slots> ... }"
// each ended by '\n'.  The reader takes exactly that: whitespace-separated tokens, one line per field in this
// order, nothing after the sixth line.
namespace {

std::vector<std::string> split_ws(const std::string& line) {
    std::vector<std::string> t;
    size_t i = 0;
    while (i < line.size()) {
        while (i < line.size() && (line[i] == ' ' || line[i] == '\t' || line[i] == '\r')) i++;
        size_t j = i;
        while (j < line.size() && line[j] != ' ' && line[j] != '\t' && line[j] != '\r') j++;
        if (j > i) t.push_back(line.substr(i, j - i));
        i = j;
    }
    return t;
}

[[noreturn]] void dev_fail(int line, const std::string& why) {
    throw std::invalid_argument("dev sidecar line " + std::to_string(line) + ": " + why);
}

int64_t dev_int(const std::string& tok, int line, int64_t lo, int64_t hi) {
    size_t k = 0;
    if (tok.empty()) dev_fail(line, "empty number");
    if (tok[0] == '-' || tok[0] == '+') k = 1;
    if (k == tok.size() || tok.size() > 12) dev_fail(line, "not an integer: '" + tok + "'");
    for (size_t i = k; i < tok.size(); i++)
        if (tok[i] < '0' || tok[i] > '9') dev_fail(line, "not an integer: '" + tok + "'");
    const int64_t v = std::stoll(tok);
    if (v < lo || v > hi) dev_fail(line, "out of range: " + tok);
    return v;
}

// "{ a b ... }" starting at token i0 (the braces are tokens of their own); the tokens between them
std::vector<std::string> dev_braced(const std::vector<std::string>& t, size_t i0, int line) {
    if (t.size() < i0 + 2 || t[i0] != "{" || t.back() != "}") dev_fail(line, "expected '{ ... }'");
    std::vector<std::string> inner(t.begin() + (long)i0 + 1, t.end() - 1);
    for (auto& x : inner)
        if (x == "{" || x == "}") dev_fail(line, "nested or stray brace");
    return inner;
}

int32_t dev_flag(const std::string& line, const char* key, int n) {
    const auto t = split_ws(line);
    if (t.size() != 2 || t[0] != key) dev_fail(n, std::string("expected '") + key + " <int>'");
    return (int32_t)dev_int(t[1], n, INT32_MIN, INT32_MAX);
}

uint32_t rot_index_n(int64_t k, uint32_t N) {
    const uint64_t M = 2ull * N, ord = N / 2;  // 5 has order N/2 in (Z/2N)^*
    int64_t e = k % (int64_t)ord;
    if (e < 0) e += (int64_t)ord;
    uint64_t r = 1, b = 5;
    for (uint64_t x = (uint64_t)e; x; x >>= 1) {
        if (x & 1) r = r * b % M;
        b = b * b % M;
    }
    return (uint32_t)r;
}

}  // namespace

DevSidecar read_dev_sidecar(const std::string& path) {
    std::ifstream is(path, std::ios::binary);
    if (!is.good()) throw std::invalid_argument("dev sidecar: cannot open " + path);
    std::string text((std::istreambuf_iterator<char>(is)), std::istreambuf_iterator<char>());
    if (text.size() > (1u << 20)) throw std::invalid_argument("dev sidecar: implausibly large");
    std::vector<std::string> lines;
    size_t a = 0;
    while (a < text.size()) {
        const size_t b = text.find('\n', a);
        if (b == std::string::npos) dev_fail((int)lines.size() + 1, "no line end (truncated file)");
        lines.push_back(text.substr(a, b - a));
        a = b + 1;
    }
    if (lines.size() != 6) throw std::invalid_argument("dev sidecar: " + std::to_string(lines.size()) + " lines, not 6");
    DevSidecar s;
    {
        const auto t = split_ws(lines[0]);
        if (t.empty()) dev_fail(1, "expected '<n> { <device> ... }'");
        const int64_t n = dev_int(t[0], 1, 1, 64);
        const auto ids = dev_braced(t, 1, 1);
        if ((int64_t)ids.size() != n) dev_fail(1, "device count does not match the list");
        s.devices.clear();
        for (auto& x : ids) s.devices.push_back((uint32_t)dev_int(x, 1, 0, 1023));
    }
    s.auto_load_ciphertexts = dev_flag(lines[1], "AutoLoadCiphertexts:", 2);
    s.auto_load_plaintexts = dev_flag(lines[2], "AutoLoadPlaintexts:", 3);
    {
        const auto t = split_ws(lines[3]);
        if (t.empty() || t[0] != "RotationIndexes:") dev_fail(4, "expected 'RotationIndexes: { ... }'");
        for (auto& x : dev_braced(t, 1, 4)) s.rotations.push_back((int32_t)dev_int(x, 4, INT32_MIN + 1, INT32_MAX));
    }
    s.key_dist = dev_flag(lines[4], "KeyDist:", 5);
    {
        const auto t = split_ws(lines[5]);
        if (t.empty() || t[0] != "BootstrapSlots:") dev_fail(6, "expected 'BootstrapSlots: { ... }'");
        for (auto& x : dev_braced(t, 1, 6)) {
            const int64_t v = dev_int(x, 6, 1, 1 << 30);
            if (v & (v - 1)) dev_fail(6, "slot count not a power of two: " + x);
            s.boot_slots.push_back((uint32_t)v);
        }
    }
    return s;
}

std::string format_dev_sidecar(const DevSidecar& s) {
    if (s.devices.empty()) throw std::invalid_argument("dev sidecar: no device");
    std::string o = std::to_string(s.devices.size()) + " { ";
    for (auto d : s.devices) o += std::to_string(d) + " ";
    o += "}\nAutoLoadCiphertexts: " + std::to_string(s.auto_load_ciphertexts) + "\n";
    o += "AutoLoadPlaintexts: " + std::to_string(s.auto_load_plaintexts) + "\n";
    o += "RotationIndexes: { ";
    for (auto r : s.rotations) o += std::to_string(r) + " ";
    o += "}\nKeyDist: " + std::to_string(s.key_dist) + "\n";
    o += "BootstrapSlots: { ";
    for (auto b : s.boot_slots) {
        if (b == 0 || (b & (b - 1))) throw std::invalid_argument("dev sidecar: slot count not a power of two");
        o += std::to_string(b) + " ";
    }
    o += "}\n";
    return o;
}

void write_dev_sidecar(const std::string& path, const DevSidecar& s) {
    const std::string text = format_dev_sidecar(s);
    std::ofstream os(path, std::ios::binary | std::ios::trunc);
    if (!os.good()) throw std::invalid_argument("dev sidecar: cannot create " + path);
    os.write(text.data(), (std::streamsize)text.size());
    os.flush();
    if (!os.good()) throw std::invalid_argument("dev sidecar: write failed: " + path);
}

std::vector<KeyLocation> resolve_rotation_keys(const std::vector<int32_t>& rotations,
                                               const std::vector<std::string>& parts) {
    if (parts.empty()) throw std::invalid_argument("rotation keys: no part files");
    uint32_t N = 0;
    std::vector<std::vector<uint32_t>> idx(parts.size());
    for (size_t p = 0; p < parts.size(); p++) {
        const SeededPartHeader h = read_seeded_part_header(parts[p]);
        if (N && h.N != N) throw std::invalid_argument("rotation keys: parts of different ring dimensions");
        N = h.N;
        idx[p] = seeded_part_indices(parts[p]);
    }
    std::vector<KeyLocation> out;
    out.reserve(rotations.size());
    for (int32_t k : rotations) {
        const uint32_t g = rot_index_n(k, N);
        bool found = false;
        for (size_t p = 0; p < parts.size() && !found; p++)
            for (size_t r = 0; r < idx[p].size(); r++)
                if (idx[p][r] == g) {
                    out.push_back(KeyLocation{(uint32_t)p, (uint32_t)r, g});
                    found = true;
                    break;
                }
        if (!found)
            throw std::invalid_argument("rotation keys: no key for rotation " + std::to_string(k) +
                                        " (automorphism index " + std::to_string(g) + ") in the parts");
    }
    return out;
}

void load_rotation_keys(Context& ctx, const std::string& dev_path, const std::vector<std::string>& parts,
                        uint64_t* const* d_evks, uint32_t n_keys) {
    const DevSidecar s = read_dev_sidecar(dev_path);
    if (s.rotations.size() != n_keys)
        throw std::invalid_argument("rotation keys: the sidecar lists " + std::to_string(s.rotations.size()) +
                                    " rotations, " + std::to_string(n_keys) + " key buffers given");
    const std::vector<KeyLocation> loc = resolve_rotation_keys(s.rotations, parts);
    for (uint32_t i = 0; i < n_keys; i++) {
        uint32_t g = 0;
        load_seeded_part_key(ctx, parts[loc[i].part], loc[i].record, &g, d_evks[i]);
        if (g != loc[i].index) throw std::logic_error("rotation keys: record index changed under the loader");
    }
}

}  // namespace fhe
