// store.cpp -- the compressed plaintext store file: base file + append journal (host only).
//
// The reference persists its compressed plaintext store with --store-file (hpc_gpu_port/gpu_real_model.cu:1887-2141):
// a base file written once, whole, through PATH.tmp and a rename; later entries appended to PATH.journal as
// self-checksummed records; a stamp naming the configuration the store was built for, refused loudly when it differs;
// an FNV-1a hash over 64-bit words as the checksum, with the reference's offset basis 1469598103934665603 (FNV's
// 14695981039346656037 with its last digit dropped; kept, or no file would match).  This file keeps that format, so that a store written by either
// side is read by the other when the stamps agree:
//   base     "FHESSMSTORE1" + 4 zero bytes | u64 stamp length (1..4096) | stamp | u64 entry count (<= 10^8) |
//            per entry: 7 int32 key fields, u64 word count, the words | u64 FNV of every entry's key fields (each as
//            the u64 of its uint32), word count and words, in file order
//   journal  per record: 7 int32 key fields, u64 word count, the words, u64 FNV of that record's key fields, count
//            and words; a record cut short or failing its hash ends the journal, and the file is truncated there
// Key fields (layer, op, chunk, rowOff, diag, half, lvl).  With a length rule (depth > 0) an entry's lvl must lie in
// [0, depth] and it holds 0 (a dead entry) or (depth + 1 - lvl) comp_cw words: a compressed plaintext's limbs.
#include <sys/statvfs.h>

#include <array>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "fhe_ssm_decode.h"

namespace fhe_ssm_detail {
void set_error(const std::string& m);  // host/decode.cpp
}

namespace {

constexpr uint64_t kFnvBasis = 1469598103934665603ULL, kFnvPrime = 1099511628211ULL;
constexpr uint64_t kMaxEntries = 100000000ULL;
constexpr uint64_t kMaxStamp = 4096;
const char kMagic[16] = {'F', 'H', 'E', 'S', 'S', 'M', 'S', 'T', 'O', 'R', 'E', '1', 0, 0, 0, 0};

using Key = std::array<int32_t, 7>;

struct Fnv {
    uint64_t h = kFnvBasis;
    void mix(uint64_t v) {
        h ^= v;
        h *= kFnvPrime;
    }
    void mix_entry(const Key& k, const std::vector<uint64_t>& w) {
        for (int32_t f : k) mix((uint64_t)(uint32_t)f);
        mix(w.size());
        for (uint64_t x : w) mix(x);
    }
};

struct Rule {
    uint32_t depth, comp_cw;
    // "" when the entry passes, else why not
    std::string check(const Key& k, uint64_t len) const {
        if (depth == 0) return "";
        if (k[6] < 0 || (uint32_t)k[6] > depth) return "entry level out of range";
        const uint64_t want = (uint64_t)(depth + 1 - (uint32_t)k[6]) * comp_cw;
        if (len != 0 && len != want) return "entry length does not match its level";
        return "";
    }
};

struct Fail : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// every entry point: 0, or a CKKS_* code with the message in fhe_ssm_last_error()
template <class F>
int guard(F&& f) {
    try {
        f();
        return CKKS_OK;
    } catch (const std::bad_alloc&) {
        fhe_ssm_detail::set_error("out of host memory");
        return CKKS_ENOMEM;
    } catch (const std::exception& e) {
        fhe_ssm_detail::set_error(e.what());
        return CKKS_EINVAL;
    }
}

// bytes left in a file from the current position (a length field above it is a corrupt file, not an allocation)
uint64_t remaining(std::ifstream& f) {
    const auto pos = f.tellg();
    f.seekg(0, std::ios::end);
    const auto end = f.tellg();
    f.seekg(pos);
    return end > pos ? (uint64_t)(end - pos) : 0;
}

}  // namespace

struct fhe_ssm_store {
    std::map<Key, std::vector<uint64_t>> entries;
};

extern "C" {

int fhe_ssm_store_create(fhe_ssm_store** st) {
    return guard([&] {
        if (!st) throw Fail("null store pointer");
        *st = new fhe_ssm_store();
    });
}

void fhe_ssm_store_destroy(fhe_ssm_store* st) { delete st; }

int fhe_ssm_store_put(fhe_ssm_store* st, const int32_t* key, const uint64_t* words, uint64_t n_words) {
    return guard([&] {
        if (!st || !key || (n_words && !words)) throw Fail("null argument");
        Key k;
        std::memcpy(k.data(), key, sizeof k);
        if (!st->entries.emplace(k, std::vector<uint64_t>(words, words + n_words)).second)
            throw Fail("duplicate entry key");
    });
}

int fhe_ssm_store_count(const fhe_ssm_store* st, uint64_t* n) {
    return guard([&] {
        if (!st || !n) throw Fail("null argument");
        *n = st->entries.size();
    });
}

int fhe_ssm_store_entry(const fhe_ssm_store* st, uint64_t i, int32_t* key, uint64_t* n_words) {
    return guard([&] {
        if (!st || !key || !n_words) throw Fail("null argument");
        if (i >= st->entries.size()) throw Fail("entry index out of range");
        auto it = st->entries.begin();
        std::advance(it, (long)i);
        std::memcpy(key, it->first.data(), sizeof(Key));
        *n_words = it->second.size();
    });
}

int fhe_ssm_store_get(const fhe_ssm_store* st, const int32_t* key, uint64_t* words, uint64_t cap, uint64_t* n_words) {
    return guard([&] {
        if (!st || !key || !n_words) throw Fail("null argument");
        Key k;
        std::memcpy(k.data(), key, sizeof k);
        auto it = st->entries.find(k);
        if (it == st->entries.end()) throw Fail("no entry with that key");
        *n_words = it->second.size();
        if (words) {
            if (cap < it->second.size()) throw Fail("buffer too small for the entry");
            std::memcpy(words, it->second.data(), it->second.size() * 8);
        }
    });
}

int fhe_ssm_store_save(const fhe_ssm_store* st, const char* path, const char* stamp) {
    return guard([&] {
        if (!st || !path || !stamp) throw Fail("null argument");
        const uint64_t sl = std::strlen(stamp);
        if (sl == 0 || sl > kMaxStamp) throw Fail("stamp length must be 1..4096");
        uint64_t need = 16 + 8 + sl + 8 + 8;
        for (const auto& kv : st->entries) need += 28 + 8 + kv.second.size() * 8;
        const std::string dir = std::filesystem::path(path).parent_path().string();
        struct statvfs sv;
        if (statvfs(dir.empty() ? "." : dir.c_str(), &sv) == 0 &&
            (uint64_t)sv.f_bavail * (uint64_t)sv.f_frsize < need)
            throw Fail("store file: not enough free space for " + std::to_string(need) + " bytes");
        const std::string tmp = std::string(path) + ".tmp";
        {
            std::ofstream f(tmp, std::ios::binary | std::ios::trunc);
            if (!f) throw Fail("store file: cannot write " + tmp);
            Fnv h;
            f.write(kMagic, 16);
            f.write((const char*)&sl, 8);
            f.write(stamp, (std::streamsize)sl);
            const uint64_t n = st->entries.size();
            f.write((const char*)&n, 8);
            for (const auto& kv : st->entries) {
                const uint64_t len = kv.second.size();
                f.write((const char*)kv.first.data(), sizeof(Key));
                f.write((const char*)&len, 8);
                if (len) f.write((const char*)kv.second.data(), (std::streamsize)(len * 8));
                h.mix_entry(kv.first, kv.second);
            }
            f.write((const char*)&h.h, 8);
            f.close();
            if (!f) {
                std::remove(tmp.c_str());
                throw Fail("store file: write failed on " + tmp);
            }
        }
        if (std::rename(tmp.c_str(), path) != 0) {
            std::remove(tmp.c_str());
            throw Fail(std::string("store file: rename failed ") + tmp + " -> " + path);
        }
    });
}

int fhe_ssm_store_load(fhe_ssm_store* st, const char* path, const char* stamp, uint32_t depth, uint32_t comp_cw,
                       uint64_t* n_loaded) {
    return guard([&] {
        if (!st || !path) throw Fail("null argument");
        if (depth && !comp_cw) throw Fail("a length rule needs comp_cw");
        std::ifstream f(path, std::ios::binary);
        if (!f) throw Fail(std::string("store file: cannot open ") + path);
        const Rule rule{depth, comp_cw};
        char magic[16];
        f.read(magic, 16);
        if (!f || std::memcmp(magic, kMagic, 12) != 0) throw Fail("store file: bad magic");
        uint64_t sl = 0;
        f.read((char*)&sl, 8);
        if (!f || sl == 0 || sl > kMaxStamp) throw Fail("store file: bad stamp length");
        std::string fstamp(sl, '\0');
        f.read(&fstamp[0], (std::streamsize)sl);
        if (!f) throw Fail("store file: truncated stamp");
        if (stamp && fstamp != stamp)
            throw Fail("store file: built for a different configuration (file stamp \"" + fstamp +
                       "\", this run's \"" + stamp + "\")");
        uint64_t n = 0;
        f.read((char*)&n, 8);
        if (!f || n > kMaxEntries) throw Fail("store file: bad entry count");
        Fnv h;
        std::map<Key, std::vector<uint64_t>> got;
        for (uint64_t i = 0; i < n; i++) {
            Key k;
            uint64_t len = 0;
            f.read((char*)k.data(), sizeof k);
            f.read((char*)&len, 8);
            if (!f) throw Fail("store file: truncated entry header");
            const std::string why = rule.check(k, len);
            if (!why.empty()) throw Fail("store file: " + why);
            if (len > remaining(f) / 8) throw Fail("store file: truncated entry data");
            std::vector<uint64_t> w(len);
            if (len) f.read((char*)w.data(), (std::streamsize)(len * 8));
            if (!f) throw Fail("store file: truncated entry data");
            h.mix_entry(k, w);
            if (st->entries.count(k) || !got.emplace(k, std::move(w)).second)
                throw Fail("store file: duplicate entry key");
        }
        uint64_t file_hash = 0;
        f.read((char*)&file_hash, 8);
        if (!f || file_hash != h.h) throw Fail("store file: checksum mismatch");
        for (auto& kv : got) st->entries.emplace(kv.first, std::move(kv.second));
        if (n_loaded) *n_loaded = n;
    });
}

int fhe_ssm_store_read_stamp(const char* path, char* stamp, uint64_t cap, uint64_t* len) {
    return guard([&] {
        if (!path || !len) throw Fail("null argument");
        std::ifstream f(path, std::ios::binary);
        if (!f) throw Fail(std::string("store file: cannot open ") + path);
        char magic[16];
        f.read(magic, 16);
        if (!f || std::memcmp(magic, kMagic, 12) != 0) throw Fail("store file: bad magic");
        uint64_t sl = 0;
        f.read((char*)&sl, 8);
        if (!f || sl == 0 || sl > kMaxStamp) throw Fail("store file: bad stamp length");
        std::string s(sl, '\0');
        f.read(&s[0], (std::streamsize)sl);
        if (!f) throw Fail("store file: truncated stamp");
        *len = sl;
        if (stamp) {
            if (cap < sl + 1) throw Fail("buffer too small for the stamp");
            std::memcpy(stamp, s.data(), sl);
            stamp[sl] = 0;
        }
    });
}

int fhe_ssm_store_append(const char* journal_path, const int32_t* key, const uint64_t* words, uint64_t n_words) {
    return guard([&] {
        if (!journal_path || !key || (n_words && !words)) throw Fail("null argument");
        Key k;
        std::memcpy(k.data(), key, sizeof k);
        std::vector<uint64_t> w(words, words + n_words);
        Fnv h;
        h.mix_entry(k, w);
        std::ofstream f(journal_path, std::ios::binary | std::ios::app);
        if (!f) throw Fail(std::string("store journal: cannot append to ") + journal_path);
        f.write((const char*)k.data(), sizeof k);
        f.write((const char*)&n_words, 8);
        if (n_words) f.write((const char*)w.data(), (std::streamsize)(n_words * 8));
        f.write((const char*)&h.h, 8);
        f.close();
        if (!f) throw Fail(std::string("store journal: append failed on ") + journal_path);
    });
}

int fhe_ssm_store_load_journal(fhe_ssm_store* st, const char* journal_path, uint32_t depth, uint32_t comp_cw,
                               uint64_t* good, uint64_t* duplicates, uint64_t* dropped_bytes) {
    return guard([&] {
        if (!st || !journal_path) throw Fail("null argument");
        if (depth && !comp_cw) throw Fail("a length rule needs comp_cw");
        uint64_t n_good = 0, n_dup = 0, dropped = 0;
        std::ifstream f(journal_path, std::ios::binary);
        if (f) {
            const Rule rule{depth, comp_cw};
            std::streamoff good_end = 0;
            for (;;) {
                Key k;
                uint64_t len = 0, rh = 0;
                f.read((char*)k.data(), sizeof k);
                if (!f) break;
                f.read((char*)&len, 8);
                if (!f || !rule.check(k, len).empty() || len > remaining(f) / 8) break;
                std::vector<uint64_t> w(len);
                if (len) f.read((char*)w.data(), (std::streamsize)(len * 8));
                if (!f) break;
                f.read((char*)&rh, 8);
                if (!f) break;
                Fnv h;
                h.mix_entry(k, w);
                if (rh != h.h) break;
                good_end = f.tellg();
                if (st->entries.emplace(k, std::move(w)).second)
                    n_good++;
                else
                    n_dup++;
            }
            f.close();
            std::error_code ec;
            const auto total = std::filesystem::file_size(journal_path, ec);
            if (!ec && (std::streamoff)total != good_end) {
                // a torn tail (a process killed mid-append): keep the good prefix, drop the rest
                dropped = (uint64_t)((std::streamoff)total - good_end);
                std::filesystem::resize_file(journal_path, (uintmax_t)good_end, ec);
                if (ec) throw Fail(std::string("store journal: cannot truncate the torn tail of ") + journal_path);
            }
        }
        if (good) *good = n_good;
        if (duplicates) *duplicates = n_dup;
        if (dropped_bytes) *dropped_bytes = dropped;
    });
}

}  // extern "C"
