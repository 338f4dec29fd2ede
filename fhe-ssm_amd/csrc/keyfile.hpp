// keyfile.hpp -- seeded key-switching-key part files and ciphertext files (see keyfile.cpp).
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

#include "engine.hpp"

namespace fhe {

struct SeededPartHeader {
    uint32_t version = 0, expander = 0, N = 0, size_q = 0, size_p = 0, num_part_q = 0, num_per_part_q = 0, count = 0;
    std::string key_tag;
    std::vector<uint64_t> moduli;  // size_q + size_p
    uint64_t header_bytes = 0;     // where the first key record starts
};

// format errors throw std::invalid_argument with the reason
SeededPartHeader read_seeded_part_header(const std::string& path);
std::vector<uint32_t> seeded_part_indices(const std::string& path);
// key `record` of the file into d_evk [dnum][2][L+K][N] (b from the file, a expanded from its seed); the file's
// layout must be ctx's
void load_seeded_part_key(Context& ctx, const std::string& path, uint32_t record, uint32_t* index, uint64_t* d_evk);
// n keys (automorphism indices, 32-byte seeds whose expansion is each key's a-half, device keys) into one part file
void write_seeded_part(Context& ctx, const std::string& path, const std::string& key_tag, uint32_t n,
                       const uint32_t* indices, const uint8_t* seeds, const uint64_t* const* d_evks);

struct CtFileHeader {
    uint32_t N = 0, level = 0, n_polys = 0;
    double scale = 0.0;
    std::vector<uint64_t> moduli;  // level of them
    uint64_t header_bytes = 0;
};

CtFileHeader read_ct_header(const std::string& path);
// a ciphertext [2][level][N] of this context (level <= cap_level) into d_ct
void load_ct(Context& ctx, const std::string& path, uint32_t cap_level, uint64_t* d_ct, uint32_t* level, double* scale);
void save_ct(Context& ctx, const std::string& path, const uint64_t* d_ct, uint32_t level, double scale);

}  // namespace fhe
