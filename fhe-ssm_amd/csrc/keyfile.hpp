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

// The FIDESlib ".dev" sidecar of a serialized context, cryptocontext.bin.dev: a six-line text file the reference
// client writes next to cryptocontext.bin (writeDevSidecar, hpc_gpu_port/mac_fhe_client.cpp:178-194) and FIDESlib's
// LoadContext reads: the device list, the auto-load flags, the rotation AMOUNTS whose keys go to the device, the
// secret-key distribution and the slot counts bootstrapping is set up for.
struct DevSidecar {
    std::vector<uint32_t> devices{0};
    int32_t auto_load_ciphertexts = 1, auto_load_plaintexts = 0, key_dist = 1;
    std::vector<int32_t> rotations;   // EvalRotate steps, in file order
    std::vector<uint32_t> boot_slots;
};
// strict: every line, its key, its braces and its integers as the writer puts them (format errors throw
// std::invalid_argument with the line and the reason)
DevSidecar read_dev_sidecar(const std::string& path);
std::string format_dev_sidecar(const DevSidecar& s);
void write_dev_sidecar(const std::string& path, const DevSidecar& s);

// where the key of each rotation of a sidecar lies among seeded part files: rotation k needs the automorphism index
// 5^k mod 2N (negative k through the order N/2 of 5; N of the parts, which must agree), looked up in the parts in
// the given order (the first record with that index)
struct KeyLocation {
    uint32_t part, record, index;
};
std::vector<KeyLocation> resolve_rotation_keys(const std::vector<int32_t>& rotations,
                                               const std::vector<std::string>& parts);
// LoadContext's rotation keys: the key of every rotation the sidecar lists, from the parts, into d_evks[i]
void load_rotation_keys(Context& ctx, const std::string& dev_path, const std::vector<std::string>& parts,
                        uint64_t* const* d_evks, uint32_t n_keys);

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
