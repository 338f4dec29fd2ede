// client.hpp -- client-side operations (keygen, encode, encrypt, decrypt); see client.cpp.
#pragma once
#include <stdint.h>

#include <vector>

#include "engine.hpp"

namespace fhe {

struct Secret {
    std::vector<int8_t> coeffs;  // ternary coefficients, length N
    uint64_t* d_eval = nullptr;  // [L+K][N] evaluation form over Q*P
};

void sample_ternary(const uint8_t seed[32], uint32_t h, int8_t* s);
Secret* secret_create(Context& ctx, const uint8_t seed[32], uint32_t h);
void secret_destroy(Secret* sk);
void expand_key_a(Context& ctx, const uint8_t seed[32], uint64_t* d_evk);
void keygen_switch(Context& ctx, const uint64_t* d_s_old, const int8_t* s_new, const uint8_t seed[32],
                   const uint8_t eseed[32], double sigma, uint64_t* d_evk);
void keygen_switch_secret(Context& ctx, const Secret& from, const Secret& to, const uint8_t seed[32],
                          const uint8_t eseed[32], double sigma, uint32_t q_limbs, uint64_t* d_evk);
void keygen_relin(Context& ctx, const Secret& sk, const uint8_t seed[32], const uint8_t eseed[32], double sigma,
                  uint64_t* d_evk);
void keygen_automorphism(Context& ctx, const Secret& sk, uint32_t g, const uint8_t seed[32], const uint8_t eseed[32],
                         double sigma, uint64_t* d_evk);
void encode(Context& ctx, const double* re, const double* im, uint32_t n_slots, uint32_t l, double scale,
            uint64_t* d_pt);
void encode_primes(Context& ctx, const double* re, const double* im, uint32_t n_slots,
                   const std::vector<uint32_t>& pmap, double scale, uint64_t* d_pt);
void encode_periodic(Context& ctx, const double* re, const double* im, uint32_t n_vec, uint32_t P, uint32_t l,
                     double scale, uint64_t* d_out);
void encode_periodic_coeffs(Context& ctx, const double* re, const double* im, uint32_t n_vec, uint32_t P,
                            double scale, int64_t* d_coef, int32_t* d_log_approx);
void expand_periodic(Context& ctx, const int64_t* d_coef, const int32_t* d_log_approx, uint32_t n_vec, uint32_t P,
                     uint32_t l, uint64_t* d_out, hipStream_t st);
void encrypt(Context& ctx, const Secret& sk, const uint64_t* d_pt, uint32_t l, const uint8_t seed[32], uint32_t index,
             uint64_t* d_ct);
void keygen_public(Context& ctx, const Secret& sk, const uint8_t seed[32], const uint8_t eseed[32], double sigma,
                   uint64_t* d_pk);
void encrypt_public(Context& ctx, const uint64_t* d_pk, const uint64_t* d_pt, uint32_t l, const uint8_t seed[32],
                    uint32_t index, uint64_t* d_ct);
void decrypt_coeffs(Context& ctx, const Secret& sk, const uint64_t* d_ct, uint32_t l, double* out);
void decrypt_decode(Context& ctx, const Secret& sk, const uint64_t* d_ct, uint32_t l, double scale, double* re,
                    double* im, uint32_t n_slots);

}  // namespace fhe
