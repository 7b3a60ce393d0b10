// Deterministic, counter-based sampling streams for key material.
//
// The reference samples keys with OpenFHE's PRNG, which cannot be
// reproduced offline, so keys are treated as inputs for parity.  This build
// defines its own seeded streams so that the same seed gives the same keys
// on the GPU and in any independent restatement:
//   draw(key, i)   = fmix64(key + (i + 1) * 0x9E3779B97F4A7C15)   (SplitMix64)
//   stream(s,t,i)  = fmix64(s ^ fmix64((t << 32) ^ i ^ 0x5851F42D4C957F2D))
//   uniform mod q  = floor((draw(2i) * 2^64 + draw(2i+1)) * q / 2^128)
//   ternary        = {0, 1, -1}[draw(i) mod 3]
//   sparse ternary = h nonzeros: for i < h, swap position i with position
//                    i + floor(draw(2i) (n - i) / 2^64) of 0..n-1 (partial
//                    Fisher-Yates), then that position gets
//                    (draw(2i+1) & 1) ? -1 : 1
//   error          = popcount(d & 0x1FFFFF) - popcount((d >> 21) & 0x1FFFFF)
//                    (centred binomial, eta = 21, sigma ~ 3.24, in place of
//                    OpenFHE's discrete Gaussian with sigma 3.19)
#pragma once

#include <stdint.h>

#include "modarith.hpp"

namespace fhe {

enum SampleTag : uint64_t {
  TAG_SECRET = 1,
  TAG_PK_A = 2,
  TAG_PK_E = 3,
  TAG_ENC_V = 4,
  TAG_ENC_E = 5,
  TAG_KSK_A = 6,
  TAG_KSK_E = 7,
  TAG_RELIN = 0x100000,
  TAG_GALOIS = 0x200000
};

FHE_HD uint64_t fmix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

FHE_HD uint64_t draw(uint64_t key, uint64_t ctr) {
  return fmix64(key + (ctr + 1) * 0x9E3779B97F4A7C15ull);
}

FHE_HD uint64_t stream_key(uint64_t seed, uint64_t tag, uint64_t index) {
  return fmix64(seed ^ fmix64((tag << 32) ^ index ^ 0x5851F42D4C957F2Dull));
}

FHE_HD uint64_t uniform_mod(uint64_t key, uint64_t i, uint64_t q) {
  const uint64_t hi = draw(key, 2 * i), lo = draw(key, 2 * i + 1);
  const u128 t = (u128)hi * q + mulhi64(lo, q);
  return (uint64_t)(t >> 64);
}

inline void sample_ternary(uint64_t key, int64_t* out, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) {
    const uint64_t d = draw(key, i) % 3;
    out[i] = d == 0 ? 0 : (d == 1 ? 1 : -1);
  }
}

// Exactly h nonzero coefficients, each +-1 (1 <= h <= n).
inline void sample_sparse_ternary(uint64_t key, int64_t* out, uint32_t n, uint32_t h) {
  uint32_t* idx = new uint32_t[n];
  for (uint32_t i = 0; i < n; ++i) {
    idx[i] = i;
    out[i] = 0;
  }
  for (uint32_t i = 0; i < h; ++i) {
    const uint32_t j = i + (uint32_t)mulhi64(draw(key, 2 * (uint64_t)i), n - i);
    const uint32_t t = idx[i];
    idx[i] = idx[j];
    idx[j] = t;
    out[idx[i]] = (draw(key, 2 * (uint64_t)i + 1) & 1) ? -1 : 1;
  }
  delete[] idx;
}

inline void sample_cbd(uint64_t key, int64_t* out, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) {
    const uint64_t d = draw(key, i);
    out[i] = (int64_t)__builtin_popcountll(d & 0x1FFFFFull) -
             (int64_t)__builtin_popcountll((d >> 21) & 0x1FFFFFull);
  }
}

}  // namespace fhe
