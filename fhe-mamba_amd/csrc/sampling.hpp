// Sampling streams for key material and encryption.
//
// Every sample is word i of a stream named by (seed, tag, index): the tag
// says what is drawn (secret, public a, public e, encryption v / e, a
// switching key's a / e, relin / Galois key), the index which limb or
// digit, and the seed which call.  Two stream families exist:
//
// CHACHA20 (the default: secure).  A context holds a 256-bit master key,
// from OS entropy unless the caller supplies one.  ChaCha20 (RFC 8439,
// 20 rounds) is the PRF:
//   call key  K1  = ChaCha20Block(master, counter 0,
//                                 nonce (lo32 seed, hi32 seed, 0)) words 0..7
//   stream        = ChaCha20 keystream under K1, nonce (tag, index, 1)
//   word i        = little-endian 64-bit word i of that keystream
//                   (block i / 8, 32-bit output words 2(i%8), 2(i%8)+1)
// Without the master key, neither a public sample (the public a) nor any
// number of them gives K1, another stream, or the secret-dependent
// samples (s, e, v): that would break ChaCha20 as a PRF.
//
// SEEDED (parity and tests only, NOT secure).  The seed alone fixes every
// sample, so the GPU and an independent restatement draw the same keys:
//   stream key    = fmix64(seed ^ fmix64((tag << 32) ^ index ^ 0x5851F42D4C957F2D))
//   word i        = fmix64(key + (i + 1) * 0x9E3779B97F4A7C15)   (SplitMix64)
// Every step of this chain can be inverted: anyone holding a public key can
// recover the seed from its a, and with it the secret.
//
// Samples from words (both families):
//   uniform mod q  = floor((word(2i) * 2^64 + word(2i+1)) * q / 2^128)
//   ternary        = {0, 1, -1}[word(i) mod 3]
//   sparse ternary = h nonzeros: for i < h, swap position i with position
//                    i + floor(word(2i) (n - i) / 2^64) of 0..n-1 (partial
//                    Fisher-Yates), then that position gets
//                    (word(2i+1) & 1) ? -1 : 1
//   error          = popcount(w & 0x1FFFFF) - popcount((w >> 21) & 0x1FFFFF)
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

// ------------------------------------------------------------- SplitMix64
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

// ------------------------------------------------------------- ChaCha20
FHE_HD uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

#define FHE_CHACHA_QR(a, b, c, d)      \
  a += b; d ^= a; d = rotl32(d, 16);   \
  c += d; b ^= c; b = rotl32(b, 12);   \
  a += b; d ^= a; d = rotl32(d, 8);    \
  c += d; b ^= c; b = rotl32(b, 7);

// RFC 8439 section 2.3: the 16 output words of the block function.
FHE_HD void chacha20_block(const uint32_t key[8], uint32_t counter, const uint32_t nonce[3],
                           uint32_t out[16]) {
  uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                    key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                    counter, nonce[0], nonce[1], nonce[2]};
  uint32_t x[16];
  for (int i = 0; i < 16; ++i) x[i] = s[i];
  for (int r = 0; r < 10; ++r) {
    FHE_CHACHA_QR(x[0], x[4], x[8], x[12])
    FHE_CHACHA_QR(x[1], x[5], x[9], x[13])
    FHE_CHACHA_QR(x[2], x[6], x[10], x[14])
    FHE_CHACHA_QR(x[3], x[7], x[11], x[15])
    FHE_CHACHA_QR(x[0], x[5], x[10], x[15])
    FHE_CHACHA_QR(x[1], x[6], x[11], x[12])
    FHE_CHACHA_QR(x[2], x[7], x[8], x[13])
    FHE_CHACHA_QR(x[3], x[4], x[9], x[14])
  }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}
#undef FHE_CHACHA_QR

// A named stream of either family (plain data: passed to kernels by value).
struct Stream {
  uint32_t secure;     // 1: ChaCha20, 0: SplitMix64
  uint32_t key[8];     // ChaCha20 call key K1
  uint32_t nonce[3];   // (tag, index, 1)
  uint64_t sm_key;     // SplitMix64 stream key
};

// Master key of a context's secure family, or null for the seeded one.
struct SamplingKey {
  bool secure = true;
  uint32_t master[8] = {0, 0, 0, 0, 0, 0, 0, 0};
};

inline Stream make_stream(const SamplingKey& k, uint64_t seed, uint64_t tag, uint64_t index) {
  Stream s{};
  s.secure = k.secure ? 1u : 0u;
  if (!k.secure) {
    s.sm_key = stream_key(seed, tag, index);
    return s;
  }
  const uint32_t n0[3] = {(uint32_t)seed, (uint32_t)(seed >> 32), 0u};
  uint32_t blk[16];
  chacha20_block(k.master, 0u, n0, blk);
  for (int i = 0; i < 8; ++i) s.key[i] = blk[i];
  s.nonce[0] = (uint32_t)tag;
  s.nonce[1] = (uint32_t)index;
  s.nonce[2] = 1u;
  return s;
}

// 64-bit words 8b .. 8b+7 of a secure stream.
FHE_HD void stream_block(const Stream& s, uint32_t b, uint64_t w[8]) {
  uint32_t o[16];
  chacha20_block(s.key, b, s.nonce, o);
  for (int i = 0; i < 8; ++i) w[i] = (uint64_t)o[2 * i] | ((uint64_t)o[2 * i + 1] << 32);
}

FHE_HD uint64_t uniform_from(uint64_t hi, uint64_t lo, uint64_t q) {
  const u128 t = (u128)hi * q + mulhi64(lo, q);
  return (uint64_t)(t >> 64);
}

// Sequential reader of a stream on the host.
class StreamReader {
 public:
  explicit StreamReader(const Stream& s) : s_(s) {}
  uint64_t word(uint64_t i) {
    if (!s_.secure) return draw(s_.sm_key, i);
    const uint64_t b = i >> 3;
    if (b != cached_) {
      stream_block(s_, (uint32_t)b, buf_);
      cached_ = b;
    }
    return buf_[i & 7];
  }

 private:
  Stream s_;
  uint64_t cached_ = ~0ull;
  uint64_t buf_[8];
};

inline void sample_ternary(const Stream& st, int64_t* out, uint32_t n) {
  StreamReader r(st);
  for (uint32_t i = 0; i < n; ++i) {
    const uint64_t d = r.word(i) % 3;
    out[i] = d == 0 ? 0 : (d == 1 ? 1 : -1);
  }
}

// Exactly h nonzero coefficients, each +-1 (1 <= h <= n).
inline void sample_sparse_ternary(const Stream& st, int64_t* out, uint32_t n, uint32_t h) {
  StreamReader r(st);
  uint32_t* idx = new uint32_t[n];
  for (uint32_t i = 0; i < n; ++i) {
    idx[i] = i;
    out[i] = 0;
  }
  for (uint32_t i = 0; i < h; ++i) {
    const uint32_t j = i + (uint32_t)mulhi64(r.word(2 * (uint64_t)i), n - i);
    const uint32_t t = idx[i];
    idx[i] = idx[j];
    idx[j] = t;
    out[idx[i]] = (r.word(2 * (uint64_t)i + 1) & 1) ? -1 : 1;
  }
  delete[] idx;
}

inline void sample_cbd(const Stream& st, int64_t* out, uint32_t n) {
  StreamReader r(st);
  for (uint32_t i = 0; i < n; ++i) {
    const uint64_t d = r.word(i);
    out[i] = (int64_t)__builtin_popcountll(d & 0x1FFFFFull) -
             (int64_t)__builtin_popcountll((d >> 21) & 0x1FFFFFull);
  }
}

}  // namespace fhe
