// Parameter selection: NTT-friendly primes and roots of unity.
//
// Restates OpenFHE 1.4.2's CKKS-RNS parameter generation as the reference
// uses it (CCParams + GenCryptoContext, FLEXIBLEAUTO scaling, HYBRID key
// switching: native/fideslib_stage0/src/packed_fideslib.cpp:1060-1068,
// src/fhemamba/ckks_probes.py:167-201):
//   * the last Q prime is FirstPrime(scaling bits) (smallest prime >= 2^b,
//     = 1 mod 2N);
//   * going down the chain, primes alternate below / above the running
//     FLEXIBLEAUTO scaling factor sf <- sf^2 / q_{i+1};
//   * q_0 = PreviousPrime(FirstPrime(first-mod bits));
//   * K special primes, K = ceil(max digit bits / 60), descending from
//     FirstPrime(60) and skipping Q primes;
//   * psi = the smallest primitive 2N-th root of unity mod q.
#pragma once

#include <stdint.h>

#include <cmath>
#include <vector>

#include "modarith.hpp"

namespace fhe {

inline bool is_prime(uint64_t n) {
  static const uint64_t bases[12] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return false;
  for (uint64_t b : bases)
    if (n % b == 0) return n == b;
  uint64_t d = n - 1;
  int s = 0;
  while (!(d & 1)) {
    d >>= 1;
    ++s;
  }
  for (uint64_t b : bases) {
    uint64_t x = host_powmod(b, d, n);
    if (x == 1 || x == n - 1) continue;
    bool composite = true;
    for (int r = 1; r < s && composite; ++r) {
      x = host_mulmod(x, x, n);
      if (x == n - 1) composite = false;
    }
    if (composite) return false;
  }
  return true;
}

inline uint64_t first_prime(uint32_t bits, uint64_t m) {
  const uint64_t q = 1ull << bits, r = q % m;
  uint64_t c = q + 1 - r + (r ? m : 0);
  while (!is_prime(c)) c += m;
  return c;
}

inline uint64_t previous_prime(uint64_t q, uint64_t m) {
  uint64_t c = q - m;
  while (!is_prime(c)) c -= m;
  return c;
}

inline uint64_t next_prime(uint64_t q, uint64_t m) {
  uint64_t c = q + m;
  while (!is_prime(c)) c += m;
  return c;
}

inline bool contains(const std::vector<uint64_t>& v, size_t from, uint64_t x) {
  for (size_t i = from; i < v.size(); ++i)
    if (v[i] == x) return true;
  return false;
}

inline uint32_t special_prime_count(const std::vector<uint64_t>& q, uint32_t dnum) {
  const uint32_t nq = (uint32_t)q.size(), alpha = (nq + dnum - 1) / dnum;
  double maxbits = 0;
  for (uint32_t s = 0; s < nq; s += alpha) {
    double bits = 0;
    for (uint32_t i = s; i < s + alpha && i < nq; ++i) bits += std::log2((double)q[i]);
    maxbits = bits > maxbits ? bits : maxbits;
  }
  return (uint32_t)std::ceil(maxbits / 60.0);
}

// Returns the Q chain (depth + 1 primes) and fills p with the special primes.
inline std::vector<uint64_t> gen_moduli(uint32_t log_n, uint32_t depth, uint32_t scale_bits,
                                        uint32_t first_bits, uint32_t dnum,
                                        std::vector<uint64_t>& p) {
  const uint64_t m = 2ull << log_n;
  const uint32_t nq = depth + 1;
  std::vector<uint64_t> q(nq, 0);
  q[nq - 1] = first_prime(scale_bits, m);
  double sf = (double)q[nq - 1];
  uint32_t cnt = 0;
  for (int i = (int)nq - 2; i >= 1; --i, ++cnt) {
    sf = sf * sf / (double)q[i + 1];
    const uint64_t sf_int = (uint64_t)std::llround(sf), sf_rem = sf_int % m;
    uint64_t c;
    if (cnt % 2 == 0) {
      c = sf_int - m - sf_rem + 1;
      do c = previous_prime(c, m);
      while (contains(q, i + 1, c));
    } else {
      c = sf_int + m - sf_rem + 1;
      do c = next_prime(c, m);
      while (contains(q, i + 1, c));
    }
    q[i] = c;
  }
  q[0] = previous_prime(first_prime(first_bits, m), m);
  const uint32_t k = special_prime_count(q, dnum);
  p.clear();
  uint64_t c = first_prime(60, m);
  while (p.size() < k) {
    c = previous_prime(c, m);
    if (!contains(q, 0, c)) p.push_back(c);
  }
  return q;
}

// Smallest primitive m-th root of unity mod q (m a power of two).
inline uint64_t min_root_of_unity(uint64_t m, uint64_t q) {
  uint64_t root = 0;
  for (uint64_t g = 2; g < q; ++g) {
    const uint64_t r = host_powmod(g, (q - 1) / m, q);
    if (host_powmod(r, m / 2, q) == q - 1) {
      root = r;
      break;
    }
  }
  const uint64_t r2 = host_mulmod(root, root, q);
  uint64_t x = root, best = root;
  for (uint64_t t = 1; t < m / 2; ++t) {
    x = host_mulmod(x, r2, q);
    if (x < best) best = x;
  }
  return best;
}

}  // namespace fhe
