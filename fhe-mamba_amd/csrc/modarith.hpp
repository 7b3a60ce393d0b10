// 64-bit modular arithmetic for primes q < 2^61 on the CDNA4 VALU.
//
// gfx950 issues v_mad_u64_u32 / v_mul_lo_u32 / v_mul_hi_u32 at full rate,
// so every helper here is written to minimise the number of 32-bit
// multiply instructions the compiler has to emit.  Ranges follow Harvey's
// lazy-reduction conventions: most helpers return values in [0, 2q) and the
// callers keep track of the bound (documented at each use).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FHE_HD __host__ __device__ __forceinline__

namespace fhe {

typedef unsigned __int128 u128;

FHE_HD uint64_t mulhi64(uint64_t a, uint64_t b) {
  return (uint64_t)(((u128)a * b) >> 64);
}

// Shoup product with a precomputed companion wp = floor(w * 2^64 / q).
// For any a < 2^64 and w < q the result is a*w mod q plus 0 or q: [0, 2q).
FHE_HD uint64_t shoup_lazy(uint64_t a, uint64_t w, uint64_t wp, uint64_t q) {
  return a * w - mulhi64(a, wp) * q;
}

// Shoup product with an approximate quotient: the low partial product
// a_lo * wp_lo and the carries of the two middle products are dropped, so
// the quotient is low by 0, 1 or 2 and the result a*w mod q plus 0..3 q lies
// in [0, 4q) for any a < 2^64 (three 32x32 multiplies for the quotient
// instead of four and the carry chain).  Needs 4q < 2^64.
FHE_HD uint64_t shoup_lazy4(uint64_t a, uint64_t w, uint64_t wp, uint64_t q) {
  const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32);
  const uint32_t p0 = (uint32_t)wp, p1 = (uint32_t)(wp >> 32);
  const uint64_t qt = (uint64_t)a1 * p1 + (((uint64_t)a0 * p1) >> 32) +
                      (((uint64_t)a1 * p0) >> 32);
  return a * w - qt * q;
}

// shoup_lazy4 with the remainder accumulated against qneg = 2^64 - q:
// a*w - qt*q = a*w + qt*qneg (mod 2^64), which the VALU forms with
// v_mad_u64_u32 accumulations and no borrow chain.  Same quotient, so the
// same value in [0, 4q).
FHE_HD uint64_t shoup_lazy4n(uint64_t a, uint64_t w, uint64_t wp, uint64_t qneg) {
  const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32);
  const uint32_t p0 = (uint32_t)wp, p1 = (uint32_t)(wp >> 32);
  const uint32_t w0 = (uint32_t)w, w1 = (uint32_t)(w >> 32);
  const uint32_t n0 = (uint32_t)qneg, n1 = (uint32_t)(qneg >> 32);
  const uint64_t qt = (uint64_t)a1 * p1 + (((uint64_t)a0 * p1) >> 32) +
                      (((uint64_t)a1 * p0) >> 32);
  const uint32_t t0 = (uint32_t)qt, t1 = (uint32_t)(qt >> 32);
  const uint64_t lo = (uint64_t)t0 * n0 + (uint64_t)a0 * w0;
  const uint32_t hi = (uint32_t)(lo >> 32) + a0 * w1 + a1 * w0 + t0 * n1 + t1 * n0;
  return ((uint64_t)hi << 32) | (uint32_t)lo;
}

// x >= m ? x - m : x for nm = 2^64 - m, m <= 2^63 and x - m < 2^63 when
// x >= m: d = x - m wraps above 2^63 exactly when x < m.
FHE_HD uint64_t lazy_sub(uint64_t x, uint64_t nm) {
  const uint64_t d = x + nm;
  return (int64_t)d < 0 ? x : d;
}

FHE_HD uint64_t reduce_2q(uint64_t x, uint64_t q) { return x >= q ? x - q : x; }

FHE_HD uint64_t reduce_4q(uint64_t x, uint64_t q) {
  x = x >= 2 * q ? x - 2 * q : x;
  return x >= q ? x - q : x;
}

FHE_HD uint64_t reduce_8q(uint64_t x, uint64_t q) {
  x = x >= 4 * q ? x - 4 * q : x;
  x = x >= 2 * q ? x - 2 * q : x;
  return x >= q ? x - q : x;
}

FHE_HD uint64_t shoup(uint64_t a, uint64_t w, uint64_t wp, uint64_t q) {
  return reduce_2q(shoup_lazy(a, w, wp, q), q);
}

FHE_HD uint64_t add_mod(uint64_t a, uint64_t b, uint64_t q) {
  uint64_t s = a + b;
  return s >= q ? s - q : s;
}

FHE_HD uint64_t sub_mod(uint64_t a, uint64_t b, uint64_t q) {
  return a >= b ? a - b : a + q - b;
}

FHE_HD uint64_t neg_mod(uint64_t a, uint64_t q) { return a ? q - a : 0; }

// Montgomery reduction of T = hi*2^64 + lo with T < q * 2^64, qinv_neg =
// -q^-1 mod 2^64.  Returns T * 2^-64 mod q in [0, q).
FHE_HD uint64_t redc(uint64_t hi, uint64_t lo, uint64_t q, uint64_t qinv_neg) {
  const uint64_t m = lo * qinv_neg;
  const uint64_t t = hi + mulhi64(m, q) + (lo != 0);
  return t >= q ? t - q : t;
}

// a * b * 2^-64 mod q for a, b < q (b typically held in Montgomery form,
// so the product comes out in the standard domain).
FHE_HD uint64_t mont_mul(uint64_t a, uint64_t b, uint64_t q, uint64_t qinv_neg) {
  const u128 p = (u128)a * b;
  return redc((uint64_t)(p >> 64), (uint64_t)p, q, qinv_neg);
}

// Montgomery reduction without the final correction: for T = hi*2^64 + lo
// with hi < q and qinv = q^-1 mod 2^64, m = lo * qinv makes T - m q a
// multiple of 2^64 whose low word cancels exactly, so
//   (T - m q) / 2^64 = hi - mulhi64(m, q)  in (-q, q),
// and the result hi + q - mulhi64(m, q) = T * 2^-64 mod q lies in (0, 2q).
FHE_HD uint64_t redc_lazy(uint64_t hi, uint64_t lo, uint64_t q, uint64_t qinv) {
  const uint64_t m = lo * qinv;
  return hi + q - mulhi64(m, q);
}

// x mod q for x < 2^18 q and q in [2^33, 2^61), from the estimate
// e = floor(float(x >> 32) * rq), rq = 2^32 / q (1 - 2^-20) rounded down.
// The float errors (three roundings of 2^-24 each) stay inside the 2^-20
// margin, so e <= floor(x / q); they cost at most 2^18 * 2^-19.9 < 1/4 of a
// quotient unit, and dropping x's low word less than 2^32 / q <= 1/2, so
// e >= floor(x / q) - 1.  Then x - e q lies in [0, 2q): one conditional
// subtraction (qneg = 2^64 - q).
FHE_HD uint64_t reduce_est(uint64_t x, uint64_t qneg, float rq) {
  const uint32_t e = (uint32_t)((float)(uint32_t)(x >> 32) * rq);
  const uint64_t r = x + (uint64_t)e * qneg;
  const uint64_t d = r + qneg;
  return (int64_t)d < 0 ? r : d;
}

// 128-bit accumulator for sums of products that are reduced once.
struct Acc128 {
  uint64_t lo, hi;
  FHE_HD Acc128() : lo(0), hi(0) {}
  FHE_HD void mac(uint64_t a, uint64_t b) {
    const u128 p = (u128)a * b;
    const uint64_t plo = (uint64_t)p;
    lo += plo;
    hi += (uint64_t)(p >> 64) + (lo < plo);
  }
};

// Host-side helpers for table construction.
inline uint64_t host_mulmod(uint64_t a, uint64_t b, uint64_t q) {
  return (uint64_t)(((u128)a * b) % q);
}
inline uint64_t host_powmod(uint64_t a, uint64_t e, uint64_t q) {
  uint64_t r = 1 % q;
  a %= q;
  while (e) {
    if (e & 1) r = host_mulmod(r, a, q);
    a = host_mulmod(a, a, q);
    e >>= 1;
  }
  return r;
}
inline uint64_t host_invmod(uint64_t a, uint64_t q) { return host_powmod(a, q - 2, q); }
inline uint64_t host_shoup(uint64_t w, uint64_t q) { return (uint64_t)(((u128)w << 64) / q); }
// -q^-1 mod 2^64 by Newton iteration (q odd).
inline uint64_t host_qinv_neg(uint64_t q) {
  uint64_t x = q;  // correct to 3 bits
  for (int i = 0; i < 6; ++i) x *= 2 - q * x;
  return ~x + 1;
}
// a * 2^64 mod q (Montgomery form).
inline uint64_t host_to_mont(uint64_t a, uint64_t q) {
  return (uint64_t)(((u128)(a % q) << 64) % q);
}

}  // namespace fhe
