// Hybrid (dnum) key switching: ModUp, key inner product, ModDown.
//
// Follows OpenFHE's KeySwitchHYBRID, which is what FIDESlib's
// DecompAndModUpConv / hoistedRotateDotKSK / modDown kernels compute for the
// reference (profiler names in results/b300/2026-09-28/long-generation/
// profiling/ncu-{modup,keyswitch}/counters.json):
//   ModUp     digit j = limbs [j*alpha, min((j+1)*alpha, nq)) of the input is
//             taken to coefficient form and fast-converted (no correction
//             term) to the complement of the digit in Q_l plus P, then NTT'd;
//             the digit's own limbs keep their evaluation-form values.
//   inner     ext_b[i] = sum_j digit_j[i] * key_j,b[i'] over Q_l + P, with i'
//             the key limb of the same modulus.
//   ModDown   out_b = (ext_b[Q] - NTT(Conv_{P->Q}(iNTT(ext_b[P])))) * P^-1.
// Rotation adds c0 and applies the Galois permutation in the same pass as
// the ModDown subtraction.
//
// Basis conversion uses Montgomery-form constants: y_k = REDC(sum_i v_i *
// [Qhat_i * 2^64]_{t_k}), one reduction per output word.  That needs the sum
// to stay below t_k * 2^64, i.e. (terms per REDC) * max source modulus <
// 2^64; the kernel reduces in chunks of `chunk` terms chosen on the host.
#include <algorithm>
#include <vector>

#include "ops.hpp"

namespace fhe {
namespace {

constexpr int TPB = 256;
constexpr int MAXSRC = 16;

inline uint32_t tpb_for(const Context& c, uint32_t per_thread) {
  const uint32_t t = c.n / per_thread;
  return t < TPB ? t : TPB;
}

// Fast basis conversion of coefficient-form limbs.
//   src:   [npoly] x (nsrc limbs of N words), poly stride src_ps
//   out:   [npoly] x positions, poly stride out_ps; target k goes to limb
//          position pos(k) = dst < L ? dst : out_nq + (dst - L)
// grid (N / blockDim, 1, npoly); one coefficient per thread.
__global__ void __launch_bounds__(TPB)
    k_convert(const uint64_t* __restrict__ src, size_t src_ps, uint64_t* __restrict__ out,
              size_t out_ps, const ModConst* __restrict__ mc, const uint32_t* __restrict__ src_idx,
              const uint64_t* __restrict__ qhat_inv, const uint64_t* __restrict__ qhat_mont,
              const uint32_t* __restrict__ dst_idx, uint32_t nsrc, uint32_t ndst, uint32_t n,
              uint32_t L, uint32_t out_nq, uint32_t chunk) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t* s = src + (size_t)blockIdx.z * src_ps;
  uint64_t* o = out + (size_t)blockIdx.z * out_ps;
  uint64_t v[MAXSRC];
#pragma unroll
  for (int i = 0; i < MAXSRC; ++i) {
    if (i < (int)nsrc) {
      const uint64_t q = mc[src_idx[i]].q;
      v[i] = shoup(s[(size_t)i * n + e], qhat_inv[2 * i], qhat_inv[2 * i + 1], q);
    }
  }
  for (uint32_t k = 0; k < ndst; ++k) {
    const uint32_t dm = dst_idx[k];
    const uint64_t t = mc[dm].q, tinv = mc[dm].qinv_neg;
    uint64_t res = 0;
    uint32_t i0 = 0;
    while (i0 < nsrc) {
      const uint32_t i1 = i0 + chunk < nsrc ? i0 + chunk : nsrc;
      Acc128 acc;
#pragma unroll
      for (int i = 0; i < MAXSRC; ++i)
        if (i >= (int)i0 && i < (int)i1) acc.mac(v[i], qhat_mont[(size_t)i * ndst + k]);
      res = add_mod(res, redc(acc.hi, acc.lo, t, tinv), t);
      i0 = i1;
    }
    const uint32_t pos = dm < L ? dm : out_nq + (dm - L);
    o[(size_t)pos * n + e] = res;
  }
}

// Fast basis conversion, specialised for NSRC source limbs and moduli below
// 2^60.  Operands are split at bit 30 (v = vh 2^30 + vl, c = ch 2^30 + cl,
// all halves < 2^30), so each 60x60-bit product is four 32x32->64 partial
// products accumulated with v_mad_u64_u32 and no carries: for NSRC <= 16
// every partial sum stays below 2^64.  The 128-bit total
//   T = A0 + (A1a + A1b) 2^30 + A2 2^60 < NSRC * 2^60 * t_k <= t_k * 2^64
// is reduced by one REDC against the Montgomery-form constants.
// grid (N / blockDim, ceil(ndst / tch), npoly): each thread converts one
// coefficient for `tch` consecutive targets.
template <int NSRC>
__device__ __forceinline__ void convert60_body(
    const uint64_t* __restrict__ s, uint64_t* __restrict__ o, const ModConst* __restrict__ mc,
    const uint32_t* __restrict__ src_idx, const uint64_t* __restrict__ qhat_inv,
    const uint64_t* __restrict__ qhat_mont, const uint32_t* __restrict__ dst_idx, uint32_t ndst,
    uint32_t n, uint32_t L, uint32_t out_nq, uint32_t tch) {
  constexpr uint32_t M30 = (1u << 30) - 1;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t vl[NSRC], vh[NSRC];
#pragma unroll
  for (int i = 0; i < NSRC; ++i) {
    const uint64_t q = mc[src_idx[i]].q;
    const uint64_t v = shoup(s[(size_t)i * n + e], qhat_inv[2 * i], qhat_inv[2 * i + 1], q);
    vl[i] = (uint32_t)v & M30;
    vh[i] = (uint32_t)(v >> 30);
  }
  const uint32_t k0 = blockIdx.y * tch, k1 = k0 + tch < ndst ? k0 + tch : ndst;
  for (uint32_t k = k0; k < k1; ++k) {
    uint64_t a0 = 0, a1a = 0, a1b = 0, a2 = 0;
#pragma unroll
    for (int i = 0; i < NSRC; ++i) {
      const uint64_t c = qhat_mont[(size_t)i * ndst + k];
      const uint32_t cl = (uint32_t)c & M30, ch = (uint32_t)(c >> 30);
      a0 += (uint64_t)vl[i] * cl;
      a1a += (uint64_t)vl[i] * ch;
      a1b += (uint64_t)vh[i] * cl;
      a2 += (uint64_t)vh[i] * ch;
    }
    const uint64_t s1 = a1a + a1b;
    const uint64_t c1 = s1 < a1a;
    const uint64_t m1 = s1 << 30, m2 = a2 << 60;
    uint64_t lo = a0 + m1;
    uint64_t hi = (s1 >> 34) + (c1 << 30) + (a2 >> 4) + (lo < m1);
    const uint64_t lo2 = lo + m2;
    hi += lo2 < m2;
    lo = lo2;
    const uint32_t dm = dst_idx[k];
    const uint32_t pos = dm < L ? dm : out_nq + (dm - L);
    o[(size_t)pos * n + e] = redc(hi, lo, mc[dm].q, mc[dm].qinv_neg);
  }
}

// grid (N / blockDim, ceil(ndst / tch), npoly): each thread converts one
// coefficient of poly blockIdx.z for `tch` consecutive targets.
template <int NSRC>
__global__ void __launch_bounds__(TPB)
    k_convert60(const uint64_t* __restrict__ src, size_t src_ps, uint64_t* __restrict__ out,
                size_t out_ps, const ModConst* __restrict__ mc,
                const uint32_t* __restrict__ src_idx, const uint64_t* __restrict__ qhat_inv,
                const uint64_t* __restrict__ qhat_mont, const uint32_t* __restrict__ dst_idx,
                uint32_t ndst, uint32_t n, uint32_t L, uint32_t out_nq, uint32_t tch) {
  convert60_body<NSRC>(src + (size_t)blockIdx.z * src_ps, out + (size_t)blockIdx.z * out_ps, mc,
                       src_idx, qhat_inv, qhat_mont, dst_idx, ndst, n, L, out_nq, tch);
}

// ModUp conversion of several digits of several ciphertexts in one launch:
// blockIdx.z = ciphertext * ndig + digit d; digit d converts its limbs
// coef[ct][src_limb[d] ..) with its own plan into digits[ct][d].
constexpr int MAXD = 8;
struct DigitPlans {
  const uint32_t* src_idx[MAXD];
  const uint64_t* qhat_inv[MAXD];
  const uint64_t* qhat_mont[MAXD];
  const uint32_t* dst_idx[MAXD];
  uint32_t ndst[MAXD];
  uint32_t src_limb[MAXD];
};

template <int NSRC>
__global__ void __launch_bounds__(TPB)
    k_convert60_digits(const uint64_t* __restrict__ coef, uint64_t* __restrict__ digits,
                       size_t digit_words, const ModConst* __restrict__ mc, const DigitPlans P,
                       uint32_t n, uint32_t L, uint32_t nq, uint32_t tch, uint32_t ndig,
                       uint32_t nd) {
  const uint32_t ct = blockIdx.z / ndig, d = blockIdx.z % ndig;
  if (blockIdx.y * tch >= P.ndst[d]) return;
  convert60_body<NSRC>(coef + ((size_t)ct * nq + P.src_limb[d]) * n,
                       digits + ((size_t)ct * nd + d) * digit_words, mc, P.src_idx[d],
                       P.qhat_inv[d], P.qhat_mont[d], P.dst_idx[d], P.ndst[d], n, L, nq, tch);
}

// The key inner product has no kernel of its own: its P limbs feed the
// first pass of ModDown's inverse NTT and its Q limbs the last pass of the
// forward NTT (ntt.hip, KskLoad / EpiStore).  Up to MAXD digits.

__device__ __forceinline__ uint32_t brev_bits(uint32_t x, uint32_t bits) {
  return __brev(x) >> (32 - bits);
}

// Galois permutation of evaluation-form limbs (no key switching).
// grid (N / blockDim, nlimb, npoly).
__global__ void __launch_bounds__(TPB)
    k_automorph(uint64_t* __restrict__ out, const uint64_t* __restrict__ in, uint32_t n,
                uint32_t log_n, uint32_t nlimb, uint32_t galois) {
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t j = brev_bits(x, log_n);
  const uint32_t ex = (uint32_t)(((2ull * j + 1) * galois) & (2 * n - 1));
  const uint32_t s = brev_bits((ex - 1) >> 1, log_n);
  const size_t base = ((size_t)blockIdx.z * nlimb + blockIdx.y) * n;
  out[base + x] = in[base + s];
}

// Key words to Montgomery form: k * 2^64 mod q = REDC(k * (2^128 mod q)).
// grid (N / blockDim, L + K, dnum * 2).
__global__ void __launch_bounds__(TPB)
    k_to_mont(uint64_t* key, const ModConst* mc, const uint64_t* fac, uint32_t n, uint32_t nm) {
  const uint32_t i = blockIdx.y;
  const ModConst m = mc[i];
  const size_t o = ((size_t)blockIdx.z * nm + i) * n + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  key[o] = mont_mul(key[o], fac[i], m.q, m.qinv_neg);
}

// Device key -> standard form (the inverse of k_to_mont), into `out`.
__global__ void __launch_bounds__(TPB)
    k_from_mont(uint64_t* out, const uint64_t* key, const ModConst* mc, const uint64_t* fac,
                uint32_t n, uint32_t nm) {
  const uint32_t i = blockIdx.y;
  const ModConst m = mc[i];
  const size_t o = ((size_t)blockIdx.z * nm + i) * n + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  out[o] = mont_mul(key[o], fac[i], m.q, m.qinv_neg);
}

// Terms per REDC so that terms * max_q < 2^64.
uint32_t redc_chunk(const Context& c, const std::vector<uint32_t>& idx) {
  uint64_t mx = 1;
  for (uint32_t i : idx) mx = c.mods[i] > mx ? c.mods[i] : mx;
  uint64_t ch = ~0ull / mx;
  if (ch > MAXSRC) ch = MAXSRC;
  return (uint32_t)(ch < 1 ? 1 : ch);
}

bool below_2_60(const Context& c, const std::vector<uint32_t>& idx) {
  for (uint32_t i : idx)
    if (c.mods[i] >= (1ull << 60)) return false;
  return true;
}

// Targets per thread: as many as possible (each thread's source words and
// their Shoup products are reused for every target it covers) while the
// launch still has >= 4096 workgroups; at least 4.
inline uint32_t convert_tch(const Context& c, uint32_t ndst, uint32_t npoly) {
  const uint64_t per = (uint64_t)(c.n / tpb_for(c, 1)) * npoly;
  uint32_t tch = ndst;
  while (tch > 4 && per * ((ndst + tch - 1) / tch) < 4096) tch = (tch + 1) / 2;
  return tch < 4 ? 4 : tch;
}

template <int NSRC>
void launch_convert60(Context& c, const ConvPlan& pl, const uint64_t* src, size_t src_ps,
                      uint64_t* out, size_t out_ps, uint32_t out_nq, uint32_t npoly) {
  const uint32_t tpb = tpb_for(c, 1), tch = convert_tch(c, pl.ndst, npoly);
  FHE_LAUNCH(c, "k_convert", k_convert60<NSRC>, dim3(c.n / tpb, (pl.ndst + tch - 1) / tch, npoly),
             dim3(tpb), 0, src, src_ps, out, out_ps, c.d_const, pl.d_src_idx32, pl.d_qhat_inv,
             pl.d_qhat_mont, pl.d_dst_idx, pl.ndst, c.n, c.L, out_nq, tch);
}

void convert(Context& c, const ConvPlan& pl, const uint64_t* src, size_t src_ps, uint64_t* out,
             size_t out_ps, uint32_t out_nq, uint32_t npoly) {
  if (pl.nsrc > MAXSRC) throw ArgError("basis conversion source larger than 16 limbs");
  if (below_2_60(c, pl.src_idx) && below_2_60(c, pl.dst_idx)) {
    switch (pl.nsrc) {
#define CASE(S) \
  case S: launch_convert60<S>(c, pl, src, src_ps, out, out_ps, out_nq, npoly); return;
      CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
      CASE(9) CASE(10) CASE(11) CASE(12) CASE(13) CASE(14) CASE(15) CASE(16)
#undef CASE
      default: break;
    }
  }
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_convert", k_convert, dim3(c.n / tpb, 1, npoly), dim3(tpb), 0, src, src_ps, out, out_ps, c.d_const, pl.d_src_idx32, pl.d_qhat_inv, pl.d_qhat_mont, pl.d_dst_idx, pl.nsrc, pl.ndst, c.n, c.L, out_nq, redc_chunk(c, pl.src_idx));
}

}  // namespace

uint32_t num_digits(const Context& c, uint32_t nq) {
  const uint32_t d = (nq + c.alpha - 1) / c.alpha;
  return d < c.dnum ? d : c.dnum;
}

void modup(Context& c, const uint64_t* a, uint32_t nq, uint64_t* digits) {
  modup_batch(c, &a, 1, nq, digits);
}

void modup_batch(Context& c, const uint64_t* const* as, uint32_t count, uint32_t nq,
                 uint64_t* digits) {
  if (nq == 0 || nq > c.L) throw ArgError("modup: bad level");
  if (count == 0) return;
  if (modup_fused_ok(c, nq, count)) {
    modup_fused(c, as, count, nq, digits);
    return;
  }
  const size_t n = c.n, ne = nq + c.K, pl = (size_t)nq * n;
  const uint32_t nd = num_digits(c, nq);
  const size_t ct_words = (size_t)nd * ne * n;
  Scratch coef(c, count * pl);
  for (uint32_t i = 0; i < count; ++i)
    hip_check(hipMemcpyAsync(coef.p + i * pl, as[i], pl * 8, hipMemcpyDeviceToDevice, c.stream),
              "modup copy");
  ntt_inverse(c, coef.p, count, pl, nq, LimbMap::contiguous(0));
  if (nd > MAXD) throw ArgError("more than 8 key-switching digits");
  // Conversions: the full-width digits in one launch when the 30-bit split
  // applies, any other digit on its own.
  std::vector<const ConvPlan*> plans(nd);
  for (uint32_t j = 0; j < nd; ++j) {
    const uint32_t s = j * c.alpha, e = s + c.alpha < nq ? s + c.alpha : nq;
    plans[j] = &c.modup_plan(s, e, nq);
  }
  uint32_t batched = 0;
  if (c.alpha <= MAXSRC) {
    while (batched < nd && plans[batched]->nsrc == c.alpha &&
           below_2_60(c, plans[batched]->src_idx) && below_2_60(c, plans[batched]->dst_idx))
      ++batched;
  }
  if (batched > 1) {
    DigitPlans P{};
    uint32_t ndst = 0;
    for (uint32_t j = 0; j < batched; ++j) {
      P.src_idx[j] = plans[j]->d_src_idx32;
      P.qhat_inv[j] = plans[j]->d_qhat_inv;
      P.qhat_mont[j] = plans[j]->d_qhat_mont;
      P.dst_idx[j] = plans[j]->d_dst_idx;
      P.ndst[j] = plans[j]->ndst;
      P.src_limb[j] = j * c.alpha;
      ndst = std::max(ndst, plans[j]->ndst);
    }
    const uint32_t tpb = tpb_for(c, 1), tch = convert_tch(c, ndst, batched * count);
    const dim3 grid(c.n / tpb, (ndst + tch - 1) / tch, batched * count);
    switch (c.alpha) {
#define CASE(S)                                                                                \
  case S:                                                                                      \
    FHE_LAUNCH(c, "k_convert", k_convert60_digits<S>, grid, dim3(tpb), 0, coef.p, digits,     \
               ne * n, c.d_const, P, c.n, c.L, nq, tch, batched, nd);                          \
    break;
      CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
      CASE(9) CASE(10) CASE(11) CASE(12) CASE(13) CASE(14) CASE(15) CASE(16)
#undef CASE
      default: throw ArgError("digit width above 16 limbs");
    }
  } else {
    batched = 0;
  }
  for (uint32_t j = batched; j < nd; ++j)
    convert(c, *plans[j], coef.p + (size_t)j * c.alpha * n, pl, digits + (size_t)j * ne * n,
            ct_words, nq, count);
  // Forward NTT of every digit's converted limbs in one two-pass launch,
  // then each digit's own limbs copied in evaluation form.
  ntt_forward_digits(c, digits, count, nd, nq);
  for (uint32_t i = 0; i < count; ++i)
    for (uint32_t j = 0; j < nd; ++j) {
      const uint32_t s = j * c.alpha, e = s + c.alpha < nq ? s + c.alpha : nq;
      hip_check(hipMemcpyAsync(digits + i * ct_words + ((size_t)j * ne + s) * n,
                               as[i] + (size_t)s * n, (size_t)(e - s) * n * 8,
                               hipMemcpyDeviceToDevice, c.stream),
                "modup digit copy");
    }
}

uint32_t galois_inverse(uint32_t g, uint32_t n) {
  // The odd residues mod 2N form a group of order N, so g^-1 = g^(N-1).
  const uint64_t m = 2ull * n;
  if (!(g & 1) || g >= m) throw ArgError("Galois element is not a unit mod 2N");
  uint64_t r = 1, b = g;
  for (uint64_t e = n - 1; e; e >>= 1, b = b * b % m)
    if (e & 1) r = r * b % m;
  return (uint32_t)r;
}

void keyswitch_batch(Context& c, const uint64_t* digits, uint32_t nq,
                     const uint64_t* const* keys, uint32_t batch, const KeySwitchOut* outs) {
  if (batch > MAX_KS_BATCH) throw ArgError("key-switch batch too large");
  const uint64_t* dg[MAX_KS_BATCH];
  for (uint32_t r = 0; r < batch; ++r) dg[r] = digits;
  keyswitch_batch(c, dg, nq, keys, batch, outs);
}

void keyswitch_batch(Context& c, const uint64_t* const* digits, uint32_t nq,
                     const uint64_t* const* keys, uint32_t batch, const KeySwitchOut* outs) {
  if (batch == 0) return;
  if (batch > MAX_KS_BATCH) throw ArgError("key-switch batch too large");
  if (c.K == 0) throw ArgError("key switching needs special primes");
  const uint32_t nd = num_digits(c, nq);
  if (nd > MAXD) throw ArgError("more than 8 key-switching digits");
  const size_t n = c.n, ne = nq + c.K, kw = (size_t)c.K * n;
  // The fused Q-limb products are reduced once: nd * q_i < 2^64 holds for
  // nd <= 8 and q_i < 2^61.
  Scratch ext(c, 2 * (size_t)batch * kw), y(c, 2 * (size_t)batch * nq * n);
  ModDownEpi epi{};
  epi.mc = c.d_const;
  epi.kl = (size_t)(c.L + c.K) * n;
  epi.nd = nd;
  epi.ne = (uint32_t)ne;
  epi.nq = nq;
  epi.L = c.L;
  for (uint32_t r = 0; r < batch; ++r) {
    epi.digits[r] = digits[r];
    epi.key[r] = keys[r];
    epi.out[r] = outs[r].out;
    epi.add[r][0] = outs[r].add0;
    epi.add[r][1] = outs[r].add1;
    epi.ginv[r] = galois_inverse(outs[r].galois, c.n);
  }
  // P limbs of the inner product (formed by the inverse NTT's first pass),
  // to coefficient form, converted to Q; then the forward NTT with the
  // Q-limb products and the combine in its last pass.
  if (moddown_fused_ok(c, nq)) {
    moddown_fused(c, ext.p, y.p, 2 * batch, nq, c.moddown_plan(nq), epi);
    return;
  }
  ntt_inverse_ksk(c, ext.p, 2 * batch, epi);
  convert(c, c.moddown_plan(nq), ext.p, kw, y.p, (size_t)nq * n, nq, 2 * batch);
  ntt_forward_moddown(c, y.p, 2 * batch, nq, epi);
}

void keyswitch_hoisted(Context& c, const uint64_t* digits, uint32_t nq,
                       const uint64_t* const* keys, const KeySwitchOut* outs, uint32_t count) {
  const size_t per_rot = 2 * (size_t)(c.K + nq) * c.n * 8;
  uint32_t batch = (uint32_t)std::max<size_t>(1, (size_t(2) << 30) / per_rot);
  batch = std::min<uint32_t>(batch, MAX_KS_BATCH);
  for (uint32_t r0 = 0; r0 < count; r0 += batch)
    keyswitch_batch(c, digits, nq, keys + r0, std::min(batch, count - r0), outs + r0);
}

void keyswitch(Context& c, const uint64_t* a, uint32_t nq, const uint64_t* key,
               const KeySwitchOut& out) {
  Scratch dig(c, num_digits(c, nq) * (size_t)(nq + c.K) * c.n);
  modup(c, a, nq, dig.p);
  keyswitch_batch(c, dig.p, nq, &key, 1, &out);
}

void rotate(Context& c, uint64_t* out, const uint64_t* ct, uint32_t nq, const uint64_t* key,
            uint32_t galois) {
  keyswitch(c, ct + (size_t)nq * c.n, nq, key, KeySwitchOut{out, ct, nullptr, galois});
}

// `count` independent key switches of polys srcs[r] ([nq][N]) with keys[r]
// into ko[r]: batched ModUps and batched ModDowns, each batch's scratch
// (digits + ext P limbs + y per key switch) kept under 2 GiB.
static void keyswitch_many(Context& c, const uint64_t* const* srcs, uint32_t nq,
                           const uint64_t* const* keys, const KeySwitchOut* ko, uint32_t count) {
  const size_t n = c.n, ne = nq + c.K;
  const uint32_t nd = num_digits(c, nq);
  const size_t ct_words = (size_t)nd * ne * n;
  const size_t per_ks = (ct_words + 2 * (size_t)(c.K + nq) * n) * 8;
  uint32_t batch = (uint32_t)std::max<size_t>(1, (size_t(2) << 30) / per_ks);
  batch = std::min<uint32_t>(batch, MAX_KS_BATCH);
  for (uint32_t r0 = 0; r0 < count; r0 += batch) {
    const uint32_t b = std::min(batch, count - r0);
    Scratch dig(c, b * ct_words);
    std::vector<const uint64_t*> dg(b);
    for (uint32_t r = 0; r < b; ++r) dg[r] = dig.p + r * ct_words;
    modup_batch(c, srcs + r0, b, nq, dig.p);
    keyswitch_batch(c, dg.data(), nq, keys + r0, b, ko + r0);
  }
}

void rotate_many(Context& c, uint64_t* const* outs, const uint64_t* const* cts, uint32_t nq,
                 const uint64_t* const* keys, const uint32_t* galois, uint32_t count) {
  std::vector<const uint64_t*> c1(count);
  std::vector<KeySwitchOut> ko(count);
  for (uint32_t r = 0; r < count; ++r) {
    c1[r] = cts[r] + (size_t)nq * c.n;
    ko[r] = KeySwitchOut{outs[r], cts[r], nullptr, galois[r]};
  }
  keyswitch_many(c, c1.data(), nq, keys, ko.data(), count);
}

void relinearize_many(Context& c, uint64_t* const* outs, const uint64_t* const* ct3s,
                      uint32_t nq, const uint64_t* key, uint32_t count) {
  const size_t pl = (size_t)nq * c.n;
  std::vector<const uint64_t*> d2(count), keys(count, key);
  std::vector<KeySwitchOut> ko(count);
  for (uint32_t r = 0; r < count; ++r) {
    d2[r] = ct3s[r] + 2 * pl;
    ko[r] = KeySwitchOut{outs[r], ct3s[r], ct3s[r] + pl, 1};
  }
  keyswitch_many(c, d2.data(), nq, keys.data(), ko.data(), count);
}

void linear_transform(Context& c, uint64_t* out, const uint64_t* ct, uint32_t nq,
                      const uint64_t* const* pts, uint32_t count, uint32_t bstep,
                      const uint64_t* const* baby_keys, const uint32_t* baby_galois,
                      const uint64_t* const* giant_keys, const uint32_t* giant_galois,
                      uint32_t n_giant_keys) {
  linear_transform_many(c, &out, &ct, 1, nq, pts, count, bstep, baby_keys, baby_galois,
                        giant_keys, giant_galois, n_giant_keys);
}

void linear_transform_many(Context& c, uint64_t* const* outs, const uint64_t* const* cts,
                           uint32_t ncts, uint32_t nq, const uint64_t* const* pts,
                           uint32_t count, uint32_t bstep, const uint64_t* const* baby_keys,
                           const uint32_t* baby_galois, const uint64_t* const* giant_keys,
                           const uint32_t* giant_galois, uint32_t n_giant_keys) {
  if (count == 0 || bstep == 0) throw ArgError("linear transform: no diagonals");
  if (ncts == 0) return;
  const size_t n = c.n, ne = nq + c.K, pl = 2 * (size_t)nq * n;
  const uint32_t giants = (count + bstep - 1) / bstep, nb = std::min(bstep, count);
  const bool batched = giants > 1 && n_giant_keys == giants - 1;
  if (giants > 1 && !batched && n_giant_keys != 1)
    throw ArgError("linear transform: one giant-step key, or one per giant step");
  for (uint32_t g = 0; g + 1 < giants && g < n_giant_keys; ++g)
    if (!giant_keys[g]) throw ArgError("linear transform: giant-step key missing");
  std::vector<uint8_t> used(nb, 0);
  for (uint32_t k = 0; k < count; ++k)
    if (pts[k]) used[k % bstep] = 1;
  const uint32_t nd = num_digits(c, nq);
  const size_t ct_words = (size_t)nd * ne * n;
  // Key switches sharing the digits of one ciphertext go out in batches of
  // at most MAX_KS_BATCH whose ModDown scratch stays under 2 GiB.
  const size_t per_rot = 2 * (size_t)(c.K + nq) * n * 8;
  const uint32_t ks_batch =
      std::min<uint32_t>((uint32_t)std::max<size_t>(1, (size_t(2) << 30) / per_rot), MAX_KS_BATCH);
  auto switch_all = [&](const std::vector<const uint64_t*>& dg,
                        const std::vector<const uint64_t*>& keys,
                        const std::vector<KeySwitchOut>& ko) {
    const uint32_t total = (uint32_t)ko.size();
    for (uint32_t r0 = 0; r0 < total; r0 += ks_batch)
      keyswitch_batch(c, dg.data() + r0, nq, keys.data() + r0, std::min(ks_batch, total - r0),
                      ko.data() + r0);
  };
  // Babies rot(ct_i) for the b some diagonal uses: every ciphertext's c1 in
  // one batched ModUp, then all (ciphertext, baby) key switches; baby 0 is
  // ct_i itself unless baby_keys[0] gives it an offset rotation.
  std::vector<const uint64_t*> baby((size_t)ncts * nb, nullptr);
  std::vector<uint32_t> ks_b;
  for (uint32_t b = 0; b < nb; ++b) {
    if (b == 0 && !baby_keys[0]) {
      for (uint32_t i = 0; i < ncts; ++i) baby[(size_t)i * nb] = cts[i];
      continue;
    }
    if (!used[b]) continue;
    if (!baby_keys[b]) throw ArgError("linear transform: baby-step key missing");
    ks_b.push_back(b);
  }
  Scratch babies(c, std::max<size_t>(1, (size_t)ncts * ks_b.size() * pl));
  if (!ks_b.empty()) {
    Scratch dig(c, (size_t)ncts * ct_words);
    std::vector<const uint64_t*> c1(ncts), dg, keys;
    std::vector<KeySwitchOut> ko;
    for (uint32_t i = 0; i < ncts; ++i) c1[i] = cts[i] + (size_t)nq * n;
    modup_batch(c, c1.data(), ncts, nq, dig.p);
    for (uint32_t i = 0; i < ncts; ++i)
      for (size_t j = 0; j < ks_b.size(); ++j) {
        const uint32_t b = ks_b[j];
        uint64_t* dst = babies.p + ((size_t)i * ks_b.size() + j) * pl;
        baby[(size_t)i * nb + b] = dst;
        dg.push_back(dig.p + i * ct_words);
        keys.push_back(baby_keys[b]);
        ko.push_back(KeySwitchOut{dst, cts[i], nullptr, baby_galois[b]});
      }
    switch_all(dg, keys, ko);
  }
  std::vector<const uint64_t*> xs, ws;
  auto inner = [&](uint32_t i, uint32_t g, uint64_t* acc, bool accumulate) {
    xs.clear();
    ws.clear();
    for (uint32_t b = 0; b < bstep; ++b) {
      const uint32_t k = g * bstep + b;
      if (k < count && pts[k]) {
        xs.push_back(baby[(size_t)i * nb + b]);
        ws.push_back(pts[k]);
      }
    }
    poly_mac_table(c, acc, xs.data(), ws.data(), (uint32_t)xs.size(), nq, accumulate);
  };
  if (batched) {
    // Every giant step's inner sum of every ciphertext, then their
    // rotations by g giant strides as one set of independent key switches,
    // then the sums.
    Scratch in(c, (size_t)ncts * giants * pl), rot(c, (size_t)ncts * (giants - 1) * pl);
    // the babies some diagonal uses (the others were not formed)
    std::vector<uint32_t> bu;
    for (uint32_t b = 0; b < nb; ++b)
      if (baby[b]) bu.push_back(b);
    const uint32_t nu = (uint32_t)bu.size();
    for (uint32_t i = 0; i < ncts; ++i) {
      uint64_t* in_i = in.p + (size_t)i * giants * pl;
      if (nu && nu <= MACG_MAX_B) {
        // the inner sums of up to MACG_MAX_G giants per pass over the babies
        std::vector<const uint64_t*> xb(nu);
        std::vector<uint64_t*> acc(giants);
        std::vector<const uint64_t*> w((size_t)giants * nu, nullptr);
        for (uint32_t j = 0; j < nu; ++j) xb[j] = baby[(size_t)i * nb + bu[j]];
        for (uint32_t g = 0; g < giants; ++g) {
          acc[g] = in_i + g * pl;
          for (uint32_t j = 0; j < nu; ++j) {
            const uint32_t k = g * bstep + bu[j];
            if (k < count) w[(size_t)g * nu + j] = pts[k];
          }
        }
        for (uint32_t g0 = 0; g0 < giants; g0 += MACG_MAX_G)
          poly_mac_giants(c, acc.data() + g0, std::min<uint32_t>(MACG_MAX_G, giants - g0),
                          xb.data(), nu, w.data() + (size_t)g0 * nu, nq);
      } else {
        for (uint32_t g = 0; g < giants; ++g) inner(i, g, in_i + g * pl, false);
      }
    }
    const size_t nr = (size_t)ncts * (giants - 1);
    std::vector<uint64_t*> ro(nr);
    std::vector<const uint64_t*> ri(nr), rk(nr);
    std::vector<uint32_t> rg(nr);
    for (uint32_t i = 0; i < ncts; ++i)
      for (uint32_t g = 1; g < giants; ++g) {
        const size_t r = (size_t)i * (giants - 1) + (g - 1);
        ro[r] = rot.p + r * pl;
        ri[r] = in.p + ((size_t)i * giants + g) * pl;
        rk[r] = giant_keys[g - 1];
        rg[r] = giant_galois[g - 1];
      }
    rotate_many(c, ro.data(), ri.data(), nq, rk.data(), rg.data(), (uint32_t)nr);
    for (uint32_t i = 0; i < ncts; ++i) {
      const uint64_t* in_i = in.p + (size_t)i * giants * pl;
      uint64_t* const* ro_i = ro.data() + (size_t)i * (giants - 1);
      if (giants <= SUM_MAX) {
        std::vector<const uint64_t*> terms(giants);
        terms[0] = in_i;
        for (uint32_t g = 1; g < giants; ++g) terms[g] = ro_i[g - 1];
        poly_sum(c, outs[i], terms.data(), giants, 2, nq);
      } else {
        poly_binary(c, OP_ADD, outs[i], in_i, ro_i[0], 2, nq);
        for (uint32_t g = 2; g < giants; ++g)
          poly_binary(c, OP_ADD, outs[i], outs[i], ro_i[g - 1], 2, nq);
      }
    }
    return;
  }
  // Giant steps by Horner's rule, every ciphertext in step: acc_i =
  // inner_{G-1}; acc_i = inner_g + rot(acc_i), the rotations of one step as
  // one batched ModUp and one set of key switches.
  Scratch acc(c, 2 * (size_t)ncts * pl);
  std::vector<uint64_t*> cur(ncts), nxt(ncts);
  for (uint32_t i = 0; i < ncts; ++i) {
    cur[i] = acc.p + (2 * (size_t)i) * pl;
    nxt[i] = acc.p + (2 * (size_t)i + 1) * pl;
    inner(i, giants - 1, cur[i], false);
  }
  if (giants > 1) {
    Scratch dig(c, (size_t)ncts * ct_words);
    std::vector<const uint64_t*> c1(ncts), dg(ncts), keys(ncts, giant_keys[0]);
    std::vector<KeySwitchOut> ko(ncts);
    for (int g = (int)giants - 2; g >= 0; --g) {
      for (uint32_t i = 0; i < ncts; ++i) {
        c1[i] = cur[i] + (size_t)nq * n;
        dg[i] = dig.p + i * ct_words;
        ko[i] = KeySwitchOut{nxt[i], cur[i], nullptr, giant_galois[0]};
      }
      modup_batch(c, c1.data(), ncts, nq, dig.p);
      switch_all(dg, keys, ko);
      for (uint32_t i = 0; i < ncts; ++i) {
        inner(i, (uint32_t)g, nxt[i], true);
        std::swap(cur[i], nxt[i]);
      }
    }
  }
  for (uint32_t i = 0; i < ncts; ++i)
    hip_check(hipMemcpyAsync(outs[i], cur[i], pl * 8, hipMemcpyDeviceToDevice, c.stream),
              "linear transform");
}

void automorph(Context& c, uint64_t* out, const uint64_t* in, uint32_t npoly, uint32_t nlimb,
               uint32_t galois) {
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_automorph", k_automorph, dim3(c.n / tpb, nlimb, npoly), dim3(tpb), 0, out, in, c.n, c.log_n, nlimb, galois);
}

void key_to_montgomery(Context& c, uint64_t* key) {
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_to_mont", k_to_mont, dim3(c.n / tpb, c.L + c.K, c.dnum * 2), dim3(tpb), 0, key, c.d_const, c.d_keyfac, c.n, c.L + c.K);
}

void key_from_montgomery(Context& c, uint64_t* out, const uint64_t* key) {
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_from_mont", k_from_mont, dim3(c.n / tpb, c.L + c.K, c.dnum * 2), dim3(tpb), 0, out, key, c.d_const, c.d_keyfac_out, c.n, c.L + c.K);
}

}  // namespace fhe
