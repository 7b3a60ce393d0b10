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

// Key inner product.  grid (N / (2 blockDim), nq + K, 1).
__global__ void __launch_bounds__(TPB)
    k_ksk_inner(const uint64_t* __restrict__ digits, const uint64_t* __restrict__ key,
                uint64_t* __restrict__ ext, const ModConst* __restrict__ mc, uint32_t n,
                uint32_t nq, uint32_t L, uint32_t K, uint32_t nd, uint32_t chunk) {
  const uint32_t i = blockIdx.y, ne = nq + K;
  const uint32_t ki = i < nq ? i : L + (i - nq);
  const uint64_t q = mc[ki].q, qinv = mc[ki].qinv_neg;
  const size_t e = 2 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
  const size_t kl = (size_t)(L + K) * n;  // key limb-set stride
  uint64_t r0x = 0, r0y = 0, r1x = 0, r1y = 0;
  uint32_t j0 = 0;
  while (j0 < nd) {
    const uint32_t j1 = j0 + chunk < nd ? j0 + chunk : nd;
    Acc128 a0x, a0y, a1x, a1y;
    for (uint32_t j = j0; j < j1; ++j) {
      const ulonglong2 d = *reinterpret_cast<const ulonglong2*>(digits + ((size_t)j * ne + i) * n + e);
      const uint64_t* kb = key + ((size_t)j * 2) * kl + (size_t)ki * n + e;
      const ulonglong2 b = *reinterpret_cast<const ulonglong2*>(kb);
      const ulonglong2 a = *reinterpret_cast<const ulonglong2*>(kb + kl);
      a0x.mac(d.x, b.x);
      a0y.mac(d.y, b.y);
      a1x.mac(d.x, a.x);
      a1y.mac(d.y, a.y);
    }
    r0x = add_mod(r0x, redc(a0x.hi, a0x.lo, q, qinv), q);
    r0y = add_mod(r0y, redc(a0y.hi, a0y.lo, q, qinv), q);
    r1x = add_mod(r1x, redc(a1x.hi, a1x.lo, q, qinv), q);
    r1y = add_mod(r1y, redc(a1y.hi, a1y.lo, q, qinv), q);
    j0 = j1;
  }
  *reinterpret_cast<ulonglong2*>(ext + (size_t)i * n + e) = make_ulonglong2(r0x, r0y);
  *reinterpret_cast<ulonglong2*>(ext + ((size_t)ne + i) * n + e) = make_ulonglong2(r1x, r1y);
}

__device__ __forceinline__ uint32_t brev_bits(uint32_t x, uint32_t bits) {
  return __brev(x) >> (32 - bits);
}

// ModDown combine with optional addends and Galois permutation.
//   out_b[i][x] = ((ext_b[i][s] - y_b[i][s]) * P^-1 + add_b[i][s]) mod q_i,
//   s = the evaluation slot that X -> X^galois moves to x (s = x if galois
//   is 1).  grid (N / blockDim, nq, 2).
__global__ void __launch_bounds__(TPB)
    k_moddown_combine(uint64_t* __restrict__ out, const uint64_t* __restrict__ ext,
                      const uint64_t* __restrict__ y, const uint64_t* __restrict__ add0,
                      const uint64_t* __restrict__ add1, const ModConst* __restrict__ mc,
                      const uint64_t* __restrict__ pinv, uint32_t n, uint32_t log_n, uint32_t nq,
                      uint32_t K, uint32_t galois) {
  const uint32_t i = blockIdx.y, b = blockIdx.z;
  const uint64_t q = mc[i].q, pi = pinv[2 * i], pis = pinv[2 * i + 1];
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t s = x;
  if (galois != 1) {
    const uint32_t j = brev_bits(x, log_n);
    const uint32_t m2 = 2 * n;
    const uint32_t ex = (uint32_t)(((2ull * j + 1) * galois) & (m2 - 1));
    s = brev_bits((ex - 1) >> 1, log_n);
  }
  const size_t ne = nq + K;
  const uint64_t ev = ext[((size_t)b * ne + i) * n + s];
  const uint64_t yv = y[((size_t)b * nq + i) * n + s];
  uint64_t r = shoup(ev + q - yv, pi, pis, q);
  const uint64_t* add = b == 0 ? add0 : add1;
  if (add) r = add_mod(r, add[(size_t)i * n + s], q);
  out[((size_t)b * nq + i) * n + x] = r;
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
    k_to_mont(uint64_t* key, const ModConst* mc, uint32_t n, uint32_t nm) {
  const uint32_t i = blockIdx.y;
  const ModConst m = mc[i];
  const size_t o = ((size_t)blockIdx.z * nm + i) * n + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  key[o] = mont_mul(key[o], m.r2, m.q, m.qinv_neg);
}

// Terms per REDC so that terms * max_q < 2^64.
uint32_t redc_chunk(const Context& c, const std::vector<uint32_t>& idx) {
  uint64_t mx = 1;
  for (uint32_t i : idx) mx = c.mods[i] > mx ? c.mods[i] : mx;
  uint64_t ch = ~0ull / mx;
  if (ch > MAXSRC) ch = MAXSRC;
  return (uint32_t)(ch < 1 ? 1 : ch);
}

void convert(Context& c, const ConvPlan& pl, const uint64_t* src, size_t src_ps, uint64_t* out,
             size_t out_ps, uint32_t out_nq, uint32_t npoly) {
  if (pl.nsrc > MAXSRC) throw ArgError("basis conversion source larger than 16 limbs");
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_convert", k_convert, dim3(c.n / tpb, 1, npoly), dim3(tpb), 0, src, src_ps, out, out_ps, c.d_const, pl.d_src_idx32, pl.d_qhat_inv, pl.d_qhat_mont, pl.d_dst_idx, pl.nsrc, pl.ndst, c.n, c.L, out_nq, redc_chunk(c, pl.src_idx));
}

}  // namespace

uint32_t num_digits(const Context& c, uint32_t nq) {
  const uint32_t d = (nq + c.alpha - 1) / c.alpha;
  return d < c.dnum ? d : c.dnum;
}

void modup(Context& c, const uint64_t* a, uint32_t nq, uint64_t* digits) {
  if (nq == 0 || nq > c.L) throw ArgError("modup: bad level");
  const size_t n = c.n, ne = nq + c.K;
  Scratch coef(c, (size_t)nq * n);
  hip_check(hipMemcpyAsync(coef.p, a, (size_t)nq * n * 8, hipMemcpyDeviceToDevice, c.stream),
            "modup copy");
  ntt_inverse(c, coef.p, 1, 0, nq, LimbMap::contiguous(0));
  const uint32_t nd = num_digits(c, nq);
  for (uint32_t j = 0; j < nd; ++j) {
    const uint32_t s = j * c.alpha, e = s + c.alpha < nq ? s + c.alpha : nq;
    uint64_t* dj = digits + (size_t)j * ne * n;
    convert(c, c.modup_plan(s, e, nq), coef.p + (size_t)s * n, 0, dj, 0, nq, 1);
    if (s > 0) ntt_forward(c, dj, 1, 0, s, LimbMap::contiguous(0));
    ntt_forward(c, dj + (size_t)e * n, 1, 0, (uint32_t)(ne - e), LimbMap{nq - e, e, c.L});
    hip_check(hipMemcpyAsync(dj + (size_t)s * n, a + (size_t)s * n, (size_t)(e - s) * n * 8,
                             hipMemcpyDeviceToDevice, c.stream),
              "modup digit copy");
  }
}

void ksk_inner(Context& c, const uint64_t* digits, uint32_t nq, const uint64_t* key_mont,
               uint64_t* ext) {
  const uint32_t nd = num_digits(c, nq);
  std::vector<uint32_t> all(c.L + c.K);
  for (uint32_t i = 0; i < c.L + c.K; ++i) all[i] = i;
  const uint32_t tpb = tpb_for(c, 2);
  FHE_LAUNCH(c, "k_ksk_inner", k_ksk_inner, dim3(c.n / (2 * tpb), nq + c.K, 1), dim3(tpb), 0, digits, key_mont, ext, c.d_const, c.n, nq, c.L, c.K, nd, redc_chunk(c, all));
}

void moddown_pair(Context& c, const uint64_t* ext, uint32_t nq, uint64_t* out,
                  const uint64_t* add0, uint32_t galois) {
  moddown_pair2(c, ext, nq, out, add0, nullptr, galois);
}

void moddown_pair2(Context& c, const uint64_t* ext, uint32_t nq, uint64_t* out,
                   const uint64_t* add0, const uint64_t* add1, uint32_t galois) {
  const size_t n = c.n, ne = nq + c.K;
  Scratch pc(c, 2 * (size_t)c.K * n), y(c, 2 * (size_t)nq * n);
  poly_copy_limbs(c, pc.p, c.K, ext + (size_t)nq * n, (uint32_t)ne, 2, c.K);
  ntt_inverse(c, pc.p, 2, (size_t)c.K * n, c.K, LimbMap::contiguous(c.L));
  convert(c, c.moddown_plan(nq), pc.p, (size_t)c.K * n, y.p, (size_t)nq * n, nq, 2);
  ntt_forward(c, y.p, 2, (size_t)nq * n, nq, LimbMap::contiguous(0));
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_moddown_combine", k_moddown_combine, dim3(c.n / tpb, nq, 2), dim3(tpb), 0, out, ext, y.p, add0, add1, c.d_const, c.d_pinv_q, c.n, c.log_n, nq, c.K, galois);
}

void automorph(Context& c, uint64_t* out, const uint64_t* in, uint32_t npoly, uint32_t nlimb,
               uint32_t galois) {
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_automorph", k_automorph, dim3(c.n / tpb, nlimb, npoly), dim3(tpb), 0, out, in, c.n, c.log_n, nlimb, galois);
}

void key_to_montgomery(Context& c, uint64_t* key) {
  const uint32_t tpb = tpb_for(c, 1);
  FHE_LAUNCH(c, "k_to_mont", k_to_mont, dim3(c.n / tpb, c.L + c.K, c.dnum * 2), dim3(tpb), 0, key, c.d_const, c.n, c.L + c.K);
}

}  // namespace fhe
