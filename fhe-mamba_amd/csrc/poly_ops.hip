// Elementwise RNS kernels: add/sub/negate, plaintext and constant products,
// tensor product, the MAC of a plaintext-ciphertext inner product, and the
// FLEXIBLEAUTO rescale.  All are HBM-bound; each thread moves two adjacent
// words with 16-byte accesses and the grid is (N/512, limb, poly) so the
// modulus constants are uniform per workgroup.
#include "ops.hpp"

namespace fhe {
namespace {

constexpr int TPB = 256;  // threads per block, 2 words per thread

struct U2 {
  uint64_t x, y;
};

__device__ __forceinline__ U2 ld2(const uint64_t* p) {
  const ulonglong2 v = *reinterpret_cast<const ulonglong2*>(p);
  return U2{v.x, v.y};
}
__device__ __forceinline__ void st2(uint64_t* p, uint64_t a, uint64_t b) {
  *reinterpret_cast<ulonglong2*>(p) = make_ulonglong2(a, b);
}

inline uint32_t tpb_for(const Context& c) { return c.n / 2 < TPB ? c.n / 2 : TPB; }
inline dim3 grid_for(const Context& c, uint32_t nlimb, uint32_t npoly) {
  return dim3(c.n / (2 * tpb_for(c)), nlimb, npoly);
}

// Word pair handled by this thread within its limb.
__device__ __forceinline__ size_t pair_off() {
  return 2 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
}
// blockIdx: x = chunk of N, y = limb, z = poly.
__device__ __forceinline__ size_t elem_off(uint32_t n, uint32_t nlimb) {
  return ((size_t)blockIdx.z * nlimb + blockIdx.y) * n + pair_off();
}

template <int OP>
__global__ void __launch_bounds__(TPB)
    k_binary(uint64_t* out, const uint64_t* a, const uint64_t* b, const ModConst* mc, uint32_t n,
             uint32_t nlimb) {
  const uint64_t q = mc[blockIdx.y].q;
  const size_t o = elem_off(n, nlimb);
  const U2 x = ld2(a + o), y = ld2(b + o);
  if (OP == OP_ADD)
    st2(out + o, add_mod(x.x, y.x, q), add_mod(x.y, y.y, q));
  else
    st2(out + o, sub_mod(x.x, y.x, q), sub_mod(x.y, y.y, q));
}

__global__ void __launch_bounds__(TPB)
    k_negate(uint64_t* out, const uint64_t* a, const ModConst* mc, uint32_t n, uint32_t nlimb) {
  const uint64_t q = mc[blockIdx.y].q;
  const size_t o = elem_off(n, nlimb);
  const U2 x = ld2(a + o);
  st2(out + o, neg_mod(x.x, q), neg_mod(x.y, q));
}

__global__ void __launch_bounds__(TPB)
    k_mul_plain(uint64_t* out, const uint64_t* a, const uint64_t* pt, const ModConst* mc,
                uint32_t n, uint32_t nlimb) {
  const ModConst m = mc[blockIdx.y];
  const size_t o = elem_off(n, nlimb);
  const size_t po = (size_t)blockIdx.y * n + pair_off();
  const U2 x = ld2(a + o), w = ld2(pt + po);
  st2(out + o, mul_mod(x.x, w.x, m), mul_mod(x.y, w.y, m));
}

__global__ void __launch_bounds__(TPB)
    k_add_plain(uint64_t* out, const uint64_t* a, const uint64_t* pt, const ModConst* mc,
                uint32_t n, uint32_t nlimb) {
  const uint64_t q = mc[blockIdx.y].q;
  const size_t o = elem_off(n, nlimb);
  U2 x = ld2(a + o);
  if (blockIdx.z == 0) {
    const size_t po = (size_t)blockIdx.y * n + pair_off();
    const U2 w = ld2(pt + po);
    x.x = add_mod(x.x, w.x, q);
    x.y = add_mod(x.y, w.y, q);
  }
  st2(out + o, x.x, x.y);
}

struct LimbConsts {
  uint64_t v[64][2];  // (value, Shoup companion)
};

__global__ void __launch_bounds__(TPB)
    k_mul_const(uint64_t* out, const uint64_t* a, LimbConsts k, const ModConst* mc, uint32_t n,
                uint32_t nlimb) {
  const uint64_t q = mc[blockIdx.y].q, w = k.v[blockIdx.y][0], ws = k.v[blockIdx.y][1];
  const size_t o = elem_off(n, nlimb);
  const U2 x = ld2(a + o);
  st2(out + o, shoup(x.x, w, ws, q), shoup(x.y, w, ws, q));
}

__global__ void __launch_bounds__(TPB)
    k_add_const(uint64_t* out, const uint64_t* a, LimbConsts k, const ModConst* mc, uint32_t n,
                uint32_t nlimb) {
  const uint64_t q = mc[blockIdx.y].q, w = blockIdx.z == 0 ? k.v[blockIdx.y][0] : 0;
  const size_t o = elem_off(n, nlimb);
  const U2 x = ld2(a + o);
  st2(out + o, add_mod(x.x, w, q), add_mod(x.y, w, q));
}

__global__ void __launch_bounds__(TPB)
    k_copy_limbs(uint64_t* out, uint32_t out_nlimb, const uint64_t* a, uint32_t a_nlimb,
                 uint32_t n) {
  const size_t e = pair_off();
  const U2 x = ld2(a + ((size_t)blockIdx.z * a_nlimb + blockIdx.y) * n + e);
  st2(out + ((size_t)blockIdx.z * out_nlimb + blockIdx.y) * n + e, x.x, x.y);
}

// Tensor: grid (N/512, nlimb, 1).
template <bool SQUARE>
__global__ void __launch_bounds__(TPB)
    k_tensor(uint64_t* out, const uint64_t* a, const uint64_t* b, const ModConst* mc, uint32_t n,
             uint32_t nlimb) {
  const ModConst m = mc[blockIdx.y];
  const size_t pl = (size_t)nlimb * n;
  const size_t o = (size_t)blockIdx.y * n + pair_off();
  const U2 a0 = ld2(a + o), a1 = ld2(a + pl + o);
  if (SQUARE) {
    const uint64_t c1x = mul_mod(a0.x, a1.x, m), c1y = mul_mod(a0.y, a1.y, m);
    st2(out + o, mul_mod(a0.x, a0.x, m), mul_mod(a0.y, a0.y, m));
    st2(out + pl + o, add_mod(c1x, c1x, m.q), add_mod(c1y, c1y, m.q));
    st2(out + 2 * pl + o, mul_mod(a1.x, a1.x, m), mul_mod(a1.y, a1.y, m));
  } else {
    const U2 b0 = ld2(b + o), b1 = ld2(b + pl + o);
    // The cross term is one reduction of a 128-bit sum of two products.
    Acc128 sx, sy;
    sx.mac(a0.x, b1.x);
    sx.mac(a1.x, b0.x);
    sy.mac(a0.y, b1.y);
    sy.mac(a1.y, b0.y);
    st2(out + o, mul_mod(a0.x, b0.x, m), mul_mod(a0.y, b0.y, m));
    st2(out + pl + o, reduce128(sx.hi, sx.lo, m), reduce128(sy.hi, sy.lo, m));
    st2(out + 2 * pl + o, mul_mod(a1.x, b1.x, m), mul_mod(a1.y, b1.y, m));
  }
}

// Fold a 128-bit accumulator to its value mod q (kept in lo).
__device__ __forceinline__ void fold(Acc128& a, const ModConst& m) {
  a.lo = reduce128(a.hi, a.lo, m);
  a.hi = 0;
}

// Every word of the MAC's operands is read exactly once: non-temporal loads
// keep them from displacing other data in the caches (5.0 -> 5.5 TB/s on the
// 64-ciphertext batch at N=2^16, 24 limbs).
__device__ __forceinline__ U2 ld2_stream(const uint64_t* p) {
  typedef unsigned long long v2u __attribute__((ext_vector_type(2)));
  const v2u v = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p));
  return U2{v.x, v.y};
}

// MAC: grid (N/128, nq) of one-wavefront workgroups (finer than
// 256-lane blocks for the scheduler: 5.5 -> 5.8 TB/s on the same batch);
// each thread takes two adjacent words of both polys of every ciphertext, so
// each plaintext word is read once for both, and accumulates the products in
// 128 bits, folding every 32 terms so the sums never overflow.
constexpr int MAC_TPB = 64;

__global__ void __launch_bounds__(MAC_TPB)
    k_mac(uint64_t* acc, const uint64_t* x, const uint64_t* w, const ModConst* mc, uint32_t n,
          uint32_t nq, uint32_t cnt) {
  const ModConst m = mc[blockIdx.y];
  const size_t limb_off = (size_t)blockIdx.y * n + pair_off();
  const size_t pl = (size_t)nq * n, xs = 2 * pl, ws = pl;
  const uint64_t* xp = x + limb_off;
  const uint64_t* wp = w + limb_off;
  Acc128 s[2][2];
  uint32_t i = 0;
  while (i < cnt) {
    const uint32_t end = i + 32 < cnt ? i + 32 : cnt;
    // Twelve independent 16-byte loads in flight per thread.
    for (; i + 4 <= end; i += 4) {
      U2 x0[4], x1[4], wv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x0[u] = ld2_stream(xp + (i + u) * xs);
        x1[u] = ld2_stream(xp + (i + u) * xs + pl);
        wv[u] = ld2_stream(wp + (i + u) * ws);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        s[0][0].mac(x0[u].x, wv[u].x);
        s[0][1].mac(x0[u].y, wv[u].y);
        s[1][0].mac(x1[u].x, wv[u].x);
        s[1][1].mac(x1[u].y, wv[u].y);
      }
    }
    for (; i < end; ++i) {
      const U2 a = ld2_stream(xp + i * xs), b = ld2_stream(xp + i * xs + pl);
      const U2 wv = ld2_stream(wp + i * ws);
      s[0][0].mac(a.x, wv.x);
      s[0][1].mac(a.y, wv.y);
      s[1][0].mac(b.x, wv.x);
      s[1][1].mac(b.y, wv.y);
    }
    fold(s[0][0], m);
    fold(s[0][1], m);
    fold(s[1][0], m);
    fold(s[1][1], m);
  }
  st2(acc + limb_off, s[0][0].lo, s[0][1].lo);
  st2(acc + pl + limb_off, s[1][0].lo, s[1][1].lo);
}

// acc[p][j] = (acc[p][j] if accumulate) + sum_i x_i[p][j] * w_i[j] mod q_j for
// ciphertexts x_i [2][nq][N] and plaintexts w_i (limb j at w_i + j * N)
// given by address; both polys per thread and the same 128-bit accumulation
// as k_mac.
__global__ void __launch_bounds__(TPB)
    k_mac_table(uint64_t* acc, const MacTable t, const ModConst* mc, uint32_t n, uint32_t nq,
                uint32_t cnt, uint32_t accumulate) {
  const ModConst m = mc[blockIdx.y];
  const size_t limb_off = (size_t)blockIdx.y * n + pair_off();
  const size_t pl = (size_t)nq * n;
  Acc128 s[2][2];
  uint32_t i = 0;
  while (i < cnt) {
    const uint32_t end = i + 32 < cnt ? i + 32 : cnt;
    for (; i + 4 <= end; i += 4) {
      U2 x0[4], x1[4], wv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x0[u] = ld2(t.x[i + u] + limb_off);
        x1[u] = ld2(t.x[i + u] + pl + limb_off);
        wv[u] = ld2(t.w[i + u] + limb_off);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        s[0][0].mac(x0[u].x, wv[u].x);
        s[0][1].mac(x0[u].y, wv[u].y);
        s[1][0].mac(x1[u].x, wv[u].x);
        s[1][1].mac(x1[u].y, wv[u].y);
      }
    }
    for (; i < end; ++i) {
      const U2 a = ld2(t.x[i] + limb_off), b = ld2(t.x[i] + pl + limb_off);
      const U2 wv = ld2(t.w[i] + limb_off);
      s[0][0].mac(a.x, wv.x);
      s[0][1].mac(a.y, wv.y);
      s[1][0].mac(b.x, wv.x);
      s[1][1].mac(b.y, wv.y);
    }
    fold(s[0][0], m);
    fold(s[0][1], m);
    fold(s[1][0], m);
    fold(s[1][1], m);
  }
  for (int p = 0; p < 2; ++p) {
    uint64_t* ap = acc + (size_t)p * pl + limb_off;
    uint64_t v0 = s[p][0].lo, v1 = s[p][1].lo;
    if (accumulate) {
      const U2 a = ld2(ap);
      v0 = add_mod(v0, a.x, m.q);
      v1 = add_mod(v1, a.y, m.q);
    }
    st2(ap, v0, v1);
  }
}

// Integer-weighted sum of ciphertexts (both polys per thread): the weight's
// residue comes from its 128-bit magnitude by one reduction per thread, and
// the 64x64-bit products of up to WSUM_MAX terms (each below 2^122) add in
// 128 bits before one final reduction.
struct WsumTable {
  const uint64_t* x[WSUM_MAX];  // [2][nl_i][N]
  uint64_t pl[WSUM_MAX];        // words per poly of term i, nl_i * N
  uint64_t mlo[WSUM_MAX], mhi[WSUM_MAX];  // |m_i|
  uint32_t neg;                 // bit i: m_i < 0
};

__global__ void __launch_bounds__(TPB)
    k_wsum(uint64_t* out, const WsumTable t, const ModConst* mc, uint32_t n, uint32_t nq,
           uint32_t cnt, uint32_t accumulate) {
  const ModConst m = mc[blockIdx.y];
  const size_t limb_off = (size_t)blockIdx.y * n + pair_off();
  Acc128 s[2][2];
  for (uint32_t i = 0; i < cnt; ++i) {
    uint64_t w = reduce128(t.mhi[i], t.mlo[i], m);
    if (((t.neg >> i) & 1u) && w) w = m.q - w;
    const U2 a = ld2(t.x[i] + limb_off), b = ld2(t.x[i] + t.pl[i] + limb_off);
    s[0][0].mac(a.x, w);
    s[0][1].mac(a.y, w);
    s[1][0].mac(b.x, w);
    s[1][1].mac(b.y, w);
  }
  const size_t pl = (size_t)nq * n;
  for (int p = 0; p < 2; ++p) {
    fold(s[p][0], m);
    fold(s[p][1], m);
    uint64_t* op = out + (size_t)p * pl + limb_off;
    uint64_t v0 = s[p][0].lo, v1 = s[p][1].lo;
    if (accumulate) {
      const U2 o = ld2(op);
      v0 = add_mod(v0, o.x, m.q);
      v1 = add_mod(v1, o.y, m.q);
    }
    st2(op, v0, v1);
  }
}

// Rescale step 1: centred lift of the (inverse-NTT'd) last limb into limbs
// i < l.  grid (N/512, l, npoly).  last: [npoly][N] coefficient form.
__global__ void __launch_bounds__(TPB)
    k_rescale_lift(uint64_t* t, const uint64_t* last, const ModConst* mc, const uint64_t* rs,
                   uint32_t n, uint32_t l, uint32_t L, uint64_t ql) {
  const uint32_t i = blockIdx.y;
  const uint64_t q = mc[i].q;
  const uint64_t qlm = rs[((size_t)l * L + i) * 4];  // q_l mod q_i
  const size_t e = pair_off();
  const U2 v = ld2(last + (size_t)blockIdx.z * n + e);
  const uint64_t half = ql >> 1;
  const ModConst m = mc[i];
  auto lift = [&](uint64_t x) -> uint64_t {
    // x mod q_i (x < 2^61 may exceed q_i), minus q_l if x is in the upper half.
    const uint64_t r = reduce_2q(x - mulhi64(x, m.mu64) * q, q);
    return x > half ? sub_mod(r, qlm, q) : r;
  };
  st2(t + ((size_t)blockIdx.z * l + i) * n + e, lift(v.x), lift(v.y));
}

// ModRaise lift: x [npoly][N] in coefficient form mod q0 -> out[p][j] =
// (x centred mod q0) mod q_j for j < nq.  grid (N/512, nq, npoly).
__global__ void __launch_bounds__(TPB)
    k_mod_raise_lift(uint64_t* out, const uint64_t* x, const ModConst* mc, uint32_t n, uint32_t nq,
                     uint64_t q0) {
  const uint32_t j = blockIdx.y;
  const ModConst m = mc[j];
  const uint64_t q = m.q;
  auto red = [&](uint64_t v) -> uint64_t { return reduce_2q(v - mulhi64(v, m.mu64) * q, q); };
  const uint64_t q0m = red(q0), half = q0 >> 1;
  const size_t e = pair_off();
  const U2 v = ld2(x + (size_t)blockIdx.z * n + e);
  auto lift = [&](uint64_t a) -> uint64_t {
    const uint64_t r = red(a);
    return a > half ? sub_mod(r, q0m, q) : r;
  };
  st2(out + ((size_t)blockIdx.z * nq + j) * n + e, lift(v.x), lift(v.y));
}

// Rescale step 2: out_i = (a_i - t_i) * q_l^-1.  grid (N/512, l, npoly).
__global__ void __launch_bounds__(TPB)
    k_rescale_combine(uint64_t* out, const uint64_t* a, const uint64_t* t, const ModConst* mc,
                      const uint64_t* rs, uint32_t n, uint32_t l, uint32_t L) {
  const uint32_t i = blockIdx.y;
  const uint64_t q = mc[i].q;
  const uint64_t inv = rs[((size_t)l * L + i) * 4 + 1], invs = rs[((size_t)l * L + i) * 4 + 2];
  const size_t e = pair_off();
  const U2 x = ld2(a + ((size_t)blockIdx.z * (l + 1) + i) * n + e);
  const U2 y = ld2(t + ((size_t)blockIdx.z * l + i) * n + e);
  st2(out + ((size_t)blockIdx.z * l + i) * n + e, shoup(x.x + q - y.x, inv, invs, q),
      shoup(x.y + q - y.y, inv, invs, q));
}

LimbConsts make_consts(const Context& c, const uint64_t* consts, uint32_t nlimb) {
  if (nlimb > 64) throw ArgError("at most 64 limbs");
  LimbConsts k{};
  for (uint32_t j = 0; j < nlimb; ++j) {
    const uint64_t q = c.mods[j];
    if (consts[j] >= q) throw ArgError("constant not reduced mod q_j");
    k.v[j][0] = consts[j];
    k.v[j][1] = host_shoup(consts[j], q);
  }
  return k;
}

// Inner sums of up to MACG_MAX_G giant steps: each thread holds one word
// position of both polys of every baby in turn and accumulates it into every
// giant's sum (128-bit, one reduction each: at most 32 products of two
// words below 2^61), so the babies are read once instead of once per giant.
// grid (N / 256, nq).
struct MacGiants {
  const uint64_t* x[MACG_MAX_B];
  const uint64_t* w[MACG_MAX_G][MACG_MAX_B];
  uint64_t* acc[MACG_MAX_G];
};

template <int G>
__global__ void __launch_bounds__(TPB)
    k_mac_giants(const MacGiants t, const ModConst* mc, uint32_t n, uint32_t nq, uint32_t nb) {
  const ModConst m = mc[blockIdx.y];
  const size_t off = (size_t)blockIdx.y * n + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t pl = (size_t)nq * n;
  Acc128 s[G][2];
  for (uint32_t b = 0; b < nb; ++b) {
    const uint64_t* xb = t.x[b];
    const uint64_t x0 = xb[off], x1 = xb[pl + off];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint64_t* w = t.w[g][b];
      if (w) {
        const uint64_t wv = w[off];
        s[g][0].mac(x0, wv);
        s[g][1].mac(x1, wv);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    uint64_t* a = t.acc[g] + off;
    a[0] = reduce128(s[g][0].hi, s[g][0].lo, m);
    a[pl] = reduce128(s[g][1].hi, s[g][1].lo, m);
  }
}

// out = sum_j in[j], reduced after every addition (values below q).
struct SumTable {
  const uint64_t* p[SUM_MAX];
};
__global__ void __launch_bounds__(TPB)
    k_sum(uint64_t* out, const SumTable t, uint32_t cnt, const ModConst* mc, uint32_t n,
          uint32_t nlimb) {
  const uint64_t q = mc[blockIdx.y].q;
  const size_t o = elem_off(n, nlimb);
  U2 acc = ld2(t.p[0] + o);
  for (uint32_t j = 1; j < cnt; ++j) {
    const U2 v = ld2(t.p[j] + o);
    acc.x = add_mod(acc.x, v.x, q);
    acc.y = add_mod(acc.y, v.y, q);
  }
  st2(out + o, acc.x, acc.y);
}

}  // namespace

void poly_binary(Context& c, BinOp op, uint64_t* out, const uint64_t* a, const uint64_t* b,
                 uint32_t npoly, uint32_t nlimb) {
  if (op == OP_ADD)
    FHE_LAUNCH(c, "k_binary", k_binary<OP_ADD>, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, a, b, c.d_const, c.n, nlimb);
  else
    FHE_LAUNCH(c, "k_binary", k_binary<OP_SUB>, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, a, b, c.d_const, c.n, nlimb);
}

void poly_sum(Context& c, uint64_t* out, const uint64_t* const* in, uint32_t cnt,
              uint32_t npoly, uint32_t nlimb) {
  if (cnt == 0 || cnt > SUM_MAX) throw ArgError("poly_sum: 1..16 inputs");
  SumTable t{};
  for (uint32_t j = 0; j < cnt; ++j) t.p[j] = in[j];
  FHE_LAUNCH(c, "k_sum", k_sum, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, t, cnt,
             c.d_const, c.n, nlimb);
}

void poly_negate(Context& c, uint64_t* out, const uint64_t* a, uint32_t npoly, uint32_t nlimb) {
  FHE_LAUNCH(c, "k_negate", k_negate, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, a, c.d_const, c.n, nlimb);
}

void poly_mul_plain(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* pt,
                    uint32_t npoly, uint32_t nlimb) {
  FHE_LAUNCH(c, "k_mul_plain", k_mul_plain, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, a, pt, c.d_const, c.n, nlimb);
}

void poly_add_plain(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* pt,
                    uint32_t npoly, uint32_t nlimb) {
  FHE_LAUNCH(c, "k_add_plain", k_add_plain, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, a, pt, c.d_const, c.n, nlimb);
}

void poly_mul_const(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* consts,
                    uint32_t npoly, uint32_t nlimb) {
  const LimbConsts k = make_consts(c, consts, nlimb);
  FHE_LAUNCH(c, "k_mul_const", k_mul_const, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, a, k, c.d_const, c.n, nlimb);
}

void poly_add_const(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* consts,
                    uint32_t npoly, uint32_t nlimb) {
  const LimbConsts k = make_consts(c, consts, nlimb);
  FHE_LAUNCH(c, "k_add_const", k_add_const, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, a, k, c.d_const, c.n, nlimb);
}

void poly_copy_limbs(Context& c, uint64_t* out, uint32_t out_nlimb, const uint64_t* a,
                     uint32_t a_nlimb, uint32_t npoly, uint32_t nlimb) {
  if (nlimb == 0 || npoly == 0) return;
  FHE_LAUNCH(c, "k_copy_limbs", k_copy_limbs, grid_for(c, nlimb, npoly), dim3(tpb_for(c)), 0, out, out_nlimb, a, a_nlimb, c.n);
}

void poly_tensor(Context& c, uint64_t* out3, const uint64_t* a, const uint64_t* b,
                 uint32_t nlimb) {
  if (a == b)
    FHE_LAUNCH(c, "k_tensor", k_tensor<true>, grid_for(c, nlimb, 1), dim3(tpb_for(c)), 0, out3, a, b, c.d_const, c.n, nlimb);
  else
    FHE_LAUNCH(c, "k_tensor", k_tensor<false>, grid_for(c, nlimb, 1), dim3(tpb_for(c)), 0, out3, a, b, c.d_const, c.n, nlimb);
}

void poly_mac(Context& c, uint64_t* acc, const uint64_t* x, const uint64_t* w, uint32_t n,
              uint32_t nq) {
  const uint32_t tpb = c.n / 2 < MAC_TPB ? c.n / 2 : MAC_TPB;
  FHE_LAUNCH(c, "k_mac", k_mac, dim3(c.n / (2 * tpb), nq, 1), dim3(tpb), 0, acc, x, w, c.d_const,
             c.n, nq, n);
}

void poly_mac_table(Context& c, uint64_t* acc, const uint64_t* const* x,
                    const uint64_t* const* w, uint32_t cnt, uint32_t nq, bool accumulate) {
  uint32_t i = 0;
  do {
    const uint32_t k = cnt - i < MAC_TABLE ? cnt - i : MAC_TABLE;
    MacTable t{};
    for (uint32_t j = 0; j < k; ++j) {
      t.x[j] = x[i + j];
      t.w[j] = w[i + j];
    }
    const uint32_t acc_flag = (accumulate || i > 0) ? 1u : 0u;
    FHE_LAUNCH(c, "k_mac_table", k_mac_table, grid_for(c, nq, 1), dim3(tpb_for(c)), 0, acc, t, c.d_const, c.n, nq, k, acc_flag);
    i += k;
  } while (i < cnt);
}

void poly_linear_wsum(Context& c, uint64_t* out, const uint64_t* const* x, const uint32_t* x_nlimb,
                      const uint64_t* weights, uint32_t cnt, uint32_t nq) {
  if (cnt == 0) throw ArgError("a weighted sum needs at least one term");
  for (uint32_t i0 = 0; i0 < cnt; i0 += WSUM_MAX) {
    const uint32_t k = cnt - i0 < WSUM_MAX ? cnt - i0 : WSUM_MAX;
    WsumTable t{};
    for (uint32_t j = 0; j < k; ++j) {
      const uint32_t i = i0 + j;
      if (x_nlimb[i] < nq) throw ArgError("a term has fewer limbs than the sum");
      uint64_t lo = weights[2 * i], hi = weights[2 * i + 1];
      if (hi >> 63) {  // magnitude of a negative two's-complement value
        lo = ~lo + 1;
        hi = ~hi + (lo == 0);
        t.neg |= 1u << j;
      }
      t.x[j] = x[i];
      t.pl[j] = (uint64_t)x_nlimb[i] * c.n;
      t.mlo[j] = lo;
      t.mhi[j] = hi;
    }
    FHE_LAUNCH(c, "k_wsum", k_wsum, grid_for(c, nq, 1), dim3(tpb_for(c)), 0, out, t, c.d_const, c.n, nq, k, i0 > 0 ? 1u : 0u);
  }
}

void poly_mod_raise(Context& c, uint64_t* out, uint32_t nq_out, const uint64_t* a,
                    uint32_t a_nlimb, uint32_t npoly) {
  if (nq_out == 0 || nq_out > c.L) throw ArgError("ModRaise: bad output level");
  Scratch low(c, (size_t)npoly * c.n);
  FHE_LAUNCH(c, "k_copy_limbs", k_copy_limbs, grid_for(c, 1, npoly), dim3(tpb_for(c)), 0, low.p, 1u, a, a_nlimb, c.n);
  ntt_inverse(c, low.p, npoly, c.n, 1, LimbMap::contiguous(0));
  FHE_LAUNCH(c, "k_mod_raise_lift", k_mod_raise_lift, grid_for(c, nq_out, npoly), dim3(tpb_for(c)), 0, out, low.p, c.d_const, c.n, nq_out, c.mods[0]);
  ntt_forward(c, out, npoly, (size_t)nq_out * c.n, nq_out, LimbMap::contiguous(0));
}

void poly_rescale(Context& c, uint64_t* out, const uint64_t* a, uint32_t npoly, uint32_t nq) {
  if (nq < 2) throw ArgError("rescale needs at least two limbs");
  if (c.log_n >= 13 && c.log_n <= 17) {
    rescale_fused(c, out, a, npoly, nq);
    return;
  }
  const uint32_t l = nq - 1;
  Scratch last(c, (size_t)npoly * c.n), t(c, (size_t)npoly * l * c.n);
  // last limb of every poly -> [npoly][N], to coefficient form with q_l
  FHE_LAUNCH(c, "k_copy_limbs", k_copy_limbs, grid_for(c, 1, npoly), dim3(tpb_for(c)), 0, last.p, 1u, a + (size_t)l * c.n, nq, c.n);
  ntt_inverse(c, last.p, npoly, c.n, 1, LimbMap::contiguous(l));
  FHE_LAUNCH(c, "k_rescale_lift", k_rescale_lift, grid_for(c, l, npoly), dim3(tpb_for(c)), 0, t.p, last.p, c.d_const, c.d_rescale, c.n, l, c.L, c.mods[l]);
  ntt_forward(c, t.p, npoly, (size_t)l * c.n, l, LimbMap::contiguous(0));
  FHE_LAUNCH(c, "k_rescale_combine", k_rescale_combine, grid_for(c, l, npoly), dim3(tpb_for(c)), 0, out, a, t.p, c.d_const, c.d_rescale, c.n, l, c.L);
}

void poly_rescale_many(Context& c, uint64_t* const* outs, const uint64_t* const* as,
                       uint32_t count, uint32_t npoly, uint32_t nq) {
  if (nq < 2) throw ArgError("rescale needs at least two limbs");
  if (c.log_n >= 13 && c.log_n <= 17) {
    rescale_fused_many(c, outs, as, count, npoly, nq);
    return;
  }
  for (uint32_t r = 0; r < count; ++r) poly_rescale(c, outs[r], as[r], npoly, nq);
}


void poly_mac_giants(Context& c, uint64_t* const* acc, uint32_t ng, const uint64_t* const* x,
                     uint32_t nb, const uint64_t* const* w, uint32_t nq) {
  if (nb == 0 || nb > MACG_MAX_B || ng > MACG_MAX_G) throw ArgError("giant-step inner sums");
  if (ng == 0) return;
  MacGiants t{};
  for (uint32_t b = 0; b < nb; ++b) t.x[b] = x[b];
  for (uint32_t g = 0; g < ng; ++g) {
    t.acc[g] = acc[g];
    for (uint32_t b = 0; b < nb; ++b) t.w[g][b] = w[(size_t)g * nb + b];
  }
  const uint32_t tpb = c.n < TPB ? c.n : TPB;
  const dim3 grid(c.n / tpb, nq);
  switch (ng) {
#define CASE(G)                                                                           \
  case G:                                                                                 \
    FHE_LAUNCH(c, "k_mac_giants", k_mac_giants<G>, grid, dim3(tpb), 0, t, c.d_const, c.n, \
               nq, nb);                                                                   \
    break;
    CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
#undef CASE
  }
}

}  // namespace fhe
