// Negacyclic RNS NTT / inverse NTT for gfx950.
//
// Forward transform = OpenFHE's ForwardTransformToBitReverseInPlace (the
// transform behind every FIDESlib NTT_ launch the reference makes,
// experiments/ntt_warp_tail/probe.cu:58-66): Cooley-Tukey stages with
// twiddles psi^brv(m+i), output slot i holding a(psi^(2 brv(i) + 1)).
// The inverse runs Gentleman-Sande stages with psi^-brv(m+i), then N^-1.
//
// Structure.  For N = 2^logN with logN >= 13 the transform is split into
// two launches over "lines":
//   COLS   line c in [0, N2): elements c + N2*u, u in [0, N1)  (stages that
//          pair elements at distance >= N2; S1 = ceil(logN/2) stages)
//   BLOCKS line b in [0, N1): elements b*N2 + u, u in [0, N2)  (the last
//          S2 = floor(logN/2) stages)
// Rings with logN <= 12 use one launch (SINGLE) per limb.  Each thread
// holds 16 elements in registers and runs 4 stages at a time (radix-16;
// the ModDown epilogue pass holds 8 and runs 3, see RHO_EPILOGUE);
// sub-passes exchange through an LDS tile padded by one word per 16 words,
// which keeps both the stride-1 and the stride-16 access patterns free of
// bank conflicts.  Workgroups are 256 threads (4096 elements, ~35 KB LDS).
//
// Arithmetic: Harvey lazy butterflies with an approximate-quotient Shoup
// product (shoup_lazy4n, result in [0, 4q)).  Forward values stay in [0, 8q),
// inverse values in [0, 4q); the final launch reduces to [0, q).  This
// needs 8q < 2^64, guaranteed by q < 2^61.
//
// Grid: (tiles per limb, poly, limb).  The limb index is the slowest grid
// dimension so consecutive workgroups share one modulus and its twiddle
// table stays hot in L2.
#include "ops.hpp"

#include <type_traits>

namespace fhe {
namespace {

enum Kind { SINGLE = 0, COLS = 1, BLOCKS = 2 };

// RHO stages per sub-pass, radix 2^RHO per thread.  Plain passes are
// ALU-bound and use radix 16 (two sub-passes for 8 stages); the ModDown
// epilogue pass uses radix 8 in its two-launch form: half the LDS and
// registers per wave, so twice the waves to cover its extra global loads.
constexpr int RHO_PLAIN = 4, RHO_EPILOGUE = 3;

template <int S, int RHO_>
struct Geo {
  static constexpr int RHO = RHO_;
  static constexpr int TPL = 1 << (S - RHO);  // threads per line
  static constexpr int LEN = 1 << S;
  static constexpr int PITCH = LEN + LEN / 16 + 1;
};

__device__ __forceinline__ uint32_t lds_idx(uint32_t line, uint32_t u, uint32_t pitch) {
  return line * pitch + u + (u >> 4);
}

// Base of launch poly p: data + p * poly_stride, or the table's entry for
// polys held in separate allocations.
template <class Map>
__device__ __forceinline__ uint64_t* poly_base(const Map&, uint64_t* data, size_t poly_stride,
                                               uint32_t p) {
  return data + (size_t)p * poly_stride;
}
__device__ __forceinline__ uint64_t* poly_base(const TableMap& m, uint64_t*, size_t, uint32_t p) {
  return m.table[p];
}

// Final stores go through `store.fin(base, offset_in_limb, value, t, q)`,
// with t = store.pre(offset_in_limb, q) when Store::kPre.
// The first pass's input comes from `load.get(offset_in_limb, q)` instead
// of data when Load::kLoad.  kPair functors also produce the terms of two
// adjacent positions from 16-byte loads in two steps, fetch2 (every load of
// the pair, issued together into an Ops2) and comb2 (the arithmetic).
// Prefetching the next pair's operands before a pair's products was
// measured slower: the extra registers cost more waves than they hide.
struct PlainLoad {
  static constexpr bool kLoad = false;
  static constexpr bool kPair = false;
  struct Ops2 {};
  __device__ __forceinline__ void fetch2(size_t, Ops2&) const {}
  __device__ __forceinline__ void comb2(const Ops2&, uint64_t, uint64_t&, uint64_t&) const {}
  __device__ __forceinline__ uint64_t get(size_t, uint64_t) const { return 0; }
};

// LDS writes of this wavefront before the call are seen by its reads after
// the call (LDS executes a wavefront's instructions in order; this keeps the
// compiler from moving accesses across).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// BLK_IN / BLK_OUT (BLOCKS kind): the first pass's input / the last pass's
// output uses the blocked layout described with blocked_off below.  A
// workgroup's tile then still occupies the words [wg0, wg0 + LINES * LEN),
// in the order p = u * LINES + line, and is staged through LDS whatever the
// window.
//
// BLOCKS launches keep every line inside one wavefront (TPL <= 64 lanes, LPW
// = 64 / TPL lines per wave), so their sub-passes exchange through LDS with
// wavefront-level ordering only, and staging of a contiguous window is done
// per wavefront over its own lines (two adjacent words per lane, one
// 1024-byte run per instruction; 8-byte accesses measured 4% slower in the
// inverse block pass).  Only blocked-layout staging, which interleaves the
// lines of the whole workgroup word by word, keeps a workgroup barrier.
struct PlainStore;
template <int S, int KIND, bool INV, int RHO_, class Store, class Load = PlainLoad,
          class Map = LimbMap, bool BLK_IN = false, bool BLK_OUT = false>
__device__ __forceinline__ void ntt_body(uint64_t* __restrict__ data, size_t poly_stride,
                                         const ModConst* __restrict__ mc,
                                         const uint64_t* __restrict__ tw_all, uint32_t log_n,
                                         Map map, uint32_t s_other, int last,
                                         const Store& store, const Load& load = Load{}) {
  using G = Geo<S, RHO_>;
  constexpr int RHO = G::RHO;
  constexpr int R = 1 << RHO;
  constexpr int LINES = KIND == SINGLE ? 1 : 256 / G::TPL;
  constexpr int NSP = (S + RHO - 1) / RHO;
  __shared__ uint64_t lds[LINES * G::PITCH];

  const uint32_t n = 1u << log_n;
  // Workgroup-uniform: a slot without work exits before any barrier.
  uint32_t pos, midx;
  if (!map.resolve(blockIdx.y, blockIdx.z, pos, midx)) return;
  // Lazy ranges (approximate Shoup products land in [0, 4q)): forward
  // stage outputs stay in [0, 8q), inverse ones in [0, 4q); 8q < 2^64 as
  // every prime is below 2^61.
  const uint64_t q = mc[midx].q, q4 = 4 * q, qneg = mc[midx].neg_q, q4neg = mc[midx].neg_q4;
  const uint64_t* __restrict__ tw = tw_all + (size_t)midx * n * 2;
  uint64_t* __restrict__ base = poly_base(map, data, poly_stride, blockIdx.y) + (size_t)pos * n;

  const uint32_t tid = threadIdx.x;
  uint32_t line, tau;
  if (KIND == COLS) {
    line = tid % LINES;
    tau = tid / LINES;
  } else {
    tau = tid % G::TPL;
    line = tid / G::TPL;
  }
  const uint32_t gline = blockIdx.x * LINES + line;
  const uint32_t twbase = KIND == BLOCKS ? (1u << s_other) + gline : 1u;
  constexpr bool WL = KIND == BLOCKS;
  static_assert(!WL || G::TPL <= 64, "a block line spans one wavefront");
  // Staged position k of this thread: per wavefront (WL) or per workgroup.
  // PAIR (every BLOCKS launch): a lane stages two adjacent positions at a
  // time, so plain staged loads and stores and the kPair functors' operands
  // are 16-byte accesses: staged position k is
  // wave * 64R + (k / 2) * 128 + 2 * lane + k % 2.
  constexpr bool PAIR = WL;
  constexpr bool PLAIN_ST = std::is_same<Store, PlainStore>::value;
  auto staged = [&](int k) -> uint32_t {
    if (PAIR)
      return (tid >> 6) * (64u * R) + (uint32_t)(k >> 1) * 128u + 2 * (tid & 63) + (k & 1);
    return WL ? (tid >> 6) * (64u * R) + (uint32_t)k * 64u + (tid & 63)
              : (uint32_t)k * blockDim.x + tid;
  };
  auto sync_lines = [&]() {
    if (WL) wave_lds_sync();
    else __syncthreads();
  };

  uint64_t x[R];
  uint64_t pre[Store::kPre ? R : 1];

#pragma unroll
  for (int sp = 0; sp < NSP; ++sp) {
    // Window [w, w + RHO) of line-local index bits held by this thread, and
    // the stage bits [blo, bhi] processed in this sub-pass.
    int w, blo, bhi;
    if (!INV) {
      const int hi = S - RHO * sp;
      w = hi >= RHO ? hi - RHO : 0;
      bhi = hi - 1;
      blo = w;
    } else {
      const int lo = RHO * sp;
      w = lo + RHO <= S ? lo : S - RHO;
      blo = lo;
      bhi = lo + RHO <= S ? lo + RHO - 1 : S - 1;
    }
    const uint32_t thi = (tau >> w) << (w + RHO), tlo = tau & ((1u << w) - 1);
    // In BLOCKS / SINGLE launches a window at bit 0 gives each thread 16
    // consecutive words; global traffic for such a window goes through LDS
    // so that lanes touch consecutive addresses.
    const bool contiguous = KIND != COLS && w == 0;

    if (sp == 0 && (contiguous || BLK_IN)) {
      const size_t wg0 = ((size_t)blockIdx.x * LINES) << S;
      if constexpr (Load::kPair && PAIR && !BLK_IN) {
#pragma unroll
        for (int k = 0; k < R; k += 2) {
          const uint32_t p = staged(k);
          typename Load::Ops2 ops;
          uint64_t v0, v1;
          load.fetch2(wg0 + p, ops);
          load.comb2(ops, q, v0, v1);
          lds[lds_idx(p >> S, p & (G::LEN - 1), G::PITCH)] = v0;
          lds[lds_idx((p + 1) >> S, (p + 1) & (G::LEN - 1), G::PITCH)] = v1;
        }
      } else if constexpr (PAIR && !Load::kLoad && !BLK_IN) {
#pragma unroll
        for (int k = 0; k < R; k += 2) {
          const uint32_t p = staged(k);
          const ulonglong2 v2 = *reinterpret_cast<const ulonglong2*>(base + wg0 + p);
          lds[lds_idx(p >> S, p & (G::LEN - 1), G::PITCH)] = v2.x;
          lds[lds_idx((p + 1) >> S, (p + 1) & (G::LEN - 1), G::PITCH)] = v2.y;
        }
      } else {
#pragma unroll
        for (int k = 0; k < R; ++k) {
          const uint32_t p = BLK_IN ? (uint32_t)k * blockDim.x + tid : staged(k);
          const uint32_t li = BLK_IN ? lds_idx(p % LINES, p / LINES, G::PITCH)
                                     : lds_idx(p >> S, p & (G::LEN - 1), G::PITCH);
          lds[li] = Load::kLoad ? load.get(wg0 + p, q) : base[wg0 + p];
        }
      }
      if (BLK_IN) __syncthreads();
      else sync_lines();
#pragma unroll
      for (int v = 0; v < R; ++v) {
        const uint32_t u = thi | ((uint32_t)v << w) | tlo;
        x[v] = lds[lds_idx(line, u, G::PITCH)];
      }
    } else if (sp == 0) {
#pragma unroll
      for (int v = 0; v < R; ++v) {
        const uint32_t u = thi | ((uint32_t)v << w) | tlo;
        const size_t g = KIND == COLS ? gline + ((size_t)u << s_other) : ((size_t)gline << S) + u;
        x[v] = Load::kLoad ? load.get(g, q) : base[g];
      }
    } else {
      sync_lines();
#pragma unroll
      for (int v = 0; v < R; ++v) {
        const uint32_t u = thi | ((uint32_t)v << w) | tlo;
        x[v] = lds[lds_idx(line, u, G::PITCH)];
      }
    }
    // Store-side terms for this thread's final positions, loaded ahead of the
    // butterflies: with the first sub-pass when the final window is
    // contiguous (staged positions do not depend on the window), else with
    // the last one.
    constexpr bool kFinalContig = !INV && KIND != COLS;
    if (Store::kPre && last && sp == (kFinalContig ? 0 : NSP - 1)) {
      const size_t wg0 = ((size_t)blockIdx.x * LINES) << S;
      if constexpr (Store::kPair && PAIR && kFinalContig) {
#pragma unroll
        for (int k = 0; k < R; k += 2) {
          typename Store::Ops2 ops;
          store.fetch2(wg0 + staged(k), ops);
          store.comb2(ops, q, pre[k], pre[k + 1]);
        }
      } else {
#pragma unroll
        for (int k = 0; k < R; ++k) {
          const uint32_t u = thi | ((uint32_t)k << w) | tlo;
          const size_t g = kFinalContig ? wg0 + staged(k)
                           : KIND == COLS ? gline + ((size_t)u << s_other)
                                          : ((size_t)gline << S) + u;
          pre[Store::kPre ? k : 0] = store.pre(g, q);
        }
      }
    }

    if (!INV) {
#pragma unroll
      for (int beta = bhi; beta >= blo; --beta) {
        const int d = 1 << (beta - w);
#pragma unroll
        for (int v = 0; v < R; ++v) {
          if (v & d) continue;
          const uint32_t u = thi | ((uint32_t)v << w) | tlo;
          const uint32_t ti = (twbase << (S - 1 - beta)) | (u >> (beta + 1));
          const uint64_t wv = tw[2 * ti], ws = tw[2 * ti + 1];
          const uint64_t X = lazy_sub(x[v], q4neg);
          const uint64_t T = shoup_lazy4n(x[v + d], wv, ws, qneg);
          x[v] = X + T;
          x[v + d] = X + q4 - T;
        }
      }
    } else {
#pragma unroll
      for (int beta = blo; beta <= bhi; ++beta) {
        const int d = 1 << (beta - w);
#pragma unroll
        for (int v = 0; v < R; ++v) {
          if (v & d) continue;
          const uint32_t u = thi | ((uint32_t)v << w) | tlo;
          const uint32_t ti = (twbase << (S - 1 - beta)) | (u >> (beta + 1));
          const uint64_t wv = tw[2 * ti], ws = tw[2 * ti + 1];
          const uint64_t X = x[v], Y = x[v + d];
          x[v + d] = shoup_lazy4n(X + q4 - Y, wv, ws, qneg);
          x[v] = lazy_sub(X + Y, q4neg);
        }
      }
    }

    if (sp == NSP - 1) {
      if (last) {
        if (!INV) {
#pragma unroll
          for (int v = 0; v < R; ++v) x[v] = reduce_8q(x[v], q);
        } else {
          const uint64_t ni = mc[midx].ninv, nis = mc[midx].ninv_sh;
#pragma unroll
          for (int v = 0; v < R; ++v) x[v] = reduce_4q(shoup_lazy4(x[v], ni, nis, q), q);
        }
      }
      if (contiguous || BLK_OUT) {
        if (sp > 0 || NSP == 1) sync_lines();
#pragma unroll
        for (int v = 0; v < R; ++v) {
          const uint32_t u = thi | ((uint32_t)v << w) | tlo;
          lds[lds_idx(line, u, G::PITCH)] = x[v];
        }
        if (BLK_OUT) __syncthreads();
        else sync_lines();
        const size_t wg0 = ((size_t)blockIdx.x * LINES) << S;
        if constexpr (PAIR && PLAIN_ST && !BLK_OUT) {
#pragma unroll
          for (int k = 0; k < R; k += 2) {
            const uint32_t p = staged(k);
            *reinterpret_cast<ulonglong2*>(base + wg0 + p) =
                ulonglong2{lds[lds_idx(p >> S, p & (G::LEN - 1), G::PITCH)],
                           lds[lds_idx((p + 1) >> S, (p + 1) & (G::LEN - 1), G::PITCH)]};
          }
        } else {
#pragma unroll
          for (int k = 0; k < R; ++k) {
            const uint32_t p = BLK_OUT ? (uint32_t)k * blockDim.x + tid : staged(k);
            const uint32_t li = BLK_OUT ? lds_idx(p % LINES, p / LINES, G::PITCH)
                                        : lds_idx(p >> S, p & (G::LEN - 1), G::PITCH);
            store.fin(base, wg0 + p, lds[li], pre[Store::kPre ? k : 0], q);
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < R; ++v) {
          const uint32_t u = thi | ((uint32_t)v << w) | tlo;
          const size_t g =
              KIND == COLS ? gline + ((size_t)u << s_other) : ((size_t)gline << S) + u;
          store.fin(base, g, x[v], pre[Store::kPre ? v : 0], q);
        }
      }
    } else {
      if (sp > 0 || (KIND != COLS && INV)) sync_lines();
#pragma unroll
      for (int v = 0; v < R; ++v) {
        const uint32_t u = thi | ((uint32_t)v << w) | tlo;
        lds[lds_idx(line, u, G::PITCH)] = x[v];
      }
    }
  }
}

// Store functors of the last pass.  kPre: the store adds a term t(s) that
// does not depend on the transform (pre), loaded for all of a thread's
// positions before the last sub-pass so its global loads overlap the
// butterflies; fin then writes f(y, t).
struct PlainStore {
  static constexpr bool kPre = false;
  static constexpr bool kPair = false;
  struct Ops2 {};
  __device__ __forceinline__ void fetch2(size_t, Ops2&) const {}
  __device__ __forceinline__ void comb2(const Ops2&, uint64_t, uint64_t&, uint64_t&) const {}
  __device__ __forceinline__ uint64_t pre(size_t, uint64_t) const { return 0; }
  __device__ __forceinline__ void fin(uint64_t* base, size_t g, uint64_t v, uint64_t,
                                      uint64_t) const {
    base[g] = v;
  }
};

__device__ __forceinline__ uint32_t brev_bits(uint32_t x, uint32_t bits) {
  return __brev(x) >> (32 - bits);
}

// Switching-key words are read once per launch: their loads are marked
// non-temporal so that they do not displace the digits, which every key
// switch of the batch re-reads, from the caches (measured ~1% faster on the
// ModDown passes; non-temporal stores of the outputs were slower).
__device__ __forceinline__ uint64_t load_stream(const uint64_t* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ ulonglong2 load_stream2(const uint64_t* p) {
  typedef unsigned long long v2u __attribute__((ext_vector_type(2)));
  const v2u v = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p));
  ulonglong2 r;
  r.x = v.x;
  r.y = v.y;
  return r;
}

// Key inner product sum_j d_j k_j reduced once by REDC (keys in Montgomery
// form).  SPLIT (every modulus below 2^60, at most 7 digits): operands split
// at bit 30 and accumulated carry-free in three 64-bit sums with
// v_mad_u64_u32, T = a0 + a1 2^30 + a2 2^60; otherwise 128-bit products.
template <int ND, bool SPLIT>
__device__ __forceinline__ uint64_t key_dot(const uint64_t* dg, size_t dstride, const uint64_t* kr,
                                            size_t kstride, uint32_t nd_rt, uint64_t q,
                                            uint64_t qinv_neg) {
  if constexpr (SPLIT && ND > 0 && ND <= 7) {
    constexpr uint32_t M30 = (1u << 30) - 1;
    uint64_t a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const uint64_t d = dg[j * dstride], k = load_stream(kr + j * kstride);
      const uint32_t dl = (uint32_t)d & M30, dh = (uint32_t)(d >> 30);
      const uint32_t kl = (uint32_t)k & M30, kh = (uint32_t)(k >> 30);
      a0 += (uint64_t)dl * kl;
      a1 += (uint64_t)dl * kh;
      a1 += (uint64_t)dh * kl;
      a2 += (uint64_t)dh * kh;
    }
    const uint64_t m1 = a1 << 30, m2 = a2 << 60;
    const uint64_t lo = a0 + m1;
    uint64_t hi = (a1 >> 34) + (a2 >> 4) + (lo < m1);
    const uint64_t lo2 = lo + m2;
    hi += lo2 < m2;
    return redc(hi, lo2, q, qinv_neg);
  } else {
    Acc128 acc;
    if (ND > 0) {
#pragma unroll
      for (int j = 0; j < ND; ++j) acc.mac(dg[j * dstride], load_stream(kr + j * kstride));
    } else {
      for (uint32_t j = 0; j < nd_rt; ++j) acc.mac(dg[j * dstride], load_stream(kr + j * kstride));
    }
    return redc(acc.hi, acc.lo, q, qinv_neg);
  }
}

// key_dot for positions s and s + 1 (s even, operands 16-byte aligned) with
// 16-byte loads, in the SPLIT form only (every modulus below 2^60, 1..7
// digits): half the load instructions of two key_dot calls.  key_fetch2
// issues the loads, key_comb2 forms the two sums.
template <int ND>
__device__ __forceinline__ void key_fetch2(const uint64_t* dg, size_t dstride, const uint64_t* kr,
                                           size_t kstride, ulonglong2* d, ulonglong2* k) {
  static_assert(ND > 0 && ND <= 7, "split key products");
#pragma unroll
  for (int j = 0; j < ND; ++j) {
    d[j] = *reinterpret_cast<const ulonglong2*>(dg + j * dstride);
    k[j] = load_stream2(kr + j * kstride);
  }
}
template <int ND>
__device__ __forceinline__ void key_comb2(const ulonglong2* d, const ulonglong2* k, uint64_t q,
                                          uint64_t qinv_neg, uint64_t& t0, uint64_t& t1) {
  constexpr uint32_t M30 = (1u << 30) - 1;
  uint64_t a0[2] = {0, 0}, a1[2] = {0, 0}, a2[2] = {0, 0};
#pragma unroll
  for (int j = 0; j < ND; ++j) {
    const uint64_t dd[2] = {d[j].x, d[j].y}, kk[2] = {k[j].x, k[j].y};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t dl = (uint32_t)dd[h] & M30, dh = (uint32_t)(dd[h] >> 30);
      const uint32_t kl = (uint32_t)kk[h] & M30, kh = (uint32_t)(kk[h] >> 30);
      a0[h] += (uint64_t)dl * kl;
      a1[h] += (uint64_t)dl * kh;
      a1[h] += (uint64_t)dh * kl;
      a2[h] += (uint64_t)dh * kh;
    }
  }
  uint64_t t[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint64_t m1 = a1[h] << 30, m2 = a2[h] << 60;
    const uint64_t lo = a0[h] + m1;
    uint64_t hi = (a1[h] >> 34) + (a2[h] >> 4) + (lo < m1);
    const uint64_t lo2 = lo + m2;
    hi += lo2 < m2;
    t[h] = redc(hi, lo2, q, qinv_neg);
  }
  t0 = t[0];
  t1 = t[1];
}

// key_comb2 with the reduction left lazy: redc_lazy, each sum in (0, 2q)
// (T < nd q^2 keeps T's high word below q for nd q < 2^64).
template <int ND>
__device__ __forceinline__ void key_comb2_lazy(const ulonglong2* d, const ulonglong2* k,
                                               uint64_t q, uint64_t qinv, uint64_t& t0,
                                               uint64_t& t1) {
  constexpr uint32_t M30 = (1u << 30) - 1;
  uint64_t a0[2] = {0, 0}, a1[2] = {0, 0}, a2[2] = {0, 0};
#pragma unroll
  for (int j = 0; j < ND; ++j) {
    const uint64_t dd[2] = {d[j].x, d[j].y}, kk[2] = {k[j].x, k[j].y};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t dl = (uint32_t)dd[h] & M30, dh = (uint32_t)(dd[h] >> 30);
      const uint32_t kl = (uint32_t)kk[h] & M30, kh = (uint32_t)(kk[h] >> 30);
      a0[h] += (uint64_t)dl * kl;
      a1[h] += (uint64_t)dl * kh;
      a1[h] += (uint64_t)dh * kl;
      a2[h] += (uint64_t)dh * kh;
    }
  }
  uint64_t t[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint64_t m1 = a1[h] << 30, m2 = a2[h] << 60;
    const uint64_t lo = a0[h] + m1;
    uint64_t hi = (a1[h] >> 34) + (a2[h] >> 4) + (lo < m1);
    const uint64_t lo2 = lo + m2;
    hi += lo2 < m2;
    t[h] = redc_lazy(hi, lo2, q, qinv);
  }
  t0 = t[0];
  t1 = t[1];
}

// ModDown epilogue (see ModDownEpi): the value at evaluation slot s goes to
// slot d(s) of the output, d being the inverse Galois permutation.  ND > 0
// fixes the digit count at compile time (ND = 0: e.nd at run time).
template <int ND, bool SPLIT = false>
struct EpiStore {
  static constexpr bool kPre = true;
  static constexpr bool kPair = SPLIT && ND > 0 && ND <= 7;
  const ModDownEpi& e;
  uint32_t n, log_n;
  // pre() for positions s and s + 1 (s even), kPair only.  The addend is
  // loaded with the key operands; without one the first digit's words are
  // read again (a cache hit) so that the load needs no branch.
  struct Ops2 {
    ulonglong2 d[kPair ? ND : 1], k[kPair ? ND : 1], add;
  };
  __device__ __forceinline__ void fetch2(size_t s, Ops2& o) const {
    if constexpr (kPair) {
      const uint32_t p = blockIdx.y, r = p >> 1, b = p & 1, i = blockIdx.z;
      const uint64_t* dg = e.digits[r] + (size_t)i * n + s;
      key_fetch2<ND>(dg, (size_t)e.ne * n, e.key[r] + (size_t)b * e.kl + (size_t)i * n + s,
                     2 * e.kl, o.d, o.k);
      const uint64_t* add = e.add[r][b];
      o.add = *reinterpret_cast<const ulonglong2*>(add ? add + (size_t)i * n + s : dg);
    }
  }
  __device__ __forceinline__ void comb2(const Ops2& o, uint64_t q, uint64_t& t0,
                                        uint64_t& t1) const {
    if constexpr (kPair) {
      const uint32_t p = blockIdx.y, r = p >> 1, b = p & 1, i = blockIdx.z;
      key_comb2<ND>(o.d, o.k, q, e.mc[i].qinv_neg, t0, t1);
      if (e.add[r][b]) {
        t0 = add_mod(t0, o.add.x, q);
        t1 = add_mod(t1, o.add.y, q);
      }
    }
  }
  // Q-limb key inner product plus the addend at position s.
  __device__ __forceinline__ uint64_t pre(size_t s, uint64_t q) const {
    const uint32_t p = blockIdx.y, r = p >> 1, b = p & 1, i = blockIdx.z;
    const uint64_t* dg = e.digits[r] + (size_t)i * n + s;
    const uint64_t* kr = e.key[r] + (size_t)b * e.kl + (size_t)i * n + s;
    const size_t dstride = (size_t)e.ne * n, kstride = 2 * e.kl;
    uint64_t t = key_dot<ND, SPLIT>(dg, dstride, kr, kstride, e.nd, q, e.mc[i].qinv_neg);
    const uint64_t* add = e.add[r][b];
    if (add) t = add_mod(t, add[(size_t)i * n + s], q);
    return t;
  }
  __device__ __forceinline__ void fin(uint64_t*, size_t s, uint64_t y, uint64_t t,
                                      uint64_t q) const {
    const uint32_t p = blockIdx.y, r = p >> 1, b = p & 1, i = blockIdx.z;
    const uint64_t res = add_mod(t, y, q);
    uint32_t d = (uint32_t)s;
    const uint32_t gi = e.ginv[r];
    if (gi != 1) {
      // 32-bit wrap-around is exact here: only the product mod 2N matters.
      const uint32_t j = brev_bits((uint32_t)s, log_n);
      const uint32_t ex = ((2u * j + 1u) * gi) & (2u * n - 1u);
      d = brev_bits((ex - 1u) >> 1, log_n);
    }
    e.out[r][((size_t)b * e.nq + i) * n + d] = res;
  }
};

template <int S, int KIND, bool INV, class Map>
__global__ void __launch_bounds__(256)
    ntt_pass(uint64_t* __restrict__ data, size_t poly_stride, const ModConst* __restrict__ mc,
             const uint64_t* __restrict__ tw_all, uint32_t log_n, Map map, uint32_t s_other,
             int last) {
  ntt_body<S, KIND, INV, RHO_PLAIN, PlainStore, PlainLoad, Map>(
      data, poly_stride, mc, tw_all, log_n, map, s_other, last, PlainStore{});
}

// Last forward pass of a batched ModDown (BLOCKS or SINGLE kind).
template <int S, int KIND>
constexpr int epilogue_rho() {
  return KIND == SINGLE ? RHO_PLAIN : RHO_EPILOGUE;
}

// P-limb key inner product as the input of ModDown's inverse NTT: launch
// poly p is key switch r = p / 2, component b = p % 2, limb t is P limb t.
template <int ND, bool SPLIT = false>
struct KskLoad {
  static constexpr bool kLoad = true;
  static constexpr bool kPair = SPLIT && ND > 0 && ND <= 7;
  const ModDownEpi& e;
  uint32_t n;
  __device__ __forceinline__ uint64_t get(size_t s, uint64_t q) const {
    const uint32_t p = blockIdx.y, r = p >> 1, b = p & 1, t = blockIdx.z;
    const uint64_t* dg = e.digits[r] + (size_t)(e.nq + t) * n + s;
    const uint64_t* kr = e.key[r] + (size_t)b * e.kl + (size_t)(e.L + t) * n + s;
    const size_t dstride = (size_t)e.ne * n, kstride = 2 * e.kl;
    return key_dot<ND, SPLIT>(dg, dstride, kr, kstride, e.nd, q, e.mc[e.L + t].qinv_neg);
  }
  // get() for positions s and s + 1 (s even), kPair only.
  struct Ops2 {
    ulonglong2 d[kPair ? ND : 1], k[kPair ? ND : 1];
  };
  __device__ __forceinline__ void fetch2(size_t s, Ops2& o) const {
    if constexpr (kPair) {
      const uint32_t p = blockIdx.y, r = p >> 1, b = p & 1, t = blockIdx.z;
      key_fetch2<ND>(e.digits[r] + (size_t)(e.nq + t) * n + s, (size_t)e.ne * n,
                     e.key[r] + (size_t)b * e.kl + (size_t)(e.L + t) * n + s, 2 * e.kl, o.d,
                     o.k);
    }
  }
  __device__ __forceinline__ void comb2(const Ops2& o, uint64_t q, uint64_t& v0,
                                        uint64_t& v1) const {
    if constexpr (kPair) key_comb2<ND>(o.d, o.k, q, e.mc[e.L + blockIdx.z].qinv_neg, v0, v1);
  }
};

// Blocked limb layout of ModDown's intermediates (P limbs between the first
// inverse pass and the fused middle kernel, y between that kernel and the
// last forward pass).  With the split index s = b * N2 + u (row b < N1,
// column u < N2 = 2^S2), rows are grouped by BLO, the line count of a radix-8
// block-pass workgroup:
//   offset(b, u) = (b / BLO) * BLO * N2 + u * BLO + b % BLO.
// A block-pass workgroup (BLO consecutive rows, all columns) then touches
// one contiguous BLO * N2 run, and a column (all rows, one u) is N1 / BLO
// runs of BLO words.
template <int S2>
constexpr int blocked_rows() {
  return 256 >> (S2 - RHO_EPILOGUE);
}

template <int S2>
__device__ __forceinline__ size_t blocked_off(uint32_t b, uint32_t u) {
  constexpr uint32_t BLO = blocked_rows<S2>();
  return (size_t)(b / BLO) * ((size_t)BLO << S2) + (size_t)u * BLO + (b % BLO);
}

// First inverse pass of ModDown (BLOCKS or SINGLE kind) fed by KskLoad.
// BLK: BLOCKS pass of the fused ModDown (moduli below 2^60), writing the
// blocked layout.
template <int S, int KIND, int ND, bool BLK>
__global__ void __launch_bounds__(256)
    ntt_pass_ksk(uint64_t* __restrict__ data, size_t poly_stride, const ModConst* __restrict__ mc,
                 const uint64_t* __restrict__ tw_all, uint32_t log_n, uint32_t s_other,
                 int last, const ModDownEpi epi) {
  ntt_body<S, KIND, true, epilogue_rho<S, KIND>(), PlainStore, KskLoad<ND, BLK>, LimbMap, false,
           BLK>(data, poly_stride, mc, tw_all, log_n, LimbMap::contiguous(epi.L), s_other, last,
                PlainStore{}, KskLoad<ND, BLK>{epi, 1u << log_n});
}

// BLK: pass of the fused ModDown (moduli below 2^60), y read from the
// blocked layout.
template <int S, int KIND, int ND, bool BLK>
__global__ void __launch_bounds__(256)
    ntt_pass_moddown(uint64_t* __restrict__ data, size_t poly_stride,
                     const ModConst* __restrict__ mc, const uint64_t* __restrict__ tw_all,
                     uint32_t log_n, uint32_t s_other, const ModDownEpi epi) {
  ntt_body<S, KIND, false, epilogue_rho<S, KIND>(), EpiStore<ND, BLK>, PlainLoad, LimbMap, BLK>(
      data, poly_stride, mc, tw_all, log_n, LimbMap::contiguous(0), s_other, 1,
      EpiStore<ND, BLK>{epi, 1u << log_n, log_n});
}

// Last forward pass of a batched ModDown over the blocked y, both polys of
// each key switch in one workgroup (ND = 1..7 digits, every modulus in
// [2^33, 2^60)).  Eight wavefronts; lane tid holds the same R = 4 positions of row
// `line` in both polys (radix 4: one row per wavefront at N2 = 256, two or
// four at 128 / 64), so the digits' words and the twiddles are loaded once
// for both key products and both transforms, and the Galois target index is
// computed once for both stores.  The workgroup's rows are one blocked
// group (LINES = BLO).  Stage order, twiddle indices and lazy ranges are
// those of ntt_body's forward BLOCKS pass; the epilogue is EpiStore's:
// out_b[d(s)] = sum_j digit_j[s] key_j,b[s] (REDC) + add_b[s] + y_b[s].
// Lazy ranges: y arrives below 16q from the middle kernel's alternating
// stages (k_convert_mid, ALT); stages with an even bit beta first bring X
// below 8q (lazy_sub at 8q), the others add to it, so values stay below
// 16q and the last stage (beta = 0) leaves them below 12q.  The key sum
// (redc_lazy, below 2q) plus the addend (below q) plus that is below 15q,
// reduced once by reduce_est.
// The key products are formed after the transform, with the stores: the
// butterflies then hold only the transform's values, and up to three digits
// the kernel fits 64 VGPRs, four 8-wave workgroups per CU (0.84 -> 0.80 ms
// for 30 key switches at N=2^16, 24 limbs, 3 digits, against forming them
// first and keeping them in registers).
// Rows per workgroup of the paired passes (one blocked group) and the LDS
// words of their two-poly tile.
template <int S>
constexpr uint32_t pair_lines() {
  return 512u >> (S - 2);
}
template <int S>
constexpr uint32_t pair_lds_words() {
  return 2 * pair_lines<S>() * ((1u << S) + (1u << S) / 16 + 1);
}

// Twiddle pair of index ti for the paired ModDown passes.  `uniform`: every
// lane of the wavefront holds the same ti (one row per wavefront, and the
// window of the row's top stages, whose indices do not depend on the lane);
// the pair is then read through the scalar cache, leaving the vector memory
// path to the key and digit streams (0.769 -> 0.762 ms for the epilogue of
// 30 key switches at N=2^16, 24 limbs).
__device__ __forceinline__ void pair_twiddle(const uint64_t* tw, uint32_t ti, bool uniform,
                                             uint64_t& wv, uint64_t& ws) {
  if (uniform) {
    typedef const uint64_t __attribute__((address_space(4))) cu64t;
    const uint32_t tiu = __builtin_amdgcn_readfirstlane(ti);
    wv = ((cu64t*)tw)[2 * tiu];
    ws = ((cu64t*)tw)[2 * tiu + 1];
  } else {
    wv = tw[2 * ti];
    ws = tw[2 * ti + 1];
  }
}

// Body of the paired epilogue for the workgroup at row group bx of limb i of
// key switch r, with its tile in lds (pair_lds_words<S>() words).
template <int S, int ND>
__device__ __forceinline__ void moddown_pair_body(const uint64_t* __restrict__ y,
                                                  const ModConst* __restrict__ mc,
                                                  const uint64_t* __restrict__ tw_all,
                                                  uint32_t log_n, uint32_t s_other,
                                                  const ModDownEpi& e, uint32_t bx, uint32_t r,
                                                  uint32_t i, uint64_t* lds_base) {
  constexpr int RHO = 2, R = 4, TPL = 1 << (S - RHO), LINES = 512 / TPL;
  constexpr int NSP = (S + RHO - 1) / RHO;
  constexpr uint32_t LEN = 1u << S, PITCH = LEN + LEN / 16 + 1;
  static_assert(TPL <= 64 && LINES * TPL == 512 && ND > 0 && ND <= 7, "pair epilogue");
  uint64_t* const lds[2] = {lds_base, lds_base + LINES * PITCH};
  const uint32_t n = 1u << log_n, tid = threadIdx.x;
  const uint64_t q = mc[i].q, q4 = 4 * q, qneg = mc[i].neg_q, q8neg = mc[i].neg_q8;
  const float rq = mc[i].rq;
  const uint64_t* __restrict__ tw = tw_all + (size_t)i * n * 2;
  const size_t ps = (size_t)e.nq * n, wg0 = ((size_t)bx * LINES) << S;
  const uint32_t tau = tid % TPL, line = tid / TPL;
  const uint32_t twbase = (1u << s_other) + bx * LINES + line;
  // Key-product and store positions of this lane: two adjacent pairs in its
  // wavefront's own 64R-word run (the wavefront's rows).
  auto staged = [&](int k) -> uint32_t {
    return (tid >> 6) * (64u * R) + (uint32_t)(k >> 1) * 128u + 2 * (tid & 63) + (k & 1);
  };

  // The blocked group of both polys into LDS, word p = u * LINES + row,
  // two adjacent words per lane (16-byte loads).
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint64_t* __restrict__ src = y + (size_t)(2 * r + h) * ps + (size_t)i * n + wg0;
#pragma unroll
    for (int k = 0; k < R; k += 2) {
      const uint32_t p = (uint32_t)k * 512u + 2 * tid;
      const ulonglong2 v = *reinterpret_cast<const ulonglong2*>(src + p);
      lds[h][lds_idx(p % LINES, p / LINES, PITCH)] = v.x;
      lds[h][lds_idx((p + 1) % LINES, (p + 1) / LINES, PITCH)] = v.y;
    }
  }
  __syncthreads();

  uint64_t x[2][R];
#pragma unroll
  for (int sp = 0; sp < NSP; ++sp) {
    const int hi = S - RHO * sp;
    const int w = hi >= RHO ? hi - RHO : 0;
    const uint32_t thi = (tau >> w) << (w + RHO), tlo = tau & ((1u << w) - 1);
    if (sp > 0) wave_lds_sync();
#pragma unroll
    for (int v = 0; v < R; ++v) {
      const uint32_t u = thi | ((uint32_t)v << w) | tlo;
      x[0][v] = lds[0][lds_idx(line, u, PITCH)];
      x[1][v] = lds[1][lds_idx(line, u, PITCH)];
    }
#pragma unroll
    for (int beta = hi - 1; beta >= w; --beta) {
      const int d = 1 << (beta - w);
#pragma unroll
      for (int v = 0; v < R; ++v) {
        if (v & d) continue;
        const uint32_t u = thi | ((uint32_t)v << w) | tlo;
        const uint32_t ti = (twbase << (S - 1 - beta)) | (u >> (beta + 1));
        uint64_t wv, ws;
        pair_twiddle(tw, ti, TPL == 64 && w + RHO >= S, wv, ws);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint64_t X = beta % 2 == 0 ? lazy_sub(x[h][v], q8neg) : x[h][v];
          const uint64_t T = shoup_lazy4n(x[h][v + d], wv, ws, qneg);
          x[h][v] = X + T;
          x[h][v + d] = X + q4 - T;
        }
      }
    }
    wave_lds_sync();
#pragma unroll
    for (int v = 0; v < R; ++v) {
      const uint32_t u = thi | ((uint32_t)v << w) | tlo;
      lds[0][lds_idx(line, u, PITCH)] = x[0][v];
      lds[1][lds_idx(line, u, PITCH)] = x[1][v];
    }
  }
  wave_lds_sync();

  // Key products of both polys at this lane's positions, the digits' words
  // read once (16-byte loads, two positions each), plus the transform, out
  // through the inverse Galois permutation.
  const uint32_t gi = e.ginv[r];
  uint64_t* const out0 = e.out[r] + (size_t)i * n;
  uint64_t* const out1 = e.out[r] + ((size_t)e.nq + i) * n;
  const size_t dstride = (size_t)e.ne * n, kstride = 2 * e.kl;
  const uint64_t* const a0 = e.add[r][0];
  const uint64_t* const a1 = e.add[r][1];
  const uint64_t qn = e.mc[i].qinv;
#pragma unroll
  for (int k = 0; k < R; k += 2) {
    const size_t s0 = wg0 + staged(k);
    const uint64_t* dg = e.digits[r] + (size_t)i * n + s0;
    const uint64_t* kr = e.key[r] + (size_t)i * n + s0;
    ulonglong2 d[ND], k0[ND], k1[ND];
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      d[j] = *reinterpret_cast<const ulonglong2*>(dg + j * dstride);
      k0[j] = load_stream2(kr + j * kstride);
      k1[j] = load_stream2(kr + e.kl + j * kstride);
    }
    const ulonglong2 av = *reinterpret_cast<const ulonglong2*>(a0 ? a0 + (size_t)i * n + s0 : dg);
    uint64_t pre[2][2];
    key_comb2_lazy<ND>(d, k0, q, qn, pre[0][0], pre[0][1]);
    key_comb2_lazy<ND>(d, k1, q, qn, pre[1][0], pre[1][1]);
    if (a0) {
      pre[0][0] += av.x;
      pre[0][1] += av.y;
    }
    if (a1) {
      const ulonglong2 bv = *reinterpret_cast<const ulonglong2*>(a1 + (size_t)i * n + s0);
      pre[1][0] += bv.x;
      pre[1][1] += bv.y;
    }
    // Positions s (even) and s + 1 = s ^ 1 land on d(s) and d(s) ^ 1: the
    // automorphism maps brev(s) + N/2 to its image plus N/2 (mod N), so the
    // pair stays an aligned pair, swapped when d(s) is odd (16-byte stores).
    const uint32_t p = staged(k);
    const uint32_t s = (uint32_t)wg0 + p;
    uint32_t dst = s;
    if (gi != 1) {
      // 32-bit wrap-around is exact here: only the product mod 2N matters.
      const uint32_t jj = brev_bits(s, log_n);
      const uint32_t ex = ((2u * jj + 1u) * gi) & (2u * n - 1u);
      dst = brev_bits((ex - 1u) >> 1, log_n);
    }
    const uint32_t l0 = lds_idx(p >> S, p & (LEN - 1), PITCH);
    const uint32_t l1 = lds_idx((p + 1) >> S, (p + 1) & (LEN - 1), PITCH);
    const uint64_t a0v = reduce_est(pre[0][0] + lds[0][l0], qneg, rq);
    const uint64_t a1v = reduce_est(pre[0][1] + lds[0][l1], qneg, rq);
    const uint64_t b0v = reduce_est(pre[1][0] + lds[1][l0], qneg, rq);
    const uint64_t b1v = reduce_est(pre[1][1] + lds[1][l1], qneg, rq);
    const bool odd = dst & 1u;
    const size_t d2 = dst & ~1u;
    *reinterpret_cast<ulonglong2*>(out0 + d2) = odd ? ulonglong2{a1v, a0v} : ulonglong2{a0v, a1v};
    *reinterpret_cast<ulonglong2*>(out1 + d2) = odd ? ulonglong2{b1v, b0v} : ulonglong2{b0v, b1v};
  }
}

template <int S, int ND>
__global__ void __launch_bounds__(512)
    __attribute__((amdgpu_waves_per_eu(ND <= 3 && S >= 7 ? 6 : ND == 4 && S >= 7 ? 8 : 1, 8)))
    ntt_pass_moddown_pair(const uint64_t* __restrict__ y, const ModConst* __restrict__ mc,
                          const uint64_t* __restrict__ tw_all, uint32_t log_n, uint32_t s_other,
                          const ModDownEpi e) {
  __shared__ uint64_t lds[pair_lds_words<S>()];
  moddown_pair_body<S, ND>(y, mc, tw_all, log_n, s_other, e, blockIdx.x, blockIdx.y, blockIdx.z,
                           lds);
}

// First inverse pass of a batched ModDown with both polys of each key
// switch in one workgroup (the counterpart of ntt_pass_moddown_pair; ND =
// 1..7 digits, every modulus below 2^60): lane tid forms the P-limb key
// products of both polys at the same positions, the digits' words read
// once, runs the first S2 inverse stages of both polys with shared
// twiddles, and the workgroup stores its rows (one blocked group) to the
// blocked layout.  The values stay in [0, 4q); N^-1 is applied later.
// Up to three digits it fits 64 VGPRs without spills, so four 8-wave
// workgroups share a CU (LDS allows four; measured 2% faster than three at
// N=2^16, 24 limbs).
// Body for the workgroup at row group bx of P limb t of key switch r, with
// its tile in lds (pair_lds_words<S>() words).
template <int S, int ND>
__device__ __forceinline__ void ksk_pair_body(uint64_t* __restrict__ ext, size_t ps,
                                              const ModConst* __restrict__ mc,
                                              const uint64_t* __restrict__ tw_all, uint32_t log_n,
                                              uint32_t s_other, const ModDownEpi& e, uint32_t bx,
                                              uint32_t r, uint32_t t, uint64_t* lds_base) {
  constexpr int RHO = 2, R = 4, TPL = 1 << (S - RHO), LINES = 512 / TPL;
  constexpr int NSP = (S + RHO - 1) / RHO;
  constexpr uint32_t LEN = 1u << S, PITCH = LEN + LEN / 16 + 1;
  static_assert(TPL <= 64 && LINES * TPL == 512 && ND > 0 && ND <= 7, "pair ksk pass");
  uint64_t* const lds[2] = {lds_base, lds_base + LINES * PITCH};
  const uint32_t n = 1u << log_n, tid = threadIdx.x;
  const uint32_t midx = e.L + t;
  const uint64_t q = mc[midx].q, q4 = 4 * q, qneg = mc[midx].neg_q, q4neg = mc[midx].neg_q4;
  const uint64_t* __restrict__ tw = tw_all + (size_t)midx * n * 2;
  const size_t wg0 = ((size_t)bx * LINES) << S;
  const uint32_t tau = tid % TPL, line = tid / TPL;
  const uint32_t twbase = (1u << s_other) + bx * LINES + line;
  auto staged = [&](int k) -> uint32_t {
    return (tid >> 6) * (64u * R) + (uint32_t)(k >> 1) * 128u + 2 * (tid & 63) + (k & 1);
  };

  // P-limb key products of both polys into LDS (this wavefront's rows), in
  // (0, 2q) as the first inverse stage accepts them.
  {
    const size_t dstride = (size_t)e.ne * n, kstride = 2 * e.kl;
    const uint64_t qn = e.mc[midx].qinv;
#pragma unroll
    for (int k = 0; k < R; k += 2) {
      const uint32_t p = staged(k);
      const size_t s = wg0 + p;
      const uint64_t* dg = e.digits[r] + (size_t)(e.nq + t) * n + s;
      const uint64_t* kr = e.key[r] + (size_t)midx * n + s;
      ulonglong2 d[ND], k0[ND], k1[ND];
#pragma unroll
      for (int j = 0; j < ND; ++j) {
        d[j] = *reinterpret_cast<const ulonglong2*>(dg + j * dstride);
        k0[j] = load_stream2(kr + j * kstride);
        k1[j] = load_stream2(kr + e.kl + j * kstride);
      }
      uint64_t v0, v1;
      const uint32_t l0 = lds_idx(p >> S, p & (LEN - 1), PITCH);
      const uint32_t l1 = lds_idx((p + 1) >> S, (p + 1) & (LEN - 1), PITCH);
      key_comb2_lazy<ND>(d, k0, q, qn, v0, v1);
      lds[0][l0] = v0;
      lds[0][l1] = v1;
      key_comb2_lazy<ND>(d, k1, q, qn, v0, v1);
      lds[1][l0] = v0;
      lds[1][l1] = v1;
    }
  }

  uint64_t x[2][R];
#pragma unroll
  for (int sp = 0; sp < NSP; ++sp) {
    const int lo = RHO * sp;
    const int w = lo + RHO <= S ? lo : S - RHO;
    const int bhi = lo + RHO <= S ? lo + RHO - 1 : S - 1;
    const uint32_t thi = (tau >> w) << (w + RHO), tlo = tau & ((1u << w) - 1);
    wave_lds_sync();
#pragma unroll
    for (int v = 0; v < R; ++v) {
      const uint32_t u = thi | ((uint32_t)v << w) | tlo;
      x[0][v] = lds[0][lds_idx(line, u, PITCH)];
      x[1][v] = lds[1][lds_idx(line, u, PITCH)];
    }
#pragma unroll
    for (int beta = lo; beta <= bhi; ++beta) {
      const int d = 1 << (beta - w);
#pragma unroll
      for (int v = 0; v < R; ++v) {
        if (v & d) continue;
        const uint32_t u = thi | ((uint32_t)v << w) | tlo;
        const uint32_t ti = (twbase << (S - 1 - beta)) | (u >> (beta + 1));
        uint64_t wv, ws;
        pair_twiddle(tw, ti, TPL == 64 && w + RHO >= S, wv, ws);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint64_t X = x[h][v], Y = x[h][v + d];
          x[h][v + d] = shoup_lazy4n(X + q4 - Y, wv, ws, qneg);
          x[h][v] = lazy_sub(X + Y, q4neg);
        }
      }
    }
    wave_lds_sync();
#pragma unroll
    for (int v = 0; v < R; ++v) {
      const uint32_t u = thi | ((uint32_t)v << w) | tlo;
      lds[0][lds_idx(line, u, PITCH)] = x[0][v];
      lds[1][lds_idx(line, u, PITCH)] = x[1][v];
    }
  }
  __syncthreads();

  // The blocked group of both polys, word p = u * LINES + row, two adjacent
  // words per lane (16-byte stores).
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint64_t* __restrict__ dst = ext + (size_t)(2 * r + h) * ps + (size_t)t * n + wg0;
#pragma unroll
    for (int k = 0; k < R; k += 2) {
      const uint32_t p = (uint32_t)k * 512u + 2 * tid;
      *reinterpret_cast<ulonglong2*>(dst + p) =
          ulonglong2{lds[h][lds_idx(p % LINES, p / LINES, PITCH)],
                     lds[h][lds_idx((p + 1) % LINES, (p + 1) / LINES, PITCH)]};
    }
  }
}

template <int S, int ND>
__global__ void __launch_bounds__(512)
    __attribute__((amdgpu_waves_per_eu(ND <= 4 ? 8 : 1, 8)))
    ntt_pass_ksk_pair(uint64_t* __restrict__ ext, size_t ps, const ModConst* __restrict__ mc,
                      const uint64_t* __restrict__ tw_all, uint32_t log_n, uint32_t s_other,
                      const ModDownEpi e) {
  __shared__ uint64_t lds[pair_lds_words<S>()];
  ksk_pair_body<S, ND>(ext, ps, mc, tw_all, log_n, s_other, e, blockIdx.x, blockIdx.y, blockIdx.z,
                       lds);
}

// ---- Rescale in four launches (ring dimensions 2^13 .. 2^17) ----
// The rescale's passes run radix 8 (RHO_EPILOGUE: eight lines of 2^S
// words, 17 KB of LDS and ~60 VGPRs per 256-lane workgroup), so one
// ciphertext's launch fits the chip in one round of workgroups.
// The inverse NTT of the last limb reads it from the input (LastLimbLoad);
// the forward column pass lifts it to modulus i as it loads (LiftLoad:
// x mod q_i, minus q_l mod q_i in the upper half, the centred lift); the
// last forward pass stores (a_i - t_i) * q_l^-1 (RescaleStore).  One launch
// set rescales up to RESCALE_MAX inputs of npoly polys each: launch poly y
// is poly y % npoly of input y / npoly, whose addresses come from a table
// in the kernel arguments.
constexpr int RESCALE_MAX = 16;
struct RescalePtrs {
  const uint64_t* a[RESCALE_MAX];
  uint64_t* out[RESCALE_MAX];
};
struct LastLimbLoad {
  static constexpr bool kLoad = true;
  static constexpr bool kPair = false;
  const uint64_t* const* a;  // RESCALE_MAX entries in kernel arguments
  uint32_t npoly;
  size_t poly_words, last_off;
  __device__ __forceinline__ uint64_t get(size_t g, uint64_t) const {
    const uint32_t y = blockIdx.y;
    return a[y / npoly][(size_t)(y % npoly) * poly_words + last_off + g];
  }
  struct Ops2 {};
  __device__ __forceinline__ void fetch2(size_t, Ops2&) const {}
  __device__ __forceinline__ void comb2(const Ops2&, uint64_t, uint64_t&, uint64_t&) const {}
};
struct LiftLoad {
  static constexpr bool kLoad = true;
  static constexpr bool kPair = false;
  const uint64_t* last;  // [npoly][N], coefficient form mod q_l, in [0, q_l)
  const ModConst* mc;
  const uint64_t* rs;
  uint32_t n, l, L;
  uint64_t half;         // q_l >> 1
  __device__ __forceinline__ uint64_t get(size_t g, uint64_t q) const {
    const uint32_t i = blockIdx.z;
    const uint64_t x = last[(size_t)blockIdx.y * n + g];
    const uint64_t r = reduce_2q(x - mulhi64(x, mc[i].mu64) * q, q);
    return x > half ? sub_mod(r, rs[((size_t)l * L + i) * 4], q) : r;
  }
  struct Ops2 {};
  __device__ __forceinline__ void fetch2(size_t, Ops2&) const {}
  __device__ __forceinline__ void comb2(const Ops2&, uint64_t, uint64_t&, uint64_t&) const {}
};
struct RescaleStore {
  static constexpr bool kPre = true;
  static constexpr bool kPair = false;
  const uint64_t* const* a;  // RESCALE_MAX entries in kernel arguments
  uint64_t* const* out;
  const uint64_t* rs;
  uint32_t n, l, L, npoly;
  __device__ __forceinline__ uint64_t pre(size_t s, uint64_t) const {
    const uint32_t y = blockIdx.y;
    return a[y / npoly][((size_t)(y % npoly) * (l + 1) + blockIdx.z) * n + s];
  }
  struct Ops2 {};
  __device__ __forceinline__ void fetch2(size_t, Ops2&) const {}
  __device__ __forceinline__ void comb2(const Ops2&, uint64_t, uint64_t&, uint64_t&) const {}
  __device__ __forceinline__ void fin(uint64_t*, size_t s, uint64_t y, uint64_t x,
                                      uint64_t q) const {
    const uint32_t i = blockIdx.z, p = blockIdx.y;
    const uint64_t* c = rs + ((size_t)l * L + i) * 4;
    out[p / npoly][((size_t)(p % npoly) * l + i) * n + s] = shoup(x + q - y, c[1], c[2], q);
  }
};

template <int S>
__global__ void __launch_bounds__(256)
    ntt_pass_rescale_in(uint64_t* __restrict__ last, const ModConst* __restrict__ mc,
                        const uint64_t* __restrict__ tw_all, uint32_t log_n, uint32_t s_other,
                        const RescalePtrs ptrs, uint32_t npoly, size_t poly_words, uint32_t l) {
  ntt_body<S, BLOCKS, true, RHO_EPILOGUE, PlainStore, LastLimbLoad>(
      last, (size_t)1 << log_n, mc, tw_all, log_n, LimbMap::contiguous(l), s_other, 0,
      PlainStore{}, LastLimbLoad{ptrs.a, npoly, poly_words, (size_t)l << log_n});
}

template <int S>
__global__ void __launch_bounds__(256)
    ntt_pass_rescale_lift(uint64_t* __restrict__ t, size_t poly_stride,
                          const ModConst* __restrict__ mc, const uint64_t* __restrict__ tw_all,
                          uint32_t log_n, uint32_t s_other, const LiftLoad ld) {
  ntt_body<S, COLS, false, RHO_EPILOGUE, PlainStore, LiftLoad>(
      t, poly_stride, mc, tw_all, log_n, LimbMap::contiguous(0), s_other, 0, PlainStore{}, ld);
}

template <int S>
__global__ void __launch_bounds__(256)
    ntt_pass_rescale_out(uint64_t* __restrict__ t, size_t poly_stride,
                         const ModConst* __restrict__ mc, const uint64_t* __restrict__ tw_all,
                         uint32_t log_n, uint32_t s_other, const RescalePtrs ptrs,
                         const uint64_t* __restrict__ rs, uint32_t l, uint32_t L,
                         uint32_t npoly) {
  ntt_body<S, BLOCKS, false, RHO_EPILOGUE, RescaleStore>(
      t, poly_stride, mc, tw_all, log_n, LimbMap::contiguous(0), s_other, 1,
      RescaleStore{ptrs.a, ptrs.out, rs, 1u << log_n, l, L, npoly});
}

// The rescale's inverse column pass over the last limb (radix 8, as the
// other rescale passes): launch poly y's single limb, modulus l.
template <int S>
__global__ void __launch_bounds__(256)
    ntt_pass_rescale_cols(uint64_t* __restrict__ data, size_t poly_stride,
                          const ModConst* __restrict__ mc, const uint64_t* __restrict__ tw_all,
                          uint32_t log_n, uint32_t s_other, uint32_t l) {
  ntt_body<S, COLS, true, RHO_EPILOGUE, PlainStore, PlainLoad, LimbMap>(
      data, poly_stride, mc, tw_all, log_n, LimbMap::contiguous(l), s_other, 1, PlainStore{});
}

// ModUp input: limb blockIdx.z of ciphertext blockIdx.y's c1, read from the
// caller's polys (the first inverse pass reads them in place of a copy).
// Each word is read once by the pass, which also stores it as the word of
// its digit's own limb ([ct][d][ne][N], d = limb / alpha): the digits keep
// c1's own limbs as they are.
constexpr int MODUP_MAX_CT = 32;
struct SrcLoad {
  static constexpr bool kLoad = true;
  static constexpr bool kPair = false;
  const uint64_t* const* src;  // MODUP_MAX_CT entries in kernel arguments
  uint32_t n;
  uint64_t* digits;
  uint32_t alpha, nd, ne;
  __device__ __forceinline__ uint64_t get(size_t g, uint64_t) const {
    const uint32_t ct = blockIdx.y, i = blockIdx.z;
    const uint64_t v = src[ct][(size_t)i * n + g];
    digits[(((size_t)ct * nd + i / alpha) * ne + i) * n + g] = v;
    return v;
  }
  struct Ops2 {};
  __device__ __forceinline__ void fetch2(size_t, Ops2&) const {}
  __device__ __forceinline__ void comb2(const Ops2&, uint64_t, uint64_t&, uint64_t&) const {}
};
struct SrcPtrs {
  const uint64_t* p[MODUP_MAX_CT];
};

// First inverse pass of a fused ModUp: c1 of each ciphertext -> coef
// (blocked layout).
template <int S>
__global__ void __launch_bounds__(256)
    ntt_pass_modup_in(uint64_t* __restrict__ coef, size_t poly_stride,
                      const ModConst* __restrict__ mc, const uint64_t* __restrict__ tw_all,
                      uint32_t log_n, uint32_t s_other, const SrcPtrs src, uint64_t* digits,
                      uint32_t alpha, uint32_t nd, uint32_t ne) {
  ntt_body<S, BLOCKS, true, RHO_EPILOGUE, PlainStore, SrcLoad, LimbMap, false, true>(
      coef, poly_stride, mc, tw_all, log_n, LimbMap::contiguous(0), s_other, 0, PlainStore{},
      SrcLoad{src.p, 1u << log_n, digits, alpha, nd, ne});
}

// Last forward pass of a fused ModUp over the digits' converted limbs
// (blocked layout in, standard out).
template <int S>
__global__ void __launch_bounds__(256)
    ntt_pass_modup_out(uint64_t* __restrict__ digits, size_t poly_stride,
                       const ModConst* __restrict__ mc, const uint64_t* __restrict__ tw_all,
                       uint32_t log_n, DigitMap map, uint32_t s_other) {
  ntt_body<S, BLOCKS, false, RHO_EPILOGUE, PlainStore, PlainLoad, DigitMap, true, false>(
      digits, poly_stride, mc, tw_all, log_n, map, s_other, 1, PlainStore{});
}

// ---- Fused middle of a batched ModDown, ring dimensions 2^13 .. 2^17 ----
//
// One workgroup per (poly, column u): the last S1 inverse stages of the K
// P limbs (the column stages; the first pass wrote the blocked P limbs), the
// scaling by N^-1 * [P/p_t]^-1 folded into one Shoup product, the fast
// conversion P -> Q_l (30-bit split MACs, one REDC per output, constants in
// Montgomery form with -P^-1 folded in), and the first S1 forward stages of
// every Q limb, written to the blocked y.  This replaces an inverse column
// pass, a conversion and a forward column pass, and the three round trips
// of the P limbs and y through HBM between them.
//
// Each column line of M = 2^S1 rows belongs to TPL = min(64, M / 4) lanes of
// one wavefront (radix M / TPL per lane), so its sub-passes exchange through
// LDS with wavefront-level ordering only; the four waves of a workgroup meet
// at a single barrier, once the converted sources are in LDS.  With one line
// per wave the modulus, its twiddles and the conversion constants are
// wavefront-uniform.  Stage order, twiddle indices and lazy ranges are those
// of the column passes of ntt_body.  Workgroups have NW waves: 4 for large
// batches, 8 when a launch has too few (poly, column) tiles to fill the
// chip, which halves each workgroup's serial line count and doubles the
// waves in flight.

template <int S1>
constexpr uint32_t mid_pitch() {
  return (1u << S1) + (1u << S1) / 16 + 1;
}
template <int S1>
constexpr int mid_lanes_per_line() {
  return (1 << S1) / 4 < 64 ? (1 << S1) / 4 : 64;
}
template <int S1, int NW>
constexpr int mid_lines() {  // lines in flight per workgroup of NW waves
  return NW * (64 / mid_lanes_per_line<S1>());
}

// What one (poly, column) tile converts.  Poly p of the launch uses plan
// p % nplan; its sources are limbs src_limb0 .. src_limb0 + nsrc - 1 of
// source group p / nplan (moduli src_mod0 + t), its targets the limbs
// pos(k) = k < skip_at ? k : k + skip_len of output group p, target k in
// the plan's constant order having modulus pos < qlimbs ? pos : L + pos -
// qlimbs (Q limbs, then P limbs).  ModDown: one plan, sources the K P limbs
// of ext poly p, targets Q limbs 0..nq-1 of y poly p.  ModUp: one plan per
// digit d, sources the digit's limbs of ciphertext p / nd, targets the
// rest of Q_l + P in the digit buffer's order (the digit's own limbs
// skipped), which is the order of Context::modup_plan's targets.
constexpr int MID_MAXPLAN = 8;
struct MidPlan {
  const uint64_t* src_scale;  // [nsrc][2]: [Q/q_t]^-1 N^-1 mod q_t (Shoup)
  const uint64_t* qhat_mont;  // [nsrc][ndst], Montgomery form w.r.t. the target
  const uint64_t* qhat_mont30;  // [nsrc][ndst], qhat_mont * 2^30 mod the target
  uint32_t nsrc, ndst, src_mod0, src_limb0, skip_at, skip_len, qlimbs;
};
struct MidArgs {
  const uint64_t* src;        // blocked, inverse block stages done, [0, 4q)
  uint64_t* out;              // blocked, forward column stages done, [0, 8q)
  size_t src_group_words, out_group_words;
  MidPlan plan[MID_MAXPLAN];
  uint32_t nplan, L;
};

// One group of at most eight conversion sources i0 .. i1 - 1 for target k:
// T_g = t + u 2^64 == sum_i v_i c_ik (mod t_k), from sources held as 30-bit
// halves (vl, vh) and the Montgomery-form tables c and c' = c 2^30 mod t_k
// split into 30-bit halves: v c == vl c + vh c', so b0 = sum vl cl + vh dl
// and b1 = sum vl ch + vh dh (each below 16 2^60 = 2^64) give T_g = b0 +
// b1 2^30, whose high word u is at most 2^30.
template <int R, uint32_t VSTEP, uint32_t PITCH, class CU64>
__device__ __forceinline__ void conv_group(const uint64_t* sbase, CU64* qhat_mont,
                                           CU64* qhat_mont30, uint32_t nq, uint32_t k,
                                           uint32_t i0, uint32_t i1, uint64_t (&t)[R],
                                           uint64_t (&u)[R]) {
  constexpr uint32_t M30 = (1u << 30) - 1;
  uint64_t b0[R], b1[R];
#pragma unroll
  for (int v = 0; v < R; ++v) b0[v] = b1[v] = 0;
  for (uint32_t i = i0; i < i1; ++i) {
    const uint64_t cv = qhat_mont[(size_t)i * nq + k];
    const uint64_t dv = qhat_mont30[(size_t)i * nq + k];
    const uint64_t* sl = sbase + (size_t)i * PITCH;
    uint64_t sv[R];
#pragma unroll
    for (int v = 0; v < R; ++v) sv[v] = sl[v * VSTEP];
    // the constants' and all R elements' reads in flight before the first
    // product: one wait a source
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t cl = (uint32_t)cv & M30, ch = (uint32_t)(cv >> 30);
    const uint32_t dl = (uint32_t)dv & M30, dh = (uint32_t)(dv >> 30);
#pragma unroll
    for (int v = 0; v < R; ++v) {
      const uint32_t vl = (uint32_t)sv[v], vh = (uint32_t)(sv[v] >> 32);
      b0[v] += (uint64_t)vl * cl + (uint64_t)vh * dl;
      b1[v] += (uint64_t)vl * ch + (uint64_t)vh * dh;
    }
  }
#pragma unroll
  for (int v = 0; v < R; ++v) {
    const uint64_t m = b1[v] << 30;
    t[v] = b0[v] + m;
    u[v] = (b1[v] >> 34) + (t[v] < m);
  }
}

// ALT: the forward column stages use the alternating lazy range of the
// paired ModDown epilogue (a stage whose global index g has logN - 1 - g
// even first brings X below 8q; values stay below 16q), and the output may
// reach 16q; otherwise every stage brings X below 4q and the output stays
// below 8q.
// Body for (poly, column) tile `tile` with (K + NL) PITCH words of lds.
template <int S1, int S2, int NW, bool ALT>
__device__ __forceinline__ void convert_mid_body(const MidArgs& a, const ModConst* __restrict__ mc,
                                                 const uint64_t* __restrict__ tw_inv,
                                                 const uint64_t* __restrict__ tw_fwd,
                                                 uint32_t tile, uint64_t* lds_dyn) {
  constexpr int M = 1 << S1, TPL = mid_lanes_per_line<S1>(), R = M / TPL;
  constexpr int RHO = R == 4 ? 2 : 3, LPW = 64 / TPL, NL = mid_lines<S1, NW>();
  constexpr int NSP = (S1 + RHO - 1) / RHO;
  constexpr uint32_t PITCH = mid_pitch<S1>(), N2 = 1u << S2;
  constexpr size_t N = (size_t)M << S2;
  constexpr uint32_t M30 = (1u << 30) - 1;
  static_assert(R * TPL == M && (1 << RHO) == R, "column split");
  const uint32_t p = tile / N2, col = tile % N2;
  const MidPlan& pl = a.plan[p % a.nplan];
  const uint32_t K = pl.nsrc, nq = pl.ndst;
  const uint64_t* const ext = a.src + (size_t)(p / a.nplan) * a.src_group_words +
                              (size_t)pl.src_limb0 * N;
  uint64_t* const y = a.out + (size_t)p * a.out_group_words;
  // The conversion tables are read-only for the whole launch: reading them
  // through the constant address space lets uniform loads use the scalar
  // cache, as for kernel-argument tables.
  typedef const uint64_t __attribute__((address_space(4))) cu64;
  cu64* const src_scale = (cu64*)pl.src_scale;
  cu64* const qhat_mont = (cu64*)pl.qhat_mont;
  cu64* const qhat_mont30 = (cu64*)pl.qhat_mont30;
  uint64_t* const src = lds_dyn;
  uint64_t* const work = lds_dyn + (size_t)K * PITCH;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63, sub = lane / TPL, tau = lane % TPL;
  const uint32_t first = wave * LPW + sub;

  // Inverse column stages of the P limbs; each limb is one line of src.
  for (uint32_t t = first; t < K; t += NL) {
    const uint32_t midx = pl.src_mod0 + t;
    const uint64_t q = mc[midx].q, q4 = 4 * q, qneg = mc[midx].neg_q, q4neg = mc[midx].neg_q4;
    const uint64_t* __restrict__ tw = tw_inv + (size_t)midx * N * 2;
    uint64_t* const line = src + (size_t)t * PITCH;
    uint64_t x[R];
    // First window (bits 0 .. RHO-1): rows R tau + v, one blocked run.
    const uint64_t* g = ext + (size_t)t * N + blocked_off<S2>(R * tau, col);
#pragma unroll
    for (int v = 0; v < R; ++v) x[v] = g[v];
#pragma unroll
    for (int sp = 0; sp < NSP; ++sp) {
      const int lo = RHO * sp;
      const int w = lo + RHO <= S1 ? lo : S1 - RHO;
      const int bhi = lo + RHO <= S1 ? lo + RHO - 1 : S1 - 1;
      const uint32_t thi = (tau >> w) << (w + RHO), tlo = tau & ((1u << w) - 1);
      if (sp > 0) {
#pragma unroll
        for (int v = 0; v < R; ++v) x[v] = line[lds_idx(0, thi | ((uint32_t)v << w) | tlo, 0)];
      }
#pragma unroll
      for (int beta = lo; beta <= bhi; ++beta) {
        const int d = 1 << (beta - w);
#pragma unroll
        for (int v = 0; v < R; ++v) {
          if (v & d) continue;
          const uint32_t u = thi | ((uint32_t)v << w) | tlo;
          const uint32_t ti = (1u << (S1 - 1 - beta)) | (u >> (beta + 1));
          const uint64_t wv = tw[2 * ti], ws = tw[2 * ti + 1];
          const uint64_t X = x[v], Y = x[v + d];
          x[v + d] = shoup_lazy4n(X + q4 - Y, wv, ws, qneg);
          x[v] = lazy_sub(X + Y, q4neg);
        }
      }
      if (sp == NSP - 1) {
        // v_t = x N^-1 [P/p_t]^-1 mod p_t, stored as 30-bit halves.
        const uint64_t f = src_scale[2 * t], fs = src_scale[2 * t + 1];
#pragma unroll
        for (int v = 0; v < R; ++v) {
          const uint64_t z = reduce_4q(shoup_lazy4(x[v], f, fs, q), q);
          x[v] = ((uint64_t)(uint32_t)(z >> 30) << 32) | ((uint32_t)z & M30);
        }
      }
      wave_lds_sync();
#pragma unroll
      for (int v = 0; v < R; ++v) line[lds_idx(0, thi | ((uint32_t)v << w) | tlo, 0)] = x[v];
      wave_lds_sync();
    }
  }
  __syncthreads();

  // Conversion into the Q limbs, one line of `work` per line in flight, then
  // their forward column stages.
  uint64_t* const line = work + (size_t)first * PITCH;
  for (uint32_t k = first; k < nq; k += NL) {
    const uint32_t kpos = k < pl.skip_at ? k : k + pl.skip_len;
    const uint32_t kmod = kpos < pl.qlimbs ? kpos : a.L + (kpos - pl.qlimbs);
    const uint64_t q = mc[kmod].q, q4 = 4 * q, qn = mc[kmod].qinv;
    const uint64_t qneg = mc[kmod].neg_q, q4neg = mc[kmod].neg_q4, q8neg = mc[kmod].neg_q8;
    const uint64_t* __restrict__ tw = tw_fwd + (size_t)kmod * N * 2;
    uint64_t x[R];
    {
      // First forward window (bits S1-RHO .. S1-1): rows thi | v << w | tlo.
      constexpr int w = S1 - RHO;
      // With w >= 4 the row fields do not interact with the u / 16 padding:
      // lds_idx(thi | v << w | tlo) = lds_idx(thi | tlo) + v * VSTEP, so one
      // address register serves a source line's R reads (immediate offsets).
      static_assert(w >= 4, "padding split");
      constexpr uint32_t VSTEP = (1u << w) + (1u << (w - 4));
      const uint32_t thi = (tau >> w) << (w + RHO), tlo = tau & ((1u << w) - 1);
      const uint64_t* const sbase = src + lds_idx(0, thi | tlo, 0);
      // Sources in groups of at most eight (conv_group); the groups' sum T
      // (K <= 16: T >> 64 < 2^32 < t) takes one Montgomery reduction.
      uint64_t tl[R], th[R];  // T = tl + th 2^64
      const uint32_t k1 = K < 8 ? K : 8;
      conv_group<R, VSTEP, PITCH>(sbase, qhat_mont, qhat_mont30, nq, k, 0, k1, tl, th);
      if (K > 8) {
        uint64_t t2[R], u2[R];
        conv_group<R, VSTEP, PITCH>(sbase, qhat_mont, qhat_mont30, nq, k, 8, K, t2, u2);
#pragma unroll
        for (int v = 0; v < R; ++v) {
          tl[v] += t2[v];
          th[v] += u2[v] + (tl[v] < t2[v]);
        }
      }
#pragma unroll
      for (int v = 0; v < R; ++v) x[v] = redc_lazy(th[v], tl[v], q, qn);  // (0, 2q)
    }
#pragma unroll
    for (int sp = 0; sp < NSP; ++sp) {
      const int hi = S1 - RHO * sp;
      const int w = hi >= RHO ? hi - RHO : 0;
      const int bhi = hi - 1;
      const uint32_t thi = (tau >> w) << (w + RHO), tlo = tau & ((1u << w) - 1);
      if (sp > 0) {
#pragma unroll
        for (int v = 0; v < R; ++v) x[v] = line[lds_idx(0, thi | ((uint32_t)v << w) | tlo, 0)];
      }
#pragma unroll
      for (int beta = bhi; beta >= w; --beta) {
        const int d = 1 << (beta - w);
#pragma unroll
        for (int v = 0; v < R; ++v) {
          if (v & d) continue;
          const uint32_t u = thi | ((uint32_t)v << w) | tlo;
          const uint32_t ti = (1u << (S1 - 1 - beta)) | (u >> (beta + 1));
          const uint64_t wv = tw[2 * ti], ws = tw[2 * ti + 1];
          const uint64_t X = !ALT ? lazy_sub(x[v], q4neg)
                             : (S2 + beta) % 2 == 0 ? lazy_sub(x[v], q8neg) : x[v];
          const uint64_t T = shoup_lazy4n(x[v + d], wv, ws, qneg);
          x[v] = X + T;
          x[v + d] = X + q4 - T;
        }
      }
      if (sp < NSP - 1) {
        wave_lds_sync();
#pragma unroll
        for (int v = 0; v < R; ++v) line[lds_idx(0, thi | ((uint32_t)v << w) | tlo, 0)] = x[v];
        wave_lds_sync();
      } else {
        // Last window (bits 0 .. RHO-1): rows R tau + v, one blocked run.
        uint64_t* g = y + (size_t)kpos * N + blocked_off<S2>(R * tau, col);
#pragma unroll
        for (int v = 0; v < R; ++v) g[v] = x[v];
      }
    }
  }
}

template <int S1, int S2, int NW, bool ALT>
__global__ void __launch_bounds__(64 * NW)
    k_convert_mid(const MidArgs a, const ModConst* __restrict__ mc,
                  const uint64_t* __restrict__ tw_inv, const uint64_t* __restrict__ tw_fwd) {
  extern __shared__ uint64_t lds_dyn[];
  // Tiles in XCD order: workgroup i runs on XCD i % 8, and each XCD takes a
  // contiguous range of (poly, column) tiles, so neighbouring columns, which
  // share cache lines of the blocked layout, meet in one L2.
  const uint32_t per = gridDim.x / 8;
  const uint32_t tile = (blockIdx.x % 8) * per + blockIdx.x / 8;
  convert_mid_body<S1, S2, NW, ALT>(a, mc, tw_inv, tw_fwd, tile, lds_dyn);
}

template <int S, int KIND, bool INV, class Map>
void launch_pass(Context& c, uint64_t* data, uint32_t npoly, size_t poly_stride, uint32_t nlimb,
                 Map map, uint32_t s_other, bool last) {
  using G = Geo<S, RHO_PLAIN>;
  const uint32_t lines = KIND == SINGLE ? 1 : 256 / G::TPL;
  const uint32_t threads = KIND == SINGLE ? G::TPL : 256;
  // COLS has N2 = 2^s_other lines per limb, BLOCKS has N1 = 2^s_other.
  const uint32_t tiles = KIND == SINGLE ? 1 : (1u << s_other) / lines;
  dim3 grid(tiles, npoly, nlimb);
  const char* const PASS_NAME =
      KIND == SINGLE ? (INV ? "ntt_inv_single" : "ntt_fwd_single")
      : KIND == COLS ? (INV ? "ntt_inv_cols" : "ntt_fwd_cols")
                     : (INV ? "ntt_inv_blocks" : "ntt_fwd_blocks");
  FHE_LAUNCH(c, PASS_NAME, (ntt_pass<S, KIND, INV, Map>), grid, dim3(threads), 0, data, poly_stride, c.d_const, INV ? c.d_tw_inv : c.d_tw_fwd, c.log_n, map, s_other, (int)last);
}

template <bool INV, class Map = LimbMap>
void launch_single(Context& c, uint64_t* data, uint32_t npoly, size_t ps, uint32_t nlimb, Map map) {
  switch (c.log_n) {
#define CASE(S) \
  case S: launch_pass<S, SINGLE, INV>(c, data, npoly, ps, nlimb, map, 0, true); break;
    CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(9) CASE(10) CASE(11) CASE(12)
#undef CASE
    default: throw ArgError("unsupported ring dimension");
  }
}

template <bool INV, class Map = LimbMap>
void launch_cols(Context& c, uint32_t s1, uint32_t s2, uint64_t* data, uint32_t npoly, size_t ps,
                 uint32_t nlimb, Map map, bool last) {
  switch (s1) {
#define CASE(S) \
  case S: launch_pass<S, COLS, INV>(c, data, npoly, ps, nlimb, map, s2, last); break;
    CASE(7) CASE(8) CASE(9)
#undef CASE
    default: throw ArgError("unsupported column pass");
  }
}

template <bool INV, class Map = LimbMap>
void launch_blocks(Context& c, uint32_t s1, uint32_t s2, uint64_t* data, uint32_t npoly, size_t ps,
                   uint32_t nlimb, Map map, bool last) {
  switch (s2) {
#define CASE(S) \
  case S: launch_pass<S, BLOCKS, INV>(c, data, npoly, ps, nlimb, map, s1, last); break;
    CASE(6) CASE(7) CASE(8)
#undef CASE
    default: throw ArgError("unsupported block pass");
  }
}

template <int S, int KIND, bool BLK = false>
void launch_moddown(Context& c, uint64_t* y, uint32_t npoly, uint32_t nq, uint32_t s_other,
                    const ModDownEpi& epi) {
  using G = Geo<S, epilogue_rho<S, KIND>()>;
  const uint32_t lines = KIND == SINGLE ? 1 : 256 / G::TPL;
  const uint32_t threads = KIND == SINGLE ? G::TPL : 256;
  const uint32_t tiles = KIND == SINGLE ? 1 : (1u << s_other) / lines;
  const char* name = KIND == SINGLE ? "ntt_fwd_single_moddown" : "ntt_fwd_blocks_moddown";
  if constexpr (BLK && KIND == BLOCKS) {
    // Both polys of each key switch in one workgroup (blocked y, digits
    // 1..7): rows per workgroup = one blocked group.
    constexpr uint32_t pair_lines = 512u >> (S - 2);
    if (npoly % 2 == 0 && epi.nd >= 1 && epi.nd <= 7) {
      const dim3 grid((1u << s_other) / pair_lines, npoly / 2, nq);
      switch (epi.nd) {
#define CASE(D)                                                                                 case D:                                                                                         FHE_LAUNCH(c, name, (ntt_pass_moddown_pair<S, D>), grid, dim3(512), 0, y, c.d_const,                     c.d_tw_fwd, c.log_n, s_other, epi);                                                return;
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7)
#undef CASE
      }
    }
  }
  switch (epi.nd) {
#define CASE(D)                                                                               \
  case D:                                                                                     \
    FHE_LAUNCH(c, name, (ntt_pass_moddown<S, KIND, D, BLK>), dim3(tiles, npoly, nq),          \
               dim3(threads),                                                                  \
               0, y, (size_t)nq * c.n, c.d_const, c.d_tw_fwd, c.log_n, s_other, epi);         \
    return;
    CASE(1) CASE(2) CASE(3)
#undef CASE
    default:
      FHE_LAUNCH(c, name, (ntt_pass_moddown<S, KIND, 0, BLK>), dim3(tiles, npoly, nq), dim3(threads), 0,
                 y, (size_t)nq * c.n, c.d_const, c.d_tw_fwd, c.log_n, s_other, epi);
  }
}

template <int S, int KIND, bool BLK = false>
void launch_ksk(Context& c, uint64_t* ext, uint32_t npoly, uint32_t s_other, bool last,
                const ModDownEpi& epi) {
  using G = Geo<S, epilogue_rho<S, KIND>()>;
  const uint32_t lines = KIND == SINGLE ? 1 : 256 / G::TPL;
  const uint32_t threads = KIND == SINGLE ? G::TPL : 256;
  const uint32_t tiles = KIND == SINGLE ? 1 : (1u << s_other) / lines;
  const char* name = KIND == SINGLE ? "ntt_inv_single_ksk" : "ntt_inv_blocks_ksk";
  const dim3 grid(tiles, npoly, c.K);
  const size_t ps = (size_t)c.K * c.n;
  if constexpr (BLK && KIND == BLOCKS) {
    // Both polys of each key switch in one workgroup (blocked output, digits
    // 1..7, no final scaling): rows per workgroup = one blocked group.
    constexpr uint32_t pair_lines = 512u >> (S - 2);
    if (!last && npoly % 2 == 0 && epi.nd >= 1 && epi.nd <= 7) {
      const dim3 pgrid((1u << s_other) / pair_lines, npoly / 2, c.K);
      switch (epi.nd) {
#define CASE(D)                                                                              \
  case D:                                                                                    \
    FHE_LAUNCH(c, name, (ntt_pass_ksk_pair<S, D>), pgrid, dim3(512), 0, ext, ps, c.d_const,  \
               c.d_tw_inv, c.log_n, s_other, epi);                                           \
    return;
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7)
#undef CASE
      }
    }
  }
  switch (epi.nd) {
#define CASE(D)                                                                         \
  case D:                                                                               \
    FHE_LAUNCH(c, name, (ntt_pass_ksk<S, KIND, D, BLK>), grid, dim3(threads), 0, ext, ps, \
               c.d_const, c.d_tw_inv, c.log_n, s_other, (int)last, epi);                \
    return;
    CASE(1) CASE(2) CASE(3)
#undef CASE
    default:
      FHE_LAUNCH(c, name, (ntt_pass_ksk<S, KIND, 0, BLK>), grid, dim3(threads), 0, ext, ps, c.d_const,
                 c.d_tw_inv, c.log_n, s_other, (int)last, epi);
  }
}

template <int S1, int NW>
size_t mid_lds_bytes(uint32_t K) {
  return (size_t)(K + mid_lines<S1, NW>()) * mid_pitch<S1>() * 8;
}

// Launches with fewer (poly, column) tiles than this use 8-wave workgroups.
constexpr uint32_t MID_SMALL_TILES = 4096;
// Launches of at most this many tiles (one ciphertext's ModUp or ModDown)
// use 16-wave workgroups.
constexpr uint32_t MID_TINY_TILES = 1024;

template <int S1, int S2, bool ALT = false>
void launch_mid(Context& c, const char* name, const MidArgs& a, uint32_t npoly,
                uint32_t max_src) {
  const uint32_t tiles = npoly << S2;
  if (tiles <= MID_TINY_TILES && mid_lds_bytes<S1, 16>(max_src) <= c.lds_per_block) {
    FHE_LAUNCH(c, name, (k_convert_mid<S1, S2, 16, ALT>), dim3(tiles), dim3(1024),
               (mid_lds_bytes<S1, 16>(max_src)), a, c.d_const, c.d_tw_inv, c.d_tw_fwd);
    return;
  }
  if (tiles < MID_SMALL_TILES && mid_lds_bytes<S1, 8>(max_src) <= c.lds_per_block) {
    FHE_LAUNCH(c, name, (k_convert_mid<S1, S2, 8, ALT>), dim3(tiles), dim3(512),
               (mid_lds_bytes<S1, 8>(max_src)), a, c.d_const, c.d_tw_inv, c.d_tw_fwd);
    return;
  }
  FHE_LAUNCH(c, name, (k_convert_mid<S1, S2, 4, ALT>), dim3(tiles), dim3(256),
             (mid_lds_bytes<S1, 4>(max_src)), a, c.d_const, c.d_tw_inv, c.d_tw_fwd);
}

// The target order of `pl` must be the one MidPlan describes (checked).
MidPlan mid_plan(const Context& c, const ConvPlan& pl, uint32_t src_mod0, uint32_t src_limb0,
                 uint32_t skip_at, uint32_t skip_len, uint32_t qlimbs) {
  for (uint32_t k = 0; k < pl.ndst; ++k) {
    const uint32_t pos = k < skip_at ? k : k + skip_len;
    if (pl.dst_idx[k] != (pos < qlimbs ? pos : c.L + (pos - qlimbs)))
      throw ArgError("conversion plan target order");
  }
  return MidPlan{pl.d_src_scale, pl.d_qhat_mont, pl.d_qhat_mont30, pl.nsrc, pl.ndst,
                 src_mod0, src_limb0, skip_at, skip_len, qlimbs};
}

bool mid_lds_fits(const Context& c, uint32_t nsrc) {
  switch (c.log_n) {
    case 13: case 14: return mid_lds_bytes<7, 4>(nsrc) <= c.lds_per_block;
    case 15: case 16: return mid_lds_bytes<8, 4>(nsrc) <= c.lds_per_block;
    case 17: return mid_lds_bytes<9, 4>(nsrc) <= c.lds_per_block;
    default: return false;
  }
}

// Every modulus of the launch in [2^33, 2^60): the fused kernels' lazy
// ranges (16q < 2^64) and reduce_est's quotient estimate (q >= 2^33).
bool below_2_60_all(const Context& c, uint32_t nq) {
  auto ok = [](uint64_t m) { return m < (1ull << 60) && m >= (1ull << 33); };
  for (uint32_t i = 0; i < nq; ++i)
    if (!ok(c.mods[i])) return false;
  for (uint32_t t = 0; t < c.K; ++t)
    if (!ok(c.mods[c.L + t])) return false;
  return true;
}

}  // namespace

bool moddown_fused_ok(const Context& c, uint32_t nq) {
  if (c.log_n < 13 || c.log_n > 17 || c.K == 0 || c.K > 16) return false;
  if (nq == 0 || nq > c.L) return false;
  return below_2_60_all(c, nq) && mid_lds_fits(c, c.K);
}

void moddown_fused(Context& c, uint64_t* ext_p, uint64_t* y, uint32_t npoly, uint32_t nq,
                   const ConvPlan& pl, const ModDownEpi& epi) {
  if (npoly == 0) return;
  if (npoly > 2 * MAX_KS_BATCH) throw ArgError("ModDown batch too large");
  if (!moddown_fused_ok(c, nq)) throw ArgError("fused ModDown does not apply");
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  MidArgs a{};
  a.src = ext_p;
  a.out = y;
  a.src_group_words = (size_t)c.K * c.n;
  a.out_group_words = (size_t)nq * c.n;
  a.plan[0] = mid_plan(c, pl, c.L, 0, nq, 0, nq);
  a.nplan = 1;
  a.L = c.L;
  // The paired epilogue (both polys of each key switch, 1..7 digits) takes
  // the middle kernel's alternating lazy range; the other epilogues the
  // plain one.
  const bool pair = npoly % 2 == 0 && epi.nd >= 1 && epi.nd <= 7;
  switch (c.log_n) {
#define CASE(LN, A, B)                                                   \
  case LN:                                                               \
    launch_ksk<B, BLOCKS, true>(c, ext_p, npoly, s1, false, epi);        \
    if (pair)                                                            \
      launch_mid<A, B, true>(c, "k_moddown_mid", a, npoly, c.K);         \
    else                                                                 \
      launch_mid<A, B>(c, "k_moddown_mid", a, npoly, c.K);               \
    launch_moddown<B, BLOCKS, true>(c, y, npoly, nq, s1, epi);           \
    return;
    CASE(13, 7, 6) CASE(14, 7, 7) CASE(15, 8, 7) CASE(16, 8, 8) CASE(17, 9, 8)
#undef CASE
    default: throw ArgError("unsupported ring dimension");
  }
  (void)s2;
}

static void rescale_launch(Context& c, uint64_t* const* outs, const uint64_t* const* as,
                           uint32_t count, uint32_t npoly, uint32_t nq);

void rescale_fused(Context& c, uint64_t* out, const uint64_t* a, uint32_t npoly, uint32_t nq) {
  rescale_fused_many(c, &out, &a, 1, npoly, nq);
}

void rescale_fused_many(Context& c, uint64_t* const* outs, const uint64_t* const* as,
                        uint32_t count, uint32_t npoly, uint32_t nq) {
  if (c.log_n < 13 || c.log_n > 17) throw ArgError("fused rescale needs N = 2^13 .. 2^17");
  if (nq < 2 || npoly == 0 || npoly > 65535) throw ArgError("rescale: bad shape");
  for (uint32_t r0 = 0; r0 < count;) {
    // inputs of one launch set: at most RESCALE_MAX, and npoly per input
    const uint32_t b = std::min<uint32_t>({count - r0, (uint32_t)RESCALE_MAX, 65535u / npoly});
    rescale_launch(c, outs + r0, as + r0, b, npoly, nq);
    r0 += b;
  }
}

// One launch set over `count` <= RESCALE_MAX inputs of npoly polys each.
static void rescale_launch(Context& c, uint64_t* const* outs, const uint64_t* const* as,
                           uint32_t count, uint32_t npoly, uint32_t nq) {
  const uint32_t l = nq - 1, n = c.n, np = count * npoly;
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  RescalePtrs ptrs{};
  for (uint32_t r = 0; r < count; ++r) {
    ptrs.a[r] = as[r];
    ptrs.out[r] = outs[r];
  }
  Scratch last(c, (size_t)np * n), t(c, (size_t)np * l * n);
  const LiftLoad lift{last.p, c.d_const, c.d_rescale, n, l, c.L, c.mods[l] >> 1};
  switch (c.log_n) {
#define CASE(LN, A, B)                                                                        \
  case LN: {                                                                                  \
    using GB = Geo<B, RHO_EPILOGUE>;                                                          \
    using GA = Geo<A, RHO_EPILOGUE>;                                                          \
    const uint32_t tb = (1u << s1) / (256 / GB::TPL), ta = (1u << s2) / (256 / GA::TPL);      \
    FHE_LAUNCH(c, "ntt_inv_blocks_rescale", (ntt_pass_rescale_in<B>), dim3(tb, np, 1),        \
               dim3(256), 0, last.p, c.d_const, c.d_tw_inv, c.log_n, s1, ptrs, npoly,         \
               (size_t)nq * n, l);                                                            \
    FHE_LAUNCH(c, "ntt_inv_cols_rescale", (ntt_pass_rescale_cols<A>), dim3(ta, np, 1),      \
               dim3(256), 0, last.p, (size_t)n, c.d_const, c.d_tw_inv, c.log_n, s2, l);   \
    FHE_LAUNCH(c, "ntt_fwd_cols_rescale", (ntt_pass_rescale_lift<A>), dim3(ta, np, l),        \
               dim3(256), 0, t.p, (size_t)l * n, c.d_const, c.d_tw_fwd, c.log_n, s2, lift);   \
    FHE_LAUNCH(c, "ntt_fwd_blocks_rescale", (ntt_pass_rescale_out<B>), dim3(tb, np, l),       \
               dim3(256), 0, t.p, (size_t)l * n, c.d_const, c.d_tw_fwd, c.log_n, s1, ptrs,    \
               c.d_rescale, l, c.L, npoly);                                                   \
    return;                                                                                   \
  }
    CASE(13, 7, 6) CASE(14, 7, 7) CASE(15, 8, 7) CASE(16, 8, 8) CASE(17, 9, 8)
#undef CASE
    default: throw ArgError("unsupported ring dimension");
  }
}

bool modup_fused_ok(const Context& c, uint32_t nq, uint32_t count) {
  if (c.log_n < 13 || c.log_n > 17 || c.K == 0 || c.alpha == 0 || c.alpha > 16) return false;
  if (nq == 0 || nq > c.L || count == 0 || count > (uint32_t)MODUP_MAX_CT) return false;
  const uint32_t nd = num_digits(c, nq);
  if (nd > (uint32_t)MID_MAXPLAN || (uint64_t)count * nd > 65535) return false;
  return below_2_60_all(c, nq) && mid_lds_fits(c, c.alpha);
}

void modup_fused(Context& c, const uint64_t* const* as, uint32_t count, uint32_t nq,
                 uint64_t* digits) {
  if (!modup_fused_ok(c, nq, count)) throw ArgError("fused ModUp does not apply");
  const size_t n = c.n;
  const uint32_t ne = nq + c.K, nd = num_digits(c, nq);
  Scratch coef(c, (size_t)count * nq * n);
  SrcPtrs sp{};
  for (uint32_t i = 0; i < count; ++i) sp.p[i] = as[i];
  MidArgs a{};
  a.src = coef.p;
  a.out = digits;
  a.src_group_words = (size_t)nq * n;
  a.out_group_words = (size_t)ne * n;
  a.nplan = nd;
  a.L = c.L;
  uint32_t max_src = 0;
  for (uint32_t d = 0; d < nd; ++d) {
    const uint32_t s0 = d * c.alpha, e0 = s0 + c.alpha < nq ? s0 + c.alpha : nq;
    a.plan[d] = mid_plan(c, c.modup_plan(s0, e0, nq), s0, s0, s0, e0 - s0, nq);
    max_src = max_src > e0 - s0 ? max_src : e0 - s0;
  }
  // The last digit is the narrowest and so has the most converted limbs.
  const uint32_t w_last = nq - (nd - 1) * c.alpha;
  const DigitMap map{c.alpha, nq, c.L, ne, nd};
  const uint32_t s1 = (c.log_n + 1) / 2;
  switch (c.log_n) {
#define CASE(LN, A, B)                                                                        \
  case LN: {                                                                                  \
    using G = Geo<B, RHO_EPILOGUE>;                                                           \
    const uint32_t tiles = (1u << s1) / (256 / G::TPL);                                       \
    FHE_LAUNCH(c, "ntt_inv_blocks_modup", (ntt_pass_modup_in<B>), dim3(tiles, count, nq),     \
               dim3(256), 0, coef.p, (size_t)nq * n, c.d_const, c.d_tw_inv, c.log_n, s1, sp,  \
               digits, c.alpha, nd, ne);                                                      \
    launch_mid<A, B>(c, "k_modup_mid", a, count * nd, max_src);                               \
    FHE_LAUNCH(c, "ntt_fwd_blocks_modup", (ntt_pass_modup_out<B>),                            \
               dim3(tiles, count * nd, ne - w_last), dim3(256), 0, digits, (size_t)ne * n,    \
               c.d_const, c.d_tw_fwd, c.log_n, map, s1);                                      \
    break;                                                                                    \
  }
    CASE(13, 7, 6) CASE(14, 7, 7) CASE(15, 8, 7) CASE(16, 8, 8) CASE(17, 9, 8)
#undef CASE
    default: throw ArgError("unsupported ring dimension");
  }
}

void ntt_forward_digits(Context& c, uint64_t* digits, uint32_t count, uint32_t nd,
                        uint32_t nq) {
  if (count == 0 || nd == 0 || nq == 0) return;
  if (nq > c.L) throw ArgError("ModUp level out of range");
  if ((uint64_t)count * nd > 65535) throw ArgError("too many digits in one launch");
  const uint32_t ne = nq + c.K;
  // The last digit is the narrowest and so has the most converted limbs.
  const uint32_t w_last = nq - (nd - 1) * c.alpha;
  const uint32_t slots = ne - w_last;
  const DigitMap map{c.alpha, nq, c.L, ne, nd};
  const size_t ps = (size_t)ne * c.n;
  const uint32_t npoly = count * nd;
  if (c.log_n <= 12) {
    launch_single<false>(c, digits, npoly, ps, slots, map);
    return;
  }
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  launch_cols<false>(c, s1, s2, digits, npoly, ps, slots, map, false);
  launch_blocks<false>(c, s1, s2, digits, npoly, ps, slots, map, true);
}

void ntt_inverse_ksk(Context& c, uint64_t* ext_p, uint32_t npoly, const ModDownEpi& epi) {
  if (npoly == 0 || c.K == 0) return;
  if (npoly > 2 * MAX_KS_BATCH) throw ArgError("key-switch batch too large");
  if (c.log_n <= 12) {
    switch (c.log_n) {
#define CASE(S) \
  case S: launch_ksk<S, SINGLE>(c, ext_p, npoly, 0, true, epi); return;
      CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(9) CASE(10) CASE(11) CASE(12)
#undef CASE
      default: throw ArgError("unsupported ring dimension");
    }
  }
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  switch (s2) {
#define CASE(S) \
  case S: launch_ksk<S, BLOCKS>(c, ext_p, npoly, s1, false, epi); break;
    CASE(6) CASE(7) CASE(8)
#undef CASE
    default: throw ArgError("unsupported block pass");
  }
  launch_cols<true>(c, s1, s2, ext_p, npoly, (size_t)c.K * c.n, c.K, LimbMap::contiguous(c.L),
                    true);
}

void ntt_forward_moddown(Context& c, uint64_t* y, uint32_t npoly, uint32_t nq,
                         const ModDownEpi& epi) {
  if (npoly == 0 || nq == 0) return;
  if (npoly > 2 * MAX_KS_BATCH) throw ArgError("ModDown batch too large");
  if (c.log_n <= 12) {
    switch (c.log_n) {
#define CASE(S) \
  case S: launch_moddown<S, SINGLE>(c, y, npoly, nq, 0, epi); return;
      CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(9) CASE(10) CASE(11) CASE(12)
#undef CASE
      default: throw ArgError("unsupported ring dimension");
    }
  }
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  launch_cols<false>(c, s1, s2, y, npoly, (size_t)nq * c.n, nq, LimbMap::contiguous(0), false);
  switch (s2) {
#define CASE(S) \
  case S: launch_moddown<S, BLOCKS>(c, y, npoly, nq, s1, epi); return;
    CASE(6) CASE(7) CASE(8)
#undef CASE
    default: throw ArgError("unsupported block pass");
  }
}

void ntt_forward(Context& c, uint64_t* data, uint32_t npoly, size_t poly_stride, uint32_t nlimb,
                 LimbMap map) {
  if (npoly == 0 || nlimb == 0) return;
  if (npoly > 65535 || nlimb > 65535) throw ArgError("too many polys or limbs in one launch");
  if (c.log_n <= 12) {
    launch_single<false>(c, data, npoly, poly_stride, nlimb, map);
    return;
  }
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  launch_cols<false>(c, s1, s2, data, npoly, poly_stride, nlimb, map, false);
  launch_blocks<false>(c, s1, s2, data, npoly, poly_stride, nlimb, map, true);
}

void ntt_forward_table(Context& c, uint64_t* const* table, uint32_t npoly, uint32_t nlimb) {
  if (npoly == 0 || nlimb == 0) return;
  if (npoly > 65535 || nlimb > c.L + c.K) throw ArgError("too many polys or limbs in one launch");
  const TableMap map{table};
  if (c.log_n <= 12) {
    launch_single<false>(c, nullptr, npoly, 0, nlimb, map);
    return;
  }
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  launch_cols<false>(c, s1, s2, nullptr, npoly, 0, nlimb, map, false);
  launch_blocks<false>(c, s1, s2, nullptr, npoly, 0, nlimb, map, true);
}

void ntt_inverse(Context& c, uint64_t* data, uint32_t npoly, size_t poly_stride, uint32_t nlimb,
                 LimbMap map) {
  if (npoly == 0 || nlimb == 0) return;
  if (npoly > 65535 || nlimb > 65535) throw ArgError("too many polys or limbs in one launch");
  if (c.log_n <= 12) {
    launch_single<true>(c, data, npoly, poly_stride, nlimb, map);
    return;
  }
  const uint32_t s1 = (c.log_n + 1) / 2, s2 = c.log_n / 2;
  launch_blocks<true>(c, s1, s2, data, npoly, poly_stride, nlimb, map, false);
  launch_cols<true>(c, s1, s2, data, npoly, poly_stride, nlimb, map, true);
}

}  // namespace fhe
