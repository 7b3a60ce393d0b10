// CKKS encode / decode on the GPU.
//
// Encode = OpenFHE CKKSPackedEncoding::Encode as restated by the
// reference's GPU encoder (native/fideslib_stage0/src/gpu_special_fft.cu):
//   special inverse FFT over `slots` values (butterfly order and twiddle
//   table of gpu_special_fft.cu:12-22, :99-108 and
//   patches/openfhe-v1.4.2-inverse-fft-plan.patch:18-60), bit reversal,
//   division by slots, multiplication by the scale, llround (ties away from
//   zero), placement of the 2*slots real/imaginary coefficients at stride
//   N / (2 slots), signed RNS lift into each limb
//   (fideslib_plaintext_rns.cu:11-23), forward NTT.
// Decode = inverse NTT, centred CRT (balanced mixed-radix / Garner, so no
// big integers), division by the scale, forward special FFT.
//
// All floating-point operations are plain IEEE double add/sub/mul/div; the
// library is compiled with -ffp-contract=off so none fuse into FMAs, which
// keeps the encoder's rounding identical to the CPU definition.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "ops.hpp"

namespace fhe {
namespace {

constexpr int TPB = 256;

inline uint32_t ilog2(uint32_t x) {
  uint32_t l = 0;
  while ((1u << l) < x) ++l;
  return l;
}

// Twiddle (cos, sin) pairs come from one glibc sincos() call per angle: that
// is what gcc-built OpenFHE evaluates for its (cos(angle), sin(angle))
// table (gcc fuses the pair), and sincos() differs from separate cos()/sin()
// in the last bit for a few angles.
inline void host_sincos(double a, double* s, double* c) { ::sincos(a, s, c); }

std::pair<double*, double*> fft_tables(Context& c, uint32_t slots) {
  std::lock_guard<std::mutex> g(c.fft_mu);
  auto it = c.fft_tables.find(slots);
  if (it != c.fft_tables.end()) return it->second;
  const uint32_t m = 4 * slots;
  std::vector<uint32_t> rot(slots);
  uint32_t p = 1;
  for (uint32_t j = 0; j < slots; ++j) {
    rot[j] = p;
    p = (uint32_t)(((uint64_t)p * 5) % m);
  }
  const size_t cnt = slots > 1 ? slots - 1 : 1;
  std::vector<double> inv(2 * cnt, 0.0), fwd(2 * cnt, 0.0);
  for (uint32_t len = 2; len <= slots; len <<= 1) {
    const uint32_t h = len / 2, lenq = 4 * len, gap = m / lenq;
    for (uint32_t j = 0; j < h; ++j) {
      const double ai = 2.0 * M_PI * ((lenq - rot[j] % lenq) * gap) / m;
      const double af = 2.0 * M_PI * ((rot[j] % lenq) * gap) / m;
      host_sincos(ai, &inv[2 * (h - 1 + j) + 1], &inv[2 * (h - 1 + j)]);
      host_sincos(af, &fwd[2 * (h - 1 + j) + 1], &fwd[2 * (h - 1 + j)]);
    }
  }
  double *di = nullptr, *df = nullptr;
  note_alloc();
  note_alloc();
  hip_check(hipMalloc(&di, inv.size() * 8), "hipMalloc fft");
  hip_check(hipMalloc(&df, fwd.size() * 8), "hipMalloc fft");
  hip_check(hipMemcpy(di, inv.data(), inv.size() * 8, hipMemcpyHostToDevice), "fft table");
  hip_check(hipMemcpy(df, fwd.data(), fwd.size() * 8, hipMemcpyHostToDevice), "fft table");
  c.fft_tables[slots] = {di, df};
  return {di, df};
}

// One stage of the special inverse FFT: (a, b) -> (a + b, (a - b) * w).
// Vector blockIdx.y of a batch of `slots`-value vectors.
__global__ void k_fft_inv_stage(double2* v, const double* tw, uint32_t slots, uint32_t len) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= slots / 2) return;
  v += (size_t)blockIdx.y * slots;
  const uint32_t h = len / 2, j = t % h, i = (t / h) * len + j;
  const double2 a = v[i], b = v[i + h];
  const double wr = tw[2 * (h - 1 + j)], wi = tw[2 * (h - 1 + j) + 1];
  const double vr = a.x - b.x, vi = a.y - b.y;
  v[i] = make_double2(a.x + b.x, a.y + b.y);
  v[i + h] = make_double2(vr * wr - vi * wi, vi * wr + vr * wi);
}

// One stage of the forward special FFT: (u, b) -> (u + b w, u - b w).
__global__ void k_fft_fwd_stage(double2* v, const double* tw, uint32_t slots, uint32_t len) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= slots / 2) return;
  v += (size_t)blockIdx.y * slots;
  const uint32_t h = len / 2, j = t % h, i = (t / h) * len + j;
  const double2 u = v[i], b = v[i + h];
  const double wr = tw[2 * (h - 1 + j)], wi = tw[2 * (h - 1 + j) + 1];
  const double vr = b.x * wr - b.y * wi, vi = b.y * wr + b.x * wi;
  v[i] = make_double2(u.x + vr, u.y + vi);
  v[i + h] = make_double2(u.x - vr, u.y - vi);
}

// The stages with len <= FFT_BLOCK pair elements inside aligned blocks of
// FFT_BLOCK values, so one workgroup runs all of them on its block in LDS:
// the same butterflies and twiddles as the per-stage kernels above, in the
// same order per element, hence the same roundings.
constexpr uint32_t FFT_BLOCK = 2048;

// Inverse stages len = top, top / 2, ..., 2 on blocks of `top` values.
__global__ void __launch_bounds__(256)
    k_fft_inv_block(double2* v, const double* tw, uint32_t top) {
  __shared__ double2 x[FFT_BLOCK];
  double2* g = v + (size_t)blockIdx.x * top;
  for (uint32_t k = threadIdx.x; k < top; k += blockDim.x) x[k] = g[k];
  __syncthreads();
  for (uint32_t len = top; len >= 2; len >>= 1) {
    const uint32_t h = len / 2;
    for (uint32_t t = threadIdx.x; t < top / 2; t += blockDim.x) {
      const uint32_t j = t % h, i = (t / h) * len + j;
      const double2 a = x[i], b = x[i + h];
      const double wr = tw[2 * (h - 1 + j)], wi = tw[2 * (h - 1 + j) + 1];
      const double vr = a.x - b.x, vi = a.y - b.y;
      x[i] = make_double2(a.x + b.x, a.y + b.y);
      x[i + h] = make_double2(vr * wr - vi * wi, vi * wr + vr * wi);
    }
    __syncthreads();
  }
  for (uint32_t k = threadIdx.x; k < top; k += blockDim.x) g[k] = x[k];
}

// Forward stages len = 2, 4, ..., top on blocks of `top` values.
__global__ void __launch_bounds__(256)
    k_fft_fwd_block(double2* v, const double* tw, uint32_t top) {
  __shared__ double2 x[FFT_BLOCK];
  double2* g = v + (size_t)blockIdx.x * top;
  for (uint32_t k = threadIdx.x; k < top; k += blockDim.x) x[k] = g[k];
  __syncthreads();
  for (uint32_t len = 2; len <= top; len <<= 1) {
    const uint32_t h = len / 2;
    for (uint32_t t = threadIdx.x; t < top / 2; t += blockDim.x) {
      const uint32_t j = t % h, i = (t / h) * len + j;
      const double2 u = x[i], b = x[i + h];
      const double wr = tw[2 * (h - 1 + j)], wi = tw[2 * (h - 1 + j) + 1];
      const double vr = b.x * wr - b.y * wi, vi = b.y * wr + b.x * wi;
      x[i] = make_double2(u.x + vr, u.y + vi);
      x[i + h] = make_double2(u.x - vr, u.y - vi);
    }
    __syncthreads();
  }
  for (uint32_t k = threadIdx.x; k < top; k += blockDim.x) g[k] = x[k];
}

__device__ __forceinline__ uint32_t brev_bits(uint32_t x, uint32_t bits) {
  return bits ? __brev(x) >> (32 - bits) : 0;
}

__device__ __forceinline__ uint64_t lift_signed(int64_t x, uint64_t q) {
  if (x >= 0) return (uint64_t)x % q;
  const uint64_t r = ((uint64_t)(-x)) % q;
  return r ? q - r : 0;
}

// x mod q for |x| < 2^63 by a Barrett step with mu64 = floor(2^64 / q): the
// quotient estimate mulhi(|x|, mu64) is at most 1 below the true quotient,
// so one conditional subtraction completes the reduction.
__device__ __forceinline__ uint64_t lift_signed_mc(int64_t x, const ModConst& m) {
  const uint64_t a = x >= 0 ? (uint64_t)x : (uint64_t)0 - (uint64_t)x;
  uint64_t r = a - mulhi64(a, m.mu64) * m.q;
  r = r >= m.q ? r - m.q : r;
  return (x >= 0 || r == 0) ? r : m.q - r;
}

// Round slot i of the transformed vector (read through the bit reversal)
// and scatter its real / imaginary coefficient into limbs blockIdx.z,
// blockIdx.z + gridDim.z, ...  With a table, vector blockIdx.y of the
// batch goes to table[blockIdx.y].
__global__ void k_round_lift(const double2* v, uint64_t* out, uint64_t* const* table,
                             const ModConst* mc, uint32_t slots, uint32_t bits, uint32_t gap,
                             uint32_t n, uint32_t nlimb, double scale, int* status) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= slots) return;
  if (table) {
    v += (size_t)blockIdx.y * slots;
    out = table[blockIdx.y];
  }
  const double2 x = v[brev_bits(i, bits)];
  const double a = (x.x / (double)slots) * scale, b = (x.y / (double)slots) * scale;
  const double lim = 4611686018427387904.0;  // 2^62
  if (!isfinite(a) || !isfinite(b) || fabs(a) >= lim || fabs(b) >= lim) {
    if (status) atomicOr(status, 1);
    return;
  }
  const int64_t ra = llround(a), rb = llround(b);
  for (uint32_t j = blockIdx.z; j < nlimb; j += gridDim.z) {
    uint64_t* o = out + (size_t)j * n;
    o[(size_t)i * gap] = lift_signed_mc(ra, mc[j]);
    o[(size_t)(i + slots) * gap] = lift_signed_mc(rb, mc[j]);
    // the other coefficients of this slot's two gap blocks are zero
    for (uint32_t z = 1; z < gap; ++z) {
      o[(size_t)i * gap + z] = 0;
      o[(size_t)(i + slots) * gap + z] = 0;
    }
  }
}

// Balanced Garner reconstruction of coefficient positions i*gap, i < 2 slots,
// then division by the scale; writes complex slot inputs of the forward FFT
// at bit-reversed positions.
template <int MAXL>
__global__ void k_crt_decode(const uint64_t* coef, double2* v, const ModConst* mc,
                             const uint64_t* garner, const uint64_t* mods, uint32_t n,
                             uint32_t nlimb, uint32_t L, uint32_t slots, uint32_t bits,
                             uint32_t gap, double scale) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 2 * slots) return;
  const size_t pos = (size_t)t * gap;
  int64_t a[MAXL];
  double val = 0.0;
  for (uint32_t i = 0; i < nlimb; ++i) {
    const uint64_t q = mc[i].q;
    uint64_t x = coef[(size_t)i * n + pos];
    for (uint32_t j = 0; j < i; ++j) {
      const uint64_t aj = lift_signed(a[j], q);
      x = shoup(sub_mod(x, aj, q), garner[((size_t)i * L + j) * 2],
                garner[((size_t)i * L + j) * 2 + 1], q);
    }
    a[i] = x > (q >> 1) ? (int64_t)x - (int64_t)q : (int64_t)x;
  }
  val = (double)a[nlimb - 1];
  for (int i = (int)nlimb - 2; i >= 0; --i) val = val * (double)mods[i] + (double)a[i];
  val = val / scale;
  const uint32_t slot = t < slots ? t : t - slots;
  double* dst = reinterpret_cast<double*>(v + brev_bits(slot, bits));
  dst[t < slots ? 0 : 1] = val;
}

// The special FFT of nvec contiguous vectors of `slots` values each.  The
// block kernels' blocks of `top` values never straddle two vectors (top
// divides slots), so they run over the batch as one array.
void run_stages(Context& c, double2* v, const double* tw, uint32_t slots, bool inverse,
                uint32_t nvec = 1) {
  if (slots < 2) return;
  const uint32_t threads = slots / 2 < TPB ? slots / 2 : TPB;
  const uint32_t blocks = (slots / 2 + threads - 1) / threads;
  const uint32_t top = slots < FFT_BLOCK ? slots : FFT_BLOCK;
  const uint32_t bthreads = top / 2 < TPB ? top / 2 : TPB;
  const uint32_t nblk = nvec * (slots / top);
  if (inverse) {
    for (uint32_t len = slots; len > top; len >>= 1)
      FHE_LAUNCH(c, "k_fft_inv_stage", k_fft_inv_stage, dim3(blocks, nvec), dim3(threads), 0, v, tw, slots, len);
    FHE_LAUNCH(c, "k_fft_inv_block", k_fft_inv_block, dim3(nblk), dim3(bthreads), 0, v, tw, top);
  } else {
    FHE_LAUNCH(c, "k_fft_fwd_block", k_fft_fwd_block, dim3(nblk), dim3(bthreads), 0, v, tw, top);
    for (uint32_t len = 2 * top; len <= slots; len <<= 1)
      FHE_LAUNCH(c, "k_fft_fwd_stage", k_fft_fwd_stage, dim3(blocks, nvec), dim3(threads), 0, v, tw, slots, len);
  }
}

void check_slots(const Context& c, uint32_t slots) {
  if (slots == 0 || (slots & (slots - 1)) || slots > c.n / 2)
    throw ArgError("slots must be a power of two <= N/2");
}

}  // namespace

bool encode(Context& c, const double* re, const double* im, uint32_t count, uint32_t slots,
            double scale, uint32_t nlimb, uint64_t* out) {
  check_slots(c, slots);
  if (count > slots) throw ArgError("more values than slots");
  if (nlimb == 0 || nlimb > c.L) throw ArgError("bad limb count");
  if (!(scale > 0) || !std::isfinite(scale)) throw ArgError("scale must be positive");
  const size_t bytes = 2 * (size_t)slots * sizeof(double);
  const auto tw = fft_tables(c, slots);
  Scratch v(c, 2 * (size_t)slots), st(c, 1);
  // Range bound: each inverse-FFT stage maps (a, b) to (a + b, (a - b) w)
  // with |w| = 1, so an output's modulus is at most the sum of the inputs'
  // and, after the division by slots, at most the largest input modulus.
  // Inputs whose bound times the scale stays below 2^62 (the margin 2^-20
  // is far above the transform's rounding) cannot fail k_round_lift's range
  // check, so nothing waits for the device; other inputs read the check's
  // status back, which waits for the stream.
  // |z|^2 < (2^62 (1 - 2^-20) / scale)^2 for every value, with NaN and
  // infinities failing the comparison.
  const double lim = 4611686018427387904.0 * (1.0 - 0x1p-20) / scale;
  const double lim2 = lim * lim;
  bool checked = !(lim2 < INFINITY);
  {
    std::lock_guard<std::mutex> g(c.staging_mu);
    Context::Staging& sg = c.staging_slot(bytes);
    double* host = static_cast<double*>(sg.host);
    int over = 0;
    for (uint32_t j = 0; j < count; ++j) {
      const double a = re[j], b = im ? im[j] : 0.0;
      host[2 * j] = a;
      host[2 * j + 1] = b;
      over |= !(a * a + b * b < lim2);
    }
    checked = checked || over;
    std::memset(host + 2 * (size_t)count, 0, bytes - 2 * (size_t)count * sizeof(double));
    hip_check(hipMemcpyAsync(v.p, host, bytes, hipMemcpyHostToDevice, c.stream),
              "encode upload");
    hip_check(hipEventRecord(sg.done, c.stream), "encode staging event");
  }
  if (checked) hip_check(hipMemsetAsync(st.p, 0, 8, c.stream), "encode status");
  run_stages(c, reinterpret_cast<double2*>(v.p), tw.first, slots, true);
  const uint32_t threads = slots < TPB ? slots : TPB;
  // k_round_lift writes every coefficient of the nlimb limbs (the slots'
  // positions and the zeros between them).
  FHE_LAUNCH(c, "k_round_lift", k_round_lift, dim3((slots + threads - 1) / threads, 1, nlimb), dim3(threads), 0, reinterpret_cast<const double2*>(v.p), out, nullptr, c.d_const, slots, ilog2(slots), c.n / (2 * slots), c.n, nlimb, scale, checked ? reinterpret_cast<int*>(st.p) : nullptr);
  if (checked) {
    int status = 0;
    hip_check(hipMemcpyAsync(&status, st.p, sizeof(int), hipMemcpyDeviceToHost, c.stream),
              "encode status");
    hip_check(hipStreamSynchronize(c.stream), "encode sync");
    if (status) return false;
  }
  ntt_forward(c, out, 1, 0, nlimb, LimbMap::contiguous(0));
  return true;
}

bool encode_many(Context& c, const double* re, const double* im, uint32_t count, uint32_t nvec,
                 uint32_t slots, double scale, uint32_t nlimb, uint64_t* const* outs) {
  check_slots(c, slots);
  if (count > slots) throw ArgError("more values than slots");
  if (nlimb == 0 || nlimb > c.L) throw ArgError("bad limb count");
  if (!(scale > 0) || !std::isfinite(scale)) throw ArgError("scale must be positive");
  const double lim = 4611686018427387904.0 * (1.0 - 0x1p-20) / scale;
  const double lim2 = lim * lim;
  const auto tw = fft_tables(c, slots);
  // Up to kChunk vectors share one staging copy and one set of launches:
  // the pointer table (padded to 16 bytes) and then the vectors' values.
  constexpr uint32_t kChunk = 16;
  for (uint32_t r0 = 0; r0 < nvec; r0 += kChunk) {
    const uint32_t m = nvec - r0 < kChunk ? nvec - r0 : kChunk;
    bool over = !(lim2 < INFINITY);
    for (uint32_t r = r0; r < r0 + m && !over; ++r)
      for (uint32_t j = 0; j < count; ++j) {
        const double a = re[(size_t)r * count + j], b = im ? im[(size_t)r * count + j] : 0.0;
        if (!(a * a + b * b < lim2)) {
          over = true;
          break;
        }
      }
    if (over) {
      // Values that may not fit take the checked single path, which
      // reports the first vector that fails.
      for (uint32_t r = r0; r < r0 + m; ++r)
        if (!encode(c, re + (size_t)r * count, im ? im + (size_t)r * count : nullptr, count, slots,
                    scale, nlimb, outs[r]))
          return false;
      continue;
    }
    const size_t tab_words = (m + 1) & ~1u, vec_words = 2 * (size_t)slots;
    const size_t words = tab_words + m * vec_words;
    Scratch buf(c, words);
    double2* v = reinterpret_cast<double2*>(buf.p + tab_words);
    {
      std::lock_guard<std::mutex> g(c.staging_mu);
      Context::Staging& sg = c.staging_slot(words * 8);
      uint64_t* host = static_cast<uint64_t*>(sg.host);
      for (uint32_t r = 0; r < m; ++r) host[r] = reinterpret_cast<uint64_t>(outs[r0 + r]);
      double* hv = reinterpret_cast<double*>(host + tab_words);
      for (uint32_t r = 0; r < m; ++r) {
        const double* rr = re + (size_t)(r0 + r) * count;
        const double* ri = im ? im + (size_t)(r0 + r) * count : nullptr;
        double* h = hv + r * vec_words;
        for (uint32_t j = 0; j < count; ++j) {
          h[2 * j] = rr[j];
          h[2 * j + 1] = ri ? ri[j] : 0.0;
        }
        std::memset(h + 2 * (size_t)count, 0, (vec_words - 2 * (size_t)count) * sizeof(double));
      }
      hip_check(hipMemcpyAsync(buf.p, host, words * 8, hipMemcpyHostToDevice, c.stream),
                "encode upload");
      hip_check(hipEventRecord(sg.done, c.stream), "encode staging event");
    }
    uint64_t* const* table = reinterpret_cast<uint64_t* const*>(buf.p);
    run_stages(c, v, tw.first, slots, true, m);
    const uint32_t threads = slots < TPB ? slots : TPB;
    FHE_LAUNCH(c, "k_round_lift", k_round_lift, dim3((slots + threads - 1) / threads, m, nlimb), dim3(threads), 0, v, nullptr, table, c.d_const, slots, ilog2(slots), c.n / (2 * slots), c.n, nlimb, scale, nullptr);
    ntt_forward_table(c, table, m, nlimb);
  }
  return true;
}

void decode(Context& c, const uint64_t* pt, uint32_t nlimb, uint32_t slots, double scale,
            double* re, double* im) {
  check_slots(c, slots);
  if (nlimb == 0 || nlimb > c.L) throw ArgError("bad limb count");
  const auto tw = fft_tables(c, slots);
  Scratch coef(c, (size_t)nlimb * c.n), v(c, 2 * (size_t)slots), mods(c, c.L);
  hip_check(hipMemcpyAsync(coef.p, pt, (size_t)nlimb * c.n * 8, hipMemcpyDeviceToDevice,
                           c.stream),
            "decode copy");
  hip_check(hipMemcpyAsync(mods.p, c.mods.data(), c.L * 8, hipMemcpyHostToDevice, c.stream),
            "decode moduli");
  ntt_inverse(c, coef.p, 1, 0, nlimb, LimbMap::contiguous(0));
  const uint32_t cnt = 2 * slots, threads = cnt < 64 ? cnt : 64;
  FHE_LAUNCH(c, "k_crt_decode", (k_crt_decode<64>), dim3((cnt + threads - 1) / threads), dim3(threads), 0, coef.p, reinterpret_cast<double2*>(v.p), c.d_const, c.d_garner, mods.p, c.n, nlimb, c.L, slots, ilog2(slots), c.n / (2 * slots), scale);
  run_stages(c, reinterpret_cast<double2*>(v.p), tw.second, slots, false);
  std::vector<double> host(2 * (size_t)slots);
  hip_check(hipMemcpyAsync(host.data(), v.p, host.size() * 8, hipMemcpyDeviceToHost, c.stream),
            "decode download");
  hip_check(hipStreamSynchronize(c.stream), "decode sync");
  for (uint32_t j = 0; j < slots; ++j) {
    re[j] = host[2 * j];
    if (im) im[j] = host[2 * j + 1];
  }
}

}  // namespace fhe
