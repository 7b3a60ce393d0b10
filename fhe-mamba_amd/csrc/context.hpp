// Device-resident CKKS-RNS context: moduli, transform tables and the basis
// conversion constants used by key switching and rescaling.
//
// Layout conventions (all device arrays are uint64 words):
//   modulus index m in [0, L+K): q_0..q_{L-1} then p_0..p_{K-1}.
//   RNS polynomial sets are limb-major: [poly][limb][N].
//   Transform tables per modulus: tw_fwd[m][k] = (psi^brv(k), Shoup),
//   tw_inv[m][k] = (psi^-brv(k), Shoup), one 16-byte pair per entry.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "modarith.hpp"
#include "sampling.hpp"

namespace fhe {

struct HipError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct StateError : std::logic_error {
  using std::logic_error::logic_error;
};
struct ArgError : std::invalid_argument {
  using std::invalid_argument::invalid_argument;
};

inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw HipError(std::string(what) + ": " + hipGetErrorString(e));
}

// Per-modulus scalar constants.
struct ModConst {
  uint64_t q;
  uint64_t qinv_neg;   // -q^-1 mod 2^64
  uint64_t mu64;       // floor(2^64 / q)
  uint64_t r64;        // 2^64 mod q
  uint64_t r64_sh;     // Shoup companion of r64
  uint64_t ninv;       // N^-1 mod q
  uint64_t ninv_sh;
  uint64_t r2;         // 2^128 mod q (to Montgomery form via redc)
  // 2^64 - q and 2^64 - 4q, read from memory so that the compiler keeps
  // additions of them (shoup_lazy4n, lazy_sub) instead of folding them back
  // into borrow-chain subtractions.
  uint64_t neg_q, neg_q4;
  uint64_t qinv;       // q^-1 mod 2^64 (redc_lazy)
  uint64_t neg_q8;     // 2^64 - 8q (lazy_sub at 8q; 0 when 8q >= 2^64)
  float rq;            // 2^32 / q (1 - 2^-20), rounded down (reduce_est)
  uint32_t pad_;
};

// x mod q for a 128-bit x = hi * 2^64 + lo (any hi): hi * (2^64 mod q) by
// Shoup and lo by a one-word Barrett step, both in [0, 2q), then reduce.
FHE_HD uint64_t reduce128(uint64_t hi, uint64_t lo, const ModConst& m) {
  const uint64_t a = shoup_lazy(hi, m.r64, m.r64_sh, m.q);
  const uint64_t b = lo - mulhi64(lo, m.mu64) * m.q;
  return reduce_4q(a + b, m.q);
}

FHE_HD uint64_t mul_mod(uint64_t a, uint64_t b, const ModConst& m) {
  const u128 p = (u128)a * b;
  return reduce128((uint64_t)(p >> 64), (uint64_t)p, m);
}

// Basis-conversion plan from a source basis to a target basis:
//   v_i = x_i * qhat_inv_i (Shoup), y_k = sum_i v_i * qhat_ik mod t_k,
// with qhat_ik stored in Montgomery form w.r.t. t_k so that one REDC of the
// 128-bit accumulator gives the standard-domain result.
struct ConvPlan {
  uint32_t nsrc = 0, ndst = 0;
  std::vector<uint32_t> src_idx, dst_idx;  // modulus indices
  uint64_t* d_qhat_inv = nullptr;          // [nsrc][2]  (value, Shoup)
  // qhat_inv_i * N^-1 mod s_i (value, Shoup): the first factor with the
  // inverse NTT's scaling folded in, for conversions fused after a transform.
  uint64_t* d_src_scale = nullptr;         // [nsrc][2]
  uint64_t* d_qhat_mont = nullptr;         // [nsrc][ndst]
  uint64_t* d_qhat_mont30 = nullptr;       // [nsrc][ndst]: qhat_mont * 2^30 mod t_k
  uint32_t* d_dst_idx = nullptr;           // [ndst]
  uint32_t* d_src_idx32 = nullptr;         // [nsrc]
};

// Optional per-launch timing with HIP events on the context stream
// (enabled by fhe_profile_begin).  Records (kernel name, start, stop).
struct Profiler {
  bool on = false;
  struct Rec {
    const char* name;
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  std::vector<hipEvent_t> spare;
  hipEvent_t get();
  void clear();
  ~Profiler();
};

class Pool {
 public:
  explicit Pool(int device) : device_(device) {}
  ~Pool();
  void* get(size_t bytes);
  void put(void* p, size_t bytes);
  void trim();

 private:
  int device_;
  std::mutex mu_;
  std::multimap<size_t, void*> free_;
};

// Allocation requests the library has made in this process: every pool
// request (fresh or reused) and every direct device or pinned-host
// allocation of tables and staging buffers.
void note_alloc();
uint64_t alloc_requests();

// Bytes from the OS CSPRNG (getrandom); throws if none are available.
void fill_entropy(void* buf, size_t bytes);

struct Context {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  uint32_t log_n = 0, n = 0, L = 0, K = 0, dnum = 0, alpha = 0;
  uint32_t lds_per_block = 65536;    // LDS a workgroup may allocate (160 KB on gfx950)
  std::vector<uint64_t> mods;        // L + K
  std::vector<uint64_t> psi;         // minimal primitive 2N-th roots
  std::vector<ModConst> hconst;

  // device tables
  ModConst* d_const = nullptr;       // [L+K]
  uint64_t* d_tw_fwd = nullptr;      // [L+K][N][2]
  uint64_t* d_tw_inv = nullptr;      // [L+K][N][2]
  // rescale: rs[l][i] = (q_l mod q_i, (q_l)^-1 mod q_i, Shoup) for i < l
  uint64_t* d_rescale = nullptr;     // [L][L][4]
  // ModDown: P^-1 mod q_i (value, Shoup)
  uint64_t* d_pinv_q = nullptr;      // [L][2]
  std::vector<uint64_t> pinv_host;   // [L] P^-1 mod q_i
  // Key words are stored as k * f_i * 2^-64 with f_i = 2^128 * P^-1 (Q limbs)
  // or 2^128 (P limbs) mod the limb's modulus: Montgomery form with P^-1
  // folded into the Q limbs, so the key inner product yields ext * P^-1.
  uint64_t* d_keyfac = nullptr;      // [L+K]
  uint64_t* d_keyfac_out = nullptr;  // [L+K]: P mod q_i (Q limbs), 1 (P limbs)

  // Garner CRT inverses g[i][j] = (q_j^-1 mod q_i, Shoup) for j < i (decode).
  uint64_t* d_garner = nullptr;      // [L][L][2]
  // Special-FFT twiddles per slot count: (inverse, forward), each [slots-1] x (cos, sin).
  std::mutex fft_mu;
  std::map<uint32_t, std::pair<double*, double*>> fft_tables;

  // Pinned host buffers staging encode inputs, so that their uploads are
  // asynchronous: a ring whose slot is reused once the copy recorded on it
  // has completed (staging_slot waits for that copy, not for the stream).
  struct Staging {
    void* host = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;
  };
  static constexpr int kStagingSlots = 16;
  std::mutex staging_mu;
  Staging staging[kStagingSlots];
  uint32_t staging_next = 0;
  // The next ring slot, holding at least `bytes`; the caller records the
  // completion of its copy out of the slot on `done`.
  Staging& staging_slot(size_t bytes);

  // Stream family for key generation and encryption: ChaCha20 under a
  // master key from OS entropy unless the caller sets one (or chooses the
  // seeded parity family).
  SamplingKey sampling;

  std::unique_ptr<Pool> pool;
  Profiler prof;
  std::mutex plan_mu;
  std::map<std::pair<uint64_t, uint64_t>, std::unique_ptr<ConvPlan>> plans;

  Context(uint32_t log_n, const uint64_t* q, uint32_t num_q, const uint64_t* p,
          uint32_t num_p, uint32_t dnum, int device);
  ~Context();

  // Conversion plan for source modulus set [s, e) of Q (or all of P when
  // s == UINT32_MAX) into target = (Q[0..nq) minus the source) + P, or for
  // ModDown P -> Q[0..nq).
  const ConvPlan& modup_plan(uint32_t s, uint32_t e, uint32_t nq);
  const ConvPlan& moddown_plan(uint32_t nq);

  void* alloc(size_t bytes) { return pool->get(bytes); }
  void release(void* p, size_t bytes) { pool->put(p, bytes); }

  // While `base` is set, Scratch carves its buffers from this caller-given
  // device region (LIFO, 256-byte aligned) instead of the pool, and throws
  // when the region is too small.  Used by the entry point that must not
  // allocate.
  struct Arena {
    uint64_t* base = nullptr;
    size_t words = 0, used = 0;
  } arena;

  // Whether the conversion plans of a key switch at nq limbs (every ModUp
  // digit and the ModDown) are built; never builds them.
  bool has_keyswitch_plans(uint32_t nq);

 private:
  // factor (optional, per target) multiplies every constant of target k.
  ConvPlan* build_plan(const std::vector<uint32_t>& src, const std::vector<uint32_t>& dst,
                       const std::vector<uint64_t>* factor = nullptr);
};

// Limb -> modulus index map for a batch of limbs: limb j < split uses
// modulus base0 + j, limb j >= split uses base1 + (j - split).
struct LimbMap {
  uint32_t split, base0, base1;
  FHE_HD uint32_t operator()(uint32_t j) const {
    return j < split ? base0 + j : base1 + (j - split);
  }
  static FHE_HD LimbMap contiguous(uint32_t limb0) { return LimbMap{0xffffffffu, limb0, 0}; }
  // Launch slot j of any poly: limb position j, modulus (*this)(j).
  FHE_HD bool resolve(uint32_t, uint32_t j, uint32_t& pos, uint32_t& mod) const {
    pos = j;
    mod = (*this)(j);
    return true;
  }
};

// Polys held in separate allocations: launch poly p lives at table[p] (a
// device array of poly base pointers, [nlimb][N] each); limb j uses
// modulus j.
struct TableMap {
  uint64_t* const* table;
  FHE_HD bool resolve(uint32_t, uint32_t j, uint32_t& pos, uint32_t& mod) const {
    pos = j;
    mod = j;
    return true;
  }
};

// The converted limbs of ModUp digits [nd][ne][N]: digit (poly) d keeps its
// own limbs [d*alpha, min((d+1)*alpha, nq)) of Q; slot t walks the other
// limbs of Q_l + P in order (position pos, modulus pos < nq ? pos :
// L + pos - nq).  Slots past the digit's count are not launched work.
struct DigitMap {
  uint32_t alpha, nq, L, ne, nd;  // poly = ciphertext * nd + digit
  FHE_HD bool resolve(uint32_t poly, uint32_t t, uint32_t& pos, uint32_t& mod) const {
    const uint32_t d = poly % nd;
    const uint32_t s = d * alpha, e = s + alpha < nq ? s + alpha : nq, w = e - s;
    if (t + w >= ne) return false;
    pos = t < s ? t : t + w;
    mod = pos < nq ? pos : L + (pos - nq);
    return true;
  }
};

// Stream-ordered scratch buffer from the context pool.  Released back to the
// pool on destruction; later work on the same stream may reuse it, which is
// safe because all of a context's kernels run in stream order.
struct Scratch {
  Context& c;
  uint64_t* p;
  size_t bytes;
  size_t mark = 0;  // arena position to restore (arena buffers only)
  Scratch(Context& ctx, size_t words) : c(ctx), p(nullptr), bytes(words * 8) {
    Context::Arena& a = ctx.arena;
    if (!a.base) {
      p = (uint64_t*)ctx.alloc(bytes);
      return;
    }
    const size_t take = (words + 31) & ~(size_t)31;
    if (take > a.words - a.used)
      throw ArgError("the operation needs more device scratch than the no-allocation limit");
    mark = a.used;
    p = a.base + a.used;
    a.used += take;
  }
  ~Scratch() {
    if (c.arena.base)
      c.arena.used = mark;
    else
      c.release(p, bytes);
  }
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
};

// Scope that brackets one kernel launch with profiling events.
struct LaunchScope {
  Context& c;
  const char* name;
  hipEvent_t b = nullptr;
  LaunchScope(Context& ctx, const char* nm) : c(ctx), name(nm) {
    if (c.prof.on) {
      hipEvent_t a = c.prof.get();
      b = c.prof.get();
      hipEventRecord(a, c.stream);
      c.prof.recs.push_back({name, a, b});
    }
  }
  ~LaunchScope() {
    if (b) hipEventRecord(b, c.stream);
  }
};

// Launch `kernel` on the context stream under a profiling scope and check
// the launch status.
#define FHE_LAUNCH(ctx, name, kernel, grid, block, shmem, ...)                      \
  do {                                                                              \
    ::fhe::LaunchScope fhe_scope_((ctx), (name));                                   \
    hipLaunchKernelGGL(kernel, grid, block, shmem, (ctx).stream, __VA_ARGS__);      \
    ::fhe::hip_check(hipGetLastError(), name);                                      \
  } while (0)

// Epilogue of the last forward-NTT pass of a batched ModDown.  Launch poly p
// is key switch r = p / 2, component b = p % 2.  The Q-limb key inner
// product is formed here,
//   ext_r[b][i][s] = REDC(sum_j digits_r[j][i][s] * key_r[j][b][i][s]),
// and carries the factor P^-1 (folded into the stored keys); y carries -P^-1
// (folded into the ModDown conversion constants), so
//   out_r[b][i][d(s)] = ext_r[b][i][s] + y[s] + add_r,b[i][s]
// equals OpenFHE's (ext - Conv(ext_P)) * P^-1 + add exactly, where d is the
// inverse of the Galois permutation of element g_r (ginv = g_r^-1 mod 2N;
// 1 means no permutation).  One REDC suffices while nd * q_i < 2^64.
constexpr int MAX_KS_BATCH = 32;
struct ModDownEpi {
  const uint64_t* digits[MAX_KS_BATCH];   // each [nd][ne][N]
  const ModConst* mc;
  const uint64_t* key[MAX_KS_BATCH];      // each [nd][2][L+K][N], Montgomery form
  uint64_t* out[MAX_KS_BATCH];            // each [2][nq][N]
  const uint64_t* add[MAX_KS_BATCH][2];   // [nq][N] or null
  uint32_t ginv[MAX_KS_BATCH];
  size_t kl;                              // words per key component, (L+K) N
  uint32_t nd, ne, nq, L;
};

// ---- kernel launchers (implemented in the .hip files) ----
void ntt_forward(Context& c, uint64_t* data, uint32_t npoly, size_t poly_stride,
                 uint32_t nlimb, LimbMap map);
void ntt_inverse(Context& c, uint64_t* data, uint32_t npoly, size_t poly_stride,
                 uint32_t nlimb, LimbMap map);
// Forward NTT of npoly one-poly [nlimb][N] operands held in separate
// allocations; `table` is a device array of their npoly base pointers.
void ntt_forward_table(Context& c, uint64_t* const* table, uint32_t npoly, uint32_t nlimb);
// Forward NTT of y [npoly][nq][N] (limb j mod q_j) whose last pass stores
// through the ModDown epilogue instead of writing y back.
void ntt_forward_moddown(Context& c, uint64_t* y, uint32_t npoly, uint32_t nq,
                         const ModDownEpi& epi);
// Inverse NTT into ext_p [2B][K][N] of the P-limb key inner products
//   ext_p[2r+b][t][s] = REDC(sum_j digits[j][nq+t][s] * key_r[j][b][L+t][s]),
// formed while the first pass loads its input (epi.digits / key / mc / kl /
// nd / ne / nq / L are used; the output fields are not).
void ntt_inverse_ksk(Context& c, uint64_t* ext_p, uint32_t npoly, const ModDownEpi& epi);
// ModDown of a key-switch batch in three launches for ring dimensions
// 2^13..2^17 with every Q_l and P modulus below 2^60: the first inverse pass
// with the P-limb inner products (into ext_p, blocked layout), one kernel
// for the inverse column stages + conversion P -> Q_l + forward column
// stages (into y, blocked), and the last forward pass with the epilogue.
bool moddown_fused_ok(const Context& c, uint32_t nq);
void moddown_fused(Context& c, uint64_t* ext_p, uint64_t* y, uint32_t npoly, uint32_t nq,
                   const ConvPlan& pl, const ModDownEpi& epi);
// Rescale of [npoly][nq][N] into out [npoly][nq-1][N] (out != a) in four
// launches, for ring dimensions 2^13..2^17.
void rescale_fused(Context& c, uint64_t* out, const uint64_t* a, uint32_t npoly, uint32_t nq);
// The same for `count` inputs as[r] into outs[r] (each [npoly][nq][N] into
// [npoly][nq-1][N], no output aliasing any input): up to 16 inputs share
// one set of launches.
void rescale_fused_many(Context& c, uint64_t* const* outs, const uint64_t* const* as,
                        uint32_t count, uint32_t npoly, uint32_t nq);
// ModUp of `count` c1 polys (nq limbs each) into digits [count][nd][nq+K][N]
// in four launches for ring dimensions 2^13..2^17 with every modulus below
// 2^60: the first inverse pass reading c1 (blocked out), one kernel for the
// inverse column stages + the conversion of every digit + the forward
// column stages, the last forward pass, and the copy of each digit's own
// limbs.
bool modup_fused_ok(const Context& c, uint32_t nq, uint32_t count);
void modup_fused(Context& c, const uint64_t* const* as, uint32_t count, uint32_t nq,
                 uint64_t* digits);
// Forward NTT of the converted limbs of the ModUp digits of `count`
// ciphertexts, [count][nd][nq+K][N].
void ntt_forward_digits(Context& c, uint64_t* digits, uint32_t count, uint32_t nd, uint32_t nq);

}  // namespace fhe
