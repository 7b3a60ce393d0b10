// Host-side construction of the device context: moduli tables, transform
// twiddles and basis-conversion plans.  Prime selection mirrors OpenFHE's
// CCParams<CryptoContextCKKSRNS> / GenCryptoContext as used by the
// reference executors (native/fideslib_stage0/src/packed_fideslib.cpp:1060-1068).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <cerrno>
#include <sys/random.h>

#include "context.hpp"
#include "params.hpp"

namespace fhe {

hipEvent_t Profiler::get() {
  if (!spare.empty()) {
    hipEvent_t e = spare.back();
    spare.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  hip_check(hipEventCreate(&e), "hipEventCreate");
  return e;
}

void Profiler::clear() {
  for (auto& r : recs) {
    spare.push_back(r.a);
    spare.push_back(r.b);
  }
  recs.clear();
}

Profiler::~Profiler() {
  clear();
  for (hipEvent_t e : spare) hipEventDestroy(e);
}

Pool::~Pool() {
  hipSetDevice(device_);
  for (auto& kv : free_) hipFree(kv.second);
}

static std::atomic<uint64_t> g_alloc_requests{0};
void note_alloc() { g_alloc_requests.fetch_add(1, std::memory_order_relaxed); }
uint64_t alloc_requests() { return g_alloc_requests.load(std::memory_order_relaxed); }

void* Pool::get(size_t bytes) {
  note_alloc();
  bytes = (bytes + 255) & ~size_t(255);
  {
    std::lock_guard<std::mutex> g(mu_);
    auto it = free_.find(bytes);
    if (it != free_.end()) {
      void* p = it->second;
      free_.erase(it);
      return p;
    }
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    // A failed hipMalloc also sets the thread's last error; clear it so the
    // next launch check does not report an allocation that the retry below
    // satisfies.
    (void)hipGetLastError();
    trim();
    hip_check(hipMalloc(&p, bytes), "hipMalloc");
  }
  return p;
}

void Pool::put(void* p, size_t bytes) {
  if (!p) return;
  bytes = (bytes + 255) & ~size_t(255);
  std::lock_guard<std::mutex> g(mu_);
  free_.emplace(bytes, p);
}

void Pool::trim() {
  std::lock_guard<std::mutex> g(mu_);
  hipDeviceSynchronize();
  for (auto& kv : free_) hipFree(kv.second);
  free_.clear();
}

// Fills buf with bytes from the kernel's CSPRNG (getrandom); fails loudly
// rather than falling back to anything weaker.
void fill_entropy(void* buf, size_t bytes) {
  uint8_t* p = static_cast<uint8_t*>(buf);
  while (bytes) {
    const ssize_t got = getrandom(p, bytes, 0);
    if (got < 0) {
      if (errno == EINTR) continue;
      throw std::runtime_error("getrandom failed: no OS entropy for the sampling key");
    }
    p += got;
    bytes -= (size_t)got;
  }
}

static uint32_t bitrev(uint32_t x, uint32_t bits) {
  uint32_t r = 0;
  for (uint32_t i = 0; i < bits; ++i) {
    r = (r << 1) | (x & 1);
    x >>= 1;
  }
  return r;
}

template <typename T>
static T* upload(const std::vector<T>& v) {
  T* d = nullptr;
  if (v.empty()) return nullptr;
  note_alloc();
  hip_check(hipMalloc(&d, v.size() * sizeof(T)), "hipMalloc(table)");
  hip_check(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "upload table");
  return d;
}

Context::Context(uint32_t log_n_, const uint64_t* q, uint32_t num_q, const uint64_t* p,
                 uint32_t num_p, uint32_t dnum_, int device_) {
  if (log_n_ < 4 || log_n_ > 17) throw ArgError("log_n must be in [4, 17]");
  if (num_q == 0 || num_q > 64 || num_p > 64) throw ArgError("1..64 Q primes and <= 64 P primes");
  if (dnum_ == 0) throw ArgError("dnum must be positive");
  device = device_;
  log_n = log_n_;
  n = 1u << log_n;
  L = num_q;
  K = num_p;
  alpha = (L + dnum_ - 1) / dnum_;
  dnum = (L + alpha - 1) / alpha;
  mods.assign(q, q + L);
  mods.insert(mods.end(), p, p + K);
  const uint64_t m2n = 2ull * n;
  for (size_t i = 0; i < mods.size(); ++i) {
    const uint64_t qi = mods[i];
    if (qi >= (1ull << 61) || qi < 3 || (qi - 1) % m2n != 0 || !is_prime(qi))
      throw ArgError("modulus " + std::to_string(qi) + " is not a prime = 1 mod 2N below 2^61");
    for (size_t j = 0; j < i; ++j)
      if (mods[j] == qi) throw ArgError("duplicate modulus");
  }
  fill_entropy(sampling.master, sizeof(sampling.master));
  sampling.secure = true;
  hip_check(hipSetDevice(device), "hipSetDevice");
  {
    int lds = 0;
    hip_check(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device),
              "hipDeviceGetAttribute(LDS)");
    lds_per_block = lds > 0 ? (uint32_t)lds : 65536u;
  }
  hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
  own_stream = true;
  pool.reset(new Pool(device));

  const uint32_t nm = L + K;
  psi.resize(nm);
  hconst.resize(nm);
  std::vector<uint64_t> fwd((size_t)nm * n * 2), inv((size_t)nm * n * 2);
  std::vector<uint64_t> pw(n), ipw(n);
  for (uint32_t i = 0; i < nm; ++i) {
    const uint64_t qi = mods[i];
    psi[i] = min_root_of_unity(m2n, qi);
    const uint64_t psi_inv = host_invmod(psi[i], qi);
    pw[0] = ipw[0] = 1;
    for (uint32_t k = 1; k < n; ++k) {
      pw[k] = host_mulmod(pw[k - 1], psi[i], qi);
      ipw[k] = host_mulmod(ipw[k - 1], psi_inv, qi);
    }
    for (uint32_t k = 0; k < n; ++k) {
      const uint32_t r = bitrev(k, log_n);
      const size_t o = ((size_t)i * n + k) * 2;
      fwd[o] = pw[r];
      fwd[o + 1] = host_shoup(pw[r], qi);
      inv[o] = ipw[r];
      inv[o + 1] = host_shoup(ipw[r], qi);
    }
    ModConst& mc = hconst[i];
    std::memset(&mc, 0, sizeof(mc));
    mc.q = qi;
    mc.qinv_neg = host_qinv_neg(qi);
    mc.mu64 = (uint64_t)(((u128)1 << 64) / qi);
    mc.r64 = (uint64_t)(((u128)1 << 64) % qi);
    mc.r64_sh = host_shoup(mc.r64, qi);
    mc.r2 = (uint64_t)((u128)mc.r64 * mc.r64 % qi);
    mc.ninv = host_invmod(n % qi, qi);
    mc.ninv_sh = host_shoup(mc.ninv, qi);
    mc.neg_q = 0 - qi;
    mc.neg_q4 = 0 - 4 * qi;
    mc.qinv = 0 - mc.qinv_neg;
    mc.neg_q8 = qi < (1ull << 61) ? 0 - 8 * qi : 0;
    {
      // Rounded down, so the quotient estimate never exceeds the quotient.
      const double want = 4294967296.0 / (double)qi * (1.0 - 1.0 / 1048576.0);
      float f = (float)want;
      while ((double)f > want) f = std::nextafter(f, 0.0f);
      mc.rq = f;
    }
  }
  d_const = upload(hconst);
  d_tw_fwd = upload(fwd);
  d_tw_inv = upload(inv);

  // Rescale constants rs[l][i] for i < l.
  std::vector<uint64_t> rs((size_t)L * L * 4, 0);
  for (uint32_t l = 1; l < L; ++l)
    for (uint32_t i = 0; i < l; ++i) {
      const uint64_t qi = mods[i], ql = mods[l] % qi;
      const uint64_t inv_ = host_invmod(ql, qi);
      const size_t o = ((size_t)l * L + i) * 4;
      rs[o] = ql;
      rs[o + 1] = inv_;
      rs[o + 2] = host_shoup(inv_, qi);
      rs[o + 3] = host_shoup(ql, qi);
    }
  d_rescale = upload(rs);

  std::vector<uint64_t> pinv((size_t)L * 2, 0);
  for (uint32_t i = 0; i < L; ++i) {
    const uint64_t qi = mods[i];
    uint64_t pm = 1 % qi;
    for (uint32_t k = 0; k < K; ++k) pm = host_mulmod(pm, mods[L + k] % qi, qi);
    const uint64_t v = host_invmod(pm, qi);
    pinv[2 * i] = v;
    pinv[2 * i + 1] = host_shoup(v, qi);
    pinv_host.push_back(v);
  }
  d_pinv_q = upload(pinv);

  std::vector<uint64_t> keyfac(nm);
  for (uint32_t i = 0; i < nm; ++i)
    keyfac[i] = i < L ? host_mulmod(pinv_host[i], hconst[i].r2, mods[i]) : hconst[i].r2;
  d_keyfac = upload(keyfac);
  // the inverse map, device key -> standard form: a Montgomery product by
  // P mod q_i undoes P^-1 R on the Q limbs, by 1 undoes R on the P limbs
  std::vector<uint64_t> keyfac_out(nm, 1);
  for (uint32_t i = 0; i < L; ++i) keyfac_out[i] = host_invmod(pinv_host[i], mods[i]);
  d_keyfac_out = upload(keyfac_out);

  std::vector<uint64_t> garner((size_t)L * L * 2, 0);
  for (uint32_t i = 0; i < L; ++i)
    for (uint32_t j = 0; j < i; ++j) {
      const uint64_t qi = mods[i], v = host_invmod(mods[j] % qi, qi);
      garner[((size_t)i * L + j) * 2] = v;
      garner[((size_t)i * L + j) * 2 + 1] = host_shoup(v, qi);
    }
  d_garner = upload(garner);
}

Context::Staging& Context::staging_slot(size_t bytes) {
  Staging& s = staging[staging_next];
  staging_next = (staging_next + 1) % kStagingSlots;
  if (s.done)
    hip_check(hipEventSynchronize(s.done), "staging wait");
  else
    hip_check(hipEventCreateWithFlags(&s.done, hipEventDisableTiming), "staging event");
  if (s.bytes < bytes) {
    if (s.host) hip_check(hipHostFree(s.host), "hipHostFree");
    s.host = nullptr;
    s.bytes = 0;
    note_alloc();
    hip_check(hipHostMalloc(&s.host, bytes, hipHostMallocDefault), "hipHostMalloc");
    s.bytes = bytes;
  }
  return s;
}

Context::~Context() {
  hipSetDevice(device);
  if (stream) hipStreamSynchronize(stream);
  for (Staging& s : staging) {
    if (s.host) hipHostFree(s.host);
    if (s.done) hipEventDestroy(s.done);
  }
  for (auto& kv : plans) {
    ConvPlan* pl = kv.second.get();
    hipFree(pl->d_qhat_inv);
    hipFree(pl->d_src_scale);
    hipFree(pl->d_qhat_mont);
    hipFree(pl->d_qhat_mont30);
    hipFree(pl->d_dst_idx);
    hipFree(pl->d_src_idx32);
  }
  hipFree(d_const);
  hipFree(d_tw_fwd);
  hipFree(d_tw_inv);
  hipFree(d_rescale);
  hipFree(d_pinv_q);
  hipFree(d_keyfac);
  hipFree(d_keyfac_out);
  hipFree(d_garner);
  for (auto& kv : fft_tables) {
    hipFree(kv.second.first);
    hipFree(kv.second.second);
  }
  pool.reset();
  if (own_stream && stream) hipStreamDestroy(stream);
}

ConvPlan* Context::build_plan(const std::vector<uint32_t>& src, const std::vector<uint32_t>& dst,
                              const std::vector<uint64_t>* factor) {
  std::unique_ptr<ConvPlan> pl(new ConvPlan);
  pl->nsrc = (uint32_t)src.size();
  pl->ndst = (uint32_t)dst.size();
  pl->src_idx = src;
  pl->dst_idx = dst;
  std::vector<uint64_t> qhat_inv(2 * src.size()), qhat_mont(src.size() * dst.size());
  std::vector<uint64_t> qhat_mont30(src.size() * dst.size());
  std::vector<uint64_t> src_scale(2 * src.size());
  for (size_t a = 0; a < src.size(); ++a) {
    const uint64_t qa = mods[src[a]];
    uint64_t h = 1 % qa;
    for (size_t b = 0; b < src.size(); ++b)
      if (b != a) h = host_mulmod(h, mods[src[b]] % qa, qa);
    const uint64_t hi = host_invmod(h, qa);
    qhat_inv[2 * a] = hi;
    qhat_inv[2 * a + 1] = host_shoup(hi, qa);
    const uint64_t sc = host_mulmod(hi, host_invmod(n % qa, qa), qa);
    src_scale[2 * a] = sc;
    src_scale[2 * a + 1] = host_shoup(sc, qa);
    for (size_t k = 0; k < dst.size(); ++k) {
      const uint64_t t = mods[dst[k]];
      uint64_t hk = 1 % t;
      for (size_t b = 0; b < src.size(); ++b)
        if (b != a) hk = host_mulmod(hk, mods[src[b]] % t, t);
      if (factor) hk = host_mulmod(hk, (*factor)[k] % t, t);
      qhat_mont[a * dst.size() + k] = host_to_mont(hk, t);
      qhat_mont30[a * dst.size() + k] =
          host_mulmod(qhat_mont[a * dst.size() + k], (1ull << 30) % t, t);
    }
  }
  pl->d_qhat_inv = upload(qhat_inv);
  pl->d_qhat_mont = upload(qhat_mont);
  pl->d_qhat_mont30 = upload(qhat_mont30);
  pl->d_src_scale = upload(src_scale);
  pl->d_dst_idx = upload(dst);
  pl->d_src_idx32 = upload(src);
  ConvPlan* raw = pl.get();
  plans[{(uint64_t)raw, (uint64_t)raw}] = std::move(pl);
  return raw;
}

const ConvPlan& Context::modup_plan(uint32_t s, uint32_t e, uint32_t nq) {
  std::lock_guard<std::mutex> g(plan_mu);
  const uint64_t key1 = ((uint64_t)1 << 63) | ((uint64_t)s << 32) | e;
  const uint64_t key2 = nq;
  auto it = plans.find({key1, key2});
  if (it != plans.end()) return *it->second;
  std::vector<uint32_t> src, dst;
  for (uint32_t i = s; i < e; ++i) src.push_back(i);
  for (uint32_t i = 0; i < nq; ++i)
    if (i < s || i >= e) dst.push_back(i);
  for (uint32_t k = 0; k < K; ++k) dst.push_back(L + k);
  ConvPlan* raw = build_plan(src, dst);
  auto node = plans.extract({(uint64_t)raw, (uint64_t)raw});
  node.key() = {key1, key2};
  plans.insert(std::move(node));
  return *raw;
}

bool Context::has_keyswitch_plans(uint32_t nq) {
  std::lock_guard<std::mutex> g(plan_mu);
  if (!plans.count({(uint64_t)1 << 62, nq})) return false;
  const uint32_t nd = (nq + alpha - 1) / alpha < dnum ? (nq + alpha - 1) / alpha : dnum;
  for (uint32_t j = 0; j < nd; ++j) {
    const uint32_t s = j * alpha, e = s + alpha < nq ? s + alpha : nq;
    if (!plans.count({((uint64_t)1 << 63) | ((uint64_t)s << 32) | e, nq})) return false;
  }
  return true;
}

const ConvPlan& Context::moddown_plan(uint32_t nq) {
  std::lock_guard<std::mutex> g(plan_mu);
  const uint64_t key1 = ((uint64_t)1 << 62), key2 = nq;
  auto it = plans.find({key1, key2});
  if (it != plans.end()) return *it->second;
  std::vector<uint32_t> src, dst;
  for (uint32_t k = 0; k < K; ++k) src.push_back(L + k);
  for (uint32_t i = 0; i < nq; ++i) dst.push_back(i);
  // ModDown subtracts the conversion and multiplies by P^-1: fold -P^-1 in.
  std::vector<uint64_t> neg_pinv(nq);
  for (uint32_t i = 0; i < nq; ++i) neg_pinv[i] = pinv_host[i] ? mods[i] - pinv_host[i] : 0;
  ConvPlan* raw = build_plan(src, dst, &neg_pinv);
  auto node = plans.extract({(uint64_t)raw, (uint64_t)raw});
  node.key() = {key1, key2};
  plans.insert(std::move(node));
  return *raw;
}

}  // namespace fhe
