// Client-side key material, encryption and decryption on the GPU.
//
// Mirrors OpenFHE's KeyGen / EvalMultKeyGen / EvalRotateKeyGen / Encrypt /
// Decrypt as called by the reference (native/fideslib_stage0/src/
// packed_fideslib.cpp:1080-1083, :204-205, :1227) with this library's
// sampling streams (sampling.hpp; ChaCha20 unless the context was switched
// to the seeded parity family):
//   public key      b = -a s + e over Q, a uniform in evaluation form
//   switching key   digit j: b_j = -a_j s_new + e_j + [P]_{q_i} s_old on the
//                   Q limbs of digit j (KeySwitchHYBRID key generation)
//   Galois key k    s_old = s, s_new = s(X^{k^-1})
//   relin key       s_old = s^2, s_new = s
//   encryption      (pk_b v + e0 + m, pk_a v + e1), v ternary
// Uniform residues are drawn on the GPU (counter-based stream, one word per
// thread); small secrets and errors are drawn on the host and lifted.
#include <vector>

#include "ops.hpp"
#include "sampling.hpp"

namespace fhe {
namespace {

constexpr int TPB = 256;

inline uint32_t tpb_for(const Context& c) { return c.n < TPB ? c.n : TPB; }

// Signed coefficients -> residues for limbs idx0 .. idx0 + nlimb.
__global__ void k_lift_signed(const int64_t* coef, uint64_t* out, const ModConst* mc, uint32_t n,
                              uint32_t idx0) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t q = mc[idx0 + blockIdx.y].q;
  const int64_t x = coef[e];
  uint64_t r;
  if (x >= 0) {
    r = (uint64_t)x % q;
  } else {
    const uint64_t m = ((uint64_t)(-x)) % q;
    r = m ? q - m : 0;
  }
  out[(size_t)blockIdx.y * n + e] = r;
}

// out[j][e] = uniform mod q_{mod0+j} from words 2e, 2e+1 of stream
// (seed, tag, index_base | j); each thread draws four consecutive samples
// (one ChaCha20 block).  `base` carries the family, the call key and the
// tag; the limb's index goes into the nonce here.
__global__ void k_uniform(uint64_t* out, const ModConst* mc, uint32_t n, Stream base,
                          uint64_t seed, uint64_t tag, uint64_t index_base, uint32_t mod0) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x, j = blockIdx.y;
  const uint64_t q = mc[mod0 + j].q;
  uint64_t w[8];
  if (base.secure) {
    Stream s = base;
    s.nonce[1] = (uint32_t)(index_base | j);
    stream_block(s, t, w);
  } else {
    const uint64_t key = stream_key(seed, tag, index_base | j);
    for (int i = 0; i < 8; ++i) w[i] = draw(key, 8ull * t + i);
  }
  uint64_t* o = out + (size_t)j * n + 4ull * t;
  for (int i = 0; i < 4; ++i) o[i] = uniform_from(w[2 * i], w[2 * i + 1], q);
}

void launch_uniform(Context& c, uint64_t* out, uint32_t nlimb, uint64_t seed, uint64_t tag,
                    uint64_t index_base, uint32_t mod0) {
  const Stream base = make_stream(c.sampling, seed, tag, 0);
  const uint32_t quads = c.n / 4, tpb = quads < TPB ? quads : TPB;
  FHE_LAUNCH(c, "k_uniform", k_uniform, dim3(quads / tpb, nlimb), dim3(tpb), 0, out, c.d_const,
             c.n, base, seed, tag, index_base, mod0);
}

// b = e - a * s (+ f * s_old when f is given); all [nlimb][N], limb j uses
// modulus mod0 + j; f is a per-limb factor array (0 outside the digit).
__global__ void k_key_combine(uint64_t* b, const uint64_t* a, const uint64_t* s,
                              const uint64_t* e, const uint64_t* s_old, const uint64_t* f,
                              const ModConst* mc, uint32_t n, uint32_t mod0) {
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x, j = blockIdx.y;
  const ModConst m = mc[mod0 + j];
  const size_t o = (size_t)j * n + x;
  uint64_t v = sub_mod(e[o], mul_mod(a[o], s[o], m), m.q);
  if (f && f[j]) v = add_mod(v, mul_mod(f[j], s_old[o], m), m.q);
  b[o] = v;
}

// ct0 = b v + e0 + m, ct1 = a v + e1 over nq limbs.
__global__ void k_encrypt(uint64_t* ct, const uint64_t* pk, const uint64_t* v, const uint64_t* e0,
                          const uint64_t* e1, const uint64_t* msg, const ModConst* mc, uint32_t n,
                          uint32_t nq, uint32_t L) {
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
  const ModConst m = mc[i];
  const size_t o = (size_t)i * n + x;
  const uint64_t b = pk[o], a = pk[(size_t)L * n + o];
  ct[o] = add_mod(add_mod(mul_mod(b, v[o], m), e0[o], m.q), msg[o], m.q);
  ct[(size_t)nq * n + o] = add_mod(mul_mod(a, v[o], m), e1[o], m.q);
}

// m = sum_p ct_p s^p.
__global__ void k_decrypt(uint64_t* msg, const uint64_t* ct, const uint64_t* s, const ModConst* mc,
                          uint32_t n, uint32_t nq, uint32_t npoly) {
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
  const ModConst m = mc[i];
  const size_t o = (size_t)i * n + x;
  uint64_t acc = ct[o], sp = s[o];
  for (uint32_t p = 1; p < npoly; ++p) {
    acc = add_mod(acc, mul_mod(ct[(size_t)p * nq * n + o], sp, m), m.q);
    sp = mul_mod(sp, s[o], m);
  }
  msg[o] = acc;
}

__global__ void k_square(uint64_t* out, const uint64_t* a, const ModConst* mc, uint32_t n) {
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
  const size_t o = (size_t)i * n + x;
  out[o] = mul_mod(a[o], a[o], mc[i]);
}

void signed_small_to_eval(Context& c, const std::vector<int64_t>& coef, uint32_t idx0,
                          uint32_t nlimb, uint64_t* out) {
  Scratch d(c, c.n);
  hip_check(hipMemcpyAsync(d.p, coef.data(), c.n * 8, hipMemcpyHostToDevice, c.stream), "lift");
  FHE_LAUNCH(c, "k_lift_signed", k_lift_signed, dim3(c.n / tpb_for(c), nlimb), dim3(tpb_for(c)), 0, reinterpret_cast<const int64_t*>(d.p), out, c.d_const, c.n, idx0);
  ntt_forward(c, out, 1, 0, nlimb, LimbMap::contiguous(idx0));
  // coef is host memory read by an async copy: finish before it can go away
  hip_check(hipStreamSynchronize(c.stream), "lift sync");
}

}  // namespace

void sample_secret_host(Context& c, uint64_t seed, int64_t* out) {
  sample_ternary(make_stream(c.sampling, seed, TAG_SECRET, 0), out, c.n);
}
void sample_sparse_secret_host(Context& c, uint64_t seed, int64_t* out, uint32_t h) {
  sample_sparse_ternary(make_stream(c.sampling, seed, TAG_SECRET, 0), out, c.n, h);
}

void signed_to_eval(Context& c, const int64_t* coef_host, uint32_t idx0, uint32_t nlimb,
                    uint64_t* out) {
  std::vector<int64_t> v(coef_host, coef_host + c.n);
  signed_small_to_eval(c, v, idx0, nlimb, out);
}

void keygen_public(Context& c, const int64_t* s_coef, uint64_t seed, uint64_t* pk) {
  const size_t n = c.n;
  Scratch s(c, c.L * n), e(c, c.L * n);
  signed_to_eval(c, s_coef, 0, c.L, s.p);
  std::vector<int64_t> ec(n);
  sample_cbd(make_stream(c.sampling, seed, TAG_PK_E, 0), ec.data(), c.n);
  signed_small_to_eval(c, ec, 0, c.L, e.p);
  uint64_t* a = pk + (size_t)c.L * n;
  launch_uniform(c, a, c.L, seed, TAG_PK_A, 0, 0);
  FHE_LAUNCH(c, "k_key_combine", k_key_combine, dim3(c.n / tpb_for(c), c.L), dim3(tpb_for(c)), 0, pk, a, s.p, e.p, nullptr, nullptr, c.d_const, c.n, 0u);
  hip_check(hipStreamSynchronize(c.stream), "keygen sync");
}

void keygen_switch(Context& c, const uint64_t* s_old, const uint64_t* s_new, uint64_t seed,
                   uint64_t tag, uint64_t* key) {
  const size_t n = c.n;
  const uint32_t nm = c.L + c.K;
  Scratch e(c, nm * n), f(c, nm);
  std::vector<int64_t> ec(n);
  std::vector<uint64_t> pmod(nm);
  for (uint32_t i = 0; i < nm; ++i) {
    uint64_t pm = 1 % c.mods[i];
    for (uint32_t k = 0; k < c.K; ++k) pm = host_mulmod(pm, c.mods[c.L + k] % c.mods[i], c.mods[i]);
    pmod[i] = pm;
  }
  std::vector<uint64_t> fac(nm);
  for (uint32_t j = 0; j < c.dnum; ++j) {
    const uint32_t s = j * c.alpha, end = s + c.alpha < c.L ? s + c.alpha : c.L;
    sample_cbd(make_stream(c.sampling, seed, tag + TAG_KSK_E, j), ec.data(), c.n);
    signed_small_to_eval(c, ec, 0, nm, e.p);
    for (uint32_t i = 0; i < nm; ++i) fac[i] = (i >= s && i < end) ? pmod[i] : 0;
    hip_check(hipMemcpyAsync(f.p, fac.data(), nm * 8, hipMemcpyHostToDevice, c.stream), "fac");
    uint64_t* b = key + ((size_t)j * 2) * nm * n;
    uint64_t* a = b + (size_t)nm * n;
    launch_uniform(c, a, nm, seed, tag + TAG_KSK_A, (uint64_t)j << 16, 0);
    FHE_LAUNCH(c, "k_key_combine", k_key_combine, dim3(c.n / tpb_for(c), nm), dim3(tpb_for(c)), 0, b, a, s_new, e.p, s_old, f.p, c.d_const, c.n, 0u);
    hip_check(hipStreamSynchronize(c.stream), "keygen sync");
  }
}

void keygen_galois(Context& c, const int64_t* s_coef, uint32_t galois, uint64_t seed,
                   uint64_t* key) {
  const uint32_t nm = c.L + c.K;
  Scratch s(c, (size_t)nm * c.n), sp(c, (size_t)nm * c.n);
  signed_to_eval(c, s_coef, 0, nm, s.p);
  automorph(c, sp.p, s.p, 1, nm, galois_inverse(galois, c.n));
  keygen_switch(c, s.p, sp.p, seed, TAG_GALOIS + ((uint64_t)galois << 3), key);
}

void keygen_relin(Context& c, const int64_t* s_coef, uint64_t seed, uint64_t* key) {
  const uint32_t nm = c.L + c.K;
  Scratch s(c, (size_t)nm * c.n), s2(c, (size_t)nm * c.n);
  signed_to_eval(c, s_coef, 0, nm, s.p);
  FHE_LAUNCH(c, "k_square", k_square, dim3(c.n / tpb_for(c), nm), dim3(tpb_for(c)), 0, s2.p, s.p, c.d_const, c.n);
  keygen_switch(c, s2.p, s.p, seed, TAG_RELIN, key);
}

void encrypt_pk(Context& c, const uint64_t* pk, const uint64_t* m, uint32_t nq, uint64_t seed,
                uint64_t* ct) {
  const size_t n = c.n;
  Scratch v(c, nq * n), e0(c, nq * n), e1(c, nq * n);
  std::vector<int64_t> tmp(n);
  sample_ternary(make_stream(c.sampling, seed, TAG_ENC_V, 0), tmp.data(), c.n);
  signed_small_to_eval(c, tmp, 0, nq, v.p);
  sample_cbd(make_stream(c.sampling, seed, TAG_ENC_E, 0), tmp.data(), c.n);
  signed_small_to_eval(c, tmp, 0, nq, e0.p);
  sample_cbd(make_stream(c.sampling, seed, TAG_ENC_E, 1), tmp.data(), c.n);
  signed_small_to_eval(c, tmp, 0, nq, e1.p);
  FHE_LAUNCH(c, "k_encrypt", k_encrypt, dim3(c.n / tpb_for(c), nq), dim3(tpb_for(c)), 0, ct, pk, v.p, e0.p, e1.p, m, c.d_const, c.n, nq, c.L);
}

void decrypt(Context& c, const uint64_t* ct, uint32_t npoly, uint32_t nq, const int64_t* s_coef,
             uint64_t* m) {
  Scratch s(c, (size_t)nq * c.n);
  signed_to_eval(c, s_coef, 0, nq, s.p);
  FHE_LAUNCH(c, "k_decrypt", k_decrypt, dim3(c.n / tpb_for(c), nq), dim3(tpb_for(c)), 0, m, ct, s.p, c.d_const, c.n, nq, npoly);
}

}  // namespace fhe
