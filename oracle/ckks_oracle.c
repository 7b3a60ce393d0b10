/*
 * CKKS-RNS CPU oracle -- TEST INFRASTRUCTURE ONLY (see ckks_oracle.h).
 *
 * Scalar C restatement of the arithmetic OpenFHE 1.4.2 performs underneath
 * the fhemamba native executors.  Each function names the reference call
 * site it stands in for.  Nothing here is tuned beyond Shoup twiddles in the
 * transforms; clarity comes first.
 */
#define _GNU_SOURCE /* sincos */
#include "ckks_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

/* ======================================================================
 * Scalar modular arithmetic
 * ====================================================================== */
uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q) {
  return (uint64_t)(((u128)a * b) % q);
}

static inline uint64_t addmod(uint64_t a, uint64_t b, uint64_t q) {
  uint64_t s = a + b;
  return s >= q ? s - q : s;
}

static inline uint64_t submod(uint64_t a, uint64_t b, uint64_t q) {
  return a >= b ? a - b : a + q - b;
}

uint64_t orc_powmod(uint64_t a, uint64_t e, uint64_t q) {
  uint64_t r = 1 % q;
  a %= q;
  while (e) {
    if (e & 1) r = orc_mulmod(r, a, q);
    a = orc_mulmod(a, a, q);
    e >>= 1;
  }
  return r;
}

uint64_t orc_invmod(uint64_t a, uint64_t q) { return orc_powmod(a, q - 2, q); }

/* Shoup companion floor(w * 2^64 / q). */
static inline uint64_t shoup_pre(uint64_t w, uint64_t q) {
  return (uint64_t)(((u128)w << 64) / q);
}

static inline uint64_t shoup_mul(uint64_t a, uint64_t w, uint64_t wp,
                                 uint64_t q) {
  uint64_t qt = (uint64_t)(((u128)a * wp) >> 64);
  uint64_t r = a * w - qt * q;
  return r >= q ? r - q : r;
}

/* Deterministic Miller-Rabin for 64-bit integers (first 12 prime bases). */
int orc_is_prime(uint64_t n) {
  static const uint64_t bases[12] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return 0;
  for (int i = 0; i < 12; ++i) {
    if (n % bases[i] == 0) return n == bases[i];
  }
  uint64_t d = n - 1;
  int s = 0;
  while ((d & 1) == 0) {
    d >>= 1;
    ++s;
  }
  for (int i = 0; i < 12; ++i) {
    uint64_t x = orc_powmod(bases[i], d, n);
    if (x == 1 || x == n - 1) continue;
    int composite = 1;
    for (int r = 1; r < s; ++r) {
      x = orc_mulmod(x, x, n);
      if (x == n - 1) {
        composite = 0;
        break;
      }
    }
    if (composite) return 0;
  }
  return 1;
}

/* OpenFHE FirstPrime: the smallest prime >= 2^bits congruent to 1 mod m
 * (reference call: CCParams / GenCryptoContext,
 * native/fideslib_stage0/src/packed_fideslib.cpp:1060-1068). */
uint64_t orc_first_prime(uint32_t bits, uint64_t m) {
  uint64_t q = (uint64_t)1 << bits;
  uint64_t r = q % m;
  uint64_t c = q + 1 - r;
  if (r > 0) c += m;
  while (!orc_is_prime(c)) c += m;
  return c;
}

uint64_t orc_previous_prime(uint64_t q, uint64_t m) {
  uint64_t c = q - m;
  while (!orc_is_prime(c)) c -= m;
  return c;
}

uint64_t orc_next_prime(uint64_t q, uint64_t m) {
  uint64_t c = q + m;
  while (!orc_is_prime(c)) c += m;
  return c;
}

static int in_list(uint64_t v, const uint64_t *list, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i)
    if (list[i] == v) return 1;
  return 0;
}

int orc_num_special_primes(const uint64_t *q, uint32_t nq, uint32_t dnum,
                           uint32_t aux_bits) {
  if (dnum == 0 || nq == 0) return -1;
  uint32_t alpha = (nq + dnum - 1) / dnum;
  double maxbits = 0.0;
  for (uint32_t s = 0; s < nq; s += alpha) {
    double bits = 0.0;
    for (uint32_t i = s; i < s + alpha && i < nq; ++i) bits += log2((double)q[i]);
    if (bits > maxbits) maxbits = bits;
  }
  return (int)ceil(maxbits / (double)aux_bits);
}

/* FLEXIBLEAUTO prime chain: the last prime is FirstPrime(scale); going down
 * the chain the primes alternate below/above the running scaling factor
 * sf_{i} = sf_{i+1}^2 / q_{i+1}; q_0 = PreviousPrime(FirstPrime(first)).
 * HYBRID special primes descend from FirstPrime(60) skipping Q primes.
 * Pinned by the 57-prime golden chain (see header). */
int orc_gen_moduli(uint32_t log_n, uint32_t depth, uint32_t scale_bits,
                   uint32_t first_bits, uint32_t dnum, uint64_t *q_out,
                   uint64_t *p_out, uint32_t p_cap) {
  const uint64_t m = (uint64_t)2 << log_n;
  const uint32_t nq = depth + 1;
  memset(q_out, 0, sizeof(uint64_t) * nq);
  uint64_t q = orc_first_prime(scale_bits, m);
  q_out[nq - 1] = q;
  double sf = (double)q;
  uint32_t cnt = 0;
  for (int i = (int)nq - 2; i >= 1; --i, ++cnt) {
    sf = sf * sf / (double)q_out[i + 1];
    uint64_t sf_int = (uint64_t)llround(sf);
    uint64_t sf_rem = sf_int % m;
    uint64_t c;
    if (cnt % 2 == 0) {
      c = sf_int - m - sf_rem + 1;
      do {
        c = orc_previous_prime(c, m);
      } while (in_list(c, q_out + i + 1, nq - i - 1));
    } else {
      c = sf_int + m - sf_rem + 1;
      do {
        c = orc_next_prime(c, m);
      } while (in_list(c, q_out + i + 1, nq - i - 1));
    }
    q_out[i] = c;
  }
  q_out[0] = orc_previous_prime(orc_first_prime(first_bits, m), m);
  int k = orc_num_special_primes(q_out, nq, dnum, 60);
  if (k < 0 || (uint32_t)k > p_cap) return -1;
  uint64_t p = orc_first_prime(60, m);
  for (int j = 0; j < k;) {
    p = orc_previous_prime(p, m);
    if (in_list(p, q_out, nq)) continue;
    p_out[j++] = p;
  }
  return k;
}

/* OpenFHE RootOfUnity returns the smallest primitive m-th root of unity. */
uint64_t orc_root_of_unity(uint64_t m, uint64_t q) {
  uint64_t root = 0;
  for (uint64_t g = 2; g < q; ++g) {
    uint64_t r = orc_powmod(g, (q - 1) / m, q);
    if (orc_powmod(r, m / 2, q) == q - 1) {
      root = r;
      break;
    }
  }
  /* Walk the odd powers root^(2t+1); all primitive roots appear. */
  uint64_t r2 = orc_mulmod(root, root, q);
  uint64_t x = root, best = root;
  for (uint64_t t = 1; t < m / 2; ++t) {
    x = orc_mulmod(x, r2, q);
    if (x < best) best = x;
  }
  return best;
}

/* ======================================================================
 * Negacyclic NTT (bit-reversed evaluation order at psi^(2 brv(i) + 1))
 * ====================================================================== */
static uint32_t bitrev(uint32_t x, uint32_t bits) {
  uint32_t r = 0;
  for (uint32_t i = 0; i < bits; ++i) {
    r = (r << 1) | (x & 1);
    x >>= 1;
  }
  return r;
}

static uint32_t ilog2(uint32_t n) {
  uint32_t l = 0;
  while ((1u << l) < n) ++l;
  return l;
}

typedef struct {
  uint64_t q, psi, ninv, ninv_sh;
  uint64_t *fw, *fw_sh, *iw, *iw_sh; /* psi^brv(k), psi^-brv(k) + Shoup */
} ntt_tab;

static void ntt_tab_init(ntt_tab *t, uint32_t n, uint64_t q, uint64_t psi) {
  uint32_t logn = ilog2(n);
  t->q = q;
  t->psi = psi;
  t->fw = malloc(sizeof(uint64_t) * n);
  t->fw_sh = malloc(sizeof(uint64_t) * n);
  t->iw = malloc(sizeof(uint64_t) * n);
  t->iw_sh = malloc(sizeof(uint64_t) * n);
  uint64_t psi_inv = orc_invmod(psi, q);
  uint64_t *pw = malloc(sizeof(uint64_t) * n), *ipw = malloc(sizeof(uint64_t) * n);
  pw[0] = 1;
  ipw[0] = 1;
  for (uint32_t i = 1; i < n; ++i) {
    pw[i] = orc_mulmod(pw[i - 1], psi, q);
    ipw[i] = orc_mulmod(ipw[i - 1], psi_inv, q);
  }
  for (uint32_t k = 0; k < n; ++k) {
    uint32_t r = bitrev(k, logn);
    t->fw[k] = pw[r];
    t->iw[k] = ipw[r];
    t->fw_sh[k] = shoup_pre(t->fw[k], q);
    t->iw_sh[k] = shoup_pre(t->iw[k], q);
  }
  free(pw);
  free(ipw);
  t->ninv = orc_invmod(n % q, q);
  t->ninv_sh = shoup_pre(t->ninv, q);
}

static void ntt_tab_free(ntt_tab *t) {
  free(t->fw);
  free(t->fw_sh);
  free(t->iw);
  free(t->iw_sh);
}

/* Cooley-Tukey, OpenFHE ForwardTransformToBitReverseInPlace order. */
static void ntt_fwd_tab(uint64_t *a, uint32_t n, const ntt_tab *t) {
  const uint64_t q = t->q;
  for (uint32_t m = 1, h = n >> 1; m < n; m <<= 1, h >>= 1) {
    for (uint32_t i = 0; i < m; ++i) {
      const uint64_t w = t->fw[m + i], wp = t->fw_sh[m + i];
      uint64_t *x = a + 2 * i * h, *y = x + h;
      for (uint32_t j = 0; j < h; ++j) {
        uint64_t u = x[j], v = shoup_mul(y[j], w, wp, q);
        x[j] = addmod(u, v, q);
        y[j] = submod(u, v, q);
      }
    }
  }
}

/* Gentleman-Sande inverse, then scale by N^-1. */
static void ntt_inv_tab(uint64_t *a, uint32_t n, const ntt_tab *t) {
  const uint64_t q = t->q;
  for (uint32_t m = n >> 1, h = 1; m >= 1; m >>= 1, h <<= 1) {
    for (uint32_t i = 0; i < m; ++i) {
      const uint64_t w = t->iw[m + i], wp = t->iw_sh[m + i];
      uint64_t *x = a + 2 * i * h, *y = x + h;
      for (uint32_t j = 0; j < h; ++j) {
        uint64_t u = x[j], v = y[j];
        x[j] = addmod(u, v, q);
        y[j] = shoup_mul(submod(u, v, q), w, wp, q);
      }
    }
  }
  for (uint32_t j = 0; j < n; ++j) a[j] = shoup_mul(a[j], t->ninv, t->ninv_sh, q);
}

void orc_ntt_fwd(uint64_t *a, uint32_t n, uint64_t q, uint64_t psi) {
  ntt_tab t;
  ntt_tab_init(&t, n, q, psi);
  ntt_fwd_tab(a, n, &t);
  ntt_tab_free(&t);
}

void orc_ntt_inv(uint64_t *a, uint32_t n, uint64_t q, uint64_t psi) {
  ntt_tab t;
  ntt_tab_init(&t, n, q, psi);
  ntt_inv_tab(a, n, &t);
  ntt_tab_free(&t);
}

void orc_ntt_naive(const uint64_t *a, uint64_t *out, uint32_t n, uint64_t q,
                   uint64_t psi) {
  uint32_t logn = ilog2(n);
  for (uint32_t i = 0; i < n; ++i) {
    uint64_t e = 2 * (uint64_t)bitrev(i, logn) + 1;
    uint64_t x = orc_powmod(psi, e, q), xp = 1, acc = 0;
    for (uint32_t j = 0; j < n; ++j) {
      acc = addmod(acc, orc_mulmod(a[j], xp, q), q);
      xp = orc_mulmod(xp, x, q);
    }
    out[i] = acc;
  }
}

void orc_negacyclic_schoolbook(const uint64_t *a, const uint64_t *b,
                               uint64_t *out, uint32_t n, uint64_t q) {
  memset(out, 0, sizeof(uint64_t) * n);
  for (uint32_t i = 0; i < n; ++i)
    for (uint32_t j = 0; j < n; ++j) {
      uint64_t p = orc_mulmod(a[i], b[j], q);
      uint32_t k = i + j;
      if (k < n)
        out[k] = addmod(out[k], p, q);
      else
        out[k - n] = submod(out[k - n], p, q);
    }
}

/* ======================================================================
 * Automorphisms X -> X^k
 * ====================================================================== */
/* Evaluation-form permutation, OpenFHE PrecomputeAutoMap semantics:
 * out[brv(j)] = in[brv(((2j+1)k mod 2N - 1)/2)]. */
void orc_automorph_ntt(const uint64_t *in, uint64_t *out, uint32_t n,
                       uint32_t k) {
  uint32_t logn = ilog2(n);
  uint64_t m = 2 * (uint64_t)n;
  for (uint32_t j = 0; j < n; ++j) {
    uint64_t e = ((2 * (uint64_t)j + 1) * k) % m;
    out[bitrev(j, logn)] = in[bitrev((uint32_t)((e - 1) / 2), logn)];
  }
}

void orc_automorph_coeff(const uint64_t *in, uint64_t *out, uint32_t n,
                         uint32_t k, uint64_t q) {
  uint64_t m = 2 * (uint64_t)n;
  for (uint32_t j = 0; j < n; ++j) {
    uint64_t e = ((uint64_t)j * k) % m;
    if (e < n)
      out[e] = in[j];
    else
      out[e - n] = in[j] ? q - in[j] : 0;
  }
}

/* Rotation by `step` slots uses the Galois element 5^step mod 2N (OpenFHE
 * FindAutomorphismIndex2nComplex; negative steps use 5^-1). */
uint32_t orc_galois_elt(int32_t step, uint32_t n) {
  int64_t order = n / 2; /* multiplicative order of 5 mod 2N */
  int64_t r = ((int64_t)step % order + order) % order;
  return (uint32_t)orc_powmod(5, (uint64_t)r, 2 * (uint64_t)n);
}

/* ======================================================================
 * Fast (approximate, uncorrected) basis conversion, OpenFHE
 * ApproxSwitchCRTBasis semantics:
 *   v_i = [x_i * (Qhat_i)^-1]_{q_i},  y_k = [sum_i v_i * Qhat_i]_{m_k}
 * ====================================================================== */
void orc_switch_basis(const uint64_t *x, const uint64_t *from_q,
                      uint32_t nfrom, uint64_t *y, const uint64_t *to_q,
                      uint32_t nto, uint32_t n) {
  uint64_t *qhat_inv = malloc(sizeof(uint64_t) * nfrom);
  uint64_t *qhat_mod = malloc(sizeof(uint64_t) * nfrom * nto);
  for (uint32_t i = 0; i < nfrom; ++i) {
    uint64_t h = 1;
    for (uint32_t j = 0; j < nfrom; ++j)
      if (j != i) h = orc_mulmod(h, from_q[j] % from_q[i], from_q[i]);
    qhat_inv[i] = orc_invmod(h, from_q[i]);
    for (uint32_t k = 0; k < nto; ++k) {
      uint64_t hk = 1;
      for (uint32_t j = 0; j < nfrom; ++j)
        if (j != i) hk = orc_mulmod(hk, from_q[j] % to_q[k], to_q[k]);
      qhat_mod[i * nto + k] = hk;
    }
  }
  uint64_t *v = malloc(sizeof(uint64_t) * nfrom);
  for (uint32_t c = 0; c < n; ++c) {
    for (uint32_t i = 0; i < nfrom; ++i)
      v[i] = orc_mulmod(x[(size_t)i * n + c], qhat_inv[i], from_q[i]);
    for (uint32_t k = 0; k < nto; ++k) {
      u128 acc = 0;
      for (uint32_t i = 0; i < nfrom; ++i) acc += (u128)v[i] * qhat_mod[i * nto + k];
      y[(size_t)k * n + c] = (uint64_t)(acc % to_q[k]);
    }
  }
  free(v);
  free(qhat_inv);
  free(qhat_mod);
}

/* ======================================================================
 * Context
 * ====================================================================== */
struct orc_ctx {
  uint32_t log_n, n, L, K, dnum, alpha;
  uint64_t *mods; /* q_0..q_{L-1}, p_0..p_{K-1} */
  ntt_tab *tabs;
};

orc_ctx *orc_ctx_create(uint32_t log_n, const uint64_t *q, uint32_t L,
                        const uint64_t *p, uint32_t K, uint32_t dnum) {
  orc_ctx *c = calloc(1, sizeof(orc_ctx));
  c->log_n = log_n;
  c->n = 1u << log_n;
  c->L = L;
  c->K = K;
  c->alpha = (L + dnum - 1) / dnum;
  c->dnum = (L + c->alpha - 1) / c->alpha; /* digits that are non-empty */
  c->mods = malloc(sizeof(uint64_t) * (L + K));
  memcpy(c->mods, q, sizeof(uint64_t) * L);
  if (K) memcpy(c->mods + L, p, sizeof(uint64_t) * K);
  c->tabs = calloc(L + K, sizeof(ntt_tab));
  for (uint32_t i = 0; i < L + K; ++i) {
    uint64_t psi = orc_root_of_unity(2 * (uint64_t)c->n, c->mods[i]);
    ntt_tab_init(&c->tabs[i], c->n, c->mods[i], psi);
  }
  return c;
}

void orc_ctx_destroy(orc_ctx *c) {
  if (!c) return;
  for (uint32_t i = 0; i < c->L + c->K; ++i) ntt_tab_free(&c->tabs[i]);
  free(c->tabs);
  free(c->mods);
  free(c);
}

uint64_t orc_ctx_psi(const orc_ctx *c, uint32_t mod_idx) {
  return c->tabs[mod_idx].psi;
}

void orc_ctx_ntt_fwd(const orc_ctx *c, uint64_t *a, uint32_t mod_idx) {
  ntt_fwd_tab(a, c->n, &c->tabs[mod_idx]);
}

void orc_ctx_ntt_inv(const orc_ctx *c, uint64_t *a, uint32_t mod_idx) {
  ntt_inv_tab(a, c->n, &c->tabs[mod_idx]);
}

void orc_ntt_fwd_batch(const orc_ctx *c, uint64_t *data, uint32_t npoly,
                       uint32_t limb0, uint32_t nlimb, int nthreads) {
  long total = (long)npoly * nlimb;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(dynamic, 1)
  for (long t = 0; t < total; ++t) {
    uint32_t j = (uint32_t)(t % nlimb);
    ntt_fwd_tab(data + (size_t)t * c->n, c->n, &c->tabs[limb0 + j]);
  }
}

void orc_ntt_inv_batch(const orc_ctx *c, uint64_t *data, uint32_t npoly,
                       uint32_t limb0, uint32_t nlimb, int nthreads) {
  long total = (long)npoly * nlimb;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(dynamic, 1)
  for (long t = 0; t < total; ++t) {
    uint32_t j = (uint32_t)(t % nlimb);
    ntt_inv_tab(data + (size_t)t * c->n, c->n, &c->tabs[limb0 + j]);
  }
}

void orc_mac_batch(const orc_ctx *c, const uint64_t *x, const uint64_t *w,
                   uint32_t ncts, uint32_t nq, uint64_t *acc, int nthreads) {
  const size_t n = c->n;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
  for (long t = 0; t < 2L * nq; ++t) {
    uint32_t poly = (uint32_t)(t / nq), l = (uint32_t)(t % nq);
    uint64_t q = c->mods[l];
    uint64_t *out = acc + (size_t)t * n;
    for (size_t e = 0; e < n; ++e) {
      u128 s = 0;
      for (uint32_t i = 0; i < ncts; ++i) {
        const uint64_t xv = x[(((size_t)i * 2 + poly) * nq + l) * n + e];
        const uint64_t wv = w[((size_t)i * nq + l) * n + e];
        s += (u128)xv * wv;
        if ((i & 31) == 31) s %= q; /* keep the 128-bit sum from overflowing */
      }
      out[e] = (uint64_t)(s % q);
    }
  }
}

/* EvalAdd on matching limbs (OpenFHE DCRTPoly operator+, per limb
 * (a + b) mod q_l): out = a + b over npoly polys of nq limbs each. */
void orc_add(const orc_ctx *c, const uint64_t *a, const uint64_t *b, uint32_t npoly,
             uint32_t nq, uint64_t *out) {
  const size_t n = c->n;
  for (size_t t = 0; t < (size_t)npoly * nq; ++t) {
    const uint64_t q = c->mods[t % nq];
    for (size_t e = 0; e < n; ++e) {
      const uint64_t s = a[t * n + e] + b[t * n + e];
      out[t * n + e] = s >= q ? s - q : s;
    }
  }
}

/* ======================================================================
 * Hybrid key switching (OpenFHE KeySwitchHYBRID: EvalKeySwitchPrecomputeCore,
 * EvalFastKeySwitchCoreExt, ApproxModDown)
 * ====================================================================== */
uint32_t orc_num_digits(const orc_ctx *c, uint32_t nq) {
  uint32_t d = (nq + c->alpha - 1) / c->alpha;
  return d < c->dnum ? d : c->dnum;
}

void orc_modup(const orc_ctx *c, const uint64_t *a, uint32_t nq,
               uint64_t *digits) {
  const uint32_t n = c->n, K = c->K, L = c->L, ext = nq + K;
  const uint32_t nd = orc_num_digits(c, nq);
  for (uint32_t j = 0; j < nd; ++j) {
    uint32_t s = j * c->alpha, e = s + c->alpha < nq ? s + c->alpha : nq;
    uint32_t sz = e - s, nto = ext - sz;
    uint64_t *tmp = malloc(sizeof(uint64_t) * sz * n);
    memcpy(tmp, a + (size_t)s * n, sizeof(uint64_t) * sz * n);
    for (uint32_t i = 0; i < sz; ++i) orc_ctx_ntt_inv(c, tmp + (size_t)i * n, s + i);
    uint64_t *to_q = malloc(sizeof(uint64_t) * nto);
    uint32_t *to_idx = malloc(sizeof(uint32_t) * nto);
    uint32_t t = 0;
    for (uint32_t i = 0; i < nq; ++i)
      if (i < s || i >= e) {
        to_idx[t] = i;
        to_q[t++] = c->mods[i];
      }
    for (uint32_t k = 0; k < K; ++k) {
      to_idx[t] = L + k;
      to_q[t++] = c->mods[L + k];
    }
    uint64_t *conv = malloc(sizeof(uint64_t) * nto * n);
    orc_switch_basis(tmp, c->mods + s, sz, conv, to_q, nto, n);
    for (uint32_t k = 0; k < nto; ++k) orc_ctx_ntt_fwd(c, conv + (size_t)k * n, to_idx[k]);
    uint64_t *dj = digits + (size_t)j * ext * n;
    t = 0;
    for (uint32_t i = 0; i < nq; ++i) {
      const uint64_t *src = (i >= s && i < e) ? a + (size_t)i * n : conv + (size_t)(t++) * n;
      memcpy(dj + (size_t)i * n, src, sizeof(uint64_t) * n);
    }
    for (uint32_t k = 0; k < K; ++k)
      memcpy(dj + (size_t)(nq + k) * n, conv + (size_t)(t++) * n, sizeof(uint64_t) * n);
    free(tmp);
    free(to_q);
    free(to_idx);
    free(conv);
  }
}

void orc_ksk_inner(const orc_ctx *c, const uint64_t *digits, uint32_t nq,
                   const uint64_t *key, uint64_t *ext) {
  const uint32_t n = c->n, K = c->K, L = c->L, ne = nq + K;
  const uint32_t nd = orc_num_digits(c, nq);
  for (uint32_t b = 0; b < 2; ++b)
    for (uint32_t i = 0; i < ne; ++i) {
      uint32_t ki = i < nq ? i : L + (i - nq);
      uint64_t q = c->mods[ki];
      uint64_t *out = ext + ((size_t)b * ne + i) * n;
      for (uint32_t e = 0; e < n; ++e) {
        uint64_t acc = 0;
        for (uint32_t j = 0; j < nd; ++j) {
          uint64_t d = digits[((size_t)j * ne + i) * n + e];
          uint64_t k = key[(((size_t)j * 2 + b) * (L + K) + ki) * n + e];
          acc = addmod(acc, orc_mulmod(d, k, q), q);
        }
        out[e] = acc;
      }
    }
}

void orc_moddown(const orc_ctx *c, const uint64_t *ext, uint32_t nq,
                 uint64_t *out) {
  const uint32_t n = c->n, K = c->K, L = c->L;
  uint64_t *pp = malloc(sizeof(uint64_t) * K * n);
  memcpy(pp, ext + (size_t)nq * n, sizeof(uint64_t) * K * n);
  for (uint32_t k = 0; k < K; ++k) orc_ctx_ntt_inv(c, pp + (size_t)k * n, L + k);
  uint64_t *conv = malloc(sizeof(uint64_t) * nq * n);
  orc_switch_basis(pp, c->mods + L, K, conv, c->mods, nq, n);
  for (uint32_t i = 0; i < nq; ++i) {
    uint64_t q = c->mods[i];
    orc_ctx_ntt_fwd(c, conv + (size_t)i * n, i);
    uint64_t pmod = 1;
    for (uint32_t k = 0; k < K; ++k) pmod = orc_mulmod(pmod, c->mods[L + k] % q, q);
    uint64_t pinv = orc_invmod(pmod, q);
    for (uint32_t e = 0; e < n; ++e) {
      uint64_t d = submod(ext[(size_t)i * n + e], conv[(size_t)i * n + e], q);
      out[(size_t)i * n + e] = orc_mulmod(d, pinv, q);
    }
  }
  free(pp);
  free(conv);
}

void orc_keyswitch(const orc_ctx *c, const uint64_t *a, uint32_t nq,
                   const uint64_t *key, uint64_t *out) {
  const uint32_t n = c->n, ne = nq + c->K, nd = orc_num_digits(c, nq);
  uint64_t *digits = malloc(sizeof(uint64_t) * nd * ne * n);
  uint64_t *ext = malloc(sizeof(uint64_t) * 2 * ne * n);
  orc_modup(c, a, nq, digits);
  orc_ksk_inner(c, digits, nq, key, ext);
  orc_moddown(c, ext, nq, out);
  orc_moddown(c, ext + (size_t)ne * n, nq, out + (size_t)nq * n);
  free(digits);
  free(ext);
}

/* OpenFHE EvalAutomorphism order: key switch c1, add c0, then permute both
 * polys (stage1 EvalRotate, stage1_mamba2_decode_fideslib.cpp:1779-1801). */
void orc_rotate(const orc_ctx *c, const uint64_t *ct, uint32_t nq,
                const uint64_t *key, uint32_t galois, uint64_t *out) {
  const uint32_t n = c->n;
  uint64_t *ks = malloc(sizeof(uint64_t) * 2 * nq * n);
  orc_keyswitch(c, ct + (size_t)nq * n, nq, key, ks);
  for (uint32_t i = 0; i < nq; ++i) {
    uint64_t q = c->mods[i];
    for (uint32_t e = 0; e < n; ++e)
      ks[(size_t)i * n + e] = addmod(ks[(size_t)i * n + e], ct[(size_t)i * n + e], q);
  }
  for (uint32_t p = 0; p < 2; ++p)
    for (uint32_t i = 0; i < nq; ++i)
      orc_automorph_ntt(ks + ((size_t)p * nq + i) * n, out + ((size_t)p * nq + i) * n, n,
                        galois);
  free(ks);
}

/* EvalFastRotation with a shared precompute (src/fideslib_rotation_batch.hpp:
 * 17-18): digits = ModUp(c1) computed once (orc_modup); per rotation the key
 * inner product, ModDown, + c0 and the permutation, as orc_rotate. */
void orc_rotate_hoisted(const orc_ctx *c, const uint64_t *ct, uint32_t nq,
                        const uint64_t *digits, const uint64_t *key, uint32_t galois,
                        uint64_t *out) {
  const uint32_t n = c->n, ne = nq + c->K;
  uint64_t *ext = malloc(sizeof(uint64_t) * 2 * ne * n);
  uint64_t *ks = malloc(sizeof(uint64_t) * 2 * nq * n);
  orc_ksk_inner(c, digits, nq, key, ext);
  orc_moddown(c, ext, nq, ks);
  orc_moddown(c, ext + (size_t)ne * n, nq, ks + (size_t)nq * n);
  for (uint32_t i = 0; i < nq; ++i) {
    uint64_t q = c->mods[i];
    for (uint32_t e = 0; e < n; ++e)
      ks[(size_t)i * n + e] = addmod(ks[(size_t)i * n + e], ct[(size_t)i * n + e], q);
  }
  for (uint32_t p = 0; p < 2; ++p)
    for (uint32_t i = 0; i < nq; ++i)
      orc_automorph_ntt(ks + ((size_t)p * nq + i) * n, out + ((size_t)p * nq + i) * n, n,
                        galois);
  free(ext);
  free(ks);
}

/* OpenFHE DropLastElementAndScale: y_i = (x_i - [lift(x_l)]_{q_i}) q_l^-1,
 * lift centred on (q_l >> 1). */
void orc_rescale(const orc_ctx *c, const uint64_t *in, uint32_t npoly,
                 uint32_t nq, uint64_t *out) {
  const uint32_t n = c->n, l = nq - 1;
  const uint64_t ql = c->mods[l];
  uint64_t *last = malloc(sizeof(uint64_t) * n), *t = malloc(sizeof(uint64_t) * n);
  for (uint32_t p = 0; p < npoly; ++p) {
    memcpy(last, in + ((size_t)p * nq + l) * n, sizeof(uint64_t) * n);
    orc_ctx_ntt_inv(c, last, l);
    for (uint32_t i = 0; i < l; ++i) {
      uint64_t q = c->mods[i];
      for (uint32_t e = 0; e < n; ++e) {
        uint64_t v = last[e];
        t[e] = v > (ql >> 1) ? submod(v % q, ql % q, q) : v % q;
      }
      orc_ctx_ntt_fwd(c, t, i);
      uint64_t inv = orc_invmod(ql % q, q);
      const uint64_t *x = in + ((size_t)p * nq + i) * n;
      uint64_t *y = out + ((size_t)p * l + i) * n;
      for (uint32_t e = 0; e < n; ++e) y[e] = orc_mulmod(submod(x[e], t[e], q), inv, q);
    }
  }
  free(last);
  free(t);
}

void orc_tensor(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
                uint32_t nq, uint64_t *out) {
  const size_t n = c->n, pl = nq * n;
  for (uint32_t i = 0; i < nq; ++i) {
    uint64_t q = c->mods[i];
    for (size_t e = 0; e < n; ++e) {
      size_t o = i * n + e;
      uint64_t a0 = a[o], a1 = a[pl + o], b0 = b[o], b1 = b[pl + o];
      out[o] = orc_mulmod(a0, b0, q);
      out[pl + o] = addmod(orc_mulmod(a0, b1, q), orc_mulmod(a1, b0, q), q);
      out[2 * pl + o] = orc_mulmod(a1, b1, q);
    }
  }
}

void orc_relinearize(const orc_ctx *c, const uint64_t *ct3, uint32_t nq,
                     const uint64_t *key, uint64_t *out) {
  const size_t n = c->n, pl = nq * n;
  uint64_t *ks = malloc(sizeof(uint64_t) * 2 * pl);
  orc_keyswitch(c, ct3 + 2 * pl, nq, key, ks);
  for (uint32_t p = 0; p < 2; ++p)
    for (uint32_t i = 0; i < nq; ++i) {
      uint64_t q = c->mods[i];
      for (size_t e = 0; e < n; ++e) {
        size_t o = p * pl + i * n + e;
        out[o] = addmod(ct3[o], ks[o], q);
      }
    }
  free(ks);
}

/* ======================================================================
 * Sampling streams.  The definition is shared with the HIP library's key
 * generation so that both produce identical keys.  Sample word i of the
 * stream named (seed, tag, index) comes from one of two families:
 *   seeded (the default here; parity only, not secure):
 *     key    = fmix64(seed ^ fmix64((tag << 32) ^ index ^ 0x5851F42D4C957F2D))
 *     word i = fmix64(key + (i + 1) * 0x9E3779B97F4A7C15)        (SplitMix64)
 *   ChaCha20 (RFC 8439) under a 256-bit master key (orc_set_sampling_key):
 *     K1     = ChaCha20Block(master, 0, nonce (lo32 seed, hi32 seed, 0))[0..7]
 *     word i = 64-bit little-endian word i of the keystream under K1 with
 *              nonce (tag, index, 1), block counter i / 8
 * Samples from words:
 *   uniform mod q = floor((word(2i) * 2^64 + word(2i+1)) * q / 2^128)
 *   ternary       = {0, 1, -1}[word(i) mod 3]
 *   sparse ternary (Hamming weight h): for i < h swap position i with
 *                   i + floor(word(2i) (n - i) / 2^64) of 0..n-1 (partial
 *                   Fisher-Yates), that position gets (word(2i+1) & 1) ? -1 : 1
 *   error         = centred binomial, eta = 21 (sigma ~ 3.24)
 * ====================================================================== */
static inline uint64_t fmix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t orc_draw(uint64_t key, uint64_t ctr) {
  return fmix64(key + (ctr + 1) * 0x9E3779B97F4A7C15ull);
}

uint64_t orc_stream_key(uint64_t seed, uint64_t tag, uint64_t index) {
  return fmix64(seed ^ fmix64((tag << 32) ^ index ^ 0x5851F42D4C957F2Dull));
}

static inline uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

/* RFC 8439 section 2.3, written from the RFC's quarter-round definition. */
void orc_chacha20_block(const uint32_t key[8], uint32_t counter, const uint32_t nonce[3],
                        uint32_t out[16]) {
  uint32_t st[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                     key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                     counter, nonce[0], nonce[1], nonce[2]};
  uint32_t x[16];
  static const int qr[8][4] = {{0, 4, 8, 12}, {1, 5, 9, 13}, {2, 6, 10, 14}, {3, 7, 11, 15},
                               {0, 5, 10, 15}, {1, 6, 11, 12}, {2, 7, 8, 13}, {3, 4, 9, 14}};
  memcpy(x, st, sizeof(x));
  for (int r = 0; r < 10; ++r)
    for (int k = 0; k < 8; ++k) {
      uint32_t *a = &x[qr[k][0]], *b = &x[qr[k][1]], *c = &x[qr[k][2]], *d = &x[qr[k][3]];
      *a += *b; *d ^= *a; *d = rotl32(*d, 16);
      *c += *d; *b ^= *c; *b = rotl32(*b, 12);
      *a += *b; *d ^= *a; *d = rotl32(*d, 8);
      *c += *d; *b ^= *c; *b = rotl32(*b, 7);
    }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + st[i];
}

static int g_secure = 0;
static uint32_t g_master[8];

void orc_set_sampling_key(const uint8_t *key32) {
  g_secure = key32 != NULL;
  for (int i = 0; key32 && i < 8; ++i)
    g_master[i] = (uint32_t)key32[4 * i] | ((uint32_t)key32[4 * i + 1] << 8) |
                  ((uint32_t)key32[4 * i + 2] << 16) | ((uint32_t)key32[4 * i + 3] << 24);
}

typedef struct {
  int secure;
  uint32_t key[8], nonce[3];
  uint64_t sm, cached, buf[8];
} orc_stream;

static orc_stream stream_open(uint64_t seed, uint64_t tag, uint64_t index) {
  orc_stream s;
  memset(&s, 0, sizeof(s));
  s.secure = g_secure;
  s.cached = ~0ull;
  if (!g_secure) {
    s.sm = orc_stream_key(seed, tag, index);
    return s;
  }
  uint32_t n0[3] = {(uint32_t)seed, (uint32_t)(seed >> 32), 0u}, blk[16];
  orc_chacha20_block(g_master, 0u, n0, blk);
  memcpy(s.key, blk, sizeof(s.key));
  s.nonce[0] = (uint32_t)tag;
  s.nonce[1] = (uint32_t)index;
  s.nonce[2] = 1u;
  return s;
}

static uint64_t stream_word(orc_stream *s, uint64_t i) {
  if (!s->secure) return orc_draw(s->sm, i);
  if (s->cached != i / 8) {
    uint32_t o[16];
    orc_chacha20_block(s->key, (uint32_t)(i / 8), s->nonce, o);
    for (int k = 0; k < 8; ++k) s->buf[k] = (uint64_t)o[2 * k] | ((uint64_t)o[2 * k + 1] << 32);
    s->cached = i / 8;
  }
  return s->buf[i % 8];
}

static orc_stream seeded_stream(uint64_t key) {
  orc_stream s;
  memset(&s, 0, sizeof(s));
  s.sm = key;
  return s;
}

static void sample_uniform(orc_stream *st, uint64_t q, uint64_t *out, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) {
    uint64_t hi = stream_word(st, 2 * (uint64_t)i), lo = stream_word(st, 2 * (uint64_t)i + 1);
    u128 t = (u128)hi * q + (uint64_t)(((u128)lo * q) >> 64);
    out[i] = (uint64_t)(t >> 64);
  }
}

static void sample_ternary(orc_stream *st, int64_t *out, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) {
    uint64_t d = stream_word(st, i) % 3;
    out[i] = d == 0 ? 0 : (d == 1 ? 1 : -1);
  }
}

static void sample_sparse_ternary(orc_stream *st, int64_t *out, uint32_t n, uint32_t h) {
  uint32_t *idx = malloc(sizeof(uint32_t) * n);
  for (uint32_t i = 0; i < n; ++i) {
    idx[i] = i;
    out[i] = 0;
  }
  for (uint32_t i = 0; i < h && i < n; ++i) {
    uint32_t j = i + (uint32_t)(((u128)stream_word(st, 2 * (uint64_t)i) * (n - i)) >> 64);
    uint32_t t = idx[i];
    idx[i] = idx[j];
    idx[j] = t;
    out[idx[i]] = (stream_word(st, 2 * (uint64_t)i + 1) & 1) ? -1 : 1;
  }
  free(idx);
}

static void sample_cbd(orc_stream *st, int64_t *out, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) {
    uint64_t d = stream_word(st, i);
    out[i] = (int64_t)__builtin_popcountll(d & 0x1FFFFFull) -
             (int64_t)__builtin_popcountll((d >> 21) & 0x1FFFFFull);
  }
}

/* Seeded-family samplers on an explicit SplitMix64 stream key. */
void orc_sample_uniform(uint64_t key, uint64_t q, uint64_t *out, uint32_t n) {
  orc_stream s = seeded_stream(key);
  sample_uniform(&s, q, out, n);
}

void orc_sample_ternary(uint64_t key, int64_t *out, uint32_t n) {
  orc_stream s = seeded_stream(key);
  sample_ternary(&s, out, n);
}

void orc_sample_sparse_ternary(uint64_t key, int64_t *out, uint32_t n, uint32_t h) {
  orc_stream s = seeded_stream(key);
  sample_sparse_ternary(&s, out, n, h);
}

void orc_sample_cbd(uint64_t key, int64_t *out, uint32_t n) {
  orc_stream s = seeded_stream(key);
  sample_cbd(&s, out, n);
}

/* Word i of stream (seed, tag, index) of the current family. */
uint64_t orc_stream_word(uint64_t seed, uint64_t tag, uint64_t index, uint64_t i) {
  orc_stream s = stream_open(seed, tag, index);
  return stream_word(&s, i);
}

enum {
  TAG_SECRET = 1,
  TAG_PK_A = 2,
  TAG_PK_E = 3,
  TAG_ENC_V = 4,
  TAG_ENC_E = 5,
  TAG_KSK_A = 6,
  TAG_KSK_E = 7,
  TAG_RELIN = 0x100000,
  TAG_GALOIS = 0x200000
};

void orc_signed_to_eval(const orc_ctx *c, const int64_t *coef, uint32_t idx0,
                        uint32_t nlimb, uint64_t *out) {
  const uint32_t n = c->n;
  for (uint32_t j = 0; j < nlimb; ++j) {
    uint64_t q = c->mods[idx0 + j];
    uint64_t *o = out + (size_t)j * n;
    for (uint32_t e = 0; e < n; ++e) {
      int64_t v = coef[e];
      o[e] = v >= 0 ? (uint64_t)v % q : (q - ((uint64_t)(-v) % q)) % q;
    }
    orc_ctx_ntt_fwd(c, o, idx0 + j);
  }
}

void orc_keygen_secret(uint64_t seed, uint32_t n, int64_t *s_coef) {
  {
    orc_stream st = stream_open(seed, TAG_SECRET, 0);
    sample_ternary(&st, s_coef, n);
  }
}

void orc_keygen_secret_sparse(uint64_t seed, uint32_t n, uint32_t h, int64_t *s_coef) {
  {
    orc_stream st = stream_open(seed, TAG_SECRET, 0);
    sample_sparse_ternary(&st, s_coef, n, h);
  }
}

void orc_keygen_public(const orc_ctx *c, const int64_t *s_coef, uint64_t seed,
                       uint64_t *pk) {
  const uint32_t n = c->n, L = c->L;
  uint64_t *s = malloc(sizeof(uint64_t) * L * n), *e = malloc(sizeof(uint64_t) * L * n);
  int64_t *ec = malloc(sizeof(int64_t) * n);
  orc_signed_to_eval(c, s_coef, 0, L, s);
  {
    orc_stream st = stream_open(seed, TAG_PK_E, 0);
    sample_cbd(&st, ec, n);
  }
  orc_signed_to_eval(c, ec, 0, L, e);
  for (uint32_t i = 0; i < L; ++i) {
    uint64_t q = c->mods[i];
    uint64_t *a = pk + ((size_t)L + i) * n, *b = pk + (size_t)i * n;
    {
      orc_stream st = stream_open(seed, TAG_PK_A, i);
      sample_uniform(&st, q, a, n);
    }
    for (uint32_t k = 0; k < n; ++k) {
      size_t o = (size_t)i * n + k;
      b[k] = submod(e[o], orc_mulmod(a[k], s[o], q), q);
    }
  }
  free(s);
  free(e);
  free(ec);
}

/* OpenFHE KeySwitchHYBRID::KeySwitchGenInternal: digit j encrypts
 * [P]_{q_i} s_old on the Q limbs of digit j under s_new. */
void orc_keygen_switch(const orc_ctx *c, const uint64_t *s_old_qp,
                       const uint64_t *s_new_qp, uint64_t seed, uint64_t tag,
                       uint64_t *key) {
  const uint32_t n = c->n, L = c->L, K = c->K, nm = L + K;
  uint64_t *e = malloc(sizeof(uint64_t) * nm * n);
  int64_t *ec = malloc(sizeof(int64_t) * n);
  for (uint32_t j = 0; j < c->dnum; ++j) {
    uint32_t s = j * c->alpha, end = s + c->alpha < L ? s + c->alpha : L;
    {
      orc_stream st = stream_open(seed, tag + TAG_KSK_E, j);
      sample_cbd(&st, ec, n);
    }
    orc_signed_to_eval(c, ec, 0, nm, e);
    for (uint32_t i = 0; i < nm; ++i) {
      uint64_t q = c->mods[i];
      uint64_t *b = key + (((size_t)j * 2 + 0) * nm + i) * n;
      uint64_t *a = key + (((size_t)j * 2 + 1) * nm + i) * n;
      {
        orc_stream st = stream_open(seed, tag + TAG_KSK_A, ((uint64_t)j << 16) | i);
        sample_uniform(&st, q, a, n);
      }
      uint64_t pmod = 1;
      for (uint32_t k = 0; k < K; ++k) pmod = orc_mulmod(pmod, c->mods[L + k] % q, q);
      int in_digit = i >= s && i < end;
      for (uint32_t k = 0; k < n; ++k) {
        size_t o = (size_t)i * n + k;
        uint64_t v = submod(e[o], orc_mulmod(a[k], s_new_qp[o], q), q);
        if (in_digit) v = addmod(v, orc_mulmod(pmod, s_old_qp[o], q), q);
        b[k] = v;
      }
    }
  }
  free(e);
  free(ec);
}

void orc_keygen_galois(const orc_ctx *c, const int64_t *s_coef, uint32_t galois,
                       uint64_t seed, uint64_t *key) {
  const uint32_t n = c->n, nm = c->L + c->K;
  uint64_t *s = malloc(sizeof(uint64_t) * nm * n), *sp = malloc(sizeof(uint64_t) * nm * n);
  orc_signed_to_eval(c, s_coef, 0, nm, s);
  /* s_new = s(X^{k^-1}) (OpenFHE EvalAutomorphismKeyGen). */
  uint32_t kinv = 1;
  {
    const uint64_t m = 2 * (uint64_t)n; /* not prime: search the odd units */
    for (uint64_t t = 1; t < m; t += 2)
      if ((t * galois) % m == 1) {
        kinv = (uint32_t)t;
        break;
      }
  }
  for (uint32_t i = 0; i < nm; ++i)
    orc_automorph_ntt(s + (size_t)i * n, sp + (size_t)i * n, n, kinv);
  orc_keygen_switch(c, s, sp, seed, TAG_GALOIS + ((uint64_t)galois << 3), key);
  free(s);
  free(sp);
}

void orc_keygen_relin(const orc_ctx *c, const int64_t *s_coef, uint64_t seed,
                      uint64_t *key) {
  const uint32_t n = c->n, nm = c->L + c->K;
  uint64_t *s = malloc(sizeof(uint64_t) * nm * n), *s2 = malloc(sizeof(uint64_t) * nm * n);
  orc_signed_to_eval(c, s_coef, 0, nm, s);
  for (uint32_t i = 0; i < nm; ++i)
    for (uint32_t k = 0; k < n; ++k) {
      size_t o = (size_t)i * n + k;
      s2[o] = orc_mulmod(s[o], s[o], c->mods[i]);
    }
  orc_keygen_switch(c, s2, s, seed, TAG_RELIN, key);
  free(s);
  free(s2);
}

void orc_encrypt_pk(const orc_ctx *c, const uint64_t *pk, const uint64_t *m,
                    uint32_t nq, uint64_t seed, uint64_t *ct) {
  const uint32_t n = c->n, L = c->L;
  int64_t *vc = malloc(sizeof(int64_t) * n), *ec = malloc(sizeof(int64_t) * n);
  uint64_t *v = malloc(sizeof(uint64_t) * nq * n), *e0 = malloc(sizeof(uint64_t) * nq * n),
           *e1 = malloc(sizeof(uint64_t) * nq * n);
  {
    orc_stream st = stream_open(seed, TAG_ENC_V, 0);
    sample_ternary(&st, vc, n);
  }
  orc_signed_to_eval(c, vc, 0, nq, v);
  {
    orc_stream st = stream_open(seed, TAG_ENC_E, 0);
    sample_cbd(&st, ec, n);
  }
  orc_signed_to_eval(c, ec, 0, nq, e0);
  {
    orc_stream st = stream_open(seed, TAG_ENC_E, 1);
    sample_cbd(&st, ec, n);
  }
  orc_signed_to_eval(c, ec, 0, nq, e1);
  for (uint32_t i = 0; i < nq; ++i) {
    uint64_t q = c->mods[i];
    for (uint32_t k = 0; k < n; ++k) {
      size_t o = (size_t)i * n + k;
      uint64_t b = pk[o], a = pk[(size_t)L * n + o];
      ct[o] = addmod(addmod(orc_mulmod(b, v[o], q), e0[o], q), m[o], q);
      ct[(size_t)nq * n + o] = addmod(orc_mulmod(a, v[o], q), e1[o], q);
    }
  }
  free(vc);
  free(ec);
  free(v);
  free(e0);
  free(e1);
}

void orc_decrypt(const orc_ctx *c, const uint64_t *ct, uint32_t npoly,
                 uint32_t nq, const int64_t *s_coef, uint64_t *m) {
  const uint32_t n = c->n;
  uint64_t *s = malloc(sizeof(uint64_t) * nq * n);
  orc_signed_to_eval(c, s_coef, 0, nq, s);
  for (uint32_t i = 0; i < nq; ++i) {
    uint64_t q = c->mods[i];
    for (uint32_t k = 0; k < n; ++k) {
      size_t o = (size_t)i * n + k;
      uint64_t acc = ct[o], sp = s[o];
      for (uint32_t p = 1; p < npoly; ++p) {
        acc = addmod(acc, orc_mulmod(ct[(size_t)p * nq * n + o], sp, q), q);
        sp = orc_mulmod(sp, s[o], q);
      }
      m[o] = acc;
    }
  }
  free(s);
}

/* ======================================================================
 * CKKS special FFT (encode/decode), restating the butterfly order and
 * twiddle table of native/fideslib_stage0/src/gpu_special_fft.cu:12-29,
 * :99-108 and patches/openfhe-v1.4.2-inverse-fft-plan.patch:18-60.
 * Plain IEEE double operations; build with -ffp-contract=off.
 * ====================================================================== */
/* OpenFHE's table entry is (cos(angle), sin(angle)); gcc at -O2 and above
 * (how OpenFHE and the reference's host code are built) fuses the pair into
 * one glibc sincos() call, whose results differ from separate cos()/sin() in
 * the last bit for a few angles.  sincos() is called explicitly so the
 * table does not depend on the optimisation level. */
static void fft_twiddle(uint32_t idx, uint32_t m, double *wr, double *wi) {
  const double angle = 2.0 * M_PI * idx / m;
  sincos(angle, wi, wr);
}

void orc_fft_special_inv(double *re, double *im, uint32_t slots) {
  const uint32_t m = 4 * slots;
  uint32_t *rot = malloc(sizeof(uint32_t) * slots);
  uint32_t p = 1;
  for (uint32_t j = 0; j < slots; ++j) {
    rot[j] = p;
    p = (uint32_t)(((uint64_t)p * 5) % m);
  }
  for (uint32_t len = slots; len >= 2; len >>= 1) {
    const uint32_t h = len / 2, lenq = 4 * len, gap = m / lenq;
    for (uint32_t i = 0; i < slots; i += len)
      for (uint32_t j = 0; j < h; ++j) {
        double wr, wi;
        fft_twiddle((lenq - rot[j] % lenq) * gap, m, &wr, &wi);
        const double ar = re[i + j], ai = im[i + j], br = re[i + j + h], bi = im[i + j + h];
        const double vr = ar - br, vi = ai - bi;
        re[i + j] = ar + br;
        im[i + j] = ai + bi;
        re[i + j + h] = vr * wr - vi * wi;
        im[i + j + h] = vi * wr + vr * wi;
      }
  }
  const uint32_t bits = ilog2(slots);
  double *tr = malloc(sizeof(double) * slots), *ti = malloc(sizeof(double) * slots);
  for (uint32_t t = 0; t < slots; ++t) {
    uint32_t s = bits ? bitrev(t, bits) : 0;
    tr[t] = re[s] / (double)slots;
    ti[t] = im[s] / (double)slots;
  }
  memcpy(re, tr, sizeof(double) * slots);
  memcpy(im, ti, sizeof(double) * slots);
  free(tr);
  free(ti);
  free(rot);
}

void orc_fft_special(double *re, double *im, uint32_t slots) {
  const uint32_t m = 4 * slots, bits = ilog2(slots);
  uint32_t *rot = malloc(sizeof(uint32_t) * slots);
  uint32_t p = 1;
  for (uint32_t j = 0; j < slots; ++j) {
    rot[j] = p;
    p = (uint32_t)(((uint64_t)p * 5) % m);
  }
  double *tr = malloc(sizeof(double) * slots), *ti = malloc(sizeof(double) * slots);
  for (uint32_t t = 0; t < slots; ++t) {
    uint32_t s = bits ? bitrev(t, bits) : 0;
    tr[t] = re[s];
    ti[t] = im[s];
  }
  memcpy(re, tr, sizeof(double) * slots);
  memcpy(im, ti, sizeof(double) * slots);
  free(tr);
  free(ti);
  for (uint32_t len = 2; len <= slots; len <<= 1) {
    const uint32_t h = len / 2, lenq = 4 * len, gap = m / lenq;
    for (uint32_t i = 0; i < slots; i += len)
      for (uint32_t j = 0; j < h; ++j) {
        double wr, wi;
        fft_twiddle((rot[j] % lenq) * gap, m, &wr, &wi);
        const double ur = re[i + j], ui = im[i + j];
        const double br = re[i + j + h], bi = im[i + j + h];
        const double vr = br * wr - bi * wi, vi = bi * wr + br * wi;
        re[i + j] = ur + vr;
        im[i + j] = ui + vi;
        re[i + j + h] = ur - vr;
        im[i + j + h] = ui - vi;
      }
  }
  free(rot);
}

int orc_encode(const orc_ctx *c, const double *re, const double *im,
               uint32_t count, uint32_t slots, double scale, uint32_t nq,
               uint64_t *out) {
  const uint32_t n = c->n, gap = n / (2 * slots);
  double *vr = calloc(slots, sizeof(double)), *vi = calloc(slots, sizeof(double));
  for (uint32_t j = 0; j < count && j < slots; ++j) {
    vr[j] = re[j];
    vi[j] = im ? im[j] : 0.0;
  }
  orc_fft_special_inv(vr, vi, slots);
  int64_t *coef = calloc(n, sizeof(int64_t));
  int status = 0;
  for (uint32_t i = 0; i < slots; ++i) {
    const double a = vr[i] * scale, b = vi[i] * scale;
    if (!isfinite(a) || !isfinite(b) || fabs(a) >= 4611686018427387904.0 ||
        fabs(b) >= 4611686018427387904.0) {
      status = -1;
      break;
    }
    coef[(size_t)i * gap] = llround(a);
    coef[(size_t)(i + slots) * gap] = llround(b);
  }
  if (status == 0) {
    for (uint32_t j = 0; j < nq; ++j) {
      uint64_t q = c->mods[j];
      uint64_t *o = out + (size_t)j * n;
      for (uint32_t e = 0; e < n; ++e) {
        int64_t v = coef[e];
        o[e] = v >= 0 ? (uint64_t)v % q : (q - ((uint64_t)(-v) % q)) % q;
      }
      orc_ctx_ntt_fwd(c, o, j);
    }
  }
  free(vr);
  free(vi);
  free(coef);
  return status;
}

/* Balanced mixed-radix (Garner) reconstruction: digits a_i in
 * (-q_i/2, q_i/2) represent the centred value sum a_i prod_{j<i} q_j. */
void orc_crt_centered(const orc_ctx *c, const uint64_t *coef, uint32_t nq,
                      double *out) {
  const uint32_t n = c->n;
  int64_t *a = malloc(sizeof(int64_t) * nq);
  uint64_t *inv = malloc(sizeof(uint64_t) * nq * nq);
  for (uint32_t i = 0; i < nq; ++i)
    for (uint32_t j = 0; j < i; ++j) inv[i * nq + j] = orc_invmod(c->mods[j] % c->mods[i], c->mods[i]);
  for (uint32_t e = 0; e < n; ++e) {
    for (uint32_t i = 0; i < nq; ++i) {
      uint64_t q = c->mods[i];
      uint64_t t = coef[(size_t)i * n + e];
      for (uint32_t j = 0; j < i; ++j) {
        uint64_t aj = a[j] >= 0 ? (uint64_t)a[j] % q : (q - ((uint64_t)(-a[j]) % q)) % q;
        t = orc_mulmod(submod(t, aj, q), inv[i * nq + j], q);
      }
      a[i] = t > (q >> 1) ? (int64_t)t - (int64_t)q : (int64_t)t;
    }
    long double v = (long double)a[nq - 1];
    for (int i = (int)nq - 2; i >= 0; --i) v = v * (long double)c->mods[i] + (long double)a[i];
    out[e] = (double)v;
  }
  free(a);
  free(inv);
}

void orc_decode(const orc_ctx *c, const uint64_t *poly, uint32_t nq,
                uint32_t slots, double scale, double *re, double *im) {
  const uint32_t n = c->n, gap = n / (2 * slots);
  uint64_t *coef = malloc(sizeof(uint64_t) * nq * n);
  memcpy(coef, poly, sizeof(uint64_t) * nq * n);
  for (uint32_t j = 0; j < nq; ++j) orc_ctx_ntt_inv(c, coef + (size_t)j * n, j);
  double *x = malloc(sizeof(double) * n);
  orc_crt_centered(c, coef, nq, x);
  for (uint32_t i = 0; i < slots; ++i) {
    re[i] = x[(size_t)i * gap] / scale;
    im[i] = x[(size_t)(i + slots) * gap] / scale;
  }
  orc_fft_special(re, im, slots);
  free(coef);
  free(x);
}
