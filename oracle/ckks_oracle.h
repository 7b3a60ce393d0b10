/*
 * CKKS-RNS CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, scalar restatement of the CKKS-RNS arithmetic that the
 * fhemamba native backend reaches through FIDESlib / OpenFHE 1.4.2
 * (native/fideslib_stage0/src/packed_fideslib.cpp:1060-1090 builds the
 * context; the hot loop calls EvalRotate / EvalFastRotation / EvalMult /
 * RescaleInPlace, packed_fideslib.cpp:117-251).  Only the test suite, the
 * smoke check and the bench's CPU-baseline leg load this library, and only
 * as the checker.  The shipped HIP library never links or calls it.
 *
 * Pinning status of each function (what it is checked against, in tests/):
 *   orc_gen_moduli       golden 57-prime OpenFHE chain (N=2^17, depth 44,
 *                        scale 59, first 60, dnum 4) from
 *                        results/b300/2026-09-28/long-accuracy/oracle-p-r3-base/native.json
 *   orc_root_of_unity    closed form: order exactly 2N; minimality by scan
 *   orc_ntt_fwd/inv      O(N^2) evaluation at psi^(2 brv(i)+1); convolution
 *                        theorem vs schoolbook negacyclic product; inverse
 *   orc_automorph_*      coefficient-domain X -> X^k closed form vs NTT-domain
 *                        permutation; decrypt(rot_r(ct)) == roll(m, r)
 *   orc_switch_basis     exact CRT with Python big integers on small inputs
 *   orc_modup/moddown,   decryption invariants (key switching preserves the
 *   orc_keyswitch        message up to small noise), big-integer CRT identity
 *                        of ModDown on tiny parameters
 *   orc_rescale          exact integer division on noiseless inputs
 *   orc_encode/decode    special FFT restated from
 *                        native/fideslib_stage0/src/gpu_special_fft.cu:12-108 and
 *                        patches/openfhe-v1.4.2-inverse-fft-plan.patch:18-60;
 *                        decode(encode(x)) == x, numpy FFT identity
 *   sampling / keygen    parity unpinned vs OpenFHE (its PRNG is not
 *                        reproducible offline); pinned by decryption
 *                        invariants only.
 */
#ifndef CKKS_ORACLE_H
#define CKKS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar modular arithmetic and number theory ---------------------- */
uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q);
uint64_t orc_powmod(uint64_t a, uint64_t e, uint64_t q);
uint64_t orc_invmod(uint64_t a, uint64_t q);
int orc_is_prime(uint64_t n);
uint64_t orc_first_prime(uint32_t bits, uint64_t m);
uint64_t orc_previous_prime(uint64_t q, uint64_t m);
uint64_t orc_next_prime(uint64_t q, uint64_t m);
uint64_t orc_root_of_unity(uint64_t m, uint64_t q);
/* FLEXIBLEAUTO Q chain (depth+1 primes) and HYBRID P primes.  Returns the
 * number of P primes written to p_out (capacity p_cap), or -1 on error. */
int orc_gen_moduli(uint32_t log_n, uint32_t depth, uint32_t scale_bits,
                   uint32_t first_bits, uint32_t dnum, uint64_t *q_out,
                   uint64_t *p_out, uint32_t p_cap);
/* Number of P primes for a given Q chain under HYBRID key switching. */
int orc_num_special_primes(const uint64_t *q, uint32_t nq, uint32_t dnum,
                           uint32_t aux_bits);

/* ---- single-limb transforms (need not be bound to a context) ---------- */
void orc_ntt_fwd(uint64_t *a, uint32_t n, uint64_t q, uint64_t psi);
void orc_ntt_inv(uint64_t *a, uint32_t n, uint64_t q, uint64_t psi);
void orc_ntt_naive(const uint64_t *a, uint64_t *out, uint32_t n, uint64_t q,
                   uint64_t psi);
void orc_negacyclic_schoolbook(const uint64_t *a, const uint64_t *b,
                               uint64_t *out, uint32_t n, uint64_t q);
void orc_automorph_ntt(const uint64_t *in, uint64_t *out, uint32_t n,
                       uint32_t k);
void orc_automorph_coeff(const uint64_t *in, uint64_t *out, uint32_t n,
                         uint32_t k, uint64_t q);
uint32_t orc_galois_elt(int32_t step, uint32_t n);
void orc_switch_basis(const uint64_t *x, const uint64_t *from_q,
                      uint32_t nfrom, uint64_t *y, const uint64_t *to_q,
                      uint32_t nto, uint32_t n);

/* ---- context-bound operations ----------------------------------------- */
typedef struct orc_ctx orc_ctx;
orc_ctx *orc_ctx_create(uint32_t log_n, const uint64_t *q, uint32_t L,
                        const uint64_t *p, uint32_t K, uint32_t dnum);
void orc_ctx_destroy(orc_ctx *c);
uint64_t orc_ctx_psi(const orc_ctx *c, uint32_t mod_idx);
/* mod_idx indexes the joint list q_0..q_{L-1}, p_0..p_{K-1}. */
void orc_ctx_ntt_fwd(const orc_ctx *c, uint64_t *a, uint32_t mod_idx);
void orc_ctx_ntt_inv(const orc_ctx *c, uint64_t *a, uint32_t mod_idx);
/* Batched limb-major transforms: data is [npoly][nlimb][N], limb j of each
 * poly uses modulus index limb0 + j.  nthreads > 1 uses OpenMP. */
void orc_ntt_fwd_batch(const orc_ctx *c, uint64_t *data, uint32_t npoly,
                       uint32_t limb0, uint32_t nlimb, int nthreads);
void orc_ntt_inv_batch(const orc_ctx *c, uint64_t *data, uint32_t npoly,
                       uint32_t limb0, uint32_t nlimb, int nthreads);
/* acc[l] = sum_i x_i[l] * w_i[l] over ncts ciphertexts ([2][nq][N] each)
 * and plaintexts ([nq][N] each); acc is [2][nq][N]. */
void orc_mac_batch(const orc_ctx *c, const uint64_t *x, const uint64_t *w,
                   uint32_t ncts, uint32_t nq, uint64_t *acc, int nthreads);

/* out = a + b mod q_l on npoly polys of nq limbs ([npoly][nq][N]). */
void orc_add(const orc_ctx *c, const uint64_t *a, const uint64_t *b, uint32_t npoly,
             uint32_t nq, uint64_t *out);

/* Hybrid key switching.  A key is [dnum][2][L+K][N] (b then a), evaluation
 * form over Q then P.  Ciphertext polys are evaluation form [nq][N]. */
uint32_t orc_num_digits(const orc_ctx *c, uint32_t nq);
void orc_modup(const orc_ctx *c, const uint64_t *a, uint32_t nq,
               uint64_t *digits /* [ndig][nq+K][N] */);
void orc_ksk_inner(const orc_ctx *c, const uint64_t *digits, uint32_t nq,
                   const uint64_t *key, uint64_t *ext /* [2][nq+K][N] */);
void orc_moddown(const orc_ctx *c, const uint64_t *ext, uint32_t nq,
                 uint64_t *out /* [nq][N] */);
void orc_keyswitch(const orc_ctx *c, const uint64_t *a, uint32_t nq,
                   const uint64_t *key, uint64_t *out /* [2][nq][N] */);
void orc_rotate(const orc_ctx *c, const uint64_t *ct, uint32_t nq,
                const uint64_t *key, uint32_t galois, uint64_t *out);
void orc_rotate_hoisted(const orc_ctx *c, const uint64_t *ct, uint32_t nq,
                        const uint64_t *digits, const uint64_t *key, uint32_t galois,
                        uint64_t *out);
void orc_rescale(const orc_ctx *c, const uint64_t *in, uint32_t npoly,
                 uint32_t nq, uint64_t *out /* [npoly][nq-1][N] */);
void orc_tensor(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
                uint32_t nq, uint64_t *out /* [3][nq][N] */);
void orc_relinearize(const orc_ctx *c, const uint64_t *ct3, uint32_t nq,
                     const uint64_t *key, uint64_t *out /* [2][nq][N] */);

/* ---- deterministic sampling (shared stream definition) ---------------- */
uint64_t orc_draw(uint64_t key, uint64_t ctr);
uint64_t orc_stream_key(uint64_t seed, uint64_t tag, uint64_t index);
void orc_sample_uniform(uint64_t key, uint64_t q, uint64_t *out, uint32_t n);
void orc_sample_ternary(uint64_t key, int64_t *out, uint32_t n);
void orc_sample_cbd(uint64_t key, int64_t *out, uint32_t n);
void orc_sample_sparse_ternary(uint64_t key, int64_t *out, uint32_t n, uint32_t h);
/* ChaCha20 block function (RFC 8439 section 2.3). */
void orc_chacha20_block(const uint32_t key[8], uint32_t counter, const uint32_t nonce[3],
                        uint32_t out[16]);
/* Sampling family of every later key generation / encryption call: NULL
 * selects the seeded family (the default), a 32-byte key the ChaCha20
 * family under that master key. */
void orc_set_sampling_key(const uint8_t *key32);
uint64_t orc_stream_word(uint64_t seed, uint64_t tag, uint64_t index, uint64_t i);

/* Signed small coefficients -> evaluation form over modulus indices
 * [idx0, idx0+nlimb). */
void orc_signed_to_eval(const orc_ctx *c, const int64_t *coef,
                        uint32_t idx0, uint32_t nlimb, uint64_t *out);
/* Key generation.  s_coef: ternary secret (N int64). */
void orc_keygen_secret(uint64_t seed, uint32_t n, int64_t *s_coef);
/* Sparse-ternary secret: exactly h coefficients +-1 (h <= n). */
void orc_keygen_secret_sparse(uint64_t seed, uint32_t n, uint32_t h, int64_t *s_coef);
void orc_keygen_public(const orc_ctx *c, const int64_t *s_coef, uint64_t seed,
                       uint64_t *pk /* [2][L][N] */);
/* Switching key from s_old to s_new, both given as evaluation form over
 * Q then P ([L+K][N]). */
void orc_keygen_switch(const orc_ctx *c, const uint64_t *s_old_qp,
                       const uint64_t *s_new_qp, uint64_t seed, uint64_t tag,
                       uint64_t *key /* [dnum][2][L+K][N] */);
void orc_keygen_galois(const orc_ctx *c, const int64_t *s_coef,
                       uint32_t galois, uint64_t seed, uint64_t *key);
void orc_keygen_relin(const orc_ctx *c, const int64_t *s_coef, uint64_t seed,
                      uint64_t *key);
void orc_encrypt_pk(const orc_ctx *c, const uint64_t *pk, const uint64_t *m,
                    uint32_t nq, uint64_t seed, uint64_t *ct /* [2][nq][N] */);
void orc_decrypt(const orc_ctx *c, const uint64_t *ct, uint32_t npoly,
                 uint32_t nq, const int64_t *s_coef, uint64_t *m /* [nq][N] */);

/* ---- CKKS encoding ---------------------------------------------------- */
void orc_fft_special_inv(double *re, double *im, uint32_t slots);
void orc_fft_special(double *re, double *im, uint32_t slots);
/* Returns 0 on success, -1 if a scaled coefficient does not fit. */
int orc_encode(const orc_ctx *c, const double *re, const double *im,
               uint32_t count, uint32_t slots, double scale, uint32_t nq,
               uint64_t *out /* [nq][N] evaluation form */);
void orc_decode(const orc_ctx *c, const uint64_t *poly, uint32_t nq,
                uint32_t slots, double scale, double *re, double *im);
/* Centered CRT value of coefficient-form residues [nq][N] as doubles. */
void orc_crt_centered(const orc_ctx *c, const uint64_t *coef, uint32_t nq,
                      double *out);

#ifdef __cplusplus
}
#endif
#endif
