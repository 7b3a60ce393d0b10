/*
 * fhecore -- MI355X (gfx950) CKKS-RNS evaluation core, C ABI.
 *
 * Replaces, for the encrypted Mamba decode hot loop, the FIDESlib /
 * OpenFHE `fideslib::CryptoContext<DCRTPoly>` calls that the reference's
 * native executors make (native/fideslib_stage0/src/packed_fideslib.cpp,
 * native/fideslib_stage0/src/stage1_mamba2_decode_fideslib.cpp) and the
 * in-tree CUDA helpers beside them.  Python binds it with ctypes
 * (fhe-mamba_amd/fhemamba_amd/_lib.py).
 *
 * Conventions
 *   - Every function returns FHE_OK (0) or an FHE_ERR_* code; no C++
 *     exception crosses the ABI.  fhe_last_error() returns the message of
 *     the calling thread's last failure.
 *   - RNS data is uint64, limb-major: [poly][limb][N].  Limb j of a
 *     ciphertext at level with `nlimb` limbs is reduced mod q_j.  Ciphertext
 *     and plaintext polys are in evaluation (NTT) form unless stated.
 *   - Moduli index the joint list q_0..q_{L-1}, p_0..p_{K-1}.
 *   - Device work is asynchronous on the context's stream; host buffers
 *     passed to *_upload / *_download / fhe_encode* / fhe_decode are only
 *     read or written during the call (encodes copy their input to a
 *     staging buffer; the others synchronise).
 *   - Where an entry point lets its output alias an input, the result may
 *     occupy new device storage: fhe_poly_data gives the current address.
 *   - Handles are owned by the caller and released explicitly.  One
 *     context is used by one host thread at a time.
 */
#ifndef FHECORE_H
#define FHECORE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FHE_OK = 0,
  FHE_ERR_ARG = 1,   /* invalid argument or shape mismatch */
  FHE_ERR_HIP = 2,   /* HIP runtime failure */
  FHE_ERR_RANGE = 3, /* value does not fit (encode) */
  FHE_ERR_STATE = 4, /* wrong object state (e.g. key for another context) */
  FHE_ERR_INTERNAL = 5
};

typedef struct fhe_context fhe_context;
typedef struct fhe_poly fhe_poly; /* device RNS poly set [npoly][nlimb][N] */
typedef struct fhe_key fhe_key;   /* hybrid switching key */

const char *fhe_last_error(void);
int fhe_abi_version(void);

/* ---- parameters --------------------------------------------------------
 * FLEXIBLEAUTO Q chain (depth+1 primes) and HYBRID P primes for ring 2^log_n.
 * Replaces CCParams<CryptoContextCKKSRNS> + GenCryptoContext prime choice
 * (native/fideslib_stage0/src/packed_fideslib.cpp:1060-1068,
 *  src/fhemamba/ckks_probes.py:180-189). */
int fhe_gen_moduli(uint32_t log_n, uint32_t depth, uint32_t scale_bits,
                   uint32_t first_bits, uint32_t dnum, uint64_t *q_out,
                   uint64_t *p_out, uint32_t p_cap, uint32_t *num_p);

/* ---- context -----------------------------------------------------------
 * Replaces GenCryptoContext + LoadContext (packed_fideslib.cpp:1060-1090,
 * stage1_mamba2_decode_fideslib.cpp:1224-1277): builds twiddle and basis
 * conversion tables on `device`. */
int fhe_context_create(uint32_t log_n, const uint64_t *q, uint32_t num_q,
                       const uint64_t *p, uint32_t num_p, uint32_t dnum,
                       int device, fhe_context **out);
int fhe_context_destroy(fhe_context *ctx);
/* log_n, num_q (L), num_p (K), dnum (non-empty digits), alpha (limbs/digit) */
int fhe_context_info(const fhe_context *ctx, uint32_t *info5);
/* Allocation requests the library has made in this process (device pool
 * requests, fresh or reused, and device or pinned-host table and staging
 * allocations).  No counterpart in the reference: a memory diagnostic, e.g.
 * to show that a stretch of calls allocated nothing. */
int fhe_alloc_count(uint64_t *count);
/* moduli (L+K) and their primitive 2N-th roots psi (L+K). */
int fhe_context_moduli(const fhe_context *ctx, uint64_t *mods, uint64_t *psi);
/* Run the context's work on a caller stream (a hipStream_t, e.g. torch's
 * current stream); NULL restores the context's own stream. */
int fhe_context_set_stream(fhe_context *ctx, void *hip_stream);
/* Replaces the per-op cudaDeviceSynchronize of packed_fideslib.cpp:40-42. */
int fhe_sync(fhe_context *ctx);

/* ---- profiling -----------------------------------------------------------
 * Bracket every kernel the context launches with HIP events on its stream
 * (the reference's phase timers and --profile-evaluation bracket,
 * packed_fideslib.cpp:1216-1220).  fhe_profile_end synchronises and writes a
 * JSON object {"kernel": [launches, total_ms], ...} into buf (cap bytes). */
int fhe_profile_begin(fhe_context *ctx);
int fhe_profile_end(fhe_context *ctx, char *buf, size_t cap);

/* ---- raw batched kernels on caller device memory ------------------------
 * Forward / inverse negacyclic NTT of data [npoly][nlimb][N] in place; limb
 * j uses modulus limb0 + j.  Replaces FIDESlib NTT_/INTT launches
 * (experiments/ntt_warp_tail/probe.cu:58-66, fideslib_plaintext_rns.cu:119-137). */
int fhe_ntt_forward(fhe_context *ctx, uint64_t *data, uint32_t npoly,
                    uint32_t nlimb, uint32_t limb0);
int fhe_ntt_inverse(fhe_context *ctx, uint64_t *data, uint32_t npoly,
                    uint32_t nlimb, uint32_t limb0);
/* acc[2][nq][N] = sum_i x_i (.) w_i for x [n][2][nq][N], w [n][nq][N]: the
 * plaintext-ciphertext inner product of a BSGS diagonal sum
 * (stage1_mamba2_decode_fideslib.cpp:575-600, packed_fideslib.cpp:447-516). */
int fhe_mac(fhe_context *ctx, const uint64_t *x, const uint64_t *w, uint32_t n,
            uint32_t nq, uint64_t *acc);

/* ---- device polys ------------------------------------------------------ */
int fhe_poly_create(fhe_context *ctx, uint32_t npoly, uint32_t nlimb,
                    fhe_poly **out);
int fhe_poly_destroy(fhe_poly *p);
int fhe_poly_shape(const fhe_poly *p, uint32_t *npoly, uint32_t *nlimb);
/* Device pointer of the [npoly][nlimb][N] array (valid until destroy or a
 * shape change). */
int fhe_poly_data(const fhe_poly *p, uint64_t **dev);
int fhe_poly_upload(fhe_poly *p, const uint64_t *host, uint32_t npoly,
                    uint32_t nlimb);
int fhe_poly_download(const fhe_poly *p, uint64_t *host);
/* Ciphertext->Clone() (packed_fideslib.cpp:118). */
int fhe_poly_copy(fhe_poly *dst, const fhe_poly *src);
/* Ciphertext SetLevel / level drop: keep the first nlimb limbs
 * (packed_fideslib.cpp:125-126, stage1_mamba2_decode_fideslib.cpp:621-628). */
int fhe_drop_limbs(fhe_poly *out, const fhe_poly *a, uint32_t nlimb);

/* ---- arithmetic (evaluation form; in-place use with out == a is allowed) -
 * EvalAdd / EvalSub (packed_fideslib.cpp:131-149, :571). */
int fhe_add(fhe_poly *out, const fhe_poly *a, const fhe_poly *b);
int fhe_sub(fhe_poly *out, const fhe_poly *a, const fhe_poly *b);
int fhe_negate(fhe_poly *out, const fhe_poly *a);
/* EvalMult(ct, pt) / EvalAdd(ct, pt) with a one-poly plaintext
 * (packed_fideslib.cpp:177-178, stage1_mamba2_decode_fideslib.cpp:1758-1761). */
int fhe_mul_plain(fhe_poly *out, const fhe_poly *ct, const fhe_poly *pt);
int fhe_add_plain(fhe_poly *out, const fhe_poly *ct, const fhe_poly *pt);
/* Per-limb constants c[j] < q_j: EvalMult(ct, double) once the double is
 * scaled to an integer (packed_fideslib.cpp:118), and EvalAdd(ct, double)
 * (packed_fideslib.cpp:162) which adds c[j] to poly 0 only. */
int fhe_mul_const(fhe_poly *out, const fhe_poly *a, const uint64_t *c);
int fhe_add_const(fhe_poly *out, const fhe_poly *a, const uint64_t *c);
/* out = sum_i m_i * xs[i] over count 2-poly ciphertexts, on their first
 * nlimb limbs (each term holds at least nlimb), with integer weights m_i as
 * two's-complement 128-bit values, weights[2i] the low and weights[2i+1]
 * the high word: the Chebyshev leaf sum, a scaled term per basis element
 * added into the accumulator (packed_fideslib.cpp:577-584), in one pass over
 * the terms.  out is [2][nlimb] and may not alias a term. */
int fhe_linear_wsum(fhe_poly *out, const fhe_poly *const *xs, const uint64_t *weights,
                    uint32_t count, uint32_t nlimb);
/* multIntScalar (native/fideslib_stage0/src/fideslib_refresh_correction.hpp:37). */
int fhe_mul_int(fhe_poly *out, const fhe_poly *a, int64_t c);
/* RescaleInPlace, FLEXIBLEAUTO (packed_fideslib.cpp:236): drop the last limb
 * with division by its prime and centred rounding. */
int fhe_rescale(fhe_poly *out, const fhe_poly *a);
/* fhe_rescale of `count` inputs of one shape at once (as[r] into outs[r]):
 * the rescales of one step of the reference's Chebyshev evaluation (the
 * basis powers of one depth before they are multiplied again,
 * src/fhemamba/ckks_probes.py:108-155) sharing one set of launches.
 * Outputs must be distinct and none may be one of the inputs. */
int fhe_rescale_many(fhe_poly *const *outs, const fhe_poly *const *as, uint32_t count);
/* ModRaise, the first step of EvalBootstrap (packed_fideslib.cpp:235-270,
 * stage1_mamba2_decode_fideslib.cpp:2127): limb 0 (mod q0) of every poly
 * of a, centred, lifted to q_0..q_{nlimb-1}; out is [npoly][nlimb]. */
int fhe_mod_raise(fhe_poly *out, const fhe_poly *a, uint32_t nlimb);
/* Tensor product of two 2-poly ciphertexts -> 3 polys (EvalMult core);
 * a == b gives the 3-product square (EvalSquareInPlace,
 * native/fideslib_stage0/src/fideslib_owned_arithmetic.hpp:10-19). */
int fhe_tensor(fhe_poly *out3, const fhe_poly *a, const fhe_poly *b);

/* ---- keys --------------------------------------------------------------
 * A hybrid switching key as [dnum][2][L+K][N] residues (b then a) in
 * evaluation form; loaded once, kept resident in HBM.  Replaces
 * EvalMultKeyGen / EvalRotateKeyGen + LoadContext key upload
 * (packed_fideslib.cpp:1080-1083). */
int fhe_key_load(fhe_context *ctx, const uint64_t *host, fhe_key **out);
/* The inverse of fhe_key_load: the key's residues [dnum][2][L+K][N] in the
 * same standard evaluation form, into `host` (for serialising the
 * evaluation keys of the client/server handoff: SerializeEvalMultKey /
 * SerializeEvalAutomorphismKey, stage1_mamba2_decode_fideslib.cpp:
 * 1466-1477). */
int fhe_key_download(const fhe_key *k, uint64_t *host);
int fhe_key_destroy(fhe_key *k);

/* ---- key switching ----------------------------------------------------
 * Hybrid key switch of one poly a [1][nq][N] -> out [2][nq][N]. */
int fhe_keyswitch(fhe_poly *out, const fhe_poly *a, const fhe_key *key);
/* Relinearize a 3-poly tensor (EvalMult(ct, ct) relinearisation,
 * packed_fideslib.cpp:147-149). */
int fhe_relinearize(fhe_poly *out, const fhe_poly *ct3, const fhe_key *key);
/* fhe_relinearize of `count` 3-poly tensors of one level at once (ct3s[r]
 * into outs[r]): the independent EvalMult relinearisations of one step of
 * the reference's Chebyshev evaluation (the basis powers of one depth and
 * the giant-step products of one tree height, src/fhemamba/ckks_probes.py:
 * 108-155) as one batched ModUp and one batched ModDown.  Outputs must be
 * distinct and none may be one of the tensors. */
int fhe_relinearize_many(fhe_poly *const *outs, const fhe_poly *const *ct3s, uint32_t count,
                         const fhe_key *key);
/* EvalRotate / EvalConjugate: key switch c1, add c0, apply X -> X^galois
 * (packed_fideslib.cpp:207-221, stage1_mamba2_decode_fideslib.cpp:1779-1801,
 *  :2342). */
int fhe_rotate(fhe_poly *out, const fhe_poly *ct, const fhe_key *key,
               uint32_t galois);
/* fhe_rotate without any device allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Same result
 * as fhe_rotate, word for word.  `out` must already hold [2][nq][N] (it may
 * be `ct`).  Intermediates live in a fixed 128 MiB device array of the
 * library, one per GPU, kept until the process ends: shapes needing more
 * (roughly N*(dnum_eff*(nq+K) + 3nq + 2K) words, + 2nq*N when out == ct)
 * give FHE_ERR_ARG.  The level's conversion tables must already exist (any
 * allocating key switch at that level builds them), else FHE_ERR_STATE.
 * Calls on one GPU share the array and are ordered on it: a call from
 * another stream (another context, or a caller stream) waits on the GPU for
 * the previous call's work before its own, and host threads take turns
 * enqueuing.  The array keeps the last call's contents. */
int fhe_rotate_noalloc(fhe_poly *out, const fhe_poly *ct, const fhe_key *key,
                       uint32_t galois);
/* EvalFastRotationPrecompute: ModUp'd digits of c1, in a new poly handle of
 * shape [dnum_eff][nq+K][N] (native/fideslib_stage0/src/fideslib_rotation_batch.hpp:17). */
int fhe_rotation_precompute(const fhe_poly *ct, fhe_poly **digits);
/* EvalFastRotation over `count` steps sharing one precompute
 * (fideslib_rotation_batch.hpp:18). */
int fhe_rotate_hoisted(const fhe_poly *ct, const fhe_poly *digits,
                       const fhe_key *const *keys, const uint32_t *galois,
                       uint32_t count, fhe_poly *const *outs);
/* EvalRotate over `count` different ciphertexts of one level at once
 * (cts[r] by keys[r] / galois[r] into outs[r]): the per-stream rotations
 * of the reference's Mamba-2 step (src/stage1_mamba2_decode_fideslib.cpp:
 * 3865-3890, 4047-4052: the same rotate-sum step on every state group) as
 * one batched ModUp and one batched ModDown.  Outputs must be distinct; an
 * output may be one of the inputs. */
int fhe_rotate_many(fhe_poly *const *outs, const fhe_poly *const *cts,
                    const fhe_key *const *keys, const uint32_t *galois,
                    uint32_t count);
/* LinearTransformInPlace(ct, rowSize = count, bStep = bstep, pts)
 * (native/fideslib_stage0/patches/fideslib-v2.1.0-linear-transform-api.patch:21-38,
 *  called at src/stage1_mamba2_decode_fideslib.cpp:3517-3531; unfused form
 *  src/packed_fideslib.cpp:447-516):
 *   out = sum_g rot_giant^g( sum_b pts[g*bstep + b] (.) rot_b(ct) )
 * with pts already pre-rotated by the caller for their giant step.
 * baby_keys[b-1] / baby_galois[b-1] rotate by b strides (b = 1..bstep-1; a
 * key may be null when no diagonal uses that baby), all babies from one
 * ModUp; giant_key rotates by bstep strides and is applied by Horner's rule
 * (required when count > bstep).  pts[k] may be null (zero diagonal); at
 * least one must be present.  Plaintexts are one-poly with at least the
 * ciphertext's limbs.  out may be ct. */
int fhe_linear_transform(fhe_poly *out, const fhe_poly *ct,
                         const fhe_poly *const *pts, uint32_t count,
                         uint32_t bstep, const fhe_key *const *baby_keys,
                         const uint32_t *baby_galois, const fhe_key *giant_key,
                         uint32_t giant_galois);
/* The same sum with the caller's pre-rotation and the giant steps folded
 * in (LinearTransformInPlace with a nonzero offset: the ciphertext rotated
 * by `offset` first, packed_fideslib.cpp:447-516; no separate counterpart):
 * baby_keys[b] / baby_galois[b] for b = 0..min(bstep, count)-1 rotate ct by
 * offset + b strides (baby_keys[0] null: baby 0 is ct itself, no offset),
 * all babies from one ModUp, so the offset costs no key switch of its own.
 * n_giant_keys = 1: giant_keys[0] rotates by bstep strides, applied by
 * Horner's rule; n_giant_keys = G - 1 (G = ceil(count / bstep)):
 * giant_keys[g-1] rotates by g * bstep strides and the G - 1 giant
 * rotations run as one batch of independent key switches. */
int fhe_linear_transform_hoisted(fhe_poly *out, const fhe_poly *ct,
                                 const fhe_poly *const *pts, uint32_t count,
                                 uint32_t bstep, const fhe_key *const *baby_keys,
                                 const uint32_t *baby_galois,
                                 const fhe_key *const *giant_keys,
                                 const uint32_t *giant_galois,
                                 uint32_t n_giant_keys);
/* fhe_linear_transform_hoisted of ncts (1..64) ciphertexts cts[i] of one
 * limb count with the same diagonals and keys, into outs[i]: the
 * bootstrap's CoeffToSlot / SlotToCoeff groups of several ciphertexts
 * refreshed at one point of a circuit (the reference's
 * LinearTransformInPlace per ciphertext, packed_fideslib.cpp:447-516, run
 * in each bootstrap of the decoder's state-group refreshes,
 * stage1_mamba2_decode_fideslib.cpp:3952-3967).  One batched ModUp for every ciphertext's babies, their key
 * switches in shared batches, the giant-step rotations of all of them as
 * one set; the same outputs as ncts single calls.  outs must be distinct;
 * an output may be any of the inputs. */
int fhe_linear_transform_hoisted_many(fhe_poly *const *outs,
                                      const fhe_poly *const *cts, uint32_t ncts,
                                      const fhe_poly *const *pts, uint32_t count,
                                      uint32_t bstep,
                                      const fhe_key *const *baby_keys,
                                      const uint32_t *baby_galois,
                                      const fhe_key *const *giant_keys,
                                      const uint32_t *giant_galois,
                                      uint32_t n_giant_keys);

/* ---- encoding -----------------------------------------------------------
 * MakeCKKSPackedPlaintext (packed_fideslib.cpp:204): special inverse FFT of
 * `count` complex values into `slots` slots, scale, round (ties away from
 * zero), RNS lift to nlimb limbs and NTT, all on the GPU
 * (native/fideslib_stage0/src/gpu_special_fft.cu:12-108,
 *  fideslib_plaintext_rns.cu:11-53).  im may be NULL. */
int fhe_encode(fhe_context *ctx, const double *re, const double *im,
               uint32_t count, uint32_t slots, double scale, uint32_t nlimb,
               fhe_poly *out);
/* nvec encodes in one call: row r of re / im (count values each, im may be
 * NULL) into outs[r], each as fhe_encode would write it.  Replaces the
 * reference decoder's look-ahead batches of MakeCKKSPackedPlaintext calls for
 * uncached BSGS diagonals (stage1_mamba2_decode_fideslib.cpp:165-167,
 * :440-447).  The vectors share the FFT, rounding and NTT launches, up to 16
 * per set.  A row whose values may not fit 62 bits after scaling is encoded
 * by the checked single path; FHE_ERR_RANGE names the first that fails (the
 * outputs of earlier rows are then written).  Outputs must be distinct. */
int fhe_encode_many(fhe_context *ctx, const double *re, const double *im,
                    uint32_t count, uint32_t nvec, uint32_t slots, double scale,
                    uint32_t nlimb, fhe_poly *const *outs);
/* Decode a decrypted one-poly plaintext: iNTT, centred CRT, /scale and the
 * forward special FFT (GetRealPackedValue, packed_fideslib.cpp:1227-1236). */
int fhe_decode(fhe_context *ctx, const fhe_poly *pt, uint32_t slots,
               double scale, double *re, double *im);

/* ---- client-side key material and encryption ---------------------------
 * Every sample below is drawn from a stream named by (seed, sample kind,
 * limb / digit).  A new context uses the ChaCha20 family under a 256-bit
 * master key from OS entropy: secure, and the seed is only a per-call
 * label.  fhe_context_set_sampling replaces the master key
 * (FHE_SAMPLING_CHACHA20 with key32 = 32 bytes, or NULL for fresh OS
 * entropy) or selects the seeded family (FHE_SAMPLING_SEEDED, key32 NULL):
 * there the seed alone fixes every sample, which makes keys reproducible
 * for parity tests and NOT secure (a public key reveals the seed).  Takes
 * effect for later calls.  No counterpart in the reference: OpenFHE draws
 * from its own PRNG (packed_fideslib.cpp:1080-1083). */
enum {
  FHE_SAMPLING_CHACHA20 = 0,
  FHE_SAMPLING_SEEDED = 1
};
int fhe_context_set_sampling(fhe_context *ctx, int mode, const uint8_t *key32);
/* Ternary secret (N int64 coefficients) and the public / switching keys
 * derived from it (KeyGen, EvalMultKeyGen, EvalRotateKeyGen:
 * packed_fideslib.cpp:1080-1083). */
int fhe_keygen_secret(fhe_context *ctx, uint64_t seed, int64_t *s_coef);
/* Sparse-ternary secret with exactly h nonzero coefficients (+-1):
 * KeyGen under SetSecretKeyDist(SPARSE_TERNARY), the Mamba-2 decoder's
 * default (native/fideslib_stage0/src/stage1_mamba2_decode_fideslib.cpp:
 * 1225, stage1_mamba2_config.hpp:211).  1 <= h <= N, else FHE_ERR_ARG. */
int fhe_keygen_secret_sparse(fhe_context *ctx, uint64_t seed, uint32_t h,
                             int64_t *s_coef);
int fhe_keygen_public(fhe_context *ctx, const int64_t *s_coef, uint64_t seed,
                      fhe_poly *pk);
int fhe_keygen_relin(fhe_context *ctx, const int64_t *s_coef, uint64_t seed,
                     fhe_key **out);
int fhe_keygen_galois(fhe_context *ctx, const int64_t *s_coef,
                      uint32_t galois, uint64_t seed, fhe_key **out);
/* Encrypt(publicKey, pt) (packed_fideslib.cpp:205) and Decrypt
 * (packed_fideslib.cpp:1227). */
int fhe_encrypt(fhe_poly *ct, const fhe_poly *pk, const fhe_poly *pt,
                uint64_t seed);
int fhe_decrypt(fhe_poly *pt, const fhe_poly *ct, const int64_t *s_coef);

#ifdef __cplusplus
}
#endif
#endif
