// Device operations on raw limb-major arrays, called by the C ABI layer.
// Shapes: a poly set is [npoly][nlimb][N]; limb j is reduced mod q_j.
#pragma once

#include "context.hpp"

namespace fhe {

enum BinOp { OP_ADD = 0, OP_SUB = 1 };

// Elementwise (out may alias an input).
// out = sum of cnt polys in[j] [npoly][nlimb][N] (cnt <= SUM_MAX), one pass.
constexpr uint32_t SUM_MAX = 16;
void poly_sum(Context& c, uint64_t* out, const uint64_t* const* in, uint32_t cnt,
              uint32_t npoly, uint32_t nlimb);
void poly_binary(Context& c, BinOp op, uint64_t* out, const uint64_t* a, const uint64_t* b,
                 uint32_t npoly, uint32_t nlimb);
void poly_negate(Context& c, uint64_t* out, const uint64_t* a, uint32_t npoly, uint32_t nlimb);
void poly_mul_plain(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* pt,
                    uint32_t npoly, uint32_t nlimb);
void poly_add_plain(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* pt,
                    uint32_t npoly, uint32_t nlimb);
// Per-limb constants (host array of nlimb values < q_j).
void poly_mul_const(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* consts,
                    uint32_t npoly, uint32_t nlimb);
void poly_add_const(Context& c, uint64_t* out, const uint64_t* a, const uint64_t* consts,
                    uint32_t npoly, uint32_t nlimb);
// Copy the first `nlimb` limbs of every poly from a (a_nlimb limbs/poly)
// into out (out_nlimb limbs/poly).
void poly_copy_limbs(Context& c, uint64_t* out, uint32_t out_nlimb, const uint64_t* a,
                     uint32_t a_nlimb, uint32_t npoly, uint32_t nlimb);
// out3 = (a0 b0, a0 b1 + a1 b0, a1 b1); a == b takes the squaring path.
void poly_tensor(Context& c, uint64_t* out3, const uint64_t* a, const uint64_t* b,
                 uint32_t nlimb);
// acc[2][nq][N] = sum_i x_i (.) w_i for x [n][2][nq][N], w [n][nq][N].
void poly_mac(Context& c, uint64_t* acc, const uint64_t* x, const uint64_t* w, uint32_t n,
              uint32_t nq);
// acc [2][nq][N] (+)= sum_i x[i] (.) w[i] for ciphertexts x[i] [2][nq][N] and
// plaintexts w[i] (first nq limbs used) given by address; cnt may be 0.
constexpr uint32_t MAC_TABLE = 64;
struct MacTable {
  const uint64_t* x[MAC_TABLE];
  const uint64_t* w[MAC_TABLE];
};
void poly_mac_table(Context& c, uint64_t* acc, const uint64_t* const* x,
                    const uint64_t* const* w, uint32_t cnt, uint32_t nq, bool accumulate);
// out [2][nq][N] = sum_i m_i * x_i mod q_j over ciphertexts x_i [2][nl_i][N]
// (nl_i >= nq; their first nq limbs), with integer weights m_i given as
// two's-complement 128-bit values (lo, hi); up to WSUM_MAX terms per launch.
constexpr uint32_t WSUM_MAX = 16;
void poly_linear_wsum(Context& c, uint64_t* out, const uint64_t* const* x, const uint32_t* x_nlimb,
                      const uint64_t* weights, uint32_t cnt, uint32_t nq);
// The inner sums of several giant steps of a BSGS transform in one pass:
// acc[g] [2][nq][N] = sum_b x[b] (.) w[g * nb + b] for g < ng, b < nb, null
// w entries skipped; every x word is read once for all g (up to
// MACG_MAX_G giants and MACG_MAX_B babies per call).
constexpr uint32_t MACG_MAX_G = 8, MACG_MAX_B = 32;
void poly_mac_giants(Context& c, uint64_t* const* acc, uint32_t ng, const uint64_t* const* x,
                     uint32_t nb, const uint64_t* const* w, uint32_t nq);
// ModRaise: limb 0 of each of npoly polys of a ([npoly][a_nlimb][N],
// evaluation form mod q0) to coefficient form, centred, lifted to
// q_0..q_{nq_out-1} and back to evaluation form in out [npoly][nq_out][N].
void poly_mod_raise(Context& c, uint64_t* out, uint32_t nq_out, const uint64_t* a,
                    uint32_t a_nlimb, uint32_t npoly);
// Drop the last limb with centred division (FLEXIBLEAUTO rescale);
// out is [npoly][nq-1][N].
void poly_rescale(Context& c, uint64_t* out, const uint64_t* a, uint32_t npoly, uint32_t nq);
// poly_rescale of `count` inputs of one shape (outs[r] must not alias any
// as[.]); at N = 2^13..2^17 up to 16 of them share one set of launches.
void poly_rescale_many(Context& c, uint64_t* const* outs, const uint64_t* const* as,
                       uint32_t count, uint32_t npoly, uint32_t nq);

// ---- hybrid key switching (keyswitch.hip) ----
uint32_t num_digits(const Context& c, uint32_t nq);
// Digits [nd][nq+K][N] (evaluation form) of a [nq][N].
void modup(Context& c, const uint64_t* a, uint32_t nq, uint64_t* digits);
// ModUp of `count` inputs as[i] [nq][N] into digits [count][nd][nq+K][N].
void modup_batch(Context& c, const uint64_t* const* as, uint32_t count, uint32_t nq,
                 uint64_t* digits);
// Result of one key switch r of a batch:
//   out_b = galois-permute((ext_b[Q] - ModDownConv(ext_b[P])) * P^-1 + add_b),
// b = 0, 1, with ext_b = sum_j digits_j (.) key_r,j,b over Q_l + P, addends
// add0 / add1 ([nq][N], may be null) and galois 1 meaning no permutation.
// out must not alias its addends.
struct KeySwitchOut {
  uint64_t* out;         // [2][nq][N]
  const uint64_t* add0;  // added to component 0 (or null)
  const uint64_t* add1;  // added to component 1 (or null)
  uint32_t galois;       // Galois element applied to the result (1 = none)
};
// B <= MAX_KS_BATCH key switches of one set of digits (keys in Montgomery
// form): one batched ModDown whose inverse NTT forms the P limbs of the
// inner product as it loads, and whose forward NTT's last pass forms the Q
// limbs and applies the combine and the Galois permutation.
void keyswitch_batch(Context& c, const uint64_t* digits, uint32_t nq,
                     const uint64_t* const* keys, uint32_t batch, const KeySwitchOut* outs);
// The same with digits[r] ([nd][nq+K][N]) per key switch.
void keyswitch_batch(Context& c, const uint64_t* const* digits, uint32_t nq,
                     const uint64_t* const* keys, uint32_t batch, const KeySwitchOut* outs);
// ModUp of a [nq][N] (evaluation form) and one key switch.
void keyswitch(Context& c, const uint64_t* a, uint32_t nq, const uint64_t* key,
               const KeySwitchOut& out);
// `count` key switches of one set of digits (keys[r] in Montgomery form), in
// batches that share one read of the digits (scratch per batch <= 2 GiB).
void keyswitch_hoisted(Context& c, const uint64_t* digits, uint32_t nq,
                       const uint64_t* const* keys, const KeySwitchOut* outs, uint32_t count);
// Rotate ct [2][nq][N] by one key: out = galois-permute(KS(c1) + (c0, 0)).
// out must not alias ct.
void rotate(Context& c, uint64_t* out, const uint64_t* ct, uint32_t nq, const uint64_t* key,
            uint32_t galois);
// Rotations of `count` different ciphertexts cts[r] [2][nq][N] by keys[r]:
// batched ModUps and batched ModDowns.  outs[r] must not alias any cts[.].
void rotate_many(Context& c, uint64_t* const* outs, const uint64_t* const* cts, uint32_t nq,
                 const uint64_t* const* keys, const uint32_t* galois, uint32_t count);
// Relinearization of `count` tensors ct3s[r] [3][nq][N] by one key:
// outs[r] = (d0, d1) + KS(d2), batched ModUps and batched ModDowns.
// outs[r] must not alias any ct3s[.].
void relinearize_many(Context& c, uint64_t* const* outs, const uint64_t* const* ct3s,
                      uint32_t nq, const uint64_t* key, uint32_t count);
// Baby-step giant-step plaintext linear transform of ct [2][nq][N]:
//   out = sum_{g < G} rot_giant^g( sum_{b < bstep} pts[g*bstep + b] (.) baby_b ),
// G = ceil(count / bstep), baby_b = ct rotated by baby_keys[b] (all babies
// from one ModUp; baby_keys[0] null: baby_0 = ct, otherwise it rotates ct by
// an offset that the other babies' keys include).  With one giant key
// (n_giant_keys = 1) the giant sum runs by Horner's rule; with one key per
// giant step (n_giant_keys = G - 1, giant_keys[g - 1] rotating by g giant
// strides) the G - 1 rotations run as one batch of independent key
// switches.  Null pts are skipped.  out may alias ct.
void linear_transform(Context& c, uint64_t* out, const uint64_t* ct, uint32_t nq,
                      const uint64_t* const* pts, uint32_t count, uint32_t bstep,
                      const uint64_t* const* baby_keys, const uint32_t* baby_galois,
                      const uint64_t* const* giant_keys, const uint32_t* giant_galois,
                      uint32_t n_giant_keys);
// The same transform (diagonals and keys) of ncts ciphertexts cts[i]
// [2][nq][N] into outs[i], in step: one batched ModUp of every
// ciphertext's c1 for the babies, their key switches in shared batches, and
// the giant-step rotations of all of them as one set of key switches (or,
// by Horner's rule, one batched ModUp and key-switch set per step).  The
// outputs are those of ncts linear_transform calls; outs[i] are distinct
// and may alias any cts[j] (every input is read before any output is
// written).
void linear_transform_many(Context& c, uint64_t* const* outs, const uint64_t* const* cts,
                           uint32_t ncts, uint32_t nq, const uint64_t* const* pts,
                           uint32_t count, uint32_t bstep, const uint64_t* const* baby_keys,
                           const uint32_t* baby_galois, const uint64_t* const* giant_keys,
                           const uint32_t* giant_galois, uint32_t n_giant_keys);
// g^-1 mod 2N for an odd Galois element g < 2N.
uint32_t galois_inverse(uint32_t g, uint32_t n);
// Galois permutation X -> X^galois of evaluation-form limbs.
void automorph(Context& c, uint64_t* out, const uint64_t* in, uint32_t npoly, uint32_t nlimb,
               uint32_t galois);
// Convert a standard-form key [dnum][2][L+K][N] to Montgomery form in place.
void key_to_montgomery(Context& c, uint64_t* key);
// The inverse: a device key back to standard form, written to `out`.
void key_from_montgomery(Context& c, uint64_t* out, const uint64_t* key);

// ---- encoding (encode.hip) ----
// Returns false if a scaled coefficient does not fit.
bool encode(Context& c, const double* re, const double* im, uint32_t count, uint32_t slots,
            double scale, uint32_t nlimb, uint64_t* out);
// nvec vectors of `count` values each (row r at re + r * count), one
// [nlimb][N] output per vector; the same result as nvec encode calls.
bool encode_many(Context& c, const double* re, const double* im, uint32_t count, uint32_t nvec,
                 uint32_t slots, double scale, uint32_t nlimb, uint64_t* const* outs);
void decode(Context& c, const uint64_t* pt, uint32_t nlimb, uint32_t slots, double scale,
            double* re, double* im);

// ---- key material (keygen.hip) ----
void sample_secret_host(Context& c, uint64_t seed, int64_t* out);
void sample_sparse_secret_host(Context& c, uint64_t seed, int64_t* out, uint32_t h);
void signed_to_eval(Context& c, const int64_t* coef_host, uint32_t idx0, uint32_t nlimb,
                    uint64_t* out);
void keygen_public(Context& c, const int64_t* s_coef, uint64_t seed, uint64_t* pk);
void keygen_switch(Context& c, const uint64_t* s_old, const uint64_t* s_new, uint64_t seed,
                   uint64_t tag, uint64_t* key);
void keygen_relin(Context& c, const int64_t* s_coef, uint64_t seed, uint64_t* key);
void keygen_galois(Context& c, const int64_t* s_coef, uint32_t galois, uint64_t seed,
                   uint64_t* key);
void encrypt_pk(Context& c, const uint64_t* pk, const uint64_t* m, uint32_t nq, uint64_t seed,
                uint64_t* ct);
void decrypt(Context& c, const uint64_t* ct, uint32_t npoly, uint32_t nq, const int64_t* s_coef,
             uint64_t* m);

}  // namespace fhe
