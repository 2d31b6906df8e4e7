/*
 * ckks_oracle.h -- CPU restatement of the RNS-CKKS evaluation path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the MI355X
 * kernels are compared against; it is loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by nothing
 * in the product path.
 *
 * The reference delegates all homomorphic arithmetic to the third-party
 * EasyFHE library, which is not vendored (reference docs/SETUP.md:15-34,
 * NOTICE:7-13) and has no pinned version.  What is restated here is the
 * published RNS-CKKS algorithm behind the call sites the reference makes
 * (llama3fhe/backend.py:177-313, operators/primitives.py:21-190,
 * operators/linear/operator.py:195-436, operators/linear/weight.py:18-47):
 *   - Cheon-Han-Kim-Kim-Song full-RNS CKKS with hybrid key switching
 *     (Han-Ki 2020, "Better bootstrapping for approximate HE", sec. 3),
 *   - negacyclic NTT in the Longa-Naehrig bit-reversed layout,
 *   - fast basis conversion (Bajard et al. 2016) for ModUp / ModDown,
 *   - canonical-embedding encoding (CKKS 2017, sec. 3.1).
 * The choices EasyFHE would pin but cannot be read here (prime selection,
 * PRNG, error distribution, secret Hamming weight, encoder rounding) are
 * fixed in this file and documented at their definition.
 *
 * Every value array is uint64 with canonical residues in [0, q).
 * A polynomial over `ell` limbs is stored limb-major: limb i at [i*N, (i+1)*N).
 * A ciphertext of degree d (2 or 3 polynomials) is [d][ell][N].
 */
#ifndef CKKS_ORACLE_H
#define CKKS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_ctx orc_ctx;

/* --- number theory ------------------------------------------------------ */
uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q);
uint64_t orc_powmod(uint64_t a, uint64_t e, uint64_t q);
int orc_is_prime(uint64_t n);
/* Primes q = 1 (mod 2N) ordered by distance from 2^bits (below first), all
 * below 2^60, skipping the `n_used` values in `used`.  Returns count found. */
int orc_gen_primes(int logN, int bits, int count, const uint64_t *used,
                   int n_used, uint64_t *out);
/* Smallest primitive 2N-th root of unity mod q. */
uint64_t orc_min_root(uint64_t q, int logN);

/* --- ChaCha20 (RFC 8439 block function) as a counter-based PRNG --------- */
void orc_chacha20_block(const uint32_t key[8], uint32_t counter,
                        const uint32_t nonce[3], uint32_t out[16]);
void orc_prng_block(uint64_t seed, uint32_t domain, uint32_t id, uint32_t sub,
                    uint32_t counter, uint32_t out[16]);

/* --- context ------------------------------------------------------------ */
/* secret_mode: 0 = sparse ternary with Hamming weight h, 1 = uniform ternary */
orc_ctx *orc_ctx_create(int logN, int L, int alpha, int dnum, int first_bits,
                        int dcrt_bits, int special_bits, uint64_t seed,
                        int secret_mode, int h);
void orc_ctx_free(orc_ctx *c);
void orc_set_threads(int n);
int orc_N(const orc_ctx *c);
int orc_L(const orc_ctx *c);
int orc_alpha(const orc_ctx *c);
int orc_digit_size(const orc_ctx *c);
void orc_primes(const orc_ctx *c, uint64_t *out); /* L + alpha values */
void orc_secret(const orc_ctx *c, int8_t *out);   /* N coefficients */
const uint64_t *orc_psi_br(const orc_ctx *c, int prime_idx);

/* --- NTT ----------------------------------------------------------------- */
void orc_ntt_fwd(const orc_ctx *c, int prime_idx, uint64_t *a);
void orc_ntt_inv(const orc_ctx *c, int prime_idx, uint64_t *a);
/* Apply to `ell` limbs starting at prime index 0, except that limb i >= q_limbs
 * uses special prime i - q_limbs (extended basis Q_ell u P). */
void orc_ntt_fwd_limbs(const orc_ctx *c, uint64_t *a, int limbs, int q_limbs);
void orc_ntt_inv_limbs(const orc_ctx *c, uint64_t *a, int limbs, int q_limbs);

/* --- automorphism X -> X^g ---------------------------------------------- */
void orc_automorphism_coeff(const orc_ctx *c, int prime_idx, uint64_t g,
                            const uint64_t *in, uint64_t *out);
void orc_automorphism_ntt(const orc_ctx *c, uint64_t g, const uint64_t *in,
                          uint64_t *out, int limbs);
uint64_t orc_galois_elt(const orc_ctx *c, int64_t rotation);

/* --- encoding ------------------------------------------------------------ */
/* cos, sin of 2 pi j / n from IEEE basic operations only. */
void orc_unit_root(long long j, long long n, double *cs, double *sn);
/* Encode `slots` complex values at `scale` into an NTT-domain plaintext over
 * `limbs` Q limbs (plus alpha P limbs when is_ext). */
int orc_encode(const orc_ctx *c, const double *re, const double *im, int slots,
               double scale, int limbs, int is_ext, uint64_t *out);
/* Coefficient-domain integer encode (before reduction): out[N] as doubles
 * (rounded values, exact integers). */
void orc_encode_coeffs(const orc_ctx *c, const double *re, const double *im,
                       int slots, double scale, double *out);
/* Decode an NTT-domain polynomial over `limbs` Q limbs. */
void orc_decode(const orc_ctx *c, const uint64_t *poly, int limbs, int slots,
                double scale, double *re, double *im);

/* --- keys --------------------------------------------------------------- */
int orc_gen_rotation_key(orc_ctx *c, uint64_t g);
int orc_gen_relin_key(orc_ctx *c);
/* Export a key: [digits][2][L+alpha][N] (b then a). Returns digits or -1. */
int orc_get_key(const orc_ctx *c, uint64_t g, uint64_t *out);

/* --- encryption ----------------------------------------------------------- */
int orc_encrypt(const orc_ctx *c, const double *re, const double *im,
                int slots, double scale, int limbs, uint32_t enc_id,
                uint64_t *ct);
void orc_decrypt_poly(const orc_ctx *c, const uint64_t *ct, int degree,
                      int limbs, uint64_t *out);
void orc_decrypt(const orc_ctx *c, const uint64_t *ct, int degree, int limbs,
                 int slots, double scale, double *re, double *im);

/* --- evaluation ----------------------------------------------------------- */
void orc_add(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
             uint64_t *out, int polys, int limbs);
void orc_sub(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
             uint64_t *out, int polys, int limbs);
void orc_mul_pt(const orc_ctx *c, const uint64_t *ct, const uint64_t *pt,
                uint64_t *out, int limbs);
void orc_mul_monomial_half(const orc_ctx *c, const uint64_t *ct, uint64_t *out,
                           int polys, int limbs, int negative);
void orc_tensor(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
                uint64_t *out3, int limbs);
void orc_modup(const orc_ctx *c, const uint64_t *d, int limbs, uint64_t *ext);
void orc_moddown(const orc_ctx *c, const uint64_t *acc, int limbs,
                 uint64_t *out);
int orc_keyswitch(const orc_ctx *c, uint64_t g, const uint64_t *d, int limbs,
                  uint64_t *out0, uint64_t *out1);
int orc_relinearize(const orc_ctx *c, const uint64_t *ct3, int limbs,
                    uint64_t *out);
int orc_rotate(const orc_ctx *c, const uint64_t *ct, int limbs, uint64_t g,
               uint64_t *out);
int orc_hoisted_rotate(const orc_ctx *c, const uint64_t *ct, int limbs,
                       const uint64_t *gs, int n, uint64_t *outs);
void orc_rescale(const orc_ctx *c, const uint64_t *ct, int polys, int limbs,
                 uint64_t *out);
int orc_hoisted_mac_sum_ext(const orc_ctx *c, const uint64_t *ct, int limbs,
                            const uint64_t *baby_gs, int B, const uint64_t *pts,
                            uint64_t giant_g, int G, uint64_t *out);
int orc_hoisted_mac_sum_double(const orc_ctx *c, const uint64_t *ct, int limbs,
                               const uint64_t *baby_gs, int B, const uint64_t *pts,
                               const uint64_t *giant_gs, int G, uint64_t *out);
void orc_mod_raise(const orc_ctx *c, const uint64_t *ct, int polys, int target,
                   uint64_t *out);
void orc_drop_limbs(const orc_ctx *c, const uint64_t *ct, int polys, int limbs,
                    int target, uint64_t *out);
int orc_hoisted_mac_sum(const orc_ctx *c, const uint64_t *ct, int limbs,
                        const uint64_t *baby_gs, int B, const uint64_t *pts,
                        uint64_t giant_g, int G, uint64_t *out);

#ifdef __cplusplus
}
#endif
#endif
