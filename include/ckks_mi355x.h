/*
 * ckks_mi355x.h -- C ABI of the MI355X (gfx950) RNS-CKKS evaluation backend.
 *
 * This is the drop-in boundary for the reference's backend: every entry point
 * below replaces one EasyFHE call that the reference's Python makes (cited as
 * reference file:line).  Handles are opaque; all functions return a status:
 *   CKKS_OK (0), CKKS_EINVAL (1, maps to Python ValueError),
 *   CKKS_ERUNTIME (2, RuntimeError), CKKS_ENOKEY (3, missing evaluation key,
 *   RuntimeError).
 * ckks_last_error() returns the calling thread's message for the last failure.
 *
 * Device work is asynchronous on one HIP stream per context; functions that
 * return host data (decrypt, decode, download) synchronise that stream.
 * Ciphertext limbs are uint64 residues in the NTT domain, layout
 * [polys][limbs][N]; an extended (QP-basis) object carries limbs + alpha
 * limbs per polynomial.  Ownership: every handle returned is owned by the
 * caller and released with its *_free function; no callee frees a handle it
 * was passed (reference llama3fhe/backend.py:336-351 release semantics).
 */
#ifndef CKKS_MI355X_H
#define CKKS_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CKKS_OK 0
#define CKKS_EINVAL 1
#define CKKS_ERUNTIME 2
#define CKKS_ENOKEY 3

typedef struct ckks_context ckks_context;
typedef struct ckks_ct ckks_ct; /* ciphertext or plaintext polynomial set */
typedef struct ckks_event ckks_event;
typedef struct ckks_tensor ckks_tensor; /* device-resident raw array (weights) */

/* Context parameters; fields follow fhe.CKKSContextSpec
 * (reference llama3fhe/application/session.py:31-45, backend.py:457-471). */
typedef struct {
  int log_n;          /* ring degree N = 2^log_n */
  int depth;          /* multiplicative depth; Q has depth + 1 limbs */
  int dnum;           /* key-switching digits over the full chain */
  int dcrt_bits;      /* bit size of q_1 .. q_depth */
  int first_mod;      /* bit size of q_0 */
  int special_bits;   /* bit size of the special primes (<= 60) */
  int secret_mode;    /* 0 sparse ternary (SPARSE_TERNARY), 1 uniform ternary */
  int hamming_weight; /* sparse secret weight */
  uint64_t seed;      /* seed of the key / encryption PRNG streams */
} ckks_params;

typedef struct {
  int N, log_n, L, alpha, digit_size, dnum, max_slots;
  double default_scale;
} ckks_context_info;

typedef struct {
  int polys, limbs, is_ext, slots, scale_degree;
  double scale;
} ckks_ct_info;

const char *ckks_last_error(void);

/* fhe.generate_client_context (reference application/session.py:31-45). */
int ckks_context_create(const ckks_params *params, ckks_context **out);
void ckks_context_destroy(ckks_context *ctx);
int ckks_context_info_get(const ckks_context *ctx, ckks_context_info *out);
/* Prime chain q_0..q_{L-1}, p_0..p_{alpha-1}. */
int ckks_context_primes(const ckks_context *ctx, uint64_t *out);
/* Secret coefficients (client side). */
int ckks_context_secret(const ckks_context *ctx, int8_t *out);
/* Native-context scale_at(limbs) / rescale_divisor_at(limbs)
 * (reference backend.py:228, operators/nonlinear/polynomial.py:59). */
double ckks_scale_at(const ckks_context *ctx, int limbs);
double ckks_rescale_divisor_at(const ckks_context *ctx, int limbs);
/* Galois element for a rotation index (2N-1 requests conjugation). */
uint64_t ckks_galois_element(const ckks_context *ctx, int64_t rotation);

/* Key generation for the CKKSContextSpec rotation list
 * (reference application/session.py:41, backend.py:469). */
int ckks_keygen_rotations(ckks_context *ctx, const int64_t *rotations, int n);
int ckks_keygen_relin(ckks_context *ctx);
int ckks_has_rotation_key(const ckks_context *ctx, int64_t rotation);
/* Evaluation key in normal form, [digits][2][L+alpha][N]; returns digits
 * through *digits.  Pass out = NULL to query the size. */
int ckks_key_download(ckks_context *ctx, uint64_t galois, uint64_t *out,
                      int *digits);
/* Drop cached keys except the listed rotations (native-context
 * clear_cuda_rotation_cache, reference operators/nonlinear/bootstrap.py:206). */
int ckks_clear_rotation_keys(ckks_context *ctx, const int64_t *keep, int n);
int ckks_synchronize(ckks_context *ctx);
/* Bytes currently held by the context's device pool (live + cached). */
int ckks_memory_info(ckks_context *ctx, size_t *live, size_t *cached);
/* Pool counters: the most bytes live at once, device memory held by the
 * pool's segments, and the device allocations made so far (the peak the
 * reference samples from torch's allocator, application/client.py:177-200). */
int ckks_memory_stats(ckks_context *ctx, size_t *peak_live, size_t *segment_bytes,
                      uint64_t *device_allocs);
int ckks_empty_cache(ckks_context *ctx);

/* client.encrypt / client.decrypt (reference backend.py:221-229,305-313,
 * application/session.py:71-77).  enc_id selects the encryption randomness
 * stream; im may be NULL. */
int ckks_encrypt(ckks_context *ctx, const double *re, const double *im,
                 int slots, int limbs, double scale, uint32_t enc_id,
                 ckks_ct **out);
int ckks_decrypt(ckks_context *ctx, const ckks_ct *ct, double *re, double *im);
/* ConstantBundle.plaintext encode of `rows` vectors of `slots` complex values
 * (reference operators/linear/weight.py:322-366, backend.py:274-297);
 * outputs one plaintext per row. */
int ckks_encode_rows(ckks_context *ctx, const double *re, const double *im,
                     int rows, int slots, int limbs, double scale, int is_ext,
                     ckks_ct **out);
/* fhe.encode_scalar (reference operators/nonlinear/polynomial.py:40-67):
 * round(value * scale) per limb; integer mode when scale == 1. */
int ckks_encode_scalar(ckks_context *ctx, double value, int limbs, double scale,
                       ckks_ct **out);
int ckks_decode(ckks_context *ctx, const ckks_ct *pt, double *re, double *im);

/* Raw transfer (parity tests and batch plumbing). */
int ckks_ct_upload(ckks_context *ctx, const uint64_t *data, int polys,
                   int limbs, int is_ext, int slots, double scale,
                   int scale_degree, ckks_ct **out);
int ckks_ct_download(ckks_context *ctx, const ckks_ct *ct, uint64_t *out);
int ckks_ct_info_get(const ckks_ct *ct, ckks_ct_info *out);
int ckks_ct_set_scale(ckks_ct *ct, double scale, int scale_degree);
int ckks_ct_copy(ckks_context *ctx, const ckks_ct *ct, ckks_ct **out);
void ckks_ct_free(ckks_ct *ct);

/* Limb-wise arithmetic: homo_add / homo_sub / homo_add_pt / homo_mul_pt /
 * homo_mul_i / homo_add_scalar / homo_mul_scalar (reference
 * operators/primitives.py:43,56,72; operators/linear/complex.py:21;
 * operators/nonlinear/polynomial.py:73,82). */
int ckks_add(ckks_context *ctx, const ckks_ct *a, const ckks_ct *b, ckks_ct **out);
int ckks_sub(ckks_context *ctx, const ckks_ct *a, const ckks_ct *b, ckks_ct **out);
/* out[i] = a[i] + b[i] (op 0) or a[i] - b[i] (op 1) for n pairs of one shape in
 * batched launches (the reference's list comprehensions over homo_add /
 * homo_sub, e.g. operators/linear/operator.py's per-chunk accumulation). */
int ckks_add_many(ckks_context *ctx, const ckks_ct *const *a, const ckks_ct *const *b, int n,
                  int op, ckks_ct **out);
int ckks_add_pt(ckks_context *ctx, const ckks_ct *a, const ckks_ct *pt, ckks_ct **out);
int ckks_mul_pt(ckks_context *ctx, const ckks_ct *a, const ckks_ct *pt, ckks_ct **out);
int ckks_mul_i(ckks_context *ctx, const ckks_ct *a, int negative, ckks_ct **out);
int ckks_add_scalar(ckks_context *ctx, const ckks_ct *a, const ckks_ct *s, ckks_ct **out);
int ckks_mul_scalar(ckks_context *ctx, const ckks_ct *a, const ckks_ct *s, ckks_ct **out);
/* homo_mul_no_relin / homo_relinearize / homo_mul_relin (reference
 * operators/attention/qk.py:399, kernel_helpers.py:155, primitives.py:25). */
int ckks_mul_no_relin(ckks_context *ctx, const ckks_ct *a, const ckks_ct *b, ckks_ct **out);
int ckks_relinearize(ckks_context *ctx, const ckks_ct *a, ckks_ct **out);
int ckks_mul_relin(ckks_context *ctx, const ckks_ct *a, const ckks_ct *b, ckks_ct **out);
/* fhe.rescale / fhe.align_to as a limb drop (reference
 * operators/linear/operator.py:386, primitives.py:145). */
int ckks_rescale(ckks_context *ctx, const ckks_ct *a, ckks_ct **out);
int ckks_drop_limbs(ckks_context *ctx, const ckks_ct *a, int target_limbs, ckks_ct **out);
/* Bootstrap ModRaise: a one-limb ciphertext (mod q_0) lifted with centered
 * coefficients to target_limbs limbs; the plaintext becomes m + q_0 I
 * (reference bs.bootstrap, operators/nonlinear/bootstrap.py:370, "modraise_first"
 * mode, bootstrap.py:29). */
int ckks_mod_raise(ckks_context *ctx, const ckks_ct *a, int target_limbs, ckks_ct **out);
/* fhe.homo_rotate (reference operators/linear/operator.py:333,
 * operators/linear/complex.py:47). */
int ckks_rotate(ckks_context *ctx, const ckks_ct *a, int64_t rotation, ckks_ct **out);
/* Batched key switching: one rotation index applied to n ciphertexts at one
 * level; the rotation key is streamed from HBM once per call (the keyswitch
 * hot path under homo_rotate). */
int ckks_rotate_many(ckks_context *ctx, const ckks_ct *const *in, int n,
                     int64_t rotation, ckks_ct **out);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * ckks_rotate_many into caller-provided outputs: out[i] must be an existing
 * degree-1 Q-basis ciphertext at the inputs' level, distinct from every
 * input; its limbs, scale and slot count are overwritten.  Every
 * intermediate lives in one fixed 256 MiB device buffer per GPU; nothing is
 * allocated or freed.  CKKS_EINVAL when the call needs more scratch than
 * that (at N = 2^16 with 36 + 12 limbs and dnum 3 one ciphertext takes
 * 186 MiB) or when the rotation keys (whose generation also builds every
 * level's constants) are missing.  Calls on one GPU (contexts on other
 * streams or threads) are ordered on the device: each call's stream waits
 * for the previous call's work (an event, no host wait), so they use the
 * buffer one after another.  Outputs' scale and slot count are written after
 * the rotation is enqueued. */
int ckks_rotate_many_noalloc(ckks_context *ctx, const ckks_ct *const *in, int n,
                             int64_t rotation, ckks_ct *const *out);
/* homo_mul_relin + rescale for n pairs (config: HMult+relin+rescale). */
int ckks_mul_relin_rescale_many(ckks_context *ctx, const ckks_ct *const *a,
                                const ckks_ct *const *b, int n, ckks_ct **out);
/* ckks_mul_relin_rescale_many followed by `primes` - 1 more rescales (1..4
 * primes in all; the step of a multi-prime level, reference
 * operators/nonlinear/polynomial.py:115-203): one key switch whose ModDown
 * divides by P and the dropped primes at once, with the words of the
 * separate steps. */
int ckks_mul_relin_rescale_many_by(ckks_context *ctx, const ckks_ct *const *a,
                                   const ckks_ct *const *b, int n, int primes, ckks_ct **out);
/* homo_mul_relin_rescale_postop for n pairs (reference
 * operators/nonlinear/polynomial.py:115-203, the Chebyshev basis steps
 * 2 T_i T_j - T_1 and 2 T_i T_j - 1):
 *   out_i = (apply_double ? 2 : 1) rescale(relin(a_i b_i)) - sub_i + scalar
 * with sub (n degree-1 ciphertexts of one limb count at or above the output
 * level, their leading limbs used) and scalar (encode_scalar at or above the
 * output level, added to component 0) each optional (NULL).  The ModDown by
 * P q_l of the relinearise-rescale applies the postop in its epilogue, so
 * the words equal those of the separate calls. */
int ckks_mul_relin_rescale_postop_many(ckks_context *ctx, const ckks_ct *const *a,
                                       const ckks_ct *const *b, int n, int apply_double,
                                       const ckks_ct *const *sub, const ckks_ct *scalar,
                                       ckks_ct **out);
/* fhe.prepare_hoisted_baby_rotations (reference operators/linear/operator.py:105):
 * one ModUp of c1 shared by all rotations. */
int ckks_hoisted_rotate(ckks_context *ctx, const ckks_ct *a,
                        const int64_t *rotations, int n, ckks_ct **out);
/* fhe.hoisted_mac_sum, strategy "normal" (reference
 * operators/linear/operator.py:320-330, operators/transform.py:108-116):
 * sum_g rot(giant)^g (sum_b pt[g B + b] * baby_b); babies as returned by
 * ckks_hoisted_rotate for the baby offsets; result unrescaled. */
int ckks_hoisted_mac_sum(ckks_context *ctx, const ckks_ct *const *babies, int B,
                         const ckks_ct *const *pts, int64_t giant_rotation,
                         int giant_count, ckks_ct **out);

/* fhe.prepare_hoisted_baby_rotations for m ciphertexts at one level (every
 * input of a linear, reference operators/linear/operator.py:100-117): one
 * batched ModUp, then each rotation's key is read once for all m;
 * out[i * n + r] = rot_{rotations[r]}(a[i]). */
int ckks_hoisted_rotate_many(ckks_context *ctx, const ckks_ct *const *a, int m,
                             const int64_t *rotations, int n, ckks_ct **out);
/* fhe.hoisted_mac_sum with precomputed babies for n ciphertexts sharing the
 * plaintexts (reference operators/linear/operator.py:320-330 for every input
 * of one chunk): baby b of ciphertext i at babies[i * B + b], plaintexts
 * pts[g * B + b]; out[i] = Horner over the giant key of sum_b pt (.) baby,
 * unrescaled.  Each baby word is read once per pass of up to 8 giant groups
 * and each plaintext word once per pass for all n (L2 re-reads aside).
 * Requires (n + min(giant_count, 8)) * B <= 8192. */
int ckks_hoisted_mac_sum_many(ckks_context *ctx, const ckks_ct *const *babies, int n, int B,
                              const ckks_ct *const *pts, int64_t giant_rotation,
                              int giant_count, ckks_ct **out);
/* fhe.hoisted_mac_sum, strategy "ext_normal" (reference
 * operators/linear/operator.py:320-330, linear/config.py:296-305): the babies
 * of `a` for baby_rotations stay in the Q u P basis (no ModDown), the
 * plaintexts are extended (is_ext, at a's level), and each giant group is
 * brought back to Q by one ModDown before the Horner chain over the giant key;
 * result unrescaled. */
int ckks_hoisted_mac_sum_ext(ckks_context *ctx, const ckks_ct *a, const int64_t *baby_rotations,
                             int B, const ckks_ct *const *pts, int64_t giant_rotation,
                             int giant_count, ckks_ct **out);
/* ckks_hoisted_mac_sum_ext for n ciphertexts at one level sharing the
 * plaintexts (bootstrap linear levels over a batch): one batched ModUp, each
 * baby key read once for all n, batched ModDowns and giant rotations. */
int ckks_hoisted_mac_sum_ext_many(ckks_context *ctx, const ckks_ct *const *a, int n,
                                  const int64_t *baby_rotations, int B,
                                  const ckks_ct *const *pts, int64_t giant_rotation,
                                  int giant_count, ckks_ct **out);
/* fhe.hoisted_mac_sum, strategy "ext_double_hoist" (reference
 * operators/linear/config.py:296-305, operators/linear/operator.py:320-330):
 * babies and plaintexts as in ckks_hoisted_mac_sum_ext; every giant group
 * g >= 1 is rotated by g * giant_rotation in the Q u P basis with its own key
 * (ModDown of its second component only, ModUp, key product, sigma of its
 * first component added), the groups are summed there and one ModDown ends
 * it; result unrescaled.  Needs the keys of g * giant_rotation, g = 1 ..
 * giant_count - 1 (the reference's key set for this strategy,
 * linear/config.py:296-305). */
int ckks_hoisted_mac_sum_double(ckks_context *ctx, const ckks_ct *a,
                                const int64_t *baby_rotations, int B, const ckks_ct *const *pts,
                                int64_t giant_rotation, int giant_count, ckks_ct **out);
/* ckks_hoisted_mac_sum_double for n <= 64 ciphertexts at one level sharing
 * the plaintexts: one batched ModUp for the babies, each key read once for
 * all n. */
int ckks_hoisted_mac_sum_double_many(ckks_context *ctx, const ckks_ct *const *a, int n,
                                     const int64_t *baby_rotations, int B,
                                     const ckks_ct *const *pts, int64_t giant_rotation,
                                     int giant_count, ckks_ct **out);
/* Linear combination in one launch for n ciphertexts (the many small
 * homo_mul_scalar / homo_add launches of a polynomial's leaf sums, reference
 * operators/nonlinear/polynomial.py:182-199):
 *   out_i = sum_t rint(weights[t]) terms[t*n + i] + rint(constant) (on c0),
 * over the first `limbs` limbs of every term; weights are already multiplied
 * by their encoding scales; the outputs carry (scale, scale_degree). */
int ckks_linear_combination(ckks_context *ctx, const ckks_ct *const *terms, int T, int n,
                            const double *weights, double constant, int limbs, double scale,
                            int scale_degree, ckks_ct **out);
/* fhe.grouped_pairwise_mac (reference operators/attention/input.py:814-826,
 * 1274-1286, 1322-1334): terms[t] times plaintext pts[t], summed per group
 * (group g takes the next group_sizes[g] terms, 1 to 64 of them), unrescaled,
 * in one launch per group that reads each word once.  All terms share one
 * level and basis (Q, or Q u P with extended plaintexts at that level; a
 * Q-basis term takes a plaintext's leading limbs) and, with their
 * plaintexts, one scale; out[g] at scale terms' x plaintexts'.  The words
 * equal those of ckks_mul_pt then ckks_add over the group. */
int ckks_grouped_mac(ckks_context *ctx, const ckks_ct *const *terms, const ckks_ct *const *pts,
                     const int *group_sizes, int n_groups, ckks_ct **out);
/* fhe.rescale for n ciphertexts of one shape in batched launches. */
int ckks_rescale_many(ckks_context *ctx, const ckks_ct *const *a, int n, ckks_ct **out);
/* `primes` rescales in a row (1..4) of each of n ciphertexts of one shape, as
 * one inverse NTT of the dropped limbs, one combined lift and one forward NTT
 * (reference: the repeated fhe.rescale of a multi-prime level step,
 * operators/nonlinear/polynomial.py:182, operators/linear/operator.py:386);
 * the words equal those of `primes` calls of ckks_rescale. */
int ckks_rescale_many_by(ckks_context *ctx, const ckks_ct *const *a, int n, int primes,
                         ckks_ct **out);
/* fhe.fast_rotate(..., output_ext=True) (reference attention/input.py:792-826):
 * hoisted rotations left in the Q u P basis, i.e. P rot_k(a) before ModDown;
 * the outputs are extended ciphertexts at a's scale. */
int ckks_hoisted_rotate_ext(ckks_context *ctx, const ckks_ct *a, const int64_t *rotations, int n,
                            ckks_ct **out);
/* fhe.moddown_from_ext (reference attention/input.py:1103-1169): an extended
 * ciphertext divided by P (centered conversion) back to the Q basis. */
int ckks_moddown_ext(ckks_context *ctx, const ckks_ct *a, ckks_ct **out);

/* Device-resident weights for the diagonal packers (the reference keeps them
 * on the GPU as EasyFHE tensors, operators/linear/gpu_packer.py:79-97). */
int ckks_tensor_upload(ckks_context *ctx, const void *data, size_t bytes, ckks_tensor **out);
int ckks_tensor_download(ckks_context *ctx, const ckks_tensor *t, void *out, size_t bytes);
void ckks_tensor_free(ckks_tensor *t);
/* Feature-major BSGS diagonals of a device weight W [D][D] (dtype 0 float64,
 * 1 float32, 2 complex128), encoded at (limbs, scale[, P limbs]):
 *   row(g, b)[slot] = W[(slot / lanes - (giant_base + g) B) mod D, (slot / lanes + b) mod D]
 * for g < giant_count, b < B, as giant_count * B plaintexts.  The gather feeds
 * the encoder directly (reference pack_token_lane_bsgs_weight_chunk_triton_gpu,
 * operators/linear/gpu_packer.py:49-177, then ConstantBundle.plaintext). */
int ckks_encode_token_lane(ckks_context *ctx, const ckks_tensor *weight, int dtype, int dimension,
                           int token_lanes, int baby_steps, int giant_base, int giant_count,
                           int slots, int limbs, double scale, int is_ext, ckks_ct **out);
/* The same diagonals of a structured physical matrix
 *   W[o, i] = column_scale[i] (real_scale[o] src[real_source[o]][real_row[o], column[i]]
 *             + 1j imag_scale[o] src[imag_source[o]][imag_row[o], column[i]])
 * (index -1 = zero padding) over 1..3 real sources (fp32 != 0: float32, else
 * float64) with shapes [n][2] and element strides [n][2]; index_maps holds
 * real_source, real_row, imag_source, imag_row, column ([5][dimension] host
 * int64), scale_maps real_scale, imag_scale, column_scale ([3][dimension] host
 * double).  Every index is checked against the shapes before the device gather
 * (reference pack_structured_token_lane_bsgs_weight_chunk_triton_gpu,
 * operators/linear/gpu_packer.py:180-424, structured_weight.py:1-20). */
int ckks_encode_structured(ckks_context *ctx, const ckks_tensor *const *sources, int n_sources,
                           int fp32, const int64_t *shapes, const int64_t *strides,
                           const int64_t *index_maps, const double *scale_maps, int dimension,
                           int token_lanes, int baby_steps, int giant_base, int giant_count,
                           int slots, int limbs, double scale, int is_ext, ckks_ct **out);

/* Raw polynomial transforms over host buffers [n_polys][limbs][N] with limb i
 * in prime i (i < q_limbs) or special prime i - q_limbs (parity tests). */
int ckks_poly_ntt(ckks_context *ctx, const uint64_t *in, uint64_t *out,
                  int n_polys, int limbs, int q_limbs, int inverse);
/* ModUp / ModDown of host buffers (parity of the key-switch stages). */
int ckks_poly_modup(ckks_context *ctx, const uint64_t *d, int limbs, uint64_t *ext);
int ckks_poly_moddown(ckks_context *ctx, const uint64_t *acc, int limbs, uint64_t *out);
/* NTT (inverse = 0) or iNTT (inverse = 1) in place over all polynomials of n
 * resident ciphertexts: the kernel pair that bench.py times. */
int ckks_ntt_many(ckks_context *ctx, ckks_ct *const *cts, int n, int inverse);

/* No counterpart in the reference: the register-only throughput probe that
 * the measurements divide kernel operation rates by.  kind 0: the fp64-path
 * modular product of limbs below 2^45 (the basis conversions' and MACs'
 * inner operation), 1: the 64-bit Shoup modular product, 2: fp64 FMA;
 * *ops_per_second receives the device-wide rate. */
int ckks_int_peak(ckks_context *ctx, int kind, double *ops_per_second);

/* Per-kernel timing, the kernel-level counterpart of the reference's device-
 * event stage timing (operators/linear/operator.py:272-291): with enable 1
 * the library records HIP events on the context stream around each launch of
 * its key kernels (NTT passes, basis conversions, key inner products, MACs,
 * tensor, rescale, limb-wise sums); ckks_profile_read synchronises the
 * stream and writes one line per kernel group recorded since the last read,
 *   "<name> <launches> <milliseconds> <algorithmic bytes> <modular ops>\n",
 * into buf (NUL-terminated, truncated to len), then clears the records.
 * Algorithmic bytes count each input word read once and each output word
 * written once. */
int ckks_profile_enable(ckks_context *ctx, int enable);
int ckks_profile_read(ckks_context *ctx, char *buf, size_t len);

/* Device events on the context stream (reference easyfhe.cuda.Event,
 * operators/linear/operator.py:273-291). */
int ckks_event_create(ckks_context *ctx, ckks_event **out);
int ckks_event_record(ckks_event *ev);
int ckks_event_elapsed_ms(ckks_event *start, ckks_event *end, float *ms);
void ckks_event_destroy(ckks_event *ev);

/* Streams a batched key switch of at least 16 ciphertexts is split over
 * (1 .. the count set at creation by CKKS_SPLIT_STREAMS, default 3); no
 * counterpart in the reference, whose library runs one stream.  1 gives the
 * one-stream order per-kernel timings need; 0 restores the creation count. */
int ckks_set_split_parts(ckks_context *ctx, int parts);

/* The operation audit of the reference's graph audit (graph.py:348
 * operation_audit), for the roofline of a whole program: out[0] key switches
 * issued, out[1] their ciphertext bytes (a key switch's input read once per
 * ModUp, each output written once: 4 l limb-polynomials for a plain one at l
 * limbs), out[2] their key bytes (each key read once per batched launch),
 * out[3] plaintext bytes of the MACs and plaintext products (each plaintext
 * limb once per launch), out[4] rescale bytes (input and output once), all
 * since the last call with reset != 0. */
int ckks_audit_read(ckks_context *ctx, double *out, int reset);

/* The context's HIP stream as an opaque handle (hipStream_t), for callers
 * that order their own launches with the library's work (the reference's
 * Triton bridge reads torch.cuda.current_stream(idx).cuda_stream,
 * operators/linear/gpu_packer.py:35-45). */
int ckks_context_stream(ckks_context *ctx, void **stream);

#ifdef __cplusplus
}
#endif
#endif
