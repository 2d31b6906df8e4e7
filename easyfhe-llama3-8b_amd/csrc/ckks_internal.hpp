// ckks_internal.hpp -- shared definitions of the gfx950 RNS-CKKS backend.
//
// Word size: every residue is a uint64 in [0, q) with q < 2^60 (the prime
// rule keeps all primes below 2^60 so that sixteen residues sum below 2^64,
// which is the bound the lazy Montgomery accumulations below rely on).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ckks_mi355x.h"
#include "device_pool.hpp"

typedef uint64_t u64;
typedef uint32_t u32;

namespace ckks {

constexpr int kMaxBatch = 64;    // explicit pointers per kernel argument block
constexpr int kMaxDigitSize = 16;  // Montgomery fold bound: 16 * 2^60 <= 2^64
constexpr int kMaxDigits = 8;
constexpr int kMaxRescaleDrop = 4;  // primes one rescale call may divide by
constexpr int kMacGroups = 2;       // giant groups of one extended MAC pass
constexpr int kMacCts = 4;          // ciphertexts per plaintext read in that pass
constexpr int kMacCtsFp = 8;        // the same for its fp64 path
constexpr int kTabGroups = 16;      // giant groups of one Q-basis MAC pass (k_mac_table)
constexpr int kTabCts = 2;          // ciphertexts per plaintext read in that pass
constexpr int kTabCtsFp = 8;        // the same for its fp64 path
constexpr int kMultiItems = 4;    // items per multi-rotation key inner product launch

// Per-prime constants, resident in device memory.
struct ModQ {
  u64 q;
  u64 qinv;  // -q^-1 mod 2^64 (Montgomery)
  u64 r2;    // 2^128 mod q
  u64 mu;    // floor(2^(2k) / q) (Barrett)
  u32 k;     // bit length of q
  u32 pad;
};

// A set of polynomials addressed either by explicit pointers (p[i]) or by a
// base and a stride (base + i * stride) when base != nullptr.
struct Batch {
  u64 *p[kMaxBatch];
  u64 *base;
  u64 stride;
};

// An internal buffer of equally spaced items.
struct Strided {
  u64 *base;
  u64 stride;
};

// Epilogue of a relinearise-rescale ModDown (the fused Chebyshev step of
// homo_mul_relin_rescale_postop): the result r becomes
//   (dbl ? 2 r : r) - sub + scal   (scal on component 0 only)
// with sub per item at component 0 (null: none), its component 1 at
// sub + sub1_off, and scal one word per output limb (null: none).
struct PostOp {
  int dbl;
  Batch sub;
  u64 sub1_off;
  const u64 *scal;
};

__device__ __forceinline__ u64 *batch_ptr(const Batch &b, int i) {
  return b.base ? b.base + (u64)i * b.stride : b.p[i];
}

// item i of a batch on the host (null for an empty batch's item 0)
inline u64 *batch_ptr_host(const Batch &b, int i) {
  return b.base ? b.base + (u64)i * b.stride : b.p[i];
}

// Kernels that form a word-by-word product a x b on load: 2 when every item
// of b is the item of a (a square, read once), else 1
inline int product_mode(const Batch &a, const Batch &b, int n_items) {
  for (int i = 0; i < n_items; i++)
    if (batch_ptr_host(a, i) != batch_ptr_host(b, i)) return 1;
  return 2;
}

// ---------------------------------------------------------------------------
// modular arithmetic (device)
// ---------------------------------------------------------------------------

// v < m ? v : v - m, the choice taken from the subtraction's borrow (no
// separate 64-bit compare)
__device__ __forceinline__ u64 csub(u64 v, u64 m) {
  u64 r;
  return __builtin_sub_overflow(v, m, &r) ? v : r;
}

__device__ __forceinline__ u64 add_mod(u64 a, u64 b, u64 q) { return csub(a + b, q); }

__device__ __forceinline__ u64 sub_mod(u64 a, u64 b, u64 q) {
  u64 r;
  return __builtin_sub_overflow(a, b, &r) ? r + q : r;
}

// Shoup: a * w mod q with ws = floor(w 2^64 / q); a < 2^64, result in [0, q).
__device__ __forceinline__ u64 shoup_mul(u64 a, u64 w, u64 ws, u64 q) {
  u64 h = __umul64hi(a, ws);
  u64 r = a * w - h * q;
  return csub(r, q);
}

// (hi, lo) += a * b
__device__ __forceinline__ void mac_wide(u64 &hi, u64 &lo, u64 a, u64 b) {
  u64 l = a * b;
  u64 h = __umul64hi(a, b);
  lo += l;
  hi += h + (lo < l ? 1 : 0);
}

// Sums of products x w of words below 2^60 in 30-bit halves: x = x1 2^30 +
// x0, w = w1 2^30 + w0 (every half below 2^30), so x w = x0 w0 + (x0 w1 +
// x1 w0) 2^30 + x1 w1 2^60 and each partial product is below 2^60: four
// 64-bit sums hold 16 products without a carry, each term one 32 x 32 + 64
// multiply-add (v_mad_u64_u32).
struct Half30 {
  u32 lo, hi;
};
__device__ __forceinline__ Half30 half30(u64 x) {
  return Half30{(u32)x & 0x3fffffffu, (u32)(x >> 30)};
}
struct Sum30 {
  u64 s00, s01, s10, s11;
};
__device__ __forceinline__ void mac30(Sum30 &a, Half30 x, Half30 w) {
  a.s00 += (u64)x.lo * w.lo;
  a.s01 += (u64)x.lo * w.hi;
  a.s10 += (u64)x.hi * w.lo;
  a.s11 += (u64)x.hi * w.hi;
}
// the sum of the four partial sums as hi 2^64 + lo
__device__ __forceinline__ void sum30_wide(const Sum30 &a, u64 &hi, u64 &lo) {
  lo = a.s00;
  hi = 0;
  const u64 m = a.s01 + a.s10;  // may wrap: the carry is bit 64 of the middle sum
  const u64 mc = m < a.s01 ? 1 : 0;
  u64 t = m << 30;
  lo += t;
  hi += (m >> 34) + (mc << 30) + (lo < t ? 1 : 0);
  t = a.s11 << 60;
  lo += t;
  hi += (a.s11 >> 4) + (lo < t ? 1 : 0);
}
// hi 2^64 + lo plus the sum of a's partial sums (a second set of sums, for
// more than 16 products)
__device__ __forceinline__ void sum30_add_wide(const Sum30 &a, u64 &hi, u64 &lo) {
  u64 h, l;
  sum30_wide(a, h, l);
  lo += l;
  hi += h + (lo < l ? 1 : 0);
}

// Montgomery reduction of x = hi 2^64 + lo < q 2^64: x 2^-64 mod q in [0, q).
__device__ __forceinline__ u64 redc(u64 hi, u64 lo, u64 q, u64 qinv) {
  u64 m = lo * qinv;
  u64 t = hi + __umul64hi(m, q) + (lo != 0 ? 1 : 0);
  return csub(t, q);
}

// Barrett reduction of x = hi 2^64 + lo < q^2 (HAC 14.42 with radix 2).
__device__ __forceinline__ u64 barrett(u64 hi, u64 lo, const ModQ &M) {
  const u32 k = M.k;
  u64 xs = (hi << (65 - k)) | (lo >> (k - 1));
  u64 ph = __umul64hi(xs, M.mu), pl = xs * M.mu;
  u64 qh = (ph << (63 - k)) | (pl >> (k + 1));
  return csub(csub(lo - qh * M.q, M.q), M.q);
}

__device__ __forceinline__ u64 mul_mod(u64 a, u64 b, const ModQ &M) {
  return barrett(__umul64hi(a, b), a * b, M);
}

__device__ __forceinline__ u64 to_mont(u64 a, const ModQ &M) {
  return redc(__umul64hi(a, M.r2), a * M.r2, M.q, M.qinv);
}

// Index map of the automorphism X -> X^g in the bit-reversed NTT domain:
// out[i] = in[autom_index(i)].
__device__ __forceinline__ u32 autom_index(u32 i, u64 g, int logN) {
  u32 r = __brev(i) >> (32 - logN);
  u64 e = ((2 * (u64)r + 1) * g) & ((2ull << logN) - 1);
  return __brev((u32)((e - 1) >> 1)) >> (32 - logN);
}

// Storage slot of key position s (N >= 1024): within each group of 1024
// positions, bits 1-3 and 4-9 of s trade places (bit 0 stays), so that the
// 16 consecutive positions a thread of the fused low pass + key product reads
// (positions 16 c0 .. 16 c0 + 15 of row r, lane (r mod 4) 16 + c0) become 8
// pairs 128 words apart, and each pair's load is contiguous across the wave.
__host__ __device__ __forceinline__ u32 key_slot(u32 s) {
  return (s & ~1023u) | (s & 1u) | (((s >> 4) & 63u) << 1) | (((s >> 1) & 7u) << 7);
}

__device__ __forceinline__ int prime_of(int limb, int q_limbs, int L) {
  return limb < q_limbs ? limb : L + (limb - q_limbs);
}

// ---------------------------------------------------------------------------
// host-side structures
// ---------------------------------------------------------------------------

// Device memory of one context: exact-size free lists plus the set of live
// blocks, so that destroying the context returns everything it allocated.
// The HIP device behind the context's pool (device_pool.hpp).
struct HipDevice {
  static bool alloc(void **p, size_t bytes) {
    if (hipMalloc(p, bytes) == hipSuccess) return true;
    (void)hipGetLastError();
    return false;
  }
  static void release(void *p) { (void)hipFree(p); }
  static size_t free_bytes() {
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) != hipSuccess) {
      (void)hipGetLastError();
      return (size_t)-1;
    }
    return fr;
  }
  static void synchronize() { (void)hipDeviceSynchronize(); }
};
using Pool = BasicPool<HipDevice>;


struct DeviceKey {
  u64 galois;
  int digits;
  // [digits][2][K][N], Montgomery form; a rotation key by g holds the word
  // of NTT position k at position autom_index(k, g) (source order), and the
  // word of position s sits at slot key_slot(s) of its row
  u64 *data;
  size_t bytes;
};

struct BCTable {  // fast basis conversion constants, device resident
  int ns, nd;
  u64 *d;  // [ns] hinv, [ns] hinv_shoup, [ns*nd] hmod (Montgomery form), [nd] Q mod t
  size_t bytes;
  // every source prime below 2^45, or all but the first: fp64 table [ns]
  // (hinv, hinv / q_i), [ns*nd] (hmod, hmod / t) with hmod in [0, t), and,
  // when the first source is wide (wide0), [nd] (2^32 hmod_0 mod t, / t);
  // null otherwise
  double *fd;
  size_t fbytes;
  int wide0;
  // int8-MFMA conversion (k_basis_convert_mfma): the balanced base-256
  // digits of M'[(s, a)][t] = [2^(8a) hmod_s]_t laid out as the MFMA B
  // operand, [n_k][n_tg][8][64] words (n_k = ceil(ns / 4) source quads,
  // n_tg = ceil(nd / 16) target groups); bit g of wide_mask: group g holds a
  // target of 2^45 or more (its digits 6 and 7 are not zero)
  u64 *mf = nullptr;
  size_t mbytes = 0;
  int n_k = 0, n_tg = 0, wide_mask = 0;
  // k_convert_h4's operands: the MFMA table with the targets of each group
  // in the order row m <- target 16 tg + 4 (m % 4) + m / 4 (so that lane
  // group g holds targets 4 e + g: a group's first targets fill every lane
  // group), [n_k][n_tg][8][64] words; and per source [N^-1 hinv]_(q_s) as
  // [ns] words, [ns] Shoup constants, [ns] (w, w / q_s) doubles (the inverse
  // high pass leaves its x N^-1 to this product), then hinv as [ns] words
  // and [ns] Shoup constants (sources of 2^45 or more, whose inverse high
  // pass runs before the kernel)
  u64 *mt = nullptr;
  u64 *sn = nullptr;
};

struct FFTTable {  // encoder tables for one slot count n
  int n;
  double *tw_fwd;  // [n/2][2] exp(+2 pi i j / n)
  double *tw_inv;  // [n/2][2] exp(-2 pi i j / n)
  double *twist;   // [n][2]   exp(-2 pi i k / 4n)
  double *untwist; // [n][2]   exp(+2 pi i k / 4n)
  u32 *perm;       // [n] r_j = (5^j mod 4n - 1) / 4
};

// Per-kernel timing (ckks_profile_enable / ckks_profile_read): HIP events on
// the context stream around a launch, with its algorithmic bytes (each input
// word read once, each output word written once) and modular operations.
struct ProfRec {
  const char *name;
  hipEvent_t a, b;
  double bytes, ops;
};

}  // namespace ckks

struct ckks_context {
  u64 serial = 0;  // unique per created context (never reused)
  ckks_params params;
  int N, logN, L, alpha, ds, K;
  hipStream_t stream;
  ckks::Pool pool;
  // pinned staging of host-to-device uploads made mid-computation: a buffer
  // is reused once the event recorded after its copy has completed
  struct StageBuf {
    void *p;
    size_t bytes;
    hipEvent_t ev;
  };
  std::vector<StageBuf> stage;
  std::vector<u64> primes;
  std::vector<int8_t> secret;
  ckks::ModQ *d_mods;  // [K]
  std::vector<ckks::ModQ> h_mods;
  u64 *d_psi, *d_psi_sh, *d_ipsi, *d_ipsi_sh;  // [K][N] each
  u64 *d_ninv;                                 // [K][2] value, shoup
  // fp64 path for primes below 2^45 (prime_fp[p] != 0): per prime [N][2]
  // doubles (w, w / q) of psi_br and psi_br^-1, and [K][2] (N^-1, N^-1 / q)
  std::vector<int> prime_fp;
  double *d_tw_fp = nullptr, *d_itw_fp = nullptr, *d_ninv_fp = nullptr;
  // per prime below 2^45: 2^-64 mod q and its quotient by q (Montgomery factor)
  double *d_rinv_fp = nullptr;
  u64 *d_secret;                               // [K][N] NTT domain
  std::map<u64, ckks::DeviceKey> keys;          // galois -> key (0 = relin)
  std::map<std::pair<int, int>, ckks::BCTable> bc_up;  // (limbs, digit)
  std::map<int, ckks::BCTable> bc_down;                // limbs
  std::map<int, u64 *> pinv;     // limbs -> [limbs][2] P^-1 mod q_i, shoup
  std::map<int, u64 *> pmod;     // limbs -> [limbs][2] P mod q_i, shoup
  u64 *d_pmod = nullptr;         // [L][2] P mod q_i, shoup (extended-basis lifts)
  std::map<std::pair<int, int>, u64 *> relin_rs;  // (limbs, primes) -> relin-rescale constants
  std::map<std::pair<int, int>, u64 *> rescale_d;  // (limbs, primes) -> rescale constants
  std::map<int, ckks::FFTTable> fft;
  std::map<int, u64 *> garner;   // K -> [K*K] q_j^-1 mod q_k
  bool prof = false;                     // per-kernel timing on
  std::vector<ckks::ProfRec> prof_recs;  // timed launches since the last read
  // operation audit since the last ckks_audit_read with reset: key switches,
  // their ciphertext bytes (input read once per ModUp, each output written
  // once), their key bytes (each key read once per launch), the plaintext
  // bytes of MACs and plaintext products, rescale bytes
  double audit[5] = {0, 0, 0, 0, 0};
  std::vector<hipEvent_t> prof_pool;     // events for reuse
  int device = 0;                  // HIP device current at creation
  u64 *noalloc_scratch = nullptr;  // that device's fixed scratch (ckks_rotate_many_noalloc)
  bool rotation_tables = false;    // every level's key-switch constants built
  // basis conversions on the int8 matrix cores (k_basis_convert_mfma, the
  // default) or the VALU kernels (environment CKKS_BASIS_CONVERT=valu when
  // the context is created); both give the same words
  bool bc_mfma = true;
  // N = 2^16 key switches run the extended digits' low NTT pass with the key
  // inner product fused (launch_ntt_low_key); environment
  // CKKS_KEYSWITCH_FUSED=0 at creation selects the separate kernels
  bool ks_fused = true;
  // with ks_fused and fp64 special primes, the special limbs of the key
  // product also take the ModDown's inverse low pass in the same kernel;
  // environment CKKS_KS_SPECIAL_INV=0 at creation keeps it separate
  bool ks_sp_inv = true;
  // N = 2^16: the ModUp's and ModDown's conversions run between the NTT
  // halves in one register-resident kernel (launch_convert_h4) where the
  // int8-MFMA table allows; environment CKKS_KS_TILE=0 at creation keeps the
  // separate high passes and conversion
  bool ks_tile = true;
  // with ks_tile and the special limbs' inverse low pass in the key product,
  // rotations and relinearisations run the fp64 Q limbs' key product with
  // the ModDown's combine in one kernel (launch_low_key_moddown), after the
  // special limbs' conversion; environment CKKS_KS_DEFER=0 at creation keeps
  // the accumulators in HBM between the two
  bool ks_defer = true;
  // batched key switches of at least kSplitMin ciphertexts per part run as
  // `split_parts` parts, the first on the context stream and the others on
  // `aux` streams (forked from and joined back into the context stream), so
  // that a latency-bound kernel of one part shares the CUs with a streaming
  // kernel of another; environment CKKS_SPLIT_STREAMS=<parts> at creation
  // (1 keeps one stream)
  static constexpr int kMaxSplit = 4;
  int split_parts = 3;
  int split_streams = 3;  // parts whose streams exist (split_parts <= this)
  hipStream_t aux[kMaxSplit - 1] = {};
  hipEvent_t fork_ev = nullptr, join_ev[kMaxSplit - 1] = {};
};

struct ckks_ct {
  ckks_context *ctx;
  u64 *d;
  size_t bytes;
  int polys, limbs, is_ext, slots, scale_degree;
  double scale;
  u64 serial;  // the owning context's serial (0: a view that owns no memory)
};

struct ckks_event {
  ckks_context *ctx;
  hipEvent_t ev;
};

struct ckks_tensor {  // raw device bytes (weights for the diagonal packers)
  ckks_context *ctx;
  void *d;
  size_t bytes;
  u64 serial;  // the owning context's serial
};

// ---------------------------------------------------------------------------
// kernel launchers (ckks_kernels.hip)
// ---------------------------------------------------------------------------
namespace ckks {

// Records one timed launch when the context profiles (scope = the launches).
// audit counters (ckks_context::audit)
inline void audit_keyswitch(ckks_context *c, int n_items, int n_keys, int q_limbs, int digits,
                            int E) {
  const double lp = 8.0 * c->N;
  c->audit[0] += (double)n_items * n_keys;
  c->audit[1] += (double)n_items * (2.0 * q_limbs + 2.0 * q_limbs * n_keys) * lp;
  c->audit[2] += (double)n_keys * digits * 2.0 * E * lp;
}
inline void audit_pt(ckks_context *c, double limb_polys) { c->audit[3] += limb_polys * 8.0 * c->N; }
inline void audit_rescale(ckks_context *c, double limb_polys) {
  c->audit[4] += limb_polys * 8.0 * c->N;
}

struct KTimer {
  ckks_context *c;
  ProfRec r{};
  bool on;
  KTimer(ckks_context *c, const char *name, double bytes, double ops);
  ~KTimer();
  KTimer(const KTimer &) = delete;
  KTimer &operator=(const KTimer &) = delete;
};

void launch_ntt(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                int l_begin, int l_count, int q_limbs, bool inverse);
// out = a op b over `limbs` limbs of `polys` polynomials (op: 0 add, 1 sub)
void launch_addsub_many(ckks_context *c, const Batch &a, const Batch &b, const Batch &out, int n,
                        int polys, int limbs, int q_limbs, int op);
void launch_addsub(ckks_context *c, const u64 *a, const u64 *b, u64 *out, int polys,
                   int limbs, int q_limbs, int op);
void launch_mul_pt(ckks_context *c, const u64 *ct, const u64 *pt, u64 *out, int polys,
                   int limbs, int q_limbs);
void launch_mul_i(ckks_context *c, const u64 *ct, u64 *out, int polys, int limbs,
                  int q_limbs, int negative);
void launch_scalar(ckks_context *c, const u64 *ct, const u64 *s, u64 *out, int polys,
                   int limbs, int q_limbs, int op);  // op 0: add to poly 0, 1: mul all
// out = a x b of degree-1 ciphertexts at `limbs` limbs: parts 1 writes d0 and
// d1, 2 writes d2, 3 all three, for limbs [l_begin, l_begin + l_count)
// (l_count -1: to the last limb) and [l_begin2, l_begin2 + l_count2)
void launch_tensor(ckks_context *c, const Batch &a, const Batch &b, const Batch &out,
                   int n_items, int limbs, int l_begin = 0, int l_count = -1, int parts = 3,
                   int l_begin2 = 0, int l_count2 = 0);
void launch_basis_convert(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                          const BCTable &t, int src_prime0, int t_split, int t_skip,
                          int q_limbs, bool centered);
void launch_copy_limbs(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                       int limb_count);
void launch_key_inner(ckks_context *c, const Batch &ext, const Batch &acc, int n_items,
                      const DeviceKey &key, int digits, int E, int q_limbs, u64 galois,
                      const Batch *own = nullptr);
// N = 2^16: the high pass of the forward NTT alone (the low pass then runs in
// launch_ntt_low_key)
void launch_ntt_fwd_high(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                         int l_begin, int l_count, int q_limbs);
// N = 2^16: the forward low pass of the extended digits ext (item it at
// ext + it ext_stride, [digits][E][N], high pass done; a digit's own limbs
// are read from own) fused with the key inner product into acc (item it at
// acc + it acc_stride, [2][E][N]); ginv = g^-1 mod 2N (1 for
// relinearisation).  The words of launch_ntt's low pass then launch_key_inner.
// With sp (only where low_key_special_fp holds), the special limbs' two
// components also take the inverse NTT's low pass, into sp.base + (2 it + c)
// sp.stride + (l - q_limbs) N, and are not written to acc: the ModDown then
// runs launch_ntt_inv_high on them.
bool low_key_special_fp(const ckks_context *c);
// The Q limbs of fp64 primes below defer_below are skipped
// (launch_low_key_moddown runs their key product with the ModDown's combine)
// With own_b, the digits' own limbs are those of own x own_b (word by word),
// formed where they are read.
void launch_ntt_low_key(ckks_context *c, const u64 *ext, size_t ext_stride, const Batch &own,
                        u64 *acc, size_t acc_stride, int n_items, const DeviceKey &key,
                        int digits, int E, int q_limbs, u64 ginv, const Strided *sp = nullptr,
                        int defer_below = 0, const Batch *own_b = nullptr,
                        bool ext_packed = false);
// N = 2^16: for the Q limbs of fp64 primes, launch_ntt_low_key's key product
// and launch_ntt_moddown's combine (addends and outputs as there, no postop)
// in one kernel, the accumulator kept in the block, for output limbs
// [0, out_limbs) (q_limbs, or the kept limbs of a relinearise-rescale, whose
// pinv is (P p_1..p_D)^-1); conv holds the ModDown's conversion after the
// forward high pass (launch_convert_h4), 2 n items of out_limbs limbs; pmod
// per Q limb [P]_q and its Shoup constant.  The special limbs' key product
// and the other Q limbs run through launch_ntt_low_key(defer_below) and
// launch_ntt_moddown(wide_only).
// With mul_b, add and mul_b are the factors a and b of the degree-2
// products whose d0 = a0 b0 and d1 = a0 b1 + a1 b0 (a1, b1 at add1_off)
// are the addend, formed in the kernel (launch_tensor then writes the d0 /
// d1 limbs other kernels read).  own_b as for launch_ntt_low_key.
void launch_low_key_moddown(ckks_context *c, const u64 *ext, size_t ext_stride, const Batch &own,
                            int n_items, const DeviceKey &key, int digits, int E, int q_limbs,
                            u64 ginv, const Batch &conv, const u64 *pinv, const u64 *pmod,
                            const Batch &add, u64 add1_off, const Batch &out, u64 out1_off,
                            int out_limbs, const Batch *mul_b = nullptr,
                            const Batch *own_b = nullptr, bool ext_packed = false);
// N = 2^16: the high pass of the inverse NTT alone, in place (after the low
// pass of launch_ntt_low_key's sp output)
void launch_ntt_inv_high(ckks_context *c, const Batch &dst, int n_items, int l_begin, int l_count,
                         int q_limbs);
void launch_moddown_combine(ckks_context *c, const Strided &acc, const Strided &conv,
                            const Batch &add0, const Batch &add1, const u64 *galois,
                            const Batch &out0, const Batch &out1, int n_items, int limbs,
                            int E, const u64 *pinv, const u64 *amul = nullptr,
                            const PostOp *post = nullptr);
// high_done: conv already went through the forward high pass
// (launch_convert_h4), only the low pass with the combine runs
void launch_ntt_moddown(ckks_context *c, const Batch &conv, int n, int limbs, const Batch &acc,
                        int E, const u64 *pinv, const Batch &add, u64 add1_off,
                        const u64 *galois, const Batch &out, u64 out1_off,
                        const u64 *amul = nullptr, const PostOp *post = nullptr,
                        bool high_done = false, bool wide_only = false);
// the forward NTT's low pass alone, in place (N = 2^16: after the high pass of
// launch_convert_h4 or launch_ntt_fwd_high)
void launch_ntt_fwd_low(ckks_context *c, const Batch &data, int n_items, int l_begin,
                        int l_count, int q_limbs);
// N = 2^16: the inverse NTT's low pass alone (its high pass then runs in
// launch_convert_h4 or launch_ntt_inv_high); with mul, of src x mul word by
// word, formed on load
void launch_ntt_inv_low(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                        int l_begin, int l_count, int q_limbs, const Batch *mul = nullptr);
// N = 2^16: launch_basis_convert of inverse-low-passed sources (src item at
// the first source limb, as launch_basis_convert's) with the inverse high
// pass before and the forward high pass of every target after, in one
// register-resident kernel; targets leave ready for the forward low pass.
// convert_h4_ok tells whether table t takes it (int8-MFMA table, at most 12
// sources and 64 targets).
bool convert_h4_ok(const ckks_context *c, const BCTable &t);
// The relinearise-rescale form (launch_bc_down_rescale's: D dropped primes,
// rtab its table) of launch_convert_h4: src items hold the special limbs
// after the inverse low pass, then the D dropped limbs of X as coefficients;
// dst takes the T = nd - D kept targets after the forward high pass.
bool convert_h4_rs_ok(const ckks_context *c, const BCTable &t, int D);
void launch_convert_h4_rs(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                          const BCTable &t, int D, const u64 *rtab);
// packed: the fp64 targets' planes in the packed form the fused key products
// read (ext_packed of launch_ntt_low_key / launch_low_key_moddown)
void launch_convert_h4(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                       const BCTable &t, int src_prime0, int t_split, int t_skip, int q_limbs,
                       bool centered, bool packed = false);
void launch_rescale_lift(ckks_context *c, const Batch &last, const Batch &w, int n_items,
                         int limbs, int D, const u64 *tab);
void launch_rescale_finish(ckks_context *c, const Batch &src, const Batch &w, const Batch &out,
                           int n_items, int T, const u64 *inv);
void launch_bc_down_rescale(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                            const BCTable &t, int D, const u64 *rtab);
void launch_rs_prep(ckks_context *c, const Strided &acc, int E, int limbs, int D, const Batch &d,
                    int n, const Strided &x);
// Feature-major BSGS diagonal geometry (token-lane packing)
struct DiagGeom {
  int D, lanes, baby, giant_base;
};
struct StructSources {  // up to three real weight matrices
  const void *p[3];
  u64 stride[3][2];  // elements per row, per column
  int fp32;
};
void launch_encode_diagonals(ckks_context *c, const void *w, int dtype, const StructSources *src,
                             const u64 *maps, const DiagGeom &gm, int rows, int slots,
                             double scale, int limbs, int is_ext, ckks_ct **out);
void launch_mod_raise(ckks_context *c, const u64 *coef, u64 *out, int polys, int target);
struct MultiKeys {  // one key and inverse Galois element per rotation
  const u64 *key[kMaxBatch];
  u64 ginv[kMaxBatch];
};
void launch_key_inner_multi(ckks_context *c, const u64 *ext, size_t ext_stride, int n_items,
                            const std::vector<const DeviceKey *> &keys,
                            const std::vector<u64> &galois_inv, const Batch &c0,
                            const u64 *const *d_outp, int digits, int E, int q_limbs);
void launch_lincomb(ckks_context *c, const u64 *d_table, int T, int n, const double *d_w,
                    double cst, u64 *const *d_outp, int limbs, u64 *wtab, u64 *ctab);
void launch_mac_table(ckks_context *c, const u64 *const *bab, int n, const u64 *const *pts, int B,
                      int G, u64 *out, int limbs);
// Queue a copy of `bytes` host bytes to device memory `dst` on the context
// stream without waiting for it (the bytes go through pinned staging first,
// so `src` may be freed on return).
void upload_async(ckks_context *c, void *dst, const void *src, size_t bytes);
void launch_mac_many(ckks_context *c, const u64 *bab, int n, const Batch &pts, int B, int G,
                     u64 *out, int E, int q_limbs);
void launch_ext_identity(ckks_context *c, const u64 *ct, u64 *out, int limbs);
void launch_ext_add_pc0(ckks_context *c, const u64 *ct, u64 *out, int limbs, u64 galois);
void launch_moddown_one(ckks_context *c, const Batch &src, Strided conv, const Batch &out,
                        int n_items, int limbs, const u64 *pinv);
void launch_ext_rot_accum(ckks_context *c, const Batch &u, const Batch &acc, const Batch &total,
                          u64 galois, int n_items, int E, int q_limbs);
// MAC over limbs_total limbs per component; limbs >= q_limbs are special
// limbs (an extended object: Q limbs then alpha P limbs)
void launch_mac(ckks_context *c, const Batch &babies, const Batch &pts, int B, u64 *out,
                int limbs_total, int q_limbs);
void launch_keygen(ckks_context *c, DeviceKey &key, u64 id, int relin, u64 galois);
// residues of a signed integer polynomial e[N] over `limbs` limbs, then NTT
void launch_expand_ntt(ckks_context *c, const long long *e, u64 *out, int limbs, int q_limbs);
void launch_encode(ckks_context *c, const double *d_re, const double *d_im, int rows,
                   int slots, double scale, int limbs, int is_ext, const Batch &out);
void launch_encrypt_finish(ckks_context *c, u64 *ct, int limbs, u32 enc_id);
void launch_decrypt_decode(ckks_context *c, const ckks_ct *ct, double *d_re, double *d_im);
void launch_scalar_encode(ckks_context *c, double v, int limbs, u64 *out);
// operations per second of the register-only probe (blocks x 256 threads,
// scratch holds one double per thread)
double launch_int_peak(ckks_context *c, int kind, double *scratch, int blocks, int iters);

}  // namespace ckks
