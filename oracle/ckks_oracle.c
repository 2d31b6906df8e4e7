/*
 * ckks_oracle.c -- CPU restatement of the RNS-CKKS evaluation path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker for the MI355X kernels): loaded by
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py, never
 * by the product path.  Compile with -ffp-contract=off so the floating-point
 * encoder performs exactly the operations written here.
 *
 * Plain C11, unsigned __int128 for products; modular reductions use `%` on
 * 128-bit values (obviously correct), except the NTT butterflies, which use
 * Shoup's precomputed-quotient multiply (pinned against an O(N^2) DFT in
 * tests/test_oracle_pins.py).
 *
 * Citations: the reference calls these operations through EasyFHE
 * (call sites listed per function); EasyFHE itself is not available, so each
 * function states the published algorithm it implements.
 */
#include "ckks_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef unsigned __int128 u128;
typedef uint64_t u64;

/* ------------------------------------------------------------------------ */
/* modular arithmetic                                                        */
/* ------------------------------------------------------------------------ */

/* Reduction of a 128-bit value modulo a 64-bit prime.  The plain build uses
 * `%` (obviously correct; the pinned checker).  ORC_FAST builds, made for
 * timing the CPU baseline, reduce the two 64-bit halves with Shoup's
 * precomputed-quotient product, x = hi 2^64 + lo == hi (2^64 mod q) + lo,
 * with the per-prime constants in a table filled at context creation; the
 * two builds give the same words (tests/test_oracle_pins.py compares them). */
#ifdef ORC_FAST
typedef struct {
  u64 q, r64, r64s, one_s;
} fastmod_t;
/* Open-addressing table of every context's primes; written only while a
 * context is created (orc_ctx_create), read by the computing threads. */
#define FM_SLOTS 1024
static fastmod_t fm_table[FM_SLOTS];

static inline unsigned fm_slot(u64 q) {
  return (unsigned)(((q >> 17) * 0x9E3779B97F4A7C15ull) >> 54);
}

static void fm_register(u64 q) {
  unsigned i = fm_slot(q);
  for (int n = 0; n < FM_SLOTS; n++, i = (i + 1) & (FM_SLOTS - 1)) {
    if (fm_table[i].q == q) return;
    if (fm_table[i].q == 0) {
      fm_table[i].r64 = (u64)((((u128)1) << 64) % q);
      fm_table[i].r64s = (u64)(((u128)fm_table[i].r64 << 64) / q);
      fm_table[i].one_s = (u64)((((u128)1) << 64) / q);
      fm_table[i].q = q;
      return;
    }
  }
}

static inline u64 fm_shoup(u64 a, u64 w, u64 ws, u64 q) {
  u64 hi = (u64)(((u128)a * ws) >> 64);
  u64 r = a * w - hi * q;
  return r >= q ? r - q : r;
}

static inline u64 mod128(u128 x, u64 q) {
  unsigned i = fm_slot(q);
  while (fm_table[i].q != q) {
    if (fm_table[i].q == 0) return (u64)(x % q); /* not a registered prime */
    i = (i + 1) & (FM_SLOTS - 1);
  }
  const fastmod_t *m = &fm_table[i];
  const u64 h = fm_shoup((u64)(x >> 64), m->r64, m->r64s, q);
  const u64 l = fm_shoup((u64)x, 1, m->one_s, q);
  const u64 s = h + l;
  return s >= q ? s - q : s;
}
#else
static inline u64 mod128(u128 x, u64 q) { return (u64)(x % q); }
#endif

uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q) { return mod128((u128)a * b, q); }

static inline u64 addmod(u64 a, u64 b, u64 q) {
  u64 s = a + b;
  return s >= q ? s - q : s;
}

static inline u64 submod(u64 a, u64 b, u64 q) { return a >= b ? a - b : a + q - b; }

uint64_t orc_powmod(uint64_t a, uint64_t e, uint64_t q) {
  u64 r = 1 % q;
  a %= q;
  while (e) {
    if (e & 1) r = orc_mulmod(r, a, q);
    a = orc_mulmod(a, a, q);
    e >>= 1;
  }
  return r;
}

static u64 invmod(u64 a, u64 q) { return orc_powmod(a % q, q - 2, q); }

static inline u64 shoup_pre(u64 w, u64 q) { return (u64)(((u128)w << 64) / q); }

static inline u64 shoup_mul(u64 a, u64 w, u64 ws, u64 q) {
  u64 hi = (u64)(((u128)a * ws) >> 64);
  u64 r = a * w - hi * q;
  return r >= q ? r - q : r;
}

/* Deterministic Miller-Rabin: the first twelve primes as bases decide every
 * n < 3.3e24 (Sorenson-Webster 2015), which covers all 64-bit integers. */
int orc_is_prime(uint64_t n) {
  static const u64 small[12] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return 0;
  for (int i = 0; i < 12; i++) {
    if (n == small[i]) return 1;
    if (n % small[i] == 0) return 0;
  }
  u64 d = n - 1;
  int r = 0;
  while ((d & 1) == 0) {
    d >>= 1;
    r++;
  }
  for (int i = 0; i < 12; i++) {
    u64 x = orc_powmod(small[i], d, n);
    if (x == 1 || x == n - 1) continue;
    int composite = 1;
    for (int k = 1; k < r; k++) {
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

static int in_list(u64 v, const u64 *list, int n) {
  for (int i = 0; i < n; i++)
    if (list[i] == v) return 1;
  return 0;
}

/* Prime selection rule (EasyFHE's rule is not readable here; this one is
 * fixed and documented): candidates 2^bits + 1, then 2^bits - k*2N + 1 and
 * 2^bits + k*2N + 1 for k = 1, 2, ... (closest to 2^bits first, the lower one
 * first at equal distance).  Candidates >= 2^60 are skipped so that sixteen
 * residues always sum below 2^64 (the lazy accumulation bound). */
int orc_gen_primes(int logN, int bits, int count, const uint64_t *used,
                   int n_used, uint64_t *out) {
  const u64 M = (u64)2 << logN;
  const u64 base = (u64)1 << bits;
  const u64 cap = (u64)1 << 60;
  int found = 0;
  for (u64 k = 0; found < count; k++) {
    u64 cands[2];
    int nc = 0;
    if (k == 0) {
      cands[nc++] = base + 1;
    } else {
      if (k * M < base) cands[nc++] = base - k * M + 1;
      cands[nc++] = base + k * M + 1;
    }
    if (k * M >= base && base + k * M + 1 >= cap) break;
    for (int i = 0; i < nc && found < count; i++) {
      u64 c = cands[i];
      if (c >= cap || c <= M) continue;
      if (in_list(c, used, n_used) || in_list(c, out, found)) continue;
      if (orc_is_prime(c)) out[found++] = c;
    }
  }
  return found;
}

/* Root rule: psi0 = x^((q-1)/2N) for the smallest x >= 2 with psi0^N = -1
 * (so psi0 has order exactly 2N), then the smallest of the primitive roots
 * psi0^k, k odd. */
uint64_t orc_min_root(uint64_t q, int logN) {
  const u64 N = (u64)1 << logN;
  const u64 M = 2 * N;
  u64 psi0 = 0;
  for (u64 x = 2;; x++) {
    psi0 = orc_powmod(x, (q - 1) / M, q);
    if (orc_powmod(psi0, N, q) == q - 1) break;
  }
  u64 sq = orc_mulmod(psi0, psi0, q);
  u64 cur = psi0, best = psi0;
  for (u64 k = 1; k < N; k++) {
    cur = orc_mulmod(cur, sq, q);
    if (cur < best) best = cur;
  }
  return best;
}

static inline uint32_t bitrev(uint32_t x, int bits) {
  uint32_t r = 0;
  for (int i = 0; i < bits; i++) {
    r = (r << 1) | (x & 1);
    x >>= 1;
  }
  return r;
}

/* ------------------------------------------------------------------------ */
/* ChaCha20 block function (RFC 8439 sec. 2.3)                              */
/* ------------------------------------------------------------------------ */

static inline uint32_t rotl32(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

#define QR(a, b, c, d)                \
  do {                                \
    a += b; d ^= a; d = rotl32(d, 16); \
    c += d; b ^= c; b = rotl32(b, 12); \
    a += b; d ^= a; d = rotl32(d, 8);  \
    c += d; b ^= c; b = rotl32(b, 7);  \
  } while (0)

void orc_chacha20_block(const uint32_t key[8], uint32_t counter,
                        const uint32_t nonce[3], uint32_t out[16]) {
  uint32_t s[16], x[16];
  s[0] = 0x61707865u;
  s[1] = 0x3320646eu;
  s[2] = 0x79622d32u;
  s[3] = 0x6b206574u;
  for (int i = 0; i < 8; i++) s[4 + i] = key[i];
  s[12] = counter;
  s[13] = nonce[0];
  s[14] = nonce[1];
  s[15] = nonce[2];
  memcpy(x, s, sizeof(s));
  for (int i = 0; i < 10; i++) {
    QR(x[0], x[4], x[8], x[12]);
    QR(x[1], x[5], x[9], x[13]);
    QR(x[2], x[6], x[10], x[14]);
    QR(x[3], x[7], x[11], x[15]);
    QR(x[0], x[5], x[10], x[15]);
    QR(x[1], x[6], x[11], x[12]);
    QR(x[2], x[7], x[8], x[13]);
    QR(x[3], x[4], x[9], x[14]);
  }
  for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

/* PRNG stream (domain, id, sub): key = (seed lo, seed hi, 0...), nonce =
 * (domain, id, sub), counter = block index. */
void orc_prng_block(uint64_t seed, uint32_t domain, uint32_t id, uint32_t sub,
                    uint32_t counter, uint32_t out[16]) {
  uint32_t key[8] = {(uint32_t)seed, (uint32_t)(seed >> 32), 0, 0, 0, 0, 0, 0};
  uint32_t nonce[3] = {domain, id, sub};
  orc_chacha20_block(key, counter, nonce, out);
}

enum { DOM_SECRET = 1, DOM_KEY_A = 2, DOM_KEY_E = 3, DOM_ENC_A = 4, DOM_ENC_E = 5 };

/* Uniform residue for coefficient k: 128 stream bits reduced mod q. */
static void sample_uniform(u64 seed, uint32_t dom, uint32_t id, uint32_t sub,
                           u64 q, u64 *out, int N) {
  uint32_t blk[16];
  for (int k = 0; k < N; k += 4) {
    orc_prng_block(seed, dom, id, sub, (uint32_t)(k >> 2), blk);
    for (int r = 0; r < 4; r++) {
      u64 lo = (u64)blk[4 * r] | ((u64)blk[4 * r + 1] << 32);
      u64 hi = (u64)blk[4 * r + 2] | ((u64)blk[4 * r + 3] << 32);
      out[k + r] = mod128(((u128)hi << 64) | lo, q);
    }
  }
}

/* Centered binomial error, eta = 21 (sigma = 3.24): coefficient k takes the
 * 64-bit word k of the stream, e = popcount(bits 0..20) - popcount(21..41). */
static void sample_cbd(u64 seed, uint32_t dom, uint32_t id, uint32_t sub,
                       int64_t *out, int N) {
  uint32_t blk[16];
  for (int k = 0; k < N; k += 8) {
    orc_prng_block(seed, dom, id, sub, (uint32_t)(k >> 3), blk);
    for (int r = 0; r < 8; r++) {
      u64 w = (u64)blk[2 * r] | ((u64)blk[2 * r + 1] << 32);
      out[k + r] = (int64_t)__builtin_popcountll(w & 0x1FFFFFull) -
                   (int64_t)__builtin_popcountll((w >> 21) & 0x1FFFFFull);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* context                                                                   */
/* ------------------------------------------------------------------------ */

typedef struct {
  u64 g;
  int digits;
  u64 *data; /* [digits][2][K][N] */
} orc_key;

struct orc_ctx {
  int logN, N, L, alpha, dnum, ds, K;
  u64 seed;
  u64 *primes;
  u64 **psi, **psi_sh, **ipsi, **ipsi_sh;
  u64 *ninv;
  int8_t *s;
  u64 *s_ntt; /* [K][N] */
  int nkeys;
  orc_key keys[512];
};

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int orc_N(const orc_ctx *c) { return c->N; }
int orc_L(const orc_ctx *c) { return c->L; }
int orc_alpha(const orc_ctx *c) { return c->alpha; }
int orc_digit_size(const orc_ctx *c) { return c->ds; }
void orc_primes(const orc_ctx *c, uint64_t *out) {
  memcpy(out, c->primes, sizeof(u64) * c->K);
}
void orc_secret(const orc_ctx *c, int8_t *out) { memcpy(out, c->s, c->N); }
const uint64_t *orc_psi_br(const orc_ctx *c, int prime_idx) { return c->psi[prime_idx]; }

/* limb index within an extended basis Q_limbs u P -> global prime index */
static inline int prime_of(const orc_ctx *c, int limb, int q_limbs) {
  return limb < q_limbs ? limb : c->L + (limb - q_limbs);
}

/* Secret key rule: sparse ternary with Hamming weight h by a partial
 * Fisher-Yates shuffle over positions, driven by 64-bit words t = 0, 1, ... of
 * stream (SECRET, 0, 0): position word, then sign word.  Uniform ternary
 * takes word k mod 3 - 1 per coefficient. */
static void gen_secret(orc_ctx *c, int mode, int h) {
  const int N = c->N;
  memset(c->s, 0, N);
  uint32_t blk[16];
  u64 word_idx = 0;
#define NEXT_U64(dst)                                                     \
  do {                                                                    \
    orc_prng_block(c->seed, DOM_SECRET, 0, 0, (uint32_t)(word_idx >> 3), \
                   blk);                                                  \
    int r_ = (int)(word_idx & 7);                                         \
    dst = (u64)blk[2 * r_] | ((u64)blk[2 * r_ + 1] << 32);               \
    word_idx++;                                                           \
  } while (0)
  if (mode == 0) {
    uint32_t *perm = (uint32_t *)malloc(sizeof(uint32_t) * N);
    for (int i = 0; i < N; i++) perm[i] = (uint32_t)i;
    for (int t = 0; t < h; t++) {
      u64 r, sg;
      NEXT_U64(r);
      NEXT_U64(sg);
      u64 j = (u64)t + r % (u64)(N - t);
      uint32_t tmp = perm[t];
      perm[t] = perm[j];
      perm[j] = tmp;
      c->s[perm[t]] = (sg & 1) ? -1 : 1;
    }
    free(perm);
  } else {
    for (int i = 0; i < N; i++) {
      u64 r;
      NEXT_U64(r);
      c->s[i] = (int8_t)((int)(r % 3) - 1);
    }
  }
#undef NEXT_U64
}

static void int_to_residues(const int64_t *v, u64 q, u64 *out, int N) {
  for (int k = 0; k < N; k++) {
    int64_t x = v[k];
    int64_t r = x % (int64_t)q;
    out[k] = (u64)(r < 0 ? r + (int64_t)q : r);
  }
}

orc_ctx *orc_ctx_create(int logN, int L, int alpha, int dnum, int first_bits,
                        int dcrt_bits, int special_bits, uint64_t seed,
                        int secret_mode, int h) {
  orc_ctx *c = (orc_ctx *)calloc(1, sizeof(orc_ctx));
  c->logN = logN;
  c->N = 1 << logN;
  c->L = L;
  c->alpha = alpha;
  c->dnum = dnum;
  c->ds = (L + dnum - 1) / dnum;
  c->K = L + alpha;
  c->seed = seed;
  const int N = c->N, K = c->K;
  c->primes = (u64 *)calloc(K, sizeof(u64));
  if (orc_gen_primes(logN, first_bits, 1, NULL, 0, c->primes) != 1) goto fail;
  if (L > 1 && orc_gen_primes(logN, dcrt_bits, L - 1, c->primes, 1,
                              c->primes + 1) != L - 1)
    goto fail;
  if (orc_gen_primes(logN, special_bits, alpha, c->primes, L, c->primes + L) !=
      alpha)
    goto fail;
#ifdef ORC_FAST
  for (int p = 0; p < K; p++) fm_register(c->primes[p]);
#endif
  c->psi = (u64 **)calloc(K, sizeof(u64 *));
  c->psi_sh = (u64 **)calloc(K, sizeof(u64 *));
  c->ipsi = (u64 **)calloc(K, sizeof(u64 *));
  c->ipsi_sh = (u64 **)calloc(K, sizeof(u64 *));
  c->ninv = (u64 *)calloc(K, sizeof(u64));
#pragma omp parallel for schedule(dynamic)
  for (int p = 0; p < K; p++) {
    u64 q = c->primes[p];
    u64 psi = orc_min_root(q, logN);
    u64 ipsi = invmod(psi, q);
    u64 *pw = (u64 *)malloc(sizeof(u64) * N), *ipw = (u64 *)malloc(sizeof(u64) * N);
    pw[0] = 1;
    ipw[0] = 1;
    for (int i = 1; i < N; i++) {
      pw[i] = orc_mulmod(pw[i - 1], psi, q);
      ipw[i] = orc_mulmod(ipw[i - 1], ipsi, q);
    }
    c->psi[p] = (u64 *)malloc(sizeof(u64) * N);
    c->psi_sh[p] = (u64 *)malloc(sizeof(u64) * N);
    c->ipsi[p] = (u64 *)malloc(sizeof(u64) * N);
    c->ipsi_sh[p] = (u64 *)malloc(sizeof(u64) * N);
    for (int i = 0; i < N; i++) {
      uint32_t r = bitrev((uint32_t)i, logN);
      c->psi[p][i] = pw[r];
      c->ipsi[p][i] = ipw[r];
      c->psi_sh[p][i] = shoup_pre(pw[r], q);
      c->ipsi_sh[p][i] = shoup_pre(ipw[r], q);
    }
    c->ninv[p] = invmod((u64)N, q);
    free(pw);
    free(ipw);
  }
  c->s = (int8_t *)calloc(N, 1);
  gen_secret(c, secret_mode, h);
  c->s_ntt = (u64 *)malloc(sizeof(u64) * (size_t)K * N);
  int64_t *sv = (int64_t *)malloc(sizeof(int64_t) * N);
  for (int k = 0; k < N; k++) sv[k] = c->s[k];
#pragma omp parallel for
  for (int p = 0; p < K; p++) {
    int_to_residues(sv, c->primes[p], c->s_ntt + (size_t)p * N, N);
    orc_ntt_fwd(c, p, c->s_ntt + (size_t)p * N);
  }
  free(sv);
  return c;
fail:
  free(c->primes);
  free(c);
  return NULL;
}

void orc_ctx_free(orc_ctx *c) {
  if (!c) return;
  for (int p = 0; p < c->K; p++) {
    free(c->psi[p]);
    free(c->psi_sh[p]);
    free(c->ipsi[p]);
    free(c->ipsi_sh[p]);
  }
  free(c->psi);
  free(c->psi_sh);
  free(c->ipsi);
  free(c->ipsi_sh);
  free(c->ninv);
  free(c->primes);
  free(c->s);
  free(c->s_ntt);
  for (int i = 0; i < c->nkeys; i++) free(c->keys[i].data);
  free(c);
}

/* ------------------------------------------------------------------------ */
/* NTT: a_hat[i] = sum_k a_k psi^((2 br(i) + 1) k)  (bit-reversed output)     */
/* ------------------------------------------------------------------------ */

#ifdef ORC_FAST
/* Timed build: Harvey's lazy butterflies (values kept in [0, 4q), Shoup
 * products left in [0, 2q)), canonical words at the end, so the outputs are
 * those of the plain transforms below (D. Harvey, "Faster arithmetic for
 * number-theoretic transforms", J. Symb. Comput. 60, 2014). */
static inline u64 shoup_lazy(u64 a, u64 w, u64 ws, u64 q) {
  u64 hi = (u64)(((u128)a * ws) >> 64);
  return a * w - hi * q;
}

void orc_ntt_fwd(const orc_ctx *c, int p, uint64_t *a) {
  const u64 q = c->primes[p], q2 = 2 * q;
  const u64 *W = c->psi[p], *Ws = c->psi_sh[p];
  const int N = c->N;
  int t = N;
  for (int m = 1; m < N; m <<= 1) {
    t >>= 1;
    for (int i = 0; i < m; i++) {
      const u64 w = W[m + i], ws = Ws[m + i];
      const int j1 = 2 * i * t;
      for (int j = j1; j < j1 + t; j++) {
        u64 u = a[j];
        u = u >= q2 ? u - q2 : u;
        const u64 v = shoup_lazy(a[j + t], w, ws, q);
        a[j] = u + v;
        a[j + t] = u - v + q2;
      }
    }
  }
  for (int j = 0; j < N; j++) {
    u64 x = a[j];
    x = x >= q2 ? x - q2 : x;
    a[j] = x >= q ? x - q : x;
  }
}

void orc_ntt_inv(const orc_ctx *c, int p, uint64_t *a) {
  const u64 q = c->primes[p], q2 = 2 * q;
  const u64 *W = c->ipsi[p], *Ws = c->ipsi_sh[p];
  const int N = c->N;
  int t = 1;
  for (int m = N >> 1; m >= 1; m >>= 1) {
    for (int i = 0; i < m; i++) {
      const u64 w = W[m + i], ws = Ws[m + i];
      const int j1 = 2 * i * t;
      for (int j = j1; j < j1 + t; j++) {
        const u64 x = a[j], y = a[j + t];
        const u64 s = x + y;
        a[j] = s >= q2 ? s - q2 : s;
        a[j + t] = shoup_lazy(x - y + q2, w, ws, q);
      }
    }
    t <<= 1;
  }
  const u64 ni = c->ninv[p], nis = shoup_pre(ni, q);
  for (int j = 0; j < N; j++) a[j] = shoup_mul(a[j], ni, nis, q);
}
#else
void orc_ntt_fwd(const orc_ctx *c, int p, uint64_t *a) {
  const u64 q = c->primes[p];
  const u64 *W = c->psi[p], *Ws = c->psi_sh[p];
  const int N = c->N;
  int t = N;
  for (int m = 1; m < N; m <<= 1) {
    t >>= 1;
    for (int i = 0; i < m; i++) {
      const u64 w = W[m + i], ws = Ws[m + i];
      const int j1 = 2 * i * t;
      for (int j = j1; j < j1 + t; j++) {
        u64 u = a[j];
        u64 v = shoup_mul(a[j + t], w, ws, q);
        a[j] = addmod(u, v, q);
        a[j + t] = submod(u, v, q);
      }
    }
  }
}

void orc_ntt_inv(const orc_ctx *c, int p, uint64_t *a) {
  const u64 q = c->primes[p];
  const u64 *W = c->ipsi[p], *Ws = c->ipsi_sh[p];
  const int N = c->N;
  int t = 1;
  for (int m = N >> 1; m >= 1; m >>= 1) {
    for (int i = 0; i < m; i++) {
      const u64 w = W[m + i], ws = Ws[m + i];
      const int j1 = 2 * i * t;
      for (int j = j1; j < j1 + t; j++) {
        u64 x = a[j], y = a[j + t];
        a[j] = addmod(x, y, q);
        a[j + t] = shoup_mul(submod(x, y, q), w, ws, q);
      }
    }
    t <<= 1;
  }
  const u64 ni = c->ninv[p];
  for (int j = 0; j < N; j++) a[j] = orc_mulmod(a[j], ni, q);
}
#endif

void orc_ntt_fwd_limbs(const orc_ctx *c, uint64_t *a, int limbs, int q_limbs) {
#pragma omp parallel for
  for (int l = 0; l < limbs; l++)
    orc_ntt_fwd(c, prime_of(c, l, q_limbs), a + (size_t)l * c->N);
}

void orc_ntt_inv_limbs(const orc_ctx *c, uint64_t *a, int limbs, int q_limbs) {
#pragma omp parallel for
  for (int l = 0; l < limbs; l++)
    orc_ntt_inv(c, prime_of(c, l, q_limbs), a + (size_t)l * c->N);
}

/* ------------------------------------------------------------------------ */
/* automorphisms                                                             */
/* ------------------------------------------------------------------------ */

void orc_automorphism_coeff(const orc_ctx *c, int p, uint64_t g,
                            const uint64_t *in, uint64_t *out) {
  const u64 q = c->primes[p];
  const u64 N = (u64)c->N, M = 2 * N;
  for (u64 k = 0; k < N; k++) {
    u64 e = (u64)((u128)k * g) & (M - 1); /* M = 2N, a power of two */
    if (e < N)
      out[e] = in[k];
    else
      out[e - N] = in[k] ? q - in[k] : 0;
  }
}

/* NTT-domain index map: out[i] = in[br(((2 br(i) + 1) g mod 2N - 1) / 2)]. */
void orc_automorphism_ntt(const orc_ctx *c, uint64_t g, const uint64_t *in,
                          uint64_t *out, int limbs) {
  const int N = c->N, logN = c->logN;
  const u64 M = 2 * (u64)N;
  uint32_t *idx = (uint32_t *)malloc(sizeof(uint32_t) * N);
  for (int i = 0; i < N; i++) {
    u64 e = (u64)((u128)(2 * (u64)bitrev((uint32_t)i, logN) + 1) * g) & (M - 1);
    idx[i] = bitrev((uint32_t)((e - 1) >> 1), logN);
  }
  for (int l = 0; l < limbs; l++) {
    const u64 *src = in + (size_t)l * N;
    u64 *dst = out + (size_t)l * N;
    for (int i = 0; i < N; i++) dst[i] = src[idx[i]];
  }
  free(idx);
}

/* Rotation index -> Galois element.  Left rotation by r (slot j receives
 * slot j + r) is X -> X^(5^r mod 2N); index 2N - 1 requests conjugation
 * (reference call sites operators/linear/complex.py:47-51,
 * operators/linear/config.py:316). */
uint64_t orc_galois_elt(const orc_ctx *c, int64_t rotation) {
  const u64 M = 2 * (u64)c->N;
  if ((u64)rotation == M - 1) return M - 1;
  int64_t half = c->N / 2;
  int64_t r = rotation % half;
  if (r < 0) r += half;
  return orc_powmod(5, (u64)r, M);
}

/* ------------------------------------------------------------------------ */
/* canonical-embedding encoder (CKKS 2017 sec. 3.1)                          */
/*                                                                           */
/* n slots, m'(Y) of degree 2n with Y = X^(N/2n).  With u_k = m'_k + i      */
/* m'_{k+n} and rho = exp(2 pi i / 4n):  z_j = m'(rho^(5^j)) =               */
/* sum_k (u_k rho^k) w^(r_j k), w = exp(2 pi i / n), r_j = (5^j mod 4n - 1)/4 */
/* so decoding is a twist followed by an n-point DFT and a slot permutation; */
/* encoding is its inverse.                                                  */
/* ------------------------------------------------------------------------ */

/* cos and sin of 2 pi j / n (n a power of two) from IEEE basic operations
 * only, so the result does not depend on the compiler or the libm in use
 * (glibc's sin and sincos differ in the last bit for some arguments):
 * integer octant reduction of 8 j / n, then Taylor series of degree 22 on
 * [0, pi/4] by Horner's rule. */
static void unit_root(long long j, long long n, double *cs, double *sn) {
  static const double PI_4 = 0.78539816339744830962;
  j %= n;
  if (j < 0) j += n;
  const long long e8 = 8 * j, o = e8 / n, r = e8 - o * n;
  const long long rr = (o & 1) ? n - r : r;
  const double x = PI_4 * ((double)rr / (double)n);
  const double x2 = x * x;
  double inv_fact[23];
  inv_fact[0] = 1.0;
  for (int k = 1; k <= 22; k++) inv_fact[k] = inv_fact[k - 1] / (double)k;
  double sp = 0.0, cp = 0.0;
  for (int k = 21; k >= 3; k -= 2) sp = (sp + (((k - 1) / 2) % 2 ? -inv_fact[k] : inv_fact[k])) * x2;
  const double S = (sp + 1.0) * x;
  for (int k = 22; k >= 2; k -= 2) cp = (cp + ((k / 2) % 2 ? -inv_fact[k] : inv_fact[k])) * x2;
  const double C = cp + 1.0;
  double c, s;
  switch (o) {
    case 0: c = C; s = S; break;
    case 1: c = S; s = C; break;
    case 2: c = -S; s = C; break;
    case 3: c = -C; s = S; break;
    case 4: c = -C; s = -S; break;
    case 5: c = -S; s = -C; break;
    case 6: c = S; s = -C; break;
    default: c = C; s = -S; break;
  }
  *cs = c;
  *sn = s;
}

void orc_unit_root(long long j, long long n, double *cs, double *sn) { unit_root(j, n, cs, sn); }

typedef struct {
  double re, im;
} cplx;

static inline cplx cmul(cplx a, cplx b) {
  cplx r;
  double t1 = a.re * b.re;
  double t2 = a.im * b.im;
  double t3 = a.re * b.im;
  double t4 = a.im * b.re;
  r.re = t1 - t2;
  r.im = t3 + t4;
  return r;
}

/* X_r = sum_k x_k exp(sign 2 pi i r k / n): radix-2 decimation in time,
 * bit-reversed input permutation, twiddle tw[j] = exp(sign 2 pi i j / n). */
static void fft_inplace(cplx *x, int n, int sign) {
  int logn = 0;
  while ((1 << logn) < n) logn++;
  for (int i = 0; i < n; i++) {
    int r = (int)bitrev((uint32_t)i, logn);
    if (r > i) {
      cplx t = x[i];
      x[i] = x[r];
      x[r] = t;
    }
  }
  cplx *tw = (cplx *)malloc(sizeof(cplx) * (n / 2 + 1));
  for (int j = 0; j < n / 2; j++) {
    double c, s;
    unit_root(j, n, &c, &s);
    tw[j].re = c;
    tw[j].im = sign > 0 ? s : -s;
  }
  for (int len = 2; len <= n; len <<= 1) {
    int half = len >> 1, step = n / len;
    for (int st = 0; st < n; st += len) {
      for (int k = 0; k < half; k++) {
        cplx u = x[st + k];
        cplx v = cmul(x[st + k + half], tw[k * step]);
        x[st + k].re = u.re + v.re;
        x[st + k].im = u.im + v.im;
        x[st + k + half].re = u.re - v.re;
        x[st + k + half].im = u.im - v.im;
      }
    }
  }
  free(tw);
}

static int slot_perm(int j, int n) {
  /* r_j = (5^j mod 4n - 1) / 4 */
  u64 e = orc_powmod(5, (u64)j, 4 * (u64)n);
  return (int)((e - 1) / 4);
}

void orc_encode_coeffs(const orc_ctx *c, const double *re, const double *im,
                       int slots, double scale, double *out) {
  const int N = c->N, n = slots, gap = N / (2 * n);
  cplx *w = (cplx *)calloc(n, sizeof(cplx));
  for (int j = 0; j < n; j++) {
    int r = slot_perm(j, n);
    w[r].re = re[j];
    w[r].im = im ? im[j] : 0.0;
  }
  fft_inplace(w, n, -1);
  const double inv_n = 1.0 / (double)n;
  memset(out, 0, sizeof(double) * N);
  for (int k = 0; k < n; k++) {
    double c, s;
    unit_root(k, 4 * (long long)n, &c, &s);
    cplx tw = {c, -s};
    cplx u = {w[k].re * inv_n, w[k].im * inv_n};
    u = cmul(u, tw);
    out[(size_t)k * gap] = rint(scale * u.re);
    out[(size_t)(k + n) * gap] = rint(scale * u.im);
  }
  free(w);
}

/* Residue of an integer-valued double (exact for any magnitude). */
static u64 double_to_residue(double v, u64 q) {
  if (fabs(v) < 9.2e18) {
    int64_t x = (int64_t)v;
    int64_t r = x % (int64_t)q;
    return (u64)(r < 0 ? r + (int64_t)q : r);
  }
  int e;
  double m = frexp(v, &e);
  int64_t mant = (int64_t)ldexp(m, 53);
  int shift = e - 53;
  int neg = mant < 0;
  u64 am = (u64)(neg ? -mant : mant) % q;
  u64 r = orc_mulmod(am, orc_powmod(2, (u64)shift, q), q);
  return neg ? (r ? q - r : 0) : r;
}

int orc_encode(const orc_ctx *c, const double *re, const double *im, int slots,
               double scale, int limbs, int is_ext, uint64_t *out) {
  const int N = c->N;
  if (slots <= 0 || slots > N / 2 || (slots & (slots - 1))) return -1;
  double *coef = (double *)malloc(sizeof(double) * N);
  orc_encode_coeffs(c, re, im, slots, scale, coef);
  int total = limbs + (is_ext ? c->alpha : 0);
#pragma omp parallel for
  for (int l = 0; l < total; l++) {
    int p = prime_of(c, l, limbs);
    u64 q = c->primes[p];
    u64 *dst = out + (size_t)l * N;
    for (int k = 0; k < N; k++) dst[k] = double_to_residue(coef[k], q);
    orc_ntt_fwd(c, p, dst);
  }
  free(coef);
  return 0;
}

/* Balanced mixed-radix (Garner) reconstruction over the first K limbs,
 * evaluated in double from the most significant digit. */
static void crt_to_double(const orc_ctx *c, const u64 *coeff, int K, double *out) {
  const int N = c->N;
  u64 *inv = (u64 *)malloc(sizeof(u64) * K * K); /* inv[j*K+k] = q_j^-1 mod q_k */
  for (int j = 0; j < K; j++)
    for (int k = 0; k < K; k++)
      inv[j * K + k] = (j == k) ? 0 : invmod(c->primes[j] % c->primes[k], c->primes[k]);
#pragma omp parallel for
  for (int i = 0; i < N; i++) {
    int64_t d[64];
    for (int k = 0; k < K; k++) {
      u64 qk = c->primes[k];
      u64 t = coeff[(size_t)k * N + i];
      for (int j = 0; j < k; j++) {
        int64_t dj = d[j] % (int64_t)qk;
        u64 djm = (u64)(dj < 0 ? dj + (int64_t)qk : dj);
        t = orc_mulmod(submod(t, djm, qk), inv[j * K + k], qk);
      }
      d[k] = t > (qk - 1) / 2 ? (int64_t)t - (int64_t)qk : (int64_t)t;
    }
    double v = (double)d[K - 1];
    for (int k = K - 2; k >= 0; k--) v = v * (double)c->primes[k] + (double)d[k];
    out[i] = v;
  }
  free(inv);
}

/* Number of leading limbs used to reconstruct a coefficient: the smallest K
 * with sum(log2 q_k) >= log2(scale) + 40, capped at `limbs` and 8. */
static int decode_limbs(const orc_ctx *c, int limbs, double scale) {
  double need = log2(scale) + 40.0, have = 0.0;
  int K = 0;
  while (K < limbs && K < 8 && have < need) have += log2((double)c->primes[K++]);
  return K < 1 ? 1 : K;
}

void orc_decode(const orc_ctx *c, const uint64_t *poly, int limbs, int slots,
                double scale, double *re, double *im) {
  const int N = c->N, n = slots, gap = N / (2 * n);
  int K = decode_limbs(c, limbs, scale);
  u64 *coeff = (u64 *)malloc(sizeof(u64) * (size_t)K * N);
  memcpy(coeff, poly, sizeof(u64) * (size_t)K * N);
  orc_ntt_inv_limbs(c, coeff, K, limbs);
  double *v = (double *)malloc(sizeof(double) * N);
  crt_to_double(c, coeff, K, v);
  cplx *x = (cplx *)malloc(sizeof(cplx) * n);
  for (int k = 0; k < n; k++) {
    double c, s;
    unit_root(k, 4 * (long long)n, &c, &s);
    cplx tw = {c, s};
    cplx u = {v[(size_t)k * gap], v[(size_t)(k + n) * gap]};
    x[k] = cmul(u, tw);
  }
  fft_inplace(x, n, +1);
  for (int j = 0; j < n; j++) {
    int r = slot_perm(j, n);
    re[j] = x[r].re / scale;
    if (im) im[j] = x[r].im / scale;
  }
  free(x);
  free(v);
  free(coeff);
}

/* ------------------------------------------------------------------------ */
/* keys                                                                      */
/* ------------------------------------------------------------------------ */

static orc_key *find_key(const orc_ctx *c, u64 g) {
  for (int i = 0; i < c->nkeys; i++)
    if (c->keys[i].g == g) return (orc_key *)&c->keys[i];
  return NULL;
}

/* Hybrid switching key from s' to s (Han-Ki 2020 sec. 3): for digit j with
 * limb set D_j = [j ds, min((j+1) ds, L)):
 *   b_j = -a_j s + e_j + [P]_q s'  on q in D_j,  -a_j s + e_j elsewhere,
 * a_j uniform from stream (KEY_A, id, j<<16 | prime), e_j from (KEY_E, id, j).
 * id is the Galois element (0 for the relinearisation key, s' = s^2). */
static int gen_switch_key(orc_ctx *c, u64 id, const u64 *sp_ntt) {
  if (c->nkeys >= 512) return -1;
  if (find_key(c, id)) return 0;
  const int N = c->N, K = c->K, L = c->L, digits = (L + c->ds - 1) / c->ds;
  orc_key *k = &c->keys[c->nkeys];
  k->g = id;
  k->digits = digits;
  k->data = (u64 *)malloc(sizeof(u64) * (size_t)digits * 2 * K * N);
  for (int j = 0; j < digits; j++) {
    int64_t *e = (int64_t *)malloc(sizeof(int64_t) * N);
    sample_cbd(c->seed, DOM_KEY_E, (uint32_t)id, (uint32_t)j, e, N);
#pragma omp parallel for
    for (int p = 0; p < K; p++) {
      const u64 q = c->primes[p];
      u64 *b = k->data + ((size_t)(j * 2 + 0) * K + p) * N;
      u64 *a = k->data + ((size_t)(j * 2 + 1) * K + p) * N;
      sample_uniform(c->seed, DOM_KEY_A, (uint32_t)id, ((uint32_t)j << 16) | (uint32_t)p,
                     q, a, N);
      u64 *en = (u64 *)malloc(sizeof(u64) * N);
      int_to_residues(e, q, en, N);
      orc_ntt_fwd(c, p, en);
      int in_digit = p < L && p >= j * c->ds && p < (j + 1) * c->ds;
      u64 Pmod = 1;
      for (int t = 0; t < c->alpha; t++) Pmod = orc_mulmod(Pmod, c->primes[L + t] % q, q);
      const u64 *s = c->s_ntt + (size_t)p * N;
      const u64 *sp = sp_ntt + (size_t)p * N;
      for (int i = 0; i < N; i++) {
        u64 v = submod(en[i], orc_mulmod(a[i], s[i], q), q);
        if (in_digit) v = addmod(v, orc_mulmod(Pmod, sp[i], q), q);
        b[i] = v;
      }
      free(en);
    }
    free(e);
  }
  c->nkeys++;
  return 0;
}

int orc_gen_rotation_key(orc_ctx *c, uint64_t g) {
  const int N = c->N, K = c->K;
  u64 *sp = (u64 *)malloc(sizeof(u64) * (size_t)K * N);
  for (int p = 0; p < K; p++)
    orc_automorphism_ntt(c, g, c->s_ntt + (size_t)p * N, sp + (size_t)p * N, 1);
  int r = gen_switch_key(c, g, sp);
  free(sp);
  return r;
}

int orc_gen_relin_key(orc_ctx *c) {
  const int N = c->N, K = c->K;
  u64 *sp = (u64 *)malloc(sizeof(u64) * (size_t)K * N);
  for (int p = 0; p < K; p++) {
    const u64 q = c->primes[p];
    for (int i = 0; i < N; i++) {
      u64 v = c->s_ntt[(size_t)p * N + i];
      sp[(size_t)p * N + i] = orc_mulmod(v, v, q);
    }
  }
  int r = gen_switch_key(c, 0, sp);
  free(sp);
  return r;
}

int orc_get_key(const orc_ctx *c, uint64_t g, uint64_t *out) {
  orc_key *k = find_key(c, g);
  if (!k) return -1;
  if (out) memcpy(out, k->data, sizeof(u64) * (size_t)k->digits * 2 * c->K * c->N);
  return k->digits;
}

/* ------------------------------------------------------------------------ */
/* encryption (secret-key RLWE, the client holds s)                          */
/* ------------------------------------------------------------------------ */

/* c1 = a from stream (ENC_A, enc_id, prime) sampled in the NTT domain,
 * c0 = -a s + e + m with e from (ENC_E, enc_id, 0). */
int orc_encrypt(const orc_ctx *c, const double *re, const double *im, int slots,
                double scale, int limbs, uint32_t enc_id, uint64_t *ct) {
  const int N = c->N;
  if (orc_encode(c, re, im, slots, scale, limbs, 0, ct) != 0) return -1;
  int64_t *e = (int64_t *)malloc(sizeof(int64_t) * N);
  sample_cbd(c->seed, DOM_ENC_E, enc_id, 0, e, N);
#pragma omp parallel for
  for (int p = 0; p < limbs; p++) {
    const u64 q = c->primes[p];
    u64 *c0 = ct + (size_t)p * N;
    u64 *c1 = ct + ((size_t)limbs + p) * N;
    sample_uniform(c->seed, DOM_ENC_A, enc_id, (uint32_t)p, q, c1, N);
    u64 *en = (u64 *)malloc(sizeof(u64) * N);
    int_to_residues(e, q, en, N);
    orc_ntt_fwd(c, p, en);
    const u64 *s = c->s_ntt + (size_t)p * N;
    for (int i = 0; i < N; i++)
      c0[i] = addmod(submod(en[i], orc_mulmod(c1[i], s[i], q), q), c0[i], q);
    free(en);
  }
  free(e);
  return 0;
}

/* m = c0 + c1 s (+ c2 s^2) in the NTT domain. */
void orc_decrypt_poly(const orc_ctx *c, const uint64_t *ct, int degree,
                      int limbs, uint64_t *out) {
  const int N = c->N;
#pragma omp parallel for
  for (int p = 0; p < limbs; p++) {
    const u64 q = c->primes[p];
    const u64 *s = c->s_ntt + (size_t)p * N;
    for (int i = 0; i < N; i++) {
      u64 acc = 0, spow = 1;
      for (int d = 0; d < degree; d++) {
        acc = addmod(acc, orc_mulmod(ct[((size_t)d * limbs + p) * N + i], spow, q), q);
        spow = orc_mulmod(spow, s[i], q);
      }
      out[(size_t)p * N + i] = acc;
    }
  }
}

void orc_decrypt(const orc_ctx *c, const uint64_t *ct, int degree, int limbs,
                 int slots, double scale, double *re, double *im) {
  u64 *m = (u64 *)malloc(sizeof(u64) * (size_t)limbs * c->N);
  orc_decrypt_poly(c, ct, degree, limbs, m);
  orc_decode(c, m, limbs, slots, scale, re, im);
  free(m);
}

/* ------------------------------------------------------------------------ */
/* evaluation                                                                */
/* ------------------------------------------------------------------------ */

void orc_add(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
             uint64_t *out, int polys, int limbs) {
  const int N = c->N;
  for (int d = 0; d < polys; d++)
    for (int p = 0; p < limbs; p++) {
      size_t o = ((size_t)d * limbs + p) * N;
      for (int i = 0; i < N; i++) out[o + i] = addmod(a[o + i], b[o + i], c->primes[p]);
    }
}

void orc_sub(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
             uint64_t *out, int polys, int limbs) {
  const int N = c->N;
  for (int d = 0; d < polys; d++)
    for (int p = 0; p < limbs; p++) {
      size_t o = ((size_t)d * limbs + p) * N;
      for (int i = 0; i < N; i++) out[o + i] = submod(a[o + i], b[o + i], c->primes[p]);
    }
}

void orc_mul_pt(const orc_ctx *c, const uint64_t *ct, const uint64_t *pt,
                uint64_t *out, int limbs) {
  const int N = c->N;
  for (int d = 0; d < 2; d++)
    for (int p = 0; p < limbs; p++) {
      size_t o = ((size_t)d * limbs + p) * N;
      for (int i = 0; i < N; i++)
        out[o + i] = orc_mulmod(ct[o + i], pt[(size_t)p * N + i], c->primes[p]);
    }
}

/* Multiplication by X^(N/2) (slots times i) or -X^(N/2) (slots times -i).
 * In the NTT domain evaluation point i is psi^(2 br(i) + 1), so X^(N/2)
 * evaluates to I (-1)^(br(i)) with I = psi^(N/2): +I for i < N/2 and -I for
 * i >= N/2. */
void orc_mul_monomial_half(const orc_ctx *c, const uint64_t *ct, uint64_t *out,
                           int polys, int limbs, int negative) {
  const int N = c->N;
  for (int p = 0; p < limbs; p++) {
    const u64 q = c->primes[p];
    /* psi_br[N/2 ... ]: psi^(br(1)) = psi^(N/2) since br(1) = N/2 */
    u64 I = c->psi[p][1];
    u64 lo = negative ? q - I : I, hi = negative ? I : q - I;
    for (int d = 0; d < polys; d++) {
      size_t o = ((size_t)d * limbs + p) * N;
      for (int i = 0; i < N; i++)
        out[o + i] = orc_mulmod(ct[o + i], i < N / 2 ? lo : hi, q);
    }
  }
}

void orc_tensor(const orc_ctx *c, const uint64_t *a, const uint64_t *b,
                uint64_t *out3, int limbs) {
  const int N = c->N;
#pragma omp parallel for
  for (int p = 0; p < limbs; p++) {
    const u64 q = c->primes[p];
    const u64 *a0 = a + (size_t)p * N, *a1 = a + ((size_t)limbs + p) * N;
    const u64 *b0 = b + (size_t)p * N, *b1 = b + ((size_t)limbs + p) * N;
    u64 *d0 = out3 + (size_t)p * N, *d1 = out3 + ((size_t)limbs + p) * N,
        *d2 = out3 + ((size_t)2 * limbs + p) * N;
    for (int i = 0; i < N; i++) {
      d0[i] = orc_mulmod(a0[i], b0[i], q);
      d1[i] = addmod(orc_mulmod(a0[i], b1[i], q), orc_mulmod(a1[i], b0[i], q), q);
      d2[i] = orc_mulmod(a1[i], b1[i], q);
    }
  }
}

/* Fast basis conversion (Bajard-Eynard-Hasan-Zucca 2016):
 * y_t = sum_i [x_i (Q/q_i)^-1]_{q_i} (Q/q_i) mod t over source primes src.
 * With `centered`, each v_i = [x_i (Q/q_i)^-1]_{q_i} is taken in
 * (-q_i/2, q_i/2], i.e. y_t -= #{i : v_i > (q_i - 1)/2} Q mod t; the
 * conversion error u Q then has |u| <= ns/2 and mean ~0 instead of
 * 0 <= u < ns (used by ModDown, where a biased u shows up in the slots). */
static void basis_convert(const orc_ctx *c, const u64 *const *x, const int *src,
                          int ns, const int *dst, int nd, u64 *const *y, int centered) {
  const int N = c->N;
  u64 *hinv = (u64 *)malloc(sizeof(u64) * ns);
  u64 *hmod = (u64 *)malloc(sizeof(u64) * ns * nd);
  u64 *qmod = (u64 *)malloc(sizeof(u64) * nd); /* Q_src mod t */
  for (int t = 0; t < nd; t++) {
    u64 qt = c->primes[dst[t]], m = 1;
    for (int j = 0; j < ns; j++) m = orc_mulmod(m, c->primes[src[j]] % qt, qt);
    qmod[t] = m;
  }
  for (int i = 0; i < ns; i++) {
    u64 qi = c->primes[src[i]];
    u64 h = 1;
    for (int j = 0; j < ns; j++)
      if (j != i) h = orc_mulmod(h, c->primes[src[j]] % qi, qi);
    hinv[i] = invmod(h, qi);
    for (int t = 0; t < nd; t++) {
      u64 qt = c->primes[dst[t]];
      u64 ht = 1;
      for (int j = 0; j < ns; j++)
        if (j != i) ht = orc_mulmod(ht, c->primes[src[j]] % qt, qt);
      hmod[i * nd + t] = ht;
    }
  }
#pragma omp parallel
  {
    u64 v[64];
#pragma omp for
    for (int k = 0; k < N; k++) {
      u64 cnt = 0;
      for (int i = 0; i < ns; i++) {
        u64 qi = c->primes[src[i]];
        v[i] = orc_mulmod(x[i][k], hinv[i], qi);
        if (centered && v[i] > (qi - 1) / 2) cnt++;
      }
      for (int t = 0; t < nd; t++) {
        u64 qt = c->primes[dst[t]];
        u128 acc = 0;
        for (int i = 0; i < ns; i++) {
          acc += (u128)v[i] * hmod[i * nd + t];
          if ((i & 15) == 15) acc = mod128(acc, qt);
        }
        y[t][k] = submod(mod128(acc, qt), orc_mulmod(cnt, qmod[t], qt), qt);
      }
    }
  }
  free(hinv);
  free(hmod);
  free(qmod);
}

/* ModUp of an NTT-domain polynomial d over Q_limbs: ext[j] over Q_limbs u P
 * for each digit j; limbs of digit j are copied, the others are the fast
 * basis conversion of the digit's coefficients, moved to the NTT domain. */
void orc_modup(const orc_ctx *c, const uint64_t *d, int limbs, uint64_t *ext) {
  const int N = c->N, ds = c->ds, E = limbs + c->alpha;
  const int digits = (limbs + ds - 1) / ds;
  u64 *coeff = (u64 *)malloc(sizeof(u64) * (size_t)limbs * N);
  memcpy(coeff, d, sizeof(u64) * (size_t)limbs * N);
  orc_ntt_inv_limbs(c, coeff, limbs, limbs);
  for (int j = 0; j < digits; j++) {
    int lo = j * ds, hi = (j + 1) * ds < limbs ? (j + 1) * ds : limbs;
    int ns = hi - lo, nd = E - ns;
    int src[64], dst[128];
    const u64 *xs[64];
    u64 *ys[128];
    u64 *base = ext + (size_t)j * E * N;
    for (int i = 0; i < ns; i++) {
      src[i] = lo + i;
      xs[i] = coeff + (size_t)(lo + i) * N;
      memcpy(base + (size_t)(lo + i) * N, d + (size_t)(lo + i) * N, sizeof(u64) * N);
    }
    int t = 0;
    for (int l = 0; l < E; l++) {
      if (l >= lo && l < hi) continue;
      dst[t] = prime_of(c, l, limbs);
      ys[t] = base + (size_t)l * N;
      t++;
    }
    basis_convert(c, xs, src, ns, dst, nd, ys, 0);
#pragma omp parallel for
    for (int l = 0; l < E; l++) {
      if (l >= lo && l < hi) continue;
      orc_ntt_fwd(c, prime_of(c, l, limbs), base + (size_t)l * N);
    }
  }
  free(coeff);
}

/* ModDown: out_i = (acc_i - Conv_{P->q_i}([acc]_P)) P^-1 mod q_i with the
 * centered conversion. */
void orc_moddown(const orc_ctx *c, const uint64_t *acc, int limbs, uint64_t *out) {
  const int N = c->N, A = c->alpha, L = c->L;
  u64 *yp = (u64 *)malloc(sizeof(u64) * (size_t)A * N);
  memcpy(yp, acc + (size_t)limbs * N, sizeof(u64) * (size_t)A * N);
  int src[64];
  const u64 *xs[64];
  for (int j = 0; j < A; j++) {
    src[j] = L + j;
    xs[j] = yp + (size_t)j * N;
  }
#pragma omp parallel for
  for (int j = 0; j < A; j++) orc_ntt_inv(c, L + j, yp + (size_t)j * N);
  int dst[64];
  u64 *ys[64];
  for (int i = 0; i < limbs; i++) {
    dst[i] = i;
    ys[i] = out + (size_t)i * N;
  }
  basis_convert(c, xs, src, A, dst, limbs, ys, 1);
#pragma omp parallel for
  for (int i = 0; i < limbs; i++) {
    const u64 q = c->primes[i];
    u64 Pm = 1;
    for (int j = 0; j < A; j++) Pm = orc_mulmod(Pm, c->primes[L + j] % q, q);
    u64 Pinv = invmod(Pm, q);
    u64 *o = out + (size_t)i * N;
    orc_ntt_fwd(c, i, o);
    const u64 *a = acc + (size_t)i * N;
    for (int k = 0; k < N; k++) o[k] = orc_mulmod(submod(a[k], o[k], q), Pinv, q);
  }
  free(yp);
}

/* Key inner product over Q_limbs u P: acc_c = sum_j ext_j key_j[c]. */
static void key_inner(const orc_ctx *c, const orc_key *k, const u64 *ext,
                      int limbs, u64 *acc0, u64 *acc1) {
  const int N = c->N, E = limbs + c->alpha, K = c->K;
  const int digits = (limbs + c->ds - 1) / c->ds;
#pragma omp parallel for
  for (int l = 0; l < E; l++) {
    int p = prime_of(c, l, limbs);
    const u64 q = c->primes[p];
    for (int i = 0; i < N; i++) {
      u128 s0 = 0, s1 = 0;
      for (int j = 0; j < digits; j++) {
        u64 x = ext[((size_t)j * E + l) * N + i];
        s0 += (u128)x * k->data[((size_t)(j * 2 + 0) * K + p) * N + i];
        s1 += (u128)x * k->data[((size_t)(j * 2 + 1) * K + p) * N + i];
      }
      acc0[(size_t)l * N + i] = mod128(s0, q);
      acc1[(size_t)l * N + i] = mod128(s1, q);
    }
  }
}

int orc_keyswitch(const orc_ctx *c, uint64_t g, const uint64_t *d, int limbs,
                  uint64_t *out0, uint64_t *out1) {
  const orc_key *k = find_key(c, g);
  if (!k) return -1;
  const int N = c->N, E = limbs + c->alpha;
  const int digits = (limbs + c->ds - 1) / c->ds;
  u64 *ext = (u64 *)malloc(sizeof(u64) * (size_t)digits * E * N);
  u64 *acc0 = (u64 *)malloc(sizeof(u64) * (size_t)E * N);
  u64 *acc1 = (u64 *)malloc(sizeof(u64) * (size_t)E * N);
  orc_modup(c, d, limbs, ext);
  key_inner(c, k, ext, limbs, acc0, acc1);
  orc_moddown(c, acc0, limbs, out0);
  orc_moddown(c, acc1, limbs, out1);
  free(ext);
  free(acc0);
  free(acc1);
  return 0;
}

int orc_relinearize(const orc_ctx *c, const uint64_t *ct3, int limbs, uint64_t *out) {
  const int N = c->N;
  size_t P = (size_t)limbs * N;
  u64 *k0 = (u64 *)malloc(sizeof(u64) * P), *k1 = (u64 *)malloc(sizeof(u64) * P);
  int r = orc_keyswitch(c, 0, ct3 + 2 * P, limbs, k0, k1);
  if (r == 0) {
    orc_add(c, ct3, k0, out, 1, limbs);
    orc_add(c, ct3 + P, k1, out + P, 1, limbs);
  }
  free(k0);
  free(k1);
  return r;
}

/* Rotation = hoisted rotation with one Galois element: ModUp(c1), then the
 * NTT-domain automorphism of each digit, key inner product, ModDown, plus
 * sigma_g(c0).  (Applying sigma before or after ModUp gives different, equally
 * valid approximate base conversions; this backend fixes "after" everywhere.) */
int orc_rotate(const orc_ctx *c, const uint64_t *ct, int limbs, uint64_t g,
               uint64_t *out) {
  return orc_hoisted_rotate(c, ct, limbs, &g, 1, out);
}

/* Hoisted rotations: one ModUp of c1, then per Galois element the NTT-domain
 * automorphism of every ModUp digit, the key inner product and ModDown.
 * g = 1 is the identity (copy, no key switch). */
int orc_hoisted_rotate(const orc_ctx *c, const uint64_t *ct, int limbs,
                       const uint64_t *gs, int n, uint64_t *outs) {
  const int N = c->N, E = limbs + c->alpha;
  const int digits = (limbs + c->ds - 1) / c->ds;
  size_t P = (size_t)limbs * N;
  for (int r = 0; r < n; r++)
    if (gs[r] != 1 && !find_key(c, gs[r])) return -1;
  u64 *ext = (u64 *)malloc(sizeof(u64) * (size_t)digits * E * N);
  u64 *extg = (u64 *)malloc(sizeof(u64) * (size_t)digits * E * N);
  u64 *acc0 = (u64 *)malloc(sizeof(u64) * (size_t)E * N);
  u64 *acc1 = (u64 *)malloc(sizeof(u64) * (size_t)E * N);
  u64 *k0 = (u64 *)malloc(sizeof(u64) * P);
  orc_modup(c, ct + P, limbs, ext);
  for (int r = 0; r < n; r++) {
    u64 *o = outs + (size_t)r * 2 * P;
    if (gs[r] == 1) {
      memcpy(o, ct, sizeof(u64) * 2 * P);
      continue;
    }
    orc_automorphism_ntt(c, gs[r], ext, extg, digits * E);
    key_inner(c, find_key(c, gs[r]), extg, limbs, acc0, acc1);
    orc_moddown(c, acc0, limbs, k0);
    orc_moddown(c, acc1, limbs, o + P);
    orc_automorphism_ntt(c, gs[r], ct, o, limbs);
    orc_add(c, o, k0, o, 1, limbs);
  }
  free(ext);
  free(extg);
  free(acc0);
  free(acc1);
  free(k0);
  return 0;
}

/* Rescale by the last prime with rounding: c'_i = (c_i - r) q_last^-1 mod q_i
 * where r is the centered residue of c mod q_last. */
void orc_rescale(const orc_ctx *c, const uint64_t *ct, int polys, int limbs,
                 uint64_t *out) {
  const int N = c->N, l1 = limbs - 1;
  const u64 ql = c->primes[l1];
  u64 *last = (u64 *)malloc(sizeof(u64) * N);
  for (int d = 0; d < polys; d++) {
    memcpy(last, ct + ((size_t)d * limbs + l1) * N, sizeof(u64) * N);
    orc_ntt_inv(c, l1, last);
#pragma omp parallel for
    for (int i = 0; i < l1; i++) {
      const u64 q = c->primes[i];
      const u64 qlm = ql % q;
      const u64 inv = invmod(qlm, q);
      u64 *r = (u64 *)malloc(sizeof(u64) * N);
      for (int k = 0; k < N; k++) {
        u64 v = last[k];
        r[k] = v > (ql - 1) / 2 ? submod(mod128(v, q), qlm, q) : mod128(v, q);
      }
      orc_ntt_fwd(c, i, r);
      const u64 *src = ct + ((size_t)d * limbs + i) * N;
      u64 *dst = out + ((size_t)d * l1 + i) * N;
      for (int k = 0; k < N; k++) dst[k] = orc_mulmod(submod(src[k], r[k], q), inv, q);
      free(r);
    }
  }
  free(last);
}

/* ModRaise (bootstrap step 1): every polynomial of a one-limb ciphertext is
 * read as integers in (-q_0/2, q_0/2] and reduced into `target` limbs. */
void orc_mod_raise(const orc_ctx *c, const uint64_t *ct, int polys, int target,
                   uint64_t *out) {
  const int N = c->N;
  const u64 q0 = c->primes[0];
  u64 *coef = (u64 *)malloc(sizeof(u64) * N);
  for (int d = 0; d < polys; d++) {
    memcpy(coef, ct + (size_t)d * N, sizeof(u64) * N);
    orc_ntt_inv(c, 0, coef);
#pragma omp parallel for
    for (int i = 0; i < target; i++) {
      const u64 q = c->primes[i];
      u64 *dst = out + ((size_t)d * target + i) * N;
      for (int k = 0; k < N; k++) {
        u64 v = coef[k];
        dst[k] = v > (q0 - 1) / 2 ? submod(mod128(v, q), q0 % q, q) : mod128(v, q);
      }
      orc_ntt_fwd(c, i, dst);
    }
  }
  free(coef);
}

void orc_drop_limbs(const orc_ctx *c, const uint64_t *ct, int polys, int limbs,
                    int target, uint64_t *out) {
  const int N = c->N;
  for (int d = 0; d < polys; d++)
    memcpy(out + (size_t)d * target * N, ct + (size_t)d * limbs * N,
           sizeof(u64) * (size_t)target * N);
}

/* BSGS diagonal MAC, "normal" strategy (reference call site
 * operators/linear/operator.py:320-330):
 *   sum_{g<G} rot_{giant}^g ( sum_{b<B} pt[g B + b] * rot_{baby_b}(ct) )
 * with babies from one hoisted ModUp and a Horner chain over giants.
 * The result is unrescaled (scale = scale_ct * scale_pt). */
int orc_hoisted_mac_sum(const orc_ctx *c, const uint64_t *ct, int limbs,
                        const uint64_t *baby_gs, int B, const uint64_t *pts,
                        uint64_t giant_g, int G, uint64_t *out) {
  const int N = c->N;
  size_t P = (size_t)limbs * N;
  u64 *babies = (u64 *)malloc(sizeof(u64) * (size_t)B * 2 * P);
  if (orc_hoisted_rotate(c, ct, limbs, baby_gs, B, babies) != 0) {
    free(babies);
    return -1;
  }
  if (G > 1 && giant_g != 1 && !find_key(c, giant_g)) {
    free(babies);
    return -1;
  }
  u64 *inner = (u64 *)malloc(sizeof(u64) * 2 * P);
  u64 *tmp = (u64 *)malloc(sizeof(u64) * 2 * P);
  for (int g = G - 1; g >= 0; g--) {
#pragma omp parallel for
    for (int p = 0; p < limbs; p++) {
      const u64 q = c->primes[p];
      for (int d = 0; d < 2; d++) {
        u64 *dst = inner + ((size_t)d * limbs + p) * N;
        for (int i = 0; i < N; i++) {
          u128 s = 0;
          for (int b = 0; b < B; b++) {
            s += (u128)babies[(size_t)b * 2 * P + ((size_t)d * limbs + p) * N + i] *
                 pts[((size_t)(g * B + b) * limbs + p) * N + i];
            if ((b & 15) == 15) s = mod128(s, q);
          }
          dst[i] = mod128(s, q);
        }
      }
    }
    if (g == G - 1) {
      memcpy(out, inner, sizeof(u64) * 2 * P);
    } else {
      orc_rotate(c, out, limbs, giant_g, tmp);
      orc_add(c, tmp, inner, out, 2, limbs);
    }
  }
  free(inner);
  free(tmp);
  free(babies);
  return 0;
}

/* Extended-basis BSGS MAC (hoisted_mac_sum strategies "ext_normal" and
 * "ext_double_hoist"): every baby stays in the Q u P basis, as
 * (P sigma(c0) + acc_0, acc_1) for a rotation or (P c0, P c1) for offset 0,
 * without its ModDown; the plaintexts carry P limbs ([G*B][limbs+alpha][N]);
 * each giant group sum_b pt_b babies_b is brought back to Q by one ModDown,
 * then the Horner chain over the giant key runs as in orc_hoisted_mac_sum. */
/* Extended-basis babies of ct for the Galois elements baby_gs (keys present):
 * bab[b] = [2][E][N] holding (P c0, P c1) for g = 1, (P sigma(c0) + acc_0, acc_1)
 * otherwise, from one ModUp of c1. */
static void ext_babies(const orc_ctx *c, const uint64_t *ct, int limbs, const uint64_t *baby_gs,
                       int B, u64 *bab) {
  const int N = c->N, A = c->alpha, L = c->L, E = limbs + A;
  const int digits = (limbs + c->ds - 1) / c->ds;
  const size_t P = (size_t)limbs * N, EP = (size_t)E * N;
  u64 *ext = (u64 *)malloc(sizeof(u64) * (size_t)digits * EP);
  u64 *extg = (u64 *)malloc(sizeof(u64) * (size_t)digits * EP);
  u64 *sc0 = (u64 *)malloc(sizeof(u64) * P);
  u64 Pm[64];
  for (int i = 0; i < limbs; i++) {
    Pm[i] = 1;
    for (int j = 0; j < A; j++) Pm[i] = orc_mulmod(Pm[i], c->primes[L + j] % c->primes[i], c->primes[i]);
  }
  orc_modup(c, ct + P, limbs, ext);
  for (int b = 0; b < B; b++) {
    u64 *b0 = bab + (size_t)b * 2 * EP, *b1 = b0 + EP;
    if (baby_gs[b] == 1) {
      memset(b0, 0, sizeof(u64) * 2 * EP);
      for (int d = 0; d < 2; d++)
        for (int i = 0; i < limbs; i++)
          for (int k = 0; k < N; k++)
            (d ? b1 : b0)[(size_t)i * N + k] =
                orc_mulmod(ct[(size_t)d * P + (size_t)i * N + k], Pm[i], c->primes[i]);
      continue;
    }
    orc_automorphism_ntt(c, baby_gs[b], ext, extg, digits * E);
    key_inner(c, find_key(c, baby_gs[b]), extg, limbs, b0, b1);
    orc_automorphism_ntt(c, baby_gs[b], ct, sc0, limbs);
    for (int i = 0; i < limbs; i++)
      for (int k = 0; k < N; k++) {
        u64 *x = b0 + (size_t)i * N + k;
        *x = addmod(*x, orc_mulmod(sc0[(size_t)i * N + k], Pm[i], c->primes[i]), c->primes[i]);
      }
  }
  free(ext);
  free(extg);
  free(sc0);
}

/* inner = sum_b pts[g B + b] * bab[b] over Q_limbs u P, both components */
static void ext_inner(const orc_ctx *c, const u64 *bab, int B, const uint64_t *pts, int g,
                      int limbs, u64 *inner_ext) {
  const int N = c->N, E = limbs + c->alpha;
  const size_t EP = (size_t)E * N;
#pragma omp parallel for
  for (int l = 0; l < E; l++) {
    const u64 q = c->primes[prime_of(c, l, limbs)];
    for (int d = 0; d < 2; d++) {
      u64 *dst = inner_ext + (size_t)d * EP + (size_t)l * N;
      for (int i = 0; i < N; i++) {
        u128 s = 0;
        for (int b = 0; b < B; b++) {
          s += (u128)bab[(size_t)b * 2 * EP + (size_t)d * EP + (size_t)l * N + i] *
               pts[((size_t)(g * B + b) * E + l) * N + i];
          if ((b & 15) == 15) s = mod128(s, q);
        }
        dst[i] = mod128(s, q);
      }
    }
  }
}

int orc_hoisted_mac_sum_ext(const orc_ctx *c, const uint64_t *ct, int limbs,
                            const uint64_t *baby_gs, int B, const uint64_t *pts,
                            uint64_t giant_g, int G, uint64_t *out) {
  const int N = c->N, A = c->alpha, E = limbs + A;
  const size_t P = (size_t)limbs * N, EP = (size_t)E * N;
  for (int b = 0; b < B; b++)
    if (baby_gs[b] != 1 && !find_key(c, baby_gs[b])) return -1;
  if (G > 1 && giant_g != 1 && !find_key(c, giant_g)) return -1;
  u64 *bab = (u64 *)malloc(sizeof(u64) * (size_t)B * 2 * EP);
  ext_babies(c, ct, limbs, baby_gs, B, bab);
  u64 *inner_ext = (u64 *)malloc(sizeof(u64) * 2 * EP);
  u64 *inner = (u64 *)malloc(sizeof(u64) * 2 * P);
  u64 *tmp = (u64 *)malloc(sizeof(u64) * 2 * P);
  for (int g = G - 1; g >= 0; g--) {
    ext_inner(c, bab, B, pts, g, limbs, inner_ext);
    orc_moddown(c, inner_ext, limbs, inner);
    orc_moddown(c, inner_ext + EP, limbs, inner + P);
    if (g == G - 1) {
      memcpy(out, inner, sizeof(u64) * 2 * P);
    } else {
      orc_rotate(c, out, limbs, giant_g, tmp);
      orc_add(c, tmp, inner, out, 2, limbs);
    }
  }
  free(bab);
  free(inner_ext);
  free(inner);
  free(tmp);
  return 0;
}

/* Double-hoisted schedule (ext_double_hoist): the babies and every giant
 * group's inner sum u_g = (u0, u1) stay in Q_limbs u P; each giant group g >= 1
 * is rotated there by its own Galois element G_g (the rotation by g giant
 * steps): v = ModDown(u1) (one polynomial), then
 *   (sigma(u0) + KS_0(sigma(v)), KS_1(sigma(v)))  before its ModDown,
 * KS = the key product of ModUp(sigma(v)); the groups are summed in Q u P and
 * one ModDown of the sum ends it.  Using sigma(u0) for P sigma(ModDown(u0))
 * and the ModDown of u1 only leaves a rounding error of a key switch's
 * ModDown size (the message is P times the decrypted value). */
int orc_hoisted_mac_sum_double(const orc_ctx *c, const uint64_t *ct, int limbs,
                               const uint64_t *baby_gs, int B, const uint64_t *pts,
                               const uint64_t *giant_gs, int G, uint64_t *out) {
  const int N = c->N, A = c->alpha, E = limbs + A;
  const int digits = (limbs + c->ds - 1) / c->ds;
  const size_t P = (size_t)limbs * N, EP = (size_t)E * N;
  for (int b = 0; b < B; b++)
    if (baby_gs[b] != 1 && !find_key(c, baby_gs[b])) return -1;
  for (int g = 1; g < G; g++)
    if (giant_gs[g] != 1 && !find_key(c, giant_gs[g])) return -1;
  u64 *bab = (u64 *)malloc(sizeof(u64) * (size_t)B * 2 * EP);
  ext_babies(c, ct, limbs, baby_gs, B, bab);
  u64 *total = (u64 *)malloc(sizeof(u64) * 2 * EP);
  u64 *inner = (u64 *)malloc(sizeof(u64) * 2 * EP);
  u64 *v = (u64 *)malloc(sizeof(u64) * P);
  u64 *ext = (u64 *)malloc(sizeof(u64) * (size_t)digits * EP);
  u64 *extg = (u64 *)malloc(sizeof(u64) * (size_t)digits * EP);
  u64 *k0 = (u64 *)malloc(sizeof(u64) * EP);
  u64 *k1 = (u64 *)malloc(sizeof(u64) * EP);
  u64 *su0 = (u64 *)malloc(sizeof(u64) * EP);
  ext_inner(c, bab, B, pts, 0, limbs, total);
  for (int g = 1; g < G; g++) {
    ext_inner(c, bab, B, pts, g, limbs, inner);
    if (giant_gs[g] == 1) {
      for (int d = 0; d < 2; d++)
        for (int l = 0; l < E; l++) {
          const u64 q = c->primes[prime_of(c, l, limbs)];
          for (int i = 0; i < N; i++) {
            const size_t o = (size_t)d * EP + (size_t)l * N + i;
            total[o] = addmod(total[o], inner[o], q);
          }
        }
      continue;
    }
    orc_moddown(c, inner + EP, limbs, v);
    orc_modup(c, v, limbs, ext);
    orc_automorphism_ntt(c, giant_gs[g], ext, extg, digits * E);
    key_inner(c, find_key(c, giant_gs[g]), extg, limbs, k0, k1);
    orc_automorphism_ntt(c, giant_gs[g], inner, su0, E);
    for (int l = 0; l < E; l++) {
      const u64 q = c->primes[prime_of(c, l, limbs)];
      for (int i = 0; i < N; i++) {
        const size_t o = (size_t)l * N + i;
        total[o] = addmod(total[o], addmod(su0[o], k0[o], q), q);
        total[EP + o] = addmod(total[EP + o], k1[o], q);
      }
    }
  }
  orc_moddown(c, total, limbs, out);
  orc_moddown(c, total + EP, limbs, out + P);
  free(bab);
  free(total);
  free(inner);
  free(v);
  free(ext);
  free(extg);
  free(k0);
  free(k1);
  free(su0);
  return 0;
}
