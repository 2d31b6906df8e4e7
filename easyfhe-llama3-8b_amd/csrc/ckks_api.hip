// ckks_api.hip -- context set-up, device memory pool, key-switching pipeline
// and the extern "C" entry points declared in include/ckks_mi355x.h.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <thread>

#include "ckks_internal.hpp"

typedef unsigned __int128 u128;
using namespace ckks;

// ===========================================================================
// errors
// ===========================================================================

static thread_local std::string g_err;

const char *ckks_last_error(void) { return g_err.c_str(); }

#define HIPCHECK(x)                                                          \
  do {                                                                       \
    hipError_t e_ = (x);                                                     \
    if (e_ != hipSuccess)                                                    \
      throw std::runtime_error(std::string(#x ": ") + hipGetErrorString(e_)); \
  } while (0)

struct KeyMissing : std::runtime_error {
  using std::runtime_error::runtime_error;
};

#define API_BEGIN try {
#define API_END                                   \
  return CKKS_OK;                                 \
  }                                               \
  catch (const std::invalid_argument &e) {        \
    g_err = e.what();                             \
    return CKKS_EINVAL;                           \
  }                                               \
  catch (const KeyMissing &e) {                   \
    g_err = e.what();                             \
    return CKKS_ENOKEY;                           \
  }                                               \
  catch (const std::exception &e) {               \
    g_err = e.what();                             \
    return CKKS_ERUNTIME;                         \
  }

static void require(bool cond, const std::string &msg) {
  if (!cond) throw std::invalid_argument(msg);
}

// Live contexts and their serials: an object released after its context was
// destroyed only drops its host record (the device memory went with the
// context; a later context may reuse the address, the serial tells them
// apart).
static std::unordered_map<ckks_context *, u64> g_live_contexts;
static u64 g_next_serial = 1;

static bool owner_alive(const ckks_context *c, u64 serial) {
  auto it = g_live_contexts.find(const_cast<ckks_context *>(c));
  return it != g_live_contexts.end() && it->second == serial;
}

// ===========================================================================
// host number theory (prime rule, roots, constants)
// ===========================================================================

static u64 mulmod_h(u64 a, u64 b, u64 q) { return (u64)(((u128)a * b) % q); }

static u64 powmod_h(u64 a, u64 e, u64 q) {
  u64 r = 1 % q;
  a %= q;
  while (e) {
    if (e & 1) r = mulmod_h(r, a, q);
    a = mulmod_h(a, a, q);
    e >>= 1;
  }
  return r;
}

static u64 invmod_h(u64 a, u64 q) { return powmod_h(a % q, q - 2, q); }

static bool is_prime_h(u64 n) {
  static const u64 bases[12] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return false;
  for (u64 b : bases) {
    if (n == b) return true;
    if (n % b == 0) return false;
  }
  u64 d = n - 1;
  int r = 0;
  while (!(d & 1)) {
    d >>= 1;
    r++;
  }
  for (u64 b : bases) {
    u64 x = powmod_h(b, d, n);
    if (x == 1 || x == n - 1) continue;
    bool comp = true;
    for (int k = 1; k < r && comp; k++) {
      x = mulmod_h(x, x, n);
      if (x == n - 1) comp = false;
    }
    if (comp) return false;
  }
  return true;
}

// Primes q = 1 mod 2N nearest to 2^bits (2^bits + 1 first, then for each
// distance k*2N the one below before the one above), never >= 2^60.
static std::vector<u64> prime_chain(int logN, int bits, int count, const std::vector<u64> &used) {
  const u64 M = (u64)2 << logN, base = (u64)1 << bits, cap = (u64)1 << 60;
  std::vector<u64> out;
  for (u64 k = 0; (int)out.size() < count; k++) {
    if (k * M >= base && base + k * M + 1 >= cap) break;
    u64 cands[2];
    int nc = 0;
    if (k == 0)
      cands[nc++] = base + 1;
    else {
      if (k * M < base) cands[nc++] = base - k * M + 1;
      cands[nc++] = base + k * M + 1;
    }
    for (int i = 0; i < nc && (int)out.size() < count; i++) {
      u64 cnd = cands[i];
      if (cnd >= cap || cnd <= M) continue;
      if (std::find(used.begin(), used.end(), cnd) != used.end()) continue;
      if (std::find(out.begin(), out.end(), cnd) != out.end()) continue;
      if (is_prime_h(cnd)) out.push_back(cnd);
    }
  }
  if ((int)out.size() != count) throw std::invalid_argument("prime search exhausted");
  return out;
}

// Smallest primitive 2N-th root: psi0 from the first x with psi0^N = -1,
// then the minimum over its odd powers.
static u64 min_root_h(u64 q, int logN) {
  const u64 N = (u64)1 << logN, M = 2 * N;
  u64 psi0 = 0;
  for (u64 x = 2;; x++) {
    psi0 = powmod_h(x, (q - 1) / M, q);
    if (powmod_h(psi0, N, q) == q - 1) break;
  }
  u64 sq = mulmod_h(psi0, psi0, q), cur = psi0, best = psi0;
  for (u64 k = 1; k < N; k++) {
    cur = mulmod_h(cur, sq, q);
    best = std::min(best, cur);
  }
  return best;
}

static u32 bitrev_h(u32 x, int bits) {
  u32 r = 0;
  for (int i = 0; i < bits; i++) {
    r = (r << 1) | (x & 1);
    x >>= 1;
  }
  return r;
}

static u64 shoup_h(u64 w, u64 q) { return (u64)(((u128)w << 64) / q); }

static ModQ make_modq(u64 q) {
  ModQ m{};
  m.q = q;
  u64 inv = q;  // Newton iteration for q^-1 mod 2^64
  for (int i = 0; i < 6; i++) inv *= 2 - q * inv;
  m.qinv = (u64)0 - inv;
  u64 r1 = (u64)((((u128)1) << 64) % q);
  m.r2 = mulmod_h(r1, r1, q);
  int k = 64 - __builtin_clzll(q);
  m.k = (u32)k;
  m.mu = (u64)((((u128)1) << (2 * k)) / q);
  return m;
}

// ChaCha20 block (RFC 8439) for the host-side secret sampler.
static inline u32 rotl_h(u32 v, int c) { return (v << c) | (v >> (32 - c)); }
static void chacha_h(u64 seed, u32 dom, u32 id, u32 sub, u32 counter, u32 out[16]) {
  u32 s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
               (u32)seed,   (u32)(seed >> 32), 0u, 0u, 0u, 0u, 0u, 0u,
               counter,     dom,         id,          sub};
  u32 x[16];
  memcpy(x, s, sizeof(s));
  auto qr = [&](int a, int b, int c, int d) {
    x[a] += x[b]; x[d] ^= x[a]; x[d] = rotl_h(x[d], 16);
    x[c] += x[d]; x[b] ^= x[c]; x[b] = rotl_h(x[b], 12);
    x[a] += x[b]; x[d] ^= x[a]; x[d] = rotl_h(x[d], 8);
    x[c] += x[d]; x[b] ^= x[c]; x[b] = rotl_h(x[b], 7);
  };
  for (int i = 0; i < 10; i++) {
    qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);
    qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);
  }
  for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

// Secret rule: sparse ternary of weight h by a partial Fisher-Yates shuffle
// (64-bit words t = 0, 1, ... of stream (SECRET, 0, 0): position word, sign
// word), or uniform ternary (word mod 3 - 1).
static std::vector<int8_t> sample_secret(u64 seed, int N, int mode, int h) {
  std::vector<int8_t> s(N, 0);
  u64 word = 0;
  auto next = [&]() {
    u32 blk[16];
    chacha_h(seed, 1, 0, 0, (u32)(word >> 3), blk);
    int r = (int)(word & 7);
    word++;
    return (u64)blk[2 * r] | ((u64)blk[2 * r + 1] << 32);
  };
  if (mode == 0) {
    std::vector<u32> perm(N);
    for (int i = 0; i < N; i++) perm[i] = (u32)i;
    for (int t = 0; t < h; t++) {
      u64 r = next(), sg = next();
      u64 j = (u64)t + r % (u64)(N - t);
      std::swap(perm[t], perm[j]);
      s[perm[t]] = (sg & 1) ? -1 : 1;
    }
  } else {
    for (int i = 0; i < N; i++) s[i] = (int8_t)((int)(next() % 3) - 1);
  }
  return s;
}

template <class F>
static void parallel_for(int n, F f) {
  unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> th;
  for (unsigned w = 0; w < hw; w++)
    th.emplace_back([&, w]() {
      for (int i = (int)w; i < n; i += (int)hw) f(i);
    });
  for (auto &t : th) t.join();
}

// ===========================================================================
// per-level constant tables (built once, device resident)
// ===========================================================================

static BCTable make_bc(ckks_context *c, const std::vector<u64> &src, const std::vector<u64> &dst) {
  const int ns = (int)src.size(), nd = (int)dst.size();
  // the conversion kernels hold one value per source in registers
  require(ns <= kMaxDigitSize, "basis conversion from more than 16 primes");
  std::vector<u64> h(2 * ns + (size_t)ns * nd + nd);
  for (int t = 0; t < nd; t++) {
    u64 m = 1;
    for (int j = 0; j < ns; j++) m = mulmod_h(m, src[j] % dst[t], dst[t]);
    h[2 * ns + (size_t)ns * nd + t] = m;
  }
  for (int i = 0; i < ns; i++) {
    const u64 qi = src[i];
    u64 prod = 1;
    for (int j = 0; j < ns; j++)
      if (j != i) prod = mulmod_h(prod, src[j] % qi, qi);
    const u64 inv = invmod_h(prod, qi);
    h[i] = inv;
    h[ns + i] = shoup_h(inv, qi);
    for (int t = 0; t < nd; t++) {
      const u64 qt = dst[t];
      u64 pt = 1;
      for (int j = 0; j < ns; j++)
        if (j != i) pt = mulmod_h(pt, src[j] % qt, qt);
      h[2 * ns + (size_t)i * nd + t] = (u64)(((u128)pt << 64) % qt);  // Montgomery form
    }
  }
  BCTable t{ns, nd, nullptr, sizeof(u64) * h.size(), nullptr, 0, 0};
  HIPCHECK(hipMalloc(&t.d, t.bytes));
  HIPCHECK(hipMemcpy(t.d, h.data(), t.bytes, hipMemcpyHostToDevice));
  // the fp64 kernel needs every source prime below 2^45, or every one but
  // the first when no target is wide (the first source's value then enters
  // as two 32-bit halves)
  bool narrow_rest = true, narrow_dst = true;
  for (int i = 1; i < ns; i++) narrow_rest = narrow_rest && src[i] < (1ull << 45);
  for (u64 q : dst) narrow_dst = narrow_dst && q < (1ull << 45);
  const bool narrow0 = src[0] < (1ull << 45);
  t.wide0 = (!narrow0 && narrow_rest && narrow_dst) ? 1 : 0;
  if ((narrow0 && narrow_rest) || t.wide0) {
    // (w, w / q) pairs for the fp64 modular product; hmod in plain form
    std::vector<double> f(2 * ((size_t)ns + (size_t)ns * nd + (t.wide0 ? nd : 0)));
    for (int i = 0; i < ns; i++) {
      f[2 * i] = (double)h[i];
      f[2 * i + 1] = (double)h[i] / (double)src[i];
    }
    for (int i = 0; i < ns; i++) {
      for (int t2 = 0; t2 < nd; t2++) {
        const u64 qt = dst[t2];
        u64 pt = 1;
        for (int j = 0; j < ns; j++)
          if (j != i) pt = mulmod_h(pt, src[j] % qt, qt);
        const size_t o = 2 * ((size_t)ns + (size_t)i * nd + t2);
        f[o] = (double)pt;
        f[o + 1] = (double)pt / (double)qt;
        if (i == 0 && t.wide0) {
          const u64 p32 = (u64)(((u128)pt << 32) % qt);
          const size_t o2 = 2 * ((size_t)ns + (size_t)ns * nd + t2);
          f[o2] = (double)p32;
          f[o2 + 1] = (double)p32 / (double)qt;
        }
      }
    }
    t.fbytes = sizeof(double) * f.size();
    HIPCHECK(hipMalloc(&t.fd, t.fbytes));
    HIPCHECK(hipMemcpy(t.fd, f.data(), t.fbytes, hipMemcpyHostToDevice));
  }
  // the MFMA B operand: for source quad i, target group tg, digit b, lane
  // l = col + 16 g (source s = 4 i + g, target t = 16 tg + col), byte a of
  // the lane's word is the balanced digit b of M'[(s, a)][t]; the balanced
  // digits of x < 2^63 are the bytes of x + 0x80..80, each xor 0x80 (as int8:
  // byte - 128, and sum (byte_b - 128) 256^b = x)
  t.n_k = (ns + 3) / 4;
  t.n_tg = (nd + 15) / 16;
  for (int t2 = 0; t2 < nd; t2++)
    if (dst[t2] >= (1ull << 45)) t.wide_mask |= 1 << (t2 / 16);
  std::vector<u64> m((size_t)t.n_k * t.n_tg * 8 * 64, 0);
  for (int s = 0; s < ns; s++) {
    for (int t2 = 0; t2 < nd; t2++) {
      const u64 qt = dst[t2];
      u64 hm = 1;
      for (int j = 0; j < ns; j++)
        if (j != s) hm = mulmod_h(hm, src[j] % qt, qt);
      const int lane = (t2 % 16) + 16 * (s % 4);
      for (int a = 0; a < 8; a++) {
        const u64 mp = mulmod_h(hm, (1ull << (8 * a)) % qt, qt);
        const u64 mb = mp + 0x8080808080808080ull;
        for (int b = 0; b < 8; b++) {
          const u64 digit = ((mb >> (8 * b)) & 0xff) ^ 0x80;
          m[(((size_t)(s / 4) * t.n_tg + t2 / 16) * 8 + b) * 64 + lane] |= digit << (8 * a);
        }
      }
    }
  }
  t.mbytes = sizeof(u64) * m.size();
  HIPCHECK(hipMalloc(&t.mf, t.mbytes));
  HIPCHECK(hipMemcpy(t.mf, m.data(), t.mbytes, hipMemcpyHostToDevice));
  // k_convert_h4's table: lane m of a group's words moves to the row of its
  // target in the transposed order (m = 4 (t % 4) + (t % 16) / 4 for t's
  // place in the group)
  std::vector<u64> mt(m.size(), 0);
  for (size_t blk = 0; blk < m.size() / 64; blk++)
    for (int gs = 0; gs < 4; gs++)
      for (int tm = 0; tm < 16; tm++) {
        const int row = 4 * (tm % 4) + tm / 4;
        mt[blk * 64 + row + 16 * gs] = m[blk * 64 + tm + 16 * gs];
      }
  HIPCHECK(hipMalloc(&t.mt, t.mbytes));
  HIPCHECK(hipMemcpy(t.mt, mt.data(), t.mbytes, hipMemcpyHostToDevice));
  std::vector<u64> sn(6 * (size_t)ns);
  const int N = c->N;
  for (int i = 0; i < ns; i++) {
    const u64 qi = src[i];
    const u64 w = mulmod_h(h[i], invmod_h((u64)N % qi, qi), qi);
    sn[i] = w;
    sn[ns + i] = shoup_h(w, qi);
    const double wf = (double)w, qf = (double)qi;
    const double wq = wf / qf;
    memcpy(&sn[2 * ns + 2 * i], &wf, 8);
    memcpy(&sn[2 * ns + 2 * i + 1], &wq, 8);
    sn[4 * ns + i] = h[i];
    sn[5 * ns + i] = shoup_h(h[i], qi);
  }
  HIPCHECK(hipMalloc(&t.sn, sizeof(u64) * sn.size()));
  HIPCHECK(hipMemcpy(t.sn, sn.data(), sizeof(u64) * sn.size(), hipMemcpyHostToDevice));
  return t;
}

static const BCTable &bc_up(ckks_context *c, int limbs, int j) {
  auto key = std::make_pair(limbs, j);
  auto it = c->bc_up.find(key);
  if (it != c->bc_up.end()) return it->second;
  const int lo = j * c->ds, hi = std::min((j + 1) * c->ds, limbs);
  const int E = limbs + c->alpha;
  std::vector<u64> src, dst;
  for (int i = lo; i < hi; i++) src.push_back(c->primes[i]);
  for (int l = 0; l < E; l++) {
    if (l >= lo && l < hi) continue;
    dst.push_back(l < limbs ? c->primes[l] : c->primes[c->L + (l - limbs)]);
  }
  return c->bc_up[key] = make_bc(c, src, dst);
}

static const BCTable &bc_down(ckks_context *c, int limbs) {
  auto it = c->bc_down.find(limbs);
  if (it != c->bc_down.end()) return it->second;
  std::vector<u64> src, dst;
  for (int j = 0; j < c->alpha; j++) src.push_back(c->primes[c->L + j]);
  for (int i = 0; i < limbs; i++) dst.push_back(c->primes[i]);
  return c->bc_down[limbs] = make_bc(c, src, dst);
}

// per Q limb i < limbs: P mod q_i and its Shoup constant
static const u64 *pmod_table(ckks_context *c, int limbs) {
  auto it = c->pmod.find(limbs);
  if (it != c->pmod.end()) return it->second;
  std::vector<u64> h(2 * (size_t)limbs);
  for (int i = 0; i < limbs; i++) {
    const u64 q = c->primes[i];
    u64 P = 1;
    for (int j = 0; j < c->alpha; j++) P = mulmod_h(P, c->primes[c->L + j] % q, q);
    h[2 * i] = P;
    h[2 * i + 1] = shoup_h(P, q);
  }
  u64 *d = nullptr;
  HIPCHECK(hipMalloc(&d, sizeof(u64) * h.size()));
  HIPCHECK(hipMemcpy(d, h.data(), sizeof(u64) * h.size(), hipMemcpyHostToDevice));
  return c->pmod[limbs] = d;
}

static const u64 *pinv_table(ckks_context *c, int limbs) {
  auto it = c->pinv.find(limbs);
  if (it != c->pinv.end()) return it->second;
  std::vector<u64> h(2 * (size_t)limbs);
  for (int i = 0; i < limbs; i++) {
    const u64 q = c->primes[i];
    u64 P = 1;
    for (int j = 0; j < c->alpha; j++) P = mulmod_h(P, c->primes[c->L + j] % q, q);
    const u64 inv = invmod_h(P, q);
    h[2 * i] = inv;
    h[2 * i + 1] = shoup_h(inv, q);
  }
  u64 *d = nullptr;
  HIPCHECK(hipMalloc(&d, sizeof(u64) * h.size()));
  HIPCHECK(hipMemcpy(d, h.data(), sizeof(u64) * h.size(), hipMemcpyHostToDevice));
  return c->pinv[limbs] = d;
}

// Relinearise-rescale constants for a ciphertext of `limbs` limbs dropping
// its last D primes p_1 = q_{limbs-1}, p_2, ... (T = limbs - D): [T][2]
// (P p_1..p_D)^-1 mod q_t + shoup, [T][2] (p_1..p_D)^-1 mod q_t + shoup, then
// the conversion's part (k_bc_down_rescale): [T][D] P p_1..p_{j-1} mod q_t
// (Montgomery), [T][D] P p_1..p_j mod q_t, [D][2] P^-1 mod p_j + shoup,
// [D][D][3] p_m mod p_j, p_m^-1 mod p_j, shoup (m < j).
static const u64 *relin_rs_table(ckks_context *c, int limbs, int D) {
  auto key = std::make_pair(limbs, D);
  auto it = c->relin_rs.find(key);
  if (it != c->relin_rs.end()) return it->second;
  const int T = limbs - D;
  auto p = [&](int j) { return c->primes[limbs - 1 - j]; };  // p_{j+1}
  auto pmod = [&](u64 q) {
    u64 P = 1;
    for (int j = 0; j < c->alpha; j++) P = mulmod_h(P, c->primes[c->L + j] % q, q);
    return P;
  };
  // u64 part, then [T][D] (P p_1..p_{j-1} mod q_t, / q_t) as doubles for the
  // fp64 kernel (targets below 2^45)
  const size_t words = 4 * (size_t)T + 2 * (size_t)T * D + 2 * (size_t)D + 3 * (size_t)D * D;
  std::vector<u64> h(words + 2 * (size_t)T * D, 0);
  u64 *pm = h.data() + 4 * (size_t)T, *pp = pm + (size_t)T * D, *pi = pp + (size_t)T * D;
  u64 *chain = pi + 2 * (size_t)D;
  double *pmf = reinterpret_cast<double *>(h.data() + words);
  for (int t = 0; t < T; t++) {
    const u64 q = c->primes[t], P = pmod(q);
    u64 prod = 1;  // p_1..p_j mod q
    for (int j = 0; j < D; j++) {
      const u64 f = mulmod_h(P, prod, q);
      pmf[2 * ((size_t)t * D + j)] = (double)f;
      pmf[2 * ((size_t)t * D + j) + 1] = (double)f / (double)q;
      pm[(size_t)t * D + j] = (u64)(((u128)f << 64) % q);
      prod = mulmod_h(prod, p(j) % q, q);
      pp[(size_t)t * D + j] = mulmod_h(P, prod, q);
    }
    const u64 inv2 = invmod_h(mulmod_h(P, prod, q), q), invq = invmod_h(prod, q);
    h[2 * t] = inv2;
    h[2 * t + 1] = shoup_h(inv2, q);
    h[2 * (size_t)T + 2 * t] = invq;
    h[2 * (size_t)T + 2 * t + 1] = shoup_h(invq, q);
  }
  for (int j = 0; j < D; j++) {
    const u64 pj = p(j), inv = invmod_h(pmod(pj), pj);
    pi[2 * j] = inv;
    pi[2 * j + 1] = shoup_h(inv, pj);
    for (int m = 0; m < j; m++) {
      u64 *e = chain + 3 * ((size_t)j * D + m);
      const u64 r = p(m) % pj, ri = invmod_h(r, pj);
      e[0] = r;
      e[1] = ri;
      e[2] = shoup_h(ri, pj);
    }
  }
  u64 *d = nullptr;
  HIPCHECK(hipMalloc(&d, sizeof(u64) * h.size()));
  HIPCHECK(hipMemcpy(d, h.data(), sizeof(u64) * h.size(), hipMemcpyHostToDevice));
  return c->relin_rs[key] = d;
}

// The one-ModDown relinearise-rescale needs the Montgomery sums of its
// conversion (alpha sources and D lifts) below q_t 2^64.
static bool relin_rs_fits(const ckks_context *c, int limbs, int D) {
  if (D < 1 || D > kMaxRescaleDrop || limbs <= D || c->alpha > kMaxDigitSize) return false;
  u128 s = 0;
  for (int j = 0; j < D; j++) s += c->primes[limbs - 1 - j];
  for (int j = 0; j < c->alpha; j++) s += c->primes[c->L + j];
  return s < ((u128)1 << 64);
}

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

static const FFTTable &fft_table(ckks_context *c, int n) {
  auto it = c->fft.find(n);
  if (it != c->fft.end()) return it->second;
  std::vector<double> fw(n > 1 ? n : 2), iv(n > 1 ? n : 2), tw(2 * (size_t)n), utw(2 * (size_t)n);
  for (int j = 0; j < n / 2; j++) {
    double cs, sn;
    unit_root(j, n, &cs, &sn);
    fw[2 * j] = cs;
    fw[2 * j + 1] = sn;
    iv[2 * j] = cs;
    iv[2 * j + 1] = -sn;
  }
  for (int k = 0; k < n; k++) {
    double cs, sn;
    unit_root(k, 4 * (long long)n, &cs, &sn);
    tw[2 * k] = cs;
    tw[2 * k + 1] = -sn;
    utw[2 * k] = cs;
    utw[2 * k + 1] = sn;
  }
  std::vector<u32> perm(n);
  for (int j = 0; j < n; j++) perm[j] = (u32)((powmod_h(5, (u64)j, 4 * (u64)n) - 1) / 4);
  FFTTable t{};
  t.n = n;
  auto up = [&](void **dst, const void *src, size_t bytes) {
    HIPCHECK(hipMalloc(dst, bytes));
    HIPCHECK(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
  };
  up((void **)&t.tw_fwd, fw.data(), sizeof(double) * fw.size());
  up((void **)&t.tw_inv, iv.data(), sizeof(double) * iv.size());
  up((void **)&t.twist, tw.data(), sizeof(double) * tw.size());
  up((void **)&t.untwist, utw.data(), sizeof(double) * utw.size());
  up((void **)&t.perm, perm.data(), sizeof(u32) * perm.size());
  return c->fft[n] = t;
}

// ===========================================================================
// context
// ===========================================================================

static u64 galois_of(const ckks_context *c, int64_t rotation) {
  const u64 M = 2 * (u64)c->N;
  if ((u64)rotation == M - 1) return M - 1;
  const int64_t half = c->N / 2;
  int64_t r = rotation % half;
  if (r < 0) r += half;
  return powmod_h(5, (u64)r, M);
}

static void build_context(ckks_context *c, const ckks_params &p) {
  require(p.log_n >= 10 && p.log_n <= 17, "log_n must be in [10, 17]");
  require(p.depth >= 0, "depth must be non-negative");
  require(p.dnum >= 1, "dnum must be positive");
  require(p.dcrt_bits >= 33 && p.dcrt_bits <= 60, "dcrt_bits must be in [33, 60]");
  require(p.first_mod >= 33 && p.first_mod <= 60, "first_mod must be in [33, 60]");
  require(p.special_bits >= 33 && p.special_bits <= 60, "special_bits must be in [33, 60]");
  c->params = p;
  c->logN = p.log_n;
  c->N = 1 << p.log_n;
  c->L = p.depth + 1;
  c->ds = (c->L + p.dnum - 1) / p.dnum;
  c->alpha = c->ds;
  c->K = c->L + c->alpha;
  require(c->ds <= kMaxDigitSize, "digit size ceil((depth+1)/dnum) must be <= 16");
  require((c->L + c->ds - 1) / c->ds <= kMaxDigits, "at most 8 key-switching digits");
  require(p.secret_mode == 0 || p.secret_mode == 1, "secret_mode must be 0 or 1");
  require(p.secret_mode == 1 || (p.hamming_weight > 0 && p.hamming_weight <= c->N),
          "hamming weight out of range");

  std::vector<u64> used;
  auto q0 = prime_chain(c->logN, p.first_mod, 1, used);
  used = q0;
  auto qs = prime_chain(c->logN, p.dcrt_bits, c->L - 1, used);
  used.insert(used.end(), qs.begin(), qs.end());
  auto ps = prime_chain(c->logN, p.special_bits, c->alpha, used);
  c->primes = used;
  c->primes.insert(c->primes.end(), ps.begin(), ps.end());
  // P must exceed every digit's modulus.
  double logP = 0;
  for (u64 v : ps) logP += log2((double)v);
  for (int j = 0; j * c->ds < c->L; j++) {
    double logD = 0;
    for (int i = j * c->ds; i < std::min((j + 1) * c->ds, c->L); i++) logD += log2((double)c->primes[i]);
    require(logP > logD, "special modulus P must exceed every digit modulus");
  }

  const int K = c->K, N = c->N;
  c->h_mods.resize(K);
  for (int i = 0; i < K; i++) c->h_mods[i] = make_modq(c->primes[i]);
  HIPCHECK(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
  HIPCHECK(hipMalloc(&c->d_mods, sizeof(ModQ) * K));
  HIPCHECK(hipMemcpy(c->d_mods, c->h_mods.data(), sizeof(ModQ) * K, hipMemcpyHostToDevice));

  std::vector<u64> psi((size_t)K * N), psi_sh((size_t)K * N), ipsi((size_t)K * N),
      ipsi_sh((size_t)K * N), ninv(2 * (size_t)K);
  parallel_for(K, [&](int pi) {
    const u64 q = c->primes[pi];
    const u64 r = min_root_h(q, c->logN), ri = invmod_h(r, q);
    std::vector<u64> pw(N), ipw(N);
    pw[0] = ipw[0] = 1;
    for (int i = 1; i < N; i++) {
      pw[i] = mulmod_h(pw[i - 1], r, q);
      ipw[i] = mulmod_h(ipw[i - 1], ri, q);
    }
    for (int i = 0; i < N; i++) {
      const u32 b = bitrev_h((u32)i, c->logN);
      const size_t o = (size_t)pi * N + i;
      psi[o] = pw[b];
      psi_sh[o] = shoup_h(pw[b], q);
      ipsi[o] = ipw[b];
      ipsi_sh[o] = shoup_h(ipw[b], q);
    }
    ninv[2 * pi] = invmod_h((u64)N, q);
    ninv[2 * pi + 1] = shoup_h(ninv[2 * pi], q);
  });
  auto up = [&](u64 **dst, const std::vector<u64> &v) {
    HIPCHECK(hipMalloc(dst, sizeof(u64) * v.size()));
    HIPCHECK(hipMemcpy(*dst, v.data(), sizeof(u64) * v.size(), hipMemcpyHostToDevice));
  };
  // fp64 tables for primes below 2^45 (exact doubles; w / q correctly rounded)
  c->prime_fp.assign(K, 0);
  for (int pi = 0; pi < K; pi++) c->prime_fp[pi] = c->primes[pi] < ((u64)1 << 45) ? 1 : 0;
  {
    std::vector<double> tw(2 * (size_t)K * N, 0.0), itw(2 * (size_t)K * N, 0.0), nv(2 * (size_t)K, 0.0),
        rv(2 * (size_t)K, 0.0);
    for (int pi = 0; pi < K; pi++) {
      if (!c->prime_fp[pi]) continue;
      const double q = (double)c->primes[pi];
      for (int i = 0; i < N; i++) {
        const size_t o = (size_t)pi * N + i;
        tw[2 * o] = (double)psi[o];
        tw[2 * o + 1] = (double)psi[o] / q;
        itw[2 * o] = (double)ipsi[o];
        itw[2 * o + 1] = (double)ipsi[o] / q;
      }
      nv[2 * pi] = (double)ninv[2 * pi];
      nv[2 * pi + 1] = (double)ninv[2 * pi] / q;
      // 2^-64 mod q: the Montgomery factor of the key words
      const u64 r = invmod_h((u64)(((u128)1 << 64) % c->primes[pi]), c->primes[pi]);
      rv[2 * pi] = (double)r;
      rv[2 * pi + 1] = (double)r / q;
    }
    if (N == 65536) {
      // The low NTT passes read the twiddles of bit positions 2..0 of a row
      // as runs of M = 2, 4, 8 per thread: store each run's m-th entries of
      // the 16 threads of a row side by side, so that one load of the 64
      // lanes touches contiguous memory ([row][m][c0] instead of
      // [row][c0][m]; entries below 8192 keep their places).
      std::vector<double> tmp(2 * (size_t)N);
      for (int pi = 0; pi < K; pi++) {
        if (!c->prime_fp[pi]) continue;
        for (std::vector<double> *t : {&tw, &itw}) {
          double *row0 = t->data() + 2 * (size_t)pi * N;
          std::copy(row0, row0 + 2 * (size_t)N, tmp.begin());
          for (int b = 0; b < 3; b++) {
            const int M = 8 >> b, base = 65536 >> (b + 1);
            for (int r = 0; r < 256; r++)
              for (int c0 = 0; c0 < 16; c0++)
                for (int m = 0; m < M; m++) {
                  const size_t to = (size_t)base + (size_t)r * 16 * M + (size_t)m * 16 + c0;
                  const size_t from = (size_t)base + (size_t)r * 16 * M + (size_t)c0 * M + m;
                  row0[2 * to] = tmp[2 * from];
                  row0[2 * to + 1] = tmp[2 * from + 1];
                }
          }
        }
      }
    }
    auto upd = [&](double **dst, const std::vector<double> &v) {
      HIPCHECK(hipMalloc(dst, sizeof(double) * v.size()));
      HIPCHECK(hipMemcpy(*dst, v.data(), sizeof(double) * v.size(), hipMemcpyHostToDevice));
    };
    upd(&c->d_tw_fp, tw);
    upd(&c->d_itw_fp, itw);
    upd(&c->d_ninv_fp, nv);
    upd(&c->d_rinv_fp, rv);
  }
  up(&c->d_psi, psi);
  up(&c->d_psi_sh, psi_sh);
  up(&c->d_ipsi, ipsi);
  up(&c->d_ipsi_sh, ipsi_sh);
  up(&c->d_ninv, ninv);
  {
    // P mod q_i (and its Shoup companion) for the extended-basis lifts
    std::vector<u64> pm(2 * (size_t)c->L);
    for (int i = 0; i < c->L; i++) {
      const u64 q = c->primes[i];
      u64 P = 1;
      for (int j = 0; j < c->alpha; j++) P = mulmod_h(P, c->primes[c->L + j] % q, q);
      pm[2 * i] = P;
      pm[2 * i + 1] = shoup_h(P, q);
    }
    up(&c->d_pmod, pm);
  }

  // secret: sampled on the host (client side), moved to every prime's NTT domain
  c->secret = sample_secret(p.seed, N, p.secret_mode, p.hamming_weight);
  std::vector<long long> sv(N);
  for (int i = 0; i < N; i++) sv[i] = c->secret[i];
  long long *d_sv = nullptr;
  HIPCHECK(hipMalloc(&d_sv, sizeof(long long) * N));
  HIPCHECK(hipMemcpy(d_sv, sv.data(), sizeof(long long) * N, hipMemcpyHostToDevice));
  HIPCHECK(hipMalloc(&c->d_secret, sizeof(u64) * (size_t)K * N));
  launch_expand_ntt(c, d_sv, c->d_secret, K, c->L);
  HIPCHECK(hipStreamSynchronize(c->stream));
  HIPCHECK(hipFree(d_sv));
}

// Pinned staging: buffers in 1 MiB units, up to 1 GiB in all; past that the
// stream is drained and the buffers too small for the request are dropped.
static constexpr size_t kStageUnit = (size_t)1 << 20, kStageCap = (size_t)1 << 30;

namespace ckks {
void upload_async(ckks_context *c, void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return;
  ckks_context::StageBuf *pick = nullptr;
  for (auto &b : c->stage) {
    if (b.bytes < bytes) continue;
    if (hipEventQuery(b.ev) == hipSuccess) {
      pick = &b;
      break;
    }
    (void)hipGetLastError();  // a copy still pending is not an error for later checks
  }
  if (!pick) {
    const size_t want = (bytes + kStageUnit - 1) / kStageUnit * kStageUnit;
    size_t total = 0;
    for (auto &b : c->stage) total += b.bytes;
    if (total + want > kStageCap) {
      HIPCHECK(hipStreamSynchronize(c->stream));
      for (auto &b : c->stage)
        if (b.bytes >= bytes) {
          pick = &b;
          break;
        }
      if (!pick) {
        for (auto &b : c->stage) {
          (void)hipHostFree(b.p);
          (void)hipEventDestroy(b.ev);
        }
        c->stage.clear();
      }
    }
    if (!pick) {
      ckks_context::StageBuf nb{nullptr, want, nullptr};
      HIPCHECK(hipHostMalloc(&nb.p, want, hipHostMallocDefault));
      if (hipEventCreateWithFlags(&nb.ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipHostFree(nb.p);
        throw std::runtime_error("hipEventCreateWithFlags failed");
      }
      c->stage.push_back(nb);
      pick = &c->stage.back();
    }
  }
  memcpy(pick->p, src, bytes);
  HIPCHECK(hipMemcpyAsync(dst, pick->p, bytes, hipMemcpyHostToDevice, c->stream));
  HIPCHECK(hipEventRecord(pick->ev, c->stream));
}
}  // namespace ckks

static void free_context(ckks_context *c) {
  if (!c) return;
  g_live_contexts.erase(c);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  for (auto &b : c->stage) {
    (void)hipHostFree(b.p);
    (void)hipEventDestroy(b.ev);
  }
  c->stage.clear();
  for (auto &r : c->prof_recs) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (auto e : c->prof_pool) (void)hipEventDestroy(e);
  for (auto &kv : c->keys) (void)hipFree(kv.second.data);
  for (auto &kv : c->bc_up) {
    (void)hipFree(kv.second.d);
    if (kv.second.fd) (void)hipFree(kv.second.fd);
    if (kv.second.mf) (void)hipFree(kv.second.mf);
    if (kv.second.mt) (void)hipFree(kv.second.mt);
    if (kv.second.sn) (void)hipFree(kv.second.sn);
  }
  for (auto &kv : c->bc_down) {
    (void)hipFree(kv.second.d);
    if (kv.second.fd) (void)hipFree(kv.second.fd);
    if (kv.second.mf) (void)hipFree(kv.second.mf);
    if (kv.second.mt) (void)hipFree(kv.second.mt);
    if (kv.second.sn) (void)hipFree(kv.second.sn);
  }
  for (auto &kv : c->pinv) (void)hipFree(kv.second);
  for (auto &kv : c->pmod) (void)hipFree(kv.second);
  for (auto &kv : c->relin_rs) (void)hipFree(kv.second);
  for (auto &kv : c->rescale_d) (void)hipFree(kv.second);
  for (auto &kv : c->garner) (void)hipFree(kv.second);
  for (auto &kv : c->fft) {
    (void)hipFree(kv.second.tw_fwd);
    (void)hipFree(kv.second.tw_inv);
    (void)hipFree(kv.second.twist);
    (void)hipFree(kv.second.untwist);
    (void)hipFree(kv.second.perm);
  }
  (void)hipFree(c->d_mods);
  (void)hipFree(c->d_psi);
  (void)hipFree(c->d_psi_sh);
  (void)hipFree(c->d_ipsi);
  (void)hipFree(c->d_ipsi_sh);
  (void)hipFree(c->d_ninv);
  (void)hipFree(c->d_pmod);
  (void)hipFree(c->d_secret);
  (void)hipFree(c->d_tw_fp);
  (void)hipFree(c->d_itw_fp);
  (void)hipFree(c->d_ninv_fp);
  (void)hipFree(c->d_rinv_fp);
  c->pool.trim();
  if (c->fork_ev) (void)hipEventDestroy(c->fork_ev);
  for (int i = 0; i < ckks_context::kMaxSplit - 1; i++) {
    if (c->join_ev[i]) (void)hipEventDestroy(c->join_ev[i]);
    if (c->aux[i]) (void)hipStreamDestroy(c->aux[i]);
  }
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

// ===========================================================================
// per-kernel timing
// ===========================================================================

namespace ckks {
static hipEvent_t prof_event(ckks_context *c) {
  if (!c->prof_pool.empty()) {
    hipEvent_t e = c->prof_pool.back();
    c->prof_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  HIPCHECK(hipEventCreate(&e));
  return e;
}

KTimer::KTimer(ckks_context *cc, const char *name, double bytes, double ops)
    : c(cc), on(cc->prof) {
  if (!on) return;
  r = ProfRec{name, prof_event(c), prof_event(c), bytes, ops};
  (void)hipEventRecord(r.a, c->stream);
}

KTimer::~KTimer() {
  if (!on) return;
  (void)hipEventRecord(r.b, c->stream);
  c->prof_recs.push_back(r);
}
}  // namespace ckks

// ===========================================================================
// fixed key-switch scratch of ckks_rotate_many_noalloc
// ===========================================================================

// 256 MiB per device, held from the library's first context on that device
// until the process ends; every context on one device shares it.
static constexpr size_t kNoAllocWords = (size_t)1 << 25;
static __device__ __align__(256) u64 scratch[kNoAllocWords];

static constexpr int kMaxDevices = 64;

// Per device: the array's device address, and the ordering of its users.
// Calls from different contexts run on different streams; each call holds
// `mu` while it enqueues, makes its stream wait on `done` (the previous
// call's completion on whatever stream it ran) and records `done` after its
// last launch, so the calls use the buffer one after another on the device
// without the host waiting.
struct NoAllocDevice {
  u64 *ptr = nullptr;
  hipEvent_t done = nullptr;
  std::mutex mu;
};
static NoAllocDevice g_noalloc[kMaxDevices];
static std::mutex g_scratch_mu;

// Resolves the device address of `scratch` on the current device (each
// device holds its own copy of the array at its own address) and creates its
// ordering event, recorded once on `stream` so that it is always in a
// recorded state; done once per device.
static u64 *device_scratch(int dev, hipStream_t stream) {
  require(dev >= 0 && dev < kMaxDevices, "device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  NoAllocDevice &nd = g_noalloc[dev];
  if (!nd.ptr) {
    void *p = nullptr;
    HIPCHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    hipEvent_t ev = nullptr;
    HIPCHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    HIPCHECK(hipEventRecord(ev, stream));
    nd.done = ev;
    nd.ptr = (u64 *)p;
  }
  return nd.ptr;
}

// ===========================================================================
// ciphertext objects
// ===========================================================================

static ckks_ct *new_ct(ckks_context *c, int polys, int limbs, int is_ext, int slots,
                       double scale, int scale_degree) {
  ckks_ct *ct = new ckks_ct();
  ct->ctx = c;
  ct->serial = c->serial;
  ct->polys = polys;
  ct->limbs = limbs;
  ct->is_ext = is_ext;
  ct->slots = slots;
  ct->scale = scale;
  ct->scale_degree = scale_degree;
  const int rows = polys == 0 ? 1 : polys;
  const int per = polys == 0 ? limbs : (limbs + (is_ext ? c->alpha : 0)) * c->N;
  ct->bytes = sizeof(u64) * (size_t)rows * per;
  ct->d = (u64 *)c->pool.alloc(ct->bytes);
  return ct;
}

static void free_ct(ckks_ct *ct) {
  if (!ct) return;
  if (ct->serial && owner_alive(ct->ctx, ct->serial)) ct->ctx->pool.release(ct->d, ct->bytes);
  delete ct;
}

static void check_ct(const ckks_context *c, const ckks_ct *ct, const char *what) {
  require(ct != nullptr, std::string(what) + ": null ciphertext");
  require(ct->ctx == c, std::string(what) + ": ciphertext belongs to another context");
}

// A ciphertext or plaintext polynomial set (polys >= 1); the per-limb
// constants of encode_scalar (polys 0) hold one word per limb and are only
// accepted where an entry point says so.
static void check_poly(const ckks_context *c, const ckks_ct *ct, const char *what) {
  check_ct(c, ct, what);
  require(ct->polys >= 1, std::string(what) + ": expects a ciphertext or plaintext, not a scalar");
}

static int poly_words(const ckks_context *c, const ckks_ct *ct) {
  return (ct->limbs + (ct->is_ext ? c->alpha : 0)) * c->N;
}

// scales of two operands that are combined limb-wise must agree to 2^-10
// relative (fixed-scale bookkeeping); the result takes the left scale.
static void check_scales(const ckks_ct *a, const ckks_ct *b) {
  const double r = fabs(a->scale - b->scale) / std::max(a->scale, b->scale);
  require(r < 1.0 / 1024.0, "operand scales differ");
}

// ===========================================================================
// key switching pipeline
// ===========================================================================

// Key-switch intermediates: blocks from the context pool, released when the
// Scratch goes out of scope, or (arena mode) consecutive ranges of a fixed
// device buffer that is never allocated or freed here.
struct Scratch {
  ckks_context *c;
  std::vector<std::pair<void *, size_t>> bufs;
  u64 *arena = nullptr;
  size_t arena_words = 0, used = 0;
  explicit Scratch(ckks_context *cc) : c(cc) {}
  Scratch(ckks_context *cc, u64 *base, size_t words) : c(cc), arena(base), arena_words(words) {}
  Scratch(const Scratch &) = delete;
  Scratch &operator=(const Scratch &) = delete;
  u64 *get(size_t words) {
    if (arena) {
      // 256-byte aligned ranges, as the pool's blocks
      const size_t w = (words + 31) & ~(size_t)31;
      if (used + w > arena_words)
        throw std::invalid_argument("fixed scratch exhausted: " + std::to_string(used + w) +
                                    " words needed, " + std::to_string(arena_words) + " held");
      u64 *p = arena + used;
      used += w;
      return p;
    }
    void *p = c->pool.alloc(sizeof(u64) * words);
    bufs.emplace_back(p, sizeof(u64) * words);
    return (u64 *)p;
  }
  ~Scratch() {
    for (auto &b : bufs) c->pool.release(b.first, b.second);
  }
};

static Batch strided(u64 *base, size_t stride) {
  Batch b{};
  b.base = base;
  b.stride = stride;
  return b;
}

// ModUp of n polynomials d[i] (NTT domain, `limbs` limbs) into
// ext = [n][digits][E][N].
// own_copy false: the digits' own limbs are not copied into ext; the key
// inner product then reads them from d (ks_inner's `own`).
// high_only (N = 2^16, own_copy false): the converted limbs get only the
// high pass of the forward NTT; launch_ntt_low_key runs the low pass.
// dmul (tile path, own_copy false): the polynomials are d[i] x dmul[i] word
// by word, formed by the inverse low pass (modup_tile_ok tells when).
// pack (high_only, own_copy false): on the tile path the fp64 limbs are
// written in the packed form of launch_convert_h4, which only the fused key
// products read; returns whether they were.
static bool ks_modup(ckks_context *c, int limbs, int n, const u64 *const *d, u64 *ext,
                     Scratch &s, bool own_copy = true, bool high_only = false,
                     const Batch *dmul = nullptr, bool pack = false) {
  const size_t N = c->N;
  const int E = limbs + c->alpha, digits = (limbs + c->ds - 1) / c->ds;
  u64 *coeff = s.get((size_t)n * limbs * N);
  Batch src{};
  for (int i = 0; i < n; i++) src.p[i] = (u64 *)d[i];
  // N = 2^16: the inverse NTT's high pass, the conversion and the targets'
  // forward high pass run as one kernel per digit; for the full NTT form
  // (not high_only) the targets' low pass follows
  bool tile = c->ks_tile;
  for (int j = 0; j < digits && tile; j++) tile = convert_h4_ok(c, bc_up(c, limbs, j));
  if (dmul && (!tile || own_copy)) throw std::logic_error("ModUp of a product: tile path only");
  if (tile) {
    const size_t est = (size_t)digits * E * N;
    const bool packed = pack && high_only && !own_copy;
    launch_ntt_inv_low(c, src, strided(coeff, (size_t)limbs * N), n, 0, limbs, limbs, dmul);
    for (int j = 0; j < digits; j++) {
      const int lo = j * c->ds, hi = std::min((j + 1) * c->ds, limbs), ns = hi - lo;
      u64 *ej = ext + (size_t)j * E * N;
      if (own_copy) {
        Batch dsrc{};
        for (int i = 0; i < n; i++) dsrc.p[i] = (u64 *)d[i] + (size_t)lo * N;
        launch_copy_limbs(c, dsrc, strided(ej + (size_t)lo * N, est), n, ns);
      }
      launch_convert_h4(c, strided(coeff + (size_t)lo * N, (size_t)limbs * N), strided(ej, est),
                        n, bc_up(c, limbs, j), lo, lo, ns, limbs, false, packed);
      if (!high_only) {
        launch_ntt_fwd_low(c, strided(ej, est), n, 0, lo, limbs);
        launch_ntt_fwd_low(c, strided(ej, est), n, hi, E - hi, limbs);
      }
    }
    return packed;
  }
  launch_ntt(c, src, strided(coeff, (size_t)limbs * N), n, 0, limbs, limbs, true);
  for (int j = 0; j < digits; j++) {
    const int lo = j * c->ds, hi = std::min((j + 1) * c->ds, limbs), ns = hi - lo;
    Batch dsrc{};
    for (int i = 0; i < n; i++) dsrc.p[i] = (u64 *)d[i] + (size_t)lo * N;
    u64 *ej = ext + (size_t)j * E * N;
    const size_t est = (size_t)digits * E * N;
    if (own_copy) launch_copy_limbs(c, dsrc, strided(ej + (size_t)lo * N, est), n, ns);
    launch_basis_convert(c, strided(coeff + (size_t)lo * N, (size_t)limbs * N), strided(ej, est), n,
                         bc_up(c, limbs, j), lo, lo, ns, limbs, false);
    if (high_only) {
      launch_ntt_fwd_high(c, strided(ej, est), strided(ej, est), n, 0, lo, limbs);
      launch_ntt_fwd_high(c, strided(ej, est), strided(ej, est), n, hi, E - hi, limbs);
    } else {
      launch_ntt(c, strided(ej, est), strided(ej, est), n, 0, lo, limbs, false);
      launch_ntt(c, strided(ej, est), strided(ej, est), n, hi, E - hi, limbs, false);
    }
  }
  return false;
}

struct KsJob {
  int ext_item;
  const DeviceKey *key;
  u64 galois;
  const u64 *add0, *add1;
  u64 *out0, *out1;
};

// The key product of the fp64 Q limbs left by ks_modup_inner for ks_moddown
// (launch_low_key_moddown): the extended digits and what it multiplies them by.
struct KsDeferred {
  // input: the Q limbs [0, below) whose key product may be deferred (-1: all,
  // where ks_moddown's tile conversion applies)
  int below = -1;
  bool on = false;
  const u64 *ext = nullptr;
  size_t est = 0;
  Batch own{};
  const Batch *own_b = nullptr;  // own x own_b is the source (ks_modup_inner's dmul)
  bool packed = false;           // ext's fp64 limbs in the packed form
  const DeviceKey *key = nullptr;
  int digits = 0;
  u64 ginv = 1;
};

// ModDown of n accumulators acc = [n][2][E][N] (Q limbs then P limbs) into
// the jobs' outputs, adding each job's addends (sigma-permuted): the P-part
// iNTT, the centered conversion, then the forward NTT with the combine.
// With ptmp given ([2 n][alpha][N]) and sp_done, ks_modup_inner's key
// product left the P part there after the inverse NTT's low pass.
static void ks_moddown(ckks_context *c, int limbs, u64 *acc, const std::vector<KsJob> &jobs,
                       Scratch &s, u64 *ptmp = nullptr, bool sp_done = false,
                       const KsDeferred *dk = nullptr) {
  const size_t N = c->N;
  const int E = limbs + c->alpha;
  const int n = (int)jobs.size();
  if (!ptmp) ptmp = s.get((size_t)n * 2 * c->alpha * N);
  const u64 *pinv = pinv_table(c, limbs);
  // the fused path addresses component 1 of the addend and of the output at
  // a fixed offset from component 0 (as every caller lays them out)
  bool uniform = n <= kMaxBatch;
  const u64 add1_off = jobs[0].add1 ? (u64)(jobs[0].add1 - jobs[0].add0) : 0;
  const u64 out1_off = (u64)(jobs[0].out1 - jobs[0].out0);
  for (int i = 0; i < n && uniform; i++)
    uniform = (jobs[i].add1 ? (u64)(jobs[i].add1 - jobs[i].add0) : 0) == add1_off &&
              (!jobs[i].add1 || jobs[i].add0) && (u64)(jobs[i].out1 - jobs[i].out0) == out1_off;
  const Batch spb = strided(ptmp - (size_t)limbs * N, (size_t)c->alpha * N);  // limb l at l N
  u64 *conv = s.get((size_t)n * 2 * limbs * N);
  // N = 2^16: the special limbs' inverse high pass, the conversion and the
  // forward high pass of the Q limbs in one kernel, then the low pass with
  // the combine
  const bool tile = c->logN == 16 && uniform && c->ks_tile && convert_h4_ok(c, bc_down(c, limbs));
  const bool deferred = dk && dk->on;
  if (deferred && !(tile && sp_done)) throw std::logic_error("deferred key product without the tile ModDown");
  if (tile) {
    if (!sp_done) launch_ntt_inv_low(c, strided(acc, E * N), spb, 2 * n, limbs, c->alpha, limbs);
    launch_convert_h4(c, strided(ptmp, (size_t)c->alpha * N), strided(conv, (size_t)limbs * N),
                      2 * n, bc_down(c, limbs), c->L, limbs, 0, limbs, true);
  } else {
    if (sp_done)
      launch_ntt_inv_high(c, spb, 2 * n, limbs, c->alpha, limbs);
    else
      launch_ntt(c, strided(acc, E * N), spb, 2 * n, limbs, c->alpha, limbs, true);
    launch_basis_convert(c, strided(ptmp, (size_t)c->alpha * N),
                         strided(conv, (size_t)limbs * N), 2 * n, bc_down(c, limbs), c->L, limbs,
                         0, limbs, true);
  }
  if (c->logN == 16 && uniform) {
    // NTT of the conversion with the combine fused into its last pass
    Batch a0{}, o0{};
    std::vector<u64> gal(n);
    for (int i = 0; i < n; i++) {
      a0.p[i] = (u64 *)jobs[i].add0;
      o0.p[i] = jobs[i].out0;
      gal[i] = jobs[i].galois;
    }
    if (deferred)
      launch_low_key_moddown(c, dk->ext, dk->est, dk->own, n, *dk->key, dk->digits, E, limbs,
                             dk->ginv, strided(conv, (size_t)limbs * N), pinv,
                             pmod_table(c, limbs), a0, add1_off, o0, out1_off, limbs,
                             nullptr, dk->own_b, dk->packed);
    launch_ntt_moddown(c, strided(conv, (size_t)limbs * N), n, limbs, strided(acc, 2 * E * N), E,
                       pinv, a0, add1_off, gal.data(), o0, out1_off, nullptr, nullptr, tile,
                       deferred);
    return;
  }
  if (deferred) throw std::logic_error("deferred key product without the fused combine");
  launch_ntt(c, strided(conv, (size_t)limbs * N), strided(conv, (size_t)limbs * N), 2 * n, 0,
             limbs, limbs, false);
  for (int b0 = 0; b0 < n; b0 += kMaxBatch) {
    const int nb = std::min(kMaxBatch, n - b0);
    Batch a0{}, a1{}, o0{}, o1{};
    std::vector<u64> gal(nb);
    for (int i = 0; i < nb; i++) {
      const KsJob &jb = jobs[b0 + i];
      a0.p[i] = (u64 *)jb.add0;
      a1.p[i] = (u64 *)jb.add1;
      o0.p[i] = jb.out0;
      o1.p[i] = jb.out1;
      gal[i] = jb.galois;
    }
    Strided sacc{acc + (size_t)b0 * 2 * E * N, 2 * E * N};
    Strided sconv{conv + (size_t)b0 * 2 * limbs * N, 2 * limbs * N};
    launch_moddown_combine(c, sacc, sconv, a0, a1, gal.data(), o0, o1, nb, limbs, E, pinv);
  }
}

// Key inner product of every job into [n][2][E][N] accumulators.  With own
// given, ext item i lacks its digits' own limbs, which are read from own[i].
static u64 *ks_inner(ckks_context *c, int limbs, const u64 *ext, const std::vector<KsJob> &jobs,
                     Scratch &s, const u64 *const *own = nullptr) {
  const size_t N = c->N;
  const int E = limbs + c->alpha, digits = (limbs + c->ds - 1) / c->ds;
  const int n = (int)jobs.size();
  const size_t est = (size_t)digits * E * N;
  u64 *acc = s.get((size_t)n * 2 * E * N);
  bool shared = true;
  for (int i = 0; i < n; i++)
    shared = shared && jobs[i].ext_item == i && jobs[i].key == jobs[0].key &&
             jobs[i].galois == jobs[0].galois;
  if (shared) {
    Batch ob{};
    if (own)
      for (int i = 0; i < n; i++) ob.p[i] = (u64 *)own[i];
    launch_key_inner(c, strided((u64 *)ext, est), strided(acc, 2 * E * N), n, *jobs[0].key,
                     digits, E, limbs, jobs[0].galois, own ? &ob : nullptr);
  } else {
    for (int i = 0; i < n; i++) {
      Batch ob{};
      if (own) ob.p[0] = (u64 *)own[jobs[i].ext_item];
      launch_key_inner(c, strided((u64 *)ext + (size_t)jobs[i].ext_item * est, 0),
                       strided(acc + (size_t)i * 2 * E * N, 0), 1, *jobs[i].key, digits, E,
                       limbs, jobs[i].galois, own ? &ob : nullptr);
    }
  }
  return acc;
}

// g^-1 mod 2N: the units mod 2N have order N / 2, so g^-1 = g^(N - 1)
static u64 galois_inverse(const ckks_context *c, u64 g) {
  const u64 two_n = 2 * (u64)c->N;
  u64 inv = 1, base = g % two_n;
  for (u64 e = c->N - 1; e; e >>= 1, base = base * base % two_n)
    if (e & 1) inv = inv * base % two_n;
  return inv;
}

// ModUp of n polynomials d[i] (NTT domain) and the key inner product of
// every job (job i takes ext item i; all share one key and Galois element)
// into [n][2][E][N] accumulators.  At N = 2^16 the extended digits get only
// the NTT's high pass and their low pass runs with the key product.  With sp
// given, *sp_done tells whether the P part went through the inverse NTT's
// low pass into sp (launch_ntt_low_key) instead of into the accumulators.
// With dk given (the caller's jobs meet ks_moddown's fused combine: one
// addend per component at a fixed offset, outputs likewise), where the
// special limbs take the inverse low pass here and the ModDown's conversion
// runs tile-resident, the fp64 Q limbs' key product is left to ks_moddown
// (dk->on), which runs it with the combine.  With dk->below >= 0 the caller
// has checked its own conversion and only Q limbs below it are deferred.
static u64 *ks_modup_inner(ckks_context *c, int limbs, int n, const u64 *const *d,
                           const std::vector<KsJob> &jobs, Scratch &s,
                           const Strided *sp = nullptr, bool *sp_done = nullptr,
                           KsDeferred *dk = nullptr, const Batch *dmul = nullptr) {
  const size_t N = c->N;
  const int E = limbs + c->alpha, digits = (limbs + c->ds - 1) / c->ds;
  const size_t est = (size_t)digits * E * N;
  u64 *ext = s.get((size_t)n * est);
  const bool fused = c->ks_fused && c->logN == 16 && n <= kMaxBatch;
  const bool spf = fused && sp && c->ks_sp_inv && low_key_special_fp(c);
  if (sp_done) *sp_done = spf;
  if (dmul && !fused) throw std::logic_error("key switch of a product: fused path only");
  // the fused key products are the only readers of ext: packed where the
  // tile path writes it
  const bool packed = ks_modup(c, limbs, n, d, ext, s, false, fused, dmul, fused);
  if (!fused) return ks_inner(c, limbs, ext, jobs, s, d);
  u64 *acc = s.get((size_t)n * 2 * E * N);
  Batch ob{};
  for (int i = 0; i < n; i++) ob.p[i] = (u64 *)d[i];
  const u64 ginv = galois_inverse(c, jobs[0].galois);
  const bool defer = dk && spf && c->ks_defer && c->ks_tile &&
                     (dk->below >= 0 || convert_h4_ok(c, bc_down(c, limbs)));
  if (dk) {
    dk->on = defer;
    if (defer) {
      dk->ext = ext;
      dk->est = est;
      dk->own = ob;
      dk->own_b = dmul;
      dk->packed = packed;
      dk->key = jobs[0].key;
      dk->digits = digits;
      dk->ginv = ginv;
    }
  }
  launch_ntt_low_key(c, ext, est, ob, acc, 2 * (size_t)E * N, n, *jobs[0].key, digits, E, limbs,
                     ginv, spf ? sp : nullptr, defer ? (dk->below >= 0 ? dk->below : limbs) : 0,
                     dmul, packed);
  return acc;
}

// Whether ks_modup_inner of n polynomials at `limbs` limbs takes the fused
// tile path, on which the polynomials may be products formed on load (dmul)
static bool modup_tile_ok(ckks_context *c, int limbs, int n) {
  if (!(c->ks_fused && c->logN == 16 && n <= kMaxBatch && c->ks_tile)) return false;
  const int digits = (limbs + c->ds - 1) / c->ds;
  for (int j = 0; j < digits; j++)
    if (!convert_h4_ok(c, bc_up(c, limbs, j))) return false;
  return true;
}

// Key inner product for every job, ModDown, and the combine with addends.
static void ks_finish(ckks_context *c, int limbs, const u64 *ext, int n_ext,
                      const std::vector<KsJob> &jobs, Scratch &s,
                      const u64 *const *own = nullptr) {
  (void)n_ext;
  u64 *acc = ks_inner(c, limbs, ext, jobs, s, own);
  ks_moddown(c, limbs, acc, jobs, s);
}

static const DeviceKey &get_key(ckks_context *c, u64 galois) {
  auto it = c->keys.find(galois);
  if (it == c->keys.end()) {
    if (galois == 0) throw KeyMissing("relinearization key not generated");
    throw KeyMissing("rotation key for Galois element " + std::to_string(galois) +
                     " not generated");
  }
  return it->second;
}

static void gen_key(ckks_context *c, u64 id, int relin, u64 galois) {
  if (c->keys.count(id)) return;
  DeviceKey k{};
  k.galois = id;
  k.digits = (c->L + c->ds - 1) / c->ds;
  k.bytes = sizeof(u64) * (size_t)k.digits * 2 * c->K * c->N;
  k.data = (u64 *)c->pool.raw_alloc(k.bytes);
  launch_keygen(c, k, id, relin, galois);
  c->keys[id] = k;
}

// Parts of a batched key switch on several streams.  run(b0, nb, s) issues
// the work of items b0 .. b0 + nb - 1 on c->stream with intermediates from
// s.  The first part goes on the context stream and part i on c->aux[i - 1],
// which waits for everything issued before it (its inputs) and is joined
// back before the function returns; every part's intermediates stay
// allocated until then, so that no block of one part is handed to another
// while still in use.  Parts keep at least kSplitMin items.
constexpr int kSplitMin = 8;

struct StreamSwap {
  ckks_context *c;
  hipStream_t saved;
  StreamSwap(ckks_context *cc, hipStream_t s) : c(cc), saved(cc->stream) { cc->stream = s; }
  ~StreamSwap() { c->stream = saved; }
};

template <typename F>
static void run_parts(ckks_context *c, int b0, int nb, F run) {
  const int parts = std::min(c->split_parts, std::max(1, nb / kSplitMin));
  if (parts <= 1) {
    Scratch s(c);
    run(b0, nb, s);
    return;
  }
  std::vector<std::unique_ptr<Scratch>> sc;
  for (int i = 0; i < parts; i++) sc.emplace_back(new Scratch(c));
  HIPCHECK(hipEventRecord(c->fork_ev, c->stream));
  for (int i = 1; i < parts; i++) HIPCHECK(hipStreamWaitEvent(c->aux[i - 1], c->fork_ev, 0));
  for (int i = 0; i < parts; i++) {
    const int lo = b0 + nb * i / parts, hi = b0 + nb * (i + 1) / parts;
    if (i == 0) {
      run(lo, hi - lo, *sc[i]);
    } else {
      StreamSwap sw(c, c->aux[i - 1]);
      run(lo, hi - lo, *sc[i]);
    }
  }
  for (int i = 1; i < parts; i++) {
    HIPCHECK(hipEventRecord(c->join_ev[i - 1], c->aux[i - 1]));
    HIPCHECK(hipStreamWaitEvent(c->stream, c->join_ev[i - 1], 0));
  }
}

// Words of key-switch scratch that rotate_batch takes for nb ciphertexts at
// `limbs` limbs (each range rounded up to 256 bytes, as Scratch hands them out).
static size_t rotate_scratch_words(const ckks_context *c, int limbs, int nb) {
  const size_t N = c->N;
  const int digits = (limbs + c->ds - 1) / c->ds, E = limbs + c->alpha;
  auto r = [](size_t w) { return (w + 31) & ~(size_t)31; };
  return r((size_t)nb * digits * E * N) + r((size_t)nb * limbs * N) + r((size_t)nb * 2 * E * N) +
         r((size_t)nb * 2 * c->alpha * N) + r((size_t)nb * 2 * limbs * N);
}

// Rotations of n ciphertexts at one level by the same Galois element.  With
// `arena` given, every intermediate lives in that fixed buffer of
// `arena_words` words (n <= 64) and nothing is allocated.
static void rotate_batch(ckks_context *c, const ckks_ct *const *in, int n, u64 g, ckks_ct **out,
                         u64 *arena = nullptr, size_t arena_words = 0,
                         size_t *arena_used = nullptr) {
  const int limbs = in[0]->limbs;
  const size_t N = c->N, P = (size_t)limbs * N;
  const DeviceKey &key = get_key(c, g);
  auto run = [&](int b0, int nb, Scratch &s) {
    std::vector<const u64 *> d(nb);
    for (int i = 0; i < nb; i++) d[i] = in[b0 + i]->d + P;
    std::vector<KsJob> jobs(nb);
    for (int i = 0; i < nb; i++)
      jobs[i] = KsJob{i, &key, g, in[b0 + i]->d, nullptr, out[b0 + i]->d, out[b0 + i]->d + P};
    u64 *ptmp = s.get((size_t)nb * 2 * c->alpha * N);
    const Strided sp{ptmp, (u64)c->alpha * N};
    bool sp_done = false;
    KsDeferred dk;
    u64 *acc = ks_modup_inner(c, limbs, nb, d.data(), jobs, s, &sp, &sp_done, &dk);
    ks_moddown(c, limbs, acc, jobs, s, ptmp, sp_done, &dk);
  };
  for (int b0 = 0; b0 < n; b0 += kMaxBatch) {
    const int nb = std::min(kMaxBatch, n - b0);
    if (arena) {
      // the fixed scratch holds one batch's intermediates: one stream
      Scratch s(c, arena, arena_words);
      run(b0, nb, s);
      if (arena_used) *arena_used = std::max(*arena_used, s.used);
    } else {
      run_parts(c, b0, nb, run);
    }
  }
}

// Relinearisation of n degree-2 ciphertexts into out.
static void relin_batch(ckks_context *c, const ckks_ct *const *in, int n, ckks_ct **out) {
  const int limbs = in[0]->limbs;
  const size_t N = c->N, P = (size_t)limbs * N;
  const DeviceKey &key = get_key(c, 0);
  auto run = [&](int b0, int nb, Scratch &s) {
    std::vector<const u64 *> d(nb);
    for (int i = 0; i < nb; i++) d[i] = in[b0 + i]->d + 2 * P;
    std::vector<KsJob> jobs(nb);
    for (int i = 0; i < nb; i++)
      jobs[i] = KsJob{i, &key, 1, in[b0 + i]->d, in[b0 + i]->d + P, out[b0 + i]->d,
                      out[b0 + i]->d + P};
    u64 *ptmp = s.get((size_t)nb * 2 * c->alpha * N);
    const Strided sp{ptmp, (u64)c->alpha * N};
    bool sp_done = false;
    KsDeferred dk;
    u64 *acc = ks_modup_inner(c, limbs, nb, d.data(), jobs, s, &sp, &sp_done, &dk);
    ks_moddown(c, limbs, acc, jobs, s, ptmp, sp_done, &dk);
  };
  for (int b0 = 0; b0 < n; b0 += kMaxBatch) run_parts(c, b0, std::min(kMaxBatch, n - b0), run);
}

// Relinearisation of n degree-2 ciphertexts followed by D rescales, as one
// ModDown by P p_1..p_D (see k_bc_down_rescale): the same words as
// relin_batch then D rescales, without the relinearised ciphertext's forward
// NTT, the inverse NTTs of the dropped limbs and the rescales' lift NTTs and
// combines.
// The postop of homo_mul_relin_rescale_postop on the host side: doubling,
// the ciphertexts subtracted (per pair, or null) and the scalar's words.
struct PostSpec {
  int dbl;
  const ckks_ct *const *sub;
  const u64 *scal;
};

static PostOp post_chunk(const ckks_context *c, const PostSpec *ps, int b0, int nb) {
  PostOp po{};
  if (!ps) return po;
  po.dbl = ps->dbl;
  po.scal = ps->scal;
  if (ps->sub) {
    for (int i = 0; i < nb; i++) po.sub.p[i] = ps->sub[b0 + i]->d;
    po.sub1_off = (u64)ps->sub[b0]->limbs * c->N;
  }
  return po;
}

// With ta / tb given, in[i] is the degree-2 product of ta[i] and tb[i], not
// yet formed (in[0 .. n - 1] spaced 3 limbs N words apart): each part forms
// its items' d2 before the ModUp and, after it, the d0 / d1 limbs that the
// ModDown reads from memory; the fused combine forms the other d0 / d1
// words from the factors.
static void relin_rescale_batch(ckks_context *c, const ckks_ct *const *in, int n, ckks_ct **out,
                                int D = 1, const PostSpec *ps = nullptr,
                                const Batch *ta = nullptr, const Batch *tb = nullptr) {
  const int limbs = in[0]->limbs, T = limbs - D, A = c->alpha;
  const size_t N = c->N, P = (size_t)limbs * N;
  const DeviceKey &key = get_key(c, 0);
  const BCTable &bt = bc_down(c, limbs);
  const u64 *rt = relin_rs_table(c, limbs, D);
  auto run = [&](int b0, int nb, Scratch &s) {
    Batch fa{}, fb{}, fb1{};
    const Batch prod = strided(in[b0]->d, 3 * P);
    std::vector<const u64 *> d(nb);
    for (int i = 0; i < nb; i++) d[i] = in[b0 + i]->d + 2 * P;
    // on the fused tile path d2 = a1 b1 is formed where the ModUp reads it
    // (dmul: d[i] = a1 and fb1 the b1 polynomials), else written first
    const bool d2_fused = ta && modup_tile_ok(c, limbs, nb);
    if (ta) {
      for (int i = 0; i < nb; i++) {
        fa.p[i] = batch_ptr_host(*ta, b0 + i);
        fb.p[i] = batch_ptr_host(*tb, b0 + i);
        fb1.p[i] = fb.p[i] + P;
        if (d2_fused) d[i] = fa.p[i] + P;
      }
      if (!d2_fused) launch_tensor(c, fa, fb, prod, nb, limbs, 0, limbs, 2);
    }
    const int E = limbs + A;
    std::vector<KsJob> jobs(nb);
    for (int i = 0; i < nb; i++) jobs[i] = KsJob{i, &key, 1, nullptr, nullptr, nullptr, nullptr};
    // per item: [A] P limbs of X, then its limbs limbs-D .. limbs-1, as
    // coefficients
    const size_t xs = (size_t)(A + D) * N;
    u64 *x = s.get((size_t)nb * 2 * xs);
    const Strided sp{x, (u64)xs};
    bool sp_done = false;
    // N = 2^16: the special limbs' inverse high pass, the conversion with the
    // lifts and the forward high pass of the kept limbs in one kernel; then,
    // without a postop, the kept fp64 limbs' key product runs with the
    // combine (launch_low_key_moddown: (acc + [P] d - conv) (P p)^-1 is
    // (acc - conv) (P p)^-1 + d p^-1), the dropped limbs' before the lift
    const bool tile = c->logN == 16 && c->ks_tile && convert_h4_rs_ok(c, bt, D);
    const PostOp po = post_chunk(c, ps, b0, nb);
    KsDeferred dk;
    dk.below = T;
    const bool may_defer = tile && !ps;
    u64 *acc = ks_modup_inner(c, limbs, nb, d.data(), jobs, s, &sp, &sp_done,
                              may_defer ? &dk : nullptr, d2_fused ? &fb1 : nullptr);
    if (ta && dk.on) {
      // d0 / d1 of the kept limbs of primes of 2^45 or more (launch_ntt_moddown's
      // combine), run by run, the last run with the dropped limbs (the lift)
      int l0 = 0;
      for (;;) {
        while (l0 < T && c->prime_fp[l0]) l0++;
        int l1 = l0;
        while (l1 < T && !c->prime_fp[l1]) l1++;
        int r0 = l1;
        while (r0 < T && c->prime_fp[r0]) r0++;
        if (r0 < T) {  // another run follows: this one alone
          launch_tensor(c, fa, fb, prod, nb, limbs, l0, l1 - l0, 1);
          l0 = r0;
          continue;
        }
        launch_tensor(c, fa, fb, prod, nb, limbs, l0, l1 - l0, 1, T, D);
        break;
      }
    } else if (ta) {
      launch_tensor(c, fa, fb, prod, nb, limbs, 0, limbs, 1);
    }
    if (tile) {
      if (!sp_done)
        launch_ntt_inv_low(c, strided(acc, (size_t)E * N), strided(x - P, xs), 2 * nb, limbs, A,
                           limbs);
    } else if (sp_done) {
      launch_ntt_inv_high(c, strided(x - P, xs), 2 * nb, limbs, A, limbs);
    } else {
      launch_ntt(c, strided(acc, (size_t)E * N), strided(x - P, xs), 2 * nb, limbs, A, limbs,
                 true);
    }
    Batch d3{}, o0{};
    for (int i = 0; i < nb; i++) {
      d3.p[i] = in[b0 + i]->d;
      o0.p[i] = out[b0 + i]->d;
    }
    u64 *xq = x + (size_t)A * N;  // slot A holds limb T
    launch_rs_prep(c, Strided{acc, (size_t)E * N}, E, limbs, D, d3, nb, Strided{xq, xs});
    launch_ntt(c, strided(xq - (size_t)T * N, xs), strided(xq - (size_t)T * N, xs), 2 * nb, T, D,
               limbs, true);
    u64 *conv = s.get((size_t)nb * 2 * T * N);
    if (tile)
      launch_convert_h4_rs(c, strided(x, xs), strided(conv, (size_t)T * N), 2 * nb, bt, D,
                           rt + 4 * (size_t)T);
    else
      launch_bc_down_rescale(c, strided(x, xs), strided(conv, (size_t)T * N), 2 * nb, bt, D,
                             rt + 4 * (size_t)T);
    std::vector<u64> gal(nb, 1);
    const u64 *amul = rt + 2 * (size_t)T;
    if (c->logN == 16) {
      if (dk.on)
        launch_low_key_moddown(c, dk.ext, dk.est, dk.own, nb, *dk.key, dk.digits, E, limbs,
                               dk.ginv, strided(conv, (size_t)T * N), rt, pmod_table(c, limbs),
                               ta ? fa : d3, P, o0, (u64)T * N, T, ta ? &fb : nullptr,
                               dk.own_b, dk.packed);
      launch_ntt_moddown(c, strided(conv, (size_t)T * N), nb, T, strided(acc, 2 * E * N), E, rt,
                         d3, P, gal.data(), o0, (u64)T * N, amul, &po, tile, dk.on);
    } else {
      Batch a1{}, o1{};
      for (int i = 0; i < nb; i++) {
        a1.p[i] = in[b0 + i]->d + P;
        o1.p[i] = out[b0 + i]->d + (size_t)T * N;
      }
      launch_ntt(c, strided(conv, (size_t)T * N), strided(conv, (size_t)T * N), 2 * nb, 0, T, T,
                 false);
      launch_moddown_combine(c, Strided{acc, 2 * E * N}, Strided{conv, 2 * T * N}, d3, a1,
                             gal.data(), o0, o1, nb, T, E, rt, amul, &po);
    }
  };
  for (int b0 = 0; b0 < n; b0 += kMaxBatch) run_parts(c, b0, std::min(kMaxBatch, n - b0), run);
}

// Constants of a rescale by the last D primes p_1 = q_{limbs-1}, p_2, ... of
// a `limbs`-limb ciphertext, T = limbs - D remaining limbs (k_rescale_lift):
// [T][2] (p_1..p_D)^-1 mod q_i + shoup; [T][D][3] p_1..p_j mod q_i (j < D
// factors), its shoup, p_{j+1} mod q_i; [D][D][3] p_m mod p_j, p_m^-1 mod
// p_j, shoup (m < j).
static const u64 *rescale_d_table(ckks_context *c, int limbs, int D) {
  auto key = std::make_pair(limbs, D);
  auto it = c->rescale_d.find(key);
  if (it != c->rescale_d.end()) return it->second;
  const int T = limbs - D;
  auto p = [&](int j) { return c->primes[limbs - 1 - j]; };  // p_{j+1}
  std::vector<u64> h(2 * (size_t)T + 3 * (size_t)T * D + 3 * (size_t)D * D, 0);
  for (int i = 0; i < T; i++) {
    const u64 q = c->primes[i];
    u64 prod = 1;
    for (int j = 0; j < D; j++) {
      u64 *e = &h[2 * (size_t)T + 3 * ((size_t)i * D + j)];
      e[0] = prod;
      e[1] = shoup_h(prod, q);
      e[2] = p(j) % q;
      prod = mulmod_h(prod, p(j) % q, q);
    }
    const u64 inv = invmod_h(prod, q);
    h[2 * i] = inv;
    h[2 * i + 1] = shoup_h(inv, q);
  }
  for (int j = 0; j < D; j++)
    for (int m = 0; m < j; m++) {
      u64 *e = &h[2 * (size_t)T + 3 * (size_t)T * D + 3 * ((size_t)j * D + m)];
      const u64 pj = p(j), pm = p(m) % pj, inv = invmod_h(pm, pj);
      e[0] = pm;
      e[1] = inv;
      e[2] = shoup_h(inv, pj);
    }
  u64 *d = nullptr;
  HIPCHECK(hipMalloc(&d, sizeof(u64) * h.size()));
  HIPCHECK(hipMemcpy(d, h.data(), sizeof(u64) * h.size(), hipMemcpyHostToDevice));
  return c->rescale_d[key] = d;
}

// Rescale n ciphertexts of `polys` polynomials each by their last D primes:
// the inverse NTT of those limbs, the combined lift (k_rescale_lift), its
// forward NTT and the combine, which at N = 2^16 runs in the NTT's last pass.
// The words equal those of D rescales in a row.
static void rescale_batch(ckks_context *c, const ckks_ct *const *in, int n, ckks_ct **out,
                          int D = 1) {
  const int limbs = in[0]->limbs, polys = in[0]->polys, T = limbs - D;
  const size_t N = c->N;
  const u64 *tab = rescale_d_table(c, limbs, D);
  const bool fused = c->logN == 16 && polys == 2;
  const int per = kMaxBatch / polys;
  audit_rescale(c, (double)n * polys * (limbs + T));
  for (int b0 = 0; b0 < n; b0 += per) {
    const int nb = std::min(per, n - b0), items = nb * polys;
    Scratch s(c);
    u64 *last = s.get((size_t)items * D * N);
    u64 *w = s.get((size_t)items * T * N);
    Batch src{}, dst{};
    for (int i = 0; i < nb; i++)
      for (int p = 0; p < polys; p++) {
        src.p[i * polys + p] = in[b0 + i]->d + (size_t)p * limbs * N;
        dst.p[i * polys + p] = out[b0 + i]->d + (size_t)p * T * N;
      }
    launch_ntt(c, src, strided(last - (size_t)T * N, (size_t)D * N), items, T, D, limbs, true);
    launch_rescale_lift(c, strided(last, (size_t)D * N), strided(w, (size_t)T * N), items, limbs,
                        D, tab);
    if (fused) {
      Batch acc{}, o{};
      for (int i = 0; i < nb; i++) {
        acc.p[i] = in[b0 + i]->d;
        o.p[i] = out[b0 + i]->d;
      }
      std::vector<u64> gal(nb, 1);
      launch_ntt_moddown(c, strided(w, (size_t)T * N), nb, T, acc, limbs, tab, Batch{}, 0,
                         gal.data(), o, (u64)T * N);
    } else {
      launch_ntt(c, strided(w, (size_t)T * N), strided(w, (size_t)T * N), items, 0, T, T, false);
      launch_rescale_finish(c, src, strided(w, (size_t)T * N), dst, items, T, tab);
    }
  }
}

// ===========================================================================
// extern "C" API
// ===========================================================================

extern "C" {

int ckks_context_create(const ckks_params *params, ckks_context **out) {
  API_BEGIN
  require(params && out, "null argument");
  ckks_context *c = new ckks_context();
  c->stream = nullptr;
  try {
    build_context(c, *params);
    // basis conversions run on the int8 matrix cores unless
    // CKKS_BASIS_CONVERT=valu selects the fp64/integer VALU kernels (same words)
    const char *bc = getenv("CKKS_BASIS_CONVERT");
    c->bc_mfma = !(bc && strcmp(bc, "valu") == 0);
    const char *kf = getenv("CKKS_KEYSWITCH_FUSED");
    c->ks_fused = !(kf && strcmp(kf, "0") == 0);
    const char *si = getenv("CKKS_KS_SPECIAL_INV");
    c->ks_sp_inv = !(si && strcmp(si, "0") == 0);
    const char *kt = getenv("CKKS_KS_TILE");
    c->ks_tile = !(kt && strcmp(kt, "0") == 0);
    const char *kd = getenv("CKKS_KS_DEFER");
    c->ks_defer = !(kd && strcmp(kd, "0") == 0);
    const char *ss = getenv("CKKS_SPLIT_STREAMS");
    if (ss) {
      c->split_parts = atoi(ss);
      require(c->split_parts >= 1 && c->split_parts <= ckks_context::kMaxSplit,
              "CKKS_SPLIT_STREAMS must be 1 .. 4");
    }
    c->split_streams = c->split_parts;
    HIPCHECK(hipEventCreateWithFlags(&c->fork_ev, hipEventDisableTiming));
    for (int i = 0; i + 1 < c->split_parts; i++) {
      // default priority, as the context stream
      HIPCHECK(hipStreamCreateWithFlags(&c->aux[i], hipStreamNonBlocking));
      HIPCHECK(hipEventCreateWithFlags(&c->join_ev[i], hipEventDisableTiming));
    }
    HIPCHECK(hipGetDevice(&c->device));
    c->noalloc_scratch = device_scratch(c->device, c->stream);
  } catch (...) {
    free_context(c);
    throw;
  }
  c->serial = g_next_serial++;
  g_live_contexts[c] = c->serial;
  *out = c;
  API_END
}

void ckks_context_destroy(ckks_context *ctx) {
  if (ctx && g_live_contexts.count(ctx)) free_context(ctx);
}

int ckks_context_info_get(const ckks_context *c, ckks_context_info *o) {
  API_BEGIN
  require(c && o, "null argument");
  o->N = c->N;
  o->log_n = c->logN;
  o->L = c->L;
  o->alpha = c->alpha;
  o->digit_size = c->ds;
  o->dnum = c->params.dnum;
  o->max_slots = c->N / 2;
  o->default_scale = ldexp(1.0, c->params.dcrt_bits);
  API_END
}

int ckks_context_primes(const ckks_context *c, uint64_t *out) {
  API_BEGIN
  require(c && out, "null argument");
  memcpy(out, c->primes.data(), sizeof(u64) * c->primes.size());
  API_END
}

int ckks_context_secret(const ckks_context *c, int8_t *out) {
  API_BEGIN
  require(c && out, "null argument");
  memcpy(out, c->secret.data(), c->secret.size());
  API_END
}

double ckks_scale_at(const ckks_context *c, int limbs) {
  (void)limbs;
  return ldexp(1.0, c->params.dcrt_bits);
}

double ckks_rescale_divisor_at(const ckks_context *c, int limbs) {
  if (limbs < 0 || limbs >= c->L) return 0.0;
  return (double)c->primes[limbs];
}

uint64_t ckks_galois_element(const ckks_context *c, int64_t rotation) {
  return galois_of(c, rotation);
}

int ckks_keygen_rotations(ckks_context *c, const int64_t *rot, int n) {
  API_BEGIN
  require(c && (rot || n == 0), "null argument");
  for (int i = 0; i < n; i++) {
    const u64 g = galois_of(c, rot[i]);
    if (g != 1) gen_key(c, g, 0, g);
  }
  // the conversion constants of every level, so that a rotation at any
  // level needs no further device allocation (ckks_rotate_many_noalloc)
  if (n > 0 && !c->rotation_tables) {
    for (int limbs = 1; limbs <= c->L; limbs++) {
      for (int j = 0; j * c->ds < limbs; j++) bc_up(c, limbs, j);
      bc_down(c, limbs);
      pinv_table(c, limbs);
      pmod_table(c, limbs);
    }
    c->rotation_tables = true;
  }
  API_END
}

int ckks_keygen_relin(ckks_context *c) {
  API_BEGIN
  require(c, "null argument");
  gen_key(c, 0, 1, 0);
  API_END
}

int ckks_has_rotation_key(const ckks_context *c, int64_t rotation) {
  const u64 g = galois_of(c, rotation);
  return g == 1 || c->keys.count(g) ? 1 : 0;
}

// key words in NTT position order and out of Montgomery form: word k of each
// row from position autom_index(k, g) of the stored key (g = 1: in place),
// stored at key_slot of it
__global__ void k_key_export(const u64 *__restrict__ key, u64 *__restrict__ out, size_t words,
                             int K, int logN, u64 g, const ModQ *__restrict__ mods) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= words) return;
  const size_t row = i >> logN;
  const u32 k = (u32)(i & (((size_t)1 << logN) - 1));
  const u32 s = g <= 1 ? k : autom_index(k, g, logN);
  const ModQ M = mods[(int)(row % K)];
  out[i] = redc(0, key[(row << logN) + key_slot(s)], M.q, M.qinv);
}

int ckks_key_download(ckks_context *c, uint64_t galois, uint64_t *out, int *digits) {
  API_BEGIN
  require(c, "null argument");
  const DeviceKey &k = get_key(c, galois);
  if (digits) *digits = k.digits;
  if (out) {
    const size_t words = k.bytes / sizeof(u64);
    u64 *tmp = (u64 *)c->pool.alloc(k.bytes);
    hipLaunchKernelGGL(k_key_export, dim3((words + 255) / 256), dim3(256), 0, c->stream, k.data,
                       tmp, words, c->K, c->logN, k.galois, c->d_mods);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipMemcpyAsync(out, tmp, k.bytes, hipMemcpyDeviceToHost, c->stream));
    HIPCHECK(hipStreamSynchronize(c->stream));
    c->pool.release(tmp, k.bytes);
  }
  API_END
}

int ckks_clear_rotation_keys(ckks_context *c, const int64_t *keep, int n) {
  API_BEGIN
  require(c, "null argument");
  std::vector<u64> kg;
  for (int i = 0; i < n; i++) kg.push_back(galois_of(c, keep[i]));
  HIPCHECK(hipStreamSynchronize(c->stream));
  for (auto it = c->keys.begin(); it != c->keys.end();) {
    if (it->first != 0 && std::find(kg.begin(), kg.end(), it->first) == kg.end()) {
      (void)hipFree(it->second.data);
      it = c->keys.erase(it);
    } else {
      ++it;
    }
  }
  API_END
}

int ckks_synchronize(ckks_context *c) {
  API_BEGIN
  require(c, "null argument");
  HIPCHECK(hipStreamSynchronize(c->stream));
  API_END
}

int ckks_memory_info(ckks_context *c, size_t *live, size_t *cached) {
  API_BEGIN
  require(c, "null argument");
  if (live) *live = c->pool.live;
  if (cached) *cached = c->pool.cached;
  API_END
}

int ckks_memory_stats(ckks_context *c, size_t *peak_live, size_t *segment_bytes,
                      uint64_t *device_allocs) {
  API_BEGIN
  require(c, "null argument");
  if (peak_live) *peak_live = c->pool.peak;
  if (segment_bytes) *segment_bytes = c->pool.segment_bytes;
  if (device_allocs) *device_allocs = c->pool.device_allocs;
  API_END
}

int ckks_empty_cache(ckks_context *c) {
  API_BEGIN
  require(c, "null argument");
  HIPCHECK(hipStreamSynchronize(c->stream));
  c->pool.trim();
  API_END
}

static void check_slots(const ckks_context *c, int slots) {
  require(slots >= 1 && slots <= c->N / 2 && !(slots & (slots - 1)),
          "slots must be a power of two in [1, N/2]");
  require(slots >= 2, "at least two slots are required");
}

static void check_limbs(const ckks_context *c, int limbs) {
  require(limbs >= 1 && limbs <= c->L, "limb count out of range [1, L]");
}

int ckks_encrypt(ckks_context *c, const double *re, const double *im, int slots, int limbs,
                 double scale, uint32_t enc_id, ckks_ct **out) {
  API_BEGIN
  require(c && re && out, "null argument");
  check_slots(c, slots);
  check_limbs(c, limbs);
  require(scale > 0, "scale must be positive");
  fft_table(c, slots);
  ckks_ct *ct = new_ct(c, 2, limbs, 0, slots, scale, 1);
  Scratch s(c);
  double *dre = (double *)s.get(slots), *dim = im ? (double *)s.get(slots) : nullptr;
  HIPCHECK(hipMemcpyAsync(dre, re, sizeof(double) * slots, hipMemcpyHostToDevice, c->stream));
  if (im)
    HIPCHECK(hipMemcpyAsync(dim, im, sizeof(double) * slots, hipMemcpyHostToDevice, c->stream));
  Batch o{};
  o.p[0] = ct->d;
  launch_encode(c, dre, dim, 1, slots, scale, limbs, 0, o);
  launch_encrypt_finish(c, ct->d, limbs, enc_id);
  HIPCHECK(hipStreamSynchronize(c->stream));  // host buffers are the caller's
  *out = ct;
  API_END
}

int ckks_decrypt(ckks_context *c, const ckks_ct *ct, double *re, double *im) {
  API_BEGIN
  require(c && re, "null argument");
  check_ct(c, ct, "decrypt");
  require(ct->polys >= 1 && !ct->is_ext, "decrypt needs a Q-basis ciphertext");
  fft_table(c, ct->slots);
  Scratch s(c);
  double *dre = (double *)s.get(ct->slots), *dim = (double *)s.get(ct->slots);
  launch_decrypt_decode(c, ct, dre, dim);
  HIPCHECK(hipMemcpyAsync(re, dre, sizeof(double) * ct->slots, hipMemcpyDeviceToHost, c->stream));
  if (im)
    HIPCHECK(hipMemcpyAsync(im, dim, sizeof(double) * ct->slots, hipMemcpyDeviceToHost, c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  API_END
}

int ckks_decode(ckks_context *c, const ckks_ct *pt, double *re, double *im) {
  return ckks_decrypt(c, pt, re, im);
}

int ckks_encode_rows(ckks_context *c, const double *re, const double *im, int rows, int slots,
                     int limbs, double scale, int is_ext, ckks_ct **out) {
  API_BEGIN
  require(c && re && out, "null argument");
  require(rows >= 1, "rows must be positive");
  check_slots(c, slots);
  check_limbs(c, limbs);
  fft_table(c, slots);
  for (int r = 0; r < rows; r++) out[r] = new_ct(c, 1, limbs, is_ext, slots, scale, 1);
  for (int r0 = 0; r0 < rows; r0 += kMaxBatch) {
    const int nr = std::min(kMaxBatch, rows - r0);
    Scratch s(c);
    double *dre = (double *)s.get((size_t)nr * slots);
    double *dim = im ? (double *)s.get((size_t)nr * slots) : nullptr;
    upload_async(c, dre, re + (size_t)r0 * slots, sizeof(double) * nr * slots);
    if (im) upload_async(c, dim, im + (size_t)r0 * slots, sizeof(double) * nr * slots);
    Batch o{};
    for (int r = 0; r < nr; r++) o.p[r] = out[r0 + r]->d;
    launch_encode(c, dre, dim, nr, slots, scale, limbs, is_ext, o);
  }
  API_END
}

int ckks_encode_scalar(ckks_context *c, double value, int limbs, double scale, ckks_ct **out) {
  API_BEGIN
  require(c && out, "null argument");
  check_limbs(c, limbs);
  ckks_ct *ct = new_ct(c, 0, limbs, 0, 0, scale, 1);
  launch_scalar_encode(c, value * scale, limbs, ct->d);
  *out = ct;
  API_END
}

int ckks_ct_upload(ckks_context *c, const uint64_t *data, int polys, int limbs, int is_ext,
                   int slots, double scale, int scale_degree, ckks_ct **out) {
  API_BEGIN
  require(c && data && out, "null argument");
  require(polys >= 1 && polys <= 3, "polys must be 1, 2 or 3");
  require(is_ext == 0 || is_ext == 1, "is_ext must be 0 or 1");
  check_limbs(c, limbs);
  check_slots(c, slots);
  require(scale > 0 && scale_degree >= 1, "scale must be positive and scale_degree at least 1");
  ckks_ct *ct = new_ct(c, polys, limbs, is_ext, slots, scale, scale_degree);
  HIPCHECK(hipMemcpyAsync(ct->d, data, ct->bytes, hipMemcpyHostToDevice, c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  *out = ct;
  API_END
}

int ckks_ct_download(ckks_context *c, const ckks_ct *ct, uint64_t *out) {
  API_BEGIN
  require(c && out, "null argument");
  check_ct(c, ct, "download");
  HIPCHECK(hipMemcpyAsync(out, ct->d, ct->bytes, hipMemcpyDeviceToHost, c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  API_END
}

int ckks_ct_info_get(const ckks_ct *ct, ckks_ct_info *o) {
  API_BEGIN
  require(ct && o, "null argument");
  o->polys = ct->polys;
  o->limbs = ct->limbs;
  o->is_ext = ct->is_ext;
  o->slots = ct->slots;
  o->scale = ct->scale;
  o->scale_degree = ct->scale_degree;
  API_END
}

int ckks_ct_set_scale(ckks_ct *ct, double scale, int scale_degree) {
  API_BEGIN
  require(ct, "null argument");
  ct->scale = scale;
  ct->scale_degree = scale_degree;
  API_END
}

int ckks_ct_copy(ckks_context *c, const ckks_ct *ct, ckks_ct **out) {
  API_BEGIN
  check_ct(c, ct, "copy");
  ckks_ct *o = new_ct(c, ct->polys, ct->limbs, ct->is_ext, ct->slots, ct->scale, ct->scale_degree);
  HIPCHECK(hipMemcpyAsync(o->d, ct->d, ct->bytes, hipMemcpyDeviceToDevice, c->stream));
  *out = o;
  API_END
}

void ckks_ct_free(ckks_ct *ct) { free_ct(ct); }

static int binary_limbwise(ckks_context *c, const ckks_ct *a, const ckks_ct *b, ckks_ct **out,
                           int op) {
  API_BEGIN
  check_poly(c, a, "add/sub");
  check_poly(c, b, "add/sub");
  require(out, "null argument");
  require(a->limbs == b->limbs, "operands must have the same limb count");
  require(a->is_ext == b->is_ext, "operands must share the basis");
  require(a->polys == b->polys, "operands must have the same degree");
  check_scales(a, b);
  ckks_ct *o = new_ct(c, a->polys, a->limbs, a->is_ext, a->slots, a->scale, a->scale_degree);
  const int total = a->limbs + (a->is_ext ? c->alpha : 0);
  launch_addsub(c, a->d, b->d, o->d, a->polys, total, a->limbs, op);
  *out = o;
  API_END
}

int ckks_add(ckks_context *c, const ckks_ct *a, const ckks_ct *b, ckks_ct **out) {
  return binary_limbwise(c, a, b, out, 0);
}

int ckks_sub(ckks_context *c, const ckks_ct *a, const ckks_ct *b, ckks_ct **out) {
  return binary_limbwise(c, a, b, out, 1);
}

int ckks_add_many(ckks_context *c, const ckks_ct *const *a, const ckks_ct *const *b, int n,
                  int op, ckks_ct **out) {
  API_BEGIN
  require(c && a && b && out && n >= 1, "null argument");
  require(op == 0 || op == 1, "op must be 0 (add) or 1 (sub)");
  // every pair is checked before any output exists
  for (int i = 0; i < n; i++) {
    check_poly(c, a[i], "add_many");
    check_poly(c, b[i], "add_many");
    require(a[i]->limbs == b[i]->limbs && a[i]->limbs == a[0]->limbs,
            "add_many operands must share one limb count");
    require(a[i]->is_ext == b[i]->is_ext && a[i]->is_ext == a[0]->is_ext,
            "add_many operands must share the basis");
    require(a[i]->polys == b[i]->polys && a[i]->polys == a[0]->polys,
            "add_many operands must share the degree");
    check_scales(a[i], b[i]);
  }
  const int limbs = a[0]->limbs, polys = a[0]->polys;
  const int total = limbs + (a[0]->is_ext ? c->alpha : 0);
  for (int i = 0; i < n; i++)
    out[i] = new_ct(c, polys, limbs, a[i]->is_ext, a[i]->slots, a[i]->scale, a[i]->scale_degree);
  for (int i0 = 0; i0 < n; i0 += kMaxBatch) {
    const int nb = std::min(kMaxBatch, n - i0);
    Batch ba{}, bb{}, bo{};
    for (int i = 0; i < nb; i++) {
      ba.p[i] = a[i0 + i]->d;
      bb.p[i] = b[i0 + i]->d;
      bo.p[i] = out[i0 + i]->d;
    }
    launch_addsub_many(c, ba, bb, bo, nb, polys, total, limbs, op);
  }
  API_END
}

int ckks_add_pt(ckks_context *c, const ckks_ct *a, const ckks_ct *pt, ckks_ct **out) {
  API_BEGIN
  check_poly(c, a, "add_pt");
  check_ct(c, pt, "add_pt");
  require(out, "null argument");
  require(pt->polys == 1 && pt->limbs >= a->limbs, "plaintext limbs below ciphertext limbs");
  require(!a->is_ext, "add_pt on a Q-basis ciphertext");
  check_scales(a, pt);
  ckks_ct *o = new_ct(c, a->polys, a->limbs, 0, a->slots, a->scale, a->scale_degree);
  const size_t P = (size_t)a->limbs * c->N;
  launch_addsub(c, a->d, pt->d, o->d, 1, a->limbs, a->limbs, 0);
  if (a->polys > 1)
    HIPCHECK(hipMemcpyAsync(o->d + P, a->d + P, sizeof(u64) * P * (a->polys - 1),
                            hipMemcpyDeviceToDevice, c->stream));
  *out = o;
  API_END
}

int ckks_mul_pt(ckks_context *c, const ckks_ct *a, const ckks_ct *pt, ckks_ct **out) {
  API_BEGIN
  check_poly(c, a, "mul_pt");
  check_ct(c, pt, "mul_pt");
  require(out, "null argument");
  require(pt->polys == 1 && pt->limbs >= a->limbs, "plaintext limbs below ciphertext limbs");
  if (a->is_ext)  // Q u P basis: the plaintext's P limbs must follow the same Q limbs
    require(pt->is_ext && pt->limbs == a->limbs,
            "an extended ciphertext needs an extended plaintext at its level");
  ckks_ct *o = new_ct(c, a->polys, a->limbs, a->is_ext, a->slots, a->scale * pt->scale,
                      a->scale_degree + pt->scale_degree);
  // a Q-basis product uses the leading (Q) limbs of an extended plaintext
  launch_mul_pt(c, a->d, pt->d, o->d, a->polys, a->limbs + (a->is_ext ? c->alpha : 0),
                a->limbs);
  *out = o;
  API_END
}

int ckks_grouped_mac(ckks_context *c, const ckks_ct *const *terms, const ckks_ct *const *pts,
                     const int *group_sizes, int n_groups, ckks_ct **out) {
  API_BEGIN
  require(c && terms && pts && group_sizes && out, "null argument");
  require(n_groups >= 1, "at least one group");
  int n = 0;
  for (int g = 0; g < n_groups; g++) {
    require(group_sizes[g] >= 1 && group_sizes[g] <= kMaxBatch,
            "a group takes 1 to 64 terms");
    n += group_sizes[g];
    out[g] = nullptr;
  }
  const ckks_ct *a0 = terms[0];
  check_poly(c, a0, "grouped_pairwise_mac");
  require(a0->polys == 2, "grouped_pairwise_mac: degree-1 ciphertexts");
  const double sc = a0->scale * pts[0]->scale;
  for (int t = 0; t < n; t++) {
    const ckks_ct *a = terms[t], *pt = pts[t];
    check_poly(c, a, "grouped_pairwise_mac");
    check_ct(c, pt, "grouped_pairwise_mac plaintext");
    require(a->polys == 2 && a->limbs == a0->limbs && a->is_ext == a0->is_ext,
            "grouped_pairwise_mac: terms at one level and basis");
    require(pt->polys == 1 && pt->limbs >= a->limbs, "plaintext limbs below ciphertext limbs");
    if (a->is_ext)
      require(pt->is_ext && pt->limbs == a->limbs,
              "an extended ciphertext needs an extended plaintext at its level");
    const double st = a->scale * pt->scale;
    require(fabs(st - sc) / std::max(st, sc) < 1.0 / 1024.0,
            "grouped_pairwise_mac: products at different scales");
  }
  const int total = a0->limbs + (a0->is_ext ? c->alpha : 0);
  int t0 = 0;
  try {
    for (int g = 0; g < n_groups; g++) {
      Batch bb{}, pb{};
      for (int b = 0; b < group_sizes[g]; b++) {
        bb.p[b] = terms[t0 + b]->d;
        pb.p[b] = pts[t0 + b]->d;
      }
      out[g] = new_ct(c, 2, a0->limbs, a0->is_ext, a0->slots, sc,
                      a0->scale_degree + pts[0]->scale_degree);
      launch_mac(c, bb, pb, group_sizes[g], out[g]->d, total, a0->limbs);
      t0 += group_sizes[g];
    }
  } catch (...) {
    for (int g = 0; g < n_groups; g++) {
      free_ct(out[g]);
      out[g] = nullptr;
    }
    throw;
  }
  API_END
}

int ckks_mul_i(ckks_context *c, const ckks_ct *a, int negative, ckks_ct **out) {
  API_BEGIN
  check_poly(c, a, "mul_i");
  require(out, "null argument");
  ckks_ct *o = new_ct(c, a->polys, a->limbs, a->is_ext, a->slots, a->scale, a->scale_degree);
  const int total = a->limbs + (a->is_ext ? c->alpha : 0);
  launch_mul_i(c, a->d, o->d, a->polys, total, a->limbs, negative);
  *out = o;
  API_END
}

int ckks_add_scalar(ckks_context *c, const ckks_ct *a, const ckks_ct *s, ckks_ct **out) {
  API_BEGIN
  check_poly(c, a, "add_scalar");
  check_ct(c, s, "add_scalar");
  require(out, "null argument");
  require(s->polys == 0 && s->limbs >= a->limbs, "scalar limbs below ciphertext limbs");
  require(!a->is_ext, "add_scalar on a Q-basis ciphertext");
  ckks_ct *o = new_ct(c, a->polys, a->limbs, 0, a->slots, a->scale, a->scale_degree);
  launch_scalar(c, a->d, s->d, o->d, a->polys, a->limbs, a->limbs, 0);
  *out = o;
  API_END
}

int ckks_mul_scalar(ckks_context *c, const ckks_ct *a, const ckks_ct *s, ckks_ct **out) {
  API_BEGIN
  check_poly(c, a, "mul_scalar");
  check_ct(c, s, "mul_scalar");
  require(out, "null argument");
  require(s->polys == 0 && s->limbs >= a->limbs, "scalar limbs below ciphertext limbs");
  require(!a->is_ext, "mul_scalar on a Q-basis ciphertext");
  ckks_ct *o = new_ct(c, a->polys, a->limbs, 0, a->slots, a->scale * s->scale,
                      a->scale_degree + (s->scale == 1.0 ? 0 : 1));
  launch_scalar(c, a->d, s->d, o->d, a->polys, a->limbs, a->limbs, 1);
  *out = o;
  API_END
}

int ckks_mul_no_relin(ckks_context *c, const ckks_ct *a, const ckks_ct *b, ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "mul");
  check_ct(c, b, "mul");
  require(out, "null argument");
  require(a->polys == 2 && b->polys == 2, "mul expects degree-1 ciphertexts");
  require(a->limbs == b->limbs, "operands must have the same limb count");
  require(!a->is_ext && !b->is_ext, "mul expects Q-basis ciphertexts");
  ckks_ct *o = new_ct(c, 3, a->limbs, 0, a->slots, a->scale * b->scale,
                      a->scale_degree + b->scale_degree);
  Batch ba{}, bb{}, bo{};
  ba.p[0] = a->d;
  bb.p[0] = b->d;
  bo.p[0] = o->d;
  launch_tensor(c, ba, bb, bo, 1, a->limbs);
  *out = o;
  API_END
}

int ckks_relinearize(ckks_context *c, const ckks_ct *a, ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "relinearize");
  require(out, "null argument");
  require(a->polys == 3, "relinearize expects a degree-2 ciphertext");
  ckks_ct *o = new_ct(c, 2, a->limbs, 0, a->slots, a->scale, a->scale_degree);
  try {
    relin_batch(c, &a, 1, &o);
  } catch (...) {
    free_ct(o);
    throw;
  }
  *out = o;
  API_END
}

int ckks_mul_relin(ckks_context *c, const ckks_ct *a, const ckks_ct *b, ckks_ct **out) {
  ckks_ct *t = nullptr;
  int rc = ckks_mul_no_relin(c, a, b, &t);
  if (rc) return rc;
  rc = ckks_relinearize(c, t, out);
  free_ct(t);
  return rc;
}

int ckks_rescale(ckks_context *c, const ckks_ct *a, ckks_ct **out) {
  API_BEGIN
  check_poly(c, a, "rescale");
  require(out, "null argument");
  require(a->limbs >= 2, "rescale needs at least two limbs");
  require(!a->is_ext, "rescale expects a Q-basis ciphertext");
  const double div = (double)c->primes[a->limbs - 1];
  ckks_ct *o = new_ct(c, a->polys, a->limbs - 1, 0, a->slots, a->scale / div,
                      std::max(1, a->scale_degree - 1));
  rescale_batch(c, &a, 1, &o);
  *out = o;
  API_END
}

int ckks_drop_limbs(ckks_context *c, const ckks_ct *a, int target, ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "drop_limbs");
  require(out, "null argument");
  require(!a->is_ext, "drop_limbs expects a Q-basis ciphertext");
  require(target >= 1 && target <= a->limbs, "target limbs out of range");
  ckks_ct *o = new_ct(c, a->polys, target, 0, a->slots, a->scale, a->scale_degree);
  if (a->polys == 0) {
    // a scalar constant: one word per limb, the leading `target` of them
    HIPCHECK(hipMemcpyAsync(o->d, a->d, sizeof(u64) * target, hipMemcpyDeviceToDevice, c->stream));
    *out = o;
    return CKKS_OK;
  }
  const size_t N = c->N;
  for (int p = 0; p < a->polys; p++)
    HIPCHECK(hipMemcpyAsync(o->d + (size_t)p * target * N, a->d + (size_t)p * a->limbs * N,
                            sizeof(u64) * target * N, hipMemcpyDeviceToDevice, c->stream));
  *out = o;
  API_END
}

int ckks_mod_raise(ckks_context *c, const ckks_ct *a, int target_limbs, ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "mod_raise");
  require(out, "null argument");
  require(a->limbs == 1 && !a->is_ext, "mod_raise expects a one-limb Q-basis ciphertext");
  require(a->polys >= 1 && a->polys <= 3, "mod_raise expects 1 to 3 polynomials");
  check_limbs(c, target_limbs);
  const size_t N = c->N;
  ckks_ct *o = new_ct(c, a->polys, target_limbs, 0, a->slots, a->scale, a->scale_degree);
  Scratch s(c);
  u64 *coef = s.get((size_t)a->polys * N);
  launch_ntt(c, strided(a->d, N), strided(coef, N), a->polys, 0, 1, 1, true);
  launch_mod_raise(c, coef, o->d, a->polys, target_limbs);
  launch_ntt(c, strided(o->d, (size_t)target_limbs * N), strided(o->d, (size_t)target_limbs * N),
             a->polys, 0, target_limbs, target_limbs, false);
  *out = o;
  API_END
}

int ckks_rotate_many(ckks_context *c, const ckks_ct *const *in, int n, int64_t rotation,
                     ckks_ct **out) {
  API_BEGIN
  require(c && in && out && n >= 1, "null argument");
  for (int i = 0; i < n; i++) {
    check_ct(c, in[i], "rotate");
    require(in[i]->polys == 2 && !in[i]->is_ext, "rotate expects degree-1 Q-basis ciphertexts");
    require(in[i]->limbs == in[0]->limbs, "batched rotation needs one common level");
  }
  const u64 g = galois_of(c, rotation);
  if (g != 1) get_key(c, g);
  std::vector<ckks_ct *> o(n, nullptr);
  for (int i = 0; i < n; i++)
    o[i] = new_ct(c, 2, in[i]->limbs, 0, in[i]->slots, in[i]->scale, in[i]->scale_degree);
  if (g == 1) {
    for (int i = 0; i < n; i++)
      HIPCHECK(hipMemcpyAsync(o[i]->d, in[i]->d, in[i]->bytes, hipMemcpyDeviceToDevice, c->stream));
  } else {
    rotate_batch(c, in, n, g, o.data());
  }
  for (int i = 0; i < n; i++) out[i] = o[i];
  API_END
}

int ckks_rotate(ckks_context *c, const ckks_ct *a, int64_t rotation, ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "rotate");
  require(out, "null argument");
  const u64 g = galois_of(c, rotation);
  if (g == 1) {
    ckks_ct *o = new_ct(c, a->polys, a->limbs, a->is_ext, a->slots, a->scale, a->scale_degree);
    HIPCHECK(hipMemcpyAsync(o->d, a->d, a->bytes, hipMemcpyDeviceToDevice, c->stream));
    *out = o;
    return CKKS_OK;
  }
  require(a->polys == 2 && !a->is_ext, "rotate expects a degree-1 Q-basis ciphertext");
  get_key(c, g);
  ckks_ct *o = new_ct(c, 2, a->limbs, 0, a->slots, a->scale, a->scale_degree);
  rotate_batch(c, &a, 1, g, &o);
  *out = o;
  API_END
}

int ckks_rotate_many_noalloc(ckks_context *c, const ckks_ct *const *in, int n, int64_t rotation,
                             ckks_ct *const *out) {
  API_BEGIN
  require(c && in && out, "null argument");
  require(n >= 1 && n <= kMaxBatch, "noalloc rotation takes 1 to 64 ciphertexts");
  check_ct(c, in[0], "rotate_noalloc");
  const int limbs = in[0]->limbs;
  for (int i = 0; i < n; i++) {
    check_ct(c, in[i], "rotate_noalloc");
    check_ct(c, out[i], "rotate_noalloc output");
    require(in[i]->polys == 2 && !in[i]->is_ext && in[i]->limbs == limbs,
            "noalloc rotation expects degree-1 Q-basis ciphertexts at one level");
    require(out[i]->polys == 2 && !out[i]->is_ext && out[i]->limbs == limbs,
            "each output must be a degree-1 Q-basis ciphertext at the input's level");
    for (int j = 0; j < n; j++)
      require(out[i]->d != in[j]->d, "an output may not be one of the inputs");
    for (int j = 0; j < i; j++) require(out[i]->d != out[j]->d, "outputs must be distinct");
  }
  const u64 g = galois_of(c, rotation);
  size_t need = 0;
  if (g != 1) {
    get_key(c, g);
    require(c->rotation_tables,
            "the key-switch constants are built with the rotation keys (ckks_keygen_rotations)");
    need = rotate_scratch_words(c, limbs, n);
    require(need <= kNoAllocWords,
            "noalloc rotation needs " + std::to_string(need * 8 >> 20) +
                " MiB of scratch, above its fixed 256 MiB: rotate fewer ciphertexts per call");
    require(c->noalloc_scratch != nullptr, "fixed scratch not resolved for this device");
  }
  if (g == 1) {
    for (int i = 0; i < n; i++)
      HIPCHECK(hipMemcpyAsync(out[i]->d, in[i]->d, in[i]->bytes, hipMemcpyDeviceToDevice,
                              c->stream));
  } else {
    NoAllocDevice &nd = g_noalloc[c->device];
    std::lock_guard<std::mutex> lk(nd.mu);
    HIPCHECK(hipStreamWaitEvent(c->stream, nd.done, 0));
    // whatever was enqueued (also if a launch below fails) uses the buffer:
    // the next call waits for it
    struct Release {
      NoAllocDevice &nd;
      hipStream_t st;
      ~Release() { (void)hipEventRecord(nd.done, st); }
    } release{nd, c->stream};
    ckks_ct *o[kMaxBatch];
    for (int i = 0; i < n; i++) o[i] = out[i];
    size_t used = 0;
    rotate_batch(c, in, n, g, o, c->noalloc_scratch, kNoAllocWords, &used);
    require(used <= need, "noalloc rotation used " + std::to_string(used) +
                              " scratch words, above the " + std::to_string(need) + " it sized");
  }
  for (int i = 0; i < n; i++) {
    out[i]->slots = in[i]->slots;
    out[i]->scale = in[i]->scale;
    out[i]->scale_degree = in[i]->scale_degree;
  }
  API_END
}

// HMult + relinearise + `primes` rescales of n pairs, with the postop of
// ps (primes == 1) folded into the ModDown epilogue when the merged path
// applies and applied by limb-wise launches otherwise.
static void mul_relin_rescale(ckks_context *c, const ckks_ct *const *a, const ckks_ct *const *b,
                              int n, int primes, const PostSpec *ps, ckks_ct **out) {
  for (int i = 0; i < n; i++) out[i] = nullptr;
  check_ct(c, a[0], "mul");
  const int limbs = a[0]->limbs;
  require(primes >= 1 && primes <= kMaxRescaleDrop, "a rescale divides by 1 to 4 primes");
  require(limbs > primes, "rescale needs more limbs than the primes it divides by");
  for (int i = 0; i < n; i++) {
    check_ct(c, a[i], "mul");
    check_ct(c, b[i], "mul");
    require(a[i]->polys == 2 && b[i]->polys == 2, "mul expects degree-1 ciphertexts");
    require(a[i]->limbs == limbs && b[i]->limbs == limbs, "one common level required");
  }
  get_key(c, 0);
  const size_t N = c->N;
  const bool merged = relin_rs_fits(c, limbs, primes);
  for (int b0 = 0; b0 < n; b0 += kMaxBatch) {
    const int nb = std::min(kMaxBatch, n - b0);
    Scratch s(c);
    u64 *t3 = s.get((size_t)nb * 3 * limbs * N);
    u64 *t2 = merged ? nullptr : s.get((size_t)nb * 2 * limbs * N);
    Batch ba{}, bb{};
    for (int i = 0; i < nb; i++) {
      ba.p[i] = a[b0 + i]->d;
      bb.p[i] = b[b0 + i]->d;
    }
    // the merged path forms the products itself, part by part
    if (!merged) launch_tensor(c, ba, bb, strided(t3, (size_t)3 * limbs * N), nb, limbs);
    std::vector<ckks_ct> v3(nb), v2(nb);
    std::vector<const ckks_ct *> p3(nb);
    std::vector<ckks_ct *> p2(nb);
    for (int i = 0; i < nb; i++) {
      v3[i] = ckks_ct{c, t3 + (size_t)i * 3 * limbs * N, 0, 3, limbs, 0, a[b0 + i]->slots, 2, 0};
      p3[i] = &v3[i];
      if (!merged) {
        v2[i] = ckks_ct{c, t2 + (size_t)i * 2 * limbs * N, 0, 2, limbs, 0, a[b0 + i]->slots, 2, 0};
        p2[i] = &v2[i];
      }
    }
    std::vector<ckks_ct *> o(nb);
    for (int i = 0; i < nb; i++) {
      double scale = a[b0 + i]->scale * b[b0 + i]->scale;
      int degree = a[b0 + i]->scale_degree + b[b0 + i]->scale_degree;
      for (int j = 0; j < primes; j++) {
        scale /= (double)c->primes[limbs - 1 - j];
        degree = std::max(1, degree - 1);
      }
      o[i] = out[b0 + i] = new_ct(c, 2, limbs - primes, 0, a[b0 + i]->slots, scale, degree);
    }
    if (merged) {
      // relin_rescale_batch indexes the subtrahends from its own first item
      PostSpec pss{};
      if (ps) pss = PostSpec{ps->dbl, ps->sub ? ps->sub + b0 : nullptr, ps->scal};
      relin_rescale_batch(c, p3.data(), nb, o.data(), primes, ps ? &pss : nullptr, &ba, &bb);
      continue;
    }
    relin_batch(c, p3.data(), nb, p2.data());
    std::vector<const ckks_ct *> cp2(p2.begin(), p2.end());
    rescale_batch(c, cp2.data(), nb, o.data(), primes);
    if (!ps) continue;
    const int T = limbs - primes;
    for (int i = 0; i < nb; i++) {
      u64 *od = o[i]->d;
      if (ps->dbl) launch_addsub(c, od, od, od, 2, T, T, 0);
      if (ps->sub) {
        const ckks_ct *sb = ps->sub[b0 + i];
        for (int comp = 0; comp < 2; comp++)
          launch_addsub(c, od + (size_t)comp * T * N, sb->d + (size_t)comp * sb->limbs * N,
                        od + (size_t)comp * T * N, 1, T, T, 1);
      }
      if (ps->scal) launch_scalar(c, od, ps->scal, od, 2, T, T, 0);
    }
  }
}

int ckks_mul_relin_rescale_many_by(ckks_context *c, const ckks_ct *const *a,
                                   const ckks_ct *const *b, int n, int primes, ckks_ct **out) {
  API_BEGIN
  require(c && a && b && out && n >= 1, "null argument");
  mul_relin_rescale(c, a, b, n, primes, nullptr, out);
  API_END
}

int ckks_mul_relin_rescale_postop_many(ckks_context *c, const ckks_ct *const *a,
                                       const ckks_ct *const *b, int n, int apply_double,
                                       const ckks_ct *const *sub, const ckks_ct *scalar,
                                       ckks_ct **out) {
  API_BEGIN
  require(c && a && b && out && n >= 1, "null argument");
  check_ct(c, a[0], "postop");
  require(a[0]->limbs >= 2, "the product needs at least two limbs");
  const int T = a[0]->limbs - 1;
  if (sub) {
    for (int i = 0; i < n; i++) {
      check_ct(c, sub[i], "postop sub");
      require(sub[i]->polys == 2 && !sub[i]->is_ext && sub[i]->limbs >= T,
              "sub must be a degree-1 Q-basis ciphertext at or above the output level");
      require(sub[i]->limbs == sub[0]->limbs, "every sub must have one limb count");
      require(a[i] && b[i], "null argument");
      const double s = a[i]->scale * b[i]->scale / (double)c->primes[T];
      const double r = fabs(s - sub[i]->scale) / std::max(s, sub[i]->scale);
      require(r < 1.0 / 1024.0, "sub's scale differs from the product's");
    }
  }
  if (scalar) {
    check_ct(c, scalar, "postop scalar");
    require(scalar->polys == 0 && scalar->limbs >= T, "scalar limbs below the output level");
  }
  PostSpec ps{apply_double ? 1 : 0, sub, scalar ? scalar->d : nullptr};
  mul_relin_rescale(c, a, b, n, 1, &ps, out);
  API_END
}

int ckks_mul_relin_rescale_many(ckks_context *c, const ckks_ct *const *a,
                                const ckks_ct *const *b, int n, ckks_ct **out) {
  return ckks_mul_relin_rescale_many_by(c, a, b, n, 1, out);
}

int ckks_hoisted_rotate(ckks_context *c, const ckks_ct *a, const int64_t *rotations, int n,
                        ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "hoisted_rotate");
  require(out && rotations && n >= 1, "null argument");
  require(a->polys == 2 && !a->is_ext, "hoisted rotation expects a degree-1 Q-basis ciphertext");
  const int limbs = a->limbs;
  const size_t N = c->N, P = (size_t)limbs * N;
  std::vector<u64> gs(n);
  for (int i = 0; i < n; i++) {
    gs[i] = galois_of(c, rotations[i]);
    if (gs[i] != 1) get_key(c, gs[i]);
  }
  std::vector<ckks_ct *> o(n);
  for (int i = 0; i < n; i++) o[i] = new_ct(c, 2, limbs, 0, a->slots, a->scale, a->scale_degree);
  std::vector<KsJob> jobs;
  for (int i = 0; i < n; i++) {
    if (gs[i] == 1)
      HIPCHECK(hipMemcpyAsync(o[i]->d, a->d, a->bytes, hipMemcpyDeviceToDevice, c->stream));
    else
      jobs.push_back(KsJob{0, &get_key(c, gs[i]), gs[i], a->d, nullptr, o[i]->d, o[i]->d + P});
  }
  if (!jobs.empty()) {
    Scratch s(c);
    const int digits = (limbs + c->ds - 1) / c->ds, E = limbs + c->alpha;
    u64 *ext = s.get((size_t)digits * E * N);
    const u64 *d = a->d + P;
    ks_modup(c, limbs, 1, &d, ext, s);
    for (size_t j0 = 0; j0 < jobs.size(); j0 += kMaxBatch) {
      std::vector<KsJob> part(jobs.begin() + j0,
                              jobs.begin() + std::min(jobs.size(), j0 + kMaxBatch));
      ks_finish(c, limbs, ext, 1, part, s);
    }
  }
  for (int i = 0; i < n; i++) out[i] = o[i];
  API_END
}

int ckks_hoisted_rotate_many(ckks_context *c, const ckks_ct *const *a, int m,
                             const int64_t *rotations, int n, ckks_ct **out) {
  API_BEGIN
  require(a && out && rotations && m >= 1 && n >= 1, "null argument");
  for (int j = 0; j < m * n; j++) out[j] = nullptr;
  const int limbs = a[0]->limbs;
  for (int i = 0; i < m; i++) {
    check_ct(c, a[i], "hoisted_rotate_many");
    require(a[i]->polys == 2 && !a[i]->is_ext && a[i]->limbs == limbs,
            "hoisted rotation expects degree-1 Q-basis ciphertexts at one level");
  }
  const size_t N = c->N, P = (size_t)limbs * N;
  std::vector<u64> gs(n);
  for (int r = 0; r < n; r++) {
    gs[r] = galois_of(c, rotations[r]);
    if (gs[r] != 1) get_key(c, gs[r]);
  }
  std::vector<ckks_ct *> o((size_t)m * n);
  for (int i = 0; i < m; i++)
    for (int r = 0; r < n; r++)
      o[(size_t)i * n + r] = new_ct(c, 2, limbs, 0, a[i]->slots, a[i]->scale, a[i]->scale_degree);
  const int digits = (limbs + c->ds - 1) / c->ds, E = limbs + c->alpha;
  for (int i0 = 0; i0 < m; i0 += kMaxBatch) {
    const int mb = std::min(kMaxBatch, m - i0);
    Scratch s(c);
    u64 *ext = nullptr;
    for (int r = 0; r < n; r++) {
      if (gs[r] == 1) {
        for (int i = i0; i < i0 + mb; i++)
          HIPCHECK(hipMemcpyAsync(o[(size_t)i * n + r]->d, a[i]->d, a[i]->bytes,
                                  hipMemcpyDeviceToDevice, c->stream));
        continue;
      }
      if (!ext) {
        // one ModUp per ciphertext, shared by every rotation
        ext = s.get((size_t)mb * digits * E * N);
        std::vector<const u64 *> d(mb);
        for (int i = 0; i < mb; i++) d[i] = a[i0 + i]->d + P;
        ks_modup(c, limbs, mb, d.data(), ext, s);
      }
      // one rotation for the whole batch: its key is read once
      const DeviceKey &key = get_key(c, gs[r]);
      std::vector<KsJob> jobs(mb);
      for (int i = 0; i < mb; i++) {
        ckks_ct *d = o[(size_t)(i0 + i) * n + r];
        jobs[i] = KsJob{i, &key, gs[r], a[i0 + i]->d, nullptr, d->d, d->d + P};
      }
      Scratch s2(c);
      ks_finish(c, limbs, ext, mb, jobs, s2);
    }
  }
  for (size_t j = 0; j < o.size(); j++) out[j] = o[j];
  API_END
}

int ckks_hoisted_mac_sum(ckks_context *c, const ckks_ct *const *babies, int B,
                         const ckks_ct *const *pts, int64_t giant_rotation, int giant_count,
                         ckks_ct **out) {
  API_BEGIN
  require(c && babies && pts && out, "null argument");
  require(B >= 1 && B <= kMaxBatch, "baby count must be in [1, 64]");
  require(giant_count >= 1, "giant_count must be positive");
  const int limbs = babies[0]->limbs;
  for (int b = 0; b < B; b++) {
    check_ct(c, babies[b], "hoisted_mac_sum");
    require(babies[b]->limbs == limbs && babies[b]->polys == 2 && !babies[b]->is_ext,
            "babies must be degree-1 Q-basis ciphertexts at one level");
  }
  for (int i = 0; i < B * giant_count; i++) {
    check_ct(c, pts[i], "hoisted_mac_sum");
    // an extended plaintext stores its Q limbs first, so its leading
    // `limbs` limbs are used as they are
    require(pts[i]->polys == 1 && pts[i]->limbs >= limbs,
            "plaintexts must be at or above the babies' level");
  }
  const u64 gg = galois_of(c, giant_rotation);
  if (giant_count > 1 && gg != 1) get_key(c, gg);
  const double scale = babies[0]->scale * pts[0]->scale;
  const int sdeg = babies[0]->scale_degree + pts[0]->scale_degree;
  const size_t N = c->N, P = (size_t)limbs * N;
  Batch bb{};
  for (int b = 0; b < B; b++) bb.p[b] = babies[b]->d;
  ckks_ct *acc = nullptr;
  Scratch s(c);
  u64 *inner = s.get(2 * P);
  for (int g = giant_count - 1; g >= 0; g--) {
    Batch bp{};
    for (int b = 0; b < B; b++) bp.p[b] = pts[g * B + b]->d;
    if (!acc) {
      acc = new_ct(c, 2, limbs, 0, babies[0]->slots, scale, sdeg);
      launch_mac(c, bb, bp, B, acc->d, limbs, limbs);
      continue;
    }
    launch_mac(c, bb, bp, B, inner, limbs, limbs);
    ckks_ct *rot = new_ct(c, 2, limbs, 0, acc->slots, scale, sdeg);
    if (gg == 1)
      HIPCHECK(hipMemcpyAsync(rot->d, acc->d, acc->bytes, hipMemcpyDeviceToDevice, c->stream));
    else {
      const ckks_ct *ac = acc;
      rotate_batch(c, &ac, 1, gg, &rot);
    }
    launch_addsub(c, rot->d, inner, acc->d, 2, limbs, limbs, 0);
    free_ct(rot);
  }
  *out = acc;
  API_END
}

// out[i] = a[i] + b[i] for n degree-1 ciphertexts at `limbs` limbs, 64 pairs
// per launch (the giant Horner chains' adds)
// (item i's second operand at b + i b_stride)
static void add_batched(ckks_context *c, const std::vector<ckks_ct *> &a, const u64 *b,
                        size_t b_stride, ckks_ct *const *out, int n, int limbs) {
  for (int b0 = 0; b0 < n; b0 += kMaxBatch) {
    const int nb = std::min(kMaxBatch, n - b0);
    Batch ba{}, bb{}, bo{};
    for (int i = 0; i < nb; i++) {
      ba.p[i] = a[b0 + i]->d;
      bb.p[i] = (u64 *)(b + (size_t)(b0 + i) * b_stride);
      bo.p[i] = out[b0 + i]->d;
    }
    launch_addsub_many(c, ba, bb, bo, nb, 2, limbs, limbs, 0);
  }
}

int ckks_hoisted_mac_sum_many(ckks_context *c, const ckks_ct *const *babies, int n, int B,
                              const ckks_ct *const *pts, int64_t giant_rotation,
                              int giant_count, ckks_ct **out) {
  API_BEGIN
  require(c && babies && pts && out, "null argument");
  require(n >= 1 && B >= 1, "ciphertext and baby counts must be positive");
  require(giant_count >= 1, "giant_count must be positive");
  require(((size_t)n + std::min(kTabGroups, giant_count)) * B <= 8192,
          "(ciphertexts + min(giants, 8)) x babies must be at most 8192 (split the batch)");
  for (int i = 0; i < n; i++) out[i] = nullptr;
  const int limbs = babies[0]->limbs;
  for (int j = 0; j < n * B; j++) {
    check_ct(c, babies[j], "hoisted_mac_sum_many");
    require(babies[j]->limbs == limbs && babies[j]->polys == 2 && !babies[j]->is_ext,
            "babies must be degree-1 Q-basis ciphertexts at one level");
  }
  for (int j = 0; j < B * giant_count; j++) {
    check_ct(c, pts[j], "hoisted_mac_sum_many");
    // an extended plaintext stores its Q limbs first
    require(pts[j]->polys == 1 && pts[j]->limbs >= limbs,
            "plaintexts must be at or above the babies' level");
  }
  const u64 gg = galois_of(c, giant_rotation);
  if (giant_count > 1 && gg != 1) get_key(c, gg);
  const size_t N = c->N, CP = 2 * (size_t)limbs * N;
  std::vector<u64> btab((size_t)n * B), ptab((size_t)B * giant_count);
  for (size_t j = 0; j < btab.size(); j++) btab[j] = (u64)babies[j]->d;
  for (size_t j = 0; j < ptab.size(); j++) ptab[j] = (u64)pts[j]->d;
  Scratch s(c);
  u64 *dbt = s.get(btab.size()), *dpt = s.get(ptab.size());
  upload_async(c, dbt, btab.data(), sizeof(u64) * btab.size());
  upload_async(c, dpt, ptab.data(), sizeof(u64) * ptab.size());
  const int GC = std::min(kTabGroups, giant_count);
  u64 *inner = s.get((size_t)GC * n * CP);
  const double scale = babies[0]->scale * pts[0]->scale;
  const int sdeg = babies[0]->scale_degree + pts[0]->scale_degree;
  int g_lo = giant_count;  // groups [g_lo, g_lo + GC) are in inner
  for (int g = giant_count - 1; g >= 0; g--) {
    if (g < g_lo) {
      g_lo = std::max(0, g - GC + 1);
      launch_mac_table(c, (const u64 *const *)dbt, n, (const u64 *const *)(dpt + (size_t)g_lo * B),
                       B, g - g_lo + 1, inner, limbs);
    }
    const u64 *ig = inner + (size_t)(g - g_lo) * n * CP;
    if (!out[0]) {
      for (int i = 0; i < n; i++) {
        out[i] = new_ct(c, 2, limbs, 0, babies[(size_t)i * B]->slots, scale, sdeg);
        HIPCHECK(hipMemcpyAsync(out[i]->d, ig + (size_t)i * CP, sizeof(u64) * CP,
                                hipMemcpyDeviceToDevice, c->stream));
      }
      continue;
    }
    // Horner: out = rot(out) + inner_g, the rotations batched over the n
    std::vector<ckks_ct *> rot(n);
    for (int i = 0; i < n; i++)
      rot[i] = new_ct(c, 2, limbs, 0, out[i]->slots, scale, sdeg);
    if (gg == 1) {
      for (int i = 0; i < n; i++)
        HIPCHECK(hipMemcpyAsync(rot[i]->d, out[i]->d, out[i]->bytes, hipMemcpyDeviceToDevice,
                                c->stream));
    } else {
      std::vector<const ckks_ct *> cur(out, out + n);
      rotate_batch(c, cur.data(), n, gg, rot.data());
    }
    add_batched(c, rot, ig, CP, out, n, limbs);
    for (int i = 0; i < n; i++) free_ct(rot[i]);
  }
  API_END
}

// Extended-basis babies of n ciphertexts for the given rotations, each
// [2][E][N] before its ModDown: (P c0, P c1) for offset 0,
// (P sigma(c0) + acc_0, acc_1) otherwise.  One ModUp per ciphertext (batched)
// is shared by all rotations; each rotation's key is read once for all n.
// dst[b * n + i] is baby b of ciphertext i.
static void ext_babies(ckks_context *c, const ckks_ct *const *a, int n, const int64_t *rotations,
                       int nr, u64 *const *dst, Scratch &s) {
  const int limbs = a[0]->limbs, E = limbs + c->alpha, digits = (limbs + c->ds - 1) / c->ds;
  const size_t N = c->N, P = (size_t)limbs * N, est = (size_t)digits * E * N;
  std::vector<u64> gal(nr);
  bool any = false;
  for (int b = 0; b < nr; b++) {
    gal[b] = galois_of(c, rotations[b]);
    if (gal[b] != 1) {
      get_key(c, gal[b]);
      any = true;
    }
  }
  u64 *ext = nullptr;
  if (any) {
    ext = s.get((size_t)n * est);
    std::vector<const u64 *> d1(n);
    for (int i = 0; i < n; i++) d1[i] = a[i]->d + P;
    ks_modup(c, limbs, n, d1.data(), ext, s);
  }
  std::vector<int> rb;
  std::vector<const DeviceKey *> keys;
  std::vector<u64> ginv;
  const u64 two_n = 2 * (u64)c->N;
  for (int b = 0; b < nr; b++) {
    if (gal[b] == 1) {
      for (int i = 0; i < n; i++) launch_ext_identity(c, a[i]->d, dst[b * n + i], limbs);
      continue;
    }
    rb.push_back(b);
    keys.push_back(&get_key(c, gal[b]));
    // the units mod 2N have order N, so g^-1 = g^(N-1)
    u64 inv = 1, base = gal[b] % two_n;
    for (u64 e = c->N - 1; e; e >>= 1, base = base * base % two_n)
      if (e & 1) inv = inv * base % two_n;
    ginv.push_back(inv);
  }
  if (rb.empty()) return;
  // every rotation of a chunk of ciphertexts in one pass over the digits
  for (int i0 = 0; i0 < n; i0 += kMultiItems) {
    const int ni = std::min(kMultiItems, n - i0);
    std::vector<const u64 *> table(rb.size() * ni);
    for (size_t r = 0; r < rb.size(); r++)
      for (int it = 0; it < ni; it++) table[r * ni + it] = dst[(size_t)rb[r] * n + i0 + it];
    u64 *dtab = s.get(table.size());
    upload_async(c, dtab, table.data(), sizeof(u64) * table.size());
    Batch c0{};
    for (int it = 0; it < ni; it++) c0.p[it] = a[i0 + it]->d;
    launch_key_inner_multi(c, ext + (size_t)i0 * est, est, ni, keys, ginv, c0,
                           (const u64 *const *)dtab, digits, E, limbs);
  }
}

// hoisted_mac_sum_ext for n ciphertexts at one level sharing the plaintexts.
static void mac_sum_ext(ckks_context *c, const ckks_ct *const *a, int n,
                        const int64_t *baby_rotations, int B, const ckks_ct *const *pts,
                        int64_t giant_rotation, int giant_count, ckks_ct **out) {
  require(n >= 1 && n <= kMaxBatch, "ciphertext count must be in [1, 64]");
  require(B >= 1 && B <= kMaxBatch, "baby count must be in [1, 64]");
  require(giant_count >= 1, "giant_count must be positive");
  const int limbs = a[0]->limbs, E = limbs + c->alpha;
  for (int i = 0; i < n; i++) {
    check_ct(c, a[i], "hoisted_mac_sum_ext");
    require(a[i]->polys == 2 && !a[i]->is_ext && a[i]->limbs == limbs,
            "hoisted_mac_sum_ext expects degree-1 Q-basis ciphertexts at one level");
  }
  for (int i = 0; i < B * giant_count; i++) {
    check_ct(c, pts[i], "hoisted_mac_sum_ext");
    require(pts[i]->polys == 1 && pts[i]->is_ext && pts[i]->limbs == limbs,
            "plaintexts must be extended (Q u P) at the ciphertexts' level");
  }
  const u64 gg = galois_of(c, giant_rotation);
  if (giant_count > 1 && gg != 1) get_key(c, gg);
  const size_t N = c->N, P = (size_t)limbs * N, EP = 2 * (size_t)E * N;
  Scratch s(c);
  u64 *bab = s.get((size_t)B * n * EP);
  std::vector<u64 *> bp((size_t)B * n);
  for (size_t k = 0; k < bp.size(); k++) bp[k] = bab + k * EP;
  ext_babies(c, a, n, baby_rotations, B, bp.data(), s);
  // the MAC of several giant groups runs as one pass over the babies
  const int GC = std::max(1, std::min(kMacGroups, kMaxBatch / B));
  u64 *inner_all = s.get((size_t)std::min(GC, giant_count) * n * EP);
  u64 *inner = s.get((size_t)n * 2 * P);
  for (int i = 0; i < n; i++) out[i] = nullptr;
  int g_lo = giant_count;  // groups [g_lo, g_lo + GC) are in inner_all
  for (int g = giant_count - 1; g >= 0; g--) {
    if (g < g_lo) {
      g_lo = std::max(0, g - GC + 1);
      const int gn = g - g_lo + 1;
      Batch ptb{};
      for (int gi = 0; gi < gn; gi++)
        for (int b = 0; b < B; b++) ptb.p[gi * B + b] = pts[(g_lo + gi) * B + b]->d;
      launch_mac_many(c, bab, n, ptb, B, gn, inner_all, E, limbs);
    }
    u64 *inner_ext = inner_all + (size_t)(g - g_lo) * n * EP;
    const bool first = out[0] == nullptr;
    std::vector<KsJob> jobs(n);
    for (int i = 0; i < n; i++) {
      if (first)
        out[i] = new_ct(c, 2, limbs, 0, a[i]->slots, a[i]->scale * pts[0]->scale,
                        a[i]->scale_degree + pts[0]->scale_degree);
      u64 *dst = first ? out[i]->d : inner + (size_t)i * 2 * P;
      jobs[i] = KsJob{0, nullptr, 1, nullptr, nullptr, dst, dst + P};
    }
    {
      Scratch s2(c);
      ks_moddown(c, limbs, inner_ext, jobs, s2);
    }
    if (first) continue;
    std::vector<ckks_ct *> rot(n);
    for (int i = 0; i < n; i++)
      rot[i] = new_ct(c, 2, limbs, 0, out[i]->slots, out[i]->scale, out[i]->scale_degree);
    if (gg == 1) {
      for (int i = 0; i < n; i++)
        HIPCHECK(hipMemcpyAsync(rot[i]->d, out[i]->d, out[i]->bytes, hipMemcpyDeviceToDevice,
                                c->stream));
    } else {
      std::vector<const ckks_ct *> cur(out, out + n);
      rotate_batch(c, cur.data(), n, gg, rot.data());
    }
    add_batched(c, rot, inner, 2 * P, out, n, limbs);
    for (int i = 0; i < n; i++) free_ct(rot[i]);
  }
}

// ModDown of m single polynomials src[i] ([E][N], NTT form, Q limbs then P
// limbs) into dst[i] ([limbs][N]): the P limbs' inverse NTT, their centred
// conversion to the Q primes, its forward NTT, then (x - conv) P^-1.
static void moddown_polys(ckks_context *c, int limbs, const std::vector<const u64 *> &src,
                          const std::vector<u64 *> &dst, Scratch &s) {
  const size_t N = c->N;
  const int m = (int)src.size();
  const u64 *pinv = pinv_table(c, limbs);
  for (int b0 = 0; b0 < m; b0 += kMaxBatch) {
    const int nb = std::min(kMaxBatch, m - b0);
    Batch sb{}, ob{};
    for (int i = 0; i < nb; i++) {
      sb.p[i] = (u64 *)src[b0 + i];
      ob.p[i] = dst[b0 + i];
    }
    u64 *ptmp = s.get((size_t)nb * c->alpha * N);
    u64 *conv = s.get((size_t)nb * limbs * N);
    const Batch spb = strided(ptmp - (size_t)limbs * N, (size_t)c->alpha * N);
    if (c->ks_tile && convert_h4_ok(c, bc_down(c, limbs))) {
      // N = 2^16: the P limbs' inverse high pass, the conversion and the
      // forward high pass in the tile-resident kernel, then the low pass
      launch_ntt_inv_low(c, sb, spb, nb, limbs, c->alpha, limbs);
      launch_convert_h4(c, strided(ptmp, (size_t)c->alpha * N), strided(conv, (size_t)limbs * N),
                        nb, bc_down(c, limbs), c->L, limbs, 0, limbs, true);
      launch_ntt_fwd_low(c, strided(conv, (size_t)limbs * N), nb, 0, limbs, limbs);
    } else {
      launch_ntt(c, sb, spb, nb, limbs, c->alpha, limbs, true);
      launch_basis_convert(c, strided(ptmp, (size_t)c->alpha * N),
                           strided(conv, (size_t)limbs * N), nb, bc_down(c, limbs), c->L, limbs, 0,
                           limbs, true);
      launch_ntt(c, strided(conv, (size_t)limbs * N), strided(conv, (size_t)limbs * N), nb, 0,
                 limbs, limbs, false);
    }
    launch_moddown_one(c, sb, Strided{conv, (size_t)limbs * N}, ob, nb, limbs, pinv);
  }
}

// hoisted_mac_sum with doubly hoisted giant steps (the reference's
// "ext_double_hoist" strategy, operators/linear/config.py:296-305) for n
// ciphertexts at one level sharing the plaintexts.  The babies and every
// giant group's inner sum u_g = (u0, u1) stay in Q u P; group g >= 1 is
// rotated there by its own key (the rotation by g giant steps): v =
// ModDown(u1) (one polynomial), then (sigma(u0) + KS_0(sigma v), KS_1(sigma v))
// with KS the key product of ModUp(sigma v), before any ModDown; the groups
// are summed in Q u P and one ModDown of the sum ends it.  Against the Horner
// chain of the extended schedule this saves, per giant group, the ModDown of
// u0 and the ModDown of the rotated accumulator.
static void mac_sum_double(ckks_context *c, const ckks_ct *const *a, int n,
                           const int64_t *baby_rotations, int B, const ckks_ct *const *pts,
                           int64_t giant_rotation, int giant_count, ckks_ct **out) {
  require(n >= 1 && n <= kMaxBatch, "ciphertext count must be in [1, 64]");
  require(B >= 1 && B <= kMaxBatch, "baby count must be in [1, 64]");
  require(giant_count >= 1, "giant_count must be positive");
  const int limbs = a[0]->limbs, E = limbs + c->alpha, digits = (limbs + c->ds - 1) / c->ds;
  for (int i = 0; i < n; i++) {
    check_ct(c, a[i], "hoisted_mac_sum_double");
    require(a[i]->polys == 2 && !a[i]->is_ext && a[i]->limbs == limbs,
            "hoisted_mac_sum_double expects degree-1 Q-basis ciphertexts at one level");
  }
  for (int i = 0; i < B * giant_count; i++) {
    check_ct(c, pts[i], "hoisted_mac_sum_double");
    require(pts[i]->polys == 1 && pts[i]->is_ext && pts[i]->limbs == limbs,
            "plaintexts must be extended (Q u P) at the ciphertexts' level");
  }
  // every giant group's own rotation key (the keys must exist before any launch)
  std::vector<u64> gal(giant_count, 1);
  for (int g = 1; g < giant_count; g++) {
    gal[g] = galois_of(c, (int64_t)g * giant_rotation);
    if (gal[g] != 1) get_key(c, gal[g]);
  }
  const size_t N = c->N, P = (size_t)limbs * N, EP = 2 * (size_t)E * N;
  const size_t est = (size_t)digits * E * N;
  Scratch s(c);
  u64 *bab = s.get((size_t)B * n * EP);
  std::vector<u64 *> bp((size_t)B * n);
  for (size_t k = 0; k < bp.size(); k++) bp[k] = bab + k * EP;
  ext_babies(c, a, n, baby_rotations, B, bp.data(), s);
  // inner sums, GC groups per MAC launch, [slot][n][2][E][N]: slot 0 holds
  // group 0's, the running sum; the other groups of a launch go to slots
  // 1..gn (the first launch's to 1..gn-1) and are folded into the sum before
  // the next launch reuses them, so at most GC + 1 groups are held at once
  const int GC = std::max(1, std::min(kMacGroups, kMaxBatch / B));
  u64 *inner = s.get((size_t)std::min(giant_count, GC + 1) * n * EP);
  u64 *total = inner;
  Batch tb{};
  for (int i = 0; i < n; i++) tb.p[i] = total + (size_t)i * EP;
  for (int g0 = 0; g0 < giant_count; g0 += GC) {
    const int gn = std::min(GC, giant_count - g0);
    u64 *dst = g0 == 0 ? inner : inner + (size_t)n * EP;
    Batch ptb{};
    for (int gi = 0; gi < gn; gi++)
      for (int b = 0; b < B; b++) ptb.p[gi * B + b] = pts[(g0 + gi) * B + b]->d;
    launch_mac_many(c, bab, n, ptb, B, gn, dst, E, limbs);
    for (int gi = g0 == 0 ? 1 : 0; gi < gn; gi++) {
      const int g = g0 + gi;
      u64 *ug = dst + (size_t)gi * n * EP;
      Batch ub{};
      for (int i = 0; i < n; i++) ub.p[i] = ug + (size_t)i * EP;
      if (gal[g] == 1) {
        launch_ext_rot_accum(c, ub, Batch{}, tb, 1, n, E, limbs);
        continue;
      }
      Scratch s2(c);
      u64 *v = s2.get((size_t)n * P);
      std::vector<const u64 *> src(n), vp(n);
      std::vector<u64 *> dstp(n);
      for (int i = 0; i < n; i++) {
        src[i] = ug + (size_t)i * EP + (size_t)E * N;  // component 1
        dstp[i] = v + (size_t)i * P;
        vp[i] = dstp[i];
      }
      moddown_polys(c, limbs, src, dstp, s2);
      u64 *ext = s2.get((size_t)n * est);
      ks_modup(c, limbs, n, vp.data(), ext, s2);
      u64 *acc = s2.get((size_t)n * EP);
      launch_key_inner(c, strided(ext, est), strided(acc, EP), n, get_key(c, gal[g]), digits,
                       E, limbs, gal[g], nullptr);
      Batch ab{};
      for (int i = 0; i < n; i++) ab.p[i] = acc + (size_t)i * EP;
      launch_ext_rot_accum(c, ub, ab, tb, gal[g], n, E, limbs);
    }
  }
  std::vector<KsJob> jobs(n);
  for (int i = 0; i < n; i++) out[i] = nullptr;
  for (int i = 0; i < n; i++) {
    out[i] = new_ct(c, 2, limbs, 0, a[i]->slots, a[i]->scale * pts[0]->scale,
                    a[i]->scale_degree + pts[0]->scale_degree);
    jobs[i] = KsJob{0, nullptr, 1, nullptr, nullptr, out[i]->d, out[i]->d + P};
  }
  Scratch s3(c);
  ks_moddown(c, limbs, total, jobs, s3);
}

int ckks_hoisted_mac_sum_double(ckks_context *c, const ckks_ct *a,
                                const int64_t *baby_rotations, int B, const ckks_ct *const *pts,
                                int64_t giant_rotation, int giant_count, ckks_ct **out) {
  API_BEGIN
  require(c && a && baby_rotations && pts && out, "null argument");
  *out = nullptr;
  mac_sum_double(c, &a, 1, baby_rotations, B, pts, giant_rotation, giant_count, out);
  API_END
}

int ckks_hoisted_mac_sum_double_many(ckks_context *c, const ckks_ct *const *a, int n,
                                     const int64_t *baby_rotations, int B,
                                     const ckks_ct *const *pts, int64_t giant_rotation,
                                     int giant_count, ckks_ct **out) {
  API_BEGIN
  require(c && a && baby_rotations && pts && out, "null argument");
  mac_sum_double(c, a, n, baby_rotations, B, pts, giant_rotation, giant_count, out);
  API_END
}

int ckks_hoisted_mac_sum_ext(ckks_context *c, const ckks_ct *a, const int64_t *baby_rotations,
                             int B, const ckks_ct *const *pts, int64_t giant_rotation,
                             int giant_count, ckks_ct **out) {
  API_BEGIN
  require(c && a && baby_rotations && pts && out, "null argument");
  mac_sum_ext(c, &a, 1, baby_rotations, B, pts, giant_rotation, giant_count, out);
  API_END
}

int ckks_hoisted_mac_sum_ext_many(ckks_context *c, const ckks_ct *const *a, int n,
                                  const int64_t *baby_rotations, int B,
                                  const ckks_ct *const *pts, int64_t giant_rotation,
                                  int giant_count, ckks_ct **out) {
  API_BEGIN
  require(c && a && baby_rotations && pts && out, "null argument");
  mac_sum_ext(c, a, n, baby_rotations, B, pts, giant_rotation, giant_count, out);
  API_END
}

int ckks_linear_combination(ckks_context *c, const ckks_ct *const *terms, int T, int n,
                            const double *weights, double constant, int limbs, double scale,
                            int scale_degree, ckks_ct **out) {
  API_BEGIN
  require(c && terms && weights && out, "null argument");
  require(T >= 1 && T <= 256, "term count must be in [1, 256]");
  require(n >= 1 && n <= 256, "ciphertext count must be in [1, 256]");
  check_limbs(c, limbs);
  for (int t = 0; t < T; t++)
    for (int i = 0; i < n; i++) {
      const ckks_ct *x = terms[(size_t)t * n + i];
      check_ct(c, x, "linear_combination");
      require(x->polys == 2 && !x->is_ext && x->limbs >= limbs,
              "terms must be degree-1 Q-basis ciphertexts with at least `limbs` limbs");
    }
  for (int t = 0; t < T; t++)
    require(std::isfinite(weights[t]) && fabs(rint(weights[t])) < ldexp(1.0, 1000),
            "weights must be finite");
  std::vector<u64> table(2 * (size_t)T * n);
  for (size_t j = 0; j < (size_t)T * n; j++) {
    table[2 * j] = (u64)terms[j]->d;
    table[2 * j + 1] = (u64)terms[j]->limbs;
  }
  std::vector<double> w(T);
  for (int t = 0; t < T; t++) w[t] = rint(weights[t]);
  for (int i = 0; i < n; i++) out[i] = nullptr;
  std::vector<u64 *> outp(n);
  for (int i = 0; i < n; i++) {
    out[i] = new_ct(c, 2, limbs, 0, terms[i]->slots, scale, scale_degree);
    outp[i] = out[i]->d;
  }
  Scratch s(c);
  u64 *dtab = s.get(table.size());
  double *dw = (double *)s.get(T);
  u64 *dout = s.get(n);
  u64 *wtab = s.get((size_t)T * limbs);
  u64 *ctab = s.get(limbs);
  upload_async(c, dtab, table.data(), sizeof(u64) * table.size());
  upload_async(c, dw, w.data(), sizeof(double) * T);
  upload_async(c, dout, outp.data(), sizeof(u64) * n);
  launch_lincomb(c, dtab, T, n, dw, rint(constant), (u64 *const *)dout, limbs, wtab, ctab);
  API_END
}

int ckks_rescale_many_by(ckks_context *c, const ckks_ct *const *a, int n, int primes,
                         ckks_ct **out) {
  API_BEGIN
  require(c && a && out, "null argument");
  require(n >= 1, "need at least one ciphertext");
  for (int i = 0; i < n; i++) out[i] = nullptr;
  for (int i = 0; i < n; i++) {
    check_ct(c, a[i], "rescale_many");
    require(!a[i]->is_ext && a[i]->polys >= 1 && a[i]->limbs == a[0]->limbs &&
                a[i]->polys == a[0]->polys,
            "rescale_many expects Q-basis ciphertexts of one shape");
  }
  require(primes >= 1 && primes <= kMaxRescaleDrop, "a rescale divides by 1 to 4 primes");
  require(a[0]->limbs > primes, "rescale needs more limbs than the primes it divides by");
  for (int i = 0; i < n; i++) {
    double scale = a[i]->scale;
    int degree = a[i]->scale_degree;
    for (int j = 0; j < primes; j++) {
      scale /= (double)c->primes[a[i]->limbs - 1 - j];
      degree = degree > 1 ? degree - 1 : 1;
    }
    out[i] = new_ct(c, a[i]->polys, a[i]->limbs - primes, 0, a[i]->slots, scale, degree);
  }
  rescale_batch(c, a, n, out, primes);
  API_END
}

int ckks_rescale_many(ckks_context *c, const ckks_ct *const *a, int n, ckks_ct **out) {
  return ckks_rescale_many_by(c, a, n, 1, out);
}

int ckks_hoisted_rotate_ext(ckks_context *c, const ckks_ct *a, const int64_t *rotations, int n,
                            ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "hoisted_rotate_ext");
  require(rotations && out, "null argument");
  require(n >= 1, "need at least one rotation");
  require(a->polys == 2 && !a->is_ext, "hoisted_rotate_ext expects a degree-1 Q-basis ciphertext");
  for (int r = 0; r < n; r++) out[r] = nullptr;
  std::vector<u64 *> dst(n);
  for (int r = 0; r < n; r++) {
    out[r] = new_ct(c, 2, a->limbs, 1, a->slots, a->scale, a->scale_degree);
    dst[r] = out[r]->d;
  }
  Scratch s(c);
  ext_babies(c, &a, 1, rotations, n, dst.data(), s);
  API_END
}

int ckks_moddown_ext(ckks_context *c, const ckks_ct *a, ckks_ct **out) {
  API_BEGIN
  check_ct(c, a, "moddown_ext");
  require(out, "null argument");
  require(a->polys == 2 && a->is_ext, "moddown_ext expects a degree-1 extended ciphertext");
  const size_t P = (size_t)a->limbs * c->N;
  ckks_ct *o = new_ct(c, 2, a->limbs, 0, a->slots, a->scale, a->scale_degree);
  Scratch s(c);
  std::vector<KsJob> jobs{KsJob{0, nullptr, 1, nullptr, nullptr, o->d, o->d + P}};
  ks_moddown(c, a->limbs, a->d, jobs, s);
  *out = o;
  API_END
}

int ckks_tensor_upload(ckks_context *c, const void *data, size_t bytes, ckks_tensor **out) {
  API_BEGIN
  require(c && data && out, "null argument");
  require(bytes > 0, "empty tensor");
  ckks_tensor *t = new ckks_tensor{c, nullptr, bytes, c->serial};
  try {
    t->d = c->pool.raw_alloc(bytes);
  } catch (...) {
    delete t;
    throw;
  }
  HIPCHECK(hipMemcpyAsync(t->d, data, bytes, hipMemcpyHostToDevice, c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  *out = t;
  API_END
}

int ckks_tensor_download(ckks_context *c, const ckks_tensor *t, void *out, size_t bytes) {
  API_BEGIN
  require(c && t && out, "null argument");
  require(t->ctx == c, "tensor belongs to another context");
  require(bytes <= t->bytes, "download larger than the tensor");
  HIPCHECK(hipMemcpyAsync(out, t->d, bytes, hipMemcpyDeviceToHost, c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  API_END
}

void ckks_tensor_free(ckks_tensor *t) {
  if (!t) return;
  if (owner_alive(t->ctx, t->serial)) {
    (void)hipStreamSynchronize(t->ctx->stream);
    (void)hipFree(t->d);
  }
  delete t;
}

static void check_diag_geom(const ckks_context *c, int D, int lanes, int baby, int giant_base,
                            int giant_count, int slots) {
  require(D > 0 && lanes > 0 && baby > 0 && giant_base >= 0 && giant_count > 0,
          "dimension, token_lanes, baby_steps, giant_count must be positive, giant_base >= 0");
  require((long long)D * lanes == slots,
          "token-lane packing needs dimension * token_lanes == slots");
  check_slots(c, slots);
}

int ckks_encode_token_lane(ckks_context *c, const ckks_tensor *w, int dtype, int D, int lanes,
                           int baby, int giant_base, int giant_count, int slots, int limbs,
                           double scale, int is_ext, ckks_ct **out) {
  API_BEGIN
  require(c && w && out, "null argument");
  require(w->ctx == c, "tensor belongs to another context");
  require(dtype >= 0 && dtype <= 2, "dtype must be 0 (float64), 1 (float32) or 2 (complex128)");
  check_diag_geom(c, D, lanes, baby, giant_base, giant_count, slots);
  check_limbs(c, limbs);
  const size_t elem = dtype == 0 ? 8 : dtype == 1 ? 4 : 16;
  require(w->bytes >= elem * (size_t)D * D, "weight tensor is smaller than dimension^2 entries");
  fft_table(c, slots);
  const int rows = baby * giant_count;
  for (int r = 0; r < rows; r++) out[r] = new_ct(c, 1, limbs, is_ext, slots, scale, 1);
  DiagGeom gm{D, lanes, baby, giant_base};
  launch_encode_diagonals(c, w->d, dtype, nullptr, nullptr, gm, rows, slots, scale, limbs,
                          is_ext, out);
  API_END
}

int ckks_encode_structured(ckks_context *c, const ckks_tensor *const *sources, int n_sources,
                           int fp32, const int64_t *shapes, const int64_t *strides,
                           const int64_t *index_maps, const double *scale_maps, int D,
                           int lanes, int baby, int giant_base, int giant_count, int slots,
                           int limbs, double scale, int is_ext, ckks_ct **out) {
  API_BEGIN
  require(c && sources && shapes && strides && index_maps && scale_maps && out,
          "null argument");
  require(n_sources >= 1 && n_sources <= 3, "one to three sources");
  check_diag_geom(c, D, lanes, baby, giant_base, giant_count, slots);
  check_limbs(c, limbs);
  StructSources src{};
  src.fp32 = fp32 ? 1 : 0;
  const size_t elem = fp32 ? 4 : 8;
  for (int s = 0; s < n_sources; s++) {
    require(sources[s] && sources[s]->ctx == c, "bad source tensor");
    const int64_t rows = shapes[2 * s], cols = shapes[2 * s + 1];
    const int64_t rst = strides[2 * s], cst = strides[2 * s + 1];
    require(rows > 0 && cols > 0 && rst >= 0 && cst >= 0, "bad source shape or strides");
    require((size_t)((rows - 1) * rst + (cols - 1) * cst + 1) * elem <= sources[s]->bytes,
            "source shape and strides exceed the tensor");
    src.p[s] = sources[s]->d;
    src.stride[s][0] = (u64)rst;
    src.stride[s][1] = (u64)cst;
  }
  // every index the gather can read is checked here, on the host
  const int64_t *rsrc = index_maps, *rrow = index_maps + D, *isrc = index_maps + 2 * (size_t)D;
  const int64_t *irow = index_maps + 3 * (size_t)D, *col = index_maps + 4 * (size_t)D;
  for (int i = 0; i < D; i++) {
    for (int part = 0; part < 2; part++) {
      const int64_t sidx = part ? isrc[i] : rsrc[i], r = part ? irow[i] : rrow[i];
      require(sidx >= -1 && sidx < n_sources, "source index out of range");
      if (sidx >= 0) require(r >= 0 && r < shapes[2 * sidx], "row index out of range");
    }
    if (col[i] >= 0)
      for (int s = 0; s < n_sources; s++)
        require(col[i] < shapes[2 * s + 1], "column index out of range");
    require(col[i] >= -1, "column index out of range");
  }
  std::vector<u64> maps(8 * (size_t)D);
  memcpy(maps.data(), index_maps, sizeof(int64_t) * 5 * (size_t)D);
  memcpy(maps.data() + 5 * (size_t)D, scale_maps, sizeof(double) * 3 * (size_t)D);
  fft_table(c, slots);
  const int rows = baby * giant_count;
  for (int r = 0; r < rows; r++) out[r] = new_ct(c, 1, limbs, is_ext, slots, scale, 1);
  Scratch s(c);
  u64 *dmaps = s.get(maps.size());
  upload_async(c, dmaps, maps.data(), sizeof(u64) * maps.size());
  DiagGeom gm{D, lanes, baby, giant_base};
  launch_encode_diagonals(c, nullptr, 0, &src, dmaps, gm, rows, slots, scale, limbs, is_ext, out);
  API_END
}

int ckks_poly_ntt(ckks_context *c, const uint64_t *in, uint64_t *out, int n_polys, int limbs,
                  int q_limbs, int inverse) {
  API_BEGIN
  require(c && in && out, "null argument");
  require(n_polys >= 1 && limbs >= 1 && limbs <= c->K, "bad shape");
  require(q_limbs >= 0 && q_limbs <= c->L && limbs - q_limbs <= c->alpha, "bad q_limbs");
  const size_t words = (size_t)n_polys * limbs * c->N;
  Scratch s(c);
  u64 *d = s.get(words);
  HIPCHECK(hipMemcpyAsync(d, in, sizeof(u64) * words, hipMemcpyHostToDevice, c->stream));
  launch_ntt(c, strided(d, (size_t)limbs * c->N), strided(d, (size_t)limbs * c->N), n_polys, 0,
             limbs, q_limbs, inverse != 0);
  HIPCHECK(hipMemcpyAsync(out, d, sizeof(u64) * words, hipMemcpyDeviceToHost, c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  API_END
}

int ckks_poly_modup(ckks_context *c, const uint64_t *dh, int limbs, uint64_t *ext_h) {
  API_BEGIN
  require(c && dh && ext_h, "null argument");
  check_limbs(c, limbs);
  const size_t N = c->N;
  const int digits = (limbs + c->ds - 1) / c->ds, E = limbs + c->alpha;
  Scratch s(c);
  u64 *d = s.get((size_t)limbs * N);
  u64 *ext = s.get((size_t)digits * E * N);
  HIPCHECK(hipMemcpyAsync(d, dh, sizeof(u64) * limbs * N, hipMemcpyHostToDevice, c->stream));
  const u64 *dp = d;
  ks_modup(c, limbs, 1, &dp, ext, s);
  HIPCHECK(hipMemcpyAsync(ext_h, ext, sizeof(u64) * digits * E * N, hipMemcpyDeviceToHost,
                          c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  API_END
}

int ckks_poly_moddown(ckks_context *c, const uint64_t *acc_h, int limbs, uint64_t *out_h) {
  API_BEGIN
  require(c && acc_h && out_h, "null argument");
  check_limbs(c, limbs);
  const size_t N = c->N;
  const int E = limbs + c->alpha;
  Scratch s(c);
  // run ModDown through the combine path with component 1 = component 0
  u64 *acc = s.get(2 * (size_t)E * N);
  u64 *ptmp = s.get(2 * (size_t)c->alpha * N);
  u64 *conv = s.get(2 * (size_t)limbs * N);
  u64 *o = s.get(2 * (size_t)limbs * N);
  HIPCHECK(hipMemcpyAsync(acc, acc_h, sizeof(u64) * E * N, hipMemcpyHostToDevice, c->stream));
  HIPCHECK(hipMemcpyAsync(acc + (size_t)E * N, acc_h, sizeof(u64) * E * N, hipMemcpyHostToDevice,
                          c->stream));
  launch_ntt(c, strided(acc, E * N), strided(ptmp - (size_t)limbs * N, (size_t)c->alpha * N), 2,
             limbs, c->alpha, limbs, true);
  launch_basis_convert(c, strided(ptmp, (size_t)c->alpha * N), strided(conv, (size_t)limbs * N), 2,
                       bc_down(c, limbs), c->L, limbs, 0, limbs, true);
  launch_ntt(c, strided(conv, (size_t)limbs * N), strided(conv, (size_t)limbs * N), 2, 0, limbs,
             limbs, false);
  Batch a0{}, a1{}, o0{}, o1{};
  o0.p[0] = o;
  o1.p[0] = o + (size_t)limbs * N;
  u64 g = 1;
  launch_moddown_combine(c, Strided{acc, 2 * (u64)E * N}, Strided{conv, 2 * (u64)limbs * N}, a0,
                         a1, &g, o0, o1, 1, limbs, E, pinv_table(c, limbs));
  HIPCHECK(hipMemcpyAsync(out_h, o, sizeof(u64) * limbs * N, hipMemcpyDeviceToHost, c->stream));
  HIPCHECK(hipStreamSynchronize(c->stream));
  API_END
}

int ckks_ntt_many(ckks_context *c, ckks_ct *const *cts, int n, int inverse) {
  API_BEGIN
  require(c && cts && n >= 1, "null argument");
  for (int b0 = 0; b0 < n; b0 += kMaxBatch) {
    const int nb = std::min(kMaxBatch, n - b0);
    const int limbs = cts[b0]->limbs, polys = cts[b0]->polys;
    Batch b{};
    for (int i = 0; i < nb; i++) {
      check_poly(c, cts[b0 + i], "ntt_many");
      require(cts[b0 + i]->limbs == limbs && cts[b0 + i]->polys == polys && !cts[b0 + i]->is_ext,
              "ntt_many needs one shape");
      b.p[i] = cts[b0 + i]->d;
    }
    // polys x limbs limb-polynomials per ciphertext: limb index runs over
    // [0, polys * limbs) and maps to prime (index mod limbs).
    for (int p = 0; p < polys; p++) {
      Batch bp{};
      for (int i = 0; i < nb; i++) bp.p[i] = b.p[i] + (size_t)p * limbs * c->N;
      launch_ntt(c, bp, bp, nb, 0, limbs, limbs, inverse != 0);
    }
  }
  API_END
}

int ckks_int_peak(ckks_context *c, int kind, double *ops_per_second) {
  API_BEGIN
  require(c && ops_per_second, "null argument");
  require(kind >= 0 && kind <= 2, "kind must be 0 (fp64 modular product), 1 (64-bit Shoup) or 2 (fp64 FMA)");
  const int blocks = 4096, iters = 2048;
  Scratch s(c);
  double *out = (double *)s.get((size_t)blocks * 256);
  launch_int_peak(c, kind, out, blocks, iters / 8);  // warm-up
  *ops_per_second = launch_int_peak(c, kind, out, blocks, iters);
  API_END
}

int ckks_profile_enable(ckks_context *c, int enable) {
  API_BEGIN
  require(c, "null argument");
  c->prof = enable != 0;
  API_END
}

int ckks_profile_read(ckks_context *c, char *buf, size_t len) {
  API_BEGIN
  require(c && buf && len > 0, "null argument");
  HIPCHECK(hipStreamSynchronize(c->stream));
  struct Sum {
    long calls = 0;
    double ms = 0, bytes = 0, ops = 0;
  };
  std::map<std::string, Sum> sums;
  for (auto &r : c->prof_recs) {
    float ms = 0;
    HIPCHECK(hipEventElapsedTime(&ms, r.a, r.b));
    Sum &s = sums[r.name];
    s.calls++;
    s.ms += ms;
    s.bytes += r.bytes;
    s.ops += r.ops;
    c->prof_pool.push_back(r.a);
    c->prof_pool.push_back(r.b);
  }
  c->prof_recs.clear();
  std::string text;
  for (auto &kv : sums) {
    char line[256];
    snprintf(line, sizeof line, "%s %ld %.6f %.6e %.6e\n", kv.first.c_str(), kv.second.calls,
             kv.second.ms, kv.second.bytes, kv.second.ops);
    text += line;
  }
  const size_t n = std::min(len - 1, text.size());
  memcpy(buf, text.data(), n);
  buf[n] = 0;
  API_END
}

int ckks_set_split_parts(ckks_context *c, int parts) {
  API_BEGIN
  require(c, "null argument");
  require(parts >= 0 && parts <= c->split_streams,
          "split parts must be 0 .. the count the context was created with");
  c->split_parts = parts ? parts : c->split_streams;
  API_END
}

int ckks_audit_read(ckks_context *c, double *out, int reset) {
  API_BEGIN
  require(c && out, "null argument");
  for (int i = 0; i < 5; i++) out[i] = c->audit[i];
  if (reset)
    for (int i = 0; i < 5; i++) c->audit[i] = 0.0;
  API_END
}

int ckks_context_stream(ckks_context *c, void **stream) {
  API_BEGIN
  require(c && stream, "null argument");
  *stream = (void *)c->stream;
  API_END
}

int ckks_event_create(ckks_context *c, ckks_event **out) {
  API_BEGIN
  require(c && out, "null argument");
  ckks_event *e = new ckks_event();
  e->ctx = c;
  HIPCHECK(hipEventCreate(&e->ev));
  *out = e;
  API_END
}

int ckks_event_record(ckks_event *e) {
  API_BEGIN
  require(e, "null argument");
  HIPCHECK(hipEventRecord(e->ev, e->ctx->stream));
  API_END
}

int ckks_event_elapsed_ms(ckks_event *a, ckks_event *b, float *ms) {
  API_BEGIN
  require(a && b && ms, "null argument");
  HIPCHECK(hipEventSynchronize(b->ev));
  HIPCHECK(hipEventElapsedTime(ms, a->ev, b->ev));
  API_END
}

void ckks_event_destroy(ckks_event *e) {
  if (!e) return;
  (void)hipEventDestroy(e->ev);
  delete e;
}

}  // extern "C"
