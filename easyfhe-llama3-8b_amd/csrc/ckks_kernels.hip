// ckks_kernels.hip -- gfx950 kernels of the RNS-CKKS backend.
//
// All kernels use 256-thread workgroups (four wave64s).  Polynomials are
// uint64 limb arrays of N residues; the NTT domain is the bit-reversed
// evaluation order a_hat[i] = a(psi^(2 br(i) + 1)).
#include <math.h>
#include <type_traits>

#include "ckks_internal.hpp"

namespace ckks {

#define HIP_OK(x)                                                          \
  do {                                                                     \
    hipError_t e_ = (x);                                                   \
    if (e_ != hipSuccess)                                                  \
      throw std::runtime_error(std::string(#x ": ") + hipGetErrorString(e_)); \
  } while (0)

#define LAUNCH_CHECK()                                                     \
  do {                                                                     \
    hipError_t e_ = hipGetLastError();                                     \
    if (e_ != hipSuccess)                                                  \
      throw std::runtime_error(std::string("kernel launch: ") +            \
                               hipGetErrorString(e_));                     \
  } while (0)

constexpr int TPB = 256;

// ===========================================================================
// NTT: two passes of LDS-staged radix-2 stages.
//   high pass: bit positions [logN - S1, logN), a tile is 2^S1 rows (stride
//              N / 2^S1) by C adjacent columns, so global loads stay
//              coalesced in C-element runs;
//   low pass:  bit positions [0, S2), a tile is R contiguous rows of 2^S2.
// Forward: high then low (Cooley-Tukey, twiddle psi_br[(N + j) >> (b + 1)]).
// Inverse: low then high (Gentleman-Sande with psi_br^-1), then x N^-1.
// ===========================================================================

template <int S, int TILE>
__global__ __launch_bounds__(TPB) void k_ntt_fwd_high(Batch src, Batch dst, int logN,
                                                      int l_begin, int q_limbs, int L,
                                                      const ModQ *__restrict__ mods,
                                                      const u64 *__restrict__ psi,
                                                      const u64 *__restrict__ psi_sh) {
  constexpr int ROWS = 1 << S;
  constexpr int C = TILE / ROWS;
  constexpr int PER = TILE / TPB;
  __shared__ u64 s[TILE];
  const int N = 1 << logN;
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const u64 q = mods[p].q;
  const u64 *W = psi + (size_t)p * N;
  const u64 *Ws = psi_sh + (size_t)p * N;
  const u64 *in = batch_ptr(src, blockIdx.y) + (size_t)limb * N;
  u64 *out = batch_ptr(dst, blockIdx.y) + (size_t)limb * N;
  const int stride = N >> S;
  const int col0 = blockIdx.x * C;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e = threadIdx.x + TPB * k;
    s[e] = in[(size_t)(e / C) * stride + col0 + (e % C)];
  }
  __syncthreads();
#pragma unroll
  for (int st = 0; st < S; st++) {
    const int h = ROWS >> (st + 1);
#pragma unroll
    for (int k = 0; k < PER / 2; k++) {
      int u = threadIdx.x + TPB * k;
      int cc = u % C, v = u / C;
      int group = v / h, pos = v % h;
      int ia = (group * 2 * h + pos) * C + cc, ib = ia + h * C;
      int ti = (1 << st) + group;
      u64 a = s[ia];
      u64 t = shoup_mul(s[ib], W[ti], Ws[ti], q);
      s[ia] = add_mod(a, t, q);
      s[ib] = sub_mod(a, t, q);
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e = threadIdx.x + TPB * k;
    out[(size_t)(e / C) * stride + col0 + (e % C)] = s[e];
  }
}

template <int S, int TILE>
__global__ __launch_bounds__(TPB) void k_ntt_fwd_low(Batch dst, int logN, int l_begin,
                                                     int q_limbs, int L,
                                                     const ModQ *__restrict__ mods,
                                                     const u64 *__restrict__ psi,
                                                     const u64 *__restrict__ psi_sh) {
  constexpr int COLS = 1 << S;
  constexpr int PER = TILE / TPB;
  __shared__ u64 s[TILE];
  const int N = 1 << logN;
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const u64 q = mods[p].q;
  const u64 *W = psi + (size_t)p * N;
  const u64 *Ws = psi_sh + (size_t)p * N;
  u64 *base = batch_ptr(dst, blockIdx.y) + (size_t)limb * N + (size_t)blockIdx.x * TILE;
#pragma unroll
  for (int k = 0; k < PER; k++) s[threadIdx.x + TPB * k] = base[threadIdx.x + TPB * k];
  __syncthreads();
#pragma unroll
  for (int st = 0; st < S; st++) {
    const int b = S - 1 - st, h = 1 << b;
#pragma unroll
    for (int k = 0; k < PER / 2; k++) {
      int u = threadIdx.x + TPB * k;
      int r = u / (COLS / 2), v = u % (COLS / 2);
      int ca = r * COLS + ((v >> b) << (b + 1)) + (v & (h - 1));
      int j = blockIdx.x * TILE + ca;
      int ti = (N + j) >> (b + 1);
      u64 a = s[ca];
      u64 t = shoup_mul(s[ca + h], W[ti], Ws[ti], q);
      s[ca] = add_mod(a, t, q);
      s[ca + h] = sub_mod(a, t, q);
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < PER; k++) base[threadIdx.x + TPB * k] = s[threadIdx.x + TPB * k];
}

template <int S, int TILE>
__global__ __launch_bounds__(TPB) void k_ntt_inv_low(Batch src, Batch dst, int logN,
                                                     int l_begin, int q_limbs, int L,
                                                     const ModQ *__restrict__ mods,
                                                     const u64 *__restrict__ ipsi,
                                                     const u64 *__restrict__ ipsi_sh) {
  constexpr int COLS = 1 << S;
  constexpr int PER = TILE / TPB;
  __shared__ u64 s[TILE];
  const int N = 1 << logN;
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const u64 q = mods[p].q;
  const u64 *W = ipsi + (size_t)p * N;
  const u64 *Ws = ipsi_sh + (size_t)p * N;
  const u64 *in = batch_ptr(src, blockIdx.y) + (size_t)limb * N + (size_t)blockIdx.x * TILE;
  u64 *out = batch_ptr(dst, blockIdx.y) + (size_t)limb * N + (size_t)blockIdx.x * TILE;
#pragma unroll
  for (int k = 0; k < PER; k++) s[threadIdx.x + TPB * k] = in[threadIdx.x + TPB * k];
  __syncthreads();
#pragma unroll
  for (int b = 0; b < S; b++) {
    const int h = 1 << b;
#pragma unroll
    for (int k = 0; k < PER / 2; k++) {
      int u = threadIdx.x + TPB * k;
      int r = u / (COLS / 2), v = u % (COLS / 2);
      int ca = r * COLS + ((v >> b) << (b + 1)) + (v & (h - 1));
      int j = blockIdx.x * TILE + ca;
      int ti = (N + j) >> (b + 1);
      u64 x = s[ca], y = s[ca + h];
      s[ca] = add_mod(x, y, q);
      s[ca + h] = shoup_mul(sub_mod(x, y, q), W[ti], Ws[ti], q);
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < PER; k++) out[threadIdx.x + TPB * k] = s[threadIdx.x + TPB * k];
}

template <int S, int TILE>
__global__ __launch_bounds__(TPB) void k_ntt_inv_high(Batch dst, int logN, int l_begin,
                                                      int q_limbs, int L,
                                                      const ModQ *__restrict__ mods,
                                                      const u64 *__restrict__ ipsi,
                                                      const u64 *__restrict__ ipsi_sh,
                                                      const u64 *__restrict__ ninv) {
  constexpr int ROWS = 1 << S;
  constexpr int C = TILE / ROWS;
  constexpr int PER = TILE / TPB;
  __shared__ u64 s[TILE];
  const int N = 1 << logN;
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const u64 q = mods[p].q;
  const u64 *W = ipsi + (size_t)p * N;
  const u64 *Ws = ipsi_sh + (size_t)p * N;
  u64 *io = batch_ptr(dst, blockIdx.y) + (size_t)limb * N;
  const int stride = N >> S;
  const int col0 = blockIdx.x * C;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e = threadIdx.x + TPB * k;
    s[e] = io[(size_t)(e / C) * stride + col0 + (e % C)];
  }
  __syncthreads();
#pragma unroll
  for (int st = S - 1; st >= 0; st--) {
    const int h = ROWS >> (st + 1);
#pragma unroll
    for (int k = 0; k < PER / 2; k++) {
      int u = threadIdx.x + TPB * k;
      int cc = u % C, v = u / C;
      int group = v / h, pos = v % h;
      int ia = (group * 2 * h + pos) * C + cc, ib = ia + h * C;
      int ti = (1 << st) + group;
      u64 x = s[ia], y = s[ib];
      s[ia] = add_mod(x, y, q);
      s[ib] = shoup_mul(sub_mod(x, y, q), W[ti], Ws[ti], q);
    }
    __syncthreads();
  }
  const u64 ni = ninv[2 * p], nis = ninv[2 * p + 1];
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e = threadIdx.x + TPB * k;
    io[(size_t)(e / C) * stride + col0 + (e % C)] = shoup_mul(s[e], ni, nis, q);
  }
}

// ===========================================================================
// N = 2^16 as a 16 x 4096 array (position j = 4096 r + c): two passes of
// register-resident radix-16 rounds (4 stages each in 16 registers per
// thread).
//   high pass, bit positions 15..12: one 16-point transform per column c,
//     held by one thread (words c + 4096 k), no exchange; every stage's
//     twiddle is the same for all columns;
//   low pass, bit positions 11..0: one 4096-word row (tile) per block: round
//     Z on bits 11..8 (thread t holds words t + 256 k, read and written
//     coalesced), then rounds A (7..4) and B (3..0) on the tile as 16 rows
//     of 256 through the padded LDS tile.
// Forward: high then low (Cooley-Tukey, twiddle psi_br[(N + j) >> (b + 1)]
// for bit b and position j); inverse: low then high (Gentleman-Sande with
// psi_br^-1), then x N^-1.  Butterflies are Harvey's lazy ones (forward
// values in [0, 4q), inverse values in [0, 2q)); only the last pass reduces
// to [0, q), so pass-to-pass data in HBM may be lazy.
// LDS layout: element (r, c) of a 16 x 256 tile at r * 272 + c + (c >> 4):
// the +1 per 16 keeps 16-apart columns in distinct banks.
// ===========================================================================

__device__ __forceinline__ u64 shoup_lazy(u64 a, u64 w, u64 ws, u64 q) {
  return a * w - __umul64hi(a, ws) * q;  // in [0, 2q) for any a < 2^64
}

// Cooley-Tukey: X, Y in [0, 4q) -> X + wY, X - wY in [0, 4q)
__device__ __forceinline__ void ct_bfly(u64 &X, u64 &Y, u64 w, u64 ws, u64 q, u64 q2) {
  const u64 x = csub(X, q2);
  const u64 t = shoup_lazy(Y, w, ws, q);
  X = x + t;
  Y = x - t + q2;
}

// Gentleman-Sande: X, Y in [0, 2q) -> X + Y, (X - Y) w in [0, 2q)
__device__ __forceinline__ void gs_bfly(u64 &X, u64 &Y, u64 w, u64 ws, u64 q, u64 q2) {
  u64 sum = X + Y;
  sum = csub(sum, q2);
  const u64 d = X - Y + q2;
  X = sum;
  Y = shoup_lazy(d, w, ws, q);
}

__device__ __forceinline__ int lds16(int r, int c) { return r * 272 + c + (c >> 4); }

// The 16 threads of tile row rl (threads 16 rl .. 16 rl + 15) belong to one
// wave, and the LDS serves one wave's instructions in order: an exchange
// within rows needs only that the compiler keeps the wave's LDS accesses on
// their side of this point, not a workgroup barrier.
__device__ __forceinline__ void row_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// row_sync when every thread's accesses on both sides stay in its row, a
// workgroup barrier otherwise (rows: wave-uniform)
__device__ __forceinline__ void tile_sync(bool rows) {
  if (rows) row_sync();
  else __syncthreads();
}

// ModDown epilogue of the forward low pass (conv items 2 i + c):
// out_c[l][k] = (acc_c[l][k] - NTT(conv_c)[l][k]) P^-1 + add_c[l][sigma(k)]
struct Galois64 {
  u64 g[kMaxBatch];
};

struct MDCombine {
  Batch acc;        // per item: [2][E][N] (component c, limb l at (c E + l) N)
  int E;
  const u64 *pinv;  // per Q limb: P^-1, shoup
  const u64 *amul;  // per Q limb: multiplier of the addend, shoup (null: 1)
  Batch add;        // per item: component-0 addend (or null)
  u64 add1_off;     // component-1 addend at add + add1_off (0: none)
  Batch out;        // per item: component-0 output
  u64 out1_off;     // component-1 output at out + out1_off
  Galois64 gal;
  PostOp post;      // postop of the relinearise-rescale step (zero: none)
};

// (dbl ? 2 r : r) - sub + scal of the postop, at word (limb, e) of an output
// component (PostOp)
__device__ __forceinline__ u64 apply_post(const PostOp &po, int item, int comp, int limb, u32 e,
                                          size_t N, u64 r, u64 q) {
  if (po.dbl) r = add_mod(r, r, q);
  const u64 *sb = batch_ptr(po.sub, item);
  if (sb) r = sub_mod(r, sb[(comp ? po.sub1_off : 0) + (size_t)limb * N + e], q);
  if (po.scal && !comp) r = add_mod(r, po.scal[limb], q);
  return r;
}

// Operands of the epilogue for the 16 outputs e(k) = tile + rl 256 + c0 + 16 k
// of one thread, loaded at kernel entry so that their latency overlaps the
// butterflies: acc - is kept, add (or 0) is summed in; the limb's constants
// (P^-1, the addend's multiplier, the postop's scalar) are read here too, so
// that the stores issue no loads but the postop's subtrahends (md_sub_load).
struct MDPrefetch {
  u64 a[16], d[16];
  u64 pinv, pinvs, am, ams, sc;
};

__device__ __forceinline__ void md_load(const MDCombine &md, int item2, int limb, u32 e0,
                                        MDPrefetch &pf) {
  const int item = item2 >> 1, comp = item2 & 1;
  const size_t N = 65536;
  const u64 *acc = batch_ptr(md.acc, item) + ((size_t)comp * md.E + limb) * N;
  const u64 *ad = batch_ptr(md.add, item);
  if (comp) ad = (ad && md.add1_off) ? ad + md.add1_off : nullptr;
  const u64 g = md.gal.g[item];
  pf.pinv = md.pinv[2 * limb];
  pf.pinvs = md.pinv[2 * limb + 1];
  pf.am = md.amul ? md.amul[2 * limb] : 0;
  pf.ams = md.amul ? md.amul[2 * limb + 1] : 0;
  pf.sc = md.post.scal && !comp ? md.post.scal[limb] : 0;
#pragma unroll
  for (int k = 0; k < 16; k++) pf.a[k] = acc[e0 + 16 * k];
#pragma unroll
  for (int k = 0; k < 16; k++) {
    const u32 e = e0 + 16 * k;
    pf.d[k] = ad ? ad[(size_t)limb * N + (g == 1 ? e : autom_index(e, g, 16))] : 0;
  }
}

// The postop's subtrahend words of the 16 outputs (all 0 without one), read
// together before the stores.
__device__ __forceinline__ void md_sub_load(const MDCombine &md, int item2, int limb, u32 e0,
                                            u64 (&sv)[16]) {
  const int item = item2 >> 1, comp = item2 & 1;
  const u64 *sb = batch_ptr(md.post.sub, item);
  if (sb) {
    sb += (comp ? md.post.sub1_off : 0) + ((size_t)limb << 16);
#pragma unroll
    for (int k = 0; k < 16; k++) sv[k] = sb[e0 + 16 * k];
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) sv[k] = 0;
  }
}

// (dbl ? 2 r : r) - s + sc with r = (a - y) P^-1 + d amul (apply_post's terms)
__device__ __forceinline__ void md_store(const MDCombine &md, int item2, int limb, u32 e, u64 y,
                                         const MDPrefetch &pf, u64 a, u64 d, u64 s, u64 q) {
  const int item = item2 >> 1, comp = item2 & 1;
  const size_t N = 65536;
  u64 r = shoup_mul(sub_mod(a, y, q), pf.pinv, pf.pinvs, q);
  if (md.amul) d = shoup_mul(d, pf.am, pf.ams, q);
  r = add_mod(r, d, q);
  if (md.post.dbl) r = add_mod(r, r, q);
  r = sub_mod(r, s, q);
  if (pf.sc) r = add_mod(r, pf.sc, q);
  u64 *o = batch_ptr(md.out, item) + (comp ? md.out1_off : 0);
  o[(size_t)limb * N + e] = r;
}

// High pass, 64-bit body: x[k] = word c + 4096 k of one column, stages on
// bits 15..12 (k bits 3..0); the twiddle of stage st and pair k is
// psi_br[2^st + (k >> (4 - st))], the same for every column.
__device__ __forceinline__ void u64_high_fwd(u64 (&x)[16], const u64 *__restrict__ W,
                                             const u64 *__restrict__ Ws, u64 q, u64 q2) {
#pragma unroll
  for (int st = 0; st < 4; st++) {
    const int half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const int ti = (1 << st) + (k >> (4 - st));
      ct_bfly(x[k], x[k + half], W[ti], Ws[ti], q, q2);
    }
  }
}

// inverse high pass on one column (lazy input, lazy output in [0, 2q))
__device__ __forceinline__ void u64_high_inv_stages(u64 (&x)[16], const u64 *__restrict__ W,
                                                    const u64 *__restrict__ Ws, u64 q, u64 q2) {
#pragma unroll
  for (int st = 3; st >= 0; st--) {
    const int half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const int ti = (1 << st) + (k >> (4 - st));
      gs_bfly(x[k], x[k + half], W[ti], Ws[ti], q, q2);
    }
  }
}

// the inverse high pass, then x N^-1 to [0, q)
__device__ __forceinline__ void u64_high_inv(u64 (&x)[16], const u64 *__restrict__ W,
                                             const u64 *__restrict__ Ws, u64 ni, u64 nis,
                                             u64 q, u64 q2) {
  u64_high_inv_stages(x, W, Ws, q, q2);
#pragma unroll
  for (int k = 0; k < 16; k++) {
    const u64 v = shoup_lazy(x[k], ni, nis, q);
    x[k] = csub(v, q);
  }
}

// Round Z of the forward low pass: x[k] = word t + 256 k of tile `tile`
// (position j = 4096 tile + 256 k + t), stages on bits 11..8 (k bits 3..0);
// twiddle index (N >> (b + 1)) + (j >> (b + 1)) does not depend on t.
__device__ __forceinline__ void u64_low_round_z(u64 (&x)[16], const u64 *__restrict__ W,
                                                const u64 *__restrict__ Ws, int tile, u64 q,
                                                u64 q2) {
#pragma unroll
  for (int st = 0; st < 4; st++) {
    const int b = 11 - st, half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const int ti = (65536 >> (b + 1)) + ((tile * 4096 + 256 * k) >> (b + 1));
      ct_bfly(x[k], x[k + half], W[ti], Ws[ti], q, q2);
    }
  }
}

// inverse round Z: stages on bits 8..11, same positions as round Z
__device__ __forceinline__ void u64_inv_round_z(u64 (&x)[16], const u64 *__restrict__ W,
                                                const u64 *__restrict__ Ws, int tile, u64 q,
                                                u64 q2) {
#pragma unroll
  for (int b = 8; b < 12; b++) {
    const int half = 1 << (b - 8);
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const int ti = (65536 >> (b + 1)) + ((tile * 4096 + 256 * k) >> (b + 1));
      gs_bfly(x[k], x[k + half], W[ti], Ws[ti], q, q2);
    }
  }
}

// Rounds of the forward low pass on one thread's 16 words of global row
// `row` (of 256): A on columns c0 + 16 k (bits 7..4), B on columns 16 c0 + j
// (bits 3..0); values in [0, 4q)
__device__ __forceinline__ void u64_low_round_a(u64 (&x)[16], const u64 *__restrict__ W,
                                                const u64 *__restrict__ Ws, int row, u64 q,
                                                u64 q2) {
#pragma unroll
  for (int st = 0; st < 4; st++) {
    const int b = 7 - st, half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const int ti = (65536 >> (b + 1)) + ((row * 256 + 16 * k) >> (b + 1));
      ct_bfly(x[k], x[k + half], W[ti], Ws[ti], q, q2);
    }
  }
}

__device__ __forceinline__ void u64_low_round_b(u64 (&x)[16], const u64 *__restrict__ W,
                                                const u64 *__restrict__ Ws, int row, int c0, u64 q,
                                                u64 q2) {
#pragma unroll
  for (int st = 4; st < 8; st++) {
    const int b = 7 - st, half = 1 << b;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      if (j & half) continue;
      const int ti = (65536 >> (b + 1)) + ((row * 256 + 16 * c0 + j) >> (b + 1));
      ct_bfly(x[j], x[j + half], W[ti], Ws[ti], q, q2);
    }
  }
}

// Round Z of tile `tile` from src (words t + 256 k), its result into the LDS
// tile for round A (word 256 k + t at lds16(k, t)).  The caller synchronises
// before (earlier reads of sm) and after.
__device__ __forceinline__ void u64_round_z_to_lds(u64 *__restrict__ sm,
                                                   const u64 *__restrict__ src,
                                                   const u64 *__restrict__ W,
                                                   const u64 *__restrict__ Ws, int tile, u64 q,
                                                   u64 q2) {
  const int t = threadIdx.x;
  u64 x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = src[t + 256 * k];
  u64_low_round_z(x, W, Ws, tile, q, q2);
#pragma unroll
  for (int k = 0; k < 16; k++) sm[lds16(k, t)] = x[k];
}

// forward, bit positions 11..0: one 4096-word tile per block; output in
// [0, q) (COMBINE: the ModDown epilogue instead of the store)
template <bool COMBINE>
__device__ __forceinline__ void k_ntt16_fwd_low_body(u64 *__restrict__ lds, Batch dst, int l_begin, int q_limbs,
                                                       int L, const ModQ *__restrict__ mods,
                                                       const u64 *__restrict__ psi,
                                                       const u64 *__restrict__ psi_sh,
                                                       MDCombine md) {
  u64 *sm = lds;
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const u64 q = mods[p].q, q2 = 2 * q;
  const u64 *W = psi + ((size_t)p << 16);
  const u64 *Ws = psi_sh + ((size_t)p << 16);
  u64 *base = batch_ptr(dst, blockIdx.y) + ((size_t)limb << 16) + (size_t)blockIdx.x * 4096;
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int row = blockIdx.x * 16 + rl;  // global row of 256
  MDPrefetch pf;
  if constexpr (COMBINE) md_load(md, blockIdx.y, limb, blockIdx.x * 4096 + rl * 256 + c0, pf);
  u64_round_z_to_lds(sm, base, W, Ws, blockIdx.x, q, q2);
  __syncthreads();
  u64 x[16];
  // round A: column = c0 + 16 k, stages on column bits 7..4; the thread
  // writes back the slots it read, which no other thread reads
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = sm[lds16(rl, c0 + 16 * k)];
  u64_low_round_a(x, W, Ws, row, q, q2);
#pragma unroll
  for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = x[k];
  row_sync();
  // round B: column = 16 c0 + j, stages on column bits 3..0
#pragma unroll
  for (int j = 0; j < 16; j++) x[j] = sm[lds16(rl, 16 * c0 + j)];
  u64_low_round_b(x, W, Ws, row, c0, q, q2);
  // store through LDS so that adjacent lanes write adjacent words
  row_sync();
#pragma unroll
  for (int j = 0; j < 16; j++) {
    sm[lds16(rl, 16 * c0 + j)] = csub(csub(x[j], q2), q);
  }
  row_sync();
  if constexpr (COMBINE) {
    const u32 e0 = blockIdx.x * 4096 + rl * 256 + c0;
    u64 sv[16];
    md_sub_load(md, blockIdx.y, limb, e0, sv);
#pragma unroll
    for (int k = 0; k < 16; k++)
      md_store(md, blockIdx.y, limb, e0 + 16 * k, sm[lds16(rl, c0 + 16 * k)], pf, pf.a[k],
               pf.d[k], sv[k], q);
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) base[rl * 256 + c0 + 16 * k] = sm[lds16(rl, c0 + 16 * k)];
  }
}

// inverse, bit positions 0..11 (first pass): input in [0, 2q), output lazy
__device__ __forceinline__ void k_ntt16_inv_low_body(u64 *__restrict__ lds, Batch src, Batch dst, int l_begin,
                                                       int q_limbs, int L,
                                                       const ModQ *__restrict__ mods,
                                                       const u64 *__restrict__ ipsi,
                                                       const u64 *__restrict__ ipsi_sh,
                                                       const Batch &mul, int mm) {
  u64 *sm = lds;
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const u64 q = mods[p].q, q2 = 2 * q;
  const u64 *W = ipsi + ((size_t)p << 16);
  const u64 *Ws = ipsi_sh + ((size_t)p << 16);
  const u64 *in = batch_ptr(src, blockIdx.y) + ((size_t)limb << 16) + (size_t)blockIdx.x * 4096;
  u64 *out = batch_ptr(dst, blockIdx.y) + ((size_t)limb << 16) + (size_t)blockIdx.x * 4096;
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int row = blockIdx.x * 16 + rl;
  u64 x[16];
  // round B^-1: column = 16 c0 + j, stages on column bits 0..3; the load
  // goes through LDS so that adjacent lanes read adjacent words (with mm,
  // of the product src x mul or src^2, formed here)
  if (mm) {
    const ModQ M = mods[p];
    const u64 *mb = mm == 2 ? in
                            : batch_ptr(mul, blockIdx.y) + ((size_t)limb << 16) +
                                  (size_t)blockIdx.x * 4096;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int e = rl * 256 + c0 + 16 * k;
      const u64 v = in[e];
      sm[lds16(rl, c0 + 16 * k)] = mul_mod(v, mm == 2 ? v : mb[e], M);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = in[rl * 256 + c0 + 16 * k];
  }
  row_sync();
#pragma unroll
  for (int j = 0; j < 16; j++) x[j] = sm[lds16(rl, 16 * c0 + j)];
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const int half = 1 << b;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      if (j & half) continue;
      const int ti = (65536 >> (b + 1)) + ((row * 256 + 16 * c0 + j) >> (b + 1));
      gs_bfly(x[j], x[j + half], W[ti], Ws[ti], q, q2);
    }
  }
  row_sync();
#pragma unroll
  for (int j = 0; j < 16; j++) sm[lds16(rl, 16 * c0 + j)] = x[j];
  row_sync();
  // round A^-1: column = c0 + 16 k, stages on column bits 4..7
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = sm[lds16(rl, c0 + 16 * k)];
#pragma unroll
  for (int b = 4; b < 8; b++) {
    const int half = 1 << (b - 4);
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const int ti = (65536 >> (b + 1)) + ((row * 256 + 16 * k) >> (b + 1));
      gs_bfly(x[k], x[k + half], W[ti], Ws[ti], q, q2);
    }
  }
  // round Z^-1 (bits 8..11) on words t + 256 k: the thread's slots go back
  // (no other thread reads them), then each thread takes one tile column
#pragma unroll
  for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = x[k];
  __syncthreads();
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = sm[lds16(k, t)];
  u64_inv_round_z(x, W, Ws, blockIdx.x, q, q2);
#pragma unroll
  for (int k = 0; k < 16; k++) out[t + 256 * k] = x[k];
}

// ---------------------------------------------------------------------------
// fp64 variant for primes q < 2^45: residues travel as signed doubles (exact
// integers) and every modular product is
//   hi = a w, lo = fma(a, w, -hi)             (a w = hi + lo exactly)
//   t  = round(a (w / q)), r = fma(-t, q, hi) + lo   in [-q, q], exact
// which needs |a| < 2^50; forward butterflies then need no reduction over
// all 16 stages (|x| <= 17 q < 2^50), inverse ones reduce every 4 stages.
// Between the two passes the data is stored as raw double bits.
// ---------------------------------------------------------------------------

#define FP_ROUND_C 6755399441055744.0  // 1.5 * 2^52: y + C keeps round(y) in its low bits

// round to nearest, ties to even (one v_rndne_f64)
__device__ __forceinline__ double fp_rint(double y) { return __builtin_rint(y); }

__device__ __forceinline__ double fp_mulmod(double a, double w, double wq, double q) {
  const double hi = __dmul_rn(a, w);
  const double lo = __fma_rn(a, w, -hi);
  const double t = fp_rint(__dmul_rn(a, wq));
  return __dadd_rn(__fma_rn(-t, q, hi), lo);
}

__device__ __forceinline__ double as_dbl(u64 v) { return __longlong_as_double((long long)v); }
__device__ __forceinline__ u64 dbl_bits(double v) { return (u64)__double_as_longlong(v); }

// exact conversions of integers in [0, 2^52): the word is the mantissa of
// 2^52 + x
constexpr u64 kTwo52Bits = 0x4330000000000000ull;
__device__ __forceinline__ double u52_to_dbl(u64 x) {
  return __dsub_rn(as_dbl(x | kTwo52Bits), 4503599627370496.0);
}
__device__ __forceinline__ u64 dbl_to_u52(double r) {
  return dbl_bits(__dadd_rn(r, 4503599627370496.0)) - kTwo52Bits;
}

// exact conversion of an integer |x| < 2^51 to a signed word: 1.5 2^52 + x
// keeps the exponent of 1.5 2^52, so its word differs from that of 1.5 2^52
// by x
__device__ __forceinline__ long long dbl_to_i51(double x) {
  return (long long)(dbl_bits(__dadd_rn(x, FP_ROUND_C)) - 0x4338000000000000ull);
}

// x -> x - round(x / q) q in [-q/2 - 1, q/2 + 1]
__device__ __forceinline__ double fp_reduce(double x, double qinv, double q) {
  return __fma_rn(-fp_rint(__dmul_rn(x, qinv)), q, x);
}

// x reduced to [0, q) as an exact double
__device__ __forceinline__ double fp_canon_d(double x, double qinv, double q) {
  const double r = fp_reduce(x, qinv, q);
  return r < 0.0 ? __dadd_rn(r, q) : r;
}

__device__ __forceinline__ u64 fp_canon(double x, double qinv, double q) {
  double r = fp_reduce(x, qinv, q);
  r = r < 0.0 ? __dadd_rn(r, q) : r;
  return dbl_to_u52(r);
}

__device__ __forceinline__ void ct_fp(double &X, double &Y, double w, double wq, double q) {
  const double t = fp_mulmod(Y, w, wq, q);
  const double x = X;
  X = __dadd_rn(x, t);
  Y = __dsub_rn(x, t);
}

__device__ __forceinline__ void gs_fp(double &X, double &Y, double w, double wq, double q) {
  const double x = X, y = Y;
  X = __dadd_rn(x, y);
  Y = fp_mulmod(__dsub_rn(x, y), w, wq, q);
}


// Twiddle table layout for the fp64 path, per prime: [N][2] doubles (w, w/q).
// High pass, fp64 body: x[k] = word c + 4096 k of one column, stages on bits
// 15..12; |x| grows by at most q per stage.
__device__ __forceinline__ void fp_high_fwd(double (&x)[16], const double2 *__restrict__ T,
                                            double q) {
#pragma unroll
  for (int st = 0; st < 4; st++) {
    const int half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const double2 w = T[(1 << st) + (k >> (4 - st))];
      ct_fp(x[k], x[k + half], w.x, w.y, q);
    }
  }
}

// inverse high pass on one column (|x| < 2^50 on entry: reduced first);
// |x| <= 8 q + 8 after
__device__ __forceinline__ void fp_high_inv_stages(double (&x)[16], const double2 *__restrict__ T,
                                                   double q, double qinv) {
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = fp_reduce(x[k], qinv, q);
#pragma unroll
  for (int st = 3; st >= 0; st--) {
    const int half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const double2 w = T[(1 << st) + (k >> (4 - st))];
      gs_fp(x[k], x[k + half], w.x, w.y, q);
    }
  }
}

// the inverse high pass, then x N^-1; result as exact doubles in [0, q)
__device__ __forceinline__ void fp_high_inv(double (&x)[16], const double2 *__restrict__ T,
                                            double2 ni, double q, double qinv) {
  fp_high_inv_stages(x, T, q, qinv);
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = fp_canon_d(fp_mulmod(x[k], ni.x, ni.y, q), qinv, q);
}

// Round Z of the fp64 forward low pass (as u64_low_round_z)
__device__ __forceinline__ void fp_low_round_z(double (&x)[16], const double2 *__restrict__ T,
                                               int tile, double q) {
#pragma unroll
  for (int st = 0; st < 4; st++) {
    const int b = 11 - st, half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const double2 w = T[(65536 >> (b + 1)) + ((tile * 4096 + 256 * k) >> (b + 1))];
      ct_fp(x[k], x[k + half], w.x, w.y, q);
    }
  }
}

// inverse round Z on bits 8..11 (entry values reduced first)
__device__ __forceinline__ void fp_inv_round_z(double (&x)[16], const double2 *__restrict__ T,
                                               int tile, double q, double qinv) {
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = fp_reduce(x[k], qinv, q);
#pragma unroll
  for (int b = 8; b < 12; b++) {
    const int half = 1 << (b - 8);
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const double2 w = T[(65536 >> (b + 1)) + ((tile * 4096 + 256 * k) >> (b + 1))];
      gs_fp(x[k], x[k + half], w.x, w.y, q);
    }
  }
}

// Round Z of tile `tile` from src (raw double words t + 256 k) into the LDS
// tile for round A (as u64_round_z_to_lds).
__device__ __forceinline__ void fp_round_z_to_lds(double *__restrict__ sm,
                                                  const u64 *__restrict__ src,
                                                  const double2 *__restrict__ T, int tile,
                                                  double q) {
  const int t = threadIdx.x;
  double x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = as_dbl(src[t + 256 * k]);
  fp_low_round_z(x, T, tile, q);
#pragma unroll
  for (int k = 0; k < 16; k++) sm[lds16(k, t)] = x[k];
}

// Rounds of the fp64 forward low pass (as u64_low_round_a/b); the table
// holds bit positions 2..0 in [row][m][c0] order
__device__ __forceinline__ void fp_low_round_a(double (&x)[16], const double2 *__restrict__ T,
                                               int row, double q) {
#pragma unroll
  for (int st = 0; st < 4; st++) {
    const int b = 7 - st, half = 8 >> st;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const double2 w = T[(65536 >> (b + 1)) + ((row * 256 + 16 * k) >> (b + 1))];
      ct_fp(x[k], x[k + half], w.x, w.y, q);
    }
  }
}

__device__ __forceinline__ void fp_low_round_b(double (&x)[16], const double2 *__restrict__ T,
                                               int row, int c0, double q) {
#pragma unroll
  for (int st = 4; st < 8; st++) {
    const int b = 7 - st, half = 1 << b;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      if (j & half) continue;
      // entry (row 256 + 16 c0 + j) >> (b + 1) of the stage, in the table's
      // [row][m][c0] order for these stages
      const double2 w = T[(65536 >> (b + 1)) + row * (128 >> b) + ((j >> (b + 1)) << 4) + c0];
      ct_fp(x[j], x[j + half], w.x, w.y, q);
    }
  }
}

template <bool COMBINE>
__device__ __forceinline__ void k_ntt16f_fwd_low_body(u64 *__restrict__ lds, Batch dst, int l_begin, int q_limbs,
                                                        int L, const ModQ *__restrict__ mods,
                                                        const double2 *__restrict__ tw,
                                                        MDCombine md) {
  double *sm = reinterpret_cast<double *>(lds);
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const double q = (double)mods[p].q, qinv = 1.0 / q;
  const double2 *T = tw + ((size_t)p << 16);
  u64 *base = batch_ptr(dst, blockIdx.y) + ((size_t)limb << 16) + (size_t)blockIdx.x * 4096;
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int row = blockIdx.x * 16 + rl;
  MDPrefetch pf;
  if constexpr (COMBINE) md_load(md, blockIdx.y, limb, blockIdx.x * 4096 + rl * 256 + c0, pf);
  fp_round_z_to_lds(sm, base, T, blockIdx.x, q);
  __syncthreads();
  double x[16];
  // round A on the thread's slots, written back in place (no other thread
  // reads them)
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = sm[lds16(rl, c0 + 16 * k)];
  fp_low_round_a(x, T, row, q);
#pragma unroll
  for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = x[k];
  row_sync();
#pragma unroll
  for (int j = 0; j < 16; j++) x[j] = sm[lds16(rl, 16 * c0 + j)];
  fp_low_round_b(x, T, row, c0, q);
  row_sync();
  u64 *smu = reinterpret_cast<u64 *>(sm);
#pragma unroll
  for (int j = 0; j < 16; j++) smu[lds16(rl, 16 * c0 + j)] = fp_canon(x[j], qinv, q);
  row_sync();
  if constexpr (COMBINE) {
    const u64 qu = mods[p].q;
    const u32 e0 = blockIdx.x * 4096 + rl * 256 + c0;
    u64 sv[16];
    md_sub_load(md, blockIdx.y, limb, e0, sv);
#pragma unroll
    for (int k = 0; k < 16; k++)
      md_store(md, blockIdx.y, limb, e0 + 16 * k, smu[lds16(rl, c0 + 16 * k)], pf, pf.a[k],
               pf.d[k], sv[k], qu);
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) base[rl * 256 + c0 + 16 * k] = smu[lds16(rl, c0 + 16 * k)];
  }
}

// The fp64 inverse low pass of one 4096-word tile held in the LDS tile sm
// (position rl 256 + c of the tile at lds16(rl, c), exact integers of
// magnitude below q),
// rows 16 tile .. 16 tile + 15 of 256: round A on bit positions 3..0 from
// the 16 consecutive positions 16 c0 + j of row rl, round B on 7..4 from
// positions c0 + 16 k, round Z on 11..8 from positions t + 256 k; the result
// (fp64 words of the pass) goes to out[t + 256 k].  The caller has
// synchronised after filling sm.
__device__ __forceinline__ void fp_inv_low_tile(double *__restrict__ sm, int tile,
                                                const double2 *__restrict__ T, double q,
                                                double qinv, u64 *__restrict__ out) {
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int row = tile * 16 + rl;
  double x[16];
#pragma unroll
  for (int j = 0; j < 16; j++) x[j] = sm[lds16(rl, 16 * c0 + j)];
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const int half = 1 << b;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      if (j & half) continue;
      // entry (row 256 + 16 c0 + j) >> (b + 1), table in [row][m][c0] order
      const double2 w = T[(65536 >> (b + 1)) + row * (128 >> b) + ((j >> (b + 1)) << 4) + c0];
      gs_fp(x[j], x[j + half], w.x, w.y, q);
    }
  }
  row_sync();
#pragma unroll
  for (int j = 0; j < 16; j++) sm[lds16(rl, 16 * c0 + j)] = x[j];
  row_sync();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = fp_reduce(sm[lds16(rl, c0 + 16 * k)], qinv, q);
#pragma unroll
  for (int b = 4; b < 8; b++) {
    const int half = 1 << (b - 4);
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k & half) continue;
      const double2 w = T[(65536 >> (b + 1)) + ((row * 256 + 16 * k) >> (b + 1))];
      gs_fp(x[k], x[k + half], w.x, w.y, q);
    }
  }
  // the thread's slots back in place, then one tile column per thread
#pragma unroll
  for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = x[k];
  __syncthreads();
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = sm[lds16(k, t)];
  fp_inv_round_z(x, T, tile, q, qinv);
#pragma unroll
  for (int k = 0; k < 16; k++) out[t + 256 * k] = dbl_bits(x[k]);
}

__device__ __forceinline__ void k_ntt16f_inv_low_body(u64 *__restrict__ lds, Batch src, Batch dst, int l_begin,
                                                        int q_limbs, int L,
                                                        const ModQ *__restrict__ mods,
                                                        const double2 *__restrict__ itw,
                                                        const Batch &mul, int mm) {
  double *sm = reinterpret_cast<double *>(lds);
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const double q = (double)mods[p].q, qinv = 1.0 / q;
  const double2 *T = itw + ((size_t)p << 16);
  const u64 *in = batch_ptr(src, blockIdx.y) + ((size_t)limb << 16) + (size_t)blockIdx.x * 4096;
  u64 *out = batch_ptr(dst, blockIdx.y) + ((size_t)limb << 16) + (size_t)blockIdx.x * 4096;
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  if (mm) {
    // the transform of src x mul (mm 1) or src^2 (mm 2), formed here: the
    // product of two words below q < 2^45 leaves fp_mulmod in (-q, q), the
    // magnitude fp_inv_low_tile takes
    const u64 *mb = mm == 2 ? in
                            : batch_ptr(mul, blockIdx.y) + ((size_t)limb << 16) +
                                  (size_t)blockIdx.x * 4096;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int e = rl * 256 + c0 + 16 * k;
      const double x = u52_to_dbl(in[e]), w = mm == 2 ? x : u52_to_dbl(mb[e]);
      sm[lds16(rl, c0 + 16 * k)] = fp_mulmod(x, w, __dmul_rn(w, qinv), q);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++)
      sm[lds16(rl, c0 + 16 * k)] = u52_to_dbl(in[rl * 256 + c0 + 16 * k]);
  }
  row_sync();
  fp_inv_low_tile(sm, blockIdx.x, T, q, qinv, out);
}

// One launch per pass over every limb of a batch: a block takes the fp64
// body when its prime is below 2^45 and the 64-bit body otherwise (q_0), so
// the few 64-bit limbs run beside the others instead of in launches of their
// own.  Both low-pass bodies share one LDS tile.
constexpr u64 kFpPrimeBound = (u64)1 << 45;

// High passes: thread = one column c = 256 blockIdx.x + t of limb
// l_begin + blockIdx.z of item blockIdx.y; words c + 4096 k, each load and
// store of a wave 512 contiguous bytes.  Forward: canonical input, lazy
// output (fp64: raw double bits); inverse: lazy input, canonical output.
__global__ __launch_bounds__(TPB) void k_ntt16m_fwd_high(Batch src, Batch dst, int l_begin,
                                                         int q_limbs, int L,
                                                         const ModQ *__restrict__ mods,
                                                         const u64 *__restrict__ psi,
                                                         const u64 *__restrict__ psi_sh,
                                                         const double2 *__restrict__ tw) {
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  const u64 *in = batch_ptr(src, blockIdx.y) + ((size_t)limb << 16) + blockIdx.x * 256 + threadIdx.x;
  u64 *out = batch_ptr(dst, blockIdx.y) + ((size_t)limb << 16) + blockIdx.x * 256 + threadIdx.x;
  const u64 qu = mods[p].q;
  if (qu < kFpPrimeBound) {
    const double q = (double)qu;
    double x[16];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = u52_to_dbl(in[4096 * k]);
    fp_high_fwd(x, tw + ((size_t)p << 16), q);
#pragma unroll
    for (int k = 0; k < 16; k++) out[4096 * k] = dbl_bits(x[k]);
  } else {
    u64 x[16];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = in[4096 * k];
    u64_high_fwd(x, psi + ((size_t)p << 16), psi_sh + ((size_t)p << 16), qu, 2 * qu);
#pragma unroll
    for (int k = 0; k < 16; k++) out[4096 * k] = x[k];
  }
}

template <bool COMBINE>
__global__ __launch_bounds__(TPB) void k_ntt16m_fwd_low(Batch dst, int l_begin, int q_limbs,
                                                        int L, const ModQ *__restrict__ mods,
                                                        const u64 *__restrict__ psi,
                                                        const u64 *__restrict__ psi_sh,
                                                        const double2 *__restrict__ tw,
                                                        MDCombine md) {
  __shared__ u64 lds[16 * 272];
  if (mods[prime_of(l_begin + blockIdx.z, q_limbs, L)].q < kFpPrimeBound)
    k_ntt16f_fwd_low_body<COMBINE>(lds, dst, l_begin, q_limbs, L, mods, tw, md);
  else
    k_ntt16_fwd_low_body<COMBINE>(lds, dst, l_begin, q_limbs, L, mods, psi, psi_sh, md);
}

// mm 1: the transform of src x mul (word by word), 2: of src^2, 0: of src
__global__ __launch_bounds__(TPB) void k_ntt16m_inv_low(Batch src, Batch dst, int l_begin,
                                                        int q_limbs, int L,
                                                        const ModQ *__restrict__ mods,
                                                        const u64 *__restrict__ ipsi,
                                                        const u64 *__restrict__ ipsi_sh,
                                                        const double2 *__restrict__ itw,
                                                        Batch mul, int mm) {
  __shared__ u64 lds[16 * 272];
  if (mods[prime_of(l_begin + blockIdx.z, q_limbs, L)].q < kFpPrimeBound)
    k_ntt16f_inv_low_body(lds, src, dst, l_begin, q_limbs, L, mods, itw, mul, mm);
  else
    k_ntt16_inv_low_body(lds, src, dst, l_begin, q_limbs, L, mods, ipsi, ipsi_sh, mul, mm);
}

__global__ __launch_bounds__(TPB) void k_ntt16m_inv_high(
    Batch dst, int l_begin, int q_limbs, int L, const ModQ *__restrict__ mods,
    const u64 *__restrict__ ipsi, const u64 *__restrict__ ipsi_sh, const u64 *__restrict__ ninv,
    const double2 *__restrict__ itw, const double2 *__restrict__ ninv_fp) {
  const int limb = l_begin + blockIdx.z;
  const int p = prime_of(limb, q_limbs, L);
  u64 *io = batch_ptr(dst, blockIdx.y) + ((size_t)limb << 16) + blockIdx.x * 256 + threadIdx.x;
  const u64 qu = mods[p].q;
  if (qu < kFpPrimeBound) {
    const double q = (double)qu, qinv = 1.0 / q;
    double x[16];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = as_dbl(io[4096 * k]);
    fp_high_inv(x, itw + ((size_t)p << 16), ninv_fp[p], q, qinv);
#pragma unroll
    for (int k = 0; k < 16; k++) io[4096 * k] = dbl_to_u52(x[k]);
  } else {
    u64 x[16];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = io[4096 * k];
    u64_high_inv(x, ipsi + ((size_t)p << 16), ipsi_sh + ((size_t)p << 16), ninv[2 * p],
                 ninv[2 * p + 1], qu, 2 * qu);
#pragma unroll
    for (int k = 0; k < 16; k++) io[4096 * k] = x[k];
  }
}

// the high passes of a batch: grid (16, items, limbs)
static void launch_fwd_high16(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                              int l_begin, int l_count, int q_limbs) {
  hipLaunchKernelGGL(k_ntt16m_fwd_high, dim3(16, n_items, l_count), dim3(TPB), 0, c->stream,
                     src, dst, l_begin, q_limbs, c->L, c->d_mods, c->d_psi, c->d_psi_sh,
                     (const double2 *)c->d_tw_fp);
  LAUNCH_CHECK();
}

static void launch_inv_high16(ckks_context *c, const Batch &dst, int n_items, int l_begin,
                              int l_count, int q_limbs) {
  hipLaunchKernelGGL(k_ntt16m_inv_high, dim3(16, n_items, l_count), dim3(TPB), 0, c->stream,
                     dst, l_begin, q_limbs, c->L, c->d_mods, c->d_ipsi, c->d_ipsi_sh,
                     c->d_ninv, (const double2 *)c->d_itw_fp, (const double2 *)c->d_ninv_fp);
  LAUNCH_CHECK();
}

// grid (tiles, items, limbs): blocks of one prime run back to back and share
// its twiddle table in L2
static void ntt16_dispatch(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                           int l_begin, int l_count, int q_limbs, bool inverse) {
  dim3 block(TPB), grid(16, n_items, l_count);
  if (!inverse) {
    launch_fwd_high16(c, src, dst, n_items, l_begin, l_count, q_limbs);
    hipLaunchKernelGGL(k_ntt16m_fwd_low<false>, grid, block, 0, c->stream, dst, l_begin, q_limbs,
                       c->L, c->d_mods, c->d_psi, c->d_psi_sh, (const double2 *)c->d_tw_fp,
                       MDCombine{});
    LAUNCH_CHECK();
  } else {
    hipLaunchKernelGGL(k_ntt16m_inv_low, grid, block, 0, c->stream, src, dst, l_begin, q_limbs,
                       c->L, c->d_mods, c->d_ipsi, c->d_ipsi_sh, (const double2 *)c->d_itw_fp,
                       Batch{}, 0);
    LAUNCH_CHECK();
    launch_inv_high16(c, dst, n_items, l_begin, l_count, q_limbs);
  }
}

template <int S1, int S2, int TILE>
static void ntt_dispatch(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                         int l_begin, int l_count, int q_limbs, bool inverse) {
  const int N = c->N;
  dim3 block(TPB);
  // grid (tiles, items, limbs): blocks of one prime run back to back and
  // share its twiddle table in L2
  dim3 g_high((N >> S1) / (TILE >> S1), n_items, l_count);
  dim3 g_low(N / TILE, n_items, l_count);
  if (!inverse) {
    hipLaunchKernelGGL((k_ntt_fwd_high<S1, TILE>), g_high, block, 0, c->stream, src, dst,
                       c->logN, l_begin, q_limbs, c->L, c->d_mods, c->d_psi, c->d_psi_sh);
    LAUNCH_CHECK();
    hipLaunchKernelGGL((k_ntt_fwd_low<S2, TILE>), g_low, block, 0, c->stream, dst, c->logN,
                       l_begin, q_limbs, c->L, c->d_mods, c->d_psi, c->d_psi_sh);
    LAUNCH_CHECK();
  } else {
    hipLaunchKernelGGL((k_ntt_inv_low<S2, TILE>), g_low, block, 0, c->stream, src, dst,
                       c->logN, l_begin, q_limbs, c->L, c->d_mods, c->d_ipsi, c->d_ipsi_sh);
    LAUNCH_CHECK();
    hipLaunchKernelGGL((k_ntt_inv_high<S1, TILE>), g_high, block, 0, c->stream, dst,
                       c->logN, l_begin, q_limbs, c->L, c->d_mods, c->d_ipsi, c->d_ipsi_sh,
                       c->d_ninv);
    LAUNCH_CHECK();
  }
}

void launch_ntt(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                int l_begin, int l_count, int q_limbs, bool inverse) {
  KTimer kt(c, inverse ? "ntt_inv" : "ntt_fwd", 16.0 * c->N * n_items * l_count,
            0.5 * c->N * c->logN * n_items * l_count);
  if (n_items <= 0 || l_count <= 0) return;
  switch (c->logN) {
    case 10: ntt_dispatch<5, 5, 1024>(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    case 11: ntt_dispatch<5, 6, 2048>(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    case 12: ntt_dispatch<6, 6, 4096>(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    case 13: ntt_dispatch<6, 7, 4096>(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    case 14: ntt_dispatch<7, 7, 4096>(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    case 15: ntt_dispatch<7, 8, 4096>(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    case 16: ntt16_dispatch(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    case 17: ntt_dispatch<8, 9, 4096>(c, src, dst, n_items, l_begin, l_count, q_limbs, inverse); break;
    default: throw std::invalid_argument("log_n must be in [10, 17]");
  }
}

void launch_ntt_inv_high(ckks_context *c, const Batch &dst, int n_items, int l_begin, int l_count,
                         int q_limbs) {
  KTimer kt(c, "ntt_inv", 16.0 * c->N * n_items * l_count, 0.5 * c->N * 4 * n_items * l_count);
  if (n_items <= 0 || l_count <= 0) return;
  if (c->logN != 16) throw std::invalid_argument("inverse high pass alone: N = 2^16 only");
  launch_inv_high16(c, dst, n_items, l_begin, l_count, q_limbs);
}

// Forward NTT of the ModDown conversion conv (2 n items, Q limbs) with the
// combine of k_moddown_combine fused into the low pass: the converted P part
// is never written back.  N = 2^16 only.
void launch_ntt_moddown(ckks_context *c, const Batch &conv, int n, int limbs, const Batch &acc,
                        int E, const u64 *pinv, const Batch &add, u64 add1_off,
                        const u64 *galois, const Batch &out, u64 out1_off, const u64 *amul,
                        const PostOp *post, bool high_done, bool wide_only) {
  // the limbs this call combines (wide_only: those of primes at or above 2^45)
  int run_limbs = limbs;
  if (wide_only) {
    run_limbs = 0;
    for (int l = 0; l < limbs; l++) run_limbs += c->prime_fp[l] ? 0 : 1;
  }
  KTimer kt(c, "ntt_fwd_moddown",
            8.0 * c->N * run_limbs *
                (6.0 * n + (batch_ptr_host(add, 0) ? (add1_off ? 2.0 : 1.0) * n : 0.0)),
            0.5 * c->N * c->logN * 2.0 * n * run_limbs);
  if (c->logN != 16 || n > kMaxBatch) throw std::invalid_argument("fused ModDown: N = 2^16, n <= 64");
  MDCombine md{};
  md.acc = acc;
  md.E = E;
  md.pinv = pinv;
  md.amul = amul;
  md.add = add;
  md.add1_off = add1_off;
  md.out = out;
  md.out1_off = out1_off;
  if (post) md.post = *post;
  for (int i = 0; i < n; i++) md.gal.g[i] = galois[i];
  if (!high_done) launch_fwd_high16(c, conv, conv, 2 * n, 0, limbs, limbs);
  // runs of limbs (wide_only: the limbs of primes at or above 2^45 alone,
  // the others being combined by launch_low_key_moddown)
  for (int l0 = 0; l0 < limbs;) {
    if (wide_only && c->prime_fp[l0]) {
      l0++;
      continue;
    }
    int l1 = l0 + 1;
    while (l1 < limbs && !(wide_only && c->prime_fp[l1])) l1++;
    hipLaunchKernelGGL(k_ntt16m_fwd_low<true>, dim3(16, 2 * n, l1 - l0), dim3(TPB), 0, c->stream,
                       conv, l0, limbs, c->L, c->d_mods, c->d_psi, c->d_psi_sh,
                       (const double2 *)c->d_tw_fp, md);
    LAUNCH_CHECK();
    l0 = l1;
  }
}

// Only the high pass of the forward NTT (bit positions 15..12), for limbs
// whose low pass runs inside launch_ntt_low_key.  N = 2^16 only.
void launch_ntt_fwd_high(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                         int l_begin, int l_count, int q_limbs) {
  KTimer kt(c, "ntt_fwd_high", 16.0 * c->N * n_items * l_count,
            0.5 * c->N * 4 * n_items * l_count);
  if (n_items <= 0 || l_count <= 0) return;
  if (c->logN != 16) throw std::invalid_argument("high pass alone: N = 2^16 only");
  launch_fwd_high16(c, src, dst, n_items, l_begin, l_count, q_limbs);
}

// ===========================================================================
// N = 2^16: the forward NTT's low pass of every digit's extended limb with
// the key inner product as its epilogue, so that the ModUp output is never
// stored in NTT form.  Block (item, tile, limb) holds the 4096 words
// tile 4096 + [0, 4096) of limb l: for each digit j it runs the low pass on
// what the high pass left in ext (or reads the digit's own limb, already in
// NTT form, from the source), then accumulates
//   acc_c[l][t] = sum_j ext_j[l][s] key_j[c][l][s],  t = autom_index(s, g^-1)
// with the key in source order (the words of k_key_inner, which reads both
// at s = autom_index(t, g)).  The automorphism maps each aligned group of 16
// words onto an aligned group of 16, so the 16 lanes holding one group of s
// (the coalesced layout s = tile 4096 + rl 256 + c0 + 16 k) write the
// accumulator at one 128-byte group of t.
// fp64 primes multiply by the Montgomery-form key words in fp64 and take
// the factor 2^-64 out once at the end; the 64-bit body reduces each digit's
// product by redc, as k_key_inner reduces their sum: the same words.
// grid (items, 16, E): the blocks of one tile and limb run back to back and
// read its key words from L2.
// ===========================================================================

struct LowKeyArgs {
  const u64 *ext;     // item it, digit j, limb l: ext + it ext_stride + ((j E + l) << 16)
  size_t ext_stride;
  // 1: the planes of fp64 limbs hold k_convert_h4's packed form (the 32 low
  // bits of a centered residue, then its 16 high bits), 0: raw double bits
  int ext_packed;
  Batch own;          // per item: the source polynomial, limb l at l << 16 (NTT form)
  // own_mul 1: the source polynomial is own x own_b word by word, 2: own^2
  // (formed where the digit's own limb is read), 0: own itself
  Batch own_b;
  int own_mul;
  u64 *acc;           // per item [2][E][N] at acc + it acc_stride
  size_t acc_stride;
  const u64 *key;     // [digits][2][K][N], Montgomery form, source order
  u64 ginv;           // inverse of the Galois element mod 2N (1: none)
  int digits, E, q_limbs, L, K, ds;
  // with sp (fp64 special primes only): component c of special limb
  // l >= q_limbs leaves through the inverse NTT's low pass, to
  // sp + (2 it + c) sp_stride + ((l - q_limbs) << 16), and acc's special
  // limbs are not written
  u64 *sp;
  size_t sp_stride;
  const double2 *itw;
};

// Offset of position sb + i's key word from key_slot(sb) (sb 16-aligned)
__device__ __forceinline__ constexpr int kword(int i) { return ((i >> 1) << 7) | (i & 1); }

// 4 consecutive words from a 32-byte aligned address, as 2 loads of 16 bytes
__device__ __forceinline__ void load4(const u64 *__restrict__ p, u64 (&v)[4]) {
  const ulonglong2 *q = reinterpret_cast<const ulonglong2 *>(p);
  const ulonglong2 x = q[0], y = q[1];
  v[0] = x.x;
  v[1] = x.y;
  v[2] = y.x;
  v[3] = y.y;
}

// 16 consecutive words from a 128-byte aligned address, as 8 loads of 16 bytes
__device__ __forceinline__ void load16(const u64 *__restrict__ p, u64 (&v)[16]) {
  const ulonglong2 *q = reinterpret_cast<const ulonglong2 *>(p);
#pragma unroll
  for (int m = 0; m < 8; m++) {
    const ulonglong2 t = q[m];
    v[2 * m] = t.x;
    v[2 * m + 1] = t.y;
  }
}

// The permuted store of one accumulator component: word(i), the thread's
// word for position s = sb + i, goes to t = autom_index(s, g^-1), inside the
// tile tb + [0, 4096); it passes through the LDS tile so that the store is
// coalesced.
template <typename F>
__device__ __forceinline__ void low_key_store(u64 *__restrict__ sm, F word, u32 sb, u64 ginv,
                                              u64 *__restrict__ out, u32 tb) {
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  __syncthreads();  // earlier reads of the tile are done
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const u32 t = ginv == 1 ? sb + i : autom_index(sb + i, ginv, 16);
    sm[lds16((t >> 8) & 15, t & 255)] = word(i);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) out[tb + rl * 256 + c0 + 16 * k] = sm[lds16(rl, c0 + 16 * k)];
}

// As low_key_store, then the inverse NTT's low pass of the permuted tile
// (fp64 words in [0, q)) from the LDS tile into out + tb (fp_inv_low_tile).
template <typename F>
__device__ __forceinline__ void low_key_store_inv(double *__restrict__ sm, F word, u32 sb,
                                                  u64 ginv, const double2 *__restrict__ T,
                                                  double q, double qinv, u64 *__restrict__ out,
                                                  u32 tb) {
  __syncthreads();  // earlier reads of the tile are done
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const u32 t = ginv == 1 ? sb + i : autom_index(sb + i, ginv, 16);
    sm[lds16((t >> 8) & 15, t & 255)] = word(i);
  }
  __syncthreads();
  fp_inv_low_tile(sm, (int)(tb >> 12), T, q, qinv, out + tb);
}

// Per digit: the low pass leaves each thread the 16 consecutive positions
// s = sb + i of round B, where the key product runs; the own limb and the
// key words are read at those positions.
// The key product of one (item, tile, limb) on an fp64 prime: per digit the
// low pass leaves each thread the 16 consecutive positions s = sb + i of
// round B, where the key product runs; the own limb and the key words are
// read at those positions.  acc0 / acc1 leave unreduced (|acc| <= digits q).
__device__ __forceinline__ void low_key_fp_acc(double *__restrict__ sm, const LowKeyArgs &a,
                                               int it, int tile, int l, int p,
                                               const ModQ *__restrict__ mods,
                                               const double2 *__restrict__ tw,
                                               double (&acc0)[16], double (&acc1)[16]) {
  const double q = (double)mods[p].q, qinv = 1.0 / q;
  const double2 *T = tw + ((size_t)p << 16);
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int row = tile * 16 + rl;
  const u32 sb = (u32)(tile * 4096 + rl * 256 + 16 * c0);
  const u32 kslot = key_slot(sb);
  const int jo = l < a.q_limbs ? l / a.ds : -1;
  for (int j = 0; j < a.digits; j++) {
    double y[16];
    if (j == jo && a.own_mul) {
      // products of words below q < 2^45, in (-q, q), four at a time
      const u64 *pa = batch_ptr(a.own, it) + ((size_t)l << 16) + sb;
      const u64 *pb = a.own_mul == 2 ? pa : batch_ptr(a.own_b, it) + ((size_t)l << 16) + sb;
#pragma unroll
      for (int i0 = 0; i0 < 16; i0 += 4) {
        u64 wa[4], wb[4];
        load4(pa + i0, wa);
        if (a.own_mul == 1) load4(pb + i0, wb);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const double x = u52_to_dbl(wa[i]), w = a.own_mul == 2 ? x : u52_to_dbl(wb[i]);
          y[i0 + i] = fp_mulmod(x, w, __dmul_rn(w, qinv), q);
        }
      }
    } else if (j == jo) {
      u64 w[16];
      load16(batch_ptr(a.own, it) + ((size_t)l << 16) + sb, w);
#pragma unroll
      for (int i = 0; i < 16; i++) y[i] = u52_to_dbl(w[i]);
    } else {
      const u64 *plane = a.ext + it * a.ext_stride + ((size_t)(j * a.E + l) << 16);
      const int t = threadIdx.x;
      // round Z on the thread's column; only its LDS writes wait for the
      // previous digit's reads of the tile
      if (a.ext_packed) {
        const u32 *lo = reinterpret_cast<const u32 *>(plane) + tile * 4096 + t;
        const short *hi =
            reinterpret_cast<const short *>(reinterpret_cast<const u32 *>(plane) + 65536) +
            tile * 4096 + t;
#pragma unroll
        for (int k = 0; k < 16; k++)
          y[k] = __fma_rn((double)hi[256 * k], 4294967296.0, (double)lo[256 * k]);
      } else {
        const u64 *src = plane + (size_t)tile * 4096;
#pragma unroll
        for (int k = 0; k < 16; k++) y[k] = as_dbl(src[t + 256 * k]);
      }
      fp_low_round_z(y, T, tile, q);
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 16; k++) sm[lds16(k, t)] = y[k];
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 16; k++) y[k] = sm[lds16(rl, c0 + 16 * k)];
      fp_low_round_a(y, T, row, q);
#pragma unroll
      for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = y[k];
      row_sync();
#pragma unroll
      for (int i = 0; i < 16; i++) y[i] = sm[lds16(rl, 16 * c0 + i)];
      fp_low_round_b(y, T, row, c0, q);
    }
    // |y| <= 17 q < 2^50: the products need no reduction first.  The key
    // words of positions sb + i sit at key_slot(sb + i) = kslot + kword(i)
    const u64 *kb = a.key + ((size_t)(2 * j) * a.K + p) * 65536 + kslot;
    const u64 *ka = kb + (size_t)a.K * 65536;
    // groups of 4 positions; each group's 8 key words are loaded one group
    // ahead of their products
    u64 kw[2][8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      kw[0][2 * i] = kb[kword(i)];
      kw[0][2 * i + 1] = ka[kword(i)];
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
      __builtin_amdgcn_sched_barrier(0);
      if (g < 3) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          kw[(g + 1) & 1][2 * i] = kb[kword(4 * (g + 1) + i)];
          kw[(g + 1) & 1][2 * i + 1] = ka[kword(4 * (g + 1) + i)];
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int e = 4 * g + i;
        const double wb = u52_to_dbl(kw[g & 1][2 * i]), wa = u52_to_dbl(kw[g & 1][2 * i + 1]);
        const double pb = fp_mulmod(y[e], wb, __dmul_rn(wb, qinv), q);
        const double pa = fp_mulmod(y[e], wa, __dmul_rn(wa, qinv), q);
        acc0[e] = j == 0 ? pb : __dadd_rn(acc0[e], pb);
        acc1[e] = j == 0 ? pa : __dadd_rn(acc1[e], pa);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <bool SPINV>
__device__ __forceinline__ void low_key_fp(double *__restrict__ sm, const LowKeyArgs &a, int it,
                                           int tile, int l, int p, const ModQ *__restrict__ mods,
                                           const double2 *__restrict__ tw,
                                           const double2 *__restrict__ rinv) {
  const double q = (double)mods[p].q, qinv = 1.0 / q;
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const u32 sb = (u32)(tile * 4096 + rl * 256 + 16 * c0);
  double acc0[16], acc1[16];
  low_key_fp_acc(sm, a, it, tile, l, p, mods, tw, acc0, acc1);
  // x 2^-64 (the keys' Montgomery factor), then canonical
  const double2 ri = rinv[p];
  auto canon_d = [&](double x) {
    const double r = fp_reduce(fp_mulmod(x, ri.x, ri.y, q), qinv, q);
    return r < 0.0 ? __dadd_rn(r, q) : r;
  };
  auto canon = [&](double x) { return dbl_to_u52(canon_d(x)); };
  const u32 tb = a.ginv == 1 ? sb & ~4095u : autom_index(sb, a.ginv, 16) & ~4095u;
  if constexpr (SPINV) {
    const double2 *Ti = a.itw + ((size_t)p << 16);
    u64 *o = a.sp + 2 * (size_t)it * a.sp_stride + ((size_t)(l - a.q_limbs) << 16);
    low_key_store_inv(sm, [&](int i) { return canon_d(acc0[i]); }, sb, a.ginv, Ti, q, qinv, o, tb);
    low_key_store_inv(sm, [&](int i) { return canon_d(acc1[i]); }, sb, a.ginv, Ti, q, qinv,
                      o + a.sp_stride, tb);
    return;
  }
  u64 *o = a.acc + it * a.acc_stride + ((size_t)l << 16);
  u64 *smu = reinterpret_cast<u64 *>(sm);
  low_key_store(smu, [&](int i) { return canon(acc0[i]); }, sb, a.ginv, o, tb);
  low_key_store(smu, [&](int i) { return canon(acc1[i]); }, sb, a.ginv, o + ((size_t)a.E << 16),
                tb);
}

__device__ __forceinline__ void low_key_64(u64 *__restrict__ sm, const LowKeyArgs &a, int it,
                                           int tile, int l, int p, const ModQ *__restrict__ mods,
                                           const u64 *__restrict__ psi,
                                           const u64 *__restrict__ psi_sh) {
  const ModQ M = mods[p];
  const u64 q = M.q, q2 = 2 * q;
  const u64 *W = psi + ((size_t)p << 16);
  const u64 *Ws = psi_sh + ((size_t)p << 16);
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int row = tile * 16 + rl;
  const u32 sb = (u32)(tile * 4096 + rl * 256 + 16 * c0);
  const u32 kslot = key_slot(sb);
  const int jo = l < a.q_limbs ? l / a.ds : -1;
  // accumulators start at 0: add_mod(0, p) = p for the canonical products
  u64 acc0[16], acc1[16];
#pragma unroll
  for (int i = 0; i < 16; i++) acc0[i] = acc1[i] = 0;
  for (int j = 0; j < a.digits; j++) {
    u64 y[16];
    if (j == jo && a.own_mul) {
      const u64 *pa = batch_ptr(a.own, it) + ((size_t)l << 16) + sb;
      const u64 *pb = a.own_mul == 2 ? pa : batch_ptr(a.own_b, it) + ((size_t)l << 16) + sb;
#pragma unroll
      for (int i0 = 0; i0 < 16; i0 += 4) {
        u64 wa[4], wb[4];
        load4(pa + i0, wa);
        if (a.own_mul == 1) load4(pb + i0, wb);
#pragma unroll
        for (int i = 0; i < 4; i++) y[i0 + i] = mul_mod(wa[i], a.own_mul == 2 ? wa[i] : wb[i], M);
      }
    } else if (j == jo) {
      load16(batch_ptr(a.own, it) + ((size_t)l << 16) + sb, y);
    } else {
      const u64 *src = a.ext + it * a.ext_stride + ((size_t)(j * a.E + l) << 16) +
                       (size_t)tile * 4096;
      // round Z on the thread's column; only its LDS writes wait for the
      // previous digit's reads of the tile
      const int t = threadIdx.x;
#pragma unroll
      for (int k = 0; k < 16; k++) y[k] = src[t + 256 * k];
      u64_low_round_z(y, W, Ws, tile, q, q2);
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 16; k++) sm[lds16(k, t)] = y[k];
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 16; k++) y[k] = sm[lds16(rl, c0 + 16 * k)];
      u64_low_round_a(y, W, Ws, row, q, q2);
#pragma unroll
      for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = y[k];
      row_sync();
#pragma unroll
      for (int i = 0; i < 16; i++) y[i] = sm[lds16(rl, 16 * c0 + i)];
      u64_low_round_b(y, W, Ws, row, c0, q, q2);
#pragma unroll
      for (int i = 0; i < 16; i++) {
        y[i] = csub(csub(y[i], q2), q);
      }
    }
    const u64 *kb = a.key + ((size_t)(2 * j) * a.K + p) * 65536 + kslot;
    const u64 *ka = kb + (size_t)a.K * 65536;
    // groups of 4 positions; each group's 8 key words are loaded one group
    // ahead of their products
    u64 kw[2][8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      kw[0][2 * i] = kb[kword(i)];
      kw[0][2 * i + 1] = ka[kword(i)];
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
      __builtin_amdgcn_sched_barrier(0);
      if (g < 3) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          kw[(g + 1) & 1][2 * i] = kb[kword(4 * (g + 1) + i)];
          kw[(g + 1) & 1][2 * i + 1] = ka[kword(4 * (g + 1) + i)];
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int e = 4 * g + i;
        const u64 b = kw[g & 1][2 * i], c = kw[g & 1][2 * i + 1];
        const u64 pb = redc(__umul64hi(y[e], b), y[e] * b, q, M.qinv);
        const u64 pa = redc(__umul64hi(y[e], c), y[e] * c, q, M.qinv);
        acc0[e] = add_mod(acc0[e], pb, q);
        acc1[e] = add_mod(acc1[e], pa, q);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  u64 *o = a.acc + it * a.acc_stride + ((size_t)l << 16);
  const u32 tb = a.ginv == 1 ? sb & ~4095u : autom_index(sb, a.ginv, 16) & ~4095u;
  low_key_store(sm, [&](int i) { return acc0[i]; }, sb, a.ginv, o, tb);
  low_key_store(sm, [&](int i) { return acc1[i]; }, sb, a.ginv, o + ((size_t)a.E << 16), tb);
}

// One kernel per body, each over a run of nl limbs of its kind starting at
// l_begin, so that each gets its own register allocation.  1-D grid of
// n_items x 16 x nl blocks, decoded so that the n_items blocks of one
// (tile, limb) share b % 8, i.e. run on one XCD (blocks go to the 8 XCDs
// round robin) and read the tile's key words into one L2.
// SPINV (fp64 bodies of special limbs with a.sp): the inverse low pass of
// the two accumulator components into a.sp instead of the stores to acc; a
// kernel of its own, so that the Q limbs' blocks keep the smaller register
// allocation of the plain body.
template <bool FP, bool SPINV = false>
__global__ __launch_bounds__(TPB, 2) void k_ntt16_low_key(LowKeyArgs a, int l_begin,
                                                                   int n_items,
                                                                   const ModQ *__restrict__ mods,
                                                                   const u64 *__restrict__ psi,
                                                                   const u64 *__restrict__ psi_sh,
                                                                   const double2 *__restrict__ tw,
                                                                   const double2 *__restrict__ rinv) {
  __shared__ u64 lds[16 * 272];
  const int b = blockIdx.x, r = b >> 3;
  const int it = r % n_items, tl = (r / n_items) * 8 + (b & 7);
  const int tile = tl & 15, l = l_begin + (tl >> 4);
  const int p = prime_of(l, a.q_limbs, a.L);
  if constexpr (FP)
    low_key_fp<SPINV>(reinterpret_cast<double *>(lds), a, it, tile, l, p, mods, tw, rinv);
  else
    low_key_64(lds, a, it, tile, l, p, mods, psi, psi_sh);
}

// ===========================================================================
// N = 2^16, fp64 Q limbs: the key product of one (item, tile, limb) and the
// ModDown's combine of the output tile it maps to, with the accumulator kept
// in the block.  After the key product (low_key_fp_acc) each component's
// values, x 2^-64 plus [P] addend, go through the LDS tile to their output
// positions t = autom_index(s, g^-1) (an aligned tile onto an aligned tile),
// so that thread (rl, c0) holds output words tb + rl 256 + c0 + 16 k.  Then,
// per component, the forward low pass of the converted special part (conv:
// launch_convert_h4's output for this limb and output tile) and
//   out = (acc - NTT(conv)) P^-1 + addend,
// the words of launch_ntt_low_key then launch_ntt_moddown (no postop).  The special
// limbs' key product (and their inverse low pass) and the ModDown's
// conversion run before it.
// ===========================================================================
// The combine's side of k_low_key_md: P^-1 per Q limb (and its quotient
// constant), the outputs, and per item either the addend (prod 0: d0 at add,
// d1 at add + add1_off, add null for none) or the factors of the degree-2
// product whose d0 = a0 b0 and d1 = a0 b1 + a1 b0 are the addend (prod 1: a0
// at add, a1 at add + add1_off, b0 and b1 likewise from mulb; prod 2: the
// square of a, mulb unused).
struct LowMD {
  const u64 *pinv;
  Batch add;
  u64 add1_off;
  Batch mulb;
  Batch out;
  u64 out1_off;
  int prod;
};


__global__ __launch_bounds__(TPB, 2) void k_low_key_md(LowKeyArgs a, LowMD md, Batch conv,
                                                       const u64 *__restrict__ pmod,
                                                       int l_begin, int n_items,
                                                       const ModQ *__restrict__ mods,
                                                       const double2 *__restrict__ tw,
                                                       const double2 *__restrict__ rinv) {
  // tile 0: the working tile; tile 1: component 1's accumulator values in
  // their output order until its combine
  __shared__ u64 lds[2 * 16 * 272];
  double *sm = reinterpret_cast<double *>(lds), *acc1t = sm + 16 * 272;
  const int b = blockIdx.x, r0 = b >> 3;
  const int it = r0 % n_items, tl = (r0 / n_items) * 8 + (b & 7);
  const int tile = tl & 15, l = l_begin + (tl >> 4);
  const int p = prime_of(l, a.q_limbs, a.L);
  const double q = (double)mods[p].q, qinv = 1.0 / q;
  const int c0 = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const u32 sb = (u32)(tile * 4096 + rl * 256 + 16 * c0);
  double acc0[16], acc1[16];
  low_key_fp_acc(sm, a, it, tile, l, p, mods, tw, acc0, acc1);
  // Everything below stays in fp64: signed exact integers congruent to the
  // words, reduced to [0, q) once at the store.  The addend of output t is
  // the word at sigma(t) = s: the thread holds it at its own positions, so
  // (acc - conv) P^-1 + add is taken as (acc + [P] add - conv) P^-1, with
  // add read here in source order.  Bounds: acc 2^-64 and [P] add each in
  // [-q, q]; the converted part after its 16 forward stages below 2^49.2
  // (entry below 2^46, at most q more per stage), so the factor of P^-1
  // sees less than 2^49.3 < 2^50, as fp_mulmod needs.
  const double2 ri = rinv[p];
  const double Pm = (double)pmod[2 * l], Pmq = __dmul_rn(Pm, qinv);
  const u64 *ad0 = batch_ptr(md.add, it);
  const u64 *ad1 = (ad0 && md.add1_off) ? ad0 + md.add1_off : nullptr;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    acc0[i] = fp_mulmod(acc0[i], ri.x, ri.y, q);
    acc1[i] = fp_mulmod(acc1[i], ri.x, ri.y, q);
  }
  if (md.prod) {
    // the addend formed here from the factors (words below q < 2^45): each
    // product |a b| < 2^90 leaves fp_mulmod within (-q, q), so d0 lies in
    // (-q, q), d1 in (-2 q, 2 q) and [P] d again in (-q, q)
    const u64 *pa0 = ad0 + ((size_t)l << 16) + sb, *pa1 = pa0 + md.add1_off;
    const u64 *pb0 = md.prod == 2 ? pa0 : batch_ptr(md.mulb, it) + ((size_t)l << 16) + sb;
    const u64 *pb1 = pb0 + md.add1_off;
    // each group of 4 positions' factor words loaded one group ahead
    u64 fx[2][2][4];
    load4(pa0, fx[0][0]);
    load4(pa1, fx[0][1]);
#pragma unroll
    for (int i0 = 0; i0 < 16; i0 += 4) {
      const int cur = (i0 >> 2) & 1;
      if (i0 + 4 < 16) {
        load4(pa0 + i0 + 4, fx[cur ^ 1][0]);
        load4(pa1 + i0 + 4, fx[cur ^ 1][1]);
      }
      const u64 *x0 = fx[cur][0], *x1 = fx[cur][1];
      if (md.prod == 2) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const double a0 = u52_to_dbl(x0[i]), a1 = u52_to_dbl(x1[i]);
          const double d0 = fp_mulmod(a0, a0, __dmul_rn(a0, qinv), q);
          const double h = fp_mulmod(a0, a1, __dmul_rn(a1, qinv), q);
          acc0[i0 + i] = __dadd_rn(acc0[i0 + i], fp_mulmod(d0, Pm, Pmq, q));
          acc1[i0 + i] = __dadd_rn(acc1[i0 + i], fp_mulmod(__dadd_rn(h, h), Pm, Pmq, q));
        }
      } else {
        u64 y0[4], y1[4];
        load4(pb0 + i0, y0);
        load4(pb1 + i0, y1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const double a0 = u52_to_dbl(x0[i]), a1 = u52_to_dbl(x1[i]);
          const double b0 = u52_to_dbl(y0[i]), b1 = u52_to_dbl(y1[i]);
          const double b0q = __dmul_rn(b0, qinv);
          const double d0 = fp_mulmod(a0, b0, b0q, q);
          const double d1 = __dadd_rn(fp_mulmod(a0, b1, __dmul_rn(b1, qinv), q),
                                      fp_mulmod(a1, b0, b0q, q));
          acc0[i0 + i] = __dadd_rn(acc0[i0 + i], fp_mulmod(d0, Pm, Pmq, q));
          acc1[i0 + i] = __dadd_rn(acc1[i0 + i], fp_mulmod(d1, Pm, Pmq, q));
        }
      }
    }
  } else if (ad0) {
    u64 d[16];
    load16(ad0 + ((size_t)l << 16) + sb, d);
#pragma unroll
    for (int i = 0; i < 16; i++) acc0[i] = __dadd_rn(acc0[i], fp_mulmod(u52_to_dbl(d[i]), Pm, Pmq, q));
  }
  if (ad1 && !md.prod) {
    u64 d[16];
    load16(ad1 + ((size_t)l << 16) + sb, d);
#pragma unroll
    for (int i = 0; i < 16; i++) acc1[i] = __dadd_rn(acc1[i], fp_mulmod(u52_to_dbl(d[i]), Pm, Pmq, q));
  }
  // sigma maps the block's tile onto one output tile: the same base for
  // every thread (uniform, so the low pass's twiddles stay scalar loads)
  const u32 tb = (u32)__builtin_amdgcn_readfirstlane(
      (int)(a.ginv == 1 ? sb & ~4095u : autom_index(sb, a.ginv, 16) & ~4095u));
  const int ot = (int)(tb >> 12);
  // the key product's reads of the working tile are done (they read the
  // thread's row, as the identity permutation writes it)
  tile_sync(a.ginv == 1);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const u32 t = a.ginv == 1 ? sb + i : autom_index(sb + i, a.ginv, 16);
    sm[lds16((t >> 8) & 15, t & 255)] = acc0[i];
    acc1t[lds16((t >> 8) & 15, t & 255)] = acc1[i];
  }
  tile_sync(a.ginv == 1);
  double av[16];
#pragma unroll
  for (int k = 0; k < 16; k++) av[k] = sm[lds16(rl, c0 + 16 * k)];
  const double2 *T = tw + ((size_t)p << 16);
  const int row = ot * 16 + rl;
  const u32 e0 = tb + rl * 256 + c0;
  const double pinv = (double)md.pinv[2 * l], pinvq = __dmul_rn(pinv, qinv);
#pragma unroll 1
  for (int comp = 0; comp < 2; comp++) {
    // forward low pass of conv's output tile: round Z on the thread's column,
    // whose LDS writes wait for earlier reads of the working tile
    const u64 *src = batch_ptr(conv, 2 * it + comp) + ((size_t)l << 16) + tb;
    double x[16];
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = as_dbl(src[threadIdx.x + 256 * k]);
    fp_low_round_z(x, T, ot, q);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) sm[lds16(k, threadIdx.x)] = x[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = sm[lds16(rl, c0 + 16 * k)];
    fp_low_round_a(x, T, row, q);
#pragma unroll
    for (int k = 0; k < 16; k++) sm[lds16(rl, c0 + 16 * k)] = x[k];
    row_sync();
#pragma unroll
    for (int j = 0; j < 16; j++) x[j] = sm[lds16(rl, 16 * c0 + j)];
    fp_low_round_b(x, T, row, c0, q);
    row_sync();
#pragma unroll
    for (int j = 0; j < 16; j++) sm[lds16(rl, 16 * c0 + j)] = x[j];
    row_sync();
    u64 *o = batch_ptr(md.out, it) + (comp ? md.out1_off : 0) + ((size_t)l << 16);
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const double acc = comp ? acc1t[lds16(rl, c0 + 16 * k)] : av[k];
      const double v = __dsub_rn(acc, sm[lds16(rl, c0 + 16 * k)]);
      o[e0 + 16 * k] = fp_canon(fp_mulmod(v, pinv, pinvq, q), qinv, q);
    }
  }
}

bool low_key_special_fp(const ckks_context *c) {
  for (int j = 0; j < c->alpha; j++)
    if (!c->prime_fp[c->L + j]) return false;
  return true;
}

static LowKeyArgs low_key_args(ckks_context *c, const u64 *ext, size_t ext_stride,
                               const Batch &own, u64 *acc, size_t acc_stride,
                               const DeviceKey &key, int digits, int E, int q_limbs, u64 ginv,
                               const Batch *own_b, int n_items, bool ext_packed) {
  if (c->logN != 16) throw std::invalid_argument("fused low pass and key product: N = 2^16 only");
  if (digits < 1 || digits > key.digits || q_limbs > c->L || E != q_limbs + c->alpha)
    throw std::invalid_argument("fused low pass and key product: shape");
  LowKeyArgs a{};
  a.ext = ext;
  a.ext_stride = ext_stride;
  a.ext_packed = ext_packed ? 1 : 0;
  a.own = own;
  if (own_b) {
    a.own_b = *own_b;
    a.own_mul = product_mode(own, *own_b, n_items);
  }
  a.acc = acc;
  a.acc_stride = acc_stride;
  a.key = key.data;
  a.ginv = ginv;
  a.digits = digits;
  a.E = E;
  a.q_limbs = q_limbs;
  a.L = c->L;
  a.K = c->K;
  a.ds = c->ds;
  return a;
}

void launch_low_key_moddown(ckks_context *c, const u64 *ext, size_t ext_stride, const Batch &own,
                            int n_items, const DeviceKey &key, int digits, int E, int q_limbs,
                            u64 ginv, const Batch &conv, const u64 *pinv, const u64 *pmod,
                            const Batch &add, u64 add1_off, const Batch &out, u64 out1_off,
                            int out_limbs, const Batch *mul_b, const Batch *own_b,
                            bool ext_packed) {
  if (n_items <= 0) return;
  if (n_items > kMaxBatch) throw std::invalid_argument("fused key product + ModDown: n <= 64");
  if (out_limbs < 1 || out_limbs > q_limbs)
    throw std::invalid_argument("fused key product + ModDown: output limbs");
  LowKeyArgs a = low_key_args(c, ext, ext_stride, own, nullptr, 0, key, digits, E, q_limbs, ginv,
                              own_b, n_items, ext_packed);
  LowMD md{};
  md.pinv = pinv;
  md.add = add;
  md.add1_off = add1_off;
  md.out = out;
  md.out1_off = out1_off;
  if (mul_b) {
    if (!batch_ptr_host(add, 0) || !add1_off)
      throw std::invalid_argument("fused key product + ModDown: product addend needs both factors");
    md.prod = product_mode(add, *mul_b, n_items);
    md.mulb = *mul_b;
  }
  // words per output limb and item: the extended digits, the conversion (2),
  // the addend (2, or the product's factors: 2 or 4) and the outputs (2)
  const double addend = md.prod == 1 ? 4.0 : 2.0;
  KTimer kt(c, "ntt_low_key_moddown",
            8.0 * c->N * ((double)n_items * (digits + 4.0 + addend) * out_limbs +
                          2.0 * digits * out_limbs),
            2.0 * c->N * out_limbs * digits * n_items +
                0.5 * c->N * 12 * 2.0 * n_items * out_limbs +
                (md.prod ? 3.0 * c->N * n_items * out_limbs : 0.0));
  for (int l0 = 0; l0 < out_limbs;) {
    if (!c->prime_fp[l0]) {
      l0++;
      continue;
    }
    int l1 = l0 + 1;
    while (l1 < out_limbs && c->prime_fp[l1]) l1++;
    hipLaunchKernelGGL(k_low_key_md, dim3(n_items * 16 * (l1 - l0)), dim3(TPB), 0, c->stream, a,
                       md, conv, pmod, l0, n_items, c->d_mods, (const double2 *)c->d_tw_fp,
                       (const double2 *)c->d_rinv_fp);
    LAUNCH_CHECK();
    l0 = l1;
  }
}

void launch_ntt_low_key(ckks_context *c, const u64 *ext, size_t ext_stride, const Batch &own,
                        u64 *acc, size_t acc_stride, int n_items, const DeviceKey &key,
                        int digits, int E, int q_limbs, u64 ginv, const Strided *sp,
                        int defer_below, const Batch *own_b, bool ext_packed) {
  KTimer kt(c, "ntt_low_key",
            8.0 * c->N * ((double)n_items * (digits * E + 2.0 * E) + 2.0 * digits * E),
            2.0 * c->N * E * digits * n_items);
  audit_keyswitch(c, n_items, 1, q_limbs, digits, E);
  if (n_items <= 0) return;
  LowKeyArgs a = low_key_args(c, ext, ext_stride, own, acc, acc_stride, key, digits, E, q_limbs,
                              ginv, own_b, n_items, ext_packed);
  if (sp) {
    if (!low_key_special_fp(c)) throw std::invalid_argument("fused special inverse: fp64 special primes only");
    a.sp = sp->base;
    a.sp_stride = sp->stride;
    a.itw = (const double2 *)c->d_itw_fp;
  }
  // runs of limbs whose primes take the same body (q_0 and wide special
  // primes the 64-bit one)
  // (with sp, the special limbs (all fp64) form a run of their own)
  auto fp_limb = [&](int l) { return c->prime_fp[l < q_limbs ? l : c->L + (l - q_limbs)] != 0; };
  // (kind 3: fp64 Q limbs below defer_below, left to launch_low_key_moddown)
  auto kind = [&](int l) {
    return fp_limb(l) ? (sp && l >= q_limbs ? 2 : (l < defer_below ? 3 : 1)) : 0;
  };
  for (int l0 = 0; l0 < E;) {
    const int k = kind(l0);
    int l1 = l0 + 1;
    while (l1 < E && kind(l1) == k) l1++;
    if (k == 3) {
      l0 = l1;
      continue;
    }
    auto kern = k == 2 ? k_ntt16_low_key<true, true>
                : k == 1 ? k_ntt16_low_key<true, false>
                         : k_ntt16_low_key<false, false>;
    hipLaunchKernelGGL(kern, dim3(n_items * 16 * (l1 - l0)), dim3(TPB), 0, c->stream, a, l0, n_items,
                       c->d_mods, c->d_psi, c->d_psi_sh, (const double2 *)c->d_tw_fp,
                       (const double2 *)c->d_rinv_fp);
    LAUNCH_CHECK();
    l0 = l1;
  }
}

// ===========================================================================
// limb-wise arithmetic; grid (N / 256, limbs, polys)
// ===========================================================================

__global__ void k_addsub(const u64 *__restrict__ a, const u64 *__restrict__ b,
                         u64 *__restrict__ out, int logN, int limbs, int q_limbs, int L,
                         const ModQ *__restrict__ mods, int op) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const size_t off = (((size_t)blockIdx.z * limbs + l) << logN) + k;
  const u64 q = mods[prime_of(l, q_limbs, L)].q;
  out[off] = op == 0 ? add_mod(a[off], b[off], q) : sub_mod(a[off], b[off], q);
}

// n pairs at once: grid (N / 256, limbs, polys n), z = item polys + poly
__global__ void k_addsub_many(Batch a, Batch b, Batch out, int logN, int polys, int limbs,
                              int q_limbs, int L, const ModQ *__restrict__ mods, int op) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const int item = blockIdx.z / polys, poly = blockIdx.z - item * polys;
  const size_t off = (((size_t)poly * limbs + l) << logN) + k;
  const u64 q = mods[prime_of(l, q_limbs, L)].q;
  const u64 x = batch_ptr(a, item)[off], y = batch_ptr(b, item)[off];
  batch_ptr(out, item)[off] = op == 0 ? add_mod(x, y, q) : sub_mod(x, y, q);
}

void launch_addsub_many(ckks_context *c, const Batch &a, const Batch &b, const Batch &out, int n,
                        int polys, int limbs, int q_limbs, int op) {
  KTimer kt(c, "limbwise", 8.0 * c->N * 3.0 * n * polys * limbs, (double)c->N * n * polys * limbs);
  if (n < 1 || n > kMaxBatch) throw std::invalid_argument("addsub_many: 1..64 pairs per launch");
  dim3 grid(c->N / TPB, limbs, polys * n);
  hipLaunchKernelGGL(k_addsub_many, grid, dim3(TPB), 0, c->stream, a, b, out, c->logN, polys,
                     limbs, q_limbs, c->L, c->d_mods, op);
  LAUNCH_CHECK();
}

void launch_addsub(ckks_context *c, const u64 *a, const u64 *b, u64 *out, int polys,
                   int limbs, int q_limbs, int op) {
  KTimer kt(c, "limbwise", 8.0 * c->N * 3.0 * polys * limbs, (double)c->N * polys * limbs);
  dim3 grid(c->N / TPB, limbs, polys);
  hipLaunchKernelGGL(k_addsub, grid, dim3(TPB), 0, c->stream, a, b, out, c->logN, limbs,
                     q_limbs, c->L, c->d_mods, op);
  LAUNCH_CHECK();
}

__global__ void k_mul_pt(const u64 *__restrict__ ct, const u64 *__restrict__ pt,
                         u64 *__restrict__ out, int logN, int limbs, int q_limbs, int L,
                         const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const size_t off = (((size_t)blockIdx.z * limbs + l) << logN) + k;
  const ModQ M = mods[prime_of(l, q_limbs, L)];
  out[off] = mul_mod(ct[off], pt[((size_t)l << logN) + k], M);
}

void launch_mul_pt(ckks_context *c, const u64 *ct, const u64 *pt, u64 *out, int polys,
                   int limbs, int q_limbs) {
  audit_pt(c, (double)limbs);
  dim3 grid(c->N / TPB, limbs, polys);
  hipLaunchKernelGGL(k_mul_pt, grid, dim3(TPB), 0, c->stream, ct, pt, out, c->logN, limbs,
                     q_limbs, c->L, c->d_mods);
  LAUNCH_CHECK();
}

// x X^(N/2): evaluation point i gives +I for i < N/2 and -I otherwise, with
// I = psi^(N/2) = psi_br[1]; negative swaps the signs.
__global__ void k_mul_i(const u64 *__restrict__ ct, u64 *__restrict__ out, int logN,
                        int limbs, int q_limbs, int L, const ModQ *__restrict__ mods,
                        const u64 *__restrict__ psi, int negative) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const size_t off = (((size_t)blockIdx.z * limbs + l) << logN) + k;
  const int p = prime_of(l, q_limbs, L);
  const ModQ M = mods[p];
  const u64 I = psi[((size_t)p << logN) + 1];
  const bool upper = k >= (1 << (logN - 1));
  const u64 f = (upper != (negative != 0)) ? M.q - I : I;
  out[off] = mul_mod(ct[off], f, M);
}

void launch_mul_i(ckks_context *c, const u64 *ct, u64 *out, int polys, int limbs,
                  int q_limbs, int negative) {
  dim3 grid(c->N / TPB, limbs, polys);
  hipLaunchKernelGGL(k_mul_i, grid, dim3(TPB), 0, c->stream, ct, out, c->logN, limbs,
                     q_limbs, c->L, c->d_mods, c->d_psi, negative);
  LAUNCH_CHECK();
}

// op 0: add the per-limb constant s[l] to polynomial 0; op 1: multiply every
// polynomial by s[l].  (A constant polynomial is the same value at every NTT
// evaluation point.)
__global__ void k_scalar(const u64 *__restrict__ ct, const u64 *__restrict__ sc,
                         u64 *__restrict__ out, int logN, int limbs, int q_limbs, int L,
                         const ModQ *__restrict__ mods, int op) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const size_t off = (((size_t)blockIdx.z * limbs + l) << logN) + k;
  const ModQ M = mods[prime_of(l, q_limbs, L)];
  u64 v = ct[off];
  if (op == 0)
    out[off] = blockIdx.z == 0 ? add_mod(v, sc[l], M.q) : v;
  else
    out[off] = mul_mod(v, sc[l], M);
}

void launch_scalar(ckks_context *c, const u64 *ct, const u64 *s, u64 *out, int polys,
                   int limbs, int q_limbs, int op) {
  dim3 grid(c->N / TPB, limbs, polys);
  hipLaunchKernelGGL(k_scalar, grid, dim3(TPB), 0, c->stream, ct, s, out, c->logN, limbs,
                     q_limbs, c->L, c->d_mods, op);
  LAUNCH_CHECK();
}

// Tensor product of degree-1 ciphertexts: (a0 b0, a0 b1 + a1 b0, a1 b1).
// grid (N / 256, limbs, items)
// parts: 1 writes d0 = a0 b0 and d1 = a0 b1 + a1 b0, 2 writes d2 = a1 b1 (3
// both), for limb la + blockIdx.y (blockIdx.y < na), else lb + blockIdx.y -
// na; two coefficients per thread.  grid (N / 512, limb count, items)
__device__ __forceinline__ void tensor_word(u64 a0, u64 a1, u64 b0, u64 b1, const ModQ &M,
                                            int parts, u64 &d0, u64 &d1, u64 &d2) {
  if (parts & 1) {
    d0 = mul_mod(a0, b0, M);
    // a0 b1 + a1 b0 < 2 q^2 < q 2^64: one Montgomery fold, then x R
    u64 hi = 0, lo = 0;
    mac_wide(hi, lo, a0, b1);
    mac_wide(hi, lo, a1, b0);
    d1 = to_mont(redc(hi, lo, M.q, M.qinv), M);
  }
  if (parts & 2) d2 = mul_mod(a1, b1, M);
}

__global__ void k_tensor(Batch a, Batch b, Batch out, int logN, int limbs, int la, int na,
                         int lb, int parts, const ModQ *__restrict__ mods) {
  const int k = 2 * (blockIdx.x * TPB + threadIdx.x);
  const int y = blockIdx.y;
  const int l = y < na ? la + y : lb + (y - na);
  const ModQ M = mods[l];
  const size_t P = (size_t)limbs << logN;
  const size_t off = ((size_t)l << logN) + k;
  const u64 *pa = batch_ptr(a, blockIdx.z), *pb = batch_ptr(b, blockIdx.z);
  u64 *po = batch_ptr(out, blockIdx.z);
  using V = ulonglong2;
  const V a1 = *reinterpret_cast<const V *>(pa + P + off);
  const V b1 = *reinterpret_cast<const V *>(pb + P + off);
  V a0{}, b0{};
  if (parts & 1) {
    a0 = *reinterpret_cast<const V *>(pa + off);
    b0 = *reinterpret_cast<const V *>(pb + off);
  }
  u64 d0[2], d1[2], d2[2];
  tensor_word(a0.x, a1.x, b0.x, b1.x, M, parts, d0[0], d1[0], d2[0]);
  tensor_word(a0.y, a1.y, b0.y, b1.y, M, parts, d0[1], d1[1], d2[1]);
  if (parts & 1) {
    *reinterpret_cast<V *>(po + off) = V{d0[0], d0[1]};
    *reinterpret_cast<V *>(po + P + off) = V{d1[0], d1[1]};
  }
  if (parts & 2) *reinterpret_cast<V *>(po + 2 * P + off) = V{d2[0], d2[1]};
}

void launch_tensor(ckks_context *c, const Batch &a, const Batch &b, const Batch &out,
                   int n_items, int limbs, int l_begin, int l_count, int parts, int l_begin2,
                   int l_count2) {
  if (l_count < 0) l_count = limbs - l_begin;
  if (n_items <= 0 || l_count + l_count2 <= 0) return;
  if (parts < 1 || parts > 3 || l_begin < 0 || l_count < 0 || l_begin + l_count > limbs ||
      l_count2 < 0 || (l_count2 > 0 && (l_begin2 < 0 || l_begin2 + l_count2 > limbs)))
    throw std::invalid_argument("tensor: parts or limb ranges");
  const int nl = l_count + l_count2;
  // a squared operand (a = b) is read once
  bool same = true;
  for (int i = 0; i < n_items && same; i++) same = batch_ptr_host(a, i) == batch_ptr_host(b, i);
  // words per coefficient: the reads of a (and b) and the writes of the parts
  const double reads = (parts & 1 ? 2.0 : 1.0) * (same ? 1.0 : 2.0);
  const double writes = (parts & 1 ? 2.0 : 0.0) + (parts & 2 ? 1.0 : 0.0);
  KTimer kt(c, "tensor", 8.0 * c->N * (reads + writes) * n_items * nl,
            ((parts & 1 ? 3.0 : 0.0) + (parts & 2 ? 1.0 : 0.0)) * c->N * n_items * nl);
  dim3 grid(c->N / (2 * TPB), nl, n_items);
  hipLaunchKernelGGL(k_tensor, grid, dim3(TPB), 0, c->stream, a, b, out, c->logN, limbs, l_begin,
                     l_count, l_begin2, parts, c->d_mods);
  LAUNCH_CHECK();
}

// ===========================================================================
// fast basis conversion (ModUp / ModDown); grid (N / 256, items)
//   v_i = [x_i (Q/q_i)^-1]_{q_i};  y_t = REDC(sum_i v_i [(Q/q_i) R]_t)
// centered: v_i is taken in (-q_i/2, q_i/2], i.e. y_t -= cnt Q mod t with
// cnt = #{i : v_i > (q_i - 1)/2}; the conversion error u Q then has zero
// mean (ModDown uses this; a biased u is amplified at the slot whose
// evaluation point is nearest 1).
// Source limbs are contiguous from src; target t is written at limb
// tl = t < t_split ? t : t + t_skip of dst, in prime prime_of(tl).
// Table: [ns] hinv, [ns] hinv shoup, [ns][nd] hmod (Montgomery), [nd] Q mod t.
// ===========================================================================

template <int MS>
__global__ __launch_bounds__(TPB) void k_basis_convert(Batch src, Batch dst, int logN, int ns,
                                                       int nd, const u64 *__restrict__ tab,
                                                       int src_prime0, int t_split, int t_skip,
                                                       int q_limbs, int L, int centered,
                                                       const ModQ *__restrict__ mods) {
  // the constant table is read at wave-uniform addresses (scalar loads)
  const u64 *st = tab;
  const u64 *in = batch_ptr(src, blockIdx.y);
  u64 *out = batch_ptr(dst, blockIdx.y);
  const int k = blockIdx.x * TPB + threadIdx.x;
  u64 v[MS];
  u64 cnt = 0;
#pragma unroll
  for (int i = 0; i < MS; i++) {
    if (i < ns) {
      const u64 qi = mods[src_prime0 + i].q;
      v[i] = shoup_mul(in[((size_t)i << logN) + k], st[i], st[ns + i], qi);
      cnt += (centered && v[i] > (qi - 1) / 2) ? 1 : 0;
    }
  }
  const u64 *hm = st + 2 * ns;
  const u64 *qm = hm + (size_t)ns * nd;
  int t = 0;
  for (; t + 1 < nd; t += 2) {
    const int tl0 = t < t_split ? t : t + t_skip;
    const int tl1 = t + 1 < t_split ? t + 1 : t + 1 + t_skip;
    const ModQ M0 = mods[prime_of(tl0, q_limbs, L)];
    const ModQ M1 = mods[prime_of(tl1, q_limbs, L)];
    u64 h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
    for (int i = 0; i < MS; i++) {
      if (i < ns) {
        mac_wide(h0, l0, v[i], hm[i * nd + t]);
        mac_wide(h1, l1, v[i], hm[i * nd + t + 1]);
      }
    }
    u64 y0 = redc(h0, l0, M0.q, M0.qinv);
    u64 y1 = redc(h1, l1, M1.q, M1.qinv);
    if (cnt) {
      y0 = sub_mod(y0, mul_mod(cnt, qm[t], M0), M0.q);
      y1 = sub_mod(y1, mul_mod(cnt, qm[t + 1], M1), M1.q);
    }
    out[((size_t)tl0 << logN) + k] = y0;
    out[((size_t)tl1 << logN) + k] = y1;
  }
  if (t < nd) {
    const int tl = t < t_split ? t : t + t_skip;
    const ModQ M = mods[prime_of(tl, q_limbs, L)];
    u64 hi = 0, lo = 0;
#pragma unroll
    for (int i = 0; i < MS; i++)
      if (i < ns) mac_wide(hi, lo, v[i], hm[i * nd + t]);
    u64 y = redc(hi, lo, M.q, M.qinv);
    if (cnt) y = sub_mod(y, mul_mod(cnt, qm[t], M), M.q);
    out[((size_t)tl << logN) + k] = y;
  }
}

// fp64 variant for source primes below 2^45: v_i = [x_i hinv_i]_{q_i} by the
// exact fp64 product (centered: v_i in (-q_i/2, q_i/2] directly), and for a
// target t below 2^45 y_t = sum_i [v_i hmod_i]_t as exact fp64 residues, one
// final reduction.  The exact integer sum is the same as the 64-bit kernel's,
// so the output words are identical; a wider target (q_0) keeps the 128-bit
// Montgomery accumulation of k_basis_convert.
template <int MS>
__global__ __launch_bounds__(TPB, 5) void k_basis_convert_fp(
    Batch src, Batch dst, int logN, int ns, int nd, const u64 *__restrict__ tab,
    const double2 *__restrict__ ftab, int src_prime0, int t_split, int t_skip, int q_limbs,
    int L, int centered, int wide0, const ModQ *__restrict__ mods) {
  // the constants are read at wave-uniform addresses straight from global
  // memory (scalar loads into SGPRs) rather than staged in LDS, which cost one
  // broadcast LDS read per product (7 % slower)
  const double2 *sf = ftab;
  const u64 *st = tab;
  const u64 *in = batch_ptr(src, blockIdx.y);
  u64 *out = batch_ptr(dst, blockIdx.y);
  const int k = blockIdx.x * TPB + threadIdx.x;
  // v_i as exact doubles: canonical, or centered when asked (only these stay
  // live across the target loop, to keep the register count and so the
  // occupancy of this latency-bound kernel up)
  double vd[MS];
  // wide first source (q_0 >= 2^45, every target narrow): its value, found
  // with the 64-bit Shoup product, enters as v_0 = va 2^32 + vd[0] with
  // vd[0] in [0, 2^32) and |va| < 2^28, both exact doubles; the products
  // with 2^32 hmod and hmod then stay within fp_mulmod's range
  double va = 0.0;
  if (wide0) {
    const u64 q0 = mods[src_prime0].q;
    const u64 v0 = shoup_mul(in[k], st[0], st[ns], q0);
    const long long sv = (centered && v0 > (q0 - 1) / 2) ? (long long)v0 - (long long)q0
                                                          : (long long)v0;
    va = (double)(sv >> 32);
    vd[0] = (double)(sv & 0xffffffffLL);
  }
#pragma unroll
  for (int i = 0; i < MS; i++) {
    if (i < ns && !(wide0 && i == 0)) {
      const double q = (double)mods[src_prime0 + i].q;
      double v = fp_mulmod(u52_to_dbl(in[((size_t)i << logN) + k]), sf[i].x, sf[i].y, q);
      v = v < 0.0 ? __dadd_rn(v, q) : v;
      v = v >= q ? __dsub_rn(v, q) : v;
      if (centered && v > __dmul_rn(__dsub_rn(q, 1.0), 0.5)) v = __dsub_rn(v, q);
      vd[i] = v;
    }
  }
  const double2 *hf = sf + ns;
  const double2 *hw = hf + (size_t)ns * nd;  // wide0: (2^32 hmod_0 mod t, / t)
  const u64 *hm = st + 2 * ns;
  const u64 *qm = hm + (size_t)ns * nd;
  // wide target (q_0): 128-bit Montgomery accumulation of the canonical v,
  // minus cnt Q for the centered ones
  auto wide = [&](int t) {
    const int tl = t < t_split ? t : t + t_skip;
    const ModQ M = mods[prime_of(tl, q_limbs, L)];
    u64 hi = 0, lo = 0, cnt = 0;
#pragma unroll
    for (int i = 0; i < MS; i++) {
      if (i < ns) {
        const double v = vd[i];
        const u64 vu = dbl_to_u52(v < 0.0 ? __dadd_rn(v, (double)mods[src_prime0 + i].q) : v);
        cnt += v < 0.0 ? 1 : 0;
        mac_wide(hi, lo, vu, hm[i * nd + t]);
      }
    }
    u64 y = redc(hi, lo, M.q, M.qinv);
    if (cnt) y = sub_mod(y, mul_mod(cnt, qm[t], M), M.q);
    out[((size_t)tl << logN) + k] = y;
  };
  auto narrow = [&](int t) {
    const int tl = t < t_split ? t : t + t_skip;
    const double q = (double)mods[prime_of(tl, q_limbs, L)].q;
    double a0 = 0.0, a1 = 0.0;
    if (wide0) a1 = fp_mulmod(va, hw[t].x, hw[t].y, q);
#pragma unroll
    for (int i = 0; i < MS; i += 2) {
      if (i < ns) {
        const double2 h = hf[i * nd + t];
        a0 = __dadd_rn(a0, fp_mulmod(vd[i], h.x, h.y, q));
      }
      if (i + 1 < ns) {
        const double2 h = hf[(i + 1) * nd + t];
        a1 = __dadd_rn(a1, fp_mulmod(vd[i + 1], h.x, h.y, q));
      }
    }
    out[((size_t)tl << logN) + k] = fp_canon(__dadd_rn(a0, a1), 1.0 / q, q);
  };
  int t = 0;
  for (; t + 1 < nd; t += 2) {
    const int tl0 = t < t_split ? t : t + t_skip;
    const int tl1 = t + 1 < t_split ? t + 1 : t + 1 + t_skip;
    const u64 q0u = mods[prime_of(tl0, q_limbs, L)].q, q1u = mods[prime_of(tl1, q_limbs, L)].q;
    if (q0u >= (1ull << 45) || q1u >= (1ull << 45)) {
      if (q0u >= (1ull << 45)) wide(t); else narrow(t);
      if (q1u >= (1ull << 45)) wide(t + 1); else narrow(t + 1);
      continue;
    }
    // two fp64 targets: four independent accumulation chains
    const double q0 = (double)q0u, q1 = (double)q1u;
    double a0 = 0.0, a1 = 0.0, b0 = 0.0, b1 = 0.0;
    if (wide0) {
      a1 = fp_mulmod(va, hw[t].x, hw[t].y, q0);
      b1 = fp_mulmod(va, hw[t + 1].x, hw[t + 1].y, q1);
    }
#pragma unroll
    for (int i = 0; i < MS; i += 2) {
      if (i < ns) {
        const double2 h0 = hf[i * nd + t], h1 = hf[i * nd + t + 1];
        a0 = __dadd_rn(a0, fp_mulmod(vd[i], h0.x, h0.y, q0));
        b0 = __dadd_rn(b0, fp_mulmod(vd[i], h1.x, h1.y, q1));
      }
      if (i + 1 < ns) {
        const double2 h0 = hf[(i + 1) * nd + t], h1 = hf[(i + 1) * nd + t + 1];
        a1 = __dadd_rn(a1, fp_mulmod(vd[i + 1], h0.x, h0.y, q0));
        b1 = __dadd_rn(b1, fp_mulmod(vd[i + 1], h1.x, h1.y, q1));
      }
    }
    out[((size_t)tl0 << logN) + k] = fp_canon(__dadd_rn(a0, a1), 1.0 / q0, q0);
    out[((size_t)tl1 << logN) + k] = fp_canon(__dadd_rn(b0, b1), 1.0 / q1, q1);
  }
  if (t < nd) {
    const int tl = t < t_split ? t : t + t_skip;
    if (mods[prime_of(tl, q_limbs, L)].q >= (1ull << 45)) wide(t); else narrow(t);
  }
}

// int8-MFMA variant (the tensor-core formulation of fast basis conversion:
// residues split into bytes, exact int32 sums on the matrix cores, one
// modular reduction per output).  For coefficients k:
//   A[k][(s, a)] = digit a of v_s(k)   (8 balanced base-256 digits)
//   B[(s, a)][(t, b)] = digit b of M'[(s, a)][t] = [2^(8a) hmod_s]_t
//   C_b[k][t] = sum_(s, a) A B,  |C_b| <= 8 ns 2^14 < 2^21
// so that sum_b C_b 256^b = sum_(s, a) d_a(v_s) 2^(8a) hmod_s = sum_s v_s
// hmod_s (mod t), the exact integer sum of the VALU kernels: the words are
// the same.  One 16x16x32 MFMA covers a quad of sources (lane group g = lane
// / 16 holds source 4 i + g of coefficient lane % 16) for one target group of
// 16 and one digit b; it computes C^T (table operand first), so lane l holds
// targets 16 tg + 4 (l / 16) .. + 3 of coefficient lane % 16 and a store
// writes 16 consecutive coefficients of each of 4 targets.
// Centered (ModDown) v_s are taken in (-q_s/2, q_s/2] as signed values.
// grid (N / (64 R chunks), items): a block stages the table in LDS once and
// converts `chunks` chunks of 4 waves x R x 16 coefficients, loading the next
// chunk's residues while it converts the current one.
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMfmaRows = 2;    // 16-coefficient column tiles per wave and chunk
constexpr int kMfmaChunks = 4;  // chunks of 4 waves x R tiles per block

// Per-target constants staged in LDS after the digit table (words per
// target): the ModQ of the target's prime (0..4), 1/q (5), the output limb
// (6), 2^32/q (7), q as a double (8); with RS also [P]_t, [P]_t / q_t
// (10, 11: the fp64 form), Montgomery [P]_t (12) and [P p]_t (13).
constexpr int kBcTgtWords = 10;
// with RSD dropped primes: per dropped prime j, ([P p_1..p_(j-1)]_t, its
// fp64 quotient), Montgomery [P p_1..p_(j-1)]_t and [P p_1..p_j]_t
__host__ __device__ constexpr int bc_tgt_words(int rsd) { return kBcTgtWords + 4 * rsd; }

// RSD > 0: the relinearise-rescale ModDown by P p_1 .. p_RSD (the dropped
// primes are the last targets, p_(j+1) at target td_j = nd - 1 - j, all in
// one target group; k_bc_down_rescale states the algebra): the dropped
// targets' group runs first; p_1's value y gives the centred lift r_0 =
// [(x - y) P^-1]_(p_1), where x is the dropped limb of X as coefficients
// (source slot ns + RSD - 1 - j for p_(j+1)), broadcast from the lanes that
// hold it; p_2's lift r_1 follows from its own value and r_0 (the rescale
// chain of k_rescale_lift); every target t < T = nd - RSD is written as
// y_t + sum_j r_j [P p_1..p_j]_t - (r_j > p_(j+1) / 2 ? [P p_1..p_(j+1)]_t : 0).
// rs: the relinearise-rescale table of k_bc_down_rescale ([T][RSD]
// Montgomery [P p_1..p_j]_t, [T][RSD] [P p_1..p_(j+1)]_t, [RSD][2] P^-1 mod
// p_(j+1) + Shoup, [RSD][RSD][3] chain constants); rsf: its fp64 part.
template <int R, int NK, int CH, int RSD = 0>
__global__ __launch_bounds__(TPB) void k_basis_convert_mfma(
    Batch src, Batch dst, int logN, int ns, int nd, const u64 *__restrict__ tab,
    const u64 *__restrict__ mtab, int n_tg, int wide_mask, int src_prime0, int t_split,
    int t_skip, int q_limbs, int L, int centered, const ModQ *__restrict__ mods,
    const u64 *__restrict__ rs = nullptr, const double2 *__restrict__ rsf = nullptr) {
  constexpr bool RS = RSD > 0;
  constexpr int RJ = RS ? RSD : 1;
  // the block's table, staged once: [NK][n_tg][8][64] words
  extern __shared__ u64 tb[];
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15, wave = threadIdx.x >> 6;
  const u64 *in = batch_ptr(src, blockIdx.y);
  u64 *out = batch_ptr(dst, blockIdx.y);
  const int kblk = blockIdx.x * CH * 64 * R;
  // per source quad i: source s = 4 i + g, its prime and Shoup constants
  u64 sq[NK], sw[NK], sws[NK];
#pragma unroll
  for (int i = 0; i < NK; i++) {
    const int s = 4 * i + g;
    const bool live = s < ns;
    sq[i] = live ? mods[src_prime0 + s].q : 1;
    sw[i] = live ? tab[s] : 0;
    sws[i] = live ? tab[ns + s] : 0;
  }
  // raw residues of the chunk being loaded (coefficient k + 16 r + col)
  u64 x[R][NK];
  u64 xd[RJ][R];  // RS: the dropped limbs of X at the same coefficients
  auto load = [&](int ch) {
    const int k0 = kblk + ch * 64 * R + wave * 16 * R;
#pragma unroll
    for (int i = 0; i < NK; i++)
#pragma unroll
      for (int r = 0; r < R; r++)
        x[r][i] = 4 * i + g < ns ? in[((size_t)(4 * i + g) << logN) + k0 + 16 * r + col] : 0;
    if constexpr (RS) {
#pragma unroll
      for (int j = 0; j < RSD; j++)
#pragma unroll
        for (int r = 0; r < R; r++)
          xd[j][r] = in[((size_t)(ns + RSD - 1 - j) << logN) + k0 + 16 * r + col];
    }
  };
  // RS: the remaining targets, the dropped targets' group
  const int T = nd - (RS ? RSD : 0), tg_d = (nd - 1) >> 4;
  load(0);
  const int words = NK * n_tg * 512;
  for (int idx = threadIdx.x; idx < words; idx += TPB) tb[idx] = mtab[idx];
  constexpr int TW = bc_tgt_words(RS ? RSD : 0);
  u64 *tgt = tb + words;
  for (int t = threadIdx.x; t < nd; t += TPB) {
    const int tl = t < t_split ? t : t + t_skip;
    const ModQ M = mods[prime_of(tl, q_limbs, L)];
    u64 *w = tgt + (size_t)t * TW;
    w[0] = M.q;
    w[1] = M.qinv;
    w[2] = M.r2;
    w[3] = M.mu;
    w[4] = (u64)M.k | ((u64)M.pad << 32);
    const double q = (double)M.q, qinv = 1.0 / q;
    w[5] = dbl_bits(qinv);
    w[6] = (u64)tl;
    w[7] = dbl_bits(4294967296.0 * qinv);
    w[8] = dbl_bits(q);
    if constexpr (RS) {
      if (t < T) {
#pragma unroll
        for (int j = 0; j < RSD; j++) {
          const size_t tj = (size_t)t * RSD + j;
          w[10 + 4 * j] = dbl_bits(rsf[tj].x);
          w[11 + 4 * j] = dbl_bits(rsf[tj].y);
          w[12 + 4 * j] = rs[tj];
          w[13 + 4 * j] = rs[(size_t)T * RSD + tj];
        }
      }
    }
  }
  // RS: the dropped primes' lift constants (uniform): P^-1 mod p_(j+1) and
  // its Shoup constant, then the chain's [p_2] mod p_1... (k_bc_down_rescale)
  const u64 *rpinv = RS ? rs + 2 * (size_t)T * RSD : nullptr;
  const u64 *rchain = RS ? rpinv + 2 * RSD : nullptr;
  __syncthreads();
  const int quad = n_tg * 512;
  for (int ch = 0; ch < CH; ch++) {
    const int k0 = kblk + ch * 64 * R + wave * 16 * R;
    // the data operand: digits of v_s at coefficient k0 + 16 r + col
    long a[R][NK];
#pragma unroll
    for (int i = 0; i < NK; i++)
#pragma unroll
      for (int r = 0; r < R; r++) {
        u64 v = shoup_mul(x[r][i], sw[i], sws[i], sq[i]);
        if (centered && v > (sq[i] - 1) / 2) v -= sq[i];  // two's complement of v - q
        a[r][i] = (long)((v + 0x8080808080808080ull) ^ 0x8080808080808080ull);
      }
    u64 xdc[RJ][R];  // RS: this chunk's dropped-limb words
    if constexpr (RS) {
#pragma unroll
      for (int j = 0; j < RSD; j++)
#pragma unroll
        for (int r = 0; r < R; r++) xdc[j][r] = xd[j][r];
    }
    if (ch + 1 < CH) load(ch + 1);  // in flight during this chunk
    u64 rv[RJ][R];
    bool rneg[RJ][R];
    for (int tt = 0; tt < n_tg; tt++) {
      // RS: the dropped target's group first
      const int tg = RS ? (tt == 0 ? tg_d : (tt <= tg_d ? tt - 1 : tt)) : tt;
      const bool wide = (wide_mask >> tg) & 1;
      const u64 *mt = tb + tg * 512 + lane;
      // C_b (rows: targets 16 tg + 4 g + e, columns: coefficients) and
      // sum_b C_b 256^b = lo + hi 2^32 with lo = sum_(b<4) C_b 256^b, hi =
      // sum_(b>=4) C_b 256^(b-4).  Digits go in pairs (b, b + 1): two
      // independent MFMA chains per tile, then D = C_b + 256 C_(b+1) in
      // int32 (|D| < 2^29.1), folded into lo / hi as exact fp64 sums (|lo|,
      // |hi| < 2^45.01); only one pair's accumulators are live at a time
      double lo[R][4], hi[R][4];
#pragma unroll
      for (int pr = 0; pr < 4; pr++) {
        if (pr >= 3 && !wide) continue;  // digits 6, 7 of a narrow table are 0
        v4i c0[R], c1[R];
#pragma unroll
        for (int r = 0; r < R; r++) c0[r] = c1[r] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < NK; i++) {
          const long b0 = (long)mt[i * quad + (2 * pr) * 64];
          const long b1 = (long)mt[i * quad + (2 * pr + 1) * 64];
#pragma unroll
          for (int r = 0; r < R; r++) {
            c0[r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(b0, a[r][i], c0[r], 0, 0, 0);
            c1[r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(b1, a[r][i], c1[r], 0, 0, 0);
          }
        }
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const double d = (double)(c0[r][e] + 256 * c1[r][e]);
            if (pr == 0) lo[r][e] = d;
            else if (pr == 1) lo[r][e] = __fma_rn(d, 65536.0, lo[r][e]);
            else if (pr == 2) hi[r][e] = d;
            else hi[r][e] = __fma_rn(d, 65536.0, hi[r][e]);
          }
      }
      if constexpr (RS) {
        if (tt == 0) {
          // each dropped target's value in its lanes, the lift from it (and
          // the earlier lifts), then the lift to every lane of the same
          // coefficient column
#pragma unroll
          for (int j = 0; j < RSD; j++) {
            const int td = nd - 1 - j, g_d = (td & 15) >> 2, e_d = td & 3;
            const u64 *wd = tgt + (size_t)td * TW;
            ModQ Mj;
            Mj.q = wd[0];
            Mj.qinv = wd[1];
            Mj.r2 = wd[2];
            Mj.mu = wd[3];
            Mj.k = (u32)wd[4];
            Mj.pad = (u32)(wd[4] >> 32);
            const u64 qd = Mj.q;
            const double q = as_dbl(wd[8]), qinv = as_dbl(wd[5]), w32q = as_dbl(wd[7]);
            const u64 pinv = rpinv[2 * j], pinvs = rpinv[2 * j + 1];
#pragma unroll
            for (int r = 0; r < R; r++) {
              const double tq = fp_rint(__dmul_rn(hi[r][e_d], w32q));
              const double y =
                  __dadd_rn(__fma_rn(-tq, q, __dmul_rn(hi[r][e_d], 4294967296.0)), lo[r][e_d]);
              u64 u = shoup_mul(sub_mod(xdc[j][r], fp_canon(y, qinv, q), qd), pinv, pinvs, qd);
#pragma unroll
              for (int m = 0; m < j; m++) {
                const u64 *cm = rchain + 3 * ((size_t)j * RSD + m);
                u64 rm = barrett(0, rv[m][r], Mj);
                if (rneg[m][r]) rm = sub_mod(rm, cm[0], qd);
                u = shoup_mul(sub_mod(u, rm, qd), cm[1], cm[2], qd);
              }
              const u64 ub = (u64)__shfl((long long)u, 16 * g_d + col);
              rv[j][r] = ub;
              rneg[j][r] = ub > (qd - 1) / 2;
            }
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = 16 * tg + 4 * g + e;
        if (t >= T) continue;
        const u64 *w = tgt + (size_t)t * TW;
        u64 *o = out + ((size_t)w[6] << logN) + k0 + col;
        if (w[0] < kFpPrimeBound) {
          // y = hi 2^32 + lo: hi 2^32 is an exact double, the quotient by
          // round(hi 2^32 / q) leaves an exact residue, one reduction after
          const double q = as_dbl(w[8]), qinv = as_dbl(w[5]), w32q = as_dbl(w[7]);
#pragma unroll
          for (int r = 0; r < R; r++) {
            const double tq = fp_rint(__dmul_rn(hi[r][e], w32q));
            double y =
                __dadd_rn(__fma_rn(-tq, q, __dmul_rn(hi[r][e], 4294967296.0)), lo[r][e]);
            if constexpr (RS) {
              // |y| < 2q; each lift's product (< 1.5 q) and [P p..]_t (< q)
              // keep it below 2^50
#pragma unroll
              for (int j = 0; j < RSD; j++) {
                y = __dadd_rn(y, fp_mulmod(u52_to_dbl(rv[j][r]), as_dbl(w[10 + 4 * j]),
                                           as_dbl(w[11 + 4 * j]), q));
                if (rneg[j][r]) y = __dsub_rn(y, u52_to_dbl(w[13 + 4 * j]));
              }
            }
            o[16 * r] = fp_canon(y, qinv, q);
          }
        } else {
          // q > 2^45 > |hi|, |lo|: one correction each, then the 64-bit product
          ModQ M;
          M.q = w[0];
          M.qinv = w[1];
          M.r2 = w[2];
          M.mu = w[3];
          M.k = (u32)w[4];
          M.pad = (u32)(w[4] >> 32);
#pragma unroll
          for (int r = 0; r < R; r++) {
            const long long hv = dbl_to_i51(hi[r][e]), lv = dbl_to_i51(lo[r][e]);
            const u64 h = hv < 0 ? (u64)(hv + (long long)M.q) : (u64)hv;
            const u64 l = lv < 0 ? (u64)(lv + (long long)M.q) : (u64)lv;
            u64 y = add_mod(mul_mod(h, 1ull << 32, M), l, M.q);
            if constexpr (RS) {
#pragma unroll
              for (int j = 0; j < RSD; j++) {
                // Montgomery form: the REDC of the product is r_j [P p..]_t
                const u64 pmM = w[12 + 4 * j], rj = rv[j][r];
                y = add_mod(y, redc(__umul64hi(rj, pmM), rj * pmM, M.q, M.qinv), M.q);
                if (rneg[j][r]) y = sub_mod(y, w[13 + 4 * j], M.q);
              }
            }
            o[16 * r] = y;
          }
        }
      }
    }
  }
}

void launch_basis_convert(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                          const BCTable &t, int src_prime0, int t_split, int t_skip,
                          int q_limbs, bool centered) {
  KTimer kt(c, "basis_convert", 8.0 * c->N * n_items * (t.ns + t.nd),
            (double)c->N * n_items * t.ns * t.nd);
  // the table is staged in LDS: tables above 64 KiB (digits of more than
  // 12 primes into more than 48 targets) take the VALU kernels
  if (c->bc_mfma && t.mf && (size_t)t.n_k * t.n_tg * 512 * sizeof(u64) <= 65536) {
    auto kern = t.n_k == 1   ? k_basis_convert_mfma<kMfmaRows, 1, kMfmaChunks>
                : t.n_k == 2 ? k_basis_convert_mfma<kMfmaRows, 2, kMfmaChunks>
                : t.n_k == 3 ? k_basis_convert_mfma<kMfmaRows, 3, kMfmaChunks>
                             : k_basis_convert_mfma<kMfmaRows, 4, kMfmaChunks>;
    const size_t lds =
        sizeof(u64) * ((size_t)t.n_k * t.n_tg * 512 + (size_t)t.nd * kBcTgtWords);
    hipLaunchKernelGGL(kern, dim3(c->N / (64 * kMfmaRows * kMfmaChunks), n_items), dim3(TPB),
                       lds, c->stream,
                       src, dst, c->logN, t.ns, t.nd, t.d, t.mf, t.n_tg, t.wide_mask,
                       src_prime0, t_split, t_skip, q_limbs, c->L, centered ? 1 : 0, c->d_mods,
                       (const u64 *)nullptr, (const double2 *)nullptr);
    LAUNCH_CHECK();
    return;
  }
  dim3 grid(c->N / TPB, n_items);
  // one register per source: a 12-source instance for digits (and P) of at
  // most 12 primes keeps the register count down
  const bool s12 = t.ns <= 12;
  if (t.fd) {
    hipLaunchKernelGGL(s12 ? k_basis_convert_fp<12> : k_basis_convert_fp<kMaxDigitSize>, grid,
                       dim3(TPB), 0, c->stream, src, dst, c->logN, t.ns, t.nd, t.d,
                       (const double2 *)t.fd, src_prime0, t_split, t_skip, q_limbs, c->L,
                       centered ? 1 : 0, t.wide0, c->d_mods);
  } else {
    hipLaunchKernelGGL(s12 ? k_basis_convert<12> : k_basis_convert<kMaxDigitSize>, grid,
                       dim3(TPB), 0, c->stream, src, dst, c->logN, t.ns, t.nd, t.d, src_prime0,
                       t_split, t_skip, q_limbs, c->L, centered ? 1 : 0, c->d_mods);
  }
  LAUNCH_CHECK();
}

// ===========================================================================
// N = 2^16: fast base conversion between the two halves of the NTTs,
// resident in registers (the ModUp of one digit, and the ModDown of the
// special limbs).  Block (64 columns, item): wave w holds columns
// 64 blockIdx.x + 16 w + col of the 16 x 4096 array; lane (g, col) takes,
// for each source quad i, source s = 4 i + g:
//   1. the inverse high pass (bits 12..15) of its 16-word column, read from
//      what the inverse low pass left (raw double bits / lazy words);
//   2. v_s = [x N^-1 Qhat_s^-1]_(q_s) (centered for the ModDown) as 8
//      balanced bytes, the data operand of k_basis_convert_mfma for
//      coefficient (row r, column col): the MFMA's 16 coefficients are the
//      wave's 16 columns of one row;
//   3. per target group and row, the int8 MFMAs and the exact fp64 fold of
//      k_basis_convert_mfma; the table (BCTable::mt) orders each group's
//      targets so that lane (g, col) holds targets 16 tg + 4 e + g of its
//      column at all 16 rows, and a group's rows e past its last target are
//      skipped by the whole wave;
//   4. the forward high pass (bits 15..12) of each of those columns, stored
//      as the low pass expects it (raw double bits / lazy words), or for
//      the fused key products (flag 8) fp64 targets in the packed form:
//      the centered residue's 32 low bits, then its 16 high bits.
// The converted limbs never exist in coefficient form in HBM: the kernel
// reads each source word and writes each target word once.  The same words
// as the inverse high pass, k_basis_convert_mfma and the forward high pass
// in a row (the same exact integers, canonical in between).
// ===========================================================================
struct H4Tabs {
  const u64 *psi, *psi_sh, *ipsi, *ipsi_sh, *ninv;
  const double2 *tw, *itw, *ninv_fp;
};

// RSD > 0: the relinearise-rescale ModDown by P p_1 .. p_RSD
// (k_basis_convert_mfma's RS form): the dropped primes are the last targets,
// p_(j+1) at target nd - 1 - j, all in one group, which runs first; its
// lanes form each lift r_j from the dropped limb of X (source slot
// ns + RSD - 1 - j, coefficient form) and leave it in LDS for every column
// and row; each kept target t < nd - RSD then adds
// r_j [P p_1..p_j]_t - (r_j > p_(j+1) / 2 ? [P p_1..p_(j+1)]_t : 0) before
// its forward high pass.  rs / rsf: launch_bc_down_rescale's tables.
template <int NK, int RSD = 0>
__global__ __launch_bounds__(TPB, 2) void k_convert_h4(
    Batch src, Batch dst, int ns, int nd, const u64 *__restrict__ tab,
    const u64 *__restrict__ mtab, int n_tg, int wide_mask, int src_prime0, int t_split,
    int t_skip, int q_limbs, int L, int flags, const ModQ *__restrict__ mods, H4Tabs nt,
    const u64 *__restrict__ rs, const double2 *__restrict__ rsf) {
  constexpr bool RS = RSD > 0;
  constexpr int TW = bc_tgt_words(RSD);
  const int T = nd - RSD;
  // flags: 1 centered (ModDown); 2 / 4: the high passes of sources / targets
  // of 2^45 or more run outside the kernel (when such primes share a launch
  // with fp64 ones, whose lanes would wait on their 64-bit butterflies);
  // 8: fp64 targets stored packed (LowKeyArgs::ext_packed), 3/4 of the bytes
  const bool centered = flags & 1, wide_src_out = flags & 2, wide_tgt_out = flags & 4;
  const bool packed = !RS && (flags & 8);  // ModUp only (never with the lifts)
  extern __shared__ u64 tb[];
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15, wave = threadIdx.x >> 6;
  const int cc = blockIdx.x * 64 + wave * 16 + col;
  const u64 *in = batch_ptr(src, blockIdx.y) + cc;
  u64 *out = batch_ptr(dst, blockIdx.y) + cc;
  // the table and per-target constants (k_basis_convert_mfma's words, and
  // the target's prime index at word 9)
  const int words = NK * n_tg * 512;
  for (int idx = threadIdx.x; idx < words; idx += TPB) tb[idx] = mtab[idx];
  u64 *tgt = tb + words;
  for (int t = threadIdx.x; t < nd; t += TPB) {
    const int tl = t < t_split ? t : t + t_skip;
    const int pt = prime_of(tl, q_limbs, L);
    const ModQ M = mods[pt];
    u64 *w = tgt + (size_t)t * TW;
    w[0] = M.q;
    w[1] = M.qinv;
    w[2] = M.r2;
    w[3] = M.mu;
    w[4] = (u64)M.k | ((u64)M.pad << 32);
    const double q = (double)M.q, qinv = 1.0 / q;
    w[5] = dbl_bits(qinv);
    w[6] = (u64)tl;
    w[7] = dbl_bits(4294967296.0 * qinv);
    w[8] = dbl_bits(q);
    w[9] = (u64)pt;
    if constexpr (RS) {
      if (t < T) {
#pragma unroll
        for (int j = 0; j < RSD; j++) {
          const size_t tj = (size_t)t * RSD + j;
          w[10 + 4 * j] = dbl_bits(rsf[tj].x);
          w[11 + 4 * j] = dbl_bits(rsf[tj].y);
          w[12 + 4 * j] = rs[tj];
          w[13 + 4 * j] = rs[(size_t)T * RSD + tj];
        }
      }
    }
  }
  // the high passes' 15 twiddles of every target's prime (forward) and every
  // source's prime (inverse), 32 words each: fp64 primes as 16 (w, w / q)
  // pairs, others as [16] psi_br and [16] Shoup constants; entry 0 is unused
  // and word 0 holds q.  Each lane group works on its own primes, so these
  // would otherwise be per-lane global loads.
  u64 *ttw = tgt + (size_t)nd * TW, *stw = ttw + (size_t)nd * 32;
  // RS: the lifts, [RSD][16 rows][64 columns of the block]
  u64 *lift = stw + (size_t)ns * 32;
  for (int idx = threadIdx.x; idx < (nd + ns) * 16; idx += TPB) {
    const int t = idx >> 4, j = idx & 15;
    const bool src_side = t >= nd;
    int pt;
    if (src_side) {
      pt = src_prime0 + (t - nd);
    } else {
      const int tl = t < t_split ? t : t + t_skip;
      pt = prime_of(tl, q_limbs, L);
    }
    u64 *w = src_side ? stw + (size_t)(t - nd) * 32 : ttw + (size_t)t * 32;
    const u64 qu = mods[pt].q;
    if (j == 0) {
      w[0] = qu;
      continue;
    }
    const size_t o = ((size_t)pt << 16) + j;
    if (qu < kFpPrimeBound) {
      const double2 v = src_side ? nt.itw[o] : nt.tw[o];
      w[2 * j] = dbl_bits(v.x);
      w[2 * j + 1] = dbl_bits(v.y);
    } else {
      w[j] = src_side ? nt.ipsi[o] : nt.psi[o];
      w[16 + j] = src_side ? nt.ipsi_sh[o] : nt.psi_sh[o];
    }
  }
  __syncthreads();
  // 1-2: the sources of this lane group
  long a[NK][16];
#pragma unroll
  for (int i = 0; i < NK; i++) {
    const int s = 4 * i + g;
    if (s < ns) {
      const u64 *sw0 = stw + (size_t)s * 32;
      const u64 qu = sw0[0];
      const u64 *ps = in + ((size_t)s << 16);
      u64 x[16];
#pragma unroll
      for (int r = 0; r < 16; r++) x[r] = ps[4096 * r];
      // v = x [N^-1 hinv]_q: the inverse pass's x N^-1 folded into the
      // conversion's first product
      if (qu < kFpPrimeBound) {
        const double q = (double)qu, qinv = 1.0 / q;
        const double2 wn = reinterpret_cast<const double2 *>(tab + 2 * ns)[s];
        double xd[16];
#pragma unroll
        for (int r = 0; r < 16; r++) xd[r] = as_dbl(x[r]);
        fp_high_inv_stages(xd, reinterpret_cast<const double2 *>(sw0), q, qinv);
        // fp_reduce of the product (in [-q, q]) leaves [-(q+1)/2, (q+1)/2]; a
        // second one gives the centered representative, |v| <= (q-1)/2, and
        // v < 0 ? v + q : v the canonical one.  The word of 1.5 2^52 + v is
        // that of 1.5 2^52 plus v, so one 64-bit add gives the bytes' offset
        // form of v's two's complement.
        constexpr u64 kBal = 0x8080808080808080ull - 0x4338000000000000ull;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          double v = fp_reduce(fp_mulmod(xd[r], wn.x, wn.y, q), qinv, q);
          v = centered ? fp_reduce(v, qinv, q) : (v < 0.0 ? __dadd_rn(v, q) : v);
          a[i][r] = (long)((dbl_bits(__dadd_rn(v, FP_ROUND_C)) + kBal) ^ 0x8080808080808080ull);
        }
      } else {
        // a prime of 2^45 or more: the inverse high pass here, or (flag 2)
        // before the kernel (with the x N^-1, x canonical)
        u64 hw = tab[4 * ns + s], hws = tab[5 * ns + s];
        if (!wide_src_out) {
          u64_high_inv_stages(x, sw0, sw0 + 16, qu, 2 * qu);
          hw = tab[s];
          hws = tab[ns + s];
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
          u64 v = shoup_mul(x[r], hw, hws, qu);
          if (centered && v > (qu - 1) / 2) v -= qu;  // two's complement of v - q
          a[i][r] = (long)((v + 0x8080808080808080ull) ^ 0x8080808080808080ull);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) a[i][r] = 0;
    }
  }
  __syncthreads();
  const int quad = n_tg * 512;
  // 3-4 run in passes (tg, h): target group tg, rows e = 2 h, 2 h + 1 of its
  // MFMA output (targets 16 tg + 4 e + g), so that a lane keeps two target
  // columns (y) beside its sources (a) in registers; each pass recomputes
  // the group's MFMAs.  RS: the pass of the dropped targets goes first.
  const int first = RS ? ((nd - 1) >> 3) : 0;  // = 2 tg + h of the last target
  for (int pp = 0; pp < 2 * n_tg; pp++) {
    const int pq = RS ? (pp == 0 ? first : (pp <= first ? pp - 1 : pp)) : pp;
    const int tg = pq >> 1, h = pq & 1;
    if (16 * tg + 8 * h >= nd) continue;  // no target in this pass
    const bool wide = (wide_mask >> tg) & 1;
    // lane m + 16 k supplies row m of the table operand; reading row
    // (m & 12) | ((m + 2 h) & 3) instead puts targets 16 tg + 4 (2 h + ee) + g
    // at accumulator entries ee = 0, 1 of lane group g (static indices)
    const u64 *mt = tb + tg * 512 + ((lane & ~3) | ((lane + 2 * h) & 3));
    // 3: values of targets 16 tg + 4 (2 h + ee) + g at rows 0..15 (for
    // targets below 2^45 exact doubles congruent to the residue, as bits;
    // words otherwise).  The lane's two targets' constants are read once per
    // pass; lanes without a target (past nd) compute unused values on the
    // fp64 path.
    bool fpt[2];
    double tqd[2], tw32[2];
#pragma unroll
    for (int ee = 0; ee < 2; ee++) {
      const int t = 16 * tg + 4 * (2 * h + ee) + g;
      const bool tv = t < nd;
      const u64 *w = tgt + (size_t)(tv ? t : 0) * TW;
      fpt[ee] = !tv || w[0] < kFpPrimeBound;
      tqd[ee] = as_dbl(w[8]);
      tw32[ee] = as_dbl(w[7]);
    }
    u64 y[2][16];
    {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        double lo[2], hi[2];
#pragma unroll
        for (int pr = 0; pr < 4; pr++) {
          if (pr >= 3 && !wide) continue;  // digits 6, 7 of a narrow table are 0
          v4i c0 = v4i{0, 0, 0, 0}, c1 = v4i{0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < NK; i++) {
            const long b0 = (long)mt[i * quad + (2 * pr) * 64];
            const long b1 = (long)mt[i * quad + (2 * pr + 1) * 64];
            c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b0, a[i][r], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b1, a[i][r], c1, 0, 0, 0);
          }
#pragma unroll
          for (int ee = 0; ee < 2; ee++) {
            const double d = (double)(c0[ee] + 256 * c1[ee]);
            if (pr == 0) lo[ee] = d;
            else if (pr == 1) lo[ee] = __fma_rn(d, 65536.0, lo[ee]);
            else if (pr == 2) hi[ee] = d;
            else hi[ee] = __fma_rn(d, 65536.0, hi[ee]);
          }
        }
#pragma unroll
        for (int ee = 0; ee < 2; ee++) {
          // fp64 targets: |y| < q / 2 + 2^45.1 < 2^46, which the forward
          // passes take as it is (|x| grows by at most q per stage, 16
          // stages, below 2^50)
          const double tq = fp_rint(__dmul_rn(hi[ee], tw32[ee]));
          u64 yv = dbl_bits(
              __dadd_rn(__fma_rn(-tq, tqd[ee], __dmul_rn(hi[ee], 4294967296.0)), lo[ee]));
          if (!fpt[ee]) {
            // a prime q of 2^45 or more: V = hi 2^32 + lo (|hi|, |lo| <
            // 2^45) less t q, t = round(V / q) from fp64 (|V / q| < 2^32, so
            // the error is below 2^-19), is exact in 64-bit two's complement
            // and lies in (-q, q); one conditional q makes it canonical
            const u64 *w = tgt + (size_t)(16 * tg + 4 * (2 * h + ee) + g) * TW;
            const u64 qw = w[0];
            const double tv = fp_rint(__fma_rn(hi[ee], as_dbl(w[7]), __dmul_rn(lo[ee], as_dbl(w[5]))));
            const u64 v = ((u64)dbl_to_i51(hi[ee]) << 32) + (u64)dbl_to_i51(lo[ee]) -
                          (u64)dbl_to_i51(tv) * qw;
            yv = (long long)v < 0 ? v + qw : v;
          }
          y[ee][r] = yv;
        }
      }
    }
    if constexpr (RS) {
      if (pp == 0) {
        // the lifts, in the lanes of each dropped target (fp64 primes; the
        // transposed order puts target t in lane group t % 4, row t % 16 / 4)
        const u64 *rpinv = rs + 2 * (size_t)T * RSD;
        const u64 *rchain = rpinv + 2 * RSD;
#pragma unroll
        for (int j = 0; j < RSD; j++) {
          const int td = nd - 1 - j, ee_d = ((td & 15) >> 2) & 1;
          if (g == (td & 3)) {
            const u64 *wd = tgt + (size_t)td * TW;
            ModQ Mj;
            Mj.q = wd[0];
            Mj.qinv = wd[1];
            Mj.r2 = wd[2];
            Mj.mu = wd[3];
            Mj.k = (u32)wd[4];
            Mj.pad = (u32)(wd[4] >> 32);
            const u64 qd = Mj.q;
            const double q = as_dbl(wd[8]), qinv = as_dbl(wd[5]);
            const u64 pinv = rpinv[2 * j], pinvs = rpinv[2 * j + 1];
            const u64 *xs = in + ((size_t)(ns + RSD - 1 - j) << 16);
#pragma unroll
            for (int r = 0; r < 16; r++) {
              // a mask select, so that y keeps static indices
              const u64 msk = 0ull - (u64)ee_d;
              const u64 yd = fp_canon(as_dbl((y[0][r] & ~msk) | (y[1][r] & msk)), qinv, q);
              u64 u = shoup_mul(sub_mod(xs[4096 * r], yd, qd), pinv, pinvs, qd);
#pragma unroll
              for (int m = 0; m < j; m++) {
                const u64 *cm = rchain + 3 * ((size_t)j * RSD + m);
                const u64 rmv = lift[(m * 16 + r) * 64 + wave * 16 + col];
                const u64 qm = tgt[(size_t)(nd - 1 - m) * TW];
                u64 rm = barrett(0, rmv, Mj);
                if (rmv > (qm - 1) / 2) rm = sub_mod(rm, cm[0], qd);
                u = shoup_mul(sub_mod(u, rm, qd), cm[1], cm[2], qd);
              }
              lift[(j * 16 + r) * 64 + wave * 16 + col] = u;
            }
          }
          __syncthreads();
        }
      }
      // every kept target adds its lifts
#pragma unroll
      for (int ee = 0; ee < 2; ee++) {
        const int t = 16 * tg + 4 * (2 * h + ee) + g;
        if (16 * tg + 4 * (2 * h + ee) >= nd || t >= T) continue;
        const u64 *w = tgt + (size_t)t * TW;
#pragma unroll
        for (int j = 0; j < RSD; j++) {
          const u64 qj = tgt[(size_t)(nd - 1 - j) * TW];
          if (w[0] < kFpPrimeBound) {
            const double q = as_dbl(w[8]);
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const u64 rj = lift[(j * 16 + r) * 64 + wave * 16 + col];
              double yv = __dadd_rn(as_dbl(y[ee][r]), fp_mulmod(u52_to_dbl(rj), as_dbl(w[10 + 4 * j]),
                                                                  as_dbl(w[11 + 4 * j]), q));
              if (rj > (qj - 1) / 2) yv = __dsub_rn(yv, u52_to_dbl(w[13 + 4 * j]));
              y[ee][r] = dbl_bits(yv);
            }
          } else {
            const u64 qu = w[0], qinvm = w[1], pmM = w[12 + 4 * j];
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const u64 rj = lift[(j * 16 + r) * 64 + wave * 16 + col];
              u64 yw = add_mod(y[ee][r], redc(__umul64hi(rj, pmM), rj * pmM, qu, qinvm), qu);
              if (rj > (qj - 1) / 2) yw = sub_mod(yw, w[13 + 4 * j], qu);
              y[ee][r] = yw;
            }
          }
        }
      }
    }
    // 4: forward high pass of each target column, stored for the low pass
#pragma unroll
    for (int ee = 0; ee < 2; ee++) {
      const int t = 16 * tg + 4 * (2 * h + ee) + g;
      if (16 * tg + 4 * (2 * h + ee) >= nd || t >= T) continue;
      const u64 *w = tgt + (size_t)t * TW;
      const u64 *tw0 = ttw + (size_t)t * 32;
      u64 *po = out + ((size_t)w[6] << 16);
      if (w[0] < kFpPrimeBound) {
        double xd[16];
#pragma unroll
        for (int r = 0; r < 16; r++) xd[r] = as_dbl(y[ee][r]);
        fp_high_fwd(xd, reinterpret_cast<const double2 *>(tw0), as_dbl(w[8]));
        if (packed) {
          // the centered residue v (|v| <= q / 2 + 1 < 2^44) as its 32 low
          // bits (u32 plane) and 16 high bits (i16 plane after it)
          u32 *plo = reinterpret_cast<u32 *>(po - cc);
          short *phi = reinterpret_cast<short *>(plo + 65536) + cc;
          plo += cc;
          const double q = as_dbl(w[8]), qinv = as_dbl(w[5]);
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const long long v = dbl_to_i51(fp_reduce(xd[r], qinv, q));
            plo[4096 * r] = (u32)v;
            phi[4096 * r] = (short)(v >> 32);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; r++) po[4096 * r] = dbl_bits(xd[r]);
        }
      } else {
        // a prime of 2^45 or more: the forward high pass here, or (flag 4)
        // stored canonical for the launch after the kernel
        if (!wide_tgt_out) {
          const u64 qu = w[0];
          u64_high_fwd(y[ee], tw0, tw0 + 16, qu, 2 * qu);
        }
#pragma unroll
        for (int r = 0; r < 16; r++) po[4096 * r] = y[ee][r];
      }
    }
  }
}

// Where a launch mixes primes of 2^45 or more with fp64 ones, k_convert_h4
// leaves the wide primes' high passes (whose 64-bit butterflies would run
// beside the fp64 ones of the other lane groups of a wave) to these
// launches: the inverse high pass of such sources before the kernel, in
// place (source s of prime src_prime0 + s sits at item limb s; the batch is
// shifted so that the pass's limb index names that prime), and the forward
// high pass of such targets after it (target t at output limb
// t < t_split ? t : t + t_skip).  Each returns the kernel's flag (2, 4) when
// the launch is mixed, else 0 and runs nothing: a launch of wide primes only
// keeps its high passes inside.
static int h4_wide_sources(ckks_context *c, const Batch &src, int n_items, int ns,
                           int src_prime0, int q_limbs) {
  int wide = 0;
  for (int s = 0; s < ns; s++) wide += c->prime_fp[src_prime0 + s] ? 0 : 1;
  if (wide == 0 || wide == ns) return 0;
  const int off = src_prime0 < c->L ? src_prime0 : q_limbs + (src_prime0 - c->L);
  for (int s0 = 0; s0 < ns;) {
    if (c->prime_fp[src_prime0 + s0]) {
      s0++;
      continue;
    }
    int s1 = s0 + 1;
    while (s1 < ns && !c->prime_fp[src_prime0 + s1]) s1++;
    Batch b = src;
    const size_t back = (size_t)off << 16;
    if (b.base) b.base -= back;
    else
      for (int i = 0; i < n_items; i++) b.p[i] -= back;
    launch_inv_high16(c, b, n_items, off + s0, s1 - s0, q_limbs);
    s0 = s1;
  }
  return 2;
}

// run: false asks only whether the launch is mixed (the flag), true runs
// the passes
static int h4_wide_targets(ckks_context *c, const Batch &dst, int n_items, int n_out,
                           int t_split, int t_skip, int q_limbs, bool run) {
  auto limb = [&](int t) { return t < t_split ? t : t + t_skip; };
  auto wide = [&](int t) {
    const int tl = limb(t);
    return !c->prime_fp[tl < q_limbs ? tl : c->L + (tl - q_limbs)];
  };
  int n_wide = 0;
  for (int t = 0; t < n_out; t++) n_wide += wide(t) ? 1 : 0;
  if (n_wide == 0 || n_wide == n_out) return 0;
  if (!run) return 4;
  for (int t0 = 0; t0 < n_out;) {
    if (!wide(t0)) {
      t0++;
      continue;
    }
    int t1 = t0 + 1;
    while (t1 < n_out && wide(t1) && limb(t1) == limb(t1 - 1) + 1) t1++;
    launch_fwd_high16(c, dst, dst, n_items, limb(t0), t1 - t0, q_limbs);
    t0 = t1;
  }
  return 4;
}

static size_t convert_h4_lds(const BCTable &t, int rsd = 0) {
  return sizeof(u64) * ((size_t)t.n_k * t.n_tg * 512 + (size_t)t.nd * bc_tgt_words(rsd) +
                        32 * (size_t)(t.nd + t.ns) + (size_t)rsd * 16 * 64);
}

bool convert_h4_ok(const ckks_context *c, const BCTable &t) {
  return c->logN == 16 && c->bc_mfma && t.mt && t.sn && t.n_k >= 1 && t.n_k <= 3 &&
         t.n_tg <= 4 && t.nd <= 64 && convert_h4_lds(t) <= 65536;
}

void launch_convert_h4(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                       const BCTable &t, int src_prime0, int t_split, int t_skip, int q_limbs,
                       bool centered, bool packed) {
  KTimer kt(c, "convert_h4", 8.0 * c->N * n_items * (t.ns + t.nd),
            (double)c->N * n_items * t.ns * t.nd);
  if (!convert_h4_ok(c, t)) throw std::invalid_argument("tile-resident conversion: shape");
  if (n_items <= 0) return;
  auto kern = t.n_k == 1 ? k_convert_h4<1, 0> : t.n_k == 2 ? k_convert_h4<2, 0> : k_convert_h4<3, 0>;
  const size_t lds = convert_h4_lds(t);
  H4Tabs nt{c->d_psi, c->d_psi_sh, c->d_ipsi, c->d_ipsi_sh, c->d_ninv,
            (const double2 *)c->d_tw_fp, (const double2 *)c->d_itw_fp,
            (const double2 *)c->d_ninv_fp};
  const int flags = (centered ? 1 : 0) | (packed ? 8 : 0) |
                    h4_wide_sources(c, src, n_items, t.ns, src_prime0, q_limbs) |
                    h4_wide_targets(c, dst, n_items, t.nd, t_split, t_skip, q_limbs, false);
  hipLaunchKernelGGL(kern, dim3(64, n_items), dim3(TPB), lds, c->stream, src, dst, t.ns, t.nd,
                     t.sn, t.mt, t.n_tg, t.wide_mask, src_prime0, t_split, t_skip, q_limbs, c->L,
                     flags, c->d_mods, nt, (const u64 *)nullptr, (const double2 *)nullptr);
  LAUNCH_CHECK();
  if (flags & 4) h4_wide_targets(c, dst, n_items, t.nd, t_split, t_skip, q_limbs, true);
}

bool convert_h4_rs_ok(const ckks_context *c, const BCTable &t, int D) {
  // the dropped targets in one pass of the kernel (one group, one half)
  if (!(D >= 1 && D <= 2 && t.nd > D && convert_h4_ok(c, t) && convert_h4_lds(t, D) <= 65536 &&
        ((t.nd - 1) >> 3) == ((t.nd - D) >> 3)))
    return false;
  for (int j = 0; j < D; j++)
    if (c->primes[t.nd - 1 - j] >= kFpPrimeBound) return false;
  return true;
}

void launch_convert_h4_rs(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                          const BCTable &t, int D, const u64 *rtab) {
  KTimer kt(c, "convert_h4_rescale", 8.0 * c->N * n_items * (t.ns + D + t.nd - D),
            (double)c->N * n_items * t.ns * t.nd);
  if (!convert_h4_rs_ok(c, t, D)) throw std::invalid_argument("tile-resident RS conversion: shape");
  if (n_items <= 0) return;
  const int T = t.nd - D;
  const double2 *rsf =
      (const double2 *)(rtab + 2 * (size_t)T * D + 2 * (size_t)D + 3 * (size_t)D * D);
  auto k1 = t.n_k == 1 ? k_convert_h4<1, 1> : t.n_k == 2 ? k_convert_h4<2, 1> : k_convert_h4<3, 1>;
  auto k2 = t.n_k == 1 ? k_convert_h4<1, 2> : t.n_k == 2 ? k_convert_h4<2, 2> : k_convert_h4<3, 2>;
  H4Tabs nt{c->d_psi, c->d_psi_sh, c->d_ipsi, c->d_ipsi_sh, c->d_ninv,
            (const double2 *)c->d_tw_fp, (const double2 *)c->d_itw_fp,
            (const double2 *)c->d_ninv_fp};
  const int flags = 1 | h4_wide_sources(c, src, n_items, t.ns, c->L, t.nd) |
                    h4_wide_targets(c, dst, n_items, T, t.nd, 0, t.nd, false);
  hipLaunchKernelGGL(D == 1 ? k1 : k2, dim3(64, n_items), dim3(TPB), convert_h4_lds(t, D),
                     c->stream, src, dst, t.ns, t.nd, t.sn, t.mt, t.n_tg, t.wide_mask, c->L,
                     t.nd, 0, t.nd, c->L, flags, c->d_mods, nt, rtab, rsf);
  LAUNCH_CHECK();
  if (flags & 4) h4_wide_targets(c, dst, n_items, T, t.nd, 0, t.nd, true);
}

// Only the low pass of the forward NTT (bit positions 11..0), in place, for
// limbs whose high pass ran inside launch_convert_h4.  N = 2^16 only.
void launch_ntt_fwd_low(ckks_context *c, const Batch &data, int n_items, int l_begin,
                        int l_count, int q_limbs) {
  KTimer kt(c, "ntt_fwd", 16.0 * c->N * n_items * l_count, 0.5 * c->N * 12 * n_items * l_count);
  if (n_items <= 0 || l_count <= 0) return;
  if (c->logN != 16) throw std::invalid_argument("low pass alone: N = 2^16 only");
  hipLaunchKernelGGL(k_ntt16m_fwd_low<false>, dim3(16, n_items, l_count), dim3(TPB), 0, c->stream,
                     data, l_begin, q_limbs, c->L, c->d_mods, c->d_psi, c->d_psi_sh,
                     (const double2 *)c->d_tw_fp, MDCombine{});
  LAUNCH_CHECK();
}

// Only the low pass of the inverse NTT (bit positions 0..11), for limbs
// whose high pass runs inside launch_convert_h4.  N = 2^16 only.
void launch_ntt_inv_low(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                        int l_begin, int l_count, int q_limbs, const Batch *mul) {
  const int mm = mul ? product_mode(src, *mul, n_items) : 0;
  KTimer kt(c, "ntt_inv", (mm == 1 ? 24.0 : 16.0) * c->N * n_items * l_count,
            (0.5 * 12 + (mm ? 1.0 : 0.0)) * c->N * n_items * l_count);
  if (n_items <= 0 || l_count <= 0) return;
  if (c->logN != 16) throw std::invalid_argument("inverse low pass alone: N = 2^16 only");
  hipLaunchKernelGGL(k_ntt16m_inv_low, dim3(16, n_items, l_count), dim3(TPB), 0, c->stream, src,
                     dst, l_begin, q_limbs, c->L, c->d_mods, c->d_ipsi, c->d_ipsi_sh,
                     (const double2 *)c->d_itw_fp, mul ? *mul : Batch{}, mm);
  LAUNCH_CHECK();
}

// ModDown conversion of a relinearisation fused with the D rescales that
// follow it (division by P p_1 .. p_D in one ModDown, bit-identical to the
// separate steps; p_1 = q_{l-1} is the last prime, p_2 the one before, ...).
// Per item (the 2 polynomials of each ciphertext) the source holds the
// ns = alpha P limbs of X = acc + P d and, at slots ns .. ns + D - 1, its
// limbs l - D .. l - 1, all as coefficients.  For each dropped prime p_j,
// y_j = conv(X_P)_{p_j} gives the relinearised coefficient
// [(X_{p_j} - y_j) P^-1]_{p_j}; the rescale chain turns these into the
// centered lifts r_j that the rescales subtract (as in k_rescale_lift).
// Written for the T = nd - D remaining limbs:
//   out_t = conv(X_P)_t + P sum_j r_j p_1 .. p_{j-1}   (mod q_t)
// so that (acc - NTT(out)) (P p_1..p_D)^-1 + d (p_1..p_D)^-1 is the result.
// tab: the ModDown conversion table to the nd = limbs Q primes; rtab:
// [T][D] P p_1..p_{j-1} mod q_t (Montgomery), [T][D] P p_1..p_j mod q_t,
// [D][2] P^-1 mod p_j + shoup, [D][D][3] p_m mod p_j, p_m^-1 mod p_j, shoup.
// The Montgomery sums stay below q_t 2^64 when sum(P primes) + sum(p_j) < 2^64.
template <int MS>
__global__ __launch_bounds__(TPB) void k_bc_down_rescale(Batch src, Batch dst, int logN, int ns,
                                                         int nd, int D,
                                                         const u64 *__restrict__ tab,
                                                         const u64 *__restrict__ rtab, int L,
                                                         const ModQ *__restrict__ mods) {
  // constants at wave-uniform addresses (scalar loads)
  const u64 *st = tab;
  const u64 *in = batch_ptr(src, blockIdx.y);
  u64 *out = batch_ptr(dst, blockIdx.y);
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int T = nd - D;
  // the sums of products (words below 2^60) as 30-bit half sums (mac30):
  // the ns source terms in one set (ns <= MS <= 16), the D lift terms in the
  // same set when MS + D <= 16, else in a second one
  constexpr bool kOneSet = MS + kMaxRescaleDrop <= 16;
  Half30 v[MS];
  u64 cnt = 0;
#pragma unroll
  for (int i = 0; i < MS; i++) {
    if (i < ns) {
      const u64 qi = mods[L + i].q;
      const u64 vi = shoup_mul(in[((size_t)i << logN) + k], st[i], st[ns + i], qi);
      v[i] = half30(vi);
      cnt += vi > (qi - 1) / 2 ? 1 : 0;
    }
  }
  const u64 *hm = st + 2 * ns;
  const u64 *qm = hm + (size_t)ns * nd;
  const u64 *pm = rtab, *pp = rtab + (size_t)T * D, *pinv = pp + (size_t)T * D;
  const u64 *chain = pinv + 2 * (size_t)D;
  u64 rv[kMaxRescaleDrop];
  Half30 rh[kMaxRescaleDrop];
  bool neg[kMaxRescaleDrop];
#pragma unroll
  for (int j = 0; j < kMaxRescaleDrop; j++) {
    if (j < D) {
      const int tj = nd - 1 - j;
      const ModQ Mj = mods[tj];
      Sum30 a{0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < MS; i++)
        if (i < ns) mac30(a, v[i], half30(hm[i * nd + tj]));
      u64 hi, lo;
      sum30_wide(a, hi, lo);
      u64 y = redc(hi, lo, Mj.q, Mj.qinv);
      if (cnt) y = sub_mod(y, mul_mod(cnt, qm[tj], Mj), Mj.q);
      const u64 xq = in[((size_t)(ns + D - 1 - j) << logN) + k];
      u64 u = shoup_mul(sub_mod(xq, y, Mj.q), pinv[2 * j], pinv[2 * j + 1], Mj.q);
#pragma unroll
      for (int m = 0; m < kMaxRescaleDrop; m++) {
        if (m < j) {
          const u64 *cm = chain + 3 * ((size_t)j * D + m);
          u64 rm = barrett(0, rv[m], Mj);
          if (neg[m]) rm = sub_mod(rm, cm[0], Mj.q);
          u = shoup_mul(sub_mod(u, rm, Mj.q), cm[1], cm[2], Mj.q);
        }
      }
      rv[j] = u;
      rh[j] = half30(u);
      neg[j] = u > (Mj.q - 1) / 2;
    }
  }
  int t = 0;
  for (; t + 1 < T; t += 2) {
    const ModQ M0 = mods[t], M1 = mods[t + 1];
    Sum30 a0{0, 0, 0, 0}, a1{0, 0, 0, 0}, b0{0, 0, 0, 0}, b1{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < MS; i++) {
      if (i < ns) {
        mac30(a0, v[i], half30(hm[i * nd + t]));
        mac30(a1, v[i], half30(hm[i * nd + t + 1]));
      }
    }
#pragma unroll
    for (int j = 0; j < kMaxRescaleDrop; j++) {
      if (j < D) {
        mac30(kOneSet ? a0 : b0, rh[j], half30(pm[(size_t)t * D + j]));
        mac30(kOneSet ? a1 : b1, rh[j], half30(pm[(size_t)(t + 1) * D + j]));
      }
    }
    u64 h0, l0, h1, l1;
    sum30_wide(a0, h0, l0);
    sum30_wide(a1, h1, l1);
    if constexpr (!kOneSet) {
      sum30_add_wide(b0, h0, l0);
      sum30_add_wide(b1, h1, l1);
    }
    u64 y0 = redc(h0, l0, M0.q, M0.qinv);
    u64 y1 = redc(h1, l1, M1.q, M1.qinv);
    if (cnt) {
      y0 = sub_mod(y0, mul_mod(cnt, qm[t], M0), M0.q);
      y1 = sub_mod(y1, mul_mod(cnt, qm[t + 1], M1), M1.q);
    }
#pragma unroll
    for (int j = 0; j < kMaxRescaleDrop; j++) {
      if (j < D && neg[j]) {
        y0 = sub_mod(y0, pp[(size_t)t * D + j], M0.q);
        y1 = sub_mod(y1, pp[(size_t)(t + 1) * D + j], M1.q);
      }
    }
    out[((size_t)t << logN) + k] = y0;
    out[((size_t)(t + 1) << logN) + k] = y1;
  }
  if (t < T) {
    const ModQ M = mods[t];
    Sum30 a0{0, 0, 0, 0}, b0{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < MS; i++)
      if (i < ns) mac30(a0, v[i], half30(hm[i * nd + t]));
#pragma unroll
    for (int j = 0; j < kMaxRescaleDrop; j++)
      if (j < D) mac30(kOneSet ? a0 : b0, rh[j], half30(pm[(size_t)t * D + j]));
    u64 h0, l0;
    sum30_wide(a0, h0, l0);
    if constexpr (!kOneSet) sum30_add_wide(b0, h0, l0);
    u64 y0 = redc(h0, l0, M.q, M.qinv);
    if (cnt) y0 = sub_mod(y0, mul_mod(cnt, qm[t], M), M.q);
#pragma unroll
    for (int j = 0; j < kMaxRescaleDrop; j++)
      if (j < D && neg[j]) y0 = sub_mod(y0, pp[(size_t)t * D + j], M.q);
    out[((size_t)t << logN) + k] = y0;
  }
}

// fp64 variant for P primes and dropped primes below 2^45 (the ModDown table
// has its fp64 part): the v_i as centered exact doubles, every narrow
// target's sum sum_i v_i hmod_i + sum_j r_j P p_1..p_{j-1} of exact fp64
// residues reduced once, minus P p_1..p_j for the negative lifts; the
// dropped primes' values and the lift chain in 64-bit arithmetic; a wide
// target (q_0) as the 64-bit kernel.  The same words.
template <int MS>
__global__ __launch_bounds__(TPB, MS <= 12 ? 5 : 4) void k_bc_down_rescale_fp(
    Batch src, Batch dst, int logN, int ns, int nd, int D, const u64 *__restrict__ tab,
    const double2 *__restrict__ ftab, const u64 *__restrict__ rtab,
    const double2 *__restrict__ frtab, int L, const ModQ *__restrict__ mods) {
  const u64 *in = batch_ptr(src, blockIdx.y);
  u64 *out = batch_ptr(dst, blockIdx.y);
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int T = nd - D;
  const double2 *sf = ftab, *hf = ftab + ns;
  double vd[MS];
#pragma unroll
  for (int i = 0; i < MS; i++) {
    if (i < ns) {
      const double q = (double)mods[L + i].q;
      double v = fp_mulmod(u52_to_dbl(in[((size_t)i << logN) + k]), sf[i].x, sf[i].y, q);
      v = v < 0.0 ? __dadd_rn(v, q) : v;
      v = v >= q ? __dsub_rn(v, q) : v;
      vd[i] = v > __dmul_rn(__dsub_rn(q, 1.0), 0.5) ? __dsub_rn(v, q) : v;
    }
  }
  const u64 *hm = tab + 2 * ns;
  const u64 *qm = hm + (size_t)ns * nd;
  const u64 *pm = rtab, *pp = rtab + (size_t)T * D, *pinv = pp + (size_t)T * D;
  const u64 *chain = pinv + 2 * (size_t)D;
  // sum_i v_i hmod_i (centered) mod the narrow prime of target t
  auto conv = [&](int t, double q) {
    double a0 = 0.0, a1 = 0.0;
#pragma unroll
    for (int i = 0; i < MS; i += 2) {
      if (i < ns) {
        const double2 h = hf[i * nd + t];
        a0 = __dadd_rn(a0, fp_mulmod(vd[i], h.x, h.y, q));
      }
      if (i + 1 < ns) {
        const double2 h = hf[(i + 1) * nd + t];
        a1 = __dadd_rn(a1, fp_mulmod(vd[i + 1], h.x, h.y, q));
      }
    }
    return __dadd_rn(a0, a1);
  };
  u64 rv[kMaxRescaleDrop];
  bool neg[kMaxRescaleDrop];
#pragma unroll
  for (int j = 0; j < kMaxRescaleDrop; j++) {
    if (j < D) {
      const int tj = nd - 1 - j;
      const ModQ Mj = mods[tj];
      const double qj = (double)Mj.q;
      const u64 y = dbl_to_u52(fp_canon_d(conv(tj, qj), 1.0 / qj, qj));
      const u64 xq = in[((size_t)(ns + D - 1 - j) << logN) + k];
      u64 u = shoup_mul(sub_mod(xq, y, Mj.q), pinv[2 * j], pinv[2 * j + 1], Mj.q);
#pragma unroll
      for (int m = 0; m < kMaxRescaleDrop; m++) {
        if (m < j) {
          const u64 *cm = chain + 3 * ((size_t)j * D + m);
          u64 rm = barrett(0, rv[m], Mj);
          if (neg[m]) rm = sub_mod(rm, cm[0], Mj.q);
          u = shoup_mul(sub_mod(u, rm, Mj.q), cm[1], cm[2], Mj.q);
        }
      }
      rv[j] = u;
      neg[j] = u > (Mj.q - 1) / 2;
    }
  }
  for (int t = 0; t < T; t++) {
    const ModQ M = mods[t];
    if (M.q >= (1ull << 45)) {
      // wide target: 128-bit Montgomery accumulation of the canonical v
      u64 hi = 0, lo = 0, cnt = 0;
#pragma unroll
      for (int i = 0; i < MS; i++) {
        if (i < ns) {
          const double v = vd[i];
          const u64 vu = v < 0.0 ? dbl_to_u52(__dadd_rn(v, (double)mods[L + i].q)) : dbl_to_u52(v);
          cnt += v < 0.0 ? 1 : 0;
          mac_wide(hi, lo, vu, hm[i * nd + t]);
        }
      }
#pragma unroll
      for (int j = 0; j < kMaxRescaleDrop; j++)
        if (j < D) mac_wide(hi, lo, rv[j], pm[(size_t)t * D + j]);
      u64 y = redc(hi, lo, M.q, M.qinv);
      if (cnt) y = sub_mod(y, mul_mod(cnt, qm[t], M), M.q);
#pragma unroll
      for (int j = 0; j < kMaxRescaleDrop; j++)
        if (j < D && neg[j]) y = sub_mod(y, pp[(size_t)t * D + j], M.q);
      out[((size_t)t << logN) + k] = y;
      continue;
    }
    const double q = (double)M.q;
    double a = conv(t, q);
#pragma unroll
    for (int j = 0; j < kMaxRescaleDrop; j++) {
      if (j < D) {
        const double2 w = frtab[(size_t)t * D + j];
        a = __dadd_rn(a, fp_mulmod(u52_to_dbl(rv[j]), w.x, w.y, q));
        if (neg[j]) a = __dsub_rn(a, u52_to_dbl(pp[(size_t)t * D + j]));
      }
    }
    out[((size_t)t << logN) + k] = dbl_to_u52(fp_canon_d(a, 1.0 / q, q));
  }
}

void launch_bc_down_rescale(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                            const BCTable &t, int D, const u64 *rtab) {
  KTimer kt(c, "basis_convert_rescale", 8.0 * c->N * n_items * (t.ns + t.nd),
            (double)c->N * n_items * t.ns * t.nd);
  if (D < 1 || D > kMaxRescaleDrop || t.nd <= D || t.ns > kMaxDigitSize)
    throw std::invalid_argument("relinearise-rescale conversion: 1 <= primes < limbs");
  // one or two dropped primes below 2^45, in one target group: the int8
  // matrix-core conversion with the lifts in its epilogue (the same words as
  // the VALU kernels)
  bool mfma = D <= 2 && c->bc_mfma && t.mf &&
              (size_t)t.n_k * t.n_tg * 512 * sizeof(u64) <= 65536 &&
              ((t.nd - 1) >> 4) == ((t.nd - D) >> 4);
  for (int j = 0; j < D && mfma; j++) mfma = c->primes[t.nd - 1 - j] < kFpPrimeBound;
  if (mfma) {
    const int T = t.nd - D;
    const double2 *rsf =
        (const double2 *)(rtab + 2 * (size_t)T * D + 2 * (size_t)D + 3 * (size_t)D * D);
    auto pick1 = t.n_k == 1   ? k_basis_convert_mfma<kMfmaRows, 1, kMfmaChunks, 1>
                 : t.n_k == 2 ? k_basis_convert_mfma<kMfmaRows, 2, kMfmaChunks, 1>
                 : t.n_k == 3 ? k_basis_convert_mfma<kMfmaRows, 3, kMfmaChunks, 1>
                              : k_basis_convert_mfma<kMfmaRows, 4, kMfmaChunks, 1>;
    auto pick2 = t.n_k == 1   ? k_basis_convert_mfma<kMfmaRows, 1, kMfmaChunks, 2>
                 : t.n_k == 2 ? k_basis_convert_mfma<kMfmaRows, 2, kMfmaChunks, 2>
                 : t.n_k == 3 ? k_basis_convert_mfma<kMfmaRows, 3, kMfmaChunks, 2>
                              : k_basis_convert_mfma<kMfmaRows, 4, kMfmaChunks, 2>;
    const size_t lds =
        sizeof(u64) * ((size_t)t.n_k * t.n_tg * 512 + (size_t)t.nd * bc_tgt_words(D));
    hipLaunchKernelGGL(D == 1 ? pick1 : pick2,
                       dim3(c->N / (64 * kMfmaRows * kMfmaChunks), n_items), dim3(TPB), lds,
                       c->stream, src, dst, c->logN, t.ns, t.nd, t.d, t.mf,
                       t.n_tg, t.wide_mask, c->L, t.nd, 0, t.nd, c->L, 1, c->d_mods, rtab, rsf);
    LAUNCH_CHECK();
    return;
  }
  dim3 grid(c->N / TPB, n_items);
  // the fp64 kernel needs the table's fp64 part and the dropped primes below
  // 2^45 (their values come from the fp64 sums)
  bool fp = t.fd != nullptr && !t.wide0;
  for (int j = 0; j < D && fp; j++) fp = c->primes[t.nd - 1 - j] < (1ull << 45);
  if (fp) {
    const int T = t.nd - D;
    const double2 *frtab =
        (const double2 *)(rtab + 2 * (size_t)T * D + 2 * (size_t)D + 3 * (size_t)D * D);
    hipLaunchKernelGGL(t.ns <= 12 ? k_bc_down_rescale_fp<12> : k_bc_down_rescale_fp<kMaxDigitSize>,
                       grid, dim3(TPB), 0, c->stream, src, dst, c->logN, t.ns, t.nd, D, t.d,
                       (const double2 *)t.fd, rtab, frtab, c->L, c->d_mods);
  } else {
    hipLaunchKernelGGL(t.ns <= 12 ? k_bc_down_rescale<12> : k_bc_down_rescale<kMaxDigitSize>,
                       grid, dim3(TPB), 0, c->stream, src, dst, c->logN, t.ns, t.nd, D, t.d, rtab,
                       c->L, c->d_mods);
  }
  LAUNCH_CHECK();
}

// X_l = acc_l + [P]_l d_l for the last D limbs l = limbs - D .. limbs - 1 of
// every item: acc items [2 n][E][N]; ciphertext i of d is batch_ptr(d, i)
// with polynomials [3][limbs][N]; written to x (strided per item2, the D
// limbs in order).  grid (N / 256, 2 n, D)
__global__ void k_rs_prep(Strided acc, int E, int limbs, int D, Batch d, Strided x, int logN,
                          const u64 *__restrict__ pmod, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int item = blockIdx.y >> 1, comp = blockIdx.y & 1;
  const size_t N = (size_t)1 << logN;
  const int l = limbs - D + blockIdx.z;
  const u64 q = mods[l].q;
  const u64 a = acc.base[blockIdx.y * acc.stride + (size_t)l * N + k];
  const u64 dv = batch_ptr(d, item)[((size_t)comp * limbs + l) * N + k];
  x.base[blockIdx.y * x.stride + (size_t)blockIdx.z * N + k] =
      add_mod(a, shoup_mul(dv, pmod[2 * l], pmod[2 * l + 1], q), q);
}

void launch_rs_prep(ckks_context *c, const Strided &acc, int E, int limbs, int D, const Batch &d,
                    int n, const Strided &x) {
  dim3 grid(c->N / TPB, 2 * n, D);
  hipLaunchKernelGGL(k_rs_prep, grid, dim3(TPB), 0, c->stream, acc, E, limbs, D, d, x, c->logN,
                     c->d_pmod, c->d_mods);
  LAUNCH_CHECK();
}

// dst[item][l] = src[item][l] for l < limb_count; grid (N / 256, limbs, items)
__global__ void k_copy_limbs(Batch src, Batch dst, int logN) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const size_t off = ((size_t)blockIdx.y << logN) + k;
  batch_ptr(dst, blockIdx.z)[off] = batch_ptr(src, blockIdx.z)[off];
}

void launch_copy_limbs(ckks_context *c, const Batch &src, const Batch &dst, int n_items,
                       int limb_count) {
  if (limb_count <= 0 || n_items <= 0) return;
  dim3 grid(c->N / TPB, limb_count, n_items);
  hipLaunchKernelGGL(k_copy_limbs, grid, dim3(TPB), 0, c->stream, src, dst, c->logN);
  LAUNCH_CHECK();
}

// ===========================================================================
// key inner product: acc_c[l] = sum_j ext_j[l][sigma(k)] key_j[c][l][k].
// One thread owns one (limb, coefficient) and keeps the key words in
// registers while it walks every item, so each key word is read from HBM
// once per call.  grid (N / 256, E)
// ===========================================================================

template <int MD>
__global__ __launch_bounds__(TPB) void k_key_inner(Batch ext, Batch acc, int n_items,
                                                   const u64 *__restrict__ key, int digits,
                                                   int E, int q_limbs, int L, int K, u64 galois,
                                                   int logN, const ModQ *__restrict__ mods,
                                                   Batch own, int has_own, int ds) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const int p = prime_of(l, q_limbs, L);
  const ModQ M = mods[p];
  const size_t N = (size_t)1 << logN;
  const u32 kk = galois == 1 ? (u32)k : autom_index((u32)k, galois, logN);
  // rotation keys are stored in source order: the word for output k at kk
  u64 kb[MD], ka[MD];
#pragma unroll
  for (int j = 0; j < MD; j++) {
    if (j < digits) {
      kb[j] = key[((size_t)(2 * j) * K + p) * N + key_slot(kk)];
      ka[j] = key[((size_t)(2 * j + 1) * K + p) * N + key_slot(kk)];
    }
  }
  // the digit holding limb l (its own limb: read from the source if given)
  const int jo = (has_own && l < q_limbs) ? l / ds : -1;
  for (int it = 0; it < n_items; it++) {
    const u64 *e = batch_ptr(ext, it);
    const u64 *o = jo >= 0 ? batch_ptr(own, it) : nullptr;
    u64 h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
    for (int j = 0; j < MD; j++) {
      if (j < digits) {
        const u64 x = j == jo ? o[(size_t)l * N + kk] : e[((size_t)j * E + l) * N + kk];
        mac_wide(h0, l0, x, kb[j]);
        mac_wide(h1, l1, x, ka[j]);
      }
    }
    u64 *a = batch_ptr(acc, it);
    a[(size_t)l * N + k] = redc(h0, l0, M.q, M.qinv);
    a[((size_t)E + l) * N + k] = redc(h1, l1, M.q, M.qinv);
  }
}

void launch_key_inner(ckks_context *c, const Batch &ext, const Batch &acc, int n_items,
                      const DeviceKey &key, int digits, int E, int q_limbs, u64 galois,
                      const Batch *own) {
  KTimer kt(c, "key_inner", 8.0 * c->N * ((double)n_items * (digits * E + 2.0 * E) + 2.0 * digits * E),
            2.0 * c->N * E * digits * n_items);
  audit_keyswitch(c, n_items, 1, q_limbs, digits, E);
  dim3 grid(c->N / TPB, E);
  Batch ob{};
  if (own) ob = *own;
  // the keys of every digit are held in registers: a 4-digit instance keeps
  // the register count (and so the occupancy) of the common dnum <= 4 down
  if (digits <= 4)
    hipLaunchKernelGGL(k_key_inner<4>, grid, dim3(TPB), 0, c->stream, ext, acc, n_items,
                       key.data, digits, E, q_limbs, c->L, c->K, galois, c->logN, c->d_mods, ob,
                       own ? 1 : 0, c->ds);
  else
    hipLaunchKernelGGL(k_key_inner<kMaxDigits>, grid, dim3(TPB), 0, c->stream, ext, acc,
                       n_items, key.data, digits, E, q_limbs, c->L, c->K, galois, c->logN,
                       c->d_mods, ob, own ? 1 : 0, c->ds);
  LAUNCH_CHECK();
}

// ===========================================================================
// Key inner products of several rotations sharing one ModUp (hoisted babies),
// written before ModDown in the Q u P basis:
//   acc_b[t] = sum_j ext_j[s] key_b,j[t],  t = pi_{g_b^-1}(s),
// i.e. the automorphism is applied on the output side, so each thread reads
// the extended digits (and c0) at its own index s once for all babies.  With
// c0 given, acc_b,0[t] += P c0[s] on the Q limbs (the extended lift).
// grid (N / 256, E); up to kMultiItems items per launch.  At N = 2^16 the
// 16 blocks of a tile of 16 rows (4096 positions, which the automorphisms
// map onto one tile) share blockIdx.x % 8, so they run on one XCD and the
// permuted stores of the tile fill whole lines in one L2.  Limbs whose prime
// is below 2^45 take fp64 products (exact residues, as the fused low pass +
// key product: the sum times 2^-64, the keys' Montgomery factor, then
// canonical; the same words).
// ===========================================================================

template <int MD>
__global__ __launch_bounds__(TPB) void k_key_inner_multi(
    Strided ext, int n_items, MultiKeys mk, int n_babies, Batch c0, const u64 *__restrict__ pmod,
    const u64 *const *__restrict__ outp, int digits, int E, int q_limbs, int L, int K, int logN,
    const ModQ *__restrict__ mods, const double2 *__restrict__ rinv) {
  int s = blockIdx.x * TPB + threadIdx.x;
  if (logN == 16) {
    const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
    s = ((((j >> 4) << 3) | xcd) << 12) + ((j & 15) << 8) + threadIdx.x;
  }
  const int l = blockIdx.y;
  const int p = prime_of(l, q_limbs, L);
  const ModQ M = mods[p];
  const size_t N = (size_t)1 << logN;
  u64 x[kMultiItems][MD];
  u64 pc[kMultiItems];
  const bool lift = l < q_limbs;
#pragma unroll
  for (int it = 0; it < kMultiItems; it++) {
    if (it < n_items) {
      const u64 *e = ext.base + (size_t)it * ext.stride;
#pragma unroll
      for (int j = 0; j < MD; j++)
        if (j < digits) x[it][j] = e[((size_t)j * E + l) * N + s];
      const u64 *c = batch_ptr(c0, it);
      pc[it] = (lift && c) ? shoup_mul(c[(size_t)l * N + s], pmod[2 * l], pmod[2 * l + 1], M.q)
                           : 0;
    }
  }
  if (M.q < kFpPrimeBound) {
    const double q = (double)M.q, qinv = 1.0 / q;
    const double2 ri = rinv[p];
    double xd[kMultiItems][MD];
#pragma unroll
    for (int it = 0; it < kMultiItems; it++)
#pragma unroll
      for (int j = 0; j < MD; j++)
        xd[it][j] = it < n_items && j < digits ? u52_to_dbl(x[it][j]) : 0.0;
    // each baby's key words are loaded one baby ahead of their products
    const u32 ks = key_slot(s);
    u64 kn[2 * MD];
#pragma unroll
    for (int j = 0; j < MD; j++) {
      if (j < digits && n_babies > 0) {
        kn[2 * j] = mk.key[0][((size_t)(2 * j) * K + p) * N + ks];
        kn[2 * j + 1] = mk.key[0][((size_t)(2 * j + 1) * K + p) * N + ks];
      }
    }
    for (int b = 0; b < n_babies; b++) {
      const u32 t = autom_index((u32)s, mk.ginv[b], logN);
      double kb[MD], kbq[MD], ka[MD], kaq[MD];
#pragma unroll
      for (int j = 0; j < MD; j++) {
        if (j < digits) {
          kb[j] = u52_to_dbl(kn[2 * j]);
          ka[j] = u52_to_dbl(kn[2 * j + 1]);
          kbq[j] = __dmul_rn(kb[j], qinv);
          kaq[j] = __dmul_rn(ka[j], qinv);
        }
      }
      if (b + 1 < n_babies) {
        const u64 *key = mk.key[b + 1];
#pragma unroll
        for (int j = 0; j < MD; j++) {
          if (j < digits) {
            kn[2 * j] = key[((size_t)(2 * j) * K + p) * N + ks];
            kn[2 * j + 1] = key[((size_t)(2 * j + 1) * K + p) * N + ks];
          }
        }
      }
#pragma unroll
      for (int it = 0; it < kMultiItems; it++) {
        if (it < n_items) {
          // |sum| < 1.5 q digits < 2^49
          double a0 = 0.0, a1 = 0.0;
#pragma unroll
          for (int j = 0; j < MD; j++) {
            if (j < digits) {
              a0 = __dadd_rn(a0, fp_mulmod(xd[it][j], kb[j], kbq[j], q));
              a1 = __dadd_rn(a1, fp_mulmod(xd[it][j], ka[j], kaq[j], q));
            }
          }
          const u64 r0 = fp_canon(fp_mulmod(a0, ri.x, ri.y, q), qinv, q);
          const u64 r1 = fp_canon(fp_mulmod(a1, ri.x, ri.y, q), qinv, q);
          u64 *o = (u64 *)outp[(size_t)b * n_items + it];
          o[(size_t)l * N + t] = add_mod(r0, pc[it], M.q);
          o[((size_t)E + l) * N + t] = r1;
        }
      }
    }
    return;
  }
  // primes of 2^45 or more: the extended words split once into 30-bit halves
  // for every baby's products, each output's sum of at most MD <= 16
  // products kept as 30-bit half sums (mac30) and reduced once
  Half30 xh[kMultiItems][MD];
#pragma unroll
  for (int it = 0; it < kMultiItems; it++)
#pragma unroll
    for (int j = 0; j < MD; j++)
      xh[it][j] = it < n_items && j < digits ? half30(x[it][j]) : Half30{0, 0};
  for (int b = 0; b < n_babies; b++) {
    const u32 t = autom_index((u32)s, mk.ginv[b], logN);
    const u64 *key = mk.key[b];
    // keys in source order: the word for output t sits at s
    Half30 kb[MD], ka[MD];
#pragma unroll
    for (int j = 0; j < MD; j++) {
      if (j < digits) {
        kb[j] = half30(key[((size_t)(2 * j) * K + p) * N + key_slot(s)]);
        ka[j] = half30(key[((size_t)(2 * j + 1) * K + p) * N + key_slot(s)]);
      }
    }
#pragma unroll
    for (int it = 0; it < kMultiItems; it++) {
      if (it < n_items) {
        Sum30 s0{0, 0, 0, 0}, s1{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < MD; j++) {
          if (j < digits) {
            mac30(s0, xh[it][j], kb[j]);
            mac30(s1, xh[it][j], ka[j]);
          }
        }
        u64 h0, l0, h1, l1;
        sum30_wide(s0, h0, l0);
        sum30_wide(s1, h1, l1);
        u64 *o = (u64 *)outp[(size_t)b * n_items + it];
        o[(size_t)l * N + t] = add_mod(redc(h0, l0, M.q, M.qinv), pc[it], M.q);
        o[((size_t)E + l) * N + t] = redc(h1, l1, M.q, M.qinv);
      }
    }
  }
}

void launch_key_inner_multi(ckks_context *c, const u64 *ext, size_t ext_stride, int n_items,
                            const std::vector<const DeviceKey *> &keys,
                            const std::vector<u64> &galois_inv, const Batch &c0,
                            const u64 *const *d_outp, int digits, int E, int q_limbs) {
  KTimer kt(c, "key_inner_multi",
            8.0 * c->N * E * ((double)n_items * digits + 2.0 * digits * keys.size() +
                              2.0 * n_items * keys.size()),
            2.0 * c->N * E * digits * (double)keys.size() * n_items);
  audit_keyswitch(c, n_items, (int)keys.size(), q_limbs, digits, E);
  if (n_items < 1 || n_items > kMultiItems) throw std::invalid_argument("key_inner_multi: items");
  const int nb = (int)keys.size();
  if (nb < 1 || nb > kMaxBatch) throw std::invalid_argument("key_inner_multi: babies");
  MultiKeys mk{};
  for (int b = 0; b < nb; b++) {
    mk.key[b] = keys[b]->data;
    mk.ginv[b] = galois_inv[b];
  }
  dim3 grid(c->N / TPB, E);
  if (digits <= 4)
    hipLaunchKernelGGL(k_key_inner_multi<4>, grid, dim3(TPB), 0, c->stream,
                       Strided{(u64 *)ext, ext_stride}, n_items, mk, nb, c0, c->d_pmod, d_outp,
                       digits, E, q_limbs, c->L, c->K, c->logN, c->d_mods,
                       (const double2 *)c->d_rinv_fp);
  else
    hipLaunchKernelGGL(k_key_inner_multi<kMaxDigits>, grid, dim3(TPB), 0, c->stream,
                       Strided{(u64 *)ext, ext_stride}, n_items, mk, nb, c0, c->d_pmod, d_outp,
                       digits, E, q_limbs, c->L, c->K, c->logN, c->d_mods,
                       (const double2 *)c->d_rinv_fp);
  LAUNCH_CHECK();
}

// ===========================================================================
// ModDown combine: out_c[l] = (acc_c[l] - conv_c[l]) P^-1 + add_c[l][sigma(k)]
// acc item layout [2][E][N], conv [2][limbs][N] (internal, strided); add_c and
// out_c are [limbs][N] polynomials per item (a null add pointer adds
// nothing).  grid (N / 256, limbs, 2 * items)
// ===========================================================================

__global__ void k_moddown_combine(Strided acc, Strided conv, Batch add0, Batch add1,
                                  Galois64 gal, Batch out0, Batch out1, int logN, int limbs,
                                  int E, const u64 *__restrict__ pinv,
                                  const u64 *__restrict__ amul, const ModQ *__restrict__ mods,
                                  PostOp post) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const int item = blockIdx.z >> 1, comp = blockIdx.z & 1;
  const size_t N = (size_t)1 << logN;
  const u64 q = mods[l].q;
  const u64 a = acc.base[item * acc.stride + ((size_t)comp * E + l) * N + k];
  const u64 v = conv.base[item * conv.stride + ((size_t)comp * limbs + l) * N + k];
  u64 r = shoup_mul(sub_mod(a, v, q), pinv[2 * l], pinv[2 * l + 1], q);
  // select the pointer, not the argument struct: a selected struct is
  // copied to per-thread scratch memory
  const u64 *ad = comp ? batch_ptr(add1, item) : batch_ptr(add0, item);
  if (ad) {
    const u64 g = gal.g[item];
    const u32 kk = g == 1 ? (u32)k : autom_index((u32)k, g, logN);
    u64 d = ad[(size_t)l * N + kk];
    if (amul) d = shoup_mul(d, amul[2 * l], amul[2 * l + 1], q);
    r = add_mod(r, d, q);
  }
  r = apply_post(post, item, comp, l, (u32)k, N, r, q);
  u64 *o = comp ? batch_ptr(out1, item) : batch_ptr(out0, item);
  o[(size_t)l * N + k] = r;
}

void launch_moddown_combine(ckks_context *c, const Strided &acc, const Strided &conv,
                            const Batch &add0, const Batch &add1, const u64 *galois,
                            const Batch &out0, const Batch &out1, int n_items, int limbs,
                            int E, const u64 *pinv, const u64 *amul, const PostOp *post) {
  KTimer kt(c, "moddown_combine", 8.0 * c->N * 2.0 * n_items * limbs * 4.0,
            2.0 * c->N * n_items * limbs);
  if (n_items > kMaxBatch) throw std::invalid_argument("moddown combine: too many items");
  Galois64 g{};
  for (int i = 0; i < n_items; i++) g.g[i] = galois[i];
  PostOp po{};
  if (post) po = *post;
  dim3 grid(c->N / TPB, limbs, 2 * n_items);
  hipLaunchKernelGGL(k_moddown_combine, grid, dim3(TPB), 0, c->stream, acc, conv, add0, add1,
                     g, out0, out1, c->logN, limbs, E, pinv, amul, c->d_mods, po);
  LAUNCH_CHECK();
}

// ===========================================================================
// rescale (rounded division by the last primes)
// ===========================================================================

// Rescale by the product of the last D primes p_1 = q_l, p_2 = q_{l-1}, ...
// in one pass, giving the words of D rescales in a row.  With v_j the
// coefficients of limb l - j + 1 (canonical mod p_j), rescale j subtracts the
// centered lift r_j of
//   u_j = (((v_j - r_1) p_1^-1 - r_2) p_2^-1 - ... - r_{j-1}) p_{j-1}^-1 mod p_j,
// so the result is (c - NTT(W)) (p_1 ... p_D)^-1 with W = sum_j r_j p_1..p_{j-1}.
// This kernel writes W mod q_i for every remaining limb i < T = limbs - D.
// last: per item [D][N], limbs l - D + 1 .. l in order (v_1 last); w: per
// item [T][N]; grid (N / 256, items).
// tab (see rescale_d_table): [T][2] (prod p)^-1 + shoup, [T][D][3] (p_1..p_{j-1}
// mod q_i, its shoup, p_j mod q_i), [D][D][3] (p_m mod p_j, p_m^-1 mod p_j, shoup).
__global__ __launch_bounds__(TPB) void k_rescale_lift(Batch last, Batch w, int logN, int limbs,
                                                      int D, const u64 *__restrict__ tab,
                                                      const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int T = limbs - D;
  const u64 *in = batch_ptr(last, blockIdx.y);
  u64 *out = batch_ptr(w, blockIdx.y);
  const u64 *tq = tab + 2 * (size_t)T;          // per target
  const u64 *tc = tq + 3 * (size_t)T * D;       // lift chain
  // r_j as canonical residues rv[j] in [0, p_j) with the sign of the lift
  u64 rv[kMaxRescaleDrop];
  bool neg[kMaxRescaleDrop];
#pragma unroll
  for (int j = 0; j < kMaxRescaleDrop; j++) {
    if (j < D) {
      const ModQ Mj = mods[limbs - 1 - j];
      u64 u = in[((size_t)(D - 1 - j) << logN) + k];  // limb l - j sits at slot D - 1 - j
#pragma unroll
      for (int m = 0; m < kMaxRescaleDrop; m++) {
        if (m < j) {
          const u64 *cm = tc + 3 * ((size_t)j * D + m);
          u64 rm = barrett(0, rv[m], Mj);
          if (neg[m]) rm = sub_mod(rm, cm[0], Mj.q);
          u = shoup_mul(sub_mod(u, rm, Mj.q), cm[1], cm[2], Mj.q);
        }
      }
      rv[j] = u;
      neg[j] = u > (Mj.q - 1) / 2;
    }
  }
  for (int i = 0; i < T; i++) {
    const ModQ M = mods[i];
    const u64 *ti = tq + 3 * (size_t)i * D;
    u64 acc = 0;
#pragma unroll
    for (int j = 0; j < kMaxRescaleDrop; j++) {
      if (j < D) {
        u64 r = barrett(0, rv[j], M);
        if (neg[j]) r = sub_mod(r, ti[3 * j + 2], M.q);
        acc = add_mod(acc, j ? shoup_mul(r, ti[3 * j], ti[3 * j + 1], M.q) : r, M.q);
      }
    }
    out[((size_t)i << logN) + k] = acc;
  }
}

void launch_rescale_lift(ckks_context *c, const Batch &last, const Batch &w, int n_items,
                         int limbs, int D, const u64 *tab) {
  KTimer kt(c, "rescale", 8.0 * c->N * n_items * limbs, (double)c->N * n_items * limbs * D);
  if (D < 1 || D > kMaxRescaleDrop || D >= limbs)
    throw std::invalid_argument("rescale: 1 <= primes dropped <= 4 and below the limb count");
  dim3 grid(c->N / TPB, n_items);
  hipLaunchKernelGGL(k_rescale_lift, grid, dim3(TPB), 0, c->stream, last, w, c->logN, limbs, D,
                     tab, c->d_mods);
  LAUNCH_CHECK();
}

// out_i = (src_i - w_i) inv_i for the T remaining limbs; grid (N / 256, T, items)
__global__ void k_rescale_finish(Batch src, Batch w, Batch out, int logN,
                                 const u64 *__restrict__ inv, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int i = blockIdx.y;
  const size_t N = (size_t)1 << logN;
  const u64 q = mods[i].q;
  const u64 a = batch_ptr(src, blockIdx.z)[(size_t)i * N + k];
  const u64 b = batch_ptr(w, blockIdx.z)[(size_t)i * N + k];
  batch_ptr(out, blockIdx.z)[(size_t)i * N + k] =
      shoup_mul(sub_mod(a, b, q), inv[2 * i], inv[2 * i + 1], q);
}

void launch_rescale_finish(ckks_context *c, const Batch &src, const Batch &w, const Batch &out,
                           int n_items, int T, const u64 *inv) {
  KTimer kt(c, "rescale", 8.0 * c->N * 3.0 * n_items * T, (double)c->N * n_items * T);
  dim3 grid(c->N / TPB, T, n_items);
  hipLaunchKernelGGL(k_rescale_finish, grid, dim3(TPB), 0, c->stream, src, w, out, c->logN, inv,
                     c->d_mods);
  LAUNCH_CHECK();
}

// ModRaise: coefficients of limb 0 (in [0, q_0)) read as integers in
// (-q_0/2, q_0/2] and reduced into limb i.  grid (N / 256, target, polys)
__global__ void k_mod_raise(const u64 *__restrict__ coef, u64 *__restrict__ out, int target,
                            int logN, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int i = blockIdx.y;
  const size_t N = (size_t)1 << logN;
  const ModQ M = mods[i];
  const u64 q0 = mods[0].q;
  const u64 v = coef[(size_t)blockIdx.z * N + k];
  u64 r = barrett(0, v, M);
  if (v > (q0 - 1) / 2) r = sub_mod(r, barrett(0, q0, M), M.q);
  out[((size_t)blockIdx.z * target + i) * N + k] = r;
}

void launch_mod_raise(ckks_context *c, const u64 *coef, u64 *out, int polys, int target) {
  dim3 grid(c->N / TPB, target, polys);
  hipLaunchKernelGGL(k_mod_raise, grid, dim3(TPB), 0, c->stream, coef, out, target, c->logN,
                     c->d_mods);
  LAUNCH_CHECK();
}

// ===========================================================================
// BSGS inner sum: out[c][l] = sum_b baby_b[c][l] * pt_b[l]
// Products are folded 16 at a time with REDC (16 q^2 < q 2^64) and the
// folded sum is multiplied back by R.  grid (N / 256, limbs, 2)
// ===========================================================================

__global__ void k_mac(Batch babies, Batch pts, int B, u64 *__restrict__ out, int logN,
                      int limbs, int q_limbs, int L, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y, comp = blockIdx.z;
  const size_t N = (size_t)1 << logN;
  const ModQ M = mods[prime_of(l, q_limbs, L)];
  const size_t off = ((size_t)comp * limbs + l) * N + k;
  u64 acc = 0, hi = 0, lo = 0;
  for (int b = 0; b < B; b++) {
    mac_wide(hi, lo, batch_ptr(babies, b)[off], batch_ptr(pts, b)[(size_t)l * N + k]);
    if ((b & 15) == 15 || b == B - 1) {
      acc = add_mod(acc, redc(hi, lo, M.q, M.qinv), M.q);
      hi = lo = 0;
    }
  }
  out[off] = to_mont(acc, M);
}

void launch_mac(ckks_context *c, const Batch &babies, const Batch &pts, int B, u64 *out,
                int limbs_total, int q_limbs) {
  KTimer kt(c, "mac", 8.0 * c->N * limbs_total * (3.0 * B + 2.0), 2.0 * c->N * limbs_total * B);
  audit_pt(c, (double)B * limbs_total);
  dim3 grid(c->N / TPB, limbs_total, 2);
  hipLaunchKernelGGL(k_mac, grid, dim3(TPB), 0, c->stream, babies, pts, B, out, c->logN,
                     limbs_total, q_limbs, c->L, c->d_mods);
  LAUNCH_CHECK();
}

// 1-D block decode of the table and extended MACs: kb, the block of 256 coefficients, and
// z, the component and input group (nz of them).  The nz blocks of one kb
// read the same plaintext words; with N / 256 a multiple of 8 they get ids 8
// apart, so they run on one XCD close in time and the words come from its L2.
__device__ __forceinline__ void mac_table_block(int nz, int logN, int &kb, int &z) {
  const int b = blockIdx.x, nkb = (1 << logN) / TPB;
  if (nkb & 7) {
    kb = b % nkb;
    z = b / nkb;
  } else {
    const int r = b >> 3;
    z = r % nz;
    kb = (r / nz) * 8 + (b & 7);
  }
}

// Extended-basis MAC of n ciphertexts sharing the plaintexts, for G giant
// groups at once: babies at bab[(b n + i)][2][E][N], plaintext of group g and
// baby b at pts[g B + b], out[(g n + i)][2][E][N].  A block takes one
// component of kMacCtsFp ciphertexts for 256 coefficients (mac_table_block:
// the blocks sharing a plaintext tile run on one XCD back to back); each
// thread walks the babies with the plaintext words of every group in
// registers: every baby word is read from HBM once for all groups.  Limbs
// whose prime is below 2^45 (with B <= 64) take the fp64 path of k_mac_table
// (exact residues, sums below 2^53, one reduction; the same words) over the
// block's ciphertexts at once, the 64-bit path kMacCts at a time; GT >= G
// groups compiled and a baby step's loads issued one step ahead of its
// products.  grid (N / 256 x 2 x input groups, E)
template <int GT>
__global__ __launch_bounds__(TPB) void k_mac_many(const u64 *__restrict__ bab, int n, Batch pts,
                                                  int B, int G, u64 *__restrict__ out, int E,
                                                  int q_limbs, int L, int logN,
                                                  const ModQ *__restrict__ mods) {
  int kb, z;
  mac_table_block(2 * ((n + kMacCtsFp - 1) / kMacCtsFp), logN, kb, z);
  const int k = kb * TPB + threadIdx.x;
  const int l = blockIdx.y, comp = z & 1, ib = (z >> 1) * kMacCtsFp;
  const size_t N = (size_t)1 << logN, EP = 2 * (size_t)E * N;
  const ModQ M = mods[prime_of(l, q_limbs, L)];
  const size_t off = ((size_t)comp * E + l) * N + k;
  if (M.q < ((u64)1 << 45) && B <= 64) {
    constexpr int IC = kMacCtsFp;
    const double q = (double)M.q, qinv = 1.0 / q;
    const size_t poff = (size_t)l * N + k;
    for (int i0 = ib; i0 < ib + IC; i0 += IC) {
      double acc[GT][IC];
#pragma unroll
      for (int g = 0; g < GT; g++)
#pragma unroll
        for (int c = 0; c < IC; c++) acc[g][c] = 0.0;
      u64 xw[IC], ww[GT];
      auto issue = [&](int b) {
#pragma unroll
        for (int c = 0; c < IC; c++) xw[c] = bab[((size_t)b * n + min(i0 + c, n - 1)) * EP + off];
#pragma unroll
        for (int g = 0; g < GT; g++) ww[g] = batch_ptr(pts, min(g, G - 1) * B + b)[poff];
      };
      issue(0);
      for (int b = 0; b < B; b++) {
        u64 xc[IC], wc[GT];
#pragma unroll
        for (int c = 0; c < IC; c++) xc[c] = xw[c];
#pragma unroll
        for (int g = 0; g < GT; g++) wc[g] = ww[g];
        if (b + 1 < B) issue(b + 1);  // the next step's words in flight
        __builtin_amdgcn_sched_barrier(0);
        double x[IC];
#pragma unroll
        for (int c = 0; c < IC; c++) x[c] = u52_to_dbl(xc[c]);
#pragma unroll
        for (int g = 0; g < GT; g++) {
          const double w = u52_to_dbl(wc[g]);
          const double wq = __dmul_rn(w, qinv);
#pragma unroll
          for (int c = 0; c < IC; c++) acc[g][c] = __dadd_rn(acc[g][c], fp_mulmod(x[c], w, wq, q));
        }
      }
#pragma unroll
      for (int g = 0; g < GT; g++)
#pragma unroll
        for (int c = 0; c < IC; c++)
          if (g < G && i0 + c < n)
            out[((size_t)g * n + i0 + c) * EP + off] = fp_canon(acc[g][c], qinv, q);
    }
    return;
  }
  static_assert(kMacCtsFp % kMacCts == 0, "a block's inputs split into 64-bit passes");
  for (int i0 = ib; i0 < ib + kMacCtsFp && i0 < n; i0 += kMacCts) {
    constexpr int IC = kMacCts;
    u64 acc[GT][IC];
    Sum30 sum[GT][IC];
#pragma unroll
    for (int g = 0; g < GT; g++)
#pragma unroll
      for (int c = 0; c < IC; c++) {
        acc[g][c] = 0;
        sum[g][c] = Sum30{0, 0, 0, 0};
      }
    // a baby step's words issued together, one step ahead of their products
    u64 xw[IC], ww[GT];
    auto issue = [&](int b) {
#pragma unroll
      for (int c = 0; c < IC; c++) xw[c] = bab[((size_t)b * n + min(i0 + c, n - 1)) * EP + off];
#pragma unroll
      for (int g = 0; g < GT; g++) ww[g] = batch_ptr(pts, min(g, G - 1) * B + b)[(size_t)l * N + k];
    };
    issue(0);
    for (int b = 0; b < B; b++) {
      u64 xc[IC], wc[GT];
#pragma unroll
      for (int c = 0; c < IC; c++) xc[c] = xw[c];
#pragma unroll
      for (int g = 0; g < GT; g++) wc[g] = ww[g];
      if (b + 1 < B) issue(b + 1);
      __builtin_amdgcn_sched_barrier(0);
      // 16 babies' products as 30-bit half sums (mac30), then reduced
      Half30 xh[IC];
#pragma unroll
      for (int c = 0; c < IC; c++) xh[c] = half30(xc[c]);
#pragma unroll
      for (int g = 0; g < GT; g++) {
        const Half30 wh = half30(wc[g]);
#pragma unroll
        for (int c = 0; c < IC; c++) mac30(sum[g][c], xh[c], wh);
      }
      if ((b & 15) == 15 || b == B - 1) {
#pragma unroll
        for (int g = 0; g < GT; g++)
#pragma unroll
          for (int c = 0; c < IC; c++) {
            u64 hi, lo;
            sum30_wide(sum[g][c], hi, lo);
            acc[g][c] = add_mod(acc[g][c], redc(hi, lo, M.q, M.qinv), M.q);
            sum[g][c] = Sum30{0, 0, 0, 0};
          }
      }
    }
#pragma unroll
    for (int g = 0; g < GT; g++)
#pragma unroll
      for (int c = 0; c < IC; c++)
        if (g < G && i0 + c < n) out[((size_t)g * n + i0 + c) * EP + off] = to_mont(acc[g][c], M);
  }
}

void launch_mac_many(ckks_context *c, const u64 *bab, int n, const Batch &pts, int B, int G,
                     u64 *out, int E, int q_limbs) {
  KTimer kt(c, "mac_many", 8.0 * c->N * E * (2.0 * n * B + (double)G * B + 2.0 * G * n),
            2.0 * c->N * E * (double)n * B * G);
  audit_pt(c, (double)G * B * E);
  if (G < 1 || G > kMacGroups || G * B > kMaxBatch)
    throw std::invalid_argument("mac_many: 1 <= groups <= 2 and groups x babies <= 64");
  dim3 grid(c->N / TPB * 2 * ((n + kMacCtsFp - 1) / kMacCtsFp), E);
  hipLaunchKernelGGL(G <= 1 ? k_mac_many<1> : k_mac_many<kMacGroups>, grid, dim3(TPB), 0,
                     c->stream, bab, n, pts, B, G, out, E, q_limbs, c->L, c->logN, c->d_mods);
  LAUNCH_CHECK();
}

// BSGS MAC of n Q-basis ciphertexts sharing G x B plaintexts, up to
// kTabGroups giant groups per pass: baby b of ciphertext i at bab[i B + b]
// ([2][limbs][N]), plaintext of group g and baby b at pts[g B + b] (limb l at
// l N), inner sum of group g for ciphertext i to out + (g n + i) 2 limbs N.
// A block takes one component of IC ciphertexts (kTabCtsFp on the fp64
// kernel, half as many with more than 8 groups, so that a thread's GT x IC
// accumulators stay within its registers; kTabCts on the 64-bit one, which
// takes more than 8 groups as passes of 8) for 256
// coefficients, each thread the babies of its coefficient with the groups'
// plaintext words in registers: a baby word is read once per pass, a
// plaintext word once per block, which the block decode below turns into
// one HBM read per 256 coefficients.  Passes of 16 groups read the babies
// half as often as passes of 8; their plaintext words serve twice as many
// blocks, from the same XCD's L2.
// Limbs whose prime is below 2^45 (with B <= 64) take the fp64 kernel: each
// product is the exact fp64 residue of fp_mulmod (|r| < 1.5 q) and the
// B-term sums stay exact integers below 2^53, reduced once at the end, so the
// words equal the 64-bit kernel's.  The two are separate kernels, each with
// its own register allocation.  GT >= G groups are compiled: the loads of a
// baby step's IC baby words and GT plaintext words issue together (groups
// beyond G re-read group G - 1 and are not stored), one step ahead of the
// products that use them.
// grid (N / 256 x 2 x input groups, limb_count), limbs from l_begin
typedef __attribute__((address_space(1))) u64 GlobalU64;

template <int GT, int IC>
__global__ __launch_bounds__(TPB) void k_mac_table_fp(const u64 *const *__restrict__ bab, int n,
                                                      const u64 *const *__restrict__ pts, int B,
                                                      int G, u64 *__restrict__ out, int limbs,
                                                      int l_begin, int logN,
                                                      const ModQ *__restrict__ mods) {
  int kb, z;
  mac_table_block(2 * ((n + IC - 1) / IC), logN, kb, z);
  const int k = kb * TPB + threadIdx.x;
  const int l = l_begin + blockIdx.y, comp = z & 1, i0 = (z >> 1) * IC;
  const size_t N = (size_t)1 << logN, CP = 2 * (size_t)limbs * N;
  const ModQ M = mods[l];
  const size_t off = ((size_t)comp * limbs + l) * N + k, poff = (size_t)l * N + k;
  const double q = (double)M.q, qinv = 1.0 / q;
  double acc[GT][IC];
#pragma unroll
  for (int g = 0; g < GT; g++)
#pragma unroll
    for (int c = 0; c < IC; c++) acc[g][c] = 0.0;
  // the tables hold device pointers: global loads, not flat ones
  u64 xw[IC], ww[GT];
  auto issue = [&](int b) {
#pragma unroll
    for (int c = 0; c < IC; c++)
      xw[c] = ((const GlobalU64 *)bab[(size_t)min(i0 + c, n - 1) * B + b])[off];
#pragma unroll
    for (int g = 0; g < GT; g++)
      ww[g] = ((const GlobalU64 *)pts[(size_t)min(g, G - 1) * B + b])[poff];
  };
  issue(0);
  for (int b = 0; b < B; b++) {
    u64 xc[IC], wc[GT];
#pragma unroll
    for (int c = 0; c < IC; c++) xc[c] = xw[c];
#pragma unroll
    for (int g = 0; g < GT; g++) wc[g] = ww[g];
    if (b + 1 < B) issue(b + 1);  // the next step's words in flight
    __builtin_amdgcn_sched_barrier(0);
    double x[IC];
#pragma unroll
    for (int c = 0; c < IC; c++) x[c] = u52_to_dbl(xc[c]);
#pragma unroll
    for (int g = 0; g < GT; g++) {
      const double w = u52_to_dbl(wc[g]);
      const double wq = __dmul_rn(w, qinv);
#pragma unroll
      for (int c = 0; c < IC; c++) acc[g][c] = __dadd_rn(acc[g][c], fp_mulmod(x[c], w, wq, q));
    }
  }
#pragma unroll
  for (int g = 0; g < GT; g++)
#pragma unroll
    for (int c = 0; c < IC; c++)
      if (g < G && i0 + c < n)
        out[((size_t)g * n + i0 + c) * CP + off] = fp_canon(acc[g][c], qinv, q);
}

// The 64-bit kernel: the sums of 16 babies' products (below q 2^64 for
// q < 2^60) kept as four 64-bit sums of 30-bit half products (mac30), then
// Montgomery-reduced; GT >= G groups compiled, a baby step's loads
// issued together one step ahead, and each block takes kTabCts ciphertexts
// (blockIdx.z = component + 2 x ciphertext group), so that a single limb (q_0)
// still fills the chip.
template <int GT, int IC>
__global__ __launch_bounds__(TPB) void k_mac_table_64(const u64 *const *__restrict__ bab, int n,
                                                      const u64 *const *__restrict__ pts, int B,
                                                      int G, u64 *__restrict__ out, int limbs,
                                                      int l_begin, int logN,
                                                      const ModQ *__restrict__ mods) {
  int kb, z;
  mac_table_block(2 * ((n + IC - 1) / IC), logN, kb, z);
  const int k = kb * TPB + threadIdx.x;
  const int l = l_begin + blockIdx.y, comp = z & 1, i0 = (z >> 1) * IC;
  const size_t N = (size_t)1 << logN, CP = 2 * (size_t)limbs * N;
  const ModQ M = mods[l];
  const size_t off = ((size_t)comp * limbs + l) * N + k, poff = (size_t)l * N + k;
  u64 acc[GT][IC];
  Sum30 sum[GT][IC];
#pragma unroll
  for (int g = 0; g < GT; g++)
#pragma unroll
    for (int c = 0; c < IC; c++) {
      acc[g][c] = 0;
      sum[g][c] = Sum30{0, 0, 0, 0};
    }
  u64 xw[IC], ww[GT];
  auto issue = [&](int b) {
#pragma unroll
    for (int c = 0; c < IC; c++)
      xw[c] = ((const GlobalU64 *)bab[(size_t)min(i0 + c, n - 1) * B + b])[off];
#pragma unroll
    for (int g = 0; g < GT; g++)
      ww[g] = ((const GlobalU64 *)pts[(size_t)min(g, G - 1) * B + b])[poff];
  };
  issue(0);
  for (int b = 0; b < B; b++) {
    u64 xc[IC], wc[GT];
#pragma unroll
    for (int c = 0; c < IC; c++) xc[c] = xw[c];
#pragma unroll
    for (int g = 0; g < GT; g++) wc[g] = ww[g];
    if (b + 1 < B) issue(b + 1);  // the next step's words in flight
    __builtin_amdgcn_sched_barrier(0);
    Half30 xh[IC];
#pragma unroll
    for (int c = 0; c < IC; c++) xh[c] = half30(xc[c]);
#pragma unroll
    for (int g = 0; g < GT; g++) {
      const Half30 wh = half30(wc[g]);
#pragma unroll
      for (int c = 0; c < IC; c++) mac30(sum[g][c], xh[c], wh);
    }
    if ((b & 15) == 15 || b == B - 1) {
#pragma unroll
      for (int g = 0; g < GT; g++)
#pragma unroll
        for (int c = 0; c < IC; c++) {
          u64 hi, lo;
          sum30_wide(sum[g][c], hi, lo);
          acc[g][c] = add_mod(acc[g][c], redc(hi, lo, M.q, M.qinv), M.q);
          sum[g][c] = Sum30{0, 0, 0, 0};
        }
    }
  }
#pragma unroll
  for (int g = 0; g < GT; g++)
#pragma unroll
    for (int c = 0; c < IC; c++)
      if (g < G && i0 + c < n) out[((size_t)g * n + i0 + c) * CP + off] = to_mont(acc[g][c], M);
}

void launch_mac_table(ckks_context *c, const u64 *const *bab, int n, const u64 *const *pts, int B,
                      int G, u64 *out, int limbs) {
  KTimer kt(c, "mac_table", 8.0 * c->N * limbs * (2.0 * n * B + (double)G * B + 2.0 * G * n),
            2.0 * c->N * limbs * (double)n * B * G);
  audit_pt(c, (double)G * B * limbs);
  if (G < 1 || G > kTabGroups || B < 1 || n < 1)
    throw std::invalid_argument("mac_table: 1 <= groups <= 16, babies and ciphertexts >= 1");
  // a thread of the fp64 kernel holds GT x IC accumulators: up to 8 groups
  // of 8 ciphertexts, or 16 groups of 4
  const bool wide = G > 8;
  auto fp_kern = G <= 1   ? k_mac_table_fp<1, kTabCtsFp>
                 : G <= 2 ? k_mac_table_fp<2, kTabCtsFp>
                 : G <= 4 ? k_mac_table_fp<4, kTabCtsFp>
                 : G <= 8 ? k_mac_table_fp<8, kTabCtsFp>
                          : k_mac_table_fp<16, kTabCtsFp / 2>;
  // the 64-bit kernel (q_0 alone, beside the others) takes more than 8
  // groups as passes of 8: one ciphertext per block measured 4x slower
  auto w_kern = [](int g) {
    return g <= 1 ? k_mac_table_64<1, kTabCts>
           : g <= 2 ? k_mac_table_64<2, kTabCts>
           : g <= 4 ? k_mac_table_64<4, kTabCts>
                    : k_mac_table_64<8, kTabCts>;
  };
  auto fp_limb = [&](int l) { return B <= 64 && c->prime_fp[l] != 0; };
  auto launch_run = [&](int l0, int l1, hipStream_t st) {
    if (fp_limb(l0)) {
      const int ic = kTabCtsFp / (wide ? 2 : 1);
      const dim3 grid(c->N / TPB * 2 * ((n + ic - 1) / ic), l1 - l0);
      hipLaunchKernelGGL(fp_kern, grid, dim3(TPB), 0, st, bab, n, pts, B, G, out, limbs, l0,
                         c->logN, c->d_mods);
      LAUNCH_CHECK();
      return;
    }
    const dim3 grid(c->N / TPB * 2 * ((n + kTabCts - 1) / kTabCts), l1 - l0);
    const size_t CP = 2 * (size_t)limbs * c->N;
    for (int g0 = 0; g0 < G; g0 += 8) {
      const int gn = std::min(8, G - g0);
      hipLaunchKernelGGL(w_kern(gn), grid, dim3(TPB), 0, st, bab, n, pts + (size_t)g0 * B, B,
                         gn, out + (size_t)g0 * n * CP, limbs, l0, c->logN, c->d_mods);
      LAUNCH_CHECK();
    }
  };
  // runs of limbs of one kind; with both kinds and a second stream, the
  // 64-bit runs (q_0) run beside the fp64 ones
  std::vector<std::pair<int, int>> runs;
  for (int l0 = 0; l0 < limbs;) {
    int l1 = l0 + 1;
    while (l1 < limbs && fp_limb(l1) == fp_limb(l0)) l1++;
    runs.emplace_back(l0, l1);
    l0 = l1;
  }
  const bool fork = runs.size() > 1 && c->aux[0] && c->stream != c->aux[0];
  if (fork) {
    HIP_OK(hipEventRecord(c->fork_ev, c->stream));
    HIP_OK(hipStreamWaitEvent(c->aux[0], c->fork_ev, 0));
  }
  for (auto [l0, l1] : runs) launch_run(l0, l1, fork && !fp_limb(l0) ? c->aux[0] : c->stream);
  if (fork) {
    HIP_OK(hipEventRecord(c->join_ev[0], c->aux[0]));
    HIP_OK(hipStreamWaitEvent(c->stream, c->join_ev[0], 0));
  }
}

// Extended-basis babies.  Offset 0: out = (P c0, P c1) on the Q limbs and 0
// on the special limbs (layout [2][limbs + alpha][N]); grid (N / 256, E, 2)
__global__ void k_ext_identity(const u64 *__restrict__ ct, u64 *__restrict__ out, int limbs,
                               int E, int logN, const u64 *__restrict__ pmod,
                               const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y, comp = blockIdx.z;
  const size_t N = (size_t)1 << logN;
  u64 v = 0;
  if (l < limbs)
    v = shoup_mul(ct[((size_t)comp * limbs + l) * N + k], pmod[2 * l], pmod[2 * l + 1],
                  mods[l].q);
  out[((size_t)comp * E + l) * N + k] = v;
}

// A rotation baby before its ModDown: out_0 += P sigma(c0) on the Q limbs.
// grid (N / 256, limbs)
__global__ void k_ext_add_pc0(const u64 *__restrict__ ct, u64 *__restrict__ out, u64 galois,
                              int logN, const u64 *__restrict__ pmod,
                              const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const size_t N = (size_t)1 << logN;
  const u64 q = mods[l].q;
  const u32 kk = autom_index((u32)k, galois, logN);
  const u64 t = shoup_mul(ct[(size_t)l * N + kk], pmod[2 * l], pmod[2 * l + 1], q);
  u64 *o = out + (size_t)l * N + k;
  *o = add_mod(*o, t, q);
}

void launch_ext_identity(ckks_context *c, const u64 *ct, u64 *out, int limbs) {
  dim3 grid(c->N / TPB, limbs + c->alpha, 2);
  hipLaunchKernelGGL(k_ext_identity, grid, dim3(TPB), 0, c->stream, ct, out, limbs,
                     limbs + c->alpha, c->logN, c->d_pmod, c->d_mods);
  LAUNCH_CHECK();
}

void launch_ext_add_pc0(ckks_context *c, const u64 *ct, u64 *out, int limbs, u64 galois) {
  dim3 grid(c->N / TPB, limbs);
  hipLaunchKernelGGL(k_ext_add_pc0, grid, dim3(TPB), 0, c->stream, ct, out, galois, c->logN,
                     c->d_pmod, c->d_mods);
  LAUNCH_CHECK();
}

// The Q limbs of a one-polynomial ModDown: out[l] = (src[l] - conv[l]) P^-1
// mod q_l, conv = the forward NTT of the centred conversion of src's P limbs
// (the first `limbs` limbs of src are the Q ones).  grid (N / 256, limbs, items)
__global__ void k_moddown_one(Batch src, Strided conv, Batch out, int logN,
                              const u64 *__restrict__ pinv, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y, it = blockIdx.z;
  const size_t N = (size_t)1 << logN, o = (size_t)l * N + k;
  const u64 q = mods[l].q;
  const u64 d = sub_mod(batch_ptr(src, it)[o], conv.base[(size_t)it * conv.stride + o], q);
  batch_ptr(out, it)[o] = shoup_mul(d, pinv[2 * l], pinv[2 * l + 1], q);
}

void launch_moddown_one(ckks_context *c, const Batch &src, Strided conv, const Batch &out,
                        int n_items, int limbs, const u64 *pinv) {
  if (n_items <= 0) return;
  dim3 grid(c->N / TPB, limbs, n_items);
  hipLaunchKernelGGL(k_moddown_one, grid, dim3(TPB), 0, c->stream, src, conv, out, c->logN,
                     pinv, c->d_mods);
  LAUNCH_CHECK();
}

// One giant group of the double-hoisted BSGS added to the running sum, all
// in Q u P (item layout [2][E][N], Q limbs then P limbs):
//   total_0[l][k] += u_0[l][autom(k, g)] + acc_0[l][k],  total_1 += acc_1,
// i.e. sigma_g of the group's first component plus the key product of its
// second; for g = 1 the group is added as it is (acc unused).
// grid (N / 256, E, items)
__global__ void k_ext_rot_accum(Batch u, Batch acc, Batch total, u64 galois, int E, int q_limbs,
                                int L, int logN, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y, it = blockIdx.z;
  const size_t N = (size_t)1 << logN, o = (size_t)l * N + k, EN = (size_t)E * N;
  const u64 q = mods[prime_of(l, q_limbs, L)].q;
  const u64 *ui = batch_ptr(u, it);
  u64 *ti = batch_ptr(total, it);
  if (galois == 1) {
    ti[o] = add_mod(ti[o], ui[o], q);
    ti[EN + o] = add_mod(ti[EN + o], ui[EN + o], q);
    return;
  }
  const u64 *ai = batch_ptr(acc, it);
  const u32 kk = autom_index((u32)k, galois, logN);
  ti[o] = add_mod(ti[o], add_mod(ui[(size_t)l * N + kk], ai[o], q), q);
  ti[EN + o] = add_mod(ti[EN + o], ai[EN + o], q);
}

void launch_ext_rot_accum(ckks_context *c, const Batch &u, const Batch &acc, const Batch &total,
                          u64 galois, int n_items, int E, int q_limbs) {
  if (n_items <= 0) return;
  dim3 grid(c->N / TPB, E, n_items);
  hipLaunchKernelGGL(k_ext_rot_accum, grid, dim3(TPB), 0, c->stream, u, acc, total, galois, E,
                     q_limbs, c->L, c->logN, c->d_mods);
  LAUNCH_CHECK();
}

// ===========================================================================
// Linear combination of n ciphertexts' terms in one launch:
//   out_i = sum_t W_t x_(t,i) + C   (C on c0 only), on the first `limbs` limbs
// of every term, W_t = rint(weight_t) and C = rint(constant) as residues.
// Terms: table of (pointer, limbs) per (t, i), t-major.  grid (N/256, limbs, 2n)
// ===========================================================================

__device__ u64 dbl_residue(double v, const ModQ &M);

__global__ void k_lincomb_prep(const double *__restrict__ w, int T, double cst, int limbs,
                               u64 *__restrict__ wtab, u64 *__restrict__ ctab,
                               const ModQ *__restrict__ mods) {
  const int l = blockIdx.x, t = threadIdx.x;
  const ModQ M = mods[l];
  if (t < T) wtab[(size_t)t * limbs + l] = to_mont(dbl_residue(w[t], M), M);
  if (t == 0) ctab[l] = dbl_residue(cst, M);
}

__global__ void k_lincomb(const u64 *__restrict__ table, int T, int n,
                          const u64 *__restrict__ wtab, const u64 *__restrict__ ctab,
                          u64 *const *__restrict__ outp, int limbs, int logN,
                          const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const int i = blockIdx.z >> 1, poly = blockIdx.z & 1;
  const size_t N = (size_t)1 << logN;
  const ModQ M = mods[l];
  u64 acc = 0, hi = 0, lo = 0;
  // each term's word loaded one term ahead of its product
  auto word = [&](int t) {
    const u64 *x = (const u64 *)table[2 * ((size_t)t * n + i)];
    const u64 tl = table[2 * ((size_t)t * n + i) + 1];
    return x[((size_t)poly * tl + l) * N + k];
  };
  u64 xn = T > 0 ? word(0) : 0;
  for (int t = 0; t < T; t++) {
    const u64 xv = xn;
    if (t + 1 < T) xn = word(t + 1);
    mac_wide(hi, lo, xv, wtab[(size_t)t * limbs + l]);
    if ((t & 15) == 15 || t == T - 1) {
      acc = add_mod(acc, redc(hi, lo, M.q, M.qinv), M.q);
      hi = lo = 0;
    }
  }
  if (poly == 0) acc = add_mod(acc, ctab[l], M.q);
  outp[i][((size_t)poly * limbs + l) * N + k] = acc;
}

void launch_lincomb(ckks_context *c, const u64 *d_table, int T, int n, const double *d_w,
                    double cst, u64 *const *d_outp, int limbs, u64 *wtab, u64 *ctab) {
  KTimer kt(c, "lincomb", 8.0 * c->N * 2.0 * n * limbs * (T + 1.0), 2.0 * c->N * n * limbs * T);
  hipLaunchKernelGGL(k_lincomb_prep, dim3(limbs), dim3(TPB), 0, c->stream, d_w, T, rint(cst),
                     limbs, wtab, ctab, c->d_mods);
  LAUNCH_CHECK();
  dim3 grid(c->N / TPB, limbs, 2 * n);
  hipLaunchKernelGGL(k_lincomb, grid, dim3(TPB), 0, c->stream, d_table, T, n, wtab, ctab, d_outp,
                     limbs, c->logN, c->d_mods);
  LAUNCH_CHECK();
}

// ===========================================================================
// ChaCha20 (RFC 8439) counter-mode PRNG: key = (seed lo, seed hi, 0, ...),
// nonce = (domain, id, sub), counter = block index.
// ===========================================================================

enum { DOM_SECRET = 1, DOM_KEY_A = 2, DOM_KEY_E = 3, DOM_ENC_A = 4, DOM_ENC_E = 5 };

__device__ __forceinline__ u32 rotl32(u32 v, int c) { return (v << c) | (v >> (32 - c)); }

#define DQR(a, b, c, d)                  \
  a += b; d ^= a; d = rotl32(d, 16);     \
  c += d; b ^= c; b = rotl32(b, 12);     \
  a += b; d ^= a; d = rotl32(d, 8);      \
  c += d; b ^= c; b = rotl32(b, 7);

__device__ void chacha_block(u64 seed, u32 dom, u32 id, u32 sub, u32 counter, u32 out[16]) {
  u32 s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
               (u32)seed,   (u32)(seed >> 32), 0u, 0u,
               0u,          0u,          0u,          0u,
               counter,     dom,         id,          sub};
  u32 x[16];
#pragma unroll
  for (int i = 0; i < 16; i++) x[i] = s[i];
#pragma unroll 1
  for (int i = 0; i < 10; i++) {
    DQR(x[0], x[4], x[8], x[12]);
    DQR(x[1], x[5], x[9], x[13]);
    DQR(x[2], x[6], x[10], x[14]);
    DQR(x[3], x[7], x[11], x[15]);
    DQR(x[0], x[5], x[10], x[15]);
    DQR(x[1], x[6], x[11], x[12]);
    DQR(x[2], x[7], x[8], x[13]);
    DQR(x[3], x[4], x[9], x[14]);
  }
#pragma unroll
  for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

// (hi 2^64 + lo) mod q for q >= 2^33: hi is reduced by Barrett (hi < q^2),
// then REDC(hi' 2^64 + lo) = x 2^-64 and x R restores the factor.
__device__ __forceinline__ u64 wide_mod(u64 hi, u64 lo, const ModQ &M) {
  const u64 h = barrett(0, hi, M);
  return to_mont(redc(h, lo, M.q, M.qinv), M);
}

// Centered binomial (eta = 21) errors, coefficient k from 64-bit word k of the
// stream.  grid (N / 8 / 256 rounded up)
__global__ void k_sample_cbd(u64 seed, u32 dom, u32 id, u32 sub, long long *e, int N) {
  const int t = blockIdx.x * TPB + threadIdx.x;
  if (8 * t >= N) return;
  u32 blk[16];
  chacha_block(seed, dom, id, sub, (u32)t, blk);
#pragma unroll
  for (int r = 0; r < 8; r++) {
    const u64 w = (u64)blk[2 * r] | ((u64)blk[2 * r + 1] << 32);
    e[8 * t + r] = (long long)__popcll(w & 0x1FFFFFull) -
                   (long long)__popcll((w >> 21) & 0x1FFFFFull);
  }
}

__device__ __forceinline__ u64 signed_residue(long long x, const ModQ &M) {
  const u64 a = x < 0 ? (u64)(-x) : (u64)x;
  const u64 r = barrett(0, a, M);
  return (x < 0 && r) ? M.q - r : r;
}

// out[l][k] = e[k] mod q_{prime_of(l)}; grid (N / 256, limbs)
__global__ void k_expand_int(const long long *__restrict__ e, u64 *__restrict__ out, int logN,
                             int q_limbs, int L, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const ModQ M = mods[prime_of(l, q_limbs, L)];
  out[((size_t)l << logN) + k] = signed_residue(e[k], M);
}

void launch_expand_ntt(ckks_context *c, const long long *e, u64 *out, int limbs, int q_limbs) {
  hipLaunchKernelGGL(k_expand_int, dim3(c->N / TPB, limbs), dim3(TPB), 0, c->stream, e, out,
                     c->logN, q_limbs, c->L, c->d_mods);
  LAUNCH_CHECK();
  Batch b{};
  b.p[0] = out;
  launch_ntt(c, b, b, 1, 0, limbs, q_limbs, false);
}

// Switching-key digit j over all K primes (p = blockIdx.y):
//   a = uniform (KEY_A, id, j << 16 | p), b = e - a s + [p in digit j] [P]_q s'
// with s' = sigma_g(s) (rotation) or s^2 (relinearisation); both stored in
// Montgomery form.  Each thread produces 4 coefficients from one block.
__global__ void k_keygen_digit(u64 seed, u32 id, int j, const u64 *__restrict__ e_ntt,
                               const u64 *__restrict__ s_ntt, const u64 *__restrict__ pmod,
                               int relin, u64 galois, int ds, u64 *__restrict__ out_b,
                               u64 *__restrict__ out_a, int logN, int L,
                               const ModQ *__restrict__ mods) {
  const int t = blockIdx.x * TPB + threadIdx.x;
  const int p = blockIdx.y;
  const size_t N = (size_t)1 << logN;
  if ((size_t)4 * t >= N) return;
  const ModQ M = mods[p];
  const bool in_digit = p < L && p / ds == j;
  u32 blk[16];
  chacha_block(seed, DOM_KEY_A, id, ((u32)j << 16) | (u32)p, (u32)t, blk);
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const u32 k = 4 * t + r;
    const u64 lo = (u64)blk[4 * r] | ((u64)blk[4 * r + 1] << 32);
    const u64 hi = (u64)blk[4 * r + 2] | ((u64)blk[4 * r + 3] << 32);
    const u64 a = wide_mod(hi, lo, M);
    const u64 s = s_ntt[p * N + k];
    u64 b = sub_mod(e_ntt[p * N + k], mul_mod(a, s, M), M.q);
    if (in_digit) {
      u64 sp;
      if (relin)
        sp = mul_mod(s, s, M);
      else
        sp = s_ntt[p * N + autom_index(k, galois, logN)];
      b = add_mod(b, mul_mod(pmod[p], sp, M), M.q);
    }
    // rotation keys in source order: the word of position k at
    // autom_index(k, g), so that a key switch reads it where it reads the
    // extended digit it multiplies
    const u32 so = key_slot(relin ? k : autom_index(k, galois, logN));
    out_b[p * N + so] = to_mont(b, M);
    out_a[p * N + so] = to_mont(a, M);
  }
}

void launch_keygen(ckks_context *c, DeviceKey &key, u64 id, int relin, u64 galois) {
  const int N = c->N, K = c->K;
  long long *e = (long long *)c->pool.alloc(sizeof(long long) * N);
  u64 *en = (u64 *)c->pool.alloc(sizeof(u64) * (size_t)K * N);
  u64 *pmod = (u64 *)c->pool.alloc(sizeof(u64) * K);
  std::vector<u64> hp(K, 0);
  for (int p = 0; p < c->L; p++) {
    unsigned __int128 acc = 1;
    for (int t = 0; t < c->alpha; t++)
      acc = (acc * (c->primes[c->L + t] % c->primes[p])) % c->primes[p];
    hp[p] = (u64)acc;
  }
  HIP_OK(hipMemcpyAsync(pmod, hp.data(), sizeof(u64) * K, hipMemcpyHostToDevice, c->stream));
  HIP_OK(hipStreamSynchronize(c->stream));  // hp is a host temporary
  for (int j = 0; j < key.digits; j++) {
    hipLaunchKernelGGL(k_sample_cbd, dim3((N / 8 + TPB - 1) / TPB), dim3(TPB), 0, c->stream,
                       c->params.seed, (u32)DOM_KEY_E, (u32)id, (u32)j, e, N);
    LAUNCH_CHECK();
    hipLaunchKernelGGL(k_expand_int, dim3(N / TPB, K), dim3(TPB), 0, c->stream, e, en, c->logN,
                       c->L, c->L, c->d_mods);
    LAUNCH_CHECK();
    Batch b{};
    b.p[0] = en;
    launch_ntt(c, b, b, 1, 0, K, c->L, false);
    u64 *ob = key.data + (size_t)(2 * j) * K * N;
    u64 *oa = key.data + (size_t)(2 * j + 1) * K * N;
    hipLaunchKernelGGL(k_keygen_digit, dim3((N / 4 + TPB - 1) / TPB, K), dim3(TPB), 0,
                       c->stream, c->params.seed, (u32)id, j, en, c->d_secret, pmod, relin,
                       galois, c->ds, ob, oa, c->logN, c->L, c->d_mods);
    LAUNCH_CHECK();
  }
  c->pool.release(e, sizeof(long long) * N);
  c->pool.release(en, sizeof(u64) * (size_t)K * N);
  c->pool.release(pmod, sizeof(u64) * K);
}

// Encryption: c1 = uniform (ENC_A, id, l) in the NTT domain,
// c0 = e - c1 s + m, with m already encoded in c0.  grid (N / 4 / 256, limbs)
__global__ void k_encrypt(u64 seed, u32 id, const u64 *__restrict__ e_ntt,
                          const u64 *__restrict__ s_ntt, u64 *__restrict__ ct, int limbs,
                          int logN, const ModQ *__restrict__ mods) {
  const int t = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const size_t N = (size_t)1 << logN;
  if ((size_t)4 * t >= N) return;
  const ModQ M = mods[l];
  u32 blk[16];
  chacha_block(seed, DOM_ENC_A, id, (u32)l, (u32)t, blk);
  u64 *c0 = ct + (size_t)l * N;
  u64 *c1 = ct + ((size_t)limbs + l) * N;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const size_t k = 4 * (size_t)t + r;
    const u64 lo = (u64)blk[4 * r] | ((u64)blk[4 * r + 1] << 32);
    const u64 hi = (u64)blk[4 * r + 2] | ((u64)blk[4 * r + 3] << 32);
    const u64 a = wide_mod(hi, lo, M);
    c1[k] = a;
    c0[k] = add_mod(sub_mod(e_ntt[l * N + k], mul_mod(a, s_ntt[l * N + k], M), M.q), c0[k], M.q);
  }
}

void launch_encrypt_finish(ckks_context *c, u64 *ct, int limbs, u32 enc_id) {
  const int N = c->N;
  long long *e = (long long *)c->pool.alloc(sizeof(long long) * N);
  u64 *en = (u64 *)c->pool.alloc(sizeof(u64) * (size_t)limbs * N);
  hipLaunchKernelGGL(k_sample_cbd, dim3((N / 8 + TPB - 1) / TPB), dim3(TPB), 0, c->stream,
                     c->params.seed, (u32)DOM_ENC_E, enc_id, 0u, e, N);
  LAUNCH_CHECK();
  hipLaunchKernelGGL(k_expand_int, dim3(N / TPB, limbs), dim3(TPB), 0, c->stream, e, en,
                     c->logN, limbs, c->L, c->d_mods);
  LAUNCH_CHECK();
  Batch b{};
  b.p[0] = en;
  launch_ntt(c, b, b, 1, 0, limbs, limbs, false);
  hipLaunchKernelGGL(k_encrypt, dim3((N / 4 + TPB - 1) / TPB, limbs), dim3(TPB), 0, c->stream,
                     c->params.seed, enc_id, en, c->d_secret, ct, limbs, c->logN, c->d_mods);
  LAUNCH_CHECK();
  c->pool.release(e, sizeof(long long) * N);
  c->pool.release(en, sizeof(u64) * (size_t)limbs * N);
}

// ===========================================================================
// canonical-embedding encoder / decoder (fp64, no contraction: the same
// operations in the same order as the CPU statement of the algorithm)
// ===========================================================================

struct cplx {
  double re, im;
};

__device__ __forceinline__ cplx cmul(cplx a, cplx b) {
  const double t1 = __dmul_rn(a.re, b.re);
  const double t2 = __dmul_rn(a.im, b.im);
  const double t3 = __dmul_rn(a.re, b.im);
  const double t4 = __dmul_rn(a.im, b.re);
  return cplx{__dsub_rn(t1, t2), __dadd_rn(t3, t4)};
}

// x[row][br(perm[j])] = z[row][j]  (perm, then the FFT's bit-reversal)
__global__ void k_fft_place(const double *__restrict__ re, const double *__restrict__ im,
                            cplx *__restrict__ x, const u32 *__restrict__ perm, int n, int logn) {
  const int j = blockIdx.x * TPB + threadIdx.x;
  if (j >= n) return;
  const size_t row = blockIdx.y;
  const u32 r = __brev(perm[j]) >> (32 - logn);
  x[row * n + r] = cplx{re[row * n + j], im ? im[row * n + j] : 0.0};
}

// Radix-2 DIT FFT of rows of n points (bit-reversed input).  Stage len
// (2, 4, .., n) takes, for every st multiple of len and k < len / 2,
//   u = x[st + k], v = x[st + k + len/2] * tw[k n / len],
//   x[st + k] = u + v, x[st + k + len/2] = u - v
// (complex product as cmul, each sum rounded once).  The stages run in two
// launches per batch of rows: len = 2 .. min(n, kFftTile) inside tiles of
// kFftTile contiguous points staged in LDS (k_fft_tile), then len =
// 2 kFftTile .. n in registers over the points r + kFftTile m of a row
// (k_fft_cols, M = n / kFftTile per thread).  The order of the stages, and
// so every rounding, is that of the stage-by-stage definition above.
constexpr int kFftTile = 2048;

// grid (n / tile, rows), tile = min(n, kFftTile)
__global__ __launch_bounds__(TPB) void k_fft_tile(cplx *__restrict__ x, int n, int tile,
                                                  const cplx *__restrict__ tw) {
  __shared__ cplx sm[kFftTile];
  cplx *row = x + (size_t)blockIdx.y * n + (size_t)blockIdx.x * tile;
  for (int i = threadIdx.x; i < tile; i += TPB) sm[i] = row[i];
  __syncthreads();
  for (int len = 2; len <= tile; len <<= 1) {
    const int half = len >> 1, step = n / len;
    for (int b = threadIdx.x; b < (tile >> 1); b += TPB) {
      const int k = b & (half - 1);
      const int i0 = 2 * (b - k) + k;
      const cplx u = sm[i0];
      const cplx v = cmul(sm[i0 + half], tw[k * step]);
      sm[i0] = cplx{__dadd_rn(u.re, v.re), __dadd_rn(u.im, v.im)};
      sm[i0 + half] = cplx{__dsub_rn(u.re, v.re), __dsub_rn(u.im, v.im)};
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < tile; i += TPB) row[i] = sm[i];
}

// grid (kFftTile / 256, rows); n = M kFftTile
template <int M>
__global__ __launch_bounds__(TPB) void k_fft_cols(cplx *__restrict__ x, int n,
                                                  const cplx *__restrict__ tw) {
  const int r = blockIdx.x * TPB + threadIdx.x;
  cplx *row = x + (size_t)blockIdx.y * n;
  cplx v[M];
#pragma unroll
  for (int m = 0; m < M; m++) v[m] = row[r + kFftTile * m];
#pragma unroll
  for (int hm = 1; hm < M; hm <<= 1) {
    const int step = n / (2 * kFftTile * hm);
#pragma unroll
    for (int m = 0; m < M; m++) {
      if (m & hm) continue;
      const int k = r + kFftTile * (m & (hm - 1));
      const cplx u = v[m];
      const cplx w = cmul(v[m + hm], tw[k * step]);
      v[m] = cplx{__dadd_rn(u.re, w.re), __dadd_rn(u.im, w.im)};
      v[m + hm] = cplx{__dsub_rn(u.re, w.re), __dsub_rn(u.im, w.im)};
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++) row[r + kFftTile * m] = v[m];
}

// In-place FFT of `rows` rows of n points (n a power of two, bit-reversed
// input) with the stage twiddles `tw` (tw[k n / len] for stage len).
static void launch_fft(ckks_context *c, cplx *x, int rows, int n, const cplx *tw) {
  if (n < 2 || rows < 1) return;
  if (rows > 65535) throw std::invalid_argument("fft: at most 65535 rows per launch");
  const int tile = n < kFftTile ? n : kFftTile;
  hipLaunchKernelGGL(k_fft_tile, dim3(n / tile, rows), dim3(TPB), 0, c->stream, x, n, tile, tw);
  LAUNCH_CHECK();
  const dim3 g(kFftTile / TPB, rows);
  switch (n / tile) {
    case 1: break;
    case 2: hipLaunchKernelGGL(k_fft_cols<2>, g, dim3(TPB), 0, c->stream, x, n, tw); break;
    case 4: hipLaunchKernelGGL(k_fft_cols<4>, g, dim3(TPB), 0, c->stream, x, n, tw); break;
    case 8: hipLaunchKernelGGL(k_fft_cols<8>, g, dim3(TPB), 0, c->stream, x, n, tw); break;
    case 16: hipLaunchKernelGGL(k_fft_cols<16>, g, dim3(TPB), 0, c->stream, x, n, tw); break;
    case 32: hipLaunchKernelGGL(k_fft_cols<32>, g, dim3(TPB), 0, c->stream, x, n, tw); break;
    default: throw std::invalid_argument("fft: at most 2^16 points");
  }
  LAUNCH_CHECK();
}

// Residue of an integer-valued double of any magnitude (exact).
__device__ u64 dbl_residue(double v, const ModQ &M) {
  if (fabs(v) < 9.2e18) return signed_residue((long long)v, M);
  const u64 bits = (u64)__double_as_longlong(v);
  const int e = (int)((bits >> 52) & 0x7ff) - 1075;
  const u64 mant = (bits & 0xFFFFFFFFFFFFFull) | (1ull << 52);
  u64 r = barrett(0, mant, M);
  for (int i = 0; i < e; i++) r = add_mod(r, r, M.q);
  return ((long long)bits < 0 && r) ? M.q - r : r;
}

// Encoder tail: u = (x_k / n) * twist_k, coefficient k gap and (k + n) gap
// get rint(scale u.re), rint(scale u.im); then residues for every limb, the
// rounded value formed once per coefficient.  grid (N / 256, rows)
__global__ void k_encode_finish(const cplx *__restrict__ x, const cplx *__restrict__ twist,
                                Batch out, int n, int logN, double scale, int total, int q_limbs,
                                int L, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;  // coefficient index
  const int N = 1 << logN, gap = N / (2 * n);
  double v = 0.0;
  if (k % gap == 0) {
    const int idx = k / gap;
    const int kk = idx < n ? idx : idx - n;
    const cplx w = x[(size_t)blockIdx.y * n + kk];
    const double inv_n = 1.0 / (double)n;
    cplx u = cplx{__dmul_rn(w.re, inv_n), __dmul_rn(w.im, inv_n)};
    u = cmul(u, twist[kk]);
    v = rint(__dmul_rn(scale, idx < n ? u.re : u.im));
  }
  u64 *o = batch_ptr(out, blockIdx.y) + k;
  for (int l = 0; l < total; l++)
    o[(size_t)l << logN] = dbl_residue(v, mods[prime_of(l, q_limbs, L)]);
}

// Encoder tail over rows already placed in x ([rows][n], slot j at
// bit-reversed perm[j]): inverse FFT, twist, rounding, residues, NTT.
static void encode_placed(ckks_context *c, cplx *x, int rows, int slots, double scale,
                          int limbs, int is_ext, const Batch &out) {
  const FFTTable &t = c->fft.at(slots);
  const int n = slots;
  launch_fft(c, x, rows, n, (const cplx *)t.tw_inv);
  const int total = limbs + (is_ext ? c->alpha : 0);
  hipLaunchKernelGGL(k_encode_finish, dim3(c->N / TPB, rows), dim3(TPB), 0, c->stream, x,
                     (const cplx *)t.twist, out, n, c->logN, scale, total, limbs, c->L,
                     c->d_mods);
  LAUNCH_CHECK();
  launch_ntt(c, out, out, rows, 0, total, limbs, false);
}

void launch_encode(ckks_context *c, const double *d_re, const double *d_im, int rows,
                   int slots, double scale, int limbs, int is_ext, const Batch &out) {
  const FFTTable &t = c->fft.at(slots);
  const int n = slots;
  int logn = 0;
  while ((1 << logn) < n) logn++;
  cplx *x = (cplx *)c->pool.alloc(sizeof(cplx) * (size_t)rows * n);
  hipLaunchKernelGGL(k_fft_place, dim3((n + TPB - 1) / TPB, rows), dim3(TPB), 0, c->stream,
                     d_re, d_im, x, t.perm, n, logn);
  LAUNCH_CHECK();
  encode_placed(c, x, rows, slots, scale, limbs, is_ext, out);
  c->pool.release(x, sizeof(cplx) * (size_t)rows * n);
}

// ---------------------------------------------------------------------------
// BSGS diagonals gathered from a device-resident weight, placed straight into
// the encoder's FFT input (the [rows, slots] block is never written):
//   row(g, b)[slot] = W[(f - (giant_base + g) B) mod D, (f + b) mod D],
//   f = slot / token_lanes, row index g B + b.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void diag_features(int row, int j, const DiagGeom &gm, int &of,
                                              int &inf) {
  const int g = gm.giant_base + row / gm.baby, b = row % gm.baby;
  const int f = j / gm.lanes;
  of = (int)(((long long)f - (long long)g * gm.baby) % gm.D);
  if (of < 0) of += gm.D;
  inf = (f + b) % gm.D;
}

// dtype 0 float64, 1 float32, 2 complex128 ([D][D] row-major)
__global__ void k_place_token_lane(const void *__restrict__ w, int dtype, DiagGeom gm,
                                   cplx *__restrict__ x, const u32 *__restrict__ perm, int n,
                                   int logn, int row0) {
  const int j = blockIdx.x * TPB + threadIdx.x;
  if (j >= n) return;
  const int row = row0 + blockIdx.y;
  int of, inf;
  diag_features(row, j, gm, of, inf);
  const size_t wi = (size_t)of * gm.D + inf;
  cplx v{0.0, 0.0};
  if (dtype == 0) v.re = ((const double *)w)[wi];
  else if (dtype == 1) v.re = (double)((const float *)w)[wi];
  else v = ((const cplx *)w)[wi];
  x[(size_t)blockIdx.y * n + (__brev(perm[j]) >> (32 - logn))] = v;
}

// W_phys[o, i] = column_scale[i] (real_scale[o] src[real_source[o]][real_row[o], column[i]]
//                + i imag_scale[o] src[imag_source[o]][imag_row[o], column[i]]);
// an index of -1 (source or column) is zero padding.  maps: [8][D] words:
// real_source, real_row, imag_source, imag_row, column (int64), real_scale,
// imag_scale, column_scale (double).
__global__ void k_place_structured(StructSources src, const u64 *__restrict__ maps, DiagGeom gm,
                                   cplx *__restrict__ x, const u32 *__restrict__ perm, int n,
                                   int logn, int row0) {
  const int j = blockIdx.x * TPB + threadIdx.x;
  if (j >= n) return;
  const int row = row0 + blockIdx.y;
  int of, inf;
  diag_features(row, j, gm, of, inf);
  const long long *mi = (const long long *)maps;
  const double *md = (const double *)maps;
  const size_t D = gm.D;
  const long long rs = mi[of], rr = mi[D + of], is = mi[2 * D + of], ir = mi[3 * D + of];
  const long long col = mi[4 * D + inf];
  const double rsc = md[5 * D + of], isc = md[6 * D + of], csc = md[7 * D + inf];
  auto read = [&](long long s, long long r) -> double {
    if (s < 0 || col < 0) return 0.0;
    const size_t idx = (size_t)r * src.stride[s][0] + (size_t)col * src.stride[s][1];
    return src.fp32 ? (double)((const float *)src.p[s])[idx] : ((const double *)src.p[s])[idx];
  };
  cplx v{read(rs, rr) * rsc * csc, read(is, ir) * isc * csc};
  x[(size_t)blockIdx.y * n + (__brev(perm[j]) >> (32 - logn))] = v;
}

void launch_encode_diagonals(ckks_context *c, const void *w, int dtype, const StructSources *src,
                             const u64 *maps, const DiagGeom &gm, int rows, int slots,
                             double scale, int limbs, int is_ext, ckks_ct **out) {
  const FFTTable &t = c->fft.at(slots);
  const int n = slots;
  int logn = 0;
  while ((1 << logn) < n) logn++;
  for (int r0 = 0; r0 < rows; r0 += kMaxBatch) {
    const int nr = std::min(kMaxBatch, rows - r0);
    cplx *x = (cplx *)c->pool.alloc(sizeof(cplx) * (size_t)nr * n);
    dim3 grid((n + TPB - 1) / TPB, nr);
    if (src)
      hipLaunchKernelGGL(k_place_structured, grid, dim3(TPB), 0, c->stream, *src, maps, gm, x,
                         t.perm, n, logn, r0);
    else
      hipLaunchKernelGGL(k_place_token_lane, grid, dim3(TPB), 0, c->stream, w, dtype, gm, x,
                         t.perm, n, logn, r0);
    LAUNCH_CHECK();
    Batch o{};
    for (int r = 0; r < nr; r++) o.p[r] = out[r0 + r]->d;
    encode_placed(c, x, nr, slots, scale, limbs, is_ext, o);
    c->pool.release(x, sizeof(cplx) * (size_t)nr * n);
  }
}

__global__ void k_scalar_encode(double v, int limbs, u64 *out, const ModQ *__restrict__ mods) {
  const int l = threadIdx.x;
  if (l < limbs) out[l] = dbl_residue(v, mods[l]);
}

void launch_scalar_encode(ckks_context *c, double v, int limbs, u64 *out) {
  hipLaunchKernelGGL(k_scalar_encode, dim3(1), dim3(TPB), 0, c->stream, rint(v), limbs, out,
                     c->d_mods);
  LAUNCH_CHECK();
}

// m = sum_d c_d s^d on the first K limbs (NTT domain).  grid (N / 256, K)
__global__ void k_dec_poly(const u64 *__restrict__ ct, int polys, int limbs,
                           const u64 *__restrict__ s_ntt, u64 *__restrict__ m, int logN,
                           const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  const int l = blockIdx.y;
  const size_t N = (size_t)1 << logN;
  const ModQ M = mods[l];
  const u64 s = s_ntt[l * N + k];
  u64 acc = 0, sp = 1;
  for (int d = 0; d < polys; d++) {
    acc = add_mod(acc, mul_mod(ct[((size_t)d * limbs + l) * N + k], sp, M), M.q);
    sp = mul_mod(sp, s, M);
  }
  m[l * N + k] = acc;
}

// Balanced Garner reconstruction of coefficient (idx gap) over K limbs, then
// x[br(k)] = (v_k + i v_{k+n}) * untwist_k for the decoding FFT.
// grid (n / 256 rounded up)
// Decryption reconstructs at most this many limbs (40-bit primes: ~320 bits,
// far above any scale times the 2^40 headroom it keeps).
constexpr int GARNER_MAX_LIMBS = 8;

__global__ void k_dec_garner(const u64 *__restrict__ m, int K, const u64 *__restrict__ inv,
                             const cplx *__restrict__ untwist, cplx *__restrict__ x, int n,
                             int logn, int logN, const ModQ *__restrict__ mods) {
  const int k = blockIdx.x * TPB + threadIdx.x;
  if (k >= n) return;
  const size_t N = (size_t)1 << logN;
  const int gap = (int)(N / (2 * n));
  double vv[2];
  for (int h = 0; h < 2; h++) {
    const size_t ci = (size_t)(k + h * n) * gap;
    // fully unrolled over the bound so that the digits stay in registers
    long long d[GARNER_MAX_LIMBS];
#pragma unroll
    for (int kk = 0; kk < GARNER_MAX_LIMBS; kk++) {
      if (kk < K) {
        const ModQ M = mods[kk];
        u64 t = m[kk * N + ci];
#pragma unroll
        for (int j = 0; j < kk; j++)
          t = mul_mod(sub_mod(t, signed_residue(d[j], M), M.q), inv[j * K + kk], M);
        d[kk] = t > (M.q - 1) / 2 ? (long long)t - (long long)M.q : (long long)t;
      }
    }
    double v = 0.0;
#pragma unroll
    for (int kk = GARNER_MAX_LIMBS - 1; kk >= 0; kk--)
      if (kk < K) v = __dadd_rn(__dmul_rn(v, (double)mods[kk].q), (double)d[kk]);
    vv[h] = v;
  }
  const u32 r = __brev((u32)k) >> (32 - logn);
  x[r] = cmul(cplx{vv[0], vv[1]}, untwist[k]);
}

__global__ void k_dec_gather(const cplx *__restrict__ x, const u32 *__restrict__ perm, int n,
                             double scale, double *__restrict__ re, double *__restrict__ im) {
  const int j = blockIdx.x * TPB + threadIdx.x;
  if (j >= n) return;
  const cplx v = x[perm[j]];
  re[j] = v.re / scale;
  im[j] = v.im / scale;
}

void launch_decrypt_decode(ckks_context *c, const ckks_ct *ct, double *d_re, double *d_im) {
  const int N = c->N, n = ct->slots;
  int logn = 0;
  while ((1 << logn) < n) logn++;
  // limbs needed: smallest K with sum log2 q >= log2(scale) + 40
  double need = log2(ct->scale) + 40.0, have = 0.0;
  int K = 0;
  while (K < ct->limbs && K < GARNER_MAX_LIMBS && have < need)
    have += log2((double)c->primes[K++]);
  if (K < 1) K = 1;
  u64 *m = (u64 *)c->pool.alloc(sizeof(u64) * (size_t)K * N);
  const bool is_pt = ct->polys == 1;
  if (is_pt) {
    HIP_OK(hipMemcpyAsync(m, ct->d, sizeof(u64) * (size_t)K * N, hipMemcpyDeviceToDevice,
                          c->stream));
  } else {
    hipLaunchKernelGGL(k_dec_poly, dim3(N / TPB, K), dim3(TPB), 0, c->stream, ct->d, ct->polys,
                       ct->limbs + (ct->is_ext ? c->alpha : 0), c->d_secret, m, c->logN,
                       c->d_mods);
    LAUNCH_CHECK();
  }
  Batch b{};
  b.p[0] = m;
  launch_ntt(c, b, b, 1, 0, K, K, true);
  if (!c->garner.count(K)) {
    std::vector<u64> inv((size_t)K * K, 0);
    for (int j = 0; j < K; j++)
      for (int k = 0; k < K; k++) {
        if (j == k) continue;
        const u64 q = c->primes[k];
        // q_j^-1 mod q_k by Fermat
        unsigned __int128 base = c->primes[j] % q, r = 1;
        u64 e = q - 2;
        while (e) {
          if (e & 1) r = (r * base) % q;
          base = (base * base) % q;
          e >>= 1;
        }
        inv[(size_t)j * K + k] = (u64)r;
      }
    u64 *d = nullptr;
    HIP_OK(hipMalloc(&d, sizeof(u64) * (size_t)K * K));
    HIP_OK(hipMemcpy(d, inv.data(), sizeof(u64) * (size_t)K * K, hipMemcpyHostToDevice));
    c->garner[K] = d;
  }
  const FFTTable &t = c->fft.at(n);
  cplx *x = (cplx *)c->pool.alloc(sizeof(cplx) * n);
  hipLaunchKernelGGL(k_dec_garner, dim3((n + TPB - 1) / TPB), dim3(TPB), 0, c->stream, m, K,
                     c->garner[K], (const cplx *)t.untwist, x, n, logn, c->logN, c->d_mods);
  LAUNCH_CHECK();
  launch_fft(c, x, 1, n, (const cplx *)t.tw_fwd);
  hipLaunchKernelGGL(k_dec_gather, dim3((n + TPB - 1) / TPB), dim3(TPB), 0, c->stream, x,
                     t.perm, n, ct->scale, d_re, d_im);
  LAUNCH_CHECK();
  c->pool.release(x, sizeof(cplx) * n);
  c->pool.release(m, sizeof(u64) * (size_t)K * N);
}

// ===========================================================================
// integer-throughput probe: eight independent chains per thread of the
// modular product the kernels use, in registers only (kind 0: the fp64-path
// product of 40-bit limbs, 1: the 64-bit Shoup product, 2: a plain fp64 FMA)
// ===========================================================================

__global__ __launch_bounds__(TPB) void k_int_peak(int kind, int iters, double *out) {
  const int t = blockIdx.x * TPB + threadIdx.x;
  const double q = 1099511480321.0, w = 774036213477.0, wq = w / q;  // q < 2^40 prime
  const u64 qi = 1152921504606830593ull, wi = 1015234567890123ull;    // q < 2^60
  const u64 ws = (u64)(((unsigned __int128)wi << 64) / qi);
  double a[8];
  u64 b[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    a[j] = (double)(t * 8 + j + 1);
    b[j] = (u64)(t * 8 + j + 1);
  }
  if (kind == 0) {
    for (int it = 0; it < iters; it++)
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] = fp_mulmod(a[j], w, wq, q);
  } else if (kind == 1) {
    for (int it = 0; it < iters; it++)
#pragma unroll
      for (int j = 0; j < 8; j++) b[j] = shoup_mul(b[j], wi, ws, qi);
  } else {
    for (int it = 0; it < iters; it++)
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] = __fma_rn(a[j], 0.999999, 1e-3);
  }
  double acc = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) acc += a[j] + (double)(b[j] & 1023);
  out[t] = acc;
}

double launch_int_peak(ckks_context *c, int kind, double *scratch, int blocks, int iters) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
    throw std::runtime_error("int peak: event creation failed");
  (void)hipEventRecord(e0, c->stream);
  hipLaunchKernelGGL(k_int_peak, dim3(blocks), dim3(TPB), 0, c->stream, kind, iters, scratch);
  (void)hipEventRecord(e1, c->stream);
  hipError_t err = hipGetLastError();
  float ms = 0;
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (err != hipSuccess) throw std::runtime_error(std::string("int peak: ") + hipGetErrorString(err));
  return 8.0 * TPB * (double)blocks * iters / (ms * 1e-3);
}

}  // namespace ckks
