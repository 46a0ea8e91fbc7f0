// Lightning-indexer scores and per-query top-k on gfx950.
//
// I[b,t,s] = sum_h w[b,t,h] * ReLU(q[b,t,h,:] . k[b,s,h,:])
// (kernels/triton/fused_indexer.py:52-60), then the k best keys per query
// (fused_indexer.py:63-73, :153-206) with ties to the lowest key index.
//
// Scores are fp64 and a fixed function of the inputs: each q.k product of
// fp32/bf16 values is exact in fp64 and is accumulated over d in increasing
// order (so fused and unfused adds agree), ReLU, then the heads are added in
// increasing h as fl(acc + fl(w*r)) -- never fused.  The CPU oracle computes
// the same expression, so selections match bit for bit.
//
// Score kernels:
//  - matrix-core tiles (prefill, 2-byte q and k): 64 queries x 64 keys per
//    workgroup on v_mfma_f64_16x16x4f64, whose in-order accumulation keeps
//    the sequential sum's bits (products of 2-byte values are exact);
//  - VALU tiles (fp32 or unaligned inputs): a 64-query x 128-key tile per
//    workgroup, 8x4 register tile per thread, q/k slices staged in LDS;
//  - per-key (decode, few queries): 64 keys per workgroup, one thread per
//    (key, head) reading the key row from LDS.
// Scores of a chunk of queries go to the workspace and the shared row top-k
// (topk.hip) selects from them.
#include <algorithm>

#include <atomic>
#include <random>

#include "common.h"

#include "topk.h"

namespace la {

struct IdxKP {
  const void *q;
  const void *k;
  const float *w;
  double *scores;  // [b][t - t0][Tk]
  int64_t B, Tq, Tk, HI, d;
  int64_t q_sb, q_st, q_sh, k_sb, k_st, k_sh, w_sb, w_st, w_sh;
  int64_t t0, tn;  // query chunk [t0, t0 + tn)
  int64_t offset;
  int64_t unit;  // tokens per key (pooled groups); key s starts at token s*unit
  int32_t dt, causal;
  // one query per chunk only (may be null): the radix top-k's first-digit
  // histogram of each batch row, [b * hist_stride + bin], fed with the valid keys
  uint32_t *hist0;
  int64_t hist_stride;
  // with rx_ready: the first workgroup of batch row b clears the row's
  // hist_stride words of radix records, then stores the call's value
  // *rx_epoch + rx_gen into rx_ready[b]; every workgroup waits for that value
  // before adding into the histogram.  rx_gen is a per-call value of the
  // host (a word left over in the workspace does not hold it by chance), and
  // the epoch word is advanced by the radix select's first launch (after this
  // kernel), so a replayed graph of the call waits for a value of its own too.
  uint64_t *rx_ready;
  const uint64_t *rx_epoch;
  uint64_t rx_gen;
  uint32_t spin_limit;  // polls before that wait is given up (0: at once)
  // the integer-limb form of bf16 q and k (indexer_limb_kernel, d == 64): per
  // 16-row block, head and limb, the block in the matrix-core operand order;
  // per row and head the packed exponent word (lm_* in the limb kernel)
  const int8_t *lq, *lk;
  const int32_t *xq, *xk;
  int64_t nqb, nkb;  // 16-row blocks per batch row of q (the chunk) and of k
};

// Status bits this file's kernels raise on the current device (read through
// la_device_status).
__device__ uint32_t la_ix_status;

constexpr int IT_Q = 64, IT_K = 128, IT_D = 64;  // tile, d slice
constexpr int IT_NT = 256;

// Tile: queries [qt*64, +64) of the chunk x keys [kt*128, +128).
// Thread (tq = tid/32, tk = tid%32) owns queries 8*tq..8*tq+7, keys 4*tk..4*tk+3.
__global__ __launch_bounds__(IT_NT) void indexer_tile_kernel(IdxKP p) {
  // rows padded by 4 floats: 16-byte aligned, at most 4-way conflicts on stores
  __shared__ float sq[IT_D][IT_Q + 4];
  __shared__ float sk[IT_D][IT_K + 4];
  const int tid = threadIdx.x;
  const int tq = tid >> 5, tk = tid & 31;
  const int64_t b = blockIdx.z;
  const int64_t q0 = (int64_t)blockIdx.y * IT_Q;  // within the chunk
  const int64_t k0 = (int64_t)blockIdx.x * IT_K;
  if (q0 >= p.tn) return;
  // causal: skip tiles whose first key is after the tile's last query
  if (p.causal) {
    const int64_t last_q = p.offset + p.t0 + min(q0 + IT_Q, p.tn) - 1;
    if (k0 * p.unit > last_q) return;
  }
  double score[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) score[i][j] = 0.0;

  for (int64_t h = 0; h < p.HI; ++h) {
    double dot[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) dot[i][j] = 0.0;
    for (int64_t d0 = 0; d0 < p.d; d0 += IT_D) {
      const int dn = (int)min((int64_t)IT_D, p.d - d0);
      __syncthreads();  // previous slice fully consumed
      // stage q (64 rows) and k (128 rows) slices, transposed to [d][row]
      for (int i = tid; i < IT_Q * IT_D; i += IT_NT) {
        const int r = i / IT_D, dd = i % IT_D;
        const int64_t t = p.t0 + q0 + r;
        float x = 0.f;
        if (dd < dn && q0 + r < p.tn)
          x = load_as_f32(p.q, b * p.q_sb + t * p.q_st + h * p.q_sh + d0 + dd, p.dt);
        sq[dd][r] = x;
      }
      for (int i = tid; i < IT_K * IT_D; i += IT_NT) {
        const int r = i / IT_D, dd = i % IT_D;
        const int64_t s = k0 + r;
        float x = 0.f;
        if (dd < dn && s < p.Tk)
          x = load_as_f32(p.k, b * p.k_sb + s * p.k_st + h * p.k_sh + d0 + dd, p.dt);
        sk[dd][r] = x;
      }
      __syncthreads();
      for (int dd = 0; dd < dn; ++dd) {
        const float4 qa = *(const float4 *)&sq[dd][tq * 8];
        const float4 qb = *(const float4 *)&sq[dd][tq * 8 + 4];
        const float4 ka = *(const float4 *)&sk[dd][tk * 4];
        const double qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const double kv[4] = {ka.x, ka.y, ka.z, ka.w};
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) dot[i][j] = __builtin_fma(qv[i], kv[j], dot[i][j]);
      }
    }
    // head epilogue: score += fl(w * relu(dot)), heads in increasing order
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t ql = q0 + tq * 8 + i;
      const int64_t t = p.t0 + min(ql, p.tn - 1);
      const double wv = (double)p.w[b * p.w_sb + t * p.w_st + h * p.w_sh];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double r = dot[i][j] > 0.0 ? dot[i][j] : 0.0;
        score[i][j] = add_product(score[i][j], wv, r);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t ql = q0 + tq * 8 + i;
    if (ql >= p.tn) continue;
    double *row = p.scores + (b * p.tn + ql) * p.Tk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t s = k0 + tk * 4 + j;
      if (s < p.Tk) row[s] = score[i][j];
    }
  }
}

// 2-byte q/k whose (head, d) rows are 16-byte aligned (the shape of config
// C2) are loaded as (head, 64-d) slices with coalesced 16-byte loads (8 lanes
// per row) and widened to fp32 (exact) for LDS.
constexpr int IT16_D = 64;  // d slice

template <bool BF>
__device__ __forceinline__ void widen8(const uint4 &v, float (&x)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (BF) {
      x[2 * e] = bf16lo(w[e]);
      x[2 * e + 1] = bf16hi(w[e]);
    } else {
      x[2 * e] = __half2float(__ushort_as_half((uint16_t)(w[e] & 0xffffu)));
      x[2 * e + 1] = __half2float(__ushort_as_half((uint16_t)(w[e] >> 16)));
    }
  }
}

// The score tile on the fp64 matrix cores (2-byte q and k): a workgroup
// covers 64 queries x 64 keys, wave w keys [k0 + 32 (w % 2), +32) x
// queries [q0 + 32 (w / 2), +32) as 2 x 2 tiles of v_mfma_f64_16x16x4f64
// (A = key rows, B = query columns, one fp64 value per lane each); three
// workgroups per CU.  gfx950 accumulates that instruction as a chain in k
// order, c = fl(fl(fl(fl(c + a0 b0) + a1 b1) + a2 b2) + a3 b3), and a product
// of two 2-byte values is exact in fp64, so chaining the instructions over d
// in increasing order yields the bits of the sequential sum (tests pin this
// on the device).  Lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]
// (d = 4 s + l / 16 of chunk s) and receives D[4 e + l / 16][l % 16], e < 4.
// q and k slices are staged in LDS as fp32 (exact) with rows padded to 68
// floats, so the 16 rows x 4 columns a fragment read touches fall in
// distinct banks; the next slice is loaded into registers during this one.
constexpr int IM_S = 68;   // LDS row stride (fp32)
constexpr int IM_K = 64;   // keys per workgroup (queries: IT_Q)
constexpr int IM_NT = 256;

template <bool BF>
__global__ __launch_bounds__(IM_NT, 3) void indexer_mfma_kernel(IdxKP p) {
  typedef double f64x4 __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) float sq[IT_Q][IM_S];
  __shared__ __align__(16) float sk[IM_K][IM_S];
  __shared__ float sw[IT_Q][8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r16 = lane & 15, kq = lane >> 4;
  const int64_t b = blockIdx.z;
  const int64_t q0 = (int64_t)blockIdx.y * IT_Q;  // within the chunk
  const int64_t k0 = (int64_t)blockIdx.x * IM_K;
  if (q0 >= p.tn) return;
  if (p.causal) {
    const int64_t last_q = p.offset + p.t0 + min(q0 + IT_Q, p.tn) - 1;
    if (k0 * p.unit > last_q) return;
  }
  const int HI = (int)p.HI, d = (int)p.d;
  for (int i = tid; i < IT_Q * HI; i += IM_NT) {
    const int r = i / HI, h = i % HI;
    const int64_t t = p.t0 + min(q0 + r, p.tn - 1);
    sw[r][h] = p.w[b * p.w_sb + t * p.w_st + h * p.w_sh];
  }
  const uint16_t *qb = (const uint16_t *)p.q + b * p.q_sb;
  const uint16_t *kb = (const uint16_t *)p.k + b * p.k_sb;
  // slice loads: chunk c (c < 512) of q is row c/8, d-chunk c%8; k likewise.
  // Rows past the chunk / key range read a clamped row.
  uint4 lq[2], lk[2];
  auto fetch = [&](int h, int d0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + u * IM_NT, r = c >> 3, dc = c & 7;
      const int64_t t = p.t0 + min(q0 + r, p.tn - 1);
      const int64_t s = min(k0 + r, p.Tk - 1);
      const int dd = min(d0 + dc * 8, d - 8);
      lq[u] = *(const uint4 *)(qb + t * p.q_st + h * p.q_sh + dd);
      lk[u] = *(const uint4 *)(kb + s * p.k_st + h * p.k_sh + dd);
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + u * IM_NT, r = c >> 3, dc = c & 7;
      float x[8];
      widen8<BF>(lq[u], x);
      *(float4 *)&sq[r][dc * 8] = float4{x[0], x[1], x[2], x[3]};
      *(float4 *)&sq[r][dc * 8 + 4] = float4{x[4], x[5], x[6], x[7]};
      widen8<BF>(lk[u], x);
      *(float4 *)&sk[r][dc * 8] = float4{x[0], x[1], x[2], x[3]};
      *(float4 *)&sk[r][dc * 8 + 4] = float4{x[4], x[5], x[6], x[7]};
    }
  };
  const int kw = w & 1, qw = w >> 1;
  f64x4 score[2][2];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) score[ib][jb] = f64x4{0.0, 0.0, 0.0, 0.0};
  const float *ka = &sk[32 * kw + r16][kq];
  const float *qa = &sq[32 * qw + r16][kq];
  fetch(0, 0);
  for (int h = 0; h < HI; ++h) {
    f64x4 dot[2][2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) dot[ib][jb] = f64x4{0.0, 0.0, 0.0, 0.0};
    for (int d0 = 0; d0 < d; d0 += IT16_D) {
      const int dn = min(IT16_D, d - d0);
      __syncthreads();  // the previous slice is consumed
      stage();
      __syncthreads();
      {  // next slice in flight during this one
        const bool last_d = d0 + IT16_D >= d;
        const int nh = last_d ? h + 1 : h, nd = last_d ? 0 : d0 + IT16_D;
        fetch(min(nh, HI - 1), nd);
      }
      auto chunk = [&](int dd) {
        double a[2], bq[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          a[i] = (double)ka[16 * i * IM_S + dd];
          bq[i] = (double)qa[16 * i * IM_S + dd];
        }
#pragma unroll
        for (int ib = 0; ib < 2; ++ib)
#pragma unroll
          for (int jb = 0; jb < 2; ++jb)
            dot[ib][jb] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[ib], bq[jb], dot[ib][jb], 0, 0, 0);
      };
      if (dn == IT16_D) {
#pragma unroll
        for (int dd = 0; dd < IT16_D; dd += 4) chunk(dd);
      } else {
        for (int dd = 0; dd < dn; dd += 4) chunk(dd);
      }
    }
    // head epilogue: score += fl(w * relu(dot)), heads in increasing order
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const double wv = (double)sw[32 * qw + 16 * jb + r16][h];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const double x = dot[ib][jb][e];
          score[ib][jb][e] = add_product(score[ib][jb][e], wv, x > 0.0 ? x : 0.0);
        }
    }
  }
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int64_t ql = q0 + 32 * qw + 16 * jb + r16;
    if (ql >= p.tn) continue;
    double *row = p.scores + (b * p.tn + ql) * p.Tk;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t s = k0 + 32 * kw + 16 * ib + 4 * e + kq;
        if (s < p.Tk) row[s] = score[ib][jb][e];
      }
  }
}

// ------------------------------------------------ integer-limb scores ----
// The same scores on the int8 matrix cores, exact: a bf16 value is
// x = m 2^(e - 134) with an integer m < 256 (sign included), so over the 64
// values of one (row, head) with least exponent E, x = X 2^(E - 134) with the
// integer X = m 2^(e - E), |X| < 2^(8 + R), R the row's exponent range.  For
// R <= 22, X is four balanced base-256 digits (limbs, int8), and the head's
// dot of a query row and a key row is the integer sum over the 16 limb pairs
// of int8 dots (v_mfma_i32_16x16x64_i8, exact in int32), scaled by
// 2^(Eq + Ek - 268).  That integer equals the fp64 sequential sum of the
// (exact) products whenever every partial sum is exact, which holds when
// Rq + Rk <= 30 (the partial sums stay below 64 * 2^(16 + Rq + Rk) <= 2^52
// units of the least product bit).  A pair outside that bound (or a row with
// an inf / nan, or R > 22) takes the sequential fp64 sum of the bf16 values
// instead, in the same order as the oracle.  The heads are then added in
// order as in the fp64 kernel.

// Packed exponent word of a (row, head): E + 1024 in bits 0-15, R in bits
// 16-23 (255: no limbs, the sequential sum is taken).
constexpr int LM_NOLIMB = 255;

// Sixteen lanes per (batch, row, head): lane j converts elements 4 j .. 4 j + 3
// and stores their limbs as one 4-byte word per limb.  Rows past n (the
// padding of the last 64-row tile) get zero limbs.
// One launch converts two runs of rows (k and the first query chunk): the
// first blocks_a workgroups take run a, the rest run b.
struct LimbRun {
  const uint16_t *src;
  int64_t sb, st, sh, r0, n, n_pad;
  int8_t *limbs;
  int32_t *xw;
};
__global__ __launch_bounds__(256) void indexer_limb_kernel(LimbRun ra, LimbRun rb, int64_t HI,
                                                           uint32_t blocks_a) {
  const bool in_a = blockIdx.x < blocks_a;
  const LimbRun &r = in_a ? ra : rb;
  const uint16_t *src = r.src;
  const int64_t sb = r.sb, st = r.st, sh = r.sh, r0 = r.r0, n = r.n, n_pad = r.n_pad;
  int8_t *limbs = r.limbs;
  int32_t *xw = r.xw;
  const uint32_t blk_x = in_a ? blockIdx.x : blockIdx.x - blocks_a;
  // a wave takes 4 consecutive rows of one head, so that its limb stores
  // fill 64-byte runs of one block
  const int64_t gt = (int64_t)blk_x * 256 + threadIdx.x;
  const int j = (int)(gt & 15);
  const int64_t rh = gt >> 4;
  const int64_t r4 = rh >> 2, h = r4 % HI, rq = r4 / HI;
  const int64_t row = (rq % (n_pad / 4)) * 4 + (rh & 3), b = rq / (n_pad / 4);
  uint2 raw = make_uint2(0u, 0u);
  if (row < n) raw = *(const uint2 *)(src + b * sb + (r0 + row) * st + h * sh + 4 * j);
  const uint32_t xs[4] = {raw.x & 0xffffu, raw.x >> 16, raw.y & 0xffffu, raw.y >> 16};
  int m[4], e[4];
  int emin = 1 << 20, emax = -1, special = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t E = (xs[u] >> 7) & 0xffu, f = xs[u] & 0x7fu;
    m[u] = E ? (int)(128u + f) : (int)f;
    e[u] = E ? (int)E : 1;
    special |= E == 255u;
    if (m[u] != 0) {
      emin = min(emin, e[u]);
      emax = max(emax, e[u]);
    }
  }
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) {  // over the row's 16 lanes
    emin = min(emin, __shfl_xor(emin, o, 64));
    emax = max(emax, __shfl_xor(emax, o, 64));
    special |= __shfl_xor(special, o, 64);
  }
  if (emax < 0) emin = emax = 0;  // all zero
  const int R = emax - emin;
  const bool nolimb = special || R > 22;
  uint32_t word[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    int X = nolimb ? 0 : m[u] << (e[u] - emin);  // |X| < 2^30
    if (xs[u] >> 15) X = -X;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int di = ((X + 128) & 255) - 128;
      word[i] |= (uint32_t)(di & 255) << (8 * u);
      X = (X - di) >> 8;
    }
  }
  // block (row / 16), lane position (row % 16) + 16 (d / 16), byte d % 16
  int8_t *blk = limbs + ((b * (n_pad / 16) + row / 16) * HI + h) * 4096;
  const int pos = (int)(row % 16) + 16 * (j / 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) *(uint32_t *)(blk + i * 1024 + pos * 16 + 4 * (j % 4)) = word[i];
  if (j == 0) xw[(b * n_pad + row) * HI + h] = (emin + 1024) | ((nolimb ? LM_NOLIMB : R) << 16);
}

// A workgroup covers 64 queries x 64 keys (the fp64 kernel's tiles; two
// workgroups per CU, for its registers); wave w keys [k0 + 32 (w % 2), +32) x
// queries [q0 + 32 (w / 2), +32) as 2 x 2 tiles of 16 x 16.  Lane l supplies
// key / query row l % 16 of a tile, d = 16 (l / 16) .. + 15 (the limb blocks
// are stored in that order), and receives D[4 (l / 16) + i][l % 16]: key
// 4 (l / 16) + i, query l % 16.
template <int HIc>
__global__ __launch_bounds__(IM_NT, 2) void indexer_i8_kernel(IdxKP p) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  // the limb blocks of one head: 4 key and 4 query 16-row blocks x 4 limbs,
  // 1 KiB each, copied by the LDS-DMA loads a head ahead (two buffers)
  __shared__ __align__(16) int8_t sl[2][2][4][4][1024];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t b = blockIdx.z;
  const int64_t q0 = (int64_t)blockIdx.y * IT_Q;  // within the chunk
  const int64_t k0 = (int64_t)blockIdx.x * IM_K;
  if (q0 >= p.tn) return;
  if (p.causal) {
    const int64_t last_q = p.offset + p.t0 + min(q0 + IT_Q, p.tn) - 1;
    if (k0 * p.unit > last_q) return;
  }
  constexpr int HI = HIc;
  const int kw = w & 1, qw = w >> 1;
  const int g4 = lane >> 4, c16 = lane & 15;
  const int64_t kbw = k0 / 16, qbw = q0 / 16;  // the workgroup's first blocks
  // wave w copies blocks 8 w .. 8 w + 7 of a head's 32 (k blocks, then q)
  auto copy_head = [&](int h) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = 8 * w + u, side = j >> 4, blk = (j >> 2) & 3, limb = j & 3;
      const int8_t *src = side == 0 ? p.lk + ((b * p.nkb + kbw + blk) * HI + h) * 4096
                                    : p.lq + ((b * p.nqb + qbw + blk) * HI + h) * 4096;
      dma16(src + limb * 1024 + lane * 16, &sl[h & 1][side][blk][limb][0]);
    }
  };
  // the head weights of this lane's two queries (registers, loaded now and
  // used one head after another)
  float wq[2][HI];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int64_t t = p.t0 + min(q0 + 32 * qw + 16 * jb + c16, p.tn - 1);
#pragma unroll
    for (int hh = 0; hh < HI; ++hh) wq[jb][hh] = p.w[b * p.w_sb + t * p.w_st + hh * p.w_sh];
  }
  double score[2][2][4];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int i = 0; i < 4; ++i) score[ib][jb][i] = 0.0;
  const uint16_t *qg = (const uint16_t *)p.q + b * p.q_sb;
  const uint16_t *kg = (const uint16_t *)p.k + b * p.k_sb;
  // a double 2^e (normal range)
  auto pow2 = [](int e) { return __longlong_as_double((long long)(e + 1023) << 52); };
  // this lane's exponent words of a head: its 4 keys of each key tile, its
  // query of each query tile (loaded with the head's copies, a head ahead)
  auto load_x = [&](int h, int32_t (&xk)[2][4], int32_t (&xq)[2]) {
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xk[ib][i] = p.xk[((b * p.nkb + kbw + 2 * kw + ib) * 16 + 4 * g4 + i) * HI + h];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) xq[jb] = p.xq[((b * p.nqb + qbw + 2 * qw + jb) * 16 + c16) * HI + h];
  };
  int32_t xk[2][4], xq[2], nxk[2][4], nxq[2];
  copy_head(0);
  load_x(0, xk, xq);
#pragma unroll
  for (int h = 0; h < HI; ++h) {
    if (h > 0) {
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int i = 0; i < 4; ++i) xk[ib][i] = nxk[ib][i];
      xq[0] = nxq[0];
      xq[1] = nxq[1];
    }
    wait_vmcnt<0>();  // this wave's copies of head h (and the words)
    __syncthreads();  // every wave's copies; head h - 1's buffer is free
    if (h + 1 < HI) {
      copy_head(h + 1);
      load_x(h + 1, nxk, nxq);
    }
    v4i A[2][4], B[2][4];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int l = 0; l < 4; ++l) A[ib][l] = *(const v4i *)&sl[h & 1][0][2 * kw + ib][l][lane * 16];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int l = 0; l < 4; ++l) B[jb][l] = *(const v4i *)&sl[h & 1][1][2 * qw + jb][l][lane * 16];
    // a 16-row block whose rows all have R <= 14 has a zero fourth limb
    // (|X| < 2^22): tiles of two such blocks take 3 x 3 limb pairs, and no
    // pair of theirs can leave the exact bound (R + R <= 28)
    bool kbig[2], qbig[2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      bool big = false;
#pragma unroll
      for (int i = 0; i < 4; ++i) big |= ((xk[ib][i] >> 16) & 0xff) > 14;
      kbig[ib] = __ballot(big) != 0;
    }
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) qbig[jb] = __ballot(((xq[jb] >> 16) & 0xff) > 14) != 0;
    double wsq[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) wsq[jb] = (double)wq[jb][h] * pow2((xq[jb] & 0xffff) - 1024 - 134);
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        double prod[4];
        if (!kbig[ib] && !qbig[jb]) {
          v4i acc[5];
#pragma unroll
          for (int g = 0; g < 5; ++g) acc[g] = v4i{0, 0, 0, 0};
#pragma unroll
          for (int la = 0; la < 3; ++la)
#pragma unroll
            for (int lb = 0; lb < 3; ++lb)
              acc[la + lb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ib][la], B[jb][lb], acc[la + lb], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // lo + m1 2^16 + top 2^32, each part within int32
            const int32_t lo = acc[0][i] + acc[1][i] * 256;
            const int32_t m1 = acc[2][i] + acc[3][i] * 256;
            double v = (double)acc[4][i];
            v = __builtin_fma(v, 65536.0, (double)m1);
            v = __builtin_fma(v, 65536.0, (double)lo);
            const double x = v * pow2((xk[ib][i] & 0xffff) - 1024 - 134);
            prod[i] = wsq[jb] * (x > 0.0 ? x : 0.0);
          }
        } else {
          v4i acc[7];
#pragma unroll
          for (int g = 0; g < 7; ++g) acc[g] = v4i{0, 0, 0, 0};
#pragma unroll
          for (int la = 0; la < 4; ++la)
#pragma unroll
            for (int lb = 0; lb < 4; ++lb)
              acc[la + lb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ib][la], B[jb][lb], acc[la + lb], 0, 0, 0);
          bool bad[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // lo + m1 2^16 + m2 2^32 + top 2^48, each part within int32
            const int32_t lo = acc[0][i] + acc[1][i] * 256;
            const int32_t m1 = acc[2][i] + acc[3][i] * 256;
            const int32_t m2 = acc[4][i] + acc[5][i] * 256;
            double v = (double)acc[6][i];
            v = __builtin_fma(v, 65536.0, (double)m2);
            v = __builtin_fma(v, 65536.0, (double)m1);
            v = __builtin_fma(v, 65536.0, (double)lo);
            const double x = v * pow2((xk[ib][i] & 0xffff) - 1024 - 134);
            prod[i] = wsq[jb] * (x > 0.0 ? x : 0.0);
            bad[i] = ((xk[ib][i] >> 16) & 0xff) + ((xq[jb] >> 16) & 0xff) > 30;
          }
          if (__ballot(bad[0] || bad[1] || bad[2] || bad[3])) {
            // outside the exact bound: the sequential fp64 sum of the values
            const int64_t ql = q0 + 32 * qw + 16 * jb + c16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int64_t s = k0 + 32 * kw + 16 * ib + 4 * g4 + i;
              if (bad[i] && ql < p.tn && s < p.Tk) {
                const uint4 *qr = (const uint4 *)(qg + (p.t0 + ql) * p.q_st + h * p.q_sh);
                const uint4 *kr = (const uint4 *)(kg + s * p.k_st + h * p.k_sh);
                double a = 0.0;
#pragma unroll 1
                for (int c = 0; c < 8; ++c) {  // 8 values per 16-byte load, in order
                  const uint4 qv = qr[c], kv = kr[c];
                  const uint32_t qw4[4] = {qv.x, qv.y, qv.z, qv.w}, kw4[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                  for (int e = 0; e < 4; ++e) {
                    a = __builtin_fma((double)bf16lo(qw4[e]), (double)bf16lo(kw4[e]), a);
                    a = __builtin_fma((double)bf16hi(qw4[e]), (double)bf16hi(kw4[e]), a);
                  }
                }
                prod[i] = (double)wq[jb][h] * (a > 0.0 ? a : 0.0);
              }
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) score[ib][jb][i] = score[ib][jb][i] + prod[i];
      }
  }
  // the 64 x 64 scores leave through LDS (the limb buffer, free now), each
  // query row written as one contiguous 512-byte run; column k of row q sits
  // at k ^ 4 (q % 16), so that the 16 rows a store instruction touches fall
  // in different banks
  __syncthreads();
  double *st = (double *)&sl[0][0][0][0][0];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = 32 * qw + 16 * jb + c16, k = 32 * kw + 16 * ib + 4 * g4 + i;
        st[q * IM_K + (k ^ (4 * (q & 15)))] = score[ib][jb][i];
      }
  __syncthreads();
  const int64_t s = k0 + lane;
#pragma unroll 4
  for (int r = w; r < IT_Q; r += 4) {
    const int64_t ql = q0 + r;
    if (ql < p.tn && s < p.Tk) p.scores[(b * p.tn + ql) * p.Tk + s] = st[r * IM_K + (lane ^ (4 * (r & 15)))];
  }
}

// Few queries (decode): 32 keys per workgroup, rows staged in LDS (fp32,
// padded); thread (key, head) computes the head's dot for every query of the
// chunk, then thread (query, key) adds the heads in order.
constexpr int ID_KEYS = 32;
constexpr int ID_MAXQ = 4;
constexpr int ID_MAXHD = 256;  // HI * d staged per key

__global__ __launch_bounds__(256) void indexer_decode_kernel(IdxKP p) {
  __shared__ float sk[ID_KEYS][ID_MAXHD + 1];
  __shared__ double sqd[ID_MAXQ][ID_MAXHD];
  __shared__ double sdot[ID_MAXQ][ID_KEYS][8];  // HI <= 8
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t k0 = (int64_t)blockIdx.x * ID_KEYS;
  const int64_t hd = p.HI * p.d;
  for (int64_t i = tid; i < p.tn * hd; i += 256) {
    const int64_t tl = i / hd, c = i % hd;
    const int64_t h = c / p.d, dd = c % p.d;
    sqd[tl][c] = load_as_f64(p.q, b * p.q_sb + (p.t0 + tl) * p.q_st + h * p.q_sh + dd, p.dt);
  }
  for (int64_t i = tid; i < ID_KEYS * hd; i += 256) {
    const int64_t r = i / hd, c = i % hd;
    const int64_t s = k0 + r;
    float x = 0.f;
    if (s < p.Tk) {
      const int64_t h = c / p.d, dd = c % p.d;
      x = load_as_f32(p.k, b * p.k_sb + s * p.k_st + h * p.k_sh + dd, p.dt);
    }
    sk[r][c] = x;
  }
  __syncthreads();
  for (int64_t pair = tid; pair < ID_KEYS * p.HI; pair += 256) {
    const int64_t r = pair % ID_KEYS, h = pair / ID_KEYS;
    for (int64_t tl = 0; tl < p.tn; ++tl) {
      double dot = 0.0;
      for (int64_t dd = 0; dd < p.d; ++dd)
        dot = __builtin_fma(sqd[tl][h * p.d + dd], (double)sk[r][h * p.d + dd], dot);
      sdot[tl][r][h] = dot;
    }
  }
  __syncthreads();
  for (int64_t i = tid; i < ID_KEYS * p.tn; i += 256) {
    const int64_t r = i % ID_KEYS, tl = i / ID_KEYS;
    const int64_t s = k0 + r;
    if (s >= p.Tk) continue;
    const int64_t t = p.t0 + tl;
    double acc = 0.0;
    for (int64_t h = 0; h < p.HI; ++h) {
      const double dv = sdot[tl][r][h];
      const double rl = dv > 0.0 ? dv : 0.0;
      acc = add_product(acc, (double)p.w[b * p.w_sb + t * p.w_st + h * p.w_sh], rl);
    }
    p.scores[(b * p.tn + tl) * p.Tk + s] = acc;
  }
}

// Few queries over a long key axis with 2-byte keys whose (head, dim) block
// is contiguous and 16-byte aligned (the decode shape of config C5).  Every
// wave works on its own: a wave tile is 64/HI keys, lane (key, head) owns
// that key's head segment of d values.  The tile is loaded with coalesced
// 16-byte loads (lane l takes chunk l of each 1 KiB step), two tiles ahead
// for HI >= 4 (one otherwise), written to the wave's LDS rows (head segments
// of 2d + 16 bytes, which puts the 64 lanes' segments on different banks)
// and read back per lane.  Lane (key, head) computes that head's dot for
// every query of the chunk, d in order (q read from LDS as fp32, exact for
// 2-byte inputs, which halves the bytes of those reads); the head lanes of a
// key are adjacent, and the first adds the heads in order and writes the
// score.  No workgroup barrier inside the loop.  The loads are issued as inline assembly and
// waited for explicitly (the compiler's waits at the loop head were for
// every outstanding load).
constexpr int IDF_KEYS = 64;  // keys per workgroup step (one wave tile per wave)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 load16_async(const void *ptr) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(ptr));
  return v;
}
// the same load through the caches (for data many waves re-read)
__device__ __forceinline__ u32x4 load16_async_cached(const void *ptr) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(ptr));
  return v;
}

// Wait until at most N loads are outstanding; the chunks are operands so
// that no use of them is moved above the wait.
template <int N, int CH>
__device__ __forceinline__ void wait_chunks(u32x4 (&v)[CH]) {
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    if (i == 0)
      asm volatile("s_waitcnt vmcnt(%1)" : "+v"(v[i]) : "n"(N));
    else
      asm volatile("" : "+v"(v[i]));
  }
}

static size_t decode16_lds(int64_t tn, int64_t HI, int64_t d, bool hist0) {
  return (size_t)(4 * 64 * (2 * d + 16) + ((tn * HI * d + 3) & ~3) * 4 + tn * HI * 8) +
         (hist0 ? RX_BINS * 4 + 16 : 0);
}

// waves per SIMD the registers are sized for (two tiles of 16-byte chunks in
// flight for HI >= 4; HI < 4 lanes hold more chunks per tile)
template <int HI>
constexpr int idf_waves_per_eu() { return HI >= 4 ? 3 : HI == 2 ? 2 : 1; }

// TN1: the chunk has one query (the decode step), so one dot per lane; BF:
// bf16 keys (else fp16)
template <int HI, bool TN1, bool BF>
__global__ __launch_bounds__(256, idf_waves_per_eu<HI>()) void indexer_decode16_kernel(IdxKP p, int tiles) {
  constexpr int NQ = TN1 ? 1 : ID_MAXQ;
  constexpr int KW = 64 / HI;            // keys per wave tile
  constexpr int CH = ID_MAXHD / 8 / HI;  // 16-byte chunks per lane (most)
  constexpr bool TWO = HI >= 4;          // two tiles in flight
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t b = blockIdx.y;
  const int d = (int)p.d;
  const int hd = HI * d;
  const int ch = d / 8;       // chunks per lane in use (<= CH)
  const int cpr = hd / 8;     // chunks per key row
  const int hs = 2 * d + 16;  // LDS head segment
  const int tn = (int)p.tn;
  unsigned char *rows = smem + w * 64 * hs;              // this wave's KW rows of HI segments
  float *sqf = (float *)(smem + 4 * 64 * hs);            // q [tn][hd] (fp32: exact for 2-byte inputs)
  double *sw = (double *)(sqf + ((tn * hd + 3) & ~3));   // head weights [tn][HI]
  uint32_t *lh = (uint32_t *)(sw + tn * HI);             // first-digit histogram (hist0)
  uint32_t *s_ok = lh + RX_BINS;                          // the flush's go-ahead (hist0)
  const bool hist = TN1 && p.hist0 != nullptr;
  // the keys the top-k sees: a causal decode query at pos sees keys s <= pos / unit
  int64_t n_v = p.Tk;
  if (p.causal) {
    const int64_t pos = p.offset + p.t0;
    n_v = pos >= 0 ? min(p.Tk, pos / p.unit + 1) : 0;
  }
  if (hist)
    for (int i = tid; i < RX_BINS; i += 256) lh[i] = 0u;
  const bool prep = hist && p.rx_ready != nullptr;
  if (prep && blockIdx.x == 0) {  // the row's radix records start from zero
    uint4 *r = (uint4 *)(p.hist0 + b * p.hist_stride);
    for (int64_t i = tid; i < p.hist_stride / 4; i += 256) r[i] = make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // every wave's zeros reach the device
    __syncthreads();
    if (tid == 0)
      __hip_atomic_store(&p.rx_ready[b], *p.rx_epoch + p.rx_gen, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Adds this workgroup's first-digit counts into the row's histogram, after
  // the row's records are cleared (a wait on the row's first workgroup, which
  // is dispatched before every other workgroup of the row and clears them
  // before anything else; the wait is bounded, a hardware-fault guard that
  // raises LA_DEV_TOPK_TIMEOUT and leaves the counts out).
  auto flush = [&]() {
    if (tid == 0) {
      uint32_t ok = 1, spins = 0;
      if (prep) {
        const uint64_t want = *p.rx_epoch + p.rx_gen;
        for (;;) {
          if (spins >= p.spin_limit) {
            ok = 0;
            __hip_atomic_fetch_or(&la_ix_status, (uint32_t)LA_DEV_TOPK_TIMEOUT, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          if (__hip_atomic_load(&p.rx_ready[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == want)
            break;
          ++spins;
          __builtin_amdgcn_s_sleep(2);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the zeros before the adds
      }
      *s_ok = ok;
    }
    __syncthreads();
    if (!*s_ok) return;
    for (int i = tid; i < RX_BINS; i += 256) {
      const uint32_t x = lh[i];
      if (x) __hip_atomic_fetch_add(&p.hist0[b * p.hist_stride + i], x, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  const uint16_t *kb = (const uint16_t *)p.k + b * p.k_sb;
  // wave tiles of this workgroup: [wt0, wt0 + 4 * tiles * HI / ... ) interleaved over waves
  const int64_t n_wt = (p.Tk + KW - 1) / KW;
  const int64_t wt0 = (int64_t)blockIdx.x * tiles * HI;  // `tiles` 64-key steps = tiles*HI wave tiles
  const int64_t wt_end = min(n_wt, wt0 + (int64_t)tiles * HI);
  const int nw = wt0 + w < wt_end ? (int)((wt_end - wt0 - w + 3) / 4) : 0;  // this wave's tiles
  for (int i = tid; i < tn * hd; i += 256) {
    const int tl = i / hd, c = i % hd;
    const int h = c / d, dd = c % d;
    sqf[tl * hd + c] = load_as_f32(p.q, b * p.q_sb + (p.t0 + tl) * p.q_st + h * p.q_sh + dd, p.dt);
  }
  for (int i = tid; i < tn * HI; i += 256)
    sw[i] = (double)p.w[b * p.w_sb + (p.t0 + i / HI) * p.w_st + (i % HI) * p.w_sh];
  __syncthreads();
  if (nw == 0) {  // no tiles for this wave: only the histogram's flush remains
    if (hist) flush();
    return;
  }
  // chunk i of lane l in the coalesced load of a wave tile: c = i*64 + l of
  // the tile's KW x cpr chunks (past the end: the tile's last chunk again).
  // The loads past the wave's last tile (issued so that every step waits for
  // the same count) read the sequence's first tile through the caches, where
  // every wave's tail finds it, instead of streaming a tile from HBM again.
  auto fetch = [&](u32x4 (&v)[CH], int k) {  // k-th tile of this wave
    const bool tail = k >= nw;  // (wave-uniform)
    const int64_t key0 = tail ? 0 : (wt0 + w + 4 * (int64_t)k) * KW;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = min(i * 64 + lane, KW * cpr - 1);
      const int64_t s = min(key0 + c / cpr, p.Tk - 1);
      const uint16_t *src = kb + s * p.k_st + (c % cpr) * 8;
      v[i] = tail ? load16_async_cached(src) : load16_async(src);
    }
  };
  auto stage = [&](const u32x4 (&v)[CH]) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = i * 64 + lane;
      if (i < ch) {
        const int r = c / cpr, col = c % cpr;
        *(u32x4 *)(rows + r * HI * hs + (col / ch) * hs + (col % ch) * 16) = v[i];
      }
    }
  };
  auto compute = [&](int k) {
    const int64_t key0 = (wt0 + w + 4 * (int64_t)k) * KW;
    const int kr = lane / HI, h = lane % HI;
    const unsigned char *seg = rows + kr * HI * hs + h * hs;
    double dot[NQ];
#pragma unroll
    for (int tl = 0; tl < NQ; ++tl) dot[tl] = 0.0;
    for (int dd = 0; dd < d; dd += 8) {
      const u32x4 kv = *(const u32x4 *)(seg + dd * 2);
      double kf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (BF) {
          kf[2 * e] = (double)bf16lo(kv[e]);
          kf[2 * e + 1] = (double)bf16hi(kv[e]);
        } else {
          kf[2 * e] = (double)__half2float(__ushort_as_half((uint16_t)(kv[e] & 0xffffu)));
          kf[2 * e + 1] = (double)__half2float(__ushort_as_half((uint16_t)(kv[e] >> 16)));
        }
      }
#pragma unroll
      for (int tl = 0; tl < NQ; ++tl) {
        if (tl >= tn) break;
        const float4 qa = *(const float4 *)&sqf[tl * hd + h * d + dd];
        const float4 qb = *(const float4 *)&sqf[tl * hd + h * d + dd + 4];
        const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) dot[tl] = __builtin_fma((double)qv[e], kf[e], dot[tl]);
      }
    }
    // heads of a key are lanes kr*HI + 0..HI-1: the first adds them in order
    const int64_t s = key0 + kr;
#pragma unroll
    for (int tl = 0; tl < NQ; ++tl) {
      if (tl >= tn) break;
      double acc = 0.0;
#pragma unroll
      for (int hh = 0; hh < HI; ++hh) {
        const double dv = __shfl(dot[tl], kr * HI + hh, 64);
        const double rl = dv > 0.0 ? dv : 0.0;
        acc = add_product(acc, sw[tl * HI + hh], rl);
      }
      if (h == 0 && s < p.Tk) p.scores[(b * p.tn + tl) * p.Tk + s] = acc;
      if (hist && h == 0 && s < n_v) atomicAdd(&lh[(uint32_t)(ord_key(acc) >> (64 - RX_RB))], 1u);
    }
  };
  u32x4 va[CH];
  if constexpr (TWO) {
    u32x4 vb[CH];
    fetch(va, 0);
    fetch(vb, 1);
    for (int k = 0; k < nw; k += 2) {
      wait_chunks<CH, CH>(va);  // vb's loads (and at most a store) may still be in flight
      stage(va);
      fetch(va, k + 2);
      compute(k);
      if (k + 1 >= nw) break;
      wait_chunks<CH, CH>(vb);
      stage(vb);
      fetch(vb, k + 3);
      compute(k + 1);
    }
  } else {
    fetch(va, 0);
    for (int k = 0; k < nw; ++k) {
      wait_chunks<0, CH>(va);
      stage(va);
      fetch(va, k + 1);
      compute(k);
    }
  }
  wait_vmcnt<0>();  // drain the last (repeated) loads before the wave ends
  if (hist) flush();
}

template <int HI, bool TN1, bool BF>
static int launch_decode16(const IdxKP &p, size_t lds, dim3 grid, int tiles, hipStream_t st) {
  if (lds > 65536) {
    static bool attr_set = false;
    if (!attr_set) {
      LA_HIP(hipFuncSetAttribute((const void *)indexer_decode16_kernel<HI, TN1, BF>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      attr_set = true;
    }
  }
  indexer_decode16_kernel<HI, TN1, BF><<<grid, 256, lds, st>>>(p, tiles);
  LA_LAUNCHED();
  return LA_OK;
}

template <int HI>
static int dispatch_decode16(const IdxKP &p, hipStream_t st) {
  const size_t lds = decode16_lds(p.tn, HI, p.d, p.hist0 != nullptr);
  // a few workgroups per CU (by LDS, at most 4), each walking consecutive
  // 64-key steps of one batch row; four rounds of them, so that the
  // dispatcher evens out workgroups that stream slower than others (one
  // round left the last ones alone on the device: C5 0.297 -> 0.288 ms)
  const int64_t per_cu = std::max<int64_t>(
      1, std::min<int64_t>(idf_waves_per_eu<HI>(), (int64_t)(160 * 1024) / (int64_t)lds));
  const int64_t n_tiles = ceil_div(p.Tk, IDF_KEYS);
  const int64_t want = std::max<int64_t>(1, (int64_t)num_cus() * per_cu * 4 / p.B);
  const int tiles = (int)std::max<int64_t>(1, ceil_div(n_tiles, want));
  const dim3 grid((unsigned)ceil_div(n_tiles, tiles), (unsigned)p.B);
  if (p.dt == LA_BF16)
    return p.tn == 1 ? launch_decode16<HI, true, true>(p, lds, grid, tiles, st)
                     : launch_decode16<HI, false, true>(p, lds, grid, tiles, st);
  return p.tn == 1 ? launch_decode16<HI, true, false>(p, lds, grid, tiles, st)
                   : launch_decode16<HI, false, false>(p, lds, grid, tiles, st);
}

static int64_t pick_chunk(const la_indexer_args *a) {
  if (a->q_chunk > 0) return std::min(a->q_chunk, a->Tq);
  const int64_t budget = (int64_t)1 << 30;  // 1 GiB of fp64 scores per pass
  const int64_t per_q = a->B * a->Tk * 8;
  int64_t c = std::max<int64_t>(1, budget / std::max<int64_t>(per_q, 1));
  if (c >= IT_Q) c = c / IT_Q * IT_Q;
  return std::min(c, a->Tq);
}

static int validate(const la_indexer_args *a) {
  LA_REQUIRE(a && a->q && a->kk && a->w && a->out_idx, "la_indexer_topk: null pointer");
  LA_REQUIRE(a->B > 0 && a->Tq > 0 && a->Tk > 0 && a->HI > 0 && a->d > 0 && a->k > 0,
             "la_indexer_topk: bad shape");
  LA_REQUIRE(a->in_dtype == LA_F32 || a->in_dtype == LA_BF16 || a->in_dtype == LA_F16,
             "la_indexer_topk: q/k must be fp32, bf16 or fp16");
  LA_REQUIRE(a->HI <= 8, "la_indexer_topk: at most 8 indexer heads");
  LA_REQUIRE(a->Tk < ((int64_t)1 << 31), "la_indexer_topk: Tk >= 2^31");
  LA_REQUIRE(a->order == 0 || a->order == 1, "la_indexer_topk: order must be 0 or 1");
  LA_REQUIRE(a->order == 0 || !a->out_val, "la_indexer_topk: index order returns no values");
  return LA_OK;
}

}  // namespace la

using namespace la;

// Top-k parameters for the queries [t0, t0 + tn) whose scores are in `scores`.
static TopkKParams topk_params(const la_indexer_args *a, double *scores, int64_t t0, int64_t tn) {
  TopkKParams tp{};
  tp.scores = scores;
  tp.row_stride = a->Tk;
  tp.G = 1;
  tp.Tq = tn;
  tp.NG = a->B * tn;
  tp.t_base = t0;
  tp.out_tq = a->Tq;
  tp.n = a->Tk;
  tp.k = a->k;
  tp.width = a->k;
  tp.pos_off = a->causal ? a->offset : 0;
  tp.pos_unit = a->causal ? std::max<int64_t>(1, a->causal_unit) : 0;
  tp.order = a->order;
  tp.out_idx = a->out_idx;
  tp.out_val = a->out_val;
  return tp;
}

// The status word read (and, with clear, reset) in one atomic exchange on the
// caller's stream.
__device__ uint32_t la_ix_status_snap;
__global__ void ix_status_kernel(int clear) {
  la_ix_status_snap = clear ? __hip_atomic_exchange(&la_ix_status, 0u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                            : __hip_atomic_load(&la_ix_status, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
}

namespace la {
int indexer_status(uint32_t *bits, bool clear, hipStream_t st) {
  ix_status_kernel<<<1, 1, 0, st>>>(clear ? 1 : 0);
  LA_LAUNCHED();
  LA_HIP(hipMemcpyFromSymbolAsync(bits, HIP_SYMBOL(la_ix_status_snap), sizeof(uint32_t), 0,
                                  hipMemcpyDeviceToHost, st));
  LA_HIP(hipStreamSynchronize(st));
  return LA_OK;
}
}  // namespace la

// A value of each call (the counter starts at a random 64-bit value and
// steps by one), for the rows' ready words: with the epoch added, no word
// left over in the workspace holds the value a call waits for.
static uint64_t next_radix_gen() {
  static std::atomic<uint64_t> gen{[] {
    std::random_device rd;
    return ((uint64_t)rd() << 32) ^ (uint64_t)rd();
  }()};
  return gen.fetch_add(1) + 1;
}

static int64_t scores_bytes(const la_indexer_args *a, int64_t chunk) {
  return (a->B * chunk * a->Tk * 8 + 255) / 256 * 256;
}

// The integer-limb score kernel applies: bf16 q and k in 16-byte aligned
// (head, 64-d) rows, a few queries or more (not the decode forms).
static bool use_limbs(const la_indexer_args *a) {
  const bool decode = a->Tq <= ID_MAXQ && a->HI * a->d <= ID_MAXHD;
  return !decode && a->in_dtype == LA_BF16 && a->d == 64 &&
         (a->HI == 1 || a->HI == 2 || a->HI == 4 || a->HI == 8) && a->q_st % 8 == 0 &&
         a->q_sh % 8 == 0 && a->q_sb % 8 == 0 && a->k_st % 8 == 0 && a->k_sh % 8 == 0 &&
         a->k_sb % 8 == 0 && (uintptr_t)a->q % 16 == 0 && (uintptr_t)a->kk % 16 == 0;
}

// 16-row blocks of a padded (64-row multiple) run of n rows
static int64_t limb_blocks(int64_t n) { return ceil_div(n, 64) * 4; }

// Bytes of the limb form: the blocks (4 KiB per block and head) and the
// exponent words (4 bytes per row and head) of q (one chunk) and of k.
static int64_t limbs_bytes(const la_indexer_args *a, int64_t chunk) {
  if (!use_limbs(a)) return 0;
  const int64_t nq = limb_blocks(chunk), nk = limb_blocks(a->Tk);
  return (a->B * (nq + nk) * a->HI * (4096 + 16 * 4) + 255) / 256 * 256;
}

extern "C" size_t la_indexer_topk_workspace(const la_indexer_args *a) {
  if (validate(a) != LA_OK) return 0;
  const int64_t chunk = pick_chunk(a);
  return (size_t)(scores_bytes(a, chunk) + topk_workspace_bytes(topk_params(a, nullptr, 0, chunk)) +
                  limbs_bytes(a, chunk));
}

extern "C" int la_indexer_topk(const la_indexer_args *a, void *stream) {
  int rc = validate(a);
  if (rc != LA_OK) return rc;
  const int64_t chunk = pick_chunk(a);
  const int64_t sc_bytes = scores_bytes(a, chunk);
  const int64_t tk_bytes = topk_workspace_bytes(topk_params(a, nullptr, 0, chunk));
  const size_t need = (size_t)(sc_bytes + tk_bytes + limbs_bytes(a, chunk));
  if (!a->workspace || (size_t)a->ws_bytes < need)
    return fail(LA_ERR_WORKSPACE, "la_indexer_topk: workspace %lld < %zu bytes",
                (long long)a->ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const bool decode = a->Tq <= ID_MAXQ && a->HI * a->d <= ID_MAXHD;
  // fast decode form: 2-byte keys, (head, dim) block contiguous and 16-byte aligned
  const bool decode16 = decode && (a->in_dtype == LA_BF16 || a->in_dtype == LA_F16) &&
                        (a->HI == 1 || a->HI == 2 || a->HI == 4 || a->HI == 8) &&
                        a->k_sh == a->d && a->d % 8 == 0 && a->k_st % 8 == 0 &&
                        a->k_sb % 8 == 0 && (uintptr_t)a->kk % 16 == 0;
  // 2-byte q and k, 16-byte aligned (head, d) rows with d a multiple of 8
  const bool tile16 = (a->in_dtype == LA_BF16 || a->in_dtype == LA_F16) && a->d % 8 == 0 &&
                      a->q_st % 8 == 0 && a->q_sh % 8 == 0 && a->q_sb % 8 == 0 &&
                      a->k_st % 8 == 0 && a->k_sh % 8 == 0 && a->k_sb % 8 == 0 &&
                      (uintptr_t)a->q % 16 == 0 && (uintptr_t)a->kk % 16 == 0;
  // the limb form of k (once per call) and its buffers; q's per chunk below
  const bool limbs = use_limbs(a);
  const int64_t nqb = limb_blocks(chunk), nkb = limb_blocks(a->Tk);
  int8_t *lk = nullptr, *lq = nullptr;
  int32_t *xk = nullptr, *xq = nullptr;
  if (limbs) {
    char *base = (char *)a->workspace + sc_bytes + (tk_bytes + 255) / 256 * 256;
    lk = (int8_t *)base;
    lq = lk + a->B * nkb * a->HI * 4096;
    xk = (int32_t *)(lq + a->B * nqb * a->HI * 4096);
    xq = xk + a->B * nkb * 16 * a->HI;
  }
  // k's limbs go with the first query chunk's, in one launch
  const LimbRun run_k{(const uint16_t *)a->kk, a->k_sb, a->k_st, a->k_sh, 0, a->Tk, nkb * 16, lk, xk};
  const uint32_t blocks_k = (uint32_t)(a->B * nkb * 16 * a->HI / 16);  // 16 lanes per (row, head)
  for (int64_t t0 = 0; t0 < a->Tq; t0 += chunk) {
    IdxKP p{};
    p.q = a->q;
    p.k = a->kk;
    p.w = a->w;
    p.scores = (double *)a->workspace;
    p.B = a->B;
    p.Tq = a->Tq;
    p.Tk = a->Tk;
    p.HI = a->HI;
    p.d = a->d;
    p.q_sb = a->q_sb; p.q_st = a->q_st; p.q_sh = a->q_sh;
    p.k_sb = a->k_sb; p.k_st = a->k_st; p.k_sh = a->k_sh;
    p.w_sb = a->w_sb; p.w_st = a->w_st; p.w_sh = a->w_sh;
    p.t0 = t0;
    p.tn = std::min(chunk, a->Tq - t0);
    p.offset = a->offset;
    p.dt = a->in_dtype;
    p.causal = a->causal;
    p.unit = std::max<int64_t>(1, a->causal_unit);
    const TopkKParams tp = topk_params(a, p.scores, t0, p.tn);
    void *tws = (char *)a->workspace + sc_bytes;
    // a decode step whose rows go to the multi-workgroup radix select: the
    // scores kernel histograms the first digit on the way
    // and clears the rows' radix records itself (no set-up launch)
    const RadixPlan R = decode16 && p.tn == 1 ? topk_long_plan(tp) : RadixPlan{};
    if (R.C > 0) {
      LA_REQUIRE(tp.NG < 65536, "la_indexer_topk: at most 65535 batch rows per call");
      const RadixRowPrep rp = radix_row_prep(tp, R, tws);
      p.hist0 = rp.rows;
      p.hist_stride = rp.row_words;
      p.rx_ready = rp.ready;
      p.rx_epoch = rp.epoch;
      p.rx_gen = next_radix_gen();
      p.spin_limit = rx_spin_limit();
    }
    if (decode16) {
      switch (a->HI) {
        case 1: rc = dispatch_decode16<1>(p, st); break;
        case 2: rc = dispatch_decode16<2>(p, st); break;
        case 4: rc = dispatch_decode16<4>(p, st); break;
        default: rc = dispatch_decode16<8>(p, st); break;
      }
      if (rc != LA_OK) return rc;
    } else if (decode) {
      indexer_decode_kernel<<<dim3((unsigned)ceil_div(a->Tk, ID_KEYS), (unsigned)a->B), 256, 0,
                              st>>>(p);
    } else {
      const dim3 grid((unsigned)ceil_div(a->Tk, IT_K), (unsigned)ceil_div(p.tn, IT_Q), (unsigned)a->B);
      const dim3 grid_m((unsigned)ceil_div(a->Tk, IM_K), (unsigned)ceil_div(p.tn, IT_Q),
                        (unsigned)a->B);
      if (limbs) {
        const LimbRun run_q{(const uint16_t *)a->q, a->q_sb, a->q_st, a->q_sh, t0, p.tn, nqb * 16, lq, xq};
        const uint32_t blocks_q = (uint32_t)(a->B * nqb * 16 * a->HI / 16);
        if (t0 == 0)
          indexer_limb_kernel<<<dim3(blocks_k + blocks_q), 256, 0, st>>>(run_k, run_q, a->HI, blocks_k);
        else
          indexer_limb_kernel<<<dim3(blocks_q), 256, 0, st>>>(run_q, run_q, a->HI, blocks_q);
        LA_LAUNCHED();
        p.lq = lq;
        p.lk = lk;
        p.xq = xq;
        p.xk = xk;
        p.nqb = nqb;
        p.nkb = nkb;
        switch (a->HI) {
          case 1: indexer_i8_kernel<1><<<grid_m, IM_NT, 0, st>>>(p); break;
          case 2: indexer_i8_kernel<2><<<grid_m, IM_NT, 0, st>>>(p); break;
          case 4: indexer_i8_kernel<4><<<grid_m, IM_NT, 0, st>>>(p); break;
          default: indexer_i8_kernel<8><<<grid_m, IM_NT, 0, st>>>(p); break;
        }
      } else if (tile16 && a->in_dtype == LA_BF16)
        indexer_mfma_kernel<true><<<grid_m, IM_NT, 0, st>>>(p);
      else if (tile16)
        indexer_mfma_kernel<false><<<grid_m, IM_NT, 0, st>>>(p);
      else
        indexer_tile_kernel<<<grid, IT_NT, 0, st>>>(p);
    }
    LA_LAUNCHED();
    rc = R.C > 0 ? topk_radix_finish(tp, R, tws, true, true, st)
                 : topk_launch_ws(tp, tws, tk_bytes, st);
    if (rc != LA_OK) return rc;
  }
  return LA_OK;
}
