// XAttention block selection on gfx950 (variants/selection.py:500-595).
//
// One workgroup per (b, query head h, query block qb) row.  The row's query
// block (blk rows, zero past Tq) is staged in LDS as fp32 (exact for the
// input types); every visible key block kb (kb*blk <= qb*blk + offset) gets
// the strided antidiagonal scores of selection.py:528-566: slot s (offset
// o = s*r, o <= 2*blk - 2) sums the entries (i, o - i) of the (query block,
// key block) gram matrix, key rows past T counting as zero rows (F.pad).
// Arithmetic is fixed so that the CPU oracle reproduces every bit:
//   entry  = sum_d q[i][d] * k[j][d] in fp64, d increasing (exact products);
//   slot   = entries added in increasing i, then times inv_sqrt_d (a host
//            constant, fl(1/fl(sqrt(D))));
//   weight = exp_det(slot - row max) (below), as a fixed-point integer
//            rint(weight * 2^F), F = 52 - ceil(log2(n_kb * n_slots)), so that
//            block masses (the sum over a block's slots) and their totals are
//            exact integer sums below 2^53 in any order;
//   threshold mode (the paper's rule, _cumulative_select, selection.py:62-69):
//            with blocks ordered by (mass desc, index asc) and C_m the sum of
//            the first m masses, keep n = 1 + #{m : C_m < ceil(alpha * Z)}
//            blocks (Z the row's total; alpha * Z > Z keeps every block);
//            found without a sort by a bitwise search for the largest mass
//            value v with sum(mass >= v) >= thr, then every block above v and
//            the first 1 + (thr - 1 - sum(mass > v)) / v blocks equal to v;
//   top-k mode: the top min(topk, n_kb) blocks by (mass desc, index asc).
// The own block (first token at qb*blk + offset) is OR'd in and the blocks
// past causality dropped (selection.py:591-592); the list is written in
// ascending order.
#include <algorithm>
#include <cmath>

#include "common.h"
#include "topk_select.h"

#pragma clang fp contract(off)

namespace la {

__host__ __device__ constexpr int64_t xa_align16(int64_t x) { return (x + 15) & ~(int64_t)15; }

// exp(x) for x <= 0 with a fixed sequence of correctly rounded operations
// (the CPU oracle runs the same sequence): 0 below -700; x = k*ln2 + r by a
// two-part ln2 (the fdlibm split) with fused multiply-adds; e^r by its
// degree-13 Taylor polynomial in Horner form (fma); times 2^k from exponent
// bits (exact, 2^k is normal for x > -700).
__device__ __forceinline__ double exp_det(double x) {
  if (!(x > -700.0)) return 0.0;
  const double kf = __builtin_rint(x * 1.4426950408889634);
  double r = __builtin_fma(-kf, 6.93147180369123816490e-01, x);
  r = __builtin_fma(-kf, 1.90821492927058770002e-10, r);
  double p = 1.6059043836821613e-10;
  p = __builtin_fma(p, r, 2.08767569878681e-09);
  p = __builtin_fma(p, r, 2.505210838544172e-08);
  p = __builtin_fma(p, r, 2.755731922398589e-07);
  p = __builtin_fma(p, r, 2.7557319223985893e-06);
  p = __builtin_fma(p, r, 2.48015873015873e-05);
  p = __builtin_fma(p, r, 0.0001984126984126984);
  p = __builtin_fma(p, r, 0.001388888888888889);
  p = __builtin_fma(p, r, 0.008333333333333333);
  p = __builtin_fma(p, r, 0.041666666666666664);
  p = __builtin_fma(p, r, 0.16666666666666666);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const double two_k = __longlong_as_double((long long)((int64_t)kf + 1023) << 52);
  return p * two_k;
}

struct XaKP {
  const void *q, *k;
  int32_t *out_idx, *out_count;
  const double *alpha;  // per query head (threshold mode)
  double *slots;        // optional: [b][h][qb - qc0][kb][slot] scored by xattn_slots_mfma_kernel
  int64_t B, Hq, Hkv, Tq, T, D;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st;
  int64_t blk, r, n_slots, offset, n_qb, n_kb, topk, width;
  double inv_sqrt_d, two_f;
  int32_t in_dt, mode;  // mode 0: threshold, 1: top-k
  // the launch covers query blocks [qc0, qc0 + n_qc) (rows (b, h, qb) of
  // that range, numbered b, h, qb - qc0 within the launch)
  int64_t qc0, n_qc;
};

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t *red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += (uint64_t)__shfl_xor((unsigned long long)v, off, 64);
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int x = 0; x < TK_NW; ++x) t += red[x];
  __syncthreads();
  return t;
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t *red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = (uint64_t)__shfl_xor((unsigned long long)v, off, 64);
    v = o > v ? o : v;
  }
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int x = 0; x < TK_NW; ++x) t = red[x] > t ? red[x] : t;
  __syncthreads();
  return t;
}

// Slot scores on the fp64 matrix cores when stride == block (>= 2): slot 0
// of (qb, kb) is entry (0, 0) and slot 1 the entries (i, block - i),
// i = 1 .. block-1, so query row qb*block + i only meets key rows kb*block +
// ((block - i) mod block): for each residue i the entries of every (qb, kb)
// form one dense gram product G_i = Q_i K_i^T (Q_i the query rows i mod
// block, K_i the key rows -i mod block).  slot0 = (0 + G_0) * inv_sqrt_d and
// slot1 = (((0 + G_1) + G_2) + ... + G_{block-1}) * inv_sqrt_d, the oracle's
// order.  A workgroup covers 64 query blocks x 64 key blocks of one (b, h);
// wave w computes key blocks [kb0 + 32 (w % 2), +32) x query blocks
// [qb0 + 32 (w / 2), +32) as 2 x 2 tiles of v_mfma_f64_16x16x4f64 (A = key
// rows, B = query rows, one value per lane; lane l supplies d = 4 c + l / 16
// of chunk c and receives D[4 e + l / 16][l % 16]).  The instruction
// accumulates in k order and a product of 2-byte values is exact in fp64,
// so the entries carry the bits of the sequential sum over d.  Rows past Tq
// or T are zero rows (F.pad).  Slices of 64 dims are staged in LDS as fp32
// (rows padded to 68 floats: conflict-free fragment reads), the next slice
// loaded into registers during this one.  Tiles wholly past causality are
// skipped.
constexpr int XM_T = 64, XM_D = 64, XM_S = XM_D + 4, XM_NT = 256;

template <bool BF>
__device__ __forceinline__ void xm_widen8(const uint4 &v, float (&x)[8]) {
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

template <bool BF>
// Three workgroups per CU (168 VGPRs; the few spills are outside the
// product loop): 5 % faster than two at 178 VGPRs without spills.
__global__ __launch_bounds__(XM_NT, 3) void xattn_slots_mfma_kernel(XaKP p) {
  typedef double f64x4 __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) float sq[XM_T][XM_S];
  __shared__ __align__(16) float sk[XM_T][XM_S];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r16 = lane & 15, kq = lane >> 4;
  const int64_t kb0 = (int64_t)blockIdx.x * XM_T, qb0 = p.qc0 + (int64_t)blockIdx.y * XM_T;
  const int64_t qend = p.qc0 + p.n_qc;  // first query block past the launch's range
  const int64_t bh = blockIdx.z, b = bh / p.Hq, h = bh % p.Hq, kvh = h / (p.Hq / p.Hkv);
  const int64_t blk = p.blk;
  const int D = (int)p.D;
  if (qb0 >= qend) return;
  const int64_t qlast = min(qb0 + XM_T, qend) - 1;
  if (kb0 * blk > qlast * blk + p.offset) return;  // every key block past causality
  const uint16_t *qbase = (const uint16_t *)p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t *kbase = (const uint16_t *)p.k + b * p.k_sb + kvh * p.k_sh;
  // slice loads: chunk c (< 512) is row c / 8, 16-byte chunk c % 8, for the
  // query rows (qb0 + row) * blk + i and the key rows (kb0 + row) * blk + j
  uint4 lq[2], lk[2];
  auto fetch = [&](int64_t i, int d0) {
    const int64_t j = (blk - i) % blk;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + u * XM_NT, r = c >> 3, dc = c & 7;
      const int dd = min(d0 + dc * 8, D - 8);
      const int64_t t = (qb0 + r) * blk + i, s = (kb0 + r) * blk + j;
      lq[u] = (qb0 + r < qend && t < p.Tq) ? *(const uint4 *)(qbase + t * p.q_st + dd)
                                              : uint4{0u, 0u, 0u, 0u};
      lk[u] = (kb0 + r < p.n_kb && s < p.T) ? *(const uint4 *)(kbase + s * p.k_st + dd)
                                             : uint4{0u, 0u, 0u, 0u};
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + u * XM_NT, r = c >> 3, dc = c & 7;
      float x[8];
      xm_widen8<BF>(lq[u], x);
      *(float4 *)&sq[r][dc * 8] = float4{x[0], x[1], x[2], x[3]};
      *(float4 *)&sq[r][dc * 8 + 4] = float4{x[4], x[5], x[6], x[7]};
      xm_widen8<BF>(lk[u], x);
      *(float4 *)&sk[r][dc * 8] = float4{x[0], x[1], x[2], x[3]};
      *(float4 *)&sk[r][dc * 8 + 4] = float4{x[4], x[5], x[6], x[7]};
    }
  };
  const int kw = w & 1, qw = w >> 1;
  const float *ka = &sk[32 * kw + r16][kq];
  const float *qa = &sq[32 * qw + r16][kq];
  // output slot of this lane's element (ib, jb, e): key block kb0 + 32 kw +
  // 16 ib + 4 e + kq, query block qb0 + 32 qw + 16 jb + r16
  auto store = [&](const f64x4 (&v)[2][2], int slot) {  // slot 0: (0 + entry) * inv_sqrt_d
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const int64_t qb = qb0 + 32 * qw + 16 * jb + r16;
      if (qb >= qend) continue;
      double *rowp = p.slots + ((bh * p.n_qc + qb - p.qc0) * p.n_kb) * p.n_slots + slot;
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t kb = kb0 + 32 * kw + 16 * ib + 4 * e + kq;
          if (kb < p.n_kb)
            rowp[kb * p.n_slots] = (slot == 0 ? 0.0 + v[ib][jb][e] : v[ib][jb][e]) * p.inv_sqrt_d;
        }
    }
  };
  f64x4 slot1[2][2];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) slot1[ib][jb] = f64x4{0.0, 0.0, 0.0, 0.0};
  fetch(0, 0);
  for (int64_t i = 0; i < blk; ++i) {
    f64x4 dot[2][2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) dot[ib][jb] = f64x4{0.0, 0.0, 0.0, 0.0};
    for (int d0 = 0; d0 < D; d0 += XM_D) {
      const int dn = min(XM_D, D - d0);
      __syncthreads();  // the previous slice is consumed
      stage();
      __syncthreads();
      {  // next slice in flight during this one
        const bool last_d = d0 + XM_D >= D;
        fetch(last_d ? min(i + 1, blk - 1) : i, last_d ? 0 : d0 + XM_D);
      }
      auto chunk = [&](int dd) {
        double a[2], bq[2];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          a[x] = (double)ka[16 * x * XM_S + dd];
          bq[x] = (double)qa[16 * x * XM_S + dd];
        }
#pragma unroll
        for (int ib = 0; ib < 2; ++ib)
#pragma unroll
          for (int jb = 0; jb < 2; ++jb)
            dot[ib][jb] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[ib], bq[jb], dot[ib][jb], 0, 0, 0);
      };
      if (dn == XM_D) {
#pragma unroll
        for (int dd = 0; dd < XM_D; dd += 4) chunk(dd);
      } else {
        for (int dd = 0; dd < dn; dd += 4) chunk(dd);
      }
    }
    if (i == 0) {
      store(dot, 0);
    } else {
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
          for (int e = 0; e < 4; ++e) slot1[ib][jb][e] = slot1[ib][jb][e] + dot[ib][jb][e];
    }
  }
  store(slot1, 1);
}

template <int KPT>
__global__ __launch_bounds__(TK_NT) void xattn_select_kernel(XaKP p) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ TkRegShared<KPT> sh;
  __shared__ uint64_t red[TK_NW];
  __shared__ double redd[TK_NW];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t lrow = blockIdx.x;  // (b, h, qb - qc0)
  const int64_t qb = p.qc0 + lrow % p.n_qc;
  const int64_t h = (lrow / p.n_qc) % p.Hq;
  const int64_t b = lrow / (p.n_qc * p.Hq);
  const int64_t row = (b * p.Hq + h) * p.n_qb + qb;  // the output row
  const int64_t kvh = h / (p.Hq / p.Hkv);
  const int64_t blk = p.blk, D = p.D, NS = p.n_slots, n_kb = p.n_kb;

  float *sq = (float *)dyn;                       // [blk][D]
  double *ss = (double *)(dyn + xa_align16(blk * D * 4));  // [n_kb][NS]
  uint32_t *bm = (uint32_t *)(ss + n_kb * NS);    // bitmap of kept blocks

  // visible key blocks: kb*blk <= qb*blk + offset
  const int64_t pos0 = qb * blk + p.offset;
  const int64_t lim = min(pos0 / blk, n_kb - 1);
  const int64_t n_vis = lim + 1;
  const int64_t kbase = b * p.k_sb + kvh * p.k_sh;

  if (p.slots) {  // scored on the matrix cores: the row's visible slots
    const double *src = p.slots + lrow * n_kb * NS;
    for (int64_t x = tid; x < n_vis * NS; x += TK_NT) ss[x] = src[x];
  } else {
    for (int64_t x = tid; x < blk * D; x += TK_NT) {
      const int64_t i = x / D, d = x % D, t = qb * blk + i;
      sq[x] = t < p.Tq ? load_as_f32(p.q, b * p.q_sb + h * p.q_sh + t * p.q_st + d, p.in_dt) : 0.f;
    }
  }
  for (int64_t x = tid; x < (n_kb + 31) / 32; x += TK_NT) bm[x] = 0u;
  __syncthreads();

  // slot scores of the visible blocks, one block per thread
  for (int64_t kb = p.slots ? n_vis : tid; kb < n_vis; kb += TK_NT) {
    for (int64_t s = 0; s < NS; ++s) {
      const int64_t o = s * p.r;
      double acc = 0.0;
      for (int64_t i = max((int64_t)0, o - blk + 1); i <= min(blk - 1, o); ++i) {
        const int64_t j = o - i, kr = kb * blk + j;
        const float *qi = sq + i * D;
        double e = 0.0;
        if (kr < p.T) {
          const int64_t ko = kbase + kr * p.k_st;
          if (p.in_dt == LA_BF16) {
            // 128 dims at a time: all sixteen 16-byte loads of the chunk are
            // issued before its (serial) fma chain
            const uint16_t *kp = (const uint16_t *)p.k + ko;
            for (int64_t d0 = 0; d0 < D; d0 += 128) {
              const int nch = (int)min((int64_t)16, (D - d0) / 8);
              uint4 kv[16];
#pragma unroll
              for (int c = 0; c < 16; ++c)
                if (c < nch) kv[c] = *(const uint4 *)(kp + d0 + 8 * c);
#pragma unroll
              for (int c = 0; c < 16; ++c) {
                if (c < nch) {
                  const uint32_t wv[4] = {kv[c].x, kv[c].y, kv[c].z, kv[c].w};
                  const float *qc = qi + d0 + 8 * c;
#pragma unroll
                  for (int u = 0; u < 4; ++u) {
                    e = __builtin_fma((double)qc[2 * u], (double)bf16lo(wv[u]), e);
                    e = __builtin_fma((double)qc[2 * u + 1], (double)bf16hi(wv[u]), e);
                  }
                }
              }
            }
          } else {
            for (int64_t d = 0; d < D; ++d)
              e = __builtin_fma((double)qi[d], (double)load_as_f32(p.k, ko + d, p.in_dt), e);
          }
        } else {
          // a zero key row (F.pad): the same operations on zeros
          for (int64_t d = 0; d < D; ++d) e = __builtin_fma((double)qi[d], 0.0, e);
        }
        acc = acc + e;
      }
      ss[kb * NS + s] = acc * p.inv_sqrt_d;
    }
  }
  __syncthreads();

  // row maximum over the visible slots (exact, any order)
  double mx = __int_as_float(0xff800000);
  for (int64_t x = tid; x < n_vis * NS; x += TK_NT) mx = fmax(mx, ss[x]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmax(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) redd[w] = mx;
  __syncthreads();
  mx = redd[0];
#pragma unroll
  for (int x = 1; x < TK_NW; ++x) mx = fmax(mx, redd[x]);

  // fixed-point block masses, kept in registers (block tid + 256 j)
  uint64_t u[KPT];
  uint64_t zpart = 0;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int64_t kb = tid + TK_NT * j;
    uint64_t m = 0;
    if (kb < n_vis) {
      for (int64_t s = 0; s < NS; ++s) {
        const double e = exp_det(ss[kb * NS + s] - mx);
        m += (uint64_t)__builtin_rint(e * p.two_f);
      }
    }
    u[j] = m;
    zpart += m;
  }
  const uint64_t Z = block_sum_u64(zpart, red);

  const uint64_t lt = lanemask_lt(lane);
  auto keep = [&](int64_t kb) {
    if (kb <= lim) atomicOr(&bm[kb >> 5], 1u << (kb & 31));
  };
  bool by_count = p.mode == 1;
  uint32_t K = (uint32_t)min(p.topk, n_kb);
  if (p.mode == 0) {
    const double thr_d = p.alpha[h] * (double)Z;
    if (thr_d > (double)Z) {  // every block
      for (int64_t kb = tid; kb < n_kb; kb += TK_NT) keep(kb);
    } else if (!(thr_d > 0.0)) {  // C_m < thr for no m: the top block alone
      by_count = true;
      K = 1;
    } else {
      const uint64_t thr = (uint64_t)ceil(thr_d);
      // largest v with sum(mass >= v) >= thr (v = 0 qualifies: the sum is Z)
      const uint64_t top = block_max_u64(
          [&] {
            uint64_t x = 0;
#pragma unroll
            for (int j = 0; j < KPT; ++j) x = u[j] > x ? u[j] : x;
            return x;
          }(),
          red);
      uint64_t v = 0;
      for (int bit = top ? 63 - __clzll((long long)top) : -1; bit >= 0; --bit) {
        const uint64_t v2 = v | (1ull << bit);
        uint64_t part = 0;
#pragma unroll
        for (int j = 0; j < KPT; ++j) part += u[j] >= v2 ? u[j] : 0ull;
        if (block_sum_u64(part, red) >= thr) v = v2;
      }
      uint64_t gpart = 0;
#pragma unroll
      for (int j = 0; j < KPT; ++j) gpart += u[j] > v ? u[j] : 0ull;
      const uint64_t s_gt = block_sum_u64(gpart, red);
      // ties at v taken in index order (block tid + 256 j: slot j, then
      // lower waves, then lower lanes)
      // v >= 1: sum(mass >= 1) = Z >= thr
      const uint64_t n_eq_take = v ? (thr - s_gt - 1) / v + 1 : 0;
      uint32_t *eqc = sh.eqc[0];  // [KPT][TK_NW]
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const bool eq = tid + TK_NT * j < n_kb && u[j] == v;
        const uint64_t bmsk = __ballot(eq);
        if (lane == 0) eqc[j * TK_NW + w] = (uint32_t)__popcll(bmsk);
      }
      __syncthreads();
      uint64_t eq_before = 0;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int64_t kb = tid + TK_NT * j;
        const bool eq = kb < n_kb && u[j] == v;
        const uint64_t bmsk = __ballot(eq);
        uint64_t rank = eq_before + (uint64_t)__popcll(bmsk & lt);
#pragma unroll
        for (int x = 0; x < TK_NW; ++x) rank += x < w ? eqc[j * TK_NW + x] : 0u;
        if (kb < n_kb && (u[j] > v || (eq && rank < n_eq_take))) keep(kb);
#pragma unroll
        for (int x = 0; x < TK_NW; ++x) eq_before += eqc[j * TK_NW + x];
      }
    }
  }
  if (by_count) {
    tk_reg_select_bits<KPT>(u, (int32_t)n_kb, K, sh, [&](int j, int32_t i, bool take) {
      if (take) keep(i);
    });
  }
  __syncthreads();
  // the own block (selection.py:591): the block whose first token is pos0
  if (tid == 0 && pos0 % blk == 0 && pos0 / blk < n_kb) keep(pos0 / blk);
  __syncthreads();
  tk_emit_bitmap_row(bm, n_kb, -1, 0, 0, p.width, p.out_idx + row * p.width, p.out_count + row,
                     sh.wtmp[1]);
}

// 64-bit lane exchanges within a wave (no LDS, no barrier): DPP moves within
// rows of 16 lanes, then the 16- and 32-lane swaps, on the two 32-bit halves.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)x, CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(x >> 32), CTRL, 0xf, 0xf, false);
  return ((uint64_t)hi << 32) | lo;
}
// (the value of lane l, the value of lane l ^ 16 or l ^ 32), lower lane first
template <bool P32>
__device__ __forceinline__ void swap_u64(uint64_t x, uint64_t &a, uint64_t &b) {
  const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
  const auto l = P32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                     : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto h = P32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                     : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  a = ((uint64_t)h[0] << 32) | l[0];
  b = ((uint64_t)h[1] << 32) | l[1];
}
// Sum (MAX = false) or maximum over the wave, in every lane.
template <bool MAX>
__device__ __forceinline__ uint64_t wave_red_u64(uint64_t x) {
  auto op = [](uint64_t a, uint64_t b) { return MAX ? (a > b ? a : b) : a + b; };
  x = op(x, dpp_u64<0xB1>(x));   // quad_perm [1,0,3,2]
  x = op(x, dpp_u64<0x4E>(x));   // quad_perm [2,3,0,1]
  x = op(x, dpp_u64<0x141>(x));  // row_half_mirror
  x = op(x, dpp_u64<0x140>(x));  // row_mirror
  uint64_t a, b;
  swap_u64<false>(x, a, b);
  x = op(a, b);
  swap_u64<true>(x, a, b);
  return op(a, b);
}

// The selection of xattn_select_kernel for rows whose slot scores are already
// in the workspace (stride == block) and that have at most 64 * KPL key
// blocks: one wave per row, block kb = lane + 64 j in slot j of the lane's
// registers, every reduction a lane exchange -- the ~40 steps of the
// threshold search take no barrier.  The arithmetic (row maximum, masses,
// the threshold and tie rules, top-k by (mass desc, block asc), the own
// block) is the block kernel's, so the lists are identical.
template <int KPL>
__global__ __launch_bounds__(256) void xattn_select_wave_kernel(XaKP p, int64_t n_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t lrow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b, h, qb - qc0)
  if (lrow >= n_rows) return;  // wave-uniform; the kernel has no barrier
  const int64_t qb = p.qc0 + lrow % p.n_qc;
  const int64_t h = (lrow / p.n_qc) % p.Hq;
  const int64_t row = (lrow / (p.n_qc * p.Hq) * p.Hq + h) * p.n_qb + qb;  // the output row
  const int64_t n_kb = p.n_kb, NS = p.n_slots, blk = p.blk;
  const int64_t pos0 = qb * blk + p.offset;
  const int64_t lim = min(pos0 / blk, n_kb - 1);
  const int64_t n_vis = lim + 1;
  const double *src = p.slots + lrow * n_kb * NS;
  const uint64_t lt = lanemask_lt(lane);

  double mx = __int_as_float(0xff800000);
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const int64_t kb = lane + 64 * j;
    if (kb < n_vis)
      for (int64_t s = 0; s < NS; ++s) mx = fmax(mx, src[kb * NS + s]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmax(mx, __shfl_xor(mx, off, 64));

  uint64_t u[KPL];
  uint64_t zpart = 0, umax = 0;
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const int64_t kb = lane + 64 * j;
    uint64_t m = 0;
    if (kb < n_vis)
      for (int64_t s = 0; s < NS; ++s) m += (uint64_t)__builtin_rint(exp_det(src[kb * NS + s] - mx) * p.two_f);
    u[j] = m;
    zpart += m;
    umax = m > umax ? m : umax;
  }
  const uint64_t Z = wave_red_u64<false>(zpart);
  const uint64_t top = wave_red_u64<true>(umax);

  uint32_t kbits = 0;  // bit j: block lane + 64 j is kept
  // Slots j >= jn hold only blocks past the visible ones (mass 0, never
  // kept): the searches skip them.  They add nothing to the sums, and as
  // ties at 0 they would rank after every visible block.
  const int jn = (int)min((int64_t)KPL, (n_vis + 63) / 64);
  auto listed = [&](int j) { return j < jn && lane + 64 * (int64_t)j < n_kb; };
  bool by_count = p.mode == 1;
  uint32_t K = (uint32_t)min(p.topk, n_kb);
  if (p.mode == 0) {
    const double thr_d = p.alpha[h] * (double)Z;
    if (thr_d > (double)Z) {  // every block
#pragma unroll
      for (int j = 0; j < KPL; ++j) kbits |= listed(j) ? 1u << j : 0u;
    } else if (!(thr_d > 0.0)) {  // C_m < thr for no m: the top block alone
      by_count = true;
      K = 1;
    } else {
      const uint64_t thr = (uint64_t)ceil(thr_d);
      // largest v with sum(mass >= v) >= thr (v = 0 qualifies: the sum is Z)
      uint64_t v = 0;
      for (int bit = top ? 63 - __clzll((long long)top) : -1; bit >= 0; --bit) {
        const uint64_t v2 = v | (1ull << bit);
        uint64_t part = 0;
#pragma unroll
        for (int j = 0; j < KPL; ++j)
          if (j < jn) part += u[j] >= v2 ? u[j] : 0ull;
        if (wave_red_u64<false>(part) >= thr) v = v2;
      }
      uint64_t gpart = 0;
#pragma unroll
      for (int j = 0; j < KPL; ++j)
        if (j < jn) gpart += u[j] > v ? u[j] : 0ull;
      const uint64_t s_gt = wave_red_u64<false>(gpart);
      const uint64_t n_eq_take = v ? (thr - s_gt - 1) / v + 1 : 0;
      // ties at v taken in block order (slot j, then lane: ascending kb)
      uint64_t eq_before = 0;
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        if (j >= jn) break;
        const bool eq = listed(j) && u[j] == v;
        const uint64_t bm = __ballot(eq);
        const uint64_t rank = eq_before + (uint64_t)__popcll(bm & lt);
        if (listed(j) && (u[j] > v || (eq && rank < n_eq_take))) kbits |= 1u << j;
        eq_before += (uint64_t)__popcll(bm);
      }
    }
  }
  if (by_count) {  // the K largest masses over the listed blocks, ties to the lower block
    uint64_t T = 0;
    for (int bit = top ? 63 - __clzll((long long)top) : -1; bit >= 0; --bit) {
      const uint64_t T2 = T | (1ull << bit);
      uint32_t c = 0;
#pragma unroll
      for (int j = 0; j < KPL; ++j)
        if (j < jn) c += (uint32_t)__popcll(__ballot(listed(j) && u[j] >= T2));
      if (c >= K) T = T2;
    }
    uint32_t gt = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j)
      if (j < jn) gt += (uint32_t)__popcll(__ballot(listed(j) && u[j] > T));
    const uint32_t need = K - gt;
    uint32_t eq_before = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      if (j >= jn) break;
      const bool eq = listed(j) && u[j] == T;
      const uint64_t bm = __ballot(eq);
      const uint32_t rank = eq_before + (uint32_t)__popcll(bm & lt);
      if (listed(j) && (u[j] > T || (eq && rank < need))) kbits |= 1u << j;
      eq_before += (uint32_t)__popcll(bm);
    }
  }
  // only visible blocks are kept, and the own block (selection.py:591)
  const int64_t own = (pos0 % blk == 0 && pos0 / blk < n_kb) ? pos0 / blk : -1;
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const int64_t kb = lane + 64 * j;
    if (kb > lim) kbits &= ~(1u << j);
    if (kb == own) kbits |= 1u << j;
  }
  // ascending list, -1 padded, count
  int32_t *out = p.out_idx + row * p.width;
  uint32_t total = 0;
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const bool k = (kbits >> j) & 1u;
    const uint64_t bm = __ballot(k);
    const uint32_t pos = total + (uint32_t)__popcll(bm & lt);
    if (k && pos < (uint32_t)p.width) out[pos] = (int32_t)(lane + 64 * j);
    total += (uint32_t)__popcll(bm);
  }
  for (int64_t jj = (int64_t)total + lane; jj < p.width; jj += 64) out[jj] = -1;
  if (lane == 0) p.out_count[row] = (int32_t)min((int64_t)total, p.width);
}

}  // namespace la

using namespace la;

static int64_t ceil_log2(int64_t x) {
  int64_t l = 0;
  while (((int64_t)1 << l) < x) ++l;
  return l;
}

static int xattn_lds(const la_xattn_select_args *a, int64_t n_kb, int64_t ns, size_t &bytes) {
  bytes = (size_t)xa_align16(a->block * a->D * 4) + (size_t)(n_kb * ns * 8) +
          (size_t)((n_kb + 31) / 32 * 4);
  return bytes <= 120 * 1024 ? LA_OK : LA_ERR_UNSUPPORTED;
}

// Slots on the matrix cores: stride == block >= 2, 2-byte q and k, 16-byte
// aligned rows with D a multiple of 8.
static bool xattn_mfma_shape(const la_xattn_select_args *a) {
  const bool two = a->in_dtype == LA_BF16 || a->in_dtype == LA_F16;
  return two && a->block >= 2 && a->stride == a->block && a->D % 8 == 0 &&
         (uintptr_t)a->q % 16 == 0 && (uintptr_t)a->k % 16 == 0 && a->q_sb % 8 == 0 &&
         a->q_sh % 8 == 0 && a->q_st % 8 == 0 && a->k_sb % 8 == 0 && a->k_sh % 8 == 0 &&
         a->k_st % 8 == 0;
}

// Query blocks scored per launch: all of them while their slot scores fit
// `avail` bytes, else a multiple of XM_T that does (0: not even XM_T do).
// The workspace asked for is bounded by XA_SLOT_BUDGET (not quadratic in T);
// a smaller workspace from the caller gives smaller chunks.
constexpr int64_t XA_SLOT_BUDGET = (int64_t)256 << 20;
static int64_t xattn_chunk_qb(const la_xattn_select_args *a, int64_t avail) {
  const int64_t n_kb = ceil_div(a->T, a->block), n_qb = ceil_div(a->Tq, a->block);
  const int64_t ns = (2 * a->block - 2) / a->stride + 1;
  const int64_t per_qb = std::max<int64_t>(a->B * a->Hq * n_kb * ns * 8, 1);
  const int64_t c = avail / per_qb;
  if (c >= n_qb) return n_qb;
  return c / XM_T * XM_T;
}

static int64_t xattn_slot_bytes(const la_xattn_select_args *a, int64_t cq) {
  const int64_t n_kb = ceil_div(a->T, a->block);
  const int64_t ns = (2 * a->block - 2) / a->stride + 1;
  return a->B * a->Hq * cq * n_kb * ns * 8;
}

// The block-per-row selection over rows [0, nrows) of the launch's chunk.
static int xattn_launch_select(const XaKP &p, int64_t n_kb, size_t lds, int64_t nrows,
                               hipStream_t st) {
  const int kpt = (int)ceil_div(n_kb, TK_NT);
  auto launch = [&](auto kern) -> int {
    if (lds > 64 * 1024)
      LA_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    kern<<<dim3((unsigned)nrows), TK_NT, lds, st>>>(p);
    return (int)LA_OK;
  };
  int rc;
  if (kpt <= 1)
    rc = launch(&xattn_select_kernel<1>);
  else if (kpt <= 4)
    rc = launch(&xattn_select_kernel<4>);
  else
    rc = launch(&xattn_select_kernel<16>);
  if (rc != LA_OK) return rc;
  LA_LAUNCHED();
  return LA_OK;
}

extern "C" size_t la_xattn_select_workspace(const la_xattn_select_args *a) {
  if (!a || a->B <= 0 || a->Hq <= 0 || a->Tq <= 0 || a->T <= 0 || a->block < 1 || a->stride < 1)
    return 0;
  if (!xattn_mfma_shape(a)) return 0;
  const int64_t cq = std::max<int64_t>(xattn_chunk_qb(a, XA_SLOT_BUDGET),
                                       std::min<int64_t>(XM_T, ceil_div(a->Tq, a->block)));
  return (size_t)xattn_slot_bytes(a, cq);
}

extern "C" int la_xattn_select(const la_xattn_select_args *a, void *stream) {
  LA_REQUIRE(a && a->q && a->k && a->out_idx && a->out_count, "la_xattn_select: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hq > 0 && a->Hkv > 0 && a->Tq > 0 && a->T > 0 && a->D > 0,
             "la_xattn_select: bad shape");
  LA_REQUIRE(a->Hq % a->Hkv == 0, "n_heads must be a multiple of n_kv_heads");
  LA_REQUIRE(a->block >= 1 && a->block <= 64 && a->stride >= 1, "la_xattn_select: block in [1, 64], stride >= 1");
  LA_REQUIRE(a->offset >= 0, "la_xattn_select: offset >= 0");
  LA_REQUIRE(a->mode == 0 || a->mode == 1, "la_xattn_select: mode 0 (threshold) or 1 (top-k)");
  LA_REQUIRE(a->mode == 1 || a->alpha, "la_xattn_select: threshold mode needs per-head alpha");
  LA_REQUIRE(a->mode == 0 || a->topk >= 1, "la_xattn_select: topk >= 1");
  LA_REQUIRE(a->in_dtype == LA_F32 || a->in_dtype == LA_BF16 || a->in_dtype == LA_F16,
             "la_xattn_select: q/k dtype");
  const int64_t n_kb = ceil_div(a->T, a->block), n_qb = ceil_div(a->Tq, a->block);
  const int64_t ns = (2 * a->block - 2) / a->stride + 1;
  LA_REQUIRE(a->width >= (a->mode == 1 ? std::min(a->topk, n_kb) + 1 : n_kb),
             "la_xattn_select: width below the largest selection");
  if (n_kb > 16 * TK_NT)
    return fail(LA_ERR_UNSUPPORTED, "la_xattn_select: at most %d key blocks", 16 * TK_NT);
  size_t lds = 0;
  if (xattn_lds(a, n_kb, ns, lds) != LA_OK)
    return fail(LA_ERR_UNSUPPORTED, "la_xattn_select: %zu bytes of LDS per row (max 120 KiB)", lds);
  if (a->in_dtype == LA_BF16)
    LA_REQUIRE((uintptr_t)a->k % 16 == 0 && a->D % 8 == 0 && a->k_sb % 8 == 0 && a->k_sh % 8 == 0 &&
                   a->k_st % 8 == 0,
               "la_xattn_select: bf16 key rows must be 16-byte aligned");
  XaKP p{};
  p.q = a->q;
  p.k = a->k;
  p.out_idx = a->out_idx;
  p.out_count = a->out_count;
  p.alpha = a->alpha;
  p.B = a->B; p.Hq = a->Hq; p.Hkv = a->Hkv; p.Tq = a->Tq; p.T = a->T; p.D = a->D;
  p.q_sb = a->q_sb; p.q_sh = a->q_sh; p.q_st = a->q_st;
  p.k_sb = a->k_sb; p.k_sh = a->k_sh; p.k_st = a->k_st;
  p.blk = a->block; p.r = a->stride; p.n_slots = ns; p.offset = a->offset;
  p.n_qb = n_qb; p.n_kb = n_kb; p.topk = a->topk; p.width = a->width;
  p.inv_sqrt_d = a->inv_sqrt_d;
  p.two_f = std::ldexp(1.0, (int)(52 - ceil_log2(n_kb * ns)));
  p.in_dt = a->in_dtype;
  p.mode = a->mode;
  const int64_t nwg = a->B * a->Hq * n_qb;
  LA_REQUIRE(nwg < ((int64_t)1 << 31), "la_xattn_select: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const int64_t cq = a->workspace && xattn_mfma_shape(a) ? xattn_chunk_qb(a, a->ws_bytes) : 0;
  if (cq > 0) {
    p.slots = (double *)a->workspace;
    LA_REQUIRE(a->B * a->Hq < 65536, "la_xattn_select: B * Hq >= 65536");
    // chunks of query blocks: score the chunk's slots, then select its rows
    for (int64_t q0 = 0; q0 < n_qb; q0 += cq) {
      p.qc0 = q0;
      p.n_qc = std::min(cq, n_qb - q0);
      const dim3 grid((unsigned)ceil_div(n_kb, XM_T), (unsigned)ceil_div(p.n_qc, XM_T),
                      (unsigned)(a->B * a->Hq));
      if (a->in_dtype == LA_BF16)
        xattn_slots_mfma_kernel<true><<<grid, XM_NT, 0, st>>>(p);
      else
        xattn_slots_mfma_kernel<false><<<grid, XM_NT, 0, st>>>(p);
      LA_LAUNCHED();
      const int64_t nrows = a->B * a->Hq * p.n_qc;
      if (n_kb <= 1024) {  // one wave per row over the scored slots
        const unsigned g4 = (unsigned)ceil_div(nrows, 4);
        if (n_kb <= 64)
          xattn_select_wave_kernel<1><<<g4, 256, 0, st>>>(p, nrows);
        else if (n_kb <= 256)
          xattn_select_wave_kernel<4><<<g4, 256, 0, st>>>(p, nrows);
        else
          xattn_select_wave_kernel<16><<<g4, 256, 0, st>>>(p, nrows);
        LA_LAUNCHED();
      } else {
        const int rc = xattn_launch_select(p, n_kb, lds, nrows, st);
        if (rc != LA_OK) return rc;
      }
    }
    return LA_OK;
  }
  p.qc0 = 0;
  p.n_qc = n_qb;
  return xattn_launch_select(p, n_kb, lds, nwg, st);
}
