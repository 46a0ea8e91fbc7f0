// Block selection for block-sparse prefill (config C3), gfx950.
//
// The block-sparse estimator of MInferenceAttention._block_sparse
// (variants/selection.py:339-353): mean-pool q and k over 64-token blocks
// (block_reduce, core.py:102-120; the tail block repeats the last row), score
// every causal block pair with the pooled dot product, keep the top-k key
// blocks per (b, h, query block), then OR the sink blocks and the local window
// (which contains the diagonal block, selection.py:351).
//
// Arithmetic is fp64 and a fixed function of the inputs: pooled sums add rows
// in order and divide by the block size; block scores add fl(qbar_d*kbar_d)
// over d in order (never fused).  The positive 1/sqrt(D) factor of the
// reference does not change the ranking and is not applied.
#include <algorithm>

#include "common.h"
#include "topk.h"

namespace la {

// Rows of sequence b: lens[b] (clamped to [0, T]) in a ragged batch, else T.
__device__ __forceinline__ int64_t seq_rows(const int32_t *lens, int64_t b, int64_t T) {
  return lens ? min(max((int64_t)lens[b], (int64_t)0), T) : T;
}

// The block a pooling workgroup writes: blk0 + blockIdx.x, or, with per-
// sequence positions, the block of positions[b] (-1 when outside [0, nb)).
__device__ __forceinline__ int64_t pool_block(int64_t blk0, const int32_t *pos, int64_t b,
                                              int64_t bs, int64_t nb) {
  if (!pos) return blk0 + blockIdx.x;
  const int64_t p = pos[b];
  return (p >= 0 && p / bs < nb) ? p / bs : -1;
}

// qbar/kbar[b][h][blk][d] = (sum_{i<bs} x[b][h][min(blk*bs+i, T_b-1)][d]) / bs
// (T_b = seq_rows; a sequence without rows pools zeros, which no list reads)
__global__ __launch_bounds__(128) void mean_pool_kernel(const void *x, int dt, int64_t T, int64_t D,
                                                        int64_t sb, int64_t sh, int64_t st,
                                                        int64_t bs, int64_t H, int64_t nb,
                                                        double *out, const int32_t *lens,
                                                        int64_t blk0, const int32_t *pos) {
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t blk = pool_block(blk0, pos, b, bs, nb);
  if (blk < 0) return;
  const int64_t base = b * sb + h * sh;
  T = seq_rows(lens, b, T);
  if (T == 0) {
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) out[((b * H + h) * nb + blk) * D + d] = 0.0;
    return;
  }
  for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
    double acc = 0.0;
    for (int64_t i = 0; i < bs; ++i) {
      const int64_t row = min(blk * bs + i, T - 1);
      acc = acc + load_as_f64(x, base + row * st + d, dt);
    }
    out[((b * H + h) * nb + blk) * D + d] = acc / (double)bs;
  }
}

// The same pooling with the block staged in LDS first: 16-byte loads, every
// row of the block in flight at once; thread d then adds the rows in order.
// Needs bs <= 64, D * element size a multiple of 16 bytes and <= 512 bytes,
// 16-byte aligned rows.
template <int ESZ, int NT>
__global__ __launch_bounds__(NT) void mean_pool_vec_kernel(const void *x, int dt, int64_t T,
                                                            int64_t D, int64_t sb, int64_t sh,
                                                            int64_t st, int64_t bs, int64_t H,
                                                            int64_t nb, double *out,
                                                            const int32_t *lens, int64_t blk0,
                                                            const int32_t *pos) {
  extern __shared__ __align__(16) unsigned char rows[];  // bs rows of D * ESZ bytes
  constexpr int CH = 64 * 512 / 16 / NT;                  // chunks per thread (max)
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t blk = pool_block(blk0, pos, b, bs, nb);
  if (blk < 0) return;  // (workgroup-uniform)
  const int tid = threadIdx.x;
  T = seq_rows(lens, b, T);
  if (T == 0) {  // (workgroup-uniform)
    for (int64_t d = tid; d < D; d += NT) out[((b * H + h) * nb + blk) * D + d] = 0.0;
    return;
  }
  const int rb = (int)(D * ESZ);  // bytes per row
  const int cpr = rb / 16;
  const int total = (int)bs * cpr;
  const char *base = (const char *)x + (b * sb + h * sh) * ESZ;
  uint4 v[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int c = tid + u * NT;
    const int64_t row = min(blk * bs + c / cpr, T - 1);
    v[u] = c < total ? *(const uint4 *)(base + row * st * ESZ + (c % cpr) * 16) : uint4{0, 0, 0, 0};
  }
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int c = tid + u * NT;
    if (c < total) *(uint4 *)(rows + (c / cpr) * rb + (c % cpr) * 16) = v[u];
  }
  __syncthreads();
  for (int64_t d = tid; d < D; d += NT) {
    double acc = 0.0;
    for (int64_t i = 0; i < bs; ++i) {
      const unsigned char *e = rows + i * rb + d * ESZ;
      double xv;
      if constexpr (ESZ == 4) {
        xv = (double)*(const float *)e;
      } else {
        const uint32_t bits = *(const uint16_t *)e;
        xv = dt == LA_BF16 ? (double)bf16_bits_to_f32(bits)
                           : (double)__half2float(__ushort_as_half((uint16_t)bits));
      }
      acc = acc + xv;
    }
    out[((b * H + h) * nb + blk) * D + d] = acc / (double)bs;
  }
}

constexpr int BS_DC = 32, BS_NT = 256;

// scores[(b*Hq+h)*nqb + i][j] = sum_d fl(qbar[b,h,i,d] * kbar[b,h/G,j,d]) for
// the TQ x TK tile (i, j), TK = (256 / (TQ / RQ)) * RK: each thread holds
// RQ x RK scores.  Row i sits at position pos0 + i*qunit and column j starts
// at j*kunit; tiles whose every column starts past every row's position are
// skipped (causal: their scores are never read).  TQ = 64 (4 x 4 per thread)
// for prefill rows; TQ = 4 (one score per thread, 64 columns) for decode,
// where a 64-row tile would compute 63 empty rows per query.
template <int TQ, int RQ, int RK>
__global__ __launch_bounds__(BS_NT) void block_score_kernel(const double *qbar, const double *kbar,
                                                            int64_t Hq, int64_t Hkv, int64_t nqb,
                                                            int64_t nkb, int64_t D, int64_t pos0,
                                                            int64_t qunit, int64_t kunit,
                                                            double *scores) {
  constexpr int TY = TQ / RQ, TX = BS_NT / TY, TK = TX * RK;
  static_assert(TY * TX == BS_NT, "tile shape");
  __shared__ double sq[BS_DC][TQ + 2];
  __shared__ double sk[BS_DC][TK + 2];
  const int tid = threadIdx.x;
  const int tq = tid / TX, tk = tid % TX;  // rows RQ*tq.., cols RK*tk..
  const int64_t i0 = (int64_t)blockIdx.y * TQ, j0 = (int64_t)blockIdx.x * TK;
  const int64_t bh = blockIdx.z;
  const int64_t b = bh / Hq, h = bh % Hq;
  if (j0 * kunit > pos0 + min(i0 + TQ - 1, nqb - 1) * qunit) return;  // all in the future
  const double *qb = qbar + bh * nqb * D;
  const double *kb = kbar + (b * Hkv + h / (Hq / Hkv)) * nkb * D;
  double acc[RQ][RK];
#pragma unroll
  for (int a = 0; a < RQ; ++a)
#pragma unroll
    for (int c = 0; c < RK; ++c) acc[a][c] = 0.0;
  for (int64_t d0 = 0; d0 < D; d0 += BS_DC) {
    const int dn = (int)min((int64_t)BS_DC, D - d0);
    __syncthreads();
    for (int x = tid; x < TQ * BS_DC; x += BS_NT) {
      const int r = x / BS_DC, dd = x % BS_DC;
      sq[dd][r] = (dd < dn && i0 + r < nqb) ? qb[(i0 + r) * D + d0 + dd] : 0.0;
    }
    for (int x = tid; x < TK * BS_DC; x += BS_NT) {
      const int r = x / BS_DC, dd = x % BS_DC;
      sk[dd][r] = (dd < dn && j0 + r < nkb) ? kb[(j0 + r) * D + d0 + dd] : 0.0;
    }
    __syncthreads();
    for (int dd = 0; dd < dn; ++dd) {
      double qv[RQ], kv[RK];
#pragma unroll
      for (int a = 0; a < RQ; ++a) qv[a] = sq[dd][RQ * tq + a];
#pragma unroll
      for (int c = 0; c < RK; ++c) kv[c] = sk[dd][RK * tk + c];
#pragma unroll
      for (int a = 0; a < RQ; ++a)
#pragma unroll
        for (int c = 0; c < RK; ++c) acc[a][c] = add_product(acc[a][c], qv[a], kv[c]);
    }
  }
#pragma unroll
  for (int a = 0; a < RQ; ++a) {
    const int64_t i = i0 + RQ * tq + a;
    if (i >= nqb) continue;
#pragma unroll
    for (int c = 0; c < RK; ++c) {
      const int64_t j = j0 + RK * tk + c;
      if (j < nkb) scores[(bh * nqb + i) * nkb + j] = acc[a][c];
    }
  }
}

// Scores of every (row, column) tile of (B * Hq) heads; the tile shape
// follows the number of rows.
static void block_scores(const double *qbar, const double *kbar, int64_t B, int64_t Hq,
                         int64_t Hkv, int64_t nqb, int64_t nkb, int64_t D, int64_t pos0,
                         int64_t qunit, int64_t kunit, double *scores, hipStream_t st) {
  if (nqb <= 4)
    block_score_kernel<4, 1, 1><<<dim3((unsigned)ceil_div(nkb, 64), (unsigned)ceil_div(nqb, 4),
                                       (unsigned)(B * Hq)),
                                  BS_NT, 0, st>>>(qbar, kbar, Hq, Hkv, nqb, nkb, D, pos0, qunit,
                                                  kunit, scores);
  else
    block_score_kernel<64, 4, 4><<<dim3((unsigned)ceil_div(nkb, 64), (unsigned)ceil_div(nqb, 64),
                                        (unsigned)(B * Hq)),
                                   BS_NT, 0, st>>>(qbar, kbar, Hq, Hkv, nqb, nkb, D, pos0, qunit,
                                                   kunit, scores);
}

// Mean of every `bs` rows of x[b][h] (rows past T_b repeat row T_b-1) into
// out[b][h][blk][d] in fp64; bs = 1 is the exact widening to fp64.  T_b is
// lens[b] (ragged batch) or T.  Blocks blk0 .. blk0 + npool - 1 (all nb by
// default), or the block of pos[b] for each sequence b (npool = 1).
static void pool_rows(const void *x, int dt, int64_t B, int64_t H, int64_t T, int64_t D, int64_t sb,
                      int64_t sh, int64_t s_t, int64_t bs, int64_t nb, double *out,
                      hipStream_t st, const int32_t *lens = nullptr, int64_t blk0 = 0,
                      int64_t npool = -1, const int32_t *pos = nullptr) {
  const int64_t esz = dt == LA_F32 ? 4 : 2;
  if (npool < 0) npool = nb;
  const dim3 grid((unsigned)npool, (unsigned)H, (unsigned)B);
  const bool vec = bs <= 64 && (D * esz) % 16 == 0 && D * esz <= 512 && (uintptr_t)x % 16 == 0 &&
                   (sb * esz) % 16 == 0 && (sh * esz) % 16 == 0 && (s_t * esz) % 16 == 0;
  const size_t lds = (size_t)(bs * D * esz);
  // 128 threads when one thread per d covers the row (the block stays in LDS
  // only while it is summed, so several blocks per CU overlap)
  if (vec && esz == 4 && D <= 128)
    mean_pool_vec_kernel<4, 128><<<grid, 128, lds, st>>>(x, dt, T, D, sb, sh, s_t, bs, H, nb, out, lens, blk0, pos);
  else if (vec && esz == 4)
    mean_pool_vec_kernel<4, 256><<<grid, 256, lds, st>>>(x, dt, T, D, sb, sh, s_t, bs, H, nb, out, lens, blk0, pos);
  else if (vec && D <= 128)
    mean_pool_vec_kernel<2, 128><<<grid, 128, lds, st>>>(x, dt, T, D, sb, sh, s_t, bs, H, nb, out, lens, blk0, pos);
  else if (vec)
    mean_pool_vec_kernel<2, 256><<<grid, 256, lds, st>>>(x, dt, T, D, sb, sh, s_t, bs, H, nb, out, lens, blk0, pos);
  else
    mean_pool_kernel<<<grid, 128, 0, st>>>(x, dt, T, D, sb, sh, s_t, bs, H, nb, out, lens, blk0, pos);
}

struct BsLayout {
  int64_t nqb, nkb, qbar_off, kbar_off, sc_off, bytes;
};

static BsLayout layout(const la_block_select_args *a) {
  BsLayout L{};
  L.nqb = ceil_div(a->T, a->block);
  L.nkb = L.nqb;
  L.qbar_off = 0;
  L.kbar_off = L.qbar_off + a->B * a->Hq * L.nqb * a->D * 8;
  L.sc_off = L.kbar_off + a->B * a->Hkv * L.nkb * a->D * 8;
  L.bytes = L.sc_off + a->B * a->Hq * L.nqb * L.nkb * 8;
  return L;
}

static int validate(const la_block_select_args *a) {
  LA_REQUIRE(a && a->q && a->k && a->out_idx, "la_block_select: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hq > 0 && a->Hkv > 0 && a->T > 0 && a->D > 0 && a->block > 0,
             "la_block_select: bad shape");
  LA_REQUIRE(a->Hq % a->Hkv == 0, "n_heads must be a multiple of n_kv_heads");
  LA_REQUIRE(a->topk >= 1 && a->sink_blocks >= 0 && a->window_blocks >= 0, "la_block_select: budget");
  LA_REQUIRE(a->width >= a->topk + a->sink_blocks + a->window_blocks,
             "la_block_select: width < topk + sink + window");
  LA_REQUIRE(a->in_dtype == LA_F32 || a->in_dtype == LA_BF16 || a->in_dtype == LA_F16,
             "la_block_select: q/k dtype");
  return LA_OK;
}

}  // namespace la

using namespace la;

extern "C" size_t la_block_select_workspace(const la_block_select_args *a) {
  if (validate(a) != LA_OK) return 0;
  return (size_t)layout(a).bytes;
}

extern "C" int la_block_select(const la_block_select_args *a, void *stream) {
  int rc = validate(a);
  if (rc != LA_OK) return rc;
  const BsLayout L = layout(a);
  if (!a->workspace || a->ws_bytes < L.bytes)
    return fail(LA_ERR_WORKSPACE, "la_block_select: workspace %lld < %lld bytes",
                (long long)a->ws_bytes, (long long)L.bytes);
  hipStream_t st = (hipStream_t)stream;
  char *ws = (char *)a->workspace;
  double *qbar = (double *)(ws + L.qbar_off);
  double *kbar = (double *)(ws + L.kbar_off);
  double *sc = (double *)(ws + L.sc_off);
  pool_rows(a->q, a->in_dtype, a->B, a->Hq, a->T, a->D, a->q_sb, a->q_sh, a->q_st, a->block, L.nqb,
            qbar, st, a->lengths);
  LA_LAUNCHED();
  pool_rows(a->k, a->in_dtype, a->B, a->Hkv, a->T, a->D, a->k_sb, a->k_sh, a->k_st, a->block, L.nkb,
            kbar, st, a->lengths);
  LA_LAUNCHED();
  block_scores(qbar, kbar, a->B, a->Hq, a->Hkv, L.nqb, L.nkb, a->D, 0, 1, 1, sc, st);
  LA_LAUNCHED();
  TopkKParams tp{};
  tp.scores = sc;
  tp.row_stride = L.nkb;
  tp.G = 1;
  tp.Tq = L.nqb;
  tp.NG = a->B * a->Hq * L.nqb;
  tp.t_base = 0;
  tp.out_tq = L.nqb;
  tp.n = L.nkb;
  tp.k = a->topk;
  tp.width = a->width;
  tp.pos_off = 0;  // query block qb: key blocks kb <= qb, own block qb
  tp.pos_unit = 1;
  tp.sink = a->sink_blocks;
  tp.window = a->window_blocks;
  tp.order = 1;
  tp.out_idx = a->out_idx;
  tp.out_count = a->out_count;
  // ragged: the query blocks of sequence b at or past its length select nothing
  tp.b_lens = a->lengths;
  tp.rows_per_b = a->Hq * L.nqb;
  tp.b_len_unit = a->block;
  return topk_launch(tp, st);
}

// ------------------------------------------------------------ gate select --
// Per-query block routing: MoBA's gate (variants/selection.py:624-634) and
// the blockwise selection of NSA (variants/native_sparse.py:78-93), which
// compute the same thing: g[j] = q_t . mean(K block j) over the visible
// blocks (start <= pos_t = offset + t), the top-k blocks by gate, and the
// query's own block OR'd in.  The gates are fp64, fl(q_d * kbar_d) added
// over d in order, without the positive 1/sqrt(D) factor (it does not change
// the ranking); ties go to the lowest block.
namespace la {
struct GsLayout {
  int64_t nkb, qbar_off, kbar_off, sc_off, bytes;
};
static GsLayout gs_layout(const la_gate_select_args *a) {
  GsLayout L{};
  L.nkb = ceil_div(a->T, a->block);
  L.qbar_off = 0;
  L.kbar_off = L.qbar_off + a->B * a->Hq * a->Tq * a->D * 8;
  // (no pooled keys when the caller keeps them)
  L.sc_off = L.kbar_off + (a->kbar ? 0 : a->B * a->Hkv * L.nkb * a->D * 8);
  L.bytes = L.sc_off + a->B * a->Hq * a->Tq * L.nkb * 8;
  return L;
}
static int gs_validate(const la_gate_select_args *a) {
  LA_REQUIRE(a && a->q && (a->k || a->kbar) && a->out_idx, "la_gate_select: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hq > 0 && a->Hkv > 0 && a->Tq > 0 && a->T > 0 && a->D > 0 &&
                 a->block > 0,
             "la_gate_select: bad shape");
  LA_REQUIRE(a->Hq % a->Hkv == 0, "n_heads must be a multiple of n_kv_heads");
  LA_REQUIRE(a->topk >= 1, "la_gate_select: topk");
  LA_REQUIRE(a->offset >= 0, "la_gate_select: offset");
  LA_REQUIRE(a->width >= std::min(a->topk, ceil_div(a->T, a->block)) + 1,
             "la_gate_select: width < min(topk, blocks) + 1");
  LA_REQUIRE(a->in_dtype == LA_F32 || a->in_dtype == LA_BF16 || a->in_dtype == LA_F16,
             "la_gate_select: q/k dtype");
  return LA_OK;
}
}  // namespace la

extern "C" size_t la_gate_select_workspace(const la_gate_select_args *a) {
  if (gs_validate(a) != LA_OK) return 0;
  return (size_t)gs_layout(a).bytes;
}

extern "C" int la_gate_select(const la_gate_select_args *a, void *stream) {
  int rc = gs_validate(a);
  if (rc != LA_OK) return rc;
  const GsLayout L = gs_layout(a);
  if (!a->workspace || a->ws_bytes < L.bytes)
    return fail(LA_ERR_WORKSPACE, "la_gate_select: workspace %lld < %lld bytes",
                (long long)a->ws_bytes, (long long)L.bytes);
  hipStream_t st = (hipStream_t)stream;
  char *ws = (char *)a->workspace;
  double *qbar = (double *)(ws + L.qbar_off);
  double *kbar = (double *)(ws + L.kbar_off);
  double *sc = (double *)(ws + L.sc_off);
  pool_rows(a->q, a->in_dtype, a->B, a->Hq, a->Tq, a->D, a->q_sb, a->q_sh, a->q_st, 1, a->Tq, qbar,
            st);  // q widened to fp64
  LA_LAUNCHED();
  if (a->kbar) {  // block means kept by the caller (la_block_means)
    kbar = const_cast<double *>(a->kbar);
  } else {
    pool_rows(a->k, a->in_dtype, a->B, a->Hkv, a->T, a->D, a->k_sb, a->k_sh, a->k_st, a->block,
              L.nkb, kbar, st);
    LA_LAUNCHED();
  }
  block_scores(qbar, kbar, a->B, a->Hq, a->Hkv, a->Tq, L.nkb, a->D, a->offset, 1, a->block, sc,
               st);
  LA_LAUNCHED();
  TopkKParams tp{};
  tp.scores = sc;
  tp.row_stride = L.nkb;
  tp.G = 1;
  tp.Tq = a->Tq;
  tp.NG = a->B * a->Hq * a->Tq;
  tp.t_base = 0;
  tp.out_tq = a->Tq;
  tp.n = L.nkb;
  tp.k = a->topk;
  tp.width = a->width;
  tp.pos_off = a->offset;  // visible: block start <= offset + t; own = (offset + t) / block
  tp.pos_unit = a->block;
  tp.sink = 0;
  tp.window = 1;  // the own block, OR'd after the top-k (selection.py:632-633)
  tp.order = 1;
  tp.out_idx = a->out_idx;
  tp.out_count = a->out_count;
  return topk_launch(tp, st);
}

// ------------------------------------------------------------ block means --
namespace la {
static int bm_validate(const la_block_means_args *a) {
  LA_REQUIRE(a && a->k && a->out, "la_block_means: null pointer");
  LA_REQUIRE(a->B > 0 && a->H > 0 && a->T > 0 && a->D > 0 && a->block > 0,
             "la_block_means: bad shape");
  LA_REQUIRE(a->in_dtype == LA_F32 || a->in_dtype == LA_BF16 || a->in_dtype == LA_F16,
             "la_block_means: k dtype");
  const int64_t nkb = ceil_div(a->T, a->block);
  if (!a->positions)
    LA_REQUIRE(a->first_block >= 0 && a->n_blocks >= 0 && a->first_block + a->n_blocks <= nkb,
               "la_block_means: blocks [%lld, %lld) outside [0, %lld)", (long long)a->first_block,
               (long long)(a->first_block + a->n_blocks), (long long)nkb);
  LA_REQUIRE(nkb < ((int64_t)1 << 31) && a->B < 65536 && a->H < 65536, "la_block_means: grid");
  return LA_OK;
}
}  // namespace la

extern "C" int la_block_means(const la_block_means_args *a, void *stream) {
  const int rc = bm_validate(a);
  if (rc != LA_OK) return rc;
  const int64_t nkb = ceil_div(a->T, a->block);
  const int64_t npool = a->positions ? 1 : a->n_blocks;
  if (npool == 0) return LA_OK;
  pool_rows(a->k, a->in_dtype, a->B, a->H, a->T, a->D, a->k_sb, a->k_sh, a->k_st, a->block, nkb,
            a->out, (hipStream_t)stream, a->lengths, a->positions ? 0 : a->first_block, npool,
            a->positions);
  LA_LAUNCHED();
  return LA_OK;
}
