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
// Two score kernels, both VALU fp64 (matrix-core accumulation order is not
// specified, so MFMA cannot reproduce these bits):
//  - tiled (prefill): a 64-query x 128-key tile per workgroup, 8x4 register
//    tile per thread, q/k slices staged in LDS as fp32 (exact for bf16);
//  - per-key (decode, few queries): 64 keys per workgroup, one thread per
//    (key, head) reading the key row from LDS.
// Scores of a chunk of queries go to the workspace and the shared row top-k
// (topk.hip) selects from them.
#include <algorithm>

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
};

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
// is contiguous and 16-byte aligned (the decode shape of config C5).  64 keys
// per workgroup, HI threads per key: the key rows are staged with coalesced
// 16-byte loads (all in flight at once) into LDS rows padded to 528 bytes;
// thread (key, head) computes that head's dot for every query of the chunk,
// d in order, and thread (query, key) then adds the heads in order.
constexpr int IDF_KEYS = 64, IDF_ROWB = 528;

__device__ __forceinline__ float half_bits_to_f32(uint32_t bits16, int dt) {
  return dt == LA_BF16 ? bf16_bits_to_f32(bits16) : __half2float(__ushort_as_half((uint16_t)bits16));
}

template <int HI>
__global__ __launch_bounds__(IDF_KEYS * HI) void indexer_decode16_kernel(IdxKP p) {
  constexpr int NT = IDF_KEYS * HI;
  constexpr int CPT = (IDF_KEYS * ID_MAXHD / 8 + NT - 1) / NT;  // 16-byte chunks per thread (max)
  __shared__ __align__(16) unsigned char sk[IDF_KEYS * IDF_ROWB];
  __shared__ double sqd[ID_MAXQ][ID_MAXHD];
  __shared__ double sdot[ID_MAXQ][IDF_KEYS][HI];
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t k0 = (int64_t)blockIdx.x * IDF_KEYS;
  const int d = (int)p.d;
  const int hd = HI * d;
  const int cpr = hd / 8;  // 16-byte chunks per key row
  const uint16_t *kb = (const uint16_t *)p.k + b * p.k_sb;
  {
    uint4 v[CPT];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * NT;
      const int r = c / cpr, col = c % cpr;
      const int64_t s = k0 + r;
      v[u] = (r < IDF_KEYS && s < p.Tk) ? *(const uint4 *)(kb + s * p.k_st + col * 8) : uint4{0, 0, 0, 0};
    }
    for (int i = tid; i < p.tn * hd; i += NT) {
      const int tl = i / hd, c = i % hd;
      const int h = c / d, dd = c % d;
      sqd[tl][c] = load_as_f64(p.q, b * p.q_sb + (p.t0 + tl) * p.q_st + h * p.q_sh + dd, p.dt);
    }
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * NT;
      if (c < IDF_KEYS * cpr) *(uint4 *)(sk + (c / cpr) * IDF_ROWB + (c % cpr) * 16) = v[u];
    }
  }
  __syncthreads();
  {
    const int h = tid % HI, r = tid / HI;
    const unsigned char *row = sk + r * IDF_ROWB + h * d * 2;
    double dot[ID_MAXQ] = {0.0, 0.0, 0.0, 0.0};
    for (int dd = 0; dd < d; dd += 8) {
      const uint4 kv = *(const uint4 *)(row + dd * 2);
      const uint32_t w4[4] = {kv.x, kv.y, kv.z, kv.w};
      double kf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[2 * e] = (double)half_bits_to_f32(w4[e] & 0xffffu, p.dt);
        kf[2 * e + 1] = (double)half_bits_to_f32(w4[e] >> 16, p.dt);
      }
#pragma unroll
      for (int tl = 0; tl < ID_MAXQ; ++tl) {
        if (tl >= p.tn) break;
        const double *qv = &sqd[tl][h * d + dd];
#pragma unroll
        for (int e = 0; e < 8; ++e) dot[tl] = __builtin_fma(qv[e], kf[e], dot[tl]);
      }
    }
#pragma unroll
    for (int tl = 0; tl < ID_MAXQ; ++tl)
      if (tl < p.tn) sdot[tl][r][h] = dot[tl];
  }
  __syncthreads();
  for (int i = tid; i < IDF_KEYS * p.tn; i += NT) {
    const int r = i % IDF_KEYS, tl = i / IDF_KEYS;
    const int64_t s = k0 + r;
    if (s >= p.Tk) continue;
    const int64_t t = p.t0 + tl;
    double acc = 0.0;
#pragma unroll
    for (int h = 0; h < HI; ++h) {
      const double dv = sdot[tl][r][h];
      const double rl = dv > 0.0 ? dv : 0.0;
      acc = add_product(acc, (double)p.w[b * p.w_sb + t * p.w_st + h * p.w_sh], rl);
    }
    p.scores[(b * p.tn + tl) * p.Tk + s] = acc;
  }
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
  tp.order = 0;
  tp.out_idx = a->out_idx;
  tp.out_val = a->out_val;
  return tp;
}

static int64_t scores_bytes(const la_indexer_args *a, int64_t chunk) {
  return (a->B * chunk * a->Tk * 8 + 255) / 256 * 256;
}

extern "C" size_t la_indexer_topk_workspace(const la_indexer_args *a) {
  if (validate(a) != LA_OK) return 0;
  const int64_t chunk = pick_chunk(a);
  return (size_t)(scores_bytes(a, chunk) + topk_workspace_bytes(topk_params(a, nullptr, 0, chunk)));
}

extern "C" int la_indexer_topk(const la_indexer_args *a, void *stream) {
  int rc = validate(a);
  if (rc != LA_OK) return rc;
  const int64_t chunk = pick_chunk(a);
  const int64_t sc_bytes = scores_bytes(a, chunk);
  const size_t need = (size_t)(sc_bytes + topk_workspace_bytes(topk_params(a, nullptr, 0, chunk)));
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
    if (decode16) {
      const dim3 grid((unsigned)ceil_div(a->Tk, IDF_KEYS), (unsigned)a->B);
      switch (a->HI) {
        case 1: indexer_decode16_kernel<1><<<grid, IDF_KEYS * 1, 0, st>>>(p); break;
        case 2: indexer_decode16_kernel<2><<<grid, IDF_KEYS * 2, 0, st>>>(p); break;
        case 4: indexer_decode16_kernel<4><<<grid, IDF_KEYS * 4, 0, st>>>(p); break;
        default: indexer_decode16_kernel<8><<<grid, IDF_KEYS * 8, 0, st>>>(p); break;
      }
    } else if (decode) {
      indexer_decode_kernel<<<dim3((unsigned)ceil_div(a->Tk, ID_KEYS), (unsigned)a->B), 256, 0,
                              st>>>(p);
    } else {
      indexer_tile_kernel<<<dim3((unsigned)ceil_div(a->Tk, IT_K), (unsigned)ceil_div(p.tn, IT_Q),
                                 (unsigned)a->B),
                            IT_NT, 0, st>>>(p);
    }
    LA_LAUNCHED();
    rc = topk_launch_ws(topk_params(a, p.scores, t0, p.tn), (char *)a->workspace + sc_bytes,
                        a->ws_bytes - sc_bytes, st);
    if (rc != LA_OK) return rc;
  }
  return LA_OK;
}
