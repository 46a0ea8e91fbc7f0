// Quest page metadata and upper-bound page scores (gfx950).
//
// page bounds : quest_pages.py:38-48 (page_bounds_torch), selection.py:181-201
// page scores : quest_pages.py:51-55 (page_scores_torch), selection.py:203-212
#include "common.h"
#include "kv_access.h"

namespace la {

// One workgroup per (page, kv head, batch); threads walk the channels, so the
// reads of one key row are coalesced.  min/max of stored values are exact.
template <int KT>
__global__ __launch_bounds__(256) void page_bounds_kernel(la_kv kv, int64_t Hkv, int64_t D,
                                                          int64_t ps, int64_t first_page,
                                                          void *mn, void *mx, int64_t m_sb,
                                                          int64_t m_sh, int64_t m_sp, int64_t m_sd,
                                                          int meta_dt) {
  const int64_t p = first_page + blockIdx.x;
  const int64_t h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int64_t len = kv_length(kv, b);
  const int64_t t0 = p * ps;
  const int64_t t1 = min(len, t0 + ps);
  for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
    float lo = __int_as_float(0x7f800000), hi = __int_as_float(0xff800000);
    for (int64_t tok = t0; tok < t1; ++tok) {
      const int64_t off = kv_row(kv, b, h, tok, Hkv, D, false) + d;
      const float x = load_as_f32(kv.k, off, KT);
      lo = fminf(lo, x);
      hi = fmaxf(hi, x);
    }
    const int64_t o = b * m_sb + h * m_sh + p * m_sp + d * m_sd;
    store_from_f32(mn, o, meta_dt, lo);
    store_from_f32(mx, o, meta_dt, hi);
  }
}

// Scores of PPT consecutive pages per thread for the G query heads that share
// one KV head.  score = sum_{d=0}^{D-1} max(q_d m_d, q_d M_d), accumulated in
// fp64 in increasing d.  Because m_d <= M_d, the max is q_d*M_d for q_d >= 0
// and q_d*m_d otherwise; both products are exact in fp64 (fp32/bf16 inputs), so
// the fused multiply-add below rounds exactly like a separate add.
template <int MT, int G, int PPT, bool VEC>
__global__ __launch_bounds__(256) void quest_scores_kernel(
    const void *q, int q_dt, int64_t Hq, int64_t Tq, int64_t D, int64_t q_sb, int64_t q_sh,
    int64_t q_st, const void *mn, const void *mx, int64_t Hkv, int64_t n_pages, int64_t m_sb,
    int64_t m_sh, int64_t m_sp, int64_t m_sd, double *scores) {
  __shared__ double qd[G * 256];
  const int64_t row = blockIdx.y;  // (b, kvh, t)
  const int64_t t = row % Tq;
  const int64_t kvh = (row / Tq) % Hkv;
  const int64_t b = row / (Tq * Hkv);
  for (int64_t i = threadIdx.x; i < G * D; i += blockDim.x) {
    const int64_t g = i / D, d = i % D;
    const int64_t h = kvh * G + g;
    qd[g * D + d] = load_as_f64(q, b * q_sb + h * q_sh + t * q_st + d, q_dt);
  }
  __syncthreads();
  const int64_t p0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * PPT;
  if (p0 >= n_pages) return;
  double acc[G][PPT];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < PPT; ++i) acc[g][i] = 0.0;
  const int64_t mbase = b * m_sb + kvh * m_sh;
  auto accumulate = [&](int64_t d, const double (&lo)[PPT], const double (&hi)[PPT]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const double qv = qd[g * D + d];
      const bool pos = qv >= 0.0;
#pragma unroll
      for (int i = 0; i < PPT; ++i) acc[g][i] = __builtin_fma(qv, pos ? hi[i] : lo[i], acc[g][i]);
    }
  };
  if (VEC && p0 + PPT <= n_pages) {
    static_assert(PPT == 4, "vector path loads 4 pages");
    if constexpr (MT == LA_BF16) {
      const uint16_t *pl = (const uint16_t *)mn + mbase + p0;
      const uint16_t *ph = (const uint16_t *)mx + mbase + p0;
#pragma unroll 8
      for (int64_t d = 0; d < D; ++d) {
        const uint2 a = *(const uint2 *)(pl + d * m_sd);
        const uint2 c = *(const uint2 *)(ph + d * m_sd);
        const double lo[PPT] = {bf16lo(a.x), bf16hi(a.x), bf16lo(a.y), bf16hi(a.y)};
        const double hi[PPT] = {bf16lo(c.x), bf16hi(c.x), bf16lo(c.y), bf16hi(c.y)};
        accumulate(d, lo, hi);
      }
    } else {
      const float *pl = (const float *)mn + mbase + p0;
      const float *ph = (const float *)mx + mbase + p0;
#pragma unroll 8
      for (int64_t d = 0; d < D; ++d) {
        const float4 a = *(const float4 *)(pl + d * m_sd);
        const float4 c = *(const float4 *)(ph + d * m_sd);
        const double lo[PPT] = {a.x, a.y, a.z, a.w};
        const double hi[PPT] = {c.x, c.y, c.z, c.w};
        accumulate(d, lo, hi);
      }
    }
  } else {
    for (int64_t d = 0; d < D; ++d) {
      double lo[PPT], hi[PPT];
      const int64_t o = mbase + d * m_sd + p0 * m_sp;
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const bool ok = p0 + i < n_pages;
        lo[i] = ok ? load_as_f64(mn, o + i * m_sp, MT) : 0.0;
        hi[i] = ok ? load_as_f64(mx, o + i * m_sp, MT) : 0.0;
      }
      accumulate(d, lo, hi);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    double *out = scores + ((b * Hq + kvh * G + g) * Tq + t) * n_pages;
#pragma unroll
    for (int i = 0; i < PPT; ++i)
      if (p0 + i < n_pages) out[p0 + i] = acc[g][i];
  }
}

template <int MT, int G>
static int launch_scores(const void *q, int q_dt, int64_t B, int64_t Hq, int64_t Tq, int64_t D,
                         int64_t q_sb, int64_t q_sh, int64_t q_st, const void *mn, const void *mx,
                         int64_t Hkv, int64_t n_pages, int64_t m_sb, int64_t m_sh, int64_t m_sp,
                         int64_t m_sd, double *scores, hipStream_t st) {
  constexpr int PPT = 4;
  const int threads = 256;
  dim3 grid((unsigned)ceil_div(n_pages, threads * PPT), (unsigned)(B * Hkv * Tq));
  const int esz = (MT == LA_BF16) ? 2 : 4;
  const bool vec = (m_sp == 1) && (m_sd % PPT == 0) && (m_sb % PPT == 0) && (m_sh % PPT == 0) &&
                   ((uintptr_t)mn % (PPT * esz) == 0) && ((uintptr_t)mx % (PPT * esz) == 0);
  if (vec)
    quest_scores_kernel<MT, G, PPT, true><<<grid, threads, 0, st>>>(
        q, q_dt, Hq, Tq, D, q_sb, q_sh, q_st, mn, mx, Hkv, n_pages, m_sb, m_sh, m_sp, m_sd, scores);
  else
    quest_scores_kernel<MT, G, PPT, false><<<grid, threads, 0, st>>>(
        q, q_dt, Hq, Tq, D, q_sb, q_sh, q_st, mn, mx, Hkv, n_pages, m_sb, m_sh, m_sp, m_sd, scores);
  LA_LAUNCHED();
  return LA_OK;
}

}  // namespace la

using namespace la;

extern "C" int la_quest_page_bounds(const la_kv *kv, int64_t B, int64_t Hkv, int64_t D,
                                    int64_t page_size, int64_t first_page, int64_t n_pages,
                                    void *page_min, void *page_max, int64_t m_sb, int64_t m_sh,
                                    int64_t m_sp, int64_t m_sd, int32_t meta_dtype, void *stream) {
  LA_REQUIRE(kv && kv->k, "la_quest_page_bounds: null key cache");
  LA_REQUIRE(page_min && page_max, "la_quest_page_bounds: null output");
  LA_REQUIRE(B > 0 && Hkv > 0 && D > 0 && page_size > 0, "la_quest_page_bounds: bad shape");
  LA_REQUIRE(first_page >= 0 && first_page <= n_pages, "la_quest_page_bounds: bad page range");
  LA_REQUIRE(kv->dtype == LA_F32 || kv->dtype == LA_BF16,
             "la_quest_page_bounds: keys must be fp32 or bf16");
  LA_REQUIRE(meta_dtype == kv->dtype,
             "la_quest_page_bounds: metadata must be stored in the key dtype (exact bounds)");
  if (kv->page_table) LA_REQUIRE(kv->page_size > 0, "la_quest_page_bounds: page_size of pool");
  if (first_page == n_pages) return LA_OK;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)(n_pages - first_page), (unsigned)Hkv, (unsigned)B);
  const int threads = D >= 256 ? 256 : (int)(((D + 63) / 64) * 64);
  if (kv->dtype == LA_F32)
    page_bounds_kernel<LA_F32><<<grid, threads, 0, st>>>(*kv, Hkv, D, page_size, first_page, page_min,
                                                         page_max, m_sb, m_sh, m_sp, m_sd, meta_dtype);
  else
    page_bounds_kernel<LA_BF16><<<grid, threads, 0, st>>>(*kv, Hkv, D, page_size, first_page,
                                                          page_min, page_max, m_sb, m_sh, m_sp, m_sd,
                                                          meta_dtype);
  LA_LAUNCHED();
  return LA_OK;
}

extern "C" int la_quest_scores(const void *q, int32_t q_dtype, int64_t B, int64_t Hq, int64_t Tq,
                               int64_t D, int64_t q_sb, int64_t q_sh, int64_t q_st,
                               const void *page_min, const void *page_max, int32_t meta_dtype,
                               int64_t Hkv, int64_t n_pages, int64_t m_sb, int64_t m_sh,
                               int64_t m_sp, int64_t m_sd, double *scores, void *stream) {
  LA_REQUIRE(q && page_min && page_max && scores, "la_quest_scores: null pointer");
  LA_REQUIRE(B > 0 && Hq > 0 && Tq > 0 && Hkv > 0 && n_pages > 0, "la_quest_scores: bad shape");
  LA_REQUIRE(D > 0 && D <= 256, "la_quest_scores: head_dim must be in [1, 256]");
  LA_REQUIRE(Hq % Hkv == 0, "la_quest_scores: n_heads must be a multiple of n_kv_heads");
  LA_REQUIRE(q_dtype == LA_F32 || q_dtype == LA_BF16 || q_dtype == LA_F16,
             "la_quest_scores: q dtype");
  const int64_t G = Hq / Hkv;
  hipStream_t st = (hipStream_t)stream;
#define LA_QS(MT, GG)                                                                            \
  return launch_scores<MT, GG>(q, q_dtype, B, Hq, Tq, D, q_sb, q_sh, q_st, page_min, page_max, \
                               Hkv, n_pages, m_sb, m_sh, m_sp, m_sd, scores, st)
#define LA_QS_G(MT)                     \
  switch (G) {                          \
    case 1: LA_QS(MT, 1);               \
    case 2: LA_QS(MT, 2);               \
    case 4: LA_QS(MT, 4);               \
    case 8: LA_QS(MT, 8);               \
    default: break;                     \
  }
  if (meta_dtype == LA_BF16) {
    LA_QS_G(LA_BF16)
  } else if (meta_dtype == LA_F32) {
    LA_QS_G(LA_F32)
  } else {
    return fail(LA_ERR_INVALID, "la_quest_scores: meta dtype must be fp32 or bf16");
  }
#undef LA_QS_G
#undef LA_QS
  return fail(LA_ERR_UNSUPPORTED, "la_quest_scores: GQA group %lld not in {1,2,4,8}", (long long)G);
}
