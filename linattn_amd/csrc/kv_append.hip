// Paged KV append with incremental Quest page bounds (and the fp8 codec).
//
// One workgroup per (b, KV head) writes the Tn new key / value rows of
// sequence b into its pages of the pool and folds them into the channel-wise
// min / max of the Quest pages they land in -- the KV concatenation of
// AttentionVariant.push_kv (core.py:219-220) and the page refresh of
// QuestAttention._refresh_pages (variants/selection.py:181-201) in one pass,
// so the bounds never round-trip through a recompute over the page.  An fp8
// pool stores codes and per-token scales with the codec of kv/quant.py:76-93
// (group = head_dim).
#include "common.h"

namespace la {

constexpr int KA_NT = 128;

struct KaKP {
  const void *k_new, *v_new;
  void *k_pool, *v_pool;
  float *k_scale, *v_scale;
  const int32_t *page_table, *positions;
  void *mn, *mx;
  int64_t Hkv, Tn, D;
  int64_t n_sb, n_sh, n_st;
  int64_t n_phys, pool_page, pt_sb, pt_pages;
  int64_t meta_page, n_pages, m_sb, m_sh, m_sp, m_sd;
  int32_t in_dt, pool_dt;
  int64_t s_stride;  // fp8: scale elements between pool rows
};

// fp32 absmax of the row over the workgroup (every thread gets it)
__device__ __forceinline__ float ka_block_max(float x, float *red) {
  x = fmaxf(x, __shfl_xor(x, 1, 64));
  x = fmaxf(x, __shfl_xor(x, 2, 64));
  x = fmaxf(x, __shfl_xor(x, 4, 64));
  x = fmaxf(x, __shfl_xor(x, 8, 64));
  x = pair32_max(pair16_max(x));
  __syncthreads();  // red is reused row after row
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < KA_NT / 64; ++i) r = fmaxf(r, red[i]);
  return r;
}

// Store one row of new values x[] (this thread's dims d = tid + KA_NT i) into
// the pool row at element offset `row` (scale slot `srow` for fp8).
template <int NPT>
__device__ __forceinline__ void ka_store_row(const KaKP &p, void *pool, float *scales, int64_t row,
                                             int64_t srow, const float (&x)[NPT], bool ok,
                                             float *red) {
  const int tid = threadIdx.x;
  if (p.pool_dt == LA_FP8_E4M3) {
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i)
      if (tid + KA_NT * i < p.D) am = fmaxf(am, fabsf(x[i]));
    // scale = max(absmax, 1e-8) / 448 and codes = fp8(x / scale), as
    // kv/quant.py:82-85 computes them in fp32 (IEEE division, RNE cast)
    const float scale = fmaxf(ka_block_max(am, red), 1e-8f) / 448.f;
    if (!ok) return;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int64_t d = tid + KA_NT * i;
      if (d < p.D) {
        const float c = x[i] / scale;
        const int w = __builtin_amdgcn_cvt_pk_fp8_f32(c, c, 0, false);
        ((uint8_t *)pool)[row + d] = (uint8_t)(w & 0xff);
      }
    }
    if (tid == 0) scales[srow * p.s_stride] = scale;
    return;
  }
  if (!ok) return;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int64_t d = tid + KA_NT * i;
    if (d < p.D) store_from_f32(pool, row + d, p.pool_dt, x[i]);
  }
}

template <int NPT>
__global__ __launch_bounds__(KA_NT) void kv_append_kernel(KaKP p) {
  __shared__ float red[KA_NT / 64];
  const int tid = threadIdx.x;
  const int64_t h = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t pos0 = p.positions[b];
  const bool meta = p.mn != nullptr;
  // running bounds of the Quest page being filled
  float lo[NPT], hi[NPT];
  int64_t cur = -1;  // its index
  auto flush = [&]() {
    if (cur < 0 || cur >= p.n_pages) return;
    // a page that starts among the new tokens holds only them; otherwise the
    // old bounds cover its earlier tokens
    const bool fresh = cur * p.meta_page >= pos0;
    const int64_t o = b * p.m_sb + h * p.m_sh + cur * p.m_sp;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int64_t d = tid + KA_NT * i;
      if (d >= p.D) continue;
      float l = lo[i], u = hi[i];
      if (!fresh) {
        l = fminf(load_as_f32(p.mn, o + d * p.m_sd, p.pool_dt), l);
        u = fmaxf(load_as_f32(p.mx, o + d * p.m_sd, p.pool_dt), u);
      }
      store_from_f32(p.mn, o + d * p.m_sd, p.pool_dt, l);
      store_from_f32(p.mx, o + d * p.m_sd, p.pool_dt, u);
    }
  };
  for (int64_t i = 0; i < p.Tn; ++i) {
    const int64_t t = pos0 + i;
    const int64_t lp = t / p.pool_page;
    const int64_t phys = (t >= 0 && lp < p.pt_pages) ? p.page_table[b * p.pt_sb + lp] : -1;
    const bool ok = phys >= 0 && phys < p.n_phys;  // other entries are not written
    const int64_t srow = (phys * p.Hkv + h) * p.pool_page + t % p.pool_page;
    const int64_t row = srow * p.D;
    const int64_t in = b * p.n_sb + h * p.n_sh + i * p.n_st;
    float kx[NPT], vx[NPT];
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int64_t d = tid + KA_NT * j;
      kx[j] = d < p.D ? load_as_f32(p.k_new, in + d, p.in_dt) : 0.f;
      vx[j] = d < p.D ? load_as_f32(p.v_new, in + d, p.in_dt) : 0.f;
    }
    ka_store_row<NPT>(p, p.k_pool, p.k_scale, row, srow, kx, ok, red);
    ka_store_row<NPT>(p, p.v_pool, p.v_scale, row, srow, vx, ok, red);
    if (meta && ok) {  // a token on an unmapped page counts in no bounds
      const int64_t mp = t / p.meta_page;
      if (mp != cur) {
        flush();
        cur = mp;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
          lo[j] = __int_as_float(0x7f800000);
          hi[j] = __int_as_float(0xff800000);
        }
      }
#pragma unroll
      for (int j = 0; j < NPT; ++j) {
        lo[j] = fminf(lo[j], kx[j]);
        hi[j] = fmaxf(hi[j], kx[j]);
      }
    }
  }
  if (meta) flush();
}

}  // namespace la

using namespace la;

extern "C" int la_paged_kv_append(const la_kv_append_args *a, void *stream) {
  LA_REQUIRE(a && a->k_new && a->v_new && a->k_pool && a->v_pool && a->page_table && a->positions,
             "la_paged_kv_append: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hkv > 0 && a->Tn >= 0 && a->D > 0, "la_paged_kv_append: bad shape");
  LA_REQUIRE(a->D <= 4 * KA_NT, "la_paged_kv_append: head_dim above 512");
  LA_REQUIRE(a->pool_page > 0 && a->n_phys > 0 && a->pt_pages > 0, "la_paged_kv_append: bad pool");
  LA_REQUIRE(a->in_dtype == LA_F32 || a->in_dtype == LA_BF16, "la_paged_kv_append: input dtype");
  const bool fp8 = a->pool_dtype == LA_FP8_E4M3;
  LA_REQUIRE(fp8 || a->pool_dtype == a->in_dtype,
             "la_paged_kv_append: the pool stores the input dtype (or fp8 codes)");
  LA_REQUIRE(!fp8 || (a->k_scale && a->v_scale), "la_paged_kv_append: fp8 pool needs scales");
  const bool meta = a->page_min != nullptr || a->page_max != nullptr;
  if (meta) {
    LA_REQUIRE(a->page_min && a->page_max, "la_paged_kv_append: both bounds tensors");
    if (fp8)
      return fail(LA_ERR_UNSUPPORTED, "la_paged_kv_append: page bounds of an fp8 pool");
    LA_REQUIRE(a->meta_page > 0 && a->n_pages > 0, "la_paged_kv_append: bad page bounds shape");
  }
  if (a->Tn == 0) return LA_OK;
  KaKP p{};
  p.k_new = a->k_new;
  p.v_new = a->v_new;
  p.k_pool = a->k_pool;
  p.v_pool = a->v_pool;
  p.k_scale = a->k_scale;
  p.v_scale = a->v_scale;
  p.s_stride = a->s_stride > 0 ? a->s_stride : 1;
  p.page_table = a->page_table;
  p.positions = a->positions;
  p.mn = meta ? a->page_min : nullptr;
  p.mx = meta ? a->page_max : nullptr;
  p.Hkv = a->Hkv;
  p.Tn = a->Tn;
  p.D = a->D;
  p.n_sb = a->n_sb;
  p.n_sh = a->n_sh;
  p.n_st = a->n_st;
  p.n_phys = a->n_phys;
  p.pool_page = a->pool_page;
  p.pt_sb = a->pt_sb;
  p.pt_pages = a->pt_pages;
  p.meta_page = a->meta_page;
  p.n_pages = a->n_pages;
  p.m_sb = a->m_sb;
  p.m_sh = a->m_sh;
  p.m_sp = a->m_sp;
  p.m_sd = a->m_sd;
  p.in_dt = a->in_dtype;
  p.pool_dt = a->pool_dtype;
  dim3 grid((unsigned)a->Hkv, (unsigned)a->B);
  hipStream_t st = (hipStream_t)stream;
  const int64_t npt = (a->D + KA_NT - 1) / KA_NT;
  if (npt == 1)
    kv_append_kernel<1><<<grid, KA_NT, 0, st>>>(p);
  else if (npt == 2)
    kv_append_kernel<2><<<grid, KA_NT, 0, st>>>(p);
  else
    kv_append_kernel<4><<<grid, KA_NT, 0, st>>>(p);
  LA_LAUNCHED();
  return LA_OK;
}
