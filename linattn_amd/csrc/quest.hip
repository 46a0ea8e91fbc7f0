// Quest page metadata and upper-bound page scores (gfx950).
//
// page bounds : quest_pages.py:38-48 (page_bounds_torch), selection.py:181-201
// page scores : quest_pages.py:51-55 (page_scores_torch), selection.py:203-212
#include <type_traits>

#include "common.h"
#include "kv_access.h"
#include "quest_select.h"
#include "topk_select.h"

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

// Wave form: a workgroup (4 waves) covers PG consecutive pages of one
// (b, KV head), a wave one page at a time.  A lane reads 16-byte chunks (LPR
// lanes per key row, 64 / LPR rows per pass, U nontemporal loads in flight),
// keeps elementwise min / max in registers, and the row groups are folded
// with lane exchanges.  The page's bounds go to LDS; once every page is done
// the workgroup writes them out row by row (for page-minor metadata, a
// channel's PG pages are one contiguous run, written by adjacent lanes, in
// place of scattered 2-byte stores).  Exact, so equal to the scalar form bit
// for bit.
template <int KT, int D, int PG>
__global__ __launch_bounds__(256) void page_bounds_wave_kernel(la_kv kv, int64_t Hkv, int64_t ps,
                                                               int64_t first_page, int64_t n_pages,
                                                               void *mn, void *mx, int64_t m_sb,
                                                               int64_t m_sh, int64_t m_sp,
                                                               int64_t m_sd, int meta_dt, int quad) {
  constexpr int ESZ = KT == LA_BF16 ? 2 : 4;
  constexpr int EPL = 16 / ESZ;
  constexpr int LPR = D / EPL;  // lanes per key row
  constexpr int RG = 64 / LPR;  // rows per pass of the wave
  constexpr int U = 16;         // loads in flight per lane
  __shared__ float sb[2][D][PG + 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t p0 = first_page + (int64_t)blockIdx.x * PG;
  const int np = (int)min((int64_t)PG, n_pages - p0);  // pages of this workgroup
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t len = kv_length(kv, b);
  const int c = lane % LPR, rg = lane / LPR;
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  // a pool whose pages are the metadata pages resolves the physical page
  // once; other pools go row by row
  const bool direct = !kv.page_table || kv.page_size == ps;
  for (int pp = w; pp < np; pp += 4) {
    const int64_t p = p0 + pp;
    const int64_t t0 = p * ps;
    const int64_t n = max((int64_t)0, min(len, t0 + ps) - t0);
    float lo[EPL], hi[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      lo[e] = __int_as_float(0x7f800000);
      hi[e] = __int_as_float(0xff800000);
    }
    int64_t base = 0, rs = 0;
    if (kv.page_table) {
      const int64_t phys = (direct && n > 0) ? kv.page_table[b * kv.pt_stride + p] : 0;
      base = (phys * Hkv + h) * ps * D;
      rs = D;
    } else {
      base = b * kv.k_sb + h * kv.k_sh + t0 * kv.k_st;
      rs = kv.k_st;
    }
    const char *kb = (const char *)kv.k + (base + c * EPL) * ESZ;
    for (int64_t r = rg; r < n; r += (int64_t)RG * U) {
      v4u v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr = r + u * RG;
        const char *src = direct ? kb + rr * rs * ESZ
                                 : (const char *)kv.k +
                                       (kv_row(kv, b, h, t0 + rr, Hkv, D, false) + c * EPL) * ESZ;
        v[u] = rr < n ? __builtin_nontemporal_load((const v4u *)src) : v4u{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (r + u * RG >= n) break;
        float x[EPL];
        if constexpr (KT == LA_BF16) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[2 * e] = bf16lo(v[u][e]);
            x[2 * e + 1] = bf16hi(v[u][e]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(v[u][e]);
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          lo[e] = fminf(lo[e], x[e]);
          hi[e] = fmaxf(hi[e], x[e]);
        }
      }
    }
    // fold the row groups (lanes c, c + LPR, c + 2 LPR, ...)
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1)
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        lo[e] = fminf(lo[e], __shfl_xor(lo[e], o, 64));
        hi[e] = fmaxf(hi[e], __shfl_xor(hi[e], o, 64));
      }
    if (rg == 0)
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        sb[0][c * EPL + e][pp] = lo[e];
        sb[1][c * EPL + e][pp] = hi[e];
      }
  }
  __syncthreads();
  // channel rows out: item (which, d, page), or with `quad` (page-minor
  // metadata whose runs of four pages are 4-element aligned, every page of
  // the workgroup valid) item (which, d, four pages) as one store
  if (quad && np == PG) {
    for (int i = threadIdx.x; i < 2 * D * PG / 4; i += 256) {
      const int pp = 4 * (i % (PG / 4)), d = (i / (PG / 4)) % D, which = i / (PG / 4 * D);
      const int64_t o = b * m_sb + h * m_sh + (p0 + pp) + (int64_t)d * m_sd;
      const float *x = &sb[which][d][pp];
      void *dst = which ? mx : mn;
      if (meta_dt == LA_F32) {
        *(float4 *)((float *)dst + o) = float4{x[0], x[1], x[2], x[3]};
      } else {
        const uint32_t a = (uint32_t)f32_to_bf16_bits(x[0]) | ((uint32_t)f32_to_bf16_bits(x[1]) << 16);
        const uint32_t z = (uint32_t)f32_to_bf16_bits(x[2]) | ((uint32_t)f32_to_bf16_bits(x[3]) << 16);
        *(uint2 *)((uint16_t *)dst + o) = uint2{a, z};
      }
    }
    return;
  }
  for (int i = threadIdx.x; i < 2 * D * PG; i += 256) {
    const int pp = i % PG, d = (i / PG) % D, which = i / (PG * D);
    if (pp >= np) continue;
    const int64_t o = b * m_sb + h * m_sh + (p0 + pp) * m_sp + (int64_t)d * m_sd;
    store_from_f32(which ? mx : mn, o, meta_dt, sb[which][d][pp]);
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
    // QD dims per batch; the next batch's loads are issued before the current
    // one is accumulated, so 2*QD loads per array are in flight per thread.
    constexpr int QD = 8;
    using V = typename std::conditional<MT == LA_BF16, uint2, float4>::type;
    const V *pl = (const V *)((const char *)mn + (mbase + p0) * (MT == LA_BF16 ? 2 : 4));
    const V *ph = (const V *)((const char *)mx + (mbase + p0) * (MT == LA_BF16 ? 2 : 4));
    const int64_t sd = m_sd / PPT;  // vectors per d step
    const int Dn = (int)D;
    auto widen = [](const V &v, double (&x)[PPT]) {
      if constexpr (MT == LA_BF16) {
        x[0] = bf16lo(v.x); x[1] = bf16hi(v.x); x[2] = bf16lo(v.y); x[3] = bf16hi(v.y);
      } else {
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
      }
    };
    V a[2][QD], c[2][QD];
    // loads are unconditional (channels past D re-read channel D-1 and are
    // not consumed): a conditional load block would make the compiler wait
    // for every outstanding load before each consume
    auto fetch = [&](int d0, int buf) {
#pragma unroll
      for (int j = 0; j < QD; ++j) {
        const int64_t d = min(d0 + j, Dn - 1);
        a[buf][j] = pl[d * sd];
        c[buf][j] = ph[d * sd];
      }
    };
    auto consume = [&](int d0, int buf) {
#pragma unroll
      for (int j = 0; j < QD; ++j) {
        if (d0 + j >= Dn) break;
        double lo[PPT], hi[PPT];
        widen(a[buf][j], lo);
        widen(c[buf][j], hi);
        accumulate(d0 + j, lo, hi);
      }
    };
    fetch(0, 0);
    for (int d0 = 0; d0 < Dn; d0 += 2 * QD) {
      fetch(d0 + QD, 1);
      consume(d0, 0);
      fetch(d0 + 2 * QD, 0);
      consume(d0 + QD, 1);
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

// Quest selection of one (b, KV head, query) in a single pass: the page
// scores of the G query heads (as in quest_scores_kernel, page-minor metadata)
// go to LDS as order keys, with the query's own page forced; each head's top-k
// is selected from there (register radix select) into a union bitmap, which
// is written in ascending page order.  Equals quest_scores_kernel followed by
// the union top-k, without the score rows leaving the chip.
// qs_nt threads: up to 2048 pages, eight waves score two pages each (four
// waves per SIMD with two workgroups per CU hide the metadata reads and the
// fp64 work behind each other); longer rows keep four waves, whose selecting
// wave holds 64 keys per lane.  One wave per head selects.
template <int KPT> constexpr int qs_nt() { return KPT <= 8 ? 512 : TK_NT; }
template <int MT, int G, int KPT>
__global__ __launch_bounds__(qs_nt<KPT>()) void quest_select_kernel(QsKP a) {
  constexpr int QS_NT = qs_nt<KPT>();
  extern __shared__ __align__(16) uint64_t keys[];  // [G][NP]
  __shared__ double qd[G * 256];
  __shared__ uint32_t wtmp[QS_NT / 64];
  __shared__ uint32_t bm[TK_NT * KPT / 32];
  const int64_t row = blockIdx.x;  // (b, kvh, t)
  const int64_t t = row % a.Tq;
  const int64_t kvh = (row / a.Tq) % a.Hkv;
  const int64_t b = row / (a.Tq * a.Hkv);
  int32_t n_v, own;
  quest_select_union<MT, G, KPT, QS_NT, QS_NT>(a, b, kvh, t, keys, qd, bm, n_v, own);
  tk_emit_bitmap_row<QS_NT>(bm, n_v, own, 0, 0, a.width, a.out_idx + row * a.width,
                            a.out_count ? a.out_count + row : nullptr, wtmp);
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
  // 16-byte rows: every row offset (pool rows or strides) a multiple of 16 bytes
  const int64_t esz = kv->dtype == LA_F32 ? 4 : 2;
  bool vec = (D == 64 || D == 128 || D == 256) && (uintptr_t)kv->k % 16 == 0;
  if (!kv->page_table)
    vec = vec && (kv->k_sb * esz) % 16 == 0 && (kv->k_sh * esz) % 16 == 0 && (kv->k_st * esz) % 16 == 0;
  if (vec) {
    constexpr int PG = 32;  // pages per workgroup
    // four pages per store: page-minor metadata (bf16 or fp32; f16 keys never
    // reach here), every run of four pages aligned
    const int64_t mes = meta_dtype == LA_F32 ? 4 : 2;
    const int quad = m_sp == 1 && m_sd % 4 == 0 && m_sh % 4 == 0 && m_sb % 4 == 0 &&
                     first_page % 4 == 0 && (uintptr_t)page_min % (4 * mes) == 0 &&
                     (uintptr_t)page_max % (4 * mes) == 0 &&
                     (meta_dtype == LA_F32 || meta_dtype == LA_BF16);
    const dim3 wgrid((unsigned)ceil_div(n_pages - first_page, (int64_t)PG), (unsigned)Hkv, (unsigned)B);
#define LA_PB(KT, DD)                                                                      \
  page_bounds_wave_kernel<KT, DD, PG><<<wgrid, 256, 0, st>>>(*kv, Hkv, page_size, first_page, \
                                                             n_pages, page_min, page_max, m_sb,  \
                                                             m_sh, m_sp, m_sd, meta_dtype, quad)
    if (kv->dtype == LA_F32) {
      if (D == 64) LA_PB(LA_F32, 64); else if (D == 128) LA_PB(LA_F32, 128); else LA_PB(LA_F32, 256);
    } else {
      if (D == 64) LA_PB(LA_BF16, 64); else if (D == 128) LA_PB(LA_BF16, 128); else LA_PB(LA_BF16, 256);
    }
#undef LA_PB
  } else if (kv->dtype == LA_F32)
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

template <int MT, int G, int KPT>
static int launch_select(const QsKP &k, int64_t rows, hipStream_t st) {
  const size_t bytes = (size_t)G * TK_NT * KPT * 8;
  if (bytes > 65536) {
    static bool attr_set = false;
    if (!attr_set) {
      LA_HIP(hipFuncSetAttribute((const void *)quest_select_kernel<MT, G, KPT>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
      attr_set = true;
    }
  }
  quest_select_kernel<MT, G, KPT><<<dim3((unsigned)rows), qs_nt<KPT>(), bytes, st>>>(k);
  LA_LAUNCHED();
  return LA_OK;
}

template <int MT, int G>
static int launch_select_kpt(const QsKP &k, int64_t rows, hipStream_t st) {
  if (k.n_pages <= 1024) return launch_select<MT, G, 4>(k, rows, st);
  if (k.n_pages <= 2048) return launch_select<MT, G, 8>(k, rows, st);
  if constexpr (G <= 4) return launch_select<MT, G, 16>(k, rows, st);
  return fail(LA_ERR_UNSUPPORTED, "la_quest_select: too many pages for one workgroup");
}

extern "C" int la_quest_select(const la_quest_select_args *a, void *stream) {
  LA_REQUIRE(a && a->q && a->page_min && a->page_max && a->out_idx, "la_quest_select: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hq > 0 && a->Tq > 0 && a->Hkv > 0 && a->n_pages > 0 && a->k > 0,
             "la_quest_select: bad shape");
  LA_REQUIRE(a->D > 0 && a->D <= 256, "la_quest_select: head_dim must be in [1, 256]");
  LA_REQUIRE(a->Hq % a->Hkv == 0, "la_quest_select: n_heads must be a multiple of n_kv_heads");
  LA_REQUIRE(a->page_size > 0, "la_quest_select: page_size");
  LA_REQUIRE(a->q_dtype == LA_F32 || a->q_dtype == LA_BF16 || a->q_dtype == LA_F16,
             "la_quest_select: q dtype");
  LA_REQUIRE(a->meta_dtype == LA_F32 || a->meta_dtype == LA_BF16, "la_quest_select: meta dtype");
  const int64_t G = a->Hq / a->Hkv;
  const int64_t esz = a->meta_dtype == LA_BF16 ? 2 : 4;
  // page-minor metadata, 4 pages per aligned vector
  const bool layout = a->m_sp == 1 && a->m_sd % 4 == 0 && a->m_sd >= a->n_pages &&
                      a->m_sb % 4 == 0 && a->m_sh % 4 == 0 &&
                      (uintptr_t)a->page_min % (4 * esz) == 0 && (uintptr_t)a->page_max % (4 * esz) == 0;
  if (!layout || a->n_pages > (G <= 4 ? 4096 : 2048) || !(G == 1 || G == 2 || G == 4 || G == 8))
    return fail(LA_ERR_UNSUPPORTED, "la_quest_select: shape or metadata layout not fused");
  QsKP k{};
  k.q = a->q;
  k.mn = a->page_min;
  k.mx = a->page_max;
  k.out_idx = a->out_idx;
  k.out_count = a->out_count;
  k.Hq = a->Hq;
  k.Hkv = a->Hkv;
  k.Tq = a->Tq;
  k.D = a->D;
  k.q_sb = a->q_sb;
  k.q_sh = a->q_sh;
  k.q_st = a->q_st;
  k.n_pages = a->n_pages;
  k.m_sb = a->m_sb;
  k.m_sh = a->m_sh;
  k.m_sd = a->m_sd;
  k.page_size = a->page_size;
  k.pos_offset = a->pos_offset;
  k.positions = a->positions;
  k.k = std::max<int64_t>(1, std::min(a->k, a->n_pages));
  k.width = G * k.k;
  k.q_dt = a->q_dtype;
  const int64_t rows = a->B * a->Hkv * a->Tq;
  hipStream_t st = (hipStream_t)stream;
#define LA_QSEL(MT)                                                  \
  switch (G) {                                                       \
    case 1: return launch_select_kpt<MT, 1>(k, rows, st);           \
    case 2: return launch_select_kpt<MT, 2>(k, rows, st);           \
    case 4: return launch_select_kpt<MT, 4>(k, rows, st);           \
    default: return launch_select_kpt<MT, 8>(k, rows, st);          \
  }
  if (a->meta_dtype == LA_BF16) {
    LA_QSEL(LA_BF16)
  } else {
    LA_QSEL(LA_F32)
  }
#undef LA_QSEL
}
