// Fused Quest page selection (variants/selection.py:203-237) as a device
// routine shared by la_quest_select and the fused select + decode kernel.
#pragma once

#include <type_traits>

#include "common.h"
#include "topk_select.h"

namespace la {

struct QsKP {
  const void *q, *mn, *mx;
  int32_t *out_idx, *out_count;
  int64_t Hq, Hkv, Tq, D, q_sb, q_sh, q_st, n_pages, m_sb, m_sh, m_sd;
  int64_t page_size, pos_offset, k, width;
  const int32_t *positions;
  int32_t q_dt;
};

// read-once metadata: nontemporal loads
__device__ __forceinline__ uint2 ntl(const uint2 *p) {
  typedef uint32_t v2u __attribute__((ext_vector_type(2)));
  const v2u x = __builtin_nontemporal_load((const v2u *)p);
  return uint2{x[0], x[1]};
}
__device__ __forceinline__ float4 ntl(const float4 *p) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  const v4f x = __builtin_nontemporal_load((const v4f *)p);
  return float4{x[0], x[1], x[2], x[3]};
}
__device__ __forceinline__ uint32_t ntl(const uint32_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ float2 ntl(const float2 *p) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f x = __builtin_nontemporal_load((const v2f *)p);
  return float2{x[0], x[1]};
}

// Metadata vector of PPT consecutive pages (page-minor layout).
template <int MT, int PPT> struct QsVec;
template <> struct QsVec<LA_BF16, 4> { using T = uint2; };
template <> struct QsVec<LA_BF16, 2> { using T = uint32_t; };
template <> struct QsVec<LA_F32, 4> { using T = float4; };
template <> struct QsVec<LA_F32, 2> { using T = float2; };

// The union selection of one (b, KV head, query t) row: fp64 upper-bound
// scores of every page for the G query heads (the first SNT threads of the
// NT-thread workgroup, 1024 / SNT pages x G heads each), the own page forced,
// each head's top-k OR'd into the bitmap bm by one wave per head.  keys
// [G][256 KPT] and qd [G][256] are scratch.  Every thread of the workgroup
// takes part in the barriers; n_v (visible pages) and own (the own page) are
// returned.
template <int MT, int G, int KPT, int NT = TK_NT, int SNT = TK_NT>
__device__ __forceinline__ void quest_select_union(const QsKP &a, int64_t b, int64_t kvh, int64_t t,
                                                   uint64_t *keys, double *qd, uint32_t *bm,
                                                   int32_t &n_v_out, int32_t &own_out) {
  constexpr int NP = TK_NT * KPT;  // pages held (>= n_pages)
  constexpr int PPT = 4 * TK_NT / SNT, QD = 8;
  static_assert(SNT <= NT && (PPT == 2 || PPT == 4), "scoring threads");
  const int tid = threadIdx.x;
  const int64_t D = a.D;
  for (int64_t i = tid; i < G * D; i += NT) {
    const int64_t g = i / D, d = i % D;
    qd[g * D + d] = load_as_f64(a.q, b * a.q_sb + (kvh * G + g) * a.q_sh + t * a.q_st + d, a.q_dt);
  }
  for (int i = tid; i < NP / 32; i += NT) bm[i] = 0u;
  const int64_t pos = (a.positions ? (int64_t)a.positions[b] : a.pos_offset) + t;
  const int64_t u_own = pos >= 0 ? pos / a.page_size : -1;
  const int32_t n_v = (int32_t)min(a.n_pages, u_own + 1);
  const int32_t own = (int32_t)min(u_own, a.n_pages - 1);
  const bool force = own >= 0 && own < n_v;
  n_v_out = n_v;
  own_out = own;
  __syncthreads();
  if (NT == SNT || tid < SNT) {  // (wave-uniform)

  using V = typename QsVec<MT, PPT>::T;
  constexpr int ESZ = MT == LA_BF16 ? 2 : 4;
  const int64_t mbase = b * a.m_sb + kvh * a.m_sh;
  const int Dn = (int)D;
  const int sd = (int)(a.m_sd / PPT);  // vectors per d step
  for (int c = 0; c < NP / (SNT * PPT); ++c) {
    const int p0 = c * SNT * PPT + tid * PPT;
    double acc[G][PPT];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < PPT; ++i) acc[g][i] = 0.0;
    if (p0 < a.m_sd) {  // m_sd = pages rounded up to 4: the padded storage
      const V *pl = (const V *)((const char *)a.mn + (mbase + p0) * ESZ);
      const V *ph = (const V *)((const char *)a.mx + (mbase + p0) * ESZ);
      V lo_v[2][QD], hi_v[2][QD];
      // channels past D re-read channel D-1 (in bounds) and are not consumed
      auto fetch = [&](int d0, int buf) {
#pragma unroll
        for (int j = 0; j < QD; ++j) {
          const int d = min(d0 + j, Dn - 1);
          lo_v[buf][j] = ntl(pl + d * sd);
          hi_v[buf][j] = ntl(ph + d * sd);
        }
      };
      auto widen = [](const V &v, double (&x)[PPT]) {
        if constexpr (MT == LA_BF16 && PPT == 4) {
          x[0] = bf16lo(v.x); x[1] = bf16hi(v.x); x[2] = bf16lo(v.y); x[3] = bf16hi(v.y);
        } else if constexpr (MT == LA_BF16) {
          x[0] = bf16lo(v); x[1] = bf16hi(v);
        } else if constexpr (PPT == 4) {
          x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        } else {
          x[0] = v.x; x[1] = v.y;
        }
      };
      auto consume = [&](int d0, int buf) {
#pragma unroll
        for (int j = 0; j < QD; ++j) {
          if (d0 + j >= Dn) break;
          double lo[PPT], hi[PPT];
          widen(lo_v[buf][j], lo);
          widen(hi_v[buf][j], hi);
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const double qv = qd[g * Dn + d0 + j];
            const bool neg = qv < 0.0;
#pragma unroll
            for (int i = 0; i < PPT; ++i) acc[g][i] = __builtin_fma(qv, neg ? lo[i] : hi[i], acc[g][i]);
          }
        }
      };
      // fetches are unconditional (a conditional load block would make the
      // compiler wait for every outstanding load before each consume)
      fetch(0, 0);
      for (int d0 = 0; d0 < Dn; d0 += 2 * QD) {
        fetch(d0 + QD, 1);
        consume(d0, 0);
        fetch(d0 + 2 * QD, 0);
        consume(d0 + QD, 1);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int pg = p0 + i;
        keys[g * NP + pg] = (force && pg == own) ? KEY_FORCED : ord_key(acc[g][i]);
      }
  }
  }
  __syncthreads();
  // each wave selects its heads' pages (w, w + waves, ...) into the union bitmap
  const uint32_t K = (uint32_t)min(a.k, (int64_t)n_v);
  const int w = tid >> 6, lane = tid & 63;
  constexpr int KPL = NP / 64;
  for (int g = w; g < G; g += NT / 64) {
    uint64_t u[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) u[j] = keys[g * NP + lane + 64 * j];
    // the wave's own key row (already in registers) is its selection scratch
    __builtin_amdgcn_wave_barrier();
    tk_wave_select_bits<KPL>(
        u, n_v, K, [&](int j, int32_t i, bool take) {
          if (take) atomicOr(&bm[i >> 5], 1u << (i & 31));
        },
        keys + g * NP);
  }
  __syncthreads();
}


}  // namespace la
