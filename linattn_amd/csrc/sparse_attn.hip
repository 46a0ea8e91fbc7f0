// Split-K exact attention over listed KV units, gfx950.
//
// Executor semantics: kernels/triton/block_sparse.py:40-75 (gather form) and
// :80-128 (one program per query row, online softmax), and the paged decode of
// kernels/c/decode_attn.c:39-133.  Differences by design: the GQA group of a
// shared list is processed together (each K/V byte is read once per group),
// a list is split over several workgroups (split-K) whose partial softmax
// states are merged in LDS and then by a combine kernel, and an empty row
// yields zeros instead of NaN (block_sparse.py:115-119 computes exp(-inf+inf)).
//
// Data movement: a wave reads `RPI` consecutive token rows per load
// instruction, 16 (or 8) contiguous bytes per lane, LPR lanes per row, so every
// instruction reads whole rows.  Page ids are resolved to physical rows when
// the split's list is staged in LDS, so a paged read is one dependent load.
// Math: fp32 online softmax in the log2 domain (q is pre-scaled by
// scale*log2(e)); exp2 is the hardware v_exp_f32.
#include <algorithm>

#include "common.h"
#include "kv_access.h"

namespace la {

constexpr int SA_NT = 256;
constexpr int SA_NW = SA_NT / 64;
constexpr int SA_MAX_EPS = 1024;  // list entries staged per workgroup

struct AttnKP {
  const void *q;
  void *out;
  const int32_t *ids;
  const int32_t *counts;
  float *ws_acc;
  float *ws_ml;
  la_kv kv;
  int64_t B, Hq, Hkv, Tq, ids_heads, ids_rows, N;
  int64_t id_sb, id_sh, id_st;
  int64_t unit, offset, splits, eps;
  int64_t q_sb, q_sh, q_st, o_sb, o_sh, o_st;
  float qscale;
  int32_t q_dt, out_dt, causal;
  int32_t staged;      // paged: every unit lies inside one physical page
  int32_t unit_shift;  // log2(unit) when unit is a power of two, else -1
};

template <int KT>
struct KvTraits;
template <>
struct KvTraits<LA_F32> {
  static constexpr int ESZ = 4, LB = 16;
  using Vec = uint4;
};
template <>
struct KvTraits<LA_BF16> {
  static constexpr int ESZ = 2, LB = 16;
  using Vec = uint4;
};
template <>
struct KvTraits<LA_FP8_E4M3> {
  static constexpr int ESZ = 1, LB = 8;
  using Vec = uint2;
};

template <int KT, int EPL>
__device__ __forceinline__ void unpack(const typename KvTraits<KT>::Vec &v, float (&x)[EPL]) {
  if constexpr (KT == LA_F32) {
    x[0] = __uint_as_float(v.x);
    x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z);
    x[3] = __uint_as_float(v.w);
  } else if constexpr (KT == LA_BF16) {
    x[0] = bf16lo(v.x); x[1] = bf16hi(v.x);
    x[2] = bf16lo(v.y); x[3] = bf16hi(v.y);
    x[4] = bf16lo(v.z); x[5] = bf16hi(v.z);
    x[6] = bf16lo(v.w); x[7] = bf16hi(v.w);
  } else {
    float2 a = fp8x2_to_f32<false>(v.x), b = fp8x2_to_f32<true>(v.x);
    float2 c = fp8x2_to_f32<false>(v.y), d = fp8x2_to_f32<true>(v.y);
    x[0] = a.x; x[1] = a.y; x[2] = b.x; x[3] = b.y;
    x[4] = c.x; x[5] = c.y; x[6] = d.x; x[7] = d.y;
  }
}

template <int KT, int D, int G, int UNR, bool PAGED>
__global__ __launch_bounds__(SA_NT) void sparse_attn_kernel(AttnKP p) {
  using Tr = KvTraits<KT>;
  using Vec = typename Tr::Vec;
  constexpr int EPL = Tr::LB / Tr::ESZ;  // elements per lane
  constexpr int LPR = D / EPL;           // lanes per token row
  constexpr int RPI = 64 / LPR;          // rows per wave instruction
  static_assert(LPR >= 1 && LPR <= 64 && 64 % LPR == 0, "row must map onto a wave");

  __shared__ int32_t s_tok0[SA_MAX_EPS];  // logical first token of each entry (-1: skip)
  __shared__ int32_t s_phys[PAGED ? SA_MAX_EPS : 1];
  __shared__ float s_acc[SA_NW][G][D];
  __shared__ float s_m[SA_NW][G], s_l[SA_NW][G];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = lane % LPR;     // chunk of D this lane owns
  const int slot = lane / LPR;  // row slot within the wave
  const int64_t r = blockIdx.y;
  const int64_t split = blockIdx.x;
  const int64_t t = r % p.Tq;
  const int64_t ih = (r / p.Tq) % p.ids_heads;
  const int64_t b = r / (p.Tq * p.ids_heads);
  const int64_t grp = p.Hq / p.Hkv;
  const int64_t kvh = (p.ids_heads == p.Hkv) ? ih : ih / grp;
  const int64_t h0 = (p.ids_heads == p.Hkv) ? ih * G : ih;  // first query head
  const int64_t lrow = (p.ids_rows == 1) ? 0 : t;
  const int32_t *list = p.ids + b * p.id_sb + ih * p.id_sh + lrow * p.id_st;
  int64_t n_e = p.N;
  if (p.counts) n_e = min(n_e, (int64_t)p.counts[(b * p.ids_heads + ih) * p.ids_rows + lrow]);
  const int64_t e0 = split * p.eps;
  const int64_t e1 = min(n_e, e0 + p.eps);
  const int64_t ne = max((int64_t)0, e1 - e0);
  const int64_t len = kv_length(p.kv, b);
  const int64_t qpos = p.causal ? (p.offset + t) : (int64_t)0x7fffffffffffffffLL;
  const int64_t lim = min(len - 1, qpos);  // last attendable token

  // Stage the split's entries: logical first token (for masking) and, for a
  // paged cache, the pool row of that token (so a token costs no page lookup).
  for (int64_t e = tid; e < ne; e += SA_NT) {
    const int32_t id = list[e0 + e];
    const int64_t tok0 = (int64_t)id * p.unit;
    const bool ok = id >= 0 && tok0 <= lim;
    s_tok0[e] = ok ? (int32_t)tok0 : -1;
    if constexpr (PAGED) {
      if (p.staged && ok) {
        const int64_t ps = p.kv.page_size;
        const int64_t phys = p.kv.page_table[b * p.kv.pt_stride + tok0 / ps];
        s_phys[e] = (int32_t)((phys * p.Hkv + kvh) * ps + tok0 % ps);
      }
    }
  }
  const int64_t k_bh = b * p.kv.k_sb + kvh * p.kv.k_sh;  // contiguous-layout bases
  const int64_t v_bh = b * p.kv.v_sb + kvh * p.kv.v_sh;
  const int64_t s_bh = b * p.kv.s_sb + kvh * p.kv.s_sh;
  const int32_t lim32 = (int32_t)min(lim, (int64_t)0x7fffffff);

  // q chunk of this lane for the G heads, pre-scaled into the log2 domain.
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t qo = b * p.q_sb + (h0 + g) * p.q_sh + t * p.q_st + c * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qf[g][e] = load_as_f32(p.q, qo + e, p.q_dt) * p.qscale;
  }
  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = __int_as_float(0xff800000);
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }
  __syncthreads();

  const int64_t F = ne * p.unit;  // flat tokens of this split
  const char *kbase = (const char *)p.kv.k;
  const char *vbase = (const char *)p.kv.v;
  constexpr int64_t WAVE_SPAN = (int64_t)RPI * UNR;
  constexpr int64_t STEP = SA_NW * WAVE_SPAN;
  struct Batch {
    Vec kr[UNR], vr[UNR];
    float ksc[UNR], vsc[UNR];
    bool ok[UNR];
  };
  // Issue the loads of the batch starting at flat token `base`.
  auto load = [&](int64_t base, Batch &bt) {
    Vec(&kr)[UNR] = bt.kr;
    Vec(&vr)[UNR] = bt.vr;
    float(&ksc)[UNR] = bt.ksc;
    float(&vsc)[UNR] = bt.vsc;
    bool(&ok)[UNR] = bt.ok;
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      // flat token indices stay below 2^31 (checked on the host)
      const int32_t f = (int32_t)base + w * (int32_t)WAVE_SPAN + u * RPI + slot;
      int32_t e, j;
      if (p.unit_shift >= 0) {
        e = f >> p.unit_shift;
        j = f & ((1 << p.unit_shift) - 1);
      } else {
        e = (int32_t)((uint32_t)f / (uint32_t)p.unit);
        j = f - e * (int32_t)p.unit;
      }
      const int32_t es = min(e, SA_MAX_EPS - 1);
      const int32_t tok0 = (f < (int32_t)F) ? s_tok0[es] : -1;
      const int32_t tok = tok0 + j;
      ok[u] = tok0 >= 0 && tok <= lim32;
      kr[u] = Vec{};
      vr[u] = Vec{};
      ksc[u] = 1.f;
      vsc[u] = 1.f;
      if (ok[u]) {
        int64_t ko, vo, so = 0;
        if constexpr (PAGED) {
          int64_t prow;
          if (p.staged) {
            prow = (int64_t)((uint32_t)s_phys[es] + (uint32_t)j);  // pool rows < 2^32
          } else {
            const int64_t ps = p.kv.page_size;
            const int64_t phys = p.kv.page_table[b * p.kv.pt_stride + tok / ps];
            prow = (phys * p.Hkv + kvh) * ps + tok % ps;
          }
          ko = vo = prow * D;
          so = prow;
        } else {
          ko = k_bh + (int64_t)tok * p.kv.k_st;
          vo = v_bh + (int64_t)tok * p.kv.v_st;
          so = s_bh + (int64_t)tok * p.kv.s_st;
        }
        kr[u] = *(const Vec *)(kbase + (ko + c * EPL) * Tr::ESZ);
        vr[u] = *(const Vec *)(vbase + (vo + c * EPL) * Tr::ESZ);
        if constexpr (KT == LA_FP8_E4M3) {
          ksc[u] = p.kv.k_scale[so];
          vsc[u] = p.kv.v_scale[so];
        }
      }
    }
  };
  // Online-softmax update with one loaded batch.
  auto process = [&](Batch &bt) {
    Vec(&kr)[UNR] = bt.kr;
    Vec(&vr)[UNR] = bt.vr;
    float(&ksc)[UNR] = bt.ksc;
    float(&vsc)[UNR] = bt.vsc;
    bool(&ok)[UNR] = bt.ok;
    float s[G][UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      float kf[EPL];
      unpack<KT, EPL>(kr[u], kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) a = __builtin_fmaf(qf[g][e], kf[e], a);
        s[g][u] = a;
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g) s[g][u] = group_sum<LPR>(s[g][u]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mb = __int_as_float(0xff800000);
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        s[g][u] = ok[u] ? s[g][u] * ksc[u] : __int_as_float(0xff800000);
        mb = fmaxf(mb, s[g][u]);
      }
      const float mn = fmaxf(m[g], mb);
      const float mu = (mn == __int_as_float(0xff800000)) ? 0.f : mn;
      const float alpha = fast_exp2(m[g] - mu);
      l[g] *= alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
      m[g] = mn;
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const float pr = fast_exp2(s[g][u] - mu);
        l[g] += pr;
        s[g][u] = pr * vsc[u];
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      float vf[EPL];
      unpack<KT, EPL>(vr[u], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(s[g][u], vf[e], acc[g][e]);
    }
  };
  // Double-buffered: the next batch's loads are in flight while one is processed.
  Batch b0, b1;
  if (F > 0) load(0, b0);
  for (int64_t base = 0; base < F; base += 2 * STEP) {
    if (base + STEP < F) load(base + STEP, b1);
    process(b0);
    if (base + STEP >= F) break;
    if (base + 2 * STEP < F) load(base + 2 * STEP, b0);
    process(b1);
  }

  // Merge the row slots of the wave (lanes that own the same chunk c).
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off, 64);
      const float lo = __shfl_xor(l[g], off, 64);
      const float mn = fmaxf(m[g], mo);
      const float mu = (mn == __int_as_float(0xff800000)) ? 0.f : mn;
      const float a = fast_exp2(m[g] - mu), bb = fast_exp2(mo - mu);
      l[g] = l[g] * a + lo * bb;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float ao = __shfl_xor(acc[g][e], off, 64);
        acc[g][e] = acc[g][e] * a + ao * bb;
      }
      m[g] = mn;
    }
  }
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_acc[w][g][c * EPL + e] = acc[g][e];
      if (c == 0) {
        s_m[w][g] = m[g];
        s_l[w][g] = l[g];
      }
    }
  }
  __syncthreads();
  // Merge the waves, then write the output or this split's partial state.
  for (int i = tid; i < G * D; i += SA_NT) {
    const int g = i / D, d = i % D;
    float M = __int_as_float(0xff800000);
#pragma unroll
    for (int x = 0; x < SA_NW; ++x) M = fmaxf(M, s_m[x][g]);
    const float Mu = (M == __int_as_float(0xff800000)) ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int x = 0; x < SA_NW; ++x) {
      const float sc = fast_exp2(s_m[x][g] - Mu);
      L += s_l[x][g] * sc;
      A += s_acc[x][g][d] * sc;
    }
    const int64_t h = h0 + g;
    if (p.splits == 1) {
      const float o = L > 0.f ? A / L : 0.f;
      store_from_f32(p.out, b * p.o_sb + h * p.o_sh + t * p.o_st + d, p.out_dt, o);
    } else {
      const int64_t pi = (r * G + g) * p.splits + split;
      p.ws_acc[pi * D + d] = A;
      if (d == 0) {
        p.ws_ml[pi * 2 + 0] = M;
        p.ws_ml[pi * 2 + 1] = L;
      }
    }
  }
}

// Merge the split partials of one (row, head): one workgroup, D threads.
__global__ __launch_bounds__(256) void sparse_attn_combine(AttnKP p, int64_t G, int64_t D) {
  const int64_t rg = blockIdx.x;
  const int64_t r = rg / G, g = rg % G;
  const int64_t t = r % p.Tq;
  const int64_t ih = (r / p.Tq) % p.ids_heads;
  const int64_t b = r / (p.Tq * p.ids_heads);
  const int64_t h = ((p.ids_heads == p.Hkv) ? ih * G : ih) + g;
  const float *ml = p.ws_ml + rg * p.splits * 2;
  float M = __int_as_float(0xff800000);
  for (int64_t s = 0; s < p.splits; ++s) M = fmaxf(M, ml[2 * s]);
  const float Mu = (M == __int_as_float(0xff800000)) ? 0.f : M;
  for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
    float L = 0.f, A = 0.f;
    for (int64_t s = 0; s < p.splits; ++s) {
      const float sc = fast_exp2(ml[2 * s] - Mu);
      L += ml[2 * s + 1] * sc;
      A += p.ws_acc[(rg * p.splits + s) * D + d] * sc;
    }
    const float o = L > 0.f ? A / L : 0.f;
    store_from_f32(p.out, b * p.o_sb + h * p.o_sh + t * p.o_st + d, p.out_dt, o);
  }
}

// Tokens per row slot per batch; two batches are in flight per wave.
template <int KT>
constexpr int unroll_for(int D) {
  return 4;
}

template <int KT, int D, int G, bool PAGED>
static int launch_attn(const AttnKP &p, hipStream_t st) {
  constexpr int UNR = unroll_for<KT>(D);
  dim3 grid((unsigned)p.splits, (unsigned)(p.B * p.ids_heads * p.Tq));
  sparse_attn_kernel<KT, D, G, UNR, PAGED><<<grid, SA_NT, 0, st>>>(p);
  LA_LAUNCHED();
  if (p.splits > 1) {
    sparse_attn_combine<<<dim3((unsigned)(p.B * p.ids_heads * p.Tq * G)), D, 0, st>>>(p, G, D);
    LA_LAUNCHED();
  }
  return LA_OK;
}

template <int KT, int D, int G>
static int dispatch_paged(const AttnKP &p, hipStream_t st) {
  if (p.kv.page_table) return launch_attn<KT, D, G, true>(p, st);
  return launch_attn<KT, D, G, false>(p, st);
}

template <int KT, int D>
static int dispatch_g(const AttnKP &p, int64_t G, hipStream_t st) {
  switch (G) {
    case 1: return dispatch_paged<KT, D, 1>(p, st);
    case 2: return dispatch_paged<KT, D, 2>(p, st);
    case 4: return dispatch_paged<KT, D, 4>(p, st);
    case 8:
      if constexpr (KT != LA_FP8_E4M3) return dispatch_paged<KT, D, 8>(p, st);
      break;
    default: break;
  }
  return fail(LA_ERR_UNSUPPORTED, "sparse attention: group of %lld heads per list", (long long)G);
}

template <int KT>
static int dispatch_d(const AttnKP &p, int64_t D, int64_t G, hipStream_t st) {
  switch (D) {
    case 64: return dispatch_g<KT, 64>(p, G, st);
    case 128: return dispatch_g<KT, 128>(p, G, st);
    default: return fail(LA_ERR_UNSUPPORTED, "sparse attention: head_dim %lld not in {64,128}", (long long)D);
  }
}

struct Plan {
  int64_t G, R, splits, eps;
  size_t ws;
};

static int plan_attn(const la_sparse_attn_args *a, const la_kv *kv, Plan &pl) {
  LA_REQUIRE(a && kv, "sparse attention: null arguments");
  LA_REQUIRE(a->q && a->out && a->ids && kv->k && kv->v, "sparse attention: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hq > 0 && a->Hkv > 0 && a->Tq > 0 && a->D > 0, "sparse attention: bad shape");
  LA_REQUIRE(a->Hq % a->Hkv == 0, "n_heads must be a multiple of n_kv_heads");
  LA_REQUIRE(a->ids_heads == a->Hkv || a->ids_heads == a->Hq,
             "sparse attention: ids must have one list per KV head or per query head");
  LA_REQUIRE(a->ids_rows == 1 || a->ids_rows == a->Tq, "sparse attention: ids rows must be 1 or Tq");
  LA_REQUIRE(a->N >= 1 && a->unit >= 1, "sparse attention: empty list width or unit");
  LA_REQUIRE(kv->T >= 1, "sparse attention: empty KV cache");
  LA_REQUIRE(a->q_dtype == LA_F32 || a->q_dtype == LA_BF16 || a->q_dtype == LA_F16, "q dtype");
  LA_REQUIRE(a->out_dtype == LA_F32 || a->out_dtype == LA_BF16 || a->out_dtype == LA_F16, "out dtype");
  LA_REQUIRE(kv->dtype == LA_F32 || kv->dtype == LA_BF16 || kv->dtype == LA_FP8_E4M3, "KV dtype");
  if (kv->dtype == LA_FP8_E4M3) LA_REQUIRE(kv->k_scale && kv->v_scale, "fp8 KV needs per-token scales");
  if (kv->page_table) LA_REQUIRE(kv->page_size >= 1 && kv->pt_stride >= 1, "paged KV: bad page size");
  {
    // every lane reads one 16-byte (fp8: 8-byte) vector of a row
    const int64_t esz = kv->dtype == LA_F32 ? 4 : kv->dtype == LA_BF16 ? 2 : 1;
    const int64_t lb = kv->dtype == LA_FP8_E4M3 ? 8 : 16;
    const int64_t epl = lb / esz;
    bool al = ((uintptr_t)kv->k % lb == 0) && ((uintptr_t)kv->v % lb == 0) && (a->D % epl == 0);
    if (!kv->page_table)
      al = al && kv->k_sb % epl == 0 && kv->k_sh % epl == 0 && kv->k_st % epl == 0 &&
           kv->v_sb % epl == 0 && kv->v_sh % epl == 0 && kv->v_st % epl == 0;
    LA_REQUIRE(al, "sparse attention: K/V rows must be contiguous and %lld-byte aligned", (long long)lb);
    LA_REQUIRE(a->N * a->unit < (int64_t)1 << 31, "sparse attention: list spans >= 2^31 tokens");
  }
  pl.G = (a->ids_heads == a->Hkv) ? a->Hq / a->Hkv : 1;
  pl.R = a->B * a->ids_heads * a->Tq;
  const int64_t min_splits = ceil_div(a->N, SA_MAX_EPS);
  int64_t splits = a->num_splits;
  if (splits <= 0) {
    const int64_t target = 2048;  // workgroups: 8 per CU
    const int64_t tokens = a->N * a->unit;
    const int64_t by_tokens = std::max<int64_t>(1, tokens / 256);
    splits = std::min(ceil_div(target, pl.R), by_tokens);
  }
  splits = std::max(splits, min_splits);
  splits = std::min(splits, a->N);
  splits = std::max<int64_t>(splits, 1);
  pl.eps = ceil_div(a->N, splits);
  splits = ceil_div(a->N, pl.eps);
  pl.splits = splits;
  pl.ws = splits > 1 ? (size_t)(pl.R * pl.G * splits) * (size_t)(a->D + 2) * sizeof(float) : 0;
  return LA_OK;
}

}  // namespace la

using namespace la;

extern "C" size_t la_sparse_attention_workspace(const la_sparse_attn_args *a, const la_kv *kv) {
  Plan pl{};
  if (plan_attn(a, kv, pl) != LA_OK) return 0;
  return pl.ws;
}

extern "C" int la_sparse_attention(const la_sparse_attn_args *a, const la_kv *kv, void *stream) {
  Plan pl{};
  int rc = plan_attn(a, kv, pl);
  if (rc != LA_OK) return rc;
  if (pl.ws > 0) {
    LA_REQUIRE(a->workspace != nullptr, "sparse attention: workspace required");
    if ((size_t)a->ws_bytes < pl.ws)
      return fail(LA_ERR_WORKSPACE, "sparse attention: workspace %lld < %zu bytes",
                  (long long)a->ws_bytes, pl.ws);
  }
  AttnKP p{};
  p.q = a->q;
  p.out = a->out;
  p.ids = a->ids;
  p.counts = a->counts;
  p.kv = *kv;
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.Tq = a->Tq;
  p.ids_heads = a->ids_heads;
  p.ids_rows = a->ids_rows;
  p.N = a->N;
  p.id_sb = a->id_sb;
  p.id_sh = a->id_sh;
  p.id_st = a->id_st;
  p.unit = a->unit;
  p.offset = a->offset;
  p.splits = pl.splits;
  p.eps = pl.eps;
  p.q_sb = a->q_sb;
  p.q_sh = a->q_sh;
  p.q_st = a->q_st;
  p.o_sb = a->o_sb;
  p.o_sh = a->o_sh;
  p.o_st = a->o_st;
  p.qscale = a->scale * 1.4426950408889634f;
  p.q_dt = a->q_dtype;
  p.out_dt = a->out_dtype;
  p.causal = a->causal;
  p.staged = kv->page_table ? (kv->page_size % a->unit == 0) : 0;
  p.unit_shift = is_pow2(a->unit) ? ilog2(a->unit) : -1;
  if (pl.splits > 1) {
    p.ws_ml = (float *)a->workspace;
    p.ws_acc = p.ws_ml + pl.R * pl.G * pl.splits * 2;
  }
  hipStream_t st = (hipStream_t)stream;
  switch (kv->dtype) {
    case LA_F32: return dispatch_d<LA_F32>(p, a->D, pl.G, st);
    case LA_BF16: return dispatch_d<LA_BF16>(p, a->D, pl.G, st);
    case LA_FP8_E4M3:
      if (pl.G > 4) return fail(LA_ERR_UNSUPPORTED, "fp8 sparse attention: group > 4");
      return dispatch_d<LA_FP8_E4M3>(p, a->D, pl.G, st);
    default: return fail(LA_ERR_INVALID, "KV dtype");
  }
}
