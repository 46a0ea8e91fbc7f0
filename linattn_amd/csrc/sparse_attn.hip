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
#include <cstdlib>

#include <mutex>

#include "common.h"
#include "kv_access.h"
#include "quest_select.h"

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

// streamed (read-once) K/V rows: nontemporal loads
__device__ __forceinline__ uint4 nt_ld(const uint4 *p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u x = __builtin_nontemporal_load((const v4u *)p);
  return uint4{x[0], x[1], x[2], x[3]};
}
__device__ __forceinline__ uint2 nt_ld(const uint2 *p) {
  typedef uint32_t v2u __attribute__((ext_vector_type(2)));
  const v2u x = __builtin_nontemporal_load((const v2u *)p);
  return uint2{x[0], x[1]};
}

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

// Work of one (row, split): which list entries it covers and where the
// row's K/V live.  Row r = (b, list head ih, query t).
struct RowCtx {
  int64_t b, t, kvh, h0, e0, ne, lim;
  int64_t k_bh, v_bh, s_bh;  // contiguous-layout bases
};

// Decodes the row of this workgroup and stages its split's entries in LDS:
// the logical first token (for masking; -1 = skip) and, for a paged cache,
// the pool row of that token, so a token costs no page-table lookup.  The
// caller synchronises before reading the staged entries.
template <int G, bool PAGED>
__device__ __forceinline__ RowCtx stage_row(const AttnKP &p, int32_t *s_tok0, int32_t *s_phys) {
  RowCtx rc;
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.y;
  const int64_t split = blockIdx.x;
  rc.t = r % p.Tq;
  const int64_t ih = (r / p.Tq) % p.ids_heads;
  rc.b = r / (p.Tq * p.ids_heads);
  const int64_t grp = p.Hq / p.Hkv;
  rc.kvh = (p.ids_heads == p.Hkv) ? ih : ih / grp;
  rc.h0 = (p.ids_heads == p.Hkv) ? ih * G : ih;  // first query head
  const int64_t lrow = (p.ids_rows == 1) ? 0 : rc.t;
  const int32_t *list = p.ids + rc.b * p.id_sb + ih * p.id_sh + lrow * p.id_st;
  int64_t n_e = p.N;
  if (p.counts) n_e = min(n_e, (int64_t)p.counts[(rc.b * p.ids_heads + ih) * p.ids_rows + lrow]);
  // the row's valid entries are spread evenly over the splits
  const int64_t eps = (n_e + p.splits - 1) / p.splits;
  rc.e0 = split * eps;
  const int64_t e1 = min(n_e, rc.e0 + eps);
  rc.ne = max((int64_t)0, e1 - rc.e0);
  const int64_t len = kv_length(p.kv, rc.b);
  const int64_t qpos = p.causal ? (p.offset + rc.t) : (int64_t)0x7fffffffffffffffLL;
  rc.lim = min(len - 1, qpos);  // last attendable token
  for (int64_t e = tid; e < rc.ne; e += SA_NT) {
    const int32_t id = list[rc.e0 + e];
    const int64_t tok0 = (int64_t)id * p.unit;
    const bool ok = id >= 0 && tok0 <= rc.lim;
    s_tok0[e] = ok ? (int32_t)tok0 : -1;
    if constexpr (PAGED) {
      if (p.staged && ok) {
        const int64_t ps = p.kv.page_size;
        const int64_t phys = p.kv.page_table[rc.b * p.kv.pt_stride + tok0 / ps];
        s_phys[e] = (int32_t)((phys * p.Hkv + rc.kvh) * ps + tok0 % ps);
      }
    }
  }
  rc.k_bh = rc.b * p.kv.k_sb + rc.kvh * p.kv.k_sh;
  rc.v_bh = rc.b * p.kv.v_sb + rc.kvh * p.kv.v_sh;
  rc.s_bh = rc.b * p.kv.s_sb + rc.kvh * p.kv.s_sh;
  return rc;
}

// Flat token f of the split (entry f / unit, token f % unit of the entry):
// returns whether it is attended and, if so, the element offsets of its K and
// V rows and the index of its scale.  Flat indices stay below 2^31 (checked
// on the host).
template <int D, bool PAGED>
__device__ __forceinline__ bool token_rows(const AttnKP &p, const RowCtx &rc, const int32_t *s_tok0,
                                           const int32_t *s_phys, int32_t f, int32_t F,
                                           int32_t lim32, int64_t &ko, int64_t &vo, int64_t &so) {
  int32_t e, j;
  if (p.unit_shift >= 0) {
    e = f >> p.unit_shift;
    j = f & ((1 << p.unit_shift) - 1);
  } else {
    e = (int32_t)((uint32_t)f / (uint32_t)p.unit);
    j = f - e * (int32_t)p.unit;
  }
  const int32_t es = min(e, SA_MAX_EPS - 1);
  const int32_t tok0 = (f < F) ? s_tok0[es] : -1;
  const int32_t tok = tok0 + j;
  if (!(tok0 >= 0 && tok <= lim32)) return false;
  if constexpr (PAGED) {
    int64_t prow;
    if (p.staged) {
      prow = (int64_t)((uint32_t)s_phys[es] + (uint32_t)j);  // pool rows < 2^32
    } else {
      const int64_t ps = p.kv.page_size;
      const int64_t phys = p.kv.page_table[rc.b * p.kv.pt_stride + tok / ps];
      prow = (phys * p.Hkv + rc.kvh) * ps + tok % ps;
    }
    ko = vo = prow * D;
    so = prow * p.kv.s_st;  // paged scales: pool row r at r * s_st
  } else {
    ko = rc.k_bh + (int64_t)tok * p.kv.k_st;
    vo = rc.v_bh + (int64_t)tok * p.kv.v_st;
    so = rc.s_bh + (int64_t)tok * p.kv.s_st;
  }
  return true;
}

// Merges the per-wave softmax states (s_m, s_l, s_acc, filled by every wave
// before a barrier) and writes the output row, or this split's partial state.
template <int G, int D, int NW = SA_NW>
__device__ __forceinline__ void finish_row(const AttnKP &p, const RowCtx &rc, int64_t r,
                                           int64_t split, const float (*s_acc)[G][D],
                                           const float (*s_m)[G], const float (*s_l)[G]) {
  for (int i = threadIdx.x; i < G * D; i += 64 * NW) {
    const int g = i / D, d = i % D;
    float M = __int_as_float(0xff800000);
#pragma unroll
    for (int x = 0; x < NW; ++x) M = fmaxf(M, s_m[x][g]);
    const float Mu = (M == __int_as_float(0xff800000)) ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int x = 0; x < NW; ++x) {
      const float sc = fast_exp2(s_m[x][g] - Mu);
      L += s_l[x][g] * sc;
      A += s_acc[x][g][d] * sc;
    }
    const int64_t h = rc.h0 + g;
    if (p.splits == 1) {
      const float o = L > 0.f ? A / L : 0.f;
      store_from_f32(p.out, rc.b * p.o_sb + h * p.o_sh + rc.t * p.o_st + d, p.out_dt, o);
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

template <int KT, int D, int G, int UNR, bool PAGED>
__global__ __launch_bounds__(SA_NT) void sparse_attn_kernel(AttnKP p) {
  using Tr = KvTraits<KT>;
  using Vec = typename Tr::Vec;
  constexpr int EPL = Tr::LB / Tr::ESZ;  // elements per lane
  constexpr int LPR = D / EPL;           // lanes per token row
  constexpr int RPI = 64 / LPR;          // rows per wave instruction
  static_assert(LPR >= 1 && LPR <= 64 && 64 % LPR == 0, "row must map onto a wave");

  __shared__ int32_t s_tok0[SA_MAX_EPS];
  __shared__ int32_t s_phys[PAGED ? SA_MAX_EPS : 1];
  __shared__ float s_acc[SA_NW][G][D];
  __shared__ float s_m[SA_NW][G], s_l[SA_NW][G];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = lane % LPR;     // chunk of D this lane owns
  const int slot = lane / LPR;  // row slot within the wave
  const RowCtx rc = stage_row<G, PAGED>(p, s_tok0, s_phys);
  const int32_t lim32 = (int32_t)min(rc.lim, (int64_t)0x7fffffff);

  // q chunk of this lane for the G heads, pre-scaled into the log2 domain.
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t qo = rc.b * p.q_sb + (rc.h0 + g) * p.q_sh + rc.t * p.q_st + c * EPL;
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

  const int32_t F = (int32_t)(rc.ne * p.unit);  // flat tokens of this split
  const char *kbase = (const char *)p.kv.k;
  const char *vbase = (const char *)p.kv.v;
  constexpr int32_t WAVE_SPAN = RPI * UNR;
  constexpr int32_t STEP = SA_NW * WAVE_SPAN;
  struct Batch {
    Vec kr[UNR], vr[UNR];
    float ksc[UNR], vsc[UNR];
    bool ok[UNR];
  };
  // Issue the loads of the batch starting at flat token `base`.
  auto load = [&](int32_t base, Batch &bt) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int32_t f = base + w * WAVE_SPAN + u * RPI + slot;
      int64_t ko = 0, vo = 0, so = 0;
      bt.ok[u] = token_rows<D, PAGED>(p, rc, s_tok0, s_phys, f, F, lim32, ko, vo, so);
      bt.kr[u] = Vec{};
      bt.vr[u] = Vec{};
      bt.ksc[u] = 1.f;
      bt.vsc[u] = 1.f;
      if (bt.ok[u]) {
        bt.kr[u] = *(const Vec *)(kbase + (ko + c * EPL) * Tr::ESZ);
        bt.vr[u] = *(const Vec *)(vbase + (vo + c * EPL) * Tr::ESZ);
        if constexpr (KT == LA_FP8_E4M3) {
          bt.ksc[u] = p.kv.k_scale[so];
          bt.vsc[u] = p.kv.v_scale[so];
        }
      }
    }
  };
  // Online-softmax update with one loaded batch.
  auto process = [&](Batch &bt) {
    float s[G][UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      float kf[EPL];
      unpack<KT, EPL>(bt.kr[u], kf);
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
        s[g][u] = bt.ok[u] ? s[g][u] * bt.ksc[u] : __int_as_float(0xff800000);
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
        s[g][u] = pr * bt.vsc[u];
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      float vf[EPL];
      unpack<KT, EPL>(bt.vr[u], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(s[g][u], vf[e], acc[g][e]);
    }
  };
  // Double-buffered: the next batch's loads are in flight while one is processed.
  Batch b0, b1;
  if (F > 0) load(0, b0);
  for (int32_t base = 0; base < F; base += 2 * STEP) {
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
  finish_row<G, D>(p, rc, blockIdx.y, blockIdx.x, s_acc, s_m, s_l);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per-lane scales of the fp8 matrix-core kernel (empty for bf16 K/V).
template <bool F8>
struct Fp8Scales {
  float k = 0.f, v[4] = {0.f, 0.f, 0.f, 0.f};
};
template <>
struct Fp8Scales<false> {};

// Maximum over the 16 lanes of a DPP row; every lane of the row gets it.
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));
  x = fmaxf(x, dpp_f32<0x4E>(x));
  x = fmaxf(x, dpp_f32<0x141>(x));
  x = fmaxf(x, dpp_f32<0x140>(x));
  return x;
}

// bf16 K/V, bf16 q, head dim 128: scores on the matrix cores.
//
// Each wave walks its own tokens, 16 per round.  S = Q K^T for the round is
// four v_mfma_f32_16x16x32_bf16 (A = the G query rows of q, zero above G;
// B = K^T, lane l holding 8 dims of token l % 16), which leaves lane
// 16*(h/4) + i holding S[head h][token i], h % 4 in the accumulator element.
// The softmax reference max is wave-uniform (round maxima by DPP row
// reductions, then readlane), so the four row slots of the PV product share
// it and merge by plain sums.  Probabilities pass through LDS to the PV
// lanes, which read V rows 16 contiguous bytes per lane (a token per 16
// lanes) and accumulate O on the VALU in fp32.
//
// fp8 e4m3 K/V with per-token scales (KT = LA_FP8_E4M3): the scores come from
// v_mfma_f32_16x16x32_fp8_fp8 on the K codes as stored.  q is quantised in
// the kernel to a two-term fp8 expansion, q ~ sq * (hi + lo), with one scale
// sq = absmax/448 over the G heads and lo = fp8(q/sq - hi) (the residual, in
// the same code units, down to the e4m3 subnormal step 2^-9), so
// S = ks_t * sq * (hi + lo).K is eight fp8 MFMAs into one accumulator per
// round and keeps q to ~2^-8 relative; the per-token K scale multiplies the
// fp32 scores, and each V row is decoded in registers with its scale folded
// into the token's weight.
// LDS of the matrix-core attention body for NW waves (G heads, D = 128).
template <int KT, int G, int NW>
struct MfmaLds {
  static constexpr int NRG = (G + 3) / 4;
  float acc[NW][G][128];
  float m[NW][G], l[NW][G];
  __attribute__((aligned(16))) float p[NW][16][4 * NRG];
  long q8[KT == LA_FP8_E4M3 ? 2 * 4 * 64 : 1];  // fp8: [term][s][lane] q codes
  float sq;                                     // fp8: their scale
};

// The attention of one row by NW waves over the entries staged in s_tok0 /
// s_phys (the caller synchronises after staging, before the body reads
// them): every wave leaves its softmax state (m, l, acc) in L and the body
// ends with a workgroup barrier, so finish_row can merge them.
template <int KT, int G, bool PAGED, bool U16, int NW>
__device__ __forceinline__ void mfma_attend(const AttnKP &p, const RowCtx &rc,
                                            const int32_t *s_tok0, const int32_t *s_phys,
                                            MfmaLds<KT, G, NW> &L) {
  constexpr bool F8 = KT == LA_FP8_E4M3;
  constexpr int ESZ = F8 ? 1 : 2;  // bytes per K/V element
  constexpr int D = 128;
  constexpr int RT = 16;            // tokens per wave round
  constexpr int NRG = (G + 3) / 4;  // DPP rows holding heads
  static_assert(G >= 1 && G <= 8, "group of at most 8 heads");
  auto &s_acc = L.acc;
  auto &s_m = L.m;
  auto &s_l = L.l;
  auto &s_p = L.p;
  long *s_q8 = L.q8;
  float &s_sq = L.sq;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = lane & 15;     // V: 8-dim chunk; K: token of the round
  const int slot = lane >> 4;  // V: token slot; K: 8-dim group within 32
  const int32_t lim32 = (int32_t)min(rc.lim, (int64_t)0x7fffffff);

  // A operand: q row c (head c < G), dims 32s + 8*slot .. +8, raw bf16 bits
  // (fp8: dims 32*slot + 8s .. +8 of the hi and lo codes, the same dims as
  // the K bytes the lane feeds to MFMA s).
  bf16x8 qa[4];
  if constexpr (!F8) {
    const uint16_t *qp = (const uint16_t *)p.q;
    const int64_t qo = rc.b * p.q_sb + (rc.h0 + c) * p.q_sh + rc.t * p.q_st + 8 * slot;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      uint16_t x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = c < G ? qp[qo + 32 * s + e] : (uint16_t)0;
      qa[s] = __builtin_bit_cast(bf16x8, x);
    }
  } else if (w == 0) {  // fp8: wave 0 writes the codes for the workgroup
    const uint16_t *qp = (const uint16_t *)p.q;
    const int64_t qo = rc.b * p.q_sb + (rc.h0 + c) * p.q_sh + rc.t * p.q_st + 32 * slot;
    float x[32];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      x[i] = c < G ? bf16_bits_to_f32(qp[qo + i]) : 0.f;
      amax = fmaxf(amax, fabsf(x[i]));
    }
    // absmax over the wave: the 4 lanes of a head, then the 16 heads
    const float am = row_max16(pair32_max(pair16_max(amax)));
    const float sq = am > 0.f ? am / 448.f : 1.f;
    if (lane == 0) s_sq = sq;
    const float inv = 1.f / sq;
#pragma unroll
    for (int i = 0; i < 32; ++i) x[i] *= inv;
    // codes of x by round to nearest; x keeps the residual
    auto term = [&](int tm) {
      uint32_t wd[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int wv = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * j], x[4 * j + 1], 0, false);
        wv = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * j + 2], x[4 * j + 3], wv, true);
        wd[j] = (uint32_t)wv;
        const float2 a = fp8x2_to_f32<false>(wd[j]), b = fp8x2_to_f32<true>(wd[j]);
        x[4 * j] -= a.x;
        x[4 * j + 1] -= a.y;
        x[4 * j + 2] -= b.x;
        x[4 * j + 3] -= b.y;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
        s_q8[(tm * 4 + s) * 64 + lane] = (long)(((uint64_t)wd[2 * s + 1] << 32) | (uint64_t)wd[2 * s]);
    };
    term(0);
    term(1);
  }
  float ms[4], ls[4];  // per DPP row: max and partial sums of heads 4*slot + e
  float acc[G][8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    ms[e] = __int_as_float(0xff800000);
    ls[e] = 0.f;
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  __syncthreads();

  const int32_t F = (int32_t)(rc.ne * p.unit);
  const char *kbase = (const char *)p.kv.k;
  const char *vbase = (const char *)p.kv.v;
  constexpr int32_t STEP = NW * RT;
  // One set of K/V registers, refilled as it is consumed: the next round's K
  // loads are issued once the current K is in the matrix core, and each V
  // row of the next round once the current one has been accumulated.
  uint4 kr[F8 ? 2 : 4];
  typename KvTraits<KT>::Vec vr[4];
  Fp8Scales<F8> f8s;  // fp8: scales of this lane's K / V tokens
  bool kok = false;
  // U16 (units of 16k tokens lying inside one page): the 16 tokens of a round
  // are consecutive rows of one entry, so the entry lookup is wave-uniform and
  // every row address is a scalar base plus a lane offset.
  const int wu = __builtin_amdgcn_readfirstlane(w);
  struct Round {
    int32_t tok;    // first token of the round (-1: nothing to attend)
    int64_t kb, vb; // element offsets of its K and V rows
    int64_t sb;     // fp8: index of its first token's scale (tokens s_st apart)
  };
  auto round_of = [&](int32_t base) {
    Round rd{-1, 0, 0, 0};
    const int32_t fw = base + wu * RT;
    if (fw >= F) return rd;
    int32_t e, j;
    if (p.unit_shift >= 0) {
      e = fw >> p.unit_shift;
      j = fw & ((1 << p.unit_shift) - 1);
    } else {
      e = (int32_t)((uint32_t)fw / (uint32_t)p.unit);
      j = fw - e * (int32_t)p.unit;
    }
    const int32_t t0 = __builtin_amdgcn_readfirstlane(s_tok0[e]);
    if (t0 < 0) return rd;
    rd.tok = t0 + j;
    if constexpr (PAGED) {
      const uint32_t prow = (uint32_t)__builtin_amdgcn_readfirstlane(s_phys[e]) + (uint32_t)j;
      rd.kb = rd.vb = (int64_t)prow * D;
      rd.sb = (int64_t)prow * p.kv.s_st;
    } else {
      rd.kb = rc.k_bh + (int64_t)rd.tok * p.kv.k_st;
      rd.vb = rc.v_bh + (int64_t)rd.tok * p.kv.v_st;
      rd.sb = rc.s_bh + (int64_t)rd.tok * p.kv.s_st;
    }
    return rd;
  };
  Round rd_next{-1, 0, 0, 0};
  // U16 loads are issued for every lane: the 16 rows of a round lie in one
  // pool page, so every row address is valid; a round with nothing to attend
  // reads the first rows of the pool instead.  Tokens that are not attended
  // have their K columns masked and their V rows zeroed after the load.
  // K: bf16, dims 32s + 8*slot (four 16-byte loads); fp8, dims 32*slot ..
  // +32 (two).  V: dims 8c .. +8 of token slot (+4u) of the round.
  const uint32_t koff = (uint32_t)((c * D + (F8 ? 32 : 8) * slot) * ESZ);
  const uint32_t voff = (uint32_t)((slot * D + 8 * c) * ESZ);
  using VVec = typename KvTraits<KT>::Vec;
  uint32_t prow_k = 0xffffffffu;  // paged token lists: pool row of this lane's K token (~0: none)
  auto load_k = [&](int32_t base) {
    if constexpr (U16) {
      rd_next = round_of(base);
      kok = rd_next.tok >= 0 && rd_next.tok + c <= lim32;
      const char *rp = rd_next.tok >= 0 ? kbase + rd_next.kb * ESZ : kbase;  // wave-uniform
#pragma unroll
      for (int s = 0; s < (F8 ? 2 : 4); ++s) kr[s] = nt_ld((const uint4 *)(rp + koff + 16 * (F8 ? 1 : 4) * s));
      if constexpr (F8) f8s.k = p.kv.k_scale[rd_next.tok >= 0 ? rd_next.sb + c * p.kv.s_st : 0];
    } else {
      int64_t ko = 0, vo = 0, so = 0;
      kok = token_rows<D, PAGED>(p, rc, s_tok0, s_phys, base + w * RT + c, F, lim32, ko, vo, so);
      if constexpr (PAGED) prow_k = kok ? (uint32_t)(ko / D) : 0xffffffffu;  // ko = pool row * D
      if constexpr (F8) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
          kr[s] = kok ? *(const uint4 *)(kbase + ko + 32 * slot + 16 * s) : uint4{0, 0, 0, 0};
        f8s.k = kok ? p.kv.k_scale[so] : 0.f;
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          kr[s] = kok ? *(const uint4 *)(kbase + (ko + 32 * s + 8 * slot) * 2) : uint4{0, 0, 0, 0};
      }
    }
  };
  auto load_v = [&](int32_t base, int u) {
    if constexpr (U16) {
      const bool ok = rd_next.tok >= 0 && rd_next.tok + 4 * u + slot <= lim32;
      const char *rp = rd_next.tok >= 0 ? vbase + rd_next.vb * ESZ : vbase;  // wave-uniform
      const VVec x = nt_ld((const VVec *)(rp + voff + 4 * u * D * ESZ));
      if constexpr (F8) vr[u] = ok ? x : uint2{0, 0}; else vr[u] = ok ? x : uint4{0, 0, 0, 0};
      if constexpr (F8) {
        const float sv =
            p.kv.v_scale[rd_next.tok >= 0 ? rd_next.sb + (4 * u + slot) * p.kv.s_st : 0];
        f8s.v[u] = ok ? sv : 0.f;
      }
    } else {
      int64_t ko = 0, vo = 0, so = 0;
      bool ok;
      if constexpr (PAGED) {
        // a paged K and V row share the pool row, which the round's K load
        // (issued first) resolved on lane 4u + slot
        const uint32_t pr = (uint32_t)__shfl((int)prow_k, 4 * u + slot, 64);
        ok = pr != 0xffffffffu;
        vo = (int64_t)pr * D;
        so = (int64_t)pr * p.kv.s_st;
      } else {
        ok = token_rows<D, PAGED>(p, rc, s_tok0, s_phys, base + w * RT + 4 * u + slot, F, lim32, ko, vo, so);
      }
      if constexpr (F8) vr[u] = ok ? *(const VVec *)(vbase + (vo + 8 * c) * ESZ) : uint2{0, 0}; else vr[u] = ok ? *(const VVec *)(vbase + (vo + 8 * c) * ESZ) : uint4{0, 0, 0, 0};
      if constexpr (F8) f8s.v[u] = ok ? p.kv.v_scale[so] : 0.f;
    }
  };
  if (F > 0) {
    load_k(0);
#pragma unroll
    for (int u = 0; u < 4; ++u) load_v(0, u);
  }
  for (int32_t base = 0; base < F; base += STEP) {
    const bool more = base + STEP < F;
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
    float kq = p.qscale;  // fp8: times the q scale and the K scale of this lane's token
    if constexpr (F8) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 &kk = kr[s >> 1];
        const long kb8 = (s & 1) ? (long)(((uint64_t)kk.w << 32) | kk.z)
                                 : (long)(((uint64_t)kk.y << 32) | kk.x);
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(s_q8[s * 64 + lane], kb8, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(s_q8[(4 + s) * 64 + lane], kb8, sacc, 0, 0, 0);
      }
      kq *= s_sq * f8s.k;
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[s], __builtin_bit_cast(bf16x8, kr[s]), sacc, 0, 0, 0);
    }
    const bool cur_ok = kok;
    if (U16 || more) load_k(base + STEP);
    __builtin_amdgcn_sched_barrier(0);
    float sv[4], mn[4];
    bool grow = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float raw = sacc[e];
      sv[e] = cur_ok ? raw * kq : __int_as_float(0xff800000);
      mn[e] = fmaxf(ms[e], row_max16(sv[e]));
      grow = grow || (slot < NRG && mn[e] - ms[e] > 8.f);
    }
    // the G heads' reference maxima are wave-uniform (DPP row 0: heads 0-3,
    // row 1: 4-7); a reference is raised (acc, l rescaled) only when a round
    // maximum exceeds it by more than 8 in the log2 domain, so the weights
    // stay below 256 and most rounds skip the rescale
    if (__ballot(grow) != 0) {
      float al[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float u = (mn[e] == __int_as_float(0xff800000)) ? 0.f : mn[e];
        al[e] = fast_exp2(ms[e] - u);
        ls[e] *= al[e];
        ms[e] = mn[e];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float af = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al[g & 3]), 16 * (g >> 2)));
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] *= af;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float u = (ms[e] == __int_as_float(0xff800000)) ? 0.f : ms[e];
      sv[e] = fast_exp2(sv[e] - u);
      ls[e] += sv[e];
    }
    if (slot < NRG) *(float4 *)&s_p[w][c][4 * slot] = float4{sv[0], sv[1], sv[2], sv[3]};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float pg[4 * NRG];
#pragma unroll
      for (int x = 0; x < NRG; ++x) {
        const float4 v4 = *(const float4 *)&s_p[w][4 * u + slot][4 * x];
        pg[4 * x + 0] = v4.x;
        pg[4 * x + 1] = v4.y;
        pg[4 * x + 2] = v4.z;
        pg[4 * x + 3] = v4.w;
      }
      float vf[8];
      unpack<KT, 8>(vr[u], vf);
      if constexpr (F8) {
#pragma unroll
        for (int g = 0; g < 4 * NRG; ++g) pg[g] *= f8s.v[u];
      }
      if (U16 || more) load_v(base + STEP, u);
      // keep each refill after the use of the registers it replaces
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = __builtin_fmaf(pg[g], vf[e], acc[g][e]);
    }
  }

  // The four token slots share the wave's reference maxima: plain sums.
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[g][e] = pair32_sum(pair16_sum(acc[g][e]));
    }
#pragma unroll
  for (int e = 0; e < 4; ++e) ls[e] = group_sum<16>(ls[e]);
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[w][g][8 * c + e] = acc[g][e];
  }
  if (c == 0 && slot < NRG) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int g = 4 * slot + e;
      if (g < G) {
        s_m[w][g] = ms[e];
        s_l[w][g] = ls[e];
      }
    }
  }
  __syncthreads();
}

template <int KT, int G, bool PAGED, bool U16>
__global__ __launch_bounds__(SA_NT, G <= 4 ? 4 : 2) void sparse_attn_mfma_kernel(AttnKP p) {
  __shared__ int32_t s_tok0[SA_MAX_EPS];
  __shared__ int32_t s_phys[PAGED ? SA_MAX_EPS : 1];
  __shared__ MfmaLds<KT, G, SA_NW> L;
  const RowCtx rc = stage_row<G, PAGED>(p, s_tok0, s_phys);
  mfma_attend<KT, G, PAGED, U16, SA_NW>(p, rc, s_tok0, s_phys, L);
  finish_row<G, 128, SA_NW>(p, rc, blockIdx.y, blockIdx.x, L.acc, L.m, L.l);
}


// ---------------------------------------------- fused Quest decode ----
// One workgroup of eight waves per (b, KV head) with one query per sequence:
// the union page selection of the G heads (quest_select_union, as in
// la_quest_select), the ascending list staged in LDS (first token and pool
// row of every page) and written out for the caller, then the matrix-core
// attention of the G heads over it by the eight waves and the merge of their
// softmax states.  The selection's page keys and widened q are dead once the
// list is staged, so the attention state reuses their LDS.
constexpr int QD_NW = 8, QD_NT = 64 * QD_NW;

template <int MT, int G, int KPT>
struct QuestDecodeLds {
  union {
    struct {
      uint64_t keys[G * TK_NT * KPT];
      double qd[G * 256];
    } sel;
    MfmaLds<LA_BF16, G, QD_NW> att;
  } u;
  uint32_t bm[TK_NT * KPT / 32];
  int32_t tok0[TK_NT * KPT];
  int32_t phys[TK_NT * KPT];
  int32_t n_e;
};

template <int MT, int G, int KPT>
__global__ __launch_bounds__(QD_NT, 4) void quest_decode_fused_kernel(QsKP a, AttnKP p) {
  __shared__ QuestDecodeLds<MT, G, KPT> L;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row = blockIdx.x;  // (b, kvh)
  const int64_t kvh = row % a.Hkv, b = row / a.Hkv;
  int32_t n_v, own;
  quest_select_union<MT, G, KPT, QD_NT>(a, b, kvh, 0, L.u.sel.keys, L.u.sel.qd, L.bm, n_v, own);
  // the last key this query attends: its position, within the cache length
  const int64_t pos = a.positions ? (int64_t)a.positions[b] : a.pos_offset;
  const int64_t lim = min(kv_length(p.kv, b) - 1, pos);
  if (w == 0) {  // the union in ascending order: LDS, out_idx, out_count
    constexpr int WPL = (TK_NT * KPT / 32 + 63) / 64;  // bitmap words per lane
    const int64_t words = (n_v + 31) / 32;
    uint32_t bits[WPL];
    uint32_t cnt = 0;
#pragma unroll
    for (int j = 0; j < WPL; ++j) {
      const int64_t x = lane * WPL + j;
      bits[j] = x < words ? L.bm[x] : 0u;
      cnt += __popc(bits[j]);
    }
    uint32_t incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t v = (uint32_t)__shfl_up((int)incl, off, 64);
      if (lane >= off) incl += v;
    }
    const uint32_t total = (uint32_t)__shfl((int)incl, 63, 64);
    uint32_t at = incl - cnt;
    int32_t *gout = a.out_idx + row * a.width;
    const int64_t ps = a.page_size;
    const int32_t *ptab = p.kv.page_table + b * p.kv.pt_stride;
#pragma unroll
    for (int j = 0; j < WPL; ++j) {
      uint32_t bb = bits[j];
      while (bb) {
        const int bit = __ffs(bb) - 1;
        const int32_t page = (int32_t)((lane * WPL + j) * 32 + bit);
        if (at < (uint32_t)a.width) {
          gout[at] = page;
          const int64_t tok0 = (int64_t)page * ps;
          const bool ok = tok0 <= lim;
          L.tok0[at] = ok ? (int32_t)tok0 : -1;
          L.phys[at] = ok ? (int32_t)(((int64_t)ptab[page] * a.Hkv + kvh) * ps) : 0;
        }
        ++at;
        bb &= bb - 1;
      }
    }
    for (int64_t jj = (int64_t)total + lane; jj < a.width; jj += 64) gout[jj] = -1;
    if (lane == 0) {
      const int32_t ne = (int32_t)min((int64_t)total, a.width);
      L.n_e = ne;
      if (a.out_count) a.out_count[row] = ne;
    }
  }
  __syncthreads();
  RowCtx rc{};
  rc.b = b;
  rc.t = 0;
  rc.kvh = kvh;
  rc.h0 = kvh * G;
  rc.e0 = 0;
  rc.ne = L.n_e;
  rc.lim = lim;
  mfma_attend<LA_BF16, G, true, true, QD_NW>(p, rc, L.tok0, L.phys, L.u.att);
  finish_row<G, 128, QD_NW>(p, rc, row, 0, L.u.att.acc, L.u.att.m, L.u.att.l);
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

// bf16 or fp8 K/V with bf16 q and head dim 128 take the matrix-core kernel.
// LA_FP8_MFMA=0 keeps fp8 K/V on the VALU kernel (fp32 dequantised scores).
static bool mfma_path(int kt, int64_t d, int q_dt) {
  static const bool fp8_mfma = [] {
    const char *e = getenv("LA_FP8_MFMA");
    return !(e && e[0] == '0');
  }();
  if (d != 128 || q_dt != LA_BF16) return false;
  return kt == LA_BF16 || (kt == LA_FP8_E4M3 && fp8_mfma);
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
  // U16: paged, and every 16-row round lies inside one entry of one page
  const bool u16 = PAGED && p.staged && p.unit % 16 == 0;
  if (mfma_path(KT, D, p.q_dt) && u16)
    sparse_attn_mfma_kernel<KT == LA_F32 ? LA_BF16 : KT, G, PAGED, true><<<grid, SA_NT, 0, st>>>(p);
  else if (mfma_path(KT, D, p.q_dt))
    sparse_attn_mfma_kernel<KT == LA_F32 ? LA_BF16 : KT, G, PAGED, false><<<grid, SA_NT, 0, st>>>(p);
  else
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
    // workgroups to aim for: the matrix-core kernel keeps 4 resident per CU
    // (so one full wave of workgroups), the VALU kernel 8 per CU
    const bool mfma = mfma_path(kv->dtype, a->D, a->q_dtype);
    const int64_t target = (int64_t)num_cus() * (mfma ? 4 : 8);
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

namespace la {

// Launch of a planned attention with its split-K partials in `ws`.
static int sparse_attention_run(const la_sparse_attn_args *a, const la_kv *kv, const Plan &pl,
                                void *ws, hipStream_t st) {
  AttnKP p{};
  p.q = a->q;
  p.out = a->out;
  p.ids = a->ids;
  p.counts = a->counts;
  p.kv = *kv;
  if (kv->page_table && p.kv.s_st <= 0) p.kv.s_st = 1;  // paged scales: contiguous by default
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
    p.ws_ml = (float *)ws;
    p.ws_acc = p.ws_ml + pl.R * pl.G * pl.splits * 2;
  }
  switch (kv->dtype) {
    case LA_F32: return dispatch_d<LA_F32>(p, a->D, pl.G, st);
    case LA_BF16: return dispatch_d<LA_BF16>(p, a->D, pl.G, st);
    case LA_FP8_E4M3:
      if (pl.G > 4) return fail(LA_ERR_UNSUPPORTED, "fp8 sparse attention: group > 4");
      return dispatch_d<LA_FP8_E4M3>(p, a->D, pl.G, st);
    default: return fail(LA_ERR_INVALID, "KV dtype");
  }
}

// Static scratch of the allocation-free entry point: one array per device,
// held until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, once per device.
constexpr size_t LA_NOALLOC_SCRATCH = LA_NOALLOC_MAX_WORKSPACE;
__device__ __align__(256) unsigned char scratch[LA_NOALLOC_SCRATCH];

constexpr int LA_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[LA_MAX_DEVICES];

// Device address of this device's scratch (looked up on its first use, with
// that device current).
static int scratch_ptr(void **out) {
  int dev = 0;
  LA_HIP(hipGetDevice(&dev));
  LA_REQUIRE(dev >= 0 && dev < LA_MAX_DEVICES, "sparse attention (no-alloc): device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    LA_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    LA_REQUIRE(ptr != nullptr, "sparse attention (no-alloc): no scratch address");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return LA_OK;
}

}  // namespace la

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
  return sparse_attention_run(a, kv, pl, a->workspace, (hipStream_t)stream);
}

extern "C" int la_sparse_attention_noalloc(const la_sparse_attn_args *a, const la_kv *kv,
                                           void *stream) {
  Plan pl{};
  int rc = plan_attn(a, kv, pl);
  if (rc != LA_OK) return rc;
  if (pl.ws > LA_NOALLOC_SCRATCH)
    return fail(LA_ERR_WORKSPACE,
                "sparse attention (no-alloc): %zu bytes of split partials exceed the %zu-byte "
                "static scratch (fewer splits, or la_sparse_attention with a workspace)",
                pl.ws, LA_NOALLOC_SCRATCH);
  void *ws = nullptr;
  if (pl.ws > 0) {
    rc = scratch_ptr(&ws);
    if (rc != LA_OK) return rc;
  }
  return sparse_attention_run(a, kv, pl, ws, (hipStream_t)stream);
}

namespace la {
template <int MT, int G>
static int launch_quest_decode(const QsKP &qk, const AttnKP &p, int64_t rows, hipStream_t st) {
  quest_decode_fused_kernel<MT, G, 4><<<dim3((unsigned)rows), QD_NT, 0, st>>>(qk, p);
  LA_LAUNCHED();
  return LA_OK;
}
}  // namespace la

extern "C" int la_quest_decode_fused(const la_quest_decode_args *a, void *stream) {
  LA_REQUIRE(a, "la_quest_decode_fused: null arguments");
  const la_quest_select_args *s = &a->select;
  const la_kv *kv = &a->kv;
  LA_REQUIRE(s->q && s->page_min && s->page_max && s->out_idx && a->out && kv->k && kv->v &&
                 kv->page_table,
             "la_quest_decode_fused: null pointer");
  LA_REQUIRE(s->B > 0 && s->Hq > 0 && s->Hkv > 0 && s->n_pages > 0 && s->k > 0 && kv->T >= 1,
             "la_quest_decode_fused: bad shape");
  LA_REQUIRE(s->Hq % s->Hkv == 0, "n_heads must be a multiple of n_kv_heads");
  LA_REQUIRE(s->page_size > 0 && kv->page_size == s->page_size && kv->pt_stride >= 1,
             "la_quest_decode_fused: page sizes of the selection and the pool differ");
  LA_REQUIRE(a->out_dtype == LA_F32 || a->out_dtype == LA_BF16 || a->out_dtype == LA_F16,
             "la_quest_decode_fused: out dtype");
  LA_REQUIRE(s->meta_dtype == LA_F32 || s->meta_dtype == LA_BF16, "la_quest_decode_fused: meta dtype");
  const int64_t G = s->Hq / s->Hkv;
  const int64_t esz = s->meta_dtype == LA_BF16 ? 2 : 4;
  const bool layout = s->m_sp == 1 && s->m_sd % 4 == 0 && s->m_sd >= s->n_pages &&
                      s->m_sb % 4 == 0 && s->m_sh % 4 == 0 &&
                      (uintptr_t)s->page_min % (4 * esz) == 0 &&
                      (uintptr_t)s->page_max % (4 * esz) == 0;
  const bool shape = s->Tq == 1 && s->D == 128 && s->q_dtype == LA_BF16 && kv->dtype == LA_BF16 &&
                     (G == 2 || G == 4) && s->n_pages <= TK_NT * 4 &&
                     s->page_size % 16 == 0 && (uintptr_t)kv->k % 16 == 0 &&
                     (uintptr_t)kv->v % 16 == 0;
  if (!layout || !shape)
    return fail(LA_ERR_UNSUPPORTED, "la_quest_decode_fused: shape or layout not fused");
  LA_REQUIRE(s->n_pages * s->page_size < ((int64_t)1 << 31), "la_quest_decode_fused: cache span");
  QsKP qk{};
  qk.q = s->q;
  qk.mn = s->page_min;
  qk.mx = s->page_max;
  qk.out_idx = s->out_idx;
  qk.out_count = s->out_count;
  qk.Hq = s->Hq;
  qk.Hkv = s->Hkv;
  qk.Tq = 1;
  qk.D = s->D;
  qk.q_sb = s->q_sb;
  qk.q_sh = s->q_sh;
  qk.q_st = s->q_st;
  qk.n_pages = s->n_pages;
  qk.m_sb = s->m_sb;
  qk.m_sh = s->m_sh;
  qk.m_sd = s->m_sd;
  qk.page_size = s->page_size;
  qk.pos_offset = s->pos_offset;
  qk.positions = s->positions;
  qk.k = std::max<int64_t>(1, std::min(s->k, s->n_pages));
  qk.width = G * qk.k;
  qk.q_dt = s->q_dtype;
  AttnKP p{};
  p.q = s->q;
  p.out = a->out;
  p.ids = s->out_idx;
  p.counts = s->out_count;
  p.kv = *kv;
  p.B = s->B;
  p.Hq = s->Hq;
  p.Hkv = s->Hkv;
  p.Tq = 1;
  p.ids_heads = s->Hkv;
  p.ids_rows = 1;
  p.N = qk.width;
  p.unit = s->page_size;
  p.offset = s->pos_offset;
  p.splits = 1;
  p.eps = qk.width;
  p.q_sb = s->q_sb;
  p.q_sh = s->q_sh;
  p.q_st = s->q_st;
  p.o_sb = a->o_sb;
  p.o_sh = a->o_sh;
  p.o_st = a->o_st;
  p.qscale = a->scale * 1.4426950408889634f;
  p.q_dt = LA_BF16;
  p.out_dt = a->out_dtype;
  p.causal = 1;
  p.staged = 1;
  p.unit_shift = is_pow2(s->page_size) ? ilog2(s->page_size) : -1;
  const int64_t rows = s->B * s->Hkv;
  hipStream_t st = (hipStream_t)stream;
  const bool bf = s->meta_dtype == LA_BF16;
  if (G == 2)
    return bf ? launch_quest_decode<LA_BF16, 2>(qk, p, rows, st) : launch_quest_decode<LA_F32, 2>(qk, p, rows, st);
  return bf ? launch_quest_decode<LA_BF16, 4>(qk, p, rows, st) : launch_quest_decode<LA_F32, 4>(qk, p, rows, st);
}
