// Block-sparse causal prefill on the gfx950 matrix cores.
//
// The executor of block_sparse_attention (kernels/triton/block_sparse.py:80-163)
// specialised for lists shared by a 64-query block: workgroup (b, h, qb) attends
// the listed 64-key blocks of KV head h / (Hq/Hkv), with the causal mask applied
// in-kernel on the diagonal block.  Head dim 128, bf16 inputs, fp32 accumulate,
// online softmax in the log2 domain.
//
// Per workgroup: 4 waves = 2 query halves (32 queries) x 2 key halves (32 of
// every 64-key block).  For every listed key block the K and V blocks (64 x
// 128, row-major) are staged in LDS, double buffered, with the global loads of
// the two following blocks in flight (two register stages) while the current
// one is multiplied.  Each wave reads only its half of K and V and uses each
// A operand for both of its 16-query groups, so a block costs 64 KiB of LDS
// reads instead of 128 KiB; the two key halves keep separate online-softmax
// states that are merged through LDS at the end.
//   S^T = K Q^T   : v_mfma_f32_16x16x32_bf16, A = K rows from LDS, B = Q rows
//                   held in registers; lane (g = lane/16, c = lane%16) ends
//                   with S^T[key 16*kt + 4g + e][query c].
//   O^T += V^T P^T: P^T is used straight from those registers as the B
//                   operand -- the contraction index k = 8g + e is mapped to key
//                   4g + e (e < 4) or 16 + 4g + (e - 4) of the wave's half,
//                   and the A operand (V^T rows) is read with the same key
//                   mapping by LDS transpose reads of the row-major V block,
//                   so neither P nor V is shuffled.
// Workgroups are remapped so that the query heads of one KV head and adjacent
// query blocks run on the same XCD (shared L2 for their common key blocks).
#include "common.h"

namespace la {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

constexpr int PF_D = 128, PF_BS = 64, PF_NT = 256;
constexpr int PF_KP = 136;  // K row stride in LDS (bf16): 272 B, conflict-free b128 reads
constexpr int PF_VP = 136;  // V row stride in LDS (bf16): 272 B

struct PfKP {
  const uint16_t *q, *k, *v;
  void *out;
  const int32_t *ids, *counts;
  int64_t B, Hq, Hkv, T;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  int64_t width, nqb;
  float qscale;  // scale * log2(e)
  int32_t causal, out_dt;
};

__global__ __launch_bounds__(PF_NT, 2) void prefill_kernel(PfKP p) {
  __shared__ __align__(16) uint16_t sK[2][PF_BS * PF_KP];
  __shared__ __align__(16) uint16_t sV[2][PF_BS * PF_VP];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  // XCD-aware order: consecutive logical ids share an XCD; logical order is
  // (b, kvh, qb, head within the group).
  const int64_t nwg = gridDim.x;
  const int64_t wg = blockIdx.x;
  const int64_t per_xcd = nwg / 8;
  const int64_t lid = (wg < per_xcd * 8) ? (wg % 8) * per_xcd + wg / 8 : wg;
  const int64_t G = p.Hq / p.Hkv;
  const int64_t hg = lid % G;
  const int64_t qb = (lid / G) % p.nqb;
  const int64_t kvh = (lid / (G * p.nqb)) % p.Hkv;
  const int64_t b = lid / (G * p.nqb * p.Hkv);
  const int64_t h = kvh * G + hg;

  const int qh = w >> 1, kh = w & 1;  // query half, key half
  int64_t q_row[2];                    // this lane's query in each 16-query group
  bf16x8 qreg[2][4];
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    q_row[qg] = qb * PF_BS + 32 * qh + 16 * qg + c16;
    const uint16_t *qp = p.q + b * p.q_sb + h * p.q_sh + min(q_row[qg], p.T - 1) * p.q_st;
#pragma unroll
    for (int s = 0; s < 4; ++s) qreg[qg][s] = *(const bf16x8 *)(qp + 32 * s + 8 * g);
  }
  const int32_t *list = p.ids + ((b * p.Hq + h) * p.nqb + qb) * p.width;
  const int n = p.counts ? min((int)p.counts[(b * p.Hq + h) * p.nqb + qb], (int)p.width)
                         : (int)p.width;

  const uint16_t *kbh = p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t *vbh = p.v + b * p.v_sb + kvh * p.v_sh;
  // global -> register staging of one key block
  // register staging of one key block (global -> registers -> LDS)
  struct Stage {
    uint4 k[4], v[4];
  };
  // thread chunk i: key (tid/16) + 16 i of the block, 8 dims at (tid%16)*8;
  // element offsets within a block are loop invariant
  const int64_t koff = (int64_t)(tid >> 4) * p.k_st + (tid & 15) * 8, kstep = 16 * p.k_st;
  const int64_t voff = (int64_t)(tid >> 4) * p.v_st + (tid & 15) * 8, vstep = 16 * p.v_st;
  auto gload = [&](int kb, Stage &r) {
    if (kb >= 0 && (int64_t)kb * PF_BS + PF_BS <= p.T) {  // a whole block: plain loads
      const uint16_t *kp = kbh + (int64_t)kb * PF_BS * p.k_st + koff;
      const uint16_t *vp = vbh + (int64_t)kb * PF_BS * p.v_st + voff;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r.k[i] = *(const uint4 *)(kp + i * kstep);
        r.v[i] = *(const uint4 *)(vp + i * vstep);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t key = (int64_t)kb * PF_BS + (tid >> 4) + 16 * i;
      const bool kok = kb >= 0 && key < p.T;  // -1 list entries read nothing
      r.k[i] = kok ? *(const uint4 *)(kbh + key * p.k_st + (tid & 15) * 8) : uint4{0, 0, 0, 0};
      r.v[i] = kok ? *(const uint4 *)(vbh + key * p.v_st + (tid & 15) * 8) : uint4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf, const Stage &r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + i * PF_NT;
      *(uint4 *)&sK[buf][(ch >> 4) * PF_KP + (ch & 15) * 8] = r.k[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + i * PF_NT;
      *(uint4 *)&sV[buf][(ch >> 4) * PF_VP + (ch & 15) * 8] = r.v[i];
    }
  };

  // m: reference maximum of the raw (unscaled) scores of this lane's query, per group
  float m[2] = {__int_as_float(0xff800000), __int_as_float(0xff800000)}, l[2] = {0.f, 0.f};
  f32x4 acc[2][8];
#pragma unroll
  for (int qg = 0; qg < 2; ++qg)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[qg][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Two register stages: while block j is multiplied out of LDS, block j+1
  // waits in registers for its LDS slot and block j+2 is being loaded.
  Stage R0, R1;
  if (n > 0) {
    gload(list[0], R0);
    lstore(0, R0);
    if (n > 1) gload(list[1], R1);
  }
  __syncthreads();
  auto step = [&](int j, Stage &load_into, const Stage &store_from) {
    const int buf = j & 1;
    const int kb = list[j];
    if (j + 2 < n) gload(list[j + 2], load_into);  // in flight for two blocks
    // S^T = K Q^T over this wave's 32 keys, both query groups
    f32x4 st[2][2];
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) {
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 a = *(const bf16x8 *)&sK[buf][(32 * kh + 16 * kt2 + c16) * PF_KP + 32 * s + 8 * g];
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[0][s], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[1][s], s1, 0, 0, 0);
      }
      st[0][kt2] = s0;
      st[1][kt2] = s1;
    }
    // mask, online softmax (column c16 = this lane's query); the positive
    // scale commutes with the max, so it is applied inside the exponent
    const int64_t key0 = (int64_t)kb * PF_BS + 32 * kh;  // first key of this half
    const bool need_mask = kb < 0 || (p.causal && key0 + 31 > qb * PF_BS + 32 * qh) ||
                           key0 + 32 > p.T;
    bf16x8 ph[2], pl[2];
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      if (need_mask) {
#pragma unroll
        for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t key = key0 + 16 * kt2 + 4 * g + e;
            if (kb < 0 || (p.causal && key > q_row[qg]) || key >= p.T)
              st[qg][kt2][e] = __int_as_float(0xff800000);
          }
      }
      float mx = fmaxf(fmaxf(fmaxf(st[qg][0][0], st[qg][0][1]), fmaxf(st[qg][0][2], st[qg][0][3])),
                       fmaxf(fmaxf(st[qg][1][0], st[qg][1][1]), fmaxf(st[qg][1][2], st[qg][1][3])));
      mx = pair32_max(pair16_max(mx));
      // m is a reference maximum: it is raised (and acc, l rescaled) only when
      // a row's maximum exceeds it by more than 2^8 in the exponent, so the
      // weights stay below 256 and the rescale is rare; the final division
      // by l is unchanged by the choice of reference.
      const float mn = fmaxf(m[qg], mx);
      if (__ballot((mn - m[qg]) * p.qscale > 8.f) != 0) {
        const float alpha = mn > m[qg] ? fast_exp2((m[qg] - mn) * p.qscale) : 1.f;
        l[qg] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[qg][dt] *= alpha;
        m[qg] = mn;
      }
      const float mu = (m[qg] == __int_as_float(0xff800000)) ? 0.f : m[qg] * p.qscale;
      // P = P_hi + P_lo in bf16 (P_lo = bf16(P - P_hi)): the product keeps ~16
      // mantissa bits of each weight, so bf16 rounding of P costs ~2^-17
      // relative instead of 2^-9 (which alone exceeds 2e-3 on rows whose mass
      // sits on a few keys).
      float pv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = fast_exp2(__builtin_fmaf(st[qg][0][e], p.qscale, -mu));
        pv[4 + e] = fast_exp2(__builtin_fmaf(st[qg][1][e], p.qscale, -mu));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) l[qg] += pv[e];
      // packed words: hw = bf16x2(P) (round to nearest), its exact fp32
      // value from the halves, lw = bf16x2(P - hi)
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{pv[2 * e], pv[2 * e + 1]}), bf16x2));
        const float h0 = __uint_as_float(hw[e] << 16), h1 = __uint_as_float(hw[e] & 0xffff0000u);
        lw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{pv[2 * e] - h0, pv[2 * e + 1] - h1}), bf16x2));
      }
      ph[qg] = __builtin_bit_cast(bf16x8, uint4{hw[0], hw[1], hw[2], hw[3]});
      pl[qg] = __builtin_bit_cast(bf16x8, uint4{lw[0], lw[1], lw[2], lw[3]});
    }
    // O^T += V^T P^T over this wave's keys; each V^T operand serves both groups
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      // V^T rows through the LDS transpose read: lane (g, j) of a 16-lane group
      // gets V[k0 + e][16 dt + j], e < 4, when lane i of the group points at
      // row k0 + i/4, columns 16 dt + 4 (i%4) .. +3
      const uint16_t *v0 = &sV[buf][(32 * kh + 4 * g + (c16 >> 2)) * PF_VP + 16 * dt + 4 * (c16 & 3)];
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)v0);
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(v0 + 16 * PF_VP));
      const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int qg = 0; qg < 2; ++qg) {
        acc[qg][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ph[qg], acc[qg][dt], 0, 0, 0);
        acc[qg][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pl[qg], acc[qg][dt], 0, 0, 0);
      }
    }
    if (j + 1 < n) lstore(buf ^ 1, store_from);
    __syncthreads();
  };
  for (int j = 0; j < n; j += 2) {
    step(j, R0, R1);
    if (j + 1 >= n) break;
    step(j + 1, R1, R0);
  }
  // l is a per-lane partial over this lane's keys; sum the 4 lane groups.
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    l[qg] = pair32_sum(pair16_sum(l[qg]));
  }
  // Merge the two key halves: the kh = 1 wave of each query half hands its
  // state to the kh = 0 wave through LDS (the K buffers are free now).
  float *red = (float *)&sK[0][0] + qh * (2 * 128 * 16 + 64);
  float *red_o = red;                   // [qg][d][query]
  float *red_ml = red + 2 * 128 * 16;   // [qg][m, l][query]
  if (kh == 1) {
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) red_o[(qg * 128 + 16 * dt + 4 * g + e) * 16 + c16] = acc[qg][dt][e];
      if (g == 0) {
        red_ml[(qg * 2 + 0) * 16 + c16] = m[qg];
        red_ml[(qg * 2 + 1) * 16 + c16] = l[qg];
      }
    }
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    const float m2 = red_ml[(qg * 2 + 0) * 16 + c16], l2 = red_ml[(qg * 2 + 1) * 16 + c16];
    const float M = fmaxf(m[qg], m2);
    const float a1 = (m[qg] == __int_as_float(0xff800000)) ? 0.f : fast_exp2((m[qg] - M) * p.qscale);
    const float a2 = (m2 == __int_as_float(0xff800000)) ? 0.f : fast_exp2((m2 - M) * p.qscale);
    const float L = l[qg] * a1 + l2 * a2;
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (q_row[qg] >= p.T) continue;
    const int64_t ob = b * p.o_sb + h * p.o_sh + q_row[qg] * p.o_st;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        r[e] = (acc[qg][dt][e] * a1 + red_o[(qg * 128 + 16 * dt + 4 * g + e) * 16 + c16] * a2) * inv;
      const int64_t o = ob + 16 * dt + 4 * g;
      if (p.out_dt == LA_BF16) {
        const bf16x2 x = __builtin_convertvector((f32x2{r[0], r[1]}), bf16x2);
        const bf16x2 y = __builtin_convertvector((f32x2{r[2], r[3]}), bf16x2);
        uint2 u;
        u.x = *(const uint32_t *)&x;
        u.y = *(const uint32_t *)&y;
        *(uint2 *)((uint16_t *)p.out + o) = u;
      } else {
        *(f32x4 *)((float *)p.out + o) = r;
      }
    }
  }
}

}  // namespace la

using namespace la;

extern "C" int la_block_sparse_prefill(const la_prefill_args *a, void *stream) {
  LA_REQUIRE(a && a->q && a->k && a->v && a->out && a->ids, "la_block_sparse_prefill: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hq > 0 && a->Hkv > 0 && a->T > 0, "la_block_sparse_prefill: bad shape");
  LA_REQUIRE(a->Hq % a->Hkv == 0, "n_heads must be a multiple of n_kv_heads");
  if (a->D != PF_D || a->block != PF_BS)
    return fail(LA_ERR_UNSUPPORTED, "la_block_sparse_prefill: head_dim 128 and 64-token blocks only");
  LA_REQUIRE(a->out_dtype == LA_F32 || a->out_dtype == LA_BF16, "la_block_sparse_prefill: out dtype");
  LA_REQUIRE(a->width >= 1, "la_block_sparse_prefill: list width");
  // 16-byte vector access of q/k/v rows and of the output
  const bool al = ((uintptr_t)a->q % 16 == 0) && ((uintptr_t)a->k % 16 == 0) &&
                  ((uintptr_t)a->v % 16 == 0) && ((uintptr_t)a->out % 16 == 0) &&
                  a->q_sb % 8 == 0 && a->q_sh % 8 == 0 && a->q_st % 8 == 0 && a->k_sb % 8 == 0 &&
                  a->k_sh % 8 == 0 && a->k_st % 8 == 0 && a->v_sb % 8 == 0 && a->v_sh % 8 == 0 &&
                  a->v_st % 8 == 0 && a->o_sb % 4 == 0 && a->o_sh % 4 == 0 && a->o_st % 4 == 0;
  LA_REQUIRE(al, "la_block_sparse_prefill: rows must be contiguous and 16-byte aligned");
  PfKP p{};
  p.q = (const uint16_t *)a->q;
  p.k = (const uint16_t *)a->k;
  p.v = (const uint16_t *)a->v;
  p.out = a->out;
  p.ids = a->ids;
  p.counts = a->counts;
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.T = a->T;
  p.q_sb = a->q_sb; p.q_sh = a->q_sh; p.q_st = a->q_st;
  p.k_sb = a->k_sb; p.k_sh = a->k_sh; p.k_st = a->k_st;
  p.v_sb = a->v_sb; p.v_sh = a->v_sh; p.v_st = a->v_st;
  p.o_sb = a->o_sb; p.o_sh = a->o_sh; p.o_st = a->o_st;
  p.width = a->width;
  p.nqb = ceil_div(a->T, PF_BS);
  p.qscale = a->scale * 1.4426950408889634f;
  p.causal = a->causal;
  p.out_dt = a->out_dtype;
  const int64_t nwg = a->B * a->Hq * p.nqb;
  LA_REQUIRE(nwg < ((int64_t)1 << 31), "la_block_sparse_prefill: too many query blocks");
  prefill_kernel<<<dim3((unsigned)nwg), PF_NT, 0, (hipStream_t)stream>>>(p);
  LA_LAUNCHED();
  return LA_OK;
}
