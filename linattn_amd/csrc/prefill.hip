// Block-sparse causal prefill on the gfx950 matrix cores.
//
// The executor of block_sparse_attention (kernels/triton/block_sparse.py:80-163)
// specialised for lists shared by a 64-query block: workgroup (b, h, qb) attends
// the listed 64-key blocks of KV head h / (Hq/Hkv), with the causal mask applied
// in-kernel on the diagonal block.  Head dim 128, bf16 inputs, fp32 accumulate,
// online softmax in the log2 domain.
//
// Per workgroup: 4 waves x 16 queries.  For every listed key block the K block
// (64 x 128) and V^T (128 x 64) are staged in LDS, double buffered, with the
// global loads of the two following blocks in flight (two register stages)
// while the current one is multiplied.
//   S^T = K Q^T   : v_mfma_f32_16x16x32_bf16, A = K rows from LDS, B = Q rows
//                   held in registers; lane (g = lane/16, c = lane%16) ends
//                   with S^T[key 16*kt + 4g + e][query c].
//   O^T += V^T P^T: P^T is used straight from those registers as the B
//                   operand -- the contraction index k = 8g + e is mapped to key
//                   32s + 4g + e (e < 4) or 32s + 16 + 4g + (e - 4), and the A
//                   operand (V^T rows) is read with the same key mapping, so no
//                   shuffle of P is needed.
// Workgroups are remapped so that the query heads of one KV head and adjacent
// query blocks run on the same XCD (shared L2 for their common key blocks).
#include "common.h"

namespace la {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_D = 128, PF_BS = 64, PF_NT = 256;
constexpr int PF_KP = 136;  // K row stride in LDS (bf16): 272 B, conflict-free b128 reads
constexpr int PF_VP = 72;   // V^T row stride in LDS (bf16): 144 B

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

__device__ __forceinline__ uint32_t pack2(uint32_t lo_src, uint32_t hi_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__global__ __launch_bounds__(PF_NT, 2) void prefill_kernel(PfKP p) {
  __shared__ __align__(16) uint16_t sK[2][PF_BS * PF_KP];
  __shared__ __align__(16) uint16_t sV[2][PF_D * PF_VP];

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

  const int64_t q_row = qb * PF_BS + w * 16 + c16;  // this lane's query
  const bool q_ok = q_row < p.T;
  bf16x8 qreg[4];
  {
    const uint16_t *qp = p.q + b * p.q_sb + h * p.q_sh + min(q_row, p.T - 1) * p.q_st;
#pragma unroll
    for (int s = 0; s < 4; ++s) qreg[s] = *(const bf16x8 *)(qp + 32 * s + 8 * g);
  }
  const int32_t *list = p.ids + ((b * p.Hq + h) * p.nqb + qb) * p.width;
  const int n = p.counts ? min((int)p.counts[(b * p.Hq + h) * p.nqb + qb], (int)p.width)
                         : (int)p.width;

  const uint16_t *kbh = p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t *vbh = p.v + b * p.v_sb + kvh * p.v_sh;
  // global -> register staging of one key block
  const int kq = tid & 15;  // V: keys 4kq..4kq+3
  const int dc = tid >> 4;  // V: dims 8dc..8dc+7
  // register staging of one key block (global -> registers -> LDS)
  struct Stage {
    uint4 k[4], v[4];
  };
  auto gload = [&](int kb, Stage &r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + i * PF_NT;  // K chunk: key ch/16, 8 dims at (ch%16)*8
      const int64_t key = (int64_t)kb * PF_BS + (ch >> 4);
      const bool kok = kb >= 0 && key < p.T;  // -1 list entries read nothing
      r.k[i] = kok ? *(const uint4 *)(kbh + key * p.k_st + (ch & 15) * 8) : uint4{0, 0, 0, 0};
      const int64_t vkey = (int64_t)kb * PF_BS + kq * 4 + i;
      const bool vok = kb >= 0 && vkey < p.T;
      r.v[i] = vok ? *(const uint4 *)(vbh + vkey * p.v_st + dc * 8) : uint4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf, const Stage &r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + i * PF_NT;
      *(uint4 *)&sK[buf][(ch >> 4) * PF_KP + (ch & 15) * 8] = r.k[i];
    }
    // V^T: row d holds keys; 4 keys x 8 dims -> 8 rows of 4 keys (8 bytes)
    const uint32_t a[4][4] = {{r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w},
                              {r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w},
                              {r.v[2].x, r.v[2].y, r.v[2].z, r.v[2].w},
                              {r.v[3].x, r.v[3].y, r.v[3].z, r.v[3].w}};
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // dims 8dc + 2j, 8dc + 2j + 1
      const uint2 lo = {pack2(a[0][j], a[1][j], 0x05040100u), pack2(a[2][j], a[3][j], 0x05040100u)};
      const uint2 hi = {pack2(a[0][j], a[1][j], 0x07060302u), pack2(a[2][j], a[3][j], 0x07060302u)};
      *(uint2 *)&sV[buf][(dc * 8 + 2 * j) * PF_VP + kq * 4] = lo;
      *(uint2 *)&sV[buf][(dc * 8 + 2 * j + 1) * PF_VP + kq * 4] = hi;
    }
  };

  // m: running max of the raw (unscaled) scores of this lane's query
  float m = __int_as_float(0xff800000), l = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

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
    // S^T = K Q^T
    f32x4 st[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 a = *(const bf16x8 *)&sK[buf][(16 * kt + c16) * PF_KP + 32 * s + 8 * g];
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[s], sacc, 0, 0, 0);
      }
      st[kt] = sacc;
    }
    // mask, online softmax (column c16 = this lane's query); the positive
    // scale commutes with the max, so it is applied inside the exponent
    const int64_t key0 = (int64_t)kb * PF_BS;
    const bool need_mask =
        kb < 0 || (p.causal && key0 + PF_BS - 1 > qb * PF_BS + w * 16) || key0 + PF_BS > p.T;
    if (need_mask) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t key = key0 + 16 * kt + 4 * g + e;
          if (kb < 0 || (p.causal && key > q_row) || key >= p.T) st[kt][e] = __int_as_float(0xff800000);
        }
    }
    float mx = __int_as_float(0xff800000);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
      mx = fmaxf(mx, fmaxf(fmaxf(st[kt][0], st[kt][1]), fmaxf(st[kt][2], st[kt][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    // rescale only when some lane's maximum grew (rare after the first blocks)
    if (__ballot(mn > m) != 0) {
      const float alpha = mn > m ? fast_exp2((m - mn) * p.qscale) : 1.f;
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
      m = mn;
    }
    const float mu = (m == __int_as_float(0xff800000)) ? 0.f : m * p.qscale;
    // P = P_hi + P_lo in bf16 (P_lo = bf16(P - P_hi)): the product keeps ~16
    // mantissa bits of each weight, so bf16 rounding of P costs ~2^-17
    // relative instead of 2^-9 (which alone exceeds 2e-3 on rows whose mass
    // sits on a few keys).
    bf16x8 ph[2], pl[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = fast_exp2(__builtin_fmaf(st[2 * s2][e], p.qscale, -mu));
        pv[4 + e] = fast_exp2(__builtin_fmaf(st[2 * s2 + 1][e], p.qscale, -mu));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) l += pv[e];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const bf16x2 h2 = __builtin_convertvector((f32x2{pv[e], pv[e + 1]}), bf16x2);
        const f32x2 hf = __builtin_convertvector(h2, f32x2);
        const bf16x2 l2 = __builtin_convertvector((f32x2{pv[e] - hf[0], pv[e + 1] - hf[1]}), bf16x2);
        ph[s2][e] = h2[0];
        ph[s2][e + 1] = h2[1];
        pl[s2][e] = l2[0];
        pl[s2][e + 1] = l2[1];
      }
    }
    // O^T += V^T P^T
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const uint16_t *vrow = &sV[buf][(16 * dt + c16) * PF_VP + 32 * s2 + 4 * g];
        const uint2 lo = *(const uint2 *)vrow;
        const uint2 hi = *(const uint2 *)(vrow + 16);
        const uint4 av = {lo.x, lo.y, hi.x, hi.y};
        const bf16x8 a = *(const bf16x8 *)&av;
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ph[s2], acc[dt], 0, 0, 0);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pl[s2], acc[dt], 0, 0, 0);
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
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (!q_ok) return;
  const int64_t ob = b * p.o_sb + h * p.o_sh + q_row * p.o_st;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const int64_t o = ob + 16 * dt + 4 * g;
    const f32x4 r = acc[dt] * inv;
    if (p.out_dt == LA_BF16) {
      const bf16x2 a = __builtin_convertvector((f32x2{r[0], r[1]}), bf16x2);
      const bf16x2 c = __builtin_convertvector((f32x2{r[2], r[3]}), bf16x2);
      uint2 u;
      u.x = *(const uint32_t *)&a;
      u.y = *(const uint32_t *)&c;
      *(uint2 *)((uint16_t *)p.out + o) = u;
    } else {
      *(f32x4 *)((float *)p.out + o) = r;
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
