// Block-sparse causal prefill on the gfx950 matrix cores.
//
// The executor of block_sparse_attention (kernels/triton/block_sparse.py:80-163)
// specialised for lists shared by a 64-query block: workgroup (b, h, qb) attends
// the listed 64-key blocks of KV head h / (Hq/Hkv), with the causal mask applied
// in-kernel on the diagonal block.  Head dim 128, bf16 inputs, fp32 accumulate,
// online softmax in the log2 domain.
//
// Precision of the PV product: the weights P go to the matrix core as fp16
// (11 significant bits; bf16's 8 alone err by up to 2^-9 of the largest weight,
// which exceeds 2e-3 on rows whose mass sits on a few keys), and the row sum is
// taken from the same rounded weights, so a rounding shared by every weight
// cancels in the division.  V is therefore converted once to fp16 by
// prefill_v16_kernel, each 64-token block scaled by a power of two 2^-e:
// e = 0 while the block's largest |v| lies in [1, 2^15); above, e > 0 (at most
// 7, so |v| < 2^22) brings it below 2^15; below 1, e < 0 (at least -8) scales
// small blocks up to [1, 2), so their values stay normal fp16 down to 2^-22.
// Every bf16 value of magnitude >= 2^(e-17) is then exact.  The kernel folds
// 2^e into the weights of that block (exp2(x + e): at most 2^(8+e) <= 2^15,
// still an fp16; e < 0 only where the block's values are small, since it
// moves weights of the block towards the fp16 subnormals) and weighs them by
// 2^-e in the row sum.  Blocks with |v| >= 2^22 raise LA_DEV_PREFILL_RANGE in
// the device status word (their fp16 copy overflows to inf), which
// block_sparse_prefill turns into an error.
//
// Per workgroup: 4 waves = 2 query halves (32 queries) x 2 key halves (32 of
// every 64-key block).  Each listed key block's K and V (64 x 128, bf16) are
// copied global -> LDS by the gfx950 LDS-DMA loads (global_load_lds_dwordx4),
// double buffered: block j+1 streams into the other buffer while block j is
// multiplied.  No registers stage the copy, and its waits are explicit (the
// loads are invisible to the compiler's wait counting, which would otherwise
// wait for the newest prefetch wherever two paths issue different loads).
// LDS rows are 256 B, unpadded; row r keeps its 16-byte chunk c at position
// c ^ swz(r), which spreads both the K row reads and the V transpose reads
// over all banks.  Each wave reads only its half of K and V and uses each A
// operand for both of its 16-query groups; the two key halves keep separate
// online-softmax states that are merged through LDS at the end.
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
#include <algorithm>
#include <climits>
#include <type_traits>

#include "common.h"

namespace la {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

constexpr int PF_D = 128, PF_BS = 64, PF_NT = 256;
constexpr int PF_BLK = PF_BS * PF_D;  // elements of one staged K or V block (16 KiB)

// Chunk swizzle of staged row r (16-byte chunks, 16 per row): a permutation
// of 0..15 over any 16 consecutive rows (K reads: 16 lanes, 16 rows, one
// chunk), and rows r and r ^ 1 never share a chunk pair {2i, 2i+1} (V
// transpose reads: 8 rows x 2 chunks per 32 lanes).
__device__ __forceinline__ int pf_swz(int r) { return (2 * (r & 7)) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int pf_swz_k(int r) { return 2 * (r & 7); }

// IEEE maximum (NaN-propagating): gfx950 v_maximum3_f32 without the
// canonicalising moves fmaxf needs in IEEE mode.
__device__ __forceinline__ float pf_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float pf_pair16_max(float x) { const float2 p = pair16(x); return pf_max(p.x, p.y); }
__device__ __forceinline__ float pf_pair32_max(float x) { const float2 p = pair32(x); return pf_max(p.x, p.y); }

// x / d and x % d for a wave-uniform x < 2^31 (shift when d = 2^sh)
__device__ __forceinline__ uint32_t pf_div(uint32_t x, uint32_t d, int sh) { return sh >= 0 ? x >> sh : x / d; }

// Three wave-uniform 32-bit reads through the scalar cache, waited for together.
__device__ __forceinline__ void sload3_i32(const int32_t *p0, const int32_t *p1, const int32_t *p2,
                                           int32_t &a, int32_t &b, int32_t &c) {
  asm volatile(
      "s_load_dword %0, %3, 0x0\n\ts_load_dword %1, %4, 0x0\n\ts_load_dword %2, %5, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(a), "=&s"(b), "=&s"(c) : "s"(p0), "s"(p1), "s"(p2) : "memory");
}

// Two wave-uniform 32-bit reads through the scalar cache, waited for together.
__device__ __forceinline__ void sload2_i32(const int32_t *p0, const int32_t *p1, int32_t &a, int32_t &b) {
  asm volatile("s_load_dword %0, %2, 0x0\n\ts_load_dword %1, %3, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(a), "=&s"(b) : "s"(p0), "s"(p1) : "memory");
}

struct PfKP {
  const uint16_t *q, *k, *v;  // v: the fp16 copy (B, Hkv, T, 128), contiguous
  const int32_t *vexp;        // (B, Hkv, nkb): V block kb holds v * 2^-vexp
  void *out;
  const int32_t *ids, *counts;
  int64_t B, Hq, Hkv, T;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  int64_t width, nqb, nkb;
  uint32_t k_blk, v_blk;  // elements between consecutive 64-token blocks of K / V
  int32_t sh_g, sh_nqb, sh_hkv;  // log2 of G, nqb, Hkv when powers of two, else -1
  float qscale;   // scale * log2(e)
  float thr_gap;  // 8 / qscale: raw-score headroom above the reference maximum
  int32_t causal, out_dt;
  const int32_t *lens;  // ragged batch: rows of sequence b (clamped to [0, T]); null: T
  const float *ks;      // fp8 K: per-token scales (B, Hkv, T) at strides s_sb, s_sh, s_st
  int64_t s_sb, s_sh, s_st;
};

// Status bits this file's kernels raise on the current device (read through
// la_device_status).
__device__ uint32_t la_pf_status;

// V (bf16 at any strides with a unit stride over D, or fp8 e4m3 codes with
// per-token fp32 scales) -> fp16, one workgroup per 64-token block of one
// (b, KV head): for the block's largest |v| with biased exponent E,
// e = min(7, E - 141) when E > 141 (so |v| * 2^-e < 2^15 when E <= 148),
// e = max(-8, E - 127) when E < 127 (|v| < 1), and 0 otherwise; then
// v16 = fp16(v * 2^-e), rounded to nearest even (fp8: v = code * scale in
// fp32, the product rounded once).  Rows past T (T_b) are not written.
template <bool F8>
__global__ __launch_bounds__(256) void prefill_v16_kernel(const void *v, const float *vs,
                                                          int64_t s_sb, int64_t s_sh, int64_t s_st,
                                                          int64_t v_sb, int64_t v_sh, int64_t v_st,
                                                          int64_t Hkv, int64_t T, int64_t nkb,
                                                          uint16_t *v16, int32_t *vexp,
                                                          const int32_t *lens) {
  __shared__ uint32_t wmax[4];
  const int64_t blk = blockIdx.x;
  const int64_t kb = blk % nkb, bh = blk / nkb;
  const int64_t b = bh / Hkv, kvh = bh % Hkv;
  const int tid = threadIdx.x;
  const int64_t Tfull = T;
  if (lens) T = min(max((int64_t)lens[b], (int64_t)0), T);  // ragged: rows past T_b are padding
  if (kb * PF_BS >= T) {  // a block of padding only: never listed
    if (tid == 0) vexp[blk] = 0;
    return;
  }
  uint16_t *dst = v16 + bh * Tfull * PF_D;
  float x[4][8];
  uint32_t mx = 0;  // largest |v| as fp32 bits (NaN above inf: e then saturates)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = kb * PF_BS + (tid >> 4) + 16 * i;
    const int col = 8 * (tid & 15);
    if (row < T) {
      if constexpr (F8) {
        const uint8_t *src = (const uint8_t *)v + b * v_sb + kvh * v_sh + row * v_st + col;
        const uint2 c = *(const uint2 *)src;
        const float sc = vs[b * s_sb + kvh * s_sh + row * s_st];
        const float2 a0 = fp8x2_to_f32<false>(c.x), a1 = fp8x2_to_f32<true>(c.x);
        const float2 a2 = fp8x2_to_f32<false>(c.y), a3 = fp8x2_to_f32<true>(c.y);
        x[i][0] = a0.x * sc; x[i][1] = a0.y * sc; x[i][2] = a1.x * sc; x[i][3] = a1.y * sc;
        x[i][4] = a2.x * sc; x[i][5] = a2.y * sc; x[i][6] = a3.x * sc; x[i][7] = a3.y * sc;
      } else {
        const uint16_t *src = (const uint16_t *)v + b * v_sb + kvh * v_sh + row * v_st + col;
        const u32x4 w = __builtin_nontemporal_load((const u32x4 *)src);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[i][2 * e] = bf16lo(w[e]);
          x[i][2 * e + 1] = bf16hi(w[e]);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = max(mx, __float_as_uint(x[i][e]) & 0x7fffffffu);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o, 64));
  if ((tid & 63) == 0) wmax[tid >> 6] = mx;
  __syncthreads();
  mx = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
  const int E = (int)(mx >> 23);
  const int e = E > 141 ? min(7, E - 141) : E < 127 ? max(-8, E - 127) : 0;
  if (tid == 0) {
    vexp[blk] = e;
    if (E > 148 && mx < 0x7f800000u)  // finite |v| >= 2^22 (inf and NaN pass through)
      __hip_atomic_fetch_or(&la_pf_status, (uint32_t)LA_DEV_PREFILL_RANGE, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = kb * PF_BS + (tid >> 4) + 16 * i;
    if (row >= T) continue;
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = __builtin_amdgcn_ldexpf(x[i][2 * j], -e);
      const float hi = __builtin_amdgcn_ldexpf(x[i][2 * j + 1], -e);
      o[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
    }
    *(uint4 *)(dst + row * PF_D + 8 * (tid & 15)) = uint4{o[0], o[1], o[2], o[3]};
  }
}

// KF8 (fp8 K/V): K is staged as its e4m3 codes (64 rows of 128 bytes, half
// the bytes of a bf16 block) and scored on the fp8 matrix cores
// (v_mfma_scale_f32_16x16x128_f8f6f4, unit block scales): q is split per
// query row into a two-term fp8 expansion q = sq (hi + lo), sq a power of two,
// hi = e4m3(q / sq), lo = e4m3(q / sq - hi), so a
// score is two fp8 products into one accumulator, then multiplied by its
// key's scale.  With sq a power of two (below) the two terms hold the bf16 q
// exactly, so the products are those of the dequantised keys and q.  Scores
// are kept in "lane units" (the true score / sq of the lane's query);
// qs = qscale * sq turns lane units into the exponent.  Without KF8,
// qs = qscale.  V (codes times scale) goes through the fp16 copy as for bf16.
template <bool KF8>
__global__ __launch_bounds__(PF_NT, 2) void prefill_kernel(PfKP p) {
  // K slots 0..1 (16 KiB each, KF8: 8 KiB), V slots 0..1 after them (16 KiB
  // each): 64 / 48 KiB, two workgroups per CU; after the loop, the key-half
  // merge area
  constexpr int KSL = KF8 ? PF_BLK / 2 : PF_BLK;  // uint16 elements of a K slot
  __shared__ __align__(16) uint16_t smem[2 * KSL + 2 * PF_BLK];
  // KF8: the per-key scales of the K block in each K slot (copied with it)
  __shared__ __align__(16) float sscale[KF8 ? 2 * PF_BS : 4];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  // XCD-aware order: consecutive logical ids share an XCD; logical order is
  // (b, kvh, qb, head within the group).
  const int64_t nwg = gridDim.x;
  const int64_t wg = blockIdx.x;
  const int64_t per_xcd = nwg / 8;
  const uint32_t lid = (uint32_t)((wg < per_xcd * 8) ? (wg % 8) * per_xcd + wg / 8 : wg);
  const uint32_t G = (uint32_t)(p.Hq / p.Hkv), nqbu = (uint32_t)p.nqb, hkvu = (uint32_t)p.Hkv;
  const uint32_t l1 = pf_div(lid, G, p.sh_g), l2 = pf_div(l1, nqbu, p.sh_nqb);
  const uint32_t l3 = pf_div(l2, hkvu, p.sh_hkv);
  const int64_t hg = lid - l1 * G;
  const int64_t qb = l1 - l2 * nqbu;
  const int64_t kvh = l2 - l3 * hkvu;
  const int64_t b = l3;
  const int64_t h = kvh * G + hg;

  const int qh = w >> 1, kh = w & 1;  // query half, key half
  const int qhu = __builtin_amdgcn_readfirstlane(qh), khu = __builtin_amdgcn_readfirstlane(kh);
  // rows of this sequence (a ragged batch's shorter sequences end early; their
  // padding rows are never read)
  const int64_t Tb = p.lens ? min(max((int64_t)sload_i32(p.lens + b), (int64_t)0), p.T) : p.T;
  const int T32 = (int)Tb, nkb32 = (int)p.nkb;
  int64_t q_row[2];                    // this lane's query in each 16-query group
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) q_row[qg] = qb * PF_BS + 32 * qh + 16 * qg + c16;
  bf16x8 qreg[2][4];  // this lane's q fragments, loaded after the first block copies are issued
  // the list length and its first two entries in one scalar wait (a list
  // entry read past the count is never used)
  const int32_t *list = p.ids + ((b * p.Hq + h) * p.nqb + qb) * p.width;
  const int32_t *cnt_p = p.counts ? p.counts + (b * p.Hq + h) * p.nqb + qb : list;
  int n, kbj, kb1;
  const int o1 = __builtin_amdgcn_readfirstlane(p.width > 1 ? 1 : 0);
  sload3_i32(cnt_p, list, list + o1, n, kbj, kb1);
  n = p.counts ? min(n, (int)p.width) : (int)p.width;
  if (qb * PF_BS >= Tb) n = 0;  // a query block past the sequence's end attends nothing

  // four output values of query group qg: dims 16 dt + 4 g .. + 3
  auto store4 = [&](int qg, int dt, f32x4 r) {
    const int64_t o = b * p.o_sb + h * p.o_sh + q_row[qg] * p.o_st + 16 * dt + 4 * g;
    if (p.out_dt == LA_BF16) {
      const bf16x2 x = __builtin_convertvector((f32x2{r[0], r[1]}), bf16x2);
      const bf16x2 y = __builtin_convertvector((f32x2{r[2], r[3]}), bf16x2);
      const u32x2 u = {__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, y)};
      __builtin_nontemporal_store(u, (u32x2 *)((uint16_t *)p.out + o));
    } else {
      __builtin_nontemporal_store(r, (f32x4 *)((float *)p.out + o));
    }
  };
  if (n <= 0) {  // an empty list attends nothing: zero rows (n is workgroup-uniform)
    if (kh == 0)
#pragma unroll
      for (int qg = 0; qg < 2; ++qg)
        if (q_row[qg] < p.T)
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) store4(qg, dt, f32x4{0.f, 0.f, 0.f, 0.f});
    return;
  }

  const uint16_t *kbh = p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t *vbh = p.v + b * p.v_sb + kvh * p.v_sh;
  const int32_t *vexp = p.vexp + (b * p.Hkv + kvh) * p.nkb;
  // a block is whole (no row past T) and listed (>= 0) iff kb < T / 64 as
  // an unsigned compare
  const uint32_t nwhole = (uint32_t)(T32 / PF_BS);
  auto whole_block = [&](int kb) { return (uint32_t)kb < nwhole; };
  // LDS slots: K x at element kslot(x), V x at vslot(x), x in {0, 1}
  auto kslot = [](int x) { return (uint32_t)(x * KSL); };
  auto vslot = [](int x) { return (uint32_t)(2 * KSL + x * PF_BLK); };
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t *)smem);
  const int wu = __builtin_amdgcn_readfirstlane(w);
  // LDS-DMA of a block: instruction t of wave w fills rows 16 t + 4 w + lane/16;
  // a lane writes chunk position lane%16 of its row and fetches global chunk
  // (lane%16) ^ swz(row)  (swz(row + 16 t) == swz(row)).  Whole blocks use a
  // block base in SGPRs and per-lane 32-bit byte offsets (no per-load VALU).
  const int drow = 4 * w + (lane >> 4);
  const int kdch = (lane & 15) ^ pf_swz_k(drow), vdch = (lane & 15) ^ pf_swz(drow);
  uint32_t kvo[4], vvo[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    kvo[t] = (uint32_t)((((int64_t)(16 * t + drow)) * p.k_st + 8 * kdch) * 2);
    vvo[t] = (uint32_t)((((int64_t)(16 * t + drow)) * p.v_st + 8 * vdch) * 2);
  }
  auto dma_part = [&](const uint16_t *bh, int64_t st, uint32_t blk, const uint32_t (&vo)[4], int dch,
                      int kb, uint32_t soff) {
    const uint32_t m0 = lds0 + 2 * (soff + 4 * wu * PF_D);
    if (whole_block(kb)) {
      const uint16_t *base = bh + (uint32_t)kb * blk;  // fits 32 bits (checked at launch)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(vo[t]), "s"(base),
                     "{m0}"(m0 + 2 * 16 * t * PF_D) : "memory");
    } else {  // a partial last block or a -1 entry: rows clamped into [0, T)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t key = min((int64_t)max(kb, 0) * PF_BS + 16 * t + drow, Tb - 1);
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(bh + key * st + 8 * dch),
                     "{m0}"(m0 + 2 * 16 * t * PF_D) : "memory");
      }
    }
  };
  // KF8 K blocks: rows of 128 bytes (8 chunks); instruction t of wave w
  // fills rows 32 t + 8 w + lane/8, a lane writes chunk position lane%8 of its
  // row and fetches global chunk (lane%8) ^ (row & 7).  Byte offsets.
  const int drow8 = 8 * w + (lane >> 3);
  const int kdch8 = (lane & 7) ^ (drow8 & 7);
  uint32_t k8o[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) k8o[t] = (uint32_t)(((int64_t)(32 * t + drow8)) * p.k_st + 16 * kdch8);
  const char *kbh8 = (const char *)p.k + b * p.k_sb + kvh * p.k_sh;  // KF8: byte strides
  auto dma_k = [&](int kb, int x) {
    if constexpr (KF8) {
      const uint32_t m0 = lds0 + 2 * kslot(x) + 8 * PF_D * wu;
      if (whole_block(kb)) {
        const char *base = kbh8 + (uint32_t)kb * p.k_blk;
#pragma unroll
        for (int t = 0; t < 2; ++t)
          asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(k8o[t]), "s"(base),
                       "{m0}"(m0 + 32 * PF_D * t) : "memory");
      } else {  // a partial last block or a -1 entry: rows clamped into [0, T)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int64_t key = min((int64_t)max(kb, 0) * PF_BS + 32 * t + drow8, Tb - 1);
          asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(kbh8 + key * p.k_st + 16 * kdch8),
                       "{m0}"(m0 + 32 * PF_D * t) : "memory");
        }
      }
    } else {
      dma_part(kbh, p.k_st, p.k_blk, kvo, kdch, kb, kslot(x));
    }
  };
  auto dma_v = [&](int kb, int x) { dma_part(vbh, p.v_st, p.v_blk, vvo, vdch, kb, vslot(x)); };
  // rows of a landed partial block that lie past T (or all rows of a -1
  // entry) are cleared, so masked keys hold zeros rather than copies
  auto clear_part = [&](int kb, uint32_t soff, int row_elems) {
    uint16_t *d = smem + soff;
    const int cpr = row_elems / 8;  // 16-byte chunks per row
    for (int ch = tid; ch < PF_BS * cpr; ch += PF_NT) {
      const int r = ch / cpr;
      if (kb < 0 || kb * PF_BS + r >= T32)
        *(uint4 *)(d + r * row_elems + 8 * (ch % cpr)) = uint4{0, 0, 0, 0};
    }
  };
  auto clear_k = [&](int kb, int x) { clear_part(kb, kslot(x), KF8 ? PF_D / 2 : PF_D); };
  auto clear_v = [&](int kb, int x) { clear_part(kb, vslot(x), PF_D); };

  // LDS element offsets of this lane's operand reads:
  // K: row 32 kh + c16 (+16 kt2), global chunk 4 s + g
  int koffs[4];
  const int ksw = pf_swz_k(c16);
#pragma unroll
  for (int s = 0; s < 4; ++s) koffs[s] = (32 * kh + c16) * PF_D + 8 * ((4 * s + g) ^ ksw);
  // KF8 K: row 32 kh + c16 (+16 kt2), the lane's 32 codes (dims 32 g .. +31)
  // are chunks 2 g and 2 g + 1 (byte offsets in the slot)
  int k8offs[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) k8offs[h] = (32 * kh + c16) * PF_D + 16 * ((2 * g + h) ^ (c16 & 7));
  auto load_k8 = [&](uint32_t soff, int kt2) {
    const char *sk8 = (const char *)(smem + soff) + 16 * kt2 * PF_D;
    const uint4 a0 = *(const uint4 *)(sk8 + k8offs[0]), a1 = *(const uint4 *)(sk8 + k8offs[1]);
    return i32x8{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z,
                 (int)a1.w};
  };
  // fp8 e4m3 K codes x fp8 e4m3 q terms (unit scales: e8m0 127)
  auto mfma8 = [](const i32x8 &a, const i32x8 &b, f32x4 c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
  };
  i32x8 qh8[2], ql8[2];  // KF8: this lane's q terms (query q_row[qg], dims 32 g .. +31)
  // V (transpose reads): row 32 kh + 4 g + c16/4 (+16), global column
  // 16 dt + 4 (c16 % 4) = chunk 2 dt + (c16/2)%2, element 4 (c16 % 2) in it
  const int vr = 4 * g + (c16 >> 2), vsw = pf_swz(vr);
  int voffs[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    voffs[dt] = (32 * kh + vr) * PF_D + 8 * ((2 * dt + ((c16 >> 1) & 1)) ^ vsw) + 4 * (c16 & 1);

  // S^T = K Q^T over this wave's 32 keys of the K block in LDS slot x
  auto scores = [&](int x, f32x4 (&st)[2][2]) {
    const uint16_t *sk = smem + kslot(x);
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) {
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KF8) {
        const i32x8 a = load_k8(kslot(x), kt2);
        s0 = mfma8(a, ql8[0], mfma8(a, qh8[0], s0));
        s1 = mfma8(a, ql8[1], mfma8(a, qh8[1], s1));
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8 a = *(const bf16x8 *)&sk[koffs[s] + 16 * kt2 * PF_D];
          s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[0][s], s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[1][s], s1, 0, 0, 0);
        }
      }
      st[0][kt2] = s0;
      st[1][kt2] = s1;
    }
  };

  // m: reference maximum of the raw (unscaled) scores of this lane's query,
  // per group; thr = m + thr_gap, the raw score above which m must be raised;
  // nmu = -m * qscale (0 while m = -inf), the exponent offset of the weights
  const float NEG_INF = __int_as_float(0xff800000);
  float qs[2] = {p.qscale, p.qscale}, tg[2] = {p.thr_gap, p.thr_gap};  // KF8: per lane and group
  auto QS = [&](int qg) {
    if constexpr (KF8) return qs[qg]; else return p.qscale;
  };
  auto TG = [&](int qg) {
    if constexpr (KF8) return tg[qg]; else return p.thr_gap;
  };
  // KF8: the 64 scales of K block kb go to LDS with its codes (wave 0: one
  // 4-byte LDS-DMA load per lane from the caller's scale tensor, counted and
  // waited for like the block copies; keys past T read the last key's scale,
  // and an empty entry block 0's, never used)
  auto dma_ks = [&](int kb, int x) {
    if constexpr (KF8) {
      if (wu == 0) {
        const int64_t key = min((int64_t)max(kb, 0) * PF_BS + lane, Tb - 1);
        const float *sp = p.ks + b * p.s_sb + kvh * p.s_sh + key * p.s_st;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(
            (uint32_t)(uintptr_t)(lds_void_t *)(sscale + x * PF_BS));
        asm volatile("global_load_lds_dword %0, off" ::"v"(sp), "{m0}"(m0) : "memory");
      }
    }
  };
  // the scores of this lane's 8 keys (16 kt2 + 4 g + e of its key half) of
  // the K block in `slot`, times their scales
  auto scale_scores = [&](f32x4 (&sc)[2][2], int slot) {
    const float *sp = sscale + slot * PF_BS + 32 * kh + 4 * g;
    f32x4 sk[2];
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) sk[kt2] = *(const f32x4 *)(sp + 16 * kt2);
#pragma unroll
    for (int qg = 0; qg < 2; ++qg)
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2) sc[qg][kt2] *= sk[kt2];
  };
  float m[2] = {NEG_INF, NEG_INF}, thr[2] = {NEG_INF, NEG_INF}, l[2] = {0.f, 0.f};
  float nmu[2] = {0.f, 0.f};
  f32x4 acc[2][8];
#pragma unroll
  for (int qg = 0; qg < 2; ++qg)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[qg][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The mask of block kbx in this wave's key half: -inf on keys past the
  // causal diagonal or past T, and on every key of a -1 entry, written over
  // the block's scores.  Only those blocks (diagonal, partial, empty) need it;
  // keys and positions fit in int32 (T < 2^30 is checked at launch).
  // Blocks kb <= mask_lim need no mask in this wave: key 32 kh + 31 of the
  // block is at most the first query of the wave's half (causal) and below T.
  const int mask_lim = min(p.causal ? (int)qb - 1 + (qhu > khu ? 1 : 0) : INT_MAX,
                           (T32 - 32 - 32 * khu) >> 6);
  auto needs_mask = [&](int kbx) { return kbx < 0 || kbx > mask_lim; };
  auto apply_mask = [&](int kbx, f32x4 (&sc)[2][2]) {
    const int key0 = kbx * PF_BS + 32 * kh;
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      const int last = min(p.causal ? (int)q_row[qg] : INT_MAX, T32 - 1);
      const int lim = kbx < 0 ? -1 : last - key0;  // keys past lim are masked
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (16 * kt2 + 4 * g + e > lim) sc[qg][kt2][e] = NEG_INF;
    }
  };
  // this lane's largest score of a block, per query group (v_max3 chains)
  auto lane_max = [&](const f32x4 (&sc)[2][2], float (&mx)[2]) {
#pragma unroll
    for (int qg = 0; qg < 2; ++qg)
      mx[qg] = pf_max(pf_max(pf_max(sc[qg][0][0], sc[qg][0][1]), pf_max(sc[qg][0][2], sc[qg][0][3])),
                      pf_max(pf_max(sc[qg][1][0], sc[qg][1][1]), pf_max(sc[qg][1][2], sc[qg][1][3])));
  };
  // Settle the reference maxima for a block whose lane maxima are mx.  m is
  // raised (and l, acc rescaled) only when some query's block maximum exceeds
  // it by more than 2^8 in the exponent, so the weights stay below 256 (fp16
  // holds them) and raises are rare; the final division by l is unchanged by
  // the choice of reference.  The test is one compare per lane (any lane over
  // its query's threshold); the exact column maximum (lane swaps) is formed
  // only then.  alpha (the factor for acc) is returned through `alpha`.
  auto settle_max = [&](float (&mx)[2], float (&alpha)[2]) {
    alpha[0] = alpha[1] = 1.f;
    if (__ballot(mx[0] > thr[0] || mx[1] > thr[1]) == 0) return false;  // the common case
    bool any = false;
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      if (__ballot(mx[qg] > thr[qg]) != 0) {
        const float cm = pf_pair32_max(pf_pair16_max(mx[qg]));
        const float mn = pf_max(m[qg], cm);
        alpha[qg] = (m[qg] == NEG_INF) ? 0.f : fast_exp2((m[qg] - mn) * QS(qg));
        m[qg] = mn;
        thr[qg] = mn + TG(qg);
        nmu[qg] = (mn == NEG_INF) ? 0.f : -mn * QS(qg);
        l[qg] *= alpha[qg];
        any = true;
      }
    }
    return any;
  };
  auto rescale_acc = [&](const float (&alpha)[2]) {
#pragma unroll
    for (int qg = 0; qg < 2; ++qg)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[qg][dt] *= alpha[qg];
  };
  // Software pipeline over the list.  Step j computes the scores of block
  // j+1 while the weights of block j are formed, then block j's PV product
  // while the maxima of block j+1 are taken.  K block x lives in K slot x % 2
  // and V block x in V slot x % 2; both are fetched one step ahead (K of
  // block j+2 and V of block j+1 during step j).  bf16 K/V: lists of up to
  // 64 entries sit in VGPR lanes (entry i in lane i, with the exponent of its
  // V block) and are read per step by v_readlane; longer lists, and every
  // list of the fp8 form (which has no registers to spare), come through the
  // scalar cache (see sload_i32).
  if (n <= 1) kb1 = 0;
  const bool lanes = !KF8 && n <= 64;
  int lv = 0, evv = 0;
  if (lanes) lv = list[min(lane, n - 1)];
  dma_k(kbj, 0);
  dma_v(kbj, 0);
  if (n > 1) dma_k(kb1, 1);
  // q, read once: streamed past the caches that keep the K/V blocks.  bf16:
  // dims 32 s + 8 g .. +7 (the bf16 MFMA operand); KF8: dims 32 g + 8 s .. +7
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    const uint16_t *qp = p.q + b * p.q_sb + h * p.q_sh + min(q_row[qg], Tb - 1) * p.q_st;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qreg[qg][s] = __builtin_nontemporal_load(
          (const bf16x8 *)(qp + (KF8 ? 32 * g + 8 * s : 32 * s + 8 * g)));
  }
  dma_ks(kbj, 0);
  if (n > 1) dma_ks(kb1, 1);
  wait_vmcnt<0>();
#pragma unroll
  for (int qg = 0; qg < 2; ++qg)
#pragma unroll
    for (int s = 0; s < 4; ++s) settle(qreg[qg][s]);  // q landed with the first blocks
  settle(lv);
  if (lanes) evv = vexp[(uint32_t)lv < (uint32_t)nkb32 ? (uint32_t)lv : 0u];
  if constexpr (KF8) {
    // q row -> 2^e (hi + lo) in e4m3 codes, 2^e putting the row's largest |q|
    // in [128, 256) (its 128 values are spread over the 4 lanes c16 + 16 g).
    // With a power-of-two scale q / 2^e keeps its bf16 significand, and two
    // e4m3 terms hold any 8-bit significand exactly (hi its top 4 bits,
    // rounded; lo = q / 2^e - hi a multiple of 2^-7 of hi's binade of at most
    // 4 significant bits) while lo stays in the e4m3 range: every element
    // of magnitude >= 2^-9 of the row's largest is represented exactly, the
    // rest within 2^-17 of it.
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      float x[32];
      float am = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 w = __builtin_bit_cast(u32x4, qreg[qg][s]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[8 * s + 2 * e] = bf16lo(w[e]);
          x[8 * s + 2 * e + 1] = bf16hi(w[e]);
        }
      }
#pragma unroll
      for (int i = 0; i < 32; ++i) am = pf_max(am, fabsf(x[i]));
      am = pf_pair32_max(pf_pair16_max(am));
      const int e = am > 0.f ? (int)((__float_as_uint(am) >> 23) & 0xff) - 127 - 7 : 0;
#pragma unroll
      for (int i = 0; i < 32; ++i) x[i] = __builtin_amdgcn_ldexpf(x[i], -e);
      // codes by round to nearest; x keeps the residual for the second term
      auto term = [&]() {
        i32x8 t;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          int wv = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * j], x[4 * j + 1], 0, false);
          wv = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * j + 2], x[4 * j + 3], wv, true);
          t[j] = wv;
          const float2 a = fp8x2_to_f32<false>((uint32_t)wv), c = fp8x2_to_f32<true>((uint32_t)wv);
          x[4 * j] -= a.x;
          x[4 * j + 1] -= a.y;
          x[4 * j + 2] -= c.x;
          x[4 * j + 3] -= c.y;
        }
        return t;
      };
      qh8[qg] = term();
      ql8[qg] = term();
      qs[qg] = __builtin_amdgcn_ldexpf(p.qscale, e);
      tg[qg] = 8.f / qs[qg];
    }
  }
  lds_barrier();
  {
    const bool c0 = !whole_block(kbj), c1 = n > 1 && !whole_block(kb1);
    if (c0) {
      clear_k(kbj, 0);
      clear_v(kbj, 0);
    }
    if (c1) clear_k(kb1, 1);
    if (c0 || c1) lds_barrier();
  }
  // scores of blocks with even / odd list position
  f32x4 sA[2][2], sB[2][2];
  scores(0, sA);
  if constexpr (KF8) scale_scores(sA, 0);
  if (needs_mask(kbj)) apply_mask(kbj, sA);
  {
    float mx[2], alpha[2];
    lane_max(sA, mx);
    settle_max(mx, alpha);  // acc is still zero: no rescale
  }
  lds_barrier();  // every wave has read K slot 0 before step 0 refills it

  // Step j: all of the step's LDS operands are read first (K of block j+1,
  // V of block j), then (A) the scores of block j+1 (of a stale slot when
  // j+1 == n: computed, unused) with the weights of block j, then (B) block
  // j's PV product with the lane maxima of block j+1.  The reads, A and B are
  // one branch-free block whose matrix and vector instructions are
  // interleaved (sched_group_barrier); the masks of diagonal / partial blocks
  // and the rare raise of a reference maximum follow it.
  // FULL: j + 2 < n (every block of the step exists: the steady state,
  // without edge conditions).
  auto step = [&](auto full, int j, const int par, f32x4 (&st)[2][2], f32x4 (&sn)[2][2]) {
    constexpr bool FULL = decltype(full)::value;
    // list entry j+2 and the exponent of V block j (V block j holds v * 2^-ev;
    // an empty or out-of-range entry reads exponent 0 from block 0)
    int kb2, ev;
    if (lanes) {
      kb2 = __builtin_amdgcn_readlane(lv, FULL ? j + 2 : min(j + 2, n - 1));
      ev = __builtin_amdgcn_readlane(evv, j);
    } else {
      const uint32_t kbe = (uint32_t)kbj < (uint32_t)nkb32 ? (uint32_t)kbj : 0u;
      sload2_i32(list + (FULL ? j + 2 : min(j + 2, n - 1)), vexp + kbe, kb2, ev);
    }
    if (!FULL && j + 2 >= n) kb2 = 0;
    if (FULL || j + 2 < n) {  // the slot held block j (scored a step ago)
      dma_k(kb2, par);
      dma_ks(kb2, par);
    }
    if (FULL || j + 1 < n) dma_v(kb1, par ^ 1);  // held block j-1 (multiplied)
    const uint16_t *sk = smem + kslot(par ^ 1);
    const uint16_t *sv = smem + vslot(par);
    bf16x8 ka[2][4];
    i32x8 ka8[2];
    f16x8 va[8];
    if constexpr (KF8) {
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2) ka8[kt2] = load_k8(kslot(par ^ 1), kt2);
    } else {
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[kt2][s] = *(const bf16x8 *)&sk[koffs[s] + 16 * kt2 * PF_D];
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      // V^T rows through the LDS transpose read: lane (g, j) of a 16-lane group
      // gets V[k0 + e][16 dt + j], e < 4, when lane i of the group points at
      // row k0 + i/4, columns 16 dt + 4 (i%4) .. +3
      const uint16_t *v0 = sv + voffs[dt];
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)v0);
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(v0 + 16 * PF_D));
      va[dt] = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
    // S^T = K Q^T for block j+1
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) {
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KF8) {
        s0 = mfma8(ka8[kt2], qh8[0], s0);
        s1 = mfma8(ka8[kt2], qh8[1], s1);
        s0 = mfma8(ka8[kt2], ql8[0], s0);
        s1 = mfma8(ka8[kt2], ql8[1], s1);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[kt2][s], qreg[0][s], s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[kt2][s], qreg[1][s], s1, 0, 0, 0);
        }
      }
      sn[0][kt2] = s0;
      sn[1][kt2] = s1;
    }
    // P = 2^ev * exp2(s*qscale - m*qscale) in fp16 (round to nearest even; at
    // most 2^(8+ev) <= 2^15); l sums the rounded weights times 2^-ev (exact:
    // 2^-ev, -8 <= ev <= 7, is a normal fp16).
    // Column c16 is this lane's query; the positive scale commutes with the
    // max, so it is applied in the exponent.
    const float evf = (float)ev;
    // 2^-ev as an fp16 pair (-8 <= ev <= 7: biased exponent 15 - ev in [8, 23])
    const uint32_t wbits = (uint32_t)(15 - ev) << 10;
    const f16x2 wl2 = __builtin_bit_cast(f16x2, wbits | (wbits << 16));
    f16x8 ph[2];
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      const float c = nmu[qg] + evf;
      float pv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = fast_exp2(__builtin_fmaf(st[qg][0][e], QS(qg), c));
        pv[4 + e] = fast_exp2(__builtin_fmaf(st[qg][1][e], QS(qg), c));
      }
      f16x2 hw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hw[e] = __builtin_convertvector((f32x2{pv[2 * e], pv[2 * e + 1]}), f16x2);
        l[qg] = __builtin_amdgcn_fdot2(hw[e], wl2, l[qg], false);
      }
      ph[qg] = __builtin_shufflevector(__builtin_shufflevector(hw[0], hw[1], 0, 1, 2, 3),
                                       __builtin_shufflevector(hw[2], hw[3], 0, 1, 2, 3), 0, 1, 2,
                                       3, 4, 5, 6, 7);
    }
    // O^T += V^T P^T over this wave's keys; each V^T operand serves both groups
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int qg = 0; qg < 2; ++qg)
        acc[qg][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[dt], ph[qg], acc[qg][dt], 0, 0, 0);
    // KF8: the key scales of block j+1, applied with its maxima (its scores
    // are ready by then; applied right after the score products, the
    // multiplies would wait for the matrix core)
    if constexpr (KF8) scale_scores(sn, par ^ 1);
    float mx[2];
    lane_max(sn, mx);
    // order within the block: the LDS reads (24, KF8: 20), then the score
    // MFMAs (16, KF8: 8 of twice the work) each followed by weight VALU work,
    // then the 16 PV MFMAs each followed by VALU work of the next block's
    // maxima
    if constexpr (KF8) {
      __builtin_amdgcn_sched_group_barrier(0x100, 20, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
      }
    } else {
      __builtin_amdgcn_sched_group_barrier(0x100, 24, 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
    }
    if (FULL || j + 1 < n) {
      if (needs_mask(kb1)) {
        apply_mask(kb1, sn);
        lane_max(sn, mx);
      }
      float alpha[2];
      if (settle_max(mx, alpha)) rescale_acc(alpha);
    }
    // this wave's loads have landed and every wave is done with the slots
    // that the next step refills
    wait_vmcnt<0>();
    lds_barrier();
    const bool ck = (FULL || j + 2 < n) && !whole_block(kb2);
    const bool cv = (FULL || j + 1 < n) && !whole_block(kb1);
    if (ck || cv) {
      if (ck) clear_k(kb2, par);
      if (cv) clear_v(kb1, par ^ 1);
      lds_barrier();
    }
    kbj = kb1;
    kb1 = kb2;
  };
  using full_t = std::integral_constant<bool, true>;
  using tail_t = std::integral_constant<bool, false>;
  int j = 0;
  for (; j + 3 < n; j += 2) {
    step(full_t{}, j, 0, sA, sB);
    step(full_t{}, j + 1, 1, sB, sA);
  }
  // the last one to three steps
  for (; j < n; j += 2) {
    step(tail_t{}, j, 0, sA, sB);
    if (j + 1 >= n) break;
    step(tail_t{}, j + 1, 1, sB, sA);
  }
  // l is a per-lane partial over this lane's keys; sum the 4 lane groups.
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    l[qg] = pair32_sum(pair16_sum(l[qg]));
  }
  // Merge the two key halves.  The two waves of a query half exchange halves
  // of their accumulators through LDS (the staging buffers are free now):
  // the kh = 0 wave finalizes dims 0..63 and the kh = 1 wave dims 64..127,
  // each with the other's partial sums of its dims and the other's m, l.
  // red_o[qh][writer kh][qg][i][lane]: the writer's acc[qg][4 (1 - kh) + i].
  f32x4 *red_o = (f32x4 *)smem;
  float *red_ml = (float *)(red_o + 2 * 2 * 2 * 4 * 64);  // [qh][kh][qg][m, l][query]
  // (the accumulator halves are picked by a wave-uniform branch: indexing
  // acc by a runtime kh would move it to scratch memory)
  auto acc_half = [&](int qg, int i, bool upper) { return upper ? acc[qg][4 + i] : acc[qg][i]; };
  {
    f32x4 *mine = red_o + ((qh * 2 + kh) * 2) * 4 * 64;
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      if (khu == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) mine[(qg * 4 + i) * 64 + lane] = acc_half(qg, i, true);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) mine[(qg * 4 + i) * 64 + lane] = acc_half(qg, i, false);
      }
      if (g == 0) {
        red_ml[(((qh * 2 + kh) * 2 + qg) * 2 + 0) * 16 + c16] = m[qg];
        red_ml[(((qh * 2 + kh) * 2 + qg) * 2 + 1) * 16 + c16] = l[qg];
      }
    }
  }
  __syncthreads();
  {
    const int ok = 1 - kh;  // the partner wave
    const f32x4 *theirs = red_o + ((qh * 2 + ok) * 2) * 4 * 64;
    f32x4 o2[2][4];
    float m2[2], l2[2];
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o2[qg][i] = theirs[(qg * 4 + i) * 64 + lane];
      m2[qg] = red_ml[(((qh * 2 + ok) * 2 + qg) * 2 + 0) * 16 + c16];
      l2[qg] = red_ml[(((qh * 2 + ok) * 2 + qg) * 2 + 1) * 16 + c16];
    }
    f32x4 r[2][4];
    bool live[2];
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      const float M = pf_max(m[qg], m2[qg]);
      const float a1 = (m[qg] == NEG_INF) ? 0.f : fast_exp2((m[qg] - M) * QS(qg));
      const float a2 = (m2[qg] == NEG_INF) ? 0.f : fast_exp2((m2[qg] - M) * QS(qg));
      const float L = l[qg] * a1 + l2[qg] * a2;
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const float b1 = a1 * inv, b2 = a2 * inv;
      if (khu == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r[qg][i] = acc_half(qg, i, false) * b1 + o2[qg][i] * b2;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) r[qg][i] = acc_half(qg, i, true) * b1 + o2[qg][i] * b2;
      }
      live[qg] = q_row[qg] < p.T;
      if (q_row[qg] >= Tb)  // padding rows of a shorter sequence are written as zeros
#pragma unroll
        for (int i = 0; i < 4; ++i) r[qg][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (p.out_dt == LA_BF16) {
#pragma unroll
      for (int qg = 0; qg < 2; ++qg)
        if (live[qg])
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int64_t o = b * p.o_sb + h * p.o_sh + q_row[qg] * p.o_st + 16 * (4 * kh + i) + 4 * g;
            const bf16x2 x = __builtin_convertvector((f32x2{r[qg][i][0], r[qg][i][1]}), bf16x2);
            const bf16x2 y = __builtin_convertvector((f32x2{r[qg][i][2], r[qg][i][3]}), bf16x2);
            const u32x2 u = {__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, y)};
            __builtin_nontemporal_store(u, (u32x2 *)((uint16_t *)p.out + o));
          }
    } else {
#pragma unroll
      for (int qg = 0; qg < 2; ++qg)
        if (live[qg])
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int64_t o = b * p.o_sb + h * p.o_sh + q_row[qg] * p.o_st + 16 * (4 * kh + i) + 4 * g;
            __builtin_nontemporal_store(r[qg][i], (f32x4 *)((float *)p.out + o));
          }
    }
  }
}

}  // namespace la

using namespace la;

namespace la {

// The status word read (and, with clear, reset) in one atomic exchange on the
// caller's stream, so a bit raised by a kernel of another stream is never lost
// between a read and a clear.
__device__ uint32_t la_pf_status_snap;
__global__ void pf_status_kernel(int clear) {
  la_pf_status_snap = clear ? __hip_atomic_exchange(&la_pf_status, 0u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                            : __hip_atomic_load(&la_pf_status, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
}

int prefill_status(uint32_t *bits, bool clear, hipStream_t st) {
  pf_status_kernel<<<1, 1, 0, st>>>(clear ? 1 : 0);
  LA_LAUNCHED();
  LA_HIP(hipMemcpyFromSymbolAsync(bits, HIP_SYMBOL(la_pf_status_snap), sizeof(uint32_t), 0,
                                  hipMemcpyDeviceToHost, st));
  LA_HIP(hipStreamSynchronize(st));
  return LA_OK;
}

static int64_t pf_align(int64_t x) { return (x + 255) / 256 * 256; }

static bool prefill_fp8(const la_prefill_args *a) { return a->kv_dtype == LA_FP8_E4M3; }

// Workspace: the fp16 copy of V (B, Hkv, T, 128) and its block exponents
// (fp8 K is staged from the caller's codes and scales directly).
static int64_t prefill_ws_bytes(const la_prefill_args *a) {
  const int64_t nkb = ceil_div(a->T, PF_BS);
  return pf_align(a->B * a->Hkv * a->T * PF_D * 2) + pf_align(a->B * a->Hkv * nkb * 4);
}

static int prefill_validate(const la_prefill_args *a) {
  LA_REQUIRE(a && a->q && a->k && a->v && a->out && a->ids, "la_block_sparse_prefill: null pointer");
  LA_REQUIRE(a->B > 0 && a->Hq > 0 && a->Hkv > 0 && a->T > 0, "la_block_sparse_prefill: bad shape");
  LA_REQUIRE(a->Hq % a->Hkv == 0, "n_heads must be a multiple of n_kv_heads");
  if (a->D != PF_D || a->block != PF_BS)
    return fail(LA_ERR_UNSUPPORTED, "la_block_sparse_prefill: head_dim 128 and 64-token blocks only");
  LA_REQUIRE(a->out_dtype == LA_F32 || a->out_dtype == LA_BF16, "la_block_sparse_prefill: out dtype");
  LA_REQUIRE(a->width >= 1, "la_block_sparse_prefill: list width");
  LA_REQUIRE(a->T < ((int64_t)1 << 30), "la_block_sparse_prefill: T must be below 2^30");
  LA_REQUIRE(a->scale > 0.f, "la_block_sparse_prefill: scale must be positive");
  if (prefill_fp8(a)) {
    LA_REQUIRE(a->k_scale && a->v_scale, "la_block_sparse_prefill: fp8 K/V need k_scale and v_scale");
    // K rows go to LDS in 16-byte pieces, V codes are read 8 bytes at a time;
    // element strides are bytes for fp8
    const bool al8 = (uintptr_t)a->k % 16 == 0 && (uintptr_t)a->v % 8 == 0 && a->k_sb % 16 == 0 &&
                     a->k_sh % 16 == 0 && a->k_st % 16 == 0 && a->v_sb % 8 == 0 &&
                     a->v_sh % 8 == 0 && a->v_st % 8 == 0;
    LA_REQUIRE(al8, "la_block_sparse_prefill: fp8 rows must be contiguous, K 16-byte and V 8-byte "
                    "aligned");
  } else {
    const bool alk = (uintptr_t)a->k % 16 == 0 && (uintptr_t)a->v % 16 == 0 && a->k_sb % 8 == 0 &&
                     a->k_sh % 8 == 0 && a->k_st % 8 == 0 && a->v_sb % 8 == 0 && a->v_sh % 8 == 0 &&
                     a->v_st % 8 == 0;
    LA_REQUIRE(alk, "la_block_sparse_prefill: rows must be contiguous and 16-byte aligned");
  }
  // 16-byte vector access of q rows and of the output
  const bool al = ((uintptr_t)a->q % 16 == 0) && ((uintptr_t)a->out % 16 == 0) &&
                  a->q_sb % 8 == 0 && a->q_sh % 8 == 0 && a->q_st % 8 == 0 &&
                  a->o_sb % 4 == 0 && a->o_sh % 4 == 0 && a->o_st % 4 == 0;
  LA_REQUIRE(al, "la_block_sparse_prefill: rows must be contiguous and 16-byte aligned");
  return LA_OK;
}

}  // namespace la

extern "C" size_t la_block_sparse_prefill_workspace(const la_prefill_args *a) {
  if (prefill_validate(a) != LA_OK) return 0;
  return (size_t)prefill_ws_bytes(a);
}

extern "C" int la_block_sparse_prefill(const la_prefill_args *a, void *stream) {
  const int rc = prefill_validate(a);
  if (rc != LA_OK) return rc;
  const int64_t ws_need = prefill_ws_bytes(a);
  LA_REQUIRE(a->workspace != nullptr, "la_block_sparse_prefill: workspace required");
  LA_REQUIRE((uintptr_t)a->workspace % 256 == 0, "la_block_sparse_prefill: workspace alignment");
  if (a->ws_bytes < ws_need)
    return fail(LA_ERR_WORKSPACE, "la_block_sparse_prefill: workspace %lld < %lld bytes",
                (long long)a->ws_bytes, (long long)ws_need);
  const int64_t nkb = ceil_div(a->T, PF_BS);
  uint16_t *v16 = (uint16_t *)a->workspace;
  int32_t *vexp = (int32_t *)((char *)a->workspace + pf_align(a->B * a->Hkv * a->T * PF_D * 2));
  hipStream_t st = (hipStream_t)stream;
  const int64_t nvb = a->B * a->Hkv * nkb;
  LA_REQUIRE(nvb < ((int64_t)1 << 31), "la_block_sparse_prefill: too many key blocks");
  const bool f8 = prefill_fp8(a);
  if (f8)
    prefill_v16_kernel<true><<<dim3((unsigned)nvb), 256, 0, st>>>(
        a->v, a->v_scale, a->s_sb, a->s_sh, a->s_st, a->v_sb, a->v_sh, a->v_st, a->Hkv, a->T, nkb,
        v16, vexp, a->lengths);
  else
    prefill_v16_kernel<false><<<dim3((unsigned)nvb), 256, 0, st>>>(
        a->v, nullptr, 0, 0, 0, a->v_sb, a->v_sh, a->v_st, a->Hkv, a->T, nkb, v16, vexp, a->lengths);
  LA_LAUNCHED();
  PfKP p{};
  p.q = (const uint16_t *)a->q;
  p.k = (const uint16_t *)a->k;  // fp8: the codes, addressed in bytes
  p.v = v16;
  p.vexp = vexp;
  p.out = a->out;
  p.ids = a->ids;
  p.counts = a->counts;
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.T = a->T;
  p.q_sb = a->q_sb; p.q_sh = a->q_sh; p.q_st = a->q_st;
  p.k_sb = a->k_sb; p.k_sh = a->k_sh; p.k_st = a->k_st;
  p.v_st = PF_D; p.v_sh = a->T * PF_D; p.v_sb = a->Hkv * a->T * PF_D;
  LA_REQUIRE(nkb * PF_BS * std::max<int64_t>(p.k_st, PF_D) < ((int64_t)1 << 31),
             "la_block_sparse_prefill: K rows of one head span >= 2^31 elements");
  p.k_blk = (uint32_t)(PF_BS * p.k_st);
  p.v_blk = (uint32_t)(PF_BS * PF_D);
  p.o_sb = a->o_sb; p.o_sh = a->o_sh; p.o_st = a->o_st;
  p.width = a->width;
  p.nqb = ceil_div(a->T, PF_BS);
  p.nkb = nkb;
  p.qscale = a->scale * 1.4426950408889634f;
  p.thr_gap = 8.f / p.qscale;
  auto log2_or = [](int64_t x) { return is_pow2(x) ? ilog2(x) : -1; };
  p.sh_g = log2_or(a->Hq / a->Hkv);
  p.sh_nqb = log2_or(p.nqb);
  p.sh_hkv = log2_or(a->Hkv);
  p.causal = a->causal;
  p.out_dt = a->out_dtype;
  p.lens = a->lengths;
  if (f8) {
    p.ks = a->k_scale;
    p.s_sb = a->s_sb; p.s_sh = a->s_sh; p.s_st = a->s_st;
  }
  const int64_t nwg = a->B * a->Hq * p.nqb;
  LA_REQUIRE(nwg < ((int64_t)1 << 31), "la_block_sparse_prefill: too many query blocks");
  if (f8)
    prefill_kernel<true><<<dim3((unsigned)nwg), PF_NT, 0, st>>>(p);
  else
    prefill_kernel<false><<<dim3((unsigned)nwg), PF_NT, 0, st>>>(p);
  LA_LAUNCHED();
  return LA_OK;
}
