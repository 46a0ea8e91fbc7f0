// Block-sparse causal prefill on the gfx950 matrix cores.
//
// The executor of block_sparse_attention (kernels/triton/block_sparse.py:80-163)
// specialised for lists shared by a 64-query block: workgroup (b, h, qb) attends
// the listed 64-key blocks of KV head h / (Hq/Hkv), with the causal mask applied
// in-kernel on the diagonal block.  Head dim 128, bf16 inputs, fp32 accumulate,
// online softmax in the log2 domain.
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
#include <climits>

#include "common.h"

namespace la {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

constexpr int PF_D = 128, PF_BS = 64, PF_NT = 256;
constexpr int PF_BLK = PF_BS * PF_D;  // elements of one staged K or V block (16 KiB)

// Chunk swizzle of staged row r (16-byte chunks, 16 per row): a permutation
// of 0..15 over any 16 consecutive rows (K reads: 16 lanes, 16 rows, one
// chunk), and rows r and r ^ 1 never share a chunk pair {2i, 2i+1} (V
// transpose reads: 8 rows x 2 chunks per 32 lanes).
__device__ __forceinline__ int pf_swz(int r) { return (2 * (r & 7)) ^ ((r >> 3) & 1); }

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
  // K slots 0..1, V slots 2..3 (64 KiB: two workgroups per CU); after the
  // loop, the key-half merge area
  __shared__ __align__(16) uint16_t smem[4 * PF_BLK];

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

  // four output values of query group qg: dims 16 dt + 4 g .. + 3
  auto store4 = [&](int qg, int dt, f32x4 r) {
    const int64_t o = b * p.o_sb + h * p.o_sh + q_row[qg] * p.o_st + 16 * dt + 4 * g;
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
  auto whole_block = [&](int kb) { return kb >= 0 && (int64_t)kb * PF_BS + PF_BS <= p.T; };
  // LDS slots of PF_BLK elements: K in 0..1, V in 2..3
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t *)smem);
  const int wu = __builtin_amdgcn_readfirstlane(w);
  // LDS-DMA of a block: instruction t of wave w fills rows 16 t + 4 w + lane/16;
  // a lane writes chunk position lane%16 of its row and fetches global chunk
  // (lane%16) ^ swz(row)  (swz(row + 16 t) == swz(row)).  Whole blocks use a
  // block base in SGPRs and per-lane 32-bit byte offsets (no per-load VALU).
  const int drow = 4 * w + (lane >> 4);
  const int dch = (lane & 15) ^ pf_swz(drow);
  uint32_t kvo[4], vvo[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    kvo[t] = (uint32_t)((((int64_t)(16 * t + drow)) * p.k_st + 8 * dch) * 2);
    vvo[t] = (uint32_t)((((int64_t)(16 * t + drow)) * p.v_st + 8 * dch) * 2);
  }
  auto dma_part = [&](const uint16_t *bh, int64_t st, const uint32_t (&vo)[4], int kb, int slot) {
    const uint32_t m0 = lds0 + 2 * (slot * PF_BLK + 4 * wu * PF_D);
    if (whole_block(kb)) {
      const uint16_t *base = bh + (int64_t)kb * PF_BS * st;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(vo[t]), "s"(base),
                     "{m0}"(m0 + 2 * 16 * t * PF_D) : "memory");
    } else {  // a partial last block or a -1 entry: rows clamped into [0, T)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t key = min((int64_t)max(kb, 0) * PF_BS + 16 * t + drow, p.T - 1);
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(bh + key * st + 8 * dch),
                     "{m0}"(m0 + 2 * 16 * t * PF_D) : "memory");
      }
    }
  };
  auto dma_k = [&](int kb, int slot) { dma_part(kbh, p.k_st, kvo, kb, slot); };
  auto dma_v = [&](int kb, int slot) { dma_part(vbh, p.v_st, vvo, kb, slot); };
  // rows of a landed partial block that lie past T (or all rows of a -1
  // entry) are cleared, so masked keys hold zeros rather than copies
  auto clear_rows = [&](int kb, int slot) {
    uint16_t *d = smem + slot * PF_BLK;
    for (int ch = tid; ch < PF_BS * 16; ch += PF_NT) {
      const int r = ch >> 4;
      if (kb < 0 || (int64_t)kb * PF_BS + r >= p.T) *(uint4 *)(d + r * PF_D + 8 * (ch & 15)) = uint4{0, 0, 0, 0};
    }
  };

  // LDS element offsets of this lane's operand reads:
  // K: row 32 kh + c16 (+16 kt2), global chunk 4 s + g
  int koffs[4];
  const int ksw = pf_swz(c16);
#pragma unroll
  for (int s = 0; s < 4; ++s) koffs[s] = (32 * kh + c16) * PF_D + 8 * ((4 * s + g) ^ ksw);
  // V (transpose reads): row 32 kh + 4 g + c16/4 (+16), global column
  // 16 dt + 4 (c16 % 4) = chunk 2 dt + (c16/2)%2, element 4 (c16 % 2) in it
  const int vr = 4 * g + (c16 >> 2), vsw = pf_swz(vr);
  int voffs[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    voffs[dt] = (32 * kh + vr) * PF_D + 8 * ((2 * dt + ((c16 >> 1) & 1)) ^ vsw) + 4 * (c16 & 1);

  // S^T = K Q^T over this wave's 32 keys of the K block in LDS slot `slot`
  auto scores = [&](int slot, f32x4 (&st)[2][2]) {
    const uint16_t *sk = smem + slot * PF_BLK;
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) {
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 a = *(const bf16x8 *)&sk[koffs[s] + 16 * kt2 * PF_D];
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[0][s], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[1][s], s1, 0, 0, 0);
      }
      st[0][kt2] = s0;
      st[1][kt2] = s1;
    }
  };

  // m: reference maximum of the raw (unscaled) scores of this lane's query, per group
  float m[2] = {__int_as_float(0xff800000), __int_as_float(0xff800000)}, l[2] = {0.f, 0.f};
  f32x4 acc[2][8];
#pragma unroll
  for (int qg = 0; qg < 2; ++qg)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[qg][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The mask of block kbx in this wave's key half: -inf on keys past the
  // causal diagonal or past T, and on every key of a -1 entry, written over
  // the block's scores.  Only those blocks (diagonal, partial, empty: a
  // wave-uniform branch) pay for it; keys and positions fit in int32
  // (T < 2^30 is checked at launch).
  auto apply_mask = [&](int kbx, f32x4 (&sc)[2][2]) {
    const int key0 = kbx * PF_BS + 32 * kh;  // first key of this half
    const bool need = kbx < 0 || (p.causal && key0 + 31 > (int)qb * PF_BS + 32 * qh) ||
                      key0 + 32 > (int)p.T;
    if (need) {
#pragma unroll
      for (int qg = 0; qg < 2; ++qg) {
        const int last = min(p.causal ? (int)q_row[qg] : INT_MAX, (int)p.T - 1);
        const int lim = kbx < 0 ? -1 : last - key0;  // keys past lim are masked
#pragma unroll
        for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (16 * kt2 + 4 * g + e > lim) sc[qg][kt2][e] = __int_as_float(0xff800000);
      }
    }
  };
  // Settle the reference maxima for a block's (masked) scores.  m is a
  // reference maximum: it is raised (and l, acc rescaled) only when a row's
  // maximum exceeds it by more than 2^8 in the exponent, so the weights stay
  // below 256 and the rescale is rare; the final division by l is unchanged
  // by the choice of reference.  Branch-free: l is scaled here, and the
  // caller rescales acc by alpha when the result is true.  `valid` false
  // leaves the state unchanged (scores of no block).
  auto settle_max = [&](const f32x4 (&sc)[2][2], bool valid, float (&alpha)[2]) {
    bool raise = false;
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      float mx = fmaxf(fmaxf(fmaxf(sc[qg][0][0], sc[qg][0][1]), fmaxf(sc[qg][0][2], sc[qg][0][3])),
                       fmaxf(fmaxf(sc[qg][1][0], sc[qg][1][1]), fmaxf(sc[qg][1][2], sc[qg][1][3])));
      mx = pair32_max(pair16_max(mx));
      const float mn = fmaxf(m[qg], mx);
      // (mn - m) is NaN while both are -inf: no raise.  Selects rather
      // than branches (the exp is computed either way).
      const bool up = (__ballot((mn - m[qg]) * p.qscale > 8.f) != 0) & valid;
      alpha[qg] = fast_exp2(up ? (m[qg] - mn) * p.qscale : 0.f);  // 0 from m = -inf
      m[qg] = up ? mn : m[qg];
      l[qg] *= alpha[qg];
      raise |= up;
    }
    return raise;
  };
  auto rescale_acc = [&](const float (&alpha)[2]) {
#pragma unroll
    for (int qg = 0; qg < 2; ++qg)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[qg][dt] *= alpha[qg];
  };
  // Software pipeline over the list.  Step j computes the scores of block
  // j+1 while the weights of block j are formed, then block j's PV product
  // while the scores of block j+1 are masked and their maxima settled.  K
  // block x lives in slot x % 2 and V block x in slot 2 + x % 2; both are
  // fetched one step ahead (K of block j+2 and V of block j+1 during step j).
  // List entries come through the scalar cache (see sload_i32).
  const int kb = sload_i32(list);              // block 0
  int kb1 = n > 1 ? sload_i32(list + 1) : 0;  // block j + 1
  dma_k(kb, 0);
  dma_v(kb, 2);
  if (n > 1) dma_k(kb1, 1);
  wait_vmcnt<0>();
#pragma unroll
  for (int qg = 0; qg < 2; ++qg)
#pragma unroll
    for (int s = 0; s < 4; ++s) settle(qreg[qg][s]);  // q landed with the first blocks
  lds_barrier();
  {
    const bool c0 = !whole_block(kb), c1 = n > 1 && !whole_block(kb1);
    if (c0) {
      clear_rows(kb, 0);
      clear_rows(kb, 2);
    }
    if (c1) clear_rows(kb1, 1);
    if (c0 || c1) lds_barrier();
  }
  f32x4 st[2][2];
  scores(0, st);
  apply_mask(kb, st);
  {
    float alpha[2];
    settle_max(st, true, alpha);  // acc is still zero: no rescale
  }
  lds_barrier();  // every wave has read K slot 0 before step 0 refills it

  // Step j: (A) the scores of block j+1 (of a stale slot when j+1 == n:
  // computed, unused) with the weights of block j, then (B) block j's PV
  // product with the maxima of block j+1.  Both halves are one branch-free
  // block whose matrix and vector instructions are interleaved
  // (sched_group_barrier), so that each wave keeps the matrix core and the
  // VALU busy at once.
  auto step = [&](int j, const int par) {
    const int kb2 = j + 2 < n ? sload_i32(list + j + 2) : 0;
    if (j + 2 < n) dma_k(kb2, par);            // held block j (scored a step ago)
    if (j + 1 < n) dma_v(kb1, 2 + (par ^ 1));  // held block j-1 (multiplied)
    f32x4 sn[2][2];
    scores(par ^ 1, sn);
    apply_mask(kb1, sn);
    // P = P_hi + P_lo in bf16 (P_lo = bf16(P - P_hi)): the product keeps ~16
    // mantissa bits of each weight, so bf16 rounding of P costs ~2^-17
    // relative instead of 2^-9 (which alone exceeds 2e-3 on rows whose mass
    // sits on a few keys).  Column c16 is this lane's query; the positive
    // scale commutes with the max, so it is applied in the exponent.
    bf16x8 ph[2], pl[2];
#pragma unroll
    for (int qg = 0; qg < 2; ++qg) {
      const float mu = (m[qg] == __int_as_float(0xff800000)) ? 0.f : m[qg] * p.qscale;
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
    const uint16_t *sv = smem + (2 + par) * PF_BLK;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      // V^T rows through the LDS transpose read: lane (g, j) of a 16-lane group
      // gets V[k0 + e][16 dt + j], e < 4, when lane i of the group points at
      // row k0 + i/4, columns 16 dt + 4 (i%4) .. +3
      const uint16_t *v0 = sv + voffs[dt];
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)v0);
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(v0 + 16 * PF_D));
      const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int qg = 0; qg < 2; ++qg) {
        acc[qg][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ph[qg], acc[qg][dt], 0, 0, 0);
        acc[qg][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pl[qg], acc[qg][dt], 0, 0, 0);
      }
    }
    float alpha[2];
    const bool raise = settle_max(sn, j + 1 < n, alpha);
    // order within the block: K reads, then the 16 score MFMAs each followed
    // by weight VALU work, then V reads, then the 32 PV MFMAs each followed
    // by VALU work of the next block's mask and maxima
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
    }
    if (raise) rescale_acc(alpha);
#pragma unroll
    for (int qg = 0; qg < 2; ++qg)
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2) st[qg][kt2] = sn[qg][kt2];
    // this wave's loads have landed and every wave is done with the slots
    // that the next step refills
    wait_vmcnt<0>();
    lds_barrier();
    const bool ck = j + 2 < n && !whole_block(kb2), cv = j + 1 < n && !whole_block(kb1);
    if (ck) clear_rows(kb2, par);
    if (cv) clear_rows(kb1, 2 + (par ^ 1));
    if (ck || cv) lds_barrier();
    kb1 = kb2;
  };
  for (int j = 0; j < n; j += 2) {
    step(j, 0);
    if (j + 1 >= n) break;
    step(j + 1, 1);
  }
  // l is a per-lane partial over this lane's keys; sum the 4 lane groups.
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    l[qg] = pair32_sum(pair16_sum(l[qg]));
  }
  // Merge the two key halves: the kh = 1 wave of each query half hands its
  // state to the kh = 0 wave through LDS (the staging buffers are free now).
  float *red = (float *)smem + qh * (2 * 128 * 16 + 64);
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
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        r[e] = (acc[qg][dt][e] * a1 + red_o[(qg * 128 + 16 * dt + 4 * g + e) * 16 + c16] * a2) * inv;
      store4(qg, dt, r);
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
  LA_REQUIRE(a->T < ((int64_t)1 << 30), "la_block_sparse_prefill: T must be below 2^30");
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
