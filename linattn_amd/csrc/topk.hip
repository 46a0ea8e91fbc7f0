// Row-wise top-k on gfx950: one workgroup (4 wave64) per row group.
//
// Selection is a radix select over a 64-bit order-preserving image of the fp64
// scores (8 passes of 8 bits, MSB first, stopping as soon as the threshold
// bucket is taken whole), followed by an index-ordered compaction in which
// threshold ties are taken lowest index first.  The k survivors are then
// either bitonic-sorted by (score desc, index asc) in LDS or OR'd into a
// bitmap (GQA union, sink, window) and emitted in ascending index order.
//
// Replaces the torch.topk selections of topk_blocks (variants/selection.py:51-59),
// QuestAttention.page_selection (selection.py:214-237), page_select_torch
// (kernels/triton/quest_pages.py:58-78) and indexer_topk_torch
// (kernels/triton/fused_indexer.py:63-73).  torch.topk leaves tie order
// unspecified; here ties go to the lowest index.
#include <algorithm>

#include "topk.h"
#include "topk_select.h"

namespace la {

constexpr int TK_BATCH = 8;  // keys read per thread before they are used
// bucket ranking of the sorted form: TKB_N key buckets (+ forced and tie
// buckets), scanned TKB_PT per thread; TKB_MAX survivors per bucket at most
constexpr int TKB_BITS = 11, TKB_N = 1 << TKB_BITS, TKB_PT = 9, TKB_S = TKB_PT * 256;
constexpr int TKB_MAX = 256;
// undecided keys the bitwise search copies to LDS once that few remain
constexpr int TK_CAND_CAP = 128;

struct TkShared {
  uint32_t hist[256];
  uint32_t wtmp[2][TK_NW];
  uint32_t sel_bin, above, bin_cnt;
};

struct RowKeys {
  const double *row;
  const uint64_t *lds;
  int64_t own;
  bool force;
  __device__ __forceinline__ uint64_t operator()(int64_t i) const {
    if (lds) return lds[i];
    if (force && i == own) return KEY_FORCED;
    return ord_key(row[i]);
  }
  // "x precedes y": higher key first, lower index on equal keys; -1 is last.
  __device__ __forceinline__ bool before(int32_t x, int32_t y) const {
    if (x < 0) return false;
    if (y < 0) return true;
    const uint64_t kx = (*this)(x), ky = (*this)(y);
    return kx > ky || (kx == ky && x < y);
  }
};

// Selects the top K of keys [0, n_v) and calls emit(index, position) for each,
// positions 0..K-1 in increasing index order.  Collective over the workgroup.
template <class Emit>
__device__ void tk_select(const RowKeys &key, int64_t n_v, int64_t K, TkShared &sh, Emit emit) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (K <= 0) return;
  uint64_t prefix = 0, mask = 0;
  uint32_t need = (uint32_t)K;
  bool all_in = true;
  if (K < n_v) {
    all_in = false;
    for (int shift = 56; shift >= 0; shift -= 8) {
      sh.hist[tid] = 0;
      __syncthreads();
      // TK_BATCH keys per thread are read before any is counted (memory-level
      // parallelism when the keys come from global memory)
      for (int64_t base = tid; base < n_v; base += TK_NT * TK_BATCH) {
        uint64_t u[TK_BATCH];
#pragma unroll
        for (int e = 0; e < TK_BATCH; ++e) {
          const int64_t i = base + e * TK_NT;
          u[e] = i < n_v ? key(i) : 0ull;
        }
#pragma unroll
        for (int e = 0; e < TK_BATCH; ++e) {
          const int64_t i = base + e * TK_NT;
          if (i < n_v && (u[e] & mask) == prefix) atomicAdd(&sh.hist[(u[e] >> shift) & 255u], 1u);
        }
      }
      __syncthreads();
      const uint32_t c = sh.hist[255 - tid];
      uint32_t tot;
      const uint32_t incl = tk_block_incl_scan(c, sh.wtmp[0], tot);
      if (incl >= need && incl - c < need) {
        sh.sel_bin = 255 - tid;
        sh.above = incl - c;
        sh.bin_cnt = c;
      }
      __syncthreads();
      need -= sh.above;
      prefix |= (uint64_t)sh.sel_bin << shift;
      mask |= 0xffull << shift;
      const bool done = (sh.bin_cnt == need);
      __syncthreads();
      if (done) {
        all_in = true;
        break;
      }
    }
  }
  // Index-ordered compaction; wave w owns a contiguous index range.
  const int64_t per = ((n_v + TK_NW - 1) / TK_NW + 63) / 64 * 64;
  const int64_t beg = (int64_t)w * per;
  const int64_t end = min(n_v, beg + per);
  uint32_t c_gt = 0, c_eq = 0;
  for (int64_t base = beg + lane; base < end; base += 64 * TK_BATCH) {
    uint64_t u[TK_BATCH];
#pragma unroll
    for (int e = 0; e < TK_BATCH; ++e) {
      const int64_t i = base + e * 64;
      u[e] = i < end ? key(i) : 0ull;
    }
#pragma unroll
    for (int e = 0; e < TK_BATCH; ++e) {
      const int64_t i = base + e * 64;
      const uint64_t um = u[e] & mask;
      c_gt += (i < end) && um > prefix;
      c_eq += (i < end) && um == prefix;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    c_gt += __shfl_xor(c_gt, off, 64);
    c_eq += __shfl_xor(c_eq, off, 64);
  }
  if (lane == 0) {
    sh.wtmp[0][w] = c_eq;
    sh.wtmp[1][w] = c_gt;
  }
  __syncthreads();
  uint32_t eq_acc = 0, eq_before = 0, sel_before = 0;
#pragma unroll
  for (int x = 0; x < TK_NW; ++x) {
    const uint32_t e = sh.wtmp[0][x], g = sh.wtmp[1][x];
    const uint32_t take_e = all_in ? e : min(e, need > eq_acc ? need - eq_acc : 0u);
    if (x < w) sel_before += g + take_e;
    if (x == w) eq_before = eq_acc;
    eq_acc += e;
  }
  __syncthreads();
  const uint64_t lt = lanemask_lt(lane);
  uint32_t eq_seen = eq_before, pos = sel_before;
  for (int64_t base0 = beg; base0 < end; base0 += 64 * TK_BATCH) {
    uint64_t u[TK_BATCH];
#pragma unroll
    for (int e = 0; e < TK_BATCH; ++e) {
      const int64_t i = base0 + e * 64 + lane;
      u[e] = i < end ? key(i) : 0ull;
    }
#pragma unroll
    for (int e = 0; e < TK_BATCH; ++e) {
      const int64_t i = base0 + e * 64 + lane;
      const bool valid = i < end;
      const uint64_t um = u[e] & mask;
      const bool is_gt = valid && um > prefix;
      const bool is_eq = valid && um == prefix;
      const uint64_t em = __ballot(is_eq);
      const uint32_t rank = eq_seen + (uint32_t)__popcll(em & lt);
      const bool take = is_gt || (is_eq && (all_in || rank < need));
      const uint64_t tm = __ballot(take);
      if (take) emit(i, pos + (uint32_t)__popcll(tm & lt));
      eq_seen += (uint32_t)__popcll(em);
      pos += (uint32_t)__popcll(tm);
    }
  }
  __syncthreads();
}

// the candidate row of a segmented top-k's final level (G = 1), or null
__device__ __forceinline__ const int32_t *tk_cand_row(const TopkKParams &p, const TkRow &rw) {
  return p.cand_idx ? p.cand_idx + ((rw.br / p.Tq) * p.G * p.Tq + rw.tl) * p.row_stride + rw.seg0
                    : nullptr;
}

__device__ __forceinline__ void tk_emit_bitmap(const TopkKParams &p, uint32_t *bm, const TkRow &rw,
                                               uint32_t *wtmp) {
  tk_emit_bitmap_row(bm, rw.n_v, rw.own, p.sink, p.window, p.width, p.out_idx + rw.orow * p.width,
                     p.out_count ? p.out_count + rw.orow : nullptr, wtmp, tk_cand_row(p, rw));
}

__global__ __launch_bounds__(TK_NT) void topk_rows_kernel(TopkKParams p) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ TkShared sh;
  const int tid = threadIdx.x;
  const TkRow rw = tk_row(p, blockIdx.x);
  const int64_t seg0 = rw.seg0, tl = rw.tl, orow = rw.orow, n_v = rw.n_v, own = rw.own, K = rw.K;
  const int64_t br = rw.br;
  const bool force = rw.force;

  unsigned char *ptr = dyn;
  uint64_t *lkeys = nullptr;
  if (p.lds_keys) {
    lkeys = (uint64_t *)ptr;
    ptr += ((p.n_lds * 8 + 15) / 16) * 16;
  }
  int32_t *sel = nullptr;
  uint64_t *skey = nullptr;  // keys of sel[], kept beside them for the sort
  uint32_t *bm = nullptr;
  if (p.use_bitmap) {
    bm = (uint32_t *)ptr;
    for (int64_t i = tid; i < p.bitmap_words; i += TK_NT) bm[i] = 0u;
  } else {
    skey = (uint64_t *)ptr;
    sel = (int32_t *)(ptr + p.p2k * 8);
  }
  __syncthreads();

  for (int64_t j = 0; j < p.G; ++j) {
    const int64_t row = ((br / p.Tq) * p.G + j) * p.Tq + tl;
    const double *rp = p.scores + row * p.row_stride + seg0;
    const int32_t *cand = p.cand_idx ? p.cand_idx + row * p.row_stride + seg0 : nullptr;
    if (lkeys) {
      for (int64_t base = tid; base < n_v; base += TK_NT * TK_BATCH) {
        double v[TK_BATCH];
#pragma unroll
        for (int e = 0; e < TK_BATCH; ++e) {
          const int64_t i = base + e * TK_NT;
          v[e] = i < n_v ? rp[i] : 0.0;
        }
#pragma unroll
        for (int e = 0; e < TK_BATCH; ++e) {
          const int64_t i = base + e * TK_NT;
          if (i < n_v) lkeys[i] = (force && i == own) ? KEY_FORCED : ord_key(v[e]);
        }
      }
      __syncthreads();
    }
    const RowKeys key{rp, lkeys, own, force};
    if (bm) {
      tk_select(key, n_v, K, sh, [&](int64_t i, uint32_t) {
        atomicOr(&bm[i >> 5], 1u << (i & 31));
      });
    } else {
      tk_select(key, n_v, K, sh, [&](int64_t i, uint32_t pos) {
        sel[pos] = (int32_t)i;
        skey[pos] = key(i);
      });
      // Bitonic sort of (skey, sel)[0, p2k) by (key desc, index asc); padding
      // entries (index -1) sort last.  Each thread handles whole pairs.
      for (int64_t i = K + tid; i < p.p2k; i += TK_NT) {
        sel[i] = -1;
        skey[i] = 0;
      }
      __syncthreads();
      const uint32_t half = (uint32_t)(p.p2k >> 1);
      for (uint32_t size = 2; size <= (uint32_t)p.p2k; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
          for (uint32_t jp = tid; jp < half; jp += TK_NT) {
            const uint32_t i = ((jp & ~(stride - 1)) << 1) | (jp & (stride - 1));
            const uint32_t l = i + stride;
            const int32_t a = sel[i], b = sel[l];
            const uint64_t ka = skey[i], kb = skey[l];
            // x precedes y: valid before padding, higher key, then lower index
            const bool b_first = b >= 0 && (a < 0 || kb > ka || (kb == ka && b < a));
            const bool a_first = a >= 0 && (b < 0 || ka > kb || (ka == kb && a < b));
            const bool up = (i & size) == 0;
            if (up ? b_first : a_first) {
              sel[i] = b;
              sel[l] = a;
              skey[i] = kb;
              skey[l] = ka;
            }
          }
          __syncthreads();
        }
      }
      // Candidate rows carry the original index of every slot; padding slots
      // (index -1) hold the lowest key, so they sort after every real one and
      // the first of them ends the list.
      if (tid == 0) sh.above = (uint32_t)K;
      __syncthreads();
      int32_t *oi = p.out_idx + orow * p.width;
      for (int64_t base = tid; base < p.width; base += TK_NT * TK_BATCH) {
        int32_t sl[TK_BATCH], id[TK_BATCH];
#pragma unroll
        for (int e = 0; e < TK_BATCH; ++e) {
          const int64_t jj = base + e * TK_NT;
          sl[e] = jj < K ? sel[jj] : -1;
        }
#pragma unroll
        for (int e = 0; e < TK_BATCH; ++e) id[e] = (cand && sl[e] >= 0) ? cand[sl[e]] : sl[e];
#pragma unroll
        for (int e = 0; e < TK_BATCH; ++e) {
          const int64_t jj = base + e * TK_NT;
          if (jj >= p.width) break;
          if (cand && sl[e] >= 0 && id[e] < 0) {
            sl[e] = -1;
            atomicMin(&sh.above, (uint32_t)jj);
          }
          oi[jj] = id[e];
          if (p.out_val) {
            // the sort keys map back to the exact scores (-0 reads as +0)
            float v = __int_as_float(0xff800000);
            if (sl[e] >= 0)
              v = (force && sl[e] == own) ? __int_as_float(0x7f800000)
                                          : (float)key_to_double(skey[jj]);
            p.out_val[orow * p.width + jj] = v;
          }
        }
      }
      __syncthreads();
      if (p.out_count && tid == 0) p.out_count[orow] = (int32_t)sh.above;
      __syncthreads();
    }
  }
  if (!bm) return;
  tk_emit_bitmap(p, bm, rw, sh.wtmp[1]);
}

// x precedes y: valid before padding (-1), higher key, then lower index.
__device__ __forceinline__ bool tk_precedes(uint64_t kx, int32_t ix, uint64_t ky, int32_t iy) {
  return ix >= 0 && (iy < 0 || kx > ky || (kx == ky && ix < iy));
}

// Bitonic compare-exchange of register pairs (e, e | S) of this thread
// (positions tid*E + e): ascending runs put the preceding element first.
template <int S, int E>
__device__ __forceinline__ void tk_local_stage(uint64_t (&key)[E], int32_t (&idx)[E], int tid,
                                               int size) {
  if constexpr (S < E) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (e & S) continue;
      const int el = e | S;
      const bool up = ((tid * E + e) & size) == 0;
      const bool sw = up ? tk_precedes(key[el], idx[el], key[e], idx[e])
                         : tk_precedes(key[e], idx[e], key[el], idx[el]);
      const uint64_t ka = key[e], kb = key[el];
      const int32_t ia = idx[e], ib = idx[el];
      key[e] = sw ? kb : ka;
      key[el] = sw ? ka : kb;
      idx[e] = sw ? ib : ia;
      idx[el] = sw ? ia : ib;
    }
  }
}

// Sorts 256*E unsigned 64-bit values descending, E per thread (thread t holds
// positions t*E .. t*E + E - 1): bitonic network with in-register, in-wave
// (shuffle) and cross-wave (LDS, `buf` of 256*E values) stages.
template <int S, int E>
__device__ __forceinline__ void tk_local_desc(uint64_t (&c)[E], int tid, int size) {
  if constexpr (S < E) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (e & S) continue;
      const int el = e | S;
      const bool down = ((tid * E + e) & size) == 0;  // descending run
      const uint64_t a = c[e], b = c[el];
      const bool sw = down ? (b > a) : (a > b);
      c[e] = sw ? b : a;
      c[el] = sw ? a : b;
    }
  }
}

template <int E>
__device__ __forceinline__ void tk_bitonic_desc(uint64_t (&c)[E], int tid, uint64_t *buf) {
  constexpr int P = TK_NT * E;
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride < E) {
        switch (stride) {
          case 1: tk_local_desc<1, E>(c, tid, size); break;
          case 2: tk_local_desc<2, E>(c, tid, size); break;
          case 4: tk_local_desc<4, E>(c, tid, size); break;
          case 8: tk_local_desc<8, E>(c, tid, size); break;
          default: break;
        }
      } else if (stride < 64 * E) {
        const int lx = stride / E;
        // position i keeps the larger of the pair when it is the lower one of
        // a descending run (or the upper one of an ascending run)
        const int i0 = tid * E;
        const bool keep_max = (((i0 & stride) == 0) == ((i0 & size) == 0));
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const uint64_t pc = __shfl_xor(c[e], lx, 64);
          c[e] = keep_max ? (pc > c[e] ? pc : c[e]) : (pc < c[e] ? pc : c[e]);
        }
      } else {
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E; ++e) buf[tid * E + e] = c[e];
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int i = tid * E + e;
          const uint64_t pc = buf[i ^ stride];
          const bool keep_max = (((i & stride) == 0) == ((i & size) == 0));
          c[e] = keep_max ? (pc > c[e] ? pc : c[e]) : (pc < c[e] ? pc : c[e]);
        }
      }
    }
  }
  __syncthreads();
}

// Register-resident top-k for rows of at most 256*KPT keys (thread t holds
// the keys of units t + 256*j).  Selection is the radix select above, started
// at the highest bit where the row's valid keys differ (common leading bits
// cost no pass), with per-wave histograms.  The survivors are either OR'd
// into a bitmap (BITMAP: unions, sink, window, index order) or sorted by
// (key desc, index asc) with a bitonic network over E registers per thread:
// partners in the same thread are swapped in place, in other lanes of the
// wave they are exchanged by shuffles, in other waves through LDS.
// Sorted rows of the longest kind (KPT 32: the indexer's) are held to four
// waves per SIMD (128 registers, 16 of them spilled; 40 KiB of LDS each, so
// four workgroups fill a CU's LDS): their steps are short and barrier-bound,
// so every further resident workgroup per CU pays (the whole C2 indexer call
// took 0.767 ms with two per CU, 0.630 with three, 0.609 with four).
template <int KPT, int E, bool BITMAP>
__global__ __launch_bounds__(TK_NT, (!BITMAP && KPT >= 32) ? 4 : 1) void topk_reg_kernel(TopkKParams p) {
  constexpr int P = TK_NT * E;  // sort width (sorted form)
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ TkRegShared<KPT> sr;
  __shared__ uint32_t s_fill, s_first_pad;
  __shared__ uint32_t s_bins[BITMAP ? 1 : TKB_S + 1];  // sorted form: bucket counts / starts
  __shared__ uint64_t s_red2[TK_NW], s_red3[TK_NW];
  __shared__ uint32_t s_tie[BITMAP ? 1 : 2 * 256];  // sorted form: tie-bucket index bits, prefixes

  const int tid = threadIdx.x, lane = tid & 63;
  const uint64_t lt = lanemask_lt(lane);
  // groups taken last first: in causal rows the valid prefix grows with the
  // group, so the longest rows start first and the short ones fill the tail
  const TkRow rw = tk_row(p, (int64_t)gridDim.x - 1 - blockIdx.x);
  const int32_t n_v = (int32_t)rw.n_v;  // n_v <= 256*KPT
  const int32_t own = (int32_t)rw.own;
  uint32_t *bm = nullptr;
  uint64_t *skey = nullptr;
  int32_t *sidx = nullptr;
  if constexpr (BITMAP) {
    bm = (uint32_t *)dyn;
    for (int64_t i = tid; i < p.bitmap_words; i += TK_NT) bm[i] = 0u;
  } else {
    skey = (uint64_t *)dyn;
    sidx = (int32_t *)(dyn + (size_t)P * 8);
  }
  if (tid == 0) s_fill = 0;
  __syncthreads();
  // the scores of the (single) row of the sorted form
  const double *rp_row = p.scores + ((rw.br / p.Tq) * p.G * p.Tq + rw.tl) * p.row_stride + rw.seg0;

  // the sorted form has one row per group (bitmap rows take the GQA groups):
  // no loop there, so nothing of the row's loads is kept across iterations
  const int64_t n_groups = BITMAP ? p.G : 1;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t row = ((rw.br / p.Tq) * p.G + g) * p.Tq + rw.tl;
    const double *rp = p.scores + row * p.row_stride + rw.seg0;
    // raw fp64 bits, mapped in place to order keys (ord_key: -0 reads as +0)
    uint64_t u[KPT];
    const uint64_t *rb = (const uint64_t *)rp;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int32_t i = tid + TK_NT * j;
      u[j] = i < n_v ? __builtin_nontemporal_load(rb + i) : 0ull;  // read once
    }
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int32_t i = tid + TK_NT * j;
      uint64_t x = (u[j] << 1) == 0 ? 0ull : u[j];
      x = (x >> 63) ? ~x : (x | 0x8000000000000000ull);
      u[j] = (rw.force && i == own) ? KEY_FORCED : x;
    }
    const uint32_t K = (uint32_t)rw.K;
    // bitmap rows (segments and unions, few rows in flight) keep the radix
    // select, which takes fewer barrier steps; sorted rows (many in flight)
    // use the bitwise search, which issues fewer instructions
    if constexpr (BITMAP) {
      tk_reg_select<KPT>(u, n_v, K, sr, [&](int j, int32_t i, bool take) {
        if (take) atomicOr(&bm[i >> 5], 1u << (i & 31));
      });
    } else {
      static_assert(KPT <= 32, "take flags in one word");
      uint32_t takem = 0;  // bit j: slot j selected
      tk_reg_select_bits<KPT>(
          u, n_v, K, sr, [&](int j, int32_t, bool take) { takem |= take ? (1u << j) : 0u; },
          skey, (uint32_t)min(P, TK_CAND_CAP));
      // the selected keys to skey / sidx[0, K): one place reservation per wave
      uint32_t wcnt = 0;
#pragma unroll
      for (int j = 0; j < KPT; ++j) wcnt += (uint32_t)__popcll(__ballot((takem >> j) & 1u));
      uint32_t base = 0;
      if (lane == 0 && wcnt) base = atomicAdd(&s_fill, wcnt);
      base = __shfl(base, 0, 64);
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const bool take = (takem >> j) & 1u;
        const uint64_t tm = __ballot(take);
        if (take) {
          const uint32_t q = base + (uint32_t)__popcll(tm & lt);
          skey[q] = u[j];
          sidx[q] = tid + TK_NT * j;
        }
        base += (uint32_t)__popcll(tm);
      }
      __syncthreads();
    }
  }
  if constexpr (BITMAP) {
    tk_emit_bitmap(p, bm, rw, sr.wtmp[1]);
  } else {
    static_assert(BITMAP || KPT <= 32, "sorted form: row indices below 8192 (tie bits)");
    // Sorted form (one row per workgroup): the K selected keys (skey / sidx,
    // in any order) are ranked by (key desc, index asc).  A counting pass
    // spreads them over buckets of their key range -- bucket 0 for a forced
    // key, then TKB_N buckets of equal key width from the largest other key
    // down to the smallest key above the minimum, and a last bucket for the
    // keys equal to the minimum (ties such as zero scores) -- and copies them
    // back in bucket order; each then counts the keys of its own bucket that
    // precede it, and the ranked (index, value) pairs leave through LDS in
    // order.  Order keys grow with the score's exponent as well as its
    // mantissa, so scores spread over many binades still fill many buckets.
    // When the range holds both signs, the buckets are laid over a signed
    // magnitude image instead (exponent and mantissa bits, clamped 24 binades
    // below the largest magnitude), so that the 2000 binades of tiny
    // magnitudes around zero take no buckets.  A row whose largest bucket
    // still holds more than TKB_MAX keys takes the bitonic sort below.
    const int32_t K = (int32_t)rw.K;
    const int w = tid >> 6;
    const int32_t *cand = p.cand_idx ? p.cand_idx + ((rw.br / p.Tq) * p.G * p.Tq + rw.tl) * p.row_stride + rw.seg0 : nullptr;
    int32_t *oi = p.out_idx + rw.orow * p.width;
    if (tid == 0) s_first_pad = (uint32_t)K;
    // magnitude bits (exponent, mantissa) of the score behind an order key
    constexpr uint64_t MAG = 0x7fffffffffffffffull;
    auto mag = [](uint64_t k) -> uint64_t { return (k >> 63) ? (k & MAG) : (~k & MAG); };
    uint64_t bkey[E];
    int32_t bidx[E];
    uint64_t mx = 0, mn = ~0ull;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid + TK_NT * e;
      bkey[e] = i < K ? skey[i] : 0ull;
      bidx[e] = i < K ? sidx[i] : -1;
      if (bidx[e] >= 0) {
        if (bkey[e] != KEY_FORCED) mx = max(mx, bkey[e]);
        mn = min(mn, bkey[e]);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      mx = max(mx, (uint64_t)__shfl_xor(mx, off, 64));
      mn = min(mn, (uint64_t)__shfl_xor(mn, off, 64));
    }
    if (lane == 0) {
      sr.red[0][w] = mx;
      sr.red[1][w] = mn;
    }
    for (int b = tid; b <= TKB_S; b += TK_NT) s_bins[b] = 0u;
    s_tie[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int x = 0; x < TK_NW; ++x) {
      mx = max(mx, sr.red[0][x]);
      mn = min(mn, sr.red[1][x]);
    }
    // over the keys above the minimum (other than a forced key): the smallest
    // one and the largest magnitude
    uint64_t mn2 = ~0ull, emax = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (bidx[e] >= 0 && bkey[e] > mn && bkey[e] != KEY_FORCED) {
        mn2 = min(mn2, bkey[e]);
        emax = max(emax, mag(bkey[e]));
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      mn2 = min(mn2, (uint64_t)__shfl_xor(mn2, off, 64));
      emax = max(emax, (uint64_t)__shfl_xor(emax, off, 64));
    }
    if (lane == 0) {
      s_red2[w] = mn2;
      s_red3[w] = emax;
    }
    __syncthreads();
#pragma unroll
    for (int x = 0; x < TK_NW; ++x) {
      mn2 = min(mn2, s_red2[x]);
      emax = max(emax, s_red3[x]);
    }
    // the bucket image: the key itself, or over a range of both signs the
    // signed magnitude above a floor 24 binades below the largest
    const bool mixed = mn2 <= mx && ((mn2 ^ mx) >> 63) != 0;
    const uint64_t floor_m = (emax >> 52) >= 24 ? ((emax >> 52) - 24) << 52 : 0ull;
    auto img = [&](uint64_t k) -> uint64_t {
      if (!mixed) return k;
      const uint64_t dm = max(mag(k), floor_m) - floor_m;
      return (k >> 63) ? (0x8000000000000000ull + dm) : (0x8000000000000000ull - dm);
    };
    const uint64_t tmx = img(mx);
    const uint64_t range = mn2 <= mx ? tmx - img(mn2) : 0ull;
    const int nbits = range ? 64 - __clzll((long long)range) : 0;
    const int shift = nbits > TKB_BITS ? nbits - TKB_BITS : 0;
    auto bucket = [&](uint64_t k) -> uint32_t {
      return k == KEY_FORCED ? 0u : k == mn ? (uint32_t)TKB_N + 1u : 1u + (uint32_t)((tmx - img(k)) >> shift);
    };
    uint32_t bk[E], slot[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (bidx[e] >= 0) {
        bk[e] = bucket(bkey[e]);
        slot[e] = atomicAdd(&s_bins[bk[e]], 1u);
        if (bk[e] == (uint32_t)TKB_N + 1u) atomicOr(&s_tie[bidx[e] >> 5], 1u << (bidx[e] & 31));
      }
    }
    __syncthreads();
    // keys tied at the minimum rank by index: prefix counts of the tie bits
    {
      const uint32_t wbits = s_tie[tid];
      uint32_t tot_t;
      const uint32_t pc = (uint32_t)__popc(wbits);
      s_tie[256 + tid] = tk_block_incl_scan(pc, sr.wtmp[0], tot_t) - pc;
    }
    // bucket starts (exclusive scan, TKB_PT bins per thread) and the largest bucket
    uint32_t c9[TKB_PT], loc = 0, big = 0;
#pragma unroll
    for (int i = 0; i < TKB_PT; ++i) {
      c9[i] = s_bins[TKB_PT * tid + i];
      loc += c9[i];
      if (TKB_PT * tid + i != TKB_N + 1) big = max(big, c9[i]);  // (the tie bucket: by index)
    }
    uint32_t tot_b;
    uint32_t run = tk_block_incl_scan(loc, sr.wtmp[0], tot_b) - loc;
#pragma unroll
    for (int i = 0; i < TKB_PT; ++i) {
      s_bins[TKB_PT * tid + i] = run;
      run += c9[i];
    }
    if (tid == 0) s_bins[TKB_S] = (uint32_t)K;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) big = max(big, (uint32_t)__shfl_xor(big, off, 64));
    if (lane == 0) sr.wtmp[1][w] = big;
    __syncthreads();
#pragma unroll
    for (int x = 0; x < TK_NW; ++x) big = max(big, sr.wtmp[1][x]);
    if (big <= (uint32_t)TKB_MAX) {
      // bucket order in skey / sidx, then the rank within the bucket
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if (bidx[e] >= 0) {
          const uint32_t j = s_bins[bk[e]] + slot[e];
          skey[j] = bkey[e];
          sidx[j] = bidx[e];
        }
      }
      __syncthreads();
      // thread t now ranks the keys at bucket-order positions t + 256 e: the
      // 64 lanes of a wave take neighbouring buckets, of similar sizes, so
      // the rank loops below diverge less than over keys in arrival order
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int i = tid + TK_NT * e;
        bkey[e] = i < K ? skey[i] : 0ull;
        bidx[e] = i < K ? sidx[i] : -1;
        bk[e] = i < K ? bucket(bkey[e]) : 0u;
      }
      uint32_t pos[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if (bidx[e] < 0) continue;
        const uint32_t b0 = s_bins[bk[e]], b1 = s_bins[bk[e] + 1];
        uint32_t r = 0;
        if (bk[e] == (uint32_t)TKB_N + 1u) {
          const int32_t ix = bidx[e];
          r = s_tie[256 + (ix >> 5)] + (uint32_t)__popc(s_tie[ix >> 5] & ((1u << (ix & 31)) - 1u));
        } else {
          for (uint32_t j = b0; j < b1; ++j) r += tk_precedes(skey[j], sidx[j], bkey[e], bidx[e]) ? 1u : 0u;
        }
        pos[e] = b0 + r;
      }
      __syncthreads();  // every bucket is read before the ranked pairs overwrite it
      // (output index, value bits) at each rank in skey, then written out in order
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if (bidx[e] < 0) continue;
        const int32_t s0 = bidx[e];
        const int32_t id = cand ? cand[s0] : s0;
        const bool pad = cand && id < 0;
        if (pad) atomicMin(&s_first_pad, pos[e]);
        const float v = pad ? __int_as_float(0xff800000)
                            : (rw.force && s0 == own) ? __int_as_float(0x7f800000)
                                                       : (float)key_to_double(bkey[e]);
        skey[pos[e]] = (uint64_t)(uint32_t)id | ((uint64_t)__float_as_uint(v) << 32);
      }
      __syncthreads();
      const int64_t kw = min((int64_t)K, p.width);
      for (int64_t jj = tid; jj < p.width; jj += TK_NT) {
        const uint64_t x = jj < kw ? skey[jj] : 0xff800000ffffffffull;  // -1, -inf past K
        // streamed out (nontemporal): the lists are not read again here
        __builtin_nontemporal_store((int32_t)(uint32_t)x, oi + jj);
        if (p.out_val)
          __builtin_nontemporal_store(__uint_as_float((uint32_t)(x >> 32)), p.out_val + rw.orow * p.width + jj);
      }
      __syncthreads();
      if (p.out_count && tid == 0) p.out_count[rw.orow] = (int32_t)s_first_pad;
      return;
    }
    // Bitonic fallback.  The K survivors are first sorted as single 64-bit
    // composites: the key with its low 13 bits replaced by 8191 - index (rows
    // hold at most 8192 units), so one unsigned compare orders them by (key
    // desc, index asc) unless two keys differ only in their low 13 bits.  The
    // result is then checked with the full keys (re-read from the row) and,
    // if any neighbouring pair is out of order, sorted again on (key, index).
    for (int32_t i = K + tid; i < P; i += TK_NT) {
      skey[i] = 0;
      sidx[i] = -1;
    }
    if (tid == 0) {
      s_first_pad = (uint32_t)K;
      s_fill = 0;  // reused as the order-violation flag
    }
    __syncthreads();
    uint64_t c[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint64_t k0 = skey[tid * E + e];
      const int32_t i0 = sidx[tid * E + e];
      c[e] = i0 >= 0 ? ((k0 & ~0x1FFFull) | (uint64_t)(0x1FFF - i0)) : 0ull;
    }
    tk_bitonic_desc<E>(c, tid, skey);
    uint64_t key[E];
    int32_t idx[E];
    {
      double v[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        idx[e] = c[e] ? 0x1FFF - (int32_t)(c[e] & 0x1FFF) : -1;
        v[e] = idx[e] >= 0 ? rp_row[idx[e]] : 0.0;
      }
#pragma unroll
      for (int e = 0; e < E; ++e)
        key[e] = idx[e] < 0 ? 0ull : (rw.force && idx[e] == own) ? KEY_FORCED : ord_key(v[e]);
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      skey[tid * E + e] = key[e];
      sidx[tid * E + e] = idx[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid * E + e;
      if (i + 1 < K && !tk_precedes(key[e], idx[e], skey[i + 1], sidx[i + 1])) atomicOr(&s_fill, 1u);
    }
    __syncthreads();
    const auto precedes = tk_precedes;
    // position i keeps, of itself and its partner, the one that comes first
    // (ascending run) or last (descending run)
    auto exchange = [&](int e, int i, int size, int stride, uint64_t pk, int32_t pi) {
      const bool lower = (i & stride) == 0, up = (i & size) == 0;
      const bool want_first = lower == up;
      const bool take = want_first ? precedes(pk, pi, key[e], idx[e]) : precedes(key[e], idx[e], pk, pi);
      if (take) {
        key[e] = pk;
        idx[e] = pi;
      }
    };
    if (s_fill) {  // exact (key, index) sort; rare
      for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          if (stride < E) {
            // partner in the same thread: constant register indices per stride
            switch (stride) {
              case 1: tk_local_stage<1, E>(key, idx, tid, size); break;
              case 2: tk_local_stage<2, E>(key, idx, tid, size); break;
              case 4: tk_local_stage<4, E>(key, idx, tid, size); break;
              case 8: tk_local_stage<8, E>(key, idx, tid, size); break;
              default: break;
            }
          } else if (stride < 64 * E) {
            const int lx = stride / E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
              const uint64_t pk = __shfl_xor(key[e], lx, 64);
              const int32_t pi = __shfl_xor(idx[e], lx, 64);
              exchange(e, tid * E + e, size, stride, pk, pi);
            }
          } else {
            __syncthreads();
#pragma unroll
            for (int e = 0; e < E; ++e) {
              skey[tid * E + e] = key[e];
              sidx[tid * E + e] = idx[e];
            }
            __syncthreads();
#pragma unroll
            for (int e = 0; e < E; ++e) {
              const int i = tid * E + e;
              exchange(e, i, size, stride, skey[i ^ stride], sidx[i ^ stride]);
            }
          }
        }
      }
    }
    int32_t id[E];
#pragma unroll
    for (int e = 0; e < E; ++e) id[e] = (cand && idx[e] >= 0) ? cand[idx[e]] : idx[e];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int64_t jj = (int64_t)tid * E + e;
      if (jj >= p.width) break;
      int32_t s = idx[e];
      if (cand && s >= 0 && id[e] < 0) {
        s = -1;
        atomicMin(&s_first_pad, (uint32_t)jj);
      }
      oi[jj] = id[e];
      if (p.out_val) {
        float v = __int_as_float(0xff800000);
        if (s >= 0)
          v = (rw.force && s == own) ? __int_as_float(0x7f800000) : (float)key_to_double(key[e]);
        p.out_val[rw.orow * p.width + jj] = v;
      }
    }
    for (int64_t jj = P + tid; jj < p.width; jj += TK_NT) {
      oi[jj] = -1;
      if (p.out_val) p.out_val[rw.orow * p.width + jj] = __int_as_float(0xff800000);
    }
    __syncthreads();
    if (p.out_count && tid == 0) p.out_count[rw.orow] = (int32_t)s_first_pad;
  }
}

// Short rows in the bitmap form (unions, sink, window): one wave per output
// row, four rows per workgroup, no workgroup barrier.  The wave holds the
// keys of units lane + 64*j (j < KPL, rows of at most 64*KPL units), selects
// each source row with tk_wave_select_bits, ORs the ballots of kept units into its
// own bitmap words, adds sink and window, and writes the kept units in
// ascending order.
template <int KPL>
__global__ __launch_bounds__(TK_NT) void topk_wave_kernel(TopkKParams p) {
  constexpr int WORDS = 2 * KPL;  // 32-bit bitmap words per row
  __shared__ uint32_t bms[TK_NW][WORDS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t gi = (int64_t)blockIdx.x * TK_NW + w;
  if (gi >= p.NG) return;  // whole wave: no barrier follows
  const TkRow rw = tk_row(p, gi);
  const int32_t n_v = (int32_t)rw.n_v;
  const int32_t own = (int32_t)rw.own;
  uint32_t *bm = bms[w];
  for (int i = lane; i < WORDS; i += 64) bm[i] = 0u;
  __builtin_amdgcn_wave_barrier();
  const uint32_t K = (uint32_t)rw.K;
  for (int64_t g = 0; g < p.G; ++g) {
    const int64_t row = ((rw.br / p.Tq) * p.G + g) * p.Tq + rw.tl;
    const uint64_t *rb = (const uint64_t *)(p.scores + row * p.row_stride + rw.seg0);
    uint64_t u[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) u[j] = lane + 64 * j < n_v ? rb[lane + 64 * j] : 0ull;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int32_t i = lane + 64 * j;
      uint64_t x = (u[j] << 1) == 0 ? 0ull : u[j];  // ord_key of the raw bits
      x = (x >> 63) ? ~x : (x | 0x8000000000000000ull);
      u[j] = (rw.force && i == own) ? KEY_FORCED : x;
    }
    tk_wave_select_bits<KPL>(u, n_v, K, [&](int j, int32_t i, bool take) {
      const uint64_t b = __ballot(take);
      if (lane == 0) {
        bm[2 * j] |= (uint32_t)b;
        bm[2 * j + 1] |= (uint32_t)(b >> 32);
      }
    });
    __builtin_amdgcn_wave_barrier();
  }
  // sink and window units
  if (n_v > 0) {
    const int64_t s_end = min(p.sink, (int64_t)n_v);
    for (int64_t i = lane; i < s_end; i += 64) atomicOr(&bm[i >> 5], 1u << (i & 31));
    if (p.window > 0 && own >= 0) {
      const int64_t w0 = max((int64_t)0, (int64_t)own - p.window + 1);
      const int64_t w1 = min((int64_t)own, (int64_t)n_v - 1);
      for (int64_t i = w0 + lane; i <= w1; i += 64) atomicOr(&bm[i >> 5], 1u << (i & 31));
    }
  }
  __builtin_amdgcn_wave_barrier();
  // ascending emission: lane x < WORDS owns word x (units past n_v are never
  // set); candidate rows drop slots without a candidate and write cand[i]
  const int32_t *cand = tk_cand_row(p, rw);
  uint32_t word = lane < WORDS ? bm[lane] : 0u;
  if (cand) {
    uint32_t bits = word;
    while (bits) {
      const int bb = __ffs(bits) - 1;
      if (cand[lane * 32 + bb] < 0) word &= ~(1u << bb);
      bits &= bits - 1;
    }
  }
  const uint32_t cnt = (uint32_t)__popc(word);
  uint32_t incl = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  const uint32_t total = __shfl(incl, 63, 64);
  uint32_t pos = incl - cnt;
  int32_t *oi = p.out_idx + rw.orow * p.width;
  uint32_t bits = word;
  while (bits) {
    const int bb = __ffs(bits) - 1;
    if (pos < (uint32_t)p.width) oi[pos] = cand ? cand[lane * 32 + bb] : (int32_t)(lane * 32 + bb);
    ++pos;
    bits &= bits - 1;
  }
  for (int64_t jj = (int64_t)total + lane; jj < p.width; jj += 64) oi[jj] = -1;
  if (p.out_count && lane == 0) p.out_count[rw.orow] = (int32_t)min((int64_t)total, p.width);
}

static int64_t align16(int64_t x) { return (x + 15) / 16 * 16; }

int64_t topk_lds_bytes(const TopkKParams &p) {
  int64_t b = 0;
  if (p.lds_keys) b += align16(p.n_lds * 8);
  if (p.use_bitmap)
    b += align16(p.bitmap_words * 4);
  else
    b += align16(p.p2k * 12);
  return b;
}

static int max_dynamic_lds() {
  static int cached = -1;
  if (cached < 0) {
    int dev = 0, v = 65536;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess) {
      cached = v;
    } else {
      cached = 65536;
    }
  }
  return cached;
}

static int64_t lds_limit() { return (int64_t)max_dynamic_lds() - (int64_t)sizeof(TkShared) - 256; }

// Plain rows (sorted or index-order rows of one head with no extras) too long
// for one workgroup's LDS go to the multi-workgroup radix select
// (topk_radix.hip).
static bool long_plain(const TopkKParams &p) {
  const bool plain = p.G == 1 && p.sink == 0 && p.window == 0 && (p.order == 0 || p.order == 1) &&
                     !p.force_own && !p.cand_idx && p.seg_len == 0;
  int64_t p2 = 1;
  while (p2 < p.k) p2 <<= 1;
  return plain && p.n * 8 + p2 * 12 + 64 > lds_limit();
}

RadixPlan topk_long_plan(const TopkKParams &p) {
  return long_plain(p) ? radix_plan(p) : RadixPlan{};
}

int64_t topk_workspace_bytes(const TopkKParams &p) {
  if (long_plain(p)) {
    const RadixPlan R = radix_plan(p);
    if (R.C > 0) return R.bytes;
  }
  return 0;
}

int topk_launch_ws(TopkKParams p, void *ws, int64_t ws_bytes, hipStream_t st) {
  if (p.NG <= 0) return LA_OK;
  if (long_plain(p)) {
    const RadixPlan R = radix_plan(p);
    if (R.C <= 0) return fail(LA_ERR_UNSUPPORTED, "topk: rows of 2^31 or more keys");
    if (!ws || ws_bytes < R.bytes)
      return fail(LA_ERR_WORKSPACE, "topk: long rows need %lld workspace bytes",
                  (long long)R.bytes);
    return topk_radix_launch(p, R, ws, st);
  }
  return topk_launch(p, st);
}

template <bool BITMAP, int KPT>
static int launch_reg_e(const TopkKParams &p, int E, size_t bytes, hipStream_t st) {
  const dim3 grid((unsigned)p.NG);
  if constexpr (BITMAP) {
    topk_reg_kernel<KPT, 1, true><<<grid, TK_NT, bytes, st>>>(p);
  } else {
    switch (E) {
      case 1: topk_reg_kernel<KPT, 1, false><<<grid, TK_NT, bytes, st>>>(p); break;
      case 2: if constexpr (KPT >= 2) topk_reg_kernel<KPT, 2, false><<<grid, TK_NT, bytes, st>>>(p); break;
      case 4: if constexpr (KPT >= 4) topk_reg_kernel<KPT, 4, false><<<grid, TK_NT, bytes, st>>>(p); break;
      case 8: if constexpr (KPT >= 8) topk_reg_kernel<KPT, 8, false><<<grid, TK_NT, bytes, st>>>(p); break;
      case 16: if constexpr (KPT >= 16) topk_reg_kernel<KPT, 16, false><<<grid, TK_NT, bytes, st>>>(p); break;
      default: return fail(LA_ERR_UNSUPPORTED, "topk: sort width");
    }
  }
  LA_LAUNCHED();
  return LA_OK;
}

// Register-resident form: rows of at most 8192 keys (16384 for the bitmap
// form; a segment's length in segmented mode); sorted output for k up to 4096
// of one row per group.
static int launch_reg(const TopkKParams &p, hipStream_t st) {
  int kpt = 1;
  while (kpt * TK_NT < p.n_lds) kpt <<= 1;
  const int64_t kk = std::min(p.k, p.n_lds);
  int64_t p2 = TK_NT;
  while (p2 < kk) p2 <<= 1;
  const int E = (int)(p2 / TK_NT);
  const size_t bytes = p.use_bitmap ? (size_t)align16(p.bitmap_words * 4) : (size_t)p2 * 12;
#define LA_TKR(B)                                          \
  switch (kpt) {                                           \
    case 1: return launch_reg_e<B, 1>(p, E, bytes, st);   \
    case 2: return launch_reg_e<B, 2>(p, E, bytes, st);   \
    case 4: return launch_reg_e<B, 4>(p, E, bytes, st);   \
    case 8: return launch_reg_e<B, 8>(p, E, bytes, st);   \
    case 16: return launch_reg_e<B, 16>(p, E, bytes, st); \
    case 32: return launch_reg_e<B, 32>(p, E, bytes, st); \
    case 64: if constexpr (B) return launch_reg_e<B, 64>(p, E, bytes, st); break; \
    default: break;                                        \
  }
  if (p.use_bitmap) {
    LA_TKR(true)
  } else {
    LA_TKR(false)
  }
#undef LA_TKR
  return fail(LA_ERR_UNSUPPORTED, "topk: row of %lld keys", (long long)p.n_lds);
}

int topk_launch(TopkKParams p, hipStream_t st) {
  if (p.NG <= 0) return LA_OK;
  p.use_bitmap = (p.G > 1 || p.sink > 0 || p.window > 0 || p.order == 1) ? 1 : 0;
  p.n_lds = p.seg_len > 0 ? std::min(p.seg_len, p.n) : p.n;
  p.bitmap_words = (p.n_lds + 31) / 32;
  int64_t p2 = 1;
  while (p2 < p.k) p2 <<= 1;
  p.p2k = p2;
  // short bitmap rows: one wave per row
  if (p.use_bitmap && p.seg_len == 0 && p.n_lds <= 1024) {
    int kpl = 1;
    while (kpl * 64 < p.n_lds) kpl <<= 1;
    const dim3 grid((unsigned)((p.NG + TK_NW - 1) / TK_NW));
    switch (kpl) {
      case 1: topk_wave_kernel<1><<<grid, TK_NT, 0, st>>>(p); break;
      case 2: topk_wave_kernel<2><<<grid, TK_NT, 0, st>>>(p); break;
      case 4: topk_wave_kernel<4><<<grid, TK_NT, 0, st>>>(p); break;
      case 8: topk_wave_kernel<8><<<grid, TK_NT, 0, st>>>(p); break;
      default: topk_wave_kernel<16><<<grid, TK_NT, 0, st>>>(p); break;
    }
    LA_LAUNCHED();
    return LA_OK;
  }
  // register-resident rows: up to 8192 keys (16384 for the bitmap form)
  if ((p.use_bitmap && p.n_lds <= 64 * TK_NT) ||
      (p.n_lds <= 32 * TK_NT && p.G == 1 && std::min(p.k, p.n_lds) <= 16 * TK_NT))
    return launch_reg(p, st);
  const int64_t limit = (int64_t)max_dynamic_lds() - (int64_t)sizeof(TkShared) - 256;
  p.lds_keys = 1;
  int64_t bytes = topk_lds_bytes(p);
  if (bytes > limit) {
    p.lds_keys = 0;
    bytes = topk_lds_bytes(p);
  }
  if (bytes > limit)
    return fail(LA_ERR_UNSUPPORTED, "topk: k=%lld / n=%lld needs %lld B of LDS (limit %lld)",
                (long long)p.k, (long long)p.n, (long long)bytes, (long long)limit);
  if (bytes > 65536) {
    static bool attr_set = false;
    if (!attr_set) {
      LA_HIP(hipFuncSetAttribute((const void *)topk_rows_kernel,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)limit));
      attr_set = true;
    }
  }
  topk_rows_kernel<<<dim3((unsigned)p.NG), TK_NT, (size_t)bytes, st>>>(p);
  LA_LAUNCHED();
  return LA_OK;
}

}  // namespace la

using namespace la;

static TopkKParams params_from_args(const la_topk_args *a) {
  TopkKParams p{};
  p.scores = a->scores;
  p.row_stride = a->row_stride;
  p.G = a->group;
  p.Tq = a->Tq;
  p.NG = a->B * (a->H / a->group) * a->Tq;
  p.t_base = 0;
  p.out_tq = a->Tq;
  p.n = a->n;
  p.k = a->k;
  p.width = a->width;
  p.n_valid_tab = a->n_valid;
  p.own_tab = a->own;
  p.pos_off = a->pos_offset;
  p.pos_unit = a->pos_unit;
  p.sink = a->sink_units;
  p.window = a->window_units;
  p.force_own = a->force_own;
  p.order = a->order;
  p.out_idx = a->out_idx;
  p.out_val = a->out_val;
  p.out_count = a->out_count;
  return p;
}

static int validate(const la_topk_args *a) {
  LA_REQUIRE(a && a->scores && a->out_idx, "la_topk_rows: null pointer");
  LA_REQUIRE(a->B > 0 && a->H > 0 && a->Tq > 0 && a->n > 0, "la_topk_rows: bad shape");
  LA_REQUIRE(a->row_stride >= a->n, "la_topk_rows: row_stride < n");
  LA_REQUIRE(a->group >= 1 && a->H % a->group == 0, "la_topk_rows: H must be a multiple of group");
  LA_REQUIRE(a->k >= 1 && a->width >= 1, "la_topk_rows: k and width must be >= 1");
  LA_REQUIRE(a->order == 0 || a->order == 1, "la_topk_rows: order must be 0 or 1");
  const bool bitmap = a->group > 1 || a->sink_units > 0 || a->window_units > 0 || a->order == 1;
  LA_REQUIRE(!(bitmap && a->out_val), "la_topk_rows: values are only produced for order 0");
  LA_REQUIRE(!(a->order == 0 && bitmap), "la_topk_rows: union/sink/window need order 1");
  if (a->order == 0) LA_REQUIRE(a->width >= a->k, "la_topk_rows: width < k");
  if (a->window_units > 0 || a->force_own)
    LA_REQUIRE(a->own != nullptr || a->pos_unit > 0, "la_topk_rows: window/force_own need own[]");
  return LA_OK;
}

extern "C" size_t la_topk_rows_workspace(const la_topk_args *a) {
  if (validate(a) != LA_OK) return 0;
  return (size_t)topk_workspace_bytes(params_from_args(a));
}

extern "C" int la_topk_rows(const la_topk_args *a, void *stream) {
  const int rc = validate(a);
  if (rc != LA_OK) return rc;
  return topk_launch_ws(params_from_args(a), a->workspace, a->ws_bytes, (hipStream_t)stream);
}
