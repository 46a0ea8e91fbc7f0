// Workgroup-collective pieces of the row top-k, shared by the top-k kernels
// and the fused Quest selection.  Ordering: order-preserving 64-bit image of
// the fp64 score (ord_key), higher first; equal keys go to the lower index.
#pragma once

#include "common.h"

namespace la {

constexpr int TK_NT = 256;  // threads of a selecting workgroup
constexpr int TK_CAND_REGS = 2;  // keys per lane of the one-wave finish
constexpr int TK_NW = TK_NT / 64;

__device__ __forceinline__ uint64_t lanemask_lt(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Inclusive scan of one value per thread across a workgroup of NT threads
// (wtmp holds NT / 64 words).  LDS_ONLY: its barriers order LDS alone (global
// loads and stores in flight stay in flight).
template <int NT = TK_NT, bool LDS_ONLY = false>
__device__ __forceinline__ uint32_t tk_block_incl_scan(uint32_t v, uint32_t *wtmp, uint32_t &total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(v, off, 64);
    if (lane >= off) v += y;
  }
  if (lane == 63) wtmp[w] = v;
  if (LDS_ONLY)
    lds_barrier();
  else
    __syncthreads();
  uint32_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    const uint32_t x = wtmp[i];
    base += (i < w) ? x : 0u;
    tot += x;
  }
  if (LDS_ONLY)
    lds_barrier();
  else
    __syncthreads();
  total = tot;
  return v + base;
}

template <int KPT>
struct TkRegShared {
  uint32_t hist[TK_NW][256];
  uint32_t eqc[KPT][TK_NW];
  uint64_t red[2][TK_NW];
  uint32_t wtmp[2][TK_NW];
  uint32_t bin, above, cnt;
  uint32_t cfill;  // candidates copied by tk_reg_select_bits
};

// Top K of the keys u[j] of units t + 256*j (t = thread), j < KPT, among the
// first n_v units.  A radix select fixes the leading bits every valid key
// shares without a pass, then resolves 8-bit digits (per-wave histograms)
// until the threshold digit is taken whole or all bits are fixed; keys equal
// to the final threshold are taken lowest index first.  emit(j, i, take) is
// then called by every thread for every slot j, in increasing j (so it may
// use wave-collective operations); `take` marks the K selected units.
// Collective over the workgroup; ends with the workgroup in step.
template <int KPT, class Emit>
__device__ __forceinline__ void tk_reg_select(const uint64_t (&u)[KPT], int32_t n_v, uint32_t K,
                                              TkRegShared<KPT> &sh, Emit emit) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint64_t lt = lanemask_lt(lane);
  uint64_t prefix = 0, mask = 0;
  uint32_t need = K;
  bool all_in = (int32_t)K >= n_v;
  if (!all_in) {
    uint64_t o = 0, a = ~0ull;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      if (tid + TK_NT * j < n_v) {
        o |= u[j];
        a &= u[j];
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      o |= __shfl_xor(o, off, 64);
      a &= __shfl_xor(a, off, 64);
    }
    if (lane == 0) {
      sh.red[0][w] = o;
      sh.red[1][w] = a;
    }
    __syncthreads();
    o = 0;
    a = ~0ull;
#pragma unroll
    for (int x = 0; x < TK_NW; ++x) {
      o |= sh.red[0][x];
      a &= sh.red[1][x];
    }
    const uint64_t diff = o ^ a;
    int top = diff ? 63 - __clzll((long long)diff) : -1;
    mask = top >= 0 ? ~((2ull << top) - 1ull) : ~0ull;  // 2ull << 63 wraps to 0
    prefix = a & mask;
    while (top >= 0) {
      const int shift = top >= 7 ? top - 7 : 0;
      const uint32_t dm = (2u << (top - shift)) - 1u;  // digit of top-shift+1 <= 8 bits
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) sh.hist[x][tid] = 0u;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        if (tid + TK_NT * j < n_v && (u[j] & mask) == prefix)
          atomicAdd(&sh.hist[w][(uint32_t)(u[j] >> shift) & dm], 1u);
      }
      __syncthreads();
      uint32_t c = 0;
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) c += sh.hist[x][255 - tid];
      uint32_t tot;
      const uint32_t incl = tk_block_incl_scan(c, sh.wtmp[0], tot);
      if (incl >= need && incl - c < need) {
        sh.bin = 255 - tid;
        sh.above = incl - c;
        sh.cnt = c;
      }
      __syncthreads();
      need -= sh.above;
      prefix |= (uint64_t)sh.bin << shift;
      mask |= (uint64_t)dm << shift;
      const bool done = sh.cnt == need;
      __syncthreads();
      if (done) {
        all_in = true;
        break;
      }
      top = shift - 1;
    }
  }
  // Keys above the threshold are all taken; keys equal to it are taken in
  // index order until `need` is met.
  if (!all_in) {
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const bool eq = tid + TK_NT * j < n_v && (u[j] & mask) == prefix;
      const uint64_t b = __ballot(eq);
      if (lane == 0) sh.eqc[j][w] = (uint32_t)__popcll(b);
    }
    __syncthreads();
  }
  uint32_t eq_before = 0;  // threshold keys in earlier slots
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int32_t i = tid + TK_NT * j;
    const bool valid = i < n_v;
    const uint64_t um = u[j] & mask;
    const bool gt = valid && um > prefix;
    const bool eq = valid && um == prefix;
    bool take = gt || (eq && all_in);
    if (!all_in) {
      const uint64_t b = __ballot(eq);
      uint32_t rank = eq_before + (uint32_t)__popcll(b & lt);
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) rank += x < w ? sh.eqc[j][x] : 0u;
      take = gt || (eq && rank < need);
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) eq_before += sh.eqc[j][x];
    }
    emit(j, i, take);
  }
  __syncthreads();
}

// Top K of the keys u[j] of units t + 256*j (t = thread), j < KPT, among the
// first n_v units: the selection of tk_reg_select by a bitwise search for the
// K-th largest key.  T starts as the leading bits all valid keys share and
// keeps the bits found so far; each step counts the keys >= T | bit (one
// vector compare per slot, counted from the lane mask on the scalar unit),
// adds the four waves' counts through LDS (one barrier per step, alternating
// slots) and keeps the bit when at least K keys reach it.
// It stops when exactly K do; else T is the K-th largest key and its ties
// are taken lowest index first.  emit(j, i, take) as in tk_reg_select.
// The keys of units past n_v are set to 0 in u (no candidate reaches 0).
// With `cand` (LDS for `cap` <= 64 * TK_CAND_REGS keys, not otherwise used
// until emit), once at most `cap` keys lie between T and the lowest key known
// to be selected whole (the undecided window), they are copied there and one
// wave finishes the search over them in registers, with no barrier per bit.
template <int KPT, class Emit>
__device__ __forceinline__ void tk_reg_select_bits(uint64_t (&u)[KPT], int32_t n_v, uint32_t K,
                                                   TkRegShared<KPT> &sh, Emit emit,
                                                   uint64_t *cand = nullptr, uint32_t cap = 0) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint32_t *cnt = sh.wtmp[0];  // [2][TK_NW] counts, alternating steps
#pragma unroll
  for (int j = 0; j < KPT; ++j) u[j] = tid + TK_NT * j < n_v ? u[j] : 0ull;
  if ((int32_t)K >= n_v) {
#pragma unroll
    for (int j = 0; j < KPT; ++j) emit(j, tid + TK_NT * j, tid + TK_NT * j < n_v);
    __syncthreads();
    return;
  }
  // the bits every valid key shares need no step: start below them
  uint64_t o = 0, a = ~0ull;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    if (tid + TK_NT * j < n_v) {
      o |= u[j];
      a &= u[j];
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    o |= __shfl_xor(o, off, 64);
    a &= __shfl_xor(a, off, 64);
  }
  if (lane == 0) {
    sh.red[0][w] = o;
    sh.red[1][w] = a;
  }
  __syncthreads();
  o = 0;
  a = ~0ull;
#pragma unroll
  for (int x = 0; x < TK_NW; ++x) {
    o |= sh.red[0][x];
    a &= sh.red[1][x];
  }
  const uint64_t diff = o ^ a;
  const int top = diff ? 63 - __clzll((long long)diff) : -1;
  uint64_t T = top >= 0 ? a & ~((2ull << top) - 1ull) : a;  // 2ull << 63 wraps to 0
  bool exact = false;
  int step = 0;
  // keys >= U (when has_u) are selected whole: `above` of them; `tot_t`
  // keys are >= T, so tot_t - above lie in the undecided window [T, U)
  uint64_t U = 0;
  bool has_u = false;
  uint32_t above = 0, tot_t = (uint32_t)n_v;
  int bit = top;
  for (; bit >= 0; --bit, ++step) {
    if (cand && tot_t - above <= cap && step > 0) {
      // copy the window's keys (workgroup-uniform decision) ...
      uint32_t *fill = &sh.cfill;
      if (tid == 0) fill[0] = 0;
      __syncthreads();
      const uint64_t lt = lanemask_lt(lane);
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const bool inw = u[j] >= T && (!has_u || u[j] < U) && tid + TK_NT * j < n_v;
        const uint64_t m = __ballot(inw);
        if (m) {
          uint32_t base = 0;
          if (lane == 0) base = atomicAdd(fill, (uint32_t)__popcll(m));
          base = __shfl(base, 0, 64);
          if (inw) cand[base + (uint32_t)__popcll(m & lt)] = u[j];
        }
      }
      const uint32_t n_c = tot_t - above;
      __syncthreads();
      // ... and let one wave finish the search over them in registers,
      // without barriers
      if (w == 0) {
        uint64_t cr[TK_CAND_REGS];
#pragma unroll
        for (int m = 0; m < TK_CAND_REGS; ++m) {
          const uint32_t i = lane + 64 * m;
          cr[m] = i < n_c ? cand[i] : 0ull;  // 0 never reaches a candidate threshold
        }
        for (; bit >= 0; --bit) {
          const uint64_t T2 = T | (1ull << bit);
          uint32_t c = above;
#pragma unroll
          for (int m = 0; m < TK_CAND_REGS; ++m)
            c += (uint32_t)__popcll(__ballot(cr[m] >= T2 && (!has_u || cr[m] < U)));
          if (c >= K) {
            T = T2;
            if (c == K) {
              exact = true;
              break;
            }
          } else {
            U = T2;
            has_u = true;
            above = c;
          }
        }
        if (lane == 0) {
          sh.red[0][0] = T;
          sh.cfill = exact ? 1u : 0u;
        }
      }
      __syncthreads();
      T = sh.red[0][0];
      exact = sh.cfill != 0;
      break;
    }
    const uint64_t T2 = T | (1ull << bit);
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < KPT; ++j) c += (uint32_t)__popcll(__ballot(u[j] >= T2));
    uint32_t *slot = cnt + (step & 1) * TK_NW;
    if (lane == 0) slot[w] = c;
    __syncthreads();
    uint32_t tot = 0;
#pragma unroll
    for (int x = 0; x < TK_NW; ++x) tot += slot[x];
    if (tot >= K) {
      T = T2;
      tot_t = tot;
      if (tot == K) {
        exact = true;
        break;
      }
    } else {
      U = T2;
      has_u = true;
      above = tot;
    }
  }
  if (exact) {
#pragma unroll
    for (int j = 0; j < KPT; ++j) emit(j, tid + TK_NT * j, tid + TK_NT * j < n_v && u[j] >= T);
    __syncthreads();
    return;
  }
  // T is the K-th largest key: every key above it, then its ties by index
  // (slot j before slot j + 1, lower waves and lanes first within a slot)
  uint32_t gt = 0;
#pragma unroll
  for (int j = 0; j < KPT; ++j) gt += (uint32_t)__popcll(__ballot(u[j] > T));
  __syncthreads();  // sh.red is read above
  if (lane == 0) sh.red[0][w] = gt;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const bool eq = tid + TK_NT * j < n_v && u[j] == T;
    const uint64_t b = __ballot(eq);
    if (lane == 0) sh.eqc[j][w] = (uint32_t)__popcll(b);
  }
  __syncthreads();
  uint32_t need = K;
#pragma unroll
  for (int x = 0; x < TK_NW; ++x) need -= (uint32_t)sh.red[0][x];
  const uint64_t lt = lanemask_lt(lane);
  uint32_t eq_before = 0;  // threshold keys in earlier slots
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int32_t i = tid + TK_NT * j;
    const bool valid = i < n_v;
    const bool eq = valid && u[j] == T;
    const uint64_t b = __ballot(eq);
    uint32_t rank = eq_before + (uint32_t)__popcll(b & lt);
#pragma unroll
    for (int x = 0; x < TK_NW; ++x) rank += x < w ? sh.eqc[j][x] : 0u;
    const bool take = (valid && u[j] > T) || (eq && rank < need);
#pragma unroll
    for (int x = 0; x < TK_NW; ++x) eq_before += sh.eqc[j][x];
    emit(j, i, take);
  }
  __syncthreads();
}

// One wave's top K of the keys u[j] of units lane + 64*j, j < KPL, among the
// first n_v units, by a bitwise search for the K-th largest key: T keeps the
// bits found so far and each step counts the keys >= T | bit with one vector
// compare per slot (the compare writes the wave's lane mask, counted on the
// scalar unit).  It stops as soon as exactly K keys reach the candidate; else
// T ends as the K-th largest key and its ties go to the lowest index.  No
// LDS and no barrier.  Same selection as tk_reg_select.  emit(j, i, take) is
// called by every lane for every slot j in increasing j.
// With `scratch` (this wave's own LDS, >= TK_WCAP keys), once at most TK_WCAP
// keys reach T the search continues over those candidates only, two per lane
// (the keys below T can no longer be selected and do not change any later
// count): the low bits cost two compares per step instead of KPL.
constexpr int TK_WCAP = 128;
template <int KPL, class Emit>
__device__ __forceinline__ void tk_wave_select_bits(const uint64_t (&u_in)[KPL], int32_t n_v,
                                                    uint32_t K, Emit emit,
                                                    uint64_t *scratch = nullptr) {
  const int lane = threadIdx.x & 63;
  uint64_t u[KPL];  // units past n_v count as key 0, which no candidate reaches
#pragma unroll
  for (int j = 0; j < KPL; ++j) u[j] = lane + 64 * j < n_v ? u_in[j] : 0ull;
  if ((int32_t)K >= n_v) {
#pragma unroll
    for (int j = 0; j < KPL; ++j) emit(j, lane + 64 * j, lane + 64 * j < n_v);
    return;
  }
  uint64_t T = 0;  // count(u >= T) >= K throughout
  bool exact = false;
  int bit = 63;
  bool narrowed = false;
  if (scratch) {
    // the bits that every valid key shares are in T from the start (every
    // valid key still reaches it): the search starts below them.  A forced
    // unit (KEY_FORCED, above every score) is left out of the prefix: it
    // reaches any T.
    uint64_t hi = 0, lo = ~0ull;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const bool valid = lane + 64 * j < n_v && u[j] != KEY_FORCED;
      hi = valid && u[j] > hi ? u[j] : hi;
      lo = valid && u[j] < lo ? u[j] : lo;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t h2 = __shfl_xor(hi, o, 64), l2 = __shfl_xor(lo, o, 64);
      hi = h2 > hi ? h2 : hi;
      lo = l2 < lo ? l2 : lo;
    }
    const uint64_t diff = hi ^ lo;
    if (hi >= lo && diff != 0) {
      const int top = 63 - __clzll(diff);  // highest differing bit
      T = hi & ~((2ull << top) - 1ull);     // (top == 63: no shared bits, T = 0)
      bit = top;
    }
  }
  for (; bit >= 0; --bit) {
    const uint64_t T2 = T | (1ull << bit);
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j) c += (uint32_t)__popcll(__ballot(u[j] >= T2));
    if (c >= K) {
      T = T2;
      if (c == K) {
        exact = true;
        break;
      }
      if (KPL > 2 && scratch && c <= (uint32_t)TK_WCAP) {
        narrowed = true;
        --bit;
        break;
      }
    }
  }
  if (KPL > 2 && narrowed) {
    // compact the keys >= T (at most TK_WCAP) and finish the search on them
    const uint64_t lt = lanemask_lt(lane);
    uint32_t base = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const bool cand = u[j] >= T;
      const uint64_t b = __ballot(cand);
      if (cand) scratch[base + (uint32_t)__popcll(b & lt)] = u[j];
      base += (uint32_t)__popcll(b);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const uint64_t v0 = (uint32_t)lane < base ? scratch[lane] : 0ull;
    const uint64_t v1 = (uint32_t)lane + 64 < base ? scratch[lane + 64] : 0ull;
    for (; bit >= 0; --bit) {
      const uint64_t T2 = T | (1ull << bit);
      const uint32_t c = (uint32_t)__popcll(__ballot(v0 >= T2)) + (uint32_t)__popcll(__ballot(v1 >= T2));
      if (c >= K) {
        T = T2;
        if (c == K) {
          exact = true;
          break;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the scratch may be reused by the caller
  }
  if (exact) {
#pragma unroll
    for (int j = 0; j < KPL; ++j) emit(j, lane + 64 * j, lane + 64 * j < n_v && u[j] >= T);
    return;
  }
  // T is the K-th largest key: every key above it, then its ties by index
  uint32_t gt = 0;
#pragma unroll
  for (int j = 0; j < KPL; ++j) gt += (uint32_t)__popcll(__ballot(u[j] > T));
  const uint32_t need = K - gt;
  const uint64_t lt = lanemask_lt(lane);
  uint32_t eq_before = 0;
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const int32_t i = lane + 64 * j;
    const bool valid = i < n_v;
    const bool eq = valid && u[j] == T;
    const uint64_t b = __ballot(eq);
    const bool take = (valid && u[j] > T) || (eq && eq_before + (uint32_t)__popcll(b & lt) < need);
    eq_before += (uint32_t)__popcll(b);
    emit(j, i, take);
  }
}

// Sink units [0, sink) and the window (own - window, own] are OR'd into the
// bitmap of kept units, which is then written in ascending index order to
// out[0, width), -1 padded; *count (if given) gets the number kept.  With
// cand (a candidate row of a segmented top-k), slot i stands for unit
// cand[i]: slots whose candidate is -1 are dropped and cand[i] is written.
template <int NT = TK_NT>
__device__ __forceinline__ void tk_emit_bitmap_row(uint32_t *bm, int64_t n_v, int64_t own,
                                                   int64_t sink, int64_t window, int64_t width,
                                                   int32_t *out, int32_t *count, uint32_t *wtmp,
                                                   const int32_t *cand = nullptr) {
  const int tid = threadIdx.x;
  if (n_v > 0) {
    const int64_t s_end = min(sink, n_v);
    for (int64_t i = tid; i < s_end; i += NT) atomicOr(&bm[i >> 5], 1u << (i & 31));
    if (window > 0 && own >= 0) {
      const int64_t w0 = max((int64_t)0, own - window + 1);
      const int64_t w1 = min(own, n_v - 1);
      for (int64_t i = w0 + tid; i <= w1; i += NT) atomicOr(&bm[i >> 5], 1u << (i & 31));
    }
  }
  __syncthreads();
  // each thread owns a run of bitmap words
  const int64_t words = (n_v + 31) / 32;
  const int64_t wpt = (words + NT - 1) / NT;
  const int64_t w_beg = min(words, (int64_t)tid * wpt), w_end = min(words, w_beg + wpt);
  uint32_t cnt = 0;
  for (int64_t x = w_beg; x < w_end; ++x) {
    if (cand) {  // candidate rows: slots without a candidate (-1) are dropped
      uint32_t bits = bm[x], keep = bits;
      while (bits) {
        const int b = __ffs(bits) - 1;
        if (cand[x * 32 + b] < 0) keep &= ~(1u << b);
        bits &= bits - 1;
      }
      bm[x] = keep;
    }
    cnt += __popc(bm[x]);
  }
  uint32_t total;
  const uint32_t incl = tk_block_incl_scan<NT>(cnt, wtmp, total);
  uint32_t pos = incl - cnt;
  for (int64_t x = w_beg; x < w_end; ++x) {
    uint32_t bits = bm[x];
    while (bits) {
      const int b = __ffs(bits) - 1;
      if (pos < (uint32_t)width) out[pos] = cand ? cand[x * 32 + b] : (int32_t)(x * 32 + b);
      ++pos;
      bits &= bits - 1;
    }
  }
  for (int64_t jj = (int64_t)total + tid; jj < width; jj += NT) out[jj] = -1;
  if (count && tid == 0) *count = (int32_t)min((int64_t)total, width);
}

}  // namespace la
