// Row-wise top-k shared by Quest page selection, block selection and the
// lightning indexer.  Ordering: score descending, index ascending on ties.
#pragma once

#include "common.h"

namespace la {

// Kernel parameters.  Group gi (one workgroup) covers rows
//   row(gi, j) = ((gi / Tq) * G + j) * Tq + gi % Tq,   j < G
// whose query index is t = gi % Tq + t_base; the output row is
//   orow = (gi / Tq) * out_tq + gi % Tq + t_base.
struct TopkKParams {
  const double *scores;
  int64_t row_stride;
  int64_t NG, G, Tq, t_base, out_tq;
  int64_t n, k, width;
  const int32_t *n_valid_tab;  // indexed by t (may be null)
  const int32_t *own_tab;      // indexed by t (may be null)
  int64_t pos_off, pos_unit;   // pos_unit > 0: tables derived from pos = pos_off + t
  int64_t sink, window;
  int32_t force_own, order;
  int32_t lds_keys;  // cache the row's keys in LDS
  int32_t use_bitmap;
  int64_t n_lds;  // keys one workgroup holds (n, or the segment length)
  int64_t bitmap_words;
  int64_t p2k;  // power of two >= k (order 0)
  int32_t *out_idx;
  float *out_val;
  int32_t *out_count;
  // segmented mode (seg_len > 0): workgroup g selects within segment g % nseg
  // of row g / nseg and writes positions within the segment to out row g
  int64_t seg_len, nseg;
  // candidate rows: output index = cand_idx[row slot] instead of the position
  const int32_t *cand_idx;
  // ragged batches (may be null): row t of batch item br / rows_per_b has no
  // units at all once t * b_len_unit >= b_lens[item] (a row past the end of a
  // shorter sequence: nothing selected, no sink, no own unit)
  const int32_t *b_lens;
  int64_t rows_per_b, b_len_unit;
};

// The row (group) a workgroup selects for, its valid prefix and forced unit.
struct TkRow {
  int64_t br, seg0, tl, t, orow, n_v, own, K;
  bool force;
};

// Quotient of a non-negative a by a positive b; with S32 (the caller has
// checked that both fit in 32 bits) in 32-bit arithmetic, a few instructions
// instead of the long 64-bit division sequence.
template <bool S32>
__device__ __forceinline__ int64_t tk_div(int64_t a, int64_t b) {
  return S32 ? (int64_t)((uint32_t)a / (uint32_t)b) : a / b;
}

// S32: every quotient taken here has a dividend and divisor below 2^32
// (tk_row_fits_32).
template <bool S32 = false>
__device__ __forceinline__ TkRow tk_row(const TopkKParams &p, int64_t gi) {
  TkRow r;
  // Segmented mode: group gi handles segment gi % nseg of row gi / nseg.
  r.br = p.seg_len > 0 ? tk_div<S32>(gi, p.nseg) : gi;
  const int64_t seg = p.seg_len > 0 ? gi - r.br * p.nseg : 0;
  r.seg0 = seg * p.seg_len;
  const int64_t bq = tk_div<S32>(r.br, p.Tq);
  r.tl = r.br - bq * p.Tq;
  r.t = r.tl + p.t_base;
  r.orow = p.seg_len > 0 ? gi : bq * p.out_tq + r.t;
  int64_t n_v = p.n;
  int64_t own = -1;
  if (p.pos_unit > 0) {
    const int64_t pos = p.pos_off + r.t;
    const int64_t u = pos >= 0 ? tk_div<S32>(pos, p.pos_unit) : -1;
    n_v = min(p.n, u + 1);
    own = min(u, p.n - 1);
  }
  if (p.n_valid_tab) n_v = min(p.n, (int64_t)p.n_valid_tab[r.t]);
  if (p.own_tab) own = (int64_t)p.own_tab[r.t];
  if (p.b_lens && r.t * p.b_len_unit >= (int64_t)p.b_lens[tk_div<S32>(r.br, p.rows_per_b)]) {
    n_v = 0;
    own = -1;
  }
  if (p.seg_len > 0) n_v = min(n_v - r.seg0, min(p.seg_len, p.n - r.seg0));
  r.n_v = max(n_v, (int64_t)0);
  r.own = own;
  r.force = p.force_own && own >= 0 && own < r.n_v;
  r.K = min(p.k, r.n_v);
  return r;
}

// Whether tk_row<true> is exact for every group of p: the dividends (group
// and row numbers, positions pos_off + t) and the divisors below 2^32.
inline bool tk_row_fits_32(const TopkKParams &p) {
  const int64_t lim = (int64_t)1 << 32;
  return p.NG < lim && p.nseg < lim && p.Tq < lim && p.pos_unit < lim && p.rows_per_b < lim &&
         p.pos_off + p.t_base + p.Tq < lim;
}

// Long plain rows split over several workgroups per row (topk_radix.hip): C
// chunks per row; workspace bytes (per-row state, digit histograms, chunk
// records, then the candidate rows of a sorted selection).  C = 0 when a row
// holds 2^31 keys or more.
struct RadixPlan {
  int64_t C = 0, bytes = 0;
};
constexpr int RX_RB = 11;  // radix digit bits
constexpr int RX_BINS = 1 << RX_RB;
RadixPlan radix_plan(const TopkKParams &p);
int topk_radix_launch(const TopkKParams &p, const RadixPlan &R, void *ws, hipStream_t st);
// The same in parts, for a scores kernel that histograms the first digit
// (the top RX_RB bits of ord_key of every valid key of row gi, added into
// rows + gi * row_words + bin of radix_row_prep) in between: set-up, that
// kernel, then the stage launches.  Or without the set-up launch
// (state_in_kernel): the scores kernel clears row gi's row_words words and
// then stores *epoch plus a value of the call into ready[gi], before any of
// its workgroups adds into the row's histogram (each waits for that value
// first); the first stage launch starts the rows from their initial state
// and advances *epoch (one word for all rows), so a replay of the same
// launches waits for a value of its own.
// Polls after which the radix select's and the decode indexer's waits on
// other workgroups give up (2^20 unless la_test_set_spin_limit changed it).
uint32_t rx_spin_limit();

struct RadixRowPrep {
  uint32_t *rows = nullptr;
  int64_t row_words = 0;
  uint64_t *ready = nullptr;
  uint64_t *epoch = nullptr;
};
RadixRowPrep radix_row_prep(const TopkKParams &p, const RadixPlan &R, void *ws);
int topk_radix_setup(const TopkKParams &p, const RadixPlan &R, void *ws, bool hist0_external,
                     hipStream_t st);
int topk_radix_finish(const TopkKParams &p, const RadixPlan &R, void *ws, bool hist0_external,
                      bool state_in_kernel, hipStream_t st);
// The radix plan when topk_launch_ws sends these rows to the radix select
// (else C = 0).
RadixPlan topk_long_plan(const TopkKParams &p);

// Workspace bytes topk_launch_ws needs (rows longer than the LDS can hold go
// to the multi-workgroup radix select).
int64_t topk_workspace_bytes(const TopkKParams &p);

// As topk_launch, with a workspace for long rows.
int topk_launch_ws(TopkKParams p, void *ws, int64_t ws_bytes, hipStream_t st);

// Dynamic LDS bytes a launch needs, or -1 when it cannot fit.
int64_t topk_lds_bytes(const TopkKParams &p);

// Fill derived fields (lds_keys, bitmap, p2k) and launch one workgroup per group.
int topk_launch(TopkKParams p, hipStream_t st);

}  // namespace la
