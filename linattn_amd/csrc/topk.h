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
};

// Workspace bytes topk_launch needs (rows longer than the LDS can hold are
// selected in segments: candidates of each level are kept in the workspace).
int64_t topk_workspace_bytes(const TopkKParams &p);

// As topk_launch, with a workspace for long rows.
int topk_launch_ws(TopkKParams p, void *ws, int64_t ws_bytes, hipStream_t st);

// Dynamic LDS bytes a launch needs, or -1 when it cannot fit.
int64_t topk_lds_bytes(const TopkKParams &p);

// Fill derived fields (lds_keys, bitmap, p2k) and launch one workgroup per group.
int topk_launch(TopkKParams p, hipStream_t st);

}  // namespace la
