// Token addressing for contiguous and paged KV caches (see la_kv in linattn_hip.h).
#pragma once

#include "common.h"

namespace la {

// Element offset of row (b, h, tok) of K (is_v = false) or V (is_v = true).
__device__ __forceinline__ int64_t kv_row(const la_kv &kv, int64_t b, int64_t h, int64_t tok,
                                          int64_t Hkv, int64_t D, bool is_v) {
  if (kv.page_table) {
    const int64_t ps = kv.page_size;
    const int64_t phys = kv.page_table[b * kv.pt_stride + tok / ps];
    return ((phys * Hkv + h) * ps + (tok % ps)) * D;
  }
  return is_v ? (b * kv.v_sb + h * kv.v_sh + tok * kv.v_st)
              : (b * kv.k_sb + h * kv.k_sh + tok * kv.k_st);
}

// Offset of the per-token fp8 scale of (b, h, tok).
__device__ __forceinline__ int64_t kv_scale_idx(const la_kv &kv, int64_t b, int64_t h, int64_t tok,
                                                int64_t Hkv) {
  if (kv.page_table) {
    const int64_t ps = kv.page_size;
    const int64_t phys = kv.page_table[b * kv.pt_stride + tok / ps];
    return (phys * Hkv + h) * ps + (tok % ps);
  }
  return b * kv.s_sb + h * kv.s_sh + tok * kv.s_st;
}

// Valid tokens of sequence b, never more than the cache holds.
__device__ __forceinline__ int64_t kv_length(const la_kv &kv, int64_t b) {
  return kv.kv_len ? min((int64_t)kv.kv_len[b], kv.T) : kv.T;
}

}  // namespace la
