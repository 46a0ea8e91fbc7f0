/*
 * linattn_hip.h -- C ABI of the MI355X (gfx950) sparse-attention hot path.
 *
 * This is the drop-in boundary that replaces the lazily imported Triton
 * backend of tongxin/linattn (src/linattn/kernels/triton/) and the ctypes C
 * decode (src/linattn/kernels/c_attention.py).  Every entry point:
 *   - takes plain device pointers, element strides and sizes (no torch types),
 *   - enqueues work on the given HIP stream and returns without a host sync,
 *   - never allocates: scratch memory comes in through `workspace`, whose size
 *     the matching *_workspace() call reports,
 *   - returns 0 on success or a la_status code; la_last_error() then holds a
 *     message for the calling thread.
 * Inputs are never written.  Shapes are validated here as well as in the
 * Python wrapper.
 *
 * Citations are path:line in the reference repository.
 */
#ifndef LINATTN_HIP_H
#define LINATTN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LA_ABI_VERSION 13

/* element types */
enum {
  LA_F32 = 0,
  LA_BF16 = 1,
  LA_F16 = 2,
  LA_FP8_E4M3 = 3, /* OCP e4m3fn, bit-identical to torch.float8_e4m3fn */
  LA_F64 = 4
};

/* status codes */
enum {
  LA_OK = 0,
  LA_ERR_INVALID = 1,     /* bad shape / argument (Python raises ValueError) */
  LA_ERR_UNSUPPORTED = 2, /* shape the kernels are not instantiated for */
  LA_ERR_HIP = 3,         /* HIP runtime error (launch, attribute) */
  LA_ERR_WORKSPACE = 4    /* workspace smaller than *_workspace() */
};

/* device status bits (la_device_status) */
enum {
  LA_DEV_TOPK_TIMEOUT = 1,  /* a wait of the multi-workgroup top-k (a chunk's look-back over
                               the row's earlier chunks) or of the decode indexer (for the
                               row's first workgroup) passed its bound (a hardware fault
                               guard: each waits only for workgroups dispatched before it) */
  LA_DEV_PREFILL_RANGE = 2  /* la_block_sparse_prefill met a finite |v| >= 2^22 (outputs inf;
                              the Python wrapper raises ValueError) */
};

/* ABI version of the loaded library (LA_ABI_VERSION). */
int la_abi_version(void);

/*
 * Status bits the kernels raised on the current device since the last clear
 * (LA_DEV_*), after the work queued on the given stream; clear != 0 resets
 * them in the same atomic exchange (a bit raised meanwhile by another stream's
 * kernel is kept for the next read).
 * Kernels report failures they detect on the device here instead of through a
 * return code (a launch returns before the kernel runs): a long row of
 * la_topk_rows / la_indexer_topk whose multi-workgroup selection hit that
 * guard comes back incomplete (the chunk that gave up writes no ids), and
 * LA_DEV_TOPK_TIMEOUT is raised.
 * No counterpart in the reference (its kernels report nothing).  Synchronous.
 */
int la_device_status(uint32_t *bits, int32_t clear, void *stream);

/*
 * Testing hook, no counterpart in the reference: the number of polls after
 * which the library's bounded waits on other workgroups (LA_DEV_TOPK_TIMEOUT)
 * give up, process-wide; 2^20 by default, 0 gives every such wait up at once
 * (so a test can drive the timeout path while every kernel still ends).
 */
int la_test_set_spin_limit(uint32_t polls);

/* Message describing the last non-zero status returned on this thread. */
const char *la_last_error(void);

/*
 * A view of a KV cache.  Two layouts:
 *  - contiguous: k/v are (B, Hkv, T, D) with element strides k_sb/k_sh/k_st
 *    (unit stride over D), as in the reference (block_sparse.py:40-57);
 *  - paged: page_table != NULL.  k/v are pools of physical pages laid out
 *    [phys_page][Hkv][page_size][D]; logical token t of sequence b lives in
 *    physical page page_table[b * pt_stride + t / page_size] at row
 *    t % page_size.  The reference has no page table; this layout is new.
 * fp8 caches carry one fp32 scale per token and KV head (kv/quant.py:90-93
 * with group_size == head_dim): contiguous scales are (B, Hkv, T) with
 * strides s_sb/s_sh/s_st; paged scales are [phys_page][Hkv][page_size] with
 * pool row r's scale at k_scale[r * s_st] / v_scale[r * s_st] (s_st = 0 reads
 * as 1; s_st = 2 with v_scale = k_scale + 1 interleaves each token's K and V
 * scales, so a token read from a random position costs one 64-byte sector of
 * scales instead of two).
 * kv_len (optional, int32 [B]) limits the valid tokens of each sequence.
 */
typedef struct {
  const void *k;
  const void *v;
  const float *k_scale;
  const float *v_scale;
  const int32_t *page_table;
  const int32_t *kv_len;
  int64_t T;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t s_sb, s_sh, s_st;
  int64_t pt_stride;
  int64_t page_size;
  int32_t dtype; /* LA_F32, LA_BF16 or LA_FP8_E4M3 */
  int32_t reserved;
} la_kv;

/*
 * Exact attention over listed KV units (blocks, pages or tokens).
 * Replaces block_sparse_attention / _block_sparse_fwd_kernel
 * (kernels/triton/block_sparse.py:131-163, torch semantics :40-75) and the
 * C paged decode (kernels/c/decode_attn.c:39-133, c_attention.py:76-111).
 *
 * ids: int32 [B][ids_heads][rows][N] with element strides id_sb/id_sh/id_st
 *   (id_st = 0 broadcasts one list over all Tq queries, the reference's
 *   (B, Hkv, N) form).  ids_heads == Hkv shares a list across a GQA group;
 *   ids_heads == Hq gives every query head its own list.  Entry u selects
 *   tokens [u*unit, (u+1)*unit); -1 entries are skipped.  A unit listed twice
 *   is attended twice, as the reference's gather does (block_sparse.py:62-68).
 * counts (optional, int32 [B][ids_heads][rows] contiguous) bounds the entries
 *   read per list.
 * Tokens >= kv length are masked (block_sparse.py:66-71); with causal != 0
 *   token j is also masked for query t when j > offset + t.
 * Scores use `scale` (the reference uses 1/sqrt(D)); softmax is fp32 online
 * softmax; an empty row yields zeros (the reference divides by max(l,1e-12)).
 * out: (B, Hq, Tq, D) with strides o_sb/o_sh/o_st in out_dtype (F32/BF16).
 * Work is split over the list ("split-K"); num_splits = 0 picks a split count.
 */
typedef struct {
  const void *q;
  void *out;
  const int32_t *ids;
  const int32_t *counts;
  void *workspace;
  int64_t ws_bytes;
  int64_t B, Hq, Hkv, Tq, D;
  int64_t q_sb, q_sh, q_st;
  int64_t o_sb, o_sh, o_st;
  int64_t ids_heads, ids_rows, N;
  int64_t id_sb, id_sh, id_st;
  int64_t unit;
  int64_t offset;
  int64_t num_splits;
  float scale;
  int32_t q_dtype;
  int32_t out_dtype;
  int32_t causal;
} la_sparse_attn_args;

size_t la_sparse_attention_workspace(const la_sparse_attn_args *a, const la_kv *kv);
int la_sparse_attention(const la_sparse_attn_args *a, const la_kv *kv, void *stream);

/*
 * la_sparse_attention without any allocation and without a workspace
 * argument: the split-K partials go to a static device array of
 * LA_NOALLOC_MAX_WORKSPACE bytes that the library keeps on every device it
 * runs on until the process ends (a->workspace / ws_bytes are ignored).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Calls whose la_sparse_attention_workspace() exceeds the
 * limit fail with LA_ERR_WORKSPACE before launching anything.  Every call on
 * one device shares that device's array: calls that overlap in time on one
 * device (other streams, other threads) race; the partials are written whole
 * by each call, so nothing needs clearing between calls.
 */
#define LA_NOALLOC_MAX_WORKSPACE ((size_t)16 << 20)
int la_sparse_attention_noalloc(const la_sparse_attn_args *a, const la_kv *kv, void *stream);

/*
 * Quest page metadata: channel-wise min / max of the keys of every page.
 * Replaces page_bounds_torch / page_update_triton
 * (kernels/triton/quest_pages.py:38-48, 84-100, 134-142) and
 * QuestAttention._refresh_pages (variants/selection.py:181-201).
 * Page p covers logical tokens [p*page_size, min(len,(p+1)*page_size)); pages
 * with no valid token get min = +inf, max = -inf (quest_pages.py:44-46).
 * page_min / page_max: [B][Hkv][n_pages][D] addressed by element strides
 * m_sb/m_sh/m_sp/m_sd (any order; page-minor m_sp == 1 is what
 * la_quest_scores reads fastest), stored in meta_dtype (the key dtype).
 * Pages [first_page, n_pages) are written; first_page > 0 gives the
 * incremental refresh after an append (selection.py:186-190).
 */
int la_quest_page_bounds(const la_kv *kv, int64_t B, int64_t Hkv, int64_t D, int64_t page_size,
                         int64_t first_page, int64_t n_pages, void *page_min, void *page_max,
                         int64_t m_sb, int64_t m_sh, int64_t m_sp, int64_t m_sd, int32_t meta_dtype,
                         void *stream);

/*
 * Quest upper-bound page scores sum_d max(q_d*m_d, q_d*M_d)
 * (quest_pages.py:51-55, selection.py:203-212), one score per query head:
 * scores[((b*Hq + h)*Tq + t)*n_pages + p], fp64.  Products of fp32 or bf16
 * values are exact in fp64 and are summed over d = 0..D-1 in order, so the
 * score is a fixed function of the inputs and selection is reproducible.
 * Masking (visibility, own page) is applied by la_topk_rows.
 */
int la_quest_scores(const void *q, int32_t q_dtype, int64_t B, int64_t Hq, int64_t Tq, int64_t D,
                    int64_t q_sb, int64_t q_sh, int64_t q_st, const void *page_min,
                    const void *page_max, int32_t meta_dtype, int64_t Hkv, int64_t n_pages,
                    int64_t m_sb, int64_t m_sh, int64_t m_sp, int64_t m_sd, double *scores,
                    void *stream);

/*
 * Quest page selection in one pass (scores + top-k + GQA union), for the
 * default union mode of QuestAttention.page_selection (variants/selection.py:
 * 214-237, union at :232-235) over page-minor metadata from
 * la_quest_page_bounds: for every (b, KV head, query t) the Hq/Hkv query
 * heads score all pages exactly as la_quest_scores does, each head keeps its
 * top k = max(1, min(k, n_pages)) visible pages (page start <= pos_offset + t)
 * with the own page forced, and the union of the heads' pages is written in
 * ascending order to out_idx[((b*Hkv + kvh)*Tq + t)*(G*k) + i], -1 padded,
 * with the number kept in out_count.  Identical to la_quest_scores followed by
 * la_topk_rows with group = G, order = 1, force_own = 1, pos_unit = page_size.
 * Returns LA_ERR_UNSUPPORTED (nothing launched) when the metadata is not
 * page-minor (m_sp == 1, m_sd a multiple of 4) or has more pages than one
 * workgroup holds (4096 for G <= 4, 2048 for G = 8); callers then use the two
 * separate entry points.
 */
typedef struct {
  const void *q;
  const void *page_min;
  const void *page_max;
  int32_t *out_idx;
  int32_t *out_count;
  int64_t B, Hq, Hkv, Tq, D;
  int64_t q_sb, q_sh, q_st;
  int64_t n_pages, m_sb, m_sh, m_sp, m_sd;
  int64_t page_size, pos_offset, k;
  int32_t q_dtype, meta_dtype;
  /* Optional per-sequence positions (ragged decode): row (b, kvh, t) uses
   * positions[b] + t in place of pos_offset + t.  NULL: pos_offset. */
  const int32_t *positions;
} la_quest_select_args;

int la_quest_select(const la_quest_select_args *a, void *stream);

/*
 * Fused Quest decode: page selection and attention in one kernel, the
 * fusion of selector and decode kernel that docs/kernels.md:89-93 describes
 * (FFD) beyond the fused top-k of quest_pages.py:110-113: the selected page
 * list never leaves the chip before it is attended.  Replaces
 * la_quest_select followed by la_sparse_attention for one decode query per
 * sequence.  One workgroup of 512 threads per (b, KV head): the
 * la_quest_select union selection of the G = Hq/Hkv query heads (select.Tq
 * == 1; the list is also written to select.out_idx / out_count exactly as
 * la_quest_select writes it; G in {2, 4}), then the matrix-core attention of the G heads
 * over those pages of the paged pool `kv` (bf16 K/V, page_table, page_size a
 * multiple of 16 and equal to select.page_size, head_dim 128, bf16 q),
 * causal at the query's position (select.pos_offset, or select.positions[b])
 * and within kv.kv_len, scale times q.k, output (B, Hq, 1, 128) at the o_*
 * element strides in out_dtype (LA_F32, LA_BF16 or LA_F16).  Other shapes
 * return LA_ERR_UNSUPPORTED with nothing launched.  No workspace.
 */
typedef struct {
  la_quest_select_args select;
  la_kv kv;
  void *out;
  int64_t o_sb, o_sh, o_st;
  float scale;
  int32_t out_dtype;
} la_quest_decode_args;

int la_quest_decode_fused(const la_quest_decode_args *a, void *stream);

/*
 * Paged KV append with Quest page bounds maintained in the same pass.
 * Fuses the KV concatenation of AttentionVariant.push_kv (core.py:219-220)
 * with the incremental refresh of QuestAttention._refresh_pages
 * (variants/selection.py:181-201), and for an fp8 pool the per-token codec of
 * kv/quant.py:76-93 (group = head_dim: scale = max(absmax, 1e-8)/448, codes =
 * e4m3fn(x / scale)).
 * The Tn new tokens of sequence b (k_new / v_new at element strides
 * n_sb/n_sh/n_st: (B, Hkv, Tn, D)) go to logical positions positions[b] ..
 * positions[b] + Tn - 1, i.e. slot t % pool_page of physical page
 * page_table[b*pt_sb + t/pool_page] of the pools (n_phys, Hkv, pool_page, D),
 * contiguous; tokens whose table entry lies outside [0, n_phys) are dropped
 * (neither stored nor counted in the bounds).  With
 * page_min / page_max ((B, Hkv, n_pages, D) at element strides
 * m_sb/m_sh/m_sp/m_sd, in the key dtype), every Quest page of meta_page tokens
 * that the new tokens touch gets its channel-wise bounds updated: a page that
 * starts at or after positions[b] is set to the new tokens' bounds, any other
 * takes min / max with its stored bounds.  For an append at the end of the
 * sequence (positions[b] = its length) this equals la_quest_page_bounds over
 * the grown sequence, bit for bit.  fp8 pools take no bounds.
 */
typedef struct {
  const void *k_new;
  const void *v_new;
  void *k_pool;
  void *v_pool;
  float *k_scale; /* fp8 pool: (n_phys, Hkv, pool_page) per-token scales */
  float *v_scale; /* (pool row r's at r * s_stride) */
  const int32_t *page_table;
  const int32_t *positions;
  void *page_min;
  void *page_max;
  int64_t B, Hkv, Tn, D;
  int64_t n_sb, n_sh, n_st;
  int64_t n_phys, pool_page, pt_sb, pt_pages;
  int64_t meta_page, n_pages, m_sb, m_sh, m_sp, m_sd;
  int32_t in_dtype;   /* LA_F32 or LA_BF16 */
  int32_t pool_dtype; /* in_dtype, or LA_FP8_E4M3 */
  int64_t s_stride;   /* fp8 pool: scale elements between pool rows (0 reads as 1;
                         2: K and V scales interleaved, v_scale = k_scale + 1) */
} la_kv_append_args;

int la_paged_kv_append(const la_kv_append_args *a, void *stream);

/*
 * Row-wise top-k with ties broken by lowest index.
 * Replaces topk_blocks (variants/selection.py:51-59), the torch.topk calls of
 * page_select_torch / page_select_triton (quest_pages.py:76-77, 159-160),
 * QuestAttention.page_selection (selection.py:214-237) and the selection of
 * MInferenceAttention._block_sparse (selection.py:339-353).
 *
 * scores: fp64 rows (b, h, t) at scores[((b*H + h)*Tq + t)*row_stride + i],
 *   i < n.  Row (b, h, t) considers i < n_valid[t] (all n when NULL).
 * pos_unit > 0 derives both tables from positions instead: with
 *   pos = pos_offset + t, n_valid = min(n, pos/pos_unit + 1) (units whose
 *   start is <= pos: the Quest visibility rule, selection.py:219-223) and
 *   own = min(pos/pos_unit, n-1) (selection.py:224); explicit tables win.
 * force_own: unit own[t] ranks above everything, inside the k budget (the
 *   Quest own-page rule, selection.py:224-231).
 * k: per row, min(k, valid) entries are kept (entries the reference would
 *   take from masked -inf scores are never read, selection.py:96-98).
 * group G > 1: the G consecutive heads h = g*G..g*G+G-1 are unioned (Quest
 *   gqa_union, selection.py:232-235).
 * sink_units / window_units (C3 composition): units [0, sink_units) and
 *   [own[t]-window_units+1, own[t]] are OR'd in after the top-k.
 * Output per group (b, g, t): out_idx[((b*(H/G)+g)*Tq+t)*width + j],
 *   -1 padded; order 0 sorts by (score desc, index asc) -- only for G == 1
 *   and no sink/window -- order 1 sorts by ascending index.  out_val
 *   (optional, order 0 only) gets the fp32 scores, -inf for padding;
 *   out_count (optional) the number of valid entries.
 */
typedef struct {
  const double *scores;
  int32_t *out_idx;
  float *out_val;
  int32_t *out_count;
  const int32_t *n_valid;
  const int32_t *own;
  void *workspace;
  int64_t ws_bytes;
  int64_t B, H, Tq, n, row_stride;
  int64_t group, k, width;
  int64_t sink_units, window_units;
  int64_t pos_offset, pos_unit;
  int32_t force_own;
  int32_t order;
} la_topk_args;

size_t la_topk_rows_workspace(const la_topk_args *a);
int la_topk_rows(const la_topk_args *a, void *stream);

/*
 * Lightning-indexer top-k (DSA): I[b,t,s] = sum_h w[b,t,h] * ReLU(q[b,t,h].k[b,s,h])
 * and the k highest-scoring keys per query, ties to the lowest index.
 * Replaces indexer_topk / indexer_topk_triton / indexer_topk_torch
 * (kernels/triton/fused_indexer.py:52-73, 153-206).
 * q_idx: (B, Tq, HI, d), k_idx: (B, Tk, HI, d) in F32 or BF16 with element
 * strides (unit stride over d); w: fp32 (B, Tq, HI) with strides.
 * Scores are computed in fp64: each q.k product is exact, summed over d in
 * order, then ReLU, then sum over heads h = 0..HI-1 of fl(w_h * relu_h).
 * causal != 0 keeps keys s <= offset + t only (an addition; the reference
 * scores every key, fused_indexer.py:63-73).  With causal_unit = m > 1 the
 * keys are pooled groups of m tokens and group s is kept when s*m <= offset+t
 * (the compressed-indexing mask of selection.py:739-747); 0 or 1 = tokens.
 * order 0: out_idx int32 (B, Tq, k) sorted by (score desc, index asc), -1
 * padded; out_val fp32 (B, Tq, k), -inf padded (optional).
 * order 1 (an addition): the same selected keys in ascending index order,
 * -1 padded, out_val must be NULL (no sort is done; the selection is the set
 * a token mask is built from, selection.py:752-761).
 * q_chunk bounds the queries scored per pass (workspace = q_chunk*Tk*8 bytes
 * plus the top-k scratch); 0 picks one.
 */
typedef struct {
  const void *q;
  const void *kk;
  const float *w;
  int32_t *out_idx;
  float *out_val;
  void *workspace;
  int64_t ws_bytes;
  int64_t B, Tq, Tk, HI, d, k;
  int64_t q_sb, q_st, q_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t w_sb, w_st, w_sh;
  int64_t offset;
  int64_t q_chunk;
  int64_t causal_unit;
  int32_t in_dtype;
  int32_t causal;
  int32_t order; /* 0 = by score (sorted), 1 = ascending index */
  int32_t reserved;
} la_indexer_args;

size_t la_indexer_topk_workspace(const la_indexer_args *a);
int la_indexer_topk(const la_indexer_args *a, void *stream);

/*
 * Block selection for block-sparse prefill (config C3 composition of
 * MInferenceAttention._block_sparse, variants/selection.py:339-353, with
 * block_reduce mean pooling, core.py:102-120): per (b, h, query block qb)
 *   score(qb, kb) = mean_pool(q)[qb] . mean_pool(k)[kb]   (fp64, in order)
 * over kb <= qb, top `topk` by (score desc, kb asc), OR the sink blocks
 * [0, sink_blocks) and the window [qb-window_blocks+1, qb].
 * q: (B, Hq, T, D), k: (B, Hkv, T, D), F32 or BF16, strides as above.
 * Output out_idx (B, Hq, nqb, width) ascending, -1 padded; out_count (B,Hq,nqb).
 * The positive 1/sqrt(D) factor of the reference does not change the ranking
 * and is not applied.
 * Ragged batches: lengths (optional, int32 [B] on the device) gives sequence
 * b's length L_b in [0, T]; its rows past L_b are padding and are never read
 * (the tail block repeats row L_b - 1), query blocks at or past L_b get empty
 * lists (count 0), and every other list equals that of a call on sequence b
 * alone with T = L_b.  The reference batches equal lengths only
 * (core.py:250-252; its roadmap, docs/roadmap.md:6-25, names this extension).
 */
typedef struct {
  const void *q;
  const void *k;
  int32_t *out_idx;
  int32_t *out_count;
  void *workspace;
  int64_t ws_bytes;
  int64_t B, Hq, Hkv, T, D;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t block, topk, sink_blocks, window_blocks, width;
  int32_t in_dtype;
  int32_t reserved;
  const int32_t *lengths; /* optional: per-sequence lengths (ragged batch) */
} la_block_select_args;

size_t la_block_select_workspace(const la_block_select_args *a);
int la_block_select(const la_block_select_args *a, void *stream);

/*
 * Per-query block routing: the gate of MoBAAttention.select
 * (variants/selection.py:624-634) and the blockwise selection of
 * NSAAttention.selection_mask (variants/native_sparse.py:78-93), which compute
 * the same lists.  For query t of (b, h) at position pos = offset + t, key
 * block j (tokens [j*block, (j+1)*block), the tail block padded by repeating
 * the last row as block_reduce does, core.py:115-117) is visible when
 * j*block <= pos; the gate is q_t . mean(K block j) in fp64 (products added
 * over d in order; the positive 1/sqrt(D) of the reference is left out, it
 * does not change the ranking); the top min(topk, visible) visible blocks are
 * kept (ties to the lowest block) and the query's own block pos/block is OR'd
 * in (selection.py:632-633).
 * q: (B, Hq, Tq, D), k: (B, Hkv, T, D) at element strides; query head h reads
 * KV head h / (Hq/Hkv).  Output: out_idx[((b*Hq + h)*Tq + t)*width + i]
 * ascending, -1 padded (width >= min(topk, blocks) + 1), out_count the number
 * kept.  Workspace: la_gate_select_workspace bytes (fp64 q, pooled keys and
 * the gate rows).  kbar (optional): the block means of k, (B, Hkv, n_kb, D)
 * fp64 contiguous as la_block_means writes them; given, k is not read and
 * not pooled (the per-step pooling of selection.py:620-624 is replaced by
 * means kept up to date on append).
 */
typedef struct {
  const void *q;
  const void *k;
  int32_t *out_idx;
  int32_t *out_count;
  void *workspace;
  int64_t ws_bytes;
  int64_t B, Hq, Hkv, Tq, T, D;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t block, topk, offset, width;
  int32_t in_dtype;
  int32_t reserved;
  const double *kbar;
} la_gate_select_args;

size_t la_gate_select_workspace(const la_gate_select_args *a);
int la_gate_select(const la_gate_select_args *a, void *stream);

/*
 * Block means of keys for the gate routing, kept across decode steps.
 * Replaces the block_reduce pooling that MoBAAttention.select repeats over
 * every key at every call (variants/selection.py:620-624; core.py:102-120):
 * a decode step re-pools only the block its new key landed in.  Block j of
 * (b, h) is written as la_gate_select pools it: fp64, rows j*block ..
 * j*block + block - 1 added in order and the sum divided by `block`, rows
 * at or past T_b repeating row T_b - 1 (T_b = lengths[b] clamped to [0, T]
 * when given, else T; a sequence without rows gets zeros).  Blocks pooled:
 * first_block .. first_block + n_blocks - 1 of every (b, h), or, with
 * `positions` (int32 (B,)), only block positions[b] / block of sequence b
 * (entries outside [0, n_kb) pool nothing).  k: (B, H, T, D) at element
 * strides, unit stride over D; out: (B, H, n_kb, D) fp64 contiguous,
 * n_kb = ceil(T / block); blocks not pooled keep their contents.  No
 * workspace.
 */
typedef struct {
  const void *k;
  double *out;
  const int32_t *positions;
  const int32_t *lengths;
  int64_t B, H, T, D;
  int64_t k_sb, k_sh, k_st;
  int64_t block, first_block, n_blocks;
  int32_t in_dtype;
  int32_t reserved;
} la_block_means_args;

int la_block_means(const la_block_means_args *a, void *stream);

/*
 * XAttention block selection: XAttention.antidiagonal_scores / select
 * (variants/selection.py:528-595).  Replaces the torch selection path of that
 * variant (no kernel backend exists for it in the reference).  Blocks of
 * `block` tokens; query block qb of (b, h) (rows past Tq are zero rows, F.pad
 * at :544) against key block kb of KV head h / (Hq/Hkv) (rows past T zero);
 * visible when kb*block <= qb*block + offset (:573-575).  Slot s, for
 * antidiagonal offset o = s*stride <= 2*block - 2 (:554), is the sum over
 * i = max(0, o-block+1) .. min(block-1, o), increasing, of the fp64 dot
 * product q[qb*block + i] . k[kb*block + o - i] (d increasing), times
 * inv_sqrt_d (the caller's fl(1/fl(sqrt(D))), :566).  Per row: weights
 * exp(slot - max) over the visible slots (a fixed fma sequence, bit-identical
 * in the CPU oracle), as integers rint(w * 2^F), F = 52 - ceil(log2(n_kb *
 * n_slots)); block mass = the sum over its slots (:576-579, unnormalised).
 *   mode 0 (threshold, _cumulative_select :62-69 / per-head thresholds
 *     :587-589): with blocks ordered by (mass desc, index asc), keep
 *     1 + #{m : C_m < ceil(alpha[h] * Z)} blocks (C_m the sum of the first m
 *     masses, Z the total; alpha[h] * Z > Z keeps all);
 *   mode 1 (top-k, :581-582): the top min(topk, n_kb) blocks in that order.
 * The own block (first token qb*block + offset) is OR'd in and blocks past
 * causality are dropped (:591-592).  Output: out_idx[((b*Hq + h)*n_qb + qb)
 * *width + i] ascending, -1 padded, width >= n_kb (mode 0) or
 * min(topk, n_kb) + 1 (mode 1); out_count[(b*Hq + h)*n_qb + qb].  Limits:
 * block <= 64, n_kb <= 4096, LDS block*D*4 + n_kb*n_slots*8 <= 120 KiB.
 * Workspace (optional): with workspace >= la_xattn_select_workspace() bytes,
 * shapes with stride == block >= 2, 2-byte q/k and 16-byte aligned rows
 * (D a multiple of 8) score on the fp64 matrix cores first (for stride ==
 * block the antidiagonal entries pair query rows i mod block with key rows
 * -i mod block: block dense gram products per head, in-order fp64
 * accumulation over d, the same bits) and the selection reads the slots from
 * the workspace; otherwise the selection kernel scores every slot itself.
 * The slots of a chunk of query blocks are scored and then selected, chunk
 * after chunk: la_xattn_select_workspace() sizes the chunk so that its slots
 * take at most 256 MiB (at least one chunk of 64 query blocks), and a smaller
 * workspace (B*Hq*64*n_kb*n_slots*8 bytes or more) gives smaller chunks with
 * the same lists.  la_xattn_select_workspace() returns 0 when no workspace
 * is used.
 */
typedef struct {
  const void *q;
  const void *k;
  int32_t *out_idx;
  int32_t *out_count;
  const double *alpha; /* device, Hq thresholds (mode 0) */
  int64_t B, Hq, Hkv, Tq, T, D;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t block, stride, offset, topk, width;
  double inv_sqrt_d;
  int32_t mode;
  int32_t in_dtype;
  void *workspace;
  int64_t ws_bytes;
} la_xattn_select_args;

size_t la_xattn_select_workspace(const la_xattn_select_args *a);
int la_xattn_select(const la_xattn_select_args *a, void *stream);

/*
 * Block-sparse causal prefill on the matrix cores (fp32 accumulate).
 * The executor of block_sparse_attention (block_sparse.py:80-163) for lists
 * shared by a whole query block: query block qb of head h attends the key
 * blocks ids[b][h][qb][0..count) of block_size 64 tokens, with the causal mask
 * j <= i applied in-kernel (the reference's selector applies it through the
 * token mask, selection.py:86-108).  q (B,Hq,T,128), k/v (B,Hkv,T,128) bf16;
 * out (B,Hq,T,128) in out_dtype (F32 or BF16).  Scores by bf16 MFMA; the
 * softmax weights and V enter the PV product as fp16 (V converted once into
 * the workspace, each 64-token block scaled by a power of two that keeps it
 * in fp16 range).  scale must be positive.  Workspace:
 * la_block_sparse_prefill_workspace() bytes, 256-byte aligned.
 * Ragged batches: lengths (optional, int32 [B] on the device) gives sequence
 * b's length L_b in [0, T]; q/k/v rows of sequence b at or past L_b are
 * padding and are never read, its output rows there are written as zeros,
 * and its other rows equal a call on sequence b alone with T = L_b.
 * fp8 K/V (kv_dtype LA_FP8_E4M3): k/v hold OCP e4m3 codes (element strides in
 * bytes, 8-byte aligned rows) with per-token fp32 scales k_scale/v_scale
 * (B, Hkv, T) at strides s_sb/s_sh/s_st, the codec of kv/quant.py:76-109
 * with group_size == head_dim.  K's codes are scored exactly (fp16 MFMA
 * against q converted per row to fp16 with a power-of-two scale) and each
 * score is multiplied by its key's scale; V is dequantized into the fp16
 * copy.  Any other kv_dtype means bf16 K/V.
 */
typedef struct {
  const void *q;
  const void *k;
  const void *v;
  void *out;
  const int32_t *ids;
  const int32_t *counts;
  void *workspace;
  int64_t ws_bytes;
  int64_t B, Hq, Hkv, T, D;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int64_t block, width;
  float scale;
  int32_t causal;
  int32_t out_dtype;
  int32_t reserved;
  const int32_t *lengths; /* optional: per-sequence lengths (ragged batch) */
  const float *k_scale;   /* fp8 K/V only: per-token scales */
  const float *v_scale;
  int64_t s_sb, s_sh, s_st;
  int32_t kv_dtype; /* LA_FP8_E4M3, or bf16 K/V */
  int32_t reserved2;
} la_prefill_args;

size_t la_block_sparse_prefill_workspace(const la_prefill_args *a);
int la_block_sparse_prefill(const la_prefill_args *a, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LINATTN_HIP_H */
