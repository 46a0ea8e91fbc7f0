"""Quest page metadata, page scores and page selection on gfx950.

Mirrors kernels/triton/quest_pages.py:38-161 (``page_update_triton``,
``page_select_triton``) and the selection of QuestAttention
(variants/selection.py:139-248).  Differences by design:

* scores are fp64 and a fixed function of the inputs (products exact, summed
  over d in order), so page ids are reproducible bit for bit;
* ties go to the lowest page index (torch.topk leaves the order unspecified);
* the own page is forced per query row (selection.py:224-231), not with the
  (T_q, T_q) block write of quest_pages.py:75 / :159 (defect for T_q > 1);
* every KV head has its own metadata (the Triton kernels ignore the head
  index, quest_pages.py:94-100, 124-130);
* metadata is stored page-minor ([B][Hkv][D][P]) and returned as a
  (B, Hkv, P, D) view, so the scoring kernel reads 4 pages per 8-byte load.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from linattn_amd import _native as N

__all__ = [
    "page_update_hip",
    "page_scores_hip",
    "page_select_hip",
    "quest_select_hip",
    "page_update_triton",
    "page_select_triton",
    "alloc_page_meta",
]


def alloc_page_meta(B: int, Hkv: int, n_pages: int, D: int, dtype: torch.dtype,
                    device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Empty (mins, maxs) with page-minor storage, viewed as (B, Hkv, P, D)."""
    p4 = (n_pages + 3) // 4 * 4
    store = torch.empty(2, B, Hkv, D, p4, dtype=dtype, device=device)
    return store[0, ..., :n_pages].transpose(-1, -2), store[1, ..., :n_pages].transpose(-1, -2)


def page_update_hip(k: torch.Tensor, page_size: int, n_pages: Optional[int] = None, *,
                    page_table: Optional[torch.Tensor] = None, pool_page_size: Optional[int] = None,
                    kv_len: Optional[torch.Tensor] = None,
                    out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                    first_page: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Channel-wise key min/max per page (quest_pages.py:38-48, 134-142).

    k: (B, Hkv, T, D) fp32/bf16, or a paged pool (n_phys, Hkv, pool_page, D)
    with ``page_table`` (B, pages) int32.  Returns (mins, maxs), each
    (B, Hkv, n_pages, D) in k's dtype; pages with no valid token hold +inf / -inf.
    ``out`` + ``first_page`` refreshes pages [first_page, n_pages) in place (the
    incremental update of selection.py:181-201)."""
    dev = N.require_gpu(k, page_table, kv_len, what="page_update_hip")
    from linattn_amd.kernels.block_sparse import _kv_struct

    if page_table is not None:
        B, Hkv, D = page_table.shape[0], k.shape[1], k.shape[3]
        pps = int(pool_page_size or k.shape[2])
        T = page_table.shape[1] * pps
        kv = _kv_struct(k, k, page_table=page_table, page_size=pps, kv_len=kv_len, k_scale=None,
                        v_scale=None, T=T, D=D, Hkv=Hkv)
    else:
        B, Hkv, T, D = k.shape
        kv = _kv_struct(k, k, page_table=None, page_size=None, kv_len=kv_len, k_scale=None,
                        v_scale=None, T=T, D=D, Hkv=Hkv)
    if n_pages is None:
        n_pages = (T + page_size - 1) // page_size
    if out is None:
        mins, maxs = alloc_page_meta(B, Hkv, n_pages, D, k.dtype, dev)
    else:
        mins, maxs = out
        if mins.shape != (B, Hkv, n_pages, D) or maxs.shape != mins.shape:
            raise ValueError("out must be two (B, Hkv, n_pages, D) tensors")
        if mins.stride() != maxs.stride():
            raise ValueError("mins and maxs must share strides")
    sb, sh, sp, sd = mins.stride()
    N.check(N.load().la_quest_page_bounds(ctypes.byref(kv), B, Hkv, D, page_size, first_page,
                                          n_pages, mins.data_ptr(), maxs.data_ptr(), sb, sh, sp,
                                          sd, N.dtype_code(mins.dtype), N.stream_handle(dev)),
            "page_update_hip")
    return mins, maxs


def page_scores_hip(q: torch.Tensor, mins: torch.Tensor, maxs: torch.Tensor,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Upper-bound scores sum_d max(q_d m_d, q_d M_d), fp64 (B, Hq, Tq, P)
    (quest_pages.py:51-55); query head h reads KV head h // (Hq/Hkv)."""
    dev = N.require_gpu(q, mins, maxs, what="page_scores_hip")
    B, Hq, Tq, D = q.shape
    Hkv, P = mins.shape[1], mins.shape[2]
    if mins.shape != (B, Hkv, P, D) or maxs.shape != mins.shape or mins.stride() != maxs.stride():
        raise ValueError("mins/maxs must be (B, Hkv, P, D) with equal strides")
    if mins.dtype != maxs.dtype:
        raise ValueError("mins/maxs dtype mismatch")
    if out is None:
        out = torch.empty(B, Hq, Tq, P, dtype=torch.float64, device=dev)
    elif out.shape != (B, Hq, Tq, P) or out.dtype != torch.float64 or not out.is_contiguous():
        raise ValueError("out must be contiguous fp64 (B, Hq, Tq, P)")
    qs = q.stride()
    ms = mins.stride()
    N.check(N.load().la_quest_scores(q.data_ptr(), N.dtype_code(q.dtype), B, Hq, Tq, D, qs[0], qs[1],
                                     qs[2], mins.data_ptr(), maxs.data_ptr(),
                                     N.dtype_code(mins.dtype), Hkv, P, ms[0], ms[1], ms[2], ms[3],
                                     out.data_ptr(), N.stream_handle(dev)),
            "page_scores_hip")
    return out


def _topk(scores: torch.Tensor, *, k: int, width: int, group: int, order: int,
          pos_offset: int, pos_unit: int, force_own: bool, with_values: bool = False,
          sink: int = 0, window: int = 0, n_valid: Optional[torch.Tensor] = None):
    B, H, Tq, n = scores.shape
    dev = scores.device
    if n_valid is not None and (n_valid.dtype != torch.int32 or n_valid.shape != (Tq,)
                                or not n_valid.is_contiguous()):
        raise ValueError("n_valid must be contiguous int32 (Tq,)")
    ids = torch.empty(B, H // group, Tq, width, dtype=torch.int32, device=dev)
    counts = torch.empty(B, H // group, Tq, dtype=torch.int32, device=dev)
    vals = torch.empty(B, H, Tq, width, dtype=torch.float32, device=dev) if with_values else None
    a = N.LaTopkArgs()
    a.scores, a.out_idx, a.out_count = scores.data_ptr(), ids.data_ptr(), counts.data_ptr()
    a.out_val = N.ptr(vals)
    a.B, a.H, a.Tq, a.n, a.row_stride = B, H, Tq, n, scores.stride(2)
    a.group, a.k, a.width = group, k, width
    a.sink_units, a.window_units = sink, window
    a.pos_offset, a.pos_unit = pos_offset, pos_unit
    a.force_own, a.order = int(force_own), order
    a.n_valid = N.ptr(n_valid)
    L = N.load()
    ws_bytes = L.la_topk_rows_workspace(ctypes.byref(a))
    ws = N.workspace(ws_bytes, dev)
    a.workspace, a.ws_bytes = N.ptr(ws), ws_bytes
    N.check(L.la_topk_rows(ctypes.byref(a), N.stream_handle(dev)), "top-k")
    return ids, counts, vals


def quest_select_hip(q: torch.Tensor, mins: torch.Tensor, maxs: torch.Tensor, *, page_size: int,
                     topk: int, offset: int = 0, gqa_union: bool = True,
                     positions: Optional[torch.Tensor] = None
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
    """QuestAttention.page_selection (selection.py:214-237) as page lists.

    Visible pages (start <= offset + t) are ranked; the query's own page is
    forced inside the budget; k = max(1, min(topk, n_pages)).  With
    ``gqa_union`` (the reference default) the G query heads of a KV head read
    the union of their pages: ids (B, Hkv, Tq, G*k) ascending, -1 padded.
    Otherwise each query head keeps its own list: ids (B, Hq, Tq, k) by
    (score desc, index asc).  Also returns counts (valid entries per list).
    ``positions`` (int32 (B,), ragged batches) replaces ``offset`` per
    sequence: query t of sequence b sits at positions[b] + t."""
    dev = N.require_gpu(q, mins, maxs, positions, what="quest_select_hip")
    B, Hq, Tq, D = q.shape
    Hkv, P = mins.shape[1], mins.shape[2]
    G = Hq // Hkv
    k = max(1, min(int(topk), P))
    if mins.shape != (B, Hkv, P, D) or maxs.shape != mins.shape or Hq % Hkv:
        raise ValueError("mins/maxs must be (B, Hkv, P, D) with Hq a multiple of Hkv")
    if positions is not None and (positions.dtype != torch.int32 or positions.shape != (B,)
                                  or not positions.is_contiguous()):
        raise ValueError("positions must be contiguous int32 (B,)")
    if gqa_union and G > 1 and mins.stride() == maxs.stride() and mins.dtype == maxs.dtype:
        # one pass: scores, per-head top-k and the union (la_quest_select)
        ids = torch.empty(B, Hkv, Tq, G * k, dtype=torch.int32, device=dev)
        counts = torch.empty(B, Hkv, Tq, dtype=torch.int32, device=dev)
        a = N.LaQuestSelectArgs()
        a.q, a.page_min, a.page_max = q.data_ptr(), mins.data_ptr(), maxs.data_ptr()
        a.out_idx, a.out_count = ids.data_ptr(), counts.data_ptr()
        a.B, a.Hq, a.Hkv, a.Tq, a.D = B, Hq, Hkv, Tq, D
        a.q_sb, a.q_sh, a.q_st = q.stride(0), q.stride(1), q.stride(2)
        a.n_pages = P
        a.m_sb, a.m_sh, a.m_sp, a.m_sd = mins.stride()
        a.page_size, a.pos_offset, a.k = page_size, offset, k
        a.q_dtype, a.meta_dtype = N.dtype_code(q.dtype), N.dtype_code(mins.dtype)
        a.positions = N.ptr(positions)
        rc = N.load().la_quest_select(ctypes.byref(a), N.stream_handle(dev))
        if rc != N.LA_ERR_UNSUPPORTED:
            N.check(rc, "quest_select_hip")
            return ids, counts
    if positions is not None:
        # two-pass path: one selection per sequence at its own position
        # (reads the positions on the host)
        parts = [quest_select_hip(q[b:b + 1], mins[b:b + 1], maxs[b:b + 1], page_size=page_size,
                                  topk=topk, offset=int(pb), gqa_union=gqa_union)
                 for b, pb in enumerate(positions.tolist())]
        return torch.cat([p[0] for p in parts]), torch.cat([p[1] for p in parts])
    scores = page_scores_hip(q, mins, maxs)
    if gqa_union and G > 1:
        ids, counts, _ = _topk(scores, k=k, width=G * k, group=G, order=1, pos_offset=offset,
                               pos_unit=page_size, force_own=True)
    else:
        ids, counts, _ = _topk(scores, k=k, width=k, group=1, order=0, pos_offset=offset,
                               pos_unit=page_size, force_own=True)
    return ids, counts


def page_select_hip(q: torch.Tensor, mins: torch.Tensor, maxim: torch.Tensor, page_size: int,
                    topk: int, *, offset: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-k page ids per query plus the page scores (quest_pages.py:58-78, 145-161).

    Returns ids int32 (B, H, Tq, k) ordered by (score desc, index asc), -1 where
    fewer than k pages are visible, and fp32 scores (B, H, Tq, P) with
    invisible pages -inf and the own page +inf, as the reference does."""
    scores = page_scores_hip(q, mins, maxim)
    B, H, Tq, P = scores.shape
    k = max(1, min(int(topk), P))
    ids, _, _ = _topk(scores, k=k, width=k, group=1, order=0, pos_offset=offset,
                      pos_unit=page_size, force_own=True)
    pos = torch.arange(Tq, device=q.device) + offset
    visible = (torch.arange(P, device=q.device) * page_size).unsqueeze(0) <= pos.unsqueeze(1)
    out = scores.to(torch.float32).masked_fill(~visible, float("-inf"))
    own = torch.clamp(pos // page_size, max=P - 1)
    out.scatter_(-1, own.view(1, 1, Tq, 1).expand(B, H, Tq, 1), float("inf"))
    return ids, out


def page_update_triton(k: torch.Tensor, page_size: int, n_pages: int):
    """Drop-in alias for kernels/triton/quest_pages.py:134 (runs the HIP kernel)."""
    return page_update_hip(k, page_size, n_pages)


def page_select_triton(q, mins, maxim, page_size: int, topk: int, *, offset: int = 0):
    """Drop-in alias for kernels/triton/quest_pages.py:145 (runs the HIP kernels)."""
    return page_select_hip(q, mins, maxim, page_size, topk, offset=offset)
