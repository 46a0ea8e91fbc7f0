"""Paged sparse decode on gfx950.

``paged_decode`` keeps the reference's single-(head, query) C entry point
(kernels/c_attention.py:76-111, kernels/c/decode_attn.c:39-133) and runs it on
the GPU.  ``quest_decode_step`` is the batched decode hot path: Quest page
selection over a paged KV pool followed by split-K attention over the selected
pages (the decode step of QuestAttention, variants/selection.py:139-248, driven
by AttentionVariant.forward, core.py:231-279).  ``quest_decode_fused`` runs
the same step as one kernel: each (b, KV head) workgroup selects its pages and
attends them without the list leaving the chip.
"""

from __future__ import annotations

import ctypes
import math
from typing import Dict, Optional, Tuple

import torch

from linattn_amd import _native as N
from linattn_amd.kernels.block_sparse import _kv_struct, sparse_attention
from linattn_amd.kernels.fused_indexer import indexer_topk
from linattn_amd.kernels.quest_pages import quest_select_hip

__all__ = ["paged_decode", "quest_decode_step", "quest_decode_fused", "indexer_decode_step",
           "quantize_fp8_per_token"]


def quantize_fp8_per_token(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp8 e4m3 codec of kv/quant.py:76-93 with group = head_dim: scale =
    max|x| / 448 per row (clamped to 1e-8), codes = (x / scale) cast to
    float8_e4m3fn.  Returns (codes, fp32 scales without the last dim)."""
    xf = x.to(torch.float32)
    scale = xf.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 448.0
    return (xf / scale).to(torch.float8_e4m3fn), scale.squeeze(-1)


def indexer_decode_step(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                        page_table: torch.Tensor, q_idx: torch.Tensor, k_idx: torch.Tensor,
                        head_weights: torch.Tensor, *, topk: int, pos: int, page_size: int,
                        k_scale: Optional[torch.Tensor] = None,
                        v_scale: Optional[torch.Tensor] = None,
                        out_dtype: Optional[torch.dtype] = None
                        ) -> Tuple[torch.Tensor, torch.Tensor]:
    """One DSA-style decode step (config C5): the lightning indexer picks
    ``topk`` tokens per sequence (causal, one list shared by every head,
    fused_indexer.py:52-73), then every query head attends those tokens of the
    paged (optionally fp8) cache.  q (B, Hq, 1, D); q_idx (B, 1, H_I, d);
    k_idx (B, T, H_I, d); head_weights (B, 1, H_I).  Returns (out, token ids):
    the selected set in ascending order, -1 padded (the attention reads a set,
    as the reference's token mask does, selection.py:752-761, so the ids are
    not sorted by score)."""
    B, Hkv = q.shape[0], k_pool.shape[1]
    _, idx = indexer_topk(q_idx, k_idx, head_weights, topk, causal=True, offset=pos, sorted=False)
    ids = idx.view(B, 1, 1, -1).expand(B, Hkv, 1, idx.shape[-1])
    out = sparse_attention(q, k_pool, v_pool, ids, unit=1, causal=True, offset=pos,
                           page_table=page_table, page_size=page_size, k_scale=k_scale,
                           v_scale=v_scale, out_dtype=out_dtype)
    return out, idx


def paged_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, page_ids: torch.Tensor, *,
                 page_size: int, kernel: str = "hip") -> Tuple[torch.Tensor, Dict[str, int]]:
    """Attention for one (head, query) over selected pages (c_attention.py:76-111).

    q: (dim,), k/v: (n_tokens, dim), page_ids: (n_pages,).  Tokens past the end
    are skipped (decode_attn.c:49).  Returns (out fp32 (dim,), stats) where
    stats counts the KV entries actually read (tails and repeated pages
    included, unlike c_attention.py:105)."""
    if kernel not in ("hip", "naive", "tiled"):
        raise ValueError(f"unknown kernel {kernel!r}")
    dim = q.numel()
    if dim > 512:
        raise ValueError("the C kernel supports head_dim <= 512")
    t = k.shape[0]
    ids = page_ids.to(torch.int32).reshape(1, 1, 1, -1).contiguous()
    out = sparse_attention(q.reshape(1, 1, 1, dim), k.reshape(1, 1, t, dim),
                           v.reshape(1, 1, t, dim), ids, unit=page_size,
                           scale=1.0 / math.sqrt(dim), out_dtype=torch.float32)
    starts = page_ids.to(torch.int64) * page_size
    per_page = torch.clamp(t - starts, min=0, max=page_size)
    read_entries = int(per_page.sum())
    stats = {"kv_entries": read_entries, "bytes": read_entries * dim * 2 * k.element_size(),
             "dense_entries": int(t)}
    return out.reshape(dim), stats


def quest_decode_step(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                      page_table: torch.Tensor, page_min: torch.Tensor, page_max: torch.Tensor, *,
                      page_size: int, topk: int, pos: Optional[int] = None,
                      positions: Optional[torch.Tensor] = None, gqa_union: bool = True,
                      kv_len: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                      out_dtype: Optional[torch.dtype] = None, num_splits: int = 0
                      ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One Quest decode step: every sequence at position ``pos``, or (ragged
    batches) sequence b at ``positions[b]`` (int32 (B,)).

    q: (B, Hq, 1, D); k/v pools (n_phys, Hkv, page_size, D); page_table int32
    (B, pages); page_min/max (B, Hkv, pages, D).  Selects ``topk`` pages per
    query head (own page forced, GQA union by default) and attends them; with
    ``positions`` the keys of sequence b are those before positions[b] + 1.
    Returns (out (B, Hq, 1, D), ids, counts)."""
    if (pos is None) == (positions is None):
        raise ValueError("pass exactly one of pos and positions")
    if positions is not None:
        if q.shape[2] != 1:
            raise ValueError("positions: one query per sequence (decode)")
        ids, counts = quest_select_hip(q, page_min, page_max, page_size=page_size, topk=topk,
                                       gqa_union=gqa_union, positions=positions)
        lens = positions + 1
        if kv_len is not None:
            lens = torch.minimum(lens, kv_len)
        out = sparse_attention(q, k_pool, v_pool, ids, unit=page_size, counts=counts,
                               causal=False, page_table=page_table, page_size=page_size,
                               kv_len=lens.to(torch.int32), scale=scale, out_dtype=out_dtype,
                               num_splits=num_splits)
        return out, ids, counts
    ids, counts = quest_select_hip(q, page_min, page_max, page_size=page_size, topk=topk,
                                   offset=pos, gqa_union=gqa_union)
    out = sparse_attention(q, k_pool, v_pool, ids, unit=page_size, counts=counts, causal=True,
                           offset=pos, page_table=page_table, page_size=page_size, kv_len=kv_len,
                           scale=scale, out_dtype=out_dtype, num_splits=num_splits)
    return out, ids, counts


def quest_decode_fused(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                       page_table: torch.Tensor, page_min: torch.Tensor, page_max: torch.Tensor, *,
                       page_size: int, topk: int, pos: Optional[int] = None,
                       positions: Optional[torch.Tensor] = None,
                       kv_len: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                       out_dtype: Optional[torch.dtype] = None
                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``quest_decode_step`` with the GQA union in one kernel
    (``la_quest_decode_fused``): per (b, KV head), the page scores, top-k of
    every query head, union and attention over the selected pages.  Same
    arguments and results (out, ids, counts); the lists equal
    ``quest_select_hip``'s bit for bit.  One query per sequence, bf16 q and
    K/V, head_dim 128, at most 1024 pages, G = Hq/Hkv in {2, 4}; raises
    NotImplementedError otherwise (``quest_decode_step`` covers every
    shape)."""
    dev = N.require_gpu(q, k_pool, v_pool, page_table, page_min, page_max, positions, kv_len,
                        what="quest_decode_fused")
    if (pos is None) == (positions is None):
        raise ValueError("pass exactly one of pos and positions")
    B, Hq, Tq, D = q.shape
    Hkv, P = page_min.shape[1], page_min.shape[2]
    if Tq != 1:
        raise ValueError("quest_decode_fused: one query per sequence")
    if page_min.shape != (B, Hkv, P, D) or page_max.shape != page_min.shape or Hq % Hkv or \
            page_min.stride() != page_max.stride() or page_min.dtype != page_max.dtype:
        raise ValueError("page_min/max must be (B, Hkv, P, D) twins with Hq a multiple of Hkv")
    if positions is not None and (positions.dtype != torch.int32 or positions.shape != (B,)
                                  or not positions.is_contiguous()):
        raise ValueError("positions must be contiguous int32 (B,)")
    G = Hq // Hkv
    k = max(1, min(int(topk), P))
    ids = torch.empty(B, Hkv, 1, G * k, dtype=torch.int32, device=dev)
    counts = torch.empty(B, Hkv, 1, dtype=torch.int32, device=dev)
    out = torch.empty(B, Hq, 1, D, dtype=out_dtype or q.dtype, device=dev)
    a = N.LaQuestDecodeArgs()
    s = a.select
    s.q, s.page_min, s.page_max = q.data_ptr(), page_min.data_ptr(), page_max.data_ptr()
    s.out_idx, s.out_count = ids.data_ptr(), counts.data_ptr()
    s.B, s.Hq, s.Hkv, s.Tq, s.D = B, Hq, Hkv, 1, D
    s.q_sb, s.q_sh, s.q_st = q.stride(0), q.stride(1), q.stride(2)
    s.n_pages = P
    s.m_sb, s.m_sh, s.m_sp, s.m_sd = page_min.stride()
    s.page_size, s.pos_offset, s.k = page_size, (pos if pos is not None else 0), k
    s.q_dtype, s.meta_dtype = N.dtype_code(q.dtype), N.dtype_code(page_min.dtype)
    s.positions = N.ptr(positions)
    T = page_table.shape[1] * page_size
    a.kv = _kv_struct(k_pool, v_pool, page_table=page_table, page_size=page_size, kv_len=kv_len,
                      k_scale=None, v_scale=None, T=T, D=D, Hkv=Hkv)
    a.out = out.data_ptr()
    a.o_sb, a.o_sh, a.o_st = out.stride(0), out.stride(1), out.stride(2)
    a.scale = float(scale if scale is not None else 1.0 / math.sqrt(D))
    a.out_dtype = N.dtype_code(out.dtype)
    rc = N.load().la_quest_decode_fused(ctypes.byref(a), N.stream_handle(dev))
    if rc == N.LA_ERR_UNSUPPORTED:
        raise NotImplementedError((N.load().la_last_error() or b"").decode(errors="replace"))
    N.check(rc, "quest_decode_fused")
    return out, ids, counts
