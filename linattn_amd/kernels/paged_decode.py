"""Paged sparse decode on gfx950.

``paged_decode`` keeps the reference's single-(head, query) C entry point
(kernels/c_attention.py:76-111, kernels/c/decode_attn.c:39-133) and runs it on
the GPU.  ``quest_decode_step`` is the batched decode hot path: Quest page
selection over a paged KV pool followed by split-K attention over the selected
pages (the decode step of QuestAttention, variants/selection.py:139-248, driven
by AttentionVariant.forward, core.py:231-279).
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from linattn_amd.kernels.block_sparse import sparse_attention
from linattn_amd.kernels.fused_indexer import indexer_topk
from linattn_amd.kernels.quest_pages import quest_select_hip

__all__ = ["paged_decode", "quest_decode_step", "indexer_decode_step", "quantize_fp8_per_token"]


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
