"""Lightning-indexer scoring fused with top-k selection on gfx950.

Mirrors kernels/triton/fused_indexer.py:153-206 (``indexer_topk``,
``indexer_topk_triton``) with the semantics of ``indexer_topk_torch``
(:63-73): I[b,t,s] = sum_h w[b,t,h] ReLU(q[b,t,h] . k[b,s,h]) and the k best
keys per query.  Differences by design: scores are exact-product fp64 sums (a
fixed function of the inputs, so indices are reproducible bit for bit), ties go
to the lowest key index, indices are int32 (as the Triton path returns,
fused_indexer.py:181), and ``causal=True`` keeps only keys s <= offset + t
(rows with fewer valid keys are padded with -1 / -inf).  The two-pass
threshold of the Triton kernels (defect D3: an invalid threshold and a
scan-order cap) is replaced by an exact radix select.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from linattn_amd import _native as N

__all__ = ["indexer_topk", "indexer_topk_hip", "indexer_topk_triton"]


def indexer_topk(q_idx: torch.Tensor, k_idx: torch.Tensor, head_weights: torch.Tensor, k: int, *,
                 backend: str = "auto", causal: bool = False, offset: int = 0,
                 causal_unit: int = 1, q_chunk: int = 0, sorted: bool = True
                 ) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
    """Top-k indexer scores: ``(values fp32 (B,Tq,k), indices int32 (B,Tq,k))``.

    q_idx: (B, Tq, H_I, d), k_idx: (B, Tk, H_I, d) in fp32/bf16/fp16;
    head_weights: (B, Tq, H_I).  ``k`` is clipped to Tk as in the reference.
    With ``causal_unit`` = m > 1 the keys are pooled groups of m tokens and
    group s is visible to query t when s*m <= offset + t.  ``sorted=False``
    (an addition) returns ``(None, indices)`` with the same selected keys in
    ascending index order, -1 padded: the token set a selection mask is built
    from (selection.py:752-761), without the sort."""
    if backend not in ("auto", "hip", "triton"):
        raise ValueError(f"backend {backend!r} is not provided by linattn_amd (only 'hip')")
    dev = N.require_gpu(q_idx, k_idx, head_weights, what="indexer_topk")
    if q_idx.dim() != 4 or k_idx.dim() != 4:
        raise ValueError("q_idx and k_idx must be (B, T, H_I, d)")
    B, Tq, HI, d = q_idx.shape
    Tk = k_idx.shape[1]
    if k_idx.shape[0] != B or k_idx.shape[2] != HI or k_idx.shape[3] != d:
        raise ValueError("q_idx / k_idx shapes disagree")
    if k_idx.dtype != q_idx.dtype:
        raise ValueError("q_idx and k_idx must share a dtype")
    if head_weights.shape != (B, Tq, HI):
        raise ValueError("head_weights must be (B, Tq, H_I)")
    if q_idx.stride(-1) != 1 or k_idx.stride(-1) != 1:
        raise ValueError("q_idx / k_idx need a unit stride over d")
    w = head_weights.to(torch.float32)
    kk = min(int(k), Tk)
    if kk < 1:
        raise ValueError("k must be >= 1")
    idx = torch.empty(B, Tq, kk, dtype=torch.int32, device=dev)
    val = torch.empty(B, Tq, kk, dtype=torch.float32, device=dev) if sorted else None
    a = N.LaIndexerArgs()
    a.q, a.kk, a.w = q_idx.data_ptr(), k_idx.data_ptr(), w.data_ptr()
    a.out_idx, a.out_val = idx.data_ptr(), (val.data_ptr() if sorted else None)
    a.order = 0 if sorted else 1
    a.B, a.Tq, a.Tk, a.HI, a.d, a.k = B, Tq, Tk, HI, d, kk
    a.q_sb, a.q_st, a.q_sh = q_idx.stride(0), q_idx.stride(1), q_idx.stride(2)
    a.k_sb, a.k_st, a.k_sh = k_idx.stride(0), k_idx.stride(1), k_idx.stride(2)
    a.w_sb, a.w_st, a.w_sh = w.stride(0), w.stride(1), w.stride(2)
    a.offset = int(offset)
    a.q_chunk = int(q_chunk)
    a.causal_unit = int(causal_unit)
    a.in_dtype = N.dtype_code(q_idx.dtype)
    a.causal = 1 if causal else 0
    L = N.load()
    ws_bytes = L.la_indexer_topk_workspace(ctypes.byref(a))
    ws = N.workspace(ws_bytes, dev)
    a.workspace, a.ws_bytes = N.ptr(ws), ws_bytes
    N.check(L.la_indexer_topk(ctypes.byref(a), N.stream_handle(dev)), "indexer_topk")
    return val, idx


indexer_topk_hip = indexer_topk


def indexer_topk_triton(q_idx, k_idx, head_weights, k: int, *, block_k: int = 128):
    """Drop-in alias for fused_indexer.py:153 (runs the HIP kernels; block_k is
    accepted for signature compatibility and has no effect)."""
    return indexer_topk(q_idx, k_idx, head_weights, k)
