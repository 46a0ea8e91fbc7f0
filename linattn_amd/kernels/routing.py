"""Per-query block routing on gfx950: MoBA's gate and NSA's blockwise selection.

MoBAAttention.select (variants/selection.py:610-640) and
NSAAttention.selection_mask (variants/native_sparse.py:78-93) compute the same
lists: the gate q_t . mean(K block j) over the blocks that start at or before
the query's position, the top ``topk`` blocks, and the query's own block OR'd
in.  ``gate_select_hip`` returns them as block lists for the executor
(``sparse_attention`` with ``unit=block``).  Gates are fp64 (products added
over d in order) and ties go to the lowest block, so the lists are a fixed
function of the inputs.
"""

from __future__ import annotations

import ctypes
from typing import Tuple

import torch

from linattn_amd import _native as N

__all__ = ["gate_select_hip", "nsa_selection_hip"]


def gate_select_hip(q: torch.Tensor, k: torch.Tensor, *, block: int, topk: int,
                    offset: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block lists (B, Hq, Tq, min(topk, n_blocks) + 1), ascending, -1 padded,
    and counts (B, Hq, Tq).  q (B, Hq, Tq, D) at positions offset + t; k
    (B, Hkv, T, D) with Hq a multiple of Hkv (query head h reads KV head
    h // (Hq/Hkv), repeat_kv of selection.py:623)."""
    dev = N.require_gpu(q, k, what="gate_select_hip")
    if q.dim() != 4 or k.dim() != 4 or q.shape[0] != k.shape[0] or q.shape[3] != k.shape[3]:
        raise ValueError("q (B, Hq, Tq, D) and k (B, Hkv, T, D) expected")
    if q.dtype != k.dtype:
        raise ValueError("q and k must share a dtype")
    B, Hq, Tq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    if Hq % Hkv:
        raise ValueError("n_heads must be a multiple of n_kv_heads")
    if q.stride(3) != 1 or k.stride(3) != 1:
        raise ValueError("q and k rows must be contiguous")
    if block <= 0 or topk < 1 or offset < 0:
        raise ValueError("block > 0, topk >= 1 and offset >= 0 required")
    n_kb = (T + block - 1) // block
    width = min(topk, n_kb) + 1
    ids = torch.empty(B, Hq, Tq, width, dtype=torch.int32, device=dev)
    counts = torch.empty(B, Hq, Tq, dtype=torch.int32, device=dev)
    a = N.LaGateSelectArgs()
    a.q, a.k, a.out_idx, a.out_count = q.data_ptr(), k.data_ptr(), ids.data_ptr(), counts.data_ptr()
    a.B, a.Hq, a.Hkv, a.Tq, a.T, a.D = B, Hq, Hkv, Tq, T, D
    a.q_sb, a.q_sh, a.q_st = q.stride(0), q.stride(1), q.stride(2)
    a.k_sb, a.k_sh, a.k_st = k.stride(0), k.stride(1), k.stride(2)
    a.block, a.topk, a.offset, a.width = block, topk, offset, width
    a.in_dtype = N.dtype_code(q.dtype)
    L = N.load()
    ws_bytes = L.la_gate_select_workspace(ctypes.byref(a))
    ws = N.workspace(ws_bytes, dev)
    a.workspace, a.ws_bytes = N.ptr(ws), ws_bytes
    N.check(L.la_gate_select(ctypes.byref(a), N.stream_handle(dev)), "gate_select_hip")
    return ids, counts


def nsa_selection_hip(q: torch.Tensor, k: torch.Tensor, *, block: int, selected_blocks: int,
                      offset: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """NSAAttention.selection_mask (native_sparse.py:78-93) as block lists:
    the same routing as MoBA with ``selected_blocks`` blocks per query."""
    return gate_select_hip(q, k, block=block, topk=selected_blocks, offset=offset)
