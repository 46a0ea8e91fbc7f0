"""Block routing on gfx950: MoBA's gate, NSA's blockwise selection and
XAttention's antidiagonal block selection.

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
import math
from typing import Optional, Sequence, Tuple, Union

import torch

from linattn_amd import _native as N

__all__ = ["block_means_hip", "gate_select_hip", "nsa_selection_hip", "xattn_select_hip"]


def block_means_hip(k: torch.Tensor, *, block: int, out: Optional[torch.Tensor] = None,
                    first_block: int = 0, n_blocks: Optional[int] = None,
                    positions: Optional[torch.Tensor] = None,
                    lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Block means of k (B, H, T, D) as ``gate_select_hip`` pools them:
    (B, H, ceil(T/block), D) fp64, each block's rows added in order and
    divided by ``block``, the tail block repeating the last row
    (block_reduce, core.py:102-120).  Pools blocks ``first_block`` ..
    ``first_block + n_blocks - 1`` (all by default) into ``out`` (allocated
    when None; other blocks keep their values), or, with ``positions``
    (int32 (B,)), only the block holding positions[b] in sequence b: a decode
    step re-pools just the block its new key joined, instead of the per-call
    pooling of every key in MoBAAttention.select (selection.py:620-624).
    ``lengths`` (int32 (B,)): rows of each sequence (the tail repeats row
    lengths[b] - 1)."""
    dev = N.require_gpu(k, positions, lengths, what="block_means_hip")
    if k.dim() != 4 or k.stride(3) != 1:
        raise ValueError("k must be (B, H, T, D) with contiguous rows")
    if k.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError("k must be fp32, bf16 or fp16")
    B, H, T, D = k.shape
    if block <= 0 or T == 0:
        raise ValueError("block > 0 and T > 0 required")
    nkb = (T + block - 1) // block
    if out is None:
        out = torch.empty(B, H, nkb, D, dtype=torch.float64, device=dev)
    elif out.shape != (B, H, nkb, D) or out.dtype != torch.float64 or not out.is_contiguous() \
            or out.device != dev:
        raise ValueError(f"out must be a contiguous fp64 ({B}, {H}, {nkb}, {D}) tensor on {dev}")
    for name, t in (("positions", positions), ("lengths", lengths)):
        if t is not None and (t.dtype != torch.int32 or t.shape != (B,)):
            raise ValueError(f"{name} must be int32 ({B},)")
    a = N.LaBlockMeansArgs()
    a.k, a.out = k.data_ptr(), out.data_ptr()
    positions = positions.contiguous() if positions is not None else None
    lengths = lengths.contiguous() if lengths is not None else None
    a.positions, a.lengths = N.ptr(positions), N.ptr(lengths)
    a.B, a.H, a.T, a.D = B, H, T, D
    a.k_sb, a.k_sh, a.k_st = k.stride(0), k.stride(1), k.stride(2)
    a.block = block
    a.first_block = first_block
    a.n_blocks = nkb - first_block if n_blocks is None else n_blocks
    a.in_dtype = N.dtype_code(k.dtype)
    N.check(N.load().la_block_means(ctypes.byref(a), N.stream_handle(dev)), "block_means_hip")
    return out


def gate_select_hip(q: torch.Tensor, k: torch.Tensor, *, block: int, topk: int,
                    offset: int = 0, kbar: Optional[torch.Tensor] = None
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block lists (B, Hq, Tq, min(topk, n_blocks) + 1), ascending, -1 padded,
    and counts (B, Hq, Tq).  q (B, Hq, Tq, D) at positions offset + t; k
    (B, Hkv, T, D) with Hq a multiple of Hkv (query head h reads KV head
    h // (Hq/Hkv), repeat_kv of selection.py:623).  ``kbar``: the block
    means of k kept by the caller (``block_means_hip``); given, k is not
    read (only its shape is used)."""
    dev = N.require_gpu(q, k, kbar, what="gate_select_hip")
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
    if kbar is not None and (kbar.shape != (B, Hkv, n_kb, D) or kbar.dtype != torch.float64
                             or not kbar.is_contiguous()):
        raise ValueError(f"kbar must be a contiguous fp64 ({B}, {Hkv}, {n_kb}, {D}) tensor")
    width = min(topk, n_kb) + 1
    ids = torch.empty(B, Hq, Tq, width, dtype=torch.int32, device=dev)
    counts = torch.empty(B, Hq, Tq, dtype=torch.int32, device=dev)
    a = N.LaGateSelectArgs()
    a.kbar = N.ptr(kbar)
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


_ALPHAS = {}


def _alphas(threshold, Hq: int, dev: torch.device) -> torch.Tensor:
    """Per-head thresholds on the device without a host sync: a device fill
    for one value, a cached copy for a per-head list."""
    if isinstance(threshold, (int, float)):
        return torch.full((Hq,), float(threshold), dtype=torch.float64, device=dev)
    th = tuple(float(x) for x in threshold)
    if len(th) == 1:
        return torch.full((Hq,), th[0], dtype=torch.float64, device=dev)
    if len(th) != Hq:
        raise ValueError("threshold: one value or one per query head")
    key = (th, str(dev))
    if key not in _ALPHAS:
        _ALPHAS[key] = torch.tensor(th, dtype=torch.float64).to(dev)
    return _ALPHAS[key]


def xattn_select_hip(q: torch.Tensor, k: torch.Tensor, *, block: int = 8, stride: int = 8,
                     threshold: Union[float, Sequence[float]] = 0.9, offset: int = 0,
                     topk: Optional[int] = None, top_ratio: Optional[float] = None,
                     max_workspace_bytes: Optional[int] = None
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
    """XAttention's block selection (XAttention.antidiagonal_scores / select,
    selection.py:528-595) for every (b, query head, query block).

    Slot scores are the strided antidiagonal sums of each (query block, key
    block) gram matrix (stride ``stride``, blocks of ``block`` tokens) times
    1/sqrt(D); the softmax over a row's visible (block, slot) pairs gives the
    block masses; ``threshold`` (a float, or one value per query head as the
    reference's ``threshold_per_head``) keeps the minimal prefix of blocks,
    by mass, whose cumulative mass reaches it (_cumulative_select,
    selection.py:62-69); with ``topk`` the top-k blocks by mass are kept
    instead (select_mode "topk").  With ``top_ratio`` (select_mode
    "top_ratio", selection.py:583-585) the cumulative mass is compared with
    the block count max(1, ceil(n_visible * ratio)) >= 1 (:598-606); the
    masses of a row are positive and sum to 1, so that count is reached only
    once every visible block is in: every visible block is kept, and no
    score is computed.  The own block is OR'd in and blocks past
    causality dropped.  Masses are exact integers of fixed-point weights from
    a deterministic exp, so ties and the threshold crossing are a fixed
    function of the inputs (ties to the lowest block).

    The slot scores of a chunk of query blocks are kept in a workspace of at
    most 256 MiB (the chunk shrinks as T grows); ``max_workspace_bytes``
    bounds it further (smaller chunks, same lists; below one chunk of 64 query
    blocks the rows are scored without a workspace).

    q (B, Hq, Tq, D) at positions offset + t; k (B, Hkv, T, D).  Returns ids
    (B, Hq, n_qb, W) ascending, -1 padded (W = n_kb, or min(topk, n_kb) + 1)
    and counts (B, Hq, n_qb)."""
    dev = N.require_gpu(q, k, what="xattn_select_hip")
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
    if not 1 <= block <= 64 or stride < 1 or offset < 0:
        raise ValueError("block in [1, 64], stride >= 1 and offset >= 0 required")
    if topk is not None and topk < 1:
        raise ValueError("topk >= 1 required")
    n_qb, n_kb = -(-Tq // block), -(-T // block)
    if top_ratio is not None:
        if not top_ratio > 0:
            raise ValueError("top_ratio > 0 required")
        # visible key blocks of query block i: kb * block <= offset + i * block
        last = torch.clamp((offset + torch.arange(n_qb, device=dev) * block) // block, max=n_kb - 1)
        kb = torch.arange(n_kb, device=dev)
        ids = torch.where(kb[None, :] <= last[:, None], kb[None, :], -1).to(torch.int32)
        ids = ids.expand(B, Hq, n_qb, n_kb).contiguous()
        counts = (last + 1).to(torch.int32).expand(B, Hq, n_qb).contiguous()
        return ids, counts
    width = min(topk, n_kb) + 1 if topk is not None else n_kb
    ids = torch.empty(B, Hq, n_qb, width, dtype=torch.int32, device=dev)
    counts = torch.empty(B, Hq, n_qb, dtype=torch.int32, device=dev)
    alpha = None
    a = N.LaXattnSelectArgs()
    if topk is None:
        alpha = _alphas(threshold, Hq, dev)
        a.alpha = alpha.data_ptr()
    a.q, a.k, a.out_idx, a.out_count = q.data_ptr(), k.data_ptr(), ids.data_ptr(), counts.data_ptr()
    a.B, a.Hq, a.Hkv, a.Tq, a.T, a.D = B, Hq, Hkv, Tq, T, D
    a.q_sb, a.q_sh, a.q_st = q.stride(0), q.stride(1), q.stride(2)
    a.k_sb, a.k_sh, a.k_st = k.stride(0), k.stride(1), k.stride(2)
    a.block, a.stride, a.offset, a.width = block, stride, offset, width
    a.topk = int(topk or 0)
    a.inv_sqrt_d = 1.0 / math.sqrt(D)
    a.mode = 0 if topk is None else 1
    a.in_dtype = N.dtype_code(q.dtype)
    L = N.load()
    ws_bytes = L.la_xattn_select_workspace(ctypes.byref(a))
    if max_workspace_bytes is not None:
        ws_bytes = min(ws_bytes, max(0, int(max_workspace_bytes)))
    ws = N.workspace(ws_bytes, dev) if ws_bytes else None
    a.workspace, a.ws_bytes = N.ptr(ws), ws_bytes
    N.check(L.la_xattn_select(ctypes.byref(a), N.stream_handle(dev)), "xattn_select_hip")
    return ids, counts
