"""Block-sparse causal prefill on gfx950: block selection + MFMA attention.

``block_select_hip`` builds the per-(b, head, query block) key-block lists of
config C3 from the block-sparse estimator of MInferenceAttention._block_sparse
(variants/selection.py:339-353): mean-pooled q.k block scores over causal
blocks, top-k with ties to the lowest block index, then the sink blocks and
the local window (which includes the diagonal block) OR'd in.

``block_sparse_prefill`` is the executor (block_sparse.py:80-163) for lists
shared by a 64-query block, run on the matrix cores (bf16 MFMA scores, fp16
MFMA weights x V, fp32 accumulation) with the causal mask applied in-kernel.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from linattn_amd import _native as N

__all__ = ["block_select_hip", "block_sparse_prefill", "sparse_prefill"]


def _s3(t):
    s = t.stride()
    return s[0], s[1], s[2]


def _lengths(lengths: Optional[torch.Tensor], B: int) -> Optional[torch.Tensor]:
    """Per-sequence lengths of a ragged batch: int32 (B,) on the device (values
    are clamped to [0, T] by the kernels)."""
    if lengths is None:
        return None
    if lengths.dtype != torch.int32 or lengths.shape != (B,):
        raise ValueError(f"lengths must be int32 ({B},)")
    return lengths.contiguous()


def block_select_hip(q: torch.Tensor, k: torch.Tensor, *, block: int = 64, topk: int = 16,
                     sink_blocks: int = 1, window_blocks: int = 4,
                     lengths: Optional[torch.Tensor] = None
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Key-block lists (B, Hq, n_qb, topk+sink+window) int32, ascending, -1
    padded, and counts (B, Hq, n_qb).  q (B, Hq, T, D), k (B, Hkv, T, D).

    ``lengths`` (int32 (B,), optional): a ragged batch padded to T; sequence
    b's rows past lengths[b] are never read, its query blocks past the end get
    empty lists, and its other lists equal a call on that sequence alone."""
    dev = N.require_gpu(q, k, lengths, what="block_select_hip")
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, T, D):
        raise ValueError("k must be (B, Hkv, T, D) with q's batch, length and head_dim")
    if q.dtype != k.dtype:
        raise ValueError("q and k must share a dtype")
    nqb = (T + block - 1) // block
    width = topk + sink_blocks + window_blocks
    ids = torch.empty(B, Hq, nqb, width, dtype=torch.int32, device=dev)
    counts = torch.empty(B, Hq, nqb, dtype=torch.int32, device=dev)
    a = N.LaBlockSelectArgs()
    a.q, a.k, a.out_idx, a.out_count = q.data_ptr(), k.data_ptr(), ids.data_ptr(), counts.data_ptr()
    a.B, a.Hq, a.Hkv, a.T, a.D = B, Hq, Hkv, T, D
    a.q_sb, a.q_sh, a.q_st = _s3(q)
    a.k_sb, a.k_sh, a.k_st = _s3(k)
    a.block, a.topk, a.sink_blocks, a.window_blocks, a.width = block, topk, sink_blocks, \
        window_blocks, width
    a.in_dtype = N.dtype_code(q.dtype)
    lengths = _lengths(lengths, B)
    a.lengths = N.ptr(lengths)
    L = N.load()
    ws_bytes = L.la_block_select_workspace(ctypes.byref(a))
    ws = N.workspace(ws_bytes, dev)
    a.workspace, a.ws_bytes = N.ptr(ws), ws_bytes
    N.check(L.la_block_select(ctypes.byref(a), N.stream_handle(dev)), "block_select_hip")
    return ids, counts


def block_sparse_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, ids: torch.Tensor,
                         counts: Optional[torch.Tensor] = None, *, block_size: int = 64,
                         causal: bool = True, scale: Optional[float] = None,
                         out_dtype: Optional[torch.dtype] = None,
                         lengths: Optional[torch.Tensor] = None,
                         k_scale: Optional[torch.Tensor] = None,
                         v_scale: Optional[torch.Tensor] = None,
                         check_range: bool = True) -> torch.Tensor:
    """Attention of every 64-query block over its listed 64-key blocks.

    q (B, Hq, T, 128) bf16; k/v (B, Hkv, T, 128) bf16, or float8_e4m3fn codes
    with per-token fp32 scales ``k_scale``/``v_scale`` (B, Hkv, T) (the codec
    of kv/quant.py:76-109, see ``quantize_fp8_per_token``); ids int32
    (B, Hq, n_qb, W) (-1 entries read nothing); counts optional (B, Hq, n_qb).
    Returns (B, Hq, T, 128) in ``out_dtype`` (default q.dtype).  ``lengths``
    (int32 (B,), optional): a ragged batch; rows of sequence b at or past
    lengths[b] are never read and come out as zeros.

    The weights multiply an fp16 copy of V scaled by a power of two per
    64-token block, which holds |v| < 2^22; a finite |v| >= 2^22 raises
    ValueError after the call (``check_range``, default True: one read of the
    device status word, a host synchronisation; with False the rows reading
    such a block come out inf and the device status word records it)."""
    dev = N.require_gpu(q, k, v, ids, counts, lengths, k_scale, v_scale,
                        what="block_sparse_prefill")
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    fp8 = k.dtype == torch.float8_e4m3fn
    if q.dtype != torch.bfloat16 or k.dtype != v.dtype or \
            k.dtype not in (torch.bfloat16, torch.float8_e4m3fn):
        raise ValueError("block_sparse_prefill runs bf16 q with bf16 or fp8 e4m3 k/v")
    if fp8:
        if k_scale is None or v_scale is None:
            raise ValueError("fp8 k/v need k_scale and v_scale")
        if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32 or \
                k_scale.shape != (B, Hkv, T) or v_scale.shape != (B, Hkv, T) or \
                k_scale.stride() != v_scale.stride():
            raise ValueError("k_scale/v_scale must be fp32 (B, Hkv, T) with equal strides")
    if k.shape != (B, Hkv, T, D) or v.shape != k.shape:
        raise ValueError("k/v must be (B, Hkv, T, D)")
    nqb = (T + block_size - 1) // block_size
    if ids.dtype != torch.int32 or ids.dim() != 4 or ids.shape[:3] != (B, Hq, nqb):
        raise ValueError(f"ids must be int32 (B, Hq, {nqb}, W)")
    ids = ids.contiguous()
    if counts is not None:
        if counts.dtype != torch.int32 or counts.shape != (B, Hq, nqb):
            raise ValueError("counts must be int32 (B, Hq, n_qb)")
        counts = counts.contiguous()
    out = torch.empty(B, Hq, T, D, dtype=out_dtype or q.dtype, device=dev)
    a = N.LaPrefillArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.ids, a.counts = ids.data_ptr(), N.ptr(counts)
    a.B, a.Hq, a.Hkv, a.T, a.D = B, Hq, Hkv, T, D
    a.q_sb, a.q_sh, a.q_st = _s3(q)
    a.k_sb, a.k_sh, a.k_st = _s3(k)
    a.v_sb, a.v_sh, a.v_st = _s3(v)
    a.o_sb, a.o_sh, a.o_st = _s3(out)
    a.block, a.width = block_size, ids.shape[3]
    a.scale = float(scale if scale is not None else 1.0 / math.sqrt(D))
    a.causal = 1 if causal else 0
    a.out_dtype = N.dtype_code(out.dtype)
    lengths = _lengths(lengths, B)
    a.lengths = N.ptr(lengths)
    if fp8:
        a.kv_dtype = N.dtype_code(k.dtype)
        a.k_scale, a.v_scale = k_scale.data_ptr(), v_scale.data_ptr()
        a.s_sb, a.s_sh, a.s_st = _s3(k_scale)
    L = N.load()
    ws_bytes = L.la_block_sparse_prefill_workspace(ctypes.byref(a))
    ws = N.workspace(ws_bytes, dev)
    a.workspace, a.ws_bytes = N.ptr(ws), ws_bytes
    N.check(L.la_block_sparse_prefill(ctypes.byref(a), N.stream_handle(dev)),
            "block_sparse_prefill")
    if check_range and N.device_status(dev, clear=False) & N.LA_DEV_PREFILL_RANGE:
        N.device_status(dev, clear=True)
        raise ValueError("block_sparse_prefill: v holds a finite value with |v| >= 2^22 "
                         "(beyond the fp16 range of the weighted V product)")
    return out


def sparse_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block: int = 64,
                   topk: int = 16, sink_blocks: int = 1, window_blocks: int = 4,
                   out_dtype: Optional[torch.dtype] = None,
                   lengths: Optional[torch.Tensor] = None
                   ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Config-C3 prefill: block selection then MFMA attention.  Returns
    (out, ids, counts).  ``lengths``: per-sequence lengths of a ragged batch."""
    ids, counts = block_select_hip(q, k, block=block, topk=topk, sink_blocks=sink_blocks,
                                   window_blocks=window_blocks, lengths=lengths)
    out = block_sparse_prefill(q, k, v, ids, counts, block_size=block, out_dtype=out_dtype,
                               lengths=lengths)
    return out, ids, counts
