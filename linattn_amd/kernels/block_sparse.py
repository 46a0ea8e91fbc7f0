"""Exact attention over selected KV units on gfx950 (the shared executor).

``block_sparse_attention`` keeps the reference's signature and semantics
(kernels/triton/block_sparse.py:131-163, torch form :40-75); ``sparse_attention``
is the general entry used by decode and the variants (paged pools, token lists,
per-query-head lists, causal masking, fp8 KV).
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from linattn_amd import _native as N

__all__ = ["sparse_attention", "block_sparse_attention", "block_sparse_attention_hip",
           "fp8_scale_pairs"]


def _strides3(t: torch.Tensor):
    s = t.stride()
    return s[0], s[1], s[2]


def _paged_scale_stride(scale: torch.Tensor, pool: torch.Tensor) -> int:
    """Element stride between the scales of consecutive pool rows of a paged
    fp8 pool (n_phys, Hkv, page_size, D): scales are (n_phys, Hkv, page_size)
    with strides (Hkv*page_size*s, page_size*s, s) -- s = 1 for a contiguous
    tensor, s = 2 for the K or V half of an interleaved (..., 2) pair tensor
    (``fp8_scale_pairs``)."""
    n_phys, Hkv, ps = pool.shape[0], pool.shape[1], pool.shape[2]
    if scale.dim() == 4 and scale.shape[3] == 1:
        scale = scale.squeeze(3)
    if scale.shape != (n_phys, Hkv, ps):
        raise ValueError("paged fp8 scales must be (n_pages, Hkv, page_size)")
    s = scale.stride(2)
    if s < 1 or scale.stride() != (Hkv * ps * s, ps * s, s):
        raise ValueError("paged fp8 scales: rows at one constant stride (contiguous, or one "
                         "half of an interleaved (n_pages, Hkv, page_size, 2) tensor)")
    return s


def fp8_scale_pairs(n_pages: int, Hkv: int, page_size: int, device) -> Tuple[torch.Tensor,
                                                                          torch.Tensor]:
    """Per-token K and V scales of a paged fp8 pool stored interleaved
    ((n_pages, Hkv, page_size, 2) fp32): returns the K and V views.  A token
    then reads both of its scales from one 8-byte pair (one memory sector)
    instead of two scattered 4-byte values."""
    pairs = torch.empty(n_pages, Hkv, page_size, 2, dtype=torch.float32, device=device)
    return pairs[..., 0], pairs[..., 1]


def _kv_struct(k: torch.Tensor, v: torch.Tensor, *, page_table: Optional[torch.Tensor],
               page_size: Optional[int], kv_len: Optional[torch.Tensor],
               k_scale: Optional[torch.Tensor], v_scale: Optional[torch.Tensor], T: int,
               D: int, Hkv: int) -> N.LaKV:
    kv = N.LaKV()
    kv.k, kv.v = k.data_ptr(), v.data_ptr()
    kv.dtype = N.dtype_code(k.dtype)
    if v.dtype != k.dtype:
        raise ValueError("k and v must share a dtype")
    kv.T = T
    if page_table is not None:
        if k.dim() != 4 or k.shape[1] != Hkv or k.shape[3] != D or not k.is_contiguous() \
                or not v.is_contiguous() or v.shape != k.shape:
            raise ValueError("paged k/v must be contiguous pools (n_pages, Hkv, page_size, D)")
        if page_size is None or k.shape[2] != page_size:
            raise ValueError("page_size must equal the pool's page dimension")
        if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.stride(1) != 1:
            raise ValueError("page_table must be int32 (B, pages) with unit last stride")
        if k.shape[0] * k.shape[1] * k.shape[2] >= 2 ** 32:
            raise ValueError("paged pool holds >= 2^32 token rows")
        kv.page_table = page_table.data_ptr()
        kv.pt_stride = page_table.stride(0)
        kv.page_size = page_size
    else:
        if k.stride(-1) != 1 or v.stride(-1) != 1:
            raise ValueError("k/v must have a unit stride over head_dim")
        kv.k_sb, kv.k_sh, kv.k_st = _strides3(k)
        kv.v_sb, kv.v_sh, kv.v_st = _strides3(v)
    if k.dtype == torch.float8_e4m3fn:
        if k_scale is None or v_scale is None:
            raise ValueError("fp8 K/V need k_scale and v_scale (one fp32 per token)")
        if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
            raise ValueError("fp8 scales must be float32")
        if k_scale.stride() != v_scale.stride() or k_scale.shape != v_scale.shape:
            raise ValueError("k_scale and v_scale must share shape and strides")
        kv.k_scale, kv.v_scale = k_scale.data_ptr(), v_scale.data_ptr()
        if page_table is None:
            kv.s_sb, kv.s_sh, kv.s_st = _strides3(k_scale)
        else:
            kv.s_st = _paged_scale_stride(k_scale, k)
    if kv_len is not None:
        if kv_len.dtype != torch.int32 or not kv_len.is_contiguous():
            raise ValueError("kv_len must be contiguous int32 (B,)")
        kv.kv_len = kv_len.data_ptr()
    return kv


def sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, ids: torch.Tensor, *,
                     unit: int, counts: Optional[torch.Tensor] = None,
                     scale: Optional[float] = None, causal: bool = False, offset: int = 0,
                     page_table: Optional[torch.Tensor] = None, page_size: Optional[int] = None,
                     kv_len: Optional[torch.Tensor] = None, k_scale: Optional[torch.Tensor] = None,
                     v_scale: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                     out_dtype: Optional[torch.dtype] = None, num_splits: int = 0,
                     no_alloc: bool = False) -> torch.Tensor:
    """Attention of q over the units listed in ``ids``.

    q: (B, Hq, Tq, D).  k/v: contiguous (B, Hkv, T, D) or, with ``page_table``
    (int32 (B, pages)), pools (n_pages, Hkv, page_size, D).
    ids: int32 (B, L, Tq|1, N) or (B, L, N) with L = Hkv (one list per GQA
    group) or L = Hq (one list per query head); entry u covers tokens
    [u*unit, (u+1)*unit); -1 entries are skipped.
    fp8 (float8_e4m3fn) K/V need fp32 per-token scales.
    Returns (B, Hq, Tq, D) in ``out_dtype`` (default q.dtype).
    ``no_alloc`` runs la_sparse_attention_noalloc: no workspace is allocated
    (the library's static per-device scratch holds the split partials; pass
    ``out`` as well for a call that allocates nothing)."""
    dev = N.require_gpu(q, k, v, ids, counts, page_table, kv_len, k_scale, v_scale,
                        what="sparse_attention")
    if q.dim() != 4:
        raise ValueError("q must have shape (B, H, T, D)")
    B, Hq, Tq, D = q.shape
    if q.stride(-1) != 1:
        raise ValueError("q must have a unit stride over head_dim")
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError("n_heads must be a multiple of n_kv_heads")
    if ids.dtype != torch.int32:
        raise ValueError("ids must be int32")
    if ids.dim() == 3:
        ids = ids.unsqueeze(2)
    if ids.dim() != 4 or ids.shape[0] != B or ids.shape[1] not in (Hkv, Hq) \
            or ids.shape[2] not in (1, Tq) or ids.stride(-1) != 1:
        raise ValueError(f"ids must be (B, Hkv|Hq, Tq|1, N) int32, got {tuple(ids.shape)}")
    if page_table is not None:
        T = page_table.shape[1] * int(page_size or 0)
    else:
        T = k.shape[2]
    if counts is not None:
        if counts.dtype != torch.int32:
            raise ValueError("counts must be int32")
        counts = counts.reshape(B, ids.shape[1], ids.shape[2]).contiguous()
    out_dtype = out_dtype or q.dtype
    if out is None:
        out = torch.empty(B, Hq, Tq, D, dtype=out_dtype, device=dev)
    elif out.shape != (B, Hq, Tq, D) or out.stride(-1) != 1:
        raise ValueError("out must be (B, Hq, Tq, D) with a unit last stride")
    kv = _kv_struct(k, v, page_table=page_table, page_size=page_size, kv_len=kv_len,
                    k_scale=k_scale, v_scale=v_scale, T=T, D=D, Hkv=Hkv)
    a = N.LaSparseAttnArgs()
    a.q, a.out, a.ids = q.data_ptr(), out.data_ptr(), ids.data_ptr()
    a.counts = N.ptr(counts)
    a.B, a.Hq, a.Hkv, a.Tq, a.D = B, Hq, Hkv, Tq, D
    a.q_sb, a.q_sh, a.q_st = _strides3(q)
    a.o_sb, a.o_sh, a.o_st = _strides3(out)
    a.ids_heads, a.ids_rows, a.N = ids.shape[1], ids.shape[2], ids.shape[3]
    a.id_sb, a.id_sh, a.id_st = _strides3(ids)
    a.unit = int(unit)
    a.offset = int(offset)
    a.num_splits = int(num_splits)
    a.scale = float(scale if scale is not None else 1.0 / math.sqrt(D))
    a.q_dtype = N.dtype_code(q.dtype)
    a.out_dtype = N.dtype_code(out.dtype)
    a.causal = 1 if causal else 0
    L = N.load()
    if no_alloc:
        N.check(L.la_sparse_attention_noalloc(ctypes.byref(a), ctypes.byref(kv),
                                              N.stream_handle(dev)), "sparse_attention(no_alloc)")
        return out
    ws_bytes = L.la_sparse_attention_workspace(ctypes.byref(a), ctypes.byref(kv))
    ws = N.workspace(ws_bytes, dev)
    a.workspace = N.ptr(ws)
    a.ws_bytes = ws_bytes
    N.check(L.la_sparse_attention(ctypes.byref(a), ctypes.byref(kv), N.stream_handle(dev)),
            "sparse_attention")
    return out


def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           block_ids: torch.Tensor, *, block_size: int, backend: str = "auto",
                           counts: Optional[torch.Tensor] = None, causal: bool = False,
                           offset: int = 0, scale: Optional[float] = None,
                           out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Exact attention over selected KV blocks (block_sparse.py:131-163).

    ``block_ids`` is (B, H_kv, n_blocks) (one list for every query) or
    (B, H_kv, T_q, n_blocks) (one per query row), as in the reference; a
    (B, H_q, ...) list gives every query head its own blocks.  Tokens >= T_k are
    masked and no causal mask is applied unless ``causal`` (the reference leaves
    causality to the selector, tests/test_kernels.py:81-82).  A block listed
    twice counts twice, as in the reference's gather.  -1 entries are skipped.
    Output dtype: q.dtype (block_sparse.py:75) unless ``out_dtype``."""
    if backend not in ("auto", "hip"):
        raise ValueError(f"backend {backend!r} is not provided by linattn_amd (only 'hip')")
    if block_size is None:
        raise ValueError("block_size is required")
    ids = block_ids
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    return sparse_attention(q, k, v, ids.contiguous(), unit=int(block_size), counts=counts,
                            causal=causal, offset=offset, scale=scale, out_dtype=out_dtype)


block_sparse_attention_hip = block_sparse_attention
