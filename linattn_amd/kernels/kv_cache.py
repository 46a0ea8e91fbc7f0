"""Paged KV cache maintenance on gfx950: append with Quest page bounds.

``paged_kv_append`` writes the new keys / values of a decode (or chunked
prefill) step into a paged pool and, in the same kernel, folds them into the
Quest page bounds -- the KV concatenation of AttentionVariant.push_kv
(core.py:219-220) plus QuestAttention._refresh_pages (variants/selection.py:
181-201) -- so that a serving loop needs no recompute pass over touched
pages.  For an fp8 pool the codec of kv/quant.py:76-93 (per-token scales,
group = head_dim) runs in the same kernel.  Sequences may sit at different
positions (ragged batches).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from linattn_amd import _native as N
from linattn_amd.kernels.block_sparse import _paged_scale_stride

__all__ = ["paged_kv_append"]


def paged_kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor,
                    v_pool: torch.Tensor, page_table: torch.Tensor, positions: torch.Tensor, *,
                    page_min: Optional[torch.Tensor] = None,
                    page_max: Optional[torch.Tensor] = None, page_size: Optional[int] = None,
                    k_scale: Optional[torch.Tensor] = None,
                    v_scale: Optional[torch.Tensor] = None) -> None:
    """Append (B, Hkv, Tn, D) keys / values at per-sequence ``positions`` (B,).

    Token t of sequence b goes to slot t % pool_page of physical page
    ``page_table[b, t // pool_page]`` of the pools (n_phys, Hkv, pool_page, D).
    With ``page_min`` / ``page_max`` (B, Hkv, n_pages, D) in the key dtype (as
    ``page_update_hip`` returns them) the bounds of every Quest page of
    ``page_size`` tokens that the new tokens touch are updated in place; for an
    append at the end of each sequence the result equals ``page_update_hip``
    over the grown cache bit for bit.  An fp8 (``torch.float8_e4m3fn``) pool
    takes ``k_scale`` / ``v_scale`` (n_phys, Hkv, pool_page) fp32 (contiguous,
    or the interleaved halves of ``fp8_scale_pairs``) and stores
    codes = e4m3(x / scale), scale = max(|x|, 1e-8) / 448 per token (no page
    bounds for fp8 pools).  Runs on the current stream; inputs are not
    modified."""
    dev = N.require_gpu(k_new, v_new, k_pool, v_pool, page_table, positions,
                        page_min, page_max, k_scale, v_scale, what="paged_kv_append")
    if k_new.dim() != 4 or v_new.shape != k_new.shape or k_new.stride() != v_new.stride():
        raise ValueError("k_new / v_new must be (B, Hkv, Tn, D) with equal shapes and strides")
    if k_new.dtype != v_new.dtype or k_new.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("k_new / v_new must both be float32 or bfloat16")
    B, Hkv, Tn, D = k_new.shape
    if k_new.stride(3) != 1:
        raise ValueError("k_new / v_new rows must be contiguous")
    if k_pool.dim() != 4 or v_pool.shape != k_pool.shape or k_pool.shape[1] != Hkv \
            or k_pool.shape[3] != D:
        raise ValueError("pools must be (n_phys, Hkv, pool_page, D) matching k_new")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if k_pool.dtype != v_pool.dtype:
        raise ValueError("k_pool / v_pool dtype mismatch")
    fp8 = k_pool.dtype == torch.float8_e4m3fn
    if not fp8 and k_pool.dtype != k_new.dtype:
        raise ValueError("the pool stores k_new's dtype (or float8_e4m3fn codes)")
    n_phys, _, pool_page, _ = k_pool.shape
    if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.shape[0] != B \
            or page_table.stride(1) != 1:
        raise ValueError("page_table must be int32 (B, pages) with unit column stride")
    if positions.dtype != torch.int32 or positions.shape != (B,) or not positions.is_contiguous():
        raise ValueError("positions must be contiguous int32 (B,)")
    a = N.LaKvAppendArgs()
    a.k_new, a.v_new = k_new.data_ptr(), v_new.data_ptr()
    a.k_pool, a.v_pool = k_pool.data_ptr(), v_pool.data_ptr()
    if fp8:
        for s in (k_scale, v_scale):
            if s is None or s.dtype != torch.float32:
                raise ValueError("fp8 pools need fp32 k_scale / v_scale (n_phys, Hkv, pool_page)")
        if k_scale.stride() != v_scale.stride():
            raise ValueError("k_scale / v_scale must share strides")
        a.s_stride = _paged_scale_stride(k_scale, k_pool)
        a.k_scale, a.v_scale = k_scale.data_ptr(), v_scale.data_ptr()
    a.page_table, a.positions = page_table.data_ptr(), positions.data_ptr()
    if (page_min is None) != (page_max is None):
        raise ValueError("pass both page_min and page_max, or neither")
    if page_min is not None:
        if fp8:
            raise ValueError("fp8 pools take no page bounds")
        if page_size is None or page_size <= 0:
            raise ValueError("page bounds need page_size")
        P = page_min.shape[2] if page_min.dim() == 4 else -1
        if page_min.shape != (B, Hkv, P, D) or page_max.shape != page_min.shape \
                or page_min.stride() != page_max.stride():
            raise ValueError("page_min / page_max must be (B, Hkv, n_pages, D) with equal strides")
        if page_min.dtype != k_new.dtype or page_max.dtype != k_new.dtype:
            raise ValueError("page bounds are stored in the key dtype")
        a.page_min, a.page_max = page_min.data_ptr(), page_max.data_ptr()
        a.meta_page, a.n_pages = int(page_size), P
        a.m_sb, a.m_sh, a.m_sp, a.m_sd = page_min.stride()
    a.B, a.Hkv, a.Tn, a.D = B, Hkv, Tn, D
    a.n_sb, a.n_sh, a.n_st = k_new.stride(0), k_new.stride(1), k_new.stride(2)
    a.n_phys, a.pool_page = n_phys, pool_page
    a.pt_sb, a.pt_pages = page_table.stride(0), page_table.shape[1]
    a.in_dtype = N.dtype_code(k_new.dtype)
    a.pool_dtype = N.dtype_code(k_pool.dtype)
    N.check(N.load().la_paged_kv_append(ctypes.byref(a), N.stream_handle(dev)), "paged_kv_append")
