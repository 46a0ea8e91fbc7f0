"""CPU oracle for the MI355X sparse-attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` (as the
checker) and the ``cpu_baseline`` leg of ``bench.py`` may import this package.
The product (``linattn_amd``) never imports it and has no CPU fallback.

This is a from-scratch restatement of the reference semantics, written with
numpy (fp64) plus ``liboracle.so`` (``oracle/csrc/la_oracle.c``, strict IEEE
fp64) for the arithmetic whose exact bits decide a selection.  Each function
cites the reference file:line it follows (paths relative to the reference
repository).

Parity status of each function is pinned in ``tests/test_oracle.py`` by
closed forms, the reference's own known-answer and invariant tests, brute force
on tiny inputs and the reference's own C decode built from source
(``oracle/_ref``).  The reference ships no golden-vector files, and its Python
is not run to make any: every function here is pinned by the checks above.
The order of ``torch.topk`` on ties is not reproduced (this build ranks ties
lowest index first), so that order is "parity unpinned" by design.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path
from typing import Optional, Sequence, Tuple

import numpy as np

__all__ = [
    "lib",
    "repeat_kv",
    "causal_mask",
    "block_reduce",
    "block_means",
    "dense_attention",
    "block_sparse_attention",
    "attend_lists",
    "page_bounds",
    "quest_scores",
    "quest_select",
    "page_select",
    "topk_rows",
    "indexer_scores",
    "indexer_topk",
    "block_select_scores",
    "block_select",
    "window_mask",
    "fp8_quantize",
    "fp8_decode",
    "effective_mask",
    "to_f64",
]

_HERE = Path(__file__).resolve().parent
_LIB: Optional[ctypes.CDLL] = None

_D = ctypes.POINTER(ctypes.c_double)
_I32 = ctypes.POINTER(ctypes.c_int32)
_I64 = ctypes.POINTER(ctypes.c_int64)
_F32 = ctypes.POINTER(ctypes.c_float)
_VP = ctypes.c_void_p
_i64 = ctypes.c_int64


def lib() -> ctypes.CDLL:
    """Load ``oracle/liboracle.so`` (built by ``make -C oracle``)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = _HERE / "liboracle.so"
    if not path.exists():
        raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
    L = ctypes.CDLL(str(path))
    L.or_quest_scores.argtypes = [_D, _D, _D, _i64, _i64, _i64, _i64, _D]
    L.or_indexer_scores.argtypes = [_D, _D, _D, _i64, _i64, _i64, _i64, _i64, _D]
    L.or_mean_pool.argtypes = [_D, _i64, _i64, _i64, _D]
    L.or_dot_rows.argtypes = [_D, _D, _i64, _i64, _i64, _D]
    L.or_topk_rows.argtypes = [_D, _i64, _i64, _I32, _I32, ctypes.c_int, _i64, _I32, _D]
    L.or_topk_rows.restype = ctypes.c_int
    L.or_fp8_e4m3fn.argtypes = [ctypes.c_uint8]
    L.or_fp8_e4m3fn.restype = ctypes.c_double
    L.or_sparse_attend.argtypes = [_D, _i64, _i64, _VP, _VP, ctypes.c_int, _F32, _F32, _I32, _i64,
                                   _i64, _i64, _i64, _i64, _i64, _I64, _i64, ctypes.c_double, _D, _D]
    L.or_sparse_attend.restype = ctypes.c_int
    L.or_exp_det.argtypes = [ctypes.c_double]
    L.or_exp_det.restype = ctypes.c_double
    L.or_xattn_select.argtypes = [_D, _D, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_double,
                                  ctypes.c_int, ctypes.c_double, _i64, _i64, _I32, _I32]
    L.or_xattn_select.restype = ctypes.c_int
    _LIB = L
    return L


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


# ----------------------------------------------------------------- dtypes --
def to_f64(x) -> np.ndarray:
    """Exact fp64 copy of a torch tensor / numpy array (fp32, bf16, fp16)."""
    try:
        import torch

        if isinstance(x, torch.Tensor):
            x = x.detach().cpu()
            if x.dtype in (torch.bfloat16, torch.float16):
                x = x.to(torch.float32)
            return x.to(torch.float64).numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(x, dtype=np.float64)


# ------------------------------------------------------------------- core --
def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """(B, Hkv, T, D) -> (B, Hkv*n_rep, T, D); core.py:84-89."""
    if n_rep == 1:
        return x
    return np.repeat(x, n_rep, axis=1)


def causal_mask(q_len: int, kv_len: int, offset: int = 0) -> np.ndarray:
    """True where key j <= offset + i; core.py:92-100."""
    qi = np.arange(q_len)[:, None] + offset
    kj = np.arange(kv_len)[None, :]
    return kj <= qi


def block_reduce(x: np.ndarray, block: int, axis: int = -2) -> np.ndarray:
    """Mean-pool blocks along ``axis``; the tail repeats the last row; core.py:102-120."""
    if block == 1:
        return x
    x = np.moveaxis(x, axis, -2)
    t = x.shape[-2]
    pad = (-t) % block
    if pad:
        x = np.concatenate([x, np.repeat(x[..., -1:, :], pad, axis=-2)], axis=-2)
    x = x.reshape(*x.shape[:-2], x.shape[-2] // block, block, x.shape[-1]).mean(axis=-2)
    return np.moveaxis(x, -2, axis)


def _softmax(s: np.ndarray) -> np.ndarray:
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(s - m)
    z = e.sum(-1, keepdims=True)
    return np.divide(e, z, out=np.zeros_like(e), where=z > 0)


def dense_attention(q, k, v, *, causal: bool = True, scale: Optional[float] = None,
                    mask: Optional[np.ndarray] = None) -> np.ndarray:
    """softmax(q k^T * scale + mask) v in fp64; core.py:148-181.

    q (B,H,Tq,D), k/v (B,Hkv,Tk,D).  ``mask`` is True where allowed.  A fully
    masked row returns zeros (the reference returns NaN there; no selector
    produces such a row, selection.py:94-107)."""
    q, k, v = to_f64(q), to_f64(k), to_f64(v)
    scale = scale if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    kr = repeat_kv(k, q.shape[1] // k.shape[1])
    vr = repeat_kv(v, q.shape[1] // v.shape[1])
    s = np.matmul(q, np.swapaxes(kr, -1, -2)) * scale
    if mask is not None:
        allow = mask
    elif causal:
        allow = causal_mask(q.shape[-2], k.shape[-2], offset=k.shape[-2] - q.shape[-2])
    else:
        allow = None
    if allow is not None:
        s = np.where(allow, s, -np.inf)
    return np.matmul(_softmax(s), vr)


def block_sparse_attention(q, k, v, block_ids, *, block_size: int) -> np.ndarray:
    """Gather the listed blocks, then softmax attention; block_sparse.py:40-75.

    ids (B, Hkv, N) or (B, Hkv, Tq, N); a listed block is gathered once per
    listing (multiset), tokens >= T_k are masked, scale 1/sqrt(D), no causal
    mask.  Extension: -1 entries are skipped."""
    q, k, v = to_f64(q), to_f64(k), to_f64(v)
    ids = np.asarray(block_ids, dtype=np.int64)
    b, hq, tq, d = q.shape
    hkv, tk = k.shape[1], k.shape[2]
    g = hq // hkv
    if ids.ndim == 3:
        ids = np.broadcast_to(ids[:, :, None, :], (b, hkv, tq, ids.shape[-1]))
    raw = ids[..., None] * block_size + np.arange(block_size)  # (B,Hkv,Tq,N,bs)
    valid = (raw < tk) & (ids[..., None] >= 0)
    raw = np.clip(raw, 0, tk - 1).reshape(b, hkv, tq, -1)
    valid = valid.reshape(b, hkv, tq, -1)
    out = np.zeros((b, hq, tq, d))
    for bi in range(b):
        for hk in range(hkv):
            ks = k[bi, hk][raw[bi, hk]]  # (Tq, M, D)
            vs = v[bi, hk][raw[bi, hk]]
            for j in range(g):
                h = hk * g + j
                s = np.einsum("td,tmd->tm", q[bi, h], ks) / math.sqrt(d)
                s = np.where(valid[bi, hk], s, -np.inf)
                out[bi, h] = np.einsum("tm,tmd->td", _softmax(s), vs)
    return out


def attend_lists(q, k, v, ids: np.ndarray, *, unit: int, scale: Optional[float] = None,
                 causal: bool = False, offset: int = 0, kv_len: Optional[Sequence[int]] = None,
                 page_table: Optional[np.ndarray] = None, page_size: int = 0,
                 k_scale=None, v_scale=None, counts: Optional[np.ndarray] = None) -> np.ndarray:
    """Exact fp64 attention of every query row over its listed units.

    Semantics of block_sparse.py:40-75 and decode_attn.c:39-65, generalised to
    what the HIP executor accepts: ids (B, L, Tq|1, N) with L = Hkv (list shared
    by the GQA group) or L = Hq (one list per query head); unit ids cover
    [u*unit, (u+1)*unit); -1 skipped; tokens >= kv_len masked; with ``causal``
    token j is masked for query t when j > offset + t.  KV is contiguous
    (B, Hkv, T, D) or, with ``page_table`` (B, P), a pool
    [phys][Hkv][page_size][D].  fp8 KV passes uint8 codes plus fp32 per-token
    scales.  Uses ``or_sparse_attend`` (C) per (row, head group)."""
    import torch

    L = lib()

    def raw(x):
        if isinstance(x, torch.Tensor):
            x = x.detach().cpu().contiguous()
            if x.dtype == torch.bfloat16:
                return x.view(torch.int16).numpy().view(np.uint16), 1
            if x.dtype == torch.float8_e4m3fn:
                return x.view(torch.uint8).numpy(), 3
            return x.to(torch.float32).numpy(), 0
        x = np.ascontiguousarray(x)
        if x.dtype == np.uint8:
            return x, 3
        return x.astype(np.float32), 0

    qf = to_f64(q)
    kr, dt = raw(k)
    vr, _ = raw(v)
    ids = np.asarray(ids, dtype=np.int64)
    B, Hq, Tq, D = qf.shape
    Lh = ids.shape[1]
    paged = page_table is not None
    Hkv = kr.shape[1]
    if paged:
        pt = np.ascontiguousarray(np.asarray(page_table, dtype=np.int32))
        T = pt.shape[1] * page_size
    else:
        T = kr.shape[2]
    group = Hq // Hkv
    G = group if Lh == Hkv else 1
    ks = vs = None
    if k_scale is not None:
        ks = np.ascontiguousarray(to_f64(k_scale).astype(np.float32))
        vs = np.ascontiguousarray(to_f64(v_scale).astype(np.float32))
    scale = scale if scale is not None else 1.0 / math.sqrt(D)
    out = np.zeros((B, Hq, Tq, D))
    for b in range(B):
        ln = T if kv_len is None else int(kv_len[b])
        for ih in range(Lh):
            kvh = ih if Lh == Hkv else ih // group
            heads = [ih * G + g for g in range(G)]
            for t in range(Tq):
                row = ids[b, ih, t if ids.shape[2] > 1 else 0]
                if counts is not None:
                    row = row[: int(counts[b, ih, t if counts.shape[2] > 1 else 0])]
                lim = ln - 1 if not causal else min(ln - 1, offset + t)
                toks = []
                for u in row:
                    if u < 0:
                        continue
                    for j in range(unit):
                        tok = int(u) * unit + j
                        if tok <= lim:
                            toks.append(tok)
                tk = np.asarray(toks if toks else [-1], dtype=np.int64)
                qv = np.ascontiguousarray(qf[b, heads, t, :])
                o = np.zeros((G, D))
                work = np.zeros(max(1, len(tk)))
                if paged:
                    kb, vb = kr, vr
                    ptr = pt[b]
                    kst = vst = sst = 0
                    ksp = ks.ctypes.data_as(_F32) if ks is not None else None
                    vsp = vs.ctypes.data_as(_F32) if vs is not None else None
                    kvh_arg = kvh
                else:
                    kb = np.ascontiguousarray(kr[b, kvh])
                    vb = np.ascontiguousarray(vr[b, kvh])
                    ptr = None
                    kst = vst = D
                    sst = 1
                    ksp = np.ascontiguousarray(ks[b, kvh]).ctypes.data_as(_F32) if ks is not None else None
                    vsp = np.ascontiguousarray(vs[b, kvh]).ctypes.data_as(_F32) if vs is not None else None
                    kvh_arg = 0
                L.or_sparse_attend(_p(qv, _D), G, D, kb.ctypes.data, vb.ctypes.data, dt, ksp, vsp,
                                   ptr.ctypes.data_as(_I32) if ptr is not None else None,
                                   page_size, Hkv, kvh_arg, kst, vst, sst, _p(tk, _I64), len(tk),
                                   scale, _p(o, _D), _p(work, _D))
                out[b, heads, t, :] = o
    return out


# ------------------------------------------------------------------ quest --
def page_bounds(k, page_size: int) -> Tuple[np.ndarray, np.ndarray]:
    """Channel-wise min/max per page, padded rows +inf/-inf; quest_pages.py:38-48."""
    k = to_f64(k)
    b, h, t, d = k.shape
    n_pages = (t + page_size - 1) // page_size
    pad = n_pages * page_size - t
    kmin = np.concatenate([k, np.full((b, h, pad, d), np.inf)], axis=2) if pad else k
    kmax = np.concatenate([k, np.full((b, h, pad, d), -np.inf)], axis=2) if pad else k
    mins = kmin.reshape(b, h, n_pages, page_size, d).min(axis=3)
    maxs = kmax.reshape(b, h, n_pages, page_size, d).max(axis=3)
    return mins, maxs


def quest_scores(q, mins, maxs) -> np.ndarray:
    """Upper bounds sum_d max(q_d m_d, q_d M_d), one per query head:
    (B,Hq,Tq,P); quest_pages.py:51-55, selection.py:203-212 (repeat_kv of the
    metadata).  fp64, d increasing (la_oracle.c)."""
    q, mins, maxs = to_f64(q), to_f64(mins), to_f64(maxs)
    B, Hq, Tq, D = q.shape
    Hkv, P = mins.shape[1], mins.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, Tq, P))
    L = lib()
    for b in range(B):
        for hk in range(Hkv):
            mn = np.ascontiguousarray(mins[b, hk])
            mx = np.ascontiguousarray(maxs[b, hk])
            for t in range(Tq):
                qv = np.ascontiguousarray(q[b, hk * G:(hk + 1) * G, t, :])
                o = np.zeros((G, P))
                L.or_quest_scores(_p(qv, _D), _p(mn, _D), _p(mx, _D), 1, G, P, D, _p(o, _D))
                out[b, hk * G:(hk + 1) * G, t, :] = o
    return out


def topk_rows(scores: np.ndarray, k: int, n_valid=None, own=None, force_own: bool = False):
    """Top-k per row by (value desc, index asc) over the first n_valid entries;
    ``own`` ranks first when ``force_own``.  Returns (idx int32 (...,k) -1
    padded, values fp64 -inf padded).  The reference's topk_blocks
    (selection.py:51-59) uses torch.topk, whose tie order is unspecified; the
    lowest-index rule is this build's specification."""
    s = np.ascontiguousarray(to_f64(scores))
    lead, n = s.shape[:-1], s.shape[-1]
    R = int(np.prod(lead)) if lead else 1
    s2 = s.reshape(R, n)
    nv = None if n_valid is None else np.ascontiguousarray(
        np.broadcast_to(np.asarray(n_valid, dtype=np.int32), lead).reshape(R))
    ow = None if own is None else np.ascontiguousarray(
        np.broadcast_to(np.asarray(own, dtype=np.int32), lead).reshape(R))
    idx = np.zeros((R, k), dtype=np.int32)
    val = np.zeros((R, k))
    rc = lib().or_topk_rows(_p(s2, _D), R, n, nv.ctypes.data_as(_I32) if nv is not None else None,
                            ow.ctypes.data_as(_I32) if ow is not None else None, int(force_own), k,
                            _p(idx, _I32), _p(val, _D))
    if rc != 0:
        raise MemoryError("or_topk_rows")
    return idx.reshape(*lead, k), val.reshape(*lead, k)


def quest_select(q, mins, maxs, *, page_size: int, topk: int, offset: int = 0,
                 gqa_union: bool = True) -> np.ndarray:
    """QuestAttention.page_selection (selection.py:214-237) as unit lists.

    Pages with start > query position are invisible; the query's own page is
    forced inside the top-k; k = max(1, min(topk, n_pages)) but only visible
    pages are ever kept (the reference's extra picks among -inf scores are
    removed by the causal mask, selection.py:94-98).  Union mode returns
    (B, Hkv, Tq, G*k) ascending, -1 padded; per-head mode (B, Hq, Tq, k) by
    (score desc, index asc)."""
    sc = quest_scores(q, mins, maxs)
    B, Hq, Tq, P = sc.shape
    Hkv = to_f64(mins).shape[1]
    G = Hq // Hkv
    pos = np.arange(Tq) + offset
    n_valid = np.minimum(P, pos // page_size + 1)
    own = np.minimum(pos // page_size, P - 1)
    k = max(1, min(topk, P))
    idx, _ = topk_rows(sc, k, n_valid=n_valid, own=own, force_own=True)
    if not gqa_union or G == 1:
        return idx
    out = np.full((B, Hkv, Tq, G * k), -1, dtype=np.int32)
    for b in range(B):
        for hk in range(Hkv):
            for t in range(Tq):
                u = np.unique(idx[b, hk * G:(hk + 1) * G, t].reshape(-1))
                u = u[u >= 0]
                out[b, hk, t, :len(u)] = u
    return out


def page_select(q, mins, maxs, page_size: int, topk: int, *, offset: int = 0):
    """page_select_torch (quest_pages.py:58-78) with the own-page scatter of
    selection.py:224-231 (defect D1 fixed): returns (ids (B,H,Tq,k) by (score
    desc, index asc), scores (B,H,Tq,P) with invisible pages -inf and the own
    page +inf).  Queries read metadata of their own KV head (GQA)."""
    sc = quest_scores(q, mins, maxs)
    B, Hq, Tq, P = sc.shape
    pos = np.arange(Tq) + offset
    visible = (np.arange(P)[None, :] * page_size) <= pos[:, None]
    sc = np.where(visible, sc, -np.inf)
    own = np.minimum(pos // page_size, P - 1)
    sc[:, :, np.arange(Tq), own] = np.inf
    k = max(1, min(topk, P))
    n_valid = np.minimum(P, pos // page_size + 1)  # visible pages are a prefix
    idx, _ = topk_rows(sc, k, n_valid=n_valid, own=own, force_own=True)
    return idx, sc


# ---------------------------------------------------------------- indexer --
def indexer_scores(q_idx, k_idx, w, *, causal: bool = False, offset: int = 0) -> np.ndarray:
    """I[b,t,s] = sum_h w[b,t,h] ReLU(q[b,t,h].k[b,s,h]); fused_indexer.py:52-60.
    fp64 canonical order (la_oracle.c); with ``causal`` keys s > offset + t are
    -inf (not scored)."""
    q, k, w = to_f64(q_idx), to_f64(k_idx), to_f64(w)
    B, Tq, HI, d = q.shape
    Tk = k.shape[1]
    out = np.full((B, Tq, Tk), -np.inf)
    L = lib()
    for b in range(B):
        qb, kb, wb = (np.ascontiguousarray(x[b]) for x in (q, k, w))
        o = np.full((Tq, Tk), -np.inf)
        L.or_indexer_scores(_p(qb, _D), _p(kb, _D), _p(wb, _D), Tq, Tk, HI, d,
                            offset if causal else -1, _p(o, _D))
        out[b] = o
    return out


def indexer_topk(q_idx, k_idx, w, k: int, *, causal: bool = False, offset: int = 0,
                 causal_unit: int = 1):
    """indexer_topk_torch (fused_indexer.py:63-73): top-k by (score desc, index
    asc), int32 indices, -1 / -inf padding when fewer than k keys are valid.
    With ``causal_unit`` = m keys are groups of m tokens and group s is visible
    when s*m <= offset + t (selection.py:739-747)."""
    sc = indexer_scores(q_idx, k_idx, w, causal=False)
    B, Tq, Tk = sc.shape
    m = max(1, causal_unit)
    nv = np.minimum(Tk, (np.arange(Tq) + offset) // m + 1) if causal else np.full(Tq, Tk)
    idx, val = topk_rows(np.where(np.isfinite(sc), sc, 0.0), k, n_valid=nv)
    return val, idx


# ----------------------------------------------------- block selection C3 --
def block_select_scores(q, k, block: int) -> np.ndarray:
    """Pooled block scores mean(q_blk) . mean(k_blk), (B,Hq,nqb,nkb); the
    MInference block-sparse estimator (selection.py:339-345) without its
    positive 1/sqrt(D) factor.  fp64 canonical order (la_oracle.c)."""
    q, k = to_f64(q), to_f64(k)
    B, Hq, T, D = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    nqb, nkb = (T + block - 1) // block, (Tk + block - 1) // block
    L = lib()
    kp = np.zeros((B, Hkv, nkb, D))
    qp = np.zeros((B, Hq, nqb, D))
    for b in range(B):
        for h in range(Hkv):
            x = np.ascontiguousarray(k[b, h])
            o = np.zeros((nkb, D))
            L.or_mean_pool(_p(x, _D), Tk, D, block, _p(o, _D))
            kp[b, h] = o
        for h in range(Hq):
            x = np.ascontiguousarray(q[b, h])
            o = np.zeros((nqb, D))
            L.or_mean_pool(_p(x, _D), T, D, block, _p(o, _D))
            qp[b, h] = o
    out = np.zeros((B, Hq, nqb, nkb))
    for b in range(B):
        for h in range(Hq):
            a = np.ascontiguousarray(qp[b, h])
            c = np.ascontiguousarray(kp[b, h // G])
            o = np.zeros((nqb, nkb))
            L.or_dot_rows(_p(a, _D), _p(c, _D), nqb, nkb, D, _p(o, _D))
            out[b, h] = o
    return out


def block_select(q, k, *, block: int, topk: int, sink_blocks: int = 1,
                 window_blocks: int = 4) -> np.ndarray:
    """Config-C3 block lists (B,Hq,nqb,W) ascending, -1 padded: top-`topk` key
    blocks kb <= qb by pooled score (selection.py:339-350, ties to the lowest
    index), OR the sink blocks [0, sink_blocks) and the local window
    [qb-window_blocks+1, qb] (which includes the diagonal block,
    selection.py:351)."""
    sc = block_select_scores(q, k, block)
    B, Hq, nqb, nkb = sc.shape
    qb = np.arange(nqb)
    idx, _ = topk_rows(sc, topk, n_valid=np.minimum(nkb, qb + 1))
    W = topk + sink_blocks + window_blocks
    out = np.full((B, Hq, nqb, W), -1, dtype=np.int32)
    for b in range(B):
        for h in range(Hq):
            for i in range(nqb):
                s = set(int(x) for x in idx[b, h, i] if x >= 0)
                s.update(range(min(sink_blocks, i + 1)))
                s.update(range(max(0, i - window_blocks + 1), i + 1))
                u = sorted(s)
                out[b, h, i, :len(u)] = u
    return out


# ------------------------------------------------------ per-query routing --
def block_means(k, block: int) -> np.ndarray:
    """The pooled keys the gate reads: block_reduce (core.py:102-120; the tail
    block repeats the last row) of k (B, H, T, D) in fp64 with each block's
    rows added in order and the sum divided by ``block`` (or_mean_pool, the
    pooling of gate_select).  Returns (B, H, ceil(T / block), D)."""
    k = to_f64(k)
    B, H, T, D = k.shape
    nkb = (T + block - 1) // block
    L = lib()
    out = np.zeros((B, H, nkb, D))
    for b in range(B):
        for h in range(H):
            x = np.ascontiguousarray(k[b, h])
            o = np.zeros((nkb, D))
            L.or_mean_pool(_p(x, _D), T, D, block, _p(o, _D))
            out[b, h] = o
    return out


def gate_select(q, k, *, block: int, topk: int, offset: int = 0) -> np.ndarray:
    """MoBA's gate routing (selection.py:610-640), also NSA's blockwise
    selection (native_sparse.py:78-93): for query t at position offset + t,
    blocks whose start is <= the position are visible; gate = q_t .
    mean(K block) (block_reduce with the tail repeating the last row,
    core.py:102-120; the positive 1/sqrt(D) left out), fp64 with products
    added over d in order (la_oracle.c); the top min(topk, n_blocks) visible
    blocks (ties to the lowest) plus the own block.  Returns (B, Hq, Tq,
    min(topk, n_blocks) + 1) ascending, -1 padded."""
    q, k = to_f64(q), to_f64(k)
    B, Hq, Tq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    nkb = (T + block - 1) // block
    L = lib()
    kp = np.zeros((B, Hkv, nkb, D))
    for b in range(B):
        for h in range(Hkv):
            x = np.ascontiguousarray(k[b, h])
            o = np.zeros((nkb, D))
            L.or_mean_pool(_p(x, _D), T, D, block, _p(o, _D))
            kp[b, h] = o
    gates = np.zeros((B, Hq, Tq, nkb))
    for b in range(B):
        for h in range(Hq):
            a = np.ascontiguousarray(q[b, h])
            c = np.ascontiguousarray(kp[b, h // G])
            o = np.zeros((Tq, nkb))
            L.or_dot_rows(_p(a, _D), _p(c, _D), Tq, nkb, D, _p(o, _D))
            gates[b, h] = o
    pos = np.arange(Tq) + offset
    n_valid = np.minimum(nkb, pos // block + 1)
    own = np.minimum(pos // block, nkb - 1)
    kk = max(1, min(topk, nkb))
    idx, _ = topk_rows(gates, kk, n_valid=n_valid)
    out = np.full((B, Hq, Tq, kk + 1), -1, dtype=np.int32)
    for b in range(B):
        for h in range(Hq):
            for t in range(Tq):
                u = sorted(set(int(x) for x in idx[b, h, t] if x >= 0) | {int(own[t])})
                out[b, h, t, :len(u)] = u
    return out


# ------------------------------------------------------------- XAttention --
def xattn_select(q, k, *, block: int = 8, stride: int = 8, threshold=0.9, offset: int = 0,
                 topk: Optional[int] = None, top_ratio: Optional[float] = None):
    """XAttention's block selection (selection.py:528-595) per (b, query
    head, query block), in the integer-mass form the kernel computes
    (la_oracle.c or_xattn_select): antidiagonal slot scores in fp64, weights
    by a deterministic exp, block masses as fixed-point integers, then the
    cumulative threshold (``threshold`` a float or one value per query head)
    or, with ``topk``, the top-k blocks; own block OR'd, invisible blocks
    dropped.  Returns (ids (B, Hq, n_qb, width) ascending, -1 padded,
    counts (B, Hq, n_qb)); width = n_kb, or min(topk, n_kb) + 1.

    ``top_ratio`` (select_mode "top_ratio", selection.py:583-585): the
    reference keeps the shortest prefix of blocks, by mass, whose cumulative
    mass reaches the count c = max(1, ceil(n_visible * ratio)) (the
    _select_with_per_head rule, :598-606, with c in place of a threshold),
    or every block when none does.  A row's masses are a softmax over its
    visible blocks: each is positive and they sum to 1 <= c, so the prefix
    reaches c only when it holds every visible block, and either way every
    visible block is kept (width n_kb)."""
    q, k = to_f64(q), to_f64(k)
    B, Hq, Tq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    n_qb, n_kb = -(-Tq // block), -(-T // block)
    if top_ratio is not None:
        ids = np.full((B, Hq, n_qb, n_kb), -1, dtype=np.int32)
        counts = np.zeros((B, Hq, n_qb), dtype=np.int32)
        for i in range(n_qb):
            n_vis = min(n_kb, (offset + i * block) // block + 1)
            c = max(1, math.ceil(n_vis * top_ratio))
            assert c >= 1  # the cumulative mass (a sum of positive masses, total 1) reaches c last
            ids[:, :, i, :n_vis] = np.arange(n_vis, dtype=np.int32)
            counts[:, :, i] = n_vis
        return ids, counts
    mode = 1 if topk is not None else 0
    width = min(topk, n_kb) + 1 if mode else n_kb
    alphas = np.broadcast_to(np.asarray(threshold, dtype=np.float64), (Hq,))
    inv = 1.0 / math.sqrt(D)
    L = lib()
    ids = np.full((B, Hq, n_qb, width), -1, dtype=np.int32)
    counts = np.zeros((B, Hq, n_qb), dtype=np.int32)
    for b in range(B):
        for h in range(Hq):
            a = np.ascontiguousarray(q[b, h])
            c = np.ascontiguousarray(k[b, h // G])
            o = np.zeros((n_qb, width), dtype=np.int32)
            n = np.zeros(n_qb, dtype=np.int32)
            rc = L.or_xattn_select(_p(a, _D), _p(c, _D), Tq, T, D, block, stride, offset, inv,
                                   mode, float(alphas[h]), int(topk or 0), width, _p(o, _I32),
                                   _p(n, _I32))
            if rc != 0:
                raise ValueError("or_xattn_select: bad arguments")
            ids[b, h], counts[b, h] = o, n
    return ids, counts


def exp_det(x: float) -> float:
    """The deterministic exp of the XAttention weights (la_oracle.c)."""
    return lib().or_exp_det(float(x))


# ------------------------------------------------------------------ local --
def window_mask(t_q: int, t_k: int, offset: int, window: int, sink: int) -> np.ndarray:
    """j <= i and (i - j < window or j < sink); local.py:47-53."""
    qi = np.arange(t_q)[:, None] + offset
    kj = np.arange(t_k)[None, :]
    return (kj <= qi) & (((qi - kj) < window) | (kj < sink))


def effective_mask(select: np.ndarray, offset: int = 0) -> np.ndarray:
    """BlockSelectionAttention.effective_mask (selection.py:86-108): the
    selection (..., Tq, Tk) intersected with causality (key j <= offset + t);
    a row left with no key reads the query's own token, position offset + t
    clamped to the last key (selection.py:100-107)."""
    sel = np.asarray(select, dtype=bool)
    tq, tk = sel.shape[-2:]
    allow = sel & causal_mask(tq, tk, offset)
    empty = ~allow.any(-1)
    own = np.minimum(np.arange(tq) + offset, tk - 1)
    fallback = np.zeros_like(allow)
    fallback[..., np.arange(tq), own] = True
    return allow | (fallback & empty[..., None])


# -------------------------------------------------------------------- fp8 --
_FP8_TABLE: Optional[np.ndarray] = None


def fp8_decode(codes: np.ndarray) -> np.ndarray:
    """OCP e4m3fn codes (uint8) -> fp64 (la_oracle.c, from the format spec)."""
    global _FP8_TABLE
    if _FP8_TABLE is None:
        _FP8_TABLE = np.array([lib().or_fp8_e4m3fn(i) for i in range(256)])
    return _FP8_TABLE[np.asarray(codes, dtype=np.uint8)]


def fp8_quantize(x):
    """Per-token (group = head_dim) fp8 e4m3 codec of kv/quant.py:76-109:
    scale = max|x| / 448 (clamped to 1e-8), codes = (x / scale) cast to
    float8_e4m3fn (torch's round-to-nearest-even cast).  Returns torch tensors
    (codes float8_e4m3fn, scales fp32 with the last dim kept as 1)."""
    import torch

    xf = x.detach().to(torch.float32)
    scale = xf.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 448.0
    codes = (xf / scale).to(torch.float8_e4m3fn)
    return codes, scale
