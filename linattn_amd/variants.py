"""``hip_*`` attention variants: the reference's variant semantics executed by
the gfx950 kernels.

Follows the backend-adapter pattern of the reference's MLX backend
(src/linattn/kernels/mlx/adapter.py:34-107): each class is an
``AttentionVariant`` whose ``attend`` builds a selection with the HIP
selection kernels and runs the HIP executor, while ``stats``/``read_budget``/
``flops``/``memory_bytes`` keep the reference's accounting.

* ``hip_quest``          QuestAttention (variants/selection.py:139-248)
* ``hip_dsa``            DSAAttention (selection.py:659-789), token or pooled-group
                         indexing, sink + window OR'd in
* ``hip_moba``           MoBAAttention (selection.py:610-640): per-query routing by
                         q . mean(K block), own block added
* ``hip_xattention``     XAttention (selection.py:500-595): strided antidiagonal
                         block scores, cumulative-mass threshold (or top-k)
* ``hip_sliding_window`` SlidingWindowAttention (variants/local.py:22-61)
* ``hip_streaming_sink`` StreamingSinkAttention (local.py:64-80)

Every variant reads exactly the mask the reference's ``effective_mask``
describes: selection intersected with causality (selection.py:86-108).
"""

from __future__ import annotations

import math
from typing import Any, Dict, Optional

import torch

from linattn_amd.core import AttnConfig, AttentionVariant
from linattn_amd.kernels.block_sparse import sparse_attention
from linattn_amd.kernels.fused_indexer import indexer_topk
from linattn_amd.kernels.quest_pages import alloc_page_meta, page_update_hip, quest_select_hip
from linattn_amd.kernels.prefill import block_sparse_prefill
from linattn_amd.kernels.routing import block_means_hip, gate_select_hip, xattn_select_hip

__all__ = ["HipAttention", "HipQuest", "HipDSA", "HipMoBA", "HipXAttention", "HipSlidingWindow",
           "HipStreamingSink", "SUPPORTED"]


def _reads_per_query(ids: torch.Tensor, unit: int, offset: int, t_k: int) -> float:
    """Mean tokens read per query row: listed units intersected with
    causality and the cache length (ids (B, L, Tq, W), -1 padded)."""
    tq = ids.shape[2]
    lim = torch.clamp(torch.arange(tq, device=ids.device) + offset + 1, max=t_k)
    start = ids.to(torch.int64) * unit
    n = torch.clamp(lim.view(1, 1, tq, 1) - start, min=0, max=unit)
    n = torch.where(ids >= 0, n, torch.zeros_like(n))
    return float(n.sum(-1).to(torch.float64).mean())


class HipAttention(AttentionVariant):
    """Base of the HIP variants."""

    family = "hip"
    reference = "base"

    def __init__(self, cfg: Optional[AttnConfig] = None, **kw: Any):
        super().__init__(cfg, **kw)
        self.name = f"hip_{self.reference}"
        self._extra: Dict[str, float] = {}

    def stats(self) -> Dict[str, float]:
        return dict(self._extra)

    def forward(self, q, k, v, *, state=None, chunk=None, causal=True, collect_stats=False):
        """The reference driver (core.py:231-279).  fp64 inputs (the reference
        validates in float64) run in fp32 on the GPU and come back as fp64."""
        if q.dtype == torch.float64:
            res = super().forward(q.float(), k.float(), v.float(), state=state, chunk=chunk,
                                  causal=causal, collect_stats=collect_stats)
            return (res[0].double(),) + tuple(res[1:])
        return super().forward(q, k, v, state=state, chunk=chunk, causal=causal,
                               collect_stats=collect_stats)


class HipQuest(HipAttention):
    """Quest page selection (selection.py:139-248) on the GPU.

    extras: ``page_size`` (default block_size), ``gqa_union`` (default True),
    ``dense_layers`` / ``layer_idx`` (default 2 / 2: sparse).  Page metadata
    lives in the state as ``page_min`` / ``page_max`` and is refreshed only for
    pages touched by new keys (selection.py:181-201)."""

    reference = "quest"

    def __init__(self, cfg=None, **kw):
        super().__init__(cfg, **kw)
        ex = self.cfg.extras
        self.dense_layers = int(ex.get("dense_layers", 2))
        self.layer_idx = int(ex.get("layer_idx", 2))
        self.page_size = int(ex.get("page_size", self.cfg.block_size))
        self.gqa_union = bool(ex.get("gqa_union", True))

    def prepare_state(self, batch, device, dtype):
        state = super().prepare_state(batch, device, dtype)
        state["page_min"] = None
        state["page_max"] = None
        return state

    def push_kv(self, state, k, v):
        start = state["k"].shape[-2]
        state = super().push_kv(state, k, v)
        kk = state["k"]
        B, Hkv, t, D = kk.shape
        ps = self.page_size
        n_pages = (t + ps - 1) // ps
        first = start // ps
        if n_pages == 0:
            return state
        mins, maxs = alloc_page_meta(B, Hkv, n_pages, D, kk.dtype, kk.device)
        if first > 0 and state["page_min"] is not None:
            mins[:, :, :first].copy_(state["page_min"][:, :, :first])
            maxs[:, :, :first].copy_(state["page_max"][:, :, :first])
        page_update_hip(kk, ps, n_pages, out=(mins, maxs), first_page=first)
        state["page_min"], state["page_max"] = mins, maxs
        return state

    def attend(self, q, state, offset: int = 0):
        k, v = state["k"], state["v"]
        t_k = k.shape[-2]
        ps = self.page_size
        n_pages = (t_k + ps - 1) // ps
        if self.layer_idx < self.dense_layers:
            ids = torch.arange(n_pages, dtype=torch.int32, device=q.device)
            ids = ids.view(1, 1, 1, -1).expand(q.shape[0], k.shape[1], 1, n_pages)
            counts = None
            self._extra = {"pages_per_query": float(n_pages)}
        else:
            ids, counts = quest_select_hip(q, state["page_min"], state["page_max"], page_size=ps,
                                           topk=self.cfg.topk_blocks, offset=offset,
                                           gqa_union=self.gqa_union)
            self._extra = {"pages_per_query": float(counts.to(torch.float64).mean())}
        out = sparse_attention(q, k, v, ids, unit=ps, counts=counts, causal=True, offset=offset,
                               out_dtype=q.dtype)
        reads = _reads_per_query(ids if ids.shape[2] == q.shape[2] else
                                 ids.expand(-1, -1, q.shape[2], -1), ps, offset, t_k)
        self._extra["reads_per_query"] = reads
        return out

    def read_budget(self, seq_len, batch=1):
        c = self.cfg
        return float(min(seq_len, c.topk_blocks * c.block_size + c.window_size))

    def flops(self, seq_len, batch=1):
        n_pages = (seq_len + self.page_size - 1) // self.page_size
        sel = 2 * batch * self.cfg.n_heads * seq_len * n_pages * self.cfg.head_dim
        return super().flops(seq_len, batch) + int(sel)


class HipSlidingWindow(HipAttention):
    """Causal window of ``window_size`` tokens plus ``sink_size`` leading
    tokens (local.py:47-53), as per-query token lists."""

    reference = "sliding_window"

    def _lists(self, t_q: int, offset: int, device) -> torch.Tensor:
        sink, win = self.cfg.sink_size, self.cfg.window_size
        pos = torch.arange(t_q, device=device).view(-1, 1) + offset
        s = torch.arange(sink, device=device).view(1, -1).expand(t_q, sink)
        s = torch.where(s <= pos, s, torch.full_like(s, -1))
        w = pos - torch.arange(win, device=device).view(1, -1)  # pos, pos-1, ...
        w = torch.where((w >= sink) & (w >= 0), w, torch.full_like(w, -1))
        return torch.cat([s, w], dim=1).to(torch.int32)

    def attend(self, q, state, offset: int = 0):
        k, v = state["k"], state["v"]
        lists = self._lists(q.shape[2], offset, q.device)
        ids = lists.view(1, 1, q.shape[2], -1).expand(q.shape[0], k.shape[1], -1, -1)
        out = sparse_attention(q, k, v, ids, unit=1, causal=True, offset=offset,
                               out_dtype=q.dtype)
        self._extra = {"reads_per_query": _reads_per_query(ids, 1, offset, k.shape[-2])}
        return out

    def read_budget(self, seq_len, batch=1):
        return float(min(seq_len, self.cfg.window_size + self.cfg.sink_size))

    def memory_bytes(self, seq_len, batch=1):
        kept = min(seq_len, self.cfg.window_size + self.cfg.sink_size)
        return int(batch * self.cfg.n_kv_heads * kept * self.cfg.head_dim * 2 * 2)


class HipStreamingSink(HipSlidingWindow):
    """StreamingLLM naming of the same computation (local.py:64-80)."""

    reference = "streaming_sink"


class HipDSA(HipAttention):
    """DeepSeek Sparse Attention (selection.py:659-789) with the lightning
    indexer on the GPU.

    The indexer projections follow the reference parameterisation: one
    (head_dim x indexer_dim) projection per (attention head, indexer head),
    drawn from ``torch.Generator().manual_seed(cfg.seed)`` times 0.02, and
    head weights softmax(1/H_I) (selection.py:700-716); ``load_indexer``
    installs trained ones.  Keys are indexed per attention head; with
    ``compress_ratio`` m > 1 the indexer scores mean-pooled groups of m keys
    (block_reduce, tail repeats the last row) and the kept groups expand to
    their tokens.  Sink tokens and the local window are OR'd in
    (selection.py:757-761).  Like the reference, the top-k ignores causality
    unless ``extras["indexer_causal"]`` (pooled groups always use the
    reference's group-start mask, selection.py:743-747); the executor then
    reads only causal tokens."""

    reference = "dsa"
    trained = True

    def __init__(self, cfg=None, **kw):
        super().__init__(cfg, **kw)
        ex = self.cfg.extras
        self.n_indexer_heads = int(ex.get("indexer_heads", 8))
        self.indexer_dim = int(ex.get("indexer_dim", 16))
        self.compress_ratio = int(ex.get("compress_ratio", self.cfg.compress_ratio))
        self.indexer_causal = bool(ex.get("indexer_causal", False))
        gen = torch.Generator().manual_seed(self.cfg.seed)
        self.q_proj = torch.randn(self.cfg.n_heads, self.n_indexer_heads, self.cfg.head_dim,
                                  self.indexer_dim, generator=gen) * 0.02
        self.head_weights = torch.full((self.n_indexer_heads,), 1.0 / self.n_indexer_heads)

    def load_indexer(self, q_proj: torch.Tensor, head_weights: torch.Tensor) -> None:
        self.q_proj = q_proj.detach().clone()
        self.head_weights = head_weights.detach().clone()

    def indexer_inputs(self, q, k):
        """(q_idx, k_idx, w) for the kernel: (B*H, Tq, E, F), (B*H, Tk', E, F),
        (B*H, Tq, E); Tk' = pooled groups when compress_ratio > 1."""
        B, H, tq, D = q.shape
        G = self.cfg.group_size
        proj = self.q_proj.to(device=q.device, dtype=torch.float32)
        qf = q.to(torch.float32)
        kf = k.to(torch.float32).repeat_interleave(G, dim=1)  # (B, H, Tk, D)
        m = self.compress_ratio
        if m > 1:
            tk = kf.shape[2]
            pad = (-tk) % m
            if pad:
                kf = torch.cat([kf, kf[:, :, -1:].expand(B, H, pad, D)], dim=2)
            kf = kf.view(B, H, -1, m, D).mean(dim=3)
        q_idx = torch.einsum("bhtd,hedf->bhtef", qf, proj)
        k_idx = torch.einsum("bhtd,hedf->bhtef", kf, proj)
        E, F = self.n_indexer_heads, self.indexer_dim
        w = torch.softmax(self.head_weights.to(q.device, torch.float32), dim=-1)
        q_idx = q_idx.reshape(B * H, tq, E, F).contiguous()
        k_idx = k_idx.reshape(B * H, -1, E, F).contiguous()
        w = w.view(1, 1, E).expand(B * H, tq, E).contiguous()
        return q_idx, k_idx, w

    def select_lists(self, q, k, offset: int) -> torch.Tensor:
        """Token lists (B, H, Tq, W) ascending, -1 padded."""
        B, H, tq, _ = q.shape
        t_k = k.shape[2]
        q_idx, k_idx, w = self.indexer_inputs(q, k)
        m = self.compress_ratio
        if m > 1:
            n_keep = max(1, self.cfg.topk_tokens // m)
            _, grp = indexer_topk(q_idx, k_idx, w, n_keep, causal=True, offset=offset,
                                  causal_unit=m)
            toks = grp.to(torch.int64).unsqueeze(-1) * m + torch.arange(m, device=q.device)
            toks = torch.where(grp.unsqueeze(-1) >= 0, toks, torch.full_like(toks, -1))
            sel = toks.view(B, H, tq, -1)
        else:
            n_keep = min(self.cfg.topk_tokens, t_k)
            _, idx = indexer_topk(q_idx, k_idx, w, n_keep, causal=self.indexer_causal,
                                  offset=offset)
            sel = idx.to(torch.int64).view(B, H, tq, -1)
        pos = torch.arange(tq, device=q.device).view(1, 1, -1, 1) + offset
        sink = torch.arange(self.cfg.sink_size, device=q.device).view(1, 1, 1, -1)
        win = pos - torch.arange(self.cfg.window_size, device=q.device).view(1, 1, 1, -1)
        extra = torch.cat([sink.expand(B, H, tq, -1), win.expand(B, H, tq, -1)], dim=-1)
        allv = torch.cat([sel, extra], dim=-1)
        allv = torch.where((allv >= 0) & (allv < t_k), allv, torch.full_like(allv, -1))
        # effective_mask's fallback (selection.py:100-107): a row with no
        # causal entry reads the query's own token (clamped to the last key)
        own = pos.clamp(max=t_k - 1).expand(B, H, tq, 1)
        empty = ~((allv >= 0) & (allv <= pos)).any(-1, keepdim=True)
        allv = torch.cat([allv, torch.where(empty, own, torch.full_like(own, -1))], dim=-1)
        allv = allv.sort(dim=-1).values
        dup = torch.zeros_like(allv, dtype=torch.bool)
        dup[..., 1:] = allv[..., 1:] == allv[..., :-1]
        allv = torch.where(dup, torch.full_like(allv, -1), allv)
        return allv.sort(dim=-1, descending=True).values.to(torch.int32)

    def attend(self, q, state, offset: int = 0):
        k, v = state["k"], state["v"]
        ids = self.select_lists(q, k, offset)
        out = sparse_attention(q, k, v, ids, unit=1, causal=True, offset=offset,
                               out_dtype=q.dtype)
        reads = _reads_per_query(ids, 1, offset, k.shape[-2])
        self._extra = {"reads_per_query": reads, "tokens_per_query": reads}
        return out

    def read_budget(self, seq_len, batch=1):
        c = self.cfg
        return float(min(seq_len, c.topk_blocks * c.block_size + c.window_size))

    def flops(self, seq_len, batch=1):
        m = max(1, self.compress_ratio)
        sel = 2 * batch * self.cfg.n_heads * seq_len * (seq_len // m) * self.indexer_dim
        return super().flops(seq_len, batch) + int(sel)


class HipMoBA(HipAttention):
    """MoBAAttention (selection.py:610-640) on the GPU: every query routes to
    the ``topk_blocks`` visible key blocks of highest gate q . mean(K block)
    (``gate_select_hip``, fp64 gates, ties to the lowest block) plus its own
    block, then the executor reads those blocks intersected with causality
    (the effective mask of selection.py:86-108)."""

    reference = "moba"

    def prepare_state(self, batch, device, dtype):
        state = super().prepare_state(batch, device, dtype)
        state["block_means"] = None
        return state

    def push_kv(self, state, k, v):
        """Append the keys and re-pool only the blocks they touched: the
        state keeps the fp64 block means the gate reads (``block_means_hip``),
        where the reference pools every key at every call
        (selection.py:620-624)."""
        start = state["k"].shape[-2]
        state = super().push_kv(state, k, v)
        kk = state["k"]
        B, Hkv, t, D = kk.shape
        if t == 0:
            return state
        bs = self.cfg.block_size
        nkb = (t + bs - 1) // bs
        first = start // bs
        old = state.get("block_means")
        if old is not None and old.shape == (B, Hkv, nkb, D) and old.device == kk.device:
            means = old  # the new keys stayed in the known blocks: refresh in place
        else:
            means = torch.empty(B, Hkv, nkb, D, dtype=torch.float64, device=kk.device)
            if old is not None and first > 0:
                means[:, :, :first].copy_(old[:, :, :first])
        block_means_hip(kk, block=bs, out=means, first_block=first, n_blocks=nkb - first)
        state["block_means"] = means
        return state

    def attend(self, q, state, offset: int = 0):
        k, v = state["k"], state["v"]
        bs = self.cfg.block_size
        ids, counts = gate_select_hip(q, k, block=bs, topk=self.cfg.topk_blocks, offset=offset,
                                      kbar=state.get("block_means"))
        out = sparse_attention(q, k, v, ids, unit=bs, counts=counts, causal=True, offset=offset,
                               out_dtype=q.dtype)
        self._extra = {"blocks_per_query": float(counts.to(torch.float64).mean()),
                       "reads_per_query": _reads_per_query(ids, bs, offset, k.shape[-2])}
        return out

    def read_budget(self, seq_len, batch=1):
        c = self.cfg
        return float(min(seq_len, c.topk_blocks * c.block_size + c.window_size))

    def flops(self, seq_len, batch=1):
        n_kb = (seq_len + self.cfg.block_size - 1) // self.cfg.block_size
        sel = 2 * batch * self.cfg.n_heads * seq_len * n_kb * self.cfg.head_dim
        return super().flops(seq_len, batch) + int(sel)


class HipXAttention(HipAttention):
    """XAttention (selection.py:500-595) on the GPU: per query block, the
    strided antidiagonal scores of every visible key block, softmax block
    masses and the minimal prefix of blocks reaching ``cfg.threshold``
    (``xattn_select_hip``), then the executor reads those blocks intersected
    with causality.

    extras: ``xattn_block`` (default 8), ``antidiagonal_stride`` (default
    ``cfg.stride``), ``select_mode`` ("threshold", default, or "topk" with
    ``cfg.topk_blocks``, or "top_ratio" with ``top_ratio``, default 0.02),
    ``threshold_per_head``.  The reference's "top_ratio" mode compares the
    cumulative probability mass (at most 1) against a block count of at
    least 1 (selection.py:583-585 with :598-606), which is reached only when
    every visible block is in: it reads every visible block, as here.
    64-token blocks over a whole bf16 prefill (offset 0,
    head_dim 128) run the MFMA prefill kernel; otherwise every query row reads
    its block's list through ``sparse_attention``."""

    reference = "xattention"

    def __init__(self, cfg=None, **kw):
        super().__init__(cfg, **kw)
        ex = self.cfg.extras
        self.block = int(ex.get("xattn_block", 8))
        self.r = int(ex.get("antidiagonal_stride", self.cfg.stride))
        self.select_mode = ex.get("select_mode", "threshold")
        if self.select_mode not in ("threshold", "topk", "top_ratio"):
            raise ValueError(f"hip_xattention: select_mode {self.select_mode!r} not supported "
                             "(threshold, topk or top_ratio)")

    def attend(self, q, state, offset: int = 0):
        k, v = state["k"], state["v"]
        blk = self.block
        if self.select_mode == "topk":
            ids, counts = xattn_select_hip(q, k, block=blk, stride=self.r, offset=offset,
                                           topk=self.cfg.topk_blocks)
        elif self.select_mode == "top_ratio":
            ids, counts = xattn_select_hip(q, k, block=blk, stride=self.r, offset=offset,
                                           top_ratio=float(self.cfg.extras.get("top_ratio", 0.02)))
        else:
            th = self.cfg.extras.get("threshold_per_head", self.cfg.threshold)
            ids, counts = xattn_select_hip(q, k, block=blk, stride=self.r, threshold=th,
                                           offset=offset)
        Tq, T = q.shape[2], k.shape[2]
        if (blk == 64 and offset == 0 and Tq == T and q.shape[3] == 128
                and q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16):
            out = block_sparse_prefill(q, k, v, ids, counts, block_size=64, out_dtype=q.dtype)
            rows = ids.repeat_interleave(blk, dim=2)[:, :, :Tq]
        else:
            rows = ids.repeat_interleave(blk, dim=2)[:, :, :Tq].contiguous()
            rcounts = counts.repeat_interleave(blk, dim=2)[:, :, :Tq].contiguous()
            out = sparse_attention(q, k, v, rows, unit=blk, counts=rcounts, causal=True,
                                   offset=offset, out_dtype=q.dtype)
        self._extra = {"blocks_per_query": float(counts.to(torch.float64).mean()),
                       "reads_per_query": _reads_per_query(rows, blk, offset, T)}
        return out

    def read_budget(self, seq_len, batch=1):
        return float(seq_len)  # data dependent: up to the whole causal prefix

    def flops(self, seq_len, batch=1):
        blk, c = self.block, self.cfg
        n_b = (seq_len + blk - 1) // blk
        sel = 2 * 2 * batch * c.n_heads * n_b * n_b * blk * blk / self.r * c.head_dim / blk
        return super().flops(seq_len, batch) + int(sel)


SUPPORTED = {
    "quest": HipQuest,
    "dsa": HipDSA,
    "moba": HipMoBA,
    "xattention": HipXAttention,
    "sliding_window": HipSlidingWindow,
    "streaming_sink": HipStreamingSink,
}
