"""Planted-structure inputs and attention-mass recall, as the reference's
selection-quality tests use them.

``structured_inputs`` restates linattn.harness.structured_inputs
(harness.py:51-86): N(0,1) q/k/v from one CPU generator, then per (b, KV
head) ``n_spikes`` runs of ``spike_width`` keys scaled by 3 and a linear
recency ramp 0.6..1.4 over the keys.  ``attention_mass`` / ``mass_recall``
restate metrics.py:67-103 and ``block_recall`` the helper of
tests/test_selection.py:158-165.  Test infrastructure only.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch


def structured_inputs(batch: int, heads: int, seq: int, dim: int, *, n_spikes: int = 4,
                      spike_width: int = 32, seed: int = 0, kv_heads: Optional[int] = None,
                      dtype: torch.dtype = torch.float32):
    g = torch.Generator(device="cpu").manual_seed(seed)
    kv_heads = kv_heads or heads
    q = torch.randn(batch, heads, seq, dim, generator=g, dtype=torch.float32)
    k = torch.randn(batch, kv_heads, seq, dim, generator=g, dtype=torch.float32)
    v = torch.randn(batch, kv_heads, seq, dim, generator=g, dtype=torch.float32)
    for b in range(batch):
        for h in range(kv_heads):
            starts = torch.randint(0, max(1, seq - spike_width), (n_spikes,), generator=g)
            for s in starts:
                s = int(s)
                k[b, h, s:s + spike_width] *= 3.0
            k[b, h] *= torch.linspace(0.6, 1.4, seq).unsqueeze(-1)
    return q.to(dtype=dtype), k.to(dtype=dtype), v.to(dtype=dtype)


def attention_mass(q: torch.Tensor, k: torch.Tensor, block: int) -> torch.Tensor:
    """Causal dense attention weights (fp64, 1/sqrt(D), GQA by head groups)
    summed into (query block, key block) cells: (B, H, n_qb, n_kb)."""
    q, k = q.double(), k.double()
    B, H, T, D = q.shape
    G = H // k.shape[1]
    kk = k.repeat_interleave(G, dim=1)
    s = torch.matmul(q, kk.transpose(-1, -2).contiguous()) / D ** 0.5
    fut = torch.arange(T).view(1, -1) > torch.arange(T).view(-1, 1)
    w = torch.softmax(s.masked_fill(fut, float("-inf")), dim=-1)
    pad = (-T) % block
    if pad:
        w = torch.nn.functional.pad(w, (0, pad, 0, pad))
    n = w.shape[-1] // block
    return w.view(B, H, n, block, n, block).sum(dim=(3, 5))


def block_recall(tok_mask: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                 block: int) -> Tuple[float, float]:
    """Mean attention-mass recall of a (B, H, T, T) token mask reduced to
    blocks (a block is kept when any of its cells is), and the fraction of
    blocks kept."""
    mass = attention_mass(q, k, block)
    T = tok_mask.shape[-1]
    nb = T // block
    red = tok_mask[..., :nb * block, :nb * block].reshape(*tok_mask.shape[:-2], nb, block, nb, block)
    red = red.any(-3).any(-1)
    m = mass[..., :nb, :nb]
    recall = (m * red).sum(-1) / m.sum(-1).clamp_min(1e-12)
    return float(recall.mean()), float(red.float().mean())


def lists_to_mask(ids: torch.Tensor, unit: int, T: int, rows_per_block: int = 1) -> torch.Tensor:
    """(B, H, R, W) unit lists (-1 padded) to a causal (B, H, T, T) token mask;
    list row r covers queries [r * rows_per_block, (r+1) * rows_per_block)."""
    ids = ids.long().cpu()
    B, H, R, W = ids.shape
    unit_mask = torch.zeros(B, H, R, (T + unit - 1) // unit + 1, dtype=torch.bool)
    safe = torch.where(ids >= 0, ids, torch.full_like(ids, unit_mask.shape[-1] - 1))
    unit_mask.scatter_(-1, safe, True)
    unit_mask[..., -1] = False
    tok = unit_mask[..., :-1].repeat_interleave(unit, dim=-1)[..., :T]
    tok = tok.repeat_interleave(rows_per_block, dim=2)[:, :, :T]
    causal = torch.arange(T).view(-1, 1) >= torch.arange(T).view(1, -1)
    return tok & causal
