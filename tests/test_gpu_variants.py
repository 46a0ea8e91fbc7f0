"""The ``hip_*`` variants behind the reference's variant API, against the CPU
oracle (the backend-parity pattern of the reference's tests/test_mlx.py:40-57:
same outputs and the same reads_per_query, to within 1)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.core import AttnConfig
from linattn_amd.registry import build

pytestmark = pytest.mark.gpu


def inputs(b, hq, hkv, t, d, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, hq, t, d, generator=g), torch.randn(b, hkv, t, d, generator=g),
            torch.randn(b, hkv, t, d, generator=g))


def cfg(**kw):
    base = dict(n_heads=4, n_kv_heads=2, head_dim=64, block_size=16, window_size=32,
                topk_blocks=3, topk_tokens=48, compress_ratio=8, sink_size=2)
    base.update(kw)
    return AttnConfig(**base)


def quest_oracle(q, k, v, c, chunk, union):
    """QuestAttention.forward semantics chunk by chunk: metadata over every key
    pushed so far, selection at the chunk's offset, causal attention."""
    T = q.shape[2]
    ps = c.extras.get("page_size", c.block_size)
    outs, reads = [], []
    for s in range(0, T, chunk):
        e = min(T, s + chunk)
        kk, vv = k[:, :, :e], v[:, :, :e]
        mn, mx = oracle.page_bounds(kk, ps)
        ids = oracle.quest_select(q[:, :, s:e], mn, mx, page_size=ps, topk=c.topk_blocks,
                                  offset=s, gqa_union=union)
        outs.append(oracle.attend_lists(q[:, :, s:e], kk, vv, ids, unit=ps, causal=True,
                                        offset=s))
        lim = np.minimum(np.arange(e - s) + s + 1, e)[None, None, :, None]
        n = np.clip(lim - ids.astype(np.int64) * ps, 0, ps) * (ids >= 0)
        reads.append(float(n.sum(-1).mean()))
    return np.concatenate(outs, axis=2), reads


@pytest.mark.parametrize("union", [True, False])
@pytest.mark.parametrize("chunk", [192, 64])
def test_hip_quest_matches_oracle(dev, union, chunk):
    c = cfg(extras={"gqa_union": union})
    q, k, v = inputs(2, 4, 2, 192, 64, seed=1)
    var = build("hip_quest", c)
    out, _, stats = var.forward(q.to(dev), k.to(dev), v.to(dev), chunk=chunk, collect_stats=True)
    ref, reads = quest_oracle(q, k, v, c, chunk, union)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5
    for s, r in zip(stats, reads):
        assert abs(s["reads_per_query"] - r) < 1.0


def test_hip_quest_full_budget_recovers_dense(dev):
    """The parity gate (test_budgets.py:64-81), float64 in and out."""
    q, k, v = inputs(1, 4, 2, 192, 64, seed=2)
    c = cfg(topk_blocks=192 // 16 + 2)
    out, _ = build("hip_quest", c).forward(q.double().to(dev), k.double().to(dev),
                                           v.double().to(dev), chunk=192)
    assert out.dtype == torch.float64
    ref = oracle.dense_attention(q, k, v)
    assert np.abs(out.cpu().numpy() - ref).max() < 1e-5


def test_hip_quest_decode_equals_prefill(dev):
    """Token-by-token decode with state equals one prefill (the cache contract
    of test_reference.py:64-77): visible pages before the own page are full in
    both modes and the own page is always read."""
    q, k, v = inputs(1, 4, 2, 80, 64, seed=3)
    var = build("hip_quest", cfg())
    pre, _ = var.forward(q.to(dev), k.to(dev), v.to(dev), chunk=80)
    state, pieces = None, []
    for i in range(80):
        o, state = var.forward(q[:, :, i:i + 1].to(dev), k[:, :, i:i + 1].to(dev),
                               v[:, :, i:i + 1].to(dev), state=state)
        pieces.append(o)
    dec = torch.cat(pieces, dim=2)
    assert state["pos"] == 80
    assert (pre - dec).abs().max().item() < 1e-5


@pytest.mark.parametrize("name", ["hip_sliding_window", "hip_streaming_sink"])
def test_hip_window_matches_oracle(dev, name):
    q, k, v = inputs(2, 4, 2, 150, 64, seed=4)
    c = cfg()
    out, _, stats = build(name, c).forward(q.to(dev), k.to(dev), v.to(dev), chunk=64,
                                           collect_stats=True)
    mask = oracle.window_mask(150, 150, 0, c.window_size, c.sink_size)
    ref = oracle.dense_attention(q, k, v, mask=mask)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5
    last = oracle.window_mask(150 - 128, 150, 128, c.window_size, c.sink_size)
    assert abs(stats[-1]["reads_per_query"] - last.sum(-1).mean()) < 1.0


@pytest.mark.parametrize("ratio", [1, 8])
def test_hip_dsa_matches_oracle(dev, ratio):
    """Indexer top-k (per attention head, the reference's projections) plus sink
    and window, then causal attention over the kept tokens."""
    c = cfg(compress_ratio=ratio, extras={"indexer_heads": 4, "indexer_dim": 16})
    q, k, v = inputs(1, 4, 2, 128, 64, seed=5)
    var = build("hip_dsa", c)
    out, _ = var.forward(q.to(dev), k.to(dev), v.to(dev), chunk=128)
    q_idx, k_idx, w = var.indexer_inputs(q.to(dev), k.to(dev))
    B, H, T = 1, 4, 128
    if ratio > 1:
        n_keep = max(1, c.topk_tokens // ratio)
        _, grp = oracle.indexer_topk(q_idx.cpu(), k_idx.cpu(), w.cpu(), n_keep, causal=True,
                                     causal_unit=ratio)
        sel = [[set() for _ in range(T)] for _ in range(H)]
        for h in range(H):
            for t in range(T):
                for gi in grp[h, t]:
                    if gi >= 0:
                        sel[h][t].update(range(gi * ratio, gi * ratio + ratio))
    else:
        _, idx = oracle.indexer_topk(q_idx.cpu(), k_idx.cpu(), w.cpu(), min(c.topk_tokens, T))
        sel = [[set(int(x) for x in idx[h, t] if x >= 0) for t in range(T)] for h in range(H)]
    mask = np.zeros((1, H, T, T), dtype=bool)
    for h in range(H):
        for t in range(T):
            s = sel[h][t] | set(range(c.sink_size)) | set(range(max(0, t - c.window_size + 1), t + 1))
            for j in s:
                if j <= t:
                    mask[0, h, t, j] = True
    ref = oracle.dense_attention(q, k, v, mask=mask)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5


def test_hip_dsa_empty_rows_read_own_token(dev):
    """No sink and no window: early queries whose indexer top-k holds only
    future keys fall back to their own token (effective_mask,
    selection.py:100-107), and every output equals the oracle's attention
    over oracle.effective_mask of the indexer selection."""
    c = cfg(compress_ratio=1, window_size=0, sink_size=0, topk_tokens=4,
            extras={"indexer_heads": 4, "indexer_dim": 16})
    q, k, v = inputs(1, 4, 2, 96, 64, seed=15)
    var = build("hip_dsa", c)
    out, _, stats = var.forward(q.to(dev), k.to(dev), v.to(dev), chunk=96, collect_stats=True)
    q_idx, k_idx, w = var.indexer_inputs(q.to(dev), k.to(dev))
    H, T = 4, 96
    _, idx = oracle.indexer_topk(q_idx.cpu(), k_idx.cpu(), w.cpu(), c.topk_tokens)
    sel = np.zeros((1, H, T, T), dtype=bool)
    for h in range(H):
        for t in range(T):
            sel[0, h, t, [x for x in idx[h, t] if x >= 0]] = True
    mask = oracle.effective_mask(sel, offset=0)
    empty = ~(sel & oracle.causal_mask(T, T, 0)).any(-1)
    assert empty.sum() > 0  # the fallback is exercised
    ref = oracle.dense_attention(q, k, v, mask=mask)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5
    assert abs(stats[0]["reads_per_query"] - mask.sum(-1).mean()) < 1e-9


# ---------------------------------------------------------------- MoBA ----
def moba_oracle(q, k, v, c, chunk):
    """MoBAAttention.forward (selection.py:610-640) chunk by chunk: routing
    over every key pushed so far at the chunk's offset, causal attention."""
    T = q.shape[2]
    outs = []
    for s in range(0, T, chunk):
        e = min(T, s + chunk)
        ids = oracle.gate_select(q[:, :, s:e], k[:, :, :e], block=c.block_size,
                                 topk=c.topk_blocks, offset=s)
        outs.append(oracle.attend_lists(q[:, :, s:e], k[:, :, :e], v[:, :, :e], ids,
                                        unit=c.block_size, causal=True, offset=s))
    return np.concatenate(outs, axis=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,T", [(4, 2, 150), (8, 8, 97)])
def test_gate_select_bit_exact(dev, dtype, hq, hkv, T):
    """Routing lists equal the oracle's bit for bit, for a prefill (every
    query, T not a multiple of the block) and for one decode query."""
    from linattn_amd.kernels.routing import gate_select_hip

    q, k, _ = inputs(2, hq, hkv, T, 64, seed=6)
    q, k = q.to(dtype), k.to(dtype)
    ids, counts = gate_select_hip(q.to(dev), k.to(dev), block=16, topk=3, offset=0)
    ref = oracle.gate_select(q, k, block=16, topk=3, offset=0)
    assert np.array_equal(ids.cpu().numpy(), ref)
    assert np.array_equal(counts.cpu().numpy(), (ref >= 0).sum(-1))
    ids1, _ = gate_select_hip(q[:, :, -1:].to(dev), k.to(dev), block=16, topk=4, offset=T - 1)
    ref1 = oracle.gate_select(q[:, :, -1:], k, block=16, topk=4, offset=T - 1)
    assert np.array_equal(ids1.cpu().numpy(), ref1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_means_cache(dev, dtype):
    """Block means kept on append: a full pooling equals the oracle's bit for
    bit (tail block padded with the last row); re-pooling only the block of
    each appended key, one token at a time (and ragged, per-sequence
    positions and lengths), leaves the cache equal to a fresh pooling; the
    routing reads the cache instead of k and returns the same lists."""
    from linattn_amd.kernels.routing import block_means_hip, gate_select_hip

    B, Hq, Hkv, T, D, bs = 2, 8, 2, 150, 64, 16
    q, k, _ = inputs(B, Hq, Hkv, T, D, seed=9)
    q, k = q.to(dtype).to(dev), k.to(dtype).to(dev)
    full = block_means_hip(k, block=bs)
    assert np.array_equal(full.cpu().numpy(), oracle.block_means(k.cpu(), bs))
    # decode: keys appended one at a time from 120 rows, only the new key's block re-pooled
    t0 = 120
    means = block_means_hip(k[:, :, :t0], block=bs)
    for t in range(t0 + 1, T + 1):
        nkb = (t + bs - 1) // bs
        if means.shape[2] != nkb:
            grown = torch.zeros(B, Hkv, nkb, D, dtype=torch.float64, device=dev)
            grown[:, :, :means.shape[2]] = means
            means = grown
        pos = torch.full((B,), t - 1, dtype=torch.int32, device=dev)
        block_means_hip(k[:, :, :t], block=bs, out=means, positions=pos)
    assert np.array_equal(means.cpu().numpy(), full.cpu().numpy())
    # ragged: sequence b holds lengths[b] rows; its last block re-pooled alone
    lens = torch.tensor([T, 97], dtype=torch.int32, device=dev)
    rag = full.clone()
    block_means_hip(k, block=bs, out=rag, positions=lens - 1, lengths=lens)
    ref1 = oracle.block_means(k[1:, :, :97].cpu(), bs)
    assert np.array_equal(rag[1, :, (97 - 1) // bs].cpu().numpy(), ref1[0, :, -1])
    assert np.array_equal(rag[0].cpu().numpy(), full[0].cpu().numpy())
    # the gate reads the cache: same lists as pooling k, and as the oracle
    for off, qq in ((0, q), (T - 1, q[:, :, -1:])):
        ids, counts = gate_select_hip(qq, k, block=bs, topk=3, offset=off, kbar=full)
        ids0, counts0 = gate_select_hip(qq, k, block=bs, topk=3, offset=off)
        assert torch.equal(ids, ids0) and torch.equal(counts, counts0)
        assert np.array_equal(ids.cpu().numpy(),
                              oracle.gate_select(qq.cpu(), k.cpu(), block=bs, topk=3, offset=off))


def test_hip_moba_decode_keeps_block_means(dev):
    """hip_moba's state carries the block means across decode steps (refreshed
    for the touched blocks only); after a prefill and 40 single-token steps
    they equal a fresh pooling of the cache, and each step's output matches
    the oracle's."""
    from linattn_amd.kernels.routing import block_means_hip

    c = cfg()
    q, k, v = inputs(1, 4, 2, 160, 64, seed=10)
    var = build("hip_moba", c)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    _, state = var.forward(qd[:, :, :120], kd[:, :, :120], vd[:, :, :120], chunk=120)
    for t in range(120, 160):
        out, state = var.forward(qd[:, :, t:t + 1], kd[:, :, t:t + 1], vd[:, :, t:t + 1],
                                 state=state, chunk=1)
        ids = oracle.gate_select(q[:, :, t:t + 1], k[:, :, :t + 1], block=c.block_size,
                                 topk=c.topk_blocks, offset=t)
        ref = oracle.attend_lists(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1], ids,
                                  unit=c.block_size, causal=True, offset=t)
        assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5
    assert torch.equal(state["block_means"], block_means_hip(state["k"], block=c.block_size))


@pytest.mark.parametrize("chunk", [160, 48])
def test_hip_moba_matches_oracle(dev, chunk):
    c = cfg()
    q, k, v = inputs(2, 4, 2, 160, 64, seed=7)
    out, _, stats = build("hip_moba", c).forward(q.to(dev), k.to(dev), v.to(dev), chunk=chunk,
                                                 collect_stats=True)
    ref = moba_oracle(q, k, v, c, chunk)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5
    assert all(s["blocks_per_query"] <= c.topk_blocks + 1 for s in stats)


def test_hip_moba_full_budget_recovers_dense(dev):
    """test_budgets.py:64-81 for MoBA, float64 in and out."""
    q, k, v = inputs(1, 4, 2, 160, 64, seed=8)
    c = cfg(topk_blocks=160 // 16 + 2)
    out, _ = build("hip_moba", c).forward(q.double().to(dev), k.double().to(dev),
                                          v.double().to(dev), chunk=160)
    assert np.abs(out.cpu().numpy() - oracle.dense_attention(q, k, v)).max() < 1e-5
