"""GPU parity of XAttention's block selection (selection.py:500-595) and the
``hip_xattention`` variant: block lists bit-exact against the CPU oracle
(oracle.xattn_select, pinned in tests/test_oracle.py), attention within 1e-5
(fp32 in and out) of the oracle's attention over those lists, and dense
attention at an unrestricted budget."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.core import AttnConfig
from linattn_amd.kernels.routing import xattn_select_hip
from linattn_amd.registry import build

pytestmark = pytest.mark.gpu


def inputs(b, hq, hkv, tq, t, d, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, tq, d, generator=g)
    k = torch.randn(b, hkv, t, d, generator=g)
    v = torch.randn(b, hkv, t, d, generator=g)
    rows = torch.randperm(t, generator=g)[: max(1, t // 20)]
    k[:, :, rows] *= 4.0  # a few dominant keys: peaked rows
    return q.to(dtype), k.to(dtype), v.to(dtype)


def check_lists(ids, counts, ref_ids, ref_counts):
    assert ids.shape == ref_ids.shape
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    assert np.array_equal(counts.cpu().numpy(), ref_counts)


@pytest.mark.parametrize("dtype,b,hq,hkv,t,d,block,stride,threshold", [
    (torch.bfloat16, 2, 4, 2, 300, 128, 8, 8, 0.9),
    (torch.float32, 1, 2, 1, 203, 64, 16, 4, [0.5, 0.95]),
    (torch.bfloat16, 1, 2, 2, 700, 128, 64, 8, 0.9),
    (torch.float32, 1, 2, 1, 61, 32, 4, 2, 0.3),
    (torch.bfloat16, 1, 2, 1, 2500, 64, 8, 8, 0.95),
    (torch.float32, 1, 1, 1, 100, 16, 8, 8, 1.5),
])
def test_xattn_select_bit_exact(dev, dtype, b, hq, hkv, t, d, block, stride, threshold):
    q, k, _ = inputs(b, hq, hkv, t, t, d, seed=31, dtype=dtype)
    ids, counts = xattn_select_hip(q.to(dev), k.to(dev), block=block, stride=stride,
                                   threshold=threshold)
    ref_ids, ref_counts = oracle.xattn_select(q, k, block=block, stride=stride,
                                              threshold=threshold)
    check_lists(ids, counts, ref_ids, ref_counts)


@pytest.mark.parametrize("t,tq,block,topk", [(300, 300, 8, 5), (8300, 64, 8, 40),
                                             (8300, 64, 8, None), (32768, 16, 8, None)])
def test_xattn_select_topk_and_offset(dev, t, tq, block, topk):
    """Top-k mode, and a chunk of queries at the end of a long cache
    (offset = T - Tq; more than 1024 key blocks per row; at T = 32768 the
    4096 key blocks take 68 KiB of LDS per row, above the default 64 KiB)."""
    q, k, _ = inputs(1, 2, 1, tq, t, 64, seed=32, dtype=torch.bfloat16)
    kw = dict(block=block, stride=8, offset=t - tq)
    if topk is not None:
        kw["topk"] = topk
    ids, counts = xattn_select_hip(q.to(dev), k.to(dev), **kw)
    ref_ids, ref_counts = oracle.xattn_select(q, k, **kw)
    check_lists(ids, counts, ref_ids, ref_counts)


@pytest.mark.parametrize("t,tq,block,threshold,topk", [
    (1000, 1000, 8, [0.0, 1.5], None),   # 125 key blocks: 4 per lane; the top block alone / every block
    (1000, 1000, 8, 0.8, 7),             # top-k, 4 per lane
    (4000, 128, 8, 0.9, 30),             # top-k at an offset, 500 blocks: 16 per lane
    (8000, 64, 8, [0.9, 0.6], None),     # threshold at an offset, 1000 blocks
    (500, 500, 4, 0.95, None),           # block = stride = 4
    (64 * 8, 64 * 8, 8, 0.7, None),      # exactly 64 key blocks: one per lane
])
def test_xattn_select_one_wave_rows(dev, t, tq, block, threshold, topk):
    """The one-wave-per-row selection (slots on the matrix cores, at most
    1024 key blocks) against the oracle, every branch of the threshold rule
    and the top-k rule at 1, 4 and 16 blocks per lane."""
    q, k, _ = inputs(1, 2, 1, tq, t, 64, seed=33, dtype=torch.bfloat16)
    kw = dict(block=block, stride=block, offset=t - tq, threshold=threshold)
    if topk is not None:
        kw["topk"] = topk
    ids, counts = xattn_select_hip(q.to(dev), k.to(dev), **kw)
    ref_ids, ref_counts = oracle.xattn_select(q, k, **kw)
    check_lists(ids, counts, ref_ids, ref_counts)


@pytest.mark.parametrize("t,tq,block,topk", [
    (8192 - 100, 8192 - 100, 8, None),  # 1012 query blocks: 16 chunks of 64, the last partial
    (1000 * 8, 300 * 8, 8, 20),         # top-k, queries at an offset: 5 chunks
    (1200 * 8, 130 * 8, 8, None),       # 1200 key blocks: the block-per-row selection per chunk
])
def test_xattn_select_chunked_workspace(dev, t, tq, block, topk):
    """A workspace bounded to one chunk of 64 query blocks: the slots are
    scored and selected chunk by chunk, with the lists of the one-pass call
    (and of the oracle on a sample of rows)."""
    q, k, _ = inputs(1, 2, 1, tq, t, 64, seed=35, dtype=torch.bfloat16)
    kw = dict(block=block, stride=block, offset=t - tq, threshold=[0.9, 0.7])
    if topk is not None:
        kw["topk"] = topk
    n_kb = -(-t // block)
    one_chunk = 2 * 64 * n_kb * 2 * 8  # B * Hq * 64 query blocks * n_kb * 2 slots * 8 B
    ids, counts = xattn_select_hip(q.to(dev), k.to(dev), max_workspace_bytes=one_chunk, **kw)
    ids1, counts1 = xattn_select_hip(q.to(dev), k.to(dev), **kw)
    assert torch.equal(ids, ids1) and torch.equal(counts, counts1)
    r0 = max(0, (tq // block // 64 - 1) * 64 - 5)
    rows = slice(r0, r0 + 10)  # straddles a chunk boundary
    ref_ids, ref_counts = oracle.xattn_select(q[:, :, rows.start * block:rows.stop * block], k,
                                              block=block, stride=block,
                                              offset=t - tq + rows.start * block,
                                              threshold=kw["threshold"], topk=topk)
    check_lists(ids[:, :, rows], counts[:, :, rows], ref_ids, ref_counts)


def test_xattn_slots_summation_order(dev):
    """Slot entries are fp64 sums over d in increasing order (the matrix-core
    scorer for stride == block relies on the in-order fp64 accumulation).
    With q = 1 every entry is its key row's sum; each key row shuffles +-2^60
    pairs with small integers, so that sum depends on the order (a small value
    added to a +-2^60 partial sum is absorbed) and so do the slots, masses and
    lists, which equal the oracle's."""
    r = np.random.default_rng(9)
    T, D = 256, 64
    big = np.ldexp(1.0, 60)
    rows = [r.permutation(np.concatenate([[big, -big, big, -big], r.integers(1, 60, size=D - 4)]))
            for _ in range(T)]
    k = torch.tensor(np.array(rows)).to(torch.bfloat16).view(1, 1, T, D)
    q = torch.ones(1, 1, T, D, dtype=torch.bfloat16)
    seq = []
    for row in k[0, 0].double().numpy():
        acc = 0.0
        for x in row:
            acc = acc + x
        seq.append(acc)
    pair = [float(np.sum(row)) for row in k[0, 0].double().numpy()]
    assert sum(a != b for a, b in zip(seq, pair)) > T // 2  # the order matters
    for thr in (0.5, 0.9):
        ids, counts = xattn_select_hip(q.to(dev), k.to(dev), block=8, stride=8, threshold=thr)
        ref_ids, ref_counts = oracle.xattn_select(q, k, block=8, stride=8, threshold=thr)
        check_lists(ids, counts, ref_ids, ref_counts)


def cfg(**kw):
    base = dict(n_heads=4, n_kv_heads=2, head_dim=64, block_size=16, topk_blocks=4)
    base.update(kw)
    return AttnConfig(**base)


def xattn_oracle(q, k, v, c, chunk, **sel):
    T = q.shape[2]
    blk = c.extras.get("xattn_block", 8)
    outs = []
    for s in range(0, T, chunk):
        e = min(T, s + chunk)
        ids, _ = oracle.xattn_select(q[:, :, s:e], k[:, :, :e], block=blk,
                                     stride=c.extras.get("antidiagonal_stride", c.stride),
                                     offset=s, **sel)
        rows = np.repeat(ids, blk, axis=2)[:, :, :e - s]
        outs.append(oracle.attend_lists(q[:, :, s:e], k[:, :, :e], v[:, :, :e], rows, unit=blk,
                                        causal=True, offset=s))
    return np.concatenate(outs, axis=2)


@pytest.mark.parametrize("chunk", [160, 48])
def test_hip_xattention_matches_oracle(dev, chunk):
    c = cfg(threshold=0.8)
    q, k, v = inputs(2, 4, 2, 160, 160, 64, seed=33)
    out, _, stats = build("hip_xattention", c).forward(q.to(dev), k.to(dev), v.to(dev),
                                                       chunk=chunk, collect_stats=True)
    ref = xattn_oracle(q, k, v, c, chunk, threshold=0.8)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5
    assert all(s["blocks_per_query"] >= 1 for s in stats)


def test_hip_xattention_prefill_kernel_path(dev):
    """64-token blocks over a bf16 prefill take the MFMA prefill kernel."""
    c = cfg(n_heads=4, n_kv_heads=2, head_dim=128, threshold=0.9,
            extras={"xattn_block": 64, "antidiagonal_stride": 8})
    q, k, v = inputs(1, 4, 2, 320, 320, 128, seed=34, dtype=torch.bfloat16)
    out, _ = build("hip_xattention", c).forward(q.to(dev), k.to(dev), v.to(dev), chunk=320)
    ref = xattn_oracle(q, k, v, c, 320, threshold=0.9)
    # bf16 output: the 2e-3 gate plus the output's own rounding (2^-9 relative)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3 + 2 ** -9 * np.abs(ref).max()


@pytest.mark.parametrize("ratio", [0.02, 0.5])
def test_hip_xattention_top_ratio(dev, ratio):
    """select_mode "top_ratio" (selection.py:583-585): lists equal the
    oracle's (every visible block) for a prefill and an offset chunk, and the
    variant's output equals the oracle's chunked forward and dense causal
    attention."""
    q, k, v = inputs(1, 4, 2, 160, 160, 64, seed=36)
    for s0 in (0, 101):
        ids, counts = xattn_select_hip(q[:, :, s0:].to(dev), k.to(dev), block=8, stride=8,
                                       offset=s0, top_ratio=ratio)
        ref_ids, ref_counts = oracle.xattn_select(q[:, :, s0:], k, block=8, stride=8, offset=s0,
                                                  top_ratio=ratio)
        check_lists(ids, counts, ref_ids, ref_counts)
    c = cfg(extras={"select_mode": "top_ratio", "top_ratio": ratio})
    out, _ = build("hip_xattention", c).forward(q.to(dev), k.to(dev), v.to(dev), chunk=48)
    ref = xattn_oracle(q, k, v, c, 48, top_ratio=ratio)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5
    dense = oracle.dense_attention(q, k, v)
    assert np.abs(out.cpu().double().numpy() - dense).max() < 1e-5


def test_hip_xattention_full_budget_recovers_dense(dev):
    """test_budgets.py:64-81 for XAttention (select_mode topk over every
    block, and a threshold above 1), float64 in and out."""
    q, k, v = inputs(1, 4, 2, 160, 160, 64, seed=35)
    dense = oracle.dense_attention(q, k, v)
    for c in (cfg(topk_blocks=160 // 8 + 2, extras={"select_mode": "topk"}),
              cfg(threshold=1.5)):
        out, _ = build("hip_xattention", c).forward(q.double().to(dev), k.double().to(dev),
                                                    v.double().to(dev), chunk=160)
        assert np.abs(out.cpu().numpy() - dense).max() < 1e-5
