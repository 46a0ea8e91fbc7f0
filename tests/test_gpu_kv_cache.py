"""GPU parity of the paged KV append with Quest page bounds, and of ragged
(per-sequence position) Quest decode.

The append must leave the pool and the page bounds exactly as a fresh
la_quest_page_bounds over the grown cache (and the oracle's page_bounds,
quest_pages.py:38-48) would; the fp8 pool must hold the codes and scales of
the kv/quant.py:76-93 codec bit for bit.  Ragged selection must equal the
per-sequence selection of QuestAttention.page_selection (selection.py:214-237)
at each sequence's own position."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.kernels.block_sparse import fp8_scale_pairs
from linattn_amd.kernels.kv_cache import paged_kv_append
from linattn_amd.kernels.paged_decode import quest_decode_step
from linattn_amd.kernels.quest_pages import page_update_hip, quest_select_hip

pytestmark = pytest.mark.gpu


def _pool(B, Hkv, D, pool_page, max_len, dtype, dev, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    pages = max_len // pool_page
    n_phys = B * pages + 3
    k_pool = torch.randn(n_phys, Hkv, pool_page, D, generator=g).to(dtype).to(dev)
    v_pool = torch.randn(n_phys, Hkv, pool_page, D, generator=g).to(dtype).to(dev)
    pt = torch.randperm(n_phys, generator=g)[:B * pages].view(B, pages).to(torch.int32).to(dev)
    return k_pool, v_pool, pt


def _expected_pool(pool, new, pt, positions, pool_page):
    exp = pool.clone()
    B, _, Tn, _ = new.shape
    for b in range(B):
        for i in range(Tn):
            t = int(positions[b]) + i
            exp[int(pt[b, t // pool_page]), :, t % pool_page, :] = new[b, :, i, :]
    return exp


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Tn,meta_page", [(1, 16), (70, 16), (70, 32), (5, 8)])
def test_append_matches_recompute(dev, dtype, Tn, meta_page):
    B, Hkv, D, pool_page, max_len = 3, 2, 128, 16, 320
    k_pool, v_pool, pt = _pool(B, Hkv, D, pool_page, max_len, dtype, dev, seed=Tn)
    positions = torch.tensor([37, 0, 200], dtype=torch.int32, device=dev)
    n_pages = max_len // meta_page
    mins, maxs = page_update_hip(k_pool, meta_page, n_pages, page_table=pt,
                                 pool_page_size=pool_page, kv_len=positions)
    g = torch.Generator(device="cpu").manual_seed(100 + Tn)
    k_new = torch.randn(B, Hkv, Tn, D, generator=g).to(dtype).to(dev)
    v_new = torch.randn(B, Hkv, Tn, D, generator=g).to(dtype).to(dev)
    k_exp = _expected_pool(k_pool, k_new, pt, positions.cpu(), pool_page)
    v_exp = _expected_pool(v_pool, v_new, pt, positions.cpu(), pool_page)
    paged_kv_append(k_new, v_new, k_pool, v_pool, pt, positions, page_min=mins, page_max=maxs,
                    page_size=meta_page)
    torch.cuda.synchronize()
    assert torch.equal(k_pool, k_exp) and torch.equal(v_pool, v_exp)
    rmin, rmax = page_update_hip(k_pool, meta_page, n_pages, page_table=pt,
                                 pool_page_size=pool_page, kv_len=positions + Tn)
    assert torch.equal(mins, rmin) and torch.equal(maxs, rmax)
    # the oracle over the logical sequence of b = 0
    L = int(positions[0]) + Tn
    seq = torch.stack([k_pool[int(pt[0, t // pool_page]), :, t % pool_page] for t in range(L)], 1)
    om, ox = oracle.page_bounds(seq.unsqueeze(0).cpu(), meta_page)
    npg = om.shape[2]
    assert np.array_equal(mins[0:1, :, :npg].cpu().double().numpy(), om)
    assert np.array_equal(maxs[0:1, :, :npg].cpu().double().numpy(), ox)


@pytest.mark.parametrize("pairs", [False, True])
def test_append_fp8_codec(dev, pairs):
    """fp8 pool append: codes and per-token scales equal the codec's, with the
    scales contiguous or interleaved (K, V) per token (fp8_scale_pairs)."""
    B, Hkv, D, pool_page, max_len, Tn = 2, 2, 128, 16, 128, 20
    g = torch.Generator(device="cpu").manual_seed(7)
    n_phys = B * (max_len // pool_page)
    pt = torch.randperm(n_phys, generator=g).view(B, -1).to(torch.int32).to(dev)
    k_pool = torch.zeros(n_phys, Hkv, pool_page, D, dtype=torch.float8_e4m3fn, device=dev)
    v_pool = torch.zeros_like(k_pool)
    if pairs:
        k_scale, v_scale = fp8_scale_pairs(n_phys, Hkv, pool_page, dev)
        k_scale.zero_()
        v_scale.zero_()
    else:
        k_scale = torch.zeros(n_phys, Hkv, pool_page, device=dev)
        v_scale = torch.zeros_like(k_scale)
    positions = torch.tensor([3, 50], dtype=torch.int32, device=dev)
    k_new = (torch.randn(B, Hkv, Tn, D, generator=g) * 3).bfloat16()
    v_new = torch.randn(B, Hkv, Tn, D, generator=g).bfloat16()
    k_new[0, 0, 0] = 0  # an all-zero row takes the 1e-8 clamp
    paged_kv_append(k_new.to(dev), v_new.to(dev), k_pool, v_pool, pt, positions,
                    k_scale=k_scale, v_scale=v_scale)
    torch.cuda.synchronize()
    for new, pool, sc in ((k_new, k_pool, k_scale), (v_new, v_pool, v_scale)):
        codes, scales = oracle.fp8_quantize(new)
        for b in range(B):
            for i in range(Tn):
                t = int(positions[b]) + i
                ph, slot = int(pt[b, t // pool_page]), t % pool_page
                got = pool[ph, :, slot].cpu().view(torch.uint8)
                assert torch.equal(got, codes[b, :, i].view(torch.uint8)), (b, i)
                assert torch.equal(sc[ph, :, slot].cpu(), scales[b, :, i, 0]), (b, i)


@pytest.mark.parametrize("Hq,union", [(8, True), (8, False), (2, True)])
def test_ragged_quest_select(dev, Hq, union):
    B, Hkv, D, ps, T = 4, 2, 64, 16, 512
    g = torch.Generator(device="cpu").manual_seed(3)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16()
    k = torch.randn(B, Hkv, T, D, generator=g).bfloat16()
    positions = torch.tensor([511, 17, 300, 0], dtype=torch.int32)
    mins, maxs = page_update_hip(k.to(dev), ps)
    ids, counts = quest_select_hip(q.to(dev), mins, maxs, page_size=ps, topk=6,
                                   gqa_union=union, positions=positions.to(dev))
    om, ox = oracle.page_bounds(k, ps)
    for b in range(B):
        ref = oracle.quest_select(q[b:b + 1], om[b:b + 1], ox[b:b + 1], page_size=ps, topk=6,
                                  offset=int(positions[b]), gqa_union=union)
        assert np.array_equal(ids[b:b + 1].cpu().numpy(), ref), b
        assert torch.equal(counts[b].cpu(), torch.from_numpy((ref[0] >= 0).sum(-1)).int())


def test_ragged_decode_after_append(dev):
    """Serving loop: append one token per sequence at ragged positions, then a
    ragged Quest decode step; every sequence matches the oracle at its own
    position (ids bit for bit, outputs within 2e-3 of fp64)."""
    B, Hq, Hkv, D, ps, max_len, topk = 4, 8, 2, 128, 16, 512, 5
    k_pool, v_pool, pt = _pool(B, Hkv, D, ps, max_len, torch.bfloat16, dev, seed=11)
    positions = torch.tensor([300, 15, 16, 511], dtype=torch.int32, device=dev)
    n_pages = max_len // ps
    mins, maxs = page_update_hip(k_pool, ps, n_pages, page_table=pt, pool_page_size=ps,
                                 kv_len=positions)
    g = torch.Generator(device="cpu").manual_seed(12)
    k_new = torch.randn(B, Hkv, 1, D, generator=g).bfloat16().to(dev)
    v_new = torch.randn(B, Hkv, 1, D, generator=g).bfloat16().to(dev)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16().to(dev)
    paged_kv_append(k_new, v_new, k_pool, v_pool, pt, positions, page_min=mins, page_max=maxs,
                    page_size=ps)
    out, ids, counts = quest_decode_step(q, k_pool, v_pool, pt, mins, maxs, page_size=ps,
                                         topk=topk, positions=positions, out_dtype=torch.float32)
    torch.cuda.synchronize()
    for b in range(B):
        L = int(positions[b]) + 1
        kb = torch.stack([k_pool[int(pt[b, t // ps]), :, t % ps] for t in range(L)], 1)
        vb = torch.stack([v_pool[int(pt[b, t // ps]), :, t % ps] for t in range(L)], 1)
        kb, vb = kb.unsqueeze(0).cpu(), vb.unsqueeze(0).cpu()
        om, ox = oracle.page_bounds(kb, ps)
        rid = oracle.quest_select(q[b:b + 1].cpu(), om, ox, page_size=ps, topk=topk,
                                  offset=L - 1)
        assert np.array_equal(ids[b:b + 1, :, :, :rid.shape[-1]].cpu().numpy(), rid), b
        ref = oracle.attend_lists(q[b:b + 1].cpu(), kb, vb, rid, unit=ps, causal=True,
                                  offset=L - 1)
        assert np.abs(out[b:b + 1].cpu().double().numpy() - ref).max() < 2e-3, b
