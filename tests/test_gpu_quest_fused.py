"""The fused Quest decode kernel (selection and attention in one launch)
against the two-kernel path and the CPU oracle: page lists bit-exact, outputs
within 2e-3 of the oracle (bf16 inputs, fp32 output) and within 1e-5 of the
two-kernel path (the same fp32 arithmetic over a different split of the
tokens among waves)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.kernels.paged_decode import quest_decode_fused, quest_decode_step
from linattn_amd.kernels.quest_pages import page_update_hip

pytestmark = pytest.mark.gpu


def paged_inputs(B, Hq, Hkv, T, D, ps, seed, dev):
    P = T // ps
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).bfloat16()
    pk = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev).bfloat16()
    pv = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev).bfloat16()
    pt = torch.randperm(B * P, generator=g, device=dev).view(B, P).to(torch.int32)
    mins, maxs = page_update_hip(pk, ps, page_table=pt)
    return q, pk, pv, pt, mins, maxs


def oracle_rows(q, pk, pv, pt, ids, ps, positions):
    """The oracle's attention of every sequence over the fused kernel's lists
    (the selected pages gathered into a compact pool)."""
    B, P = pt.shape
    q_h, pt_h, ids_h = q.cpu(), pt.cpu().long(), ids.cpu().numpy()
    outs = []
    for b in range(B):
        rid = ids_h[b:b + 1]
        sel = np.unique(rid[rid >= 0])
        phys = pt_h[b, torch.from_numpy(sel).long()]
        ck, cv = pk[phys.to(pk.device)].cpu(), pv[phys.to(pv.device)].cpu()
        cpt = np.zeros((1, P), dtype=np.int32)
        cpt[0, sel] = np.arange(sel.size, dtype=np.int32)
        outs.append(oracle.attend_lists(q_h[b:b + 1], ck, cv, rid, unit=ps, causal=True,
                                        offset=int(positions[b]), page_table=cpt, page_size=ps))
    return np.concatenate(outs)


@pytest.mark.parametrize("hq,hkv", [(16, 4), (8, 4)])
def test_fused_equals_two_kernel_and_oracle(dev, hq, hkv):
    B, T, D, ps, topk = 3, 8192, 128, 64, 16
    q, pk, pv, pt, mins, maxs = paged_inputs(B, hq, hkv, T, D, ps, seed=hq + hkv, dev=dev)
    out, ids, counts = quest_decode_fused(q, pk, pv, pt, mins, maxs, page_size=ps, topk=topk,
                                          pos=T - 1, out_dtype=torch.float32)
    out2, ids2, counts2 = quest_decode_step(q, pk, pv, pt, mins, maxs, page_size=ps, topk=topk,
                                            pos=T - 1, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(counts, counts2)
    assert (out - out2).abs().max().item() < 1e-5
    rid = oracle.quest_select(q.cpu(), mins.cpu(), maxs.cpu(), page_size=ps, topk=topk,
                              offset=T - 1, gqa_union=True)
    assert np.array_equal(ids.cpu().numpy(), rid)
    ref = oracle_rows(q, pk, pv, pt, ids, ps, [T - 1] * B)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3


def test_fused_ragged_positions_and_kv_len(dev):
    """Per-sequence positions, some inside a page (the own page is partly
    visible), and a cache length below the position for one sequence."""
    B, Hq, Hkv, T, D, ps, topk = 4, 16, 4, 4096, 128, 64, 8
    q, pk, pv, pt, mins, maxs = paged_inputs(B, Hq, Hkv, T, D, ps, seed=5, dev=dev)
    positions = torch.tensor([T - 1, 2000, 77, 3071], dtype=torch.int32, device=dev)
    kv_len = torch.tensor([T, 2001, 78, 3000], dtype=torch.int32, device=dev)
    out, ids, counts = quest_decode_fused(q, pk, pv, pt, mins, maxs, page_size=ps, topk=topk,
                                          positions=positions, kv_len=kv_len,
                                          out_dtype=torch.float32)
    out2, ids2, counts2 = quest_decode_step(q, pk, pv, pt, mins, maxs, page_size=ps, topk=topk,
                                            positions=positions, kv_len=kv_len,
                                            out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(counts, counts2)
    assert (out - out2).abs().max().item() < 1e-5
    for b, p in enumerate(positions.tolist()):
        rid = oracle.quest_select(q[b:b + 1].cpu(), mins[b:b + 1].cpu(), maxs[b:b + 1].cpu(),
                                  page_size=ps, topk=topk, offset=p, gqa_union=True)
        assert np.array_equal(ids[b:b + 1].cpu().numpy(), rid), b
    # the oracle reads keys up to min(position, kv_len - 1)
    lim = torch.minimum(positions, kv_len - 1).tolist()
    ref = oracle_rows(q, pk, pv, pt, ids, ps, lim)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3


@pytest.mark.parametrize("hq,hkv", [(8, 1), (4, 4)])
def test_fused_rejects_unsupported_shapes(dev, hq, hkv):
    """G = 8 (the selection scratch would not fit) and G = 1 (per-head lists,
    kept in score order by quest_select_hip) are not fused."""
    B, T, D, ps = 1, 1024, 128, 64
    q, pk, pv, pt, mins, maxs = paged_inputs(B, hq, hkv, T, D, ps, seed=6, dev=dev)
    with pytest.raises(NotImplementedError):
        quest_decode_fused(q, pk, pv, pt, mins, maxs, page_size=ps, topk=4, pos=T - 1)
    with pytest.raises(ValueError):
        quest_decode_fused(q, pk, pv, pt, mins, maxs, page_size=ps, topk=4)


def test_fused_config4_full_size(dev):
    """C4 (B=64, T=65536, page 64, 32/8 heads, D=128, bf16, 2048-token
    budget): the fused kernel's lists equal the two-kernel path's for all 512
    (b, KV head) lists, which the two-kernel test pins against the oracle for
    every sequence; outputs within 1e-5 of that path."""
    B, Hq, Hkv, T, D, ps, topk = 64, 32, 8, 65536, 128, 64, 32
    q, pk, pv, pt, mins, maxs = paged_inputs(B, Hq, Hkv, T, D, ps, seed=0, dev=dev)
    out, ids, counts = quest_decode_fused(q, pk, pv, pt, mins, maxs, page_size=ps, topk=topk,
                                          pos=T - 1, out_dtype=torch.float32)
    out2, ids2, counts2 = quest_decode_step(q, pk, pv, pt, mins, maxs, page_size=ps, topk=topk,
                                            pos=T - 1, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(counts, counts2)
    assert (out - out2).abs().max().item() < 1e-5
    for b in (0, 63):
        ref = oracle_rows(q[b:b + 1], pk, pv, pt[b:b + 1], ids[b:b + 1], ps, [T - 1])
        assert np.abs(out[b:b + 1].cpu().double().numpy() - ref).max() < 2e-3
