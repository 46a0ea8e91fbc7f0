"""GPU parity: Quest metadata / scores / selection and the sparse-attention
executor against the CPU oracle.

Bars: page ids and scores bit-exact; attention within 1e-5 (fp32), 2e-3 (bf16
inputs, fp32 output) and 1e-2 (fp8 KV versus the fp8-dequantised oracle).
Inputs follow the reference harness recipe (harness.py:43-48): a CPU
torch.Generator draws q, k, v in that order from N(0, 1).
"""

from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.kernels.block_sparse import block_sparse_attention, sparse_attention
from linattn_amd.kernels.paged_decode import paged_decode, quest_decode_step
from linattn_amd.kernels.quest_pages import (page_scores_hip, page_select_hip, page_update_hip,
                                              quest_select_hip)

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def make_inputs(b, hq, hkv, t_q, t_k, d, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t_q, d, generator=g)
    k = torch.randn(b, hkv, t_k, d, generator=g)
    v = torch.randn(b, hkv, t_k, d, generator=g)
    return q, k, v


def to_pool(k, v, ps, seed=1):
    """Scatter contiguous (B, Hkv, T, D) caches into a pool through a random
    page table (pages of ps tokens)."""
    B, Hkv, T, D = k.shape
    P = T // ps
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(B * P, generator=g)
    pt = perm.view(B, P).to(torch.int32)
    pk = torch.empty(B * P, Hkv, ps, D, dtype=k.dtype)
    pv = torch.empty_like(pk)
    kk = k.view(B, Hkv, P, ps, D).permute(0, 2, 1, 3, 4)
    vv = v.view(B, Hkv, P, ps, D).permute(0, 2, 1, 3, 4)
    pk[pt.view(-1).long()] = kk.reshape(B * P, Hkv, ps, D)
    pv[pt.view(-1).long()] = vv.reshape(B * P, Hkv, ps, D)
    return pk, pv, pt


# -------------------------------------------------------------- quest ----
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_page_bounds_exact(dev, dtype):
    q, k, v = make_inputs(2, 4, 2, 1, 100, 64)
    k = k.to(dtype)
    mins, maxs = page_update_hip(k.to(dev), 16)
    om, ox = oracle.page_bounds(k, 16)
    assert np.array_equal(oracle.to_f64(mins), om)
    assert np.array_equal(oracle.to_f64(maxs), ox)
    # the same cache through a page table
    kp = torch.cat([k, torch.zeros(2, 2, 12, 64, dtype=dtype)], dim=2)
    pk, pv, pt = to_pool(kp, kp, 16)
    pm, px = page_update_hip(pk.to(dev), 16, page_table=pt.to(dev),
                             kv_len=torch.tensor([100, 100], dtype=torch.int32, device=dev))
    assert torch.equal(pm.cpu(), mins.cpu()) and torch.equal(px.cpu(), maxs.cpu())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2), (32, 8)])
def test_quest_scores_bit_exact(dev, dtype, hq, hkv):
    q, k, _ = make_inputs(2, hq, hkv, 3, 333, 128, seed=hq)
    q, k = q.to(dtype), k.to(dtype)
    mins, maxs = page_update_hip(k.to(dev), 16)
    got = page_scores_hip(q.to(dev), mins, maxs).cpu().numpy()
    ref = oracle.quest_scores(q, mins.cpu(), maxs.cpu())
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("union", [False, True])
@pytest.mark.parametrize("hq,hkv,tq,offset", [(8, 8, 1, 4095), (8, 2, 1, 2000), (4, 2, 40, 0),
                                               (32, 8, 5, 1000)])
def test_quest_select_bit_exact(dev, union, hq, hkv, tq, offset):
    t = 4096 if offset >= 1000 else 64
    q, k, _ = make_inputs(1, hq, hkv, tq, t, 64, seed=3)
    mins, maxs = page_update_hip(k.to(dev), 16)
    ids, counts = quest_select_hip(q.to(dev), mins, maxs, page_size=16, topk=16, offset=offset,
                                   gqa_union=union)
    ref = oracle.quest_select(q, mins.cpu(), maxs.cpu(), page_size=16, topk=16, offset=offset,
                              gqa_union=union)
    assert np.array_equal(ids.cpu().numpy(), ref)
    assert np.array_equal(counts.cpu().numpy(), (ref >= 0).sum(-1))


@pytest.mark.parametrize("hq,hkv,ps,t", [(32, 8, 16, 16384), (16, 2, 64, 65536), (8, 4, 8, 4000)])
def test_quest_select_fused_equals_two_pass(dev, hq, hkv, ps, t):
    """The one-pass union selection (page-minor metadata) equals scores +
    top-k run separately (row-major metadata takes that path), including
    queries whose position cuts the page range short."""
    q, k, _ = make_inputs(2, hq, hkv, 3, t, 64, seed=hq + ps)
    q, k = q.bfloat16(), k.bfloat16()
    mins, maxs = page_update_hip(k.to(dev), ps)
    for offset in (t - 3, t // 3, 5):
        a, ca = quest_select_hip(q.to(dev), mins, maxs, page_size=ps, topk=24, offset=offset)
        b, cb = quest_select_hip(q.to(dev), mins.contiguous(), maxs.contiguous(), page_size=ps,
                                 topk=24, offset=offset)
        assert torch.equal(a, b) and torch.equal(ca, cb), offset


def test_page_select_api_matches_reference_semantics(dev):
    """page_select_torch (quest_pages.py:58-78) with the D1 fix."""
    q, k, _ = make_inputs(1, 4, 4, 24, 96, 32, seed=5)
    mins, maxs = page_update_hip(k.to(dev), 8)
    ids, scores = page_select_hip(q.to(dev), mins, maxs, 8, 3, offset=40)
    rid, rsc = oracle.page_select(q, mins.cpu(), maxs.cpu(), 8, 3, offset=40)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(scores.cpu().numpy(), rsc.astype(np.float32))


def test_quest_known_answer_last_page(dev):
    """test_selection.py:68-91 on the GPU."""
    q = torch.zeros(1, 2, 32, 16)
    k = torch.zeros(1, 2, 32, 16)
    k[:, :, 24:, :] = 50.0
    q[:, :, :, 0] = 1.0
    mins, maxs = page_update_hip(k.to(dev), 8)
    ids, _ = quest_select_hip(q.to(dev), mins, maxs, page_size=8, topk=1, offset=0,
                              gqa_union=False)
    assert 3 in ids[0, 0, 31].tolist()


# ----------------------------------------------------------- executor ----
def _lists(b, heads, rows, n, n_units, seed, holes=True):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, n_units, (b, heads, rows, n), generator=g, dtype=torch.int32)
    if holes:
        ids[..., -1] = -1
    return ids


@pytest.mark.parametrize("hq,hkv,lists_per", [(8, 8, "kv"), (8, 2, "kv"), (8, 2, "q"),
                                               (32, 8, "kv")])
@pytest.mark.parametrize("d", [64, 128])
def test_sparse_attention_fp32(dev, hq, hkv, lists_per, d):
    q, k, v = make_inputs(2, hq, hkv, 3, 203, d, seed=7)  # 203: ragged last block
    heads = hkv if lists_per == "kv" else hq
    ids = _lists(2, heads, 3, 9, (203 + 15) // 16, seed=8)
    ids[0, 0, 0, 1] = ids[0, 0, 0, 0]  # a repeated block counts twice
    out = sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), unit=16)
    ref = oracle.attend_lists(q, k, v, ids.numpy(), unit=16)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5


def test_sparse_attention_causal_counts_kvlen_splits(dev):
    q, k, v = make_inputs(3, 8, 2, 4, 256, 64, seed=9)
    ids = _lists(3, 2, 4, 12, 16, seed=10, holes=False)
    counts = torch.tensor([[[12, 5, 0, 12], [3, 12, 12, 1]]] * 3, dtype=torch.int32)
    kv_len = torch.tensor([256, 100, 17], dtype=torch.int32)
    ref = None
    for splits in (1, 0, 5, 12):
        out = sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), unit=16,
                               counts=counts.to(dev), causal=True, offset=60,
                               kv_len=kv_len.to(dev), num_splits=splits)
        if ref is None:
            ref = np.zeros((3, 8, 4, 64))
            for b in range(3):
                ref[b:b + 1] = oracle.attend_lists(q[b:b + 1], k[b:b + 1], v[b:b + 1],
                                                   ids[b:b + 1].numpy(), unit=16,
                                                   counts=counts[b:b + 1].numpy(), causal=True,
                                                   offset=60, kv_len=[int(kv_len[b])])
        assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5, splits


def test_sparse_attention_empty_rows_give_zeros(dev):
    q, k, v = make_inputs(1, 4, 4, 2, 64, 64)
    ids = torch.full((1, 4, 2, 3), -1, dtype=torch.int32)
    ids[0, 1, 0, 0] = 7  # block 7 lies past T = 64 -> still empty
    out = sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), unit=16)
    assert torch.count_nonzero(out) == 0


def test_sparse_attention_bf16(dev):
    q, k, v = make_inputs(2, 32, 8, 1, 4096, 128, seed=11)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    ids = _lists(2, 8, 1, 40, 64, seed=12)
    out = sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), unit=64,
                           out_dtype=torch.float32)
    ref = oracle.attend_lists(q, k, v, ids.numpy(), unit=64)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (32, 8), (16, 2)])
@pytest.mark.parametrize("unit,paged", [(64, True), (16, True), (32, False), (1, True), (8, True)])
def test_sparse_attention_bf16_matrix_core_paths(dev, hq, hkv, unit, paged):
    """bf16 q and K/V at head dim 128 take the matrix-core kernel: whole
    16-row rounds inside one page (unit a multiple of 16, paged) or per-token
    row lookups (any other unit or layout).  Causal masking with an offset, a
    ragged kv length, per-list counts and several split counts."""
    B, T, D, ps = 2, 1024, 128, 64
    q, k, v = make_inputs(B, hq, hkv, 2, T, D, seed=hq + unit)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    n_units = T // unit
    n = min(24, n_units) if unit > 1 else 300
    ids = _lists(B, hkv, 2, n, n_units, seed=unit, holes=True)
    counts = torch.tensor([[[n, n - 3]] * hkv, [[n - 7, n]] * hkv], dtype=torch.int32)
    kv_len = torch.tensor([T, 700], dtype=torch.int32)
    offset = 900
    kw = dict(unit=unit, counts=counts.to(dev), causal=True, offset=offset, kv_len=kv_len.to(dev),
              out_dtype=torch.float32)
    if paged:
        pk, pv, pt = to_pool(k, v, ps)
        args = (pk.to(dev), pv.to(dev))
        kw.update(page_table=pt.to(dev), page_size=ps)
    else:
        args = (k.to(dev), v.to(dev))
    ref = np.zeros((B, hq, 2, D))
    for b in range(B):
        ref[b:b + 1] = oracle.attend_lists(q[b:b + 1], k[b:b + 1], v[b:b + 1], ids[b:b + 1].numpy(),
                                           unit=unit, counts=counts[b:b + 1].numpy(), causal=True,
                                           offset=offset, kv_len=[int(kv_len[b])])
    for splits in (1, 0, 3):
        out = sparse_attention(q.to(dev), *args, ids.to(dev), num_splits=splits, **kw)
        err = np.abs(out.cpu().double().numpy() - ref).max()
        assert err < 2e-3, (splits, err)


@pytest.mark.parametrize("paged", [False, True])
def test_sparse_attention_fp8(dev, paged):
    """fp8 e4m3 K/V with per-token scales (kv/quant.py:90-93, group = head_dim)."""
    q, k, v = make_inputs(2, 8, 2, 1, 1024, 128, seed=13)
    kc, ks = oracle.fp8_quantize(k)
    vc, vs = oracle.fp8_quantize(v)
    ks, vs = ks.squeeze(-1), vs.squeeze(-1)
    ids = _lists(2, 1, 1, 300, 1024, seed=14).expand(2, 2, 1, 300).contiguous()  # token ids
    qb = q.bfloat16()
    if paged:
        pk, pv, pt = to_pool(kc.view(torch.uint8), vc.view(torch.uint8), 64)
        psk, psv, _ = to_pool(ks.unsqueeze(-1), vs.unsqueeze(-1), 64)
        out = sparse_attention(qb.to(dev), pk.view(torch.float8_e4m3fn).to(dev),
                               pv.view(torch.float8_e4m3fn).to(dev), ids.to(dev), unit=1,
                               page_table=pt.to(dev), page_size=64,
                               k_scale=psk.squeeze(-1).contiguous().to(dev),
                               v_scale=psv.squeeze(-1).contiguous().to(dev),
                               out_dtype=torch.float32)
    else:
        out = sparse_attention(qb.to(dev), kc.to(dev), vc.to(dev), ids.to(dev), unit=1,
                               k_scale=ks.to(dev), v_scale=vs.to(dev), out_dtype=torch.float32)
    ref = oracle.attend_lists(qb, kc, vc, ids.numpy(), unit=1, k_scale=ks, v_scale=vs)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-2


@pytest.mark.parametrize("unit,causal", [(16, False), (64, True)])
def test_sparse_attention_fp8_page_lists(dev, unit, causal):
    """fp8 page lists on the paged pool (the matrix-core kernel's rounds of 16
    rows inside one page), GQA groups of 4 and of 1, causal cut mid-page."""
    q, k, v = make_inputs(2, 8, 2, 1, 1024, 128, seed=15)
    kc, ks = oracle.fp8_quantize(k)
    vc, vs = oracle.fp8_quantize(v)
    ks, vs = ks.squeeze(-1), vs.squeeze(-1)
    n_units = 1024 // unit
    pk, pv, pt = to_pool(kc.view(torch.uint8), vc.view(torch.uint8), 64)
    psk, psv, _ = to_pool(ks.unsqueeze(-1), vs.unsqueeze(-1), 64)
    kw = dict(unit=unit, page_table=pt.to(dev), page_size=64,
              k_scale=psk.squeeze(-1).contiguous().to(dev),
              v_scale=psv.squeeze(-1).contiguous().to(dev), out_dtype=torch.float32)
    off = 1000 if causal else 0
    qb = q.bfloat16()
    for heads in (2, 8):  # one list per KV head (G = 4) or per query head (G = 1)
        ids = _lists(2, heads, 1, n_units // 3, n_units, seed=16 + heads)
        out = sparse_attention(qb.to(dev), pk.view(torch.float8_e4m3fn).to(dev),
                               pv.view(torch.float8_e4m3fn).to(dev), ids.to(dev), causal=causal,
                               offset=off, **kw)
        ref = oracle.attend_lists(qb, kc, vc, ids.numpy(), unit=unit, causal=causal, offset=off,
                                  k_scale=ks, v_scale=vs)
        # fp8 MFMA scores with q as a two-term fp8 expansion (~2^-8 relative)
        assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3, heads


def test_paged_pool_equals_contiguous(dev):
    q, k, v = make_inputs(2, 32, 8, 1, 1024, 128, seed=15)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    pk, pv, pt = to_pool(k, v, 64)
    ids = _lists(2, 8, 1, 10, 16, seed=16)
    a = sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), unit=64,
                         out_dtype=torch.float32)
    b = sparse_attention(q.to(dev), pk.to(dev), pv.to(dev), ids.to(dev), unit=64,
                         page_table=pt.to(dev), page_size=64, out_dtype=torch.float32)
    assert torch.equal(a, b)


def test_block_sparse_full_selection_equals_dense(dev):
    """test_kernels.py:71-83 on the GPU (fp32)."""
    q, k, v = make_inputs(1, 2, 2, 32, 32, 64)
    ids = torch.arange(4, dtype=torch.int32).view(1, 1, 1, -1).expand(1, 2, 32, 4).contiguous()
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), block_size=8)
    ref = oracle.dense_attention(q, k, v, causal=False)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5


def test_block_sparse_random_blocks_bf16(dev):
    """test_kernels.py:126-138 (the reference's GPU parity test) in bf16."""
    torch.manual_seed(0)
    b, h, t, d, bs = 1, 4, 128, 64, 32
    q = torch.randn(b, h, t, d).bfloat16()
    k = torch.randn(b, h, t, d).bfloat16()
    v = torch.randn(b, h, t, d).bfloat16()
    ids = torch.randint(0, t // bs, (b, h, t, 2))
    ids[..., 1] = torch.arange(t) // bs
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), block_size=bs,
                                 out_dtype=torch.float32)
    ref = oracle.block_sparse_attention(q, k, v, ids.numpy(), block_size=bs)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3
    out2 = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), ids.to(dev), block_size=bs)
    assert out2.dtype == torch.bfloat16


def test_paged_decode_api_matches_reference_c(dev):
    """paged_decode (c_attention.py:76-111) against the reference's own C
    decode when built (oracle/_ref), else the oracle; test_kernels.py:31-44."""
    torch.manual_seed(0)
    t, dim, page = 4096, 64, 8
    k = torch.randn(t, dim)
    v = torch.randn(t, dim)
    q = torch.randn(dim)
    pages = torch.arange(0, 128)
    out, stats = paged_decode(q.to(dev), k.to(dev), v.to(dev), pages.to(dev), page_size=page)
    assert stats["kv_entries"] == 128 * page
    ref = oracle.attend_lists(q.view(1, 1, 1, dim).double(), k.view(1, 1, t, dim),
                              v.view(1, 1, t, dim), pages.view(1, 1, 1, -1).numpy(), unit=page)
    assert np.abs(out.cpu().double().numpy() - ref[0, 0, 0]).max() < 1e-5
    lib = ROOT / "oracle" / "_ref" / "libdecode_attn.so"
    if lib.exists():
        import ctypes

        L = ctypes.CDLL(str(lib))
        f = ctypes.POINTER(ctypes.c_float)
        i = ctypes.POINTER(ctypes.c_int32)
        L.paged_decode_tiled.argtypes = [f, f, f, i, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_float, f]
        ids = pages.to(torch.int32).contiguous()
        cref = torch.zeros(dim)
        L.paged_decode_tiled(ctypes.cast(q.data_ptr(), f), ctypes.cast(k.data_ptr(), f),
                             ctypes.cast(v.data_ptr(), f), ctypes.cast(ids.data_ptr(), i), 128,
                             page, dim, t, 1.0 / math.sqrt(dim), ctypes.cast(cref.data_ptr(), f))
        assert torch.allclose(out.cpu(), cref, atol=2e-4)


# ------------------------------------------------------------- configs ----
def test_config1_quest_decode_fp32(dev):
    """C1: B=1, H=Hkv=8, D=64, T=4096, page 16, top-16 pages, fp32, seed 0."""
    B, H, T, D, ps, topk = 1, 8, 4096, 64, 16, 16
    q, k, v = make_inputs(B, H, H, 1, T, D, seed=0)
    mins, maxs = page_update_hip(k.to(dev), ps)
    pk, pv, pt = to_pool(k, v, ps)
    out, ids, counts = quest_decode_step(q.to(dev), pk.to(dev), pv.to(dev), pt.to(dev), mins, maxs,
                                         page_size=ps, topk=topk, pos=T - 1)
    om, ox = oracle.page_bounds(k, ps)
    rid = oracle.quest_select(q, om, ox, page_size=ps, topk=topk, offset=T - 1)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert (counts.cpu() == topk).all() and (ids[..., 0] >= 0).all()
    assert (ids == T // ps - 1).any(-1).all()  # own page always read
    ref = oracle.attend_lists(q, k, v, rid, unit=ps, causal=True, offset=T - 1)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 1e-5


@pytest.mark.parametrize("union", [True, False])
def test_config4_paged_quest_decode_full_size(dev, union):
    """C4 at full size: B=64, T=65536, page 64, 32/8 heads, D=128, bf16, a
    permuted page table, 2048-token budget with the last page forced.
    Every list is checked by properties on the GPU (own page present, sorted
    and unique, selected scores dominate unselected ones with the index tie
    rule), and every one of the 64 sequences against the oracle: the page
    bounds of all 8 KV heads and the page ids bit for bit (the oracle selects
    from its own bounds), outputs within 2e-3."""
    B, Hq, Hkv, T, D, ps, topk = 64, 32, 8, 65536, 128, 64, 32
    P = T // ps
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).bfloat16()
    pool_k = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev).bfloat16()
    pool_v = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev).bfloat16()
    pt = torch.randperm(B * P, generator=g, device=dev).view(B, P).to(torch.int32)
    mins, maxs = page_update_hip(pool_k, ps, page_table=pt)
    out, ids, counts = quest_decode_step(q, pool_k, pool_v, pt, mins, maxs, page_size=ps,
                                         topk=topk, pos=T - 1, gqa_union=union,
                                         out_dtype=torch.float32)
    torch.cuda.synchronize()
    G = Hq // Hkv
    scores = page_scores_hip(q, mins, maxs)  # (B, Hq, 1, P)
    if union:
        assert ids.shape == (B, Hkv, 1, G * topk)
    # properties over the whole batch
    valid = ids >= 0
    assert torch.equal(valid.sum(-1).to(torch.int32), counts)
    assert (ids == P - 1).any(-1).all()
    s = ids.masked_fill(~valid, 1 << 30).sort(-1).values
    if union:
        assert (s[..., 1:] > s[..., :-1])[valid[..., 1:]].all()  # ascending, unique
    # per query head: the kept pages are the top-k by (score desc, index asc)
    sc = scores.squeeze(2).clone()
    sc[..., P - 1] = float("inf")
    rank_keys = torch.argsort(-sc, dim=-1, stable=True)[..., :topk]
    want = torch.zeros_like(sc, dtype=torch.bool).scatter_(-1, rank_keys, True)
    if union:
        want_kv = want.view(B, Hkv, G, P).any(2)
        got_kv = torch.zeros(B, Hkv, P, dtype=torch.int32, device=dev)
        idc = ids.squeeze(2).clamp(min=0).long()
        got_kv.scatter_reduce_(-1, idc, valid.squeeze(2).to(torch.int32), reduce="amax")
        assert torch.equal(got_kv.bool(), want_kv)
    else:
        got = torch.zeros(B, Hq, P, dtype=torch.bool, device=dev)
        got.scatter_(-1, ids.squeeze(2).long(), True)
        assert torch.equal(got, want)
    # the page bounds of every sequence and KV head against the oracle's, and
    # the oracle's selection from the oracle's own bounds (one sequence per
    # thread: each gathers its 1024 pages and takes their channel min/max)
    mins_h, maxs_h, q_h = mins.cpu(), maxs.cpu(), q.cpu()
    pool_h = pool_k.cpu()
    pt_h = pt.cpu().long()

    def oracle_bounds(b):
        kb = pool_h[pt_h[b]].permute(1, 0, 2, 3).reshape(1, Hkv, T, D)
        om, ox = oracle.page_bounds(kb, ps)
        ok = (np.array_equal(oracle.to_f64(mins_h[b:b + 1]), om)
              and np.array_equal(oracle.to_f64(maxs_h[b:b + 1]), ox))
        return ok, om, ox

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4)) as ex:
        bounds = list(ex.map(oracle_bounds, range(B)))
    del pool_h
    assert all(ok for ok, _, _ in bounds), [b for b, (ok, _, _) in enumerate(bounds) if not ok]
    # every sequence against the oracle: its selected pages gathered into a
    # compact pool, addressed through a remapped page table
    ids_h, out_h = ids.cpu().numpy(), out.cpu().double().numpy()
    for b in range(B):
        _, om, ox = bounds[b]
        rid = oracle.quest_select(q_h[b:b + 1], om, ox, page_size=ps,
                                  topk=topk, offset=T - 1, gqa_union=union)
        assert np.array_equal(ids_h[b:b + 1], rid), b
        sel = np.unique(rid[rid >= 0])
        phys = pt_h[b, torch.from_numpy(sel).long()]
        ck, cv = pool_k[phys.to(dev)].cpu(), pool_v[phys.to(dev)].cpu()
        cpt = np.zeros((1, P), dtype=np.int32)
        cpt[0, sel] = np.arange(sel.size, dtype=np.int32)
        ref = oracle.attend_lists(q_h[b:b + 1], ck, cv, rid, unit=ps, causal=True, offset=T - 1,
                                  page_table=cpt, page_size=ps)
        assert np.abs(out_h[b:b + 1] - ref).max() < 2e-3, b
