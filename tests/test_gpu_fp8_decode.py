"""Config C5: fp8 e4m3 KV (per-token scales) sparse decode driven by the
lightning indexer, on a paged cache.  Token ids bit-exact against the oracle;
outputs within 1e-2 of the oracle's fp8-dequantised path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.kernels.block_sparse import fp8_scale_pairs
from linattn_amd.kernels.paged_decode import indexer_decode_step, quantize_fp8_per_token

pytestmark = pytest.mark.gpu


def c5_inputs(B, Hq, Hkv, T, D, ps, HI, d, seed, dev, pairs=False):
    """Seeded C5 inputs; with ``pairs`` the per-token K and V scales are the
    interleaved halves of one (pages, Hkv, page, 2) tensor (fp8_scale_pairs)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    P = T // ps
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).bfloat16()
    kf = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev)
    vf = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev)
    kc, ks = quantize_fp8_per_token(kf)
    vc, vs = quantize_fp8_per_token(vf)
    del kf, vf
    if pairs:
        ks2, vs2 = fp8_scale_pairs(B * P, Hkv, ps, dev)
        ks2.copy_(ks)
        vs2.copy_(vs)
        ks, vs = ks2, vs2
    pt = torch.randperm(B * P, generator=g, device=dev).view(B, P).to(torch.int32)
    q_idx = torch.randn(B, 1, HI, d, generator=g, device=dev).bfloat16()
    k_idx = torch.randn(B, T, HI, d, generator=g, device=dev).bfloat16()
    w = torch.rand(B, 1, HI, generator=g, device=dev)
    return q, kc, vc, ks, vs, pt, q_idx, k_idx, w


def test_quantizer_matches_the_reference_codec(dev):
    """quantize_fp8_per_token == kv/quant.py fp8 with group = head_dim."""
    x = torch.randn(64, 5, 128)
    c, s = quantize_fp8_per_token(x.to(dev))
    rc, rs = oracle.fp8_quantize(x)
    # the GPU may divide by 448 through a reciprocal: scales agree to 1 ulp and
    # codes almost everywhere (a code can move by one step at a rounding tie)
    assert torch.allclose(s.cpu(), rs.squeeze(-1), rtol=2.0 ** -23, atol=0)
    diff = c.view(torch.uint8).cpu().int() - rc.view(torch.uint8).int()
    assert (diff != 0).float().mean() < 1e-3 and diff.abs().max() <= 1


def index_order(ri):
    """The oracle's (score desc) lists as the selected set in ascending order,
    -1 padded: the form the decode step returns."""
    out = np.full_like(ri, -1)
    for r in np.ndindex(ri.shape[:-1]):
        v = np.sort(ri[r][ri[r] >= 0])
        out[r][:v.size] = v
    return out


def check_rows(out, idx, q, kc, vc, ks, vs, pt, q_idx, k_idx, w, b, topk, pos, ps):
    ri = oracle.indexer_topk(q_idx[b:b + 1].cpu(), k_idx[b:b + 1].cpu(), w[b:b + 1].cpu(), topk,
                             causal=True, offset=pos)[1]
    assert np.array_equal(idx[b:b + 1].cpu().numpy(), index_order(ri))
    Hkv = kc.shape[1]
    ids = np.broadcast_to(ri.reshape(1, 1, 1, -1), (1, Hkv, 1, ri.shape[-1]))
    ref = oracle.attend_lists(q[b:b + 1].cpu(), kc.cpu(), vc.cpu(), ids, unit=1, causal=True,
                              offset=pos, page_table=pt[b:b + 1].cpu().numpy(), page_size=ps,
                              k_scale=ks.cpu(), v_scale=vs.cpu())
    err = np.abs(out[b:b + 1].cpu().double().numpy() - ref).max()
    assert err < 1e-2, err


@pytest.mark.parametrize("pairs", [False, True])
def test_fp8_indexer_decode_small(dev, pairs):
    B, Hq, Hkv, T, D, ps, HI, d, topk = 2, 8, 2, 8192, 128, 64, 4, 64, 512
    x = c5_inputs(B, Hq, Hkv, T, D, ps, HI, d, seed=3, dev=dev, pairs=pairs)
    q, kc, vc, ks, vs, pt, q_idx, k_idx, w = x
    out, idx = indexer_decode_step(q, kc, vc, pt, q_idx, k_idx, w, topk=topk, pos=T - 1,
                                   page_size=ps, k_scale=ks, v_scale=vs, out_dtype=torch.float32)
    for b in range(B):
        check_rows(out, idx, *x, b, topk, T - 1, ps)


def test_fp8_indexer_decode_mid_sequence(dev):
    """Decode at an earlier position: keys after it are not selectable."""
    B, Hq, Hkv, T, D, ps, HI, d, topk = 1, 4, 1, 4096, 128, 64, 4, 64, 1024
    x = c5_inputs(B, Hq, Hkv, T, D, ps, HI, d, seed=4, dev=dev)
    q, kc, vc, ks, vs, pt, q_idx, k_idx, w = x
    out, idx = indexer_decode_step(q, kc, vc, pt, q_idx, k_idx, w, topk=topk, pos=700,
                                   page_size=ps, k_scale=ks, v_scale=vs, out_dtype=torch.float32)
    assert (idx[0, 0, :701] >= 0).all() and (idx[0, 0, 701:] == -1).all()
    assert idx.max() <= 700
    check_rows(out, idx, *x, 0, topk, 700, ps)


def test_config5_fp8_decode_full_size(dev):
    """C5: batch 16, context 131072, 64-token pages, 32/8 heads, D=128, fp8 KV,
    indexer (4 x 64, bf16) top-4096.  All lists checked for structure, and
    every one of the 16 sequences against the oracle: token ids bit for bit,
    outputs within 1e-2 of the fp8-dequantised attention.  The scales are
    stored interleaved (K, V) per token, as the benchmark stores them."""
    B, Hq, Hkv, T, D, ps, HI, d, topk = 16, 32, 8, 131072, 128, 64, 4, 64, 4096
    x = c5_inputs(B, Hq, Hkv, T, D, ps, HI, d, seed=0, dev=dev, pairs=True)
    q, kc, vc, ks, vs, pt, q_idx, k_idx, w = x
    out, idx = indexer_decode_step(q, kc, vc, pt, q_idx, k_idx, w, topk=topk, pos=T - 1,
                                   page_size=ps, k_scale=ks, v_scale=vs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert (idx >= 0).all() and (idx < T).all()
    s = idx.sort(-1).values
    assert (s[..., 1:] > s[..., :-1]).all()
    assert torch.isfinite(out).all()
    # the oracle on every sequence (its pages only, to bound host memory)
    idx_h, out_h = idx.cpu().numpy(), out.cpu().double().numpy()
    for b in range(B):
        sel_pages = torch.unique(pt[b]).long()
        remap = torch.full((kc.shape[0],), -1, dtype=torch.int32, device=dev)
        remap[sel_pages] = torch.arange(sel_pages.numel(), dtype=torch.int32, device=dev)
        pt_b = remap[pt[b].long()].view(1, -1)
        ri = oracle.indexer_topk(q_idx[b:b + 1].cpu(), k_idx[b:b + 1].cpu(), w[b:b + 1].cpu(),
                                 topk, causal=True, offset=T - 1)[1]
        assert np.array_equal(idx_h[b:b + 1], index_order(ri)), b
        ids = np.broadcast_to(ri.reshape(1, 1, 1, -1), (1, Hkv, 1, topk))
        ref = oracle.attend_lists(q[b:b + 1].cpu(), kc[sel_pages].cpu(), vc[sel_pages].cpu(),
                                  ids, unit=1, causal=True, offset=T - 1,
                                  page_table=pt_b.cpu().numpy(), page_size=ps,
                                  k_scale=ks[sel_pages].cpu(), v_scale=vs[sel_pages].cpu())
        assert np.abs(out_h[b:b + 1] - ref).max() < 1e-2, b
