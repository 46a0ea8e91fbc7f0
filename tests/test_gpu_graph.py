"""The C5 decode step (decode indexer, multi-launch radix top-k, split-K fp8
paged attention and its combine) captured into a HIP graph and replayed:
every replay equals the eager step bit for bit.  The per-call value the
decode indexer keys its rows' ready words on is baked into a graph, so a
replay relies on the device-side epoch that the radix select's first launch
advances; eager steps run between the replays."""

from __future__ import annotations

import pytest
import torch

from linattn_amd import _native as N
from linattn_amd.kernels.block_sparse import fp8_scale_pairs
from linattn_amd.kernels.paged_decode import indexer_decode_step, quantize_fp8_per_token

pytestmark = pytest.mark.gpu


def _inputs(dev, seed):
    B, Hq, Hkv, T, D, ps, HI, d = 2, 32, 8, 69632, 128, 64, 4, 64
    P = T // ps
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).bfloat16()
    kc, ks = quantize_fp8_per_token(torch.randn(B * P, Hkv, ps, D, generator=g, device=dev))
    vc, vs = quantize_fp8_per_token(torch.randn(B * P, Hkv, ps, D, generator=g, device=dev))
    ksp, vsp = fp8_scale_pairs(B * P, Hkv, ps, dev)
    ksp.copy_(ks)
    vsp.copy_(vs)
    pt = torch.randperm(B * P, generator=g, device=dev).view(B, P).to(torch.int32)
    q_idx = torch.randn(B, 1, HI, d, generator=g, device=dev).bfloat16()
    k_idx = torch.randn(B, T, HI, d, generator=g, device=dev).bfloat16()
    w = torch.rand(B, 1, HI, generator=g, device=dev)
    return (q, kc, vc, pt, q_idx, k_idx, w), dict(topk=4096, pos=T - 1, page_size=ps,
                                                   k_scale=ksp, v_scale=vsp)


def test_c5_step_graph_replays_equal_eager(dev):
    args, kw = _inputs(dev, 3)
    N.device_status(dev)
    out_ref, idx_ref = indexer_decode_step(*args, **kw)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            indexer_decode_step(*args, **kw)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, idx_g = indexer_decode_step(*args, **kw)
    for rep in range(4):
        out_g.zero_()
        idx_g.fill_(-2)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx_g, idx_ref), rep
        assert torch.equal(out_g, out_ref), rep
        out_e, idx_e = indexer_decode_step(*args, **kw)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(idx_e, idx_ref) and torch.equal(out_e, out_ref), rep
    assert N.device_status(dev) == 0
