"""GPU parity of config C3: block selection (bit-exact lists) and the MFMA
block-sparse causal prefill (within 2e-3 of the fp64 oracle, fp32 output)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.kernels.prefill import block_select_hip, block_sparse_prefill, sparse_prefill

pytestmark = pytest.mark.gpu


def c3_inputs(b, hq, hkv, t, d, seed, outliers=True, device="cpu"):
    """q/k/v ~ N(0,1); 1% of key rows per (b, kv head) scaled by 8 (a seeded
    permutation drawn after v)."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g, device=device)
    k = torch.randn(b, hkv, t, d, generator=g, device=device)
    v = torch.randn(b, hkv, t, d, generator=g, device=device)
    if outliers:
        n_out = max(1, t // 100)
        for bi in range(b):
            for h in range(hkv):
                rows = torch.randperm(t, generator=g, device=device)[:n_out]
                k[bi, h, rows] *= 8.0
    return q.bfloat16(), k.bfloat16(), v.bfloat16()


def oracle_rows(q, k, v, ids, counts, b, h, qbs, block=64):
    """fp64 attention of the query rows of blocks ``qbs`` of head h over the
    listed blocks (causal)."""
    T = q.shape[2]
    G = q.shape[1] // k.shape[1]
    out = {}
    for qb in qbs:
        t0, t1 = qb * block, min(T, (qb + 1) * block)
        lst = ids[b, h, qb, :counts[b, h, qb]].cpu().numpy()
        rows = np.broadcast_to(lst, (1, 1, t1 - t0, len(lst)))
        ref = oracle.attend_lists(q[b:b + 1, h:h + 1, t0:t1], k[b:b + 1, h // G:h // G + 1],
                                  v[b:b + 1, h // G:h // G + 1], rows, unit=block, causal=True,
                                  offset=t0)
        out[qb] = ref[0, 0]
    return out


@pytest.mark.parametrize("T", [1000, 1024])
def test_block_select_bit_exact(dev, T):
    q, k, _ = c3_inputs(2, 4, 2, T, 128, seed=1)
    ids, counts = block_select_hip(q.to(dev), k.to(dev), block=64, topk=3, sink_blocks=1,
                                   window_blocks=2)
    ref = oracle.block_select(q, k, block=64, topk=3, sink_blocks=1, window_blocks=2)
    assert np.array_equal(ids.cpu().numpy(), ref)
    assert np.array_equal(counts.cpu().numpy(), (ref >= 0).sum(-1))


@pytest.mark.parametrize("T,hq,hkv", [(1000, 4, 2), (512, 8, 8)])
def test_prefill_matches_oracle(dev, T, hq, hkv):
    q, k, v = c3_inputs(1, hq, hkv, T, 128, seed=2)
    out, ids, counts = sparse_prefill(q.to(dev), k.to(dev), v.to(dev), topk=4, sink_blocks=1,
                                      window_blocks=2, out_dtype=torch.float32)
    torch.cuda.synchronize()
    nqb = (T + 63) // 64
    for h in range(hq):
        ref = oracle_rows(q, k, v, ids.cpu(), counts.cpu(), 0, h, range(nqb))
        for qb, r in ref.items():
            got = out[0, h, qb * 64:qb * 64 + r.shape[0]].cpu().double().numpy()
            assert np.abs(got - r).max() < 2e-3, (h, qb)


def test_prefill_full_selection_is_dense_causal(dev):
    """Every causal block listed: the executor must equal dense causal
    attention (test_kernels.py:71-83 plus the causal mask)."""
    q, k, v = c3_inputs(1, 2, 1, 320, 128, seed=3, outliers=False)
    nqb = 5
    ids = torch.full((1, 2, nqb, nqb), -1, dtype=torch.int32)
    for i in range(nqb):
        ids[:, :, i, :i + 1] = torch.arange(i + 1, dtype=torch.int32)
    out = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), ids.to(dev),
                               out_dtype=torch.float32)
    ref = oracle.dense_attention(q, k, v)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3
    out_b = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), ids.to(dev))
    assert out_b.dtype == torch.bfloat16
    assert np.abs(out_b.cpu().double().numpy() - ref).max() < 1.6e-2  # bf16 output rounding


def test_prefill_empty_list_gives_zeros(dev):
    q, k, v = c3_inputs(1, 1, 1, 128, 128, seed=4, outliers=False)
    ids = torch.full((1, 1, 2, 3), -1, dtype=torch.int32)
    out = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), ids.to(dev),
                               out_dtype=torch.float32)
    assert torch.count_nonzero(out) == 0


def test_config3_full_size(dev):
    """C3: B=2, T=32768, 32/8 heads, D=128, 64x64 blocks, sink + 4-block window
    + top-16.  Lists of two heads are checked bit for bit against the oracle;
    output rows of five query blocks per head against the fp64 oracle."""
    B, Hq, Hkv, T, D = 2, 32, 8, 32768, 128
    q, k, v = c3_inputs(B, Hq, Hkv, T, D, seed=0, device=dev)
    out, ids, counts = sparse_prefill(q, k, v, topk=16, sink_blocks=1, window_blocks=4,
                                      out_dtype=torch.float32)
    torch.cuda.synchronize()
    nqb = T // 64
    assert (counts >= 1).all() and (counts <= 21).all()
    qb_idx = torch.arange(nqb, device=dev)
    assert (ids.max(-1).values <= qb_idx).all()  # causal
    assert ((ids == qb_idx.view(1, 1, -1, 1)).any(-1)).all()  # diagonal block present
    assert (ids[..., 0] == 0).all()  # sink
    for b, h in ((0, 0), (1, 13)):
        kvh = h // (Hq // Hkv)
        qc, kc, vc = q[b:b + 1, h:h + 1].cpu(), k[b:b + 1, kvh:kvh + 1].cpu(), \
            v[b:b + 1, kvh:kvh + 1].cpu()
        ref = oracle.block_select(qc, kc, block=64, topk=16, sink_blocks=1, window_blocks=4)
        assert np.array_equal(ids[b:b + 1, h:h + 1].cpu().numpy(), ref)
        ids_c, counts_c = ids[b:b + 1, h:h + 1].cpu(), counts[b:b + 1, h:h + 1].cpu()
        rows = oracle_rows(qc, kc, vc, ids_c, counts_c, 0, 0, (0, 1, 17, 300, nqb - 1))
        for qb, r in rows.items():
            got = out[b, h, qb * 64:(qb + 1) * 64].cpu().double().numpy()
            assert np.abs(got - r).max() < 2e-3, (b, h, qb)
