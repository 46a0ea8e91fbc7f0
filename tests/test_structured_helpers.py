"""CPU checks of the planted-structure helpers used by the GPU selection
quality tests."""

from __future__ import annotations

import torch

from structured import attention_mass, block_recall, lists_to_mask, structured_inputs


def test_structured_inputs_plant_spikes_and_recency():
    q, k, v = structured_inputs(1, 4, 192, 32, kv_heads=2, seed=1)
    assert q.shape == (1, 4, 192, 32) and k.shape == v.shape == (1, 2, 192, 32)
    # same seed, same tensors; a different seed differs
    q2, k2, _ = structured_inputs(1, 4, 192, 32, kv_heads=2, seed=1)
    assert torch.equal(q, q2) and torch.equal(k, k2)
    assert not torch.equal(k, structured_inputs(1, 4, 192, 32, kv_heads=2, seed=2)[1])
    # the recency ramp: late keys carry larger norms on average
    nrm = k.norm(dim=-1)
    assert nrm[..., -48:].mean() > nrm[..., :48].mean()


def test_attention_mass_rows_and_full_mask_recall():
    q, k, _ = structured_inputs(1, 4, 96, 16, kv_heads=2, seed=3)
    m = attention_mass(q, k, 16)
    # every query spends mass 1: a query block of 16 queries spends 16
    assert torch.allclose(m.sum(-1), torch.full_like(m.sum(-1), 16.0))
    # causal: no mass above the diagonal blocks
    assert float(torch.triu(m, diagonal=1).abs().max()) == 0.0
    full = torch.ones(1, 4, 96, 96, dtype=torch.bool) & (
        torch.arange(96).view(-1, 1) >= torch.arange(96).view(1, -1))
    recall, kept = block_recall(full, q, k, 16)
    assert abs(recall - 1.0) < 1e-12 and abs(kept - 21 / 36) < 1e-6


def test_lists_to_mask():
    ids = torch.tensor([[[[0, 2, -1], [1, -1, -1]]]], dtype=torch.int32)  # 2 rows of blocks
    m = lists_to_mask(ids, 4, 8, rows_per_block=4)
    want = torch.zeros(8, 8, dtype=torch.bool)
    want[:4, 0:4] = True   # row block 0 lists blocks 0 and 2 (2 is in the future)
    want[4:, 4:8] = True   # row block 1 lists block 1
    want &= torch.arange(8).view(-1, 1) >= torch.arange(8).view(1, -1)
    assert torch.equal(m[0, 0], want)
