"""la_sparse_attention_noalloc (static per-device scratch, no workspace)
against la_sparse_attention (workspace from the caller), through the C-ABI:
two calls in a row, the second on a smaller input, and the size limit."""

from __future__ import annotations

import pytest
import torch

from linattn_amd import _native as N
from linattn_amd.kernels.block_sparse import sparse_attention

pytestmark = pytest.mark.gpu


def paged_case(B, Hq, Hkv, T, D, ps, n_list, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    P = T // ps
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).bfloat16()
    pk = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev).bfloat16()
    pv = torch.randn(B * P, Hkv, ps, D, generator=g, device=dev).bfloat16()
    pt = torch.randperm(B * P, generator=g, device=dev).view(B, P).to(torch.int32)
    ids = torch.stack([torch.randperm(P, generator=g, device=dev)[:n_list].sort().values
                       for _ in range(B * Hkv)]).view(B, Hkv, 1, n_list).to(torch.int32)
    ids[..., -1] = P - 1
    return q, pk, pv, pt, ids


def test_noalloc_matches_workspace_entry_two_calls(dev):
    """Call 1 (B=16) then call 2 (B=3, fewer splits) on the no-alloc entry:
    each output equals la_sparse_attention's on the same input bit for bit
    (same kernels, same split plan), and the second call is not disturbed by
    the partials the first left in the shared scratch."""
    results = []
    for B, T, n_list in ((16, 16384, 96), (3, 4096, 20)):
        q, pk, pv, pt, ids = paged_case(B, 32, 8, T, 128, 64, n_list, seed=B, dev=dev)
        kw = dict(unit=64, causal=True, offset=T - 1, page_table=pt, page_size=64,
                  out_dtype=torch.float32)
        out_na = torch.empty(B, 32, 1, 128, dtype=torch.float32, device=dev)
        sparse_attention(q, pk, pv, ids, out=out_na, no_alloc=True, **kw)
        ref = sparse_attention(q, pk, pv, ids, **kw)
        torch.cuda.synchronize()
        results.append((out_na, ref))
    for out_na, ref in results:
        assert torch.isfinite(ref).all()
        assert torch.equal(out_na, ref)


def test_noalloc_rejects_partials_beyond_the_scratch(dev):
    """A split plan whose partials exceed LA_NOALLOC_MAX_WORKSPACE fails with
    a clear error before anything is launched; the workspace entry runs it."""
    B, T = 64, 8192
    q, pk, pv, pt, ids = paged_case(B, 32, 8, T, 128, 64, 64, seed=5, dev=dev)
    kw = dict(unit=64, causal=True, offset=T - 1, page_table=pt, page_size=64, num_splits=64)
    need = B * 8 * 4 * 64 * (128 + 2) * 4
    assert need > N.NOALLOC_MAX_WORKSPACE
    with pytest.raises(RuntimeError, match="static scratch"):
        sparse_attention(q, pk, pv, ids, no_alloc=True, **kw)
    out = sparse_attention(q, pk, pv, ids, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
