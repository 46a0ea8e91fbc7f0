"""GPU parity of the lightning-indexer top-k (config C2 and the decode form
used by config C5) against the CPU oracle: indices bit-exact, values equal to
the oracle's fp64 scores rounded to fp32."""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
from linattn_amd.kernels.fused_indexer import indexer_topk

pytestmark = pytest.mark.gpu


def inputs(b, tq, tk, hi, d, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, tq, hi, d, generator=g).to(dtype)
    k = torch.randn(b, tk, hi, d, generator=g).to(dtype)
    w = torch.rand(b, tq, hi, generator=g)
    return q, k, w


def check(q, k, w, kk, dev, *, causal=False, offset=0, q_chunk=0):
    val, idx = indexer_topk(q.to(dev), k.to(dev), w.to(dev), kk, causal=causal, offset=offset,
                            q_chunk=q_chunk)
    rv, ri = oracle.indexer_topk(q, k, w, min(kk, k.shape[1]), causal=causal, offset=offset)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert np.array_equal(val.cpu().numpy(), rv.astype(np.float32))
    return idx


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_indexer_small_noncausal(dev, dtype):
    """fused_indexer.py:52-73 semantics (no causal mask), k < Tk."""
    q, k, w = inputs(2, 37, 300, 3, 16, seed=1, dtype=dtype)
    check(q, k, w, 50, dev)


def test_indexer_k_clipped_to_tk(dev):
    q, k, w = inputs(1, 9, 20, 2, 8, seed=2)
    val, idx = indexer_topk(q.to(dev), k.to(dev), w.to(dev), 64)
    assert idx.shape == (1, 9, 20)
    assert (np.sort(idx.cpu().numpy(), -1) == np.arange(20)).all()


@pytest.mark.parametrize("chunk", [0, 64, 100])
def test_indexer_causal_ties_and_padding(dev, chunk):
    """Causal rows with fewer valid keys than k are -1 padded; ReLU zeros tie
    and go to the lowest indices."""
    q, k, w = inputs(1, 200, 200, 4, 64, seed=3, dtype=torch.bfloat16)
    idx = check(q, k, w, 96, dev, causal=True, offset=0, q_chunk=chunk)
    assert (idx[0, 10, 11:] == -1).all() and (idx[0, 199] >= 0).all()


def test_indexer_causal_with_offset(dev):
    q, k, w = inputs(2, 70, 517, 4, 64, seed=4, dtype=torch.bfloat16)
    check(q, k, w, 128, dev, causal=True, offset=517 - 70)


def index_order(ri):
    """The oracle's (score desc) lists as ascending sets, -1 padded."""
    out = np.full_like(ri, -1)
    for r in np.ndindex(ri.shape[:-1]):
        v = np.sort(ri[r][ri[r] >= 0])
        out[r][:v.size] = v
    return out


@pytest.mark.parametrize("tq,tk,kk,offset", [
    (5, 600, 64, 400),      # short rows: one wave per row
    (3, 9000, 700, 8000),   # register rows
    (2, 70000, 4096, 69000),  # long rows: segmented levels, candidate rows
    (1, 70000, 4096, 3000),   # fewer visible keys than k: -1 padded
])
def test_indexer_index_order(dev, tq, tk, kk, offset):
    """sorted=False: the same selection as ascending sets, no values."""
    q, k, w = inputs(1, tq, tk, 4, 64, seed=11 + tq, dtype=torch.bfloat16)
    val, idx = indexer_topk(q.to(dev), k.to(dev), w.to(dev), kk, causal=True, offset=offset,
                            sorted=False)
    assert val is None
    _, ri = oracle.indexer_topk(q, k, w, kk, causal=True, offset=offset)
    assert np.array_equal(idx.cpu().numpy(), index_order(ri))


@pytest.mark.parametrize("tq", [1, 3])
@pytest.mark.parametrize("hi,d,dtype", [(4, 64, torch.bfloat16), (1, 256, torch.bfloat16),
                                        (2, 128, torch.float16), (8, 32, torch.bfloat16)])
def test_indexer_decode_form(dev, tq, hi, d, dtype):
    """A few queries against a long key axis (the per-key kernel: 2-byte keys,
    hi threads per key)."""
    q, k, w = inputs(3, tq, 5000, hi, d, seed=5 + hi, dtype=dtype)
    check(q, k, w, 512, dev, causal=True, offset=5000 - tq)


@pytest.mark.parametrize("offset,kk,sorted_", [
    (50000, 4096, True),     # causal row, threshold above the ReLU zeros
    (50000, 4096, False),
    (50000, 48000, False),   # threshold among the tied zeros: lowest indices first
    (4200, 4096, True),      # the same, sorted (4201 visible keys, about 260 zeros)
    (None, 4096, True),      # every key visible
    (None, 69990, False),
])
def test_indexer_decode_long_row(dev, offset, kk, sorted_):
    """One query against 70000 keys: the multi-workgroup radix select, with
    the first digit histogrammed by the scores kernel."""
    q, k, w = inputs(2, 1, 70000, 4, 64, seed=31, dtype=torch.bfloat16)
    causal = offset is not None
    if sorted_:
        check(q, k, w, kk, dev, causal=causal, offset=offset or 0)
        return
    val, idx = indexer_topk(q.to(dev), k.to(dev), w.to(dev), kk, causal=causal,
                            offset=offset or 0, sorted=False)
    _, ri = oracle.indexer_topk(q, k, w, kk, causal=causal, offset=offset or 0)
    assert np.array_equal(idx.cpu().numpy(), index_order(ri))


def test_indexer_summation_order_is_sequential(dev):
    """The tiled score kernel adds q.k products over d in increasing order
    (the matrix-core form relies on gfx950's in-order fp64 accumulation).
    Each key row is a shuffle of +-2^60 pairs and small integers, so its
    fp64 sum depends on the order (a small value added to a +-2^60 partial
    sum is absorbed); with q = 1 and w = 1 the score is relu(sum).  The
    ranking of every key and the values equal the oracle's sequential sums;
    an unordered or pairwise sum would change them."""
    r = np.random.default_rng(7)
    Tq, Tk, d = 64, 256, 64
    big = np.ldexp(1.0, 60)
    rows = []
    for _ in range(Tk):
        vals = np.concatenate([[big, -big, big, -big], r.integers(1, 100, size=d - 4)])
        rows.append(r.permutation(vals))
    k = torch.tensor(np.array(rows), dtype=torch.float64).to(torch.bfloat16).view(1, Tk, 1, d)
    q = torch.ones(1, Tq, 1, d, dtype=torch.bfloat16)
    w = torch.ones(1, Tq, 1)
    seq = [0.0] * Tk
    for j, row in enumerate(k[0, :, 0].double().numpy()):
        acc = 0.0
        for x in row:
            acc = acc + x
        seq[j] = max(acc, 0.0)
    assert len(set(seq)) > 20  # the order matters for these rows
    check(q, k, w, Tk, dev)
    val, _ = indexer_topk(q.to(dev), k.to(dev), w.to(dev), Tk)
    want = np.sort(np.array(seq))[::-1].astype(np.float32)
    assert np.array_equal(val[0, 0].cpu().numpy(), want)
    assert np.array_equal(val[0, -1].cpu().numpy(), want)


def limb_rows(n, hi, d, ranges, seed):
    """bf16 rows whose (row, head) exponent range R (largest minus least
    exponent of the non-zero values) is one of `ranges`, cycled over rows and
    heads; -1 gives an all-zero row, -2 a row of subnormals only, -3 a row
    mixing subnormals with values near 1 (R above 120)."""
    r = np.random.default_rng(seed)
    x = np.zeros((n, hi, d))
    for i in range(n):
        for h in range(hi):
            R = ranges[(i * hi + h) % len(ranges)]
            sign = r.choice([-1.0, 1.0], size=d)
            mant = 1.0 + r.integers(0, 128, size=d) / 128.0
            if R == -1:
                continue
            if R == -2:
                x[i, h] = sign * r.integers(1, 128, size=d) * 2.0 ** -133
                continue
            e = r.integers(0, max(R, 0) + 1, size=d)
            e[0], e[-1] = 0, max(R, 0)
            if R == -3:
                e = np.where(r.random(d) < 0.5, 0, 1)
                x[i, h] = sign * mant * np.where(e == 0, 2.0 ** -130, 1.0)
                continue
            x[i, h] = sign * mant * 2.0 ** (e - R // 2 - r.integers(-3, 4))
    return torch.tensor(x, dtype=torch.float64).to(torch.bfloat16).unsqueeze(0)


@pytest.mark.parametrize("hi", [1, 4, 8])
@pytest.mark.parametrize("causal", [False, True])
def test_indexer_limb_exponent_ranges(dev, hi, causal):
    """The integer-limb score path (bf16, d = 64) at every branch of its
    exactness rule, bit for bit against the oracle's sequential fp64 sums:
    16-row blocks whose rows all have R <= 14 (three limbs a side) next to
    blocks of R 15-22 (four limbs), query/key pairs with Rq + Rk <= 30 and
    pairs above it (the sequential sum), rows with R > 22, subnormal rows,
    all-zero rows and mixed signs; rows are ranked in full (k = Tk), so a
    wrong score of any key moves it."""
    Tq, Tk = 160, 192
    narrow = [0, 3, 7, 10, 14]
    wide = [15, 16, 18, 20, 22]
    odd = [23, 30, -1, -2, -3, 14, 9]
    q = torch.cat([limb_rows(64, hi, 64, narrow, seed=11),
                   limb_rows(64, hi, 64, wide + narrow, seed=12),
                   limb_rows(32, hi, 64, odd, seed=13)], dim=1)
    k = torch.cat([limb_rows(64, hi, 64, wide, seed=14),
                   limb_rows(64, hi, 64, narrow, seed=15),
                   limb_rows(64, hi, 64, odd + narrow, seed=16)], dim=1)
    w = torch.rand(1, Tq, hi, generator=torch.Generator().manual_seed(17))
    check(q, k, w, Tk, dev, causal=causal, offset=Tk - Tq if causal else 0)


def test_config2_indexer_full_size(dev):
    """C2: B=1, T=8192, 4 heads of dim 64, bf16 q/k, w ~ U(0,1), causal top-2048,
    int32 indices.  Every one of the 8192 rows against the oracle bit for bit
    (indices and fp32 values), in chunks of 256 query rows on a thread pool
    (the oracle's C scorer releases the GIL)."""
    T, HI, d, kk = 8192, 4, 64, 2048
    q, k, w = inputs(1, T, T, HI, d, seed=0, dtype=torch.bfloat16)
    val, idx = indexer_topk(q.to(dev), k.to(dev), w.to(dev), kk, causal=True)
    torch.cuda.synchronize()
    t = torch.arange(T, device=dev)
    n_valid = torch.clamp(t + 1, max=kk)
    got = (idx[0] >= 0).sum(-1)
    assert torch.equal(got, n_valid)
    idx_h, val_h = idx[0].cpu().numpy(), val[0].cpu().numpy()
    chunk = 256

    def job(t0):
        rv, ri = oracle.indexer_topk(q[:, t0:t0 + chunk], k, w[:, t0:t0 + chunk], kk,
                                     causal=True, offset=t0)
        ok_i = np.array_equal(idx_h[t0:t0 + chunk], ri[0])
        ok_v = np.array_equal(val_h[t0:t0 + chunk], rv[0].astype(np.float32))
        return t0, ok_i, ok_v

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4)) as ex:
        res = list(ex.map(job, range(0, T, chunk)))
    bad = [(t0, oi, ov) for t0, oi, ov in res if not (oi and ov)]
    assert not bad, bad
