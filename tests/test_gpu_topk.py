"""The row top-k kernel alone against the oracle's ranking (value desc, index
asc), on rows built to stress it: heavy exact ties, short valid prefixes, and
rows longer than one workgroup's LDS (the multi-workgroup radix select)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from linattn_amd import _native as N
from linattn_amd.kernels.quest_pages import _topk

pytestmark = pytest.mark.gpu


def run(scores, k, *, pos_offset=0, pos_unit=0):
    B, H, Tq, n = scores.shape
    ids, counts, vals = _topk(scores, k=k, width=k, group=1, order=0, pos_offset=pos_offset,
                              pos_unit=pos_unit, force_own=False, with_values=True)
    return ids, vals


@pytest.mark.parametrize("n,k", [(1000, 100), (8192, 2048), (40000, 3000), (131072, 4096)])
def test_topk_ties_and_prefixes(dev, n, k):
    g = torch.Generator().manual_seed(n)
    # integer-valued scores: ~n/7 exact ties per value
    sc = torch.randint(-3, 4, (1, 1, 3, n), generator=g).double()
    sc[0, 0, 1] = torch.randn(n, generator=g, dtype=torch.float64)  # a tie-free row
    sc[0, 0, 2, ::3] = 0.0
    pos_offset = n - 2  # rows t = 0, 1, 2 see n - 1, n, n keys (causal prefix)
    ids, vals = run(sc.to(dev), k, pos_offset=pos_offset, pos_unit=1)
    nv = np.minimum(n, np.arange(3) + pos_offset + 1)
    ri, rv = oracle.topk_rows(sc[0, 0].numpy(), k, n_valid=nv)
    assert np.array_equal(ids[0, 0].cpu().numpy(), ri)
    assert np.array_equal(vals[0, 0].cpu().numpy(), rv.astype(np.float32))


@pytest.mark.parametrize("order", [1, 0])
def test_topk_wide_many_batches_short_prefixes(dev, order):
    """The multi-workgroup radix select over many rows (300 rows of 65536
    keys in one call), with valid prefixes shorter than k, equal to k and in
    between; ascending-index (order 1) and sorted (order 0) output.  The
    device status stays clean."""
    n, k, Tq = 65536, 3000, 300
    g = torch.Generator().manual_seed(11)
    sc = torch.randint(-50, 50, (1, 1, Tq, n), generator=g).double()
    sc[0, 0, ::3] = torch.randn(Tq // 3, n, generator=g, dtype=torch.float64)
    nv = torch.randint(k, n + 1, (Tq,), generator=g).to(torch.int32)
    nv[:6] = torch.tensor([1, 100, k - 1, k, k + 1, 2 * k], dtype=torch.int32)
    N.device_status(dev)
    ids, counts, _ = _topk(sc.to(dev), k=k, width=k, group=1, order=order, pos_offset=0,
                           pos_unit=0, force_own=False, n_valid=nv.to(dev))
    assert N.device_status(dev) == 0
    ri, _ = oracle.topk_rows(sc[0, 0].numpy(), k, n_valid=nv.numpy())
    want = ri if order == 0 else np.sort(np.where(ri < 0, n, ri), axis=-1)
    if order == 1:
        want = np.where(want == n, -1, want)
    assert np.array_equal(ids[0, 0].cpu().numpy(), want)
    assert np.array_equal(counts[0, 0].cpu().numpy(), np.minimum(nv.numpy(), k))


@pytest.mark.parametrize("order", [1, 0])
def test_topk_radix_long_rows_every_depth(dev, order):
    """Long rows of the multi-workgroup radix select (200000 keys, 49 chunks):
    a row of equal keys (every digit pass runs, then index ties), a row of
    keys equal above their lowest bits, a row whose valid prefix is shorter
    than k (everything taken), an empty row, an ordinary row, and a row whose
    keys share their leading 28 bits (the three chunk-parallel digits: 11, 6
    and 11 bits) and spread over the next digit's 2048 values (too many to
    collect: the one-workgroup finish runs, exact ties remain).  The device
    status stays clean, and a second call on the same scores gives the same
    result (the per-call state starts from scratch)."""
    n, k = 200000, 5000
    g = torch.Generator().manual_seed(13)
    sc = torch.randn(1, 1, 6, n, generator=g, dtype=torch.float64)
    sc[0, 0, 0] = 0.75
    sc[0, 0, 1] = 1.5 + torch.randint(0, 4, (n,), generator=g).double() * 2.0 ** -51
    sc[0, 0, 5] = 1.5 + torch.randint(0, 2048, (n,), generator=g).double() * 2.0 ** -27
    nv = torch.tensor([n, n, k - 7, 0, n - 3, n], dtype=torch.int32)
    N.device_status(dev)
    for _ in range(2):
        ids, counts, _ = _topk(sc.to(dev), k=k, width=k, group=1, order=order, pos_offset=0,
                               pos_unit=0, force_own=False, n_valid=nv.to(dev))
        assert N.device_status(dev) == 0
        ri, _ = oracle.topk_rows(sc[0, 0].numpy(), k, n_valid=nv.numpy())
        want = ri if order == 0 else np.sort(np.where(ri < 0, n, ri), axis=-1)
        if order == 1:
            want = np.where(want == n, -1, want)
        assert np.array_equal(ids[0, 0].cpu().numpy(), want)
        assert np.array_equal(counts[0, 0].cpu().numpy(), np.minimum(nv.numpy(), k))


@pytest.mark.parametrize("order", [1, 0])
def test_topk_radix_candidates(dev, order):
    """Long rows whose keys matching the threshold prefix are few enough to
    collect (at most 4096): every workgroup of the row then settles the
    remaining digits from the collected keys alone (each wave on its own up
    to 1024 keys, the whole workgroup above).  Valid prefixes of 3000 and
    4096 keys (collected before any pass), 4097 (one pass first), 1024 and
    1025; 4096 keys in one first-digit bin above small noise, over 8 values
    (the settle runs down to the last bit, then index ties), 4097 such keys
    (too many: the chunk-parallel passes and the one-workgroup finish) and
    1020 (the wave settle, ties); 4096 distinct keys in that bin; a row of
    negative keys."""
    n, k = 200000, 1000
    g = torch.Generator().manual_seed(17)
    sc = torch.randn(1, 1, 10, n, generator=g, dtype=torch.float64)
    for r, (m, vals) in {3: (4096, 8), 4: (4097, 8), 5: (4096, None), 9: (1020, 8)}.items():
        sc[0, 0, r] *= 0.01  # below 0.5: outside the [2, 8) bin of the first digit
        pos = torch.randperm(n, generator=g)[:m]
        if vals is None:
            sc[0, 0, r, pos] = 3.0 + torch.randperm(m, generator=g).double() * 2.0 ** -30
        else:
            sc[0, 0, r, pos] = 3.0 + torch.randint(0, vals, (m,), generator=g).double() * 2.0 ** -40
    sc[0, 0, 6] = -1.0 - sc[0, 0, 6].abs()
    nv = torch.tensor([3000, 4096, 4097, n, n, n, n, 1024, 1025, n], dtype=torch.int32)
    N.device_status(dev)
    for _ in range(2):
        ids, counts, _ = _topk(sc.to(dev), k=k, width=k, group=1, order=order, pos_offset=0,
                               pos_unit=0, force_own=False, n_valid=nv.to(dev))
        assert N.device_status(dev) == 0
        ri, _ = oracle.topk_rows(sc[0, 0].numpy(), k, n_valid=nv.numpy())
        want = ri if order == 0 else np.sort(ri, axis=-1)
        assert np.array_equal(ids[0, 0].cpu().numpy(), want)
        assert np.array_equal(counts[0, 0].cpu().numpy(), np.minimum(nv.numpy(), k))


def test_topk_short_rows_pad(dev):
    sc = torch.randn(1, 2, 5, 300, dtype=torch.float64)
    ids, vals = run(sc.to(dev), 64, pos_offset=0, pos_unit=8)  # t visible units: t//8 + 1
    for h in range(2):
        ri, rv = oracle.topk_rows(sc[0, h].numpy(), 64, n_valid=np.arange(5) // 8 + 1)
        assert np.array_equal(ids[0, h].cpu().numpy(), ri)
    assert (ids[0, :, :, 1:] == -1).all()


def test_topk_sorted_keys_differing_in_low_bits(dev):
    """Scores that differ only in their lowest mantissa bits (the sorted form
    first orders truncated keys, then must detect and repair the order)."""
    g = torch.Generator().manual_seed(7)
    n = 3000
    base = torch.full((1, 1, 2, n), 1.5, dtype=torch.float64)
    steps = torch.randperm(n, generator=g).to(torch.float64)
    sc = base + steps * 2.0 ** -51  # ulps apart: equal above the low 13 bits
    sc[0, 0, 1] = torch.randn(n, generator=g, dtype=torch.float64)  # an ordinary row
    ids, vals = run(sc.to(dev), 700)
    ri, rv = oracle.topk_rows(sc[0, 0].numpy(), 700)
    assert np.array_equal(ids[0, 0].cpu().numpy(), ri)
    assert np.array_equal(vals[0, 0].cpu().numpy(), rv.astype(np.float32))


def _check_values(got, want64):
    """fp32 values of the selection against the oracle's fp64 scores: equal
    to the rounded score where it is an fp32 number, and +-inf with the
    score's sign where it lies beyond the fp32 range (the far outliers of
    the spread rows); -inf padding where the oracle pads."""
    got = np.asarray(got)
    big = np.isfinite(want64) & (np.abs(want64) > np.finfo(np.float32).max)
    finite = np.isfinite(want64) & ~big
    with np.errstate(over="ignore"):
        want32 = want64.astype(np.float32)
    assert np.array_equal(got[finite], want32[finite])
    assert np.array_equal(got[big], np.where(want64[big] > 0, np.inf, -np.inf).astype(np.float32))
    pad = ~np.isfinite(want64)
    assert np.array_equal(got[pad], want32[pad])
    return int(big.sum())


def _spread_rows(n, seed):
    """Rows for the sorted form's bucket ranking: ReLU sums with exact zeros
    (ties at the minimum), both signs, far outliers, scores over many
    binades and few distinct values."""
    g = torch.Generator().manual_seed(seed)
    relu = (torch.randn(n, 4, generator=g, dtype=torch.float64).clamp(min=0)
            * torch.rand(4, generator=g, dtype=torch.float64)).sum(1)
    rows = [relu, relu.clone(), torch.randn(n, generator=g, dtype=torch.float64) * 3.0,
            torch.randn(n, generator=g, dtype=torch.float64),
            torch.exp(torch.randn(n, generator=g, dtype=torch.float64) * 20.0),
            torch.randint(0, 5, (n,), generator=g).double() * 0.5]
    rows[3][17], rows[3][n // 2] = 1e300, -1e300
    return torch.stack(rows).view(1, 1, len(rows), n)


@pytest.mark.parametrize("n,k", [(8192, 2048), (5000, 4096), (3000, 512)])
def test_topk_sorted_bucket_rank_rows(dev, n, k):
    """Sorted selections whose survivors stress the bucket ranking: ties at
    the minimum, mixed signs, far outliers (the bitonic fallback), many
    binades; prefixes shorter and longer than k."""
    sc = _spread_rows(n, n + k)
    Tq = sc.shape[2]
    nv = torch.tensor([n, k + 60, n, n, n, n - 1], dtype=torch.int32)[:Tq]
    ids, counts, vals = _topk(sc.to(dev), k=k, width=k, group=1, order=0, pos_offset=0,
                              pos_unit=0, force_own=False, with_values=True,
                              n_valid=nv.to(dev))
    ri, rv = oracle.topk_rows(sc[0, 0].numpy(), k, n_valid=nv.numpy())
    assert np.array_equal(ids[0, 0].cpu().numpy(), ri)
    assert _check_values(vals[0, 0].cpu().numpy(), rv) >= 1  # row 3's 1e300 is selected
    assert np.array_equal(counts[0, 0].cpu().numpy(), np.minimum(k, nv.numpy()))


def test_topk_sorted_forced_own(dev):
    """A forced own unit ranks first (value +inf) above every bucket."""
    n, k = 6000, 1024
    sc = _spread_rows(n, 3)
    Tq = sc.shape[2]
    pos_offset = n - Tq - 500  # rows see n - Tq - 499 + t keys; own = the last visible
    ids, counts, vals = _topk(sc.to(dev), k=k, width=k, group=1, order=0,
                              pos_offset=pos_offset, pos_unit=1, force_own=True,
                              with_values=True)
    t = np.arange(Tq)
    nv = np.minimum(n, pos_offset + t + 1)
    ri, rv = oracle.topk_rows(sc[0, 0].numpy(), k, n_valid=nv, own=nv - 1, force_own=True)
    assert np.array_equal(ids[0, 0].cpu().numpy(), ri)
    assert (ids[0, 0, :, 0].cpu().numpy() == nv - 1).all()
    assert _check_values(vals[0, 0, :, 1:].cpu().numpy(), rv[:, 1:]) >= 1


@pytest.mark.parametrize("n,group", [(60, 1), (500, 2), (1024, 4), (3000, 2)])
def test_topk_union_sink_window(dev, n, group):
    """Bitmap form (one wave per row for short rows, register form for long):
    per-head top-k with the own unit forced, union over the group, sink and
    window units added, ascending order, -1 padded, counts."""
    g = torch.Generator().manual_seed(n + group)
    Tq, k, sink, window, unit = 5, 7, 2, 3, 16
    sc = torch.randint(-4, 5, (1, 2 * group, Tq, n), generator=g).double()
    pos_offset = n * unit - Tq - 40  # queries see all but the last few units
    width = group * k + sink + window
    ids, counts, _ = _topk(sc.to(dev), k=k, width=width, group=group, order=1,
                           pos_offset=pos_offset, pos_unit=unit, force_own=True, sink=sink,
                           window=window)
    for hg in range(2):
        for t in range(Tq):
            pos = pos_offset + t
            own = min(pos // unit, n - 1)
            n_v = min(n, pos // unit + 1)
            keep = set()
            for j in range(group):
                row = sc[0, hg * group + j, t].numpy()
                ri, _ = oracle.topk_rows(row, min(k, n_v), n_valid=n_v, own=own, force_own=True)
                keep.update(int(x) for x in ri if x >= 0)
            keep.update(range(min(sink, n_v)))
            keep.update(range(max(0, own - window + 1), own + 1))
            want = sorted(keep)[:width]
            got = ids[0, hg, t].cpu().numpy()
            assert list(got[:len(want)]) == want and (got[len(want):] == -1).all(), (hg, t)
            assert int(counts[0, hg, t]) == len(want)


def test_radix_waits_give_up_when_forced(dev):
    """The bounded waits between workgroups (a chunk's look-back over the
    row's earlier chunks in the multi-workgroup top-k, the decode indexer's
    wait for a row's first workgroup) are forced to give up at once through
    the testing hook (a limit of 0 polls): every kernel still ends,
    LA_DEV_TOPK_TIMEOUT is raised, and with the default limit restored the
    same calls return the oracle's selection with a clean status."""
    from linattn_amd.kernels.fused_indexer import indexer_topk

    lib = N.load()
    n, k = 200000, 5000
    g = torch.Generator().manual_seed(23)
    sc = torch.randn(1, 1, 3, n, generator=g, dtype=torch.float64)
    nv = torch.tensor([n, 3000, n - 5], dtype=torch.int32)
    q = torch.randn(1, 1, 4, 64, generator=g).bfloat16()
    kk = torch.randn(1, 70000, 4, 64, generator=g).bfloat16()
    w = torch.rand(1, 1, 4, generator=g)

    def run_topk():
        return _topk(sc.to(dev), k=k, width=k, group=1, order=1, pos_offset=0, pos_unit=0,
                     force_own=False, n_valid=nv.to(dev))

    def run_indexer():
        return indexer_topk(q.to(dev), kk.to(dev), w.to(dev), 4096, sorted=False)

    N.device_status(dev)
    try:
        assert lib.la_test_set_spin_limit(0) == N.LA_OK
        run_topk()
        assert N.device_status(dev) & N.LA_DEV_TOPK_TIMEOUT
        run_indexer()
        assert N.device_status(dev) & N.LA_DEV_TOPK_TIMEOUT
    finally:
        lib.la_test_set_spin_limit(1 << 20)
    ids, counts, _ = run_topk()
    assert N.device_status(dev) == 0
    ri, _ = oracle.topk_rows(sc[0, 0].numpy(), k, n_valid=nv.numpy())
    want = np.sort(np.where(ri < 0, n, ri), axis=-1)
    assert np.array_equal(ids[0, 0].cpu().numpy(), np.where(want == n, -1, want))
    _, idx = run_indexer()
    assert N.device_status(dev) == 0
    _, r2 = oracle.indexer_topk(q, kk, w, 4096)
    want2 = np.sort(r2.reshape(-1))
    assert np.array_equal(idx.cpu().numpy().reshape(-1), want2)
