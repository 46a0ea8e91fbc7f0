"""GPU parity of config C3: block selection (bit-exact lists) and the MFMA
block-sparse causal prefill (within 2e-3 of the fp64 oracle, fp32 output)."""

from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
from linattn_amd import _native as N
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


@pytest.mark.parametrize("causal", [False, True])
def test_prefill_multiset_lists_with_holes(dev, causal):
    """Hand-made lists: unsorted, one block listed twice (attended twice, as
    the reference's gather does, block_sparse.py:62-68), -1 holes between
    entries, a partial last key block (T = 300), and future blocks (read whole
    without the causal mask, cut by it with the mask; the diagonal block is
    always listed so every row sees its own token)."""
    T, hq, hkv = 300, 4, 2
    q, k, v = c3_inputs(1, hq, hkv, T, 128, seed=7)
    nqb, W = 5, 7
    g = np.random.default_rng(7)
    ids = np.full((1, hq, nqb, W), -1, dtype=np.int32)
    for h in range(hq):
        for qb in range(nqb):
            picks = list(g.choice(nqb, size=3, replace=False))
            lst = [qb, picks[0], picks[1], picks[0], -1, picks[2], -1]
            g.shuffle(lst)
            ids[0, h, qb] = lst
    out = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(ids).to(dev),
                               causal=causal, out_dtype=torch.float32)
    torch.cuda.synchronize()
    G = hq // hkv
    for h in range(hq):
        for qb in range(nqb):
            t0, t1 = qb * 64, min(T, (qb + 1) * 64)
            rows = np.broadcast_to(ids[0, h, qb], (1, 1, t1 - t0, W))
            ref = oracle.attend_lists(q[:, h:h + 1, t0:t1], k[:, h // G:h // G + 1],
                                      v[:, h // G:h // G + 1], rows, unit=64, causal=causal,
                                      offset=t0)
            got = out[0, h, t0:t1].cpu().double().numpy()
            assert np.abs(got - ref[0, 0]).max() < 2e-3, (h, qb)


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_long_lists(dev, causal):
    """Lists of 64, 65 and 100 entries: the kernel keeps lists of up to 64
    entries in VGPR lanes and reads longer ones through the scalar cache, so
    both paths and the 64/65 boundary run.  Causal: every block up to the
    diagonal (query blocks 63, 64 and 99); non-causal: seeded multisets of
    any blocks, -1 padded.  Within 2e-3 of the fp64 oracle."""
    T, hq, hkv, W = 6400, 2, 1, 100
    q, k, v = c3_inputs(1, hq, hkv, T, 128, seed=9)
    nqb = T // 64
    ids = np.full((1, hq, nqb, W), -1, dtype=np.int32)
    g = np.random.default_rng(9)
    check = {63: 64, 64: 65, 99: 100}
    for h in range(hq):
        for qb in range(nqb):
            if causal:
                n = qb + 1
                ids[0, h, qb, :n] = np.arange(n)
            else:
                n = check.get(qb, int(g.integers(1, W + 1)))
                ids[0, h, qb, :n] = g.integers(0, nqb, size=n)
    out = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(ids).to(dev),
                               causal=causal, out_dtype=torch.float32)
    torch.cuda.synchronize()
    for h in range(hq):
        for qb, n in check.items():
            assert (ids[0, h, qb] >= 0).sum() == n
            t0 = qb * 64
            rows = np.broadcast_to(ids[0, h, qb], (1, 1, 64, W))
            ref = oracle.attend_lists(q[:, h:h + 1, t0:t0 + 64], k, v, rows, unit=64,
                                      causal=causal, offset=t0)
            got = out[0, h, t0:t0 + 64].cpu().double().numpy()
            assert np.abs(got - ref[0, 0]).max() < 2e-3, (h, qb)


def test_prefill_empty_list_gives_zeros(dev):
    q, k, v = c3_inputs(1, 1, 1, 128, 128, seed=4, outliers=False)
    ids = torch.full((1, 1, 2, 3), -1, dtype=torch.int32)
    out = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), ids.to(dev),
                               out_dtype=torch.float32)
    assert torch.count_nonzero(out) == 0


def test_config3_full_size(dev):
    """C3: B=2, T=32768, 32/8 heads, D=128, 64x64 blocks, sink + 4-block window
    + top-16.  The lists of all 64 (b, head) pairs are checked bit for bit
    against the oracle (one pair per thread); output rows of five query blocks
    of two heads against the fp64 oracle."""
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
    ids_h, q_h, k_h = ids.cpu().numpy(), q.cpu(), k.cpu()

    def lists_equal(bh):
        b, h = divmod(bh, Hq)
        kvh = h // (Hq // Hkv)
        ref = oracle.block_select(q_h[b:b + 1, h:h + 1], k_h[b:b + 1, kvh:kvh + 1], block=64,
                                  topk=16, sink_blocks=1, window_blocks=4)
        return bh, np.array_equal(ids_h[b:b + 1, h:h + 1], ref)

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4)) as ex:
        res = list(ex.map(lists_equal, range(B * Hq)))
    assert all(ok for _, ok in res), [bh for bh, ok in res if not ok]
    for b, h in ((0, 0), (1, 13)):
        kvh = h // (Hq // Hkv)
        qc, kc, vc = q[b:b + 1, h:h + 1].cpu(), k[b:b + 1, kvh:kvh + 1].cpu(), \
            v[b:b + 1, kvh:kvh + 1].cpu()
        ids_c, counts_c = ids[b:b + 1, h:h + 1].cpu(), counts[b:b + 1, h:h + 1].cpu()
        rows = oracle_rows(qc, kc, vc, ids_c, counts_c, 0, 0, (0, 1, 17, 300, nqb - 1))
        for qb, r in rows.items():
            got = out[b, h, qb * 64:(qb + 1) * 64].cpu().double().numpy()
            assert np.abs(got - r).max() < 2e-3, (b, h, qb)


def fp64_block_attention(q, k, v, ids, counts, chunk=256):
    """fp64 attention of every (b, h, query block) over its listed 64-key
    blocks with the causal mask, on the device (torch fp64 matmuls over the
    gathered blocks), as (B, Hq, T, D)."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G, nqb, W = Hq // Hkv, ids.shape[2], ids.shape[3]
    dev = q.device
    out = torch.zeros(B, Hq, T, D, dtype=torch.float64, device=dev)
    flat_ids = ids.reshape(-1, W).long()
    flat_cnt = counts.reshape(-1).long()
    ar64 = torch.arange(64, device=dev)
    for s0 in range(0, B * Hq * nqb, chunk):
        i = torch.arange(s0, min(s0 + chunk, B * Hq * nqb), device=dev)
        b, h, qb = i // (Hq * nqb), (i // nqb) % Hq, i % nqb
        lst = flat_ids[i]
        ok = (lst >= 0) & (torch.arange(W, device=dev)[None, :] < flat_cnt[i][:, None])
        tok = (lst.clamp(min=0)[:, :, None] * 64 + ar64).reshape(len(i), -1)
        tok_ok = ok[:, :, None].expand(-1, -1, 64).reshape(len(i), -1) & (tok < T)
        tok = tok.clamp(max=T - 1)
        qrow = (qb[:, None] * 64 + ar64).clamp(max=T - 1)
        qg = q[b[:, None], h[:, None], qrow].double()
        kg = k[b[:, None], (h // G)[:, None], tok].double()
        vg = v[b[:, None], (h // G)[:, None], tok].double()
        sc = torch.bmm(qg, kg.transpose(1, 2).contiguous()) / math.sqrt(D)
        allow = tok_ok[:, None, :] & (tok[:, None, :] <= qrow[:, :, None])
        sc = sc.masked_fill(~allow, float("-inf"))
        o = torch.bmm(torch.softmax(sc, dim=-1), vg)
        rows = qb[:, None] * 64 + ar64
        keep = rows < T
        out[b[:, None].expand_as(rows)[keep], h[:, None].expand_as(rows)[keep], rows[keep]] = o[keep]
    return out


def test_config3_every_row_within_tolerance(dev):
    """C3 at full size (2 x 32 x 32768 query rows): every output row of the
    fp32-output prefill within 2e-3 of fp64 attention over its lists; the
    bf16 output within bf16 rounding of it."""
    B, Hq, Hkv, T, D = 2, 32, 8, 32768, 128
    q, k, v = c3_inputs(B, Hq, Hkv, T, D, seed=0, device=dev)
    out, ids, counts = sparse_prefill(q, k, v, topk=16, sink_blocks=1, window_blocks=4,
                                      out_dtype=torch.float32)
    ref = fp64_block_attention(q, k, v, ids, counts)
    err = (out.double() - ref).abs()
    assert err.max().item() < 2e-3, err.max().item()
    out_b = block_sparse_prefill(q, k, v, ids, counts)
    assert out_b.dtype == torch.bfloat16
    assert ((out_b.double() - ref).abs() <= ref.abs() * 2.0 ** -8 + 2e-3).all()


def test_prefill_large_v_blocks(dev):
    """V blocks whose values reach 2^15..2^22 are converted to fp16 with a
    power-of-two block exponent (folded back into the weights): outputs stay
    within 2e-3 relative to the value scale.  A finite |v| >= 2^22 raises
    ValueError (its fp16 copy would overflow); with check_range=False the
    rows come out inf and LA_DEV_PREFILL_RANGE is raised on the device."""
    q, k, v = c3_inputs(1, 4, 2, 512, 128, seed=6, outliers=False)
    v = v.float()
    v[0, 0, 128:192] *= 2.0 ** 18   # block 2 of KV head 0: e = 5 or 6
    v[0, 1, 448:512] *= 2.0 ** 19   # block 7 of KV head 1 (|v| < 2^22): e = 6 or 7
    v = v.bfloat16()
    nqb = 8
    ids = torch.full((1, 4, nqb, nqb), -1, dtype=torch.int32)
    for i in range(nqb):
        ids[:, :, i, :i + 1] = torch.arange(i + 1, dtype=torch.int32)
    N.device_status(dev)
    out = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), ids.to(dev),
                               out_dtype=torch.float32)
    assert N.device_status(dev) == 0
    ref = oracle.dense_attention(q, k, v)
    scale = np.abs(v.double().numpy()).max(axis=(2, 3))[:, np.repeat(np.arange(2), 2)]
    err = np.abs(out.cpu().double().numpy() - ref).max(axis=(2, 3))
    assert (err < 2e-3 * np.maximum(scale, 1.0)).all(), (err, scale)
    # a finite value beyond the fp16 range of its scaled block is an error
    v2 = v.clone()
    v2[0, 0, 5, 3] = 2.0 ** 23
    with pytest.raises(ValueError):
        block_sparse_prefill(q.to(dev), k.to(dev), v2.to(dev), ids.to(dev),
                             out_dtype=torch.float32)
    assert N.device_status(dev) == 0  # the error consumed the status bit
    out2 = block_sparse_prefill(q.to(dev), k.to(dev), v2.to(dev), ids.to(dev),
                                out_dtype=torch.float32, check_range=False)
    assert N.device_status(dev) & N.LA_DEV_PREFILL_RANGE
    assert not torch.isfinite(out2[0, :2]).all()


def test_prefill_small_v_blocks_keep_relative_precision(dev):
    """V blocks of small magnitude (|v| ~ 2^-18, below the fp16 normal range)
    are scaled up by their block exponent (by up to 2^8): outputs keep 2e-3
    relative precision, not only absolute."""
    q, k, v = c3_inputs(1, 2, 1, 256, 128, seed=8, outliers=False)
    v = (v.float() * 2.0 ** -20).bfloat16()
    nqb = 4
    ids = torch.full((1, 2, nqb, nqb), -1, dtype=torch.int32)
    for i in range(nqb):
        ids[:, :, i, :i + 1] = torch.arange(i + 1, dtype=torch.int32)
    out = block_sparse_prefill(q.to(dev), k.to(dev), v.to(dev), ids.to(dev),
                               out_dtype=torch.float32)
    ref = oracle.dense_attention(q, k, v)
    scale = float(np.abs(v.double().numpy()).max())
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-3 * scale


def test_ragged_batch_equals_one_call_per_sequence(dev):
    """A ragged batch (lengths 1000, 517, 64 and 0, padded to 1000) gives, for
    each sequence, the lists and outputs of a call on that sequence alone; its
    query blocks past the end get empty lists and its padding rows come out
    as zeros.  Padding rows hold NaN: reading any of them would show."""
    Tm, hq, hkv = 1000, 4, 2
    lens = [1000, 517, 64, 0]
    B = len(lens)
    q, k, v = c3_inputs(B, hq, hkv, Tm, 128, seed=11)
    for b, L in enumerate(lens):
        q[b, :, L:] = float("nan")
        k[b, :, L:] = float("nan")
        v[b, :, L:] = float("nan")
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    lengths = torch.tensor(lens, dtype=torch.int32, device=dev)
    kw = dict(topk=3, sink_blocks=1, window_blocks=2)
    out, ids, counts = sparse_prefill(q, k, v, out_dtype=torch.float32, lengths=lengths, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    nqb = (Tm + 63) // 64
    for b, L in enumerate(lens):
        nb = (L + 63) // 64
        assert (counts[b, :, nb:] == 0).all() and (ids[b, :, nb:] == -1).all()
        assert (out[b, :, L:] == 0).all()
        if L == 0:
            continue
        o1, i1, c1 = sparse_prefill(q[b:b + 1, :, :L], k[b:b + 1, :, :L], v[b:b + 1, :, :L],
                                    out_dtype=torch.float32, **kw)
        assert torch.equal(ids[b:b + 1, :, :nb], i1), b
        assert torch.equal(counts[b:b + 1, :, :nb], c1), b
        assert torch.equal(out[b:b + 1, :, :L], o1), b
    # the lists of the full-length sequence also match the CPU oracle
    ref = oracle.block_select(q[:1].cpu(), k[:1].cpu(), block=64, **kw)
    assert np.array_equal(ids[:1].cpu().numpy(), ref)
    assert nqb == ids.shape[2]


@pytest.mark.parametrize("T,hq,hkv", [(1000, 4, 2), (512, 8, 8)])
def test_prefill_fp8_kv_matches_dequantised_oracle(dev, T, hq, hkv):
    """fp8 e4m3 K/V with per-token scales (kv/quant.py:76-109): the prefill
    equals fp64 attention over the dequantised cache (codes times scales, the
    oracle's fp8 reader) within 2e-3, inside the 1e-2 fp8 gate of the north
    star.  The K codes are scored on the fp8 matrix cores against q as a
    two-term fp8 expansion per query row with a power-of-two scale (which
    holds a bf16 q exactly), each score times its key's scale; V is
    dequantised into fp16."""
    from linattn_amd.kernels.paged_decode import quantize_fp8_per_token
    q, k, v = c3_inputs(1, hq, hkv, T, 128, seed=21)
    kc, ks = quantize_fp8_per_token(k.float())
    vc, vs = quantize_fp8_per_token(v.float())
    ids, counts = block_select_hip(q.to(dev), k.to(dev), block=64, topk=4, sink_blocks=1,
                                   window_blocks=2)
    out = block_sparse_prefill(q.to(dev), kc.to(dev), vc.to(dev), ids, counts,
                               out_dtype=torch.float32, k_scale=ks.to(dev), v_scale=vs.to(dev))
    torch.cuda.synchronize()
    nqb = (T + 63) // 64
    ids_c, counts_c = ids.cpu(), counts.cpu()
    for h in range(hq):
        for qb in range(nqb):
            t0, t1 = qb * 64, min(T, (qb + 1) * 64)
            lst = ids_c[0, h, qb, :counts_c[0, h, qb]].numpy()
            rows = np.broadcast_to(lst, (1, 1, t1 - t0, len(lst)))
            kvh = h // (hq // hkv)
            ref = oracle.attend_lists(q[:, h:h + 1, t0:t1], kc[:, kvh:kvh + 1], vc[:, kvh:kvh + 1],
                                      rows, unit=64, causal=True, offset=t0,
                                      k_scale=ks[:, kvh:kvh + 1], v_scale=vs[:, kvh:kvh + 1])
            got = out[0, h, t0:t1].cpu().double().numpy()
            assert np.abs(got - ref[0, 0]).max() < 2e-3, (h, qb)


def test_prefill_fp8_ragged_equals_per_sequence(dev):
    """fp8 K/V and a ragged batch together: each sequence as if alone."""
    from linattn_amd.kernels.paged_decode import quantize_fp8_per_token
    Tm, lens = 640, [640, 300]
    q, k, v = c3_inputs(2, 4, 2, Tm, 128, seed=22)
    kc, ks = quantize_fp8_per_token(k.float())
    vc, vs = quantize_fp8_per_token(v.float())
    q, kc, vc, ks, vs = q.to(dev), kc.to(dev), vc.to(dev), ks.to(dev), vs.to(dev)
    lengths = torch.tensor(lens, dtype=torch.int32, device=dev)
    ids, counts = block_select_hip(q, k.to(dev), topk=3, sink_blocks=1, window_blocks=2,
                                   lengths=lengths)
    out = block_sparse_prefill(q, kc, vc, ids, counts, out_dtype=torch.float32, lengths=lengths,
                               k_scale=ks, v_scale=vs)
    for b, L in enumerate(lens):
        nb = (L + 63) // 64
        o1 = block_sparse_prefill(q[b:b + 1, :, :L], kc[b:b + 1, :, :L], vc[b:b + 1, :, :L],
                                  ids[b:b + 1, :, :nb].contiguous(), counts[b:b + 1, :, :nb],
                                  out_dtype=torch.float32, k_scale=ks[b:b + 1, :, :L],
                                  v_scale=vs[b:b + 1, :, :L])
        assert torch.equal(out[b:b + 1, :, :L], o1), b
        assert (out[b, :, L:] == 0).all()
