"""Pins the CPU oracle before it is trusted as the GPU checker.

Each oracle function is checked against something other than its own formula:
the reference's known-answer tests (cited), closed forms computed by a
different route, brute force on tiny inputs, invariants a plausible mistake
would break, and the reference's own C decode built from its source
(oracle/_ref, built by oracle/Makefile when the reference tree is present).
"""

from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

ROOT = Path(__file__).resolve().parents[1]
REF_LIB = ROOT / "oracle" / "_ref" / "libdecode_attn.so"


def rng(seed=0):
    return np.random.default_rng(seed)


# --------------------------------------------------------------- core ----
def test_dense_matches_manual_softmax():
    """test_reference.py:13-22: the oracle equals an explicit softmax."""
    r = rng(0)
    q, k, v = (r.standard_normal((2, 2, 5, 8)) for _ in range(3))
    out = oracle.dense_attention(q, k, v)
    for b in range(2):
        for h in range(2):
            for i in range(5):
                s = np.array([q[b, h, i] @ k[b, h, j] / math.sqrt(8) for j in range(i + 1)])
                w = np.exp(s - s.max())
                w /= w.sum()
                ref = sum(w[j] * v[b, h, j] for j in range(i + 1))
                assert np.allclose(out[b, h, i], ref, atol=1e-12)


def test_causal_mask_truth_table():
    """test_reference.py:25-29."""
    m = oracle.causal_mask(3, 6, offset=3)
    assert m[0].tolist() == [True, True, True, True, False, False]
    assert m[2].tolist() == [True] * 6


def test_repeat_kv():
    """test_reference.py:32-36."""
    x = np.arange(8, dtype=np.float64).reshape(1, 2, 1, 4)
    e = oracle.repeat_kv(x, 3)
    assert e.shape == (1, 6, 1, 4)
    assert np.array_equal(e[:, 0], e[:, 1]) and np.array_equal(e[:, 3], x[:, 1])


def test_block_reduce_tail_repeats_last_row():
    """core.py:102-120: the tail block is padded with copies of the last row."""
    x = np.arange(10, dtype=np.float64).reshape(1, 1, 5, 2)
    p = oracle.block_reduce(x, 4)
    assert p.shape == (1, 1, 2, 2)
    assert np.allclose(p[0, 0, 0], x[0, 0, :4].mean(0))
    assert np.allclose(p[0, 0, 1], x[0, 0, 4])


# ---------------------------------------------------------- executor ----
def test_block_sparse_full_selection_is_unmasked_dense():
    """test_kernels.py:71-83 (fp64, 1e-10)."""
    r = rng(0)
    b, h, t, d, bs = 1, 2, 32, 16, 8
    q, k, v = (r.standard_normal((b, h, t, d)) for _ in range(3))
    ids = np.broadcast_to(np.arange(t // bs), (b, h, t, t // bs))
    out = oracle.block_sparse_attention(q, k, v, ids, block_size=bs)
    assert np.allclose(out, oracle.dense_attention(q, k, v, causal=False), atol=1e-10)


def test_block_sparse_equals_dense_over_token_mask():
    """Brute force: listed blocks (set, tails clipped) == dense over that mask."""
    r = rng(1)
    b, hq, hkv, t, d, bs = 1, 4, 2, 37, 8, 8
    q = r.standard_normal((b, hq, 5, d))
    k, v = (r.standard_normal((b, hkv, t, d)) for _ in range(2))
    ids = np.array([[[0, 4, 2], [1, 3, -1]]])  # (B, Hkv, N); block 4 is a 5-token tail
    out = oracle.block_sparse_attention(q, k, v, ids, block_size=bs)
    for hk in range(hkv):
        allow = np.zeros(t, bool)
        for u in ids[0, hk]:
            if u >= 0:
                allow[u * bs:(u + 1) * bs] = True
        mask = np.broadcast_to(allow, (5, t))
        for g in range(2):
            h = hk * 2 + g
            ref = oracle.dense_attention(q[:, h:h + 1], k[:, hk:hk + 1], v[:, hk:hk + 1], mask=mask)
            assert np.allclose(out[:, h:h + 1], ref, atol=1e-12)


def test_block_sparse_duplicate_block_counts_twice():
    """block_sparse.py:62-68 gathers a repeated id twice (multiset)."""
    r = rng(2)
    q = r.standard_normal((1, 1, 1, 4))
    k, v = (r.standard_normal((1, 1, 8, 4)) for _ in range(2))
    out = oracle.block_sparse_attention(q, k, v, np.array([[[0, 0, 1]]]), block_size=4)
    kk = np.concatenate([k[0, 0, :4], k[0, 0, :4], k[0, 0, 4:8]])
    vv = np.concatenate([v[0, 0, :4], v[0, 0, :4], v[0, 0, 4:8]])
    s = kk @ q[0, 0, 0] / 2.0
    w = np.exp(s - s.max())
    assert np.allclose(out[0, 0, 0], (w / w.sum()) @ vv, atol=1e-12)


def test_attend_lists_matches_block_sparse_and_paging():
    """attend_lists (C) == gather form, contiguous and through a page table."""
    r = rng(3)
    B, Hq, Hkv, T, D, ps = 2, 4, 2, 64, 16, 8
    q = torch.from_numpy(r.standard_normal((B, Hq, 1, D)))
    k = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float()
    v = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float()
    ids = np.array([[[[0, 3, 7, -1]], [[1, 2, -1, -1]]], [[[5, 6, 0, 1]], [[7, -1, -1, -1]]]])
    a = oracle.attend_lists(q, k, v, ids, unit=ps)
    bsa = oracle.block_sparse_attention(q.numpy(), k.double().numpy(), v.double().numpy(),
                                        ids[:, :, 0, :], block_size=ps)
    assert np.allclose(a, bsa, atol=1e-12)
    # the same cache through a random page table
    P = T // ps
    perm = r.permutation(B * P)
    pt = perm.reshape(B, P).astype(np.int32)
    pool_k = torch.zeros(B * P, Hkv, ps, D)
    pool_v = torch.zeros(B * P, Hkv, ps, D)
    for b in range(B):
        for p in range(P):
            pool_k[pt[b, p]] = k[b, :, p * ps:(p + 1) * ps]
            pool_v[pt[b, p]] = v[b, :, p * ps:(p + 1) * ps]
    ap = oracle.attend_lists(q, pool_k, pool_v, ids, unit=ps, page_table=pt, page_size=ps)
    assert np.allclose(ap, a, atol=1e-12)


def test_attend_lists_causal_and_empty():
    r = rng(4)
    q = torch.from_numpy(r.standard_normal((1, 1, 3, 8)))
    k = torch.from_numpy(r.standard_normal((1, 1, 16, 8))).float()
    v = torch.from_numpy(r.standard_normal((1, 1, 16, 8))).float()
    ids = np.array([[[[0, 1, 2, 3]]]])
    out = oracle.attend_lists(q, k, v, ids, unit=4, causal=True, offset=5)
    ref = oracle.dense_attention(q.numpy(), k.double().numpy(), v.double().numpy(),
                                 mask=oracle.causal_mask(3, 16, offset=5))
    assert np.allclose(out, ref, atol=1e-12)
    empty = oracle.attend_lists(q, k, v, np.full((1, 1, 1, 2), -1), unit=4)
    assert np.array_equal(empty, np.zeros_like(empty))


def _token_mask(ids, unit, tq, tk, offset, causal=True):
    """Token mask of unit lists (B, L, Tq, N): the units' tokens below Tk,
    intersected with causality."""
    B, L = ids.shape[:2]
    m = np.zeros((B, L, tq, tk), dtype=bool)
    for b in range(B):
        for h in range(L):
            for t in range(tq):
                for u in ids[b, h, t if ids.shape[2] > 1 else 0]:
                    if u >= 0:
                        m[b, h, t, u * unit:min(tk, (u + 1) * unit)] = True
    if causal:
        m &= oracle.causal_mask(tq, tk, offset)
    return m


def test_attend_lists_bf16_elements_match_dense():
    """The bf16 element reader of attend_lists (raw 16-bit words) against
    dense attention over the same values widened by torch, through the token
    mask of the lists (GQA lists shared by two query heads)."""
    r = rng(32)
    B, Hq, Hkv, T, D, unit, Tq, off = 2, 4, 2, 48, 16, 8, 3, 30
    k = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).bfloat16()
    v = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).bfloat16()
    q = torch.from_numpy(r.standard_normal((B, Hq, Tq, D))).bfloat16()
    # distinct units per row (a repeated unit would be attended twice), one
    # of them visible, some slots empty
    ids = np.stack([np.stack([np.stack([np.r_[3, r.choice([0, 1, 2, 4, 5], 2, replace=False)]
                                        for _ in range(Tq)]) for _ in range(Hkv)])
                    for _ in range(B)])
    ids[r.random(ids.shape) < 0.2] = -1
    ids[..., 0] = 3
    got = oracle.attend_lists(q, k, v, ids, unit=unit, causal=True, offset=off)
    mask = np.repeat(_token_mask(ids, unit, Tq, T, off), Hq // Hkv, axis=1)
    ref = oracle.dense_attention(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                 mask=mask)
    assert np.abs(got - ref).max() < 1e-12


@pytest.mark.parametrize("paged", [False, True])
def test_attend_lists_fp8_elements_match_dequantised_dense(paged):
    """The fp8 reader of attend_lists (e4m3fn codes times the per-token K and
    V scales) against dense attention over K and V dequantised by torch,
    code.float() * scale (kv/quant.py:105-109), contiguous and through a
    page table."""
    r = rng(33)
    B, Hq, Hkv, T, D, ps, Tq, off = 2, 4, 2, 64, 16, 8, 2, 50
    kf = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float() * 3
    vf = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float()
    ks = kf.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 448.0
    vs = vf.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 448.0
    kc, vc = (kf / ks).to(torch.float8_e4m3fn), (vf / vs).to(torch.float8_e4m3fn)
    # torch's own e4m3fn decode, times the scale in fp64 (exact: a 4-bit code
    # mantissa times a 24-bit scale); the reference's fp32 product
    # (kv/quant.py:105-109) rounds it to within 2^-24 relative
    kd, vd = kc.to(torch.float64) * ks.double(), vc.to(torch.float64) * vs.double()
    assert torch.allclose(kd.float(), kc.to(torch.float32) * ks, rtol=2.0 ** -23, atol=0)
    q = torch.from_numpy(r.standard_normal((B, Hq, Tq, D)))
    ids = np.stack([np.stack([np.stack([np.r_[1, r.choice(np.r_[0, 2:T // ps], 3, replace=False)]
                                        for _ in range(Tq)]) for _ in range(Hkv)])
                    for _ in range(B)])
    ids[r.random(ids.shape) < 0.2] = -1
    ids[..., 0] = 1
    mask = np.repeat(_token_mask(ids, ps, Tq, T, off), Hq // Hkv, axis=1)
    ref = oracle.dense_attention(q.numpy(), kd.double().numpy(), vd.double().numpy(), mask=mask)
    if not paged:
        got = oracle.attend_lists(q, kc, vc, ids, unit=ps, causal=True, offset=off,
                                  k_scale=ks, v_scale=vs)
    else:
        P = T // ps
        pt = r.permutation(B * P).reshape(B, P).astype(np.int32)
        pk = torch.zeros(B * P, Hkv, ps, D, dtype=torch.float8_e4m3fn)
        pv = torch.zeros_like(pk)
        pks = torch.zeros(B * P, Hkv, ps)
        pvs = torch.zeros(B * P, Hkv, ps)
        for b in range(B):
            for p in range(P):
                sl = slice(p * ps, (p + 1) * ps)
                pk[pt[b, p]], pv[pt[b, p]] = kc[b, :, sl], vc[b, :, sl]
                pks[pt[b, p]], pvs[pt[b, p]] = ks[b, :, sl, 0], vs[b, :, sl, 0]
        got = oracle.attend_lists(q, pk, pv, ids, unit=ps, causal=True, offset=off,
                                  page_table=pt, page_size=ps, k_scale=pks, v_scale=pvs)
    assert np.abs(got - ref).max() < 1e-12


def test_effective_mask_fallback_reads_own_token():
    """selection.py:100-107: a row whose selection is empty, or entirely in
    the future, reads the query's own token; other rows are the selection
    intersected with causality."""
    sel = np.zeros((1, 1, 4, 6), dtype=bool)
    sel[0, 0, 1, 5] = True          # only a future key (query 1 sits at 3)
    sel[0, 0, 2, [0, 5]] = True     # one past key and one future key
    m = oracle.effective_mask(sel, offset=2)
    assert m[0, 0, 0].tolist() == [False, False, True, False, False, False]
    assert m[0, 0, 1].tolist() == [False, False, False, True, False, False]
    assert m[0, 0, 2].tolist() == [True, False, False, False, False, False]
    assert m[0, 0, 3].tolist() == [False, False, False, False, False, True]
    # past the last key, the own position clamps to it
    m2 = oracle.effective_mask(np.zeros((1, 2), dtype=bool), offset=5)
    assert m2.tolist() == [[False, True]]


@pytest.mark.skipif(not REF_LIB.exists(), reason="reference C decode not built (oracle/_ref)")
def test_attend_lists_matches_reference_c_decode():
    """The reference's own decode_attn.c (built from source into oracle/_ref)
    against the oracle, at the reference test's shape and tolerance
    (test_kernels.py:31-44: T=4096, D=64, page 8, atol 2e-4)."""
    L = ctypes.CDLL(str(REF_LIB))
    f32p = ctypes.POINTER(ctypes.c_float)
    i32p = ctypes.POINTER(ctypes.c_int32)
    for name in ("paged_decode_naive", "paged_decode_tiled"):
        getattr(L, name).argtypes = [f32p, f32p, f32p, i32p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_float, f32p]
    torch.manual_seed(0)
    t, dim, page = 4096, 64, 8
    k = torch.randn(t, dim)
    v = torch.randn(t, dim)
    q = torch.randn(dim)
    for pages in (torch.arange(0, 128), torch.randperm(t // page)[:37]):
        ids = pages.to(torch.int32).contiguous()
        ref = oracle.attend_lists(q.view(1, 1, 1, dim).double(), k.view(1, 1, t, dim),
                                  v.view(1, 1, t, dim), ids.view(1, 1, 1, -1).numpy(), unit=page)
        for name in ("paged_decode_naive", "paged_decode_tiled"):
            out = torch.zeros(dim)
            getattr(L, name)(q.data_ptr() and ctypes.cast(q.data_ptr(), f32p),
                             ctypes.cast(k.data_ptr(), f32p), ctypes.cast(v.data_ptr(), f32p),
                             ctypes.cast(ids.data_ptr(), i32p), ids.numel(), page, dim, t,
                             1.0 / math.sqrt(dim), ctypes.cast(out.data_ptr(), f32p))
            assert np.allclose(out.numpy(), ref[0, 0, 0], atol=2e-4), name


# -------------------------------------------------------------- quest ----
def test_page_bounds_bruteforce():
    """test_kernels.py:98-105 plus a ragged tail padded with +/-inf."""
    r = rng(5)
    k = r.standard_normal((1, 2, 30, 8))
    mins, maxs = oracle.page_bounds(k, 8)
    for p in range(4):
        chunk = k[..., p * 8:(p + 1) * 8, :]
        assert np.array_equal(mins[..., p, :], chunk.min(-2))
        assert np.array_equal(maxs[..., p, :], chunk.max(-2))


def test_quest_scores_are_upper_bounds_and_exact_for_single_token_pages():
    """Defining properties of the Quest bound (selection.py:140-152): it is >=
    q.k for every key of the page, and equals q.k when the page holds one key."""
    r = rng(6)
    q = r.standard_normal((1, 4, 3, 16)).astype(np.float32)
    k = r.standard_normal((1, 2, 40, 16)).astype(np.float32)
    mins, maxs = oracle.page_bounds(k, 8)
    s = oracle.quest_scores(q, mins, maxs)
    qd, kd = q.astype(np.float64), k.astype(np.float64)
    for h in range(4):
        dots = np.einsum("td,sd->ts", qd[0, h], kd[0, h // 2])
        for p in range(5):
            assert np.all(s[0, h, :, p] >= dots[:, p * 8:(p + 1) * 8].max(-1) - 1e-12)
    m1, x1 = oracle.page_bounds(k, 1)
    s1 = oracle.quest_scores(q, m1, x1)
    for h in range(4):
        assert np.allclose(s1[0, h], np.einsum("td,sd->ts", qd[0, h], kd[0, h // 2]), atol=1e-12)


def test_topk_rows_tie_rule_bruteforce():
    """Ranking = sorted by (-value, index) over the valid prefix; the forced
    entry first.  Integer-valued scores make ties frequent."""
    r = rng(7)
    s = r.integers(-3, 4, size=(50, 20)).astype(np.float64)
    nv = r.integers(0, 21, size=50)
    own = r.integers(0, 20, size=50)
    for force in (False, True):
        idx, val = oracle.topk_rows(s, 6, n_valid=nv, own=own, force_own=force)
        for i in range(50):
            items = [(-(math.inf if force and j == own[i] else s[i, j]), j) for j in range(nv[i])]
            want = [j for _, j in sorted(items)][:6]
            assert idx[i].tolist() == want + [-1] * (6 - len(want))
            if len(want) and force and own[i] < nv[i]:
                assert idx[i, 0] == own[i] and val[i, 0] == math.inf


def test_quest_known_answer_last_page():
    """test_selection.py:68-91: the high-scoring last page (3) is selected for the
    final query (a (T_q, T_q) own-page write would collapse the selection)."""
    q = np.zeros((1, 2, 32, 16))
    k = np.zeros((1, 2, 32, 16))
    k[:, :, 24:, :] = 50.0
    q[:, :, :, 0] = 1.0
    mins, maxs = oracle.page_bounds(k, 8)
    ids = oracle.quest_select(q, mins, maxs, page_size=8, topk=1, offset=0, gqa_union=False)
    assert 3 in ids[0, 0, 31].tolist()
    # earlier queries see only their own page (the budget is one page)
    assert ids[0, 0, 5].tolist() == [0]
    assert ids[0, 0, 17].tolist() == [2]


def test_quest_union_reads_at_least_shared():
    """test_selection.py:54-65: union over the GQA group reads >= per-head."""
    r = rng(8)
    q = r.standard_normal((1, 4, 1, 16))
    k = r.standard_normal((1, 2, 160, 16))
    mins, maxs = oracle.page_bounds(k, 16)
    u = oracle.quest_select(q, mins, maxs, page_size=16, topk=3, offset=159, gqa_union=True)
    s = oracle.quest_select(q, mins, maxs, page_size=16, topk=3, offset=159, gqa_union=False)
    assert u.shape == (1, 2, 1, 6) and s.shape == (1, 4, 1, 3)
    for hk in range(2):
        got = set(u[0, hk, 0].tolist()) - {-1}
        assert got == set(s[0, 2 * hk:2 * hk + 2, 0].reshape(-1).tolist())
        assert 9 in got  # own page of position 159
    assert (u >= 0).sum() / 2 >= (s >= 0).sum() / 4


def test_quest_full_budget_recovers_dense():
    """test_budgets.py:64-81: with every page selected the output is dense causal
    attention (here at every decode position of a short sequence)."""
    r = rng(9)
    B, Hq, Hkv, T, D, ps = 1, 4, 2, 48, 8, 8
    q = torch.from_numpy(r.standard_normal((B, Hq, T, D)))
    k = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float()
    v = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float()
    mins, maxs = oracle.page_bounds(k, ps)
    ids = oracle.quest_select(q, mins, maxs, page_size=ps, topk=T // ps + 2, offset=0)
    out = oracle.attend_lists(q, k, v, ids, unit=ps, causal=True, offset=0)
    ref = oracle.dense_attention(q.numpy(), k.double().numpy(), v.double().numpy())
    assert np.abs(out - ref).max() < 1e-12


def _page_select_bruteforce(q, mins, maxs, page_size, topk, offset):
    """page_select_torch (quest_pages.py:58-78) spelled out per row: the bound
    as an elementwise maximum summed by numpy, visibility and the own page of
    selection.py:219-231, then a sort by (-score, page)."""
    q, mins, maxs = (np.asarray(x, dtype=np.float64) for x in (q, mins, maxs))
    B, Hq, Tq, D = q.shape
    Hkv, P = mins.shape[1], mins.shape[2]
    G = Hq // Hkv
    k = max(1, min(topk, P))
    scores = np.zeros((B, Hq, Tq, P))
    ids = np.full((B, Hq, Tq, k), -1, dtype=np.int64)
    for b in range(B):
        for h in range(Hq):
            for t in range(Tq):
                pos = offset + t
                qv = q[b, h, t][None, :]
                bound = np.maximum(qv * mins[b, h // G], qv * maxs[b, h // G]).sum(-1)
                own = min(pos // page_size, P - 1)
                row = np.array([bound[p] if p * page_size <= pos else -math.inf
                                for p in range(P)])
                row[own] = math.inf
                scores[b, h, t] = row
                vis = [p for p in range(P) if p * page_size <= pos]
                want = sorted(vis, key=lambda p: (-row[p], p))[:k]
                ids[b, h, t, :len(want)] = want
    return ids, scores


def test_page_select_integer_inputs_bruteforce():
    """oracle.page_select == brute force, exactly: small-integer q and keys
    make every product and sum exact, and make ties frequent (the tie rule)."""
    r = rng(30)
    B, Hq, Hkv, T, D, ps = 2, 4, 2, 40, 6, 4
    q = r.integers(-2, 3, size=(B, Hq, 5, D)).astype(np.float64)
    k = r.integers(-3, 4, size=(B, Hkv, T, D)).astype(np.float64)
    mins, maxs = oracle.page_bounds(k, ps)
    for offset, topk in ((17, 3), (0, 2), (35, 20)):
        ids, sc = oracle.page_select(q, mins, maxs, ps, topk, offset=offset)
        want_ids, want_sc = _page_select_bruteforce(q, mins, maxs, ps, topk, offset)
        assert np.array_equal(sc, want_sc), offset
        assert np.array_equal(ids, want_ids), offset


def test_page_select_real_inputs_own_page_per_query():
    """Real-valued inputs: scores agree with the elementwise form to rounding,
    the ids exactly; with Tq > 1 only entry (t, own(t)) of each row is +inf
    (defect D1 of quest_pages.py:74-75 is not reproduced)."""
    r = rng(31)
    B, Hq, Hkv, T, D, ps, Tq, offset = 1, 4, 1, 64, 16, 8, 6, 20
    q = r.standard_normal((B, Hq, Tq, D))
    k = r.standard_normal((B, Hkv, T, D))
    mins, maxs = oracle.page_bounds(k, ps)
    ids, sc = oracle.page_select(q, mins, maxs, ps, 3, offset=offset)
    want_ids, want_sc = _page_select_bruteforce(q, mins, maxs, ps, 3, offset)
    fin = np.isfinite(want_sc)
    assert np.array_equal(fin, np.isfinite(sc))
    assert np.allclose(sc[fin], want_sc[fin], rtol=0, atol=1e-12)
    assert np.array_equal(ids, want_ids)
    for t in range(Tq):
        own = (offset + t) // ps
        assert np.array_equal(np.isposinf(sc[0, :, t]).nonzero()[1], np.full(Hq, own))
        assert ids[0, 0, t, 0] == own


# ------------------------------------------------------------ indexer ----
def test_indexer_scores_closed_form():
    """fused_indexer.py:52-60 computed by numpy einsum (another summation route)."""
    r = rng(10)
    b, tq, tk, hi, d = 2, 7, 11, 3, 8
    qi = r.standard_normal((b, tq, hi, d)).astype(np.float32)
    ki = r.standard_normal((b, tk, hi, d)).astype(np.float32)
    w = r.random((b, tq, hi)).astype(np.float32)
    got = oracle.indexer_scores(qi, ki, w)
    relu = np.maximum(np.einsum("bqhd,bkhd->bqkh", qi.astype(np.float64), ki.astype(np.float64)), 0)
    ref = (relu * w.astype(np.float64)[:, :, None, :]).sum(-1)
    assert np.allclose(got, ref, atol=1e-12)
    gc = oracle.indexer_scores(qi, ki, w, causal=True, offset=2)
    for t in range(tq):
        assert np.all(np.isneginf(gc[:, t, t + 3:]))
        assert np.allclose(gc[:, t, :t + 3], ref[:, t, :t + 3], atol=1e-12)


def test_indexer_topk_bruteforce_with_ties():
    """Top-k == sorted by (-score, index); ReLU zeros tie exactly."""
    r = rng(11)
    b, tq, tk, hi, d, kk = 1, 6, 40, 2, 4, 12
    qi = r.standard_normal((b, tq, hi, d))
    ki = r.standard_normal((b, tk, hi, d))
    w = r.random((b, tq, hi))
    val, idx = oracle.indexer_topk(qi, ki, w, kk, causal=True, offset=20)
    sc = oracle.indexer_scores(qi, ki, w, causal=True, offset=20)
    for t in range(tq):
        nv = min(tk, 20 + t + 1)
        want = sorted(range(nv), key=lambda j: (-sc[0, t, j], j))[:kk]
        assert idx[0, t].tolist() == want
        assert (sc[0, t, :nv] == 0).sum() > 0  # ties at zero are exercised
    v2, i2 = oracle.indexer_topk(qi, ki, w, 30, causal=True, offset=0)
    assert i2[0, 0].tolist() == [0] + [-1] * 29 and np.isneginf(v2[0, 0, 1:]).all()


# --------------------------------------------------- block selection ----
def test_block_select_structure_and_ranking():
    """C3 lists: causal (kb <= qb), contain sink 0, the window and the diagonal,
    and the extra blocks are the top-k of an independent pooled score."""
    r = rng(12)
    B, Hq, Hkv, T, D, bs = 1, 4, 2, 256, 16, 16
    q = r.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = r.standard_normal((B, Hkv, T, D)).astype(np.float32)
    ids = oracle.block_select(q, k, block=bs, topk=3, sink_blocks=1, window_blocks=2)
    qp = oracle.block_reduce(q.astype(np.float64), bs)
    kp = oracle.repeat_kv(oracle.block_reduce(k.astype(np.float64), bs), 2)
    sc = np.einsum("bhid,bhjd->bhij", qp, kp)
    for h in range(Hq):
        for i in range(T // bs):
            s = [x for x in ids[0, h, i].tolist() if x >= 0]
            assert s == sorted(set(s)) and max(s) <= i
            assert 0 in s and i in s and (i == 0 or i - 1 in s)
            top = sorted(range(i + 1), key=lambda j: (-sc[0, h, i, j], j))[:3]
            assert set(top) <= set(s)
            assert len(s) == len(set(top) | {0} | set(range(max(0, i - 1), i + 1)))


# ------------------------------------------------- per-query routing ----
def test_gate_select_ranking_bruteforce():
    """MoBA gate routing (selection.py:610-640): lists hold only visible
    blocks, always the own block, and otherwise exactly the top-k of an
    independent gate computed by einsum over numpy block means (tail block
    padded with the last row, core.py:115-117)."""
    r = rng(13)
    B, Hq, Hkv, T, D, bs, kk = 1, 4, 2, 90, 8, 16, 3  # T not a multiple of bs
    q = r.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = r.standard_normal((B, Hkv, T, D)).astype(np.float32)
    ids = oracle.gate_select(q, k, block=bs, topk=kk, offset=0)
    nkb = (T + bs - 1) // bs
    kpad = np.concatenate([k, np.repeat(k[:, :, -1:], nkb * bs - T, axis=2)], axis=2)
    kbar = kpad.astype(np.float64).reshape(B, Hkv, nkb, bs, D).mean(3)
    gates = np.einsum("bhtd,bhjd->bhtj", q.astype(np.float64), np.repeat(kbar, Hq // Hkv, axis=1))
    assert ids.shape == (B, Hq, T, kk + 1)
    for h in range(Hq):
        for t in range(T):
            s = [x for x in ids[0, h, t].tolist() if x >= 0]
            own = t // bs
            assert s == sorted(set(s)) and max(s) == own and own in s
            top = sorted(range(own + 1), key=lambda j: (-gates[0, h, t, j], j))[:kk]
            assert set(s) == set(top) | {own}


def test_block_means_pins():
    """The gate's pooled keys (block_reduce, core.py:102-120): on small
    integers every summation order is exact, so they equal numpy's mean of the
    tail-padded blocks bit for bit; the tail block of a hand-made input is
    (sum of its rows + copies of the last row) / block; on normal data they
    agree with numpy's (pairwise) mean to rounding."""
    r = rng(21)
    x = r.integers(-50, 50, size=(2, 3, 37, 5)).astype(np.float64)
    bs = 8
    m = oracle.block_means(x, bs)
    nkb = (37 + bs - 1) // bs
    pad = np.concatenate([x, np.repeat(x[:, :, -1:], nkb * bs - 37, axis=2)], axis=2)
    assert np.array_equal(m, pad.reshape(2, 3, nkb, bs, 5).mean(3))
    y = np.array([[1.0, 2.0], [3.0, 5.0], [7.0, 11.0]]).reshape(1, 1, 3, 2)
    assert np.array_equal(oracle.block_means(y, 2)[0, 0],
                          np.array([[2.0, 3.5], [7.0, 11.0]]))
    assert np.array_equal(oracle.block_means(y, 4)[0, 0], np.array([[(1 + 3 + 7 + 7) / 4.0,
                                                                       (2 + 5 + 11 + 11) / 4.0]]))
    z = r.standard_normal((1, 2, 100, 16))
    assert np.allclose(oracle.block_means(z, 16), oracle.block_reduce(z, 16), rtol=0, atol=1e-15)


def test_gate_select_full_budget_recovers_dense():
    """test_budgets.py:64-81 for MoBA: with every block routed the output is
    dense causal attention; with an offset (decode) as well."""
    r = rng(14)
    B, Hq, Hkv, T, D, bs = 1, 4, 2, 40, 8, 8
    q = torch.from_numpy(r.standard_normal((B, Hq, T, D)))
    k = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float()
    v = torch.from_numpy(r.standard_normal((B, Hkv, T, D))).float()
    ids = oracle.gate_select(q, k, block=bs, topk=T // bs + 2, offset=0)
    out = oracle.attend_lists(q, k, v, ids, unit=bs, causal=True, offset=0)
    dense = oracle.dense_attention(q.numpy(), k.double().numpy(), v.double().numpy())
    assert np.abs(out - dense).max() < 1e-12
    ids1 = oracle.gate_select(q[:, :, -1:], k, block=bs, topk=T // bs + 2, offset=T - 1)
    out1 = oracle.attend_lists(q[:, :, -1:], k, v, ids1, unit=bs, causal=True, offset=T - 1)
    assert np.abs(out1 - dense[:, :, -1:]).max() < 1e-12


# ----------------------------------------------------------------- fp8 ----
def test_fp8_decode_matches_torch_for_all_codes():
    """The oracle's e4m3fn decoder (from the OCP spec) against torch's dtype,
    which is the reference's codec (kv/quant.py:90-93)."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    got = oracle.fp8_decode(codes.numpy())
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got)) and nan.sum() == 2
    assert np.array_equal(got[~nan], ref[~nan])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9


def test_fp8_constant_group_roundtrips_exactly():
    """test_quantization_geometry.py:6-16: a constant group is reproduced."""
    x = torch.full((2, 3, 64), 0.75)
    codes, scale = oracle.fp8_quantize(x)
    back = codes.to(torch.float32) * scale
    assert torch.equal(back, x)
    y = torch.randn(4, 128)
    c, s = oracle.fp8_quantize(y)
    assert torch.allclose(c.to(torch.float32) * s, y, rtol=2 ** -4, atol=0)
    assert torch.allclose(s.squeeze(-1), y.abs().amax(-1) / 448)


def test_window_mask():
    """local.py:47-53."""
    m = oracle.window_mask(4, 8, 4, window=2, sink=1)
    assert m[0].tolist() == [True, False, False, True, True, False, False, False]
    assert m[3].tolist() == [True, False, False, False, False, False, True, True]


# --------------------------------------------------------- XAttention ----
def test_exp_det_matches_libm():
    """The deterministic exp of the XAttention weights against math.exp:
    within 4 ulp over [-700, 0]; exp(0) = 1; 0 below -700."""
    xs = np.concatenate([-np.logspace(-12, np.log10(699.9), 2000), [-0.0, 0.0, -1e-300, -699.99]])
    for x in xs:
        got, ref = oracle.exp_det(x), math.exp(x)
        assert abs(got - ref) <= 4 * math.ulp(ref), (x, got, ref)
    assert oracle.exp_det(0.0) == 1.0
    assert oracle.exp_det(-700.0) == 0.0 and oracle.exp_det(-1e9) == 0.0


def _xattn_float_reference(q, k, *, block, stride, threshold, offset, topk=None, top_ratio=None):
    """XAttention.select (selection.py:528-595) restated with numpy floats:
    antidiagonal sums by einsum over the whole (query block, key block) gram
    tensor, fp64 softmax over the visible (block, slot) pairs, a stable sort
    of the block masses and their cumulative sum.  Independent of the
    oracle's integer masses; equal selections unless a mass tie or the
    threshold crossing sits within rounding."""
    q, k = q.astype(np.float64), k.astype(np.float64)
    Tq, D = q.shape
    T = k.shape[0]
    n_qb, n_kb = -(-Tq // block), -(-T // block)
    qp = np.zeros((n_qb * block, D)); qp[:Tq] = q
    kp = np.zeros((n_kb * block, D)); kp[:T] = k
    gram = np.einsum("aid,bjd->abij", qp.reshape(n_qb, block, D), kp.reshape(n_kb, block, D))
    offs = list(range(0, 2 * block - 1, stride))
    S = np.zeros((n_qb, n_kb, len(offs)))
    ii = np.arange(block)
    for s, o in enumerate(offs):
        jj = o - ii
        ok = (jj >= 0) & (jj < block)
        S[..., s] = gram[:, :, ii[ok], jj[ok]].sum(-1)
    S /= math.sqrt(D)
    out = []
    for qb in range(n_qb):
        pos0 = qb * block + offset
        vis = np.arange(n_kb) * block <= pos0
        flat = np.where(vis[:, None], S[qb], -np.inf)
        p = np.exp(flat - flat.max())
        mass = (p / p.sum()).sum(-1)
        order = sorted(range(n_kb), key=lambda j: (-mass[j], j))
        if topk is not None:
            n_keep = min(topk, n_kb)
        elif top_ratio is not None:  # _select_with_per_head with a block count (:583-585)
            c = max(1.0, math.ceil(vis.sum() * top_ratio))
            reached = np.cumsum(mass[order]) >= c
            n_keep = int(reached.argmax()) + 1 if reached.any() else n_kb
        else:
            cs = np.cumsum(mass[order])
            n_keep = min(int((cs < threshold).sum()) + 1, n_kb)
        sel = set(order[:n_keep])
        if pos0 % block == 0 and pos0 // block < n_kb:
            sel.add(pos0 // block)
        out.append(sorted(j for j in sel if vis[j]))
    return out


@pytest.mark.parametrize("block,stride,threshold,offset,topk,T,top_ratio", [
    (8, 8, 0.9, 0, None, 203, None), (8, 4, 0.6, 0, None, 128, None),
    (16, 8, 0.95, 5, None, 150, None), (4, 2, 0.5, 0, None, 61, None),
    (8, 8, None, 0, 3, 203, None), (8, 8, 1.5, 0, None, 100, None),
    (8, 8, None, 0, None, 203, 0.02), (4, 2, None, 7, None, 150, 0.3)])
def test_xattn_select_matches_float_restatement(block, stride, threshold, offset, topk, T,
                                                top_ratio):
    r = rng(21)
    B, Hq, Hkv, D = 1, 2, 1, 32
    Tq = T - offset
    q = r.standard_normal((B, Hq, Tq, D)).astype(np.float32)
    k = r.standard_normal((B, Hkv, T, D)).astype(np.float32)
    k[0, 0, r.permutation(T)[:T // 10]] *= 4.0  # peaked rows
    ids, counts = oracle.xattn_select(q, k, block=block, stride=stride,
                                      threshold=threshold if threshold else 0.9, offset=offset,
                                      topk=topk, top_ratio=top_ratio)
    for h in range(Hq):
        ref = _xattn_float_reference(q[0, h], k[0, 0], block=block, stride=stride,
                                     threshold=threshold, offset=offset, topk=topk,
                                     top_ratio=top_ratio)
        for qb, lst in enumerate(ref):
            got = [int(x) for x in ids[0, h, qb] if x >= 0]
            assert got == lst, (h, qb, got, lst)
            assert counts[0, h, qb] == len(lst)


def test_xattn_known_answer():
    """Two 2-token blocks, stride 1: slot scores by hand.  q rows (1,0),
    (0,1); k rows (1,0), (0,1), (5,0), (0,5).  Query block 1 sees key block 0
    (slots: q0.k0 = 1, q0.k1 + q1.k0 = 0, q1.k1 = 1) and key block 1 (slots 5,
    0, 5), so block 1 holds e^5-weighted mass and alone reaches 0.9; block 0
    (the own block of query block 0) is listed only for query block 0."""
    q = np.array([[[[1.0, 0.0], [0.0, 1.0], [1.0, 0.0], [0.0, 1.0]]]], dtype=np.float32)
    k = np.array([[[[1.0, 0.0], [0.0, 1.0], [5.0, 0.0], [0.0, 5.0]]]], dtype=np.float32)
    ids, counts = oracle.xattn_select(q * math.sqrt(2), k, block=2, stride=1, threshold=0.9)
    assert ids[0, 0, 0].tolist() == [0, -1] and counts[0, 0, 0] == 1
    assert ids[0, 0, 1].tolist() == [1, -1] and counts[0, 0, 1] == 1
    ids, _ = oracle.xattn_select(q * math.sqrt(2), k, block=2, stride=1, threshold=0.99999)
    assert ids[0, 0, 1].tolist() == [0, 1]


def test_xattn_full_budget_recovers_dense():
    """threshold > 1 (or top-k over every block) reads every visible block:
    attention over the selection equals dense causal attention
    (test_budgets.py:64-81)."""
    r = rng(22)
    q = r.standard_normal((1, 2, 70, 16)).astype(np.float32)
    k = r.standard_normal((1, 1, 70, 16)).astype(np.float32)
    v = r.standard_normal((1, 1, 70, 16)).astype(np.float32)
    for kw in (dict(threshold=1.5), dict(topk=100), dict(top_ratio=0.02)):
        ids, counts = oracle.xattn_select(q, k, block=8, stride=8, **kw)
        rows = np.repeat(ids, 8, axis=2)[:, :, :70]
        out = oracle.attend_lists(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                  rows, unit=8, causal=True)
        dense = oracle.dense_attention(q.astype(np.float64), np.repeat(k, 2, 1).astype(np.float64),
                                       np.repeat(v, 2, 1).astype(np.float64), causal=True)
        assert np.abs(out - dense).max() < 1e-12
