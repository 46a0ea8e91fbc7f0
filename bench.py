"""Benchmark of the MI355X sparse-attention hot path (one GPU).

Headline workload: paged Quest sparse decode, bf16 KV,
batch 64, context 65536 per sequence in 64-token pages behind a randomly
permuted page table, 32 query / 8 KV heads, head_dim 128, a 2048-token budget
(32 pages per query head, the last page forced), GQA union of the group's
pages (the reference default, variants/selection.py:232-235).

A step = one decode step for all 64 sequences: Quest page scores, top-k page
selection and the GQA union, attention over the selected pages, as one kernel
(``quest_decode_fused``); the same step as two launches (``quest_select_hip``,
then the split-K ``sparse_attention``) is timed beside it.  Inputs (query, KV
pool, page table, page metadata) are resident in HBM before timing starts.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline]

Prints one JSON line (see the driver contract in the repository docs).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD public spec

C4 = dict(B=64, Hq=32, Hkv=8, T=65536, D=128, page=64, topk=32, seed=0)
STEP_KERNEL = "quest_decode_fused_kernel"  # the C4 step: selection and attention in one kernel
ATTN_KERNEL = "sparse_attn_mfma_kernel"  # the attention launch of the two-launch step
COPY_MIB = 1024
TRAFFIC_FILE = "profiles/c4_step_traffic.json"
ATTN_TRAFFIC_FILE = "profiles/c4_attention_traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=16, help="sequences timed on the CPU")
    ap.add_argument("--shared", action="store_true",
                    help="per-query-head page lists instead of the GQA union")
    ap.add_argument("--pmc-workload", choices=["c3", "c5"],
                    help="one warm-up and one timed step of C3 (prefill) or C5 (fp8 decode), "
                         "then a device copy of COPY_MIB MiB; run under rocprofv3 --pmc")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="C4 only, then a device copy of COPY_MIB MiB (the counter scale "
                         "reference); run under rocprofv3 --pmc")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc runs of --pmc-probe (FETCH_SIZE, then "
                         "WRITE_SIZE) into " + TRAFFIC_FILE + " and " + ATTN_TRAFFIC_FILE)
    return ap.parse_args()


def setup_c4(dev, cfg):
    import torch

    from linattn_amd.kernels.quest_pages import page_update_hip

    B, Hq, Hkv, T, D, ps = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["T"], cfg["D"], cfg["page"]
    P = T // ps
    g = torch.Generator(device=dev).manual_seed(cfg["seed"])
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).to(torch.bfloat16)
    pool_k = torch.empty(B * P, Hkv, ps, D, dtype=torch.bfloat16, device=dev)
    pool_v = torch.empty_like(pool_k)
    chunk = 4096
    for i in range(0, B * P, chunk):  # bounded fp32 temporaries
        pool_k[i:i + chunk] = torch.randn(min(chunk, B * P - i), Hkv, ps, D, generator=g, device=dev)
    for i in range(0, B * P, chunk):
        pool_v[i:i + chunk] = torch.randn(min(chunk, B * P - i), Hkv, ps, D, generator=g, device=dev)
    pt = torch.randperm(B * P, generator=g, device=dev).view(B, P).to(torch.int32)
    mins, maxs = page_update_hip(pool_k, ps, page_table=pt)
    torch.cuda.synchronize()
    return q, pool_k, pool_v, pt, mins, maxs


def cpu_info():
    """CPU model (/proc/cpuinfo), os.cpu_count() and the cores this process
    may run on."""
    import os

    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "cpu_count": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0))}


def _timed_pool(tasks, threads, min_s):
    """Run the independent tasks (callables; the oracle's C kernels and torch's
    CPU ops release the GIL) over `threads` worker threads, one pass over all of
    them at a time: one untimed pass, then passes until min_s seconds have gone
    by.  Each worker holds torch's intra-op parallelism at one thread (the
    setting is per calling thread), so that `threads` is the parallelism.
    Returns (tasks per pass, best pass in s)."""
    from concurrent.futures import ThreadPoolExecutor

    import torch

    nt = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        with ThreadPoolExecutor(max_workers=threads,
                                initializer=lambda: torch.set_num_threads(1)) as ex:
            list(ex.map(lambda f: f(), tasks))  # warm-up
            best, t_end = float("inf"), time.perf_counter() + min_s
            while True:
                t0 = time.perf_counter()
                list(ex.map(lambda f: f(), tasks))
                t1 = time.perf_counter()
                best = min(best, t1 - t0)
                if t1 >= t_end:
                    return len(tasks), best
    finally:
        torch.set_num_threads(nt)


def cpu_baseline(q, pool_k, pool_v, pt, mins, maxs, cfg, n_seq, union, keep):
    """The CPU oracle (oracle/: C kernels + numpy, a from-scratch port of the
    reference's semantics) on bounded samples of the same inputs, copied from
    the device: C4 (Quest step), C2 (indexer top-k), C3 (blockwise prefill
    over the selected blocks), C5 (indexer + top-k + fp8 attention).  Each leg
    runs on every core this process may use and on 4 threads (the reference's
    bench pins 4, bench/bench_decode.py:56); independent units (sequences,
    query rows, query blocks) go to a thread pool.  `value` is the C4 leg on
    every core."""
    import numpy as np

    import oracle

    info = cpu_info()
    oracle.lib()
    legs = {}
    all_t = info["affinity"]

    def run(name, tasks, units_per_task, unit, note, scale=1.0):
        out = {"unit": unit, "sample": note}
        for label, th in (("all", all_t), ("4", min(4, all_t))):
            n, dt = _timed_pool(tasks, th, CPU_LEG_S)
            out[f"value_{label}_threads"] = float(f"{n * units_per_task * scale / dt:.4g}")
            out[f"threads_{label}"] = th
        legs[name] = out

    # C4: page scores, top-k and attention per sequence
    B, Hkv, T, D, ps = cfg["B"], cfg["Hkv"], cfg["T"], cfg["D"], cfg["page"]
    seqs = []
    for b in range(n_seq):
        kb = pool_k[pt[b].long()].permute(1, 0, 2, 3).reshape(1, Hkv, T, D).cpu()
        vb = pool_v[pt[b].long()].permute(1, 0, 2, 3).reshape(1, Hkv, T, D).cpu()
        seqs.append((q[b:b + 1].cpu(), kb, vb, mins[b:b + 1].cpu(), maxs[b:b + 1].cpu()))

    def c4_task(sq):
        qb, kb, vb, mb, xb = sq
        def f():
            ids = oracle.quest_select(qb, mb, xb, page_size=ps, topk=cfg["topk"], offset=T - 1,
                                      gqa_union=union)
            oracle.attend_lists(qb, kb, vb, ids, unit=ps, causal=True, offset=T - 1)
        return f

    run("c4", [c4_task(x) for x in seqs], 1, "tok/s",
        f"{n_seq} of {B} sequences of config 4 (page scores, top-k, attention), one per task")
    del seqs

    # C2: 128 query rows spread evenly over [0, T) (their causal key counts
    # average the full workload's), 2 rows per task
    c2 = keep.get("c2")
    if c2:
        Tq = c2["q"].shape[1]
        rows = np.linspace(0, Tq - 1, 128).astype(np.int64)
        k2 = oracle.to_f64(c2["k"])  # converted once, as the GPU's keys are resident

        def c2_task(r):
            qr, wr = oracle.to_f64(c2["q"][:, r]), oracle.to_f64(c2["w"][:, r])
            def f():
                for i, t in enumerate(r):
                    oracle.indexer_topk(qr[:, i:i + 1], k2[:, :t + 1], wr[:, i:i + 1],
                                        c2["topk"], causal=True, offset=int(t))
            return f

        run("c2", [c2_task(rows[i:i + 2]) for i in range(0, 128, 2)], 2, "queries/s",
            "128 query rows of config 2 evenly spaced over the 8192 positions (causal scores over "
            "their key prefix, top-2048), 2 rows per task")

    # C3: 64 (b, head, query block) items spread over the batch, heads and
    # positions; a mask-free blockwise loop in torch fp32 (gather the selected
    # key blocks, one causal 64 x 64 triangle on the diagonal block only),
    # checked on its first item against the fp64 oracle
    c3 = keep.get("c3")
    if c3:
        import torch

        bs = c3["block"]
        Bq, Hq, nqb = c3["ids"].shape[:3]
        D3 = c3["q"].shape[-1]
        G = Hq // c3["k"].shape[1]
        rng = np.random.default_rng(0)
        items = [(int(rng.integers(Bq)), int(rng.integers(Hq)), int(x))
                 for x in np.linspace(0, nqb - 1, 64).astype(np.int64)]
        pairs = sum(int(c3["counts"][b, h, qb]) for b, h, qb in items)
        kv3 = {}  # fp32 K/V heads as (blocks, 64, D), made before timing
        tri = torch.ones(bs, bs, dtype=torch.bool).tril()

        def c3_item(it):
            b, h, qb = it
            key = (b, h // G)
            if key not in kv3:
                kv3[key] = tuple(c3[n][b, h // G].float().view(-1, bs, D3) for n in "kv")
            kb, vb = kv3[key]
            lst = c3["ids"][b, h, qb, :c3["counts"][b, h, qb]].long()
            lst = lst[lst <= qb]  # causal: blocks past the query block hold no visible key
            qq = c3["q"][b, h, qb * bs:(qb + 1) * bs].float() * (1.0 / math.sqrt(D3))
            diag = lst == qb
            def f():
                s_ = (qq @ kb[lst].reshape(-1, D3).T).view(bs, -1, bs)
                s_[:, diag] = s_[:, diag].masked_fill(~tri.unsqueeze(1), float("-inf"))
                p_ = torch.softmax(s_.reshape(bs, -1), -1)
                return p_ @ vb[lst].reshape(-1, D3)
            return f

        tasks = [c3_item(it) for it in items]
        b, h, qb = items[0]
        lst = c3["ids"][b, h, qb, :c3["counts"][b, h, qb]].numpy()
        want = oracle.attend_lists(c3["q"][b:b + 1, h:h + 1, qb * bs:(qb + 1) * bs],
                                   c3["k"][b:b + 1, h // G:h // G + 1],
                                   c3["v"][b:b + 1, h // G:h // G + 1],
                                   np.broadcast_to(lst, (1, 1, bs, len(lst))), unit=bs,
                                   causal=True, offset=qb * bs)[0, 0]
        err = float(np.abs(tasks[0]().double().numpy() - want).max())
        flop_per_pair = bs * bs * D3 * 2 * 2
        run("c3", tasks, pairs / len(items), "TFLOP/s",
            "64 (b, head, query block) items of config 3 evenly spaced over the query blocks; "
            "mask-free blockwise loop in torch fp32 over the GPU-selected key blocks (the "
            "selection not timed); useful FLOPs as on the GPU", scale=flop_per_pair / 1e12)
        legs["c3"]["max_abs_err_vs_oracle_item0"] = float(f"{err:.3g}")

    # C5: per sequence, indexer over all 131072 keys, top-4096, fp8 attention
    c5 = keep.get("c5")
    if c5:
        T5, k5 = c5["T"], c5["topk"]

        for sq in c5["seqs"]:  # indexer operands converted once, as on the GPU they are resident
            for n in ("q_idx", "k_idx", "w"):
                sq[n] = oracle.to_f64(sq[n])

        def c5_task(sq):
            def f():
                _, idx = oracle.indexer_topk(sq["q_idx"], sq["k_idx"], sq["w"], k5, causal=True,
                                             offset=T5 - 1)
                ids = np.broadcast_to(idx.reshape(1, 1, 1, -1),
                                      (1, sq["kc"].shape[1], 1, idx.shape[-1]))
                oracle.attend_lists(sq["q"], sq["kc"], sq["vc"], ids, unit=1, causal=True,
                                    offset=T5 - 1, k_scale=sq["ks"], v_scale=sq["vs"])
            return f

        run("c5", [c5_task(sq) for sq in c5["seqs"]], 1, "tok/s",
            f"{len(c5['seqs'])} of 16 sequences of config 5 (indexer over 131072 keys, top-4096, "
            "fp8 attention of 32 heads), one per task")

    c4 = legs["c4"]
    return {"value": c4["value_all_threads"], "unit": "tok/s", "cores": c4["threads_all"],
            "kind": "port",
            "sample": f"config 4 leg: {c4['sample']}; one warm-up pass, then the best pass of "
                      f"{CPU_LEG_S:.0f}+ s of passes per leg and thread count; CPU oracle (C + "
                      f"numpy) on {c4['threads_all']} threads",
            "cpu": info, "legs": legs}


FP64_VALU_PEAK_TFLOPS = 78.6  # MI355X fp64 vector, AMD public spec
CPU_LEG_S = 3.0  # CPU work timed per baseline leg and thread count
C5_CPU_SEQ = 16  # C5 sequences copied to the host for its CPU leg (all of them)


SETTLE_MS = 150.0  # untimed run-in before each measurement (see settle())


def settle(fn, min_ms=None, max_calls=4000):
    """Untimed calls of ``fn`` until the device has spent ``min_ms`` on them.

    The MI355X's clocks follow the load with a lag: after a change of
    workload (setup, another benchmark, an idle pause) the same C4 step runs
    10-12 % slower for its first ~20 ms and reaches its steady time only
    after ~60 steps (measured per 10 steps: 0.40, 0.38, 0.37, 0.36, 0.356 ms).
    A measurement after a few warm-up calls would time that ramp instead of
    the steady state a serving loop runs in.  Returns the calls made."""
    import torch

    min_ms = SETTLE_MS if min_ms is None else min_ms
    done, spent = 0, 0.0
    while spent < min_ms and done < max_calls:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(10):
            fn()
        b.record()
        torch.cuda.synchronize()
        spent += a.elapsed_time(b)
        done += 10
    return done


def time_cuda(fn, steps, warmup):
    import torch

    settle(fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def bench_c2(dev, steps, warmup, keep=None):
    """Config 2: fused indexer + causal top-2048, bf16, B=1, T=8192, 4x64 heads.
    ``keep`` (a dict) receives host copies of the inputs for the CPU leg."""
    import torch

    from linattn_amd.kernels.fused_indexer import indexer_topk

    T, HI, d, kk = 8192, 4, 64, 2048
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(1, T, HI, d, generator=g, device=dev).bfloat16()
    k = torch.randn(1, T, HI, d, generator=g, device=dev).bfloat16()
    w = torch.rand(1, T, HI, generator=g, device=dev)
    ms = time_cuda(lambda: indexer_topk(q, k, w, kk, causal=True), steps, warmup)
    if keep is not None:
        keep["c2"] = {"q": q.cpu(), "k": k.cpu(), "w": w.cpu(), "topk": kk}
    pairs = T * (T + 1) // 2
    flops = pairs * HI * d * 2  # exact fp64 q.k products
    tflops = flops / (ms * 1e-3) / 1e12
    return {"workload": "C2 indexer top-2048, causal, T=8192, 4x64 heads, bf16",
            "queries_per_s": round(T / (ms * 1e-3), 1), "ms": round(ms, 4),
            "score_tflops_fp64": round(tflops, 2),
            "frac_fp64_valu_peak": round(tflops / FP64_VALU_PEAK_TFLOPS, 4),
            "note": "score_tflops_fp64: the exact fp64 q.k product work (512 FLOP per causal "
                    "pair) over the whole call, scores and top-k; bf16 scores are computed "
                    "exactly as int8 limb products on the matrix cores"}


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, AMD public spec


def bench_c3(dev, steps, warmup, keep=None):
    """Config 3: block-sparse causal prefill, bf16, B=2, T=32768, 32/8 heads,
    D=128, 64x64 blocks, sink + 4-block window + top-16 by pooled scores."""
    import torch

    from linattn_amd.kernels.prefill import block_select_hip, block_sparse_prefill

    B, Hq, Hkv, T, D, bs = 2, 32, 8, 32768, 128, 64
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, Hq, T, D, generator=g, device=dev)
    k = torch.randn(B, Hkv, T, D, generator=g, device=dev)
    v = torch.randn(B, Hkv, T, D, generator=g, device=dev)
    for b in range(B):
        for h in range(Hkv):
            rows = torch.randperm(T, generator=g, device=dev)[:T // 100]
            k[b, h, rows] *= 8.0
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    ids, counts = block_select_hip(q, k, block=bs, topk=16, sink_blocks=1, window_blocks=4)
    ms_sel = time_cuda(lambda: block_select_hip(q, k, block=bs, topk=16, sink_blocks=1,
                                                window_blocks=4), steps, warmup)
    # check_range=False: no host read of the device status word after each call
    # (it would synchronise every call); the inputs are in range by construction
    ms = time_cuda(lambda: block_sparse_prefill(q, k, v, ids, counts, block_size=bs,
                                                check_range=False), steps, warmup)
    pairs = int(counts.sum())
    flops = pairs * bs * bs * D * 2 * 2  # QK^T and PV, diagonal blocks counted whole
    tflops = flops / (ms * 1e-3) / 1e12
    if keep is not None:
        keep["c3"] = {"q": q.cpu(), "k": k.cpu(), "v": v.cpu(), "ids": ids.cpu(),
                      "counts": counts.cpu(), "block": bs}
    # the same lists over an fp8 e4m3 cache (per-token scales, kv/quant.py:76-109)
    from linattn_amd.kernels.paged_decode import quantize_fp8_per_token
    kc, ks = quantize_fp8_per_token(k.float())
    vc, vs = quantize_fp8_per_token(v.float())
    ms8 = time_cuda(lambda: block_sparse_prefill(q, kc, vc, ids, counts, block_size=bs, k_scale=ks,
                                                 v_scale=vs, check_range=False), steps, warmup)
    del kc, vc
    return {"workload": "C3 block-sparse causal prefill, B=2, T=32768, 32/8 heads, D=128, bf16",
            "selected_block_pairs": pairs, "ms_prefill": round(ms, 4),
            "ms_block_select": round(ms_sel, 4), "TFLOPs": round(tflops, 1),
            "frac_mfma_bf16_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "ms_prefill_fp8_kv": round(ms8, 4),
            "TFLOPs_fp8_kv": round(flops / (ms8 * 1e-3) / 1e12, 1),
            "note": "useful FLOPs (bf16 QK^T, fp16 weights x V); ms_prefill includes the fp16 V "
                    "conversion pre-pass; *_fp8_kv: the same lists over an fp8 e4m3 K/V cache "
                    "(K codes scored on the fp8 matrix cores against q as two e4m3 terms, "
                    "per-key scales, V dequantized to fp16)"}


def bench_c5(dev, steps, warmup, keep=None):
    """Config 5: fp8 e4m3 KV (per-token fp32 scales) sparse decode, batch 16,
    context 131072 in 64-token pages, 32/8 heads, D=128; the indexer (4 x 64,
    bf16) picks 4096 tokens per sequence."""
    import torch

    from linattn_amd.kernels.block_sparse import fp8_scale_pairs
    from linattn_amd.kernels.paged_decode import indexer_decode_step, quantize_fp8_per_token

    B, Hq, Hkv, T, D, ps, HI, d, topk = 16, 32, 8, 131072, 128, 64, 4, 64, 4096
    P = T // ps
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).bfloat16()
    kc = torch.empty(B * P, Hkv, ps, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.empty_like(kc)
    # each token's K and V scales side by side (one 8-byte pair per token)
    ks, vs = fp8_scale_pairs(B * P, Hkv, ps, dev)
    chunk = 4096
    for dst, sdst in ((kc, ks), (vc, vs)):
        for i in range(0, B * P, chunk):
            n = min(chunk, B * P - i)
            c, s = quantize_fp8_per_token(torch.randn(n, Hkv, ps, D, generator=g, device=dev))
            dst[i:i + n], sdst[i:i + n] = c, s
    pt = torch.randperm(B * P, generator=g, device=dev).view(B, P).to(torch.int32)
    q_idx = torch.randn(B, 1, HI, d, generator=g, device=dev).bfloat16()
    k_idx = torch.randn(B, T, HI, d, generator=g, device=dev).bfloat16()
    w = torch.rand(B, 1, HI, generator=g, device=dev)

    def step():
        return indexer_decode_step(q, kc, vc, pt, q_idx, k_idx, w, topk=topk, pos=T - 1,
                                   page_size=ps, k_scale=ks, v_scale=vs)

    ms = time_cuda(step, steps, warmup)
    if keep is not None:  # host copies of the first C5_CPU_SEQ sequences (contiguous K/V)
        seqs = []
        for b in range(C5_CPU_SEQ):
            rows = pt[b].long()
            seqs.append({
                "q": q[b:b + 1].cpu(), "q_idx": q_idx[b:b + 1].cpu(), "k_idx": k_idx[b:b + 1].cpu(),
                "w": w[b:b + 1].cpu(),
                "kc": kc[rows].permute(1, 0, 2, 3).reshape(1, Hkv, T, D).cpu(),
                "vc": vc[rows].permute(1, 0, 2, 3).reshape(1, Hkv, T, D).cpu(),
                "ks": ks[rows].permute(1, 0, 2).reshape(1, Hkv, T).cpu(),
                "vs": vs[rows].permute(1, 0, 2).reshape(1, Hkv, T).cpu()})
        keep["c5"] = {"seqs": seqs, "topk": topk, "T": T}
    bytes_step = (B * T * HI * d * 2            # indexer keys
                  + B * Hkv * topk * D * 2       # fp8 K and V of the kept tokens
                  + B * Hkv * topk * 2 * 4)      # their scales
    gbs = bytes_step / (ms * 1e-3) / 1e9
    return {"workload": "C5 fp8-KV indexer sparse decode, B=16, T=131072, top-4096",
            "tok_per_s": round(B / (ms * 1e-3), 1), "ms": round(ms, 4),
            "bytes_per_step": bytes_step, "GBps": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def bench_page_bounds(dev, pool_k, pt, mins, maxs, cfg, steps, warmup):
    """Quest metadata built from scratch over the whole C4 key pool (64 x 1024
    pages of 8 KV heads): channel min/max of every page (quest_pages.py:38-48),
    in place.  The step keeps them up to date on append; this is the full
    rebuild a cache load or a prefill does."""
    from linattn_amd.kernels.quest_pages import page_update_hip

    ps = cfg["page"]
    ms = time_cuda(lambda: page_update_hip(pool_k, ps, page_table=pt, out=(mins, maxs)), steps,
                   warmup)
    nbytes = pool_k.numel() * pool_k.element_size() + 2 * mins.numel() * mins.element_size()
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": "Quest page bounds of the C4 key pool (8.6 GB of bf16 keys, 64 x 1024 pages x 8 KV heads)",
            "ms": round(ms, 4), "bytes": nbytes, "GBps": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def bench_serving(dev, q, pool_k, pool_v, pt, mins, maxs, cfg, steps, warmup):
    """C4 shapes as a ragged serving step: every sequence at its own position
    (uniform in [T/2, T-1)) appends one token (K/V into the paged pool, Quest
    page bounds updated in the same kernel), then a ragged Quest decode step
    attends.  Runs after the headline (it writes into the pool)."""
    import torch

    from linattn_amd.kernels.kv_cache import paged_kv_append
    from linattn_amd.kernels.paged_decode import quest_decode_step

    B, Hkv, T, D, ps = cfg["B"], cfg["Hkv"], cfg["T"], cfg["D"], cfg["page"]
    g = torch.Generator(device=dev).manual_seed(1)
    positions = torch.randint(T // 2, T - 1, (B,), generator=g, device=dev).to(torch.int32)
    k_new = torch.randn(B, Hkv, 1, D, generator=g, device=dev).to(torch.bfloat16)
    v_new = torch.randn(B, Hkv, 1, D, generator=g, device=dev).to(torch.bfloat16)

    def append():
        paged_kv_append(k_new, v_new, pool_k, pool_v, pt, positions, page_min=mins,
                        page_max=maxs, page_size=ps)

    def step():
        append()
        quest_decode_step(q, pool_k, pool_v, pt, mins, maxs, page_size=ps, topk=cfg["topk"],
                          positions=positions)

    ms_append = time_cuda(append, steps, warmup)
    ms_step = time_cuda(step, steps, warmup)
    # K, V rows read and written, bounds of the touched page read and written
    append_bytes = B * Hkv * D * 2 * (2 + 2) + B * Hkv * D * 2 * 2 * 2
    return {"workload": "ragged serving step on C4 shapes: append 1 token + page bounds, "
                        "ragged Quest select + attend (positions uniform in [T/2, T-1))",
            "ms_append": round(ms_append, 4), "append_bytes": append_bytes,
            "ms_step": round(ms_step, 4), "tok_per_s": round(B / (ms_step * 1e-3), 1)}


def bench_moba(dev, steps, warmup):
    """MoBA decode (selection.py:610-640; the same routing is NSA's selection
    branch): B=16, 32/8 heads, D=128, T=16384 bf16, 64-token blocks, top-16
    blocks + own block per query head.  The step keeps the fp64 block means
    of K (as hip_moba's state does): it re-pools only the block of the newest
    key, routes on the cached means and attends.  ``ms_route_repool`` is the
    routing that pools every key per call, as the reference does."""
    import torch

    from linattn_amd.kernels.block_sparse import sparse_attention
    from linattn_amd.kernels.routing import block_means_hip, gate_select_hip

    B, Hq, Hkv, T, D, bs, topk = 16, 32, 8, 16384, 128, 64, 16
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=g, device=dev).to(torch.bfloat16)
    kbar = block_means_hip(k, block=bs)
    newest = torch.full((B,), T - 1, dtype=torch.int32, device=dev)

    def refresh():  # the block the step's key joined
        block_means_hip(k, block=bs, out=kbar, positions=newest)

    def route():
        return gate_select_hip(q, k, block=bs, topk=topk, offset=T - 1, kbar=kbar)

    def route_repool():
        return gate_select_hip(q, k, block=bs, topk=topk, offset=T - 1)

    ids, counts = route()
    ids0, counts0 = route_repool()
    same = bool(torch.equal(ids, ids0) and torch.equal(counts, counts0))

    def step():
        refresh()
        i, c = route()
        sparse_attention(q, k, v, i, unit=bs, counts=c, causal=True, offset=T - 1)

    ms_refresh = time_cuda(refresh, steps, warmup)
    ms_route = time_cuda(route, steps, warmup)
    ms_repool = time_cuda(route_repool, steps, warmup)
    ms_step = time_cuda(step, steps, warmup)
    pool_bytes = B * Hkv * T * D * 2
    mean_bytes = kbar.numel() * 8
    att_bytes = int(counts.sum()) * bs * D * 2 * 2
    return {"workload": "MoBA decode, B=16, T=16384, 32/8 heads, D=128, bf16, block 64, top-16",
            "ms_step": round(ms_step, 4), "tok_per_s": round(B / (ms_step * 1e-3), 1),
            "ms_refresh_means": round(ms_refresh, 4), "ms_route": round(ms_route, 4),
            "route_GBps": round(mean_bytes / (ms_route * 1e-3) / 1e9, 1),
            "ms_route_repool": round(ms_repool, 4),
            "repool_GBps": round(pool_bytes / (ms_repool * 1e-3) / 1e9, 1),
            "lists_equal_repool": same, "attend_bytes": att_bytes,
            "note": "block means (fp64, 33.5 MB) kept on append; the refresh re-pools the newest "
                    "key's block of every (b, KV head)"}


def bench_xattn(dev, steps, warmup):
    """XAttention block selection (selection.py:528-595) at its defaults
    (8-token blocks, antidiagonal stride 8, threshold 0.9): B=1, T=8192,
    32/8 heads, D=128, bf16 prefill.  Every (query block, visible key block)
    pair costs 8 antidiagonal dot products of D (fp64, exact)."""
    import torch

    from linattn_amd.kernels.routing import xattn_select_hip

    B, Hq, Hkv, T, D, blk, r = 1, 32, 8, 8192, 128, 8, 8
    g = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn(B, Hq, T, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g, device=dev).to(torch.bfloat16)

    def sel():
        return xattn_select_hip(q, k, block=blk, stride=r, threshold=0.9)

    ids, counts = sel()
    ms = time_cuda(sel, steps, warmup)
    n_qb = T // blk
    pairs = B * Hq * n_qb * (n_qb + 1) // 2
    entries = sum(min(blk - 1, o) - max(0, o - blk + 1) + 1 for o in range(0, 2 * blk - 1, r))
    tflops = pairs * entries * D * 2 / (ms * 1e-3) / 1e12
    return {"workload": "XAttention selection, B=1, T=8192, 32/8 heads, D=128, bf16, "
                        "block 8, stride 8, threshold 0.9",
            "ms_select": round(ms, 4), "blocks_per_row": round(float(counts.float().mean()), 2),
            "frac_causal_blocks_kept": round(int(counts.sum()) / pairs, 4),
            "score_tflops_fp64": round(tflops, 2),
            "frac_fp64_valu_peak": round(tflops / FP64_VALU_PEAK_TFLOPS, 4)}


def _counter_rows(d):
    import csv
    import glob

    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    return list(csv.DictReader(open(files[0])))


def traffic_from(fetch_dir, write_dir):
    """HBM bytes per launch of the C4 step kernel and of the attention kernel
    of the two-launch step from FETCH_SIZE and WRITE_SIZE (KiB per dispatch),
    each scaled by what the same counter reads for the device copy of COPY_MIB
    MiB that --pmc-probe ends with."""
    copy_bytes = COPY_MIB << 20
    for kernel, fname in ((STEP_KERNEL, TRAFFIC_FILE), (ATTN_KERNEL, ATTN_TRAFFIC_FILE)):
        out = {"kernel": kernel, "copy_bytes": copy_bytes}
        for d, name in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
            rows = [r for r in _counter_rows(d) if r["Counter_Name"] == name]
            per = {}  # dispatch -> summed counter (over the counter's dimensions)
            for r in rows:
                if kernel in r["Kernel_Name"]:
                    per[r["Dispatch_Id"]] = per.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
            copies = {}
            for r in rows:
                if "copyBuffer" in r["Kernel_Name"]:
                    copies[r["Dispatch_Id"]] = copies.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
            if not per or not copies:
                raise SystemExit(f"{name}: {kernel} or copy dispatches missing in {d}")
            kern = list(per.values())
            ref = max(copies.values())  # the COPY_MIB copy is the largest copy in the probe
            factor = copy_bytes / (ref * 1024.0)
            out[name] = {"kib_per_launch": sum(kern) / len(kern), "launches": len(kern),
                         "copy_kib": ref, "scale": round(factor, 4),
                         "bytes_per_launch": round(sum(kern) / len(kern) * 1024.0 * factor)}
        out["traffic_bytes"] = out["FETCH_SIZE"]["bytes_per_launch"] + out["WRITE_SIZE"]["bytes_per_launch"]
        out["commands"] = [
            f"rocprofv3 --pmc {c} --output-format csv -d <dir> -o run -- python -u bench.py --pmc-probe"
            for c in ("FETCH_SIZE", "WRITE_SIZE")]
        path = ROOT / fname
        path.write_text(json.dumps(out, indent=1) + "\n")
        print(json.dumps(out))
    return 0


def main() -> int:
    args = parse()
    if args.traffic_from:
        return traffic_from(*args.traffic_from)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        return 2
    import torch

    from linattn_amd.kernels.block_sparse import sparse_attention
    from linattn_amd.kernels.paged_decode import quest_decode_fused
    from linattn_amd.kernels.quest_pages import quest_select_hip

    dev = torch.device("cuda:0")
    global SETTLE_MS
    if args.pmc_workload or args.pmc_probe:
        SETTLE_MS = 0.0  # counter runs profile one warm-up and one timed call
    if args.pmc_workload:
        res = {"c3": bench_c3, "c5": bench_c5}[args.pmc_workload](dev, 1, 1)
        a = torch.empty(COPY_MIB << 20, dtype=torch.uint8, device=dev)
        torch.empty_like(a).copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_workload": args.pmc_workload, "copy_bytes": COPY_MIB << 20, **res}))
        return 0
    cfg = dict(C4)
    union = not args.shared
    q, pool_k, pool_v, pt, mins, maxs = setup_c4(dev, cfg)
    B, Hq, Hkv, T, D, ps = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["T"], cfg["D"], cfg["page"]
    pos = T - 1
    stream = torch.cuda.current_stream(dev)

    def select():
        return quest_select_hip(q, mins, maxs, page_size=ps, topk=cfg["topk"], offset=pos,
                                gqa_union=union)

    def attend(ids, counts):
        return sparse_attention(q, pool_k, pool_v, ids, unit=ps, counts=counts, causal=True,
                                offset=pos, page_table=pt, page_size=ps)

    def two_launch_step():
        ids, counts = select()
        attend(ids, counts)

    def fused_step():
        return quest_decode_fused(q, pool_k, pool_v, pt, mins, maxs, page_size=ps,
                                  topk=cfg["topk"], pos=pos)

    # The step: Quest selection and attention of every (b, KV head) in one
    # kernel (GQA union lists); with per-head lists (--shared) the two launches.
    c4_step = fused_step if union else two_launch_step

    def loop_ms(fn, n):
        """n calls with events only around the loop (an event record between
        kernels costs a few microseconds of idle GPU)."""
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(stream)
        for _ in range(n):
            fn()
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / n

    settle_calls = settle(c4_step)
    for _ in range(args.warmup):
        c4_step()
    torch.cuda.synchronize()
    ms_step = loop_ms(c4_step, args.steps)  # the headline

    # The two-launch step beside it (select, then attend): its time, the
    # split with events around each launch on the launch stream (the event
    # gaps stay inside the per-kernel figures), and the attention launch
    # alone back to back on the last selection (kernel and split combine).
    settle(two_launch_step)
    ms_two = loop_ms(two_launch_step, args.steps)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        ev[i][0].record(stream)
        ids, counts = select()
        ev[i][1].record(stream)
        attend(ids, counts)
        ev[i][2].record(stream)
    torch.cuda.synchronize()
    ms_sel = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps
    ms_att = sum(e[1].elapsed_time(e[2]) for e in ev) / args.steps
    ms_launch = loop_ms(lambda: attend(ids, counts), args.steps)
    lists_equal = None
    if union:
        _, fids, fcounts = fused_step()
        lists_equal = bool(torch.equal(fids, ids) and torch.equal(fcounts, counts))

    # algorithmic bytes, from the actual selection
    n_pages_read = int(counts.sum())  # distinct (b, list head, page) triples
    lists_heads = ids.shape[1]
    kv_row_bytes = D * 2 * 2  # K and V, bf16
    att_bytes = n_pages_read * ps * kv_row_bytes
    if lists_heads == Hq:  # per-query-head lists share KV heads; count distinct pages
        sel = torch.zeros(B, Hkv, T // ps, dtype=torch.bool, device=dev)
        g = Hq // Hkv
        idl = ids.view(B, Hkv, g, -1).clamp(min=0).long().reshape(B, Hkv, -1)
        sel.scatter_(-1, idl, True)
        att_bytes = int(sel.sum()) * ps * kv_row_bytes
    att_bytes += q.numel() * 2 + B * Hq * D * 2 + ids.numel() * 4
    if args.pmc_probe:
        a = torch.empty(COPY_MIB << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": True, "attn_bytes": att_bytes, "copy_bytes": COPY_MIB << 20}))
        return 0

    def traffic_of(fname, kernel):
        tpath = ROOT / fname
        if tpath.exists():
            rec = json.loads(tpath.read_text())
            if rec.get("kernel") == kernel:
                return rec.get("traffic_bytes")
        return None

    # selection traffic: page min+max read, q read, lists and counts written;
    # the fused union selector keeps its fp64 score rows on chip, the per-head
    # form writes them and reads them back for the top-k
    meta_bytes = 2 * mins.numel() * 2 + q.numel() * 2 + ids.numel() * 4 + counts.numel() * 4
    if not (union and Hq > Hkv):
        meta_bytes += B * Hq * (T // ps) * 8 * 2
    step_bytes = att_bytes + meta_bytes
    tok_s = B / (ms_step * 1e-3)
    att_gbs = att_bytes / (ms_launch * 1e-3) / 1e9
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9
    two_gbs = step_bytes / (ms_two * 1e-3) / 1e9
    if union:  # the step is one kernel: its roofline is the step's
        roofline = {"bound": "hbm", "kernel": STEP_KERNEL,
                    "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                    "traffic": traffic_of(TRAFFIC_FILE, STEP_KERNEL),
                    "bytes_per_launch": step_bytes, "ms_per_launch": round(ms_step, 4)}
    else:
        roofline = {"bound": "hbm", "kernel": ATTN_KERNEL + " (+ split combine)",
                    "achieved": round(att_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(att_gbs / HBM_PEAK_GBS, 4),
                    "traffic": traffic_of(ATTN_TRAFFIC_FILE, ATTN_KERNEL),
                    "bytes_per_launch": att_bytes, "ms_per_launch": round(ms_launch, 4)}

    result = {
        "metric": "sparse decode tok/s (paged Quest, 64K ctx, batch 64)",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"ms": SETTLE_MS, "steps": settle_calls,
                   "note": "untimed steps run before the warm-up until the device has run the "
                           "step for this long (its clocks ramp up over ~20 ms of load)"},
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1), seeded; random page table",
        "config": {"workload": "C4 paged Quest sparse decode", "batch": B, "context": T,
                   "page_size": ps, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D,
                   "budget_tokens": cfg["topk"] * ps, "gqa": "union" if union else "per-head",
                   "step": ("quest_decode_fused: page scores, top-k, GQA union and attention in "
                            "one kernel" if union else "quest_select_hip + sparse_attention")},
        "roofline": roofline,
        "step": {"bytes": step_bytes, "GBps": round(step_gbs, 1),
                 "frac_hbm": round(step_gbs / HBM_PEAK_GBS, 4),
                 "pages_read_per_kv_list": round(n_pages_read / (B * lists_heads), 2)},
        "two_launch_step": {"ms": round(ms_two, 4), "tok_per_s": round(B / (ms_two * 1e-3), 1),
                            "GBps": round(two_gbs, 1), "frac_hbm": round(two_gbs / HBM_PEAK_GBS, 4),
                            "ms_select": round(ms_sel, 4), "ms_attend": round(ms_att, 4),
                            "lists_equal_fused": lists_equal,
                            "attention_roofline": {
                                "kernel": ATTN_KERNEL + " (+ split combine)",
                                "achieved": round(att_gbs, 1), "frac": round(att_gbs / HBM_PEAK_GBS, 4),
                                "traffic": traffic_of(ATTN_TRAFFIC_FILE, ATTN_KERNEL),
                                "bytes_per_launch": att_bytes, "ms_per_launch": round(ms_launch, 4)}},
    }
    # side configurations: a few untimed calls first (clocks settle)
    sub, sub_w = max(3, args.steps // 4), 10
    keep = None if args.no_cpu_baseline else {}
    result["page_bounds"] = bench_page_bounds(dev, pool_k, pt, mins, maxs, cfg, sub, sub_w)
    result["indexer"] = bench_c2(dev, sub, sub_w, keep)
    result["prefill"] = bench_c3(dev, sub, sub_w, keep)
    result["fp8_decode"] = bench_c5(dev, sub, sub_w, keep)
    result["moba_decode"] = bench_moba(dev, sub, sub_w)
    result["xattn_select"] = bench_xattn(dev, max(3, args.steps // 10), 3)
    result["serving"] = bench_serving(dev, q, pool_k, pool_v, pt, mins, maxs, cfg, sub, sub_w)
    if not args.no_cpu_baseline:
        cb = cpu_baseline(q, pool_k, pool_v, pt, mins, maxs, cfg, args.cpu_sample, union, keep)
        # achieved GB/s of the decode legs, at the GPU step's algorithmic bytes per token
        for leg, per_tok in (("c4", step_bytes / B),
                             ("c5", result["fp8_decode"]["bytes_per_step"] / 16)):
            if leg in cb["legs"]:
                for lab in ("all", "4"):
                    v = cb["legs"][leg][f"value_{lab}_threads"]
                    cb["legs"][leg][f"GBps_{lab}_threads"] = round(v * per_tok / 1e9, 3)
        result["cpu_baseline"] = cb
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
