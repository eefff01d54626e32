"""Benchmark of the paged decode hot path on one MI355X.

Headline workload: ragged batched decode, Llama-2-7B attention shape --
64 rows with lengths U[128, 8192] (seed 1236), 32 q / 32 kv heads, head_dim
128, fp16, 16-token pages scattered over a pool of (pages + 1024).  One step
is one decode-attention pass over the batch: the device-side plan kernel and
the decode kernel, inputs already resident in HBM.

value = algorithmic bytes per step / measured step time (GB/s), where the
algorithmic bytes are K+V of every valid token + q + o + page tables.  The
roofline object reports the decode kernel alone (per-launch HIP events on
the stream it runs on) against MI355X's 8 TB/s HBM peak.

Also reported: the Qwen3-8B decode-layer latency (1 row x 2048 tokens, 32/8
heads, bf16), the per-layer LoRA delta time of 64 tokens over 4 adapters,
end-to-end tok/s of a Qwen3-8B-shaped random-init decoder with rank-16
no-merge LoRA under hipGraph replay (4 rows behind a 2048-token shared
prefix; 1 row at 32768 tokens), and the CPU baseline (the torch fp32 CPU
path on every host core, on a bounded subset of the headline's rows).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode-attn achieved HBM GB/s (% peak); tok/s Qwen3-8B-shape LoRA decode"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_kernel_ragged64_mha_fp16.traffic.json"


# End-to-end legs: Qwen3-8B-shaped decode with rank-16 LoRA on all 7 modules.
E2E_LEGS = {
    "shared": ("e2e_qwen3_8b_lora_r16_4x(2048_shared+64)", dict(prefix_len=2048, suffix_len=64, rows=4, steps=128)),
    "long": ("e2e_qwen3_8b_lora_r16_1x32768", dict(prefix_len=0, suffix_len=32768, rows=1, steps=128)),
}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=20.0, help="CPU baseline sample budget")
    p.add_argument("--no-extra", action="store_true", help="headline workload only")
    p.add_argument("--no-e2e", action="store_true", help="skip the end-to-end Qwen3-8B-shaped decode legs")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also run a 1 GiB device copy (for scaling rocprofv3 FETCH/WRITE_SIZE)")
    p.add_argument("--e2e-only", choices=sorted(E2E_LEGS),
                   help="run only this end-to-end decode leg and print its result (for profiling)")
    p.add_argument("--lora-only", action="store_true",
                   help="run only the per-layer LoRA delta timing and print its result (for profiling)")
    p.add_argument("--e2e-steps", type=int, default=None,
                   help="decode steps of each timed end-to-end call (default 128; fewer for counter runs)")
    return p.parse_args()


def ragged_mha_workload(device, seed=1236):
    import torch

    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 8193, size=64).tolist()
    ps, h, d = 16, 32, 128
    n_pages = [math.ceil(L / ps) for L in lens]
    total = sum(n_pages)
    pool = total + 1024
    gen = torch.Generator(device=device).manual_seed(seed)
    cache = torch.randn((pool, 2, ps, h, d), device=device, dtype=torch.float16, generator=gen)
    q = (torch.randn((64, h, d), device=device, generator=gen) / math.sqrt(d)).to(torch.float16)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(seed))[:total].to(torch.int32)
    indptr = torch.tensor(np.concatenate([[0], np.cumsum(n_pages)]), dtype=torch.int32)
    last = torch.tensor([L - ps * (n - 1) for L, n in zip(lens, n_pages)], dtype=torch.int32)
    return dict(name="ragged64_mha_fp16", q=q, cache=cache, indptr=indptr, indices=perm, last=last,
                hq=h, hkv=h, d=d, ps=ps, lens=lens, dtype_bytes=2)


def qwen3_layer_workload(device, seed=1235):
    import torch

    ps, hq, hkv, d, pool, L = 16, 32, 8, 128, 4096, 2048
    gen = torch.Generator(device=device).manual_seed(seed)
    cache = torch.randn((pool, 2, ps, hkv, d), device=device, dtype=torch.bfloat16, generator=gen)
    q = torch.randn((1, hq, d), device=device, generator=gen).to(torch.bfloat16)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(seed))[: L // ps].to(torch.int32)
    return dict(name="qwen3_layer_b1_2048_bf16", q=q, cache=cache,
                indptr=torch.tensor([0, L // ps], dtype=torch.int32), indices=perm,
                last=torch.tensor([ps], dtype=torch.int32), hq=hq, hkv=hkv, d=d, ps=ps, lens=[L], dtype_bytes=2)


def algorithmic_bytes(w):
    from oracle.paged_decode import algorithmic_bytes as ab

    return ab(w["indptr"].tolist(), w["last"].tolist(), w["ps"], w["hq"], w["hkv"], w["d"], w["dtype_bytes"], w["dtype_bytes"])


def time_decode(w, steps, warmup):
    """(ms per step, per-launch decode-kernel ms, per-launch merge-kernel ms).

    A step is the plan kernel, the decode kernel and the merge kernel; the
    two run kernels are launched as two calls so HIP events on their stream
    bracket each one.
    """
    import torch

    from pagelora_amd import _lib
    from pagelora_amd.attention_backend import PagedDecodeAttention

    dev = w["q"].device
    be = PagedDecodeAttention(device=dev, workspace_mb=256, num_qo_heads=w["hq"], num_kv_heads=w["hkv"],
                              head_dim=w["d"], page_size=w["ps"])
    be.plan_decode(paged_kv_indptr=w["indptr"], paged_kv_indices=w["indices"], paged_kv_last_page_len=w["last"])
    out = torch.empty_like(w["q"])
    for _ in range(warmup):
        be.replan_decode()
        be.run_decode_into(w["q"], w["cache"], out)
    stream = torch.cuda.current_stream(dev)  # the stream every kernel is launched on
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t0.record(stream)
    for i in range(steps):
        be.replan_decode()
        ev[i][0].record(stream)
        be.run_decode_into(w["q"], w["cache"], out, flags=_lib.PL_DECODE_SKIP_MERGE)
        ev[i][1].record(stream)
        be.run_decode_into(w["q"], w["cache"], out, flags=_lib.PL_DECODE_MERGE_ONLY)
        ev[i][2].record(stream)
    t1.record(stream)
    torch.cuda.synchronize(dev)
    decode = [e[0].elapsed_time(e[1]) for e in ev]
    merge = [e[1].elapsed_time(e[2]) for e in ev]
    return t0.elapsed_time(t1) / steps, decode, merge


def time_decode_spaced(w, steps, warmup, evict_bytes=0):
    """Per-step times of a small decode workload, each step measured on its own.

    A small step (tens of microseconds) is shorter than the host's time to
    issue its three launches, so back-to-back timing would measure the host.
    Each step is therefore preceded by GPU work that keeps the device busy
    while the host queues the step: a spin (warm caches) or, with
    ``evict_bytes``, a fill of that many bytes, which also evicts the step's
    K/V from the L2 and the Infinity Cache (cold caches).  Events bracket the
    plan, decode and merge kernels; returns per-step lists in ms
    (step = plan + decode + merge, decode, merge).
    """
    import torch

    from pagelora_amd import _lib
    from pagelora_amd.attention_backend import PagedDecodeAttention

    dev = w["q"].device
    be = PagedDecodeAttention(device=dev, workspace_mb=256, num_qo_heads=w["hq"], num_kv_heads=w["hkv"],
                              head_dim=w["d"], page_size=w["ps"])
    be.plan_decode(paged_kv_indptr=w["indptr"], paged_kv_indices=w["indices"], paged_kv_last_page_len=w["last"])
    out = torch.empty_like(w["q"])
    junk = torch.empty(evict_bytes, dtype=torch.uint8, device=dev) if evict_bytes else None
    stream = torch.cuda.current_stream(dev)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for i in range(warmup + steps):
        if junk is not None:
            junk.fill_(i & 0xFF)
        else:
            torch.cuda._sleep(200_000)  # ~0.1 ms of spinning while the host queues the step
        e = ev[i - warmup] if i >= warmup else None
        if e: e[0].record(stream)
        be.replan_decode()
        if e: e[1].record(stream)
        be.run_decode_into(w["q"], w["cache"], out, flags=_lib.PL_DECODE_SKIP_MERGE)
        if e: e[2].record(stream)
        be.run_decode_into(w["q"], w["cache"], out, flags=_lib.PL_DECODE_MERGE_ONLY)
        if e: e[3].record(stream)
        if i % 16 == 15:
            torch.cuda.synchronize(dev)  # bounded queue
    torch.cuda.synchronize(dev)
    step = [e[0].elapsed_time(e[3]) for e in ev]
    decode = [e[1].elapsed_time(e[2]) for e in ev]
    merge = [e[2].elapsed_time(e[3]) for e in ev]
    return step, decode, merge


def time_step_graph(w, steps=50, warmup=10, evict_bytes=0):
    """One decode step (plan + decode + merge) captured in a hipGraph and
    replayed behind a spin (warm caches) or a fill of ``evict_bytes`` (cold),
    events only around each replay; returns the median step in us."""
    import torch

    from pagelora_amd.attention_backend import PagedDecodeAttention

    dev = w["q"].device
    be = PagedDecodeAttention(device=dev, workspace_mb=256, num_qo_heads=w["hq"], num_kv_heads=w["hkv"],
                              head_dim=w["d"], page_size=w["ps"])
    be.plan_decode(paged_kv_indptr=w["indptr"], paged_kv_indices=w["indices"], paged_kv_last_page_len=w["last"])
    out = torch.empty_like(w["q"])

    def step():
        be.replan_decode()
        be.run_decode_into(w["q"], w["cache"], out)

    for _ in range(3):
        step()
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    junk = torch.empty(evict_bytes, dtype=torch.uint8, device=dev) if evict_bytes else None
    ts = []
    for i in range(warmup + steps):
        if junk is not None:
            junk.fill_(i & 0xFF)
        else:
            torch.cuda._sleep(200_000)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize(dev)
        if i >= warmup:
            ts.append(a.elapsed_time(b) * 1e3)
    return float(np.median(ts))


def time_lora(device, steps=20, layers=16):
    """Per-layer no-merge LoRA delta: 64 tokens over 4 adapters, r=16, the 7
    Qwen3-8B modules in their 4 groups (q/k/v, o, gate/up, down).  ``layers``
    layers, each with its own x, A, B and outputs (16 x 22.8 MB, more than the
    Infinity Cache holds), are captured in one hipGraph the way a decoder's
    step holds them, and each replay is queued behind a spin so the events
    time the GPU rather than the host's launch rate.  Two forms: the four
    groups in one pl_lora_delta_groups call (two launches per layer), and one
    pl_lora_delta call per group (eight launches per layer).  Returns
    (grouped ms, per-group-calls ms, algorithmic bytes) per layer, medians
    over ``steps`` replays."""
    import torch

    from pagelora_amd.lora import lora_delta_, lora_delta_groups_

    gen = torch.Generator(device=device).manual_seed(1237)
    T, H, I, r, n = 64, 4096, 12288, 16, 4
    ids = torch.randint(0, n, (T,), generator=gen, device=device, dtype=torch.int32)
    model = []
    nbytes = 0
    for layer in range(layers):
        groups = []
        for fin, outs in ((H, [4096, 1024, 1024]), (H, [4096]), (H, [I, I]), (I, [H])):
            x = torch.randn((T, fin), device=device, generator=gen).to(torch.bfloat16)
            mods = []
            for fout in outs:
                A = (torch.randn((n, r, fin), device=device, generator=gen) / fin**0.5).to(torch.bfloat16)
                B = (torch.randn((n, fout, r), device=device, generator=gen) * 0.01).to(torch.bfloat16)
                out = torch.zeros((T, fout), device=device, dtype=torch.bfloat16)
                mods.append((A, B, out, 2.0))
                if layer == 0:
                    nbytes += (A.numel() + B.numel()) * 2 + out.numel() * 4
            if layer == 0:
                nbytes += x.numel() * 2
            groups.append((x, mods))
        model.append(groups)

    def grouped():
        for groups in model:
            lora_delta_groups_(groups, ids)

    def per_group():
        for groups in model:
            for x, mods in groups:
                lora_delta_(x, mods, ids)

    result = []
    for fn in (grouped, per_group):
        for _ in range(2):
            fn()  # sizes the workspace before capture
        torch.cuda.synchronize(device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        ts = []
        for i in range(steps + 2):
            torch.cuda._sleep(1_000_000)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            torch.cuda.synchronize(device)
            if i >= 2:
                ts.append(a.elapsed_time(b) / layers)
        result.append(float(np.median(ts)))
    return result[0], result[1], nbytes


def e2e_decode(device, *, prefix_len, suffix_len, rows, steps, seed=5, warm_steps=2):
    """Qwen3-8B-shaped random-init decoder (36 layers, hidden 4096, 32/8 heads,
    head_dim 128, bf16) with rank-16 LoRA on all 7 modules: ``rows`` requests
    behind a shared ``prefix_len``-token prefix in shared pages plus their own
    ``suffix_len`` random-id tokens, then ``steps`` greedy steps under hipGraph
    replay.  tok/s = generated tokens / decode seconds (the graph is captured
    in a short warm-up call first, outside the timed region).  Timed twice,
    both from the prompts' own context (``prefix_len + suffix_len`` tokens):
    with the page table grown on the device inside the captured step
    (``tok_per_s``, the default path), then packed on the host and uploaded
    every step; after each warm-up and timed call the rows are rewound to
    the prompts (their pages stay allocated, the next call overwrites the
    slots).  Both legs start from the prefill's greedy token, so their
    tokens must agree (``tokens_match``)."""
    import torch

    from pagelora_amd.decoder import QWEN3_8B, DecoderWeights
    from pagelora_amd.generation import BatchGenerator, prefill_requests
    from pagelora_amd.kv_pool import PagedKVPool

    cfg = QWEN3_8B
    w = DecoderWeights(cfg, n_adapters=1, device=device, seed=0)
    print(f"[bench] e2e {rows} x ({prefix_len} shared + {suffix_len}): weights ready", file=sys.stderr, flush=True)
    ps = 16
    pages = (prefix_len + rows * (suffix_len + 2 * (steps + warm_steps) + 16)) // ps + 8 * rows + 8
    pool = PagedKVPool(num_layers=cfg.num_layers, capacity_pages=pages, page_size=ps, num_kv_heads=cfg.num_kv_heads,
                       head_dim=cfg.head_dim, dtype=torch.bfloat16, device=device)
    g = torch.Generator().manual_seed(seed)
    prefix = torch.randint(0, cfg.vocab, (prefix_len,), generator=g) if prefix_len else None
    prompts = [torch.randint(0, cfg.vocab, (suffix_len,), generator=g) for _ in range(rows)]
    t = time.perf_counter()
    reqs, first, _ = prefill_requests(w, pool, prompts, shared_prefix=prefix)
    torch.cuda.synchronize(device)
    prefill_s = time.perf_counter() - t
    print(f"[bench] e2e: prefill {prefill_s:.2f} s", file=sys.stderr, flush=True)
    gen = BatchGenerator(w, pool, use_graph=True)

    def rewind(n):
        for r in reqs:
            r.length -= n

    context = reqs[0].length
    gen.generate(reqs, first, steps=warm_steps, device_tables=True)
    rewind(warm_steps)
    res = gen.generate(reqs, first, steps=steps, device_tables=True)
    rewind(steps)
    print(f"[bench] e2e: {res.decode_tokens_per_s:.1f} tok/s with device tables", file=sys.stderr, flush=True)
    gen.generate(reqs, first, steps=warm_steps)
    rewind(warm_steps)
    host = gen.generate(reqs, first, steps=steps)
    out = {
        "tok_per_s": round(res.decode_tokens_per_s, 1),
        "ms_per_step": round(res.decode_seconds / steps * 1e3, 3),
        "rows": rows,
        "context_at_start": context,
        "steps": steps,
        "hip_graph": res.used_graph,
        "graph_captures": res.graph_captures,
        "page_table": "device (reserve uploads: %d)" % res.extra["reserve_uploads"],
        "host_tables": {"tok_per_s": round(host.decode_tokens_per_s, 1),
                        "ms_per_step": round(host.decode_seconds / steps * 1e3, 3),
                        "context_at_start": context},
        "tokens_match": bool(torch.equal(res.tokens, host.tokens)),
        "prefill_s": round(prefill_s, 2),
    }
    del w, pool, gen
    torch.cuda.empty_cache()
    return out


def _cpu_threads() -> int:
    """Threads for the CPU baseline: every core this process may run on
    (bounded by OMP_NUM_THREADS when the host sets it)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def _median_s(fn, warmup=2, runs=10):
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return float(np.median(ts))


def cpu_baseline(w, budget_s):
    """The torch fp32 CPU path (oracle.torch_cpu) on the host's cores: paged
    gather, fp32 upcast and softmax(q.K^T/sqrt(D)).V per row, over a bounded
    subset of the workload's rows (as many, in row order, as fit ~budget_s
    for 2 warm-ups + 10 timed runs); median of the 10 runs, algorithmic GB/s
    of those rows."""
    import torch

    from oracle import paged_decode as opd
    from oracle import torch_cpu as tc

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    cache = w["cache"].cpu()
    q = w["q"].cpu()
    indptr, indices, last = w["indptr"].numpy(), w["indices"].numpy(), w["last"].numpy()
    # pick the row subset from one pass (which also warms the pages)
    rows, spent = [], 0.0
    for b in range(len(last)):
        t = time.perf_counter()
        tc.paged_decode(q, cache, indptr, indices, last, rows=[b])
        spent += time.perf_counter() - t
        rows.append(b)
        if spent >= budget_s / 12:
            break
    sec = _median_s(lambda: tc.paged_decode(q, cache, indptr, indices, last, rows=rows))
    sub_indptr = [0]
    for b in rows:
        sub_indptr.append(sub_indptr[-1] + int(indptr[b + 1] - indptr[b]))
    nb = opd.algorithmic_bytes(sub_indptr, [int(last[b]) for b in rows], w["ps"], w["hq"], w["hkv"], w["d"], 2, 2)
    return {
        "value": round(nb / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"torch fp32 CPU path (oracle/torch_cpu.py), {threads} threads (os.cpu_count() {os.cpu_count()}); "
                  f"rows 0..{rows[-1]} of the 64 ({sum(w['lens'][b] for b in rows)} of {sum(w['lens'])} tokens), "
                  f"median of 10 after 2 warm-ups: {sec * 1e3:.1f} ms per pass",
    }


def cpu_small_configs():
    """The torch fp32 CPU path on the three small workloads (batch 4 x 512
    tokens fp32, GQA 4; batch 1 x 2048 bf16, GQA 4; the LoRA delta of 64
    tokens over 4 adapters and 7 modules): algorithmic GB/s, the median of
    10 runs after 2 warm-ups, all threads."""
    import torch

    from oracle import paged_decode as opd
    from oracle import torch_cpu as tc

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    res = {}
    for name, B, L, dtype, kvb, seed in (("b4_512_fp32_gqa4", 4, 512, torch.float32, 4, 1234),
                                         ("b1_2048_bf16_gqa4", 1, 2048, torch.bfloat16, 2, 1235)):
        ps, hq, hkv, d = 16, 32, 8, 128
        npg = L // ps
        gen = torch.Generator().manual_seed(seed)
        pool = 256 if B == 4 else 4096
        cache = torch.randn((pool, 2, ps, hkv, d), generator=gen).to(dtype)
        q = torch.randn((B, hq, d), generator=gen).to(dtype)
        indices = torch.randperm(pool, generator=torch.Generator().manual_seed(seed))[: B * npg]
        indptr = list(range(0, B * npg + 1, npg))
        last = [ps] * B
        sec = _median_s(lambda: tc.paged_decode(q, cache, indptr, indices, last))
        nb = opd.algorithmic_bytes(indptr, last, ps, hq, hkv, d, kvb, kvb)
        res[name] = {"GBps": round(float(nb) / sec / 1e9, 3), "ms": round(sec * 1e3, 3), "algorithmic_bytes": int(nb)}
    gen = torch.Generator().manual_seed(1237)
    T, H, I, r, n = 64, 4096, 12288, 16, 4
    ids = torch.randint(0, n, (T,), generator=gen)
    mods, nb = [], 0
    for fin, fout in ((H, 4096), (H, 1024), (H, 1024), (H, 4096), (H, I), (H, I), (I, H)):
        x = torch.randn((T, fin), generator=gen).to(torch.bfloat16)
        A = (torch.randn((n, r, fin), generator=gen) / fin**0.5).to(torch.bfloat16)
        Bm = (torch.randn((n, fout, r), generator=gen) * 0.01).to(torch.bfloat16)
        mods.append((x, A, Bm))
        nb += (A.numel() + Bm.numel()) * 2 + T * fout * 4 + x.numel() * 2
    sec = _median_s(lambda: [tc.lora_delta(x, ids, A, Bm, 2.0, intermediate=torch.bfloat16) for x, A, Bm in mods])
    res["lora_64tok_4adapters_7modules"] = {"GBps": round(float(nb) / sec / 1e9, 3), "ms": round(sec * 1e3, 3),
                                            "algorithmic_bytes": int(nb)}
    res["note"] = (f"torch fp32 CPU path (oracle/torch_cpu.py), {threads} threads, median of 10 after 2 warm-ups; "
                   "same algorithmic-byte definitions as the GPU legs")
    return res


def copy_calibration(device):
    import torch

    x = torch.ones(1 << 30, dtype=torch.uint8, device=device)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize(device)
    print(f"[bench] copy calibration: 3 dispatches of a {1 << 30}-byte device copy", file=sys.stderr)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (every box here has one GPU)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    legs = {k: (name, dict(kw, steps=args.e2e_steps or kw["steps"])) for k, (name, kw) in E2E_LEGS.items()}
    if args.copy_calibration and (args.e2e_only or args.lora_only):
        copy_calibration(dev)
    if args.e2e_only:
        name, kw = legs[args.e2e_only]
        print(json.dumps({"leg": name, **e2e_decode(dev, **kw)}), flush=True)
        return
    if args.lora_only:
        grouped, per_group, nbytes = time_lora(dev)
        print(json.dumps({"leg": "lora_delta_64tok_4adapters_7modules", "us_per_layer": round(grouped * 1e3, 2),
                          "us_per_layer_one_call_per_group": round(per_group * 1e3, 2),
                          "algorithmic_bytes": nbytes}), flush=True)
        return
    if args.copy_calibration:
        copy_calibration(dev)

    w = ragged_mha_workload(dev)
    nbytes = algorithmic_bytes(w)
    ms_step, per_launch, merge_ms = time_decode(w, args.steps, args.warmup)
    kern_ms = float(np.mean(per_launch))
    value = nbytes / (ms_step * 1e-3) / 1e9
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
    extra = {
        "decode_kernel_us": round(kern_ms * 1e3, 2),
        "decode_kernel_us_min": round(min(per_launch) * 1e3, 2),
        "merge_kernel_us": round(float(np.mean(merge_ms)) * 1e3, 2),
        "algorithmic_bytes_per_step": nbytes,
        "tokens": int(sum(w["lens"])),
    }
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w, args.cpu_seconds)
        if not args.no_extra:
            extra["cpu_oracle_small_configs"] = cpu_small_configs()
    del w
    torch.cuda.empty_cache()
    if not args.no_extra:
        w2 = qwen3_layer_workload(dev)
        nb2 = algorithmic_bytes(w2)
        leg = {"algorithmic_bytes": nb2,
               "timing": "events around each kernel, the step queued behind GPU work; step_us_graph: the step "
                         "(plan + decode + merge; batches of up to 16 rows launch no plan kernel) captured in a "
                         "hipGraph, events around each replay"}
        for tag, evict in (("warm", 0), ("cold", 512 << 20)):
            st2, per2, merge2 = time_decode_spaced(w2, max(args.steps, 100), args.warmup, evict_bytes=evict)
            dk = float(np.median(per2))
            leg[tag] = {
                "decode_kernel_us": round(dk * 1e3, 2),
                "merge_kernel_us": round(float(np.median(merge2)) * 1e3, 2),
                "step_us_incl_plan": round(float(np.median(st2)) * 1e3, 2),
                "algorithmic_GBps": round(nb2 / (dk * 1e-3) / 1e9, 1),
                "step_us_graph": round(time_step_graph(w2, evict_bytes=evict), 2),
            }
        leg["cold"]["note"] = "a 512 MiB fill before each step evicts the K/V from the L2 and the 256 MB Infinity Cache"
        extra["qwen3_layer_b1_2048_bf16"] = leg
        del w2
        torch.cuda.empty_cache()
        lora_ms, lora_each_ms, lora_bytes = time_lora(dev)
        extra["lora_delta_64tok_4adapters_7modules"] = {
            "us_per_layer": round(lora_ms * 1e3, 2),
            "algorithmic_GBps": round(lora_bytes / (lora_ms * 1e-3) / 1e9, 1),
            "algorithmic_bytes": lora_bytes,
            "form": "the layer's 4 groups in one pl_lora_delta_groups call (2 launches); 16 distinct layers in "
                    "one hipGraph, replayed behind a spin",
            "us_per_layer_one_call_per_group": round(lora_each_ms * 1e3, 2),
        }
    if not args.no_extra and not args.no_e2e:
        for name, kw in legs.values():
            extra[name] = e2e_decode(dev, **kw)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "ragged batched paged decode attention, Llama-2-7B shape: batch 64, seq lens U[128,8192] "
                        "(seed 1236), 32 q / 32 kv heads, head_dim 128, fp16, page_size 16, random pages in a "
                        "pool of pages+1024",
            "global_batch": 64,
            "page_size": 16,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
