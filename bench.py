"""Paged-attention decode benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

A step is one call of the paged-attention op on one batch (config c2 by
default: decode, B=32, Qwen2.5-0.5B heads 14/2/64, block 16, fp16, lognormal
contexts).  Inputs are resident in HBM before timing.  The op is called on R
independent replicas (caches, tables, queries) whose combined footprint is
>= 1.2 GB, cycled in order, so KV is read from HBM and not from the 256 MB
Infinity Cache.  The K timed calls are replayed from a HIP graph captured over
the R replicas (a serving loop issues them the same way), bracketed by
device synchronisation, and timed with HIP events on the launch stream.

Prints one JSON line: value = algorithmic KV GB/s (sum_i 2*L_i*Hkv*D*itemsize
per call / time per call), plus us/call, % of the 8 TB/s HBM peak, the
reshape_and_cache time for the batch's new tokens, and a CPU baseline: the
repo's torch gather+SDPA oracle timed on this host on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

METRIC = "paged-attn decode HBM GB/s (% of peak) + µs/call, B=32 Qwen-0.5B heads"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"fp16": 2500.0, "bf16": 2500.0}

WORKLOADS = {
    "c1": "decode B=8 ctx U[64,512] Hq14/Hkv2/D64 block16 fp16, 256-block pool",
    "c2": "decode B=32 ctx lognormal(1024,0.8) clip[16,8192] Hq14/Hkv2/D64 block16 fp16, pool 1.25x",
    "c3": "mixed: 28 decode (lognormal 1024,0.8) + 4x512-token prefill chunks on ctx U[0,2048], "
          "Hq14/Hkv2/D64 block16 fp16, T=2076",
    "c4": "decode B=64 ctx lognormal(4096,1.0) clip[128,32768] Hq28/Hkv4/D128 bf16",
}


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--block-size", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--replica-gb", type=float, default=1.2,
                    help="minimum combined footprint of the replicas cycled through")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-calls", type=int, default=20)
    ap.add_argument("--eager", action="store_true", help="also time K eager (non-graph) calls")
    return ap.parse_args(argv)


def _case_bytes(case) -> int:
    t = [case.query, case.k_cache, case.v_cache, case.md.block_tables]
    return sum(x.numel() * x.element_size() for x in t)


def _cpu_baseline(case_gpu, calls, gpu_out):
    """Time the repo's torch gather+SDPA oracle on this host (bounded sample).

    The sample is the benchmarked replica itself, copied to host memory, so
    the parity gate compares the GPU output with the oracle on identical inputs.
    """
    import torch

    from nanoserve_amd.attention import AttentionMetadata
    from oracle.paged_attention import paged_attention_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    md = case_gpu.md
    md_cpu = AttentionMetadata(**{k: (v.cpu() if isinstance(v, torch.Tensor) else v)
                                  for k, v in md.__dict__.items()})
    q, kc, vc = case_gpu.query.cpu(), case_gpu.k_cache.cpu(), case_gpu.v_cache.cpu()
    # Parity gate for the benchmarked replica: fp32-accumulated oracle vs the GPU output.
    ref = paged_attention_ref(q, kc, vc, md_cpu, case_gpu.scale)
    err = (gpu_out.float().cpu() - ref).abs().max().item()
    for _ in range(3):
        paged_attention_ref(q, kc, vc, md_cpu, case_gpu.scale, upcast=False)
    ts = []
    t_end = time.perf_counter() + 30.0
    for _ in range(calls):
        t0 = time.perf_counter()
        paged_attention_ref(q, kc, vc, md_cpu, case_gpu.scale, upcast=False)
        ts.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end:
            break
    med = statistics.median(ts)
    return {
        "value": case_gpu.kv_bytes() / med / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "ms_per_call": med * 1e3,
        "sample": f"{case_gpu.config} seed {case_gpu.seed} (the first benchmarked replica): median of "
                  f"{len(ts)} calls after 3 warm-up, torch gather+SDPA in "
                  f"{str(q.dtype).replace('torch.', '')} on {torch.get_num_threads()} threads "
                  f"({platform.processor() or platform.machine()})",
    }, err


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share: --gpus {args.gpus} is not supported "
              "(the attention path shards by sequence with no collective; run N=1)", file=sys.stderr)
        return 2

    import torch

    from nanoserve_amd import paged_attention_hip, reshape_and_cache
    from nanoserve_amd.workloads import make_case

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # ---- replicas ---------------------------------------------------------
    cases, total = [], 0
    while total < args.replica_gb * 1e9 or len(cases) < 2:
        c = make_case(args.config, seed=args.seed + len(cases), device=dev, gen_device=dev,
                      block_size=args.block_size)
        cases.append(c)
        total += _case_bytes(c)
    R = len(cases)
    dtype = cases[0].query.dtype
    dname = {torch.float16: "fp16", torch.bfloat16: "bf16"}[dtype]
    kv_bytes = [c.kv_bytes() for c in cases]

    # New-token K/V of each replica for the cache-write timing.
    news = []
    for c in cases:
        g = torch.Generator(device=dev).manual_seed(c.seed + 100)
        shape = (c.md.num_tokens, c.num_kv_heads, c.head_dim)
        news.append((torch.randn(shape, generator=g, device=dev).to(dtype),
                     torch.randn(shape, generator=g, device=dev).to(dtype)))

    def attn(i):
        c = cases[i]
        return paged_attention_hip(c.query, c.k_cache, c.v_cache, c.md, c.scale)

    def write(i):
        c = cases[i]
        reshape_and_cache(news[i][0], news[i][1], c.k_cache, c.v_cache, c.md.slot_mapping)

    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        # Write-then-attend, as the model's call site does: every replica's
        # new-token K/V goes in first.  Rewriting the same rows later leaves
        # the caches unchanged, so first_out stays the output of replica 0.
        for i in range(R):
            write(i)
        first_out = attn(0).clone()
        for w in range(max(args.warmup, R)):
            attn(w % R)
            write(w % R)
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize()

    def capture(fn, idxs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in idxs:
                fn(i)
        return g

    K = args.steps
    full, rem = divmod(K, R)
    g_attn = capture(attn, range(R))
    g_attn_rem = capture(attn, range(rem)) if rem else None
    g_write = capture(write, range(R))

    def timed(graph, graph_rem, reps):
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            graph.replay()
        if graph_rem is not None:
            graph_rem.replay()
        end.record()
        end.synchronize()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e-3

    t_attn = timed(g_attn, g_attn_rem, full)
    bytes_total = full * sum(kv_bytes) + sum(kv_bytes[:rem])
    s_per_call = t_attn / K
    gbs = bytes_total / t_attn / 1e9

    t_write = timed(g_write, None, max(1, K // R))
    write_us = t_write / (max(1, K // R) * R) * 1e6

    eager_us = None
    if args.eager:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(K):
            attn(k % R)
        torch.cuda.synchronize()
        eager_us = (time.perf_counter() - t0) / K * 1e6

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": s_per_call * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: {WORKLOADS[args.config]}",
            "block_size": cases[0].k_cache.shape[1],
            "global_batch": cases[0].md.num_seqs,
            "tokens_per_call": cases[0].md.num_tokens,
            "replicas": R,
            "replica_footprint_gb": round(total / 1e9, 3),
            "seeds": f"{args.seed}..{args.seed + R - 1}",
            "kv_bytes_per_call_mean": sum(kv_bytes) / R,
            "timing": "HIP-graph replay of K calls cycling the replicas, hipEvents on the launch stream",
        },
        "us_per_call": round(s_per_call * 1e6, 3),
        "pct_of_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
        "reshape_and_cache_us": round(write_us, 3),
    }
    if args.config == "c3":
        flops = sum(c.prefill_flops() for c in cases) / R
        result["prefill_flops_per_call"] = flops
        result["mfma_tflops"] = round(flops / s_per_call / 1e12, 2)
    if eager_us is not None:
        result["eager_us_per_call"] = round(eager_us, 2)
    if not args.no_cpu_baseline:
        cpu, err = _cpu_baseline(cases[0], args.cpu_calls, first_out)
        result["cpu_baseline"] = cpu
        result["max_abs_err_vs_oracle"] = err
        tol = 2e-3 if dtype == torch.float16 else 1e-2
        if not err <= tol:
            print(f"parity gate failed: max abs err {err:.3e} > {tol}", file=sys.stderr)
            print(json.dumps(result))
            return 1
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
