"""Paged-attention decode benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

A step is one serving step's worth of the paged-attention op: the engine
builds one AttentionMetadata (block tables, lengths) per step and every layer
of the model calls attention with it on that layer's own K/V cache and
queries (reference qwen2.py:105-113, model_runner.py:85-168).  So a step here
is --layers (24, Qwen2.5-0.5B) calls on one batch (config c2 by default:
decode, B=32, Qwen2.5-0.5B heads 14/2/64, block 16, fp16, lognormal
contexts), each with its own freshly drawn caches and queries.  The benchmark
holds several distinct steps (different seeds, i.e. different length draws
and block tables), enough that their caches together exceed 1.2 GB, so K/V
are always read from HBM and not from the 256 MB Infinity Cache.  Inputs are
resident in HBM before timing.

Exactly K steps are timed: they are replayed from HIP graphs captured over
the steps (a serving loop issues them the same way), cycling the distinct
steps, bracketed by device synchronisation and timed with HIP events on the
launch stream.  --cold adds a pass in which every call has its own metadata
too (nothing shared, every table read cold).

Prints one JSON line: value = algorithmic KV GB/s (sum_i 2*L_i*Hkv*D*itemsize
per call, summed over the timed calls / time), plus us per call, % of the
8 TB/s HBM peak, the reshape_and_cache time for the batch's new tokens, and a
CPU baseline: the repo's torch gather+SDPA oracle timed on this host on a
bounded sample.

Other modes: --config c5 runs the engine benchmark (config 5), --floors the
launch and streaming-read floors, --ref-grid the reference's own grid of
uniform-context decode shapes, --copy-calibration the known-size copy that
scales rocprofv3 byte counters.
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
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA

WORKLOADS = {
    "c1": "decode B=8 ctx U[64,512] Hq14/Hkv2/D64 block16 fp16, 256-block pool",
    "c2": "decode B=32 ctx lognormal(1024,0.8) clip[16,8192] Hq14/Hkv2/D64 block16 fp16, pool 1.25x",
    "c3": "mixed: 28 decode (lognormal 1024,0.8) + 4x512-token prefill chunks on ctx U[0,2048], "
          "Hq14/Hkv2/D64 block16 fp16, T=2076",
    "c4": "decode B=64 ctx lognormal(4096,1.0) clip[128,32768] Hq28/Hkv4/D128 bf16",
    "c5": "engine: Qwen2.5-0.5B architecture, random-init weights quantised to INT4 g128 (lm_head fp16), "
          "32 concurrent requests, prompts lognormal(256,0.7) clip[16,2048], outputs lognormal(128,0.7) "
          "clip[8,1024], greedy, ignore_eos, fp16, block 16",
}
C5_METRIC = "engine output tok/s + p99 TPOT, Qwen2.5-0.5B INT4 g128, 32 lognormal requests"


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="serving steps timed (each --layers calls)")
    ap.add_argument("--warmup", type=int, default=20, help="serving steps replayed before timing")
    ap.add_argument("--config", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--block-size", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--layers", type=int, default=24,
                    help="attention calls per serving step sharing one metadata (Qwen2.5-0.5B: 24)")
    ap.add_argument("--min-steps", type=int, default=4, help="distinct serving steps (length draws)")
    ap.add_argument("--replica-gb", type=float, default=1.2,
                    help="minimum combined K/V footprint of the calls cycled through")
    ap.add_argument("--cold", action="store_true",
                    help="also time steps whose calls each have their own metadata (cold metadata)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-calls", type=int, default=20)
    ap.add_argument("--eager", action="store_true", help="also time K eager (non-graph) calls")
    ap.add_argument("--floors", action="store_true",
                    help="only time an empty launch and streaming reads of c2's byte counts and exit")
    ap.add_argument("--ref-grid", action="store_true",
                    help="only run the reference's B x uniform-ctx grid (with its correctness gate) and exit")
    ap.add_argument("--int4-gemm", action="store_true",
                    help="only time ns_int4_linear on the Qwen2.5-0.5B projections at prefill sizes "
                         "(and the reference's dequantise + library GEMM steps beside it) and exit")
    ap.add_argument("--copy-calibration", type=float, default=None, metavar="MB",
                    help="only run 5 plain device copies of MB megabytes (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings) and exit")
    return ap.parse_args(argv)


def _bench_engine(torch, args):
    """Config 5: the whole serving loop with the HIP kernels inside the model."""
    from nanoserve_amd.engine import LLMEngine, SamplingParams, SchedulerConfig, summarize
    from nanoserve_amd.model import Qwen2Config, Qwen2ForCausalLM, random_init_
    from nanoserve_amd.quant import quantize_model
    from nanoserve_amd.workloads import c5_requests

    cfg = Qwen2Config()
    model = random_init_(Qwen2ForCausalLM(cfg, max_position=4096), std=0.02, seed=args.seed)
    model = model.half().to("cuda")
    qreport = quantize_model(model, 128, skip=("lm_head",))
    model.fuse_projections()
    block_size = args.block_size or 16

    reqs = c5_requests(32, args.seed, cfg.vocab_size)

    def run(use_graphs):
        eng = LLMEngine(model, num_blocks=8192, block_size=block_size, device="cuda",
                        scheduler_config=SchedulerConfig(max_num_batched_tokens=2048, max_num_seqs=256),
                        max_model_len=4096, use_graphs=use_graphs)
        if use_graphs:
            eng.runner.graphs.capture_all()  # capture is set-up, not serving time
        # Warm-up: a short run of the same shape mix (kernels, allocator, workspaces).
        for toks, n in c5_requests(8, args.seed + 7, cfg.vocab_size):
            eng.add_request(toks[:64], SamplingParams(max_new_tokens=min(n, 16), ignore_eos=True))
        eng.run_all()
        eng.finished.clear()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for toks, n in reqs:
            eng.add_request(toks, SamplingParams(max_new_tokens=n, ignore_eos=True))
        steps = 0
        while eng.has_unfinished_requests:
            eng.step()
            steps += 1
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        summ = summarize([s.metrics for s in eng.finished], wall)
        return summ, steps, wall, eng.scheduler.num_preemptions

    eager, _, eager_wall, _ = run(False)
    summ, steps, wall, preemptions = run(True)
    result = {
        "metric": C5_METRIC,
        "value": round(summ["output_tok_per_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": wall / steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 activations, int4 g128 weights",
        "data": "synthetic (random-init weights, random token ids)",
        "config": {"workload": f"c5: {WORKLOADS['c5']}", "requests": 32,
                   "prompt_tokens": summ["prompt_tokens"], "output_tokens": summ["output_tokens"],
                   "max_num_batched_tokens": 2048, "block_size": block_size},
        "tpot_p50_ms": round(summ["tpot_p50_ms"], 3),
        "tpot_p99_ms": round(summ["tpot_p99_ms"], 3),
        "ttft_p50_ms": round(summ["ttft_p50_ms"], 2),
        "ttft_p99_ms": round(summ["ttft_p99_ms"], 2),
        "e2e_p99_ms": round(summ["e2e_p99_ms"], 2),
        "wall_time_s": round(wall, 3),
        "preemptions": preemptions,
        "decode_steps": "HIP-graph replay of the whole decode step (one graph per batch bucket)",
        "eager_engine": {"output_tok_per_s": round(eager["output_tok_per_s"], 2),
                         "tpot_p99_ms": round(eager["tpot_p99_ms"], 3), "wall_time_s": round(eager_wall, 3)},
        "weights": {k: round(v, 2) if isinstance(v, float) else v for k, v in qreport.items()},
    }
    print(json.dumps(result))
    return 0


def _copy_calibration(torch, mb):
    n = int(mb * 1e6) // 16 * 16
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "kib": n / 1024, "copies": 5}))
    return 0


def graph_capture(graph, stream=None, pool=None):
    """nanoserve_amd.capture.graph_capture (imported on use: torch loads late here)."""
    from nanoserve_amd.capture import graph_capture as capture

    return capture(graph, stream=stream, pool=pool)


def _graph_time(torch, stream, launch, n, reps=3):
    """Seconds per launch of `launch(i)` for i in [0, n), captured in one HIP
    graph and replayed (best of `reps` timed replays after one warm replay)."""
    with torch.cuda.stream(stream):
        for i in range(n):
            launch(i)
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with graph_capture(g, stream=stream):
        for i in range(n):
            launch(i)
    best = float("inf")
    with torch.cuda.stream(stream):
        g.replay()
        stream.synchronize()
        for _ in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            g.replay()
            end.record(stream)
            end.synchronize()
            best = min(best, start.elapsed_time(end) * 1e-3 / n)
    return best


def _int4_gemm(torch, args):
    """int4_linear at prefill token counts on the Qwen2.5-0.5B projections (fp16
    activations, INT4 g128 weights, each projection with the epilogue the model
    gives it), graph-replayed: as Int4Linear calls it inside a captured graph
    (method "auto", the figure the line reports), the tiled GEMM alone
    ("fused", what "auto" runs eagerly), and the reference's
    QuantLinear steps (dequantize_int4 then F.linear, then the epilogue as tensor
    ops) on the same operands.  The HIP calls run with a split-K workspace, as
    Int4Linear does."""
    from nanoserve_amd.quant import int4_linear, quantize_int4_groupwise, splitk_workspace_bytes

    stream = torch.cuda.Stream()
    gen = torch.Generator().manual_seed(args.seed)
    rows = []
    for name, K, N, epi in (("qkv", 896, 1152, "bias"), ("o_proj", 896, 896, "residual"),
                            ("gate_up", 896, 9728, "silu_mul"), ("down_proj", 4864, 896, "residual")):
        packed, scales, zeros = (t.to("cuda") for t in
                                 quantize_int4_groupwise(torch.randn(N, K, generator=gen) * 0.05, 128))
        ws = torch.zeros(max(splitk_workspace_bytes(N, K), 256), dtype=torch.uint8, device="cuda")
        for M in (256, 1024, 2048):
            x = torch.randn(M, K, generator=gen).half().to("cuda")
            bias = (torch.randn(N, generator=gen) * 0.1).half().to("cuda") if epi == "bias" else None
            res = torch.randn(M, N, generator=gen).half().to("cuda") if epi == "residual" else None
            t = {}
            # "dequant" first: its eager warm-up takes the weight scratch that
            # "auto" may use inside a capture.
            for method in ("dequant", "fused", "auto"):
                def launch(i, method=method):
                    int4_linear(x, packed, scales, zeros, bias, 128, residual=res, silu_mul=epi == "silu_mul",
                                method=method, workspace=ws if method != "dequant" else None)
                t[method] = _graph_time(torch, stream, launch, 20)
            flops = 2 * M * N * K
            rows.append({"proj": name, "tokens": M, "N": N, "K": K, "epilogue": epi,
                         "us": round(t["auto"] * 1e6, 2), "tflops": round(flops / t["auto"] / 1e12, 1),
                         "frac_of_mfma_peak": round(flops / t["auto"] / 1e12 / MFMA_PEAK_TFLOPS, 4),
                         "tiled_gemm_us": round(t["fused"] * 1e6, 2),
                         "reference_steps_us": round(t["dequant"] * 1e6, 2)})
    print(json.dumps({"int4_gemm": rows, "device": torch.cuda.get_device_name(0),
                      "timing": "HIP-graph replay of 20 back-to-back calls, hipEvents, best of 3",
                      "mfma_peak_tflops": MFMA_PEAK_TFLOPS,
                      "reference_steps": "ns_int4_dequantize + torch F.linear (hipBLASLt) + epilogue ops"}))
    return 0


def _floors(torch, args):
    """What any kernel pays on this device, graph-replayed back to back: an empty
    launch, and one streaming read of N bytes from HBM (each launch reads its own
    slice of a pool larger than the 256 MB MALL), for c2's byte counts and a
    large read.  ns_stream_read (csrc/floors.hip, a library of its own that only
    this mode loads) is the kernel for both."""
    import ctypes

    from nanoserve_amd import _build, _lib

    if not _build.FLOORS_LIB_PATH.exists():
        raise FileNotFoundError(f"{_build.FLOORS_LIB_PATH} is not built (python -m nanoserve_amd._build)")
    lib = ctypes.CDLL(str(_build.FLOORS_LIB_PATH))
    lib.ns_stream_read.restype = ctypes.c_int
    lib.ns_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    stream = torch.cuda.Stream()
    sink = torch.zeros(65536, dtype=torch.int32, device="cuda")
    pool_bytes = int(args.replica_gb * 1e9) // 4096 * 4096
    pool = torch.randint(0, 255, (pool_bytes,), dtype=torch.uint8, device="cuda")
    rows = []
    for grid in (256, 512, 1024):
        t = _graph_time(torch, stream, lambda i: _lib.check(
            lib.ns_stream_read(None, 0, sink.data_ptr(), grid, stream.cuda_stream), "ns_stream_read"), 200)
        rows.append({"what": "empty launch", "grid": grid, "us_per_launch": round(t * 1e6, 3)})
    c2_seed0, c2_mean = 18_071_552, 21_328_640  # algorithmic K/V bytes of the c2 calls (seed 0; four seeds)
    for nbytes in (c2_seed0, c2_mean, 64 << 20, 1 << 30):
        nbytes = nbytes // 16 * 16
        per = max(1, min(pool_bytes // nbytes, 200))
        best = None
        for grid in (256, 512, 1024, 2048, 4096):
            def launch(i, nbytes=nbytes, grid=grid):
                src = pool.data_ptr() + (i % per) * nbytes
                _lib.check(lib.ns_stream_read(src, nbytes, sink.data_ptr(), grid, stream.cuda_stream),
                           "ns_stream_read")
            t = _graph_time(torch, stream, launch, per if nbytes < (256 << 20) else 2)
            if best is None or t < best[1]:
                best = (grid, t)
        grid, t = best
        rows.append({"what": "streaming read", "bytes": nbytes, "best_grid": grid,
                     "us_per_launch": round(t * 1e6, 3), "gbs": round(nbytes / t / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)})
    print(json.dumps({"floors": rows, "device": torch.cuda.get_device_name(0),
                      "timing": "HIP-graph replay of back-to-back launches, hipEvents, best of 3"}))
    return 0


def _uniform_case(torch, batch, ctx, dev):
    """The reference's grid case (bench/bench_attention.py:83-121): `batch`
    sequences of exactly `ctx` tokens, Hq14/Hkv2/D64, block 16, fp16, caches of
    exactly the blocks needed, block tables a seeded random permutation (int32)."""
    from nanoserve_amd.workloads import PagedCase, metadata_for

    bs, hq, hkv, d = 16, 14, 2, 64
    per = -(-ctx // bs)
    nb = batch * per
    g = torch.Generator().manual_seed(0)
    kc = torch.randn(nb, bs, hkv, d, generator=g).half().to(dev)
    vc = torch.randn(nb, bs, hkv, d, generator=g).half().to(dev)
    perm = torch.randperm(nb, generator=g).tolist()
    tables = [perm[i * per:(i + 1) * per] for i in range(batch)]
    q = torch.randn(batch, hq, d, generator=g).half().to(dev)
    md = metadata_for([ctx] * batch, [1] * batch, tables, bs, dev, index_dtype=torch.int32)
    return PagedCase("grid", 0, q, kc, vc, md, 1.0 / math.sqrt(d), [ctx] * batch, [1] * batch, tables)


def _ref_grid(torch, args):
    """The reference's measurement grid on this GPU: B in {1, 8, 32} x uniform
    ctx in {128, 512, 1024, 2048, 4096}, with its correctness gate before timing
    (reference bench/bench_attention.py:124-240).  Like the reference, each
    case's caches are reused by every timed call (so small cases run from the
    MALL); times are HIP-graph replays of 50 calls and eager calls through the
    Python shim, after 10 warm-up calls."""
    from nanoserve_amd import paged_attention_hip

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    rows = []
    for batch in (1, 8, 32):
        for ctx in (128, 512, 1024, 2048, 4096):
            case = _uniform_case(torch, batch, ctx, dev)
            out = paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale)
            err = _oracle_err(case, out)
            row = {"batch": batch, "ctx": ctx, "max_abs_err_vs_oracle": err}
            if not err <= 2e-3:
                row["status"] = "MISMATCH"
                rows.append(row)
                continue
            call = lambda i: paged_attention_hip(case.query, case.k_cache, case.v_cache, case.md, case.scale)
            t_graph = _graph_time(torch, stream, call, 50)
            with torch.cuda.stream(stream):
                for i in range(10):
                    call(i)
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record(stream)
                for i in range(50):
                    call(i)
                end.record(stream)
            end.synchronize()
            t_eager = start.elapsed_time(end) * 1e-3 / 50
            kv = 2 * batch * ctx * 2 * 64 * 2  # bench_attention.py:178-180
            row.update({"kv_bytes": kv, "graph_us": round(t_graph * 1e6, 3), "eager_us": round(t_eager * 1e6, 3),
                        "graph_gbs": round(kv / t_graph / 1e9, 1), "eager_gbs": round(kv / t_eager / 1e9, 1)})
            rows.append(row)
            print(json.dumps(row), flush=True)
            del case
    print(json.dumps({"ref_grid": rows, "device": torch.cuda.get_device_name(0)}))
    return 1 if any(r.get("status") == "MISMATCH" for r in rows) else 0


def _profiled_traffic(args):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE + WRITE_SIZE for
    this exact workload (profiles/paged_decode_<config>_traffic.md), or None."""
    if (args.seed != 0 or args.block_size is not None or args.layers != 24 or args.min_steps != 4
            or args.steps % args.min_steps):
        return None, None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"paged_decode_{args.config}_traffic.md")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        if line.startswith("machine-readable:"):
            kv = dict(tok.split("=") for tok in line.split(":", 1)[1].split())
            return int(kv["traffic_bytes_per_launch"]), os.path.relpath(path, os.path.dirname(path) + "/..")
    return None, None


def _kv_footprint(case) -> int:
    return case.k_cache.numel() * case.k_cache.element_size() * 2


def _cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo), else the machine type."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _cpu_baseline(case_gpu, calls, gpu_out):
    """Time the repo's torch gather+SDPA oracle on this host (bounded sample).

    The sample is the first benchmarked call itself, copied to host memory, so
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
    # Parity gate for the benchmarked call: fp32-accumulated oracle vs the GPU output.
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
        "sample": f"{case_gpu.config} seed {case_gpu.seed} (the first benchmarked call): median of "
                  f"{len(ts)} calls after 3 warm-up, torch gather+SDPA in "
                  f"{str(q.dtype).replace('torch.', '')} on {torch.get_num_threads()} threads "
                  f"({_cpu_model()})",
    }, err


def _oracle_err(case_gpu, gpu_out):
    """Max abs difference between a GPU output and the fp32 CPU oracle on the same inputs."""
    import torch

    from nanoserve_amd.attention import AttentionMetadata
    from oracle.paged_attention import paged_attention_ref

    md = case_gpu.md
    md_cpu = AttentionMetadata(**{k: (v.cpu() if isinstance(v, torch.Tensor) else v)
                                  for k, v in md.__dict__.items()})
    ref = paged_attention_ref(case_gpu.query.cpu(), case_gpu.k_cache.cpu(), case_gpu.v_cache.cpu(),
                              md_cpu, case_gpu.scale)
    return (gpu_out.float().cpu() - ref).abs().max().item()


def _build_steps(args, dev, shared):
    """Serving steps to cycle through.  With shared=True a step is --layers
    attention calls that share one metadata (lengths, block tables) but each
    have their own K/V caches, as the layers of one engine step do
    (reference qwen2.py:105-113); with shared=False every call of the step has
    its own metadata too.  Steps are added until their combined K/V footprint
    exceeds --replica-gb (so K/V come from HBM, not the 256 MB MALL) and
    there are at least --min-steps of them."""
    from nanoserve_amd.workloads import make_case, make_layer

    steps, total, j = [], 0, 0
    while total < args.replica_gb * 1e9 or j < args.min_steps:
        calls = []
        for layer in range(args.layers):
            if layer == 0 or not shared:
                seed = args.seed + j if layer == 0 else 10_000 + 1000 * (args.seed + j) + layer
                c = make_case(args.config, seed=seed, device=dev, gen_device=dev, block_size=args.block_size)
            else:
                c = make_layer(calls[0], seed=1000 * (args.seed + j) + layer, gen_device=dev)
            calls.append(c)
            total += _kv_footprint(c)
        steps.append(calls)
        j += 1
    return steps, total


def _rope_inputs(torch, calls, news):
    """Per call: a q output buffer and cos/sin for the new tokens' positions."""
    from nanoserve_amd import RotaryEmbedding

    c0 = calls[0]
    rot = RotaryEmbedding(c0.head_dim, max(c.md.max_seq_len for c in calls) + 1, device=c0.query.device)
    out = []
    for c in calls:
        pos = []
        for sl, ql in zip(c.md.seq_lens_cpu, c.md.query_lens_cpu):
            pos += range(sl - ql, sl)
        cos, sin = rot.cos_sin(torch.tensor(pos, device=c.query.device), c.query.dtype)
        out.append((torch.empty_like(c.query), cos, sin))
    return out


def _rope_bytes(c) -> int:
    """Algorithmic HBM bytes of one fused rotary + cache write call.

    Per token: read q, k, v rows and the cos/sin rows, write rotated q and
    the K and V cache rows: 2 * (Hq + 2*Hkv) * D + 2 * D elements.
    """
    T, Hq, D = c.query.shape
    return T * (2 * (Hq + 2 * c.num_kv_heads) * D + 2 * D) * c.query.element_size()


def _time_steps(torch, steps, news, K, warmup, stream):
    """Warm up, capture the serving steps in one HIP graph, time exactly K steps.

    Step k of the timed sequence is steps[k % R] (R = len(steps)): the graph of
    all R steps is replayed K // R times, then a graph of the first K % R
    steps once, so the timed calls are exactly K * calls-per-step calls and
    their bytes are summed exactly."""
    from nanoserve_amd import paged_attention_hip, reshape_and_cache, rope_reshape_and_cache

    calls = [c for st in steps for c in st]
    R, L = len(steps), len(steps[0])

    def attn(i):
        # The reference's call site unchanged (qwen2.py:59-65): one call per
        # layer with the step's shared metadata and no per-step hook; the
        # step's first call builds the device-side decode plan on its md.
        c = calls[i]
        return paged_attention_hip(c.query, c.k_cache, c.v_cache, c.md, c.scale)

    def write(i):
        c = calls[i]
        reshape_and_cache(news[i][0], news[i][1], c.k_cache, c.v_cache, c.md.slot_mapping)

    def run_steps(n, keep=None):
        for j in range(n):
            for i in range(j * L, (j + 1) * L):
                out = attn(i)
                if keep is not None:
                    keep[i] = out  # graph-owned: holds the latest replay's result

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        # Write-then-attend, as the model's call site does (reference
        # qwen2.py:57-65): every call's new-token K/V goes in first.  Rewriting
        # the same rows later leaves the caches unchanged.
        for i in range(len(calls)):
            write(i)
        first_out = attn(0).clone()
        run_steps(R)
    torch.cuda.synchronize()

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with graph_capture(g, stream=stream):
            fn()
        return g

    full, rem = divmod(K, R)
    replay_outs = {}
    g_all = capture(lambda: run_steps(R, replay_outs))
    g_rem = capture(lambda: run_steps(rem)) if rem else None
    g_write = capture(lambda: [write(i) for i in range(len(calls))])

    def timed(graph, reps, graph_rem=None, warm=1):
        with torch.cuda.stream(stream):
            for _ in range(warm):
                graph.replay()
            stream.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(reps):
                graph.replay()
            if graph_rem is not None:
                graph_rem.replay()
            end.record(stream)
        end.synchronize()
        return start.elapsed_time(end) * 1e-3

    warm_reps = max(1, -(-warmup // R))
    # Timed twice (the reference's run-twice check, diagnose.py:241-263); the
    # line reports the mean and flags a spread over 15%.
    t_runs = [timed(g_all, full, g_rem, warm_reps), timed(g_all, full, g_rem, 1)]
    t_attn = sum(t_runs) / 2
    n_calls = K * L
    kv = [c.kv_bytes() for c in calls]
    bytes_total = full * sum(kv) + sum(kv[:rem * L])
    t_write = timed(g_write, 1)

    # Fused rotary + cache write of the same new tokens (q rotated into a
    # separate buffer so the timed attention inputs stay as they are).
    # Afterwards the plain write is replayed once more, which puts the caches
    # back to the state the attention outputs above were computed on.
    rope_in = _rope_inputs(torch, calls, news)

    def rope(i):
        c, (q_out, cos, sin) = calls[i], rope_in[i]
        rope_reshape_and_cache(c.query, news[i][0], news[i][1], cos, sin, c.k_cache, c.v_cache,
                               c.md.slot_mapping, out=q_out)

    with torch.cuda.stream(stream):
        for i in range(len(calls)):
            rope(i)
    stream.synchronize()
    g_rope = capture(lambda: [rope(i) for i in range(len(calls))])
    t_rope = timed(g_rope, 1)
    with torch.cuda.stream(stream):
        g_write.replay()
    stream.synchronize()
    rope_bytes = sum(_rope_bytes(c) for c in calls) / len(calls)
    # The timed replays cycled every call's data through the same split-K
    # workspace: check a few replayed outputs against the oracle.
    g_all.replay()
    stream.synchronize()
    checked = sorted({0, 1, len(calls) // 2, len(calls) - 1})
    replay_err = max(_oracle_err(calls[i], replay_outs[i]) for i in checked)
    timed_steps = [steps[k % R] for k in range(min(K, R))]
    del g_all, g_rem, g_write, g_rope, rope_in
    return {
        "replay_err": replay_err,
        "replay_checked": checked,
        "s_per_call": t_attn / n_calls,
        "s_per_step": t_attn / K,
        "runs_us_per_call": [t / n_calls * 1e6 for t in t_runs],
        "gbs": bytes_total / t_attn / 1e9,
        "write_us": t_write / len(calls) * 1e6,
        "rope_us": t_rope / len(calls) * 1e6,
        "rope_bytes": rope_bytes,
        "kv_mean_timed": bytes_total / n_calls,
        "calls_timed": n_calls,
        "seeds_timed": sorted({st[0].seed for st in timed_steps}),
        "first_out": first_out,
        "attn": attn,
    }


def _time_attn_variant(torch, steps, K, stream, per_step_plan=True, host_lists=True):
    """Microseconds per attention call of K graph-replayed serving steps, for
    the variants the line reports beside its main figure: the step's metadata
    without any host-side lengths (host_lists=False: the engine's graph
    replays, which never pass host copies), and every call planning its decode
    rows inside the call (per_step_plan=False: a caller whose layers do not
    share one plan, e.g. one that builds a new metadata object per call)."""
    import dataclasses

    from nanoserve_amd.attention import _attention

    mds = {}
    for st in steps:
        md = st[0].md
        if not host_lists:
            md = dataclasses.replace(md, seq_lens_cpu=None, query_start_loc_cpu=None, query_lens_cpu=None)
        md = dataclasses.replace(md, decode_plan=None)
        mds[id(st[0].md)] = md
    calls = [(c, mds[id(st[0].md)]) for st in steps for c in st]
    R, L = len(steps), len(steps[0])

    def run(n):
        for j in range(n):
            for i in range(j * L, (j + 1) * L):
                c, md = calls[i]
                _attention(c.query, c.k_cache, c.v_cache, md, c.scale, share_plan=per_step_plan)

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run(R)
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with graph_capture(g, stream=stream):
        run(R)
    reps = max(1, -(-K // R))
    with torch.cuda.stream(stream):
        g.replay()
        stream.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            g.replay()
        end.record(stream)
    end.synchronize()
    del g
    return start.elapsed_time(end) * 1e3 / (reps * R * L)


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share: --gpus {args.gpus} is not supported "
              "(the attention path shards by sequence with no collective; run N=1)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration is not None:
        return _copy_calibration(torch, args.copy_calibration)
    if args.floors:
        return _floors(torch, args)
    if args.int4_gemm:
        return _int4_gemm(torch, args)
    if args.ref_grid:
        return _ref_grid(torch, args)
    if args.config == "c5":
        return _bench_engine(torch, args)
    stream = torch.cuda.Stream(dev)

    def new_tokens(calls):
        out = []
        for i, c in enumerate(calls):
            g = torch.Generator(device=dev).manual_seed(1_000_003 + i)
            shape = (c.md.num_tokens, c.num_kv_heads, c.head_dim)
            out.append((torch.randn(shape, generator=g, device=dev).to(c.query.dtype),
                        torch.randn(shape, generator=g, device=dev).to(c.query.dtype)))
        return out

    K = args.steps
    steps, total = _build_steps(args, dev, shared=True)
    calls = [c for st in steps for c in st]
    dtype = calls[0].query.dtype
    dname = {torch.float16: "fp16", torch.bfloat16: "bf16"}[dtype]
    res = _time_steps(torch, steps, new_tokens(calls), K, args.warmup, stream)

    no_host_us = _time_attn_variant(torch, steps, K, stream, per_step_plan=True, host_lists=False)
    per_call_plan_us = _time_attn_variant(torch, steps, K, stream, per_step_plan=False, host_lists=False)

    eager_us = None
    if args.eager:
        attn = res["attn"]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            for k in range(K * args.layers):
                attn(k % len(calls))
        torch.cuda.synchronize()
        eager_us = (time.perf_counter() - t0) / (K * args.layers) * 1e6

    gbs, s_per_call = res["gbs"], res["s_per_call"]
    traffic, traffic_src = _profiled_traffic(args)
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": res["s_per_step"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: {WORKLOADS[args.config]}",
            "step": f"one serving step: {args.layers} attention calls (one per layer) sharing the step's "
                    "metadata, each over its own K/V caches",
            "block_size": calls[0].k_cache.shape[1],
            "global_batch": calls[0].md.num_seqs,
            "tokens_per_call": calls[0].md.num_tokens,
            "layers_per_step": args.layers,
            "distinct_steps": len(steps),
            "kv_footprint_gb": round(total / 1e9, 3),
            "calls_timed": res["calls_timed"],
            "seeds_timed": res["seeds_timed"],
            "kv_bytes_per_call_mean": res["kv_mean_timed"],
            "timing": "HIP-graph replay of exactly K serving steps cycling the distinct steps, "
                      "hipEvents on the launch stream; each step = one device-side decode-plan launch "
                      "(ns_paged_decode_plan) + the attention calls, all inside the timed region",
        },
        "us_per_call": round(s_per_call * 1e6, 3),
        "timed_runs_us_per_call": [round(x, 3) for x in res["runs_us_per_call"]],
        "run_spread_pct": round(100.0 * (max(res["runs_us_per_call"]) - min(res["runs_us_per_call"]))
                                / min(res["runs_us_per_call"]), 2),
        "run_spread_over_15pct": (max(res["runs_us_per_call"]) - min(res["runs_us_per_call"]))
                                 > 0.15 * min(res["runs_us_per_call"]),
        "pct_of_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "no_host_plan_us": round(no_host_us, 3),
        "per_call_plan_us": round(per_call_plan_us, 3),
        "plan_note": "the decode plan is built on the device from seq_lens in every variant: us_per_call "
                     "calls paged_attention_hip as the reference's qwen2.py does (one md per step, no per-step "
                     "hook), so the step's first call builds the plan and the other layers reuse it; "
                     "no_host_plan_us does the same with the metadata's host-side lengths removed (as the "
                     "engine's graph replays run); per_call_plan_us plans inside every attention call",
        "reshape_and_cache_us": round(res["write_us"], 3),
        "rope_reshape_and_cache": {
            "us_per_call": round(res["rope_us"], 3),
            "bytes_per_call": int(res["rope_bytes"]),
            "gbs": round(res["rope_bytes"] / (res["rope_us"] * 1e-6) / 1e9, 2),
            "frac_of_hbm_peak": round(res["rope_bytes"] / (res["rope_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "note": "fused rotary of q,k + cache write of k,v for the call's new tokens (graph replay)",
        },
        "replay_max_abs_err_vs_oracle": res["replay_err"],
    }
    if traffic is not None:
        result["roofline"]["traffic_source"] = f"{traffic_src} (FETCH_SIZE x2.0 + WRITE_SIZE x1.0, copy-calibrated)"
    if args.config == "c3":
        flops = sum(c.prefill_flops() for c in calls) / len(calls)
        result["prefill_flops_per_call"] = flops
        result["mfma_tflops"] = round(flops / s_per_call / 1e12, 2)
    if eager_us is not None:
        result["eager_us_per_call"] = round(eager_us, 2)
    first_case, first_out = calls[0], res["first_out"]
    del res

    if args.cold:
        del calls, steps
        cold, _ = _build_steps(args, dev, shared=False)
        cold_calls = [c for st in cold for c in st]
        r2 = _time_steps(torch, cold, new_tokens(cold_calls), K, args.warmup, stream)
        result["cold_metadata"] = {
            "us_per_call": round(r2["s_per_call"] * 1e6, 3),
            "gbs": round(r2["gbs"], 2),
            "calls_timed": r2["calls_timed"],
            "note": "every call with its own block tables and lengths (no step shares metadata)",
        }
        del cold, cold_calls, r2

    if not args.no_cpu_baseline:
        cpu, err = _cpu_baseline(first_case, args.cpu_calls, first_out)
        result["cpu_baseline"] = cpu
        result["max_abs_err_vs_oracle"] = err
        tol = 2e-3 if dtype == torch.float16 else 1e-2
        if not (err <= tol and result["replay_max_abs_err_vs_oracle"] <= tol):
            print(f"parity gate failed: max abs err {err:.3e} (first call), "
                  f"{result['replay_max_abs_err_vs_oracle']:.3e} (replayed calls) > {tol}", file=sys.stderr)
            print(json.dumps(result))
            return 1
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
