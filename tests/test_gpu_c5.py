"""Config 5 on the GPU: the engine at Qwen2.5-0.5B size with every HIP kernel inside.

The workload is config 5's own (reference tests/test_integration.py:90-163,
results/sweep.json:523-551): the 24-layer Qwen2.5-0.5B architecture (hidden
896, 14/2 heads, head_dim 64, intermediate 4864, vocab 151936) with
random-init weights quantised to INT4 g128 (lm_head fp16), 32 requests with
config 5's lognormal prompt lengths (workloads.c5_requests, seed 0), greedy
with ignore_eos.  Output lengths are config 5's, capped at MAX_NEW so the
test runs in seconds; decode steps replay HIP graphs.

Checks:
  * every request ends with exactly its length and every KV block returns;
  * every emitted token is the greedy choice of a teacher-forced replay of
    the request (one prefill of prompt + outputs), fp16 near-ties aside;
  * the graph-replayed engine emits the eager engine's tokens;
  * one decode step of all 32 sequences matches the float32 CPU oracle
    (oracle/qwen2.py) within 1e-2 (max |diff| / max |oracle|).

Decoding 32 sequences after graph warm-up at batches of 16 and fewer also
exercises the INT4 split-K workspace shared by token counts that split
differently (down_proj: 4 splits up to 16 tokens, 2 up to 32).
"""

from __future__ import annotations

import pytest
import torch

from nanoserve_amd.block_manager import BlockSpaceManager
from nanoserve_amd.engine import LLMEngine, ModelRunner
from nanoserve_amd.kv_cache import PagedKVCache
from nanoserve_amd.model import Qwen2Config, Qwen2ForCausalLM, random_init_
from nanoserve_amd.quant import quantize_model
from nanoserve_amd.scheduling import SamplingParams, SchedulerConfig, Sequence
from nanoserve_amd.workloads import c5_requests
from oracle.qwen2 import qwen2_forward_ref, relative_error

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2
MAX_NEW = 8
NUM_BLOCKS = 2048
BLOCK = 16


def _say(msg: str) -> None:
    print(f"[c5] {msg}", flush=True)


@pytest.fixture(scope="module")
def model():
    _say("building the 24-layer INT4 model")
    m = random_init_(Qwen2ForCausalLM(Qwen2Config(), max_position=4096), std=0.02, seed=0)
    m = m.half().to(DEV)
    quantize_model(m, 128, skip=("lm_head",))
    m.fuse_projections()
    return m.eval().requires_grad_(False)


@pytest.fixture(scope="module")
def requests(model):
    reqs = c5_requests(32, 0, model.config.vocab_size)
    return [(toks, min(n, MAX_NEW)) for toks, n in reqs]


def _serve(model, requests, use_graphs):
    eng = LLMEngine(model, num_blocks=NUM_BLOCKS, block_size=BLOCK, device=DEV,
                    scheduler_config=SchedulerConfig(max_num_batched_tokens=2048, max_num_seqs=256),
                    max_model_len=4096, use_graphs=use_graphs)
    if use_graphs:
        eng.runner.graphs.capture_all()
    for toks, n in requests:
        eng.add_request(toks, SamplingParams(max_new_tokens=n, ignore_eos=True))
    out = eng.run_all()
    torch.cuda.synchronize()
    return out, eng


@pytest.fixture(scope="module")
def served(model, requests):
    _say("serving with graphs")
    graph_out, graph_eng = _serve(model, requests, True)
    _say("serving eagerly")
    eager_out, eager_eng = _serve(model, requests, False)
    return graph_out, graph_eng, eager_out, eager_eng


def test_c5_every_request_finishes_and_no_block_leaks(served, requests):
    graph_out, graph_eng, eager_out, eager_eng = served
    for out, eng in ((graph_out, graph_eng), (eager_out, eager_eng)):
        assert [len(s.output_token_ids) for s in out] == [n for _, n in requests]
        assert [s.prompt_token_ids for s in out] == [t for t, _ in requests]
        bm = eng.block_manager
        assert bm.num_free_blocks == bm.num_total_blocks
        assert not eng.has_unfinished_requests


def test_c5_graph_replay_emits_the_eager_tokens(served):
    graph_out, _, eager_out, _ = served
    total = sum(len(s.output_token_ids) for s in eager_out)
    same = sum(a == b for g, e in zip(graph_out, eager_out) for a, b in zip(g.output_token_ids, e.output_token_ids))
    assert same >= 0.95 * total, f"{same} of {total} tokens agree"


@torch.inference_mode()
def test_c5_tokens_are_greedy_under_teacher_forcing(model, served):
    """Replay each request's prompt + outputs in one prefill; each output token
    must be (up to fp16 near-ties) the argmax of the logits before it."""
    graph_out, *_ = served
    cache = PagedKVCache(NUM_BLOCKS, BLOCK, model.num_layers, model.num_kv_heads, model.head_dim,
                         torch.float16, DEV)
    bm = BlockSpaceManager(BLOCK, NUM_BLOCKS, watermark=0.0)
    runner = ModelRunner(model, cache, bm, DEV)
    replay, rows, picks = [], [], []
    for s in graph_out:
        full = s.prompt_token_ids + s.output_token_ids[:-1]
        r = Sequence(s.seq_id, full, SamplingParams(max_new_tokens=1, ignore_eos=True))
        assert bm.allocate(r, len(full))
        replay.append((r, len(full)))
    ids, pos, md, _, _ = runner.build_inputs(replay)
    off = 0
    for (r, n), s in zip(replay, graph_out):
        p = len(s.prompt_token_ids)
        rows.extend(range(off + p - 1, off + n))
        picks.extend(s.output_token_ids)
        off += n
    _say(f"teacher-forced replay of {off} tokens")
    hidden = model(ids, pos, cache, md, runner.attn_fn)
    logits = model.compute_logits(hidden, torch.tensor(rows, device=DEV)).float()
    picked = logits.gather(1, torch.tensor(picks, device=DEV)[:, None])[:, 0]
    gap = (logits.max(dim=1).values - picked).cpu()
    scale = logits.abs().max(dim=1).values.cpu()
    assert bool((gap <= 5 * TOL * scale).all()), f"max gap {float((gap / scale).max()):.3e} of the row scale"
    assert float((gap == 0).float().mean()) >= 0.9, "most tokens must be the exact argmax"


@torch.inference_mode()
def test_c5_decode_step_matches_the_oracle(model, requests):
    """Prefill all 32 prompts, then one decode step of all 32 sequences, checked
    against the float32 CPU oracle on the same cache contents."""
    cache = PagedKVCache(NUM_BLOCKS, BLOCK, model.num_layers, model.num_kv_heads, model.head_dim,
                         torch.float16, DEV)
    bm = BlockSpaceManager(BLOCK, NUM_BLOCKS, watermark=0.0)
    runner = ModelRunner(model, cache, bm, DEV)
    seqs = [Sequence(i, toks, SamplingParams(max_new_tokens=2, ignore_eos=True)) for i, (toks, _) in
            enumerate(requests)]
    plan = [(s, len(s.prompt_token_ids)) for s in seqs]
    for s, n in plan:
        assert bm.allocate(s, n)
    ids, pos, md, samp, _ = runner.build_inputs(plan)
    logits = model.compute_logits(model(ids, pos, cache, md, runner.attn_fn), samp)
    first = logits.argmax(dim=-1).tolist()
    for (s, n), t in zip(plan, first):
        s.mark_computed(n)
        s.output_token_ids.append(t)
    torch.cuda.synchronize()
    kc = [t.cpu() for t in cache.k_cache]
    vc = [t.cpu() for t in cache.v_cache]
    step = [(s, 1) for s in seqs]
    for s, _ in step:
        assert bm.allocate(s, s.num_tokens)
    ids, pos, md, samp, _ = runner.build_inputs(step)
    got = model.compute_logits(model(ids, pos, cache, md, runner.attn_fn), samp).float()
    torch.cuda.synchronize()
    _say(f"oracle decode step: 32 rows, contexts {min(md.seq_lens_cpu)}..{max(md.seq_lens_cpu)}")
    want, _, _ = qwen2_forward_ref(model, ids, pos, kc, vc, md, samp)
    err = relative_error(got, want)
    _say(f"decode-step logits: relative error {err:.2e}")
    assert err < TOL
