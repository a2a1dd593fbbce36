"""The engine harness on the GPU: the Qwen2 forward with every HIP kernel inside.

The model runs INT4 projections (ns_int4_linear), the fused rotary + cache
write (ns_rope_reshape_and_cache) and paged attention (ns_paged_attention);
the oracle (oracle/qwen2.py, pinned against transformers on the CPU) runs the
reference forward in float32.  Bounds: logits within 1e-2 of the oracle's
(max |diff| / max |oracle|, fp16 activations rounded after every op), and the
reference's model properties (tests/test_model.py:54-136) within the same
bound: incremental decode == one-shot prefill, chunked == one-shot, and a
sequence's logits independent of its batchmates.  The engine's integration
properties (tests/test_integration.py:38-166) -- chunked prefill, preemption,
one request at a time and requests added mid-flight -- are checked as: every
request ends with its length, no block leaks, every emitted token is the
model's greedy choice under a teacher-forced replay (fp16 near-ties aside),
and nine in ten tokens match the plain run.
"""

from __future__ import annotations

import pytest
import torch

from nanoserve_amd.block_manager import BlockSpaceManager
from nanoserve_amd.engine import LLMEngine, ModelRunner, SamplingParams, SchedulerConfig, Sequence
from nanoserve_amd.kv_cache import PagedKVCache
from nanoserve_amd.model import Qwen2Config, Qwen2ForCausalLM, random_init_
from nanoserve_amd.quant import quantize_model
from oracle.qwen2 import qwen2_forward_ref, relative_error

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2
TINY = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, rope_theta=10000.0, tie_word_embeddings=False)


def _model(cfg_kw=TINY, dtype=torch.float16, int4=True, fuse=True, seed=0, std=0.05):
    m = random_init_(Qwen2ForCausalLM(Qwen2Config(**cfg_kw), max_position=2048), std=std, seed=seed)
    m = m.to(dtype).to(DEV)
    if int4:
        quantize_model(m, 128)
    if fuse:
        m.fuse_projections()
    return m.eval().requires_grad_(False)


def _runner(model, num_blocks=64, block_size=8):
    cache = PagedKVCache(num_blocks, block_size, model.num_layers, model.num_kv_heads, model.head_dim,
                         model.model.embed_tokens.weight.dtype, DEV)
    bm = BlockSpaceManager(block_size, num_blocks, watermark=0.0)
    return ModelRunner(model, cache, bm, DEV), bm


def _seq(i, tokens, max_new=4):
    return Sequence(i, list(tokens), SamplingParams(max_new_tokens=max_new, ignore_eos=True))


_LENS = [(5, 6), (33, 3), (17, 9), (70, 4), (2, 12), (40, 7)]  # (prompt, output) lengths


def _tokens(n, vocab, seed):
    return torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


@torch.inference_mode()
def _step(runner, bm, plan):
    """Run one forward over plan [(seq, q)]; return (logits of sampled rows, sample_seqs, md, ids, pos)."""
    for s, q in plan:
        assert bm.allocate(s, s.num_computed_tokens + q)
    ids, pos, md, si, seqs = runner.build_inputs(plan)
    hidden = runner.model(ids, pos, runner.kv_cache, md, runner.attn_fn)
    logits = runner.model.compute_logits(hidden, si) if si is not None else None
    for s, q in plan:
        s.mark_computed(q)
    return logits, seqs, md, ids, pos


@pytest.mark.parametrize("int4,fuse,dtype", [(True, True, torch.float16), (True, False, torch.float16),
                                             (False, True, torch.float16), (True, True, torch.bfloat16)])
def test_forward_matches_oracle_on_a_mixed_batch(int4, fuse, dtype):
    model = _model(int4=int4, fuse=fuse, dtype=dtype)
    runner, bm = _runner(model)
    a, b = _seq(0, _tokens(21, 512, 1)), _seq(1, _tokens(9, 512, 2))
    kc = [t.cpu() for t in runner.kv_cache.k_cache]
    vc = [t.cpu() for t in runner.kv_cache.v_cache]
    # Step 1: both prefill; step 2: a decodes while c prefills beside it.
    logits, seqs, md, ids, pos = _step(runner, bm, [(a, 21), (b, 9)])
    want, kc, vc = qwen2_forward_ref(model, ids, pos, kc, vc, md, torch.tensor([20, 29]))
    torch.cuda.synchronize()
    assert relative_error(logits, want) < (TOL if dtype == torch.float16 else 3 * TOL)
    a.output_token_ids.append(int(want[0].argmax()))
    c = _seq(2, _tokens(30, 512, 3))
    logits, seqs, md, ids, pos = _step(runner, bm, [(a, 1), (c, 30)])
    want, _, _ = qwen2_forward_ref(model, ids, pos, kc, vc, md, torch.tensor([0, 30]))
    torch.cuda.synchronize()
    assert relative_error(logits, want) < (TOL if dtype == torch.float16 else 3 * TOL)


@pytest.mark.parametrize("cfg_kw,dtype,tol", [
    (TINY, torch.float32, 1e-4),                                       # float32 model: the generic kernel
    (dict(TINY, hidden_size=128, intermediate_size=256), torch.float16, TOL),  # head size 32
])
def test_forward_of_shapes_outside_the_mfma_kernels_matches_oracle(cfg_kw, dtype, tol):
    """A float32 model and a head size of 32 run attention on the generic kernel (the
    reference's model config takes any float dtype, config.py:15); the rest of the forward
    (rotary + cache write, norms, unquantised projections) is unchanged.  Prefill of two
    sequences, then one decodes while a third prefills."""
    model = _model(cfg_kw, dtype=dtype, int4=False)
    runner, bm = _runner(model)
    a, b = _seq(0, _tokens(21, 512, 1)), _seq(1, _tokens(9, 512, 2))
    kc = [t.cpu() for t in runner.kv_cache.k_cache]
    vc = [t.cpu() for t in runner.kv_cache.v_cache]
    logits, seqs, md, ids, pos = _step(runner, bm, [(a, 21), (b, 9)])
    want, kc, vc = qwen2_forward_ref(model, ids, pos, kc, vc, md, torch.tensor([20, 29]))
    torch.cuda.synchronize()
    assert logits.dtype == dtype and relative_error(logits, want) < tol
    a.output_token_ids.append(int(want[0].argmax()))
    c = _seq(2, _tokens(30, 512, 3))
    logits, seqs, md, ids, pos = _step(runner, bm, [(a, 1), (c, 30)])
    want, _, _ = qwen2_forward_ref(model, ids, pos, kc, vc, md, torch.tensor([0, 30]))
    torch.cuda.synchronize()
    assert relative_error(logits, want) < tol


def test_qwen_half_billion_shapes_two_layers_match_oracle():
    cfg = dict(num_hidden_layers=2)  # Qwen2.5-0.5B widths: hidden 896, 14/2 heads, D 64, vocab 151936
    model = _model(cfg, std=0.02)
    runner, bm = _runner(model, num_blocks=32, block_size=16)
    a, b = _seq(0, _tokens(40, 151936, 4)), _seq(1, _tokens(7, 151936, 5))
    kc = [t.cpu() for t in runner.kv_cache.k_cache]
    vc = [t.cpu() for t in runner.kv_cache.v_cache]
    logits, _, md, ids, pos = _step(runner, bm, [(a, 40), (b, 7)])
    want, _, _ = qwen2_forward_ref(model, ids, pos, kc, vc, md, torch.tensor([39, 46]))
    torch.cuda.synchronize()
    assert relative_error(logits, want) < TOL


@pytest.mark.parametrize("block_size", [8, 16])
def test_token_by_token_matches_one_shot_prefill(block_size):
    model = _model()
    toks = _tokens(23, 512, 6)
    r1, bm1 = _runner(model, block_size=block_size)
    whole, *_ = _step(r1, bm1, [(_seq(0, toks), 23)])
    r2, bm2 = _runner(model, block_size=block_size)
    s = _seq(0, toks)
    for _ in range(23):
        last, *_ = _step(r2, bm2, [(s, 1)])
    torch.cuda.synchronize()
    assert relative_error(last, whole) < TOL


def test_chunked_prefill_matches_one_shot():
    model = _model()
    toks = _tokens(30, 512, 7)
    r1, bm1 = _runner(model)
    whole, *_ = _step(r1, bm1, [(_seq(0, toks), 30)])
    r2, bm2 = _runner(model)
    s = _seq(0, toks)
    for q in (7, 11, 12):
        last, *_ = _step(r2, bm2, [(s, q)])
    torch.cuda.synchronize()
    assert relative_error(last, whole) < TOL


def test_logits_are_independent_of_batchmates():
    model = _model()
    a_t, b_t = _tokens(12, 512, 8), _tokens(25, 512, 9)
    r1, bm1 = _runner(model)
    alone, *_ = _step(r1, bm1, [(_seq(0, a_t), 12)])
    r2, bm2 = _runner(model)
    sa, sb = _seq(0, a_t), _seq(1, b_t)
    together, seqs, *_ = _step(r2, bm2, [(sa, 12), (sb, 25)])
    torch.cuda.synchronize()
    assert relative_error(together[seqs.index(sa)][None], alone) < TOL


def test_engine_runs_requests_to_completion_deterministically():
    def run(num_blocks):
        model = _model(seed=3)
        eng = LLMEngine(model, num_blocks=num_blocks, block_size=8, device=DEV,
                        scheduler_config=SchedulerConfig(max_num_batched_tokens=64, max_num_seqs=8),
                        max_model_len=256)
        lens = [(5, 6), (33, 3), (17, 9), (70, 4), (2, 12), (40, 7)]
        for i, (p, n) in enumerate(lens):
            eng.add_request(_tokens(p, 512, 100 + i), SamplingParams(max_new_tokens=n, ignore_eos=True))
        out = eng.run_all()
        assert [len(s.output_token_ids) for s in out] == [n for _, n in lens]
        assert all(0 <= t < 512 for s in out for t in s.output_token_ids)
        return [s.output_token_ids for s in out], eng.scheduler.num_preemptions

    toks1, pre1 = run(128)
    toks2, _ = run(128)
    assert toks1 == toks2 and pre1 == 0
    # A cache too small for all requests at once: sequences are preempted and recomputed.
    _, pre3 = run(16)
    assert pre3 > 0


def test_first_greedy_token_matches_oracle_when_not_a_near_tie():
    model = _model(seed=4)
    runner, bm = _runner(model)
    kc = [t.cpu() for t in runner.kv_cache.k_cache]
    vc = [t.cpu() for t in runner.kv_cache.v_cache]
    seqs = [_seq(i, _tokens(5 + 7 * i, 512, 200 + i)) for i in range(4)]
    for s in seqs:
        assert bm.allocate(s, s.prompt_len)
    ids, pos, md, si, order = runner.build_inputs([(s, s.prompt_len) for s in seqs])
    got = runner.execute([(s, s.prompt_len) for s in seqs])
    want, _, _ = qwen2_forward_ref(model, ids, pos, kc, vc, md, si)
    top2 = want.topk(2, dim=-1).values
    checked = 0
    for i, (s, tok) in enumerate(got):
        margin = float(top2[i, 0] - top2[i, 1])
        if margin > 5 * TOL * float(want.abs().max()):
            assert tok == int(want[i].argmax())
            checked += 1
    assert checked >= 1


def test_decode_logits_do_not_depend_on_a_prefilling_batchmate():
    """One sequence decoding beside another's prefill in a mixed batch (reference
    tests/test_model.py:99-126): the decoding row's logits are those of the step alone."""
    model = _model(seed=9)
    a, b = _tokens(9, 512, 31), _tokens(17, 512, 32)

    def decode_of_a(with_neighbour):
        runner, bm = _runner(model)
        sa = _seq(0, a)
        logits, *_ = _step(runner, bm, [(sa, len(a))])
        sa.output_token_ids.append(int(logits[0].argmax()))
        plan = [(sa, 1)] + ([(_seq(1, b), len(b))] if with_neighbour else [])
        logits, seqs, *_ = _step(runner, bm, plan)
        return logits[seqs.index(sa)]

    assert relative_error(decode_of_a(True), decode_of_a(False)) < TOL


def test_block_size_does_not_change_logits():
    """Prefill chunks and decode steps over caches of 4- to 32-token blocks give the
    same logits (reference tests/test_model.py:129-136)."""
    model = _model(seed=10)
    tokens = _tokens(37, 512, 33)
    outs = []
    for bs in (4, 8, 16, 32):
        runner, bm = _runner(model, num_blocks=256 // bs, block_size=bs)
        s = _seq(0, tokens)
        for q in (10, 1, 1, 25):
            logits, *_ = _step(runner, bm, [(s, q)])
        outs.append(logits[0])
    for o in outs[1:]:
        assert relative_error(o, outs[0]) < TOL


@pytest.mark.parametrize("batch", [3, 8])
def test_decode_graph_replays_match_eager_steps(batch):
    """Decode steps replayed from the captured graph (padded to a bucket) give the eager step's logits."""
    model = _model(seed=5)
    r_e, bm_e = _runner(model, num_blocks=96)
    r_g, bm_g = _runner(model, num_blocks=96)
    from nanoserve_amd.engine import DecodeGraphs
    r_g.graphs = DecodeGraphs(r_g, (1, 2, 4, 8), max_model_len=256)
    prompts = [_tokens(3 + 11 * i, 512, 300 + i) for i in range(batch)]
    se = [_seq(i, p, max_new=64) for i, p in enumerate(prompts)]
    sg = [_seq(i, p, max_new=64) for i, p in enumerate(prompts)]
    logits, seqs, *_ = _step(r_e, bm_e, [(s, s.prompt_len) for s in se])
    _step(r_g, bm_g, [(s, s.prompt_len) for s in sg])
    toks = logits.argmax(-1).tolist()
    for step in range(5):
        for a, b_, t in zip(se, sg, toks):
            a.output_token_ids.append(t)
            b_.output_token_ids.append(t)
        want, *_ = _step(r_e, bm_e, [(s, 1) for s in se])
        for s in sg:
            assert bm_g.allocate(s, s.num_computed_tokens + 1)
        with torch.inference_mode():
            got_tokens = r_g.execute([(s, 1) for s in sg])
        got = r_g.graphs.last_logits
        torch.cuda.synchronize()
        assert relative_error(got, want) < TOL, f"step {step}"
        assert [t for _, t in got_tokens] == got.argmax(-1).tolist()
        toks = want.argmax(-1).tolist()


@pytest.mark.parametrize("dtype,int4", [(torch.float16, True), (torch.float32, False)])
def test_engine_with_graphs_completes_the_same_requests(dtype, int4):
    """float32 (unquantised) runs attention on the generic kernel inside the graphs."""
    def run(graphs):
        model = _model(seed=6, dtype=dtype, int4=int4)
        eng = LLMEngine(model, num_blocks=128, block_size=8, device=DEV,
                        scheduler_config=SchedulerConfig(max_num_batched_tokens=64, max_num_seqs=8),
                        max_model_len=256, use_graphs=graphs)
        lens = [(5, 6), (33, 3), (17, 9), (70, 4), (2, 12), (40, 7)]
        for i, (p, n) in enumerate(lens):
            eng.add_request(_tokens(p, 512, 400 + i), SamplingParams(max_new_tokens=n, ignore_eos=True))
        out = eng.run_all()
        assert [len(s.output_token_ids) for s in out] == [n for _, n in lens]
        return [s.output_token_ids for s in out]

    eager, graphed = run(False), run(True)
    # Greedy tokens agree except where the eager and graphed attention grids
    # round a near-tie differently; require most of them to agree.
    same = sum(a == b for x, y in zip(eager, graphed) for a, b in zip(x, y))
    total = sum(len(x) for x in eager)
    assert same >= 0.9 * total, f"{same}/{total} tokens agree"


@pytest.mark.parametrize("mid_flight", [False, True])
def test_pipelined_decode_gives_the_unpipelined_tokens(mid_flight):
    """Launching decode step N+1 before reading step N's tokens back (ids
    gathered on the device) changes no token, no length and leaks no block."""
    def run(pipeline):
        model = _model(seed=11)
        eng = LLMEngine(model, num_blocks=64, block_size=8, device=DEV,
                        scheduler_config=SchedulerConfig(max_num_batched_tokens=64, max_num_seqs=8),
                        max_model_len=256, use_graphs=True, pipeline_decode=pipeline)
        reqs = [(_tokens(p, 512, 900 + i), SamplingParams(max_new_tokens=n, ignore_eos=True))
                for i, (p, n) in enumerate(_LENS)]
        first = reqs[:3] if mid_flight else reqs
        for r in first:
            eng.add_request(*r)
        out = []
        if mid_flight:
            for _ in range(6):
                out += eng.step()
            for r in reqs[3:]:
                eng.add_request(*r)
        while eng.has_unfinished_requests:
            out += eng.step()
        out.sort(key=lambda s: s.seq_id)
        assert eng.block_manager.num_free_blocks == 64
        assert all(m.end >= m.first_token > 0 for m in (s.metrics for s in out))
        return [s.output_token_ids for s in out]

    plain, piped = run(False), run(True)
    assert [len(t) for t in piped] == [n for _, n in _LENS]
    assert piped == plain and all(t >= 0 for seq in piped for t in seq)


def test_decode_graphs_switch_context_buckets_as_sequences_grow():
    """Contexts crossing the 256- and 512-token bounds pick larger-grid graphs; logits stay eager's."""
    model = _model(seed=7)
    r_e, bm_e = _runner(model, num_blocks=256)
    r_g, bm_g = _runner(model, num_blocks=256)
    from nanoserve_amd.engine import DecodeGraphs
    r_g.graphs = DecodeGraphs(r_g, (1, 2, 4), max_model_len=1024)
    assert r_g.graphs.ctx_sizes == [256, 512, 1024]
    prompts = [_tokens(n, 512, 500 + n) for n in (250, 509, 40)]
    se = [_seq(i, p, max_new=64) for i, p in enumerate(prompts)]
    sg = [_seq(i, p, max_new=64) for i, p in enumerate(prompts)]
    logits, *_ = _step(r_e, bm_e, [(s, s.prompt_len) for s in se])
    _step(r_g, bm_g, [(s, s.prompt_len) for s in sg])
    toks = logits.argmax(-1).tolist()
    used = set()
    for step in range(8):
        for a, b_, t in zip(se, sg, toks):
            a.output_token_ids.append(t)
            b_.output_token_ids.append(t)
        want, *_ = _step(r_e, bm_e, [(s, 1) for s in se])
        for s in sg:
            assert bm_g.allocate(s, s.num_computed_tokens + 1)
        longest = max(s.num_computed_tokens + 1 for s in sg)
        used.add(next(c for c in r_g.graphs.ctx_sizes if c >= longest))
        with torch.inference_mode():
            r_g.execute([(s, 1) for s in sg])
        got = r_g.graphs.last_logits
        torch.cuda.synchronize()
        assert relative_error(got, want) < TOL, f"step {step}"
        toks = want.argmax(-1).tolist()
    assert used == {512, 1024}


# ---- engine integration (reference tests/test_integration.py:38-166) -------------


@torch.inference_mode()
def _teacher_forced_logits(model, tokens):
    """Logits of every position of `tokens`, one-shot prefill into a fresh cache."""
    runner, bm = _runner(model, num_blocks=64, block_size=8)
    s = _seq(0, tokens)
    assert bm.allocate(s, len(tokens))
    ids, pos, md, _, _ = runner.build_inputs([(s, len(tokens))])
    hidden = runner.model(ids, pos, runner.kv_cache, md, runner.attn_fn)
    return runner.model.compute_logits(hidden, torch.arange(len(tokens), device=DEV)).float()


def _assert_greedy(model, seq):
    """Every generated token is the model's argmax at its position, up to fp16 near-ties."""
    full = seq.prompt_token_ids + seq.output_token_ids
    logits = _teacher_forced_logits(model, full[:-1])
    rows = logits[len(seq.prompt_token_ids) - 1:]
    picked = rows.gather(1, torch.tensor(seq.output_token_ids, device=DEV)[:, None])[:, 0]
    gap = rows.max(dim=1).values - picked
    assert float(gap.max()) <= 5 * TOL * float(rows.abs().max()), (seq.seq_id, gap.tolist())


def _run_engine(model, mode):
    budget, max_seqs, blocks = {"plain": (512, 8, 128), "chunked": (16, 8, 128), "preempting": (64, 8, 14),
                                "one_at_a_time": (512, 1, 128), "mid_flight": (64, 8, 128)}[mode]
    eng = LLMEngine(model, num_blocks=blocks, block_size=8, device=DEV,
                    scheduler_config=SchedulerConfig(max_num_batched_tokens=budget, max_num_seqs=max_seqs),
                    max_model_len=256)
    reqs = [(_tokens(p, 512, 700 + i), SamplingParams(max_new_tokens=n, ignore_eos=True))
            for i, (p, n) in enumerate(_LENS)]
    # Count the steps that mix prefill and decode rows.
    eng.mixed_steps = 0
    schedule = eng.scheduler.schedule

    def counting_schedule():
        out = schedule()
        eng.mixed_steps += bool(out.num_prefill_seqs and out.num_decode_seqs)
        return out

    eng.scheduler.schedule = counting_schedule
    if mode == "mid_flight":
        for r in reqs[:3]:
            eng.add_request(*r)
        out = []
        for _ in range(4):
            out += eng.step()
        for r in reqs[3:]:
            eng.add_request(*r)
        while eng.has_unfinished_requests:
            out += eng.step()
        out.sort(key=lambda s: s.seq_id)
    else:
        for r in reqs:
            eng.add_request(*r)
        out = eng.run_all()
    return out, eng


@pytest.mark.parametrize("mode", ["chunked", "preempting", "one_at_a_time", "mid_flight"])
def test_engine_serves_every_request_greedily_however_it_is_batched(mode):
    model = _model(seed=8)
    plain, _ = _run_engine(model, "plain")
    out, eng = _run_engine(model, mode)
    assert [len(s.output_token_ids) for s in out] == [n for _, n in _LENS]
    assert eng.block_manager.num_free_blocks == eng.block_manager.num_total_blocks  # nothing leaked
    if mode == "preempting":
        assert eng.scheduler.num_preemptions > 0
    if mode == "chunked":
        assert eng.mixed_steps > 0
    for s in out:
        _assert_greedy(model, s)
    same = sum(a == b for x, y in zip(plain, out) for a, b in zip(x.output_token_ids, y.output_token_ids))
    assert same >= 0.9 * sum(n for _, n in _LENS), f"{same} tokens agree with the plain run"
