"""The engine harness on the CPU: model oracle and runner bookkeeping.

* The model oracle (oracle/qwen2.py) is pinned against an independent
  implementation: transformers' own Qwen2ForCausalLM on identical float32
  weights (the reference's third model property, reference
  tests/test_model.py:1-14), both for one-shot prefill and for incremental
  decode through the paged cache.
* The runner's metadata is the engine layout (model_runner.py:85-147).
"""

from __future__ import annotations

import pytest
import torch

from nanoserve_amd.block_manager import BlockSpaceManager
from nanoserve_amd.engine import ModelRunner, summarize
from nanoserve_amd.scheduling import RequestMetrics, SamplingParams, Sequence
from nanoserve_amd.metadata import ScheduledSeq, build_metadata
from nanoserve_amd.model import Qwen2Config, Qwen2ForCausalLM, random_init_
from oracle.qwen2 import qwen2_forward_ref, relative_error

TINY = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, rope_theta=10000.0,
            tie_word_embeddings=False, max_position_embeddings=512)


def _tiny_pair(seed=0):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(seed)
    hf = transformers.Qwen2ForCausalLM(transformers.Qwen2Config(**TINY)).eval()
    ours = Qwen2ForCausalLM(Qwen2Config(**TINY))
    missing, unexpected = ours.load_state_dict(hf.state_dict(), strict=False)
    assert not missing, missing
    assert all("rotary" in u for u in unexpected), unexpected
    return hf, ours


def _paged(tokens, block_size, num_blocks, start=0):
    """Metadata for one sequence computing positions [start, len(tokens)); the
    table runs backwards so physical order differs from logical order."""
    table = list(range(num_blocks))[::-1]
    _, md = build_metadata([ScheduledSeq(table, start, len(tokens))], block_size, "cpu")
    return md


def test_model_state_dict_names_match_transformers():
    _tiny_pair()


def test_oracle_forward_matches_transformers_one_shot():
    hf, ours = _tiny_pair(1)
    tokens = torch.randint(0, 512, (23,), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        want = hf(tokens[None]).logits[0]
    L, NB, BS = 2, 4, 8
    kc = [torch.zeros(NB, BS, 2, 64) for _ in range(L)]
    vc = [torch.zeros(NB, BS, 2, 64) for _ in range(L)]
    md = _paged(tokens.tolist(), BS, NB)
    got, _, _ = qwen2_forward_ref(ours, tokens, torch.arange(23), kc, vc, md)
    assert relative_error(got, want) < 1e-4


def test_oracle_incremental_decode_matches_transformers():
    """Prefill 15 tokens, then decode 5 one at a time through the paged cache."""
    hf, ours = _tiny_pair(3)
    tokens = torch.randint(0, 512, (20,), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        want = hf(tokens[None]).logits[0]
    L, NB, BS = 2, 4, 8
    kc = [torch.zeros(NB, BS, 2, 64) for _ in range(L)]
    vc = [torch.zeros(NB, BS, 2, 64) for _ in range(L)]
    md = _paged(tokens[:15].tolist(), BS, NB)
    got, kc, vc = qwen2_forward_ref(ours, tokens[:15], torch.arange(15), kc, vc, md)
    assert relative_error(got, want[:15]) < 1e-4
    for t in range(15, 20):
        md = _paged(tokens[:t + 1].tolist(), BS, NB, start=t)
        got, kc, vc = qwen2_forward_ref(ours, tokens[t:t + 1], torch.tensor([t]), kc, vc, md)
        assert relative_error(got[0], want[t]) < 1e-4


def _seq(i, n_prompt, max_new=4):
    return Sequence(i, list(range(n_prompt)), SamplingParams(max_new_tokens=max_new, ignore_eos=True))


# ---- runner metadata -------------------------------------------------------
def test_build_inputs_matches_the_runner_layout():
    bm = BlockSpaceManager(4, 32, watermark=0.0)
    r = ModelRunner(model=None, kv_cache=type("C", (), {"block_size": 4})(), block_manager=bm, device="cpu")
    a, b = _seq(0, 9), _seq(1, 3)
    a.output_token_ids = [100, 101]
    a.num_computed_tokens = 10          # decoding its 11th token
    for s_, n in ((a, 11), (b, 3)):
        assert bm.allocate(s_, n)
    ids, pos, md, samp, seqs = r.build_inputs([(a, 1), (b, 3)])
    assert ids.tolist() == [101, 0, 1, 2]
    assert pos.tolist() == [10, 0, 1, 2]
    assert samp.tolist() == [0, 3] and seqs == [a, b]
    _, ref = build_metadata([ScheduledSeq(a.block_table, 10, 11, 0), ScheduledSeq(b.block_table, 0, 3, 1)], 4, "cpu")
    for f in ("slot_mapping", "query_start_loc", "seq_lens", "block_tables"):
        assert torch.equal(getattr(md, f), getattr(ref, f)), f
    assert md.seq_lens_cpu == [11, 3] and md.query_start_loc_cpu == [0, 1, 4] and not md.is_decode_only


def test_summary_percentiles_and_tpot():
    recs = []
    for i in range(100):
        m = RequestMetrics(i, 10, arrival=0.0, start=0.0, first_token=0.1, end=0.1 + 0.01 * i, output_tokens=11)
        recs.append(m)
    s = summarize(recs, wall_time=2.0)
    assert s["output_tokens"] == 1100 and s["output_tok_per_s"] == 550.0
    assert abs(s["tpot_p50_ms"] - 0.01 * 49.5 / 10 * 1e3) < 1e-6
    assert abs(s["tpot_p99_ms"] - 0.01 * 98.01 / 10 * 1e3) < 1e-6


def test_random_init_is_seeded_and_tied():
    cfg = Qwen2Config(**{**TINY, "tie_word_embeddings": True})
    a = random_init_(Qwen2ForCausalLM(cfg), seed=5)
    b = random_init_(Qwen2ForCausalLM(cfg), seed=5)
    assert a.lm_head.weight is a.model.embed_tokens.weight
    for (n1, p1), (_, p2) in zip(a.named_parameters(), b.named_parameters()):
        assert torch.equal(p1, p2), n1
    assert torch.equal(a.model.layers[0].input_layernorm.weight, torch.ones(256))


# ---- object lifetimes around graph capture ----------------------------------
def test_an_engine_with_decode_graphs_is_freed_without_the_cycle_collector():
    """Dropping an engine frees its decode graphs (and their pinned staging
    buffers) at once, by reference counting.  Were the graphs and the runner
    to reference each other, they would live until some later cycle
    collection, which may run inside another engine's graph capture: freeing
    a pinned buffer that served a non_blocking copy records an event on the
    copy's stream, which HIP refuses during a capture, and the process
    aborts."""
    import gc
    import weakref

    from nanoserve_amd.engine import LLMEngine

    model = Qwen2ForCausalLM(Qwen2Config(**TINY))
    was = gc.isenabled()
    gc.disable()
    try:
        eng = LLMEngine(model, num_blocks=16, block_size=8, device="cpu", max_model_len=256, use_graphs=True)
        graphs = weakref.ref(eng.runner.graphs)
        runner = weakref.ref(eng.runner)
        del eng
        assert graphs() is None and runner() is None
    finally:
        if was:
            gc.enable()


def test_no_cycle_collection_collects_first_and_holds_the_collector_off():
    import gc
    import weakref

    from nanoserve_amd.capture import no_cycle_collection

    class Node:
        pass

    a, b = Node(), Node()
    a.other, b.other = b, a  # a cycle only the collector can free
    dead = weakref.ref(a)
    del a, b
    was = gc.isenabled()
    gc.enable()
    try:
        with no_cycle_collection():
            assert dead() is None  # collected on entry, before any capture starts
            assert not gc.isenabled()
        assert gc.isenabled()
    finally:
        if not was:
            gc.disable()
