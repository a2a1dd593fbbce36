"""The engine harness on the CPU: model oracle, scheduler and runner bookkeeping.

* The model oracle (oracle/qwen2.py) is pinned against an independent
  implementation: transformers' own Qwen2ForCausalLM on identical float32
  weights (the reference's third model property, reference
  tests/test_model.py:1-14), both for one-shot prefill and for incremental
  decode through the paged cache.
* The scheduler follows the reference rules (scheduler.py:91-262): running
  first, token budget, chunked prefill, newest-first preemption by recompute.
* The runner's metadata is the engine layout (model_runner.py:85-147).
"""

from __future__ import annotations

import pytest
import torch

from nanoserve_amd.block_manager import BlockSpaceManager
from nanoserve_amd.engine import (ModelRunner, RequestMetrics, SamplingParams, Scheduler, SchedulerConfig,
                                  Sequence, SeqStatus, summarize)
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


# ---- scheduler -------------------------------------------------------------
def _seq(i, n_prompt, max_new=4):
    return Sequence(i, list(range(n_prompt)), SamplingParams(max_new_tokens=max_new, ignore_eos=True))


def _sched(budget=64, max_seqs=8, blocks=64, bs=4, chunked=True):
    bm = BlockSpaceManager(bs, blocks, watermark=0.0)
    return Scheduler(SchedulerConfig(budget, max_seqs, chunked), bm), bm


def _finish_step(out):
    """What the runner and engine do after a step: advance, emit a token when due."""
    for seq, q in out.scheduled:
        seq.advance_computed(q)
        if seq.num_computed_tokens == seq.num_tokens:
            seq.output_token_ids.append(0)
            seq.check_stop(None)


def test_budget_is_shared_and_prompts_are_chunked():
    s, _ = _sched(budget=10)
    a, b = _seq(0, 7), _seq(1, 9)
    s.add(a)
    s.add(b)
    out = s.schedule()
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 7), (1, 3)]
    _finish_step(out)
    out = s.schedule()
    # a decodes first (running sequences get the budget first), b continues its prefill.
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 1), (1, 6)]


def test_unchunked_prefill_waits_for_a_whole_budget():
    s, _ = _sched(budget=10, chunked=False)
    a, b = _seq(0, 7), _seq(1, 9)
    s.add(a)
    s.add(b)
    out = s.schedule()
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 7)]
    with pytest.raises(ValueError):
        s2, _ = _sched(budget=8, chunked=False)
        s2.add(_seq(2, 9))
        s2.schedule()


def test_max_num_seqs_caps_admission():
    s, _ = _sched(budget=100, max_seqs=2)
    for i in range(3):
        s.add(_seq(i, 5))
    out = s.schedule()
    assert [x.seq_id for x, _ in out.scheduled] == [0, 1]
    assert len(s.waiting) == 1


def test_out_of_blocks_preempts_the_newest_and_recomputes():
    # 6 blocks of 4 tokens: two 11-token prompts take 3 blocks each; the first
    # decode step needs a 4th block for sequence 0 and evicts sequence 1.
    s, bm = _sched(budget=64, blocks=6, bs=4)
    a, b = _seq(0, 11, max_new=8), _seq(1, 11, max_new=8)
    s.add(a)
    s.add(b)
    _finish_step(s.schedule())
    assert bm.num_free_blocks == 0
    _finish_step(s.schedule())  # both decode a 12th token: still 3 blocks each
    out = s.schedule()          # position 12 needs a 4th block
    assert [x.seq_id for x in out.preempted] == [1]
    assert b.status is SeqStatus.PREEMPTED and b.num_computed_tokens == 0 and b.block_table == []
    assert s.waiting[0] is b and b.num_preemptions == 1
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 1)]
    # Recompute later covers prompt + generated tokens in one prefill.
    assert b.num_uncomputed_tokens == 13


def test_request_larger_than_the_cache_is_rejected():
    s, _ = _sched(budget=64, blocks=2, bs=4)
    s.add(_seq(0, 8, max_new=4))
    _finish_step(s.schedule())
    with pytest.raises(ValueError):
        s.schedule()


def test_finished_sequences_release_their_blocks():
    s, bm = _sched(budget=64, blocks=16, bs=4)
    a = _seq(0, 5, max_new=1)
    s.add(a)
    _finish_step(s.schedule())
    assert a.status is SeqStatus.FINISHED_LENGTH
    assert s.free_finished() == [a]
    assert bm.num_free_blocks == 16 and not s.has_work


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
