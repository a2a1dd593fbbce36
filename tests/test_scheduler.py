"""Continuous-batching rules of nanoserve_amd.scheduling (CPU only).

Bookkeeping bugs in a scheduler show up as livelock, leaked blocks or wrong
batches, never as a numerical error, so these run in milliseconds on the CPU
with a stand-in for the runner.  They cover the behaviours the reference pins
for its scheduler (reference tests/test_scheduler.py:49-286, scheduler.py:
91-262) that shape config 5's batches: admission under the token budget and
the sequence cap, chunked and unchunked prefill, running sequences first,
block exhaustion, newest-first eviction by recompute to the front of the
queue, requests too large for the cache, and progress under heavy pressure.
"""

from __future__ import annotations

import pytest

from nanoserve_amd.block_manager import BlockSpaceManager
from nanoserve_amd.scheduling import SamplingParams, Scheduler, SchedulerConfig, Sequence, SeqState


def make(blocks=64, bs=16, budget=1024, max_seqs=256, chunked=True, preemption="recompute"):
    bm = BlockSpaceManager(bs, blocks, watermark=0.0)
    cfg = SchedulerConfig(max_num_batched_tokens=budget, max_num_seqs=max_seqs, enable_chunked_prefill=chunked,
                          preemption_mode=preemption)
    return Scheduler(cfg, bm), bm


def req(i, prompt, max_new=8):
    return Sequence(i, list(range(prompt)), SamplingParams(max_new_tokens=max_new, ignore_eos=True))


def step(s, out):
    """The runner's and engine's part of a step: KV computed, a token when due, stops, frees."""
    for seq, q in out.scheduled:
        seq.mark_computed(q)
        if seq.num_computed_tokens == seq.num_tokens:
            seq.output_token_ids.append(1)
            seq.check_done(None)
    return s.free_finished()


def drain(s, limit=20_000):
    done = []
    for _ in range(limit):
        out = s.schedule()
        if not out:
            break
        done += step(s, out)
    return done


def test_nothing_to_schedule():
    s, _ = make()
    out = s.schedule()
    assert not out and out.num_batched_tokens == 0 and not s.has_work


def test_prefill_then_decode_steps():
    s, _ = make()
    s.add(req(0, 10, max_new=3))
    out = s.schedule()
    assert [q for _, q in out.scheduled] == [10]
    assert (out.num_prefill_seqs, out.num_decode_seqs, out.num_batched_tokens) == (1, 0, 10)
    step(s, out)
    out = s.schedule()
    assert [q for _, q in out.scheduled] == [1]
    assert (out.num_prefill_seqs, out.num_decode_seqs) == (0, 1)


def test_budget_is_shared_and_prompts_are_chunked():
    s, _ = make(budget=10, bs=4)
    a, b = req(0, 7), req(1, 9)
    s.add(a)
    s.add(b)
    out = s.schedule()
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 7), (1, 3)]
    step(s, out)
    out = s.schedule()
    # a decodes first (running sequences get the budget first), b continues its prefill.
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 1), (1, 6)]


def test_step_never_exceeds_the_token_budget():
    s, _ = make(budget=100)
    for i in range(5):
        s.add(req(i, 40))
    for _ in range(30):
        out = s.schedule()
        if not out:
            break
        assert out.num_batched_tokens <= 100
        step(s, out)


def test_sequence_cap_limits_the_batch():
    s, _ = make(budget=10_000, max_seqs=3)
    for i in range(10):
        s.add(req(i, 8))
    out = s.schedule()
    assert len(out.scheduled) == 3 and len(s.waiting) == 7


def test_everything_finishes_and_every_block_returns():
    s, bm = make(blocks=128)
    for i in range(6):
        s.add(req(i, 20, max_new=5))
    done = drain(s)
    assert sorted(x.seq_id for x in done) == list(range(6))
    assert all(len(x.output_token_ids) == 5 and x.state is SeqState.DONE_LENGTH for x in done)
    assert bm.num_free_blocks == 128 and not s.has_work


def test_a_long_prompt_is_prefilled_in_budget_sized_chunks():
    s, _ = make(budget=64)
    s.add(req(0, 200, max_new=2))
    chunks = []
    while True:
        out = s.schedule()
        seq, q = out.scheduled[0]
        if not seq.in_prompt:
            break
        chunks.append(q)
        step(s, out)
    assert sum(chunks) == 200 and max(chunks) == 64 and len(chunks) == 4


def test_a_big_prompt_does_not_stall_running_decodes():
    s, _ = make(budget=64)
    s.add(req(0, 8, max_new=50))
    step(s, s.schedule())
    s.add(req(1, 500, max_new=2))
    out = s.schedule()
    assert (out.num_decode_seqs, out.num_prefill_seqs) == (1, 1)
    assert out.scheduled[0] == (s.running[0], 1) and out.num_batched_tokens == 64


def test_without_chunking_a_prompt_is_scheduled_whole_or_not_at_all():
    s, _ = make(budget=64, chunked=False)
    s.add(req(0, 40))
    s.add(req(1, 40))
    out = s.schedule()
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 40)]


def test_without_chunking_a_prompt_over_the_budget_raises():
    s, _ = make(budget=32, chunked=False)
    s.add(req(0, 100))
    with pytest.raises(ValueError, match="max_num_batched_tokens"):
        s.schedule()


def test_admission_stops_when_the_blocks_run_out():
    s, bm = make(blocks=4, budget=10_000)
    for i in range(10):
        s.add(req(i, 32))  # two 16-token blocks each
    out = s.schedule()
    assert [x.seq_id for x, _ in out.scheduled] == [0, 1]
    assert bm.num_free_blocks == 0 and len(s.waiting) == 8


def test_admission_keeps_the_watermark_but_growth_may_use_it():
    bm = BlockSpaceManager(4, 10, watermark=0.2)
    s = Scheduler(SchedulerConfig(max_num_batched_tokens=1000, max_num_seqs=8), bm)
    s.add(req(0, 32, max_new=40))  # 8 blocks: exactly what admission may take
    s.add(req(1, 4))
    out = s.schedule()
    assert [x.seq_id for x, _ in out.scheduled] == [0] and bm.num_free_blocks == 2
    for _ in range(8):  # decoding fills the reserve
        step(s, out)
        out = s.schedule()
    assert bm.num_free_blocks < 2 and not out.preempted


def test_out_of_blocks_evicts_the_newest_and_recomputes():
    # 6 blocks of 4 tokens: two 11-token prompts take 3 blocks each; the first
    # decode step needs a 4th block for sequence 0 and evicts sequence 1.
    s, bm = make(budget=64, blocks=6, bs=4)
    a, b = req(0, 11, max_new=8), req(1, 11, max_new=8)
    s.add(a)
    s.add(b)
    step(s, s.schedule())
    assert bm.num_free_blocks == 0
    step(s, s.schedule())  # both decode a 12th token: still 3 blocks each
    out = s.schedule()     # position 12 needs a 4th block
    assert [x.seq_id for x in out.preempted] == [1] and s.num_preemptions == 1
    assert b.state is SeqState.EVICTED and b.num_computed_tokens == 0 and b.block_table == []
    assert s.waiting[0] is b and b.num_evictions == 1
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 1)]
    # Its generated tokens stay; the recompute prefills prompt and outputs together.
    assert b.pending_tokens == 13 and b.token_slice(10, 13) == [10, 1, 1]


def test_an_evicted_request_goes_to_the_front_of_the_queue():
    s, _ = make(blocks=4, budget=10_000)
    for i in range(2):
        s.add(req(i, 32, max_new=200))
    step(s, s.schedule())
    newcomer = req(99, 16, max_new=4)
    s.add(newcomer)
    for _ in range(60):
        out = s.schedule()
        if out.preempted:
            break
        step(s, out)
    assert out.preempted and s.waiting[0] is out.preempted[0] and newcomer in s.waiting


def test_without_preemption_exhaustion_raises_instead_of_evicting():
    # The reference's ablation (scheduler.py:213-243): the case that evicts
    # sequence 1 under "recompute" stops the engine under "none", and nothing
    # was evicted before the error.
    s, bm = make(budget=64, blocks=6, bs=4, preemption="none")
    a, b = req(0, 11, max_new=8), req(1, 11, max_new=8)
    s.add(a)
    s.add(b)
    step(s, s.schedule())
    step(s, s.schedule())
    with pytest.raises(RuntimeError, match="preemption_mode='none'"):
        s.schedule()
    assert s.num_preemptions == 0 and b.state is SeqState.RUNNING and len(b.block_table) == 3


def test_without_preemption_a_fitting_workload_still_completes():
    s, bm = make(blocks=64, budget=256, preemption="none")
    for i in range(6):
        s.add(req(i, 40, max_new=12))
    done = drain(s)
    assert len(done) == 6 and s.num_preemptions == 0 and bm.num_free_blocks == 64


def test_without_preemption_an_oversized_request_is_still_a_value_error():
    s, _ = make(blocks=2, budget=10_000, preemption="none")
    s.add(req(0, 16, max_new=200))
    with pytest.raises(ValueError, match="cannot fit the KV cache"):
        drain(s, limit=400)


def test_unknown_preemption_modes_are_rejected():
    with pytest.raises(ValueError, match="preemption_mode"):
        SchedulerConfig(preemption_mode="swap")
    assert SchedulerConfig().preemption_mode == "recompute"


def test_a_request_larger_than_the_cache_is_rejected():
    s, _ = make(blocks=2, budget=10_000)
    s.add(req(0, 16, max_new=200))
    with pytest.raises(ValueError, match="cannot fit the KV cache"):
        drain(s, limit=400)


def test_the_queue_drains_under_constant_eviction():
    s, bm = make(blocks=12, budget=512)
    for i in range(8):
        s.add(req(i, 48, max_new=24))
    done = drain(s)
    assert len(done) == 8 and all(len(x.output_token_ids) == 24 for x in done)
    assert s.num_preemptions > 0 and bm.num_free_blocks == 12


def test_running_sequences_are_served_before_new_ones():
    s, _ = make(budget=4)
    s.add(req(0, 4, max_new=10))
    step(s, s.schedule())
    s.add(req(1, 64, max_new=10))
    out = s.schedule()
    assert out.scheduled[0][0].seq_id == 0 and out.scheduled[0][1] == 1


def test_finished_sequences_release_their_blocks():
    s, bm = make(budget=64, blocks=16, bs=4)
    a = req(0, 5, max_new=1)
    s.add(a)
    step(s, s.schedule())
    assert a.state is SeqState.DONE_LENGTH and bm.num_free_blocks == 16 and not s.has_work


def test_eos_stops_unless_ignored():
    a = Sequence(0, [1, 2], SamplingParams(max_new_tokens=5))
    a.output_token_ids.append(7)
    assert a.check_done(7) and a.state is SeqState.DONE_EOS
    b = Sequence(1, [1, 2], SamplingParams(max_new_tokens=5, ignore_eos=True))
    b.output_token_ids.append(7)
    assert not b.check_done(7) and b.state is SeqState.QUEUED
