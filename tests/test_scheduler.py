"""Continuous-batching rules of nanoserve_amd.engine.Scheduler (CPU only).

Bookkeeping bugs in a scheduler show up as livelock, leaked blocks or wrong
batches, never as a numerical error, so these run in milliseconds on the CPU
with a stand-in for the runner.  They cover the behaviours the reference pins
for its scheduler (reference tests/test_scheduler.py:49-286, scheduler.py:
91-262): admission under the token budget and the sequence cap, chunked and
unchunked prefill, running sequences first, block exhaustion, newest-first
preemption by recompute to the front of the queue, the no-preemption mode
failing loudly, requests too large for the cache, progress under heavy
pressure, and the step statistics.
"""

from __future__ import annotations

import pytest

from nanoserve_amd.block_manager import BlockSpaceManager
from nanoserve_amd.engine import SamplingParams, Scheduler, SchedulerConfig, Sequence, SeqStatus


def make(blocks=64, bs=16, budget=1024, max_seqs=256, chunked=True, preemption="recompute"):
    bm = BlockSpaceManager(bs, blocks, watermark=0.0)
    cfg = SchedulerConfig(max_num_batched_tokens=budget, max_num_seqs=max_seqs,
                          enable_chunked_prefill=chunked, preemption_mode=preemption)
    return Scheduler(cfg, bm), bm


def req(i, prompt, max_new=8):
    return Sequence(i, [7] * prompt, SamplingParams(max_new_tokens=max_new, ignore_eos=True))


def step(s, out):
    """The runner's and engine's part of a step: KV computed, a token when due, stops, frees."""
    for seq, q in out.scheduled:
        seq.advance_computed(q)
        if seq.num_computed_tokens == seq.num_tokens:
            seq.output_token_ids.append(1)
            seq.check_stop(None)
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
    assert all(len(x.output_token_ids) == 5 and x.status is SeqStatus.FINISHED_LENGTH for x in done)
    assert bm.num_free_blocks == 128 and not s.has_work


def test_a_long_prompt_is_prefilled_in_budget_sized_chunks():
    s, _ = make(budget=64)
    s.add(req(0, 200, max_new=2))
    chunks = []
    while True:
        out = s.schedule()
        seq, q = out.scheduled[0]
        if not seq.is_prefilling:
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
    assert s.stats.mixed_steps == 1


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


def _fill_and_grow(s, extra=None):
    """Two 32-token prompts fill 4 blocks; decoding then needs a fifth."""
    for i in range(2):
        s.add(req(i, 32, max_new=200))
    step(s, s.schedule())
    if extra is not None:
        s.add(extra)
    for _ in range(60):
        out = s.schedule()
        if out.preempted:
            return out
        step(s, out)
    raise AssertionError("no preemption happened")


def test_growth_past_the_cache_preempts_the_newest_by_recompute():
    s, bm = make(blocks=4, budget=10_000)
    out = _fill_and_grow(s)
    victim = out.preempted[0]
    assert victim.seq_id == 1 and s.stats.total_preemptions == 1 == s.num_preemptions
    assert victim.status is SeqStatus.PREEMPTED and victim.block_table == [] and victim.num_computed_tokens == 0
    # Its generated tokens stay; the recompute prefills prompt and outputs together.
    assert victim.output_token_ids and victim.num_uncomputed_tokens == 32 + len(victim.output_token_ids)
    assert [(x.seq_id, q) for x, q in out.scheduled] == [(0, 1)]


def test_a_preempted_request_goes_to_the_front_of_the_queue():
    s, _ = make(blocks=4, budget=10_000)
    newcomer = req(99, 16, max_new=4)
    out = _fill_and_grow(s, extra=newcomer)
    assert s.waiting[0] is out.preempted[0] and newcomer in s.waiting


def test_without_preemption_exhaustion_raises_instead_of_stalling():
    s, _ = make(blocks=4, budget=10_000, preemption="none")
    for i in range(2):
        s.add(req(i, 32, max_new=200))
    with pytest.raises(RuntimeError, match="preemption disabled"):
        drain(s, limit=60)
    with pytest.raises(ValueError):
        Scheduler(SchedulerConfig(preemption_mode="swap"), BlockSpaceManager(16, 4, watermark=0.0))


def test_a_request_larger_than_the_cache_is_rejected():
    for mode in ("recompute", "none"):
        s, _ = make(blocks=2, budget=10_000, preemption=mode)
        s.add(req(0, 16, max_new=200))
        with pytest.raises(ValueError, match="KV blocks"):
            drain(s, limit=400)


def test_the_queue_drains_under_constant_preemption():
    s, bm = make(blocks=12, budget=512)
    for i in range(8):
        s.add(req(i, 48, max_new=24))
    done = drain(s)
    assert len(done) == 8 and all(len(x.output_token_ids) == 24 for x in done)
    assert s.stats.total_preemptions > 0 and bm.num_free_blocks == 12


def test_running_sequences_are_served_before_new_ones():
    s, _ = make(budget=4)
    s.add(req(0, 4, max_new=10))
    step(s, s.schedule())
    s.add(req(1, 64, max_new=10))
    out = s.schedule()
    assert out.scheduled[0][0].seq_id == 0 and out.scheduled[0][1] == 1


def test_statistics_count_every_token():
    s, _ = make(blocks=256)
    for i in range(4):
        s.add(req(i, 32, max_new=6))
    drain(s)
    st = s.stats
    assert st.total_prefill_tokens == 4 * 32
    assert st.total_decode_tokens == 4 * 5  # the last token is sampled, never fed back
    assert st.total_steps == 6 and st.mean_batch_size == 4.0 and st.total_preemptions == 0
