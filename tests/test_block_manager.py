"""Paging arithmetic of nanoserve_amd.block_manager (CPU only).

The slot mapping is the cache write's addressing contract: an off-by-one
silently reads or overwrites another sequence's KV.  These tests cover the
behaviours the reference pins for its block manager (reference
tests/test_block_manager.py:22-171): allocation round trips and failures,
incremental growth, the watermark, the closed-form slot formula
(block_manager.py:131-132), contiguity inside a block, the decode step's slot,
running past the table, and no aliasing between live sequences -- plus the
block-run emission against a per-token brute force.
"""

from __future__ import annotations

import random

import pytest

from nanoserve_amd.block_manager import BlockSpaceManager, slots_for_range
from nanoserve_amd.scheduling import SamplingParams, Sequence
from oracle.paged_attention import slot_mapping_ref


def _seq(seq_id=0, prompt_len=10):
    return Sequence(seq_id, list(range(prompt_len)), SamplingParams(max_new_tokens=5))


class _Owner:
    def __init__(self, seq_id=0):
        self.seq_id = seq_id
        self.block_table: list[int] = []


def test_allocation_round_trip_and_counts():
    m = BlockSpaceManager(4, 8, watermark=0.0)
    s = _Owner()
    assert m.allocate(s, 12) and len(s.block_table) == 3 and m.num_free_blocks == 5
    m.free(s)
    assert m.num_free_blocks == 8 and s.block_table == []


def test_short_pool_takes_nothing_and_double_free_raises():
    m = BlockSpaceManager(4, 2, watermark=0.0)
    s = _Owner()
    assert not m.allocate(s, 12)
    assert m.num_free_blocks == 2 and s.block_table == []
    assert m.allocate(s, 8)
    held = list(s.block_table)
    m.free(s)
    s.block_table = held
    with pytest.raises(ValueError):
        m.free(s)
    with pytest.raises(ValueError):
        BlockSpaceManager(16, 0)


def test_blocks_are_never_handed_out_twice():
    m = BlockSpaceManager(1, 16, watermark=0.0)
    x, y = _Owner(0), _Owner(1)
    m.allocate(x, 5)
    m.allocate(y, 5)
    assert not set(x.block_table) & set(y.block_table)
    m.free(x)
    z = _Owner(2)
    m.allocate(z, 5)
    assert not set(z.block_table) & set(y.block_table)
    assert sorted(set(z.block_table) | set(y.block_table)) == sorted(z.block_table + y.block_table)


def test_blocks_for_rounds_up():
    m = BlockSpaceManager(16, 100)
    assert [m.blocks_for(n) for n in (0, 1, 16, 17, 32, 33)] == [0, 1, 1, 2, 2, 3]


def test_allocation_grows_incrementally():
    m = BlockSpaceManager(4, 100)
    s = _seq(prompt_len=10)
    assert m.allocate(s, 10) and len(s.block_table) == 3
    assert m.allocate(s, 12) and len(s.block_table) == 3
    assert m.allocate(s, 13) and len(s.block_table) == 4
    assert m.blocks_needed(s, 20) == 1


def test_failed_allocation_leaves_no_partial_state():
    m = BlockSpaceManager(4, 2, watermark=0.0)
    s = _seq(prompt_len=20)
    assert not m.allocate(s, 20)
    assert s.block_table == [] and m.num_free_blocks == 2


def test_watermark_reserves_headroom_for_admission_only():
    m = BlockSpaceManager(4, 100, watermark=0.1)
    assert m.watermark_blocks == 10
    s = _seq(prompt_len=4 * 95)
    assert not m.can_allocate(s, 4 * 95)
    assert m.can_allocate(s, 4 * 95, respect_watermark=False)
    assert m.allocate(s, 4 * 95)  # growth of a running sequence may use the reserve


def test_free_returns_every_block():
    m = BlockSpaceManager(8, 32)
    seqs = [_seq(i, prompt_len=20) for i in range(4)]
    for s in seqs:
        assert m.allocate(s, 20)
    assert m.num_free_blocks == 32 - 4 * 3
    for s in seqs:
        m.free(s)
    assert m.num_free_blocks == 32 and all(s.block_table == [] for s in seqs)


def test_slot_mapping_matches_the_closed_form():
    m = BlockSpaceManager(4, 16)
    s = _seq(prompt_len=10)
    m.allocate(s, 10)
    bt = s.block_table
    assert m.slot_mapping(s, 0, 10) == [bt[p // 4] * 4 + p % 4 for p in range(10)]
    assert m.slot_mapping(s, 0, 10) == slot_mapping_ref(bt, 0, 10, 4)


def test_slots_are_contiguous_inside_a_block():
    m = BlockSpaceManager(8, 16)
    s = _seq(prompt_len=8)
    m.allocate(s, 8)
    slots = m.slot_mapping(s, 0, 8)
    assert slots == list(range(slots[0], slots[0] + 8))


def test_decode_step_slot_continues_the_tail_block():
    m = BlockSpaceManager(4, 16)
    s = _seq(prompt_len=6)
    m.allocate(s, 6)
    prefill = m.slot_mapping(s, 0, 6)
    m.allocate(s, 7)
    assert m.slot_mapping(s, 6, 7) == [prefill[4] + 2]  # block 1, offset 2


def test_slot_mapping_past_the_table_raises():
    m = BlockSpaceManager(4, 16)
    s = _seq(prompt_len=4)
    m.allocate(s, 4)
    with pytest.raises(IndexError):
        m.slot_mapping(s, 0, 5)


def test_live_sequences_never_share_a_slot():
    m = BlockSpaceManager(4, 64)
    seen = set()
    for i in range(5):
        s = _seq(i, prompt_len=13)
        m.allocate(s, 13)
        slots = set(m.slot_mapping(s, 0, 13))
        assert not seen & slots
        seen |= slots


def test_reused_blocks_do_not_alias_live_ones():
    m = BlockSpaceManager(4, 8, watermark=0.0)
    a, b = _seq(0, 8), _seq(1, 8)
    m.allocate(a, 8)
    m.allocate(b, 8)
    live_b = set(m.slot_mapping(b, 0, 8))
    m.free(a)
    c = _seq(2, 8)
    assert m.allocate(c, 8)
    assert not set(m.slot_mapping(c, 0, 8)) & live_b


def test_block_runs_equal_per_token_brute_force():
    rng = random.Random(5)
    for _ in range(200):
        bs = rng.choice([1, 2, 4, 8, 16, 32])
        table = rng.sample(range(500), rng.randint(1, 12))
        end = rng.randint(0, len(table) * bs)
        start = rng.randint(0, end)
        assert slots_for_range(table, start, end, bs) == slot_mapping_ref(table, start, end, bs)
