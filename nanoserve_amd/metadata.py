"""Build AttentionMetadata for one step the way the engine's runner does.

Follows reference ModelRunner.build_inputs / _stage (model_runner.py:52-147):
the batch is flattened in scheduler order with no padding; for each sequence
computing positions [start, end) it appends `end - start` query rows, the
slots of those positions, `query_start_loc` prefix sums and `seq_lens = end`;
block tables are truncated to ceil(max_seq_len / block_size) columns and
zero-padded (block 0 is a real block, which is why kernels bound every loop by
the sequence length).  All integer vectors travel to the device in one int64
copy and the metadata tensors are views into that buffer.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .attention import AttentionMetadata
from .block_manager import slots_for_range


@dataclass
class ScheduledSeq:
    """One sequence's share of a step: compute positions [start, end)."""

    block_table: list[int]
    start: int
    end: int
    seq_id: int = 0
    token_ids: list[int] = field(default_factory=list)


def build_metadata(batch: list[ScheduledSeq], block_size: int, device) -> tuple[torch.Tensor, AttentionMetadata]:
    """Return (positions, metadata) for a flattened step over `batch`."""
    if not batch:
        raise ValueError("empty batch")
    positions: list[int] = []
    slots: list[int] = []
    qsl = [0]
    seq_lens: list[int] = []
    query_lens: list[int] = []
    for s in batch:
        q = s.end - s.start
        positions.extend(range(s.start, s.end))
        slots.extend(slots_for_range(s.block_table, s.start, s.end, block_size, s.seq_id))
        qsl.append(qsl[-1] + q)
        seq_lens.append(s.end)
        query_lens.append(q)

    max_seq_len = max(seq_lens)
    max_blocks = -(-max_seq_len // block_size)
    bt_flat: list[int] = []
    for s in batch:
        row = s.block_table[:max_blocks]
        bt_flat.extend(row)
        bt_flat.extend([0] * (max_blocks - len(row)))

    chunks = [positions, slots, qsl, seq_lens, bt_flat]
    host = torch.tensor([v for c in chunks for v in c], dtype=torch.int64)
    dev = host.to(device)
    views, off = [], 0
    for c in chunks:
        views.append(dev[off:off + len(c)])
        off += len(c)
    pos_t, slot_t, qsl_t, sl_t, bt_t = views

    md = AttentionMetadata(
        slot_mapping=slot_t,
        query_start_loc=qsl_t,
        seq_lens=sl_t,
        block_tables=bt_t.view(len(batch), max_blocks),
        max_query_len=max(query_lens),
        max_seq_len=max_seq_len,
        num_seqs=len(batch),
        num_tokens=len(positions),
        is_decode_only=all(q == 1 for q in query_lens),
        query_lens_cpu=query_lens,
        seq_lens_cpu=seq_lens,
        query_start_loc_cpu=qsl,
    )
    return pos_t, md
