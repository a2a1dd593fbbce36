"""Cache-block ownership and the position -> cache-slot translation.

Pure Python, no torch.  The translation is the addressing contract every
kernel here consumes (reference nanoserve/block_manager.py:93-157): a
sequence owns a list of physical block ids, its `block_table`, and token
position `pos` lives in slot

    slot = block_table[pos // block_size] * block_size + pos % block_size

of the cache viewed as [num_blocks * block_size, num_kv_heads, head_dim].
Asking for a position past the table raises IndexError.

Free blocks are kept on a stack, so a freed block is the next one handed out
(its lines are the likeliest to still sit in the GPU's last-level cache).
Which physical ids a sequence gets is not part of the contract.
"""

from __future__ import annotations


class BlockSpaceManager:
    """Hands cache blocks to sequences and translates their positions to slots.

    A sequence is any object with a `block_table` list (and, for error
    messages, a `seq_id`).  Tables only grow in place; `free` gives the
    sequence a new empty list.  `watermark` holds a fraction of the blocks
    back from `can_allocate` (admission of new requests), never from
    `allocate` (growth of admitted ones), so running sequences can still
    grow when admission stops (reference block_manager.py:64-86).
    """

    def __init__(self, block_size: int, num_gpu_blocks: int, watermark: float = 0.01) -> None:
        if block_size <= 0 or num_gpu_blocks <= 0:
            raise ValueError(f"need a positive block size and block count, got {block_size} and {num_gpu_blocks}")
        self.block_size = block_size
        self.num_total_blocks = num_gpu_blocks
        self.watermark_blocks = int(watermark * num_gpu_blocks)
        self._free_stack = list(range(num_gpu_blocks - 1, -1, -1))  # block 0 on top
        self._held = bytearray(num_gpu_blocks)                      # 1 while some table holds the block

    @property
    def num_free_blocks(self) -> int:
        return len(self._free_stack)

    def blocks_for(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def blocks_needed(self, seq, num_tokens: int) -> int:
        """Blocks `seq` lacks to address positions [0, num_tokens)."""
        return max(self.blocks_for(num_tokens) - len(seq.block_table), 0)

    def can_allocate(self, seq, num_tokens: int, respect_watermark: bool = True) -> bool:
        spare = len(self._free_stack) - (self.watermark_blocks if respect_watermark else 0)
        return self.blocks_needed(seq, num_tokens) <= spare

    def allocate(self, seq, num_tokens: int) -> bool:
        """Extend seq.block_table to cover [0, num_tokens); False (nothing taken) if blocks are short."""
        need = self.blocks_needed(seq, num_tokens)
        if need > len(self._free_stack):
            return False
        for _ in range(need):
            b = self._free_stack.pop()
            self._held[b] = 1
            seq.block_table.append(b)
        return True

    def free(self, seq) -> None:
        """Return every block of `seq` and give it an empty table."""
        table = seq.block_table
        for b in table:
            if not self._held[b]:
                raise ValueError(f"block {b} of sequence {getattr(seq, 'seq_id', '?')} is not held: "
                                 "freed twice or never allocated")
        for b in reversed(table):
            self._held[b] = 0
            self._free_stack.append(b)
        seq.block_table = []

    def slot_mapping(self, seq, start: int, end: int) -> list[int]:
        """Cache slots of positions [start, end) of `seq`."""
        return slots_for_range(seq.block_table, start, end, self.block_size, getattr(seq, "seq_id", "?"))


def slots_for_range(block_table: list[int], start: int, end: int, block_size: int,
                    seq_id="?") -> list[int]:
    """Slots of positions [start, end) through `block_table`.

    Each block contributes one contiguous range of slots, so the list is built
    a block at a time.  Raises IndexError when `end` runs past the table.
    """
    if end <= start:
        return []
    last = (end - 1) // block_size
    if last >= len(block_table):
        raise IndexError(f"sequence {seq_id}: position {end - 1} lies in block {last}, past its "
                         f"{len(block_table)}-block table")
    slots: list[int] = []
    for i in range(start // block_size, last + 1):
        lo = max(start, i * block_size)
        hi = min(end, (i + 1) * block_size)
        shift = (block_table[i] - i) * block_size  # slot - position inside block i
        slots.extend(range(lo + shift, hi + shift))
    return slots
