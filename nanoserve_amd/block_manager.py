"""Physical KV block allocation and logical-to-physical slot translation.

Pure Python, no torch.  This is the addressing contract the kernels consume
(reference nanoserve/block_manager.py:27-173): a sequence owns a block table
of physical block ids, and token position `pos` lives in cache slot

    slot = block_table[pos // block_size] * block_size + pos % block_size

of the [num_blocks * block_size, Hkv, D] cache view.  `slot_mapping` emits the
slots of [start, end) a whole block run at a time and raises IndexError past
the table, like reference block_manager.py:124-157.
"""

from __future__ import annotations

from collections import deque


class BlockAllocator:
    """FIFO free list over physical blocks [0, num_blocks)."""

    def __init__(self, num_blocks: int) -> None:
        if num_blocks <= 0:
            raise ValueError(f"num_blocks must be positive, got {num_blocks}")
        self.num_blocks = num_blocks
        self._free: deque[int] = deque(range(num_blocks))
        self._used: set[int] = set()

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_used(self) -> int:
        return len(self._used)

    def allocate(self, n: int = 1) -> list[int]:
        if n > len(self._free):
            raise MemoryError(f"requested {n} blocks, {len(self._free)} free")
        got = [self._free.popleft() for _ in range(n)]
        self._used.update(got)
        return got

    def free(self, blocks: list[int]) -> None:
        for b in blocks:
            if b not in self._used:
                raise ValueError(f"double free of block {b}")
            self._used.remove(b)
            self._free.append(b)

    def reset(self) -> None:
        self._free = deque(range(self.num_blocks))
        self._used.clear()


class BlockSpaceManager:
    """Owns the allocator and every sequence's block table.

    A sequence is any object with a mutable `block_table` list (and, for the
    reporting helpers, `num_tokens` / `seq_id`).  `watermark` keeps a fraction
    of the blocks out of reach of new admissions so running sequences can
    still grow (reference block_manager.py:64-86).
    """

    def __init__(self, block_size: int, num_gpu_blocks: int, watermark: float = 0.01) -> None:
        self.block_size = block_size
        self.allocator = BlockAllocator(num_gpu_blocks)
        self.watermark_blocks = int(watermark * num_gpu_blocks)

    @property
    def num_free_blocks(self) -> int:
        return self.allocator.num_free

    @property
    def num_total_blocks(self) -> int:
        return self.allocator.num_blocks

    def blocks_for(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def blocks_needed(self, seq, num_tokens: int) -> int:
        return max(0, self.blocks_for(num_tokens) - len(seq.block_table))

    def can_allocate(self, seq, num_tokens: int, respect_watermark: bool = True) -> bool:
        budget = self.allocator.num_free - (self.watermark_blocks if respect_watermark else 0)
        return self.blocks_needed(seq, num_tokens) <= budget

    def allocate(self, seq, num_tokens: int) -> bool:
        """Grow seq.block_table to address num_tokens; False when out of blocks."""
        need = self.blocks_needed(seq, num_tokens)
        if need == 0:
            return True
        if need > self.allocator.num_free:
            return False
        seq.block_table.extend(self.allocator.allocate(need))
        return True

    def free(self, seq) -> None:
        if seq.block_table:
            self.allocator.free(seq.block_table)
            seq.block_table = []

    def slot_mapping(self, seq, start: int, end: int) -> list[int]:
        """Cache slots of logical positions [start, end) of `seq`."""
        return slots_for_range(seq.block_table, start, end, self.block_size,
                               getattr(seq, "seq_id", "?"))

    def utilization(self) -> float:
        return self.allocator.num_used / self.allocator.num_blocks

    def fragmentation_waste(self, seqs) -> int:
        """Allocated-but-unused token slots; at most block_size - 1 per sequence."""
        return sum(len(s.block_table) * self.block_size - s.num_tokens for s in seqs if s.block_table)


def slots_for_range(block_table: list[int], start: int, end: int, block_size: int,
                    seq_id="?") -> list[int]:
    """Slots of positions [start, end) through `block_table`, one block run per step."""
    out: list[int] = []
    pos = start
    while pos < end:
        idx, off = divmod(pos, block_size)
        if idx >= len(block_table):
            raise IndexError(
                f"seq {seq_id}: position {pos} needs block {idx} but block_table has "
                f"{len(block_table)} entries")
        run = min(block_size - off, end - pos)
        first = block_table[idx] * block_size + off
        out.extend(range(first, first + run))
        pos += run
    return out
