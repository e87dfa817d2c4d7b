"""Host-side bookkeeping of the paged KV pool: which pool blocks hold each
sequence's tokens.

Mirrors nanoPD/block_manager/block_manager.py:11-115:
- the allocator is a LIFO free list that starts as [0 .. N-1], so the first
  allocation returns the highest block index;
- blocks are reference counted, and fork shares a table;
- append_slot returns the (old, new) pair of a copy-on-write when the block
  the next token goes to is shared.

The copy itself runs on the GPU with paged_kernels.copy_blocks, which the
reference never performs (block_manager.py:91-96 only returns the pair).
"""
from __future__ import annotations

from typing import Optional


class BlockAllocator:
    """LIFO allocator of pool blocks with reference counts
    (block_manager.py:11-39)."""

    def __init__(self, num_blocks: int):
        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        self._free = list(range(num_blocks))
        self._ref = [0] * num_blocks
        self.num_total_blocks = num_blocks

    def allocate(self) -> int:
        if not self._free:
            raise MemoryError("OOM: no free KV blocks")
        b = self._free.pop()
        self._ref[b] = 1
        return b

    def share(self, b: int) -> None:
        self._ref[b] += 1

    def free(self, b: int) -> None:
        if self._ref[b] <= 0:
            raise ValueError(f"block {b} is not allocated")
        self._ref[b] -= 1
        if self._ref[b] == 0:
            self._free.append(b)

    def ref_count(self, b: int) -> int:
        return self._ref[b]

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)


class BlockSpaceManager:
    """Per-sequence block tables over one pool (block_manager.py:41-115)."""

    def __init__(self, block_size: int, num_blocks: int):
        self.block_size = block_size
        self.allocator = BlockAllocator(num_blocks)
        self._tables: dict[int, list[int]] = {}

    def blocks_for(self, num_tokens: int) -> int:
        return (num_tokens + self.block_size - 1) // self.block_size

    def can_allocate(self, num_tokens: int) -> bool:
        return self.allocator.num_free_blocks >= self.blocks_for(num_tokens)

    def allocate(self, seq_id: int, num_tokens: int) -> list[int]:
        """Blocks for a new sequence's first num_tokens tokens (the prompt)."""
        if seq_id in self._tables:
            raise ValueError(f"sequence {seq_id} already has a block table")
        self._tables[seq_id] = [self.allocator.allocate() for _ in range(self.blocks_for(num_tokens))]
        return self._tables[seq_id]

    def can_append_slot(self, num_seqs: int = 1) -> bool:
        return self.allocator.num_free_blocks >= num_seqs

    def append_slot(self, seq_id: int, position: int) -> Optional[tuple[int, int]]:
        """Make room for the token at `position` (0-based). Returns (old, new)
        when the block it goes to was shared and has been replaced by a private
        copy target, else None (block_manager.py:72-98)."""
        table = self._tables[seq_id]
        if position // self.block_size + 1 > len(table):
            table.append(self.allocator.allocate())
            return None
        last = table[-1]
        if self.allocator.ref_count(last) > 1:
            new = self.allocator.allocate()
            self.allocator.free(last)
            table[-1] = new
            return (last, new)
        return None

    def fork(self, parent_id: int, child_id: int) -> None:
        table = list(self._tables[parent_id])
        for b in table:
            self.allocator.share(b)
        self._tables[child_id] = table

    def free(self, seq_id: int) -> None:
        for b in self._tables.pop(seq_id, []):
            self.allocator.free(b)

    def block_table(self, seq_id: int) -> list[int]:
        return self._tables[seq_id]

    @property
    def num_free_blocks(self) -> int:
        return self.allocator.num_free_blocks
