"""Host block bookkeeping used to build verify-step inputs.

A small Python mirror of the reference's KV block manager, which stays in Go and
is untouched by the drop-in (internal/kvcache/block_pool.go:32-114,
internal/kvcache/block_table.go:24-124). It exists so tests and the benchmark can
produce slot mappings and block tables exactly as the engine would:
slot = physical_block * block_size + offset; a new block is taken when the offset
is 0; Truncate releases blocks that become empty; shared (refcount > 1) blocks are
only ever full prefix blocks, so appends never land in them.
"""
from __future__ import annotations


class OutOfBlocks(RuntimeError):
    pass


class BlockPool:
    """Refcounted pool (block_pool.go). Allocate pops from the end of the free list."""

    def __init__(self, total_blocks: int, block_size: int, order=None):
        self.block_size = block_size
        self.total = total_blocks
        self.refcounts = [0] * total_blocks
        self.free = list(order) if order is not None else list(range(total_blocks))

    def allocate(self, n: int) -> list[int]:
        if n <= 0:
            return []
        if n > len(self.free):
            raise OutOfBlocks(f"need {n}, have {len(self.free)}")
        got = self.free[len(self.free) - n:]
        del self.free[len(self.free) - n:]
        for b in got:
            self.refcounts[b] = 1
        return got

    def ref(self, b: int) -> None:
        if 0 <= b < self.total and self.refcounts[b] > 0:
            self.refcounts[b] += 1

    def release(self, b: int) -> None:
        if not (0 <= b < self.total) or self.refcounts[b] <= 0:
            return
        self.refcounts[b] -= 1
        if self.refcounts[b] == 0:
            self.free.append(b)

    def num_free(self) -> int:
        return len(self.free)


class BlockTable:
    """Per-sequence logical -> physical block map (block_table.go)."""

    def __init__(self, pool: BlockPool):
        self.pool = pool
        self.blocks: list[int] = []
        self.num_tokens = 0

    def attach_shared(self, blocks: list[int]) -> None:
        """Attach full, already-written prefix blocks (MatchPrefix, block_table.go:87-106)."""
        for b in blocks:
            self.pool.ref(b)
            self.blocks.append(b)
            self.num_tokens += self.pool.block_size

    def append(self) -> int:
        bs = self.pool.block_size
        off = self.num_tokens % bs
        if off == 0:
            self.blocks.append(self.pool.allocate(1)[0])
        slot = self.blocks[self.num_tokens // bs] * bs + off
        self.num_tokens += 1
        return slot

    def append_n(self, n: int) -> list[int]:
        return [self.append() for _ in range(n)]

    def slot_mapping(self) -> list[int]:
        bs = self.pool.block_size
        return [self.blocks[i // bs] * bs + i % bs for i in range(self.num_tokens)]

    def truncate(self, n: int) -> None:
        if n <= 0 or n > self.num_tokens:
            return
        bs = self.pool.block_size
        for _ in range(n):
            self.num_tokens -= 1
            if self.num_tokens % bs == 0 and len(self.blocks) > self.num_tokens // bs:
                self.pool.release(self.blocks.pop())

    def free(self) -> None:
        for b in self.blocks:
            self.pool.release(b)
        self.blocks = []
        self.num_tokens = 0
