"""CPU restatement of the reference's KV block manager -- test infrastructure.

This module is the oracle for the native block manager
(vllm-jax_amd/csrc/block_manager.cpp): only tests import it.  It restates
``KVCacheManager`` of vllm/src/kv_cache_manager.py:14-70 -- a FIFO queue of
free blocks, a per-request list of blocks, reference counts -- with request
state passed in as (request id, token count) instead of a Request object.
"""
from __future__ import annotations

from collections import deque


def ceil_div(a: int, b: int) -> int:
    """kv_cache_manager.py:7."""
    return (a + b - 1) // b


class BlockManagerOracle:
    """kv_cache_manager.py:14-70, block for block."""

    def __init__(self, num_blocks: int, block_size: int):
        # :16-22: every block starts free, queued in id order
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.ref = [0] * num_blocks
        self.free = deque(range(num_blocks))
        self.tables: dict[int, list[int]] = {}

    def block_table(self, rid: int) -> list[int]:
        """:24-27 (creates an empty table on first use)."""
        return self.tables.setdefault(rid, [])

    def can_allocate(self, rid: int, num_tokens: int, is_prefill: bool) -> bool:
        """:29-41."""
        table = self.block_table(rid)
        if is_prefill:
            return ceil_div(num_tokens, self.block_size) <= len(self.free)
        assert len(table) > 0
        if num_tokens % self.block_size != 0:
            return True
        return len(self.free) > 0

    def allocate(self, rid: int, num_tokens: int, is_prefill: bool) -> None:
        """:43-60: prefill fills the table to ceil(n / bs) blocks; decode adds
        one block when n is a multiple of the block size."""
        table = self.block_table(rid)
        if is_prefill:
            needed = ceil_div(num_tokens, self.block_size)
            while len(table) < needed:
                b = self.free.popleft()
                self.ref[b] += 1
                table.append(b)
            return
        assert len(table) > 0
        if num_tokens % self.block_size == 0:
            b = self.free.popleft()
            self.ref[b] += 1
            table.append(b)

    def deallocate(self, rid: int) -> None:
        """:62-70: blocks whose count drops to 0 return to the back of the queue."""
        table = self.block_table(rid)
        for b in table:
            self.ref[b] -= 1
            if self.ref[b] == 0:
                self.free.append(b)
        table.clear()
