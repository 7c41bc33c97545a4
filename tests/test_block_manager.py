"""The native KV block manager against the restated reference manager, and
its prefix-caching and copy-on-write additions (host only, no device)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import PKG
from oracle.kv_cache_manager_oracle import BlockManagerOracle

KVCacheManager = __import__("vllm_jax_amd.kv_cache_manager", fromlist=["KVCacheManager"]).KVCacheManager


class Req:
    """The parts of vllm/src/request.py the manager reads."""
    _next = 10_000

    def __init__(self, token_ids, rid=None):
        self.token_ids = list(token_ids)
        if rid is None:
            Req._next += 1
            rid = Req._next
        self.id = rid

    def __len__(self):
        return len(self.token_ids)


# ---------------------------------------------------------------------------
# the oracle, pinned by hand-worked traces of kv_cache_manager.py
# ---------------------------------------------------------------------------
def test_oracle_hand_trace():
    m = BlockManagerOracle(8, 4)
    assert m.can_allocate(0, 10, True)
    m.allocate(0, 10, True)                  # ceil(10/4) = 3 blocks, FIFO
    assert m.block_table(0) == [0, 1, 2]
    m.allocate(1, 5, True)
    assert m.block_table(1) == [3, 4]
    m.allocate(0, 11, False)                 # 11 % 4 != 0: nothing
    m.allocate(0, 12, False)                 # 12 % 4 == 0: one block ahead
    assert m.block_table(0) == [0, 1, 2, 5]
    m.deallocate(0)                          # back of the queue, table order
    assert list(m.free) == [6, 7, 0, 1, 2, 5]
    assert not m.can_allocate(2, 25, True)   # 7 blocks > 6 free
    assert m.can_allocate(1, 7, False)
    m.allocate(2, 24, True)
    assert m.block_table(2) == [6, 7, 0, 1, 2, 5]
    assert not m.can_allocate(1, 8, False)   # a new block is due and none is free
    assert m.ref[0] == 1 and m.ref[3] == 1


# ---------------------------------------------------------------------------
# native manager == oracle (prefix caching off)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("seed,num_blocks,bs", [(0, 64, 16), (1, 40, 4), (2, 300, 256), (3, 17, 1)])
def test_matches_reference_on_random_traces(seed, num_blocks, bs):
    rng = np.random.default_rng(seed)
    ora = BlockManagerOracle(num_blocks, bs)
    nat = KVCacheManager(num_blocks, bs)
    live = {}  # rid -> token count
    for step in range(600):
        op = rng.integers(0, 10)
        if op < 3 or not live:
            rid = int(rng.integers(0, 1 << 40))
            n = int(rng.integers(1, 6 * bs + 2))
            r = Req(range(n), rid)
            a = ora.can_allocate(rid, n, True)
            assert nat.can_allocate(r, True) == a
            if a:
                ora.allocate(rid, n, True)
                nat.allocate_slots(r, True)
                live[rid] = n
        elif op < 8:
            rid = list(live)[int(rng.integers(0, len(live)))]
            n = live[rid] + 1
            r = Req(range(n), rid)
            a = ora.can_allocate(rid, n, False)
            assert nat.can_allocate(r, False) == a
            if a:
                ora.allocate(rid, n, False)
                nat.allocate_slots(r, False)
                live[rid] = n
        else:
            rid = list(live)[int(rng.integers(0, len(live)))]
            ora.deallocate(rid)
            nat.deallocate(Req([], rid))
            del live[rid]
        assert nat.num_free_blocks == len(ora.free)
        for rid in live:
            assert nat.block_ids(Req([], rid)) == ora.block_table(rid)
    for b in range(num_blocks):
        assert nat.ref_count(b) == ora.ref[b]


def test_allocation_failure_raises_index_error():
    nat = KVCacheManager(2, 4)
    with pytest.raises(IndexError):
        nat.allocate_slots(Req(range(9)), True)
    with pytest.raises(AssertionError):
        nat.can_allocate(Req(range(3)), False)   # decode without blocks (kv_cache_manager.py:38)


# ---------------------------------------------------------------------------
# prefix caching
# ---------------------------------------------------------------------------
def test_prefix_blocks_are_shared_and_counted():
    bs = 16
    m = KVCacheManager(32, bs, enable_prefix_caching=True)
    shared = list(range(1000, 1000 + 40))                  # 2.5 blocks of common prefix
    a = Req(shared + [1, 2, 3, 4, 5])                      # 45 tokens
    b = Req(shared + [7, 8, 9])                            # 43 tokens
    m.allocate_slots(a, True)
    assert m.num_cached_tokens(a) == 0
    ta = m.block_ids(a)
    assert m.can_allocate(b, True)
    free_before = m.num_free_blocks
    m.allocate_slots(b, True)
    tb = m.block_ids(b)
    assert tb[:2] == ta[:2] and tb[2] != ta[2]             # the partial third block is private
    assert m.num_cached_tokens(b) == 2 * bs
    assert free_before - m.num_free_blocks == 1
    assert [m.ref_count(x) for x in tb] == [2, 2, 1]
    # a prompt equal to a's first two blocks: only blocks before its last token are reused
    c = Req(shared[:32])
    m.allocate_slots(c, True)
    assert m.block_ids(c)[0] == ta[0] and m.block_ids(c)[1] != ta[1]
    assert m.num_cached_tokens(c) == bs


def test_same_tokens_after_a_different_block_do_not_match():
    bs = 8
    m = KVCacheManager(16, bs, enable_prefix_caching=True)
    x = list(range(8))
    a = Req([99] * 8 + x + [1])
    b = Req([98] * 8 + x + [1])                            # block 1 tokens equal, predecessor differs
    m.allocate_slots(a, True)
    m.allocate_slots(b, True)
    assert not set(m.block_ids(a)) & set(m.block_ids(b))
    assert m.num_cached_tokens(b) == 0


def test_freed_cached_blocks_are_reused_until_evicted():
    bs = 4
    m = KVCacheManager(6, bs, enable_prefix_caching=True)
    p = list(range(50, 59))                                # 9 tokens: blocks 0,1 full, 2 partial
    a = Req(p)
    m.allocate_slots(a, True)
    ta = m.block_ids(a)
    m.deallocate(a)
    assert m.num_free_blocks == 6
    b = Req(p)
    assert m.can_allocate(b, True)
    m.allocate_slots(b, True)
    assert m.block_ids(b)[:2] == ta[:2] and m.num_cached_tokens(b) == 8
    m.deallocate(b)
    # fill the pool with unrelated prompts: the cached blocks are handed out again
    fill = Req(range(1000, 1000 + 24))
    m.allocate_slots(fill, True)
    m.deallocate(fill)
    c = Req(p)
    m.allocate_slots(c, True)
    assert m.num_cached_tokens(c) == 0


def test_can_allocate_counts_free_cached_hits():
    bs = 4
    m = KVCacheManager(4, bs, enable_prefix_caching=True)
    p = list(range(13))                                    # 4 blocks, 3 before the last token
    a = Req(p)
    m.allocate_slots(a, True)
    m.deallocate(a)                                        # all 4 free, 3 of them cached
    b = Req(p)
    assert m.can_allocate(b, True)                         # 3 hits (free) + 1 new = 4 free blocks
    m.allocate_slots(b, True)
    assert m.num_free_blocks == 0 and m.num_cached_tokens(b) == 12


# ---------------------------------------------------------------------------
# fork + copy-on-write
# ---------------------------------------------------------------------------
def test_fork_then_decode_copies_the_shared_tail():
    bs = 16
    m = KVCacheManager(10, bs)
    parent = Req(range(20))                                # blocks [0, 1], tail block 1 partial
    m.allocate_slots(parent, True)
    child = Req(range(20))
    m.fork(parent, child)
    assert m.block_ids(child) == [0, 1] and m.ref_count(1) == 2
    child.token_ids.append(7)                              # child writes position 20 (block 1)
    assert m.can_allocate(child, False)
    m.allocate_slots(child, False)
    assert m.block_ids(child) == [0, 2]
    assert m.take_block_copies() == ([1], [2])
    assert m.take_block_copies() == ([], [])
    assert [m.ref_count(b) for b in (0, 1, 2)] == [2, 1, 1]
    parent.token_ids.append(5)
    m.allocate_slots(parent, False)                        # block 1 is private again: no copy
    assert m.block_ids(parent) == [0, 1] and m.take_block_copies() == ([], [])
    m.deallocate(parent)
    m.deallocate(child)
    assert m.num_free_blocks == 10


def test_refused_prefill_after_prefix_hit_changes_nothing():
    # Sequence 2 would take two cached blocks and then needs more free blocks
    # than there are: the refusal must leave tables, reference counts and the
    # free queue as they were, and a later retry must find the prefix again.
    bs = 4
    m = KVCacheManager(5, bs, enable_prefix_caching=True)
    p = list(range(100, 109))                              # 9 tokens: 2 full blocks + 1 partial
    a = Req(p)
    m.allocate_slots(a, True)
    ta = m.block_ids(a)
    assert [m.ref_count(x) for x in range(5)] == [1, 1, 1, 0, 0] and m.num_free_blocks == 2
    big = Req(p[:8] + list(range(500, 509)))               # 17 tokens: 2 hits + 3 new > 2 free
    assert not m.can_allocate(big, True)
    with pytest.raises(IndexError):
        m.allocate_slots(big, True)
    assert m.block_ids(big) == [] and m.num_free_blocks == 2
    assert [m.ref_count(x) for x in range(5)] == [1, 1, 1, 0, 0]
    m.deallocate(a)
    assert m.num_free_blocks == 5 and [m.ref_count(x) for x in range(5)] == [0] * 5
    # the retry fits now and still finds the two cached blocks
    assert m.can_allocate(big, True)
    m.allocate_slots(big, True)
    assert m.block_ids(big)[:2] == ta[:2] and m.num_cached_tokens(big) == 8


def test_refused_decode_with_copy_on_write_changes_nothing():
    # A forked sequence whose next token both falls into a shared block and
    # opens a new one needs two free blocks; with one free the call must fail
    # before the copy-on-write moves anything.
    bs = 4
    m = KVCacheManager(3, bs)
    parent = Req(range(7))                                 # blocks [0, 1], block 1 holds 3 tokens
    m.allocate_slots(parent, True)
    child = Req(range(7))
    m.fork(parent, child)
    child.token_ids.append(1)                              # 8 tokens: writes block 1 (shared), 8 % 4 == 0
    assert not m.can_allocate(child, False)
    with pytest.raises(IndexError):
        m.allocate_slots(child, False)
    assert m.block_ids(child) == [0, 1] and m.take_block_copies() == ([], [])
    assert [m.ref_count(x) for x in range(3)] == [2, 2, 0] and m.num_free_blocks == 1
