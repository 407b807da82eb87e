"""Block manager (host): the producer of the block tables the kernels read. Invariants
follow the reference's tests/test_block_manager.py; fork and copy-on-write are this
build's additions."""

from __future__ import annotations

import random

import pytest

from engine.runtime.block_manager import BlockAllocator, BlockManager, OutOfBlocks, chain_hash


def test_slot_formula_and_growth():
    """Reference tests/test_block_manager.py:38-46: slot = table[p // bs] * bs + p % bs."""
    bm = BlockManager(num_blocks=10, block_size=4, enable_prefix_caching=False)
    table = bm.grow(1, 6)
    assert len(table) == 2 and bm.num_free_blocks == 8
    for p in range(6):
        assert bm.slot(1, p) == table[p // 4] * 4 + p % 4
    assert bm.grow(1, 8) == table and bm.num_free_blocks == 8  # still fits
    bm.grow(1, 9)
    assert len(bm.tables[1]) == 3
    bm.check_no_leaks()
    bm.free(1)
    assert bm.num_free_blocks == 10
    bm.check_no_leaks()


def test_out_of_blocks_and_double_free():
    bm = BlockManager(num_blocks=2, block_size=4, enable_prefix_caching=False)
    assert not bm.can_grow(1, 9)
    with pytest.raises(OutOfBlocks):
        bm.grow(1, 9)
    a = BlockAllocator(1)
    b = a.allocate()
    a.free(b)
    with pytest.raises(ValueError):
        a.free(b)
    with pytest.raises(ValueError):
        a.incref(b)


def test_prefix_cache_shares_full_blocks_and_evicts_lru():
    bm = BlockManager(num_blocks=8, block_size=4)
    toks = list(range(100, 111))  # 11 tokens: two full blocks + 3
    bm.grow(1, len(toks))
    bm.register_full_blocks(1, toks, len(toks))
    assert bm.num_cached_blocks == 2
    # Same first 9 tokens: both full blocks match (the last token is never matched).
    assert bm.match_prefix(2, toks[:9]) == 8
    assert bm.tables[2] == bm.tables[1][:2]
    assert bm.allocator.refcount(bm.tables[1][0]) == 2
    # Exactly 8 tokens: only the first block (the 8th token must be computed).
    assert bm.match_prefix(3, toks[:8]) == 4
    bm.check_no_leaks()
    for s in (1, 2, 3):
        bm.free(s)
    bm.check_no_leaks()
    assert bm.num_free_blocks == 8 and bm.num_cached_blocks == 2
    # Evictable blocks are reused least recently released first, and leave the cache.
    first_cached = set(bm.allocator.cached.values())
    taken = bm.grow(4, 8 * 4)
    assert set(taken[-2:]) == first_cached and bm.num_cached_blocks == 0
    bm.check_no_leaks()


def test_chain_hash_depends_on_prefix():
    assert chain_hash(None, [1, 2]) == chain_hash(None, [1, 2])
    assert chain_hash(None, [1, 2]) != chain_hash(chain_hash(None, [0]), [1, 2])


def test_fork_then_copy_on_write():
    bm = BlockManager(num_blocks=8, block_size=4)
    bm.grow(1, 6)  # blocks A (full) and B (2 of 4 used)
    a, b = bm.tables[1]
    bm.fork(1, 2)
    assert bm.tables[2] == [a, b] and bm.allocator.refcount(b) == 2
    bm.check_no_leaks()
    # Child writes token 6 into shared block B: it gets a private copy.
    pairs = bm.prepare_write(2, 6, 7)
    assert len(pairs) == 1 and pairs[0][0] == b
    c = pairs[0][1]
    assert bm.tables[2] == [a, c] and bm.tables[1] == [a, b]
    assert bm.allocator.refcount(b) == 1 and bm.allocator.refcount(a) == 2
    # The parent now owns B alone: it writes in place.
    assert bm.prepare_write(1, 6, 7) == []
    # Writing past a block boundary grows the table; the full shared block A is never
    # written, so it stays shared.
    assert bm.prepare_write(2, 7, 10) == [] and len(bm.tables[2]) == 3
    assert bm.allocator.refcount(a) == 2
    bm.check_no_leaks()
    bm.free(1)
    bm.free(2)
    bm.check_no_leaks()
    assert bm.num_free_blocks == 8


def test_copy_on_write_needs_a_free_block():
    bm = BlockManager(num_blocks=2, block_size=4, enable_prefix_caching=False)
    bm.grow(1, 6)
    bm.fork(1, 2)
    assert not bm.can_write(2, 6, 7)
    with pytest.raises(OutOfBlocks):
        bm.prepare_write(2, 6, 7)
    bm.check_no_leaks()


def test_random_workload_keeps_invariants():
    """Random grow / fork / write / free sequences never break the invariants."""
    rng = random.Random(0)
    bm = BlockManager(num_blocks=40, block_size=4)
    lens: dict[int, int] = {}
    nxt = 0
    for _ in range(2000):
        op = rng.random()
        if op < 0.3 or not lens:
            n = rng.randint(1, 20)
            if bm.can_grow(nxt, n):
                bm.grow(nxt, n)
                lens[nxt] = n
                nxt += 1
        elif op < 0.45:
            parent = rng.choice(list(lens))
            bm.fork(parent, nxt)
            lens[nxt] = lens[parent]
            nxt += 1
        elif op < 0.8:
            s = rng.choice(list(lens))
            n = rng.randint(1, 5)
            if bm.can_write(s, lens[s], lens[s] + n):
                for src, dst in bm.prepare_write(s, lens[s], lens[s] + n):
                    assert src != dst and bm.allocator.refcount(dst) == 1
                lens[s] += n
                # every block the writer touches is now its own
                assert bm.shared_blocks(s, lens[s] - n, lens[s]) == []
        else:
            s = rng.choice(list(lens))
            bm.free(s)
            del lens[s]
        bm.check_no_leaks()
