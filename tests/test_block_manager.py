"""Block manager (host): the producer of the block tables the kernels read. The slot
formula is the reference's (tests/test_block_manager.py:38-46 of the reference); sharing
by fork and copy-on-write are this build's."""

from __future__ import annotations

import random

import pytest

from engine.runtime.block_manager import BlockManager, BlockPool, OutOfBlocks


def test_slot_formula_and_growth():
    """slot = table[p // bs] * bs + p % bs; growth adds blocks only when needed."""
    bm = BlockManager(num_blocks=10, block_size=4)
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


def test_out_of_blocks_and_double_release():
    bm = BlockManager(num_blocks=2, block_size=4)
    assert not bm.can_grow(1, 9)
    with pytest.raises(OutOfBlocks):
        bm.grow(1, 9)
    assert bm.tables.get(1, []) == []  # nothing half-allocated
    pool = BlockPool(1)
    b = pool.take()
    pool.release(b)
    with pytest.raises(ValueError):
        pool.release(b)
    with pytest.raises(ValueError):
        pool.share(b)
    pool.take()
    with pytest.raises(OutOfBlocks):
        pool.take()


def test_lifo_reuse():
    pool = BlockPool(4)
    a, b = pool.take(), pool.take()
    assert (a, b) == (0, 1)
    pool.release(a)
    assert pool.take() == a  # the most recently released block comes back first


def test_fork_shares_then_copy_on_write():
    bm = BlockManager(num_blocks=8, block_size=4)
    bm.grow(1, 10)  # blocks for tokens 0..9: the last one partly filled
    parent = list(bm.tables[1])
    child = bm.fork(1, 2)
    assert child == parent and all(bm.pool.refcount(b) == 2 for b in parent)
    bm.check_no_leaks()
    # The child appends token 10: block 2 is shared, so it gets a private copy.
    assert bm.shared_blocks(2, 10, 11) == [2]
    pairs = bm.prepare_write(2, 10, 11)
    assert pairs == [(parent[2], bm.tables[2][2])] and bm.tables[2][2] != parent[2]
    assert bm.tables[2][:2] == parent[:2] and bm.tables[1] == parent
    assert bm.pool.refcount(parent[2]) == 1 and bm.pool.refcount(bm.tables[2][2]) == 1
    # Now the parent's block 2 is private again: no copy for its own append.
    assert bm.prepare_write(1, 10, 11) == []
    bm.check_no_leaks()
    bm.free(1)
    bm.free(2)
    bm.check_no_leaks()
    assert bm.num_free_blocks == 8 and bm.copies_total == 1


def test_fork_of_a_prefix_and_growth_past_it():
    """Sharing the full blocks of a common prompt prefix: new tokens go to new blocks,
    no copy is needed."""
    bm = BlockManager(num_blocks=16, block_size=4)
    bm.grow(1, 14)
    shared = bm.fork(1, 2, num_tokens=8)
    assert shared == bm.tables[1][:2]
    assert bm.prepare_write(2, 8, 13) == []  # tokens 8..12: fresh blocks 2..3
    assert len(bm.tables[2]) == 4 and bm.tables[2][2:] != bm.tables[1][2:4]
    with pytest.raises(ValueError):
        bm.fork(1, 2)  # the child exists
    with pytest.raises(ValueError):
        bm.fork(1, 3, num_tokens=17)  # more than the parent holds
    bm.check_no_leaks()


def test_copy_on_write_needs_a_free_block():
    bm = BlockManager(num_blocks=2, block_size=4)
    bm.grow(1, 3)
    bm.fork(1, 2)
    bm.grow(3, 4)  # the last free block
    assert not bm.can_write(2, 3, 4)
    with pytest.raises(OutOfBlocks):
        bm.prepare_write(2, 3, 4)
    bm.check_no_leaks()


def test_leak_check_catches_corruption():
    bm = BlockManager(num_blocks=4, block_size=4)
    bm.grow(1, 8)
    bm.pool.refs[bm.tables[1][0]] = 2  # a missing owner
    with pytest.raises(AssertionError):
        bm.check_no_leaks()
    bm = BlockManager(num_blocks=4, block_size=4)
    bm.grow(1, 4)
    bm.pool._stack.append(bm.pool._stack[0])  # listed free twice
    with pytest.raises(AssertionError):
        bm.check_no_leaks()


def test_random_workload_keeps_invariants():
    """Random grow / fork / write / free sequences: the invariants hold after every
    operation, and every copy pair moves a block that was shared to a private one."""
    rnd = random.Random(0)
    bm = BlockManager(num_blocks=40, block_size=4)
    lengths: dict[int, int] = {}
    next_id = 0
    for _ in range(2000):
        op = rnd.random()
        live = list(lengths)
        if op < 0.3 or not live:
            n = rnd.randint(1, 12)
            if bm.can_grow(next_id, n):
                bm.grow(next_id, n)
                lengths[next_id] = n
                next_id += 1
        elif op < 0.45:
            parent = rnd.choice(live)
            keep = rnd.randint(1, lengths[parent])
            bm.fork(parent, next_id, num_tokens=keep)
            lengths[next_id] = keep
            next_id += 1
        elif op < 0.85:
            s = rnd.choice(live)
            start, end = lengths[s], lengths[s] + rnd.randint(1, 6)
            if bm.can_write(s, start, end):
                before = list(bm.tables[s])
                for src, dst in bm.prepare_write(s, start, end):
                    assert src in before and dst not in before
                    assert bm.pool.refcount(dst) == 1
                lengths[s] = end
        else:
            s = rnd.choice(live)
            bm.free(s)
            del lengths[s]
        bm.check_no_leaks()
        for s, n in lengths.items():
            assert len(bm.tables[s]) == -(-n // 4)
    for s in list(lengths):
        bm.free(s)
    bm.check_no_leaks()
    assert bm.num_free_blocks == 40
