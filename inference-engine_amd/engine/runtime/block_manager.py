"""KV block bookkeeping on the host: the producer of the block tables the HIP kernels read,
with copy-on-write.

Layout contract (the reference's, engine/runtime/block_manager.py:1-14, :171-174): a
sequence's table lists the physical blocks that hold its tokens in order, and token
``p`` lives in slot ``table[p // block_size] * block_size + p % block_size``.

Sharing. Blocks carry reference counts. ``fork`` gives a new sequence the leading blocks
of an existing one (a whole sequence for beam-style forks, or the full blocks of a
common prompt prefix) without copying any K/V. A block that more than one table holds
must not be written in place: ``prepare_write`` first swaps a private copy into the
writer's table and returns the (src, dst) pairs that ``PagedKVCache.copy_blocks`` (HIP)
must copy, every layer, K and V, before the step's append. The reference shares only
full prompt blocks it never writes again, so it has no copy-on-write
(block_manager.py:130-150); its content-hash prefix cache (lookup, LRU eviction) is
scheduling policy and is not part of this build.

Free blocks are a LIFO stack: the most recently released block is reused first.
``check_no_leaks`` recounts every table against the reference counts and the stack.
"""

from __future__ import annotations

import numpy as np


class OutOfBlocks(RuntimeError):
    """No free KV block; callers check ``can_grow`` / ``can_write`` first."""


class BlockPool:
    """Reference counts of ``num_blocks`` physical blocks and a stack of the free ones."""

    def __init__(self, num_blocks: int) -> None:
        if num_blocks < 1:
            raise ValueError("num_blocks must be >= 1")
        self.num_blocks = num_blocks
        self.refs = np.zeros(num_blocks, dtype=np.int32)
        self._stack = list(range(num_blocks - 1, -1, -1))  # block 0 is taken first

    @property
    def num_free(self) -> int:
        return len(self._stack)

    def refcount(self, block: int) -> int:
        return int(self.refs[block])

    def take(self) -> int:
        """A free block, now owned once."""
        if not self._stack:
            raise OutOfBlocks("no free KV blocks")
        block = self._stack.pop()
        self.refs[block] = 1
        return block

    def share(self, block: int) -> None:
        """One more owner of an owned block."""
        if self.refs[block] < 1:
            raise ValueError(f"block {block} is free; only owned blocks can be shared")
        self.refs[block] += 1

    def release(self, block: int) -> None:
        """One owner fewer; the last one returns the block to the stack."""
        if self.refs[block] < 1:
            raise ValueError(f"block {block} released while free")
        self.refs[block] -= 1
        if self.refs[block] == 0:
            self._stack.append(block)

    def free_blocks(self) -> list[int]:
        return list(self._stack)


class BlockManager:
    """Per-sequence block tables over a ``BlockPool``."""

    def __init__(self, num_blocks: int, block_size: int = 16) -> None:
        if block_size < 1:
            raise ValueError("block_size must be >= 1")
        self.block_size = block_size
        self.pool = BlockPool(num_blocks)
        self.tables: dict[int, list[int]] = {}
        self.copies_total = 0  # copy-on-write pairs handed out

    @property
    def num_free_blocks(self) -> int:
        return self.pool.num_free

    def _blocks_for(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def blocks_needed(self, seq_id: int, num_tokens: int) -> int:
        """Blocks ``seq_id`` must add to hold ``num_tokens`` tokens in all."""
        return max(self._blocks_for(num_tokens) - len(self.tables.get(seq_id, ())), 0)

    def can_grow(self, seq_id: int, num_tokens: int) -> bool:
        return self.blocks_needed(seq_id, num_tokens) <= self.pool.num_free

    def grow(self, seq_id: int, num_tokens: int) -> list[int]:
        """Room for ``num_tokens`` tokens in ``seq_id`` (new blocks at the end); returns
        its table."""
        need = self.blocks_needed(seq_id, num_tokens)
        if need > self.pool.num_free:
            raise OutOfBlocks(f"sequence {seq_id} needs {need} more blocks, "
                              f"{self.pool.num_free} free")  # fmt: skip
        table = self.tables.setdefault(seq_id, [])
        table.extend(self.pool.take() for _ in range(need))
        return table

    def fork(self, parent_id: int, child_id: int, num_tokens: int | None = None) -> list[int]:
        """``child_id`` starts with the blocks that hold the parent's first
        ``num_tokens`` tokens (all of its blocks if None, a partly filled last one
        included); each gains an owner and nothing is copied. Returns the child's
        table."""
        if child_id in self.tables:
            raise ValueError(f"sequence {child_id} already has blocks")
        parent = self.tables[parent_id]
        n = len(parent) if num_tokens is None else self._blocks_for(num_tokens)
        if n > len(parent):
            raise ValueError(f"sequence {parent_id} holds {len(parent)} blocks, not {n}")
        for block in parent[:n]:
            self.pool.share(block)
        self.tables[child_id] = list(parent[:n])
        return self.tables[child_id]

    def shared_blocks(self, seq_id: int, start: int, end: int) -> list[int]:
        """Table indices of ``seq_id``'s blocks that tokens [start, end) would write and
        that another table also holds."""
        table = self.tables.get(seq_id, [])
        hi = min(self._blocks_for(end), len(table))
        return [i for i in range(start // self.block_size, hi) if self.pool.refs[table[i]] > 1]

    def can_write(self, seq_id: int, start: int, end: int) -> bool:
        """Enough free blocks to grow to ``end`` tokens and copy every shared block."""
        need = self.blocks_needed(seq_id, end) + len(self.shared_blocks(seq_id, start, end))
        return need <= self.pool.num_free

    def prepare_write(self, seq_id: int, start: int, end: int) -> list[tuple[int, int]]:
        """Make tokens [start, end) of ``seq_id`` writable: each shared block in that
        range is replaced in this table by a fresh block (the others keep the original),
        and the table grows to ``end`` tokens. Returns the (src, dst) block pairs whose
        K/V must be copied before the write."""
        if not self.can_write(seq_id, start, end):
            raise OutOfBlocks(f"sequence {seq_id} cannot write tokens [{start}, {end})")
        table = self.tables.setdefault(seq_id, [])
        pairs = []
        for i in self.shared_blocks(seq_id, start, end):
            fresh = self.pool.take()
            self.pool.release(table[i])
            pairs.append((table[i], fresh))
            table[i] = fresh
        self.grow(seq_id, end)
        self.copies_total += len(pairs)
        return pairs

    def free(self, seq_id: int) -> None:
        for block in self.tables.pop(seq_id, ()):
            self.pool.release(block)

    def slot(self, seq_id: int, position: int) -> int:
        """Flat pool slot of token ``position`` of ``seq_id``."""
        bs = self.block_size
        return self.tables[seq_id][position // bs] * bs + position % bs

    def check_no_leaks(self) -> None:
        """Every block is either on the free stack once (refcount 0) or held by exactly
        as many table entries as its refcount says."""
        pool = self.pool
        held = np.zeros(pool.num_blocks, dtype=np.int64)
        for table in self.tables.values():
            np.add.at(held, np.asarray(table, dtype=np.int64), 1)
        bad = np.nonzero(held != pool.refs)[0]
        if bad.size:
            b = int(bad[0])
            raise AssertionError(f"block {b}: refcount {pool.refcount(b)}, held {held[b]} times")
        free = pool.free_blocks()
        if len(set(free)) != len(free):
            raise AssertionError("a block is on the free stack twice")
        if sorted(free) != np.nonzero(pool.refs == 0)[0].tolist():
            raise AssertionError("the free stack and the zero refcounts disagree")
