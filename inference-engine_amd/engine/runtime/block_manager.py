"""KV block bookkeeping on the host: the producer of the block tables the HIP kernels
read. Same layout, invariants and public names as the reference's
``engine/runtime/block_manager.py`` (``BlockAllocator`` :26-84, ``chain_hash`` :87-88,
``BlockManager`` :91-191), plus copy-on-write, which the reference lacks.

A sequence's block table lists the physical blocks holding its tokens, in order; token
``p`` lives in slot ``table[p // block_size] * block_size + p % block_size``.

Prefix caching: a full block is keyed by a hash of its tokens chained with the key of
the block before it, so equal keys mean equal prefixes. Registered blocks are shared
(reference-counted) by later sequences that start with the same tokens; when the last
owner lets go, such a block stays findable but reclaimable, least recently used first.

Copy-on-write (this build's addition): ``fork`` lets a child sequence share every block
of its parent, including the partly filled last one. Before a step writes tokens into a
block that more than one sequence holds, ``prepare_write`` gives the writer a private
copy: it allocates a fresh block, swaps it into the writer's table and returns the
(src, dst) pair for ``copy_blocks`` (HIP), which must run before the step's K/V append.
The reference never needs this because it shares only full blocks and always leaves the
last prompt token to compute (reference block_manager.py:130-150).
"""

from __future__ import annotations

from collections import OrderedDict, deque
from collections.abc import Sequence


class OutOfBlocks(RuntimeError):
    """No free KV block; callers check ``can_grow`` / ``can_write`` first."""


class BlockAllocator:
    """Reference counts over ``num_blocks`` blocks, a FIFO of free blocks and an LRU of
    evictable ones (refcount 0 but still registered under a content hash)."""

    def __init__(self, num_blocks: int) -> None:
        if num_blocks < 1:
            raise ValueError("num_blocks must be >= 1")
        self.num_blocks = num_blocks
        self._refs = [0] * num_blocks
        self._free: deque[int] = deque(range(num_blocks))
        self._evictable: OrderedDict[int, None] = OrderedDict()
        self.block_hash: dict[int, int] = {}  # registered block -> content key
        self.cached: dict[int, int] = {}  # content key -> registered block

    @property
    def num_free(self) -> int:
        """Blocks an ``allocate`` can hand out: free ones plus evictable ones."""
        return len(self._free) + len(self._evictable)

    def refcount(self, block: int) -> int:
        return self._refs[block]

    def allocate(self) -> int:
        if self._free:
            block = self._free.popleft()
        elif self._evictable:
            block = next(iter(self._evictable))  # least recently released
            del self._evictable[block]
            del self.cached[self.block_hash.pop(block)]
        else:
            raise OutOfBlocks("no free KV blocks")
        self._refs[block] = 1
        return block

    def acquire_cached(self, block: int) -> None:
        """One more owner for a registered block (revived if it was evictable)."""
        if self._refs[block] == 0:
            del self._evictable[block]
        self._refs[block] += 1

    def incref(self, block: int) -> None:
        if self._refs[block] == 0:
            raise ValueError(f"block {block} is not owned; cannot share it")
        self._refs[block] += 1

    def free(self, block: int) -> None:
        if self._refs[block] == 0:
            raise ValueError(f"double free of block {block}")
        self._refs[block] -= 1
        if self._refs[block]:
            return
        if block in self.block_hash:
            self._evictable[block] = None  # most recently released at the end
        else:
            self._free.append(block)

    def register(self, block: int, key: int) -> None:
        """Make a full, owned block findable by its content key (first one wins)."""
        if key not in self.cached and block not in self.block_hash:
            self.cached[key] = block
            self.block_hash[block] = key


def chain_hash(parent: int | None, tokens: Sequence[int]) -> int:
    """Content key of a full block: its tokens chained with the previous block's key."""
    return hash((parent, tuple(tokens)))


class BlockManager:
    """Per-sequence block tables over a ``BlockAllocator``."""

    def __init__(self, num_blocks: int, block_size: int = 16,
                 enable_prefix_caching: bool = True) -> None:  # fmt: skip
        self.block_size = block_size
        self.enable_prefix_caching = enable_prefix_caching
        self.allocator = BlockAllocator(num_blocks)
        self.tables: dict[int, list[int]] = {}
        # Per sequence: leading blocks registered so far and the last one's key.
        self._registered: dict[int, tuple[int, int | None]] = {}
        self.copies_total = 0

    @property
    def num_free_blocks(self) -> int:
        return self.allocator.num_free

    @property
    def num_cached_blocks(self) -> int:
        return len(self.allocator.cached)

    def blocks_needed(self, seq_id: int, num_tokens: int) -> int:
        """Blocks ``seq_id`` must add to hold ``num_tokens`` tokens in all."""
        have = len(self.tables.get(seq_id, ()))
        return max(-(-num_tokens // self.block_size) - have, 0)

    def can_grow(self, seq_id: int, num_tokens: int) -> bool:
        return self.blocks_needed(seq_id, num_tokens) <= self.allocator.num_free

    def grow(self, seq_id: int, num_tokens: int) -> list[int]:
        """Room for ``num_tokens`` tokens in ``seq_id``; returns its block table."""
        need = self.blocks_needed(seq_id, num_tokens)
        if need > self.allocator.num_free:
            raise OutOfBlocks(f"sequence {seq_id} needs {need} more blocks")
        table = self.tables.setdefault(seq_id, [])
        for _ in range(need):
            table.append(self.allocator.allocate())
        return table

    def match_prefix(self, seq_id: int, token_ids: Sequence[int]) -> int:
        """Attach registered blocks that match the start of a new sequence's tokens;
        returns how many tokens now have K/V in place. The last token is never matched:
        its logits are needed."""
        if not self.enable_prefix_caching or seq_id in self.tables:
            return 0
        bs = self.block_size
        table: list[int] = []
        key = None
        for start in range(0, len(token_ids) - bs, bs):
            nxt = chain_hash(key, token_ids[start : start + bs])
            block = self.allocator.cached.get(nxt)
            if block is None:
                break
            self.allocator.acquire_cached(block)
            table.append(block)
            key = nxt
        if table:
            self.tables[seq_id] = table
            self._registered[seq_id] = (len(table), key)
        return len(table) * bs

    def register_full_blocks(self, seq_id: int, token_ids: Sequence[int],
                             num_computed: int) -> None:  # fmt: skip
        """Register each block of ``seq_id`` that is now full of computed tokens."""
        if not self.enable_prefix_caching:
            return
        done, key = self._registered.get(seq_id, (0, None))
        table, bs = self.tables[seq_id], self.block_size
        full = min(num_computed // bs, len(table))
        for i in range(done, full):
            key = chain_hash(key, token_ids[i * bs : (i + 1) * bs])
            self.allocator.register(table[i], key)
        self._registered[seq_id] = (max(done, full), key)

    def fork(self, parent_id: int, child_id: int) -> list[int]:
        """The child shares every block of the parent (each gains an owner), the partly
        filled last one included; returns the child's table."""
        if child_id in self.tables:
            raise ValueError(f"sequence {child_id} already has blocks")
        table = list(self.tables[parent_id])
        for block in table:
            self.allocator.incref(block)
        self.tables[child_id] = table
        if parent_id in self._registered:
            self._registered[child_id] = self._registered[parent_id]
        return table

    def shared_blocks(self, seq_id: int, start: int, end: int) -> list[int]:
        """Indices into ``seq_id``'s table of blocks that tokens [start, end) would write
        and that another sequence also holds."""
        table, bs = self.tables.get(seq_id, []), self.block_size
        last = min(-(-end // bs), len(table))
        return [i for i in range(start // bs, last)
                if self.allocator.refcount(table[i]) > 1]  # fmt: skip

    def can_write(self, seq_id: int, start: int, end: int) -> bool:
        """Enough free blocks to grow to ``end`` tokens and copy every shared block."""
        need = self.blocks_needed(seq_id, end) + len(self.shared_blocks(seq_id, start, end))
        return need <= self.allocator.num_free

    def prepare_write(self, seq_id: int, start: int, end: int) -> list[tuple[int, int]]:
        """Make tokens [start, end) of ``seq_id`` writable: grow the table to ``end``
        tokens and replace every shared block in the range by a private copy. Returns the
        (src, dst) block pairs to copy, K and V of every layer, before the write."""
        if not self.can_write(seq_id, start, end):
            raise OutOfBlocks(f"sequence {seq_id} cannot write tokens [{start}, {end})")
        shared = self.shared_blocks(seq_id, start, end)
        done = self._registered.get(seq_id, (0, None))[0]
        if shared and shared[0] < done:
            raise ValueError(f"sequence {seq_id}: tokens [{start}, {end}) would rewrite "
                             f"registered block {shared[0]}")  # fmt: skip
        pairs = []
        table = self.tables.setdefault(seq_id, [])
        for i in shared:
            src = table[i]
            dst = self.allocator.allocate()
            self.allocator.free(src)  # drops this sequence's share; others keep it
            table[i] = dst
            pairs.append((src, dst))
        self.grow(seq_id, end)
        self.copies_total += len(pairs)
        return pairs

    def free(self, seq_id: int) -> None:
        self._registered.pop(seq_id, None)
        for block in self.tables.pop(seq_id, ()):
            self.allocator.free(block)

    def slot(self, seq_id: int, position: int) -> int:
        """Flat pool slot of token ``position`` of ``seq_id`` (reference :171-174)."""
        table, bs = self.tables[seq_id], self.block_size
        return table[position // bs] * bs + position % bs

    def check_no_leaks(self) -> None:
        """Allocator invariants against the live tables (reference :176-191)."""
        a = self.allocator
        owners: dict[int, int] = {}
        for table in self.tables.values():
            for block in table:
                owners[block] = owners.get(block, 0) + 1
        free, evictable = set(a._free), set(a._evictable)
        assert len(free) == len(a._free), "a block is listed twice as free"
        assert not free & evictable, "a block is both free and evictable"
        assert not (free | evictable) & owners.keys(), "a block is both free and owned"
        assert len(free) + len(evictable) + len(owners) == a.num_blocks, "blocks leaked"
        for block, n in owners.items():
            assert a.refcount(block) == n, f"block {block}: {a.refcount(block)} refs, {n} owners"
        assert all(b in a.block_hash for b in evictable), "evictable block without a key"
        assert all(a.cached[k] == b for b, k in a.block_hash.items()), "key maps disagree"
