"""Decode steps as hipGraph replays (reference engine/runtime/cuda_graphs.py:20-108,
``DecodeGraphs``): the whole forward pass of a decode step is captured once per
batch-size bucket and replayed, so hundreds of launches become one.

Graphs need fixed shapes and addresses, so every input lives in a static buffer sized
for the largest bucket; a step of B sequences copies its token ids, positions, block
tables and context lengths in, pads to the next bucket and replays. Padding rows have
context length 1 and a table of the scratch block (a block the allocator never hands
out), so they write and read only that block.

Differences from the reference: the slot mapping is not copied in -- the captured step
starts with the HIP slot builder (``decode_slots``), which derives every sequence's
new slot from the tables and lengths already on the device -- and the attention inside
is this build's HIP decode kernel, whose grid depends only on static shapes (context
lengths are read from device memory), so one graph serves every length.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch

from engine.runtime.paged_cache import PagedBatch, PagedKVCache, decode_slots

BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 192, 256)


class DecodeGraphs:
    """``model(input_ids [1, n], positions [1, n], batch: PagedBatch) -> logits
    [n, 1, vocab]`` captured per bucket n."""

    def __init__(self, model: Callable, cache: PagedKVCache, scratch_block: int,
                 max_batch: int, max_blocks_per_seq: int) -> None:  # fmt: skip
        self.model, self.cache = model, cache
        dev = cache.k.device
        self.sizes = [s for s in BUCKETS if s < max_batch] + [max_batch]
        b, w = self.sizes[-1], max_blocks_per_seq
        self.max_width = w
        self.scratch_block = scratch_block
        self.ids = torch.zeros(1, b, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, b, dtype=torch.long, device=dev)
        self.tables = torch.full((b, w), scratch_block, dtype=torch.int32, device=dev)
        self.ctx = torch.ones(b, dtype=torch.int32, device=dev)
        self.slots = torch.zeros(b, dtype=torch.int64, device=dev)  # written in-graph
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.outputs: dict[int, torch.Tensor] = {}
        self._batches: dict[int, PagedBatch] = {}
        self._capture()

    def _batch(self, n: int) -> PagedBatch:
        return PagedBatch(cache=self.cache, slot_mapping=self.slots[:n],
                          last_index=torch.arange(n, device=self.ids.device),
                          block_tables=self.tables[:n], context_lens=self.ctx[:n])  # fmt: skip

    def _step(self, n: int, batch: PagedBatch) -> torch.Tensor:
        decode_slots(self.tables[:n], self.ctx[:n], self.cache.block_size,
                     self.cache.k.shape[1], out=self.slots[:n])  # fmt: skip
        return self.model(self.ids[:, :n], self.pos[:, :n], batch)

    def _capture(self) -> None:
        pool = None
        for n in reversed(self.sizes):  # largest first: smaller graphs reuse its pool
            batch = self._batch(n)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):  # warm-up outside the capture
                    self._step(n, batch)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                out = self._step(n, batch)
            pool = graph.pool()
            # The graph reads the batch's tensors by address: keep them alive.
            self.graphs[n], self.outputs[n], self._batches[n] = graph, out, batch
        torch.cuda.synchronize()

    def can_run(self, batch_size: int, width: int) -> bool:
        return batch_size <= self.sizes[-1] and width <= self.max_width

    def run(self, ids: Sequence[int], positions: Sequence[int], slots: Sequence[int] | None,
            tables: Sequence[Sequence[int]], context_lens: Sequence[int]) -> torch.Tensor:  # fmt: skip
        """One decode step for len(ids) sequences -> logits [B, 1, vocab]. ``slots`` is
        accepted for the reference's call signature and not used: the captured step
        builds the slot mapping on the device."""
        del slots
        b = len(ids)
        n = next(s for s in self.sizes if s >= b)
        pad = n - b
        width = max(len(t) for t in tables)
        if width > self.max_width:
            raise ValueError(f"DecodeGraphs: table width {width} > {self.max_width}")
        rows = [list(t) + [self.scratch_block] * (width - len(t)) for t in tables]
        rows += [[self.scratch_block] * width] * pad
        self.ids[0, :n].copy_(torch.tensor(list(ids) + [0] * pad), non_blocking=True)
        self.pos[0, :n].copy_(torch.tensor(list(positions) + [0] * pad), non_blocking=True)
        self.ctx[:n].copy_(torch.tensor(list(context_lens) + [1] * pad, dtype=torch.int32))
        self.tables[:n, :width].copy_(torch.tensor(rows, dtype=torch.int32))
        self.graphs[n].replay()
        return self.outputs[n][:b]
