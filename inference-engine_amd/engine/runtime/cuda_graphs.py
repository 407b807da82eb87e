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


# Mixed steps (some sequences reading prompt tokens) by total tokens in the step.
TOKEN_BUCKETS = (16, 32, 64, 128, 256, 384, 512, 768, 1024, 1536, 2048)


class MixedGraphs:
    """Mixed steps as hipGraph replays, one graph per token bucket for the whole step.

    The reference captures mixed steps piecewise, with attention run eagerly between the
    per-layer graphs, because its attention changes shape every step (reference
    engine/runtime/cuda_graphs.py:116-228). Here attention is this build's HIP kernels,
    which read every piece of step metadata -- decode rows and their tables and lengths,
    chunk offsets, chunk tables and contexts -- from device memory and size their grids
    from static bounds only (the chunked-prefill grid from the bucket size), so the
    whole step, all layers included, is one graph.

    A step of t tokens runs in the smallest bucket n > t: rows t .. n-1 are padding
    tokens (token 0, writing their K/V into the scratch block, never sampled). Padding
    decode rows (context 1 on the scratch block) and padding chunk-row indices point at
    row n - 1, a padding row, so whatever they compute lands there; padding chunks have
    no tokens. Every op outside attention treats rows independently, so real rows
    compute exactly what they would in an eager step.
    """

    def __init__(self, model: Callable, cache: PagedKVCache, scratch_block: int,
                 max_seqs: int, max_tokens: int, max_blocks_per_seq: int) -> None:  # fmt: skip
        self.model, self.cache = model, cache
        dev = cache.k.device
        cap = min(max_tokens + 1, TOKEN_BUCKETS[-1])
        self.sizes = [s for s in TOKEN_BUCKETS if s < cap] + [cap]
        t, b, w = self.sizes[-1], max_seqs, max_blocks_per_seq
        self.max_seqs, self.max_width = b, w
        self.scratch_block = scratch_block
        self.scratch_slot = scratch_block * cache.block_size
        i64, i32 = torch.int64, torch.int32
        self.ids = torch.zeros(1, t, dtype=i64, device=dev)
        self.pos = torch.zeros(1, t, dtype=i64, device=dev)
        self.slots = torch.full((t,), self.scratch_slot, dtype=i64, device=dev)
        self.last = torch.zeros(b, dtype=i64, device=dev)
        self.dec_rows = torch.zeros(b, dtype=i64, device=dev)
        self.dec_tables = torch.full((b, w), scratch_block, dtype=i32, device=dev)
        self.dec_ctx = torch.ones(b, dtype=i32, device=dev)
        self.ch_rows = torch.zeros(t, dtype=i64, device=dev)
        self.ch_tables = torch.full((b, w), scratch_block, dtype=i32, device=dev)
        self.ch_ctx = torch.zeros(b, dtype=i32, device=dev)
        self.cu_q = torch.zeros(b + 1, dtype=i32, device=dev)
        self.row_tables = torch.full((t, w), scratch_block, dtype=i32, device=dev)
        self.row_ctx = torch.ones(t, dtype=i32, device=dev)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.outputs: dict[int, torch.Tensor] = {}
        self._batches: dict[int, PagedBatch] = {}
        self._capture()

    def _batch(self, n: int) -> PagedBatch:
        return PagedBatch(
            cache=self.cache, slot_mapping=self.slots[:n], last_index=self.last, mixed=True,
            decode_rows=self.dec_rows, block_tables=self.dec_tables, context_lens=self.dec_ctx,
            chunk_rows=self.ch_rows[:n], chunk_tables=self.ch_tables, chunk_ctx=self.ch_ctx,
            cu_seqlens_q=self.cu_q, max_query_len=n, row_tables=self.row_tables[:n],
            row_ctx=self.row_ctx[:n])  # fmt: skip

    def _reset(self, n: int) -> None:
        """Every metadata buffer to its padding value for bucket n (an all-padding step)."""
        self.ids.zero_()
        self.pos.zero_()
        self.slots.fill_(self.scratch_slot)
        self.last.zero_()
        self.dec_rows.fill_(n - 1)
        self.dec_tables.fill_(self.scratch_block)
        self.dec_ctx.fill_(1)
        self.ch_rows.fill_(n - 1)
        self.ch_tables.fill_(self.scratch_block)
        self.ch_ctx.zero_()
        self.cu_q.zero_()
        self.row_tables.fill_(self.scratch_block)
        self.row_ctx.fill_(1)

    def _capture(self) -> None:
        pool = None
        for n in reversed(self.sizes):  # largest first: smaller graphs reuse its pool
            self._reset(n)
            batch = self._batch(n)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):  # warm-up outside the capture
                    self.model(self.ids[:, :n], self.pos[:, :n], batch)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                out = self.model(self.ids[:, :n], self.pos[:, :n], batch)
            pool = graph.pool()
            self.graphs[n], self.outputs[n], self._batches[n] = graph, out, batch
        torch.cuda.synchronize()

    def can_run(self, num_tokens: int, num_seqs: int, width: int) -> bool:
        return (num_tokens < self.sizes[-1] and num_seqs <= self.max_seqs
                and width <= self.max_width)  # fmt: skip

    def run(self, ids: Sequence[int], positions: Sequence[int],
            batch: PagedBatch) -> torch.Tensor:  # fmt: skip
        """One mixed step: the step's flattened token ids and positions and its mixed
        ``PagedBatch`` (built as for an eager step) -> logits [B, 1, vocab]."""
        t, b = len(ids), batch.last_index.numel()
        n = next(s for s in self.sizes if s > t)
        self._reset(n)
        self.ids[0, :t].copy_(torch.tensor(list(ids)), non_blocking=True)
        self.pos[0, :t].copy_(torch.tensor(list(positions)), non_blocking=True)
        self.slots[:t].copy_(batch.slot_mapping)
        self.last[:b].copy_(batch.last_index)
        if batch.decode_rows is not None:
            d, w = batch.block_tables.shape
            self.dec_rows[:d].copy_(batch.decode_rows)
            self.dec_tables[:d, :w].copy_(batch.block_tables)
            self.dec_ctx[:d].copy_(batch.context_lens)
        if batch.chunk_rows is not None:
            tq = batch.chunk_rows.numel()
            c, w = batch.chunk_tables.shape
            self.ch_rows[:tq].copy_(batch.chunk_rows)
            self.ch_tables[:c, :w].copy_(batch.chunk_tables)
            self.ch_ctx[:c].copy_(batch.chunk_ctx)
            self.cu_q[: c + 1].copy_(batch.cu_seqlens_q)
            self.cu_q[c + 1 :].fill_(tq)  # padding chunks: empty
            self.row_tables[:tq, :w].copy_(batch.row_tables)
            self.row_ctx[:tq].copy_(batch.row_ctx)
        self.graphs[n].replay()
        return self.outputs[n][:b]
