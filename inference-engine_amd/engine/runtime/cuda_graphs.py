"""Decode and mixed steps as hipGraph replays, with the constructor and ``run`` signatures
of the reference's ``DecodeGraphs`` / ``MixedGraphs`` (engine/runtime/cuda_graphs.py:23-108,
:116-228). torch's CUDA graph API is hipGraph on ROCm.

Both capture the whole step once per size bucket and replay it: every kernel of this
build reads the step's metadata from device memory and sizes its grid from static
bounds only, so one graph serves every context length and every mix of sequences that
fits the bucket. Padding rows write and read only the scratch block, a block the
allocator never hands out.
"""

from __future__ import annotations

import bisect
from collections.abc import Callable, Sequence

import numpy as np
import torch

from engine.kernels import paged_attention as pa
from engine.runtime.paged_cache import PagedBatch, PagedKVCache, decode_slots

# Batch-size buckets of decode graphs (the reference's table).
BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 192, 256)


class DecodeGraphs:
    """Decode steps of ``model(input_ids [1, n], positions [1, n], batch) -> logits
    [n, 1, vocab]`` as one graph per batch bucket n.

    Step metadata lives in one int32 device block laid out as
    ``[ctx (M) | ids (M) | positions (M) | prefix groups (P) | tables (M, W)]`` for the
    largest bucket M and table width W, so bucket n's data is the contiguous prefix of
    3 M + P + n W entries. A step fills a pinned host copy of that prefix with numpy and
    sends it with a single asynchronous copy; the captured graph widens ids and
    positions to int64, builds the slot mapping on the device (``decode_slots``) and runs
    the model. Padding rows have context length 1 in the scratch block.

    ``cascade`` (needs the model's ``num_heads``): every step also looks for sequences
    whose tables start with the same blocks (``shared_prefixes``, at least
    ``cascade_min_blocks``; the ``max_groups`` largest groups) and lays them out in the
    prefix-groups region in a fixed shape per bucket -- K pieces, max_groups chunks per
    piece, member rows n apart -- which the captured decode calls read as their
    ``prefix_groups``: each shared prefix is read once per layer-step for its whole
    group. A step without groups runs the plain decode inside the same graph. Every
    chunk slot adds workgroups to the prefix pass whether a group fills it or not (at
    config 3, 256 sequences: 128.7 us per layer-step with one slot, 129.5 with two),
    hence the default of the one largest group (one shared system prompt); engines with
    several popular prefixes raise ``max_groups``.
    """

    def __init__(self, model: Callable, cache: PagedKVCache, scratch_block: int,
                 max_batch: int, max_blocks_per_seq: int, *, cascade: bool = False,
                 num_heads: int | None = None, cascade_min_blocks: int = 16,
                 max_groups: int = 1) -> None:  # fmt: skip
        if max_batch < 1 or max_blocks_per_seq < 1:
            raise ValueError("DecodeGraphs: max_batch and max_blocks_per_seq must be >= 1")
        if cascade and not num_heads:
            raise ValueError("DecodeGraphs: cascade needs the model's num_heads")
        self.model, self.cache, self.scratch_block = model, cache, scratch_block
        self.sizes = sorted({s for s in BUCKETS if s < max_batch} | {max_batch})
        self.max_width = max_blocks_per_seq
        top, w = self.sizes[-1], max_blocks_per_seq
        dev = cache.k.device
        self.cascade, self.min_blocks, self.max_groups = cascade, cascade_min_blocks, max_groups
        # Per bucket: (pieces, chunk slots per piece, piece table width) of its layout.
        self._shape: dict[int, tuple[int, int, int]] = {}
        pre = 0
        if cascade:
            nkv = cache.k.shape[2]
            for n in self.sizes:
                k = pa.cascade_pieces(n, num_heads, nkv, dev, dtype=cache.k.dtype,
                                      head_dim=cache.k.shape[-1], block_size=cache.block_size)  # fmt: skip
                self._shape[n] = (k, max_groups, -(-w // k))
                pre = max(pre, pa.prefix_entries(n, *self._shape[n], n))
        self._pre_len = pre
        self._host = torch.zeros(3 * top + pre + top * w, dtype=torch.int32, pin_memory=True)
        self._meta = torch.zeros_like(self._host, device=dev)
        h = self._host.numpy()
        self._h_ctx, self._h_ids, self._h_pos = h[:top], h[top : 2 * top], h[2 * top : 3 * top]
        self._h_pre = h[3 * top : 3 * top + pre]
        self._h_tab = h[3 * top + pre :].reshape(top, w)
        self._ctx, self._ids = self._meta[:top], self._meta[top : 2 * top]
        self._pos = self._meta[2 * top : 3 * top]
        self._pre = self._meta[3 * top : 3 * top + pre]
        self._tab = self._meta[3 * top + pre :].view(top, w)
        self._slots = torch.empty(top, dtype=torch.int64, device=dev)
        self._sent = torch.cuda.Event()  # the host block may be rewritten once this fires
        self._sent.record()
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._logits: dict[int, torch.Tensor] = {}
        self._batches = {n: self._batch_of(n) for n in self.sizes}
        self.groups_last_step = 0
        self._stage(top, [], [], [], [])  # an all-padding step for the warm-up
        self._meta.copy_(self._host)
        pool = torch.cuda.graph_pool_handle()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up outside any capture: libraries pick kernels
            for n in self.sizes:
                self._forward(n)
        torch.cuda.current_stream().wait_stream(side)
        for n in self.sizes:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                self._logits[n] = self._forward(n)
            self._graphs[n] = graph
        torch.cuda.synchronize()

    def _batch_of(self, n: int) -> PagedBatch:
        """The decode batch of bucket n, all of whose tensors are views of the static
        buffers (the graph reads them by address)."""
        flat = torch.arange(n, device=self._meta.device)
        batch = PagedBatch(cache=self.cache, slot_mapping=self._slots[:n], kv_slots=flat,
                           q_index=flat[:, None], q_valid=torch.ones_like(flat[:, None], dtype=torch.bool),
                           attn_mask=None, last_index=flat, use_kernel=True,
                           block_tables=self._tab[:n], context_lens=self._ctx[:n])  # fmt: skip
        if self.cascade:
            k, slots, width = self._shape[n]
            batch.prefix_groups = pa.prefix_view(self._pre, n, k, slots, width, members=n,
                                                  max_members=n)  # fmt: skip
        return batch

    def _forward(self, n: int) -> torch.Tensor:
        batch = self._batches[n]
        decode_slots(batch.block_tables, batch.context_lens, self.cache.block_size,
                     self.cache.k.shape[1], out=batch.slot_mapping)  # fmt: skip
        ids = self._ids[:n].to(torch.int64)[None]
        pos = self._pos[:n].to(torch.int64)[None]
        return self.model(ids, pos, batch)

    def _stage(self, n: int, ids, positions, tables, context_lens) -> None:
        """Write bucket n's metadata into the pinned host block (after the previous
        step's copy has left it)."""
        self._sent.synchronize()
        b = len(ids)
        self._h_ctx[:n] = 1
        self._h_ctx[:b] = context_lens
        self._h_ids[:n] = 0
        self._h_ids[:b] = ids
        self._h_pos[:n] = 0
        self._h_pos[:b] = positions
        self._h_tab[b:n, 0] = self.scratch_block
        for r, row in enumerate(tables):
            self._h_tab[r, : len(row)] = row
        if self.cascade:
            k, slots, width = self._shape[n]
            groups = pa.shared_prefixes(self._h_tab[:b], self._h_ctx[:b], self.cache.block_size,
                                        self.min_blocks) if b else []  # fmt: skip
            # the largest first: a step with more groups than chunk slots leaves the
            # smallest ones to the plain decode
            groups.sort(key=lambda g: -len(g[0]) * g[1])
            groups = groups[:slots]
            pa.fill_prefix(self._h_pre, n, k, slots, width, self._h_tab, groups,
                            self.cache.block_size, n)  # fmt: skip
            self.groups_last_step = len(groups)

    def can_run(self, batch_size: int, width: int) -> bool:
        return batch_size <= self.sizes[-1] and width <= self.max_width

    def run(self, ids: Sequence[int], positions: Sequence[int], slots: Sequence[int] | None,
            tables: Sequence[Sequence[int]], context_lens: Sequence[int]) -> torch.Tensor:  # fmt: skip
        """One decode step for len(ids) sequences -> logits [B, 1, vocab]. ``slots`` is
        accepted for the reference's signature and ignored: the graph derives them from
        the tables and lengths."""
        del slots
        b = len(ids)
        if not 1 <= b <= self.sizes[-1]:
            raise ValueError(f"DecodeGraphs: batch {b} outside 1..{self.sizes[-1]}")
        width = max(len(t) for t in tables)
        if width > self.max_width:
            raise ValueError(f"DecodeGraphs: table width {width} > {self.max_width}")
        n = self.sizes[bisect.bisect_left(self.sizes, b)]
        self._stage(n, np.asarray(ids), np.asarray(positions), tables, np.asarray(context_lens))
        top = self.sizes[-1]
        used = 3 * top + self._pre_len + n * self.max_width
        self._meta[:used].copy_(self._host[:used], non_blocking=True)
        self._sent.record()
        self._graphs[n].replay()
        return self._logits[n][:b]


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

    ``max_blocks_per_seq`` (table width of the static buffers) defaults to the pool's
    block count, which holds any table.
    """

    def __init__(self, model: Callable, cache: PagedKVCache, scratch_block: int,
                 max_seqs: int, max_tokens: int,
                 max_blocks_per_seq: int | None = None) -> None:  # fmt: skip
        self.model, self.cache = model, cache
        dev = cache.k.device
        cap = min(max_tokens + 1, TOKEN_BUCKETS[-1])
        self.sizes = [s for s in TOKEN_BUCKETS if s < cap] + [cap]
        w = max_blocks_per_seq or cache.num_blocks
        t, b = self.sizes[-1], max_seqs
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
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.outputs: dict[int, torch.Tensor] = {}
        self._batches: dict[int, PagedBatch] = {}
        self._capture()

    def _batch(self, n: int) -> PagedBatch:
        empty = torch.zeros(0, dtype=torch.int64, device=self.ids.device)
        return PagedBatch(
            cache=self.cache, slot_mapping=self.slots[:n], kv_slots=empty, q_index=empty,
            q_valid=torch.zeros(0, dtype=torch.bool, device=self.ids.device), attn_mask=None,
            last_index=self.last, use_kernel=False, mixed=True, decode_rows=self.dec_rows,
            block_tables=self.dec_tables, context_lens=self.dec_ctx, chunks=[],
            chunk_rows=self.ch_rows[:n], chunk_tables=self.ch_tables, chunk_ctx=self.ch_ctx,
            cu_seqlens_q=self.cu_q, max_query_len=n)  # fmt: skip

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

    def can_run(self, num_tokens: int, num_seqs: int, width: int | None = None) -> bool:
        return (num_tokens < self.sizes[-1] and num_seqs <= self.max_seqs
                and (width is None or width <= self.max_width))  # fmt: skip

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
        if batch.block_tables is not None:
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
        self.graphs[n].replay()
        return self.outputs[n][:b]
