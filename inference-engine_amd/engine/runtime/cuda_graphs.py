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

    Static metadata lives in two device blocks: int64 ``[ids | positions | slots |
    chunk rows (T each) | last | decode rows (S each)]`` and int32 ``[decode ctx | chunk
    ctx (S each) | cu_q (S + 1) | decode tables | chunk tables (S x W each)]`` for the
    largest bucket T, ``max_seqs`` S and table width W. W is ``max_blocks_per_seq`` or,
    by default, the blocks of the longest sequence the model and pool allow
    (``model.cfg.max_position_embeddings`` capped by the pool, the bound the reference's
    engine gives its decode graphs, engine/runtime/engine.py:75-77, :96-99). A step
    writes only the rows and columns it uses: the kernels never read a table column
    past a context's last block, so stale entries there are harmless, and a padding
    decode row reads column 0 only, which is the one column reset when a row turns
    into padding. A step's cost therefore follows its own size, not W or the pool.
    """

    def __init__(self, model: Callable, cache: PagedKVCache, scratch_block: int,
                 max_seqs: int, max_tokens: int,
                 max_blocks_per_seq: int | None = None) -> None:  # fmt: skip
        if max_seqs < 1 or max_tokens < 1:
            raise ValueError("MixedGraphs: max_seqs and max_tokens must be >= 1")
        self.model, self.cache, self.scratch_block = model, cache, scratch_block
        self.scratch_slot = scratch_block * cache.block_size
        top = min(max_tokens + 1, TOKEN_BUCKETS[-1])
        self.sizes = sorted({s for s in TOKEN_BUCKETS if s < top} | {top})
        self.max_seqs = max_seqs
        self.max_width = max_blocks_per_seq or _longest_table(model, cache)
        big_t, s, w = self.sizes[-1], max_seqs, self.max_width
        dev = cache.k.device
        self._i64 = torch.zeros(4 * big_t + 2 * s, dtype=torch.int64, device=dev)
        ids, pos, self._slots, self._ch_rows, self._last, self._dec_rows = torch.split(
            self._i64, [big_t, big_t, big_t, big_t, s, s])
        self._tok = self._i64[: 2 * big_t].view(2, big_t)  # ids and positions, rows 0 / 1
        self._ids, self._pos = ids.view(1, big_t), pos.view(1, big_t)
        self._i32 = torch.zeros(3 * s + 1 + 2 * s * w, dtype=torch.int32, device=dev)
        dctx, cctx, self._cu_q, dtab, ctab = torch.split(
            self._i32, [s, s, s + 1, s * w, s * w])
        self._dec_ctx, self._ch_ctx = dctx, cctx
        self._dec_tab, self._ch_tab = dtab.view(s, w), ctab.view(s, w)
        # ids and positions go up in one asynchronous copy from pinned memory
        self._host_tok = torch.zeros(2, big_t, dtype=torch.int64, pin_memory=True)
        self._sent = torch.cuda.Event()
        self._sent.record()
        # what the previous step wrote: (tokens, decode rows, chunks, bucket)
        self._prev = (big_t, s, s, big_t)
        self._dec_tab.fill_(scratch_block)
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._logits: dict[int, torch.Tensor] = {}
        self._views = {n: self._batch_of(n) for n in self.sizes}
        self._pad(self.sizes[-1], 0, 0, 0)  # an all-padding step for the warm-up
        pool = torch.cuda.graph_pool_handle()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up outside any capture: libraries pick kernels
            for n in self.sizes:
                self._pad(n, 0, 0, 0)
                self._forward(n)
        torch.cuda.current_stream().wait_stream(side)
        for n in self.sizes:
            self._pad(n, 0, 0, 0)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                self._logits[n] = self._forward(n)
            self._graphs[n] = graph
        torch.cuda.synchronize()

    def _batch_of(self, n: int) -> PagedBatch:
        """Bucket n's mixed batch, every tensor a view of the static blocks (the graph
        reads them by address)."""
        empty = torch.zeros(0, dtype=torch.int64, device=self._i64.device)
        return PagedBatch(
            cache=self.cache, slot_mapping=self._slots[:n], kv_slots=empty, q_index=empty,
            q_valid=torch.zeros(0, dtype=torch.bool, device=self._i64.device), attn_mask=None,
            last_index=self._last, use_kernel=False, mixed=True, decode_rows=self._dec_rows,
            block_tables=self._dec_tab, context_lens=self._dec_ctx, chunks=[],
            chunk_rows=self._ch_rows[:n], chunk_tables=self._ch_tab, chunk_ctx=self._ch_ctx,
            cu_seqlens_q=self._cu_q, max_query_len=n)  # fmt: skip

    def _forward(self, n: int) -> torch.Tensor:
        return self.model(self._ids[:, :n], self._pos[:, :n], self._views[n])

    def _pad(self, n: int, t: int, d: int, c: int, tq: int = 0) -> None:
        """Padding for bucket n around a step of t tokens, d decode rows, c chunks of tq
        tokens in all: only what this step leaves unwritten and the previous step (or
        a smaller bucket) may have left stale."""
        t_prev, d_prev, _, _ = self._prev
        self._tok[:, t:n].zero_()
        self._slots[t:n].fill_(self.scratch_slot)
        self._last.zero_()  # stale indices could point past this bucket
        self._dec_rows[d:].fill_(n - 1)
        self._dec_ctx[d:].fill_(1)
        if d < d_prev:  # rows that were real and now pad read column 0 only
            self._dec_tab[d:d_prev, 0].fill_(self.scratch_block)
        self._ch_rows[tq:n].fill_(n - 1)
        self._ch_ctx[c:].zero_()
        self._cu_q[c + 1 :].fill_(tq)  # padding chunks: empty
        self._prev = (t, d, c, n)

    def can_run(self, num_tokens: int, num_seqs: int, width: int | None = None) -> bool:
        return (num_tokens < self.sizes[-1] and num_seqs <= self.max_seqs
                and (width is None or width <= self.max_width))  # fmt: skip

    def run(self, ids: Sequence[int], positions: Sequence[int],
            batch: PagedBatch) -> torch.Tensor:  # fmt: skip
        """One mixed step: the step's flattened token ids and positions and its mixed
        ``PagedBatch`` (built as for an eager step) -> logits [B, 1, vocab]."""
        t = len(ids)
        if not 1 <= t < self.sizes[-1]:
            raise ValueError(f"MixedGraphs: {t} tokens outside 1..{self.sizes[-1] - 1}")
        n = self.sizes[bisect.bisect_right(self.sizes, t)]
        d = 0 if batch.block_tables is None else batch.block_tables.shape[0]
        c = 0 if batch.chunk_rows is None else batch.chunk_tables.shape[0]
        tq = 0 if batch.chunk_rows is None else batch.chunk_rows.numel()
        for rows, width in ((d, None if d == 0 else batch.block_tables.shape[1]),
                            (c, None if c == 0 else batch.chunk_tables.shape[1])):
            if rows > self.max_seqs or (width is not None and width > self.max_width):
                raise ValueError(f"MixedGraphs: {rows} rows of width {width} exceed "
                                 f"{self.max_seqs} x {self.max_width}")  # fmt: skip
        self._sent.synchronize()  # the previous step's copy has left the host block
        h = self._host_tok.numpy()
        h[0, :t] = ids
        h[1, :t] = positions
        self._tok[:, :t].copy_(self._host_tok[:, :t], non_blocking=True)
        self._sent.record()
        self._pad(n, t, d, c, tq)
        self._slots[:t].copy_(batch.slot_mapping)
        self._last[: batch.last_index.numel()].copy_(batch.last_index)
        if d:
            w = batch.block_tables.shape[1]
            self._dec_rows[:d].copy_(batch.decode_rows)
            self._dec_tab[:d, :w].copy_(batch.block_tables)
            self._dec_ctx[:d].copy_(batch.context_lens)
        if c:
            w = batch.chunk_tables.shape[1]
            self._ch_rows[:tq].copy_(batch.chunk_rows)
            self._ch_tab[:c, :w].copy_(batch.chunk_tables)
            self._ch_ctx[:c].copy_(batch.chunk_ctx)
            self._cu_q[: c + 1].copy_(batch.cu_seqlens_q)
        self._graphs[n].replay()
        return self._logits[n][: batch.last_index.numel()]


def _longest_table(model: Callable, cache: PagedKVCache) -> int:
    """Blocks of the longest sequence: the model's position limit capped by the pool
    (less the scratch block), as the reference's engine bounds max_model_len."""
    bs = cache.block_size
    pool_tokens = max(cache.num_blocks - 1, 1) * bs
    limit = getattr(getattr(model, "cfg", None), "max_position_embeddings", None)
    tokens = min(limit, pool_tokens) if limit else pool_tokens
    return -(-tokens // bs)
