"""Paged KV pool with a HIP append and block copy; the layout and ``write`` signature of
the reference's ``engine/runtime/paged_cache.py`` (``PagedKVCache``, :22-49).

The pool is one flat array of slots per layer: k, v are [layers, num_blocks *
block_size, nkv, hd]; slot ``s`` of block ``b`` is row ``b * block_size + s``. A whole
block of one layer is a contiguous [block_size, nkv, hd] span, which is what the
decode kernel streams and what ``copy_blocks`` moves.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from engine.kernels import _native


@dataclass(frozen=True)
class KVShape:
    """The three model fields the pool needs (the reference reads them off its
    ModelConfig, engine/config.py); any object with these attributes works."""

    num_hidden_layers: int
    num_key_value_heads: int
    head_dim: int


class PagedKVCache:
    def __init__(
        self,
        cfg: KVShape,
        num_blocks: int,
        block_size: int = 16,
        device: str | torch.device = "cuda",
        dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        self.num_blocks, self.block_size = num_blocks, block_size
        shape = (cfg.num_hidden_layers, num_blocks * block_size, cfg.num_key_value_heads,
                 cfg.head_dim)  # fmt: skip
        self.k = torch.zeros(shape, device=device, dtype=dtype)
        self.v = torch.zeros(shape, device=device, dtype=dtype)

    @staticmethod
    def bytes_per_block(cfg: KVShape, block_size: int, dtype: torch.dtype) -> int:
        per_token = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim
        return per_token * block_size * torch.tensor([], dtype=dtype).element_size()

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor) -> None:
        """k, v: [N, nkv, hd] for the step's new tokens; slots: [N] int64 flat slot ids.

        Same result as ``self.k[layer].index_copy_(0, slots, k.to(self.k.dtype))`` and
        the V twin (reference :42-45), in one HIP launch for both pools. Slots outside
        the pool are skipped rather than faulting the GPU (IndexError, as index_copy_
        raises, with ``_native.set_debug_checks(True)`` or PKV_DEBUG_CHECKS=1).
        """
        kv_append(self.k[layer], self.v[layer], k, v, slots)

    def gather(self, layer: int, kv_slots: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """kv_slots: [B, max_ctx] -> k, v: [B, max_ctx, nkv, hd] (reference :47-49)."""
        return self.k[layer][kv_slots], self.v[layer][kv_slots]

    def copy_blocks(self, block_mapping: torch.Tensor) -> None:
        """Copy-on-write: for every layer and each (src, dst) row of ``block_mapping``
        ([n, 2] int64 on the pool's device) copy block src over block dst, K and V.
        The reference has no such operation (its prefix cache never writes a shared
        block, engine/runtime/block_manager.py:130-150)."""
        copy_blocks(self.k, self.v, block_mapping, self.block_size)


def kv_append(
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    slots: torch.Tensor,
) -> None:
    """k_pool[slots[i]] = k[i].to(pool dtype), likewise v, for one layer's pools
    [num_slots, nkv, hd]. k, v: [N, nkv, hd] with unit stride in hd (else copied)."""
    what = "kv_append"
    dev = _native.require_gpu(what, k_pool, v_pool, k, v, slots)
    if slots.dtype != torch.int64:
        raise RuntimeError(f"{what}: expected a long tensor for slots, got {slots.dtype}")
    if k_pool.dim() != 3 or k_pool.shape != v_pool.shape or k_pool.stride() != v_pool.stride():
        raise ValueError(f"{what}: pools must be equal [num_slots, nkv, hd] tensors")
    if k_pool.dtype != v_pool.dtype:
        raise TypeError(f"{what}: pools must share one dtype")
    n = slots.numel()
    if slots.dim() != 1 or k.shape != (n, *k_pool.shape[1:]) or v.shape != k.shape:
        raise IndexError(f"{what}: {n} slots for k {tuple(k.shape)}, v {tuple(v.shape)}, "
                         f"pool rows {tuple(k_pool.shape[1:])}")  # fmt: skip
    if k.dtype != v.dtype:
        raise TypeError(f"{what}: k and v must share one dtype")
    if k_pool.stride(2) != 1:
        raise ValueError(f"{what}: pool needs unit stride in head_dim")
    if n == 0:
        return
    if _native.debug_checks():
        _native.check_slots(what, slots, k_pool.shape[0])
    if k.stride(2) != 1:
        k = k.contiguous()
    if v.stride(2) != 1:
        v = v.contiguous()
    slots = slots.contiguous()
    status = _native.lib().pkv_kv_append(
        k_pool.data_ptr(), v_pool.data_ptr(), _native.dtype_code(k_pool.dtype, what),
        k_pool.stride(0), k_pool.stride(1), k_pool.shape[0],
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), _native.dtype_code(k.dtype, what),
        slots.data_ptr(), n, k_pool.shape[1], k_pool.shape[2], _native.stream_of(dev),
    )  # fmt: skip
    _native.check(status, what)


def copy_blocks(
    k_pool: torch.Tensor, v_pool: torch.Tensor, block_mapping: torch.Tensor, block_size: int
) -> None:
    """For pools [L, num_blocks * block_size, nkv, hd] (or one layer, 3-D) and
    block_mapping [n, 2] int64 (src, dst) on the pools' device: every layer's block dst
    becomes a copy of block src, in K and V. No dst may also appear as a src."""
    what = "copy_blocks"
    dev = _native.require_gpu(what, k_pool, v_pool, block_mapping)
    if k_pool.shape != v_pool.shape or k_pool.dtype != v_pool.dtype:
        raise ValueError(f"{what}: K and V pools must match")
    if k_pool.dim() == 3:
        k_pool, v_pool = k_pool[None], v_pool[None]
    if k_pool.dim() != 4 or not (k_pool[0].is_contiguous() and v_pool[0].is_contiguous()):
        raise ValueError(f"{what}: pools must be [L, slots, nkv, hd], contiguous per layer")
    if k_pool.stride() != v_pool.stride():
        raise ValueError(f"{what}: K and V pools need equal strides")
    if block_mapping.dtype != torch.int64 or block_mapping.dim() != 2 or \
            block_mapping.shape[1] != 2:  # fmt: skip
        raise ValueError(f"{what}: block_mapping must be an int64 [n, 2] tensor")
    n = block_mapping.shape[0]
    if n == 0:
        return
    layers, slots, nkv, hd = k_pool.shape
    if slots % block_size:
        raise ValueError(f"{what}: {slots} slots not a multiple of block_size {block_size}")
    elt = k_pool.element_size()
    if _native.debug_checks():
        _native.check_slots(what, block_mapping.reshape(-1), slots // block_size)
    block_mapping = block_mapping.contiguous()
    status = _native.lib().pkv_copy_blocks(
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0) * elt, layers,
        block_size * nkv * hd * elt, slots // block_size, block_mapping.data_ptr(), n,
        _native.stream_of(dev),
    )  # fmt: skip
    _native.check(status, what)


def decode_slots(block_tables: torch.Tensor, context_lens: torch.Tensor, block_size: int,
                 num_slots: int, out: torch.Tensor | None = None) -> torch.Tensor:  # fmt: skip
    """Slot of each sequence's newest token, ``table[(n-1)//bs]*bs + (n-1)%bs`` with
    n = context_lens[b], computed on the device (int64 [B]; -1 where n < 1 or the block
    lies past the table or the pool: the append skips it). The reference builds these on
    the host (engine/runtime/paged_cache.py:140-143, engine/runtime/cuda_graphs.py:104);
    on the device a captured decode step needs only tables and lengths copied in."""
    what = "decode_slots"
    dev = _native.require_gpu(what, block_tables, context_lens)
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise TypeError(f"{what}: block_tables and context_lens must be int32")
    b = context_lens.numel()
    if block_tables.dim() != 2 or block_tables.shape[0] != b or block_tables.stride(1) != 1 \
            or not context_lens.is_contiguous():  # fmt: skip
        raise ValueError(f"{what}: block_tables [B, W] (unit column stride), context_lens [B]")
    if out is None:
        out = torch.empty(b, dtype=torch.int64, device=dev)
    elif out.dtype != torch.int64 or out.shape != (b,) or not out.is_contiguous():
        raise ValueError(f"{what}: out must be a contiguous int64 [B] tensor")
    status = _native.lib().pkv_decode_slots(
        out.data_ptr(), block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
        context_lens.data_ptr(), b, block_size, num_slots, _native.stream_of(dev))  # fmt: skip
    _native.check(status, what)
    return out


@dataclass
class PagedBatch:
    """Everything attention needs for one step, built once and shared by all layers.

    The fields and their meaning are the reference's (engine/runtime/paged_cache.py:52-77),
    so its unchanged call sites -- ``Attention._paged`` (engine/model/layers.py:191-225),
    which tests ``use_kernel``, then ``mixed``, else gathers; ``Attention._mixed``
    (:227-266), which sends decode rows to the decode kernel, then ``varlen``, then loops
    over ``chunks`` -- dispatch these batches as they dispatch the reference's:

    * decode steps (every sequence adds one token): ``use_kernel`` True,
      ``block_tables`` / ``context_lens`` for the decode kernel;
    * mixed steps: ``use_kernel`` False, ``mixed`` True, the decode rows as above, and
      every longer run of new tokens (a prompt or prompt chunk, its queries last in its
      context) described for the chunked-prefill kernel by the ``chunk_*`` fields. The
      reference's ``varlen`` (gathered slots for FlashAttention) is None and ``chunks``
      (one SDPA per chunk) is empty, so the only line of ``_mixed`` that changes is the
      varlen call (layers.py:246-253), which becomes ``paged_prefill_attention`` over
      the ``chunk_*`` fields, for every dtype and head size;
    * ``use_kernel=False`` builds: the reference's gather metadata (``kv_slots``,
      ``q_index``, ``q_valid``, ``attn_mask``) for its PyTorch path; this build's call
      site (engine.model.layers.paged_attention) rejects them.

    A step's new tokens from every sequence are flattened into one row of N tokens;
    sequence i owns the next query_lens[i] of them.
    """

    cache: PagedKVCache
    slot_mapping: torch.Tensor  # [N] int64: where each new token's K/V is written
    kv_slots: torch.Tensor  # [B, max_ctx] slot of every context position (gather path)
    q_index: torch.Tensor  # [B, max_q] flat token index of each padded query (gather path)
    q_valid: torch.Tensor  # [B, max_q] bool (gather path)
    attn_mask: torch.Tensor | None  # [B, 1, max_q, max_ctx] bool (gather path)
    last_index: torch.Tensor  # [B] flat index of each sequence's last new token
    use_kernel: bool = False
    block_tables: torch.Tensor | None = None  # [Bd, W] int32: decode rows
    context_lens: torch.Tensor | None = None  # [Bd] int32, new token included
    mixed: bool = False
    decode_rows: torch.Tensor | None = None  # [Bd] int64 flat token index
    chunks: list | None = None  # the reference's per-chunk SDPA list: always empty here
    varlen: tuple | None = None  # the reference's FlashAttention varlen inputs: None here
    # Chunked-prefill kernel inputs of a mixed step (None without prompt chunks):
    chunk_rows: torch.Tensor | None = None  # [Tq] int64 flat index of every chunk token
    chunk_tables: torch.Tensor | None = None  # [C, W] int32
    chunk_ctx: torch.Tensor | None = None  # [C] int32 context incl. the chunk's tokens
    cu_seqlens_q: torch.Tensor | None = None  # [C + 1] int32 offsets into chunk_rows
    max_query_len: int = 0
    # Decode steps with cascade on: the groups of sequences sharing leading blocks
    # (engine.kernels.paged_attention.PrefixGroups), or None.
    prefix_groups: object | None = None

    @classmethod
    def build(
        cls,
        cache: PagedKVCache,
        block_tables: Sequence[Sequence[int]],
        context_lens: Sequence[int],
        query_lens: Sequence[int],
        device: str | torch.device,
        use_kernel: bool = False,
        force_mixed: bool = False,
        *,
        device_slots: bool = False,
        cascade: bool = False,
        num_heads: int | None = None,
        cascade_min_blocks: int = 16,
    ) -> PagedBatch:
        """Per sequence, in flattened order: its block table, its context length after
        this step (new tokens included) and its number of new tokens (reference :80-127).

        With ``use_kernel``: a step where every sequence adds one token (and not
        ``force_mixed``) is a decode batch; any other step is a mixed batch -- a single
        sequence's prompt included, which the reference would gather, since the chunk
        kernel serves it. Without: the reference's gather metadata.
        Extensions (keyword-only): ``device_slots``: decode steps compute the slot
        mapping on the device from the uploaded tables instead of on the host.
        ``cascade``: decode steps look for sequences whose tables start with the same
        blocks (prompt prefixes shared through a fork; at least ``cascade_min_blocks``
        of them, fully covered) and attend to each shared prefix once per group
        (``paged_decode_attention(prefix_groups=)``); needs the model's ``num_heads``.
        Copy-on-write copies are the caller's, before the step (``cache.copy_blocks``).
        """
        if not query_lens:
            raise ValueError("PagedBatch: empty step")
        if len(block_tables) != len(query_lens) or len(context_lens) != len(query_lens):
            raise ValueError("PagedBatch: one table, context length and query length per "
                             "sequence")  # fmt: skip
        if not use_kernel:
            return cls._gather(cache, block_tables, context_lens, query_lens, device)
        if max(query_lens) == 1 and not force_mixed:
            batch = cls._decode(cache, block_tables, context_lens, device, device_slots)
            if cascade:
                if num_heads is None:
                    raise ValueError("PagedBatch: cascade needs the model's num_heads")
                from engine.kernels.paged_attention import find_prefix_groups

                batch.prefix_groups = find_prefix_groups(
                    cls._tables(block_tables), list(context_lens), cache.block_size,
                    num_heads, cache.k.shape[2], device, min_blocks=cascade_min_blocks,
                    dtype=cache.k.dtype, head_dim=cache.k.shape[-1])  # fmt: skip
            return batch
        return cls._mixed(cache, block_tables, context_lens, query_lens, device)

    @staticmethod
    def _tables(rows: Sequence[Sequence[int]]) -> torch.Tensor:
        width = max(1, max(len(t) for t in rows))
        return torch.tensor([list(t) + [0] * (width - len(t)) for t in rows], dtype=torch.int32)

    @staticmethod
    def _check(table: Sequence[int], ctx: int, q: int, bs: int) -> None:
        if q < 1 or ctx < q:
            raise ValueError(f"PagedBatch: {q} new tokens in a context of {ctx}")
        if -(-ctx // bs) > len(table):
            raise ValueError(f"PagedBatch: a table of {len(table)} blocks cannot hold "
                             f"{ctx} tokens")  # fmt: skip

    @classmethod
    def _gather(cls, cache: PagedKVCache, block_tables, context_lens, query_lens,
                device) -> PagedBatch:  # fmt: skip
        """The reference's metadata for its PyTorch gather path (reference :100-127):
        every context slot, padded query indices, and the bottom-right causal mask
        (query i of a sequence with q new tokens in a context of n sees keys up to
        n - q + i; padded query rows see key 0 only, so no row is all masked)."""
        bs = cache.block_size
        b, max_q, max_ctx = len(query_lens), max(query_lens), max(context_lens)
        kv = torch.zeros(b, max_ctx, dtype=torch.int64)
        slot_mapping: list[int] = []
        for i, (table, ctx, q) in enumerate(zip(block_tables, context_lens, query_lens,
                                                strict=True)):  # fmt: skip
            cls._check(table, ctx, q, bs)
            pos = torch.arange(ctx)
            kv[i, :ctx] = torch.tensor(list(table), dtype=torch.int64)[pos // bs] * bs + pos % bs
            slot_mapping += kv[i, ctx - q : ctx].tolist()
        qlens = torch.tensor(list(query_lens))
        ctxs = torch.tensor(list(context_lens))
        starts = torch.cumsum(qlens, 0) - qlens
        col = torch.arange(max_q)
        q_valid = col[None] < qlens[:, None]
        q_index = torch.where(q_valid, starts[:, None] + col[None], 0)
        q_pos = (ctxs - qlens)[:, None] + col[None]  # [B, max_q] absolute query positions
        k_pos = torch.arange(max_ctx)
        see = (k_pos[None, None] <= q_pos[:, :, None]) & (k_pos[None] < ctxs[:, None])[:, None]
        see |= ~q_valid[:, :, None] & (k_pos == 0)[None, None]
        return cls(cache=cache,
                   slot_mapping=torch.tensor(slot_mapping, dtype=torch.int64, device=device),
                   kv_slots=kv.to(device), q_index=q_index.to(device),
                   q_valid=q_valid.to(device), attn_mask=see[:, None].to(device),
                   last_index=(starts + qlens - 1).to(device))  # fmt: skip

    @classmethod
    def _decode(cls, cache: PagedKVCache, block_tables, context_lens, device,
                device_slots: bool) -> PagedBatch:  # fmt: skip
        """Reference :130-156: tables padded with block 0, the new token's slot."""
        bs, b = cache.block_size, len(context_lens)
        for table, ctx in zip(block_tables, context_lens, strict=True):
            cls._check(table, ctx, 1, bs)
        tables = cls._tables(block_tables).to(device)
        ctx = torch.tensor(list(context_lens), dtype=torch.int32, device=device)
        if device_slots:
            slots = decode_slots(tables, ctx, bs, cache.k.shape[1])
        else:
            slots = torch.tensor(
                [t[(n - 1) // bs] * bs + (n - 1) % bs
                 for t, n in zip(block_tables, context_lens, strict=True)],
                dtype=torch.int64, device=device)  # fmt: skip
        flat = torch.arange(b, device=device)
        return cls(cache=cache, slot_mapping=slots, kv_slots=flat, q_index=flat[:, None],
                   q_valid=torch.ones(b, 1, dtype=torch.bool, device=device), attn_mask=None,
                   last_index=flat, use_kernel=True, block_tables=tables,
                   context_lens=ctx)  # fmt: skip

    @classmethod
    def _mixed(cls, cache: PagedKVCache, block_tables, context_lens, query_lens,
               device) -> PagedBatch:  # fmt: skip
        """Reference :159-229 without the gather: decode rows keep their tables; every
        run of q > 1 new tokens becomes a chunk whose queries sit at positions
        ctx - q .. ctx - 1 of its context (bottom-right causal)."""
        bs = cache.block_size
        slots: list[int] = []
        dec_rows, dec_tables, dec_ctx = [], [], []
        ch_rows, ch_tables, ch_ctx, ch_q = [], [], [], []
        start = 0
        for table, ctx, q in zip(block_tables, context_lens, query_lens, strict=True):
            cls._check(table, ctx, q, bs)
            slots.extend(table[p // bs] * bs + p % bs for p in range(ctx - q, ctx))
            if q == 1:
                dec_rows.append(start)
                dec_tables.append(table)
                dec_ctx.append(ctx)
            else:
                ch_rows.extend(range(start, start + q))
                ch_tables.append(table)
                ch_ctx.append(ctx)
                ch_q.append(q)
            start += q
        qlens = torch.tensor(list(query_lens), device=device)
        empty = torch.zeros(0, dtype=torch.int64, device=device)
        batch = cls(cache=cache,
                    slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
                    kv_slots=empty, q_index=empty,
                    q_valid=torch.zeros(0, dtype=torch.bool, device=device), attn_mask=None,
                    last_index=torch.cumsum(qlens, 0) - 1, use_kernel=False, mixed=True,
                    decode_rows=torch.tensor(dec_rows, dtype=torch.int64, device=device),
                    chunks=[])  # fmt: skip
        if dec_rows:
            batch.block_tables = cls._tables(dec_tables).to(device)
            batch.context_lens = torch.tensor(dec_ctx, dtype=torch.int32, device=device)
        if ch_rows:
            cu = torch.zeros(len(ch_q) + 1, dtype=torch.int32)
            cu[1:] = torch.cumsum(torch.tensor(ch_q, dtype=torch.int32), 0)
            batch.chunk_rows = torch.tensor(ch_rows, dtype=torch.int64, device=device)
            batch.chunk_tables = cls._tables(ch_tables).to(device)
            batch.chunk_ctx = torch.tensor(ch_ctx, dtype=torch.int32, device=device)
            batch.cu_seqlens_q = cu.to(device)
            batch.max_query_len = max(ch_q)
        return batch


def varlen_available(t: torch.Tensor) -> bool:
    """Whether mixed steps would gather for FlashAttention's varlen kernel
    (reference engine/runtime/paged_cache.py:232-240, which its tests call and
    monkeypatch). Never here: the chunked-prefill kernel reads the paged pool in place, so
    ``PagedBatch.varlen`` stays None for every device, dtype and torch version."""
    del t
    return False
