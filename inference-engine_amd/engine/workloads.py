"""Seeded synthetic decode steps shaped like the engine's own metadata.

Each builder returns a ``DecodeStep``: one layer's K/V pool, the step's queries, the new
K/V rows with their ``slot_mapping``, and ``block_tables`` / ``context_lens`` in the
layout the reference's block manager and ``PagedBatch._decode`` produce (reference
engine/runtime/paged_cache.py:130-156, engine/runtime/block_manager.py:171-174):

- tables are int32 [B, W] padded with block 0, W fixed by the longest context the
  config allows (the engine's ``max_blocks_per_seq``, a static shape);
- context_lens count the token appended this step; its slot is
  ``table[(n-1) // bs] * bs + (n-1) % bs``;
- physical blocks are scattered over the pool in random order, so the last block of a
  sequence is usually partly filled.

Values are N(0, 1). Generation runs on ``device`` with a generator seeded by ``seed``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass
class DecodeStep:
    name: str
    q: torch.Tensor  # [B, nh, hd]
    k_cache: torch.Tensor  # [num_slots, nkv, hd]
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # [B, W] int32
    context_lens: torch.Tensor  # [B] int32, includes the appended token
    block_size: int
    new_k: torch.Tensor  # [B, nkv, hd] this step's rows
    new_v: torch.Tensor
    slot_mapping: torch.Tensor  # [B] int64
    cow_mapping: torch.Tensor | None = None  # [n, 2] int64 (src, dst) before the append
    info: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes the decode attention reads: sum(ctx) * 2 * nkv * hd * elt."""
        _, nkv, hd = self.k_cache.shape
        total = int(self.context_lens.sum())
        return total * 2 * nkv * hd * self.k_cache.element_size()

    def unique_kv_bytes(self) -> int:
        """K+V bytes of distinct physical slots read (shared prefix blocks count once)."""
        _, nkv, hd = self.k_cache.shape
        bs = self.block_size
        slots = set()
        tabs = self.block_tables.cpu().tolist()
        for row, n in zip(tabs, self.context_lens.cpu().tolist(), strict=True):
            for p in range(0, n, bs):
                blk = row[p // bs]
                for off in range(min(bs, n - p)):
                    slots.add(blk * bs + off)
        return len(slots) * 2 * nkv * hd * self.k_cache.element_size()


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, dtype, device, g) -> torch.Tensor:
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)


def _finish(name, ctx_list, tables_list, width, num_blocks, bs, nh, nkv, hd, dtype, device,
            g, cow=None, info=None) -> DecodeStep:  # fmt: skip
    b = len(ctx_list)
    tables = torch.zeros(b, width, dtype=torch.int32)
    for i, t in enumerate(tables_list):
        tables[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    slots = [t[(n - 1) // bs] * bs + (n - 1) % bs for t, n in zip(tables_list, ctx_list, strict=True)]
    k = _randn((num_blocks * bs, nkv, hd), dtype, device, g)
    v = _randn((num_blocks * bs, nkv, hd), dtype, device, g)
    return DecodeStep(
        name=name,
        q=_randn((b, nh, hd), dtype, device, g),
        k_cache=k,
        v_cache=v,
        block_tables=tables.to(device),
        context_lens=torch.tensor(ctx_list, dtype=torch.int32, device=device),
        block_size=bs,
        new_k=_randn((b, nkv, hd), dtype, device, g),
        new_v=_randn((b, nkv, hd), dtype, device, g),
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        cow_mapping=None if cow is None else torch.tensor(cow, dtype=torch.int64, device=device),
        info=info or {},
    )


def _scattered(ctx_list, bs, pool_factor, width, g) -> tuple[list[list[int]], int]:
    need = [-(-n // bs) for n in ctx_list]
    num_blocks = max(math.ceil(pool_factor * sum(need)), sum(need), width)
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables, at = [], 0
    for k in need:
        tables.append(perm[at : at + k])
        at += k
    return tables, num_blocks


def config1(device="cpu", seed: int = 0) -> DecodeStep:
    """Llama-3.2-1B-shaped layer: B=8, ctx ~ U[32, 512], 32 q heads, 8 KV heads, hd 64,
    fp16, block 16; tables = randperm(256).view(8, 32)."""
    g = torch.Generator().manual_seed(seed)
    gd = _gen(device, seed + 1)
    bs, b = 16, 8
    ctx = torch.randint(32, 513, (b,), generator=g).tolist()
    perm = torch.randperm(256, generator=g).view(b, 32).tolist()
    tables = [row[: -(-n // bs)] for row, n in zip(perm, ctx, strict=True)]
    step = _finish("c1_llama1b_fp16", ctx, tables, 32, 256, bs, 32, 8, 64, torch.float16, device, gd)
    step.block_tables = torch.tensor(perm, dtype=torch.int32, device=device)  # full permutation
    return step


def config2(device="cpu", seed: int = 0, batch: int = 64) -> DecodeStep:
    """Llama-3.2-3B decode: B=64, ctx ~ U[1024, 4096], 24 q heads, 8 KV heads, hd 128,
    bf16, block 16, pool = 1.5x the live blocks, W = 256."""
    g = torch.Generator().manual_seed(seed)
    gd = _gen(device, seed + 1)
    bs = 16
    ctx = torch.randint(1024, 4097, (batch,), generator=g).tolist()
    width = 4096 // bs
    tables, nblk = _scattered(ctx, bs, 1.5, width, g)
    return _finish("c2_llama3b_bf16", ctx, tables, width, nblk, bs, 24, 8, 128, torch.bfloat16,
                   device, gd)  # fmt: skip


def config2_1b(device="cpu", seed: int = 0, batch: int = 64) -> DecodeStep:
    """Config 2's batch and contexts (B=64, ctx ~ U[1024, 4096], bf16, block 16) at the
    Llama-3.2-1B head shape of config 1 (32 q heads, 8 KV heads, hd 64): the head-dim-64
    decode path at a bandwidth-bound size. Not a BASELINE config."""
    g = torch.Generator().manual_seed(seed)
    gd = _gen(device, seed + 1)
    bs = 16
    ctx = torch.randint(1024, 4097, (batch,), generator=g).tolist()
    width = 4096 // bs
    tables, nblk = _scattered(ctx, bs, 1.5, width, g)
    return _finish("c2_llama1b_shape_bf16", ctx, tables, width, nblk, bs, 32, 8, 64,
                   torch.bfloat16, device, gd)  # fmt: skip


def config3(device="cpu", seed: int = 0, batch: int = 256, cow: int = 64) -> DecodeStep:
    """Prefix-shared decode at the 3B shape: every sequence's first 128 table entries are
    the same physical blocks (2,048 shared tokens), then a private tail of U[0, 1024]
    tokens plus the appended one. ``cow`` sequences get the last shared block copied to
    a fresh block (``cow_mapping``) and their table entry repointed before the append."""
    g = torch.Generator().manual_seed(seed)
    gd = _gen(device, seed + 1)
    bs, shared = 16, 128
    tails = torch.randint(0, 1025, (batch,), generator=g).tolist()
    ctx = [shared * bs + t + 1 for t in tails]
    width = shared + -(-(1024 + 1) // bs)
    private = [-(-n // bs) - shared for n in ctx]
    live = shared + sum(private) + cow
    num_blocks = math.ceil(1.5 * live)
    perm = torch.randperm(num_blocks, generator=g).tolist()
    prefix, at = perm[:shared], shared
    tables = []
    for k in private:
        tables.append(prefix + perm[at : at + k])
        at += k
    pairs = []
    for i in range(min(cow, batch)):
        fresh = perm[at]
        at += 1
        pairs.append((prefix[-1], fresh))
        tables[i][shared - 1] = fresh
    return _finish("c3_prefix_shared_bf16", ctx, tables, width, num_blocks, bs, 24, 8, 128,
                   torch.bfloat16, device, gd, cow=pairs or None,
                   info={"shared_blocks": shared})  # fmt: skip


def config4(device="cpu", seed: int = 0, batch: int = 32) -> DecodeStep:
    """Long-context skewed batch at the Llama-3-8B shape: ctx log-uniform in
    [128, 32768], 32 q heads, 8 KV heads, hd 128, bf16, block 16, W = 2048."""
    g = torch.Generator().manual_seed(seed)
    gd = _gen(device, seed + 1)
    bs = 16
    u = torch.rand(batch, generator=g, dtype=torch.float64)
    ctx = torch.exp(math.log(128) + u * (math.log(32768) - math.log(128))).round().long()
    ctx = ctx.clamp(128, 32768).tolist()
    width = 32768 // bs
    tables, nblk = _scattered(ctx, bs, 1.5, width, g)
    return _finish("c4_llama8b_longctx_bf16", ctx, tables, width, nblk, bs, 32, 8, 128,
                   torch.bfloat16, device, gd)  # fmt: skip


def custom(ctx_list, nh, nkv, hd, block_size, dtype, device="cpu", seed: int = 0,
           extra_blocks: int = 3, width: int | None = None) -> DecodeStep:  # fmt: skip
    """Any shape: tables scattered over a pool of B * max_blocks + extra_blocks blocks,
    as the reference's kernel test builds them (reference tests/test_kernels.py:24-33)."""
    g = torch.Generator().manual_seed(seed)
    gd = _gen(device, seed + 1)
    bs = block_size
    max_blocks = max(1, max(-(-max(n, 1) // bs) for n in ctx_list))
    w = width or max_blocks
    nblk = len(ctx_list) * max_blocks + extra_blocks
    perm = torch.randperm(nblk, generator=g).tolist()
    tables = [perm[i * max_blocks : i * max_blocks + -(-max(n, 1) // bs)]
              for i, n in enumerate(ctx_list)]  # fmt: skip
    return _finish(f"custom_{nh}_{nkv}_{hd}_bs{bs}", list(ctx_list), tables, w, nblk, bs, nh,
                   nkv, hd, dtype, device, gd)  # fmt: skip


@dataclass
class MixedStep:
    """A chunked-prefill step: prompt chunks and decode sequences over one pool."""

    name: str
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_size: int
    # prompt chunks
    q_chunks: torch.Tensor  # [T, nh, hd]
    chunk_tables: torch.Tensor  # [C, W] int32
    chunk_ctx: torch.Tensor  # [C] int32 (own tokens included)
    cu_q: torch.Tensor  # [C + 1] int32
    max_query_len: int
    # decode rows
    decode: DecodeStep
    # this step's new K/V rows (chunk tokens, then decode tokens) and their slots
    new_k: torch.Tensor
    new_v: torch.Tensor
    slot_mapping: torch.Tensor
    info: dict = field(default_factory=dict)

    def prefill_flops(self) -> int:
        """Algorithmic FLOPs of the chunk attention: 4 * hd per (query head, visible key)."""
        nh, hd = self.q_chunks.shape[1], self.q_chunks.shape[2]
        pairs = 0
        for c in range(self.chunk_ctx.numel()):
            ql = int(self.cu_q[c + 1] - self.cu_q[c])
            prefix = int(self.chunk_ctx[c]) - ql
            pairs += ql * prefix + ql * (ql + 1) // 2
        return pairs * nh * hd * 4


def config5(device="cpu", seed: int = 0) -> MixedStep:
    """Mixed chunked-prefill step at the Llama-3-8B shape (32 q heads, 8 KV heads, hd
    128, bf16, block 16): 4 prompt chunks of 512 tokens, chunk i after a cached prefix
    of i * 1024 tokens, plus 120 decode sequences with contexts U[256, 2048]."""
    g = torch.Generator().manual_seed(seed)
    gd = _gen(device, seed + 1)
    bs, nh, nkv, hd, dt = 16, 32, 8, 128, torch.bfloat16
    chunk_len = 512
    chunk_ctx = [chunk_len + 1024 * i for i in range(4)]
    dec_ctx = torch.randint(256, 2049, (120,), generator=g).tolist()
    all_ctx = chunk_ctx + dec_ctx
    width = max(-(-n // bs) for n in all_ctx)
    tables, nblk = _scattered(all_ctx, bs, 1.5, width, g)
    k = _randn((nblk * bs, nkv, hd), dt, device, g=gd)
    v = _randn((nblk * bs, nkv, hd), dt, device, g=gd)

    def table_tensor(rows):
        t = torch.zeros(len(rows), width, dtype=torch.int32)
        for i, r in enumerate(rows):
            t[i, : len(r)] = torch.tensor(r, dtype=torch.int32)
        return t.to(device)

    slots = []
    for t, n in zip(tables[:4], chunk_ctx, strict=True):
        slots += [t[p // bs] * bs + p % bs for p in range(n - chunk_len, n)]
    for t, n in zip(tables[4:], dec_ctx, strict=True):
        slots.append(t[(n - 1) // bs] * bs + (n - 1) % bs)
    n_new = len(slots)
    decode = DecodeStep(
        name="c5_decode", q=_randn((120, nh, hd), dt, device, gd), k_cache=k, v_cache=v,
        block_tables=table_tensor(tables[4:]),
        context_lens=torch.tensor(dec_ctx, dtype=torch.int32, device=device), block_size=bs,
        new_k=torch.empty(0), new_v=torch.empty(0),
        slot_mapping=torch.tensor(slots[4 * chunk_len :], dtype=torch.int64, device=device),
    )  # fmt: skip
    return MixedStep(
        name="c5_mixed_llama8b_bf16", k_cache=k, v_cache=v, block_size=bs,
        q_chunks=_randn((4 * chunk_len, nh, hd), dt, device, gd),
        chunk_tables=table_tensor(tables[:4]),
        chunk_ctx=torch.tensor(chunk_ctx, dtype=torch.int32, device=device),
        cu_q=torch.tensor([chunk_len * i for i in range(5)], dtype=torch.int32, device=device),
        max_query_len=chunk_len, decode=decode,
        new_k=_randn((n_new, nkv, hd), dt, device, gd),
        new_v=_randn((n_new, nkv, hd), dt, device, gd),
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
    )  # fmt: skip


CONFIGS = {"c1": config1, "c2": config2, "c3": config3, "c4": config4, "c2_1b": config2_1b}
