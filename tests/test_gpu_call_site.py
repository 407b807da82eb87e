"""The reference's attention call site, unchanged apart from its varlen line, on this
build's ``PagedBatch`` and HIP kernels.

``reference_dispatch`` below follows the reference's ``Attention._paged`` /
``Attention._mixed`` (engine/model/layers.py:191-266) step for step on the same fields:
head-major q [nh, N, hd] and k, v [nkv, N, hd] as the reference passes them; the cache
write with transposed k, v; ``use_kernel`` -> decode kernel; ``mixed`` -> decode rows
(``block_tables`` not None), then ``varlen`` (None here), then the loop over ``chunks``
(empty here); else the gather path. The one line this build changes is the varlen call
(layers.py:246-253), which becomes ``paged_prefill_attention`` over the chunk fields.
Results are checked against the oracle: decode rows and chunk rows separately.
"""

from __future__ import annotations

import os

import pytest
import torch

from engine.kernels.paged_attention import paged_decode_attention, paged_prefill_attention
from engine.runtime.paged_cache import KVShape, PagedBatch, PagedKVCache
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
THREADS = min(16, os.cpu_count() or 1)


def reference_dispatch(layer: int, q, k, v, batch: PagedBatch):
    """Reference layers.py:191-266 in its own order, the varlen line swapped."""
    batch.cache.write(layer, k.transpose(0, 1), v.transpose(0, 1), batch.slot_mapping)
    if batch.use_kernel:
        out = paged_decode_attention(q.transpose(0, 1), batch.cache.k[layer],
                                     batch.cache.v[layer], batch.block_tables,
                                     batch.context_lens, batch.cache.block_size)  # fmt: skip
        return out.flatten(1)
    if batch.mixed:
        cache = batch.cache
        qt = q.transpose(0, 1)
        out = torch.empty_like(qt)
        if batch.block_tables is not None:
            rows = batch.decode_rows
            out[rows] = paged_decode_attention(
                qt[rows].contiguous(), cache.k[layer], cache.v[layer], batch.block_tables,
                batch.context_lens, cache.block_size).to(out.dtype)  # fmt: skip
        assert batch.varlen is None  # the reference's FlashAttention inputs: never built
        if batch.chunk_rows is not None:  # the swapped line (reference :246-253)
            rows = batch.chunk_rows
            out[rows] = paged_prefill_attention(
                qt[rows], cache.k[layer], cache.v[layer], batch.chunk_tables, batch.chunk_ctx,
                cache.block_size, batch.cu_seqlens_q, batch.max_query_len).to(out.dtype)  # fmt: skip
        for _ in batch.chunks:
            raise AssertionError("per-chunk SDPA entries: the reference's gather path")
        return out.flatten(1)
    raise AssertionError("gather path: not reached with use_kernel=True")


def _case(dtype, nh, nkv, hd, bs, qlens, ctxs, seed):
    g = torch.Generator().manual_seed(seed)
    cache = PagedKVCache(KVShape(2, nkv, hd), 64, bs, DEV, dtype)
    cache.k.copy_(torch.randn(cache.k.shape, generator=g).to(dtype))
    cache.v.copy_(torch.randn(cache.v.shape, generator=g).to(dtype))
    perm = torch.randperm(64, generator=g).tolist()
    tables, at = [], 0
    for n in ctxs:
        nb = -(-n // bs)
        tables.append(perm[at : at + nb])
        at += nb
    n_tok = sum(qlens)
    q = torch.randn(nh, n_tok, hd, generator=g).to(dtype)
    k = torch.randn(nkv, n_tok, hd, generator=g).to(dtype)
    v = torch.randn(nkv, n_tok, hd, generator=g).to(dtype)
    return cache, tables, q, k, v


def _expected(cache, layer, tables, ctxs, qlens, q):
    """The oracle per sequence: a decode row over its whole context, a chunk's rows
    bottom-right causal over theirs. Returns [N, nh, hd] fp32 in flattened order."""
    kc, vc = cache.k[layer].cpu(), cache.v[layer].cpu()
    bs = cache.block_size
    qt = q.transpose(0, 1).contiguous().cpu()
    outs, start = [], 0
    for t, n, ql in zip(tables, ctxs, qlens, strict=True):
        tab = torch.tensor([t], dtype=torch.int32)
        rows = qt[start : start + ql]
        if ql == 1:
            outs.append(oracle.decode_attention(rows, kc, vc, tab, torch.tensor([n], dtype=torch.int32),
                                                bs, threads=THREADS))  # fmt: skip
        else:
            outs.append(oracle.prefill_attention(rows, kc, vc, tab,
                                                 torch.tensor([0, ql], dtype=torch.int32),
                                                 torch.tensor([n], dtype=torch.int32), bs,
                                                 threads=THREADS))  # fmt: skip
        start += ql
    return torch.cat(outs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize(("nh", "nkv", "hd", "bs"), [(4, 2, 16, 4), (8, 2, 64, 16), (24, 8, 128, 16)])
@pytest.mark.parametrize("kind", ["decode", "mixed", "one_prompt", "chunks_only"])
def test_reference_call_site_dispatch(dtype, nh, nkv, hd, bs, kind):
    """Decode batches, mixed batches (decode rows + a later chunk + a whole prompt), a
    single sequence's prompt and a step of chunks only, through the reference's dispatch
    order: within 2e-3 of the oracle (fp32: 1e-4, the reference's fp32 tolerance)."""
    print("[case] call site", dtype, nh, nkv, hd, bs, kind, flush=True)
    qlens, ctxs = {
        "decode": ([1, 1, 1], [37, 1, 130]),
        "mixed": ([1, 5, 1, 9], [40, 21, 3, 9]),
        "one_prompt": ([23], [23]),
        "chunks_only": ([7, 3], [30, 3]),
    }[kind]
    cache, tables, q, k, v = _case(dtype, nh, nkv, hd, bs, qlens, ctxs, seed=hd + bs)
    batch = PagedBatch.build(cache, tables, ctxs, qlens, DEV, use_kernel=True)
    assert batch.use_kernel == (kind == "decode") and batch.mixed == (kind != "decode")
    got = reference_dispatch(1, q.to(DEV), k.to(DEV), v.to(DEV), batch)
    torch.cuda.synchronize()
    assert got.shape == (sum(qlens), nh * hd) and got.dtype == dtype
    want = _expected(cache, 1, tables, ctxs, qlens, q).reshape(sum(qlens), nh * hd)
    tol = 1e-4 if dtype == torch.float32 else 2e-3 + 2.0**-8 * want.abs().max().item()
    assert (got.float().cpu() - want).abs().max().item() <= tol
    # The build's own call site gives the same bits.
    from engine.model.layers import paged_attention

    again = paged_attention(1, q.transpose(0, 1).contiguous().to(DEV),
                            k.transpose(0, 1).contiguous().to(DEV),
                            v.transpose(0, 1).contiguous().to(DEV), batch)  # fmt: skip
    assert torch.equal(again, got)


def test_gather_batches_are_refused_by_the_kernel_call_site():
    from engine.model.layers import paged_attention

    cache = PagedKVCache(KVShape(1, 2, 16), 8, 4, DEV, torch.float32)
    batch = PagedBatch.build(cache, [[1, 2]], [6], [6], DEV)  # use_kernel=False
    with pytest.raises(ValueError):
        paged_attention(0, torch.zeros(6, 4, 16, device=DEV), torch.zeros(6, 2, 16, device=DEV),
                        torch.zeros(6, 2, 16, device=DEV), batch)  # fmt: skip
