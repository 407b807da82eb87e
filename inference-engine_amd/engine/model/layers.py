"""The attention call site of the paged path: what the reference's
``Attention._paged`` / ``Attention._mixed`` (engine/model/layers.py:191-266) do once q,
k and v are projected, on this build's HIP kernels only.

Only the KV and attention work lives here; projections, RoPE, norms and the MLP are the
model's and outside this path.
"""

from __future__ import annotations

import torch

from engine.kernels.paged_attention import (
    PREFILL_HEAD_DIMS,
    paged_decode_attention,
    paged_prefill_attention,
)
from engine.runtime.paged_cache import PagedBatch


def paged_attention(layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    batch: PagedBatch, out: torch.Tensor | None = None) -> torch.Tensor:  # fmt: skip
    """One layer's paged attention over a step's flattened tokens.

    q: [N, nh, hd]; k, v: [N, nkv, hd] (token-major; the reference passes the same data
    head-major and transposes, layers.py:200). Appends k, v at ``batch.slot_mapping``
    (HIP append), then:
      * decode steps: the decode kernel over ``block_tables`` / ``context_lens``
        (reference layers.py:201-212), with cascade over shared prefixes when the batch
        carries ``prefix_groups``;
      * mixed steps: decode rows through the decode kernel and prompt chunks through
        the chunked-prefill kernel (reference layers.py:227-266, where chunks go to
        FlashAttention varlen or per-chunk SDPA). Chunk shapes the prefill kernel does
        not take (fp32, head_dim 16) use the decode kernel once per chunk token, each
        seeing its causal prefix: the same attention, the K/V re-read per token.
    ``out`` ([N, nh, hd]) receives the result in place. Returns [N, nh * hd].
    """
    cache = batch.cache
    cache.write(layer_idx, k, v, batch.slot_mapping)
    kc, vc, bs = cache.k[layer_idx], cache.v[layer_idx], cache.block_size
    if not batch.mixed:
        res = paged_decode_attention(q, kc, vc, batch.block_tables, batch.context_lens, bs,
                                     out=out, prefix_groups=batch.prefix_groups)  # fmt: skip
        return res.flatten(1)
    if out is None:
        out = torch.empty_like(q)
    if batch.decode_rows is not None:
        rows = batch.decode_rows
        out[rows] = paged_decode_attention(q[rows], kc, vc, batch.block_tables,
                                           batch.context_lens, bs).to(out.dtype)  # fmt: skip
    if batch.chunk_rows is not None:
        rows = batch.chunk_rows
        if q.dtype in (torch.bfloat16, torch.float16) and q.shape[-1] in PREFILL_HEAD_DIMS:
            res = paged_prefill_attention(q[rows], kc, vc, batch.chunk_tables, batch.chunk_ctx,
                                          bs, batch.cu_seqlens_q, batch.max_query_len)  # fmt: skip
        else:
            res = paged_decode_attention(q[rows], kc, vc, batch.row_tables, batch.row_ctx, bs)
        out[rows] = res.to(out.dtype)
    return out.flatten(1)
