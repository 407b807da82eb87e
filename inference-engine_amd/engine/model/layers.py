"""The attention call site of the paged path: what the reference's
``Attention._paged`` / ``Attention._mixed`` (engine/model/layers.py:191-266) do once q,
k and v are projected, on this build's HIP kernels only.

The dispatch follows the reference's order on the same ``PagedBatch`` fields:
``use_kernel`` (a decode step: the decode kernel), then ``mixed`` (decode rows through
the decode kernel, prompt chunks through the chunked-prefill kernel where the reference
gathers for FlashAttention varlen, layers.py:246-253), else the reference's gather path,
which this build does not run. Projections, RoPE, norms and the MLP are the model's and
outside this path.
"""

from __future__ import annotations

import torch

from engine.kernels.paged_attention import paged_decode_attention, paged_prefill_attention
from engine.runtime.paged_cache import PagedBatch


def paged_attention(layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    batch: PagedBatch, out: torch.Tensor | None = None) -> torch.Tensor:  # fmt: skip
    """One layer's paged attention over a step's flattened tokens (reference
    ``Attention._paged``, layers.py:191-225).

    q: [N, nh, hd]; k, v: [N, nkv, hd] (token-major; the reference passes the same data
    head-major and transposes, layers.py:200). Appends k, v at ``batch.slot_mapping``
    (HIP append), then runs the decode kernel for decode batches (with cascade over
    shared prefixes when the batch carries ``prefix_groups``) or ``mixed_attention``
    for mixed ones. ``out`` ([N, nh, hd]) receives the result in place. Returns
    [N, nh * hd].
    """
    cache = batch.cache
    cache.write(layer_idx, k, v, batch.slot_mapping)
    if batch.use_kernel:
        res = paged_decode_attention(q, cache.k[layer_idx], cache.v[layer_idx],
                                     batch.block_tables, batch.context_lens, cache.block_size,
                                     out=out, prefix_groups=batch.prefix_groups)  # fmt: skip
        return res.flatten(1)
    if batch.mixed:
        return mixed_attention(layer_idx, q, batch, out=out)
    raise ValueError("paged_attention: a gather batch (PagedBatch.build(use_kernel=False)) "
                     "is the reference's PyTorch path; build with use_kernel=True")  # fmt: skip


def mixed_attention(layer_idx: int, q: torch.Tensor, batch: PagedBatch,
                    out: torch.Tensor | None = None) -> torch.Tensor:  # fmt: skip
    """Attention of a mixed step whose K/V are already written (reference
    ``Attention._mixed``, layers.py:227-266): decode rows through the decode kernel,
    every prompt chunk through the chunked-prefill kernel (all dtypes and head sizes; the
    reference's ``chunks`` list of per-chunk SDPA calls stays empty). q: [N, nh, hd];
    ``out`` ([N, nh, hd]) receives the result in place. Returns [N, nh * hd]."""
    if batch.chunks:
        raise ValueError("mixed_attention: per-chunk SDPA entries (PagedBatch.chunks) "
                         "belong to the reference's gather path")  # fmt: skip
    cache = batch.cache
    kc, vc, bs = cache.k[layer_idx], cache.v[layer_idx], cache.block_size
    if out is None:
        out = torch.empty_like(q)
    if batch.block_tables is not None:
        rows = batch.decode_rows
        out[rows] = paged_decode_attention(q[rows], kc, vc, batch.block_tables,
                                           batch.context_lens, bs).to(out.dtype)  # fmt: skip
    if batch.chunk_rows is not None:
        rows = batch.chunk_rows
        out[rows] = paged_prefill_attention(q[rows], kc, vc, batch.chunk_tables,
                                            batch.chunk_ctx, bs, batch.cu_seqlens_q,
                                            batch.max_query_len).to(out.dtype)  # fmt: skip
    return out.flatten(1)
