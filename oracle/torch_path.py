"""The reference's CPU path for one decode layer-step, restated with PyTorch CPU ops.

BASELINE INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it on the host cores;
nothing in the product imports it. It is not the checker (the C oracle is).

What the reference does for a decode layer-step when no GPU kernel runs:

- append: ``PagedKVCache.write`` (reference engine/runtime/paged_cache.py:42-45), one
  ``index_copy_`` of the new K rows and one of the V rows into the layer's pools;
- attention: ``reference_decode_attention`` (reference
  engine/kernels/paged_attention.py:192-211): per sequence, gather its context slots
  through the block table, upcast to fp32, repeat each KV head for its query group,
  softmax(q . K^T * hd^-0.5) . V, and cast to q's dtype.
"""

from __future__ import annotations

import torch


def append(k_pool, v_pool, new_k, new_v, slots) -> None:
    """index_copy_ of this step's K and V rows into one layer's pools."""
    k_pool.index_copy_(0, slots, new_k.to(k_pool.dtype))
    v_pool.index_copy_(0, slots, new_v.to(v_pool.dtype))


def decode_attention(q, k_pool, v_pool, block_tables, context_lens, block_size) -> torch.Tensor:
    """[B, nh, hd] in q.dtype: each sequence's gathered context, fp32 softmax attention."""
    b, nh, hd = q.shape
    groups = nh // k_pool.shape[1]
    scale = hd**-0.5
    out = torch.empty_like(q)
    for i in range(b):
        n = int(context_lens[i])
        pos = torch.arange(n)
        slots = block_tables[i, pos // block_size].long() * block_size + pos % block_size
        k = k_pool[slots].float().repeat_interleave(groups, dim=1)  # [n, nh, hd]
        v = v_pool[slots].float().repeat_interleave(groups, dim=1)
        qi = q[i].float()  # [nh, hd]
        w = torch.softmax(torch.einsum("hd,nhd->hn", qi, k) * scale, dim=-1)
        out[i] = torch.einsum("hn,nhd->hd", w, v).to(q.dtype)
    return out


def decode_layer_step(q, k_pool, v_pool, block_tables, context_lens, block_size, new_k,
                      new_v, slots) -> torch.Tensor:  # fmt: skip
    """The append, then the attention: one layer of a decode step."""
    append(k_pool, v_pool, new_k, new_v, slots)
    return decode_attention(q, k_pool, v_pool, block_tables, context_lens, block_size)
