"""Paged KV pool with a HIP append and block copy; the layout and ``write`` signature of
the reference's ``engine/runtime/paged_cache.py`` (``PagedKVCache``, :22-49).

The pool is one flat array of slots per layer: k, v are [layers, num_blocks *
block_size, nkv, hd]; slot ``s`` of block ``b`` is row ``b * block_size + s``. A whole
block of one layer is a contiguous [block_size, nkv, hd] span, which is what the
decode kernel streams and what ``copy_blocks`` moves.
"""

from __future__ import annotations

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
        the pool are skipped rather than faulting the GPU.
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
    block_mapping = block_mapping.contiguous()
    status = _native.lib().pkv_copy_blocks(
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0) * elt, layers,
        block_size * nkv * hd * elt, slots // block_size, block_mapping.data_ptr(), n,
        _native.stream_of(dev),
    )  # fmt: skip
    _native.check(status, what)
