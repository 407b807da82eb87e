"""Python face of the C oracle (oracle/paged_kv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline, never by the product path.

All functions take CPU torch tensors (bf16/fp16 as raw 16-bit storage) and call the C
restatement. Reference functions restated (file:line in the reference repository):

- ``kv_append``: PagedKVCache.write, engine/runtime/paged_cache.py:42-45
- ``decode_attention``: reference_decode_attention, engine/kernels/paged_attention.py:192-211
- ``prefill_attention``: the bottom-right causal chunk attention of PagedBatch._mixed /
  Attention._mixed, engine/runtime/paged_cache.py:182-194, engine/model/layers.py:246-265
- ``copy_blocks``, ``decode_partials``, ``combine``: build-defined (no reference code);
  pinned by slice equality and by the combine == single-pass identity.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libpkv_oracle.so")
DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_p, _i64, _i32, _int, _dbl = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int,
                              ctypes.c_double)  # fmt: skip
_SIG = {
    "or_kv_append": (None, [_p, _p, _int, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64,
                            _int, _p, _i64, _int, _int]),
    "or_copy_blocks": (None, [_p, _p, _i64, _int, _i64, _i64, _p, _i64]),
    "or_decode_attention": (_int, [_p, _p, _i64, _i64, _p, _p, _int, _i64, _i64, _p, _i64, _p,
                                   _int, _int, _int, _int, _int, _dbl, _int]),
    "or_decode_partials": (_int, [_p, _p, _p, _i64, _i64, _p, _p, _int, _i64, _i64, _p, _i64,
                                  _p, _int, _int, _int, _int, _int, _dbl, _int, _int]),
    "or_combine": (None, [_p, _p, _p, _i64, _int, _int]),
    "or_prefill_attention": (_int, [_p, _p, _i64, _i64, _p, _p, _int, _i64, _i64, _p, _i64,
                                    _p, _p, _int, _int, _int, _int, _int, _dbl, _int]),
    "or_cvt_f32_to_bf16_n": (None, [_p, _p, _i64]),
    "or_cvt_f32_to_f16_n": (None, [_p, _p, _i64]),
    "or_cvt_f16_to_f32_n": (None, [_p, _p, _i64]),
    "or_cvt_bf16_to_f32_n": (None, [_p, _p, _i64]),
}  # fmt: skip
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from oracle import build as _build  # noqa: PLC0415

            _build.build()
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def _cpu(t: torch.Tensor) -> torch.Tensor:
    if t.device.type != "cpu":
        raise ValueError("oracle functions take CPU tensors")
    return t


# ---- conversions -------------------------------------------------------------------


def to_bf16_bits(x: torch.Tensor) -> torch.Tensor:
    """float32 -> bfloat16 bit patterns (int16 tensor), round to nearest even."""
    x = _cpu(x).contiguous().float()
    y = torch.empty(x.shape, dtype=torch.int16)
    lib().or_cvt_f32_to_bf16_n(x.data_ptr(), y.data_ptr(), x.numel())
    return y


def to_f16_bits(x: torch.Tensor) -> torch.Tensor:
    x = _cpu(x).contiguous().float()
    y = torch.empty(x.shape, dtype=torch.int16)
    lib().or_cvt_f32_to_f16_n(x.data_ptr(), y.data_ptr(), x.numel())
    return y


def from_f16_bits(x: torch.Tensor) -> torch.Tensor:
    x = _cpu(x).contiguous()
    y = torch.empty(x.shape, dtype=torch.float32)
    lib().or_cvt_f16_to_f32_n(x.data_ptr(), y.data_ptr(), x.numel())
    return y


def from_bf16_bits(x: torch.Tensor) -> torch.Tensor:
    x = _cpu(x).contiguous()
    y = torch.empty(x.shape, dtype=torch.float32)
    lib().or_cvt_bf16_to_f32_n(x.data_ptr(), y.data_ptr(), x.numel())
    return y


# ---- KV append and block copy ----------------------------------------------------------


def kv_append(k_pool, v_pool, k, v, slots) -> None:
    """In place: pool[slots[i]] = k[i] converted to the pool dtype (one layer's pools
    [num_slots, nkv, hd]); slots outside the pool are skipped."""
    for t in (k_pool, v_pool, k, v, slots):
        _cpu(t)
    assert k_pool.stride(2) == 1 and k.stride(2) == 1 and v.stride(2) == 1
    assert k_pool.stride() == v_pool.stride()
    slots = slots.contiguous()
    lib().or_kv_append(
        k_pool.data_ptr(), v_pool.data_ptr(), DT[k_pool.dtype], k_pool.stride(0),
        k_pool.stride(1), k_pool.shape[0], k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), DT[k.dtype], slots.data_ptr(),
        slots.numel(), k_pool.shape[1], k_pool.shape[2],
    )  # fmt: skip


def copy_blocks(k_pool, v_pool, mapping, block_size: int) -> None:
    """In place, pools [L, slots, nkv, hd] (contiguous): block dst = block src, every
    layer, pairs applied in order."""
    _cpu(k_pool), _cpu(v_pool), _cpu(mapping)
    if k_pool.dim() == 3:
        k_pool, v_pool = k_pool[None], v_pool[None]
    assert k_pool.is_contiguous() and v_pool.is_contiguous()
    layers, slots, nkv, hd = k_pool.shape
    elt = k_pool.element_size()
    mapping = mapping.contiguous()
    lib().or_copy_blocks(k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0) * elt, layers,
                         block_size * nkv * hd * elt, slots // block_size, mapping.data_ptr(),
                         mapping.shape[0])  # fmt: skip


# ---- attention ---------------------------------------------------------------------------


def decode_attention(q, k_cache, v_cache, block_tables, context_lens, block_size: int,
                     scale: float | None = None, threads: int = 0) -> torch.Tensor:  # fmt: skip
    """fp32 [B, nh, hd]: softmax(scale q.K^T) V over each sequence's paged context."""
    for t in (q, k_cache, v_cache, block_tables, context_lens):
        _cpu(t)
    b, nh, hd = q.shape
    assert q.dtype == k_cache.dtype == v_cache.dtype and q.stride(2) == 1
    assert k_cache.stride() == v_cache.stride() and k_cache.stride(2) == 1
    assert block_tables.dtype == torch.int32 and context_lens.dtype == torch.int32
    assert block_tables.stride(1) == 1
    ctx = context_lens.contiguous()
    out = torch.empty(b, nh, hd, dtype=torch.float32)
    rc = lib().or_decode_attention(
        out.data_ptr(), q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(),
        v_cache.data_ptr(), DT[q.dtype], k_cache.stride(0), k_cache.stride(1),
        block_tables.data_ptr(), block_tables.stride(0), ctx.data_ptr(), b, nh,
        k_cache.shape[1], hd, block_size, hd**-0.5 if scale is None else scale, threads,
    )  # fmt: skip
    if rc:
        raise ValueError(f"or_decode_attention rejected its arguments ({rc})")
    return out


def decode_partials(q, k_cache, v_cache, block_tables, context_lens, block_size: int,
                    split_tokens: int, n_splits: int, scale: float | None = None):  # fmt: skip
    """Per-split softmax states: ml float64 [B, nh, S, 2] (max, sum), acc [B, nh, S, hd]."""
    b, nh, hd = q.shape
    ctx = context_lens.contiguous()
    ml = torch.empty(b, nh, n_splits, 2, dtype=torch.float64)
    acc = torch.empty(b, nh, n_splits, hd, dtype=torch.float64)
    rc = lib().or_decode_partials(
        ml.data_ptr(), acc.data_ptr(), q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), DT[q.dtype], k_cache.stride(0),
        k_cache.stride(1), block_tables.data_ptr(), block_tables.stride(0), ctx.data_ptr(),
        b, nh, k_cache.shape[1], hd, block_size, hd**-0.5 if scale is None else scale,
        split_tokens, n_splits,
    )  # fmt: skip
    if rc:
        raise ValueError(f"or_decode_partials rejected its arguments ({rc})")
    return ml, acc


def combine(ml: torch.Tensor, acc: torch.Tensor) -> torch.Tensor:
    """Log-sum-exp merge of split states along dim -2 -> fp32 [..., hd]."""
    *lead, s, hd = acc.shape
    ml, acc = ml.contiguous(), acc.contiguous()
    rows = 1
    for x in lead:
        rows *= x
    out = torch.empty(*lead, hd, dtype=torch.float32)
    lib().or_combine(out.data_ptr(), ml.data_ptr(), acc.data_ptr(), rows, s, hd)
    return out


def prefill_attention(q, k_cache, v_cache, block_tables, cu_q, context_lens,
                      block_size: int, scale: float | None = None,
                      threads: int = 0) -> torch.Tensor:  # fmt: skip
    """fp32 [T, nh, hd] for prompt chunks back to back: chunk c has query rows
    [cu_q[c], cu_q[c+1]) and context context_lens[c] through table row c; query i of a
    chunk of length n sits at position ctx - n + i and sees keys 0..ctx - n + i."""
    t, nh, hd = q.shape
    assert q.stride(2) == 1 and cu_q.dtype == torch.int32 and context_lens.dtype == torch.int32
    cu_q, ctx = cu_q.contiguous(), context_lens.contiguous()
    out = torch.empty(t, nh, hd, dtype=torch.float32)
    rc = lib().or_prefill_attention(
        out.data_ptr(), q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(),
        v_cache.data_ptr(), DT[q.dtype], k_cache.stride(0), k_cache.stride(1),
        block_tables.data_ptr(), block_tables.stride(0), cu_q.data_ptr(), ctx.data_ptr(),
        ctx.numel(), nh, k_cache.shape[1], hd, block_size,
        hd**-0.5 if scale is None else scale, threads,
    )  # fmt: skip
    if rc:
        raise ValueError(f"or_prefill_attention rejected its arguments ({rc})")
    return out
