"""Fused element-wise kernels beside the paged path: RMSNorm tail, in-place RoPE and
SiLU-and-multiply, one HIP launch each (csrc/fused.hip through lib/libpaged_kv.so).
Same names, signatures and contract as the reference's ``engine/kernels/fused.py``
(:38-131): every result is bitwise identical to the PyTorch ops it replaces, rounding
where they round, with the device library's exp and IEEE division and no multiply-add
contraction. RMSNorm leaves the per-row scale rsqrt(mean(x^2) + eps) to PyTorch: the
reference leaves it the mean (a fused sum adds in another order), and on ROCm PyTorch's
rsqrt can differ from the device library's in the last fp32 bit.
"""

from __future__ import annotations

import os

import torch

from engine.kernels import _native

# ENGINE_FUSED_KERNELS=0 makes callers use the plain PyTorch ops (for comparisons).
ENABLED = os.environ.get("ENGINE_FUSED_KERNELS", "1") != "0"


def available(t: torch.Tensor) -> bool:
    """Reference :41-42: enabled, on a GPU, and the HIP library loads."""
    if not (ENABLED and t.is_cuda):
        return False
    try:
        _native.lib()
    except (RuntimeError, OSError):
        return False
    return True


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """weight * (x_fp32 * rsqrt(mean(x_fp32^2) + eps)).to(x.dtype) over the last dim
    (reference :93-111)."""
    what = "rms_norm"
    dev = _native.require_gpu(what, x, weight)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    weight = weight.contiguous()
    if weight.shape != (shape[-1],):
        raise ValueError(f"{what}: weight {tuple(weight.shape)} for rows of {shape[-1]}")
    inv = torch.rsqrt(x2.float().pow(2).mean(-1) + eps)
    out = torch.empty(x2.shape, dtype=torch.promote_types(weight.dtype, x.dtype), device=dev)
    status = _native.lib().pkv_rms_norm(
        out.data_ptr(), _native.dtype_code(out.dtype, what), out.stride(0),
        x2.data_ptr(), _native.dtype_code(x.dtype, what), x2.stride(0), inv.data_ptr(),
        weight.data_ptr(), _native.dtype_code(weight.dtype, what), x2.shape[0], x2.shape[1],
        _native.stream_of(dev))  # fmt: skip
    _native.check(status, what)
    return out.view(shape)


def rope_(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> None:
    """In place: x [N, heads, hd] (unit stride in hd), cos / sin [N, hd] float32
    (reference :114-121)."""
    what = "rope_"
    dev = _native.require_gpu(what, x, cos, sin)
    if x.dim() != 3 or x.stride(-1) != 1:
        raise ValueError(f"{what}: x must be [N, heads, hd] with unit stride in hd")
    n, heads, hd = x.shape
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise TypeError(f"{what}: cos and sin must be float32")
    if cos.shape != (n, hd) or sin.shape != cos.shape or cos.stride() != sin.stride() \
            or cos.stride(-1) != 1:  # fmt: skip
        raise ValueError(f"{what}: cos, sin must be equal [N, hd] tensors, unit stride in hd")
    status = _native.lib().pkv_rope(
        x.data_ptr(), _native.dtype_code(x.dtype, what), x.stride(0), x.stride(1),
        cos.data_ptr(), sin.data_ptr(), cos.stride(0), n, heads, hd,
        _native.stream_of(dev))  # fmt: skip
    _native.check(status, what)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """F.silu(gate) * up, each rounded to the input dtype as PyTorch does
    (reference :124-131)."""
    what = "silu_mul"
    dev = _native.require_gpu(what, gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError(f"{what}: gate and up must match in shape and dtype")
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    status = _native.lib().pkv_silu_mul(
        out.data_ptr(), gate.data_ptr(), up.data_ptr(), _native.dtype_code(gate.dtype, what),
        gate.numel(), _native.stream_of(dev))  # fmt: skip
    _native.check(status, what)
    return out
