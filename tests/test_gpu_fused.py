"""Fused element-wise kernels (RMSNorm tail, RoPE, SiLU x up) through the C ABI: bitwise
identical to the PyTorch ops they replace, as the reference's
tests/test_kernels.py:218-254 require of its Triton kernels."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from engine.kernels import fused

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(*a):
    print("[case]", *a, flush=True)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("nh", "hd"), [(8, 64), (32, 128), (3, 16), (5, 12)])
def test_rope_is_bitwise_identical(dtype, nh, hd):
    """HF's q * cos + rotate_half(q) * sin with cos / sin cast to the model dtype (hd 12:
    half a row is not a whole 16-byte access, so the per-element kernel runs)."""
    _say("rope", dtype, nh, hd)
    g = torch.Generator(device=DEV).manual_seed(0)
    n = 77
    q = torch.randn(n, nh, hd, device=DEV, generator=g).to(dtype)
    pos = torch.arange(n, device=DEV) * 37
    inv = 1.0 / (500000 ** (torch.arange(0, hd, 2, device=DEV).float() / hd))
    emb = torch.cat([pos[:, None].float() * inv] * 2, -1)
    cos, sin = emb.cos(), emb.sin()
    want = q * cos[:, None].to(dtype) + _rotate_half(q) * sin[:, None].to(dtype)
    got = q.clone()
    fused.rope_(got, cos, sin)
    assert torch.equal(got, want)


def test_rope_strided_heads_in_place():
    """q and k as views of one projection output (head stride > hd)."""
    _say("rope strided")
    g = torch.Generator(device=DEV).manual_seed(1)
    n, nh, nkv, hd = 19, 8, 2, 64
    qkv = torch.randn(n, (nh + 2 * nkv) * hd, device=DEV, generator=g).to(torch.bfloat16)
    k = qkv[:, nh * hd : (nh + nkv) * hd].view(n, nkv, hd)
    before = qkv.clone()
    emb = torch.randn(n, hd, device=DEV, generator=g)
    cos, sin = emb.cos(), emb.sin()
    want = k * cos[:, None].to(k.dtype) + _rotate_half(k) * sin[:, None].to(k.dtype)
    fused.rope_(k, cos, sin)
    assert torch.equal(k, want)
    # nothing outside k changed
    assert torch.equal(qkv[:, : nh * hd], before[:, : nh * hd])
    assert torch.equal(qkv[:, (nh + nkv) * hd :], before[:, (nh + nkv) * hd :])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(64, 1000), (7, 999)])
def test_silu_mul_is_bitwise_identical(dtype, shape):
    """(7, 999): an element count that is no whole number of 16-byte accesses."""
    _say("silu_mul", dtype, shape)
    g = torch.Generator(device=DEV).manual_seed(2)
    gate = (torch.randn(*shape, device=DEV, generator=g) * 4).to(dtype)
    up = torch.randn(*shape, device=DEV, generator=g).to(dtype)
    gate[0, :6] = torch.tensor([0.0, -0.0, 88.0, -88.0, 1e-30, -1e-30]).to(dtype)
    assert torch.equal(fused.silu_mul(gate, up), F.silu(gate) * up)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim", [2048, 3072, 100, 1000])
def test_rms_norm_is_bitwise_identical(dtype, dim):
    """Reference tests/test_kernels.py:240-254."""
    _say("rms_norm", dtype, dim)
    g = torch.Generator(device=DEV).manual_seed(3)
    x = (torch.randn(300, dim, device=DEV, generator=g) * 3).to(dtype)
    w = torch.randn(dim, device=DEV, generator=g).to(dtype)
    xf = x.float()
    want = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(x.dtype)
    assert torch.equal(fused.rms_norm(x, w, 1e-5), want)


def test_rms_norm_mixed_dtypes_and_shapes():
    """fp32 weight on bf16 activations (promotes to fp32), 3-D input, strided rows."""
    _say("rms_norm mixed")
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(4, 33, 256, device=DEV, generator=g).to(torch.bfloat16)
    w = torch.randn(256, device=DEV, generator=g)
    xf = x.float()
    want = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype)
    got = fused.rms_norm(x, w, 1e-6)
    assert got.dtype == torch.float32 and torch.equal(got, want)
    xs = torch.randn(50, 512, device=DEV, generator=g).to(torch.float16)[:, :300]
    ws = torch.randn(300, device=DEV, generator=g).to(torch.float16)
    xsf = xs.float()
    want = ws * (xsf * torch.rsqrt(xsf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(xs.dtype)
    assert torch.equal(fused.rms_norm(xs, ws, 1e-5), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_misaligned_views_take_the_per_element_path(dtype):
    """Views one element off a 16-byte boundary cannot use the 16-byte kernels; the
    per-element ones run and stay bitwise identical to PyTorch."""
    _say("fused misaligned", dtype)
    g = torch.Generator(device=DEV).manual_seed(5)
    # SiLU x up on flat views starting one element in
    base_g = (torch.randn(8 * 512 + 1, device=DEV, generator=g) * 4).to(dtype)
    base_u = torch.randn(8 * 512 + 1, device=DEV, generator=g).to(dtype)
    gate, up = base_g[1:], base_u[1:]
    assert torch.equal(fused.silu_mul(gate, up), F.silu(gate) * up)
    # RMSNorm over rows whose first element is misaligned
    xb = (torch.randn(40 * 256 + 1, device=DEV, generator=g) * 3).to(dtype)
    x = xb[1:].view(40, 256)
    w = torch.randn(257, device=DEV, generator=g).to(dtype)[1:]
    xf = x.float()
    want = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(dtype)
    assert torch.equal(fused.rms_norm(x, w, 1e-5), want)
    # RoPE on a head view starting one element in
    n, nh, hd = 9, 4, 64
    qb = torch.randn(n * nh * hd + 1, device=DEV, generator=g).to(dtype)
    q = qb[1:].view(n, nh, hd)
    emb = torch.randn(n, hd, device=DEV, generator=g)
    cos, sin = emb.cos(), emb.sin()
    want_q = q * cos[:, None].to(dtype) + _rotate_half(q) * sin[:, None].to(dtype)
    fused.rope_(q, cos, sin)
    assert torch.equal(q, want_q)
