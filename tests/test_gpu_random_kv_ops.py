"""Seeded random shapes for the byte-exact kernels, through the C ABI: the KV append
(pool and new dtypes, head sizes off the 16-byte path, head-major and token-major new
rows, skipped slots), the block copy (layers, block sizes, pairs that fan one source out
or point past the pool) and the fused element-wise kernels (RoPE, SiLU x up, RMSNorm
tail), each bit for bit against the oracle or the PyTorch ops the reference runs. Each
case prints its shape first. PKV_RANDOM_CASES_SCALE=N multiplies the number of seeds."""

from __future__ import annotations

import os
import random

import pytest
import torch
import torch.nn.functional as F

from engine.kernels import fused
from engine.runtime.paged_cache import KVShape, PagedKVCache, kv_append
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SCALE = max(1, int(os.environ.get("PKV_RANDOM_CASES_SCALE", "1")))
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _say(*a):
    print("[case]", *a, flush=True)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.uint8)


@pytest.mark.parametrize("seed", range(24 * SCALE))
def test_append_random(seed):
    r = random.Random(3000 + seed)
    pool_dt, new_dt = r.choice(DTYPES), r.choice(DTYPES)
    hd = r.choice([1, 6, 12, 16, 40, 64, 96, 128, 256])
    nkv = r.choice([1, 2, 3, 8])
    nslots = r.choice([16, 500, 4096])
    n = r.choice([0, 1, r.randint(2, 16), r.randint(16, nslots)])
    head_major = r.random() < 0.5  # the call site's transposes of [nkv, N, hd] projections
    skipped = r.choice([0, 0, r.randint(0, n)])
    _say("append", seed, dict(pool=pool_dt, new=new_dt, hd=hd, nkv=nkv, nslots=nslots, n=n,
                              head_major=head_major, skipped=skipped))  # fmt: skip
    g = torch.Generator(device=DEV).manual_seed(seed)
    k_pool = torch.randn(nslots, nkv, hd, device=DEV, generator=g).to(pool_dt)
    v_pool = torch.randn(nslots, nkv, hd, device=DEV, generator=g).to(pool_dt)
    if head_major:
        k = torch.randn(nkv, n, hd, device=DEV, generator=g).to(new_dt).transpose(0, 1)
        v = torch.randn(nkv, n, hd, device=DEV, generator=g).to(new_dt).transpose(0, 1)
    else:
        k = torch.randn(n, nkv, hd, device=DEV, generator=g).to(new_dt)
        v = torch.randn(n, nkv, hd, device=DEV, generator=g).to(new_dt)
    slots = torch.randperm(nslots, device=DEV, generator=g)[:n].clone()
    if skipped:  # slots past either end of the pool are skipped
        which = torch.randperm(n, device=DEV, generator=g)[:skipped]
        slots[which] = torch.where(which % 2 == 0, torch.full_like(which, -1), torch.full_like(which, nslots + 7))
    valid = (slots >= 0) & (slots < nslots)
    want_k, want_v = k_pool.clone(), v_pool.clone()
    want_k.index_copy_(0, slots[valid], k[valid].to(pool_dt))
    want_v.index_copy_(0, slots[valid], v[valid].to(pool_dt))
    kc, vc = k_pool.cpu(), v_pool.cpu()
    oracle.kv_append(kc, vc, k.cpu(), v.cpu(), slots.cpu())
    kv_append(k_pool, v_pool, k, v, slots)
    torch.cuda.synchronize()
    assert torch.equal(_bits(k_pool), _bits(want_k)) and torch.equal(_bits(v_pool), _bits(want_v))
    assert torch.equal(_bits(k_pool.cpu()), _bits(kc)) and torch.equal(_bits(v_pool.cpu()), _bits(vc))


@pytest.mark.parametrize("seed", range(16 * SCALE))
def test_copy_blocks_random(seed):
    r = random.Random(4000 + seed)
    dtype = r.choice(DTYPES)
    bs = r.choice([1, 3, 4, 16, 32])
    nkv, hd = r.choice([1, 2, 8]), r.choice([2, 12, 64, 128])
    layers, nblk = r.choice([1, 2, 5]), r.choice([8, 120])
    npairs = r.randint(0, nblk // 2)
    _say("copy_blocks", seed, dict(dtype=dtype, bs=bs, nkv=nkv, hd=hd, layers=layers, nblk=nblk,
                                   npairs=npairs))  # fmt: skip
    cache = PagedKVCache(KVShape(layers, nkv, hd), nblk, bs, device=DEV, dtype=dtype)
    cache.k.normal_()
    cache.v.normal_()
    # Destinations distinct and never a source (copy-on-write pairs); a source may feed
    # several destinations; a few destinations lie past the pool (skipped).
    perm = r.sample(range(nblk), nblk)
    srcs = perm[: max(1, nblk // 2)]
    dsts = perm[max(1, nblk // 2) :][:npairs]
    pairs = [[r.choice(srcs), d if r.random() > 0.1 else nblk + d] for d in dsts]
    pt = torch.tensor(pairs, dtype=torch.int64, device=DEV).reshape(-1, 2)
    kc, vc = cache.k.cpu(), cache.v.cpu()
    oracle.copy_blocks(kc, vc, pt.cpu(), bs)
    cache.copy_blocks(pt)
    torch.cuda.synchronize()
    assert torch.equal(_bits(cache.k.cpu()), _bits(kc)) and torch.equal(_bits(cache.v.cpu()), _bits(vc))


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


@pytest.mark.parametrize("seed", range(24 * SCALE))
def test_fused_random(seed):
    r = random.Random(5000 + seed)
    dtype = r.choice(DTYPES)
    n = r.choice([1, 7, 300, 2168])
    nh, hd = r.choice([1, 3, 8, 32]), r.choice([2, 12, 16, 64, 128, 256])
    dim = r.choice([1, 100, 999, 2048, 4096])
    _say("fused", seed, dict(dtype=dtype, n=n, nh=nh, hd=hd, dim=dim))
    g = torch.Generator(device=DEV).manual_seed(seed)
    # RoPE in place on [n, nh, hd] with HF's cast of cos / sin to the model dtype.
    q = torch.randn(n, nh, hd, device=DEV, generator=g).to(dtype)
    pos = torch.randint(0, 8192, (n,), device=DEV, generator=g)
    inv = 1.0 / (500000 ** (torch.arange(0, hd, 2, device=DEV).float() / hd))
    emb = torch.cat([pos[:, None].float() * inv] * 2, -1)
    cos, sin = emb.cos(), emb.sin()
    want = q * cos[:, None].to(dtype) + _rotate_half(q) * sin[:, None].to(dtype)
    got = q.clone()
    fused.rope_(got, cos, sin)
    assert torch.equal(got, want), "rope"
    # SiLU(gate) * up.
    gate = (torch.randn(n, dim, device=DEV, generator=g) * 4).to(dtype)
    up = torch.randn(n, dim, device=DEV, generator=g).to(dtype)
    assert torch.equal(fused.silu_mul(gate, up), F.silu(gate) * up), "silu_mul"
    # RMSNorm: the reference's expression.
    x = (torch.randn(n, dim, device=DEV, generator=g) * 3).to(dtype)
    w = torch.randn(dim, device=DEV, generator=g).to(dtype)
    xf = x.float()
    want = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(x.dtype)
    assert torch.equal(fused.rms_norm(x, w, 1e-5), want), "rms_norm"
