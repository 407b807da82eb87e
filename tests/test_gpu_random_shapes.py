"""Seeded random shapes through the C ABI against the oracle. Decode attention: batch,
ragged and empty contexts, block size (powers of two and not), head dim, GQA group,
dtype and work split all drawn per case. Chunked prefill: chunk counts and lengths,
cached prefixes, empty chunks, block sizes, head dims, groups and dtype (fp32 and
head_dim 16 take the VALU kernel). Each case comes from
its own seed and prints its shape first, so a failure names a reproducible case.
PKV_RANDOM_CASES_SCALE=N multiplies the number of seeds (here and in the cascade's
random test)."""

from __future__ import annotations

import os
import random

import pytest
import torch

from engine import workloads
from engine.kernels import paged_attention as pa
from oracle import oracle
from test_gpu_prefill import _chunks, _run

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
THREADS = min(16, os.cpu_count() or 1)
ATOL = 2e-3
# PKV_RANDOM_CASES_SCALE=N draws N times as many seeds per random test (default 1).
SCALE = max(1, int(os.environ.get("PKV_RANDOM_CASES_SCALE", "1")))


def _say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("seed", range(32 * SCALE))
def test_decode_random_shape(seed):
    r = random.Random(seed)
    hd = r.choice([16, 32, 64, 128, 128, 128, 256])
    nkv = r.choice([1, 2, 4, 8])
    groups = r.choice([1, 2, 3, 4, 5, 6, 8])
    bs = r.choice([1, 3, 4, 8, 16, 16, 32])
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    ctx = [r.choice([0, 1, r.randint(2, 64), r.randint(65, 700)]) for _ in range(r.randint(1, 12))]
    wgs = r.choice([None, None, 1, 3, 17, 256, 900])
    _say("decode", seed, dict(hd=hd, nkv=nkv, groups=groups, bs=bs, dtype=dtype, ctx=ctx, wgs=wgs))
    step = workloads.custom(ctx, nkv * groups, nkv, hd, bs, dtype, DEV, seed=seed)
    args = (step.q, step.k_cache, step.v_cache, step.block_tables, step.context_lens, bs)
    out32 = torch.empty(step.q.shape, dtype=torch.float32, device=DEV)
    pa.paged_decode_attention(*args, out=out32, num_workgroups=wgs)
    outq = pa.paged_decode_attention(*args, num_workgroups=wgs)
    torch.cuda.synchronize()
    want = oracle.decode_attention(step.q.cpu(), step.k_cache.cpu(), step.v_cache.cpu(),
                                   step.block_tables.cpu(), step.context_lens.cpu(), bs,
                                   threads=THREADS)  # fmt: skip
    assert (out32.cpu() - want).abs().max().item() <= ATOL
    assert torch.equal(outq.cpu(), out32.cpu().to(dtype))


@pytest.mark.parametrize("seed", range(12 * SCALE))
def test_decode_random_large_batch(seed):
    """Batches past one wave (65 .. 1,100 sequences): the stream pass stages the batch's
    lengths, first columns and unit offsets in LDS up to 1,024 sequences and walks them
    64 at a time beyond that; ragged and empty contexts, work splits that leave ranges
    empty or cut every sequence."""
    r = random.Random(500 + seed)
    hd = r.choice([64, 128, 128])
    nkv = r.choice([1, 2, 8])
    groups = r.choice([1, 3, 4])
    bs = r.choice([8, 12, 16, 16, 32])
    dtype = r.choice([torch.bfloat16, torch.float16])
    batch = r.choice([65, r.randint(66, 300), r.randint(300, 1024), r.randint(1025, 1100)])
    ctx = [r.choice([0, 1, r.randint(2, 48), r.randint(49, 400)]) for _ in range(batch)]
    wgs = r.choice([None, None, 5, 256, 3000])
    _say("decode large batch", seed, dict(hd=hd, nkv=nkv, groups=groups, bs=bs, dtype=dtype,
                                          batch=batch, sum_ctx=sum(ctx), wgs=wgs))  # fmt: skip
    step = workloads.custom(ctx, nkv * groups, nkv, hd, bs, dtype, DEV, seed=seed)
    args = (step.q, step.k_cache, step.v_cache, step.block_tables, step.context_lens, bs)
    out32 = torch.empty(step.q.shape, dtype=torch.float32, device=DEV)
    pa.paged_decode_attention(*args, out=out32, num_workgroups=wgs)
    torch.cuda.synchronize()
    want = oracle.decode_attention(step.q.cpu(), step.k_cache.cpu(), step.v_cache.cpu(),
                                   step.block_tables.cpu(), step.context_lens.cpu(), bs,
                                   threads=THREADS)  # fmt: skip
    assert (out32.cpu() - want).abs().max().item() <= ATOL


@pytest.mark.parametrize("seed", range(28 * SCALE))
def test_prefill_random_shape(seed):
    r = random.Random(1000 + seed)
    hd = r.choice([16, 32, 64, 128, 128, 256])
    nkv = r.choice([1, 2, 4, 8])
    groups = r.choice([1, 2, 3, 4, 8])
    bs = r.choice([4, 12, 16, 16, 32])
    dtype = r.choice([torch.bfloat16, torch.float16, torch.bfloat16, torch.float32])
    spec = []
    for _ in range(r.randint(1, 6)):
        qn = r.choice([0, 1, r.randint(2, 40), r.randint(41, 200)])
        spec.append((qn, qn + r.choice([0, r.randint(1, 50), r.randint(51, 400)])))
    _say("prefill", seed, dict(hd=hd, nkv=nkv, groups=groups, bs=bs, dtype=dtype, spec=spec))
    q, k, v, tables, ctx, cu = _chunks(spec, nkv * groups, nkv, hd, bs, dtype, seed=seed)
    max_q = max(max(qn for qn, _ in spec), 1)
    got = _run(q, k, v, tables, ctx, cu, bs, max_q)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs, threads=THREADS)
    assert got.shape == want.shape
    if got.numel():  # every chunk may be empty (then there is nothing to compare)
        assert (got - want).abs().max().item() <= ATOL
