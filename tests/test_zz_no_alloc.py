"""The decode entry point that allocates nothing (C ``pkv_paged_decode_noalloc``: the
split-K scratch is a static per-GPU device array) against the allocating entry point
(``pkv_paged_decode``) through the C ABI: two calls in a row, the second with a smaller
input, each bit-identical to the allocating call at the same work split (same kernels)
and within 2e-3 of the oracle; shapes whose scratch exceeds the array are refused
before launch."""

from __future__ import annotations

import os

import pytest
import torch

from engine import workloads
from engine.kernels import _native
from engine.kernels import paged_attention as pa
from oracle import oracle

DEV = torch.device("cuda:0")
THREADS = min(16, os.cpu_count() or 1)


def _say(*a):
    print("[case]", *a, flush=True)


def _direct_noalloc(step, out, wgs):
    """pkv_paged_decode_noalloc called straight through ctypes."""
    b, nh, hd = step.q.shape
    k = step.k_cache
    return _native.lib().pkv_paged_decode_noalloc(
        out.data_ptr(), _native.dtype_code(out.dtype, "t"), out.stride(0), out.stride(1),
        step.q.data_ptr(), step.q.stride(0), step.q.stride(1), k.data_ptr(),
        step.v_cache.data_ptr(), _native.dtype_code(k.dtype, "t"), k.stride(0), k.stride(1),
        k.shape[0], step.block_tables.data_ptr(), step.block_tables.stride(0),
        step.block_tables.shape[1], step.context_lens.data_ptr(), b, nh, k.shape[1], hd,
        step.block_size, hd**-0.5, wgs, torch.cuda.current_stream().cuda_stream)  # fmt: skip


@pytest.mark.gpu
def test_noalloc_decode_matches_allocating_entry_point():
    steps = [
        ("config2 full", workloads.config2(DEV, seed=0), None),
        ("smaller: 5 sequences, hd 64, 8 heads", workloads.custom(
            [1, 40, 300, 17, 999], 8, 2, 64, 16, torch.bfloat16, DEV, seed=1), 37),
        # the library's default split at a small batch: the one-launch split pass, which
        # needs no scratch (the array is neither sized nor looked up for it)
        ("default split: config1", workloads.config1(DEV, seed=2), 0),
        ("default split: 3 sequences, hd 128", workloads.custom(
            [5, 200, 64], 24, 8, 128, 16, torch.bfloat16, DEV, seed=3), 0),
    ]  # fmt: skip
    for name, step, wgs in steps:
        _say("noalloc", name, "workgroups", wgs)
        args = (step.q, step.k_cache, step.v_cache, step.block_tables, step.context_lens,
                step.block_size)  # fmt: skip
        b, nh, hd = step.q.shape
        if wgs == 0:  # the default on both entry points
            n_wg = None
            assert _native.lib().pkv_decode_default_workgroups(
                _native.dtype_code(step.k_cache.dtype, "t"), hd, nh, step.k_cache.shape[1], b,
                step.block_tables.shape[1], step.block_size) == 0, name  # fmt: skip
        else:
            n_wg = wgs or pa.decode_workgroups(DEV, step.q.dtype, hd, nh, step.k_cache.shape[1])
        want32 = torch.empty(step.q.shape, dtype=torch.float32, device=DEV)
        pa.paged_decode_attention(*args, out=want32, num_workgroups=n_wg)
        got32 = torch.full_like(want32, float("nan"))
        pa.paged_decode_attention_noalloc(*args, out=got32, num_workgroups=n_wg)
        gotq = torch.empty_like(step.q)
        _native.check(_direct_noalloc(step, gotq, n_wg or 0), "noalloc direct")
        torch.cuda.synchronize()
        assert torch.equal(got32, want32), name
        assert torch.equal(gotq, want32.to(step.q.dtype)), name
        ref = oracle.decode_attention(step.q.cpu(), step.k_cache.cpu(), step.v_cache.cpu(),
                                      step.block_tables.cpu(), step.context_lens.cpu(),
                                      step.block_size, threads=THREADS)  # fmt: skip
        assert (got32.cpu() - ref).abs().max().item() <= 2e-3, name
    # Scratch beyond the static array: refused before launch, out untouched.
    step = steps[1][1]
    out = torch.zeros(step.q.shape, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError, match="no-alloc"):
        pa.paged_decode_attention_noalloc(step.q, step.k_cache, step.v_cache, step.block_tables,
                                          step.context_lens, step.block_size, out=out,
                                          num_workgroups=1 << 20)  # fmt: skip
    torch.cuda.synchronize()
    assert not out.any()
