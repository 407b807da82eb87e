"""Every BASELINE config in full against the CPU oracle, through the C ABI (the bar of
the reference's tests/test_kernels.py:17-37 and :182-215, at this build's tolerance):

- KV append and copy-on-write: the whole pools bit-exact against the oracle's own
  append and block copy on the same inputs;
- attention: every sequence (decode) and every query row (prefill) within max-abs 2e-3
  of the oracle's fp32 result, and the q.dtype output equal to the kernel's fp32 result
  rounded by torch (so within 2e-3 plus half an output ulp of the oracle).

Each test prints its case first (flushed), so a failing GPU step names it.
"""

from __future__ import annotations

import os

import pytest
import torch

from engine import workloads
from engine.kernels import paged_attention as pa
from engine.runtime.paged_cache import copy_blocks, kv_append
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
THREADS = min(16, os.cpu_count() or 1)
ATOL = 2e-3


def _say(*a):
    print("[case]", *a, flush=True)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8)


def _append_both(k_dev, v_dev, new_k, new_v, slots):
    """The HIP append on the device pools and the oracle's on CPU copies of them; the
    whole pools must then be equal bit for bit. Returns the CPU pools."""
    kc, vc = k_dev.cpu(), v_dev.cpu()
    oracle.kv_append(kc, vc, new_k.cpu(), new_v.cpu(), slots.cpu())
    kv_append(k_dev, v_dev, new_k, new_v, slots)
    torch.cuda.synchronize()
    assert torch.equal(_bits(k_dev.cpu()), _bits(kc)), "K pool differs from the oracle"
    assert torch.equal(_bits(v_dev.cpu()), _bits(vc)), "V pool differs from the oracle"
    return kc, vc


def _decode_both(step, kc, vc, **kw):
    """fp32 and q.dtype results of the decode kernel against the oracle, all rows."""
    args = (step.q, step.k_cache, step.v_cache, step.block_tables, step.context_lens,
            step.block_size)  # fmt: skip
    out32 = torch.empty(step.q.shape, dtype=torch.float32, device=DEV)
    pa.paged_decode_attention(*args, out=out32, **kw)
    outq = pa.paged_decode_attention(*args, **kw)
    torch.cuda.synchronize()
    want = oracle.decode_attention(step.q.cpu(), kc, vc, step.block_tables.cpu(),
                                   step.context_lens.cpu(), step.block_size, threads=THREADS)  # fmt: skip
    err = (out32.cpu() - want).abs().max().item()
    assert err <= ATOL, f"fp32 max|err| {err}"
    assert torch.equal(_bits(outq), _bits(out32.to(step.q.dtype))), "q.dtype rounding"
    return err


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_config_decode_full(name):
    """Configs 1 and 2: append, then decode attention over every sequence."""
    _say("config", name)
    step = workloads.CONFIGS[name](DEV, seed=0)
    kc, vc = _append_both(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)
    _decode_both(step, kc, vc)  # default split: config 1 takes the one-kernel split pass
    b, nh, hd = step.q.shape
    nkv = step.k_cache.shape[1]
    _decode_both(step, kc, vc, num_workgroups=pa.decode_workgroups(DEV, step.q.dtype, hd, nh, nkv))


@pytest.mark.parametrize("cascade", [False, True])
def test_config3_full(cascade):
    """Config 3: 256 sequences on one 2,048-token prefix. The copy-on-write of the last
    shared block for 64 of them (whole pools bit-exact), the append, then decode of
    all 256 sequences, plain and with cascade over the shared prefix."""
    _say("config3", "cascade" if cascade else "plain")
    step = workloads.config3(DEV, seed=0)
    kc, vc = step.k_cache.cpu(), step.v_cache.cpu()
    oracle.copy_blocks(kc, vc, step.cow_mapping.cpu(), step.block_size)
    copy_blocks(step.k_cache, step.v_cache, step.cow_mapping, step.block_size)
    torch.cuda.synchronize()
    assert torch.equal(_bits(step.k_cache.cpu()), _bits(kc))
    assert torch.equal(_bits(step.v_cache.cpu()), _bits(vc))
    kc, vc = _append_both(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)
    kw = {}
    if cascade:
        nh, nkv = step.q.shape[1], step.k_cache.shape[1]
        pg = pa.find_prefix_groups(step.block_tables.cpu(), step.context_lens.cpu(),
                                   step.block_size, nh, nkv, DEV)  # fmt: skip
        # All 256 share the first 127 blocks (the 128th was copied for 64 of them).
        assert pg is not None and pg.members == step.batch
        kw["prefix_groups"] = pg
    _decode_both(step, kc, vc, **kw)


@pytest.mark.parametrize("wgs", [None, 97, 1024])
def test_config4_full(wgs):
    """Config 4 (32 sequences, contexts log-uniform up to 32k): every sequence, under
    the default work split and two others (fewer and more workgroups than CUs)."""
    _say("config4", wgs)
    step = workloads.config4(DEV, seed=0)
    kc, vc = _append_both(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)
    _decode_both(step, kc, vc, num_workgroups=wgs)


def test_config5_full_step():
    """Config 5's whole mixed step: the 2,168-row append (4 prompt chunks of 512 tokens,
    then 120 decode tokens) bit-exact, every one of the 2,048 prefill rows and every one
    of the 120 decode rows within 2e-3 of the oracle, q.dtype outputs equal to the
    rounded fp32 ones."""
    _say("config5 step")
    m = workloads.config5(DEV, seed=0)
    assert m.slot_mapping.numel() == 2168
    kc, vc = _append_both(m.k_cache, m.v_cache, m.new_k, m.new_v, m.slot_mapping)
    args = (m.q_chunks, m.k_cache, m.v_cache, m.chunk_tables, m.chunk_ctx, m.block_size,
            m.cu_q, m.max_query_len)  # fmt: skip
    out32 = torch.empty(m.q_chunks.shape, dtype=torch.float32, device=DEV)
    pa.paged_prefill_attention(*args, out=out32)
    outq = pa.paged_prefill_attention(*args)
    torch.cuda.synchronize()
    assert torch.equal(_bits(outq), _bits(out32.to(m.q_chunks.dtype))), "prefill rounding"
    want = oracle.prefill_attention(m.q_chunks.cpu(), kc, vc, m.chunk_tables.cpu(), m.cu_q.cpu(),
                                    m.chunk_ctx.cpu(), m.block_size, threads=THREADS)  # fmt: skip
    assert want.shape[0] == 2048
    err = (out32.cpu() - want).abs().amax(dim=(1, 2))
    assert err.max().item() <= ATOL, f"prefill rows over 2e-3: {torch.nonzero(err > ATOL)[:8].tolist()}"
    d = m.decode
    assert d.batch == 120
    _decode_both(d, kc, vc)
