"""Parity of the HIP path (through the C ABI) with the CPU oracle on the same seeded
inputs. Append and block copy: bit-exact. Attention: the unrounded fp32 result within
max-abs 2e-3 of the oracle, and the q.dtype result equal to that fp32 result rounded
(so within 2e-3 plus half an output ulp of the oracle).

Each test prints the case it is about to run (flushed) so a failing GPU step names it.
"""

from __future__ import annotations

import math
import os

import pytest
import torch

from engine import workloads
from engine.kernels import _native
from engine.kernels import paged_attention as pa
from engine.runtime.paged_cache import PagedKVCache, KVShape, copy_blocks, decode_slots, kv_append
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
THREADS = min(16, os.cpu_count() or 1)
ATOL = 2e-3  # max-abs error of the fp32 attention result


def _say(*a):
    print("[case]", *a, flush=True)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8)


def _check_attention(step, wgs=None, ctx_for_oracle=None, what=""):
    """Run the kernel with fp32 and native-dtype outputs, compare with the oracle."""
    args = (step.q, step.k_cache, step.v_cache, step.block_tables, step.context_lens,
            step.block_size)  # fmt: skip
    out32 = torch.empty(step.q.shape, dtype=torch.float32, device=DEV)
    pa.paged_decode_attention(*args, out=out32, num_workgroups=wgs)
    outq = pa.paged_decode_attention(*args, num_workgroups=wgs)
    torch.cuda.synchronize()
    ctx = step.context_lens.cpu() if ctx_for_oracle is None else ctx_for_oracle
    want = oracle.decode_attention(step.q.cpu(), step.k_cache.cpu(), step.v_cache.cpu(),
                                   step.block_tables.cpu(), ctx, step.block_size,
                                   threads=THREADS)  # fmt: skip
    err = (out32.cpu() - want).abs().max().item()
    assert err <= ATOL, f"{what}: fp32 max|err| {err}"
    # The q.dtype output is exactly the fp32 result rounded by torch's own conversion.
    assert torch.equal(_bits(outq), _bits(out32.to(step.q.dtype))), f"{what}: rounding"
    return out32, err


# ---- KV append ---------------------------------------------------------------------------


@pytest.mark.parametrize(
    ("pool_dt", "new_dt"),
    [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
     (torch.float32, torch.float32), (torch.bfloat16, torch.float32),
     (torch.float16, torch.float32), (torch.float32, torch.bfloat16),
     (torch.bfloat16, torch.float16)],
)  # fmt: skip
@pytest.mark.parametrize("hd", [16, 64, 128, 12])
def test_append_bit_exact(pool_dt, new_dt, hd):
    _say("append", pool_dt, new_dt, hd)
    g = torch.Generator(device=DEV).manual_seed(1)
    nslots, nkv, n = 4096, 8, 300
    k_pool = torch.randn(nslots, nkv, hd, device=DEV, generator=g).to(pool_dt)
    v_pool = torch.randn(nslots, nkv, hd, device=DEV, generator=g).to(pool_dt)
    # call-site layout: transposes of [nkv, N, hd] projections
    k = torch.randn(nkv, n, hd, device=DEV, generator=g).to(new_dt).transpose(0, 1)
    v = torch.randn(nkv, n, hd, device=DEV, generator=g).to(new_dt).transpose(0, 1)
    slots = torch.randperm(nslots, device=DEV, generator=g)[:n]
    kc, vc = k_pool.cpu(), v_pool.cpu()
    oracle.kv_append(kc, vc, k.cpu(), v.cpu(), slots.cpu())
    want_k, want_v = k_pool.clone(), v_pool.clone()
    want_k.index_copy_(0, slots, k.to(pool_dt))
    want_v.index_copy_(0, slots, v.to(pool_dt))
    kv_append(k_pool, v_pool, k, v, slots)
    torch.cuda.synchronize()
    assert torch.equal(_bits(k_pool.cpu()), _bits(kc)) and torch.equal(_bits(v_pool.cpu()), _bits(vc))
    assert torch.equal(_bits(k_pool), _bits(want_k)) and torch.equal(_bits(v_pool), _bits(want_v))


def test_append_special_values_match_device_conversion():
    """NaN, inf, rounding ties and subnormals convert exactly as torch does on the GPU."""
    _say("append special values")
    vals = [float("nan"), float("inf"), float("-inf"), 0.0, -0.0, 65520.0, 1e-45, 3e38,
            1.0 + 2.0**-9, 1.0 + 3 * 2.0**-9, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 2.0**-25]  # fmt: skip
    x = torch.tensor(vals * 2, dtype=torch.float32)  # 26 values
    k = torch.zeros(1, 2, 16)
    k.view(-1)[:26] = x
    k = k.to(DEV)
    slots = torch.tensor([3], device=DEV)
    for pool_dt in (torch.bfloat16, torch.float16):
        kp = torch.zeros(8, 2, 16, dtype=pool_dt, device=DEV)
        vp = torch.zeros_like(kp)
        kv_append(kp, vp, k, -k, slots)
        want = torch.zeros_like(kp)
        want.index_copy_(0, slots, k.to(pool_dt))
        torch.cuda.synchronize()
        assert torch.equal(_bits(kp), _bits(want)), pool_dt


def test_append_edge_cases():
    _say("append edge cases")
    kp = torch.zeros(32, 2, 16, dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    k = torch.randn(4, 2, 16, device=DEV).to(torch.bfloat16)
    v = torch.randn(4, 2, 16, device=DEV).to(torch.bfloat16)
    kv_append(kp, vp, k[:0], v[:0], torch.zeros(0, dtype=torch.int64, device=DEV))  # N = 0
    assert not kp.any()
    # Out-of-range slots are skipped, the rest land.
    kv_append(kp, vp, k, v, torch.tensor([5, -1, 32, 31], device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(kp[5], k[0]) and torch.equal(kp[31], k[3]) and torch.equal(vp[31], v[3])
    assert int((kp != 0).any(-1).any(-1).sum()) == 2
    with pytest.raises(RuntimeError, match="long"):
        kv_append(kp, vp, k, v, torch.tensor([1, 2, 3, 4], dtype=torch.int32, device=DEV))
    with pytest.raises(IndexError):
        kv_append(kp, vp, k, v, torch.tensor([1, 2, 3], device=DEV))



def test_debug_checks_raise_like_the_reference():
    """With the opt-in metadata checks on, metadata the kernels would skip or mask
    raises IndexError before any launch (index_copy_ and the reference's gather raise
    there), nothing is written, and good metadata still gives the unchecked results."""
    _say("debug checks")
    step = workloads.custom([50, 300, 7], 8, 2, 64, 16, torch.bfloat16, DEV, seed=3)
    args = (step.q, step.k_cache, step.v_cache, step.block_tables, step.context_lens, 16)
    plain = pa.paged_decode_attention(*args)
    prev = _native.set_debug_checks(True)
    try:
        kp = torch.zeros(32, 2, 16, dtype=torch.bfloat16, device=DEV)
        vp = torch.zeros_like(kp)
        k = torch.randn(2, 2, 16, device=DEV).to(torch.bfloat16)
        with pytest.raises(IndexError, match="outside the pool"):
            kv_append(kp, vp, k, k, torch.tensor([5, 32], device=DEV))
        torch.cuda.synchronize()
        assert not kp.any()
        kv_append(kp, vp, k, k, torch.tensor([5, 31], device=DEV))
        torch.cuda.synchronize()
        assert torch.equal(kp[31], k[1])
        assert torch.equal(pa.paged_decode_attention(*args), plain)
        nblk = step.k_cache.shape[0] // 16
        bad = step.block_tables.clone()
        bad[1, 3] = nblk  # a used column of sequence 1 (300 tokens)
        with pytest.raises(IndexError, match="sequence 1 column 3"):
            pa.paged_decode_attention(step.q, step.k_cache, step.v_cache, bad,
                                      step.context_lens, 16)  # fmt: skip
        long_ctx = step.context_lens.clone()
        long_ctx[0] = step.block_tables.shape[1] * 16 + 1
        with pytest.raises(IndexError, match="context_lens"):
            pa.paged_decode_attention(step.q, step.k_cache, step.v_cache, step.block_tables,
                                      long_ctx, 16)  # fmt: skip
        with pytest.raises(IndexError, match="outside the pool"):
            copy_blocks(step.k_cache, step.v_cache,
                        torch.tensor([[0, nblk]], device=DEV), 16)  # fmt: skip
        cu = torch.tensor([0, 3, 2], dtype=torch.int32, device=DEV)
        q_rows = torch.randn(3, 8, 64, device=DEV).to(torch.bfloat16)
        with pytest.raises(IndexError, match="cu_seqlens_q"):
            pa.paged_prefill_attention(q_rows, step.k_cache, step.v_cache,
                                       step.block_tables[:2].contiguous(),
                                       step.context_lens[:2].contiguous(), 16, cu, 3)  # fmt: skip
    finally:
        _native.set_debug_checks(prev)

def test_paged_cache_write_all_layers():
    _say("PagedKVCache.write")
    cfg = KVShape(num_hidden_layers=3, num_key_value_heads=8, head_dim=128)
    cache = PagedKVCache(cfg, num_blocks=64, block_size=16, device=DEV, dtype=torch.bfloat16)
    ref = PagedKVCache(cfg, num_blocks=64, block_size=16, device=DEV, dtype=torch.bfloat16)
    for layer in range(3):
        k = torch.randn(64, 8, 128, device=DEV)
        v = torch.randn(64, 8, 128, device=DEV)
        slots = torch.randperm(1024, device=DEV)[:64]
        cache.write(layer, k, v, slots)
        ref.k[layer].index_copy_(0, slots, k.to(torch.bfloat16))
        ref.v[layer].index_copy_(0, slots, v.to(torch.bfloat16))
    torch.cuda.synchronize()
    assert torch.equal(_bits(cache.k), _bits(ref.k)) and torch.equal(_bits(cache.v), _bits(ref.v))


# ---- block copy --------------------------------------------------------------------------


@pytest.mark.parametrize(("bs", "nkv", "hd", "dtype"),
                         [(16, 8, 128, torch.bfloat16), (4, 2, 16, torch.float32),
                          (1, 1, 2, torch.float16)])  # fmt: skip
def test_copy_blocks_bit_exact(bs, nkv, hd, dtype):
    _say("copy_blocks", bs, nkv, hd, dtype)
    layers, nblk = 4, 200
    cfg = KVShape(layers, nkv, hd)
    cache = PagedKVCache(cfg, nblk, bs, device=DEV, dtype=dtype)
    cache.k.normal_()
    cache.v.normal_()
    pairs = torch.tensor([[7, 100], [7, 101], [50, 3], [199, 150], [0, 250]], device=DEV)
    kc, vc = cache.k.cpu(), cache.v.cpu()
    oracle.copy_blocks(kc, vc, pairs.cpu(), bs)
    cache.copy_blocks(pairs)
    torch.cuda.synchronize()
    assert torch.equal(_bits(cache.k.cpu()), _bits(kc)) and torch.equal(_bits(cache.v.cpu()), _bits(vc))


# ---- decode attention --------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("nh", "nkv", "hd"), [(32, 8, 64), (24, 8, 128), (4, 2, 16)])
@pytest.mark.parametrize("block_size", [4, 16])
def test_decode_reference_matrix(dtype, nh, nkv, hd, block_size):
    """The reference's kernel test cases (reference tests/test_kernels.py:17-37)."""
    _say("decode matrix", dtype, nh, nkv, hd, block_size)
    step = workloads.custom([1, 17, 200, 64, 333], nh, nkv, hd, block_size, dtype, DEV, seed=0)
    _check_attention(step, what="matrix")
    # the reference's own PyTorch oracle, run on the GPU, agrees to its bf16 tolerance
    got = pa.paged_decode_attention(step.q, step.k_cache, step.v_cache, step.block_tables,
                                    step.context_lens, step.block_size)  # fmt: skip
    ref = pa.reference_decode_attention(step.q, step.k_cache, step.v_cache, step.block_tables,
                                        step.context_lens, step.block_size)  # fmt: skip
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(got, ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("hd", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 6, 8, 16])
def test_decode_head_dims_and_groups(hd, groups):
    _say("decode hd/groups", hd, groups)
    nkv = 2
    step = workloads.custom([3, 40, 129, 700], nkv * groups, nkv, hd, 16, torch.bfloat16, DEV,
                            seed=hd + groups)  # fmt: skip
    _check_attention(step, what=f"hd{hd} g{groups}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("block_size", [16, 12])
def test_decode_hd64_stream_pass_matrix_pv(dtype, groups, block_size):
    """The stream-K pass at head_dim 64 multiplies P.V on the matrix cores (each wave's V
    rows staged in LDS and read back transposed, P as a hi + lo pair): oracle parity over
    1-4 query heads per wave and sub-groups, tile-aligned and tile-splitting block sizes,
    ragged, tile-boundary and empty contexts, several work splits (pieces cut anywhere),
    and agreement with the one-launch split pass (P.V on the VALU) to fp32 rounding."""
    _say("decode hd64 stream pass", dtype, groups, block_size)
    nkv = 2
    ctx = [0, 1, 15, 16, 17, 31, 32, 33, 250, 1000, 1999]
    step = workloads.custom(ctx, nkv * groups, nkv, 64, block_size, dtype, DEV,
                            seed=64 + groups + block_size)  # fmt: skip
    for wgs in (2, 7, 64):
        out32, _ = _check_attention(step, wgs=wgs, what=f"g{groups} bs{block_size} wgs{wgs}")
        assert not out32[0].any()  # empty context: 0
    if pa.default_workgroups(DEV, dtype, 64, nkv * groups, nkv, len(ctx),
                             step.block_tables.shape[1], block_size) == 0:  # fmt: skip
        split = torch.empty_like(out32)
        pa.paged_decode_attention(step.q, step.k_cache, step.v_cache, step.block_tables,
                                  step.context_lens, block_size, out=split)  # fmt: skip
        torch.cuda.synchronize()
        assert (out32 - split).abs().max().item() <= 1e-5


def test_decode_hd64_fp16_tiny_weights_keep_their_mass():
    """fp16 P on the matrix cores: one dominant key and 30,000 keys whose weights (2^-26
    of it, ~1.5e-8) lie below half of fp16's smallest subnormal. Their V of 8 carries
    ~3.6e-3 of the output, so weights rounded to zero in fp16 would miss the 2e-3 bar;
    the kernel scales P by 2^7 before packing it (and O back) so they stay."""
    _say("decode hd64 fp16 tiny weights")
    n = 30_001
    step = workloads.custom([n], 4, 1, 64, 16, torch.float16, DEV, seed=5)
    step.q.zero_()
    step.q[:, :, 0] = 16.0
    step.k_cache.zero_()
    step.v_cache.fill_(8.0)
    dom = int(step.block_tables[0, 0]) * 16  # token 0's slot
    # score difference 16 * 9 = 144, times scale * log2(e) = 0.125 * 1.4427: ~26 in log2
    step.k_cache[dom, :, 0] = 9.0
    step.v_cache[dom] = 0.0
    # one workgroup: every key in the dominant key's piece (other pieces would take
    # their own exponent reference, where these weights are not small)
    out32, err = _check_attention(step, wgs=1, what="tiny weights")
    w = 2.0 ** (-144 * 0.125 / math.log(2))
    want = 8 * (n - 1) * w / (1 + (n - 1) * w)
    assert want > 3e-3
    assert abs(out32[0, 0, 0].item() - want) < 2e-4


@pytest.mark.parametrize("block_size", [1, 2, 3, 8, 32])
def test_decode_block_sizes(block_size):
    _say("decode block size", block_size)
    step = workloads.custom([1, 5, 31, 97, 260], 8, 2, 64, block_size, torch.bfloat16, DEV, seed=2)
    _check_attention(step, what=f"bs{block_size}")


@pytest.mark.parametrize("wgs", [1, 2, 3, 7, 16, 64, 255, 1000, 5000])
def test_decode_partition_invariance(wgs):
    """combine(pieces) == single pass: every way of cutting the contexts among
    workgroups (including more workgroups than work units) gives the oracle's answer."""
    _say("decode workgroups", wgs)
    step = workloads.custom([1, 16, 17, 250, 1000, 2049, 0, 5], 24, 8, 128, 16,
                            torch.bfloat16, DEV, seed=3)  # fmt: skip
    out32, _ = _check_attention(step, wgs=wgs, what=f"wgs{wgs}")
    assert not out32[6].any()


def test_decode_edge_cases():
    _say("decode edge cases")
    step = workloads.custom([0, 1, 40, 64], 8, 2, 64, 16, torch.bfloat16, DEV, seed=4, width=6)
    out32, _ = _check_attention(step, what="ctx0")
    assert not out32[0].any()  # empty context -> 0
    # Context longer than the table covers: clamped to W * block_size.
    over = step.context_lens.clone()
    over[3] = 10_000
    step.context_lens = over
    _check_attention(step, ctx_for_oracle=torch.tensor([0, 1, 40, 96], dtype=torch.int32),
                     what="ctx clamp")  # fmt: skip
    # A block id outside the pool masks its tokens instead of faulting.
    step.context_lens = torch.tensor([0, 1, 40, 64], dtype=torch.int32, device=DEV)
    bad = step.block_tables.clone()
    bad[2, 2] = 1 << 20  # third block of a 40-token sequence: positions 32..39 masked
    bad[1, 0] = -7  # the only block of the 1-token sequence: nothing left, output 0
    step.block_tables = bad
    # Every way of cutting the work, so a piece may start (or consist of) masked tiles.
    for wgs in (None, 1, 2, 5, 9, 64):
        out32, _ = _check_attention(
            step, wgs=wgs, ctx_for_oracle=torch.tensor([0, 0, 32, 64], dtype=torch.int32),
            what=f"oob block wgs={wgs}")  # fmt: skip
        assert not out32[1].any()


def test_decode_table_row_stride_and_graph_padding_rows():
    """Graph-buffer contract (reference cuda_graphs.py:39-43, :99-106): tables are a
    view of a wider static buffer; padding rows have ctx = 1 and read a scratch block."""
    _say("decode table stride + padding rows")
    real = workloads.custom([50, 300, 7], 24, 8, 128, 16, torch.bfloat16, DEV, seed=5)
    scratch = real.k_cache.shape[0] // 16 - 1
    wide = torch.full((8, 40), scratch, dtype=torch.int32, device=DEV)
    wide[:3, : real.block_tables.shape[1]] = real.block_tables
    ctx = torch.ones(8, dtype=torch.int32, device=DEV)
    ctx[:3] = real.context_lens
    q = torch.randn(8, 24, 128, device=DEV).to(torch.bfloat16)
    q[:3] = real.q
    step = workloads.DecodeStep("padded", q, real.k_cache, real.v_cache, wide[:, :20], ctx, 16,
                                real.new_k, real.new_v, real.slot_mapping)  # fmt: skip
    assert step.block_tables.stride(0) == 40
    _check_attention(step, what="padded")


@pytest.mark.parametrize("split", ["stream", "default"])
def test_graph_capture_replay(split):
    """Append + decode captured once in a hipGraph, replayed with new lengths and tables
    (the DecodeGraphs pattern, reference engine/runtime/cuda_graphs.py:64-108): the
    stream-K split with a workspace allocated outside the capture, and the default split
    (here the one-kernel split pass, chosen from static shapes only)."""
    _say("graph capture", split)
    b, nh, nkv, hd, bs, width, nblk = 16, 24, 8, 128, 16, 64, 1200
    k_pool = torch.randn(nblk * bs, nkv, hd, device=DEV).to(torch.bfloat16)
    v_pool = torch.randn_like(k_pool)
    q_s = torch.zeros(b, nh, hd, device=DEV, dtype=torch.bfloat16)
    tables_s = torch.zeros(b, width, dtype=torch.int32, device=DEV)
    ctx_s = torch.ones(b, dtype=torch.int32, device=DEV)
    slots_s = torch.zeros(b, dtype=torch.int64, device=DEV)
    nk_s = torch.zeros(b, nkv, hd, device=DEV, dtype=torch.bfloat16)
    nv_s = torch.zeros_like(nk_s)
    out_s = torch.empty(b, nh, hd, device=DEV, dtype=torch.bfloat16)
    wgs, ws = None, None
    if split == "stream":
        wgs = pa.decode_workgroups(DEV, torch.bfloat16, hd, nh, nkv)
        ws = pa.decode_workspace(DEV, b, nh, hd, wgs)  # allocated outside the capture
    else:
        assert pa.default_workgroups(DEV, torch.bfloat16, hd, nh, nkv, b, width, bs) == 0

    def body():
        kv_append(k_pool, v_pool, nk_s, nv_s, slots_s)
        pa.paged_decode_attention(q_s, k_pool, v_pool, tables_s, ctx_s, bs, out=out_s,
                                  num_workgroups=wgs, workspace=ws)  # fmt: skip

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        body()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()

    for rep in range(3):
        g = torch.Generator().manual_seed(100 + rep)
        ctx = torch.randint(1, width * bs + 1, (b,), generator=g, dtype=torch.int32)
        perm = torch.randperm(nblk, generator=g)[: b * width].view(b, width).int()
        slots = perm[torch.arange(b), (ctx - 1) // bs].long() * bs + (ctx - 1) % bs
        q_s.copy_(torch.randn(b, nh, hd, generator=g).to(torch.bfloat16))
        tables_s.copy_(perm)
        ctx_s.copy_(ctx)
        slots_s.copy_(slots)
        nk_s.copy_(torch.randn(b, nkv, hd, generator=g).to(torch.bfloat16))
        nv_s.copy_(torch.randn(b, nkv, hd, generator=g).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got = out_s.clone()
        # eager on the same (already appended) pool
        want = pa.paged_decode_attention(q_s, k_pool, v_pool, tables_s, ctx_s, bs,
                                         num_workgroups=wgs)  # fmt: skip
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(want)), f"replay {rep}"
        ref = oracle.decode_attention(q_s.cpu(), k_pool.cpu(), v_pool.cpu(), tables_s.cpu(),
                                      ctx_s.cpu(), bs, threads=THREADS)  # fmt: skip
        assert (got.float().cpu() - ref).abs().max().item() <= ATOL + 2.0**-8 * ref.abs().max().item()
        assert torch.equal(_bits(k_pool[slots_s]), _bits(nk_s))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("nh", "nkv", "hd"),
                         [(32, 8, 64), (24, 8, 128), (8, 2, 64), (16, 1, 128), (40, 8, 128)])
@pytest.mark.parametrize("block_size", [16, 4, 12, 32])
def test_decode_split_pass(dtype, nh, nkv, hd, block_size):
    """The one-kernel split pass of small batches (default split, chosen from static
    shapes: pairs fit the CUs, tables of at most 2,048 tokens): empty, one-token,
    tile-boundary and long contexts, groups of 1-5 heads per wave (sub-groups at 5),
    block sizes that split tiles (4, 12) or not; oracle parity and agreement with the
    stream-K split on the same inputs."""
    _say("decode split", dtype, nh, nkv, hd, block_size)
    ctx = [0, 1, 17, 129, 700, 2000]
    step = workloads.custom(ctx, nh, nkv, hd, block_size, dtype, DEV, seed=hd + block_size)
    w = step.block_tables.shape[1]
    assert w * block_size <= 2048
    assert pa.default_workgroups(DEV, dtype, hd, nh, nkv, len(ctx), w, block_size) == 0
    out32, _ = _check_attention(step, what="split")
    assert not out32[0].any()  # empty context: 0
    stream = torch.empty_like(out32)
    pa.paged_decode_attention(step.q, step.k_cache, step.v_cache, step.block_tables,
                              step.context_lens, block_size, out=stream,
                              num_workgroups=pa.decode_workgroups(DEV, dtype, hd, nh, nkv))  # fmt: skip
    torch.cuda.synchronize()
    assert (out32 - stream).abs().max().item() <= 1e-5


def test_decode_default_split_keeps_stream_k_for_large_shapes():
    """Tables wider than 2,048 tokens, or more (sequence, task) pairs than CUs, or fp32,
    or head_dim 256: the default split is the stream-K pass."""
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    bf = torch.bfloat16
    assert pa.default_workgroups(DEV, bf, 128, 24, 8, 64, 256, 16) > 0  # config 2
    assert pa.default_workgroups(DEV, bf, 128, 24, 8, 8, 129, 16) > 0  # 2,064 tokens
    assert pa.default_workgroups(DEV, bf, 128, 24, 8, cus // 8 + 1, 32, 16) > 0
    assert pa.default_workgroups(DEV, torch.float32, 128, 24, 8, 8, 32, 16) > 0
    assert pa.default_workgroups(DEV, bf, 256, 24, 8, 8, 32, 16) > 0
    assert pa.default_workgroups(DEV, torch.float16, 64, 32, 8, 8, 32, 16) == 0  # config 1


@pytest.mark.parametrize("wgs", [7, 300])
def test_workspace_reuse_and_garbage(wgs):
    """The scratch may hold anything (here NaN bit patterns) and be reused across calls
    of different shapes: results stay identical and match the oracle."""
    _say("workspace reuse", wgs)
    ws = pa.decode_workspace(DEV, 6, 32, 128, wgs)
    ws.fill_(0xFF)  # 0xFFFFFFFF is a NaN
    small = workloads.custom([3, 40], 32, 8, 128, 16, torch.bfloat16, DEV, seed=12)
    step = workloads.custom([1, 700, 33, 2049, 16, 5000], 32, 8, 128, 16, torch.bfloat16,
                            DEV, seed=11)  # fmt: skip
    outs = []
    for s_ in (step, small, step, small, step):
        o = pa.paged_decode_attention(s_.q, s_.k_cache, s_.v_cache, s_.block_tables,
                                      s_.context_lens, 16, num_workgroups=wgs, workspace=ws)  # fmt: skip
        if s_ is step:
            outs.append(o)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(_bits(o), _bits(outs[0]))
    _check_attention(step, wgs=wgs, what=f"ws{wgs}")


@pytest.mark.parametrize("bs", [16, 4, 3])
def test_decode_slots_on_device(bs):
    """The device slot builder against the host formula of PagedBatch._decode
    (reference engine/runtime/paged_cache.py:140-143), with graph-style tables (row
    stride > W), padding rows (ctx 1), and the cases it must map to -1: ctx < 1, a block
    past the table, a block id outside the pool."""
    _say("decode_slots", bs)
    g = torch.Generator().manual_seed(bs)
    b, w, nblk = 37, 9, 50
    full = torch.randint(0, nblk, (b, w + 3), generator=g, dtype=torch.int32)
    tables = full[:, :w]
    ctx = torch.randint(1, w * bs + 1, (b,), generator=g, dtype=torch.int32)
    ctx[0], ctx[1], ctx[2] = 0, -5, w * bs + 1  # no token; negative; past the table
    ctx[3] = 1  # a graph padding row
    tables[4, (int(ctx[4]) - 1) // bs] = nblk + 7  # outside the pool
    want = []
    for i in range(b):
        n = int(ctx[i])
        blk = (n - 1) // bs if n >= 1 else -1
        s_ = int(tables[i, blk]) * bs + (n - 1) % bs if 0 <= blk < w else -1
        want.append(s_ if 0 <= s_ < nblk * bs else -1)
    got = decode_slots(full.to(DEV)[:, :w], ctx.to(DEV), bs, nblk * bs)
    torch.cuda.synchronize()
    assert got.cpu().tolist() == want
    assert want[0] == want[1] == want[2] == want[4] == -1 and want[3] >= 0


def test_native_library_is_loaded_from_tree():
    lib = _native.lib()
    assert os.path.samefile(lib._name, _native.LIB_PATH)
    assert pa.available(DEV)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block_size", [4, 16, 32])
@pytest.mark.parametrize("wgs", [None, 1, 7])
def test_decode_hd64_two_subtile_steps(dtype, block_size, wgs):
    """hd 64 steps through two 16-token sub-tiles at a time (V rows of the second on the
    other half of the lane columns): the Llama-3.2-1B shape (32 q / 8 KV heads), long and
    ragged contexts so both sub-tiles carry live tokens, whole sequences (one workgroup)
    and cut ones."""
    _say("decode hd64 sub-tiles", dtype, block_size, wgs)
    step = workloads.custom([1, 15, 16, 17, 31, 32, 33, 300, 777, 1500], 32, 8, 64,
                            block_size, dtype, DEV, seed=64 + block_size)  # fmt: skip
    _check_attention(step, wgs=wgs, what=f"hd64 bs{block_size} wgs{wgs}")
