"""Parity of the chunked-prefill kernels (through the C ABI) -- the matrix-core kernel for
16-bit K/V at head_dim 32-256, the VALU kernel for fp32 and head_dim 16 -- with the CPU
oracle's bottom-right causal chunk attention (the semantics of the reference's PagedBatch._mixed
and Attention._mixed, engine/runtime/paged_cache.py:182-194, engine/model/layers.py:
246-265). The fp32 result must be within max-abs 2e-3 of the oracle; the q.dtype result
equals that fp32 result rounded by torch."""

from __future__ import annotations

import os

import pytest
import torch

from engine.kernels import paged_attention as pa
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
THREADS = min(16, os.cpu_count() or 1)
ATOL = 2e-3


def _say(*a):
    print("[case]", *a, flush=True)


def _bits(t):
    return t.view(torch.uint8)


def _chunks(spec, nh, nkv, hd, bs, dtype, seed, extra_blocks=5):
    """spec: [(new tokens q_c, context n_c)], tables scattered over a shared pool."""
    g = torch.Generator().manual_seed(seed)
    nblk = sum(-(-n // bs) for _, n in spec) + extra_blocks
    perm = torch.randperm(nblk, generator=g)
    width = max(-(-n // bs) for _, n in spec)
    tables = torch.zeros(len(spec), width, dtype=torch.int32)
    at = 0
    for i, (_, n) in enumerate(spec):
        nb = -(-n // bs)
        tables[i, :nb] = perm[at : at + nb].int()
        at += nb
    k = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    v = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    qlens = [q for q, _ in spec]
    cu = torch.tensor([0, *torch.tensor(qlens).cumsum(0).tolist()], dtype=torch.int32)
    q = torch.randn(int(cu[-1]), nh, hd, generator=g).to(dtype)
    ctx = torch.tensor([n for _, n in spec], dtype=torch.int32)
    return q, k, v, tables, ctx, cu


def _run(q, k, v, tables, ctx, cu, bs, max_q):
    args = (q.to(DEV), k.to(DEV), v.to(DEV), tables.to(DEV), ctx.to(DEV), bs, cu.to(DEV), max_q)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    pa.paged_prefill_attention(*args, out=out32)
    outq = pa.paged_prefill_attention(*args)
    torch.cuda.synchronize()
    assert torch.equal(_bits(outq), _bits(out32.to(q.dtype))), "rounding of the fp32 result"
    return out32.cpu()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("nh", "nkv", "hd"),
                         [(8, 2, 64), (4, 2, 128), (24, 8, 128), (6, 2, 32), (4, 2, 16)])
def test_prefill_reference_varlen_spec(dtype, nh, nkv, hd):
    """The reference's own mixed-step spec (tests/test_kernels.py:199), block size 4; its
    tiny model's shape (4 q / 2 KV heads, hd 16) included. fp32 also within the
    reference's fp32 tolerance, 1e-4 (tests/test_kernels.py:36)."""
    _say("prefill varlen spec", dtype, nh, nkv, hd)
    spec = [(1, 9), (6, 6), (1, 3), (5, 13), (3, 20), (1, 1)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, 4, dtype, seed=0)
    got = _run(q, k, v, tables, ctx, cu, 4, max(s for s, _ in spec))
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, 4, threads=THREADS)
    err = (got - want).abs().max().item()
    assert err <= (1e-4 if dtype == torch.float32 else ATOL), err


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize(("nh", "nkv", "hd", "bs"),
                         [(4, 2, 16, 4), (8, 8, 256, 16), (12, 2, 64, 3), (5, 1, 128, 16),
                          (8, 1, 32, 8)])  # fmt: skip
def test_prefill_valu_kernel_shapes(dtype, nh, nkv, hd, bs):
    """The VALU kernel (fp32 at every head dim, 16-bit at hd 16 only; the bf16 cases at
    other dims cross-check the matrix-core kernel on the same inputs): multi-tile
    contexts (64-key tiles, 32 at hd 256), query tiles of 16 tokens cut mid-chunk, groups
    of 1-12 heads (sub-groups of 4 with masked heads), block sizes that are not powers
    of two, empty chunks."""
    _say("prefill valu", dtype, nh, nkv, hd, bs)
    spec = [(37, 300), (16, 16), (0, 7), (1, 129), (70, 70), (17, 200)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, dtype, seed=hd + nh + bs)
    got = _run(q, k, v, tables, ctx, cu, bs, 70)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs, threads=THREADS)
    err = (got - want).abs().max().item()
    assert err <= (1e-4 if dtype == torch.float32 else ATOL), err


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_prefill_valu_non_causal_rows_and_lse(dtype):
    """pkv_paged_prefill_ex on the VALU kernel: causal = 0 (every query sees the chunk's
    whole context), queries gathered through q_rows, log2 normalisers."""
    _say("prefill valu ex", dtype)
    _check_ex(dtype, 4, 2, 16, 4, [(3, 21), (5, 9)], seed=11)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("nh", "nkv", "hd", "bs"), [(8, 2, 128, 16), (4, 1, 64, 12)])
def test_prefill_matrix_non_causal_rows_and_lse(dtype, nh, nkv, hd, bs):
    """The same on the matrix-core kernel (the cascade's prefix pass), whose fp16 weights
    carry a power-of-two factor that its log2 normalisers must leave out; contexts of
    several key tiles in both key halves."""
    _say("prefill matrix ex", dtype, nh, nkv, hd, bs)
    # fp16 weights are rounded once (relative error <= 2^-11 each), so the sum is within
    # a factor 1 + 2^-11 of the exact one: log2(1 + 2^-11) = 7.04e-4
    lse_tol = 8e-4 if dtype == torch.float16 else 1e-4
    _check_ex(dtype, nh, nkv, hd, bs, [(3, 700), (5, 9), (2, 130)], seed=12, lse_tol=lse_tol)


def _check_ex(dtype, nh, nkv, hd, bs, spec, seed, lse_tol=1e-4):
    """Non-causal attention of one query over n keys is the decode oracle with context n;
    the normaliser is checked in float64 from its definition."""
    from engine.kernels import _native

    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, dtype, seed=seed)
    t = q.shape[0]
    rows = torch.randperm(t, generator=torch.Generator().manual_seed(1)).int()
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = torch.empty(t, nh, hd, dtype=torch.float32, device=DEV)
    lse = torch.empty(t, nh, dtype=torch.float32, device=DEV)
    td, cd, cud, rd = tables.to(DEV), ctx.to(DEV), cu.to(DEV), rows.to(DEV)
    st = _native.lib().pkv_paged_prefill_ex(
        out.data_ptr(), _native.PKV_F32, out.stride(0), out.stride(1), qd.data_ptr(),
        qd.stride(0), qd.stride(1), kd.data_ptr(), vd.data_ptr(), _native.dtype_code(dtype, "t"),
        kd.stride(0), kd.stride(1), kd.shape[0], td.data_ptr(), td.stride(0), td.shape[1],
        cd.data_ptr(), cud.data_ptr(), len(spec), max(a for a, _ in spec), nh, nkv, hd, bs,
        hd**-0.5, 0,
        rd.data_ptr(), lse.data_ptr(), torch.cuda.current_stream().cuda_stream)  # fmt: skip
    _native.check(st, "prefill_ex")
    torch.cuda.synchronize()
    owner = torch.repeat_interleave(torch.arange(len(spec)), torch.tensor([a for a, _ in spec]))
    row_tables = tables[owner].contiguous()
    row_ctx = ctx[owner].contiguous()
    want = oracle.decode_attention(q[rows.long()].contiguous(), k, v, row_tables, row_ctx, bs,
                                   threads=THREADS)  # fmt: skip
    err = (out.cpu() - want).abs().max().item()
    assert err <= (1e-4 if dtype == torch.float32 else ATOL), err
    g = nh // nkv
    for i in range(t):
        n = int(row_ctx[i])
        pos = torch.arange(n)
        sl = row_tables[i, pos // bs].long() * bs + pos % bs
        kk = k[sl].double().repeat_interleave(g, 1)  # [n, nh, hd]
        sc = (kk * q[rows[i].long()].double()[None]).sum(-1) * hd**-0.5 / torch.log(
            torch.tensor(2.0, dtype=torch.float64))  # log2 units
        ref = torch.logsumexp(sc * torch.log(torch.tensor(2.0, dtype=torch.float64)), 0) / \
            torch.log(torch.tensor(2.0, dtype=torch.float64))  # fmt: skip
        assert (lse[i].cpu().double() - ref).abs().max().item() <= lse_tol, i


@pytest.mark.parametrize(("nh", "nkv"), [(32, 8), (24, 8), (8, 8), (16, 1)])
@pytest.mark.parametrize("bs", [16, 1, 8])
def test_prefill_groups_and_block_sizes(nh, nkv, bs):
    _say("prefill groups/bs", nh, nkv, bs)
    spec = [(70, 70), (33, 200), (128, 129), (1, 77), (200, 450)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, 128, bs, torch.bfloat16, seed=nh + bs)
    got = _run(q, k, v, tables, ctx, cu, bs, 200)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs, threads=THREADS)
    assert (got - want).abs().max().item() <= ATOL


@pytest.mark.parametrize(("hd", "bs"), [(256, 16), (64, 12), (128, 24), (32, 2)])
def test_prefill_long_contexts_both_key_halves(hd, bs):
    """Contexts of many key tiles, odd and even counts, split between the workgroup's
    two key halves (the second half's tiles all past some rows' causal limit); block
    sizes that are not powers of two take the per-lane gather path."""
    _say("prefill long contexts", hd, bs)
    spec = [(100, 491), (37, 300), (64, 64), (1, 1000), (130, 130)]
    q, k, v, tables, ctx, cu = _chunks(spec, 8, 2, hd, bs, torch.bfloat16, seed=hd + bs)
    got = _run(q, k, v, tables, ctx, cu, bs, 130)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs, threads=THREADS)
    assert (got - want).abs().max().item() <= ATOL


def _check_first_last(spec, q, k, v, tables, cu, got, bs):
    """The oracle on each chunk's first and last 16 query tokens (as their own sub-chunks
    with the same visible keys)."""
    for part in ("first", "last"):
        rows, sub_ctx, sub_cu = [], [], [0]
        for c, (ql, n) in enumerate(spec):
            start = int(cu[c]) + (0 if part == "first" else ql - 16)
            rows.append(torch.arange(start, start + 16))
            # the first 16 queries see keys up to n - ql + 15: a context of n - ql + 16
            sub_ctx.append(n - ql + 16 if part == "first" else n)
            sub_cu.append(sub_cu[-1] + 16)
        rows = torch.cat(rows)
        want = oracle.prefill_attention(q[rows], k, v, tables, torch.tensor(sub_cu, dtype=torch.int32),
                                        torch.tensor(sub_ctx, dtype=torch.int32), bs,
                                        threads=THREADS)  # fmt: skip
        err = (got[rows] - want).abs().max().item()
        assert err <= ATOL, (part, err)


def test_prefill_config5_chunks_first_and_last_tokens():
    """Config 5's prompt chunks (Llama-3-8B shape): 4 chunks of 512 tokens after cached
    prefixes of 0, 1024, 2048, 3072 tokens (512 work items: the whole grid is resident,
    heavy and light items share CUs)."""
    _say("prefill config5")
    bs, nh, nkv, hd = 16, 32, 8, 128
    spec = [(512, 512 + 1024 * i) for i in range(4)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, torch.bfloat16, seed=5)
    got = _run(q, k, v, tables, ctx, cu, bs, 512)
    _check_first_last(spec, q, k, v, tables, cu, got, bs)


def test_prefill_grid_larger_than_the_gpu():
    """Two 2,048-token chunks at the Llama-3-8B shape: 1,024 work items, more than the
    GPU holds at once, so they run heaviest first instead of paired."""
    _say("prefill long chunks")
    bs, nh, nkv, hd = 16, 32, 8, 128
    spec = [(2048, 2048), (2048, 2560)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, torch.bfloat16, seed=6)
    got = _run(q, k, v, tables, ctx, cu, bs, 2048)
    _check_first_last(spec, q, k, v, tables, cu, got, bs)


def test_prefill_whole_prompt_is_causal_attention():
    """A chunk with no cached prefix (ctx == q) is plain causal attention: torch SDPA
    with is_causal=True, computed here in float32 on the gathered rows."""
    _say("prefill causal")
    bs, nh, nkv, hd = 16, 8, 2, 128
    q, k, v, tables, ctx, cu = _chunks([(300, 300)], nh, nkv, hd, bs, torch.bfloat16, seed=9)
    got = _run(q, k, v, tables, ctx, cu, bs, 300)
    slots = (tables[0, torch.arange(300) // bs].long() * bs + torch.arange(300) % bs)
    kk = k[slots].float().permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
    vv = v[slots].float().permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
    want = torch.nn.functional.scaled_dot_product_attention(
        q.float().permute(1, 0, 2), kk, vv, is_causal=True).permute(1, 0, 2)
    assert (got - want).abs().max().item() <= ATOL


def test_prefill_grid_bound_and_empty_chunks():
    """max_query_len larger than every chunk (a graph bucket), and zero-length chunks."""
    _say("prefill bounds")
    spec = [(0, 10), (5, 5), (0, 0), (17, 40)]
    q, k, v, tables, ctx, cu = _chunks(spec, 8, 2, 64, 4, torch.bfloat16, seed=3)
    got = _run(q, k, v, tables, ctx, cu, 4, 256)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, 4, threads=THREADS)
    assert (got - want).abs().max().item() <= ATOL


@pytest.mark.parametrize("n_chunks", [63, 64, 70])
def test_prefill_many_chunks(n_chunks):
    """Up to 63 chunks one wave ranks them (and reads each chunk's offsets from the
    lanes); from 64 on they keep their order and every workgroup loads its own chunk's
    offsets. Both sides of that boundary, ragged lengths and empty chunks included."""
    _say("prefill many chunks", n_chunks)
    g = torch.Generator().manual_seed(n_chunks)
    qs = torch.randint(0, 20, (n_chunks,), generator=g).tolist()
    spec = [(qn, qn + int(torch.randint(0, 60, (1,), generator=g))) for qn in qs]
    q, k, v, tables, ctx, cu = _chunks(spec, 8, 2, 64, 16, torch.bfloat16, seed=n_chunks)
    got = _run(q, k, v, tables, ctx, cu, 16, max(qs))
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, 16, threads=THREADS)
    assert (got - want).abs().max().item() <= ATOL


@pytest.mark.parametrize("hd", [64, 128])
def test_prefill_bf16_values_beyond_fp16(hd):
    """bf16 caches keep V in bf16 on the matrix cores: values outside fp16's range pass
    through. Some V rows of chunks 0 and 2 are scaled by 3e6 and -7e4 (fp16 would hold
    them as +-inf): every output is finite and within 2e-3 of the oracle relative to the
    largest |V| its chunk reads, the other chunks within 2e-3."""
    _say("prefill bf16 V beyond fp16", hd)
    spec = [(40, 300), (33, 33), (64, 500), (1, 90)]
    q, k, v, tables, ctx, cu = _chunks(spec, 8, 2, hd, 16, torch.bfloat16, seed=hd)
    scale = [1.0] * len(spec)
    for c, f in ((0, 3e6), (2, -7e4)):
        blocks = tables[c, : -(-int(ctx[c]) // 16)]
        rows = (blocks[:, None] * 16 + torch.arange(16)).flatten()[::5]
        v[rows, :, : hd // 2] = (v[rows, :, : hd // 2].float() * f).to(torch.bfloat16)
        scale[c] = v[rows].float().abs().max().item()
    assert scale[0] > 65504 and scale[2] > 65504
    got = _run(q, k, v, tables, ctx, cu, 16, max(s for s, _ in spec))
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, 16, threads=THREADS)
    assert torch.isfinite(got).all()
    for c in range(len(spec)):
        lo, hi = int(cu[c]), int(cu[c + 1])
        err = (got[lo:hi] - want[lo:hi]).abs().max().item()
        assert err <= ATOL * scale[c], (c, err, scale[c])


def test_prefill_fp16_tiny_weights_keep_their_mass():
    """fp16 P on the matrix cores: one dominant key (the first) and 60,000 keys whose
    weights (2^-26 of it, ~1.5e-8) lie below half of fp16's smallest subnormal. The first
    key half's 30,000 of them carry ~3.6e-3 of the output through their V of 8, so
    weights rounded to zero in fp16 would miss the 2e-3 bar; the kernel's exponent offset
    scales P by 2^7 so they stay. The second half takes its own exponent reference."""
    import math

    _say("prefill fp16 tiny weights")
    n = 60_001
    q, k, v, tables, ctx, cu = _chunks([(1, n)], 4, 1, 64, 16, torch.float16, seed=6)
    q.zero_()
    q[:, :, 0] = 16.0
    k.zero_()
    v.fill_(8.0)
    dom = int(tables[0, 0]) * 16  # key 0's slot
    # score difference 16 * 9 = 144, times scale * log2(e) = 0.125 * 1.4427: ~26 in log2
    k[dom, :, 0] = 9.0
    v[dom] = 0.0
    got = _run(q, k, v, tables, ctx, cu, 16, 1)
    w = 2.0 ** (-144 * 0.125 / math.log(2))
    want = 8 * (n - 1) * w / (1 + (n - 1) * w)
    assert want > 7e-3
    err = (got[0] - want).abs().max().item()
    assert err < 2e-4, err


def _prefill_c_abi(entry, q, k, v, tables, ctx, cu, bs, max_q, workspace=None):
    """One call of pkv_paged_prefill (entry "plain") or pkv_paged_prefill_ws ("ws", with
    ``workspace``: None = none) through the C ABI; fp32 output on the CPU."""
    from engine.kernels import _native

    nh, hd = q.shape[1], q.shape[2]
    nkv = k.shape[1]
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    td, cd, cud = tables.to(DEV), ctx.to(DEV), cu.to(DEV)
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device=DEV)
    args = [out.data_ptr(), _native.PKV_F32, out.stride(0), out.stride(1), qd.data_ptr(),
            qd.stride(0), qd.stride(1), kd.data_ptr(), vd.data_ptr(), _native.dtype_code(q.dtype, "t"),
            kd.stride(0), kd.stride(1), kd.shape[0], td.data_ptr(), td.stride(0), td.shape[1],
            cd.data_ptr(), cud.data_ptr(), len(ctx), max_q, nh, nkv, hd, bs, hd**-0.5]  # fmt: skip
    stream = torch.cuda.current_stream().cuda_stream
    if entry == "plain":
        st = _native.lib().pkv_paged_prefill(*args, stream)
    else:
        ws = workspace
        st = _native.lib().pkv_paged_prefill_ws(
            *args, ws.data_ptr() if ws is not None else None,
            ws.numel() if ws is not None else 0, stream)  # fmt: skip
    _native.check(st, entry)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize(("nh", "nkv", "hd", "bs"),
                         [(32, 8, 128, 16), (8, 2, 64, 12), (4, 1, 256, 16), (6, 2, 32, 1),
                          (16, 2, 128, 32), (12, 4, 64, 16)])  # fmt: skip
def test_prefill_bf16_fp16_copy_of_v(nh, nkv, hd, bs):
    """bf16 caches through pkv_paged_prefill_ws: each chunk's V copied to fp16 once per
    call, P multiplied once in fp16. Within 2e-3 of the oracle, like the bf16 hi + lo
    product of pkv_paged_prefill on the same inputs; contexts across several 256-token
    tiles of the copy, empty and one-token chunks, block sizes that are not powers of two."""
    _say("prefill fp16 V copy", nh, nkv, hd, bs)
    spec = [(37, 700), (1, 1), (0, 5), (64, 64), (100, 1030), (16, 300)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, torch.bfloat16, seed=hd + bs + nh)
    need = pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, len(spec), tables.shape[1], bs)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ws.fill_(0xFF)  # scratch: whatever it held before must not matter
    got = _prefill_c_abi("ws", q, k, v, tables, ctx, cu, bs, 100, ws)
    hilo = _prefill_c_abi("plain", q, k, v, tables, ctx, cu, bs, 100)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs, threads=THREADS)
    assert (got - want).abs().max().item() <= ATOL
    assert (hilo - want).abs().max().item() <= ATOL
    # the same call again on the dirty workspace: the same bits
    again = _prefill_c_abi("ws", q, k, v, tables, ctx, cu, bs, 100, ws)
    assert torch.equal(got, again)


def test_prefill_workspace_too_small_is_the_plain_call():
    """A workspace below pkv_prefill_workspace_bytes (or none) runs the bf16 hi + lo
    kernel: bit for bit the output of pkv_paged_prefill."""
    _say("prefill small workspace")
    bs, nh, nkv, hd = 16, 8, 2, 128
    spec = [(20, 400), (5, 90)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, torch.bfloat16, seed=21)
    need = pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, len(spec), tables.shape[1], bs)
    plain = _prefill_c_abi("plain", q, k, v, tables, ctx, cu, bs, 20)
    short = torch.empty(need - 16, dtype=torch.uint8, device=DEV)
    assert torch.equal(_prefill_c_abi("ws", q, k, v, tables, ctx, cu, bs, 20, short), plain)
    assert torch.equal(_prefill_c_abi("ws", q, k, v, tables, ctx, cu, bs, 20, None), plain)
    # fp16 caches and tables past 65,536 tokens take no copy: workspace size 0
    assert pa.prefill_workspace_bytes(torch.float16, hd, nkv, 2, 32, bs) == 0
    assert pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, 2, 4097, bs) == 0
    assert pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, 2, 4096, bs) > 0


def test_prefill_fp16_copy_scales_tiles_beyond_fp16():
    """Tiles of the fp16 V copy whose |V| reaches 2^16 are stored times 2^-k and the
    matrix-core kernel rescales its accumulators between tiles of different k: chunk 0
    has a 256-token tile of values near 3e5 between ordinary ones, chunk 1 starts with
    values near -2e5 and goes on with ordinary ones, chunk 2 is ordinary. Each chunk
    within 2e-3 of the oracle relative to the largest |V| it reads."""
    _say("prefill fp16 copy scaled tiles")
    bs, nh, nkv, hd = 16, 8, 2, 128
    spec = [(30, 1000), (40, 700), (20, 300)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, torch.bfloat16, seed=22)

    def rows_of(c, t0, t1):
        pos = torch.arange(t0, t1)
        return tables[c, pos // bs].long() * bs + pos % bs

    big0, big1 = rows_of(0, 256, 512), rows_of(1, 0, 100)
    v[big0] = (v[big0].float() * 3e5).to(torch.bfloat16)
    v[big1] = (v[big1].float() * -2e5).to(torch.bfloat16)
    need = pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, len(spec), tables.shape[1], bs)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    got = _prefill_c_abi("ws", q, k, v, tables, ctx, cu, bs, 40, ws)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs, threads=THREADS)
    assert torch.isfinite(got).all()
    for c, rows in enumerate((big0, big1, None)):
        lo, hi = int(cu[c]), int(cu[c + 1])
        scale = max(1.0, v[rows].float().abs().max().item()) if rows is not None else 1.0
        err = (got[lo:hi] - want[lo:hi]).abs().max().item()
        assert err <= ATOL * scale, (c, err, scale)


def test_prefill_fp16_copy_at_the_widest_table():
    """The fp16 copy at its widest table, 65,536 tokens: one chunk whose context is the
    whole table, so its 256 region tiles' scale exponents fill the kernel's window of four
    bytes per lane. The last tile holds values near 3e6 (a nonzero exponent in the
    window's last byte), and its keys are query 0's head-0 vector doubled, so that
    query attends almost only to that tile and a misread exponent would be off by 2^k.
    Within 2e-3 of the oracle relative to the largest |V|; one block wider takes no
    copy."""
    _say("prefill fp16 copy widest table")
    bs, nh, nkv, hd = 16, 4, 1, 64
    n = 65536
    spec = [(6, n)]
    q, k, v, tables, ctx, cu = _chunks(spec, nh, nkv, hd, bs, torch.bfloat16, seed=23)
    assert tables.shape[1] * bs == n
    pos = torch.arange(n - 256, n)
    big = tables[0, pos // bs].long() * bs + pos % bs
    v[big] = (v[big].float() * 3e6).to(torch.bfloat16)
    k[big, 0] = (q[0, 0].float() * 2).to(torch.bfloat16)
    need = pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, 1, tables.shape[1], bs)
    assert need > 0
    assert pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, 1, tables.shape[1] + 1, bs) == 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ws.fill_(0xFF)
    got = _prefill_c_abi("ws", q, k, v, tables, ctx, cu, bs, 6, ws)
    want = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs, threads=THREADS)
    scale = v[big].float().abs().max().item()
    assert torch.isfinite(got).all()
    assert want[0, 0].abs().max().item() > 0.01 * scale  # query 0 reads the big tile
    assert (got - want).abs().max().item() <= ATOL * scale


@pytest.mark.parametrize("workspace", ["inside", "given"])
def test_prefill_fp16_copy_under_graph_replay(workspace):
    """The two-dispatch bf16 prefill call (fp16 copy of V, then the matrix-core kernel)
    captured in a hipGraph: its workspace allocated inside the capture (from the graph's
    pool) or passed in. Three replays with new queries, new K/V, new block tables and
    context lengths (within the captured table width), eager work and synchronisations
    between them; every replay bit-equal to the eager call and within 2e-3 of the oracle."""
    _say("prefill fp16 copy graph", workspace)
    bs, nh, nkv, hd, width, max_q = 16, 8, 2, 128, 40, 48
    n_chunks = 3
    nblk = n_chunks * width + 4
    k_pool = torch.zeros(nblk * bs, nkv, hd, dtype=torch.bfloat16, device=DEV)
    v_pool = torch.zeros_like(k_pool)
    q_s = torch.zeros(n_chunks * max_q, nh, hd, dtype=torch.bfloat16, device=DEV)
    tables_s = torch.zeros(n_chunks, width, dtype=torch.int32, device=DEV)
    ctx_s = torch.ones(n_chunks, dtype=torch.int32, device=DEV)
    cu_s = torch.zeros(n_chunks + 1, dtype=torch.int32, device=DEV)
    out_s = torch.empty(q_s.shape, dtype=torch.float32, device=DEV)
    ws = None
    if workspace == "given":
        need = pa.prefill_workspace_bytes(torch.bfloat16, hd, nkv, n_chunks, width, bs)
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)

    def body():
        pa.paged_prefill_attention(q_s, k_pool, v_pool, tables_s, ctx_s, bs, cu_s, max_q,
                                   out=out_s, workspace=ws)  # fmt: skip

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        body()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()

    for rep in range(3):
        g = torch.Generator().manual_seed(200 + rep)
        qlen = torch.randint(0, max_q + 1, (n_chunks,), generator=g)
        ctx = torch.clamp(qlen + torch.randint(0, width * bs - max_q, (n_chunks,), generator=g),
                          max=width * bs)  # fmt: skip
        cu = torch.zeros(n_chunks + 1, dtype=torch.int32)
        cu[1:] = qlen.cumsum(0).int()
        q_s.copy_(torch.randn(q_s.shape, generator=g).to(torch.bfloat16))
        k_pool.copy_(torch.randn(k_pool.shape, generator=g).to(torch.bfloat16))
        v_pool.copy_(torch.randn(v_pool.shape, generator=g).to(torch.bfloat16))
        tables_s.copy_(torch.randperm(nblk, generator=g)[: n_chunks * width].view(n_chunks, width).int())
        ctx_s.copy_(ctx.int())
        cu_s.copy_(cu)
        graph.replay()
        torch.cuda.synchronize()
        got = out_s.clone()
        want = torch.empty_like(out_s)
        pa.paged_prefill_attention(q_s, k_pool, v_pool, tables_s, ctx_s, bs, cu_s, max_q,
                                   out=want)  # fmt: skip
        torch.cuda.synchronize()
        rows = int(cu[-1])
        assert torch.equal(got[:rows], want[:rows]), f"replay {rep}"
        ref = oracle.prefill_attention(q_s[:rows].cpu(), k_pool.cpu(), v_pool.cpu(),
                                       tables_s.cpu(), cu, ctx_s.cpu(), bs, threads=THREADS)
        assert (got[:rows].cpu() - ref).abs().max().item() <= ATOL, f"replay {rep}"
