"""Pins the CPU oracle (oracle/paged_kv_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something independent of its own formula:
torch library routines (Tensor.to, index_copy_, scaled_dot_product_attention in
float64), closed-form special cases, and brute force on tiny inputs. The sensitivity
tests plant plausible mistakes in the oracle's *inputs* (a wrong GQA head mapping, a
dropped scale, an off-by-one block index) and require the checks to catch them.

The reference stores no numeric golden vectors for this path (its kernel tests compare
against its own PyTorch oracle, reference tests/test_kernels.py:17-37); the shapes and
context lengths those tests use are in tests/golden/reference_kernel_cases.json.
"""

from __future__ import annotations

import json
import math
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kernel_cases.json")


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16)


def _special_floats() -> torch.Tensor:
    vals = [0.0, -0.0, 1.0, -1.0, math.inf, -math.inf, 65504.0, 65519.99, 65520.0, 70000.0,
            6.1035156e-05, 6.0e-08, 2.98e-08, 5.96e-08, 1e-45, -1e-45, 3.0e38, -3.0e38,
            1.00390625, 1.0078125, 1.01171875]  # fmt: skip
    # Every bf16 / fp16 rounding tie: x.5 ulp patterns above 1 and in the subnormal range.
    ties = [1.0 + (2 * i + 1) * 2.0**-9 for i in range(16)]
    ties += [1.0 + (2 * i + 1) * 2.0**-11 for i in range(16)]
    ties += [(2 * i + 1) * 2.0**-25 for i in range(16)]
    return torch.tensor(vals + ties + [-t for t in ties], dtype=torch.float32)


def _random_floats(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    bits = torch.randint(-(2**31), 2**31, (n,), generator=g, dtype=torch.int64).to(torch.int32)
    x = bits.view(torch.float32)
    x = x[~torch.isnan(x)]
    return torch.cat([x, torch.randn(n, generator=g) * 100, torch.randn(n, generator=g) * 1e-5])


# ---- conversions: pinned to torch's Tensor.to() (a library routine) ----------------------


def test_f32_to_bf16_matches_torch(oracle_lib):
    x = torch.cat([_special_floats(), _random_floats(200_000, 1)])
    assert torch.equal(oracle.to_bf16_bits(x), _bits(x.to(torch.bfloat16)))


def test_f32_to_bf16_nan_is_canonical(oracle_lib):
    nans = torch.tensor([0x7FC00001, 0x7F800001, -0x00400000, 0x7FFFFFFF],
                        dtype=torch.int32).view(torch.float32)  # fmt: skip
    got = oracle.to_bf16_bits(nans)
    # c10's scalar rounding (used by torch on ROCm devices) returns 0x7FC0 for every NaN;
    # torch's vectorised CPU path returns 0xFFFF instead, so on the CPU only NaN-ness is
    # comparable. The GPU tests compare the kernel with torch's device conversion.
    assert (got == 0x7FC0).all()
    assert torch.isnan(nans.to(torch.bfloat16)).all()


def test_f32_to_f16_matches_torch(oracle_lib):
    x = torch.cat([_special_floats(), _random_floats(200_000, 2)])
    assert torch.equal(oracle.to_f16_bits(x), _bits(x.to(torch.float16)))


def test_f16_bf16_to_f32_exhaustive(oracle_lib):
    allbits = torch.arange(-(2**15), 2**15, dtype=torch.int32).to(torch.int16)
    want16 = allbits.view(torch.float16).float()
    got16 = oracle.from_f16_bits(allbits)
    same = (got16 == want16) | (torch.isnan(got16) & torch.isnan(want16))
    assert same.all()
    wantb = allbits.view(torch.bfloat16).float()
    gotb = oracle.from_bf16_bits(allbits)
    assert torch.equal(gotb.view(torch.int32), wantb.view(torch.int32))


# ---- KV append: pinned to index_copy_ ----------------------------------------------------


@pytest.mark.parametrize(
    ("pool_dt", "new_dt"),
    [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
     (torch.float32, torch.float32), (torch.bfloat16, torch.float32),
     (torch.float16, torch.float32), (torch.float32, torch.bfloat16),
     (torch.float16, torch.bfloat16)],
)  # fmt: skip
def test_kv_append_matches_index_copy(oracle_lib, pool_dt, new_dt):
    g = torch.Generator().manual_seed(3)
    slots_n, nkv, hd, n = 96, 4, 32, 20
    k_pool = torch.randn(slots_n, nkv, hd, generator=g).to(pool_dt)
    v_pool = torch.randn(slots_n, nkv, hd, generator=g).to(pool_dt)
    # The call-site layout: a transposed [nkv, N, hd] projection (reference layers.py:200).
    k = torch.randn(nkv, n, hd, generator=g).to(new_dt).transpose(0, 1)
    v = torch.randn(nkv, n, hd, generator=g).to(new_dt).transpose(0, 1)
    slots = torch.randperm(slots_n, generator=g)[:n]
    want_k, want_v = k_pool.clone(), v_pool.clone()
    want_k.index_copy_(0, slots, k.to(pool_dt))
    want_v.index_copy_(0, slots, v.to(pool_dt))
    oracle.kv_append(k_pool, v_pool, k, v, slots)
    assert torch.equal(_bits(k_pool) if pool_dt != torch.float32 else k_pool,
                       _bits(want_k) if pool_dt != torch.float32 else want_k)  # fmt: skip
    assert torch.equal(v_pool.view(torch.uint8), want_v.view(torch.uint8))


def test_kv_append_skips_out_of_range_and_brute_force(oracle_lib):
    k_pool = torch.zeros(8, 1, 4, dtype=torch.float32)
    v_pool = torch.zeros(8, 1, 4, dtype=torch.float32)
    k = torch.arange(16, dtype=torch.float32).view(4, 1, 4)
    v = -k
    slots = torch.tensor([7, -1, 8, 2])
    oracle.kv_append(k_pool, v_pool, k, v, slots)
    want = torch.zeros(8, 1, 4)
    want[7], want[2] = k[0], k[3]
    assert torch.equal(k_pool, want) and torch.equal(v_pool, -want)


# ---- block copy: pinned to slice assignment ------------------------------------------------


def test_copy_blocks_matches_slices(oracle_lib):
    g = torch.Generator().manual_seed(4)
    layers, nblk, bs, nkv, hd = 3, 10, 4, 2, 8
    k = torch.randn(layers, nblk * bs, nkv, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(layers, nblk * bs, nkv, hd, generator=g).to(torch.bfloat16)
    pairs = torch.tensor([[1, 5], [1, 6], [3, 0], [9, 12]])  # last pair out of range: skipped
    want_k, want_v = k.clone(), v.clone()
    for s, d in pairs.tolist():
        if d >= nblk:
            continue
        want_k[:, d * bs : (d + 1) * bs] = want_k[:, s * bs : (s + 1) * bs]
        want_v[:, d * bs : (d + 1) * bs] = want_v[:, s * bs : (s + 1) * bs]
    oracle.copy_blocks(k, v, pairs, bs)
    assert torch.equal(_bits(k), _bits(want_k)) and torch.equal(_bits(v), _bits(want_v))


# ---- decode attention: pinned to float64 SDPA over the dense gather ----------------------


def _sdpa_decode(q, k_cache, v_cache, tables, ctx, bs):
    """Independent statement: gather each context densely, repeat KV heads, float64 SDPA."""
    b, nh, hd = q.shape
    nkv = k_cache.shape[1]
    outs = []
    for i in range(b):
        n = int(ctx[i])
        if n == 0:
            outs.append(torch.zeros(nh, hd, dtype=torch.float64))
            continue
        slots = torch.tensor([int(tables[i, p // bs]) * bs + p % bs for p in range(n)])
        kk = k_cache[slots].double().permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
        vv = v_cache[slots].double().permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
        o = F.scaled_dot_product_attention(q[i].double()[:, None, :], kk, vv)
        outs.append(o[:, 0])
    return torch.stack(outs)


def _golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("nh", "nkv", "hd"), [(32, 8, 64), (24, 8, 128), (4, 2, 16)])
@pytest.mark.parametrize("block_size", [4, 16])
def test_decode_matches_sdpa(oracle_lib, dtype, nh, nkv, hd, block_size):
    """The reference kernel test's own matrix (reference tests/test_kernels.py:17-37)."""
    case = _golden_cases()["test_paged_decode_matches_reference"]
    assert [nh, nkv, hd] in case["heads"] and block_size in case["block_sizes"]
    ctx = torch.tensor(case["context_lens"], dtype=torch.int32)
    g = torch.Generator().manual_seed(0)
    b = len(ctx)
    max_blocks = -(-int(ctx.max()) // block_size)
    nblk = b * max_blocks + 3
    tables = torch.randperm(nblk, generator=g)[: b * max_blocks].int().view(b, max_blocks)
    k = torch.randn(nblk * block_size, nkv, hd, generator=g).to(dtype)
    v = torch.randn(nblk * block_size, nkv, hd, generator=g).to(dtype)
    q = torch.randn(b, nh, hd, generator=g).to(dtype)
    got = oracle.decode_attention(q, k, v, tables, ctx, block_size)
    want = _sdpa_decode(q, k, v, tables, ctx, block_size)
    assert (got.double() - want).abs().max().item() < 1e-5


def test_decode_special_cases(oracle_lib):
    bs, nkv, nh, hd = 4, 2, 6, 16
    g = torch.Generator().manual_seed(5)
    nblk = 12
    k = torch.randn(nblk * bs, nkv, hd, generator=g)
    v = torch.randn(nblk * bs, nkv, hd, generator=g)
    tables = torch.randperm(nblk, generator=g)[:9].int().view(3, 3)
    q = torch.randn(3, nh, hd, generator=g)
    # ctx = 1: the output is the single V row of the first slot, for every query head.
    ctx1 = torch.tensor([1, 1, 1], dtype=torch.int32)
    out = oracle.decode_attention(q, k, v, tables, ctx1, bs)
    for i in range(3):
        slot = int(tables[i, 0]) * bs
        for h in range(nh):
            assert torch.allclose(out[i, h], v[slot, h // (nh // nkv)], atol=1e-7)
    # Identical keys: uniform weights, the output is the mean of the context's V rows.
    kc = k.clone()
    kc[:] = kc[0]
    ctx = torch.tensor([5, 12, 9], dtype=torch.int32)
    out = oracle.decode_attention(q, kc, v, tables, ctx, bs)
    for i in range(3):
        n = int(ctx[i])
        slots = [int(tables[i, p // bs]) * bs + p % bs for p in range(n)]
        mean = v[slots].mean(0)  # [nkv, hd]
        assert torch.allclose(out[i], mean.repeat_interleave(nh // nkv, 0), atol=1e-6)
    # Empty context gives zeros.
    out = oracle.decode_attention(q, k, v, tables, torch.tensor([0, 3, 0], dtype=torch.int32), bs)
    assert (out[0] == 0).all() and (out[2] == 0).all()


def test_decode_dominant_score_picks_one_row(oracle_lib):
    bs, nkv, nh, hd = 4, 1, 1, 16
    nblk = 4
    g = torch.Generator().manual_seed(6)
    k = torch.randn(nblk * bs, nkv, hd, generator=g) * 0.01
    v = torch.randn(nblk * bs, nkv, hd, generator=g)
    tables = torch.tensor([[2, 0, 3]], dtype=torch.int32)
    target = 3 * bs + 1  # position 9 of the context (block 3, offset 1)
    k[target, 0] = 40.0
    q = torch.ones(1, nh, hd)
    out = oracle.decode_attention(q, k, v, tables, torch.tensor([10], dtype=torch.int32), bs)
    assert torch.allclose(out[0, 0], v[target, 0], atol=1e-6)


def test_decode_identity_table_is_dense_attention(oracle_lib):
    """bs = 1 with table[p] = p reduces to dense attention: causal-free SDPA in float64."""
    g = torch.Generator().manual_seed(7)
    n, nkv, nh, hd = 37, 2, 4, 32
    k = torch.randn(n, nkv, hd, generator=g)
    v = torch.randn(n, nkv, hd, generator=g)
    q = torch.randn(1, nh, hd, generator=g)
    tables = torch.arange(n, dtype=torch.int32)[None]
    out = oracle.decode_attention(q, k, v, tables, torch.tensor([n], dtype=torch.int32), 1)
    kk = k.double().permute(1, 0, 2).repeat_interleave(2, 0)
    vv = v.double().permute(1, 0, 2).repeat_interleave(2, 0)
    want = F.scaled_dot_product_attention(q[0].double()[:, None], kk, vv)[:, 0]
    assert (out[0].double() - want).abs().max() < 1e-6


# ---- sensitivity: plausible mistakes must fail the checks --------------------------------


def _case(dtype=torch.float32, seed=8):
    g = torch.Generator().manual_seed(seed)
    bs, nkv, nh, hd = 4, 2, 8, 16
    ctx = torch.tensor([7, 30, 13], dtype=torch.int32)
    nblk = 30
    tables = torch.randperm(nblk, generator=g)[:24].int().view(3, 8)
    k = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    v = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    q = torch.randn(3, nh, hd, generator=g).to(dtype)
    return q, k, v, tables, ctx, bs


def test_sensitivity_wrong_gqa_mapping_is_caught(oracle_lib):
    q, k, v, tables, ctx, bs = _case()
    want = _sdpa_decode(q, k, v, tables, ctx, bs)
    nh, nkv = q.shape[1], k.shape[1]
    # h % nkv instead of h // G: permute the query heads so head h lands on KV head h % nkv.
    perm = torch.tensor([(h % nkv) * (nh // nkv) + h // nkv for h in range(nh)])
    mutant = oracle.decode_attention(q[:, perm], k, v, tables, ctx, bs)[:, perm.argsort()]
    assert (mutant.double() - want).abs().max() > 1e-2


def test_sensitivity_missing_scale_is_caught(oracle_lib):
    q, k, v, tables, ctx, bs = _case()
    want = _sdpa_decode(q, k, v, tables, ctx, bs)
    mutant = oracle.decode_attention(q, k, v, tables, ctx, bs, scale=1.0)
    assert (mutant.double() - want).abs().max() > 1e-2


def test_sensitivity_off_by_one_block_is_caught(oracle_lib):
    q, k, v, tables, ctx, bs = _case()
    want = _sdpa_decode(q, k, v, tables, ctx, bs)
    shifted = torch.roll(tables, 1, dims=1)
    mutant = oracle.decode_attention(q, k, v, shifted, ctx, bs)
    assert (mutant.double() - want).abs().max() > 1e-2


# ---- split-K combine: combine(partials over any partition) == single pass ----------------


@pytest.mark.parametrize("split_tokens", [1, 3, 4, 16, 64, 1000])
def test_combine_equals_single_pass(oracle_lib, split_tokens):
    q, k, v, tables, ctx, bs = _case(torch.bfloat16, seed=9)
    n_splits = -(-int(ctx.max()) // split_tokens) + 2  # trailing splits are empty
    ml, acc = oracle.decode_partials(q, k, v, tables, ctx, bs, split_tokens, n_splits)
    got = oracle.combine(ml, acc)
    want = oracle.decode_attention(q, k, v, tables, ctx, bs)
    assert (got - want).abs().max() < 1e-6
    # Each partial alone is the softmax over its own slice: l = sum exp(s - m) > 0 for
    # live splits and the per-split normalised output is a convex combination of V rows.
    live = ml[..., 1] > 0
    assert torch.isfinite(ml[..., 0][live]).all()


# ---- chunked prefill: bottom-right causal, pinned to masked SDPA ------------------------


def test_prefill_matches_masked_sdpa(oracle_lib):
    g = torch.Generator().manual_seed(10)
    bs, nkv, nh, hd = 4, 2, 4, 16
    chunks = [(6, 6), (5, 13), (3, 20), (1, 1)]  # (new tokens, context) as in reference :199
    nblk = 40
    perm = torch.randperm(nblk, generator=g)
    w = -(-max(c for _, c in chunks) // bs)
    tables = torch.zeros(len(chunks), w, dtype=torch.int32)
    at = 0
    for i, (_, c) in enumerate(chunks):
        nb = -(-c // bs)
        tables[i, :nb] = perm[at : at + nb].int()
        at += nb
    k = torch.randn(nblk * bs, nkv, hd, generator=g)
    v = torch.randn(nblk * bs, nkv, hd, generator=g)
    qlens = [q for q, _ in chunks]
    cu = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0)), dtype=torch.int32)
    q = torch.randn(int(cu[-1]), nh, hd, generator=g)
    ctx = torch.tensor([c for _, c in chunks], dtype=torch.int32)
    got = oracle.prefill_attention(q, k, v, tables, cu, ctx, bs)
    for i, (n, c) in enumerate(chunks):
        slots = torch.tensor([int(tables[i, p // bs]) * bs + p % bs for p in range(c)])
        kk = k[slots].double().permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
        vv = v[slots].double().permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
        qq = q[cu[i] : cu[i + 1]].double().permute(1, 0, 2)
        # The reference's FP32 chunk mask (paged_cache.py:190-191).
        mask = torch.arange(c)[None, :] <= (c - n) + torch.arange(n)[:, None]
        want = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask).permute(1, 0, 2)
        assert (got[cu[i] : cu[i + 1]].double() - want).abs().max() < 1e-6
        if c == n:  # whole prompt in one chunk: plain causal attention
            want_c = F.scaled_dot_product_attention(qq, kk, vv, is_causal=True).permute(1, 0, 2)
            assert (got[cu[i] : cu[i + 1]].double() - want_c).abs().max() < 1e-6
