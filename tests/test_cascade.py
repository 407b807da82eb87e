"""Cascade decode over shared prefixes: prefix groups found from the block tables, the
shared blocks attended once per group (chunked-prefill kernel, non-causal), each
sequence's private tail by the decode kernel, which merges the two by log-sum-exp. No counterpart in
the reference (its decode reads every sequence's whole context); the result must be the
same attention (the reference's semantics, engine/kernels/paged_attention.py:192-211)."""

from __future__ import annotations

import os

import pytest
import torch

from engine.kernels import paged_attention as pa

THREADS = min(16, os.cpu_count() or 1)


def _shared_batch(b=12, shared_blocks=20, bs=16, tails=None, extra=3, seed=0, width=None):
    """b sequences, the first b - extra holding the same `shared_blocks` blocks first,
    then private blocks; the last `extra` sequences fully private."""
    g = torch.Generator().manual_seed(seed)
    tails = tails if tails is not None else torch.randint(0, 70, (b,), generator=g).tolist()
    ctx = [shared_blocks * bs + t for t in tails]
    width = width or max(-(-n // bs) for n in ctx) + 2
    nblk = shared_blocks + sum(-(-n // bs) for n in ctx) + 5
    perm = torch.randperm(nblk, generator=g).int()
    tables = torch.zeros(b, width, dtype=torch.int32)
    shared = perm[:shared_blocks]
    at = shared_blocks
    for i in range(b):
        nb = -(-ctx[i] // bs)
        if i < b - extra:
            tables[i, :shared_blocks] = shared
            own = nb - shared_blocks
            tables[i, shared_blocks:nb] = perm[at : at + own]
            at += own
        else:
            tables[i, :nb] = perm[at : at + nb]
            at += nb
    return tables, torch.tensor(ctx, dtype=torch.int32), nblk


def test_prefix_groups_cover_every_context_exactly():
    """Per sequence: its prefix pieces (through the piece tables) followed by its tail
    (through its own table from first_block on) visit exactly its own slots 0 .. n-1."""
    bs = 16
    for seed, tails in ((0, None), (1, [0] * 12), (2, [5, 16, 0, 33, 1, 64, 2, 3, 4, 5, 6, 7])):
        tables, ctx, _ = _shared_batch(tails=tails, seed=seed)
        pg = pa.find_prefix_groups(tables, ctx, bs, 24, 8, "cpu", min_blocks=4,
                                   target_workgroups=200)  # fmt: skip
        assert pg is not None and pg.members == 9
        s_total = pg.members
        for b in range(tables.shape[0]):
            n = int(ctx[b])
            own = [int(tables[b, p // bs]) * bs + p % bs for p in range(n)]
            seen = []
            r = int(pg.prefix_row[b])
            if r >= 0:
                for k in range(pg.pieces):
                    row = r + k * s_total
                    c = int(torch.searchsorted(pg.cu_q, torch.tensor([row], dtype=torch.int32),
                                               right=True)) - 1  # fmt: skip
                    assert int(pg.q_rows[row]) == b
                    for p in range(int(pg.ctx[c])):
                        seen.append(int(pg.tables[c, p // bs]) * bs + p % bs)
            fb = int(pg.first_block[b])
            assert (r >= 0) == (fb > 0)
            seen += [int(tables[b, fb + p // bs]) * bs + p % bs for p in range(n - fb * bs)]
            assert seen == own, b


def test_no_groups_when_nothing_is_shared():
    tables = torch.arange(40, dtype=torch.int32).view(4, 10)
    assert pa.find_prefix_groups(tables, torch.full((4,), 160), 16, 8, 2, "cpu") is None


@pytest.mark.gpu
@pytest.mark.parametrize("wgs", [None, 1, 7])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("nh", "nkv", "hd", "bs"), [(24, 8, 128, 16), (8, 2, 64, 4), (16, 16, 256, 16),
                                                    (8, 4, 32, 16), (16, 4, 64, 32)])  # fmt: skip
def test_cascade_matches_oracle(dtype, nh, nkv, hd, bs, wgs):
    """The prefix parts merge where each sequence finishes: in the decode kernel itself
    for a sequence one workgroup holds whole (every one of them at wgs=1), in the
    combine pass for one cut between workgroups (many at wgs=7)."""
    from oracle import oracle

    dev = torch.device("cuda:0")
    tails = [0, 1, 15, 16, 17, 40, 100, 3, 0, 9, 60, 2]  # empty tails included
    tables, ctx, nblk = _shared_batch(tails=tails, bs=bs, seed=hd)
    g = torch.Generator().manual_seed(7)
    k = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    v = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    q = torch.randn(len(tails), nh, hd, generator=g).to(dtype)
    pg = pa.find_prefix_groups(tables, ctx, bs, nh, nkv, dev, min_blocks=4,
                               target_workgroups=64)  # fmt: skip
    assert pg is not None and pg.pieces > 1
    args = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), bs)
    got32 = torch.empty(q.shape, dtype=torch.float32, device=dev)
    ws = pa.decode_workspace(dev, len(tails), nh, hd, wgs, cascade=True) if wgs else None
    pa.paged_decode_attention(*args, out=got32, prefix_groups=pg, num_workgroups=wgs,
                              workspace=ws)  # fmt: skip
    gotq = pa.paged_decode_attention(*args, prefix_groups=pg, num_workgroups=wgs)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, k, v, tables, ctx, bs, threads=THREADS)
    assert (got32.cpu() - want).abs().max().item() <= 2e-3
    assert torch.equal(gotq.cpu(), got32.cpu().to(dtype))


@pytest.mark.gpu
def test_cascade_config3_matches_plain_decode():
    """Config 3 in full (256 sequences on one 2,048-token prefix, CoW'd last shared
    block for 64 of them): cascade == the plain decode kernel within 1e-3."""
    from engine import workloads
    from engine.runtime.paged_cache import copy_blocks, kv_append

    dev = torch.device("cuda:0")
    step = workloads.config3(dev, seed=0)
    copy_blocks(step.k_cache, step.v_cache, step.cow_mapping, step.block_size)
    kv_append(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)
    nh, nkv = step.q.shape[1], step.k_cache.shape[1]
    pg = pa.find_prefix_groups(step.block_tables.cpu(), step.context_lens.cpu(),
                               step.block_size, nh, nkv, dev)  # fmt: skip
    assert pg is not None and pg.members == step.batch
    args = (step.q, step.k_cache, step.v_cache, step.block_tables, step.context_lens,
            step.block_size)  # fmt: skip
    plain = torch.empty(step.q.shape, dtype=torch.float32, device=dev)
    casc = torch.empty_like(plain)
    pa.paged_decode_attention(*args, out=plain)
    pa.paged_decode_attention(*args, out=casc, prefix_groups=pg)
    torch.cuda.synchronize()
    assert (plain - casc).abs().max().item() <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("wgs", [None, 1000])
def test_cascade_many_parts_and_pieces(wgs):
    """11 prefix parts per sequence (the combine folds them 8 at a time) and, at 1,000
    workgroups, a 2,000-token tail cut into more than 64 pieces (merged 64 records at a
    time): still the oracle's attention."""
    from oracle import oracle

    dev = torch.device("cuda:0")
    tails = [2000, 0, 5, 100, 17, 1, 64, 33, 0, 250, 9, 3]
    tables, ctx, nblk = _shared_batch(tails=tails, shared_blocks=48, bs=16, seed=11)
    g = torch.Generator().manual_seed(12)
    k = torch.randn(nblk * 16, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(nblk * 16, 8, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(len(tails), 24, 128, generator=g).to(torch.bfloat16)
    pg = pa.find_prefix_groups(tables, ctx, 16, 24, 8, dev, min_blocks=4, pieces=11)
    assert pg is not None and pg.pieces == 11
    args = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), 16)
    got = torch.empty(q.shape, dtype=torch.float32, device=dev)
    pa.paged_decode_attention(*args, out=got, prefix_groups=pg, num_workgroups=wgs)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, k, v, tables, ctx, 16, threads=THREADS)
    assert (got.cpu() - want).abs().max().item() <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize(("b", "nh", "nkv", "hd", "bs", "dtype"), [
    (65, 24, 8, 128, 16, torch.bfloat16),
    (130, 32, 8, 64, 32, torch.float16),
    (300, 24, 8, 128, 16, torch.bfloat16),
    (96, 64, 8, 64, 16, torch.bfloat16),    # 8 heads a group: two rows of tasks (grid y 2)
    (200, 16, 16, 128, 16, torch.float16),  # 16 KV heads: two rows of tasks
])  # fmt: skip
@pytest.mark.parametrize("pwg", [None, 1, 7, 10_000])
def test_cascade_one_launch_matches_two_launches(b, nh, nkv, hd, bs, dtype, pwg):
    """Batches of 65-1,024 sequences at head_dim 64/128 run the prefix pass on the first
    workgroups of the decode pass's launch (they then stream a share of the units); the
    library's choice of how many (None), one workgroup taking every prefix item in turn,
    7, and more than the GPU holds (two launches). Five sequences share nothing, tails
    include empty ones. Same result as the two launches within 1e-3 (the unit ranges are
    cut elsewhere), the oracle's within 2e-3."""
    from oracle import oracle

    dev = torch.device("cuda:0")
    print("[case] one launch", b, nh, nkv, hd, bs, dtype, pwg, flush=True)
    tables, ctx, nblk = _shared_batch(b=b, shared_blocks=24, bs=bs, extra=5, seed=b)
    g = torch.Generator().manual_seed(b + 1)
    k = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    v = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    q = torch.randn(b, nh, hd, generator=g).to(dtype)
    assert pa.cascade_one_launch(dtype, hd, nh, nkv, bs, b, dev)
    pg = pa.find_prefix_groups(tables, ctx, bs, nh, nkv, dev, min_blocks=4, dtype=dtype,
                               head_dim=hd)  # fmt: skip
    assert pg is not None and pg.members == b - 5
    args = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), bs)
    one = torch.empty(q.shape, dtype=torch.float32, device=dev)
    two = torch.empty_like(one)
    pa.paged_decode_attention(*args, out=one, prefix_groups=pg, prefix_workgroups=pwg)
    pa.paged_decode_attention(*args, out=two, prefix_groups=pg, prefix_workgroups=-1)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, k, v, tables, ctx, bs, threads=THREADS)
    assert (one - two).abs().max().item() <= 1e-3
    assert (one.cpu() - want).abs().max().item() <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("pieces", [3, 8])
def test_cascade_one_launch_several_items_per_workgroup(pieces):
    """More prefix items than prefix workgroups (3 or 8 pieces of a 40-block prefix for
    256 sequences, 6 row blocks x 8 KV heads each, on 16 prefix workgroups): each
    workgroup runs items back to back, its rings refilled after every merge."""
    from oracle import oracle

    dev = torch.device("cuda:0")
    b, nh, nkv, hd, bs = 256, 24, 8, 128, 16
    tables, ctx, nblk = _shared_batch(b=b, shared_blocks=40, bs=bs, extra=0, seed=pieces)
    g = torch.Generator().manual_seed(pieces)
    k = torch.randn(nblk * bs, nkv, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(nblk * bs, nkv, hd, generator=g).to(torch.bfloat16)
    q = torch.randn(b, nh, hd, generator=g).to(torch.bfloat16)
    pg = pa.find_prefix_groups(tables, ctx, bs, nh, nkv, dev, min_blocks=4, pieces=pieces)
    assert pg.pieces == pieces
    args = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), bs)
    got = torch.empty(q.shape, dtype=torch.float32, device=dev)
    pa.paged_decode_attention(*args, out=got, prefix_groups=pg, prefix_workgroups=16)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, k, v, tables, ctx, bs, threads=THREADS)
    assert (got.cpu() - want).abs().max().item() <= 2e-3


def _static_layout(n, pieces, slots, width, tables, ctx, bs, min_blocks, groups=None):
    """The fixed-shape layout a captured decode step reads (stride n, `slots` chunks per
    piece), filled on the host for one step's tables: (flat int32 array, groups used)."""
    import numpy as np

    flat = np.zeros(pa.prefix_entries(n, pieces, slots, width, n), dtype=np.int32)
    tab = np.zeros((n, tables.shape[1]), dtype=np.int32)
    tab[: tables.shape[0]] = tables.numpy()
    if groups is None:
        groups = pa.shared_prefixes(tab[: tables.shape[0]], ctx.numpy(), bs, min_blocks)
    groups = groups[:slots]
    pa.fill_prefix(flat, n, pieces, slots, width, tab, groups, bs, n)
    return flat, groups


def test_static_prefix_layout_covers_every_context_exactly():
    """The fixed layout of a graph bucket (n rows apart between pieces, a fixed number of
    chunk slots per piece): every grouped sequence's prefix pieces plus its tail visit
    exactly its own slots; rows past the groups' members sit in the piece's last chunk
    with q_rows -1 (whether or not a group holds that chunk); padding rows and
    ungrouped sequences get no prefix; cu_q never decreases and ends at pieces * n."""
    import numpy as np

    bs = 16
    t1, c1, _ = _shared_batch(b=10, shared_blocks=12, tails=[3, 0, 40, 17, 1, 16, 9, 2, 5, 7],
                              extra=3, seed=4)  # fmt: skip
    t2, c2, _ = _shared_batch(b=6, shared_blocks=9, tails=[1, 2, 3, 4, 5, 6], extra=1, seed=5)
    t2 = t2 + 1000  # a second group on other blocks
    w = max(t1.shape[1], t2.shape[1])
    tables = torch.zeros(16, w, dtype=torch.int32)
    tables[:10, : t1.shape[1]] = t1
    tables[10:16, : t2.shape[1]] = t2
    ctx = torch.cat([c1, c2])
    n, pieces = 24, 3  # bucket 24 for 16 sequences
    width = -(-w // pieces)
    for min_blocks, slots in ((4, 4), (4, 2), (4, 1), (10, 1), (100, 1)):
        flat, groups = _static_layout(n, pieces, slots, width, tables, ctx, bs, min_blocks)
        pg = pa.prefix_view(torch.from_numpy(flat), n, pieces, slots, width, members=n,
                             max_members=n)  # fmt: skip
        assert len(groups) == min({4: 2, 10: 1, 100: 0}[min_blocks], slots)
        cu = pg.cu_q.tolist()
        assert cu[0] == 0 and cu[-1] == pieces * n and all(a <= b for a, b in zip(cu, cu[1:]))
        chunk_of = np.searchsorted(np.asarray(cu), np.arange(pieces * n), side="right") - 1
        members = sum(len(m) for m, _ in groups)
        for k in range(pieces):
            for r in range(members, n):  # rows past the members: skipped
                row = k * n + r
                assert int(pg.q_rows[row]) == -1 and chunk_of[row] == k * slots + slots - 1
        for b in range(n):
            r = int(pg.prefix_row[b])
            fb = int(pg.first_block[b])
            if b >= 16:  # padding rows
                assert r == -1 and fb == 0
                continue
            seqn = int(ctx[b])
            own = [int(tables[b, p // bs]) * bs + p % bs for p in range(seqn)]
            seen = []
            if r >= 0:
                for k in range(pieces):
                    row = r + k * n
                    c = chunk_of[row]
                    assert int(pg.q_rows[row]) == b
                    seen += [int(pg.tables[c, p // bs]) * bs + p % bs for p in range(int(pg.ctx[c]))]
            assert (r >= 0) == (fb > 0)
            seen += [int(tables[b, fb + p // bs]) * bs + p % bs for p in range(seqn - fb * bs)]
            assert seen == own, (min_blocks, slots, b)


@pytest.mark.gpu
def test_cascade_static_layout_graph_replays_match_oracle():
    """One captured decode call with fixed-shape prefix groups (what DecodeGraphs holds
    per bucket), replayed over steps whose metadata is rewritten in place: config 3 in
    full (one group of 256), the same batch with no group (plain decode inside the
    graph), and a smaller batch padded to the bucket with two groups -- each replay
    against the oracle, bit-identical replays of one step."""
    import numpy as np

    from engine import workloads
    from engine.runtime.paged_cache import copy_blocks, kv_append
    from oracle import oracle

    dev = torch.device("cuda:0")
    step = workloads.config3(dev, seed=0)
    copy_blocks(step.k_cache, step.v_cache, step.cow_mapping, step.block_size)
    kv_append(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)
    n, nh, hd = step.q.shape
    nkv, bs, w = step.k_cache.shape[1], step.block_size, step.block_tables.shape[1]
    pieces = pa.cascade_pieces(n, nh, nkv, dev)
    slots, width = 2, -(-w // pieces)  # two groups fill both: spare rows join the second's
    meta = torch.zeros(pa.prefix_entries(n, pieces, slots, width, n), dtype=torch.int32,
                       device=dev)  # fmt: skip
    tables = torch.zeros(n, w, dtype=torch.int32, device=dev)
    ctx = torch.ones(n, dtype=torch.int32, device=dev)
    q = step.q.clone()
    out = torch.empty(n, nh, hd, dtype=torch.float32, device=dev)
    pg = pa.prefix_view(meta, n, pieces, slots, width, members=n, max_members=n)

    def call():
        pa.paged_decode_attention(q, step.k_cache, step.v_cache, tables, ctx, bs, out=out,
                                  prefix_groups=pg)  # fmt: skip

    def load(tab, cx, qq, min_blocks):
        b = tab.shape[0]
        flat, groups = _static_layout(n, pieces, slots, width, tab, cx, bs, min_blocks)
        meta.copy_(torch.from_numpy(flat))
        tables.zero_()
        tables[:b] = tab.to(dev)
        ctx.fill_(1)
        ctx[:b] = cx.to(dev)
        q[:b] = qq
        return groups

    load(step.block_tables.cpu(), step.context_lens.cpu(), step.q, 16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()

    # a smaller batch: sequences 0-99 keep the group, 100-179 move to a second group on
    # copies of the prefix blocks, padded to 256 rows
    small_tab = step.block_tables[:180].cpu().clone()
    used = set(step.block_tables.flatten().tolist()) | set(step.cow_mapping.flatten().tolist())
    free = torch.tensor([x for x in range(step.k_cache.shape[0] // bs) if x not in used][:127],
                        dtype=torch.int64)  # fmt: skip
    assert free.numel() == 127
    pairs = torch.stack([step.block_tables[150, :127].long().cpu(), free], 1).to(dev)
    copy_blocks(step.k_cache, step.v_cache, pairs, bs)
    small_tab[100:180, :127] = free.to(torch.int32)
    cases = [("config 3, one group", step.block_tables.cpu(), step.context_lens.cpu(), 16, 1),
             ("config 3, no group", step.block_tables.cpu(), step.context_lens.cpu(), 10**6, 0),
             ("180 of 256 rows, two groups", small_tab, step.context_lens[:180].cpu(), 16, 2)]
    kc, vc = step.k_cache.cpu(), step.v_cache.cpu()
    for name, tab, cx, min_blocks, n_groups in cases:
        print("[case]", name, flush=True)
        groups = load(tab, cx, step.q[: tab.shape[0]], min_blocks)
        assert len(groups) == n_groups
        graph.replay()
        torch.cuda.synchronize()
        first = out.clone()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first), name
        b = tab.shape[0]
        want = oracle.decode_attention(step.q[:b].cpu(), kc, vc, tab, cx, bs, threads=THREADS)
        err = (out[:b].cpu() - want).abs().max().item()
        assert err <= 2e-3, (name, err)
        assert np.isfinite(out.cpu().numpy()).all(), name


def test_prefix_groups_must_match_the_call():
    """A PrefixGroups built for another step is refused before any launch: the kernels
    read first_block[b] and prefix_row[b] for every sequence b and the prefix pass's
    tables by chunk, so wrong lengths, dtypes or layouts would read out of bounds."""
    import dataclasses

    tables, ctx, _ = _shared_batch(seed=3)
    pg = pa.find_prefix_groups(tables, ctx, 16, 24, 8, "cpu", min_blocks=4,
                               target_workgroups=64)  # fmt: skip
    cpu = torch.device("cpu")
    b = tables.shape[0]
    pa._check_prefix_groups(pg, b, cpu, "t")  # the step it was built for
    with pytest.raises(ValueError, match="built for"):
        pa._check_prefix_groups(pg, b + 1, cpu, "t")
    for name in ("first_block", "prefix_row", "q_rows", "cu_q", "ctx", "tables"):
        t = getattr(pg, name)
        for bad in (t.long(), t.t() if t.dim() == 2 else t[::2]):
            if bad.dtype == torch.int32 and bad.is_contiguous() and bad.shape == t.shape:
                continue
            with pytest.raises(ValueError):
                pa._check_prefix_groups(dataclasses.replace(pg, **{name: bad}), b, cpu, "t")
    with pytest.raises(ValueError, match="disagree"):
        pa._check_prefix_groups(dataclasses.replace(pg, pieces=pg.pieces + 1), b, cpu, "t")
    with pytest.raises(ValueError, match="disagree"):
        pa._check_prefix_groups(dataclasses.replace(pg, cu_q=pg.cu_q[:-1].contiguous()), b,
                                cpu, "t")  # fmt: skip


@pytest.mark.gpu
def test_decode_refuses_prefix_groups_of_another_step():
    """Through paged_decode_attention on the GPU: groups built for a 12-sequence step,
    called with 11 sequences, raise ValueError and launch nothing."""
    dev = torch.device("cuda:0")
    tables, ctx, nblk = _shared_batch(seed=8)
    k = torch.randn(nblk * 16, 8, 128, device=dev).to(torch.bfloat16)
    q = torch.randn(tables.shape[0], 24, 128, device=dev).to(torch.bfloat16)
    pg = pa.find_prefix_groups(tables, ctx, 16, 24, 8, dev, min_blocks=4)
    assert pg is not None
    with pytest.raises(ValueError, match="built for"):
        pa.paged_decode_attention(q[:-1], k, k, tables[:-1].to(dev), ctx[:-1].to(dev), 16,
                                  prefix_groups=pg)  # fmt: skip


def _groups_batch(r, b, n_groups, bs, tail_max):
    """b sequences: n_groups groups each sharing its own run of 4-40 leading blocks (two
    or more members), the rest private; tails of 0..tail_max tokens."""
    sizes, left = [], b
    for g in range(n_groups):
        k = r.randint(2, max(2, left // (n_groups - g) if g < n_groups - 1 else left))
        k = min(k, left - 2 * (n_groups - g - 1))
        sizes.append(k)
        left -= k
    shared = [r.randint(4, 40) for _ in sizes]
    tails = [r.choice([0, 1, r.randint(2, tail_max)]) for _ in range(b)]
    member_of = []
    for g, k in enumerate(sizes):
        member_of += [g] * k
    member_of += [-1] * (b - len(member_of))
    r.shuffle(member_of)
    ctx = [(shared[g] * bs if g >= 0 else 0) + t + (1 if g < 0 else 0) for g, t in zip(member_of, tails)]
    width = max(-(-n // bs) for n in ctx) + 1
    nblk = sum(shared) + sum(-(-n // bs) for n in ctx) + 4
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(r.randint(0, 1 << 30)))
    at = 0
    prefix = []
    for sh in shared:
        prefix.append(perm[at : at + sh].int())
        at += sh
    tables = torch.zeros(b, width, dtype=torch.int32)
    for i, (g, n) in enumerate(zip(member_of, ctx)):
        nb = -(-n // bs)
        head = 0
        if g >= 0:
            tables[i, : shared[g]] = prefix[g]
            head = shared[g]
        tables[i, head:nb] = perm[at : at + nb - head].int()
        at += nb - head
    return tables, torch.tensor(ctx, dtype=torch.int32), nblk


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(14 * max(1, int(os.environ.get("PKV_RANDOM_CASES_SCALE", "1")))))
def test_cascade_random_shapes(seed):
    """Seeded random cascade steps: 65-600 sequences in 1-3 prefix groups (shared runs of
    4-40 blocks) plus private sequences, empty and short tails, head_dim 64/128, groups
    1-8, blocks of 16/32/64 tokens, bf16/fp16, pieces and prefix workgroups drawn or left
    to the library; one launch where the shapes allow, two launches otherwise. Against
    the oracle within 2e-3, and against the two-launch form within 1e-3."""
    import random

    from oracle import oracle

    r = random.Random(4000 + seed)
    dev = torch.device("cuda:0")
    hd = r.choice([64, 128])
    nkv = r.choice([1, 2, 8])
    groups = r.choice([1, 2, 3, 4, 8])
    bs = r.choice([16, 32, 64])
    dtype = r.choice([torch.bfloat16, torch.float16])
    b = r.choice([65, r.randint(66, 300), r.randint(300, 600)])
    n_groups = r.choice([1, 1, 2, 3])
    pieces = r.choice([None, None, 1, 2, 4])
    pwg = r.choice([None, None, 1, 9, 40])
    nh = nkv * groups
    tables, ctx, nblk = _groups_batch(r, b, n_groups, bs, 200)
    print("[case] cascade random", seed, dict(b=b, hd=hd, nkv=nkv, groups=groups, bs=bs,
                                              dtype=dtype, n_groups=n_groups, pieces=pieces,
                                              pwg=pwg), flush=True)  # fmt: skip
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    v = torch.randn(nblk * bs, nkv, hd, generator=g).to(dtype)
    q = torch.randn(b, nh, hd, generator=g).to(dtype)
    pg = pa.find_prefix_groups(tables, ctx, bs, nh, nkv, dev, min_blocks=4, pieces=pieces,
                               dtype=dtype, head_dim=hd)  # fmt: skip
    assert pg is not None
    args = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), bs)
    one = torch.empty(q.shape, dtype=torch.float32, device=dev)
    two = torch.empty_like(one)
    pa.paged_decode_attention(*args, out=one, prefix_groups=pg, prefix_workgroups=pwg)
    pa.paged_decode_attention(*args, out=two, prefix_groups=pg, prefix_workgroups=-1)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, k, v, tables, ctx, bs, threads=THREADS)
    assert (one.cpu() - want).abs().max().item() <= 2e-3
    assert (one - two).abs().max().item() <= 1e-3
