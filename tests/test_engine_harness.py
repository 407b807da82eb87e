"""End-to-end greedy-token identity through the paged path.

CPU tests (torch-only "reference" attention backend) pin the harness itself: block
tables, chunked prefill, prefix-cache hits, fork with copy-on-write and the
``PagedBatch`` metadata must give the static loop's tokens. The GPU tests run the same
engine on the HIP kernels (tests/test_kernels.py:40-179 of the reference is the
pattern: engine tokens == static-loop tokens, graphs == eager, mixed steps)."""

from __future__ import annotations

import pytest
import torch

from engine.runtime.paged_cache import PagedBatch, PagedKVCache
from tiny_llama import ReferenceBackend, TinyConfig, TinyEngine, TinyLlama, static_greedy

SHARED = [7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18]
PROMPTS = {"a": [5, 6, 7], "b": SHARED + [1, 2], "c": [99], "d": SHARED + [3],
           "e": list(range(20, 41)), "f": SHARED}  # fmt: skip


def _model(dtype=torch.float32, device="cpu", **cfg) -> TinyLlama:
    torch.manual_seed(0)
    return TinyLlama(TinyConfig(**cfg), seed=0).to(device=device, dtype=dtype).eval()


def _oracle(model, prompts, max_tokens):
    return {rid: static_greedy(model, p, max_tokens) for rid, p in prompts.items()}


def _check_logits(eng, prompts, max_tokens, atol):
    """Every sampled token's logits against the static loop's (same tokens assumed)."""
    worst = 0.0
    for rid, p in prompts.items():
        _, want = static_greedy(eng.model, p, max_tokens, with_logits=True)
        got = torch.stack(eng.logits[rid])
        worst = max(worst, (got - want).abs().max().item())
    assert worst <= atol, f"logits differ from the static loop by {worst}"
    return worst


def _run_staggered(eng: TinyEngine, prompts, max_tokens):
    """Prompts join one per step while earlier ones decode: mixed steps."""
    got = {rid: [] for rid in prompts}
    pending = list(prompts.items())
    while pending or eng.has_unfinished():
        if pending:
            rid, p = pending.pop(0)
            eng.add_request(rid, p, max_tokens)
        for rid, tok in eng.step():
            got[rid].append(tok)
    return got


def test_paged_batch_metadata_matches_definitions():
    """slot_mapping, chunk offsets and per-token causal contexts against their
    definitions (reference engine/runtime/paged_cache.py:80-229)."""
    cfg = TinyConfig()
    cache = PagedKVCache(cfg, 40, 4, "cpu", torch.float32)
    tables = [[3, 9, 1], [0], [5, 6, 7, 8], [2, 4]]
    ctx = [10, 1, 13, 6]
    qlen = [1, 1, 5, 6]  # two decode rows, a later chunk, a whole prompt
    b = PagedBatch.build(cache, tables, ctx, qlen, "cpu", use_kernel=True)
    # The reference's dispatch (layers.py:200-212) tests use_kernel before mixed:
    # mixed batches must not claim the decode kernel; chunks stay empty, varlen None.
    assert b.mixed and not b.use_kernel and b.chunks == [] and b.varlen is None
    want_slots = [t[p // 4] * 4 + p % 4 for t, n, q in zip(tables, ctx, qlen)
                  for p in range(n - q, n)]  # fmt: skip
    assert b.slot_mapping.tolist() == want_slots
    assert b.last_index.tolist() == [0, 1, 6, 12]
    assert b.decode_rows.tolist() == [0, 1]
    assert b.context_lens.tolist() == [10, 1]
    assert b.chunk_rows.tolist() == list(range(2, 13))
    assert b.cu_seqlens_q.tolist() == [0, 5, 11] and b.max_query_len == 6
    assert b.chunk_ctx.tolist() == [13, 6]
    assert b.chunk_tables[0].tolist() == [5, 6, 7, 8] and b.chunk_tables[1].tolist()[:2] == [2, 4]
    d = PagedBatch.build(cache, tables[:2], ctx[:2], [1, 1], "cpu", use_kernel=True)
    assert d.use_kernel and not d.mixed and d.slot_mapping.tolist() == want_slots[:2]
    assert d.block_tables.tolist() == [[3, 9, 1], [0, 0, 0]]  # padded with block 0
    # One sequence's prompt with the kernel: a mixed batch (the chunk kernel takes it).
    one = PagedBatch.build(cache, tables[2:3], ctx[2:3], qlen[2:3], "cpu", use_kernel=True)
    assert one.mixed and not one.use_kernel and one.block_tables is None
    assert one.chunk_rows.tolist() == list(range(5)) and one.decode_rows.numel() == 0
    with pytest.raises(ValueError):
        PagedBatch.build(cache, [[1]], [9], [2], "cpu", use_kernel=True)  # table too short


def test_paged_batch_gather_metadata_matches_definitions():
    """use_kernel=False: the reference's gather metadata (paged_cache.py:100-127) --
    every context slot, padded query indices and the bottom-right causal mask."""
    cfg = TinyConfig()
    cache = PagedKVCache(cfg, 40, 4, "cpu", torch.float32)
    tables = [[3, 9, 1], [5, 6, 7, 8]]
    ctx, qlen = [10, 13], [1, 5]
    g = PagedBatch.build(cache, tables, ctx, qlen, "cpu")
    assert not g.use_kernel and not g.mixed
    for i, (t, n) in enumerate(zip(tables, ctx)):
        assert g.kv_slots[i, :n].tolist() == [t[p // 4] * 4 + p % 4 for p in range(n)]
    assert g.slot_mapping.tolist() == [g.kv_slots[0, 9].item()] + g.kv_slots[1, 8:13].tolist()
    assert g.q_valid.tolist() == [[True] + [False] * 4, [True] * 5]
    assert g.q_index.tolist() == [[0, 0, 0, 0, 0], [1, 2, 3, 4, 5]]
    assert g.last_index.tolist() == [0, 5]
    m = g.attn_mask[:, 0]
    assert m.shape == (2, 5, 13)
    assert m[0, 0].tolist() == [True] * 10 + [False] * 3  # decode row: its whole context
    # Padded query rows: keys k <= n - q + i inside the context, plus key 0 always.
    for i in range(1, 5):
        assert m[0, i].tolist() == [(k <= 9 + i and k < 10) or k == 0 for k in range(13)]
    assert m[1].any(-1).all()  # no row is fully masked
    for i in range(5):  # query i of the chunk sits at 8 + i
        assert m[1, i].tolist() == [k <= 8 + i for k in range(13)]


def test_paged_batch_cascade_groups():
    """Decode steps with cascade: sequences whose tables start with the same blocks get
    prefix groups (their shared blocks, fully covered); nothing shared: none."""
    cfg = TinyConfig()
    cache = PagedKVCache(cfg, 32, 4, "cpu", torch.float32)
    shared = [1, 2, 3]
    tables = [shared + [10, 11], shared + [12], [20, 21, 22, 23]]
    b = PagedBatch.build(cache, tables, [18, 14, 15], [1, 1, 1], "cpu", use_kernel=True,
                         cascade=True, num_heads=cfg.num_attention_heads,
                         cascade_min_blocks=2)  # fmt: skip
    pg = b.prefix_groups
    assert pg is not None and pg.members == 2
    assert pg.first_block.tolist() == [3, 3, 0] and pg.prefix_row.tolist()[2] == -1
    none = PagedBatch.build(cache, tables[2:], [15], [1], "cpu", use_kernel=True, cascade=True,
                            num_heads=cfg.num_attention_heads, cascade_min_blocks=2)  # fmt: skip
    assert none.prefix_groups is None
    with pytest.raises(ValueError):
        PagedBatch.build(cache, tables, [18, 14, 15], [1, 1, 1], "cpu", use_kernel=True,
                         cascade=True)


@pytest.mark.parametrize("budget", [4096, 8])
def test_engine_reference_backend_matches_static_loop(budget):
    model = _model()
    want = _oracle(model, PROMPTS, 10)
    eng = TinyEngine(model, ReferenceBackend(), num_blocks=64, block_size=4,
                     max_num_batched_tokens=budget)  # fmt: skip
    assert _run_staggered(eng, PROMPTS, 10) == want
    _check_logits(eng, PROMPTS, 10, atol=1e-4)
    assert any(not s["decode_only"] for s in eng.log) and any(s["decode_only"] for s in eng.log)
    assert eng.bm.num_free_blocks == 64
    # Prompts "b", "d", "f" share 12 tokens: later ones forked the first one's blocks.
    assert eng.prefix_hits > 0


def test_engine_fork_copy_on_write_reference_backend():
    """A child forked mid-decode with a different pending token shares the parent's
    partly filled last block; both must still match their own static loops."""
    model = _model()
    prompt = list(range(30, 41))  # 11 tokens: last block of 4 partly filled
    eng = TinyEngine(model, ReferenceBackend(), num_blocks=32, block_size=4)
    eng.add_request("p", prompt, 8)
    for _ in range(3):  # prefill + 2 decodes -> 13 computed, 1 pending
        eng.step()
    parent = eng.running[0]
    assert parent.num_computed == 13 and len(parent.out) == 3
    forced = (parent.out[-1] + 1) % model.cfg.vocab_size
    eng.fork("p", "c", next_token=forced)
    while eng.has_unfinished():
        eng.step()
    assert sum(s["copies"] for s in eng.log) >= 1
    _check_fork(eng, model, prompt, parent.out[:2], forced, atol=1e-4)
    assert eng.bm.num_free_blocks == 32


def _check_fork(eng, model, prompt, shared_out, forced, atol):
    """Parent tokens and logits == static loop on the prompt; the child's tokens after
    the fork and their logits == static loop on prompt + shared outputs + forced."""
    want_p, logits_p = static_greedy(model, prompt, 8, with_logits=True)
    assert eng.done["p"] == want_p
    assert (torch.stack(eng.logits["p"]) - logits_p).abs().max().item() <= atol
    want_c, logits_c = static_greedy(model, prompt + shared_out + [forced], 5,
                                     with_logits=True)  # fmt: skip
    assert eng.done["c"] == shared_out + [forced] + want_c
    got_c = torch.stack(eng.logits["c"][3:])
    assert (got_c - logits_c).abs().max().item() <= atol


# --- GPU: the same engine on the HIP kernels ----------------------------------------


def _cuda_model(dtype, **cfg):
    return _model(dtype=dtype, device="cuda", **cfg)


@pytest.mark.gpu
@pytest.mark.parametrize("budget", [4096, 8])
def test_engine_kernels_match_static_loop_fp32(budget):
    """fp32: decode kernel (fp32 instantiation) and, for prompt chunks, the VALU
    chunked-prefill kernel. Tokens and logits == the static loop."""
    from tiny_llama import KernelBackend

    model = _cuda_model(torch.float32)
    want = _oracle(model, PROMPTS, 10)
    eng = TinyEngine(model, KernelBackend(), num_blocks=64, block_size=4,
                     max_num_batched_tokens=budget)  # fmt: skip
    assert _run_staggered(eng, PROMPTS, 10) == want
    _check_logits(eng, PROMPTS, 10, atol=2e-4)
    assert eng.bm.num_free_blocks == 64 and eng.prefix_hits > 0


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("hd", "bs"), [(64, 4), (128, 16)])
def test_engine_kernels_match_reference_backend_16bit(dtype, hd, bs):
    """16-bit: decode kernel + MFMA chunked-prefill kernel against the same engine on the
    reference's gather-then-attention (fp32 math, rounded to the model dtype), on the
    same flattened steps: identical tokens, logits within rounding. A sequence may part
    only at a step where the reference's own two best logits lie within that rounding
    tolerance of each other (a 16-bit tie, which any other order of rounding can break
    the other way; this bf16 model has one, at a gap of exactly 0); it is compared up to
    there. The fp32 engine tests above admit no such exception."""
    from tiny_llama import KernelBackend

    model = _cuda_model(dtype, hidden_size=4 * hd, num_attention_heads=4,
                        num_key_value_heads=2)  # fmt: skip
    runs = {}
    for backend in (ReferenceBackend(), KernelBackend()):
        eng = TinyEngine(model, backend, num_blocks=64, block_size=bs,
                         max_num_batched_tokens=8)  # fmt: skip
        runs[backend.name] = (_run_staggered(eng, PROMPTS, 10), eng)
    atol = 0.05  # 16-bit activations: a few ulps of the logits
    worst, parted = 0.0, []
    for r in PROMPTS:
        got, want = runs["kernel"][0][r], runs["reference"][0][r]
        assert len(got) == len(want), r
        for i, (tg, tw) in enumerate(zip(got, want)):
            lg = runs["kernel"][1].logits[r][i].float()
            lw = runs["reference"][1].logits[r][i].float()
            worst = max(worst, (lg - lw).abs().max().item())
            if tg != tw:
                top = torch.topk(lw, 2).values
                assert (top[0] - top[1]).item() <= atol, (r, i, tg, tw, top.tolist())
                parted.append((r, i))
                break
    assert worst <= atol, worst
    assert len(parted) <= 1, parted


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_engine_cascade_decode_matches_plain(dtype):
    """Decode steps with cascade over prompt prefixes shared by forking blocks:
    the plain decode's tokens, logits within 16-bit rounding."""
    from tiny_llama import KernelBackend

    model = _cuda_model(dtype)
    prompts = {"b": SHARED + [1, 2], "d": SHARED + [3], "f": SHARED, "g": SHARED + [4, 5, 6]}
    runs = {}
    for min_blocks in (None, 2):
        eng = TinyEngine(model, KernelBackend(), num_blocks=64, block_size=4,
                         cascade_min_blocks=min_blocks)  # fmt: skip
        runs[min_blocks] = (_run_staggered(eng, prompts, 12), eng)
    assert any(s["cascade"] for s in runs[2][1].log)
    assert runs[2][0] == runs[None][0]
    worst = max((torch.stack(runs[2][1].logits[r]) -
                 torch.stack(runs[None][1].logits[r])).abs().max().item()
                for r in prompts)  # fmt: skip
    assert worst <= 0.05, worst


@pytest.mark.gpu
@pytest.mark.parametrize("groups", [1, 2])
def test_decode_graphs_cascade_two_prefix_families(groups):
    """Two prompt families, each sharing its own prefix: with one group slot the graphs
    cascade the larger family and decode the other plainly, with two both -- the plain
    decode's tokens either way."""
    from tiny_llama import KernelBackend

    model = _cuda_model(torch.bfloat16)
    other = [40, 41, 42, 43, 44, 45, 46, 47, 48, 49, 50, 51]
    prompts = {"b": SHARED + [1, 2], "d": SHARED + [3], "f": SHARED, "p": other + [9],
               "q": other, "r": other + [7, 8]}  # fmt: skip
    runs = {}
    for graphs, min_blocks in ((False, None), (True, 2)):
        eng = TinyEngine(model, KernelBackend(), num_blocks=96, block_size=4, max_num_seqs=8,
                         graphs=graphs, cascade_min_blocks=min_blocks,
                         cascade_groups=groups)  # fmt: skip
        runs[graphs] = (_run_staggered(eng, prompts, 10), eng)
    log = runs[True][1].log
    assert any(s["graph"] and s["cascade"] for s in log)
    assert max(s["groups"] for s in log if s["graph"]) == groups
    assert runs[True][0] == runs[False][0]
    worst = max((torch.stack(runs[True][1].logits[r]) -
                 torch.stack(runs[False][1].logits[r])).abs().max().item()
                for r in prompts)  # fmt: skip
    assert worst <= 0.05, worst
    assert runs[True][1].bm.num_free_blocks == 96


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_graphs_cascade_matches_plain(dtype):
    """Decode steps replayed from hipGraphs with cascade on: each step's prefix groups
    are laid out in the graphs' static buffers (groups come and go between replays of
    one graph, and steps without any run the plain decode inside it). Same tokens as the
    eager plain decode, logits within 16-bit rounding."""
    from tiny_llama import KernelBackend

    model = _cuda_model(dtype)
    prompts = {"b": SHARED + [1, 2], "d": SHARED + [3], "a": [5, 6, 7], "f": SHARED,
               "g": SHARED + [4, 5, 6]}  # fmt: skip
    runs = {}
    for graphs, min_blocks in ((False, None), (True, 2)):
        eng = TinyEngine(model, KernelBackend(), num_blocks=64, block_size=4, max_num_seqs=8,
                         graphs=graphs, cascade_min_blocks=min_blocks)  # fmt: skip
        runs[graphs] = (_run_staggered(eng, prompts, 12), eng)
    log = runs[True][1].log
    assert any(s["graph"] and s["cascade"] for s in log)
    assert runs[True][0] == runs[False][0]
    worst = max((torch.stack(runs[True][1].logits[r]) -
                 torch.stack(runs[False][1].logits[r])).abs().max().item()
                for r in prompts)  # fmt: skip
    assert worst <= 0.05, worst
    assert runs[True][1].bm.num_free_blocks == 64


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_graphs_match_eager(dtype):
    """Decode steps replayed from hipGraphs (slot mapping built on the device, padding
    rows on the scratch block) give the eager engine's tokens and logits."""
    from tiny_llama import KernelBackend

    model = _cuda_model(dtype)
    prompts = dict(list(PROMPTS.items())[:3])  # three sequences pad to the 4-bucket
    runs = {}
    for graphs in (False, True):
        eng = TinyEngine(model, KernelBackend(), num_blocks=64, block_size=4, max_num_seqs=8,
                         graphs=graphs)  # fmt: skip
        runs[graphs] = (eng.generate(prompts, 30), eng)
    assert runs[True][0] == runs[False][0]
    assert sum(s["graph"] for s in runs[True][1].log) >= 20
    # Padding to the bucket changes only the GEMM row count: rounding-level differences.
    atol = 1e-4 if dtype == torch.float32 else 0.05
    for r in prompts:
        diff = torch.stack(runs[True][1].logits[r]) - torch.stack(runs[False][1].logits[r])
        assert diff.abs().max().item() <= atol, r
    if dtype == torch.float32:
        assert runs[True][0] == _oracle(model, prompts, 30)
    assert runs[True][1].bm.num_free_blocks == 64


@pytest.mark.gpu
@pytest.mark.parametrize("graphs", [False, True])
def test_engine_fork_copy_on_write_kernels(graphs):
    """Fork mid-decode on the HIP path: copy_blocks gives the child its own copy of the
    shared partly filled block before the append; both match their static loops."""
    from tiny_llama import KernelBackend

    model = _cuda_model(torch.float32)
    prompt = list(range(30, 41))
    eng = TinyEngine(model, KernelBackend(), num_blocks=32, block_size=4, graphs=graphs)
    eng.add_request("p", prompt, 8)
    for _ in range(3):
        eng.step()
    parent = eng.running[0]
    forced = (parent.out[-1] + 1) % model.cfg.vocab_size
    eng.fork("p", "c", next_token=forced)
    while eng.has_unfinished():
        eng.step()
    assert sum(s["copies"] for s in eng.log) >= 1
    _check_fork(eng, model, prompt, parent.out[:2], forced, atol=2e-4)
    assert eng.bm.num_free_blocks == 32


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("budget", [4096, 8])
def test_mixed_graphs_match_eager(dtype, budget):
    """Mixed steps replayed as one hipGraph per token bucket (prompts joining while
    others decode, chunked under budget 8, shared prompt prefixes) give the eager engine's
    tokens; in fp32 also the static loop's. Decode-only steps use DecodeGraphs."""
    from tiny_llama import KernelBackend

    model = _cuda_model(dtype)
    prompts = dict(PROMPTS, g=list(range(50, 90)))
    runs = {}
    for graphs in (False, True):
        eng = TinyEngine(model, KernelBackend(), num_blocks=64, block_size=4, max_num_seqs=8,
                         max_num_batched_tokens=budget, graphs=graphs,
                         mixed_graphs=graphs)  # fmt: skip
        runs[graphs] = (_run_staggered(eng, prompts, 12), eng)
        assert eng.bm.num_free_blocks == 64
    assert runs[True][0] == runs[False][0]
    log = runs[True][1].log
    assert sum(s["mixed_graph"] for s in log) >= 3 and sum(s["graph"] for s in log) >= 3
    assert not any(s["mixed_graph"] or s["graph"] for s in runs[False][1].log)
    atol = 1e-4 if dtype == torch.float32 else 0.05
    for r in prompts:
        diff = torch.stack(runs[True][1].logits[r]) - torch.stack(runs[False][1].logits[r])
        assert diff.abs().max().item() <= atol, r
    if dtype == torch.float32:
        assert runs[True][0] == _oracle(model, prompts, 12)


@pytest.mark.gpu
def test_mixed_graphs_step_cost_follows_the_step_not_the_pool():
    """MixedGraphs built with the reference's five arguments (engine/runtime/engine.py:
    110-112) sizes its tables by the model's longest sequence, not by the pool, and a
    step writes only what it uses: pools of 2,000 and 40,000 blocks give the same static
    buffers, the same logits and the same run() time (within noise)."""
    import time

    from engine.runtime.cuda_graphs import MixedGraphs
    from tiny_llama import KernelBackend

    model = _cuda_model(torch.bfloat16)
    model.attend = KernelBackend().attend
    tables, ctx, qlens = [[0, 1, 2], [3, 4], [5, 6]], [9, 6, 5], [1, 1, 5]
    ids = [11, 12, 20, 21, 22, 23, 24]
    positions = [8, 5, 0, 1, 2, 3, 4]
    times, logits, sizes = {}, {}, {}
    for blocks in (2_000, 40_000):
        cache = PagedKVCache(model.cfg, blocks + 1, 4, "cuda", torch.bfloat16)
        graphs = MixedGraphs(model, cache, blocks, 64, 64)
        assert graphs.max_width == model.cfg.max_position_embeddings // 4
        sizes[blocks] = (graphs._i32.numel(), graphs._i64.numel())
        batch = PagedBatch.build(cache, tables, ctx, qlens, "cuda", use_kernel=True,
                                 force_mixed=True)  # fmt: skip
        for _ in range(3):
            graphs.run(ids, positions, batch)
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(5):  # best of 5 rounds of 20 steps
            t0 = time.perf_counter()
            for _ in range(20):
                out = graphs.run(ids, positions, batch)
            torch.cuda.synchronize()
            best = min(best, (time.perf_counter() - t0) / 20)
        times[blocks], logits[blocks] = best, out.clone()
    assert sizes[2_000] == sizes[40_000]
    assert torch.equal(logits[2_000], logits[40_000])
    assert times[40_000] <= 1.3 * times[2_000] + 50e-6, times


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_elementwise_kernels_change_nothing(dtype):
    """RMSNorm, RoPE and SiLU x up on the fused HIP kernels: every logit of every step is
    bitwise the same as with the PyTorch ops (reference engine/kernels/fused.py's
    contract), through chunked prefill, decode and graph replays."""
    from tiny_llama import KernelBackend

    runs = {}
    for use in (False, True):
        model = _cuda_model(dtype).use_fused(use)
        eng = TinyEngine(model, KernelBackend(), num_blocks=64, block_size=4,
                         max_num_batched_tokens=8, graphs=True, mixed_graphs=True)  # fmt: skip
        runs[use] = (_run_staggered(eng, PROMPTS, 10), eng)
    assert runs[True][0] == runs[False][0]
    for r in PROMPTS:
        assert torch.equal(torch.stack(runs[True][1].logits[r]),
                           torch.stack(runs[False][1].logits[r])), r  # fmt: skip
