"""Benchmark of the paged-KV hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c2] [--layers L]

Default workload (BASELINE.json's metric): config 2, a Llama-3.2-3B decode step (B=64,
contexts U[1024, 4096], 24 q / 8 KV heads, hd 128, bf16, 16-token blocks). A step is one
layer-step of paged decode attention (stream-K pass + combine) over the batch on cuda:0.
L independent layer pools (default 4, ~1 GB each at config 2) are used in rotation, so
every step reads K/V the previous step did not touch, as consecutive layers of a model
do; the 256 MB last-level cache cannot serve them.

Timing. ``value`` is the mean time per layer-step over exactly ``--steps`` layer-steps
(the L pools in rotation) captured in hipGraphs of at least 32 calls and replayed (the
reference runs decode steps as CUDA-graph replays, engine/runtime/cuda_graphs.py; a model
step's graph holds every layer), between events bracketed by synchronize(). ``eager_us``
is the mean of per-call events around eager calls (includes per-call launch costs).
``roofline.achieved`` = algorithmic K+V bytes (sum(ctx) * 2 * nkv * hd * 2 B) / the
graph-replay time per layer-step. ``cpu_baseline`` times the reference's CPU path (torch
index_copy_ append + gather -> fp32 softmax -> PV) on the host cores, for the bench's
config and, at config 2, for config 1 beside it.

``--config c5`` measures the mixed chunked-prefill step of config 5 instead (append of
2,168 rows, MFMA prefill of 4 x 512-token chunks, decode of 120 sequences); its line
reports the prefill's TFLOP/s against the bf16 MFMA peak and the append's GB/s.
``--config c3`` adds the copy-on-write of the config's 64 block pairs across a 28-layer
pool (``cow_*``: algorithmic bytes, and unique bytes with the shared source once) and the
same decode with cascade over the shared prefix (``cascade_*``, GB/s on unique bytes).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "inference-engine_amd"))

HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_traffic.json")
GRAPH_CALLS = 32  # calls captured per timed hipGraph (see graph_us)
WARM_SECONDS = 0.3  # untimed load before the first timing (see warm_clocks)
DECODE_SOURCES = ("common.h", "decode_kernels.h", "decode.hip")  # what the stream pass is built from
METRIC = "paged decode attn us/layer-step + achieved HBM GB/s (% of 8 TB/s), 3B shape"


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "c2_1b"])
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--workgroups", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-graph", action="store_true", help="time eager calls only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", choices=["cascade", "cow", "append", "fused"], default=None,
                    help="time one part alone, e.g. under a profiler: cascade decode or "
                         "the copy-on-write (config c3), the KV append or the fused "
                         "element-wise kernels (config c5)")  # fmt: skip
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 5 plain 1 GiB device-to-device copies: the known-size "
                         "kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE")  # fmt: skip
    return ap.parse_args()


def cpu_model() -> str:
    """The host CPU's model name (first 'model name' line of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def host_threads() -> tuple[int, str]:
    """Threads for the CPU baseline: the cores this process may run on, capped at the
    pool's per-GPU CPU share (OMP_NUM_THREADS, 16 on the GPU boxes, which run one GPU per
    job on a shared host); and a note of what the host reports."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    share = int(os.environ.get("OMP_NUM_THREADS") or avail or 1)
    n = max(1, min(avail or 1, share))
    return n, (f"os.cpu_count()={os.cpu_count()}, affinity={avail}, "
               f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS')}")


def cpu_baseline(step, budget_s: float) -> dict:
    """The reference's CPU path for one decode layer-step (index_copy_ append, then the
    per-sequence gather -> fp32 softmax -> PV of reference_decode_attention), restated with
    torch CPU ops in oracle/torch_path.py, on a CPU copy of the step's inputs: median of
    >= 5 timed reps after one warm-up, within about ``budget_s`` seconds."""
    import torch

    from oracle import torch_path

    n, note = host_threads()
    torch.set_num_threads(n)
    cpu = {k: getattr(step, k).cpu() for k in ("q", "k_cache", "v_cache", "block_tables",
                                                "context_lens", "new_k", "new_v", "slot_mapping")}

    def run():
        torch_path.decode_layer_step(cpu["q"], cpu["k_cache"], cpu["v_cache"],
                                     cpu["block_tables"], cpu["context_lens"], step.block_size,
                                     cpu["new_k"], cpu["new_v"], cpu["slot_mapping"])  # fmt: skip

    run()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 30):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(med * 1e6, 1),
        "unit": "us/layer-step",
        "gbps": round(step.kv_bytes() / med / 1e9, 2),
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"full {step.name} layer-step (batch {step.batch}): the reference's CPU "
                  f"path (index_copy_ append + per-sequence gather, fp32 softmax, PV) in torch "
                  f"on CPU, median of {len(times)} reps; torch threads "
                  f"{torch.get_num_threads()} ({note}), {cpu_model()}",
    }  # fmt: skip


def traffic_of(step_name: str) -> tuple[int | None, str]:
    """HBM bytes per dispatch of the workload's dominant kernel (the decode stream pass;
    the matrix-core prefill at config 5) from the committed rocprofv3 counter summary, if
    it was measured on the sources built now (the SHA-256 of the entry's source files,
    the decode sources by default, is stored with it); otherwise None and why."""
    import hashlib

    if not os.path.exists(TRAFFIC_FILE):
        return None, "no counter profile"
    with open(TRAFFIC_FILE) as f:
        entry = json.load(f).get(step_name)
    if not entry:
        return None, f"no counter profile for {step_name}"
    h = hashlib.sha256()
    for name in entry.get("source_files", DECODE_SOURCES):
        with open(os.path.join(ROOT, "inference-engine_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    if entry.get("sources_sha256") != h.hexdigest():
        return None, "stale: the counter profile was taken on other kernel sources"
    return entry["bytes"], f"{entry['source']} (sources {h.hexdigest()[:12]})"


def warm_clocks(torch, fns, seconds: float = WARM_SECONDS) -> None:
    """Untimed calls of the workload itself until `seconds` of wall time passed: the GPU's
    clock ramps up over tens of milliseconds of load, and a timing taken right after a few
    milliseconds of warm-up read up to ~10% slow at config 5."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for f in fns:
            f()
        torch.cuda.synchronize()


def eager_us(torch, fns, steps: int, warmup: int) -> list[float]:
    """Per-call event times (µs) of fns called round-robin."""
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]  # fmt: skip
    for i, (a, z) in enumerate(ev):
        a.record()
        fns[i % len(fns)]()
        z.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(z) * 1e3 for a, z in ev]


def graph_us(torch, fns, steps: int, warmup: int) -> tuple[float, float]:
    """Time exactly `steps` calls of fns (round-robin) as hipGraph replays: a graph of at
    least GRAPH_CALLS calls replayed steps // G times, then one graph of the remaining
    calls. A real engine replays a whole multi-layer step per graph; with a few calls per
    graph the host's launch of each replay (~40 µs here) outlasts the GPU work and its gap
    would land in the per-call time. Returns (µs per call, wall seconds of the timed
    region)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(side)
    steps = max(1, steps)
    g_calls = min(steps, len(fns) * max(1, -(-GRAPH_CALLS // len(fns))))
    full, rem = divmod(steps, g_calls)

    def capture(n):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n):
                fns[i % len(fns)]()
        return graph

    graph = capture(g_calls)
    tail = capture(rem) if rem else None
    # at least three untimed replays: the first replays of a process's first graph ran
    # ~8% slow at config 5 even after warm_clocks (one-time set-up of graph execution)
    for _ in range(max(3, -(-warmup // g_calls))):
        graph.replay()
    if tail is not None:
        tail.replay()
    torch.cuda.synchronize()
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record()
    for _ in range(full):
        graph.replay()
    if tail is not None:
        tail.replay()
    z.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return a.elapsed_time(z) * 1e3 / steps, wall


def decode_setup(args, torch):
    """The config's decode step after its copy-on-write and append, the layer pools used
    in rotation, the output buffer and the workgroup count."""
    from engine import workloads
    from engine.kernels import paged_attention as pa
    from engine.runtime.paged_cache import copy_blocks, kv_append

    dev = torch.device("cuda:0")
    step = workloads.CONFIGS[args.config](dev, seed=args.seed)
    if step.cow_mapping is not None:
        copy_blocks(step.k_cache, step.v_cache, step.cow_mapping, step.block_size)
    kv_append(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)
    pools = [(step.k_cache, step.v_cache)]
    for _ in range(args.layers - 1):
        pools.append((torch.randn_like(step.k_cache), torch.randn_like(step.v_cache)))
    return step, pools, torch.empty_like(step.q), args.workgroups  # None: default split


def bench_decode(args, torch) -> dict:
    from engine.kernels import paged_attention as pa
    from engine.runtime.paged_cache import kv_append

    step, pools, out, wgs = decode_setup(args, torch)
    b, nh, hd = step.q.shape
    nkv = step.k_cache.shape[1]
    w = step.block_tables.shape[1]
    # What the decode call runs: 0 = the one-kernel per-sequence split pass, else the
    # stream-K pass over that many workgroups (plus its combine).
    plan = wgs or pa.default_workgroups(step.q.device, step.q.dtype, hd, nh, nkv, b, w,
                                        step.block_size)  # fmt: skip

    def attn_fn(k, v):
        return lambda: pa.paged_decode_attention(
            step.q, k, v, step.block_tables, step.context_lens, step.block_size, out=out,
            num_workgroups=wgs)  # fmt: skip

    fns = [attn_fn(k, v) for k, v in pools]
    warm_clocks(torch, fns)
    per = eager_us(torch, fns, args.steps, args.warmup)
    eager_mean = statistics.fmean(per)
    if args.no_graph:
        value, wall = eager_mean, None
    else:
        value, wall = graph_us(torch, fns, args.steps, args.warmup)

    def append():
        kv_append(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)

    append_us = graph_us(torch, [append] * 8, 400, 16)[0]

    kv_bytes = step.kv_bytes()
    gbps = kv_bytes / (value * 1e-6) / 1e9
    traffic, traffic_source = traffic_of(step.name)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(value / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if step.q.dtype == torch.bfloat16 else str(step.q.dtype).split(".")[-1],
        "data": "synthetic (seeded N(0,1) pools and queries; scattered block tables)",
        "config": {
            "workload": step.name,
            "batch": b,
            "num_heads": nh,
            "num_kv_heads": nkv,
            "head_dim": hd,
            "block_size": step.block_size,
            "table_width": w,
            "sum_ctx": int(step.context_lens.sum()),
            "workgroups": plan,
            "decode_pass": "split (one kernel)" if plan == 0 else "stream-k + combine",
            "layer_pools": len(pools),
            "timing": "eager" if args.no_graph else "hipgraph replay",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
        },
        "traffic_source": traffic_source,
        # achieved / frac cover the whole decode call the C ABI exposes (one
        # pkv_paged_decode: the split pass, or the stream pass + combine); traffic is the
        # stream pass's (the combine's own bytes are in the profile summary)
        "roofline_scope": "pkv_paged_decode call (" +
                          ("split pass" if plan == 0 else "stream pass + combine") + ")",
        "kv_bytes_per_step": kv_bytes,
        "eager_us": round(eager_mean, 2),
        "eager_median_us": round(statistics.median(per), 2),
        "append_us": round(append_us, 2),
    }
    if wall is not None:
        line["timed_wall_s"] = round(wall, 4)
    if step.cow_mapping is not None:
        line["unique_kv_bytes_per_step"] = step.unique_kv_bytes()
        line["unique_gbps"] = round(line["unique_kv_bytes_per_step"] / (value * 1e-6) / 1e9, 1)
        line.update(bench_cow(torch, step))
        line.update(bench_cascade(args, torch, step, pools, out, wgs,
                                  line["unique_kv_bytes_per_step"]))  # fmt: skip
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(step, args.cpu_seconds)
        if step.name.startswith("c2"):  # config 1 beside it: the reference's CPU-run case
            from engine import workloads

            line["cpu_baseline_c1"] = cpu_baseline(workloads.config1("cpu", seed=args.seed),
                                                   min(5.0, args.cpu_seconds))  # fmt: skip
    return line


def bench_cascade(args, torch, step, pools, out, wgs, unique_bytes) -> dict:
    """The same layer-steps with cascade decode as the engine's decode graphs run it:
    prefix groups found from the block tables on the host, laid out in the graphs'
    fixed shape (one group slot, pieces for the batch size), each shared prefix read once
    per group; timed as hipGraph replays."""
    import numpy as np

    from engine.kernels import paged_attention as pa

    n, nh = step.q.shape[0], step.q.shape[1]
    nkv, bs, w = step.k_cache.shape[1], step.block_size, step.block_tables.shape[1]
    tables = step.block_tables.cpu().numpy()
    groups = pa.shared_prefixes(tables, step.context_lens.cpu().numpy(), bs)
    if not groups:
        return {"cascade": None}
    pieces = pa.cascade_pieces(n, nh, nkv, step.q.device, dtype=step.k_cache.dtype,
                               head_dim=step.q.shape[2], block_size=bs)  # fmt: skip
    slots = 1  # DecodeGraphs' default
    width = -(-w // pieces)
    flat = np.zeros(pa.prefix_entries(n, pieces, slots, width, n), dtype=np.int32)
    groups.sort(key=lambda g: -len(g[0]) * g[1])
    pa.fill_prefix(flat, n, pieces, slots, width, tables, groups[:slots], bs, n)
    pg = pa.prefix_view(torch.from_numpy(flat).to(step.q.device), n, pieces, slots, width,
                        members=n, max_members=n)  # fmt: skip

    def fn(k, v):
        return lambda: pa.paged_decode_attention(
            step.q, k, v, step.block_tables, step.context_lens, bs, out=out,
            num_workgroups=wgs, prefix_groups=pg)  # fmt: skip

    us = graph_us(torch, [fn(k, v) for k, v in pools], args.steps, args.warmup)[0]
    gbps = unique_bytes / (us * 1e-6) / 1e9
    return {"cascade_us": round(us, 2), "cascade_unique_gbps": round(gbps, 1),
            "cascade_unique_frac": round(gbps / HBM_PEAK_GBPS, 4),
            "cascade_groups": min(len(groups), slots), "cascade_pieces": pieces,
            "cascade_one_launch": pa.cascade_one_launch(step.k_cache.dtype, step.q.shape[2], nh,
                                                        nkv, bs, n, step.q.device),
            "cascade_layout": f"decode-graph fixed shape: {slots} group slot(s)"}


def bench_cow(torch, step, layers: int = 28, blocks: int = 2048) -> dict:
    """Copy-on-write of the step's pairs across a whole model's pool (28 layers, the
    3B depth): every pair copies one 16-token block of every layer, K and V."""
    from engine.runtime.paged_cache import copy_blocks

    bs = step.block_size
    _, nkv, hd = step.k_cache.shape
    kp = torch.empty(layers, blocks * bs, nkv, hd, dtype=step.k_cache.dtype,
                     device=step.k_cache.device)  # fmt: skip
    vp = torch.empty_like(kp)
    pairs = step.cow_mapping.shape[0]
    mapping = torch.stack([torch.full((pairs,), 3, dtype=torch.int64),
                           torch.arange(pairs, dtype=torch.int64) + 100], 1).to(kp.device)  # fmt: skip
    us = graph_us(torch, [lambda: copy_blocks(kp, vp, mapping, bs)] * 8, 400, 16)[0]
    blk = bs * nkv * hd * kp.element_size()
    moved = 2 * pairs * layers * blk * 2  # K+V, every pair read + written
    # config 3 copies one shared block to every destination: its reads hit the cache
    srcs = int(torch.unique(mapping[:, 0]).numel())
    unique = 2 * layers * blk * (srcs + pairs)
    return {"cow_pairs": pairs, "cow_layers": layers, "cow_us": round(us, 2),
            "cow_bytes": moved, "cow_gbps": round(moved / (us * 1e-6) / 1e9, 1),
            "cow_unique_bytes": unique,
            "cow_unique_gbps": round(unique / (us * 1e-6) / 1e9, 1)}


def bench_append(args, torch) -> dict:
    """Config 5's KV append alone (2,168 new rows into the 8B-shaped pool), graph replay."""
    from engine import workloads
    from engine.runtime.paged_cache import kv_append

    m = workloads.config5(torch.device("cuda:0"), seed=args.seed)

    def append():
        kv_append(m.k_cache, m.v_cache, m.new_k, m.new_v, m.slot_mapping)

    us = graph_us(torch, [append] * 8, 8 * args.steps, args.warmup)[0]
    nbytes = 2 * m.new_k.numel() * m.new_k.element_size() * 2  # K and V, read + written
    return {"config": {"workload": m.name, "rows": int(m.slot_mapping.numel())},
            "append_us": round(us, 2), "append_bytes": nbytes,
            "append_gbps": round(nbytes / (us * 1e-6) / 1e9, 1)}  # fmt: skip


def bench_fused(args, torch) -> dict:
    """The fused element-wise kernels at config 5's step shape (Llama-3-8B: 2,168 token
    rows, hidden 4,096, 32 q / 8 KV heads of 128, intermediate 14,336), bf16, graph
    replay, each beside the PyTorch expression it replaces. Bytes are what the operation
    must move: RMSNorm x in + out (its per-row rsqrt(mean(x^2)) stays a PyTorch
    reduction, inside the timed call), RoPE q and k in place + cos and sin (fp32),
    SiLU x up gate and up in + out."""
    import torch.nn.functional as F

    from engine.kernels import fused

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    n, hidden, nh, nkv, hd, inter, eps = 2168, 4096, 32, 8, 128, 14336, 1e-5
    bf = torch.bfloat16
    x = torch.randn(n, hidden, device=dev, generator=g).to(bf)
    w = torch.randn(hidden, device=dev, generator=g).to(bf)
    q = torch.randn(n, nh, hd, device=dev, generator=g).to(bf)
    k = torch.randn(n, nkv, hd, device=dev, generator=g).to(bf)
    inv_freq = 1.0 / (500000 ** (torch.arange(0, hd, 2, device=dev).float() / hd))
    emb = torch.arange(n, device=dev).float()[:, None] * inv_freq
    emb = torch.cat([emb, emb], -1)
    cos, sin = emb.cos(), emb.sin()
    gate = torch.randn(n, inter, device=dev, generator=g).to(bf)
    up = torch.randn(n, inter, device=dev, generator=g).to(bf)

    def rot(t):
        h = t.shape[-1] // 2
        return torch.cat((-t[..., h:], t[..., :h]), -1)

    def torch_rms():
        xf = x.float()
        return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(bf)

    def torch_rope():
        c, s_ = cos[:, None].to(bf), sin[:, None].to(bf)
        return q * c + rot(q) * s_, k * c + rot(k) * s_

    cases = {
        "rms_norm": (lambda: fused.rms_norm(x, w, eps), torch_rms, 2 * x.numel() * 2),
        "rope": (lambda: (fused.rope_(q, cos, sin), fused.rope_(k, cos, sin)), torch_rope,
                 (q.numel() + k.numel()) * 2 * 2 + 2 * cos.numel() * 4),
        "silu_mul": (lambda: fused.silu_mul(gate, up), lambda: F.silu(gate) * up,
                     3 * gate.numel() * 2),
    }  # fmt: skip
    res = {}
    for name, (mine, ref, nbytes) in cases.items():
        us = graph_us(torch, [mine] * 8, 8 * args.steps, args.warmup)[0]
        ref_us = graph_us(torch, [ref] * 8, 8 * args.steps, args.warmup)[0]
        res[name] = {"us": round(us, 2), "bytes": nbytes,
                     "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "torch_us": round(ref_us, 2)}  # fmt: skip
    return {"config": {"workload": "c5_llama8b_elementwise_bf16", "rows": n}, "fused": res}


def bench_mixed(args, torch) -> dict:
    from engine import workloads
    from engine.kernels import paged_attention as pa
    from engine.runtime.paged_cache import kv_append

    dev = torch.device("cuda:0")
    m = workloads.config5(dev, seed=args.seed)
    d = m.decode
    out_c = torch.empty_like(m.q_chunks)
    out_d = torch.empty_like(d.q)
    nh, hd = d.q.shape[1], d.q.shape[2]
    wgs = args.workgroups  # None: the library's default split

    def append():
        kv_append(m.k_cache, m.v_cache, m.new_k, m.new_v, m.slot_mapping)

    def prefill():
        pa.paged_prefill_attention(m.q_chunks, m.k_cache, m.v_cache, m.chunk_tables,
                                   m.chunk_ctx, m.block_size, m.cu_q, m.max_query_len,
                                   out=out_c)  # fmt: skip

    def decode():
        pa.paged_decode_attention(d.q, d.k_cache, d.v_cache, d.block_tables, d.context_lens,
                                  d.block_size, out=out_d, num_workgroups=wgs)  # fmt: skip

    append()
    warm_clocks(torch, [append, prefill, decode])
    t_pre = graph_us(torch, [prefill] * 4, args.steps, args.warmup)[0]
    t_dec = graph_us(torch, [decode] * 4, args.steps, args.warmup)[0]
    t_app = graph_us(torch, [append] * 4, args.steps, args.warmup)[0]
    per_call, wall = graph_us(torch, [append, prefill, decode], 3 * args.steps, args.warmup)
    step_us = 3 * per_call  # one step = append + prefill + decode
    flops = m.prefill_flops()
    tflops = flops / (t_pre * 1e-6) / 1e12
    dec_gbps = d.kv_bytes() / (t_dec * 1e-6) / 1e9
    # append: every new row read once and written once, K and V
    app_bytes = 2 * m.new_k.numel() * m.new_k.element_size() * 2
    traffic, traffic_source = traffic_of(m.name)
    return {
        "metric": "mixed chunked-prefill layer-step us (config 5)",
        "value": round(step_us, 2),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_us / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) pool and queries; scattered block tables)",
        "config": {"workload": m.name, "chunks": "4 x 512 tokens after 0/1k/2k/3k cached",
                   "decode_batch": d.batch, "num_heads": nh, "head_dim": hd,
                   "timing": "hipgraph replay"},  # fmt: skip
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
        },
        "traffic_source": traffic_source,
        "roofline_scope": "paged_prefill_attention call (fp16 V copy + matrix-core prefill)",
        "prefill_us": round(t_pre, 2),
        "prefill_gflop": round(flops / 1e9, 2),
        "decode_us": round(t_dec, 2),
        "decode_gbps": round(dec_gbps, 1),
        "append_us": round(t_app, 2),
        "append_bytes": app_bytes,
        "append_gbps": round(app_bytes / (t_app * 1e-6) / 1e9, 1),
        "timed_wall_s": round(wall, 4),
    }


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the decode path has no "
              "cross-GPU exchange on one box); run with --gpus 1", file=sys.stderr)  # fmt: skip
        return 2

    import torch

    need = {"cascade": "c3", "cow": "c3", "append": "c5", "fused": "c5"}.get(args.only)
    if need and args.config != need:
        print(f"bench.py: --only {args.only} needs --config {need}", file=sys.stderr)
        return 2
    if args.only == "cascade":
        step, pools, out, wgs = decode_setup(args, torch)
        line = {"config": {"workload": step.name, "layer_pools": len(pools)},
                **bench_cascade(args, torch, step, pools, out, wgs, step.unique_kv_bytes())}
    elif args.only == "cow":
        step, _, _, _ = decode_setup(args, torch)
        line = {"config": {"workload": step.name}, **bench_cow(torch, step)}
    elif args.only == "append":
        line = bench_append(args, torch)
    elif args.only == "fused":
        line = bench_fused(args, torch)
    elif args.config == "c5":
        line = bench_mixed(args, torch)
    else:
        line = bench_decode(args, torch)
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
