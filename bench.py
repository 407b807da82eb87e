"""Benchmark of the paged decode attention hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c2] [--layers L]

A step is one layer-step of paged decode attention (stream-K pass + combine) over the
config's batch, on cuda:0. L independent layer pools (default 4, ~1 GB each at config 2)
are used in rotation, so every step reads K/V that the previous step did not touch,
as consecutive layers of a model do; the 256 MB last-level cache cannot serve them.
Timing: torch.cuda.Event pairs around every launch on torch's current stream, which is
the stream the library launches on; the timed region is bracketed by synchronize().

Prints one JSON line: value = mean microseconds per layer-step of decode attention;
roofline.achieved = algorithmic K+V bytes (sum(ctx) * 2 * nkv * hd * 2 B) / the mean
launch duration. cpu_baseline times the C oracle on the same config on host cores.
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_traffic.json")


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4"])
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--workgroups", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 5 plain 1 GiB device-to-device copies: the known-size "
                         "kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE")  # fmt: skip
    return ap.parse_args()


def cpu_baseline(step, budget_s: float) -> dict:
    """The C oracle (double-accumulating scalar restatement of the reference's CPU
    gather-then-attention path) on the full config batch, OpenMP over host cores."""
    from oracle import oracle

    threads = min(16, os.cpu_count() or 1)
    args = (step.q.cpu(), step.k_cache.cpu(), step.v_cache.cpu(), step.block_tables.cpu(),
            step.context_lens.cpu(), step.block_size)  # fmt: skip
    oracle.decode_attention(*args, threads=threads)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        oracle.decode_attention(*args, threads=threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(med * 1e6, 1),
        "unit": "us/layer-step",
        "gbps": round(step.kv_bytes() / med / 1e9, 2),
        "cores": threads,
        "kind": "port",
        "sample": f"full {step.name} layer-step (batch {step.batch}), median of {len(times)} "
                  f"reps; C oracle in float64, OpenMP {threads} threads, host "
                  f"os.cpu_count()={os.cpu_count()}",
    }  # fmt: skip


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the decode path has no "
              "cross-GPU exchange on one box); run with --gpus 1", file=sys.stderr)  # fmt: skip
        return 2

    import torch

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
    b, nh, hd = step.q.shape
    nkv = step.k_cache.shape[1]
    w = step.block_tables.shape[1]
    wgs = args.workgroups or pa.decode_workgroups(dev, step.q.dtype, hd, nh, nkv)
    out = torch.empty_like(step.q)

    def attn(i: int) -> None:
        k, v = pools[i % len(pools)]
        pa.paged_decode_attention(step.q, k, v, step.block_tables, step.context_lens,
                                  step.block_size, out=out, num_workgroups=wgs)  # fmt: skip

    for i in range(args.warmup):
        attn(i)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]  # fmt: skip
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record()
        attn(i)
        ev[i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [a.elapsed_time(z) * 1e3 for a, z in ev]  # microseconds
    mean_us = statistics.fmean(per)

    # KV append of the same batch (one layer), timed the same way.
    ap_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(50)]  # fmt: skip
    for a, z in ap_ev:
        a.record()
        kv_append(step.k_cache, step.v_cache, step.new_k, step.new_v, step.slot_mapping)
        z.record()
    torch.cuda.synchronize()
    append_us = statistics.fmean(a.elapsed_time(z) * 1e3 for a, z in ap_ev)

    kv_bytes = step.kv_bytes()
    gbps = kv_bytes / (mean_us * 1e-6) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get(step.name)
    line = {
        "metric": "paged decode attn us/layer-step + achieved HBM GB/s (% of 8 TB/s), 3B shape",
        "value": round(mean_us, 2),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if step.q.dtype == torch.bfloat16 else str(step.q.dtype).split(".")[-1],
        "data": "synthetic (seeded N(0,1) pools, queries; scattered block tables)",
        "config": {
            "workload": step.name,
            "batch": b,
            "num_heads": nh,
            "num_kv_heads": nkv,
            "head_dim": hd,
            "block_size": step.block_size,
            "table_width": w,
            "sum_ctx": int(step.context_lens.sum()),
            "workgroups": wgs,
            "layer_pools": len(pools),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
        },
        "kv_bytes_per_step": kv_bytes,
        "median_us": round(statistics.median(per), 2),
        "append_us": round(append_us, 2),
    }
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(step, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
