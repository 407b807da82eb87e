"""CPU checks of the drop-in boundary: the C ABI library loads and exports every symbol
include/paged_kv.h declares, its host-side validation rejects bad arguments before any
launch, and the Python wrappers mirror the reference's signatures and errors. No
compute call reaches a GPU here."""

from __future__ import annotations

import inspect
import os
import re

import pytest
import torch

from engine import workloads
from engine.kernels import _native
from engine.kernels import paged_attention as pa
from engine.runtime import paged_cache

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "paged_kv.h")


def _declared() -> list[str]:
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(pkv_\w+)\s*\(", text, re.M)


def test_header_symbols_are_exported_and_bound():
    names = _declared()
    assert len(names) >= 7
    lib = _native.lib()
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(names)
    assert lib.pkv_abi_version() == _native.ABI_VERSION


def test_status_strings():
    lib = _native.lib()
    assert lib.pkv_status_string(0) == b"ok"
    for code in (-1, -2, -3, -4, -5, -6, -7):
        assert lib.pkv_status_string(code) != b"unknown error"


def test_noalloc_decode_refuses_oversized_scratch_before_launch():
    """pkv_paged_decode_noalloc checks its workspace against the static scratch
    (PKV_NOALLOC_SCRATCH_BYTES) before touching any pointer or the GPU: a work split
    whose records exceed it returns PKV_E_SCRATCH (the pointers here are never read)."""
    lib = _native.lib()
    fake = 1 << 20  # aligned, never dereferenced
    need = lib.pkv_decode_workspace_bytes(1 << 20, 1, 64, 256)
    assert need > _native.PKV_NOALLOC_SCRATCH_BYTES
    st = lib.pkv_paged_decode_noalloc(fake, 2, 64 * 256, 256, fake, 64 * 256, 256, fake, fake,
                                      2, 8 * 256, 256, 1024, fake, 64, 64, fake, 1, 64, 8,
                                      256, 16, 0.0625, 1 << 20, None)  # fmt: skip
    assert st == -7
    assert b"no-alloc" in lib.pkv_status_string(st)


def test_workspace_arithmetic():
    lib = _native.lib()
    assert lib.pkv_decode_workspace_bytes(1, 64, 24, 128) == 0
    recs = 256 * 2 * 24
    assert lib.pkv_decode_workspace_bytes(256, 64, 24, 128) >= 64 * 16 + recs * (128 + 2) * 4

    # cascade: room for every finished sequence's fp32 output and normaliser, any wgs
    for wgs in (1, 256):
        plain = lib.pkv_decode_workspace_bytes(wgs, 64, 24, 128)
        assert lib.pkv_cascade_workspace_bytes(wgs, 64, 24, 128) >= plain + 64 * 24 * 129 * 4

    # without a GPU the device query fails cleanly
    if not torch.cuda.is_available():
        assert lib.pkv_decode_workgroups(2, 128, 24, 8) == -6
    assert lib.pkv_decode_workgroups(2, 96, 24, 8) == -2
    assert lib.pkv_decode_workgroups(9, 128, 24, 8) == -1
    # the default split's plan: shape errors before any device query
    assert lib.pkv_decode_default_workgroups(2, 96, 24, 8, 8, 32, 16) == -2
    assert lib.pkv_decode_default_workgroups(2, 128, 24, 8, 8, 32, 0) == -2
    if not torch.cuda.is_available():  # the plan needs the CU count
        assert lib.pkv_decode_default_workgroups(2, 128, 24, 8, 8, 32, 16) == -6


def test_prefill_workspace_arithmetic():
    """pkv_prefill_workspace_bytes: one scale byte per 256-token tile of every (chunk, KV
    head) (rows of a multiple of 4 bytes, the area rounded up to 256), then every
    chunk's region at the table's width rounded up to 256 tokens, fp16; 0 for shapes
    that take no copy; PKV_E_SHAPE for bad ones. Host arithmetic only (no GPU)."""
    lib = _native.lib()
    # bf16 (2), hd 128, 8 KV heads, 4 chunks, 224 blocks of 16 = 3,584 tokens -> 3,584
    kstride = (3584 // 256 + 3) // 4 * 4
    k_area = (4 * 8 * kstride + 255) // 256 * 256
    assert lib.pkv_prefill_workspace_bytes(2, 128, 8, 4, 224, 16) == k_area + 4 * 3584 * 8 * 128 * 2
    # widths round up to 256 tokens: 10 blocks of 12 = 120 tokens -> 256
    k_area = (3 * 2 * 4 + 255) // 256 * 256
    assert lib.pkv_prefill_workspace_bytes(2, 64, 2, 3, 10, 12) == k_area + 3 * 256 * 2 * 64 * 2
    assert lib.pkv_prefill_workspace_bytes(2, 128, 8, 0, 224, 16) == 0  # no chunks
    assert lib.pkv_prefill_workspace_bytes(1, 128, 8, 4, 224, 16) == 0  # fp16 caches
    assert lib.pkv_prefill_workspace_bytes(0, 128, 8, 4, 224, 16) == 0  # fp32 caches
    assert lib.pkv_prefill_workspace_bytes(2, 16, 8, 4, 224, 16) == 0   # hd 16: VALU kernel
    assert lib.pkv_prefill_workspace_bytes(2, 128, 8, 4, 4097, 16) == 0  # past 65,536 tokens
    assert lib.pkv_prefill_workspace_bytes(2, 128, 8, 4, 4096, 16) > 0
    assert lib.pkv_prefill_workspace_bytes(7, 128, 8, 4, 224, 16) == -1  # no such dtype
    assert lib.pkv_prefill_workspace_bytes(2, 96, 8, 4, 224, 16) == -2
    assert lib.pkv_prefill_workspace_bytes(2, 128, 0, 4, 224, 16) == -2
    assert lib.pkv_prefill_workspace_bytes(2, 128, 8, 4, 224, 0) == -2
    assert lib.pkv_prefill_workspace_bytes(2, 128, 8, -1, 224, 16) == -2
    assert pa.prefill_workspace_bytes(torch.bfloat16, 128, 8, 4, 224, 16) > 0
    with pytest.raises(ValueError):
        pa.prefill_workspace_bytes(torch.bfloat16, 128, 8, 4, 224, 0)


def test_prefill_ws_rejects_before_launch():
    """pkv_paged_prefill_ws checks the workspace after the common prefill arguments:
    negative bytes, or bytes without a pointer -> PKV_E_WORKSPACE; a workspace not
    16-byte aligned -> PKV_E_ALIGN; no chunks -> success with nothing launched."""
    lib = _native.lib()
    base = [1 << 12, 2, 8 * 128, 128, 1 << 12, 8 * 128, 128, 1 << 12, 1 << 12, 2, 2 * 128,
            128, 64, 1 << 12, 4, 4, 1 << 12, 1 << 12, 1, 4, 8, 2, 128, 16, 0.088]  # fmt: skip
    assert lib.pkv_paged_prefill_ws(*base, None, -1, None) == -4
    assert lib.pkv_paged_prefill_ws(*base, None, 4096, None) == -4
    assert lib.pkv_paged_prefill_ws(*base, (1 << 12) + 4, 4096, None) == -3
    empty = list(base)
    empty[18] = 0  # n_chunks
    assert lib.pkv_paged_prefill_ws(*empty, None, 0, None) == 0


def _decode_args(**over):
    a = dict(out=1 << 12, out_dtype=2, osb=24 * 128, osh=128, q=1 << 12, qsb=24 * 128,
             qsh=128, k=1 << 12, v=1 << 12, kv_dtype=2, kss=1024, ksh=128, num_slots=64,
             tables=1 << 12, tsb=4, w=4, ctx=1 << 12, batch=2, nh=24, nkv=8, hd=128, bs=16,
             scale=0.088, wgs=1, ws=None, ws_bytes=0, stream=None)  # fmt: skip
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize(
    ("over", "code"),
    [({"kv_dtype": 7}, -1), ({"out_dtype": 1}, -1), ({"hd": 96}, -2), ({"nh": 20}, -2),
     ({"wgs": -1}, -2), ({"bs": 0}, -2), ({"q": (1 << 12) + 2}, -3),
     ({"kss": 1020}, -3), ({"q": None}, -5),
     ({"wgs": 4}, -4)],
)  # fmt: skip
def test_decode_rejects_before_launch(over, code):
    """Every rejection happens on the host: these calls never reach the GPU."""
    assert _native.lib().pkv_paged_decode(*_decode_args(**over)) == code


@pytest.mark.parametrize(
    ("pre", "code"),
    [((None, 1 << 12, 1 << 12, 2, 4), -5), ((1 << 12, None, 1 << 12, 2, 4), -5),
     (((1 << 12) + 4, 1 << 12, 1 << 12, 2, 4), -3), ((1 << 12, 1 << 12, 1 << 12, -1, 4), -2),
     ((1 << 12, 1 << 12, 1 << 12, 2, -4), -2)],
)  # fmt: skip
def test_cascade_decode_rejects_before_launch(pre, code):
    """pkv_paged_decode_ex's prefix parts: missing or misaligned buffers and negative
    counts are refused on the host."""
    a = _decode_args()
    args = a[:-1] + [1 << 12, None, *pre, None]  # first_block, lse, prefix..., stream
    assert _native.lib().pkv_paged_decode_ex(*args) == code


def _cascade_args(dec=None, **pre):
    a = _decode_args(**(dec or {}))[:-1]  # without the stream
    p = dict(first_block=1 << 12, lse=None, ptab=1 << 12, ptsb=4, pw=4, pctx=1 << 12,
             pcu=1 << 12, pchunks=1, pmaxq=2, pqrows=1 << 12, pout=1 << 12, plse=1 << 12,
             prow=1 << 12, parts=1, pstride=2, pwg=0, stream=None)  # fmt: skip
    p.update(pre)
    return a + list(p.values())


@pytest.mark.parametrize(
    ("dec", "pre", "code"),
    [({}, {"pout": None}, -5), ({}, {"plse": None}, -5), ({}, {"prow": None}, -5),
     ({}, {"parts": 0}, -2), ({}, {"pchunks": -1}, -2), ({}, {"pout": (1 << 12) + 4}, -3),
     ({}, {"pchunks": 0}, -2), ({}, {"pmaxq": 0}, -2),
     ({"out": (1 << 12) + 2}, {}, -3), ({"out": (1 << 12) + 2}, {"pwg": -1}, -3),
     ({}, {}, -4), ({"kv_dtype": 7}, {}, -1)],
)  # fmt: skip
def test_cascade_one_call_rejects_before_launch(dec, pre, code):
    """pkv_cascade_decode checks the prefix pass's and the decode pass's arguments on the
    host before it launches either pass (a 2-sequence batch takes the two-launch form;
    its decode arguments, here without the workspace a cut needs, are checked before
    the prefix pass is launched). An empty prefix layout (no chunks or no queries) with
    prefix parts to merge is refused: nothing would write the parts the merge reads."""
    assert _native.lib().pkv_cascade_decode(*_cascade_args(dec, **pre)) == code


def test_cascade_one_launch_tiny_split_rejects_before_launch():
    """A batch the one-launch form takes (100 sequences, 16-bit, head_dim 128) with 1-3
    workgroups in all: the default choice of prefix workgroups handles the tiny split
    (no division by zero), and a misaligned output is still refused before any launch."""
    lib = _native.lib()
    for wgs in (1, 2, 3):
        args = _cascade_args({"out": (1 << 12) + 2, "batch": 100, "wgs": wgs})
        assert lib.pkv_cascade_decode(*args) == -3


def test_cascade_one_launch_query():
    """Shapes without a one-launch form answer 0 on any machine: batches of at most 64
    sequences, fp32 caches, head_dim 256, blocks that are not a power of two >= 16."""
    lib = _native.lib()
    for kv, hd, bs, batch in ((2, 128, 16, 64), (0, 128, 16, 256), (2, 256, 16, 256),
                              (2, 128, 12, 256), (2, 128, 8, 256), (2, 128, 16, 1025)):
        assert lib.pkv_cascade_one_launch(kv, hd, 24, 8, bs, batch) == 0
    assert not pa.cascade_one_launch(torch.bfloat16, 128, 24, 8, 16, 256, torch.device("cpu"))


def test_append_and_copy_reject_before_launch():
    lib = _native.lib()
    # bad dtype code
    assert lib.pkv_kv_append(1 << 12, 1 << 12, 5, 1024, 128, 64, 1 << 12, 1024, 128, 1 << 12,
                             1024, 128, 2, 1 << 12, 4, 8, 128, None) == -1  # fmt: skip
    # zero tokens: a no-op success
    assert lib.pkv_kv_append(None, None, 2, 1024, 128, 64, None, 1024, 128, None, 1024, 128,
                             2, None, 0, 8, 128, None) == 0  # fmt: skip
    assert lib.pkv_copy_blocks(None, None, 0, 1, 4096, 8, None, 0, None) == 0
    assert lib.pkv_copy_blocks(None, None, 0, 1, 4096, 8, None, 3, None) == -5
    assert lib.pkv_copy_blocks(1 << 12, 1 << 12, 0, 1, 0, 8, 1 << 12, 3, None) == -2


def test_python_signatures_mirror_reference():
    sig = inspect.signature(pa.paged_decode_attention)
    assert list(sig.parameters)[:7] == ["q", "k_cache", "v_cache", "block_tables",
                                        "context_lens", "block_size", "block_n"]  # fmt: skip
    assert sig.parameters["block_n"].default == 64
    ref = inspect.signature(pa.reference_decode_attention)
    assert list(ref.parameters) == ["q", "k_cache", "v_cache", "block_tables", "context_lens",
                                    "block_size"]  # fmt: skip
    w = inspect.signature(paged_cache.PagedKVCache.write)
    assert list(w.parameters) == ["self", "layer", "k", "v", "slots"]
    assert pa.HAS_TRITON is False
    assert pa.use_gqa_kernel(torch.bfloat16, 4, 64)
    assert not pa.use_gqa_kernel(torch.float32, 4, 64)
    assert not pa.use_gqa_kernel(torch.bfloat16, 4, 48)


def test_varlen_available_keeps_the_reference_surface(monkeypatch):
    """The reference exports varlen_available (engine/runtime/paged_cache.py:232-240) and
    its tests call and monkeypatch it (tests/test_kernels.py:191, :211). Here it exists,
    takes one tensor, and is False for every device and dtype: mixed steps never gather
    for varlen, whatever it returns."""
    assert list(inspect.signature(paged_cache.varlen_available).parameters) == ["t"]
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        assert paged_cache.varlen_available(torch.zeros(2, dtype=dt)) is False
    monkeypatch.setattr(paged_cache, "varlen_available", lambda t: True)
    cfg = paged_cache.KVShape(2, 2, 16)
    cache = paged_cache.PagedKVCache(cfg, 8, 4, device="cpu")
    batch = paged_cache.PagedBatch.build(cache, [[0, 1], [2]], [6, 1], [3, 1], "cpu",
                                         use_kernel=True)  # fmt: skip
    assert batch.mixed and batch.varlen is None and batch.chunks == []


def test_cpu_tensors_fail_loudly():
    """No CPU fallback: the product path refuses CPU tensors instead of computing."""
    step = workloads.custom([5, 9], 4, 2, 16, 4, torch.bfloat16)
    assert not pa.available(torch.device("cpu"))
    with pytest.raises(ValueError, match="GPU"):
        pa.paged_decode_attention(step.q, step.k_cache, step.v_cache, step.block_tables,
                                  step.context_lens, step.block_size)  # fmt: skip
    with pytest.raises(ValueError, match="GPU"):
        paged_cache.kv_append(step.k_cache, step.v_cache, step.new_k, step.new_v,
                              step.slot_mapping)  # fmt: skip
    cfg = paged_cache.KVShape(2, 2, 16)
    cache = paged_cache.PagedKVCache(cfg, 4, 4, device="cpu")
    with pytest.raises(ValueError, match="GPU"):
        cache.copy_blocks(torch.tensor([[0, 1]]))
    assert paged_cache.PagedKVCache.bytes_per_block(cfg, 4, torch.bfloat16) == 2 * 2 * 2 * 16 * 4 * 2


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _native.lib()


def test_workload_generators_follow_engine_layout():
    for make in (workloads.config1, lambda d, seed: workloads.config2(d, seed, batch=8),
                 lambda d, seed: workloads.config4(d, seed, batch=6)):  # fmt: skip
        step = make("cpu", seed=1)
        bs = step.block_size
        tabs = step.block_tables.tolist()
        ctx = step.context_lens.tolist()
        used = []
        for row, n in zip(tabs, ctx, strict=True):
            nb = -(-n // bs)
            assert nb <= len(row)
            used += row[:nb]
        assert len(used) == len(set(used)), "physical blocks must not be shared"
        assert max(used) * bs < step.k_cache.shape[0]
        # slot of the appended token: table[(n-1)//bs]*bs + (n-1)%bs (reference :140-143)
        want = [row[(n - 1) // bs] * bs + (n - 1) % bs for row, n in zip(tabs, ctx, strict=True)]
        assert step.slot_mapping.tolist() == want
    c2 = workloads.config2("cpu", seed=0, batch=8)
    assert tuple(c2.q.shape) == (8, 24, 128) and c2.k_cache.dtype == torch.bfloat16
    assert all(1024 <= n <= 4096 for n in c2.context_lens.tolist())
    assert c2.block_tables.shape[1] == 256
    c3 = workloads.config3("cpu", seed=0, batch=16, cow=4)
    shared = c3.info["shared_blocks"]
    rows = c3.block_tables.tolist()
    assert all(r[: shared - 1] == rows[0][: shared - 1] for r in rows)
    src, dst = zip(*c3.cow_mapping.tolist(), strict=True)
    assert len(set(src)) == 1 and len(set(dst)) == 4
    assert [r[shared - 1] for r in rows[:4]] == list(dst)
    assert c3.unique_kv_bytes() < c3.kv_bytes()


def test_debug_checks_follow_the_kernels_masking_rule():
    """The opt-in metadata checks (CPU tensors here: they are plain torch ops) accept
    exactly what the kernels read in bounds: a slot is live when it is in [0, num_slots),
    and a table column is read for the tokens the context puts in it -- a partly used
    last block may end past a whole-block boundary as long as its used tokens fit."""
    slots = torch.tensor([0, 5, 63])
    _native.check_slots("t", slots, 64)
    for bad in ([64], [-1], [3, 70]):
        with pytest.raises(IndexError, match="outside the pool"):
            _native.check_slots("t", torch.tensor(bad), 64)
    _native.check_slots("t", torch.tensor([], dtype=torch.int64), 0)

    bs, num_slots = 4, 30  # 7 whole blocks and 2 slots of block 7
    tables = torch.tensor([[1, 7, 99], [6, 0, -5]], dtype=torch.int32)
    _native.check_tables("t", tables, torch.tensor([6, 5], dtype=torch.int32), bs, num_slots)
    # block 7 holds only slots 28, 29: a third token in it is out of the pool
    with pytest.raises(IndexError, match="column 1"):
        _native.check_tables("t", tables, torch.tensor([7, 5], dtype=torch.int32), bs, num_slots)
    # column 2 (id 99) becomes used
    with pytest.raises(IndexError, match="sequence 0 column 2"):
        _native.check_tables("t", torch.tensor([[1, 2, 99], [6, 0, -5]], dtype=torch.int32),
                             torch.tensor([9, 5], dtype=torch.int32), bs, num_slots)  # fmt: skip
    # negative id in a used column
    with pytest.raises(IndexError, match="sequence 1 column 2"):
        _native.check_tables("t", tables, torch.tensor([2, 9], dtype=torch.int32), bs, num_slots)
    # a context longer than the table covers, or negative
    for n in (13, -1):
        with pytest.raises(IndexError, match="context_lens"):
            _native.check_tables("t", tables, torch.tensor([n, 1], dtype=torch.int32), bs,
                                 num_slots)  # fmt: skip
    # first= skips the leading columns (the cascade tail reads from there on)
    _native.check_tables("t", tables[:, 1:].contiguous(), torch.tensor([2, 1], dtype=torch.int32),
                         bs, num_slots)  # fmt: skip
    _native.check_tables("t", tables, torch.tensor([2, 1], dtype=torch.int32), bs, num_slots,
                         first=1)  # fmt: skip


def test_debug_checks_switch():
    prev = _native.set_debug_checks(True)
    try:
        assert _native.debug_checks()
        assert _native.set_debug_checks(False) is True
        assert not _native.debug_checks()
    finally:
        _native.set_debug_checks(prev)


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                      ([], {"WORLD_SIZE": "2"})])  # fmt: skip
def test_bench_refuses_more_than_one_gpu(argv, env):
    """bench.py measures one GPU: asked for more (or launched as one rank of several) it
    exits with status 2 and says so, before it imports torch or touches a device."""
    import subprocess
    import sys

    run_env = {**os.environ, **env}
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *argv],
                       capture_output=True, text=True, env=run_env, timeout=60)  # fmt: skip
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def _bench():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_committed_traffic_profiles_match_the_sources():
    """Every counter entry the bench can report as roofline.traffic was measured on the
    kernel sources committed now (a source edit needs a new rocprofv3 FETCH_SIZE /
    WRITE_SIZE pass), and its byte counts are consistent."""
    import json

    bench = _bench()
    entries = json.load(open(bench.TRAFFIC_FILE))
    assert set(entries) >= {"c1_llama1b_fp16", "c2_llama3b_bf16", "c3_prefix_shared_bf16",
                            "c4_llama8b_longctx_bf16", "c5_mixed_llama8b_bf16"}  # fmt: skip
    for name, e in entries.items():
        assert e["bytes"] == e["read_bytes"] + e["write_bytes"], name
        assert os.path.exists(os.path.join(ROOT, e["source"])), name
        got, why = bench.traffic_of(name)
        assert got == e["bytes"], f"{name}: {why}"


def test_stale_traffic_profile_is_not_reported(monkeypatch, tmp_path):
    import json

    bench = _bench()
    entries = json.load(open(bench.TRAFFIC_FILE))
    entries["c2_llama3b_bf16"]["sources_sha256"] = "0" * 64
    f = tmp_path / "traffic.json"
    f.write_text(json.dumps(entries))
    monkeypatch.setattr(bench, "TRAFFIC_FILE", str(f))
    got, why = bench.traffic_of("c2_llama3b_bf16")
    assert got is None and "stale" in why
    assert bench.traffic_of("no_such_workload") == (None, "no counter profile for no_such_workload")
