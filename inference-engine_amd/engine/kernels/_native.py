"""ctypes binding of lib/libpaged_kv.so (C ABI declared in include/paged_kv.h).

The library is the only compute path: if it is missing or cannot be loaded, every
entry point raises. ``import torch`` happens first so the library's libamdhip64.so.7
dependency resolves to the HIP runtime torch has already loaded.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(
    os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
    "lib",
    "libpaged_kv.so",
)
ABI_VERSION = 5
PKV_NOALLOC_SCRATCH_BYTES = 32 << 20  # include/paged_kv.h

PKV_F32, PKV_F16, PKV_BF16 = 0, 1, 2
DTYPE_CODE = {torch.float32: PKV_F32, torch.float16: PKV_F16, torch.bfloat16: PKV_BF16}

# Every symbol include/paged_kv.h declares, with (restype, argtypes).
_i32, _i64, _f32, _p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
SIGNATURES: dict[str, tuple] = {
    "pkv_abi_version": (ctypes.c_int, []),
    "pkv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "pkv_kv_append": (
        ctypes.c_int,
        [_p, _p, ctypes.c_int, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64,
         ctypes.c_int, _p, _i64, _i32, _i32, _p],
    ),  # fmt: skip
    "pkv_copy_blocks": (ctypes.c_int, [_p, _p, _i64, _i32, _i64, _i64, _p, _i64, _p]),
    "pkv_decode_slots": (ctypes.c_int, [_p, _p, _i64, _i32, _p, _i32, _i32, _i64, _p]),
    "pkv_decode_workgroups": (_i32, [ctypes.c_int, _i32, _i32, _i32]),
    "pkv_decode_default_workgroups": (_i32, [ctypes.c_int, _i32, _i32, _i32, _i32, _i32, _i32]),
    "pkv_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "pkv_cascade_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "pkv_paged_decode": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _i64,            # out
         _p, _i64, _i64,                          # q
         _p, _p, ctypes.c_int, _i64, _i64, _i64,  # k, v caches
         _p, _i64, _i32,                          # block tables
         _p, _i32, _i32, _i32, _i32, _i32,        # ctx, batch, nh, nkv, hd, bs
         _f32, _i32, _p, _i64, _p],               # scale, wgs, workspace, stream
    ),  # fmt: skip
    "pkv_paged_decode_noalloc": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _i64,            # out
         _p, _i64, _i64,                          # q
         _p, _p, ctypes.c_int, _i64, _i64, _i64,  # k, v caches
         _p, _i64, _i32,                          # block tables
         _p, _i32, _i32, _i32, _i32, _i32,        # ctx, batch, nh, nkv, hd, bs
         _f32, _i32, _p],                         # scale, wgs, stream
    ),  # fmt: skip
    "pkv_rms_norm": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _p, ctypes.c_int, _i64, _p, _p, ctypes.c_int, _i64, _i64, _p],
    ),  # fmt: skip
    "pkv_rope": (ctypes.c_int, [_p, ctypes.c_int, _i64, _i64, _p, _p, _i64, _i64, _i32, _i32, _p]),
    "pkv_silu_mul": (ctypes.c_int, [_p, _p, _p, ctypes.c_int, _i64, _p]),
    "pkv_paged_decode_ex": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _i64,            # out
         _p, _i64, _i64,                          # q
         _p, _p, ctypes.c_int, _i64, _i64, _i64,  # k, v caches
         _p, _i64, _i32,                          # block tables
         _p, _i32, _i32, _i32, _i32, _i32,        # ctx, batch, nh, nkv, hd, bs
         _f32, _i32, _p, _i64,                    # scale, wgs, workspace
         _p, _p,                                  # first_block, lse
         _p, _p, _p, _i32, _i64,                  # prefix out, lse, row, parts, stride
         _p],                                     # stream
    ),  # fmt: skip
    "pkv_cascade_one_launch": (_i32, [ctypes.c_int, _i32, _i32, _i32, _i32, _i32]),
    "pkv_cascade_decode": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _i64,            # out
         _p, _i64, _i64,                          # q
         _p, _p, ctypes.c_int, _i64, _i64, _i64,  # k, v caches
         _p, _i64, _i32,                          # block tables
         _p, _i32, _i32, _i32, _i32, _i32,        # ctx, batch, nh, nkv, hd, bs
         _f32, _i32, _p, _i64,                    # scale, wgs, workspace
         _p, _p,                                  # first_block, lse
         _p, _i64, _i32,                          # prefix tables, stride, width
         _p, _p, _i32, _i32, _p,                  # prefix ctx, cu_q, chunks, max queries, q_rows
         _p, _p, _p, _i32, _i64,                  # prefix out, lse, row, parts, stride
         _i32, _p],                               # prefix workgroups, stream
    ),  # fmt: skip
    "pkv_paged_prefill_ex": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _i64,            # out
         _p, _i64, _i64,                          # q
         _p, _p, ctypes.c_int, _i64, _i64, _i64,  # k, v caches
         _p, _i64, _i32,                          # block tables
         _p, _p, _i32, _i32,                      # ctx, cu_q, n_chunks, max_query_len
         _i32, _i32, _i32, _i32, _f32,            # nh, nkv, hd, bs, scale
         _i32, _p, _p, _p],                       # causal, q_rows, lse, stream
    ),  # fmt: skip
    "pkv_paged_prefill": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _i64,            # out
         _p, _i64, _i64,                          # q
         _p, _p, ctypes.c_int, _i64, _i64, _i64,  # k, v caches
         _p, _i64, _i32,                          # block tables
         _p, _p, _i32, _i32,                      # ctx, cu_q, n_chunks, max_query_len
         _i32, _i32, _i32, _i32, _f32, _p],       # nh, nkv, hd, bs, scale, stream
    ),  # fmt: skip
    "pkv_prefill_workspace_bytes": (_i64, [ctypes.c_int, _i32, _i32, _i32, _i32, _i32]),
    "pkv_paged_prefill_ws": (
        ctypes.c_int,
        [_p, ctypes.c_int, _i64, _i64,            # out
         _p, _i64, _i64,                          # q
         _p, _p, ctypes.c_int, _i64, _i64, _i64,  # k, v caches
         _p, _i64, _i32,                          # block tables
         _p, _p, _i32, _i32,                      # ctx, cu_q, n_chunks, max_query_len
         _i32, _i32, _i32, _i32, _f32,            # nh, nkv, hd, bs, scale
         _p, _i64, _p],                           # workspace, bytes, stream
    ),  # fmt: skip
}

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it is not built or not loadable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"paged-KV HIP library not built ({LIB_PATH} missing); build it with "
                    "`python inference-engine_amd/csrc/build.py`"
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = restype, argtypes
            if handle.pkv_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"{LIB_PATH}: ABI version {handle.pkv_abi_version()}, expected {ABI_VERSION}"
                )
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Map a C ABI status to an exception: negative codes reject arguments (ValueError),
    positive ones are HIP launch errors (RuntimeError)."""
    if status == 0:
        return
    msg = lib().pkv_status_string(status).decode()
    if status < 0:
        raise ValueError(f"{what}: {msg} (status {status})")
    raise RuntimeError(f"{what}: HIP error {status}: {msg}")


def dtype_code(dtype: torch.dtype, what: str) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {dtype}") from None


def stream_of(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (captured into graphs as-is)."""
    return torch.cuda.current_stream(device).cuda_stream


# Opt-in checks of step metadata. The kernels never fault on bad metadata: the append
# skips slots outside the pool, and decode / prefill leave tokens whose slot falls
# outside the pool out of the softmax. The reference raises instead (index_copy_ and
# its gather index the pool, engine/runtime/paged_cache.py:42-49). With the checks on
# (environment PKV_DEBUG_CHECKS=1, or set_debug_checks(True)) every call first checks
# its metadata on the device and raises IndexError, as the reference would. Each check
# reads one flag back (a stream synchronisation), and is skipped while a graph is
# being captured.
_debug_checks = os.environ.get("PKV_DEBUG_CHECKS", "0") not in ("", "0")


def set_debug_checks(on: bool) -> bool:
    """Turn the metadata checks on or off; returns the previous setting."""
    global _debug_checks
    prev, _debug_checks = _debug_checks, bool(on)
    return prev


def debug_checks() -> bool:
    """Whether this call checks its metadata: on, and no graph capture under way."""
    if not _debug_checks:
        return False
    return not (torch.cuda.is_available() and torch.cuda.is_current_stream_capturing())


def check_slots(what: str, slots: torch.Tensor, num_slots: int) -> None:
    """IndexError unless every slot lies in [0, num_slots) (index_copy_'s rule)."""
    if slots.numel() and bool(((slots < 0) | (slots >= num_slots)).any()):
        bad = slots[(slots < 0) | (slots >= num_slots)][:4].tolist()
        raise IndexError(f"{what}: slots {bad} outside the pool of {num_slots} slots")


def check_tables(what: str, block_tables: torch.Tensor, context_lens: torch.Tensor,
                 block_size: int, num_slots: int, first: int = 0) -> None:  # fmt: skip
    """IndexError unless each row's first context_lens[b] tokens, read through columns
    first.. of its table, all have a slot in [0, num_slots): the context fits the table,
    and every used block id is non-negative with its used tokens inside the pool."""
    w = block_tables.shape[1] - first
    if context_lens.numel() == 0:
        return
    n = context_lens.long()
    if bool(((n < 0) | (n > w * block_size)).any()):
        raise IndexError(f"{what}: context_lens {n.min().item()}..{n.max().item()} outside "
                         f"[0, {w * block_size}] (the table's {w} columns)")  # fmt: skip
    if w <= 0:
        return
    cols = torch.arange(w, device=n.device) * block_size
    used = (n[:, None] - cols[None]).clamp(0, block_size)  # tokens each column holds
    bid = block_tables[:, first:].long()
    bad = (used > 0) & ((bid < 0) | (bid * block_size + used > num_slots))
    if bool(bad.any()):
        row, col = (int(x) for x in bad.nonzero()[0])
        raise IndexError(f"{what}: sequence {row} column {col + first}: block id "
                         f"{int(bid[row, col])} outside the pool of {num_slots} slots "
                         f"(block_size {block_size})")  # fmt: skip


def require_gpu(what: str, *tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError(f"{what}: tensors must be on a GPU device, got {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"{what}: all tensors must be on {dev}, got {t.device}")
    return dev
