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
ABI_VERSION = 3
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


def require_gpu(what: str, *tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError(f"{what}: tensors must be on a GPU device, got {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"{what}: all tensors must be on {dev}, got {t.device}")
    return dev
