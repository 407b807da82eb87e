"""Paged attention on MI355X (gfx950), same call signatures as the reference's
``engine/kernels/paged_attention.py``.

``paged_decode_attention`` runs hand-written HIP kernels through the C ABI of
lib/libpaged_kv.so, chosen by the library from static shapes:

1. a stream-K pass: the contexts of all sequences, laid end to end, are split evenly
   over as many workgroups as the GPU holds at once. One wave per KV head streams its
   share of K/V rows straight from the paged pool through the block table with 16-byte
   non-temporal loads, computes the scores of every query head sharing that KV head
   (GQA: each K/V row is read once for the whole group; on the matrix cores for 16-bit
   caches at head_dim 64 and 128) and keeps an fp32 online softmax. Sequences inside one
   workgroup's share are written directly; a combine pass merges, with log-sum-exp
   weights, the pieces of the sequences cut by a share boundary.
2. for small batches (every sequence's KV heads fit the CUs), one launch in which a
   workgroup's waves split one sequence and merge through LDS: no combine, no scratch.

With ``prefix_groups`` (cascade decode) the shared prefix of each group is attended once
for all its members by the chunked-prefill kernel (``paged_prefill_attention``'s), and
the decode passes read only each sequence's private blocks.

The grids depend only on the device and static shapes, never on the context lengths
(device data), so one hipGraph capture serves every length, as the reference's
CUDA-graph decode requires (reference engine/runtime/cuda_graphs.py:10-11). Nothing here
allocates outside torch's caching allocator or synchronises (the opt-in metadata checks
of ``_native.set_debug_checks`` excepted).
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import numpy as np
import torch

from engine.kernels import _native

# The reference exposes HAS_TRITON for engine/kernels/fused.py (reference
# engine/kernels/paged_attention.py:29-35). This build has no Triton anywhere.
HAS_TRITON = False

SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)
_default_wgs: dict[tuple, int] = {}
_default_plan: dict[tuple, int] = {}


def available(device: torch.device) -> bool:
    """True when ``device`` is a GPU and the HIP library loads (reference :38-39)."""
    if device.type != "cuda":
        return False
    try:
        _native.lib()
    except (RuntimeError, OSError):
        return False
    return True


def use_gqa_kernel(dtype: torch.dtype, groups: int, head_dim: int) -> bool:
    """Reference :182-189. Here one kernel serves every dtype and group size (query heads
    sharing a KV head are always read together), so this only reports whether the
    reference would have picked its grouped kernel for these arguments."""
    return (
        dtype in (torch.bfloat16, torch.float16)
        and groups <= 16
        and head_dim >= 16
        and head_dim & (head_dim - 1) == 0
    )


def decode_workgroups(device: torch.device, dtype: torch.dtype, head_dim: int,
                      num_heads: int, num_kv_heads: int) -> int:  # fmt: skip
    """Workgroups the decode kernel uses by default: as many as ``device`` holds at once
    for this shape (a device property, so graph captures stay valid). Cached."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, dtype, head_dim, num_heads, num_kv_heads)
    wgs = _default_wgs.get(key)
    if wgs is None:
        with torch.cuda.device(idx):
            wgs = _native.lib().pkv_decode_workgroups(
                _native.dtype_code(dtype, "decode_workgroups"), head_dim, num_heads,
                num_kv_heads)  # fmt: skip
        _native.check(min(wgs, 0), "decode_workgroups")
        _default_wgs[key] = wgs
    return wgs


def default_workgroups(device: torch.device, dtype: torch.dtype, head_dim: int,
                       num_heads: int, num_kv_heads: int, batch: int, max_blocks: int,
                       block_size: int) -> int:  # fmt: skip
    """What a call with the default split runs: 0 for the one-kernel per-sequence split
    (small batches of 16-bit K/V at head_dim 64/128; no workspace), else the stream-K
    workgroup count. Static shapes only (a graph captured with it stays valid)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, dtype, head_dim, num_heads, num_kv_heads, batch, max_blocks, block_size)
    wgs = _default_plan.get(key)
    if wgs is None:
        with torch.cuda.device(idx):
            wgs = _native.lib().pkv_decode_default_workgroups(
                _native.dtype_code(dtype, "default_workgroups"), head_dim, num_heads,
                num_kv_heads, batch, max_blocks, block_size)  # fmt: skip
        _native.check(min(wgs, 0), "default_workgroups")
        _default_plan[key] = wgs
    return wgs


def decode_workspace(device: torch.device, batch: int, num_heads: int, head_dim: int,
                     num_workgroups: int, *, cascade: bool = False) -> torch.Tensor | None:  # fmt: skip
    """Scratch for ``paged_decode_attention(..., num_workgroups=n, workspace=)``, e.g. to
    allocate it outside a hipGraph capture (None when the call needs none); ``cascade``:
    large enough for a call with ``prefix_groups`` too."""
    lib = _native.lib()
    query = lib.pkv_cascade_workspace_bytes if cascade else lib.pkv_decode_workspace_bytes
    nbytes = query(num_workgroups, batch, num_heads, head_dim)
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


@dataclass
class PrefixGroups:
    """Decode sequences that share leading KV blocks (a common prompt prefix held once in
    the pool), laid out for cascade decode. Built by ``find_prefix_groups``; all tensors
    int32 on the device. With S grouped sequences and K pieces per shared prefix:

    - first_block [B]: blocks of b's shared prefix (0 for ungrouped sequences): the
      decode pass starts there;
    - prefix_row [B]: b's row among the grouped sequences (-1: ungrouped); its k-th
      prefix part is row prefix_row[b] + k * S of the prefix pass;
    - q_rows [K * S], cu_q [K * C + 1], ctx [K * C], tables [K * C, W']: the prefix pass
      as K * C non-causal chunks (chunk k * C + g = piece k of group g: the group's
      queries against blocks [k P_g, (k + 1) P_g) of its prefix).
    """

    first_block: torch.Tensor
    prefix_row: torch.Tensor
    q_rows: torch.Tensor
    cu_q: torch.Tensor
    ctx: torch.Tensor
    tables: torch.Tensor
    members: int
    pieces: int
    max_members: int


def shared_prefixes(tables: np.ndarray, context_lens: np.ndarray, block_size: int,
                    min_blocks: int = 16) -> list[tuple[np.ndarray, int]]:  # fmt: skip
    """Groups of a decode batch's sequences that start with the same physical blocks, as
    (members ascending, shared blocks) in order of first block id.

    Sequences whose first block is the same form a group (at least two members); its
    shared prefix is the longest run of leading blocks every member's table holds and
    every member's context covers completely, kept if at least ``min_blocks`` long.
    tables: int [B, W]; context_lens: int [B] (host arrays)."""
    tables = np.asarray(tables)
    b, w = tables.shape
    full = np.minimum(np.asarray(context_lens, dtype=np.int64) // block_size, w)
    eligible = full >= min_blocks
    if w == 0 or int(eligible.sum()) < 2:
        return []
    firsts = np.where(eligible, tables[:, 0].astype(np.int64), -1)
    order = np.argsort(firsts, kind="stable")
    ranked = firsts[order]
    starts = np.flatnonzero(np.r_[True, ranked[1:] != ranked[:-1]])
    groups = []
    for lo, hi in zip(starts, np.r_[starts[1:], b], strict=True):
        if ranked[lo] < 0 or hi - lo < 2:
            continue
        members = order[lo:hi]  # stable sort: already ascending
        rows = tables[members]
        lcp = np.cumprod(rows == rows[:1], axis=1).sum(1)
        shared = int(np.minimum(lcp, full[members]).min())
        if shared >= min_blocks:
            groups.append((members, shared))
    return groups


def find_prefix_groups(block_tables: Sequence[Sequence[int]] | torch.Tensor,
                       context_lens: Sequence[int] | torch.Tensor, block_size: int,
                       num_heads: int, num_kv_heads: int, device: torch.device, *,
                       min_blocks: int = 16, target_workgroups: int | None = None,
                       pieces: int | None = None, dtype: torch.dtype | None = None,
                       head_dim: int | None = None) -> PrefixGroups | None:  # fmt: skip
    """The ``shared_prefixes`` groups of a decode batch laid out for cascade decode
    (host-side, from the tables the engine's block manager produced); None when no group
    qualifies. Each prefix is cut into K pieces (K >= 1, pieces of at least 4 blocks),
    K = ``pieces`` if given. Otherwise, when the cache's ``dtype`` and ``head_dim`` are
    given and the library runs these shapes' prefix and decode passes as one launch, K is
    ``one_launch_pieces`` of the prefix pass's work items; else K is the most whose
    prefix pass has at most ``target_workgroups`` workgroups (default: the GPU's CU
    count, one workgroup per CU -- a second per CU shares the same matrix cores and only
    adds parts to merge)."""
    tables = torch.as_tensor(block_tables, dtype=torch.int32).cpu().numpy()
    ctx = torch.as_tensor(context_lens, dtype=torch.int64).cpu().numpy()
    groups = shared_prefixes(tables, ctx, block_size, min_blocks)
    if not groups:
        return None
    b = tables.shape[0]
    g_count = len(groups)
    sizes = [len(m) for m, _ in groups]
    s_total = sum(sizes)
    max_members = max(sizes)
    dev = torch.device(device)
    if pieces is None:
        per_piece = _prefix_workgroups(max_members, num_heads // num_kv_heads, num_kv_heads)
        if dtype is not None and head_dim is not None and \
                cascade_one_launch(dtype, head_dim, num_heads, num_kv_heads, block_size, b, dev):  # fmt: skip
            pieces = one_launch_pieces(per_piece * g_count, dev)
        else:
            if target_workgroups is None:
                target_workgroups = _cu_count(dev)
            pieces = target_workgroups // (per_piece * g_count)
    pieces = max(1, min(pieces, min(sh for _, sh in groups) // 4))
    width = max(-(-shared // pieces) for _, shared in groups)
    host = np.zeros(prefix_entries(b, pieces, g_count, width, s_total), dtype=np.int32)
    fill_prefix(host, b, pieces, g_count, width, tables, groups, block_size, s_total)
    return prefix_view(torch.from_numpy(host).to(dev), b, pieces, g_count, width,
                        members=s_total, max_members=max_members)  # fmt: skip


def _cu_count(dev: torch.device) -> int:
    return torch.cuda.get_device_properties(dev).multi_processor_count \
        if dev.type == "cuda" else 256  # fmt: skip


def _prefix_workgroups(members: int, groups: int, num_kv_heads: int) -> int:
    """Workgroups of one prefix piece of a group: 128 query rows (member x query head of
    one KV head) per workgroup, for every KV head."""
    return max(1, -(-members * groups // 128) * num_kv_heads)


def cascade_one_launch(dtype: torch.dtype, head_dim: int, num_heads: int, num_kv_heads: int,
                       block_size: int, batch: int, device: torch.device) -> bool:  # fmt: skip
    """Whether cascade decode of ``batch`` sequences at these shapes runs its prefix pass
    and decode pass as one launch on ``device`` (``pkv_cascade_one_launch``)."""
    code = _native.DTYPE_CODE.get(dtype)
    if torch.device(device).type != "cuda" or code is None:
        return False
    return _native.lib().pkv_cascade_one_launch(code, head_dim, num_heads, num_kv_heads,
                                                block_size, batch) == 1  # fmt: skip


def one_launch_pieces(items: int, device: torch.device, max_pieces: int = 8) -> int:
    """Pieces per prefix for the one-launch cascade, whose prefix pass has ``items`` work
    items per piece: about 7/32 of the GPU's workgroups in items, one per prefix
    workgroup (measured on 256 CUs at 96-512 sequences sharing a 2,048-token prefix)."""
    target = 7 * _cu_count(torch.device(device)) / 32
    return max(1, min(max_pieces, round(target / max(1, items))))


def cascade_pieces(batch: int, num_heads: int, num_kv_heads: int, device: torch.device,
                   max_pieces: int = 8, *, dtype: torch.dtype | None = None,
                   head_dim: int | None = None, block_size: int | None = None) -> int:  # fmt: skip
    """Pieces per shared prefix for a captured step of ``batch`` sequences. With the
    cache's ``dtype``, ``head_dim`` and ``block_size`` given and a one-launch cascade
    for these shapes: ``one_launch_pieces`` of one group's prefix items; else as many
    as keep one group's prefix pass within one workgroup per CU (at most
    ``max_pieces``)."""
    per_piece = _prefix_workgroups(batch, num_heads // num_kv_heads, num_kv_heads)
    if dtype is not None and head_dim is not None and block_size is not None and \
            cascade_one_launch(dtype, head_dim, num_heads, num_kv_heads, block_size, batch,
                               device):  # fmt: skip
        return one_launch_pieces(per_piece, device, max_pieces)
    return max(1, min(max_pieces, _cu_count(torch.device(device)) // per_piece))


# Layout of prefix groups in one int32 array, for a batch of n sequences, K pieces, C
# chunks per piece, piece tables W' wide and member rows S apart between pieces:
# first_block [n] | prefix_row [n] | q_rows [K S] | cu_q [K C + 1] | ctx [K C] |
# tables [K C, W']. Part k of grouped sequence b is row prefix_row[b] + k S of the
# prefix pass.
def prefix_entries(n: int, pieces: int, slots: int, width: int, stride: int) -> int:
    chunks = pieces * slots
    return 2 * n + pieces * stride + 2 * chunks + 1 + chunks * width


def prefix_view(flat: torch.Tensor, n: int, pieces: int, groups: int, width: int, *,
                 members: int, max_members: int) -> PrefixGroups:  # fmt: skip
    chunks = pieces * groups
    at = [0]

    def take(count: int) -> torch.Tensor:
        t = flat[at[0] : at[0] + count]
        at[0] += count
        return t

    return PrefixGroups(first_block=take(n), prefix_row=take(n), q_rows=take(pieces * members),
                        cu_q=take(chunks + 1), ctx=take(chunks),
                        tables=take(chunks * width).view(chunks, width), members=members,
                        pieces=pieces, max_members=max_members)  # fmt: skip


def fill_prefix(host: np.ndarray, n: int, pieces: int, slots: int, width: int,
                tables: np.ndarray, groups: list[tuple[np.ndarray, int]], block_size: int,
                stride: int) -> None:  # fmt: skip
    """Write ``groups`` (at most ``slots``) into the flat layout above: ``slots`` chunks per
    piece, the groups' member rows ``stride`` apart between pieces. Sequences outside
    every group get first_block 0 and prefix_row -1. Rows of a piece past its groups'
    members (when stride exceeds them) belong to the piece's last chunk, with q_rows -1:
    the prefix pass skips them (a workgroup holding only such rows leaves at once)."""
    if len(groups) > slots:
        raise ValueError(f"prefix groups: {len(groups)} groups for {slots} chunk slots")
    chunks = pieces * slots
    o_pr, o_qr = n, 2 * n
    o_cu = o_qr + pieces * stride
    o_ctx = o_cu + chunks + 1
    o_tab = o_ctx + chunks
    host[: o_tab + chunks * width] = 0
    host[o_pr : o_pr + n] = -1
    host[o_qr : o_qr + pieces * stride] = -1
    ptab = host[o_tab : o_tab + chunks * width].reshape(chunks, width)
    ends, row = [], 0
    for g, (members, shared) in enumerate(groups):
        size = len(members)
        host[members] = shared  # first_block
        host[o_pr + members] = np.arange(row, row + size)
        pb = -(-shared // pieces)
        for k in range(pieces):
            host[o_qr + k * stride + row : o_qr + k * stride + row + size] = members
            lo, hi = min(k * pb, shared), min((k + 1) * pb, shared)
            c = k * slots + g
            ptab[c, : hi - lo] = tables[members[0], lo:hi]
            host[o_ctx + c] = (hi - lo) * block_size
        row += size
        ends.append(row)
    if row > stride:
        raise ValueError(f"prefix groups: {row} member rows for a stride of {stride}")
    # cu_q: chunk k * slots + g ends at k S + (its group's last row); unused chunks of a
    # piece are empty but for the last, which runs to the next piece's first row.
    cu = np.zeros(chunks + 1, dtype=np.int64)
    for k in range(pieces):
        for g in range(slots):
            c = k * slots + g
            cu[c + 1] = k * stride + (ends[g] if g < len(ends) else row)
        cu[(k + 1) * slots] = (k + 1) * stride
    host[o_cu : o_cu + chunks + 1] = cu


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
    block_n: int = 64,
    *,
    out: torch.Tensor | None = None,
    num_workgroups: int | None = None,
    workspace: torch.Tensor | None = None,
    prefix_groups: PrefixGroups | None = None,
    prefix_workgroups: int | None = None,
) -> torch.Tensor:
    """q: [B, nh, hd]; k_cache, v_cache: [num_slots, nkv, hd] (one layer);
    block_tables: [B, max_blocks] int32; context_lens: [B] int32 -> [B, nh, hd].

    Reference: engine/kernels/paged_attention.py:140-179. ``block_n`` (the reference's
    Triton tile) is accepted and ignored. Extensions: ``out`` receives the result in
    place ([B, nh, hd], q.dtype or float32 for the unrounded fp32 result) and
    ``num_workgroups`` sets how many workgroups share the contexts in the stream-K split
    (default: the library's choice from static shapes -- for small batches at head_dim
    64/128 one kernel that splits each sequence among one workgroup's waves, else as
    many stream-K workgroups as the GPU holds at once); ``workspace`` (uint8, from
    ``decode_workspace`` with ``decode_workgroups()``) replaces the scratch otherwise
    taken from torch's caching allocator on each call.
    ``prefix_groups`` (from ``find_prefix_groups``) turns on cascade decode for 16-bit
    caches at head_dim 32-256: each group's shared prefix is read once for all its
    members on the matrix cores (the chunked-prefill kernel, non-causal, one fp32 part
    per piece with its log-sum-exp), then the decode kernel reads only each sequence's
    private blocks and merges the parts into its softmax as it finishes each sequence.
    Other shapes ignore it (the plain decode is exact). Where the shapes allow it, the
    prefix pass and the decode pass share one launch: ``prefix_workgroups`` of the
    workgroups (None: the library's default) take the prefix items while the others
    stream the private blocks; a negative value runs them as two launches.
    """
    del block_n
    what = "paged_decode_attention"
    dev = _check_decode_args(what, q, k_cache, v_cache, block_tables, context_lens, block_size)
    b, nh, hd = q.shape
    nkv = k_cache.shape[1]
    kv_code = _native.dtype_code(k_cache.dtype, what)

    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    else:
        _check_out(what, out, q, dev)
    if b == 0:
        return out

    max_blocks = block_tables.shape[1]
    lib = _native.lib()
    cascade = prefix_groups is not None and q.dtype in (torch.bfloat16, torch.float16) \
        and hd in PREFILL_HEAD_DIMS  # fmt: skip
    if cascade:
        _check_prefix_groups(prefix_groups, b, dev, what)
    # None: the library's default (C: 0): the one-kernel split for small batches (no
    # workspace), else the stream-K split over decode_workgroups() workgroups.
    wg_arg = 0 if num_workgroups is None else num_workgroups
    if num_workgroups is None:
        num_workgroups = decode_workgroups(dev, q.dtype, hd, nh, nkv) if cascade else \
            default_workgroups(dev, q.dtype, hd, nh, nkv, b, max_blocks, block_size)  # fmt: skip
    query = lib.pkv_cascade_workspace_bytes if cascade else lib.pkv_decode_workspace_bytes
    ws_bytes = query(num_workgroups, b, nh, hd) if num_workgroups else 0
    ws = None
    if ws_bytes and workspace is not None:
        if workspace.device != dev or workspace.dtype != torch.uint8 or \
                workspace.numel() < ws_bytes or not workspace.is_contiguous():  # fmt: skip
            raise ValueError(f"{what}: workspace must be a contiguous uint8 tensor of at "
                             f"least {ws_bytes} bytes on {dev}")  # fmt: skip
        ws = workspace
    elif ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    common = (
        out.data_ptr(), _native.dtype_code(out.dtype, what), out.stride(0), out.stride(1),
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), kv_code,
        k_cache.stride(0), k_cache.stride(1), k_cache.shape[0],
        block_tables.data_ptr(), block_tables.stride(0), max_blocks,
        context_lens.data_ptr(), b, nh, nkv, hd, block_size,
        hd**-0.5, wg_arg, ws.data_ptr() if ws is not None else None, ws_bytes,
    )  # fmt: skip
    if cascade:
        pg = prefix_groups
        rows = pg.pieces * pg.members
        o_pre = torch.empty(rows, nh, hd, dtype=torch.float32, device=dev)
        lse_pre = torch.empty(rows, nh, dtype=torch.float32, device=dev)
        pwg = 0 if prefix_workgroups is None else prefix_workgroups
        status = lib.pkv_cascade_decode(
            *common, pg.first_block.data_ptr(), None,
            pg.tables.data_ptr(), pg.tables.stride(0), pg.tables.shape[1],
            pg.ctx.data_ptr(), pg.cu_q.data_ptr(), pg.ctx.numel(), pg.max_members,
            pg.q_rows.data_ptr(), o_pre.data_ptr(), lse_pre.data_ptr(),
            pg.prefix_row.data_ptr(), pg.pieces, pg.members, pwg, _native.stream_of(dev),
        )  # fmt: skip
    else:
        status = lib.pkv_paged_decode_ex(*common, None, None, None, None, None, 0, 0,
                                         _native.stream_of(dev))  # fmt: skip
    _native.check(status, what)
    return out


def paged_decode_attention_noalloc(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
    *,
    out: torch.Tensor,
    num_workgroups: int | None = None,
) -> torch.Tensor:
    """``paged_decode_attention`` for callers that cannot allocate: the split-K scratch
    is a static per-GPU device array of the library (C ``pkv_paged_decode_noalloc``), the
    result goes to the caller's ``out`` ([B, nh, hd], q.dtype or float32), and q must be
    contiguous. Same kernels and results as ``paged_decode_attention`` at the same
    ``num_workgroups``. Shapes whose scratch exceeds ``_native.PKV_NOALLOC_SCRATCH_BYTES``
    raise ValueError; calls that overlap on one GPU (other streams) race on the scratch.
    No counterpart in the reference."""
    what = "paged_decode_attention_noalloc"
    dev = _check_decode_args(what, q, k_cache, v_cache, block_tables, context_lens, block_size)
    b, nh, hd = q.shape
    nkv = k_cache.shape[1]
    if not q.is_contiguous():
        raise ValueError(f"{what}: q must be contiguous (no copy is made)")
    _check_out(what, out, q, dev)
    if b == 0:
        return out
    if num_workgroups is None:
        num_workgroups = 0  # the library's default split
    status = _native.lib().pkv_paged_decode_noalloc(
        out.data_ptr(), _native.dtype_code(out.dtype, what), out.stride(0), out.stride(1),
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), _native.dtype_code(k_cache.dtype, what),
        k_cache.stride(0), k_cache.stride(1), k_cache.shape[0],
        block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
        context_lens.data_ptr(), b, nh, nkv, hd, block_size, hd**-0.5, num_workgroups,
        _native.stream_of(dev),
    )  # fmt: skip
    _native.check(status, what)
    return out


def _check_out(what: str, out: torch.Tensor, q: torch.Tensor, dev: torch.device) -> None:
    if out.shape != q.shape or out.dtype not in (q.dtype, torch.float32) or \
            out.stride(2) != 1 or out.device != dev:  # fmt: skip
        raise ValueError(f"{what}: out must be [B, nh, hd] of {q.dtype} or float32 on {dev}")


def _check_decode_args(what, q, k_cache, v_cache, block_tables, context_lens,
                       block_size) -> torch.device:  # fmt: skip
    """The decode entry points' argument checks (before any launch); returns the device."""
    dev = _native.require_gpu(what, q, k_cache, v_cache, block_tables, context_lens)
    if q.dim() != 3 or k_cache.dim() != 3 or v_cache.dim() != 3:
        raise ValueError(f"{what}: q, k_cache, v_cache must be 3-D")
    b, nh, hd = q.shape
    nkv = k_cache.shape[1]
    if v_cache.shape != k_cache.shape or k_cache.shape[2] != hd:
        raise ValueError(f"{what}: cache shapes {tuple(k_cache.shape)}, "
                         f"{tuple(v_cache.shape)} do not match q {tuple(q.shape)}")  # fmt: skip
    if nh % nkv:
        raise ValueError(f"{what}: {nh} query heads not a multiple of {nkv} KV heads")
    if hd not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{what}: head_dim {hd} not in {SUPPORTED_HEAD_DIMS}")
    if q.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise TypeError(f"{what}: q {q.dtype} and caches {k_cache.dtype}/{v_cache.dtype} "
                        "must share one dtype")  # fmt: skip
    if k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1:
        raise ValueError(f"{what}: k_cache and v_cache need equal strides, unit in head_dim")
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise TypeError(f"{what}: block_tables and context_lens must be int32")
    if block_tables.dim() != 2 or block_tables.shape[0] != b or block_tables.stride(1) != 1:
        raise ValueError(f"{what}: block_tables must be [B, max_blocks] with unit column stride")
    if context_lens.shape != (b,) or not context_lens.is_contiguous():
        raise ValueError(f"{what}: context_lens must be a contiguous [B] tensor")
    if block_size <= 0:
        raise ValueError(f"{what}: block_size must be positive")
    if _native.debug_checks():
        _native.check_tables(what, block_tables, context_lens, block_size, k_cache.shape[0])
    return dev


def _check_prefix_groups(pg: PrefixGroups, batch: int, dev: torch.device, what: str) -> None:
    """The kernels read first_block[b] and prefix_row[b] for every sequence b and the
    prefix pass's tables by chunk: a PrefixGroups built for another step (another batch
    size or order) must be rejected before launch, not read out of bounds."""
    fields = {"first_block": pg.first_block, "prefix_row": pg.prefix_row, "q_rows": pg.q_rows,
              "cu_q": pg.cu_q, "ctx": pg.ctx, "tables": pg.tables}  # fmt: skip
    for name, t in fields.items():
        if t.dtype != torch.int32 or t.device != dev or not t.is_contiguous():
            raise ValueError(f"{what}: prefix_groups.{name} must be a contiguous int32 "
                             f"tensor on {dev}")  # fmt: skip
    if pg.first_block.shape != (batch,) or pg.prefix_row.shape != (batch,):
        raise ValueError(f"{what}: prefix_groups built for {pg.first_block.numel()} "
                         f"sequences, called with {batch}")  # fmt: skip
    chunks = pg.ctx.numel()
    if pg.pieces < 1 or pg.members < 1 or chunks % pg.pieces or \
            pg.cu_q.shape != (chunks + 1,) or pg.tables.dim() != 2 or \
            pg.tables.shape[0] != chunks or pg.q_rows.shape != (pg.pieces * pg.members,):  # fmt: skip
        raise ValueError(f"{what}: prefix_groups fields disagree with each other")


def reference_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
) -> torch.Tensor:
    """Plain PyTorch gather-then-attention, one sequence at a time (reference :192-211):
    the slow path the kernel is checked against. fp32 math, result cast to q.dtype."""
    outs = []
    groups = q.shape[1] // k_cache.shape[1]
    scale = q.shape[-1] ** -0.5
    for i in range(q.shape[0]):
        n = int(context_lens[i])
        pos = torch.arange(n, device=q.device)
        slots = block_tables[i, pos // block_size].long() * block_size + pos % block_size
        k = k_cache[slots].float().repeat_interleave(groups, dim=1).transpose(0, 1).contiguous()
        v = v_cache[slots].float().repeat_interleave(groups, dim=1).transpose(0, 1).contiguous()
        w = torch.softmax((k @ q[i].float()[:, :, None])[..., 0] * scale, dim=-1)  # [nh, n]
        outs.append((w[:, None, :] @ v)[:, 0])  # [nh, hd]
    return torch.stack(outs).to(q.dtype)


PREFILL_HEAD_DIMS = (32, 64, 128, 256)


def paged_prefill_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
    cu_seqlens_q: torch.Tensor,
    max_query_len: int,
    *,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Bottom-right causal attention of prompt chunks over the paged pool.

    q: [T, nh, hd] -- the query tokens of all chunks back to back; chunk c owns rows
    cu_seqlens_q[c] .. cu_seqlens_q[c+1]-1. block_tables: int32 [C, W];
    context_lens: int32 [C], tokens in the cache for chunk c including its own (which
    come last). Query i of a chunk of q_c tokens attends to keys 0 .. ctx_c - q_c + i.
    -> [T, nh, hd] in q.dtype (or ``out``, q.dtype or float32).

    Replaces the gather of every chunk's context slots plus the FlashAttention varlen call
    of the reference (engine/model/layers.py:246-253; metadata built at
    engine/runtime/paged_cache.py:182-202) without materialising the gathered K/V.
    ``max_query_len`` bounds every chunk (it sizes the grid: one graph per bucket).
    16-bit caches at head_dim 32-256 run on the matrix cores (the reference's
    FlashAttention shapes); fp32 caches and head_dim 16 (the reference's per-chunk SDPA
    path, layers.py:254-265) on a VALU kernel that stages each K/V tile in LDS once per
    16 query tokens. For bf16 caches the call first writes each chunk's V as fp16 (per
    256-token tile scaled by a power of two that keeps it inside fp16's range) into a
    workspace, so that P enters the second product once, in fp16, instead of as a bf16
    hi + lo pair; ``workspace`` (a CUDA byte tensor of at least
    ``prefill_workspace_bytes(...)``) supplies it, else the call allocates one of that
    size through torch (at most ``PREFILL_WORKSPACE_MAX_BYTES``; beyond it, and for other
    dtypes, the call takes no copy).
    """
    what = "paged_prefill_attention"
    dev = _native.require_gpu(what, q, k_cache, v_cache, block_tables, context_lens,
                              cu_seqlens_q)  # fmt: skip
    if q.dim() != 3 or k_cache.dim() != 3 or v_cache.shape != k_cache.shape:
        raise ValueError(f"{what}: q [T, nh, hd] and equal caches [slots, nkv, hd] expected")
    t, nh, hd = q.shape
    nkv = k_cache.shape[1]
    if k_cache.shape[2] != hd or nh % nkv:
        raise ValueError(f"{what}: cache {tuple(k_cache.shape)} does not fit q {tuple(q.shape)}")
    if hd not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{what}: head_dim {hd} not in {SUPPORTED_HEAD_DIMS}")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise TypeError(f"{what}: q {q.dtype} and caches {k_cache.dtype}/{v_cache.dtype} "
                        "must share one dtype")  # fmt: skip
    if k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1:
        raise ValueError(f"{what}: k_cache and v_cache need equal strides, unit in head_dim")
    for name, x in (("block_tables", block_tables), ("context_lens", context_lens),
                    ("cu_seqlens_q", cu_seqlens_q)):  # fmt: skip
        if x.dtype != torch.int32:
            raise TypeError(f"{what}: {name} must be int32")
    n_chunks = context_lens.numel()
    if block_tables.dim() != 2 or block_tables.shape[0] != n_chunks or \
            block_tables.stride(1) != 1 or cu_seqlens_q.shape != (n_chunks + 1,):  # fmt: skip
        raise ValueError(f"{what}: block_tables [C, W], context_lens [C], cu_seqlens_q [C+1]")
    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype not in (q.dtype, torch.float32) or \
            out.stride(2) != 1 or out.device != dev:  # fmt: skip
        raise ValueError(f"{what}: out must be [T, nh, hd] of {q.dtype} or float32 on {dev}")
    if block_size <= 0:
        raise ValueError(f"{what}: block_size must be positive")
    if n_chunks == 0 or t == 0:
        return out
    if _native.debug_checks():
        _check_chunks(what, block_tables, context_lens, block_size, k_cache.shape[0],
                      cu_seqlens_q, t, max_query_len)  # fmt: skip
    context_lens = context_lens.contiguous()
    cu_seqlens_q = cu_seqlens_q.contiguous()
    kv_code = _native.dtype_code(k_cache.dtype, what)
    if workspace is None:
        need = prefill_workspace_bytes(k_cache.dtype, hd, nkv, n_chunks, block_tables.shape[1],
                                       block_size)  # fmt: skip
        if 0 < need <= PREFILL_WORKSPACE_MAX_BYTES:
            workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif not workspace.is_contiguous() or workspace.device != dev:
        raise ValueError(f"{what}: workspace must be a contiguous tensor on {dev}")
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    status = _native.lib().pkv_paged_prefill_ws(
        out.data_ptr(), _native.dtype_code(out.dtype, what), out.stride(0), out.stride(1),
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), kv_code,
        k_cache.stride(0), k_cache.stride(1), k_cache.shape[0],
        block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
        context_lens.data_ptr(), cu_seqlens_q.data_ptr(), n_chunks, int(max_query_len),
        nh, nkv, hd, block_size, hd**-0.5, ws_ptr, ws_bytes, _native.stream_of(dev),
    )  # fmt: skip
    _native.check(status, what)
    return out


# Largest workspace paged_prefill_attention allocates by itself for the fp16 V copy.
PREFILL_WORKSPACE_MAX_BYTES = 1 << 30


def prefill_workspace_bytes(dtype: torch.dtype, head_dim: int, num_kv_heads: int,
                            n_chunks: int, max_blocks: int, block_size: int) -> int:
    """Workspace bytes with which a prefill call of these static shapes writes the fp16
    copy of every chunk's V (0: the shapes take none; pkv_prefill_workspace_bytes)."""
    n = _native.lib().pkv_prefill_workspace_bytes(
        _native.DTYPE_CODE.get(dtype, -1), head_dim, num_kv_heads, n_chunks, max_blocks,
        block_size)  # fmt: skip
    if n < 0:
        _native.check(n, "prefill_workspace_bytes")
    return int(n)


def _check_chunks(what, block_tables, context_lens, block_size, num_slots, cu_seqlens_q,
                  num_rows, max_query_len) -> None:  # fmt: skip
    """Prefill metadata under the debug checks: cu_seqlens_q non-decreasing from 0 within
    q's rows, every chunk at most max_query_len rows and no longer than its context, and
    every context token's slot inside the pool. The kernel clamps or masks each of these
    instead (a chunk past max_query_len loses its last rows)."""
    cu = cu_seqlens_q.long()
    q_len = cu[1:] - cu[:-1]
    if int(cu[0]) != 0 or bool((q_len < 0).any()) or int(cu[-1]) > num_rows:
        raise IndexError(f"{what}: cu_seqlens_q must rise from 0 to at most {num_rows}")
    if bool((q_len > max_query_len).any()) or bool((q_len > context_lens.long()).any()):
        raise IndexError(f"{what}: a chunk is longer than max_query_len {max_query_len} or "
                         "than its context")  # fmt: skip
    _native.check_tables(what, block_tables, context_lens, block_size, num_slots)
