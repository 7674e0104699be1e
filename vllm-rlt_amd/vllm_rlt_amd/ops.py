"""Tensor-level entry points over the librlt_kv C ABI.

Each function validates shapes, dtypes and devices on the host (raising
ValueError, as the reference's callers expect) and then enqueues the HIP
kernel on the current stream of the tensors' device.  Nothing here computes on
the CPU and nothing falls back to another implementation.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _native
from ._native import check, dtype_code, int64_array, stream_handle


def _require_rocm(*tensors: torch.Tensor) -> torch.device:
    device = tensors[0].device
    if device.type != "cuda":
        raise ValueError("the hip backend requires a ROCm device")
    for t in tensors[1:]:
        if t.device != device:
            raise ValueError("all tensors must be on the same ROCm device")
    return device


def _require_int(t: torch.Tensor, dtype: torch.dtype, name: str, ndim: int = 1) -> None:
    if t.dtype != dtype or t.ndim != ndim:
        raise ValueError(f"{name} must be a {ndim}-D {dtype} tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def kv_append(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    layer: int,
    write_blocks: torch.Tensor,
    write_offsets: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    n_rows: int | None = None,
) -> None:
    """key_cache[write_blocks[i], layer, write_offsets[i]] = k[i] (and V) for i < n_rows.

    Mirrors the index_put pair of vllm_rlt/core/kv_cache_manager.py:531-532.
    """
    device = _require_rocm(key_cache, value_cache, write_blocks, write_offsets, k, v)
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must share shape and strides")
    if key_cache.ndim != 5:
        raise ValueError("caches must be [blocks, layers, page, kv_heads, head_dim]")
    nb, nl, page, hkv, d = key_cache.shape
    for t, name in ((k, "k"), (v, "v")):
        if t.ndim != 3 or t.shape[1:] != (hkv, d):
            raise ValueError(f"{name} must have shape [batch, {hkv}, {d}]")
        if t.dtype != key_cache.dtype:
            raise ValueError(f"{name} must use dtype {key_cache.dtype}")
    _require_int(write_blocks, torch.int64, "write_blocks")
    _require_int(write_offsets, torch.int64, "write_offsets")
    n = len(write_blocks) if n_rows is None else n_rows
    if n > min(len(write_blocks), len(write_offsets), k.shape[0], v.shape[0]):
        raise ValueError("n_rows exceeds the provided rows")
    lib = _native.load()
    rc = lib.rlt_kv_append(
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int64_array(key_cache.stride()),
        k.data_ptr(),
        int64_array(k.stride()),
        v.data_ptr(),
        int64_array(v.stride()),
        write_blocks.data_ptr(),
        write_offsets.data_ptr(),
        n,
        layer,
        nl,
        nb,
        page,
        hkv,
        d,
        dtype_code(key_cache.dtype),
        stream_handle(device),
    )
    check(rc, "rlt_kv_append")


def rope_kv_append(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    layer: int,
    write_blocks: torch.Tensor,
    write_offsets: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    out: torch.Tensor | None = None,
    n_rows: int | None = None,
) -> torch.Tensor:
    """Rotate q and k by (cos, sin), append rotated k and v; returns rotated q.

    One launch for the rotation of vllm_rlt/models/ouro.py:104-109
    (q * cos + rotate_half(q) * sin, same for k) and the index_put pair of
    vllm_rlt/core/kv_cache_manager.py:531-532.  cos and sin are the per-row
    [batch, head_dim] tables the model computes once per traversal (a
    broadcast [batch, 1, head_dim] view is accepted).  Rows below n_rows
    (default: all of write_blocks) are written; q is rotated for every row.
    `out` may be q itself.
    """
    device = _require_rocm(key_cache, value_cache, write_blocks, write_offsets, q, k, v, cos, sin)
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must share shape and strides")
    if key_cache.ndim != 5:
        raise ValueError("caches must be [blocks, layers, page, kv_heads, head_dim]")
    nb, nl, page, hkv, d = key_cache.shape
    if d % 2:
        raise ValueError("head_dim must be even for split-half RoPE")
    rows = q.shape[0]
    if q.ndim != 3 or q.shape[2] != d or q.shape[1] % hkv:
        raise ValueError(f"q must have shape [batch, heads, {d}] with heads a multiple of {hkv}")
    for t, name in ((k, "k"), (v, "v")):
        if t.ndim != 3 or t.shape != (rows, hkv, d):
            raise ValueError(f"{name} must have shape [{rows}, {hkv}, {d}]")
    if cos.ndim == 3 and cos.shape[1] == 1:
        cos = cos[:, 0]
    if sin.ndim == 3 and sin.shape[1] == 1:
        sin = sin[:, 0]
    if cos.shape != (rows, d) or sin.shape != (rows, d) or cos.stride() != sin.stride():
        raise ValueError(f"cos and sin must be [{rows}, {d}] with equal strides")
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (cos, "cos"), (sin, "sin")):
        if t.dtype != key_cache.dtype:
            raise ValueError(f"{name} must use dtype {key_cache.dtype}")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError("out must match q")
    _require_int(write_blocks, torch.int64, "write_blocks")
    _require_int(write_offsets, torch.int64, "write_offsets")
    n = len(write_blocks) if n_rows is None else n_rows
    if n > min(len(write_blocks), len(write_offsets), rows):
        raise ValueError("n_rows exceeds the provided rows")
    rc = _native.load().rlt_rope_kv_append(
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int64_array(key_cache.stride()),
        q.data_ptr(),
        int64_array(q.stride()),
        k.data_ptr(),
        int64_array(k.stride()),
        v.data_ptr(),
        int64_array(v.stride()),
        cos.data_ptr(),
        sin.data_ptr(),
        int64_array(cos.stride()),
        out.data_ptr(),
        int64_array(out.stride()),
        write_blocks.data_ptr(),
        write_offsets.data_ptr(),
        rows,
        n,
        layer,
        nl,
        nb,
        page,
        q.shape[1],
        hkv,
        d,
        dtype_code(key_cache.dtype),
        stream_handle(device),
    )
    check(rc, "rlt_rope_kv_append")
    return out


def _row_bytes(t: torch.Tensor, name: str) -> int:
    if t.ndim != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D with contiguous rows")
    return t.shape[1] * t.element_size()


def gather_rows(pool: torch.Tensor, slots: torch.Tensor, out: torch.Tensor, count: int) -> torch.Tensor:
    """out[r] = pool[slots[r]] for r < count, zeros for the remaining rows of out.

    gather_kernel of vllm_rlt/kernels/routing.py:45-59 (RoutingBank.gather,
    vllm_rlt/worker/async_state.py:93-102).  Returns out.
    """
    device = _require_rocm(pool, slots, out)
    _require_int(slots, torch.int64, "slots")
    row_bytes = _row_bytes(pool, "pool")
    if _row_bytes(out, "out") != row_bytes or out.dtype != pool.dtype:
        raise ValueError("out rows must match pool rows")
    if not 0 <= count <= min(out.shape[0], slots.numel()):
        raise ValueError("count exceeds the rows of out or slots")
    rc = _native.load().rlt_gather_rows(
        pool.data_ptr(), pool.stride(0) * pool.element_size(), pool.shape[0], slots.data_ptr(), count,
        out.shape[0], out.data_ptr(), out.stride(0) * out.element_size(), row_bytes, stream_handle(device),
    )
    check(rc, "rlt_gather_rows")
    return out


def scatter_rows(values: torch.Tensor, slots: torch.Tensor, pool: torch.Tensor, count: int | None = None) -> None:
    """pool[slots[r]] = values[r] for r < count (scatter_kernel, vllm_rlt/kernels/routing.py:62-76)."""
    device = _require_rocm(values, slots, pool)
    _require_int(slots, torch.int64, "slots")
    row_bytes = _row_bytes(pool, "pool")
    if _row_bytes(values, "values") != row_bytes or values.dtype != pool.dtype:
        raise ValueError("values rows must match pool rows")
    n = values.shape[0] if count is None else count
    if not 0 <= n <= min(values.shape[0], slots.numel()):
        raise ValueError("count exceeds the rows of values or slots")
    rc = _native.load().rlt_scatter_rows(
        values.data_ptr(), values.stride(0) * values.element_size(), slots.data_ptr(), n, pool.data_ptr(),
        pool.stride(0) * pool.element_size(), pool.shape[0], row_bytes, stream_handle(device),
    )
    check(rc, "rlt_scatter_rows")


def patch_tables(patches: torch.Tensor, count: int, tables: torch.Tensor) -> None:
    """tables.view(-1)[patches[i, 0]] = patches[i, 1] for i < count (rlt_patch_tables).

    patches: contiguous int64 [n, 2] on the tables' device or in pinned host
    memory (read in place); indices distinct.  tables: contiguous int32.
    """
    device = _require_rocm(tables)
    if patches.dtype != torch.int64 or patches.ndim != 2 or patches.shape[1] != 2 or not patches.is_contiguous():
        raise ValueError("patches must be contiguous int64 [n, 2]")
    if patches.device.type == "cpu":
        if not patches.is_pinned():
            raise ValueError("host patches must be pinned")
    elif patches.device != device:
        raise ValueError("patches must be pinned host memory or on the tables' device")
    if tables.dtype != torch.int32 or not tables.is_contiguous():
        raise ValueError("tables must be contiguous int32")
    if not 0 <= count <= patches.shape[0]:
        raise ValueError("count exceeds the patch rows")
    check(
        _native.load().rlt_patch_tables(patches.data_ptr(), count, tables.data_ptr(), tables.numel(), stream_handle(device)),
        "rlt_patch_tables",
    )


def decode_workspace_bytes(n_rows: int, num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """Bytes of split-K partials rlt_paged_decode needs for a batch of n_rows (shape only)."""
    return int(_native.load().rlt_paged_decode_workspace_bytes(n_rows, num_q_heads, num_kv_heads, head_dim))


def static_device_bytes() -> int:
    """Device bytes the library holds per device it has run on (rlt_static_device_bytes)."""
    return int(_native.load().rlt_static_device_bytes())


def prefill_workspace_bytes(
    total_q: int, num_seqs: int, table_width: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
    page_size: int, dtype: torch.dtype,
) -> int:
    """Bytes rlt_paged_prefill needs (0 on the MFMA path: bf16/fp16, head_dim 64/128, page 16)."""
    return int(
        _native.load().rlt_paged_prefill_workspace_bytes(
            total_q, num_seqs, table_width, num_q_heads, num_kv_heads, head_dim, page_size, dtype_code(dtype)
        )
    )


# rlt_paged_decode's split plan: rows are cut into splits of 256 tokens, and
# a row needing more than 64 splits doubles the split length until 64 cover it.
DECODE_SPLIT_TOKENS = 256
DECODE_MAX_SPLITS = 64
# rlt_paged_decode_shared_prefix serves batches of at most this many rows.
DECODE_SHARED_PREFIX_MAX_ROWS = 8192


def decode_split_len(length: int) -> int:
    """Split length rlt_paged_decode uses for a row of `length` tokens."""
    per = DECODE_SPLIT_TOKENS
    while -(-int(length) // per) > DECODE_MAX_SPLITS:
        per <<= 1
    return per


GROUP_FIELDS = 5  # (first member, member count, first page, page count, split length)


@dataclass(frozen=True)
class PrefixGroups:
    """Decode rows grouped by the prefix-cache pages their tables begin with.

    `hint` is the int32 device buffer rlt_paged_decode_shared_prefix reads:
    row_group [n_rows] (-1: none), n_groups records of (first member, member
    count, first page, page count, split length), item_start [n_groups + 1],
    the member rows of every group, then every group's shared page ids.
    """

    hint: torch.Tensor
    n_rows: int
    n_groups: int
    n_members: int
    n_pages: int
    n_items: int
    group_size: int  # q heads per KV head the item counts were sized for (at least the call's)


def prefix_group_layout(row_pages, lengths, page: int, group_size: int):
    """Host int32 hint and its counts (n_groups, n_members, n_pages, n_items, group_size), or None.

    row_pages[r]: the prefix-cache page ids row r's table begins with (empty
    or None: the row reads no shared prefix).  Rows group by those pages cut
    to whole splits of their own split length (decode_split_len of their
    length), and by that split length; rows whose pages cover no whole split
    stay out.  A group's page list is its first member's; rows join a group by
    its first and last page and page count, so building the layout costs
    O(1) per row beyond the group lists (the device compares every page of a
    member's split before it takes it, so a row whose middle pages differ only
    reads its own pages in the split pass).  group_size is the number of q
    heads per KV head (a larger value only adds empty work items; the hint
    serves calls up to it).  Groups appear in first-member order and list
    members in batch order, so the layout is a function of the rows alone.
    """
    n_rows = len(row_pages)
    if len(lengths) != n_rows:
        raise ValueError("one length per row")
    groups: dict = {}  # (first page, last page, pages, split length) -> (group, page list)
    row_group = np.full(n_rows, -1, dtype=np.int32)
    for r, (pages, n) in enumerate(zip(row_pages, lengths)):
        if pages is None or not len(pages) or int(n) <= 0:
            continue
        split = decode_split_len(int(n))
        cut = len(pages) * page // split * split // page
        if cut == 0:
            continue
        key = (int(pages[0]), int(pages[cut - 1]), cut, split)
        entry = groups.get(key)
        if entry is None:
            entry = groups[key] = (len(groups), pages[:cut])
        row_group[r] = entry[0]
    if not groups:
        return None
    members = [[] for _ in groups]
    for r in np.nonzero(row_group >= 0)[0]:
        members[row_group[r]].append(int(r))
    records, item_start, page_lists = [], [0], []
    member0 = page0 = 0
    for (_, _, cut, split), (g, pages) in groups.items():
        count = len(members[g])
        splits = min(cut * page // split, DECODE_MAX_SPLITS - 1)
        records.append((member0, count, page0, cut, split))
        item_start.append(item_start[-1] + splits * (-(-count * group_size // 64)))
        page_lists.append(np.asarray(pages, dtype=np.int32))
        member0 += count
        page0 += cut
    flat_members = [r for m in members for r in m]
    hint = np.concatenate(
        [
            row_group,
            np.asarray(records, dtype=np.int32).reshape(-1),
            np.asarray(item_start, dtype=np.int32),
            np.asarray(flat_members, dtype=np.int32),
            *page_lists,
        ]
    ).astype(np.int32)
    return hint, len(groups), len(flat_members), page0, item_start[-1], int(group_size)


def prefix_groups(row_pages, lengths, page: int, group_size: int, device) -> PrefixGroups | None:
    """The PrefixGroups of a decode batch on `device` (prefix_group_layout), or None."""
    layout = prefix_group_layout(row_pages, lengths, page, group_size)
    if layout is None:
        return None
    hint, *counts = layout
    return PrefixGroups(torch.from_numpy(hint).to(device), len(row_pages), *counts)


def _decode_inputs(q, key_cache, value_cache, block_tables, context_lengths, out):
    """Validated decode geometry: (device, rows, hq, hkv, d, page, num_blocks, out)."""
    device = _require_rocm(q, key_cache, value_cache, block_tables, context_lengths)
    if q.ndim != 3 or key_cache.ndim != 4:
        raise ValueError("q must be [rows, heads, head_dim] and caches [blocks, page, kv_heads, head_dim]")
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must share shape and strides")
    nb, page, hkv, d = key_cache.shape
    rows, hq, qd = q.shape
    if qd != d:
        raise ValueError(f"q head_dim {qd} does not match cache head_dim {d}")
    if hq == 0 or hq % hkv:
        raise ValueError("query heads must be a positive multiple of KV heads")
    if q.dtype != key_cache.dtype or value_cache.dtype != key_cache.dtype:
        raise ValueError("q, key_cache and value_cache must share a dtype")
    if block_tables.dtype != torch.int32 or block_tables.ndim != 2 or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be int32 [rows, width] with contiguous rows")
    if block_tables.shape[0] != rows or context_lengths.shape != (rows,):
        raise ValueError("block_tables and context_lengths must have one entry per row")
    _require_int(context_lengths, torch.int32, "context_lengths")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != device:
        raise ValueError("out must match q")
    return device, rows, hq, hkv, d, page, nb, out


def _decode_workspace(workspace, rows, hq, hkv, d, device):
    need = decode_workspace_bytes(rows, hq, hkv, d)
    if workspace is None:
        return torch.empty(need, dtype=torch.uint8, device=device)
    if workspace.numel() * workspace.element_size() < need or workspace.device != device:
        raise ValueError(f"workspace must hold {need} bytes on {device}")
    return workspace


def _serves(groups: PrefixGroups | None, rows: int, group_size: int) -> bool:
    """Whether a hint applies: batches above the row limit, or with more q heads per
    KV head than its items were sized for, read their prefixes per row (the hint
    is an optimisation only)."""
    return groups is not None and rows <= DECODE_SHARED_PREFIX_MAX_ROWS and group_size <= groups.group_size


def _prefix_call(groups: PrefixGroups, rows: int, block_tables: torch.Tensor):
    """Checked ctypes arguments of a PrefixGroups hint (rlt_paged_decode_shared_prefix)."""
    if not 0 < groups.group_size <= 64:
        raise ValueError("prefix groups need a group size in [1, 64]")
    _require_rocm(groups.hint)
    _require_int(groups.hint, torch.int32, "prefix groups")
    size = rows + (GROUP_FIELDS + 1) * groups.n_groups + 1 + groups.n_members + groups.n_pages
    if groups.n_rows != rows or groups.hint.numel() != size or not groups.hint.is_contiguous():
        raise ValueError(f"prefix groups must be a contiguous int32 hint for {rows} rows")
    if groups.n_pages > groups.n_groups * block_tables.shape[1]:
        raise ValueError("a prefix group is wider than the block tables")
    return [groups.hint.data_ptr(), groups.n_groups, groups.n_members, groups.n_pages, groups.n_items]


def paged_decode_append(
    q: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lengths: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    write_blocks: torch.Tensor,
    write_offsets: torch.Tensor,
    n_write: int | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    scale: float | None = None,
    shared_prefix: PrefixGroups | None = None,
) -> torch.Tensor:
    """KV append of rows [0, n_write) then decode attention, in one launch (rlt_paged_decode_append).

    key_cache / value_cache are layer slices [blocks, page, kv_heads, head_dim]
    and are written.  Same pages and output bits as kv_append followed by
    paged_decode, provided no row reads a slot another row writes (a decode
    batch with one row per request and depth).  With `shared_prefix` the
    groups' prefix pages are read once per launch
    (rlt_paged_decode_shared_prefix with its append arguments).
    """
    device, rows, hq, hkv, d, page, nb, out = _decode_inputs(q, key_cache, value_cache, block_tables, context_lengths, out)
    _require_rocm(q, k_new, v_new, write_blocks, write_offsets)
    n = write_blocks.shape[0] if n_write is None else int(n_write)
    for t, name in ((k_new, "k_new"), (v_new, "v_new")):
        if t.ndim != 3 or t.shape[1:] != (hkv, d) or t.shape[0] < n or t.dtype != key_cache.dtype:
            raise ValueError(f"{name} must be [>= n_write, {hkv}, {d}] {key_cache.dtype}")
    _require_int(write_blocks, torch.int64, "write_blocks")
    _require_int(write_offsets, torch.int64, "write_offsets")
    if not 0 <= n <= min(rows, write_blocks.shape[0], write_offsets.shape[0]):
        raise ValueError("n_write must be in [0, rows] and covered by write_blocks / write_offsets")
    if rows == 0:
        return out
    workspace = _decode_workspace(workspace, rows, hq, hkv, d, device)
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    common = [
        q.data_ptr(), int64_array(q.stride()), key_cache.data_ptr(), value_cache.data_ptr(),
        int64_array(key_cache.stride()), block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
        context_lengths.data_ptr(), out.data_ptr(), int64_array(out.stride()), rows, hq, hkv, d, page, nb, scale,
        dtype_code(q.dtype), k_new.data_ptr(), int64_array(k_new.stride()), v_new.data_ptr(),
        int64_array(v_new.stride()), write_blocks.data_ptr(), write_offsets.data_ptr(), n,
    ]
    tail = [workspace.data_ptr(), workspace.numel() * workspace.element_size(), stream_handle(device)]
    if _serves(shared_prefix, rows, hq // hkv):
        rc = _native.load().rlt_paged_decode_shared_prefix(
            *common, *_prefix_call(shared_prefix, rows, block_tables), *tail
        )
        check(rc, "rlt_paged_decode_shared_prefix")
        return out
    rc = _native.load().rlt_paged_decode_append(*common, *tail)
    check(rc, "rlt_paged_decode_append")
    return out


def paged_decode(
    q: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lengths: torch.Tensor,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    scale: float | None = None,
    shared_prefix: PrefixGroups | None = None,
) -> torch.Tensor:
    """Paged decode attention over layer-slice caches [blocks, page, kv_heads, head_dim].

    Same contract as torch_paged_attention (vllm_rlt/kernels/paged_attention.py:12-36):
    returns a new tensor like q unless out is given.  With `shared_prefix` each
    group's prefix pages are read once for all its rows
    (rlt_paged_decode_shared_prefix); the result is the same attention.
    """
    device, rows, hq, hkv, d, page, nb, out = _decode_inputs(q, key_cache, value_cache, block_tables, context_lengths, out)
    if rows == 0:
        return out
    workspace = _decode_workspace(workspace, rows, hq, hkv, d, device)
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    if _serves(shared_prefix, rows, hq // hkv):
        rc = _native.load().rlt_paged_decode_shared_prefix(
            q.data_ptr(), int64_array(q.stride()), key_cache.data_ptr(), value_cache.data_ptr(),
            int64_array(key_cache.stride()), block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
            context_lengths.data_ptr(), out.data_ptr(), int64_array(out.stride()), rows, hq, hkv, d, page, nb, scale,
            dtype_code(q.dtype), None, None, None, None, None, None, 0,
            *_prefix_call(shared_prefix, rows, block_tables),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), stream_handle(device),
        )
        check(rc, "rlt_paged_decode_shared_prefix")
        return out
    rc = _native.load().rlt_paged_decode(
        q.data_ptr(),
        int64_array(q.stride()),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int64_array(key_cache.stride()),
        block_tables.data_ptr(),
        block_tables.stride(0),
        block_tables.shape[1],
        context_lengths.data_ptr(),
        out.data_ptr(),
        int64_array(out.stride()),
        rows,
        hq,
        hkv,
        d,
        page,
        nb,
        scale,
        dtype_code(q.dtype),
        workspace.data_ptr(),
        workspace.numel() * workspace.element_size(),
        stream_handle(device),
    )
    check(rc, "rlt_paged_decode")
    return out


def _rows_aligned16(t: torch.Tensor) -> bool:
    """Innermost dim contiguous and every row start 16-byte aligned."""
    size = t.element_size()
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((st * size) % 16 == 0 for st in t.stride()[:-1])


def rows_aligned16(*tensors: torch.Tensor) -> bool:
    """Whether every tensor's rows are 16-byte aligned (the prefill MFMA path's requirement)."""
    return all(_rows_aligned16(t) for t in tensors)


def paged_prefill(
    q: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lengths: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    max_seqlen_q: int,
    out: torch.Tensor | None = None,
    scale: float | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Packed bottom-right-causal prefill (FlashPagedAttention.prefill, flash_attention.py:66-96).

    The MFMA path needs no workspace; other shapes (fp32, unaligned rows,
    other head sizes) run each query row as a decode row and need
    prefill_workspace_bytes(...) bytes, allocated here unless `workspace`
    (a uint8 device tensor at least that large) is given.
    """
    device = _require_rocm(q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q)
    if q.ndim != 3 or key_cache.ndim != 4:
        raise ValueError("q must be [tokens, heads, head_dim] and caches [blocks, page, kv_heads, head_dim]")
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must share shape and strides")
    nb, page, hkv, d = key_cache.shape
    total, hq, qd = q.shape
    if qd != d or hq == 0 or hq % hkv:
        raise ValueError("q must have head_dim matching the cache and a positive multiple of KV heads")
    if q.dtype != key_cache.dtype:
        raise ValueError("q and the caches must share a dtype")
    if block_tables.dtype != torch.int32 or block_tables.ndim != 2 or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be int32 [sequences, width] with contiguous rows")
    _require_int(context_lengths, torch.int32, "context_lengths")
    _require_int(cu_seqlens_q, torch.int32, "cu_seqlens_q")
    nseq = block_tables.shape[0]
    if context_lengths.shape != (nseq,) or cu_seqlens_q.shape != (nseq + 1,):
        raise ValueError("context_lengths and cu_seqlens_q must describe one entry per sequence")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != device:
        raise ValueError("out must match q")
    if total == 0 or nseq == 0:
        return out
    width = block_tables.shape[1]
    lib = _native.load()
    code = dtype_code(q.dtype)
    if not all(_rows_aligned16(t) for t in (q, out, key_cache, value_cache)):
        code = _native.RLT_FLOAT32  # the MFMA path needs 16-byte rows; size the per-token fallback
    need = int(lib.rlt_paged_prefill_workspace_bytes(total, nseq, width, hq, hkv, d, page, code))
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    elif workspace.numel() * workspace.element_size() < need or workspace.device != device:
        raise ValueError(f"workspace must hold {need} bytes on {device}")
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    rc = lib.rlt_paged_prefill(
        q.data_ptr(),
        int64_array(q.stride()),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int64_array(key_cache.stride()),
        block_tables.data_ptr(),
        block_tables.stride(0),
        width,
        context_lengths.data_ptr(),
        cu_seqlens_q.data_ptr(),
        nseq,
        total,
        max_seqlen_q,
        out.data_ptr(),
        int64_array(out.stride()),
        hq,
        hkv,
        d,
        page,
        nb,
        scale,
        dtype_code(q.dtype),
        workspace.data_ptr(),
        workspace.numel() * workspace.element_size(),
        stream_handle(device),
    )
    check(rc, "rlt_paged_prefill")
    return out


def _pool_dims(key_cache: torch.Tensor, value_cache: torch.Tensor):
    if key_cache.ndim != 5 or key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError("caches must be matching [blocks, layers, page, kv_heads, head_dim] tensors")
    return key_cache.shape


def kv_copy_token(
    key_cache: torch.Tensor, value_cache: torch.Tensor, src_block: int, dst_blocks, offset: int
) -> None:
    """cache[dst, :, offset] = cache[src_block, :, offset] for every dst (all layers, K and V).

    Mirrors the exit copies of finalize_token, vllm_rlt/core/kv_cache_manager.py:601-611.
    """
    device = _require_rocm(key_cache, value_cache)
    nb, nl, page, hkv, d = _pool_dims(key_cache, value_cache)
    dst = list(dst_blocks)
    rc = _native.load().rlt_kv_copy_token(
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int64_array(key_cache.stride()),
        src_block,
        int64_array(dst or [0]),
        len(dst),
        offset,
        nl,
        nb,
        page,
        hkv,
        d,
        dtype_code(key_cache.dtype),
        stream_handle(device),
    )
    check(rc, "rlt_kv_copy_token")


def kv_finalize(
    descriptors: torch.Tensor,
    tables: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    max_loops: int,
    count: int | None = None,
) -> None:
    """Batched LAST-EXITED exit copies (finalize_kernel, vllm_rlt/kernels/routing.py:80-109).

    descriptors: int64 [n, 3] of (slot, exit depth, position), device or pinned host.
    tables: int32 [slots, planes, width] device-resident page tables.
    """
    device = _require_rocm(key_cache, value_cache, tables)
    nb, nl, page, hkv, d = _pool_dims(key_cache, value_cache)
    if descriptors.dtype != torch.int64 or descriptors.ndim != 2 or descriptors.shape[1] != 3:
        raise ValueError("descriptors must be int64 [n, 3]")
    if not descriptors.is_contiguous():
        raise ValueError("descriptors must be contiguous")
    if descriptors.device.type == "cpu" and not descriptors.is_pinned():
        raise ValueError("host descriptors must be pinned")
    if tables.dtype != torch.int32 or tables.ndim != 3 or not tables.is_contiguous():
        raise ValueError("tables must be contiguous int32 [slots, planes, width]")
    n = descriptors.shape[0] if count is None else count
    rc = _native.load().rlt_kv_finalize(
        descriptors.data_ptr(),
        n,
        tables.data_ptr(),
        tables.shape[2],
        tables.shape[1],
        tables.shape[0],
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int64_array(key_cache.stride()),
        nl,
        nb,
        hkv,
        d,
        page,
        max_loops,
        dtype_code(key_cache.dtype),
        stream_handle(device),
    )
    check(rc, "rlt_kv_finalize")


def kv_gather(
    key_cache: torch.Tensor, value_cache: torch.Tensor, layer: int, table: torch.Tensor, length: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """Ordered [length, kv_heads, head_dim] K and V of one table (read(), kv_cache_manager.py:616-637)."""
    device = _require_rocm(key_cache, value_cache, table)
    nb, nl, page, hkv, d = _pool_dims(key_cache, value_cache)
    _require_int(table, torch.int32, "table")
    if length < 0 or (length + page - 1) // page > table.numel():
        raise ValueError("length exceeds the table")
    out_k = torch.empty((length, hkv, d), dtype=key_cache.dtype, device=device)
    out_v = torch.empty_like(out_k)
    if length == 0:
        return out_k, out_v
    rc = _native.load().rlt_kv_gather(
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int64_array(key_cache.stride()),
        layer,
        table.data_ptr(),
        length,
        out_k.data_ptr(),
        out_v.data_ptr(),
        nl,
        nb,
        page,
        hkv,
        d,
        dtype_code(key_cache.dtype),
        stream_handle(device),
    )
    check(rc, "rlt_kv_gather")
    return out_k, out_v


def build_decode_metadata(
    descriptors: torch.Tensor,
    count: int,
    size: int,
    tables: torch.Tensor,
    page_size: int,
    slots: torch.Tensor,
    positions: torch.Tensor,
    lengths: torch.Tensor,
    blocks: torch.Tensor,
    offsets: torch.Tensor,
    out_tables: torch.Tensor,
    out_width: int,
) -> None:
    """Per-row routing metadata on the device (metadata_kernel, vllm_rlt/kernels/routing.py:8-41)."""
    device = _require_rocm(tables, slots, positions, lengths, blocks, offsets, out_tables)
    if tables.dtype != torch.int32 or tables.ndim != 3 or not tables.is_contiguous():
        raise ValueError("tables must be contiguous int32 [slots, planes, width]")
    if descriptors.dtype != torch.int64 or descriptors.ndim != 2 or descriptors.shape[1] != 3:
        raise ValueError("descriptors must be int64 [n, 3]")
    if descriptors.device.type == "cpu" and not descriptors.is_pinned():
        raise ValueError("host descriptors must be pinned")
    if out_tables.dtype != torch.int32 or out_tables.ndim != 2 or out_tables.stride(1) != 1:
        raise ValueError("out_tables must be int32 [rows, width] with contiguous rows")
    for t, dt, name in (
        (slots, torch.int64, "slots"),
        (positions, torch.int64, "positions"),
        (lengths, torch.int32, "lengths"),
        (blocks, torch.int64, "blocks"),
        (offsets, torch.int64, "offsets"),
    ):
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous {dt}")
    if min(slots.numel(), positions.numel(), lengths.numel(), out_tables.shape[0]) < size:
        raise ValueError("output buffers are smaller than size")
    if min(blocks.numel(), offsets.numel(), descriptors.shape[0]) < count:
        raise ValueError("descriptor/address buffers are smaller than count")
    rc = _native.load().rlt_build_decode_metadata(
        descriptors.data_ptr(),
        count,
        size,
        tables.data_ptr(),
        tables.shape[0],
        tables.shape[2],
        tables.shape[1],
        page_size,
        slots.data_ptr(),
        positions.data_ptr(),
        lengths.data_ptr(),
        blocks.data_ptr(),
        offsets.data_ptr(),
        out_tables.data_ptr(),
        out_tables.stride(0),
        out_width,
        stream_handle(device),
    )
    check(rc, "rlt_build_decode_metadata")


def stage_prefill(source: torch.Tensor, target: torch.Tensor, target32: torch.Tensor, n: int) -> None:
    """Copy n int64 values to int64 and int32 device buffers (stage_prefill, prefill_metadata.py:8-12)."""
    device = _require_rocm(target, target32)
    if source.dtype != torch.int64 or target.dtype != torch.int64 or target32.dtype != torch.int32:
        raise ValueError("stage_prefill expects int64 source/target and int32 target32")
    if source.device.type == "cpu" and not source.is_pinned():
        raise ValueError("host source must be pinned")
    if min(source.numel(), target.numel(), target32.numel()) < n:
        raise ValueError("buffers are smaller than n")
    check(
        _native.load().rlt_stage_prefill(
            source.data_ptr(), target.data_ptr(), target32.data_ptr(), n, stream_handle(device)
        ),
        "rlt_stage_prefill",
    )


def expand_prefill(
    positions: torch.Tensor,
    sequences: torch.Tensor,
    tables: torch.Tensor,
    page_size: int,
    blocks: torch.Tensor,
    offsets: torch.Tensor,
    n: int,
) -> None:
    """Per-token write addresses of a packed prefill (expand_prefill, prefill_metadata.py:16-32)."""
    device = _require_rocm(positions, sequences, tables, blocks, offsets)
    if tables.dtype != torch.int32 or tables.ndim != 2 or not tables.is_contiguous():
        raise ValueError("tables must be contiguous int32 [sequences, width]")
    for t, name in ((positions, "positions"), (sequences, "sequences"), (blocks, "blocks"), (offsets, "offsets")):
        if t.dtype != torch.int64 or t.numel() < n:
            raise ValueError(f"{name} must be int64 with at least n entries")
    check(
        _native.load().rlt_expand_prefill(
            positions.data_ptr(),
            sequences.data_ptr(),
            tables.data_ptr(),
            tables.shape[0],
            tables.shape[1],
            page_size,
            blocks.data_ptr(),
            offsets.data_ptr(),
            n,
            stream_handle(device),
        ),
        "rlt_expand_prefill",
    )
