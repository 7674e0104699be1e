"""Page export / import: preemption snapshots and the prefill-to-decode segment format.

The byte-range format is the reference's (vllm_rlt/pd/transport.py:18-68),
because a decode-side peer pairs its segments with ours one by one: a
request's valid token range [start, end) becomes one segment per whole page
(all layers, one contiguous block) and one per layer for a partially valid
page, for K and V and every storage depth; partition_segments bounds each
transfer by bytes and descriptor count.  The transport that moves segments
between processes (NIXL in the reference) is outside this package; here a
batch of segments the device can address (same device, or pinned host memory)
is executed by one rlt_copy_segments launch.

Preemption (vllm_rlt/engine/preemption.py:68-138) moves whole pages between
the pool and host memory.  The reference copies one page at a time into
pageable memory; here one rlt_kv_export_pages launch writes every page of the
request straight into pinned host memory (no device temporary on a full GPU),
and rlt_kv_import_pages restores them.
"""

from __future__ import annotations

from copy import deepcopy

import torch

from . import _native
from ._native import check, stream_handle


def transfer_info(cache, hidden: torch.Tensor | None = None) -> dict:
    """Pool geometry in bytes, as NixlConnector advertises it (vllm_rlt/pd/transport.py:80-97)."""
    k = cache.key_cache
    element = k.element_size()
    info = dict(
        key_ptr=k.data_ptr(),
        value_ptr=cache.value_cache.data_ptr(),
        device=k.device.index,
        num_blocks=cache.num_blocks,
        block_size=cache.block_size,
        num_layers=cache.num_layers,
        depths=cache.storage_depths,
        block_bytes=k.stride(0) * element,
        layer_bytes=k.stride(1) * element,
        token_bytes=k.stride(2) * element,
    )
    if hidden is not None:
        info["hidden_ptr"] = hidden.data_ptr()
        info["hidden_bytes"] = hidden.stride(0) * hidden.element_size()
    return info


def _page_pieces(info: dict, lo: int, hi: int) -> list[tuple[int, int]]:
    """(offset inside one page's block, bytes) pieces that hold tokens [lo, hi) of the page.

    All tokens valid: the whole block (every layer) is one piece.  Otherwise
    each layer's slice of the page holds the tokens at the same place, so the
    page contributes one piece per layer, in layer order.
    """
    if hi - lo == info["block_size"]:
        return [(0, info["block_bytes"])]
    first, size = lo * info["token_bytes"], (hi - lo) * info["token_bytes"]
    stride = info["layer_bytes"]
    return [(first + layer * stride, size) for layer in range(info["num_layers"])]


def kv_segments(info: dict, tables, start: int, end: int) -> list[tuple[int, int, int]]:
    """(address, bytes, device) ranges that hold tokens [start, end) of every table.

    The order is part of the format, since a peer pairs its own segments with
    these one by one (vllm_rlt/pd/transport.py:18-46, paired at
    vllm_rlt/pd/worker.py:214-229): tables (storage depths) in order; within a
    table, pages in logical order; within a page, the key pool's pieces, then
    the value pool's.  A page whose tokens are all in the range is a single
    segment of its whole block; a partially covered page gives one segment per
    layer, so bytes of tokens outside the range are never sent.  Every table
    is checked before any segment is returned, with the reference's messages.
    """
    page = info["block_size"]
    if not 0 <= start < end:
        raise ValueError("invalid KV range")
    first_page, last_page = start // page, (end - 1) // page
    # The valid token window of each touched page, relative to that page.
    windows = [
        (logical, max(start, logical * page) - logical * page, min(end, (logical + 1) * page) - logical * page)
        for logical in range(first_page, last_page + 1)
    ]
    pieces = [_page_pieces(info, lo, hi) for _, lo, hi in windows]
    bases = (info["key_ptr"], info["value_ptr"])
    device, block_bytes, num_blocks = info["device"], info["block_bytes"], info["num_blocks"]
    out = []
    for table in tables:
        if len(table) * page < end:
            raise ValueError("KV range exceeds allocation")
        blocks = [table[logical] for logical, _, _ in windows]
        if any(not 0 <= b < num_blocks for b in blocks):
            raise ValueError("physical block outside registered pool")
        for block, page_pieces in zip(blocks, pieces):
            out.extend(
                (base + block * block_bytes + offset, size, device)
                for base in bases
                for offset, size in page_pieces
            )
    return out


def partition_segments(source, target, byte_limit: int, descriptor_limit: int):
    """Cut paired source/target segments into transfers (vllm_rlt/pd/transport.py:49-68).

    Returns a list of (source pieces, target pieces, bytes).  The pairs are
    laid end to end as one byte stream and cut greedily: a transfer closes as
    soon as it holds byte_limit bytes or descriptor_limit pieces, and a
    segment that straddles a cut continues, at the same offset on both sides,
    in the next transfer.  Zero-byte segments produce no piece.  Each pair must
    have equal sizes ("incompatible source/target KV geometry" otherwise,
    checked for every pair before anything is returned).
    """
    source, target = list(source), list(target)
    if len(source) != len(target) or any(s[1] != t[1] for s, t in zip(source, target)):
        raise ValueError("incompatible source/target KV geometry")
    if byte_limit <= 0 or descriptor_limit <= 0:
        raise ValueError("transfer limits must be positive")
    transfers = []
    pending_src, pending_dst, room = [], [], byte_limit
    for (s_addr, size, s_dev), (t_addr, _, t_dev) in zip(source, target):
        offset = 0
        while offset < size:
            take = min(size - offset, room)
            pending_src.append((s_addr + offset, take, s_dev))
            pending_dst.append((t_addr + offset, take, t_dev))
            offset += take
            room -= take
            if room == 0 or len(pending_src) == descriptor_limit:
                transfers.append((pending_src, pending_dst, byte_limit - room))
                pending_src, pending_dst, room = [], [], byte_limit
    if pending_src:
        transfers.append((pending_src, pending_dst, byte_limit - room))
    return transfers


def _inside(address: int, size: int, regions) -> bool:
    for t in regions:
        lo = t.data_ptr()
        if lo <= address and address + size <= lo + t.numel() * t.element_size():
            return True
    return False


def copy_segments(source, target, regions, device: torch.device | str = "cuda") -> int:
    """Execute paired (address, bytes, device) segments with one launch; returns bytes copied.

    Every source and target range must lie inside one of `regions` (the
    tensors the addresses were taken from), which is checked before launch.
    """
    device = torch.device(device)
    source, target = list(source), list(target)
    if len(source) != len(target):
        raise ValueError("incompatible source/target KV geometry")
    for (sa, sn, _), (ta, tn, _) in zip(source, target):
        if sn != tn or sn < 0:
            raise ValueError("incompatible source/target KV geometry")
        if not _inside(sa, sn, regions) or not _inside(ta, tn, regions):
            raise ValueError("segment outside the registered tensors")
    if not source:
        return 0
    table = torch.tensor([[s[0] for s in source], [t[0] for t in target], [s[1] for s in source]], dtype=torch.int64)
    table = table.pin_memory().to(device, non_blocking=True)
    total, largest = sum(s[1] for s in source), max(s[1] for s in source)
    rc = _native.load().rlt_copy_segments(
        table[0].data_ptr(), table[1].data_ptr(), table[2].data_ptr(), len(source), largest, stream_handle(device)
    )
    check(rc, "rlt_copy_segments")
    return total


def _page_bytes(cache) -> int:
    k = cache.key_cache
    return k.stride(0) * k.element_size()


def export_pages(cache, blocks, keys: torch.Tensor | None = None, values: torch.Tensor | None = None):
    """keys[i] = key_cache[blocks[i]], values[i] = value_cache[blocks[i]] (whole pages, bitwise).

    Destinations default to new pinned host tensors [n, *page_shape]; device
    tensors of that shape work too.  The copy is enqueued on the current stream.
    """
    k = cache.key_cache
    n = len(blocks)
    if any(not 0 <= b < cache.num_blocks for b in blocks):
        raise ValueError("physical block outside the pool")
    shape = (n, *k.shape[1:])
    if keys is None:
        keys = torch.empty(shape, dtype=k.dtype, pin_memory=True)
    if values is None:
        values = torch.empty(shape, dtype=k.dtype, pin_memory=True)
    _check_rows(cache, keys, values, n)
    ids = torch.tensor(list(blocks), dtype=torch.int64).pin_memory().to(k.device, non_blocking=True)
    rc = _native.load().rlt_kv_export_pages(
        k.data_ptr(), cache.value_cache.data_ptr(), _page_bytes(cache), _page_bytes(cache), cache.num_blocks,
        ids.data_ptr(), n, keys.data_ptr(), values.data_ptr(), _page_bytes(cache),
        stream_handle(k.device),
    )
    check(rc, "rlt_kv_export_pages")
    return keys, values


def import_pages(cache, blocks, keys: torch.Tensor, values: torch.Tensor) -> None:
    """key_cache[blocks[i]] = keys[i], value_cache[blocks[i]] = values[i] (whole pages, bitwise)."""
    k = cache.key_cache
    n = len(blocks)
    if any(not 0 <= b < cache.num_blocks for b in blocks):
        raise ValueError("physical block outside the pool")
    _check_rows(cache, keys, values, n)
    ids = torch.tensor(list(blocks), dtype=torch.int64).pin_memory().to(k.device, non_blocking=True)
    rc = _native.load().rlt_kv_import_pages(
        k.data_ptr(), cache.value_cache.data_ptr(), _page_bytes(cache), _page_bytes(cache), cache.num_blocks,
        ids.data_ptr(), n, keys.data_ptr(), values.data_ptr(), _page_bytes(cache),
        stream_handle(k.device),
    )
    check(rc, "rlt_kv_import_pages")


def _check_rows(cache, keys, values, n):
    k = cache.key_cache
    if not (k.is_contiguous() and cache.value_cache.is_contiguous()):
        raise ValueError("page export needs contiguous pools")
    for t, name in ((keys, "keys"), (values, "values")):
        if t.shape != (n, *k.shape[1:]) or t.dtype != k.dtype or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous {k.dtype} [{n}, {', '.join(map(str, k.shape[1:]))}]")
        if t.device.type == "cpu" and not t.is_pinned():
            raise ValueError(f"host {name} must be pinned")
        if t.device.type != "cpu" and t.device != k.device:
            raise ValueError(f"{name} must live on {k.device} or in pinned host memory")


def snapshot_request(cache, request_id: str, hidden: torch.Tensor | None = None, token: torch.Tensor | None = None):
    """The page and bookkeeping part of PreemptionManager.preempt (vllm_rlt/engine/preemption.py:74-99).

    Copies every page of the request (all planes) to pinned host memory with
    one launch, waits for it, and returns the snapshot; the caller then frees
    the request's pages.
    """
    allocation = cache._get_allocation(request_id)
    blocks = [b for table in allocation.block_tables for b in table]
    if any(not 0 <= b < cache.num_blocks for b in blocks):
        raise ValueError("physical block outside the pool")
    keys, values = export_pages(cache, blocks)
    torch.cuda.current_stream(cache.device).synchronize()
    return dict(
        maximum=allocation.max_tokens,
        pages=len(allocation.block_tables[0]),
        written=deepcopy(allocation.written),
        keys=keys,
        values=values,
        hidden=None if hidden is None else hidden.cpu().clone(),
        token=None if token is None else token.cpu().clone(),
    )


def restore_request(cache, request_id: str, snapshot: dict) -> bool:
    """The page part of PreemptionManager.resume (vllm_rlt/engine/preemption.py:113-138).

    False if the pool cannot take the request back; otherwise its pages are
    allocated afresh, refilled from the snapshot and its written positions
    restored.
    """
    frontier = min(snapshot["maximum"], snapshot["pages"] * cache.block_size)
    if not cache.allocate(request_id, snapshot["maximum"], initial_tokens=frontier):
        return False
    allocation = cache._get_allocation(request_id)
    blocks = [b for table in allocation.block_tables for b in table]
    import_pages(cache, blocks, snapshot["keys"], snapshot["values"])
    allocation.written = snapshot["written"]
    torch.cuda.current_stream(cache.device).synchronize()
    return True
