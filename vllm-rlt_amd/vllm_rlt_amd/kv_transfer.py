"""Page export / import: preemption snapshots and the prefill-to-decode segment format.

The byte-range format is the reference's (vllm_rlt/pd/transport.py:18-68): a
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
from itertools import zip_longest

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


def kv_segments(info: dict, tables, start: int, end: int):
    """(address, bytes, device) ranges holding tokens [start, end) of every table (depth).

    A fully valid page is one segment (all layers); a partial page is one
    segment per layer covering only its valid tokens, so unused tail bytes are
    never sent (vllm_rlt/pd/transport.py:18-46).
    """
    page = info["block_size"]
    if not 0 <= start < end:
        raise ValueError("invalid KV range")
    for table in tables:
        if end > len(table) * page:
            raise ValueError("KV range exceeds allocation")
        for logical in range(start // page, (end - 1) // page + 1):
            block = table[logical]
            if not 0 <= block < info["num_blocks"]:
                raise ValueError("physical block outside registered pool")
            lo = max(start - logical * page, 0)
            hi = min(end - logical * page, page)
            for base in (info["key_ptr"], info["value_ptr"]):
                address = base + block * info["block_bytes"]
                if lo == 0 and hi == page:
                    yield (address, info["block_bytes"], info["device"])
                else:
                    for layer in range(info["num_layers"]):
                        yield (
                            address + layer * info["layer_bytes"] + lo * info["token_bytes"],
                            (hi - lo) * info["token_bytes"],
                            info["device"],
                        )


def partition_segments(source, target, byte_limit: int, descriptor_limit: int):
    """Pair source and target segments into transfers of at most byte_limit bytes and
    descriptor_limit descriptors, splitting segments where needed (vllm_rlt/pd/transport.py:49-68)."""
    local, remote, size = [], [], 0
    for src, dst in zip_longest(source, target):
        if src is None or dst is None or src[1] != dst[1]:
            raise ValueError("incompatible source/target KV geometry")
        offset = 0
        while offset < src[1]:
            amount = min(src[1] - offset, byte_limit - size)
            local.append((src[0] + offset, amount, src[2]))
            remote.append((dst[0] + offset, amount, dst[2]))
            size += amount
            offset += amount
            if size == byte_limit or len(local) == descriptor_limit:
                yield local, remote, size
                local, remote, size = [], [], 0
    if local:
        yield local, remote, size


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
