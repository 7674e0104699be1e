"""Host bookkeeping of the paged KV pool: pages, depth planes, prefix sharing.

KVPageBook is everything the KV cache manager decides on the host -- which
physical page holds which (request, depth plane, logical page), which
positions of which layer are initialised, which full prompt pages are shared
through the prefix cache -- with no device tensors.  KVCacheManager adds the
pool and the HIP data path on top of it.

Semantics restated from vllm_rlt/core/kv_cache_manager.py (line numbers cited
per method).  Depth indices are 0-based; LAST-EXITED keeps one storage plane
per loop depth, SHARED a single plane every depth writes.
"""

from __future__ import annotations

import hashlib
from collections import OrderedDict
from collections.abc import Sequence
from dataclasses import dataclass, field
from numbers import Integral
from typing import Any

import numpy as np
import torch

LAYOUTS = ("last_exited", "shared")


def _is_index(value) -> bool:
    return isinstance(value, Integral) and not isinstance(value, bool)


@dataclass
class WrittenPrefix:
    """Positions of one (plane, layer) that hold valid KV (kv_cache_manager.py:22-41).

    `prefix` is the length of the contiguous written run starting at 0;
    positions written ahead of it wait in `pending` until the gap closes.
    """

    prefix: int = 0
    pending: set = field(default_factory=set)

    def add(self, position: int) -> None:
        if position < self.prefix:
            return
        if position != self.prefix:
            self.pending.add(position)
            return
        frontier = position + 1
        while frontier in self.pending:
            self.pending.discard(frontier)
            frontier += 1
        self.prefix = frontier

    def __contains__(self, position: int) -> bool:
        return position < self.prefix or position in self.pending


@dataclass
class Allocation:
    """One request's pages: block_tables[plane][logical page] (kv_cache_manager.py:44-50)."""

    max_tokens: int
    block_tables: tuple
    written: list
    transfer_leases: set = field(default_factory=set)
    release_requested: bool = False
    # Leading pages of every plane taken from the prefix cache at admission
    # (shared read-only with other requests; fixed for the request's life).
    prefix_pages: int = 0


@dataclass(frozen=True, eq=False)
class PreparedKVBatch:
    """Per-traversal metadata, borrowed by every layer (kv_cache_manager.py:53-71).

    rows: (allocation, depth, position) per row.  position_ids, write_blocks,
    write_offsets: int64 [rows].  block_tables: int32 [rows or sequences, W],
    padded with -1.  context_lengths: int32, position + 1 of each table row.
    cu_seqlens_q / max_seqlen_q describe packed prefill sequences.
    """

    owner: Any
    rows: tuple
    allocations: tuple
    position_ids: torch.Tensor
    write_blocks: torch.Tensor
    write_offsets: torch.Tensor
    block_tables: torch.Tensor
    context_lengths: torch.Tensor
    writable: bool
    cu_seqlens_q: torch.Tensor | None = None
    max_seqlen_q: int = 1
    # Rows grouped by the prefix-cache pages they read, when the manager shares
    # those reads (an ops.PrefixGroups; no counterpart in the reference's batch).
    shared_prefix: Any = None


@dataclass
class BatchPlan:
    """Host arrays of a prepared batch before they are placed on the device."""

    rows: tuple
    allocations: tuple
    positions: np.ndarray  # int64 [n]
    write_blocks: np.ndarray  # int64 [n]
    write_offsets: np.ndarray  # int64 [n]
    tables: np.ndarray  # int32 [t, W]
    lengths: np.ndarray  # int32 [t]
    cu_seqlens: np.ndarray | None  # int32 [s + 1]
    max_seqlen_q: int
    writable: bool


class _PagePool:
    """Physical pages with reference counts; unreferenced pages wait on a LIFO stack.

    The stack starts as [n-1, ..., 1, 0], so the first pages handed out are
    0, 1, 2, ... (kv_cache_manager.py:137, :142).  A page is held once per
    request table that lists it and once per prefix-index entry that names it.
    """

    __slots__ = ("free", "refs")

    def __init__(self, count: int):
        self.free = list(range(count - 1, -1, -1))
        self.refs = [0] * count

    def retain(self, pages) -> None:
        refs = self.refs
        for b in pages:
            refs[b] += 1

    def release(self, pages) -> None:
        """Drop one hold per page, in the order given; a page left unheld is pushed (:175-180)."""
        refs, free = self.refs, self.free
        for b in pages:
            refs[b] -= 1
            if refs[b] == 0:
                free.append(b)
            elif refs[b] < 0:
                raise AssertionError(f"page {b} released more often than held")

    def take(self, count: int) -> list:
        """The top `count` pages of the stack, top first, each now held once."""
        if not 0 <= count <= len(self.free):
            raise AssertionError(f"cannot take {count} of {len(self.free)} free pages")
        cut = len(self.free) - count
        pages = self.free[cut:][::-1]
        del self.free[cut:]
        for b in pages:
            if self.refs[b]:
                raise AssertionError(f"free page {b} is still held")
            self.refs[b] = 1
        return pages


class _PrefixIndex:
    """Cached full prompt pages, least recently used first (kv_cache_manager.py:194-251).

    A key names a whole token prefix up to the end of one page: the sha256 of
    the previous page's key followed by the page's tokens as little-endian
    int64, starting from the empty key.  A value holds the page's physical id
    in every storage plane.  The index keeps one pool hold on each of them.
    """

    __slots__ = ("page", "entries")

    def __init__(self, page_tokens: int):
        self.page = page_tokens
        self.entries: OrderedDict = OrderedDict()

    def keys(self, tokens):
        """Keys of the full pages of `tokens`, computed lazily in page order."""
        step = self.page
        whole = len(tokens) - len(tokens) % step
        if not whole:
            return
        data = memoryview(np.asarray(tokens[:whole], dtype="<i8").tobytes())
        key = b""
        for start in range(0, whole * 8, step * 8):
            h = hashlib.sha256(key)
            h.update(data[start : start + step * 8])
            key = h.digest()
            yield key

    def match(self, tokens) -> tuple:
        """The cached pages of the longest indexed run of `tokens`' full pages, marked recently used."""
        run = []
        for key in self.keys(tokens):
            pages = self.entries.get(key)
            if pages is None:
                break
            self.entries.move_to_end(key)
            run.append(pages)
        return tuple(run)

    def add_run(self, tokens, tables, pool: _PagePool) -> None:
        """Index every full page of `tokens` not indexed yet; page i is (table[i] for each plane)."""
        for index, key in enumerate(self.keys(tokens)):
            if key not in self.entries:
                pages = tuple(table[index] for table in tables)
                pool.retain(pages)
                self.entries[key] = pages

    def evict_oldest(self):
        """Remove the least recently used entry and return its pages (None when empty)."""
        if not self.entries:
            return None
        return self.entries.popitem(last=False)[1]

    def reclaimable(self, pool: _PagePool) -> int:
        """Indexed pages no request holds (the index's hold is their last)."""
        return sum(1 for pages in self.entries.values() for b in pages if pool.refs[b] == 1)


@dataclass
class _DeferredPublish:
    """A publication waiting for the device writes behind `event` (kv_cache_manager.py:201-209)."""

    request_id: str
    allocation: Allocation
    tokens: tuple
    length: int
    event: Any


def _widen(tables: tuple, fresh: list, per_plane: int) -> tuple:
    """Plane d's table followed by fresh[d * per_plane:(d + 1) * per_plane]."""
    return tuple(table + tuple(fresh[d * per_plane : (d + 1) * per_plane]) for d, table in enumerate(tables))


class KVPageBook:
    """Page allocator, prefix cache and per-position validity of a paged KV pool."""

    def __init__(
        self,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        num_blocks: int,
        block_size: int,
        max_loops: int,
        layout: str = "last_exited",
        enable_prefix_caching: bool = False,
        incremental_allocation: bool = False,
        watermark_ratio: float = 0.0,
    ):
        # kv_cache_manager.py:98-108, 113-116, 137-147
        for name, value in (
            ("num_layers", num_layers),
            ("num_kv_heads", num_kv_heads),
            ("head_dim", head_dim),
            ("num_blocks", num_blocks),
            ("block_size", block_size),
            ("max_loops", max_loops),
        ):
            if not _is_index(value) or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
            setattr(self, name, int(value))
        if layout not in LAYOUTS:
            raise ValueError("unsupported KV layout")
        self.layout = layout
        self.storage_depths = self.max_loops if layout == "last_exited" else 1
        if enable_prefix_caching and layout != "last_exited":
            raise ValueError("prefix caching requires last_exited KV")
        self.enable_prefix_caching = enable_prefix_caching
        self.incremental_allocation = incremental_allocation
        self.watermark_blocks = int(watermark_ratio * self.num_blocks)
        self._pool = _PagePool(self.num_blocks)
        self._index = _PrefixIndex(self.block_size)
        self._deferred: list = []
        self._allocations: dict[str, Allocation] = {}
        self.prefix_hits = self.prefix_queries = 0

    # ------------------------------------------------------------------ pool
    # The page holds, free stack and prefix entries under the names the
    # reference's scheduler and tests read (scheduler.py:207, test_cdb_runtime.py:176).
    @property
    def _refs(self) -> list:
        return self._pool.refs

    @property
    def _free_blocks(self) -> list:
        return self._pool.free

    @property
    def _prefixes(self) -> OrderedDict:
        return self._index.entries

    @property
    def num_free_blocks(self) -> int:
        """Free pages plus cached prefix pages only the cache still holds (:149-153)."""
        return len(self._pool.free) + self._index.reclaimable(self._pool)

    @property
    def num_used_blocks(self) -> int:
        return self.num_blocks - self.num_free_blocks

    def required_blocks(self, max_tokens: int) -> int:
        """Pages over all planes for max_tokens positions (:170-173)."""
        if not _is_index(max_tokens) or max_tokens <= 0:
            raise ValueError("max_tokens must be a positive integer")
        return -(-max_tokens // self.block_size) * self.storage_depths

    def _take_pages(self, count: int):
        """`count` fresh pages, evicting least recently used prefixes while short; None if
        even an empty index leaves too few (:182-192)."""
        pool = self._pool
        while len(pool.free) < count:
            evicted = self._index.evict_oldest()
            if evicted is None:
                return None
            pool.release(evicted)
        return pool.take(count)

    # --------------------------------------------------------- prefix cache
    def poll_prefixes(self) -> None:
        """Publish deferred prefixes whose completion event has fired, in arrival order (:201-209).

        A request freed (or freed and re-admitted) since it asked is dropped.
        """
        waiting, self._deferred = self._deferred, []
        for item in waiting:
            if self._allocations.get(item.request_id) is not item.allocation:
                continue
            if item.event is not None and not item.event.query():
                self._deferred.append(item)
            else:
                self.publish_prefix(item.request_id, item.tokens, item.length)

    def publish_prefix(self, request_id, tokens, length, event=None) -> None:
        """Index full prompt pages written at every depth and layer for reuse (:211-238).

        The last prompt token is never published (its hidden state is not
        cached), and only pages every (plane, layer) has written contiguously
        from position 0 qualify.  With an event, publication waits for it.
        """
        if not self.enable_prefix_caching:
            return
        allocation = self._get_allocation(request_id)
        if event is not None:
            self._deferred.append(_DeferredPublish(request_id, allocation, tuple(tokens), length, event))
            return
        publishable = tokens[: min(length, len(tokens) - 1)]
        written = min(w.prefix for plane in allocation.written for w in plane)
        self._index.add_run(publishable[: written - written % self.block_size], allocation.block_tables, self._pool)

    def lookup_prefix(self, tokens) -> tuple:
        """Longest cached run of full pages of tokens[:-1], refreshed as recently used (:240-251)."""
        if not self.enable_prefix_caching:
            return ()
        self.poll_prefixes()
        return self._index.match(tokens[:-1])

    # ----------------------------------------------------------- allocation
    def allocate(self, request_id: str, max_tokens: int, *, initial_tokens=None, prefix=()) -> bool:
        """Reserve capacity and pages for the initial frontier (:253-293).

        Plane d's table is the prefix pages' plane-d entries followed by that
        plane's share of the fresh pages.  On failure nothing stays held.
        """
        if not isinstance(request_id, str) or not request_id:
            raise ValueError("request_id must be a nonempty string")
        if request_id in self._allocations:
            raise ValueError(f"request {request_id!r} already owns KV blocks")
        needed = self.required_blocks(max_tokens)
        if needed > self.num_blocks:
            raise ValueError(f"request needs {needed} physical KV blocks, but the pool has {self.num_blocks}")
        frontier = max_tokens if initial_tokens is None else initial_tokens
        if not 0 < frontier <= max_tokens:
            raise ValueError("invalid initial KV frontier")
        pages = -(-frontier // self.block_size)
        if len(prefix) > pages:
            raise ValueError("prefix exceeds initial KV frontier")
        # Hold the prefix pages first so that making room cannot evict them.
        aliased = [b for entry in prefix for b in entry]
        self._pool.retain(aliased)
        tail = pages - len(prefix)
        fresh = self._take_pages(tail * self.storage_depths)
        if fresh is None:
            self._pool.release(aliased)
            return False
        heads = tuple(tuple(entry[d] for entry in prefix) for d in range(self.storage_depths))
        cached = len(prefix) * self.block_size
        written = [[WrittenPrefix(prefix=cached) for _ in range(self.num_layers)] for _ in range(self.storage_depths)]
        self._allocations[request_id] = Allocation(
            int(max_tokens), _widen(heads, fresh, tail), written, prefix_pages=len(prefix)
        )
        self.prefix_queries += 1
        self.prefix_hits += cached
        return True

    def ensure_capacity(self, request_id, tokens) -> bool:
        """Grow every plane's table to cover `tokens` positions (:295-310)."""
        allocation = self._get_allocation(request_id)
        if not 0 < tokens <= allocation.max_tokens:
            raise ValueError("KV growth exceeds logical capacity")
        extra = -(-tokens // self.block_size) - len(allocation.block_tables[0])
        if extra <= 0:
            return True
        fresh = self._take_pages(extra * self.storage_depths)
        if fresh is None:
            return False
        allocation.block_tables = _widen(allocation.block_tables, fresh, extra)
        return True

    def free(self, request_id: str) -> None:
        """Release a request's pages, or defer while a transfer holds them (:312-319).

        Pages go back table by table, each table from its last page to its first.
        """
        allocation = self._allocations.get(request_id)
        if allocation is None:
            return
        if allocation.transfer_leases:
            allocation.release_requested = True
            return
        del self._allocations[request_id]
        self._pool.release(b for table in allocation.block_tables for b in reversed(table))

    def pin_transfer(self, request_id: str, transfer_id: str) -> None:
        allocation = self._get_allocation(request_id)
        if allocation.release_requested:
            raise RuntimeError("cannot transfer KV scheduled for release")
        allocation.transfer_leases.add(transfer_id)

    def unpin_transfer(self, request_id: str, transfer_id: str) -> None:
        allocation = self._get_allocation(request_id)
        allocation.transfer_leases.discard(transfer_id)
        if allocation.release_requested and not allocation.transfer_leases:
            self.free(request_id)

    def mark_imported_prefix(self, request_id: str, length: int, *, start=0) -> None:
        """Declare positions [0, length) valid on every plane and layer after an import (:333-344)."""
        allocation = self._get_allocation(request_id)
        if type(length) is not int or not 0 < length <= allocation.max_tokens:
            raise ValueError("imported prefix exceeds reserved capacity")
        if allocation.release_requested:
            raise RuntimeError("cannot activate cancelled KV")
        if any(w.prefix != start or w.pending for plane in allocation.written for w in plane):
            raise RuntimeError("KV prefix was already initialized")
        for plane in allocation.written:
            for w in plane:
                w.prefix = length

    def get_block_table(self, request_id: str, depth: int) -> tuple:
        self._validate_depth(depth)
        return self._get_allocation(request_id).block_tables[self._plane(depth)]

    def _plane(self, depth: int) -> int:
        return depth if self.layout == "last_exited" else 0

    def _get_allocation(self, request_id: str) -> Allocation:
        allocation = self._allocations.get(request_id)
        if allocation is None:
            raise KeyError(f"request {request_id!r} has no KV allocation")
        return allocation

    # ----------------------------------------------------------- validation
    def _validate_layer(self, layer: int) -> None:
        if not _is_index(layer) or not 0 <= layer < self.num_layers:
            raise ValueError(f"layer must be in [0, {self.num_layers})")

    def _validate_depth(self, depth: int) -> None:
        if not _is_index(depth) or not 0 <= depth < self.max_loops:
            raise ValueError(f"depth must be in [0, {self.max_loops})")

    def _validate_position(self, allocation: Allocation, position: int) -> None:
        if not _is_index(position) or not 0 <= position < allocation.max_tokens:
            raise ValueError(f"position must be in [0, {allocation.max_tokens})")

    def _validate_rows(self, request_ids, depths, positions):
        """(allocation, depth, position) per row, checked before anything mutates (:383-396)."""
        if isinstance(positions, torch.Tensor):
            if positions.ndim != 1 or positions.dtype not in (torch.int32, torch.int64):
                raise ValueError("positions must be a one-dimensional integer tensor")
            positions = positions.tolist()
        if not len(request_ids) == len(depths) == len(positions):
            raise ValueError("request_ids, depths, and positions must have equal lengths")
        rows = []
        for request_id, depth, position in zip(request_ids, depths, positions):
            allocation = self._get_allocation(request_id)
            self._validate_depth(depth)
            self._validate_position(allocation, position)
            rows.append((allocation, int(depth), int(position)))
        return rows

    def _require_prefix(self, allocation, layer, depth, length) -> None:
        """Attention may only read an initialised contiguous history (:536-543)."""
        if length > allocation.written[self._plane(depth)][layer].prefix:
            raise RuntimeError(
                f"uninitialized KV history at layer {layer}, depth {depth}, context length {length}; "
                "write preceding tokens and finalize early exits before attention"
            )

    def _require_live_batch(self, batch: PreparedKVBatch) -> None:
        """A prepared batch is only valid for the allocations it was built from (:480-485)."""
        if batch.owner is not self:
            raise ValueError("prepared KV batch belongs to a different cache manager")
        for request_id, allocation in batch.allocations:
            if self._allocations.get(request_id) is not allocation:
                raise RuntimeError(f"stale prepared KV batch for request {request_id!r}")

    def _supports_packed_prefill(self) -> bool:
        return False

    # --------------------------------------------------------- batch plans
    def _plan_batch(self, request_ids, depths, positions, *, for_write=True, packed_prefill=False) -> BatchPlan:
        """Layer-independent addresses of a traversal (_prepare_batch, :398-478).

        Row i writes (tables[plane][pos // page], pos % page).  Tables are cut
        to W = max(pos // page + 1) and padded with -1; context length is
        pos + 1.  A packed prefill groups consecutive rows of one
        (request, depth) into a sequence whose table and length are those of
        its last row.
        """
        rows = tuple(self._validate_rows(request_ids, depths, positions))
        page = self.block_size
        blocks = [a.block_tables[self._plane(d)][p // page] for a, d, p in rows]
        offsets = [p % page for _, _, p in rows]
        if for_write and len(set(zip(blocks, offsets))) != len(rows):
            raise ValueError("a write batch cannot contain duplicate request/depth/position addresses")
        width = max((p // page + 1 for _, _, p in rows), default=0)
        table_rows = rows
        cumulative = None
        max_query = 1
        if packed_prefill:
            if self.layout != "last_exited" or not self._supports_packed_prefill():
                raise ValueError("packed prefill requires LAST_EXITED and a packed-prefill attention backend")
            cumulative, last_rows, seen = [0], [], set()
            for i, (allocation, depth, position) in enumerate(rows):
                key = (id(allocation), depth)
                continuing = i > 0 and key == (id(rows[i - 1][0]), rows[i - 1][1])
                if continuing:
                    if position != rows[i - 1][2] + 1:
                        raise ValueError("packed prefill positions must be contiguous")
                    last_rows[-1] = rows[i]
                    cumulative[-1] = i + 1
                else:
                    if key in seen:
                        raise ValueError("packed prefill request/depth must form one sequence")
                    seen.add(key)
                    last_rows.append(rows[i])
                    cumulative.append(i + 1)
            table_rows = tuple(last_rows)
            max_query = max((b - a for a, b in zip(cumulative, cumulative[1:])), default=1)
        tables = np.full((len(table_rows), width), -1, dtype=np.int32)
        for i, (allocation, depth, _) in enumerate(table_rows):
            cut = allocation.block_tables[self._plane(depth)][:width]
            tables[i, : len(cut)] = cut
        owners = dict(zip(request_ids, (a for a, _, _ in rows)))
        return BatchPlan(
            rows=rows,
            allocations=tuple(owners.items()),
            positions=np.array([p for _, _, p in rows], dtype=np.int64),
            write_blocks=np.array(blocks, dtype=np.int64),
            write_offsets=np.array(offsets, dtype=np.int64),
            tables=tables,
            lengths=np.array([p + 1 for _, _, p in table_rows], dtype=np.int32),
            cu_seqlens=None if cumulative is None else np.array(cumulative, dtype=np.int32),
            max_seqlen_q=max_query,
            writable=for_write,
        )

    def _batch_from_plan(self, plan: BatchPlan) -> PreparedKVBatch:
        """Host-tensor form of a plan; the device manager overrides this with one upload."""
        return PreparedKVBatch(
            owner=self,
            rows=plan.rows,
            allocations=plan.allocations,
            position_ids=torch.from_numpy(plan.positions),
            write_blocks=torch.from_numpy(plan.write_blocks),
            write_offsets=torch.from_numpy(plan.write_offsets),
            block_tables=torch.from_numpy(plan.tables),
            context_lengths=torch.from_numpy(plan.lengths),
            writable=plan.writable,
            cu_seqlens_q=None if plan.cu_seqlens is None else torch.from_numpy(plan.cu_seqlens),
            max_seqlen_q=plan.max_seqlen_q,
        )

    def _prepare_batch(
        self,
        request_ids: Sequence[str],
        depths: Sequence[int],
        positions,
        *,
        for_write: bool = True,
        packed_prefill: bool = False,
    ) -> PreparedKVBatch:
        """Build layer-independent addresses once; initialise no KV slot."""
        plan = self._plan_batch(request_ids, depths, positions, for_write=for_write, packed_prefill=packed_prefill)
        return self._batch_from_plan(plan)

    def _require_history(self, batch: PreparedKVBatch) -> None:
        """Every row's earlier positions hold KV at every layer (a whole-core replay's precondition)."""
        for allocation, depth, position in batch.rows:
            for layer in range(self.num_layers):
                self._require_prefix(allocation, layer, depth, position)

    def _record_all_layers(self, batch: PreparedKVBatch) -> None:
        """Mark every row's position written at every layer (after a whole-core replay)."""
        for layer in range(self.num_layers):
            self._record_written(batch, layer)

    def _record_written(self, batch: PreparedKVBatch, layer: int) -> None:
        for allocation, depth, position in batch.rows:
            allocation.written[self._plane(depth)][layer].add(position)
