"""Slot-resident request state and descriptor banks for asynchronous decode (hip backend).

The runner drives this through the names of vllm_rlt/worker/async_state.py
(AsyncState: .hidden .tokens .tables .width .slots .free .owners .banks
.index .use_uva, prepare(), release(); a bank: .host .count .size .width
.descriptor .done .ready_event, record_done(), transfer(), gather(),
scatter(); used at vllm_rlt/worker/model_runner.py:167-179, 333-340,
360-430, 462-463, 504-564, 584-589).  The mechanism underneath is this
package's own:

* Page tables live on the device, [max_seqs, planes, width] int32, and are
  patched, never re-uploaded.  Each request's lease records how many entries
  of every plane the device already holds.  A bank ships only what is
  missing: a new request's whole table once, then a growing request's new
  pages.  transfer() applies all of a step's patches in one rlt_patch_tables
  launch.
* A bank keeps the step's (slot, depth, position) descriptors and its table
  patches in one pinned host buffer.  With use_uva the kernels read it in
  place (pinned memory is device-addressable on ROCm); otherwise one
  non-blocking copy moves descriptors and patches together.
* The routing outputs (slots, positions, write blocks/offsets, lengths,
  depth-resolved tables) sit in two device arenas per bank, allocated once,
  so their addresses never change (a captured graph may read them).
* A bank is rewritten only after the event of its last reader (record_done)
  has completed; a request slot returns to the free list only on release().
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np
import torch

from . import ops
from .page_book import PreparedKVBatch

DEFAULT_BANKS = 4
FINALIZE_BANKS = 2


@dataclass
class _Lease:
    """One request's residency in a state slot."""

    slot: int
    request: int  # id() of the request object that took the slot
    allocation: object  # the page-book allocation whose tables the device holds
    shipped: list  # table entries per plane already patched into the device tables


class RoutingBank:
    """Descriptors, table patches and routing outputs of one step."""

    def __init__(self, owner: "AsyncState", rows: int, *, control_only: bool = False):
        self.owner = owner
        self.rows = int(rows)
        self.control_only = control_only
        self.done = self.ready_event = None
        self.descriptor = None
        self.count = self.size = self.width = 0
        self.imports: list = []
        self.n_patches = 0
        self._staging = None  # device copy of the pinned buffer (use_uva=False)
        self._alloc_host(patch_capacity=0 if control_only else 4 * self.rows)
        if control_only:
            return
        device = owner.cache.device
        # Arena of int64 outputs: slots, positions, write blocks, write offsets.
        self._i64 = torch.empty((4, self.rows), dtype=torch.int64, device=device)
        self.slots, self.positions, self.blocks, self.offsets = self._i64.unbind(0)
        # Arena of int32 outputs: lengths, then the depth-resolved table rows.
        self._i32 = torch.zeros(self.rows * (1 + owner.width), dtype=torch.int32, device=device)
        self.lengths = self._i32[: self.rows]
        self.tables = self._i32[self.rows :].view(self.rows, owner.width)
        self.hidden = torch.empty((self.rows, owner.hidden.shape[1]), dtype=owner.hidden.dtype, device=device)
        self.tokens = torch.empty((self.rows, 1), dtype=torch.int64, device=device)

    @staticmethod
    def device_bytes(rows: int, width: int, hidden_size: int, element_size: int, staging_patches: int = 0) -> int:
        """Device memory one transferring bank holds (arenas, hidden and token rows).

        staging_patches > 0 adds the device copy of the pinned buffer that a
        bank without UVA keeps, at that patch capacity.
        """
        arenas = rows * (4 * 8 + 4 * (1 + width) + hidden_size * element_size + 8)
        staging = 8 * (3 * rows + 2 * staging_patches) if staging_patches else 0
        return arenas + staging

    @staticmethod
    def staging_capacity_bound(rows: int, max_num_seqs: int, planes: int, width: int) -> int:
        """Largest patch capacity a bank reaches: a step ships at most every plane's
        whole table of each of its requests, and the capacity starts at 4 x rows and
        grows to max(need, twice the old capacity)."""
        need = min(rows, max_num_seqs) * planes * width
        return max(4 * rows, 2 * need)

    # ------------------------------------------------------------ host side
    def _alloc_host(self, patch_capacity: int) -> None:
        """One pinned int64 buffer: [rows, 3] descriptors, then [capacity, 2] patches."""
        self.patch_capacity = int(patch_capacity)
        self._pinned = torch.empty(3 * self.rows + 2 * self.patch_capacity, dtype=torch.int64, pin_memory=True)
        self.host = self._pinned[: 3 * self.rows].view(self.rows, 3)
        self._patches = self._pinned[3 * self.rows :].view(self.patch_capacity, 2)
        self._staging = None

    def acquire(self) -> None:
        """Wait for the last GPU reader of the previous step, then start empty."""
        if self.done is not None:
            self.done.synchronize()
        self.imports.clear()
        self.n_patches = 0
        self.descriptor = None

    def add_patches(self, flat_start: int, entries) -> None:
        """Queue tables.view(-1)[flat_start + j] = entries[j]."""
        count = len(entries)
        if not count:
            return
        end = self.n_patches + count
        if end > self.patch_capacity:
            # The bank is acquired (no reader left), so its buffer can be replaced.
            kept = self._patches[: self.n_patches].clone()
            descriptors = self.host.clone()
            self._alloc_host(max(end, 2 * self.patch_capacity))
            self.host.copy_(descriptors)
            self._patches[: self.n_patches].copy_(kept)
        patch = self._patches.numpy()[self.n_patches : end]
        patch[:, 0] = np.arange(flat_start, flat_start + count, dtype=np.int64)
        patch[:, 1] = entries
        self.n_patches = end

    # ------------------------------------------------------------ device side
    def _device_source(self, stream) -> torch.Tensor:
        """The pinned buffer itself (use_uva) or its device copy, moved with one transfer."""
        if self.owner.use_uva:
            return self._pinned
        used = 3 * self.rows + 2 * self.n_patches
        if self._staging is None:
            self._staging = torch.empty_like(self._pinned, device=self.owner.cache.device)
        self._staging[:used].copy_(self._pinned[:used], non_blocking=True)
        return self._staging

    def transfer(self, batch: PreparedKVBatch | None = None):
        """Apply table patches and imported states, build the routing metadata on the device.

        Returns `batch` with its fields pointing at this bank's device outputs.
        """
        owner = self.owner
        device = owner.cache.device
        stream = torch.cuda.current_stream(device)
        source = self._device_source(stream)
        if self.n_patches:
            patches = source[3 * self.rows : 3 * self.rows + 2 * self.n_patches].view(self.n_patches, 2)
            ops.patch_tables(patches, self.n_patches, owner.tables)
        for slot, hidden in self.imports:
            hidden.record_stream(stream)
            owner.hidden[slot].copy_(hidden)
        self.descriptor = source[: 3 * self.rows].view(self.rows, 3)[: max(self.count, 1)]
        ops.build_decode_metadata(
            self.descriptor, self.count, self.size, owner.tables, owner.page, self.slots, self.positions,
            self.lengths, self.blocks, self.offsets, self.tables, self.width,
        )
        self.ready_event = torch.cuda.Event()
        self.ready_event.record(stream)
        return None if batch is None else self.device_batch(batch)

    def device_batch(self, batch: PreparedKVBatch) -> PreparedKVBatch:
        """`batch` reading positions, addresses, lengths and tables from this bank."""
        n, size = self.count, self.size
        return replace(
            batch,
            position_ids=self.positions[:size],
            write_blocks=self.blocks[:n],
            write_offsets=self.offsets[:n],
            block_tables=self.tables[:size, : self.width],
            context_lengths=self.lengths[:size],
        )

    def record_done(self) -> None:
        """Mark the bank busy until the current stream's queued work completes."""
        self.done = torch.cuda.Event()
        self.done.record(torch.cuda.current_stream(self.owner.cache.device))

    def gather(self, tokens: bool = False) -> torch.Tensor:
        """Batch-ordered hidden states (or token ids) of the routed rows; pad rows read zeros."""
        pool, out = (self.owner.tokens, self.tokens) if tokens else (self.owner.hidden, self.hidden)
        ops.gather_rows(pool, self.slots, out[: self.size], self.count)
        return out[: self.size, 0] if tokens else out[: self.size]

    def scatter(self, values: torch.Tensor, tokens: bool = False) -> None:
        """Store the first `count` batch rows back into their request slots."""
        if tokens:
            ops.scatter_rows(values.reshape(-1, 1), self.slots, self.owner.tokens, self.count)
        else:
            ops.scatter_rows(values, self.slots, self.owner.hidden, self.count)


class AsyncState:
    """Request slots, device page tables and a ring of routing banks."""

    def __init__(self, cache, config, scheduler, rows: int, *, use_uva: bool = True, banks: int = DEFAULT_BANKS):
        self.cache = cache
        self.use_uva = use_uva
        self.page = cache.block_size
        self.width = -(-config.max_position_embeddings // self.page)
        self.planes = cache.storage_depths
        seqs = scheduler.max_num_seqs
        device = cache.device
        self.hidden = torch.empty((seqs, config.hidden_size), dtype=cache.key_cache.dtype, device=device)
        self.tokens = torch.zeros((seqs, 1), dtype=torch.int64, device=device)
        self.tables = torch.zeros((seqs, self.planes, self.width), dtype=torch.int32, device=device)
        self.owners: dict[str, _Lease] = {}
        self.slots: dict[str, int] = {}  # request id -> slot (the runner's state_slots)
        self.free = list(range(seqs - 1, -1, -1))  # pop() hands out 0, 1, 2, ...
        self.banks = [RoutingBank(self, rows) for _ in range(banks)]
        self.finalize_banks = [RoutingBank(self, seqs, control_only=True) for _ in range(FINALIZE_BANKS)]
        self.index = self.finalize_index = 0

    @staticmethod
    def device_bytes(max_num_seqs: int, rows: int, hidden_size: int, width: int, planes: int, element_size: int,
                     banks: int = DEFAULT_BANKS, use_uva: bool = True) -> int:
        """Device memory an AsyncState of this shape allocates (without UVA, each bank's
        staging copy at its largest capacity included)."""
        pools = max_num_seqs * (hidden_size * element_size + 8 + planes * width * 4)
        patches = 0 if use_uva else RoutingBank.staging_capacity_bound(rows, max_num_seqs, planes, width)
        return pools + banks * RoutingBank.device_bytes(rows, width, hidden_size, element_size, patches)

    def _next_bank(self, finalize: bool) -> RoutingBank:
        if finalize:
            bank = self.finalize_banks[self.finalize_index]
            self.finalize_index = (self.finalize_index + 1) % len(self.finalize_banks)
        else:
            bank = self.banks[self.index]
            self.index = (self.index + 1) % len(self.banks)
        bank.acquire()
        return bank

    def _slot_for(self, request, bank: RoutingBank) -> int:
        """The request's slot; a first visit leases one and queues its imported state."""
        rid = request.request_id
        allocation = self.cache._get_allocation(rid)
        lease = self.owners.get(rid)
        if lease is None:
            if not self.free:
                raise RuntimeError("every request state slot is leased; release finished requests first")
            lease = _Lease(self.free.pop(), id(request), allocation, [0] * self.planes)
            self.owners[rid] = lease
            self.slots[rid] = lease.slot
            hidden = getattr(request, "hidden_state", None)
            if hidden is not None:
                bank.imports.append((lease.slot, hidden))
                request.hidden_state = self.hidden[lease.slot]
        elif lease.request != id(request) or lease.allocation is not allocation:
            raise RuntimeError(f"request {rid!r} still holds the state slot of an earlier owner; release it first")
        if not bank.control_only:
            self._ship_tables(lease, allocation.block_tables, bank)
        return lease.slot

    def _ship_tables(self, lease: _Lease, tables, bank: RoutingBank) -> None:
        """Queue the table entries of every plane the device does not hold yet.

        An allocation's existing entries never change (growth appends pages),
        so the device copy stays valid and only the new tail moves.
        """
        for plane, entries in enumerate(tables):
            have = lease.shipped[plane]
            if len(entries) > self.width:
                raise ValueError(f"a block table of {len(entries)} pages exceeds the routing width {self.width}")
            if len(entries) > have:
                bank.add_patches((lease.slot * self.planes + plane) * self.width + have, entries[have:])
                lease.shipped[plane] = len(entries)

    def prepare(self, requests, depths, positions, size, *, recurrent=False, finalize=False):
        """Fill the next bank with the step's descriptors; a recurrent step also gets its batch.

        Depths route only recurrent and finalize steps; other stages read depth 0.
        Finalize banks are never transferred: their requests' tables are on the
        device already from the recurrent steps before them.
        """
        bank = self._next_bank(finalize)
        n = len(requests)
        if not 0 < n <= size <= bank.rows:
            raise ValueError(f"a routed step needs 0 < rows <= size <= {bank.rows}")
        bank.count, bank.size = n, size
        bank.width = max(p // self.page for p in positions) + 1
        routed = recurrent or finalize
        descriptors = np.empty((n, 3), dtype=np.int64)
        for i, (request, depth, position) in enumerate(zip(requests, depths, positions)):
            descriptors[i] = (self._slot_for(request, bank), depth if routed else 0, position)
        bank.host.numpy()[:n] = descriptors
        if not recurrent:
            return bank, None
        return bank, self._routed_batch(bank, requests, depths, positions)

    def _routed_batch(self, bank: RoutingBank, requests, depths, positions) -> PreparedKVBatch:
        """A writable batch whose device fields are this bank's (valid after transfer())."""
        cache = self.cache
        ids = [r.request_id for r in requests]
        rows = tuple(cache._validate_rows(ids, depths, positions))
        slots = {
            (allocation.block_tables[cache._plane(depth)][position // self.page], position % self.page)
            for allocation, depth, position in rows
        }
        if len(slots) != len(rows):
            raise ValueError("duplicate KV write addresses in a routed batch")
        n, size = bank.count, bank.size
        return PreparedKVBatch(
            owner=cache,
            rows=rows,
            allocations=tuple({rid: row[0] for rid, row in zip(ids, rows)}.items()),
            position_ids=bank.host[:n, 2],
            write_blocks=bank.blocks[:n],
            write_offsets=bank.offsets[:n],
            block_tables=bank.tables[:size, : bank.width],
            context_lengths=bank.lengths[:size],
            writable=True,
        )

    def release(self, rid: str) -> None:
        """Return a finished request's slot; its device tables are overwritten by the next lease."""
        lease = self.owners.pop(rid, None)
        self.slots.pop(rid, None)
        if lease is not None:
            self.free.append(lease.slot)
