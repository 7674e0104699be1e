"""Stable request slots and event-owned routing banks for asynchronous decode on ROCm.

Mirrors vllm_rlt/worker/async_state.py (RoutingBank :16-112, AsyncState
:115-216) with the same names, arguments and ownership rules, over the HIP
kernels of librlt_kv.so:

* page tables stay on the device, [max_seqs, planes, W] int32, with a row
  uploaded only when the request's table changed;
* each step's (slot, depth, position) descriptors go into a pinned host bank
  and rlt_build_decode_metadata turns them into write addresses, lengths and
  depth-resolved tables on the device;
* hidden states and tokens live in slot-indexed device pools, moved to and
  from batch order by rlt_gather_rows / rlt_scatter_rows;
* no bank or request slot is reused until its last GPU reader completed
  (events recorded by the caller's stream).

The reference reads descriptors through UVA on CUDA and copies them to the
device on ROCm (vllm_rlt/worker/model_runner.py:175).  The metadata kernel
here reads pinned host descriptors directly on ROCm, so use_uva defaults to
True; use_uva=False keeps the copy.
"""

from __future__ import annotations

import math
from dataclasses import replace

import torch

from . import ops
from .page_book import PreparedKVBatch


class RoutingBank:
    def __init__(self, owner: "AsyncState", rows: int, *, control_only: bool = False):
        self.owner = owner
        self.host = torch.empty((rows, 3), dtype=torch.int64, pin_memory=True)
        self.done = self.ready_event = None
        self.uploads = []
        self.imports = []
        self.descriptor = None
        self.count = self.size = self.width = 0
        if control_only:
            return
        device = owner.cache.device
        self.slots = torch.empty(rows, dtype=torch.int64, device=device)
        self.positions = torch.empty_like(self.slots)
        self.blocks = torch.empty_like(self.slots)
        self.offsets = torch.empty_like(self.slots)
        self.lengths = torch.empty(rows, dtype=torch.int32, device=device)
        self.tables = torch.zeros((rows, owner.width), dtype=torch.int32, device=device)
        self.hidden = torch.empty((rows, owner.hidden.shape[1]), dtype=owner.hidden.dtype, device=device)
        self.tokens = torch.empty((rows, 1), dtype=torch.int64, device=device)

    def acquire(self) -> None:
        """Wait until the bank's previous readers finished (async_state.py:38-43)."""
        if self.done is not None:
            self.done.synchronize()
        self.uploads.clear()
        self.imports.clear()
        self.descriptor = None

    def transfer(self, batch: PreparedKVBatch | None = None):
        """Upload changed tables and imported states, then build the metadata (async_state.py:45-87)."""
        owner = self.owner
        device = owner.cache.device
        for slot, table in self.uploads:
            owner.tables[slot, :, : table.shape[1]].copy_(table, non_blocking=True)
        for slot, hidden in self.imports:
            hidden.record_stream(torch.cuda.current_stream(device))
            owner.hidden[slot].copy_(hidden)
        self.descriptor = (
            self.host[: max(self.count, 1)]
            if owner.use_uva
            else self.host[: max(self.count, 1)].to(device, non_blocking=True)
        )
        ops.build_decode_metadata(
            self.descriptor,
            self.count,
            self.size,
            owner.tables,
            owner.cache.block_size,
            self.slots,
            self.positions,
            self.lengths,
            self.blocks,
            self.offsets,
            self.tables,
            self.width,
        )
        self.ready_event = torch.cuda.Event()
        self.ready_event.record(torch.cuda.current_stream(device))
        if batch is None:
            return None
        return replace(
            batch,
            position_ids=self.positions[: self.size],
            context_lengths=self.lengths[: self.size],
            write_blocks=self.blocks[: self.count],
            write_offsets=self.offsets[: self.count],
            block_tables=self.tables[: self.size, : self.width],
        )

    def record_done(self) -> None:
        self.done = torch.cuda.Event()
        self.done.record(torch.cuda.current_stream(self.owner.cache.device))

    def gather(self, tokens: bool = False) -> torch.Tensor:
        """Batch-ordered hidden states (or tokens) of the bank's rows; padding rows read 0 (:93-102)."""
        pool = self.owner.tokens if tokens else self.owner.hidden
        output = self.tokens if tokens else self.hidden
        ops.gather_rows(pool, self.slots, output[: self.size], self.count)
        return output[: self.size, 0] if tokens else output[: self.size]

    def scatter(self, values: torch.Tensor, tokens: bool = False) -> None:
        """Write the batch's first `count` rows back to their slots (:104-112)."""
        pool = self.owner.tokens if tokens else self.owner.hidden
        values = values.reshape(-1, 1) if tokens else values
        ops.scatter_rows(values, self.slots, pool, self.count)


class AsyncState:
    def __init__(self, cache, config, scheduler, rows: int, *, use_uva: bool = True, banks: int = 4):
        self.cache = cache
        self.use_uva = use_uva
        self.width = math.ceil(config.max_position_embeddings / cache.block_size)
        self.planes = config.total_ut_steps if cache.layout == "last_exited" else 1
        self.hidden = torch.empty(
            (scheduler.max_num_seqs, config.hidden_size), dtype=cache.key_cache.dtype, device=cache.device
        )
        self.tokens = torch.empty((scheduler.max_num_seqs, 1), dtype=torch.int64, device=cache.device)
        self.tables = torch.zeros(
            (scheduler.max_num_seqs, self.planes, self.width), dtype=torch.int32, device=cache.device
        )
        self.slots = {}
        self.table_versions = {}
        self.owners = {}
        self.free = list(reversed(range(scheduler.max_num_seqs)))
        self.banks = [RoutingBank(self, rows) for _ in range(banks)]
        self.finalize_banks = [RoutingBank(self, scheduler.max_num_seqs, control_only=True) for _ in range(2)]
        self.index = self.finalize_index = 0

    def ensure_slot(self, request, bank: RoutingBank) -> int:
        """The request's device slot; queues a table upload when its tables changed (:145-170)."""
        rid = request.request_id
        allocation = self.cache._get_allocation(rid)
        if rid in self.slots:
            if self.owners[rid] != (id(request), id(allocation)):
                raise RuntimeError("request slot reused before retiring its previous owner")
            slot = self.slots[rid]
            if self.table_versions.get(rid) != allocation.block_tables:
                table = torch.tensor(allocation.block_tables, dtype=torch.int32).pin_memory()
                bank.uploads.append((slot, table))
                self.table_versions[rid] = allocation.block_tables
            return slot
        if not self.free:
            raise RuntimeError("no retired request state slots")
        slot = self.free.pop()
        self.slots[rid] = slot
        self.owners[rid] = (id(request), id(allocation))
        table = torch.tensor(allocation.block_tables, dtype=torch.int32).pin_memory()
        bank.uploads.append((slot, table))
        self.table_versions[rid] = allocation.block_tables
        if getattr(request, "hidden_state", None) is not None:
            bank.imports.append((slot, request.hidden_state))
            request.hidden_state = self.hidden[slot]
        return slot

    def prepare(self, requests, depths, positions, size, *, recurrent=False, finalize=False):
        """Fill the next bank's descriptors; for recurrent steps also a borrowed batch (:172-210)."""
        if finalize:
            bank = self.finalize_banks[self.finalize_index]
            self.finalize_index = (self.finalize_index + 1) % len(self.finalize_banks)
        else:
            bank = self.banks[self.index]
            self.index = (self.index + 1) % len(self.banks)
        bank.acquire()
        bank.count, bank.size = len(requests), size
        bank.width = max(p // self.cache.block_size + 1 for p in positions)
        descriptors = [
            (self.ensure_slot(r, bank), d if recurrent or finalize else 0, p)
            for r, d, p in zip(requests, depths, positions)
        ]
        # A plain list stays host-owned; only the pinned snapshot is device-readable.
        bank.host.numpy()[: len(descriptors)] = descriptors
        batch = None
        if recurrent:
            ids = [r.request_id for r in requests]
            rows = tuple(self.cache._validate_rows(ids, depths, positions))
            addresses = [
                (a.block_tables[self.cache._plane(d)][p // self.cache.block_size], p % self.cache.block_size)
                for a, d, p in rows
            ]
            if len(set(addresses)) != len(addresses):
                raise ValueError("duplicate KV write addresses")
            batch = PreparedKVBatch(
                owner=self.cache,
                rows=rows,
                allocations=tuple(dict(zip(ids, (a for a, _, _ in rows))).items()),
                position_ids=bank.host[: len(rows), 2],
                write_blocks=bank.blocks[: len(rows)],
                write_offsets=bank.offsets[: len(rows)],
                block_tables=bank.tables[:size, : bank.width],
                context_lengths=bank.lengths[:size],
                writable=True,
            )
        return bank, batch

    def release(self, rid: str) -> None:
        self.table_versions.pop(rid, None)
        self.owners.pop(rid, None)
        slot = self.slots.pop(rid, None)
        if slot is not None:
            self.free.append(slot)
