"""Reusable per-step workspace: fixed-width prepared batches from pinned host buffers.

Mirrors vllm_rlt/worker/buffers.py (Workspace :29-96) with the same names,
arguments, padding and ownership rules:

* every buffer is allocated once, [rows] or [rows, width], so the device
  tensors a prepared batch points at keep their addresses from step to step
  (a captured graph can read them);
* ``prepare`` fills rows [0, n) and zeroes rows [n, size): pad rows get
  position 0, context length 0, an all-zero table row and no write address,
  so attention returns zeros for them and the append writes n rows only;
* table rows are zero-padded past the request's table (the kernels never
  read past ceil(length / page));
* the host side waits for the event of the previous step's last reader
  before it overwrites the pinned inputs (``acquire`` / ``release``).

Workspace.device_bytes gives the device memory one Workspace holds, which the
capacity planner (memory.py) budgets.
"""

from __future__ import annotations

import numpy as np
import torch

from .page_book import PreparedKVBatch

__all__ = ["Workspace"]

_INT64 = ("tokens", "positions", "blocks", "offsets")
_INT32 = ("tables", "lengths")


class Workspace:
    def __init__(self, rows: int, width: int, hidden_size: int, device, dtype: torch.dtype):
        device = torch.device(device)
        self.device = device
        self.rows, self.width = int(rows), int(width)
        self.hidden = torch.empty((rows, hidden_size), device=device, dtype=dtype)
        self.event = None
        pinned = device.type == "cuda"
        self.host: dict[str, torch.Tensor] = {}
        self.gpu: dict[str, torch.Tensor] = {}
        for name in _INT64 + _INT32:
            shape = (rows, width) if name == "tables" else (rows,)
            kind = torch.int32 if name in _INT32 else torch.int64
            self.host[name] = torch.empty(shape, dtype=kind, pin_memory=pinned)
            self.gpu[name] = torch.empty(shape, dtype=kind, device=device)

    @staticmethod
    def device_bytes(rows: int, width: int, hidden_size: int, element_size: int) -> int:
        """Device memory of one Workspace: hidden rows, four int64 and two int32 fields."""
        return rows * (hidden_size * element_size + 4 * 8 + 4 + 4 * width)

    def acquire(self) -> None:
        """Wait for the last reader of the previous step's inputs (buffers.py:49-51)."""
        if self.event is not None:
            self.event.synchronize()

    def release(self) -> None:
        """Mark the buffers busy until the current stream's queued work is done (:53-56)."""
        if self.device.type == "cuda":
            self.event = torch.cuda.Event()
            self.event.record(torch.cuda.current_stream(self.device))

    def tokens(self, ids, size: int) -> torch.Tensor:
        """Token ids in rows [0, len(ids)), zeros up to `size`, on the device (:58-63)."""
        host = self.host["tokens"][:size]
        host.zero_()
        host[: len(ids)] = torch.as_tensor(ids, dtype=host.dtype)
        self.gpu["tokens"][:size].copy_(host, non_blocking=True)
        return self.gpu["tokens"][:size]

    def prepare(self, cache, ids, depths, positions, size: int) -> PreparedKVBatch:
        """A writable prepared batch of n rows padded to `size` (:65-96)."""
        rows = tuple(cache._validate_rows(ids, depths, positions))
        n = len(rows)
        if not n <= size <= self.rows:
            raise ValueError(f"size must be in [{n}, {self.rows}]")
        page = cache.block_size
        tables = [a.block_tables[cache._plane(d)] for a, d, _ in rows]
        position = np.fromiter((p for _, _, p in rows), dtype=np.int64, count=n)
        blocks = np.fromiter((t[p // page] for t, (_, _, p) in zip(tables, rows)), dtype=np.int64, count=n)
        offsets = position % page
        if len(set(zip(blocks.tolist(), offsets.tolist()))) != n:
            raise ValueError("duplicate KV write addresses")
        if any(len(t) > self.width for t in tables):
            raise ValueError(f"a block table is wider than the workspace ({self.width} pages)")

        host = {name: self.host[name].numpy() for name in self.host}
        host["positions"][:size] = 0
        host["lengths"][:size] = 0
        host["tables"][:size] = 0
        host["positions"][:n] = position
        host["lengths"][:n] = position + 1
        host["blocks"][:n] = blocks
        host["offsets"][:n] = offsets
        for i, table in enumerate(tables):
            host["tables"][i, : len(table)] = table
        for name in ("positions", "lengths", "tables", "blocks", "offsets"):
            count = n if name in ("blocks", "offsets") else size
            self.gpu[name][:count].copy_(self.host[name][:count], non_blocking=True)
        owners = dict(zip(ids, (a for a, _, _ in rows)))
        return PreparedKVBatch(
            owner=cache,
            rows=rows,
            allocations=tuple(owners.items()),
            position_ids=self.gpu["positions"][:size],
            write_blocks=self.gpu["blocks"][:n],
            write_offsets=self.gpu["offsets"][:n],
            block_tables=self.gpu["tables"][:size],
            context_lengths=self.gpu["lengths"][:size],
            writable=True,
        )
