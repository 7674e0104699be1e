"""Event-owned pinned bank for packed chunked-prefill metadata of every loop depth.

Mirrors vllm_rlt/worker/prefill_metadata.py (PrefillMetadataBank :12-110)
with the same names, arguments and ownership rules.  One host description
covers all depths:

    [tokens n | positions n | sequence n | ends q | cumulative q + 1 |
     tables depths x q x W]                                  (int64, pinned)

where consecutive rows of one request form one packed sequence (q of them),
ends = last position + 1 (the sequence's context length), cumulative = the
cu_seqlens of the packed queries, and W = max(position) // page + 1 with
tables cut to W and padded with -1.  rlt_stage_prefill reads the pinned
buffer directly and writes it to an int64 and an int32 device copy (one
transfer for all depths); rlt_expand_prefill then derives each depth's
per-row write addresses on the device.  ``metadata(depth)`` returns views of
those buffers as a prepared batch, equal field by field to the manager's
``_prepare_batch(..., packed_prefill=True)`` for that depth.

The pinned buffer and the device outputs are reused: ``prepare`` waits for
the event ``release`` recorded after the last consumer, so neither is
overwritten while a queued kernel still reads it.  Buffers grow to the next
power of two and are never shrunk.
"""

from __future__ import annotations

import numpy as np
import torch

from . import ops
from .page_book import PreparedKVBatch


class PrefillMetadataBank:
    def __init__(self, cache):
        self.cache = cache
        self.done = None
        self.capacity = 0
        self.row_capacity = 0

    def prepare(self, ids, positions, tokens) -> torch.Tensor:
        """Stage the packed metadata of all depths; returns the device token ids (:19-88)."""
        if self.done is not None:
            self.done.synchronize()
        cache = self.cache
        ids = list(ids)
        positions = [int(p) for p in (positions.tolist() if isinstance(positions, torch.Tensor) else positions)]
        tokens = tokens.tolist() if isinstance(tokens, torch.Tensor) else list(tokens)
        n = len(ids)
        if not n or len(positions) != n or len(tokens) != n:
            raise ValueError("ids, positions and tokens must be non-empty and of equal length")
        allocations = cache._allocations
        owners = {rid: allocations[rid] for rid in ids}
        self.ids, self.positions = ids, positions
        self.allocations = tuple(owners.items())

        # Packed sequences: runs of equal consecutive ids.
        starts = [i for i in range(n) if i == 0 or ids[i] != ids[i - 1]]
        q = len(starts)
        bounds = starts + [n]
        sequence = np.repeat(np.arange(q, dtype=np.int64), np.diff(bounds))
        ends = np.array([positions[b - 1] + 1 for b in bounds[1:]], dtype=np.int64)
        cumulative = np.array(bounds, dtype=np.int64)
        cumulative[0] = 0
        page = cache.block_size
        width = max(positions) // page + 1
        depths = cache.storage_depths
        tables = np.full((depths, q, width), -1, dtype=np.int64)
        for s, b in enumerate(starts):
            allocation = allocations[ids[b]]
            for depth in range(depths):
                cut = allocation.block_tables[depth][:width]
                tables[depth, s, : len(cut)] = cut

        sizes = (n, n, n, q, q + 1, depths * q * width)
        total = sum(sizes)
        if total > self.capacity:
            self.capacity = 1 << (total - 1).bit_length()
            self.host = torch.empty(self.capacity, dtype=torch.int64, pin_memory=True)
            self.device = torch.empty(self.capacity, dtype=torch.int64, device=cache.device)
            self.device32 = torch.empty(self.capacity, dtype=torch.int32, device=cache.device)
        np.concatenate(
            (np.asarray(tokens, dtype=np.int64), np.asarray(positions, dtype=np.int64), sequence, ends, cumulative,
             tables.reshape(-1)),
            out=self.host.numpy()[:total],
        )
        ops.stage_prefill(self.host, self.device, self.device32, total)

        self.n, self.q, self.width = n, q, width
        self.tokens = self.device[:n]
        self.position_ids = self.device[n : 2 * n]
        seq = self.device[2 * n : 3 * n]
        self.lengths = self.device32[3 * n : 3 * n + q]
        self.cu = self.device32[3 * n + q : 3 * n + 2 * q + 1]
        self.tables = self.device32[3 * n + 2 * q + 1 : total].view(depths, q, width)
        if n > self.row_capacity:
            self.row_capacity = 1 << (n - 1).bit_length()
            self.block_storage = torch.empty((depths, self.row_capacity), dtype=torch.int64, device=cache.device)
            self.offset_storage = torch.empty_like(self.block_storage)
        self.blocks = self.block_storage[:, :n]
        self.offsets = self.offset_storage[:, :n]
        for depth in range(depths):
            ops.expand_prefill(
                self.position_ids, seq, self.tables[depth], page, self.blocks[depth], self.offsets[depth], n
            )
        self.max_query = int(np.diff(cumulative).max())
        return self.tokens

    def metadata(self, depth: int) -> PreparedKVBatch:
        """The packed prefill batch of one depth, as views of the staged buffers (:90-106)."""
        plane = self.cache._plane(depth)
        rows = tuple((self.cache._allocations[rid], depth, pos) for rid, pos in zip(self.ids, self.positions))
        return PreparedKVBatch(
            self.cache,
            rows,
            self.allocations,
            self.position_ids,
            self.blocks[plane],
            self.offsets[plane],
            self.tables[plane],
            self.lengths,
            True,
            self.cu,
            self.max_query,
        )

    def release(self) -> None:
        """Record the point after which the staged buffers may be reused (:108-110)."""
        self.done = torch.cuda.Event()
        self.done.record(torch.cuda.current_stream(self.cache.device))
