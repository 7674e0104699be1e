"""HIP-graph capture and replay of a recurrent decode core over the paged KV path.

Mirrors RecurrentGraphs (vllm_rlt/worker/cuda_graph.py:32-122): one graph per
decode batch size, captured on first use over static metadata buffers and the
graph-capturable DeviceCache proxy, replayed afterwards; batches it cannot
serve (too large, packed prefill, empty, or a new size once the graph budget
is spent) run eagerly through the real cache.  History is validated on the
host before launch, and the written positions are recorded after replay, so
capture never freezes or repeats host bookkeeping.

The core is any callable core(hidden, batch, cache) -> tensor or tuple of
tensors that performs the per-layer write / attend through
cache._write_prepared(_rotary) and cache._attend_prepared (the reference's
model.recurrent_prepared, vllm_rlt/models/ouro.py:209-217); the model itself
is outside this package.
"""

from __future__ import annotations

import math
from dataclasses import replace
from types import SimpleNamespace

import torch

from .device_cache import DeviceCache


class RecurrentGraphs:
    def __init__(self, core, cache, *, max_batch_size: int, max_graphs: int, max_positions: int):
        self.core, self.cache = core, cache
        self.max_batch_size, self.max_graphs = max_batch_size, max_graphs
        self.width = math.ceil(max_positions / cache.block_size)
        self.entries = {}
        self.pool = torch.cuda.graph_pool_handle()
        self.capture_stream = torch.cuda.Stream(device=cache.device)
        self.last_event = None
        self.captures = self.replays = self.fallbacks = 0

    @torch.inference_mode()
    def run(self, hidden: torch.Tensor, batch):
        count = len(batch.rows)
        if len(batch.position_ids) != count:
            batch = replace(
                batch,
                position_ids=batch.position_ids[:count],
                context_lengths=batch.context_lengths[:count],
                block_tables=batch.block_tables[:count],
            )
        if (
            count > self.max_batch_size
            or not count
            or batch.cu_seqlens_q is not None
            or (count not in self.entries and len(self.entries) >= self.max_graphs)
        ):
            self.fallbacks += 1
            return self.core(hidden, batch, self.cache)
        cache = self.cache
        cache._require_live_batch(batch)
        # One position per (request, depth): validate history before launch.
        for allocation, depth, pos in batch.rows:
            for layer in range(cache.num_layers):
                cache._require_prefix(allocation, layer, depth, pos)
        stream = torch.cuda.current_stream(cache.device)
        if self.last_event is not None:
            stream.wait_event(self.last_event)
        entry = self.entries.get(count)
        if entry is None:
            device = cache.device
            entry = SimpleNamespace(
                hidden=torch.empty_like(hidden[:count]),
                metadata=SimpleNamespace(
                    position_ids=torch.empty(count, device=device, dtype=torch.long),
                    write_blocks=torch.empty(count, device=device, dtype=torch.long),
                    write_offsets=torch.empty(count, device=device, dtype=torch.long),
                    block_tables=torch.zeros((count, self.width), device=device, dtype=torch.int32),
                    context_lengths=torch.empty(count, device=device, dtype=torch.int32),
                ),
            )
        entry.hidden.copy_(hidden[:count])
        for name in ("position_ids", "write_blocks", "write_offsets", "context_lengths"):
            getattr(entry.metadata, name).copy_(getattr(batch, name)[:count])
        width = batch.block_tables.shape[1]
        entry.metadata.block_tables[:, :width].copy_(batch.block_tables[:count])
        if count not in self.entries:
            # First-use capture is outside steady-state timing; capture cannot race other launches.
            torch.cuda.synchronize(cache.device)
            proxy = DeviceCache(cache)
            with torch.cuda.stream(self.capture_stream):
                for _ in range(2):
                    self.core(entry.hidden, entry.metadata, proxy)
            self.capture_stream.synchronize()
            entry.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(entry.graph, pool=self.pool, stream=self.capture_stream):
                entry.output = self.core(entry.hidden, entry.metadata, proxy)
            self.entries[count] = entry
            self.captures += 1
        entry.graph.replay()
        # Outputs must outlive the graph-private buffers' next reuse.
        output = entry.output
        output = output.clone() if isinstance(output, torch.Tensor) else tuple(
            t.clone() if t is not None else None for t in output
        )
        self.last_event = torch.cuda.Event()
        self.last_event.record(stream)
        for allocation, depth, pos in batch.rows:
            for layer in range(cache.num_layers):
                allocation.written[cache._plane(depth)][layer].add(pos)
        self.replays += 1
        return output
