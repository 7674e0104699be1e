"""HIP-graph capture and replay of a recurrent decode core over the paged KV path.

RecurrentGraphs keeps the surface the runner uses (vllm_rlt/worker/cuda_graph.py:
32-122 as called at vllm_rlt/worker/model_runner.py:85-92, 390-398): run(hidden,
batch) returns what the core returns, and the captures / replays / fallbacks
counters.  The core is any callable core(hidden, batch, cache) that writes and
attends through cache._write_prepared(_rotary) / cache._attend_prepared (the
model's recurrent pass, vllm_rlt/models/ouro.py:209-217); the model itself is
outside this package.

Design:
* GraphCache holds graphs under any hashable key, each captured once on a
  private stream after warm-up runs, all in one memory pool.  bench.py
  captures its loop-step through the same class.
* One graph per decode row count (and per whether the batch's rows are
  independent, when the core's fused append-and-attend is captured).
  Replays must give the eager bits, and a model's GEMMs may choose other
  kernels at other row counts, so batches are never padded up to a shared
  size.
* A graph reads a StaticBatch: one int64 arena [3, rows] (positions, write
  blocks, write offsets) and one int32 arena (lengths, then the [rows, width]
  tables), loaded from the live batch before each replay.
* The warm-up runs before the first capture of a row count grow the attention
  backend's workspace for it, so the captured kernels keep one workspace
  address and the capture itself allocates none of it.
* Host bookkeeping stays out of the graph: the manager checks every row's
  history before a replay and records the written positions after it.
* Batches a graph cannot serve run eagerly through the real cache: too many
  rows, packed prefill, an empty batch, or a new row count once the graph
  budget is spent.
"""

from __future__ import annotations

from dataclasses import replace

import torch

from .device_cache import DeviceCache


class GraphCache:
    """Graphs keyed by the caller, captured on a private stream into one memory pool."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.pool = torch.cuda.graph_pool_handle()
        self.stream = torch.cuda.Stream(device=self.device)
        self.entries: dict = {}

    def __contains__(self, key) -> bool:
        return key in self.entries

    def __len__(self) -> int:
        return len(self.entries)

    def get(self, key):
        """(graph, output) captured under `key`, or None."""
        return self.entries.get(key)

    def capture(self, key, fn, *, warmups: int = 2):
        """Capture fn() under `key` and return (graph, output).

        The device is drained first (a capture must not race other work), then
        fn runs `warmups` times eagerly on the private stream, so lazily sized
        buffers reach their final size before capture.
        """
        torch.cuda.synchronize(self.device)
        with torch.cuda.stream(self.stream):
            for _ in range(warmups):
                fn()
        self.stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool, stream=self.stream):
            output = fn()
        self.entries[key] = (graph, output)
        return graph, output


class StaticBatch:
    """Fixed-address decode metadata for `rows` rows and tables `width` pages wide.

    Carries the fields a prepared batch exposes to the kernels.
    """

    def __init__(self, rows: int, width: int, device):
        self.size, self.width = rows, width
        self._i64 = torch.zeros((3, rows), dtype=torch.int64, device=device)
        self._i32 = torch.zeros(rows * (1 + width), dtype=torch.int32, device=device)
        self.position_ids, self.write_blocks, self.write_offsets = self._i64.unbind(0)
        self.context_lengths = self._i32[:rows]
        self.block_tables = self._i32[rows:].view(rows, width)
        self.cu_seqlens_q = None
        self.shared_prefix = None

    @staticmethod
    def device_bytes(rows: int, width: int) -> int:
        return rows * (3 * 8 + 4 * (1 + width))

    def load(self, batch) -> None:
        """Copy a live batch's first `size` rows in (stream-ordered device copies)."""
        n = self.size
        self.position_ids.copy_(batch.position_ids[:n])
        self.write_blocks.copy_(batch.write_blocks[:n])
        self.write_offsets.copy_(batch.write_offsets[:n])
        self.context_lengths.copy_(batch.context_lengths[:n])
        width = batch.block_tables.shape[1]
        if width > self.width:
            raise ValueError(f"batch tables are {width} pages wide; the graph holds {self.width}")
        # Columns past the batch's width keep stale entries: the kernels never
        # read a table entry past ceil(length / page).
        self.block_tables[:, :width].copy_(batch.block_tables[:n])


class _Entry:
    def __init__(self, hidden: torch.Tensor, batch: StaticBatch):
        self.hidden, self.batch = hidden, batch
        self.graph = self.output = None


class RecurrentGraphs:
    def __init__(self, core, cache, *, max_batch_size: int, max_graphs: int, max_positions: int):
        self.core, self.cache = core, cache
        self.max_batch_size, self.max_graphs = max_batch_size, max_graphs
        self.width = -(-max_positions // cache.block_size)
        self.graphs = GraphCache(cache.device)
        self._entries: dict[int, _Entry] = {}
        self._last_replay = None  # event after the latest replay (static inputs are reused)
        self.captures = self.replays = self.fallbacks = 0

    def _serves(self, key, batch) -> bool:
        if not 0 < key[0] <= self.max_batch_size or batch.cu_seqlens_q is not None:
            return False
        return key in self._entries or len(self._entries) < self.max_graphs

    def _entry(self, key, hidden: torch.Tensor) -> _Entry:
        entry = self._entries.get(key)
        if entry is None:
            rows = key[0]
            entry = _Entry(torch.empty_like(hidden[:rows]), StaticBatch(rows, self.width, self.cache.device))
        return entry

    def _capture(self, key, entry: _Entry) -> None:
        # The warm-up runs grow the attention backend's workspace for the
        # graph's rows, so the captured kernels see its final address.
        proxy = DeviceCache(self.cache, fused_append=key[1])
        entry.graph, entry.output = self.graphs.capture(key, lambda: self.core(entry.hidden, entry.batch, proxy))
        self._entries[key] = entry
        self.captures += 1

    @staticmethod
    def _unpadded(batch, rows: int):
        """The batch cut to its real rows (a runner may pad it to a larger size)."""
        if len(batch.position_ids) == rows:
            return batch
        return replace(
            batch,
            position_ids=batch.position_ids[:rows],
            context_lengths=batch.context_lengths[:rows],
            block_tables=batch.block_tables[:rows],
        )

    @torch.inference_mode()
    def run(self, hidden: torch.Tensor, batch):
        rows = len(batch.rows)
        # Graphs are keyed by row count and by whether the batch's rows are
        # independent (then the core's fused append-and-attend is captured).
        fused = rows > 0 and batch.cu_seqlens_q is None and self.cache._rows_independent(batch)
        key = (rows, fused)
        if not self._serves(key, batch):
            self.fallbacks += 1
            return self.core(hidden, self._unpadded(batch, rows), self.cache)
        cache = self.cache
        cache._require_live_batch(batch)
        cache._require_history(batch)
        stream = torch.cuda.current_stream(cache.device)
        if self._last_replay is not None:
            stream.wait_event(self._last_replay)  # the previous replay still reads the static inputs
        entry = self._entry(key, hidden)
        entry.hidden.copy_(hidden[:rows])
        entry.batch.load(batch)
        if entry.graph is None:
            self._capture(key, entry)
        entry.graph.replay()
        # The graph's outputs are overwritten by its next replay: hand out copies.
        output = entry.output
        if isinstance(output, torch.Tensor):
            output = output.clone()
        else:
            output = tuple(None if t is None else t.clone() for t in output)
        self._last_replay = torch.cuda.Event()
        self._last_replay.record(stream)
        cache._record_all_layers(batch)
        self.replays += 1
        return output
