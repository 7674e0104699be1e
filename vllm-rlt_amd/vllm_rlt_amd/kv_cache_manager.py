"""Paged KV cache manager with the HIP data path (drop-in for vllm_rlt's KVCacheManager).

Same constructor, methods and error behaviour as
vllm_rlt/core/kv_cache_manager.py:74-637; the host bookkeeping lives in
KVPageBook, every byte of KV moves through librlt_kv.so:

  _write_prepared -> rlt_kv_append       (index_put pair, :531-532)
  _attend_prepared -> rlt_paged_decode / rlt_paged_prefill (:570-586)
  finalize_token  -> rlt_kv_copy_token   (exit copies, :601-611)
  read            -> rlt_kv_gather       (ordered gather, :631-637)

The only backend is "hip" on a ROCm device; there is no CPU path.
"""

from __future__ import annotations

from numbers import Integral

import torch

from . import ops
from .page_book import BatchPlan, KVPageBook, PreparedKVBatch
from .paged_attention import HipPagedAttention

BACKENDS = ("hip",)
DTYPES = (torch.float32, torch.float16, torch.bfloat16)

# Reference-compatible alias of the batch type.
_PreparedKVBatch = PreparedKVBatch


class KVCacheManager(KVPageBook):
    """Own a fixed physical page pool shared by request/depth allocations.

    ``num_blocks`` counts physical blocks across all recurrence depths; every
    block holds K and V for all decoder layers.  Depth indices are 0-based.
    """

    def __init__(
        self,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        num_blocks: int,
        block_size: int,
        max_loops: int,
        device: str | torch.device = "cuda",
        dtype: torch.dtype = torch.bfloat16,
        backend: str = "hip",
        layout: str = "last_exited",
        enable_prefix_caching: bool = False,
        incremental_allocation: bool = False,
        watermark_ratio: float = 0.0,
        share_prefix_reads: bool = True,
    ):
        super().__init__(
            num_layers,
            num_kv_heads,
            head_dim,
            num_blocks,
            block_size,
            max_loops,
            layout=layout,
            enable_prefix_caching=enable_prefix_caching,
            incremental_allocation=incremental_allocation,
            watermark_ratio=watermark_ratio,
        )
        if backend not in BACKENDS:
            raise ValueError("unknown attention backend")
        if dtype not in DTYPES:
            raise ValueError("KV dtype must be float32, float16, or bfloat16")
        device = torch.device(device)
        if device.type != "cuda" or not torch.version.hip:
            raise ValueError("the hip attention backend requires a ROCm device")
        self.backend = backend
        self.dtype = dtype
        # Decode rows whose pages came from the prefix cache read those pages
        # once per launch for all rows that share them, one group per plane
        # and prefix (rlt_paged_decode_shared_prefix).  Which splits take that
        # path depends on the row's own allocation, and each row's result on
        # its own q and pages, so a row's bits do not depend on the batch.
        self.share_prefix_reads = bool(share_prefix_reads)
        self._query_group = 8  # q heads per KV head, learnt from the first attention call
        self.attention = HipPagedAttention(device, dtype, self.head_dim, self.block_size)
        self.attention_info = self.attention.info
        shape = (self.num_blocks, self.num_layers, self.block_size, self.num_kv_heads, self.head_dim)
        self.key_cache = torch.empty(shape, device=device, dtype=dtype)
        self.value_cache = torch.empty_like(self.key_cache)
        # Resolve an implicit device index to the storage device once.
        self.device = self.key_cache.device

    @property
    def bytes_per_block(self) -> int:
        return 2 * self.num_layers * self.block_size * self.num_kv_heads * self.head_dim * self.key_cache.element_size()

    def _supports_packed_prefill(self) -> bool:
        return bool(getattr(self.attention, "supports_packed_prefill", False))

    # ------------------------------------------------------------ metadata
    def _batch_from_plan(self, plan: BatchPlan) -> PreparedKVBatch:
        """Pack the plan into one pinned buffer and upload it with a single copy."""
        n = len(plan.positions)
        t, w = plan.tables.shape
        s = 0 if plan.cu_seqlens is None else len(plan.cu_seqlens)
        found = None
        if self.share_prefix_reads and plan.cu_seqlens is None and len(plan.rows) == t:
            row_pages = [
                allocation.block_tables[self._plane(depth)][: allocation.prefix_pages] if allocation.prefix_pages else ()
                for allocation, depth, _ in plan.rows
            ]
            # The prefix pass's item counts depend on the q heads per KV head,
            # which the first attention call tells; until then they are sized
            # for the widest group it serves.
            found = ops.prefix_group_layout(row_pages, plan.lengths, self.block_size, self._query_group)
        hint32 = 0 if found is None else len(found[0])
        n64 = 3 * n
        n32 = t * w + t + s + hint32
        bytes64 = 8 * n64
        total = bytes64 + (4 * n32 + 7) // 8 * 8
        host = torch.empty(max(total, 8), dtype=torch.uint8, pin_memory=True)
        if n64:
            h64 = host[:bytes64].view(torch.int64).numpy()
            h64[:n] = plan.positions
            h64[n : 2 * n] = plan.write_blocks
            h64[2 * n :] = plan.write_offsets
        if n32:
            h32 = host[bytes64 : bytes64 + 4 * n32].view(torch.int32).numpy()
            h32[: t * w] = plan.tables.reshape(-1)
            h32[t * w : t * w + t] = plan.lengths
            if s:
                h32[t * w + t : t * w + t + s] = plan.cu_seqlens
            if found is not None:
                base = t * w + t + s
                h32[base : base + hint32] = found[0]
        dev = host.to(self.device, non_blocking=True)
        d64 = dev[:bytes64].view(torch.int64) if n64 else torch.empty(0, dtype=torch.int64, device=self.device)
        d32 = (
            dev[bytes64 : bytes64 + 4 * n32].view(torch.int32)
            if n32
            else torch.empty(0, dtype=torch.int32, device=self.device)
        )
        return PreparedKVBatch(
            owner=self,
            rows=plan.rows,
            allocations=plan.allocations,
            position_ids=d64[:n],
            write_blocks=d64[n : 2 * n],
            write_offsets=d64[2 * n : 3 * n],
            block_tables=d32[: t * w].view(t, w),
            context_lengths=d32[t * w : t * w + t],
            writable=plan.writable,
            cu_seqlens_q=d32[t * w + t : t * w + t + s] if s else None,
            max_seqlen_q=plan.max_seqlen_q,
            shared_prefix=None if found is None else self._prefix_groups_view(d32, t * w + t + s, t, found),
        )

    @staticmethod
    def _prefix_groups_view(d32, base, t, found):
        hint, *counts = found
        return ops.PrefixGroups(d32[base : base + len(hint)], t, *counts)

    # ------------------------------------------------------------ tensors
    def _validate_tensor(self, tensor, batch_size, name, *, query=False) -> None:
        """Shape, head count, device and dtype of k / v / q (:487-496)."""
        if tensor.ndim != 3 or tensor.shape[0] != batch_size or tensor.shape[-1] != self.head_dim:
            raise ValueError(f"{name} must have shape [batch, heads, {self.head_dim}]")
        if query:
            if tensor.shape[1] == 0 or tensor.shape[1] % self.num_kv_heads:
                raise ValueError("query heads must be a positive multiple of KV heads")
            self._query_group = min(tensor.shape[1] // self.num_kv_heads, 64)
        elif tensor.shape[1] != self.num_kv_heads:
            raise ValueError(f"{name} must have {self.num_kv_heads} KV heads")
        if tensor.device != self.device or tensor.dtype != self.dtype:
            raise ValueError(f"{name} must use device {self.device} and dtype {self.dtype}")

    # ---------------------------------------------------------------- KV ops
    @torch.no_grad()
    def write(self, layer, request_ids, depths, positions, k, v) -> None:
        """Write a packed batch before attend; address validation precedes tensor validation (:498-517)."""
        self._validate_layer(layer)
        batch = self._prepare_batch(request_ids, depths, positions)
        self._write_prepared(layer, batch, k, v)

    @torch.no_grad()
    def _write_prepared(self, layer: int, batch: PreparedKVBatch, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append the rows' K/V at their (block, layer, offset) slots (:520-534)."""
        self._validate_layer(layer)
        self._require_live_batch(batch)
        if not batch.writable:
            raise ValueError("a read-only prepared KV batch cannot be written")
        self._validate_tensor(k, len(batch.position_ids), "k")
        self._validate_tensor(v, len(batch.position_ids), "v")
        if not batch.rows:
            return
        ops.kv_append(
            self.key_cache, self.value_cache, layer, batch.write_blocks, batch.write_offsets, k, v, n_rows=len(batch.rows)
        )
        self._record_written(batch, layer)

    @torch.no_grad()
    def _write_prepared_rotary(
        self,
        layer: int,
        batch: PreparedKVBatch,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        position_embeddings: tuple[torch.Tensor, torch.Tensor],
    ) -> torch.Tensor:
        """Rotate q and k and append the rows' K/V in one launch; returns rotated q.

        The fused form of the caller's rotation (vllm_rlt/models/ouro.py:104-109,
        q * cos + rotate_half(q) * sin with the traversal's position_embeddings)
        followed by _write_prepared (:520-534).  Pages and the returned q are
        bit-identical to the unfused sequence.
        """
        self._validate_layer(layer)
        self._require_live_batch(batch)
        if not batch.writable:
            raise ValueError("a read-only prepared KV batch cannot be written")
        self._validate_tensor(q, len(batch.position_ids), "q", query=True)
        self._validate_tensor(k, len(batch.position_ids), "k")
        self._validate_tensor(v, len(batch.position_ids), "v")
        cos, sin = position_embeddings
        out = ops.rope_kv_append(
            self.key_cache, self.value_cache, layer, batch.write_blocks, batch.write_offsets, q, k, v, cos, sin,
            n_rows=len(batch.rows),
        )
        if batch.rows:
            self._record_written(batch, layer)
        return out

    @torch.no_grad()
    def attend(self, layer, request_ids, depths, positions, q) -> torch.Tensor:
        """Causal GQA at each row's own position and recurrence depth (:545-557)."""
        self._validate_layer(layer)
        batch = self._prepare_batch(request_ids, depths, positions, for_write=False)
        return self._attend_prepared(layer, batch, q)

    @torch.no_grad()
    def _attend_prepared(self, layer: int, batch: PreparedKVBatch, q: torch.Tensor) -> torch.Tensor:
        """Decode rows, or packed prefill sequences when cu_seqlens_q is set (:559-586)."""
        self._validate_layer(layer)
        self._require_live_batch(batch)
        self._validate_tensor(q, len(batch.position_ids), "q", query=True)
        if not batch.rows:
            return torch.empty_like(q)
        for allocation, depth, position in batch.rows:
            self._require_prefix(allocation, layer, depth, position + 1)
        if batch.cu_seqlens_q is not None:
            return self.attention.prefill(
                q,
                self.key_cache[:, layer],
                self.value_cache[:, layer],
                batch.block_tables,
                batch.context_lengths,
                batch.cu_seqlens_q,
                batch.max_seqlen_q,
            )
        shared_prefix = getattr(batch, "shared_prefix", None)  # absent from batches built by other code
        if shared_prefix is not None:
            return self.attention(
                q, self.key_cache[:, layer], self.value_cache[:, layer], batch.block_tables, batch.context_lengths,
                shared_prefix=shared_prefix,
            )
        return self.attention(
            q, self.key_cache[:, layer], self.value_cache[:, layer], batch.block_tables, batch.context_lengths
        )

    def _rows_independent(self, batch: PreparedKVBatch) -> bool:
        """No row of this decode batch reads a KV slot another row writes.

        Holds when every (request, storage plane) has one row: a row writes
        only its own plane's private page at its own position, and pages
        shared between requests (an aliased prefix) are never written.
        """
        if batch.cu_seqlens_q is not None:
            return False
        planes = {(id(allocation), self._plane(depth)) for allocation, depth, _ in batch.rows}
        return len(planes) == len(batch.rows)

    @torch.no_grad()
    def _write_attend_prepared(
        self, layer: int, batch: PreparedKVBatch, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor
    ) -> torch.Tensor:
        """_write_prepared then _attend_prepared (:520-586) as one launch where that gives the same bits.

        A decode batch whose rows are independent (_rows_independent) runs
        rlt_paged_decode_append (rlt_paged_decode_shared_prefix with its
        append when the batch carries prefix groups); any other batch (packed
        prefill, a request twice on one plane) runs the two steps.
        """
        if not self._rows_independent(batch):
            self._write_prepared(layer, batch, k, v)
            return self._attend_prepared(layer, batch, q)
        self._validate_layer(layer)
        self._require_live_batch(batch)
        if not batch.writable:
            raise ValueError("a read-only prepared KV batch cannot be written")
        n = len(batch.position_ids)
        self._validate_tensor(k, n, "k")
        self._validate_tensor(v, n, "v")
        self._validate_tensor(q, n, "q", query=True)
        if not batch.rows:
            return torch.empty_like(q)
        # Each row's history before its new token must already be there.
        for allocation, depth, position in batch.rows:
            self._require_prefix(allocation, layer, depth, position)
        out = self.attention.decode_append(
            q, self.key_cache[:, layer], self.value_cache[:, layer], batch.block_tables, batch.context_lengths,
            k, v, batch.write_blocks, batch.write_offsets, n_write=len(batch.rows),
            shared_prefix=getattr(batch, "shared_prefix", None),
        )
        self._record_written(batch, layer)
        return out

    @torch.no_grad()
    def finalize_token(self, request_id: str, position: int, exit_depth: int) -> None:
        """Copy the exit depth's K/V of one token into every unexecuted depth (:588-614)."""
        allocation = self._get_allocation(request_id)
        self._validate_depth(exit_depth)
        self._validate_position(allocation, position)
        exit_plane = self._plane(exit_depth)
        if any(position not in allocation.written[exit_plane][layer] for layer in range(self.num_layers)):
            raise RuntimeError("cannot finalize a token before every layer has written its exit depth")
        if self.layout == "shared":
            return
        logical_page, offset = divmod(position, self.block_size)
        source = allocation.block_tables[exit_plane][logical_page]
        targets = range(exit_depth + 1, self.max_loops)
        destinations = [allocation.block_tables[self._plane(d)][logical_page] for d in targets]
        if destinations:
            ops.kv_copy_token(self.key_cache, self.value_cache, source, destinations, offset)
        for depth in targets:
            for layer in range(self.num_layers):
                allocation.written[self._plane(depth)][layer].add(position)

    @torch.no_grad()
    def read(self, layer: int, request_id: str, depth: int, length: int | None = None):
        """[length, kv_heads, head_dim] K and V of a fully initialised prefix (:616-637)."""
        self._validate_layer(layer)
        self._validate_depth(depth)
        allocation = self._get_allocation(request_id)
        plane = self._plane(depth)
        if length is None:
            length = allocation.written[plane][layer].prefix
        if not isinstance(length, Integral) or isinstance(length, bool) or not 0 <= length <= allocation.max_tokens:
            raise ValueError("read length exceeds the request's reserved token budget")
        self._require_prefix(allocation, layer, depth, length)
        pages = -(-length // self.block_size)
        table = torch.tensor(allocation.block_tables[plane][:pages], dtype=torch.int32).to(self.device)
        return ops.kv_gather(self.key_cache, self.value_cache, layer, table, int(length))
