"""Graph-capturable cache proxy for a recurrent core (vllm_rlt/worker/cuda_graph.py:10-29).

DeviceCache exposes only the GPU side of _write_prepared / _attend_prepared:
no host bookkeeping, no validation that reads device memory, no allocation
beyond the caching allocator, so a 24-layer core that calls it can be captured
in a HIP graph and replayed.  The caller owns the written-position records.
"""

from __future__ import annotations

from . import ops


class DeviceCache:
    """fused_append: _write_attend_prepared runs one rlt_paged_decode_append
    launch (the captured batches' rows are independent) instead of the two
    steps."""

    def __init__(self, cache, *, fused_append: bool = False):
        self.cache = cache
        self.fused_append = fused_append

    def _write_prepared(self, layer, batch, k, v):
        cache = self.cache
        ops.kv_append(cache.key_cache, cache.value_cache, layer, batch.write_blocks, batch.write_offsets, k, v)

    def _write_prepared_rotary(self, layer, batch, q, k, v, position_embeddings):
        cache = self.cache
        cos, sin = position_embeddings
        return ops.rope_kv_append(
            cache.key_cache, cache.value_cache, layer, batch.write_blocks, batch.write_offsets, q, k, v, cos, sin
        )

    def _attend_prepared(self, layer, batch, q):
        cache = self.cache
        return cache.attention(
            q, cache.key_cache[:, layer], cache.value_cache[:, layer], batch.block_tables, batch.context_lengths,
            shared_prefix=getattr(batch, "shared_prefix", None),
        )

    def _write_attend_prepared(self, layer, batch, q, k, v):
        if not self.fused_append:
            self._write_prepared(layer, batch, k, v)
            return self._attend_prepared(layer, batch, q)
        cache = self.cache
        return cache.attention.decode_append(
            q, cache.key_cache[:, layer], cache.value_cache[:, layer], batch.block_tables, batch.context_lengths,
            k, v, batch.write_blocks, batch.write_offsets, shared_prefix=getattr(batch, "shared_prefix", None),
        )
