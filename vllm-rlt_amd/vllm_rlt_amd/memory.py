"""Startup KV pool sizing for the hip backend.

Mirrors vllm_rlt/core/memory.py:11-129 (budget_blocks, plan_cache) and
vllm_rlt/worker/buffers.py:10-26 (execution_buffer_bytes): explicit block or
byte overrides first; otherwise a peak-memory probe on the device, then the
free memory under gpu_memory_utilization minus the probe's peak (doubled for
concurrent streams), the runner's static buffers, dynamic metadata, the
configured reserve and the graph reserve, clamped to the blocks all
concurrent full-context requests could use.

The probe itself -- a full-depth forward of the model over a temporary KV
manager -- belongs to the model, which is outside this package: the caller
passes it as `probe(cache, request_ids, positions)`.  In place of the torch
backend's long-context attention scratch, the hip backend budgets its own
decode workspace (split partials for the largest decode batch).
"""

from __future__ import annotations

import math

import torch

from . import ops


def budget_blocks(available_bytes: int, bytes_per_block: int) -> int:
    """Whole blocks that fit in available_bytes (vllm_rlt/core/memory.py:11-18)."""
    blocks = int(available_bytes) // bytes_per_block
    if blocks < 1:
        raise ValueError("no memory remains for KV blocks; reduce execution limits or memory reserve")
    return blocks


def execution_buffer_bytes(config, scheduler, cache, execution, element_size: int) -> int:
    """Static runner workspaces and async routing banks (vllm_rlt/worker/buffers.py:10-26)."""
    rows = scheduler.max_num_batched_tokens
    if execution.pad_to_power_of_two:
        rows = 1 << (rows - 1).bit_length()
    width = math.ceil(config.max_position_embeddings / cache.block_size)
    hidden = config.hidden_size * element_size
    total = 0
    if execution.static_buffers:
        total += 4 * rows * (hidden + 4 * width + 36) + scheduler.max_num_seqs * hidden
    if execution.async_scheduling:
        planes = config.total_ut_steps if cache.layout == "last_exited" else 1
        total += 4 * rows * (hidden + 4 * width + 68)
        total += scheduler.max_num_seqs * (hidden + 8 + planes * width * 4)
        total += 2 * scheduler.max_num_seqs * 24
    return total


def bytes_per_block(config, block_size: int, element_size: int) -> int:
    """K and V of one page at every layer (vllm_rlt/core/memory.py:24-32)."""
    return 2 * config.num_hidden_layers * block_size * config.num_key_value_heads * config.head_dim * element_size


@torch.inference_mode()
def plan_cache(config, cache, scheduler, execution, *, dtype: torch.dtype, device, probe=None, memory_info=None):
    """(num_blocks, details) for a KV pool of `config`'s shape on `device`.

    `cache` carries the reference's CacheConfig fields (num_blocks,
    kv_cache_memory_bytes, block_size, layout, gpu_memory_utilization,
    memory_reserve_bytes).  `memory_info` overrides (free, total) device
    bytes; by default they are read from the device after the allocator's
    cache is emptied.
    """
    from .kv_cache_manager import KVCacheManager

    device = torch.device(device)
    element = torch.empty((), dtype=dtype).element_size()
    per_block = bytes_per_block(config, cache.block_size, element)
    if cache.num_blocks is not None:
        return cache.num_blocks, {"source": "blocks", "bytes_per_block": per_block}
    if cache.kv_cache_memory_bytes is not None:
        return budget_blocks(cache.kv_cache_memory_bytes, per_block), {"source": "bytes", "bytes_per_block": per_block}
    if device.type != "cuda":
        return 256, {"source": "cpu_default", "bytes_per_block": per_block}
    torch.cuda.synchronize(device)
    with torch.cuda.device(device):
        torch.cuda.empty_cache()
    free_before, total = memory_info if memory_info is not None else torch.cuda.mem_get_info(device)
    reserved = torch.cuda.memory_reserved(device)
    allocated = torch.cuda.memory_allocated(device)
    torch.cuda.reset_peak_memory_stats(device)
    count = min(scheduler.max_num_batched_tokens, scheduler.max_num_seqs * config.max_position_embeddings)
    if execution.pad_to_power_of_two:
        count = 1 << (count - 1).bit_length()
    peak = 0
    if probe is not None:
        lengths = [
            min(config.max_position_embeddings, count - start)
            for start in range(0, count, config.max_position_embeddings)
        ]
        probe_cache = KVCacheManager(
            num_layers=config.num_hidden_layers,
            num_kv_heads=config.num_key_value_heads,
            head_dim=config.head_dim,
            max_loops=config.total_ut_steps,
            num_blocks=sum(math.ceil(n / cache.block_size) for n in lengths) * config.total_ut_steps,
            block_size=cache.block_size,
            device=device,
            dtype=dtype,
        )
        ids, positions = [], []
        for index, length in enumerate(lengths):
            rid = f"profile-{index}"
            probe_cache.allocate(rid, length)
            ids.extend([rid] * length)
            positions.extend(range(length))
        probe(probe_cache, ids, positions)
        torch.cuda.synchronize(device)
        peak = max(0, torch.cuda.max_memory_allocated(device) - allocated)
        del probe_cache
    # The hip decode keeps split partials for every row of the largest batch.
    workspace = ops.decode_workspace_bytes(
        count, config.num_attention_heads, config.num_key_value_heads, config.head_dim
    )
    buffers = execution_buffer_bytes(config, scheduler, cache, execution, element)
    metadata = scheduler.max_num_batched_tokens * math.ceil(config.max_position_embeddings / cache.block_size) * 4
    budget = min(free_before, int(total * cache.gpu_memory_utilization) - reserved)
    concurrent_peak = peak * (2 if execution.async_scheduling and execution.multi_stream else 1)
    graph_reserve = execution.cuda_graph_memory_reserve_bytes if execution.cuda_graphs else 0
    budget -= concurrent_peak + workspace + buffers + metadata + cache.memory_reserve_bytes + graph_reserve
    useful_blocks = (
        math.ceil(config.max_position_embeddings / cache.block_size)
        * (config.total_ut_steps if cache.layout == "last_exited" else 1)
        * scheduler.max_num_seqs
    )
    blocks = min(budget_blocks(budget, per_block), useful_blocks)
    return blocks, dict(
        source="device_profile",
        bytes_per_block=per_block,
        profile_peak_bytes=peak,
        concurrent_peak_bytes=concurrent_peak,
        max_useful_blocks=useful_blocks,
        graph_reserve_bytes=graph_reserve,
        static_buffer_bytes=buffers,
        decode_workspace_bytes=workspace,
        kv_budget_bytes=int(budget),
    )
