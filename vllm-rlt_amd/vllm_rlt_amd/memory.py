"""KV pool sizing for the hip backend.

Keeps the entry points the engine and tests call (plan_cache, budget_blocks:
vllm_rlt/engine/llm_engine.py:48-50, tests/test_cdb_runtime.py:269) and the
reference's override rules (vllm_rlt/core/memory.py): an explicit block count
or byte budget wins, and a CPU device gets a fixed default.

The device budget is this package's own.  It adds up what will actually be
allocated next to the pool, asking each allocating object for its size:

* the attention backend's grow-only workspace at its final size
  (HipPagedAttention.workspace_size_for over rlt_paged_decode_workspace_bytes
  for the largest decode batch and rlt_paged_prefill_workspace_bytes for the
  per-token prefill path, which the pool's dtype and shape decide), and with
  graphs the outgrown workspaces captured graphs keep alive (less than the
  largest graph's workspace: powers of two below it);
* the library's static device array (rlt_static_device_bytes);
* the runner's static Workspaces and slot pool, and the AsyncState pools and
  routing banks (their device_bytes(), with each bank's staging copy of its
  pinned buffer when descriptors do not go through UVA, as on ROCm);
* per captured graph its StaticBatch, plus the configured graph reserve for
  the graphs' private activations;
* the model's activation peak (doubled when the core and boundary streams
  overlap): measured around a caller-supplied probe, or around the
  reference's own profiling pass when a model is given without one (a
  temporary pool, prelude, the recurrent pass at every depth, coda;
  vllm_rlt/core/memory.py:37-76), or given as activation_bytes;
* the configured memory reserve.

The pool gets the rest of min(free memory, utilisation x total - reserved),
in whole pages, and never more pages than every concurrent request could use.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field

import torch

from . import ops
from .async_state import AsyncState
from .buffers import Workspace
from .graphs import StaticBatch
from .paged_attention import HipPagedAttention

CPU_DEFAULT_BLOCKS = 256  # vllm_rlt/core/memory.py: pools on a CPU device


def budget_blocks(available_bytes: int, bytes_per_block: int) -> int:
    """Whole pages of bytes_per_block in available_bytes; at least one, else ValueError."""
    blocks = int(available_bytes) // int(bytes_per_block)
    if blocks < 1:
        raise ValueError("no memory remains for KV blocks; reduce execution limits or memory reserve")
    return blocks


def bytes_per_block(config, block_size: int, element_size: int) -> int:
    """K and V of one page at every layer."""
    return 2 * config.num_hidden_layers * block_size * config.num_key_value_heads * config.head_dim * element_size


def _pow2(n: int) -> int:
    return 1 << (max(int(n), 1) - 1).bit_length()


@dataclass
class MemoryPlan:
    """Where the device memory goes, in bytes; `costs` are the non-KV allocations."""

    source: str
    bytes_per_block: int
    num_blocks: int = 0
    costs: dict = field(default_factory=dict)
    budget_bytes: int = 0  # min(free, utilisation x total - reserved) before costs
    kv_bytes: int = 0  # what remains for pages
    max_useful_blocks: int = 0

    def as_dict(self) -> dict:
        return asdict(self)


_DTYPES = {2: torch.bfloat16, 4: torch.float32}


def execution_bytes(config, scheduler, cache, execution, element_size: int, num_q_heads=None, dtype=None) -> dict:
    """Device bytes of everything the runner and this package allocate beside the pool."""
    dtype = dtype or _DTYPES[element_size]
    page = cache.block_size
    width = -(-config.max_position_embeddings // page)
    rows = scheduler.max_num_batched_tokens
    if execution.pad_to_power_of_two:
        rows = _pow2(rows)
    hidden = config.hidden_size
    planes = config.total_ut_steps if cache.layout == "last_exited" else 1
    heads = num_q_heads or config.num_attention_heads
    costs = {}
    # One backend workspace serves decode partials and the per-token prefill path.
    decode = ops.decode_workspace_bytes(rows, heads, config.num_key_value_heads, config.head_dim)
    # Zero on the MFMA prefill path; the per-token path's rows otherwise.
    prefill = ops.prefill_workspace_bytes(
        rows, scheduler.max_num_seqs, width, heads, config.num_key_value_heads, config.head_dim, page, dtype
    )
    costs["attention_workspace"] = HipPagedAttention.workspace_size_for(max(decode, prefill))
    costs["library_static"] = ops.static_device_bytes()
    if execution.static_buffers:
        costs["static_workspaces"] = 4 * Workspace.device_bytes(rows, width, hidden, element_size)
        costs["state_slots"] = scheduler.max_num_seqs * hidden * element_size
    if execution.async_scheduling:
        costs["async_state"] = AsyncState.device_bytes(
            scheduler.max_num_seqs, rows, hidden, width, planes, element_size,
            use_uva=getattr(execution, "use_uva", False),
        )
    if execution.cuda_graphs:
        graph_rows = min(execution.cuda_graph_max_batch_size, rows)
        costs["graph_inputs"] = execution.cuda_graph_max_graphs * (
            StaticBatch.device_bytes(graph_rows, width) + graph_rows * hidden * element_size
        )
        costs["graph_reserve"] = execution.cuda_graph_memory_reserve_bytes
        graph_decode = ops.decode_workspace_bytes(graph_rows, heads, config.num_key_value_heads, config.head_dim)
        costs["graph_held_workspaces"] = HipPagedAttention.workspace_size_for(graph_decode)
    return costs


def _profiling_pass(model, cache, scheduler, execution, device, dtype):
    """The reference's activation probe (vllm_rlt/core/memory.py:46-76) on this package's pool.

    One step of the largest token count, cut into requests of at most
    max_position_embeddings tokens, runs the prelude, the recurrent pass at
    every depth over a temporary LAST-EXITED pool sized for exactly those
    tokens, and the coda.  The temporary pool counts in the peak, as in the
    reference.
    """
    from .kv_cache_manager import KVCacheManager

    config = model.config
    count = min(scheduler.max_num_batched_tokens, scheduler.max_num_seqs * config.max_position_embeddings)
    if execution.pad_to_power_of_two:
        count = _pow2(count)
    longest = config.max_position_embeddings
    lengths = [min(longest, count - start) for start in range(0, count, longest)]

    def probe():
        pages = sum(-(-n // cache.block_size) for n in lengths) * config.total_ut_steps
        kv = KVCacheManager(
            config.num_hidden_layers, config.num_key_value_heads, config.head_dim, pages, cache.block_size,
            config.total_ut_steps, device=device, dtype=dtype, backend="hip",
        )
        ids, positions = [], []
        for index, n in enumerate(lengths):
            rid = f"profile-{index}"
            kv.allocate(rid, n)
            ids += [rid] * n
            positions += list(range(n))
        hidden = model.prelude(torch.zeros(count, dtype=torch.long, device=device))
        for depth in range(config.total_ut_steps):
            hidden, _ = model.recurrent(hidden, ids, [depth] * count, positions, kv)
        model.coda(hidden)

    return probe


def _measure_probe(probe, device) -> int:
    """Peak bytes allocated above the current level while probe() runs."""
    torch.cuda.synchronize(device)
    base = torch.cuda.memory_allocated(device)
    torch.cuda.reset_peak_memory_stats(device)
    probe()
    torch.cuda.synchronize(device)
    return max(0, torch.cuda.max_memory_allocated(device) - base)


@torch.inference_mode()
def plan_cache(config_or_model, cache, scheduler, execution, backend: str = "hip", *, dtype=None, device=None,
               probe=None, activation_bytes=None, memory_info=None):
    """(num_blocks, plan dict) for a KV pool on `device`.

    The first argument is a model (its .config, parameter dtype and device are
    used) or a config with dtype/device given.  `cache` carries the
    reference's CacheConfig fields (num_blocks, kv_cache_memory_bytes,
    block_size, layout, gpu_memory_utilization, memory_reserve_bytes).
    The activation peak comes from `probe()` (the caller's largest step), or
    is `activation_bytes`, or, for a model given with neither, from the
    reference's profiling pass over the model's prelude / recurrent / coda.
    A device plan for a bare config needs a probe or activation_bytes: an
    unbudgeted activation peak would hand its memory to the pool.
    `memory_info` overrides the device's (free, total) bytes.
    """
    if backend != "hip":
        raise ValueError("unknown attention backend")
    config = getattr(config_or_model, "config", config_or_model)
    if hasattr(config_or_model, "parameters"):
        parameter = next(config_or_model.parameters())
        dtype = dtype or parameter.dtype
        device = device or parameter.device
    if dtype is None or device is None:
        raise ValueError("plan_cache needs a model, or dtype and device")
    device = torch.device(device)
    element = torch.empty((), dtype=dtype).element_size()
    per_block = bytes_per_block(config, cache.block_size, element)
    if cache.num_blocks is not None:
        plan = MemoryPlan("blocks", per_block, num_blocks=cache.num_blocks)
        return plan.num_blocks, plan.as_dict()
    if cache.kv_cache_memory_bytes is not None:
        plan = MemoryPlan("bytes", per_block, num_blocks=budget_blocks(cache.kv_cache_memory_bytes, per_block))
        return plan.num_blocks, plan.as_dict()
    if device.type != "cuda":
        plan = MemoryPlan("cpu_default", per_block, num_blocks=CPU_DEFAULT_BLOCKS)
        return plan.num_blocks, plan.as_dict()

    if probe is None and activation_bytes is None:
        if not all(hasattr(config_or_model, name) for name in ("prelude", "recurrent", "coda")):
            raise ValueError(
                "plan_cache needs a model (prelude/recurrent/coda), a probe or activation_bytes to budget activations"
            )
        probe = _profiling_pass(config_or_model, cache, scheduler, execution, device, dtype)
    costs = execution_bytes(config, scheduler, cache, execution, element, dtype=dtype)
    peak = _measure_probe(probe, device) if probe is not None else int(activation_bytes)
    overlap = execution.async_scheduling and execution.multi_stream
    costs["activation_peak"] = peak * (2 if overlap else 1)
    costs["reserve"] = cache.memory_reserve_bytes
    if memory_info is None:
        torch.cuda.synchronize(device)
        with torch.cuda.device(device):
            torch.cuda.empty_cache()  # cached but unused segments count as free
        memory_info = torch.cuda.mem_get_info(device)
    free, total = memory_info
    budget = min(int(free), int(total * cache.gpu_memory_utilization) - torch.cuda.memory_reserved(device))
    kv_bytes = budget - sum(costs.values())
    planes = config.total_ut_steps if cache.layout == "last_exited" else 1
    useful = -(-config.max_position_embeddings // cache.block_size) * planes * scheduler.max_num_seqs
    plan = MemoryPlan(
        "device_profile", per_block, num_blocks=min(budget_blocks(kv_bytes, per_block), useful), costs=costs,
        budget_bytes=budget, kv_bytes=kv_bytes, max_useful_blocks=useful,
    )
    return plan.num_blocks, plan.as_dict()
