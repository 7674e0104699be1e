"""KV pool sizing rules (CPU): overrides, the page size and the budgeted allocations.

The override rules follow vllm_rlt/core/memory.py (explicit blocks, explicit
bytes, CPU default) and tests/test_cdb_runtime.py:269 (budget_blocks refuses
a budget below one page).  The device costs are this package's own: each
item must equal what the allocating object reports for the same shape.
"""

from types import SimpleNamespace

import pytest
import torch

from vllm_rlt_amd import memory, ops
from vllm_rlt_amd.async_state import AsyncState
from vllm_rlt_amd.buffers import Workspace
from vllm_rlt_amd.graphs import StaticBatch
from vllm_rlt_amd.paged_attention import HipPagedAttention

OURO = SimpleNamespace(
    num_hidden_layers=24, num_key_value_heads=16, num_attention_heads=16, head_dim=128, hidden_size=2048,
    max_position_embeddings=65536, total_ut_steps=4,
)


def cache_config(**overrides):
    values = dict(
        num_blocks=None, kv_cache_memory_bytes=None, block_size=16, layout="last_exited",
        gpu_memory_utilization=0.9, memory_reserve_bytes=256 << 20,
    )
    values.update(overrides)
    return SimpleNamespace(**values)


SCHED = SimpleNamespace(max_num_seqs=8, max_num_batched_tokens=128)


def execution(**overrides):
    values = dict(
        async_scheduling=False, multi_stream=True, static_buffers=False, pad_to_power_of_two=False,
        cuda_graphs=False, cuda_graph_max_batch_size=128, cuda_graph_max_graphs=16,
        cuda_graph_memory_reserve_bytes=1 << 30,
    )
    values.update(overrides)
    return SimpleNamespace(**values)


def test_ouro_page_is_three_mebibytes():
    # One page of K+V at every layer: 2 x 24 x 16 x 16 x 128 x 2 bytes.
    assert memory.bytes_per_block(OURO, 16, 2) == 3 * 1024 * 1024


def test_overrides_and_cpu_default():
    per = memory.bytes_per_block(OURO, 16, 2)
    plan = dict(dtype=torch.bfloat16, device="cpu")
    assert memory.plan_cache(OURO, cache_config(num_blocks=77), SCHED, execution(), **plan)[0] == 77
    blocks, info = memory.plan_cache(OURO, cache_config(kv_cache_memory_bytes=11 * per - 1), SCHED, execution(), **plan)
    assert blocks == 10 and info["source"] == "bytes" and info["bytes_per_block"] == per
    assert memory.plan_cache(OURO, cache_config(), SCHED, execution(), **plan)[0] == memory.CPU_DEFAULT_BLOCKS
    with pytest.raises(ValueError, match="no memory remains"):
        memory.budget_blocks(per - 1, per)
    with pytest.raises(ValueError, match="no memory remains"):
        memory.budget_blocks(-1, per)
    with pytest.raises(ValueError, match="backend"):
        memory.plan_cache(OURO, cache_config(), SCHED, execution(), "torch", **plan)
    with pytest.raises(ValueError, match="dtype and device"):
        memory.plan_cache(OURO, cache_config(), SCHED, execution())


def test_costs_follow_the_enabled_features():
    cfg = cache_config()
    plain = memory.execution_bytes(OURO, SCHED, cfg, execution(), 2)
    assert set(plain) == {"attention_workspace", "library_static"}
    full = memory.execution_bytes(
        OURO, SCHED, cfg, execution(static_buffers=True, async_scheduling=True, cuda_graphs=True), 2
    )
    assert set(full) == {
        "attention_workspace", "library_static", "static_workspaces", "state_slots", "async_state", "graph_inputs",
        "graph_reserve", "graph_held_workspaces",
    }
    assert all(v > 0 for v in full.values())


def test_costs_equal_what_each_object_reports():
    cfg = cache_config()
    width = 65536 // 16
    costs = memory.execution_bytes(
        OURO, SCHED, cfg, execution(static_buffers=True, async_scheduling=True, cuda_graphs=True), 2
    )
    rows = SCHED.max_num_batched_tokens
    decode = ops.decode_workspace_bytes(rows, 16, 16, 128)
    assert costs["attention_workspace"] == HipPagedAttention.workspace_size_for(decode) >= decode
    assert costs["static_workspaces"] == 4 * Workspace.device_bytes(rows, width, 2048, 2)
    # Without UVA (the ROCm runner's choice) every bank keeps a device copy of its pinned buffer.
    assert costs["async_state"] == AsyncState.device_bytes(8, rows, 2048, width, 4, 2, use_uva=False)
    assert costs["graph_inputs"] == 16 * (StaticBatch.device_bytes(128, width) + 128 * 2048 * 2)
    assert costs["graph_held_workspaces"] == HipPagedAttention.workspace_size_for(decode)
    assert costs["library_static"] == ops.static_device_bytes() == 64 << 20
    # SHARED stores one plane: smaller device tables.
    shared = memory.execution_bytes(OURO, SCHED, cache_config(layout="shared"), execution(async_scheduling=True), 2)
    assert shared["async_state"] == AsyncState.device_bytes(8, rows, 2048, width, 1, 2, use_uva=False)
    assert shared["async_state"] < costs["async_state"]
    uva = memory.execution_bytes(OURO, SCHED, cfg, execution(async_scheduling=True, use_uva=True), 2)
    assert uva["async_state"] == AsyncState.device_bytes(8, rows, 2048, width, 4, 2)


def test_staging_bound_covers_a_step_that_ships_every_table_whole():
    from vllm_rlt_amd.async_state import RoutingBank

    rows, seqs, planes, width = 16, 8, 4, 4096
    bound = RoutingBank.staging_capacity_bound(rows, seqs, planes, width)
    # Replay the bank's growth rule for the largest step: 8 new requests x 4 planes x 4096 pages.
    capacity, need = 4 * rows, seqs * planes * width
    while capacity < need:
        capacity = max(need, 2 * capacity)
    assert capacity <= bound
    extra = RoutingBank.device_bytes(rows, width, 2048, 2, bound) - RoutingBank.device_bytes(rows, width, 2048, 2)
    assert extra == 8 * (3 * rows + 2 * bound)


def test_device_plan_of_a_bare_config_needs_a_probe_or_activation_bytes():
    plan = dict(dtype=torch.bfloat16, device="cuda", memory_info=(8 << 30, 16 << 30))
    with pytest.raises(ValueError, match="activation"):
        memory.plan_cache(OURO, cache_config(), SCHED, execution(), **plan)


def test_per_token_prefill_is_budgeted_for_every_dtype_that_takes_it():
    cfg = cache_config()
    # bf16 at head_dim 256 (no MFMA tile) takes the per-token path like fp32 does.
    wide = SimpleNamespace(**{**vars(OURO), "head_dim": 256})
    need = ops.prefill_workspace_bytes(128, 8, 4096, 16, 16, 256, 16, torch.bfloat16)
    assert need > 0
    costs = memory.execution_bytes(wide, SCHED, cfg, execution(), 2, dtype=torch.bfloat16)
    assert costs["attention_workspace"] >= need
    # Page 32 leaves the MFMA path too.
    big_page = ops.prefill_workspace_bytes(128, 8, 2048, 16, 16, 128, 32, torch.bfloat16)
    costs = memory.execution_bytes(OURO, SCHED, cache_config(block_size=32), execution(), 2)
    assert big_page > 0 and costs["attention_workspace"] >= big_page


def test_padding_rounds_rows_up_and_fp32_budgets_the_per_token_prefill():
    cfg = cache_config()
    odd = SimpleNamespace(max_num_seqs=8, max_num_batched_tokens=100)
    padded = execution(static_buffers=True, pad_to_power_of_two=True)
    assert memory.execution_bytes(OURO, odd, cfg, padded, 2) == memory.execution_bytes(OURO, SCHED, cfg, padded, 2)
    fp32 = memory.execution_bytes(OURO, SCHED, cfg, execution(), 4)["attention_workspace"]
    prefill = ops.prefill_workspace_bytes(128, 8, 4096, 16, 16, 128, 16, torch.float32)
    assert fp32 >= prefill > 0
    assert ops.prefill_workspace_bytes(128, 8, 4096, 16, 16, 128, 16, torch.bfloat16) == 0
