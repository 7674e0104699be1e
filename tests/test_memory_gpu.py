"""Device-profiled KV pool sizing (GPU).

The probe's peak and every budgeted allocation come out of the pool's share,
and each budgeted item matches what the allocating object really takes.
"""

from types import SimpleNamespace

import pytest
import torch

from vllm_rlt_amd import memory

pytestmark = pytest.mark.gpu

CONFIG = SimpleNamespace(
    num_hidden_layers=4, num_key_value_heads=4, num_attention_heads=8, head_dim=64, hidden_size=512,
    max_position_embeddings=256, total_ut_steps=4,
)
CACHE = SimpleNamespace(
    num_blocks=None, kv_cache_memory_bytes=None, block_size=16, layout="last_exited", gpu_memory_utilization=0.9,
    memory_reserve_bytes=64 << 20,
)
SCHED = SimpleNamespace(max_num_seqs=4, max_num_batched_tokens=64)


def execution(**overrides):
    values = dict(
        async_scheduling=False, multi_stream=True, static_buffers=False, pad_to_power_of_two=False,
        cuda_graphs=False, cuda_graph_max_batch_size=32, cuda_graph_max_graphs=4,
        cuda_graph_memory_reserve_bytes=1 << 30,
    )
    values.update(overrides)
    return SimpleNamespace(**values)


def test_probe_peak_and_costs_reduce_the_pool():
    free, total = 8 << 30, 16 << 30
    plan = dict(dtype=torch.bfloat16, device="cuda", memory_info=(free, total))
    base_blocks, base = memory.plan_cache(CONFIG, CACHE, SCHED, execution(), **plan)
    calls = []

    def probe():
        calls.append(1)
        scratch = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        scratch.fill_(1)

    blocks, info = memory.plan_cache(CONFIG, CACHE, SCHED, execution(async_scheduling=True), probe=probe, **plan)
    assert calls == [1]
    assert info["costs"]["activation_peak"] >= 2 * (256 << 20)  # doubled: core and boundary streams overlap
    assert info["kv_bytes"] == info["budget_bytes"] - sum(info["costs"].values())
    assert base["kv_bytes"] - info["kv_bytes"] >= 2 * (256 << 20)
    per = info["bytes_per_block"]
    useful = 256 // 16 * 4 * 4
    assert info["max_useful_blocks"] == useful
    assert blocks == min(info["kv_bytes"] // per, useful) and base_blocks == min(base["kv_bytes"] // per, useful)


def test_budgeted_items_match_the_real_allocations():
    from vllm_rlt_amd import KVCacheManager
    from vllm_rlt_amd.async_state import AsyncState

    ex = execution(async_scheduling=True)
    _, info = memory.plan_cache(CONFIG, CACHE, SCHED, ex, dtype=torch.bfloat16, device="cuda")
    cache = KVCacheManager(4, 4, 64, 64, 16, 4, device="cuda", dtype=torch.bfloat16)
    rows = SCHED.max_num_batched_tokens
    cache.attention.reserve_decode(rows, CONFIG.num_attention_heads, CONFIG.num_key_value_heads)
    assert cache.attention.workspace_bytes == info["costs"]["attention_workspace"]
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    state = AsyncState(cache, CONFIG, SCHED, rows)
    taken = torch.cuda.memory_allocated() - before
    # The caching allocator rounds each tensor up to 512 bytes.
    assert info["costs"]["async_state"] <= taken <= info["costs"]["async_state"] + 64 * 512
    del state


def test_planned_pool_fits_on_the_device():
    from vllm_rlt_amd import KVCacheManager

    big = SimpleNamespace(**{**vars(CONFIG), "max_position_embeddings": 1 << 20})
    sched = SimpleNamespace(max_num_seqs=64, max_num_batched_tokens=64)
    cache = SimpleNamespace(**{**vars(CACHE), "gpu_memory_utilization": 0.1})
    blocks, info = memory.plan_cache(big, cache, sched, execution(), dtype=torch.bfloat16, device="cuda")
    assert info["source"] == "device_profile" and blocks > 1000
    manager = KVCacheManager(4, 4, 64, blocks, 16, 4, device="cuda", dtype=torch.bfloat16)
    assert manager.num_free_blocks == blocks
    del manager
    torch.cuda.empty_cache()
