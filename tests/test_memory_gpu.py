"""Device-profiled KV pool sizing (GPU): the probe's peak and the hip decode workspace come out of the budget."""

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
        cuda_graphs=False, cuda_graph_memory_reserve_bytes=1 << 30,
    )
    values.update(overrides)
    return SimpleNamespace(**values)


def test_probe_peak_and_workspace_reduce_the_budget():
    free, total = 8 << 30, 16 << 30
    base_blocks, base = memory.plan_cache(
        CONFIG, CACHE, SCHED, execution(), dtype=torch.bfloat16, device="cuda", memory_info=(free, total)
    )
    seen = {}

    def probe(cache, ids, positions):
        # The probe sees a full-depth manager with every profiling row allocated.
        seen["rows"] = len(ids)
        seen["blocks"] = cache.num_blocks
        scratch = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        scratch.fill_(1)

    blocks, info = memory.plan_cache(
        CONFIG, CACHE, SCHED, execution(async_scheduling=True), dtype=torch.bfloat16, device="cuda", probe=probe,
        memory_info=(free, total),
    )
    assert seen == {"rows": 64, "blocks": 4 * 4}  # 64 tokens at 16 per page, 4 depths
    assert info["profile_peak_bytes"] >= 256 << 20
    assert info["concurrent_peak_bytes"] == 2 * info["profile_peak_bytes"]
    assert base["kv_budget_bytes"] - info["kv_budget_bytes"] >= 2 * (256 << 20)
    assert info["decode_workspace_bytes"] > 0
    per = info["bytes_per_block"]
    useful = 256 // 16 * 4 * 4
    assert blocks == min(info["kv_budget_bytes"] // per, useful) and base_blocks == min(base["kv_budget_bytes"] // per, useful)


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
