"""KV pool sizing rules (CPU): overrides, the per-page byte count and buffer budgets.

Follows vllm_rlt/core/memory.py:11-129 and vllm_rlt/worker/buffers.py:10-26.
"""

from types import SimpleNamespace

import pytest
import torch

from vllm_rlt_amd import memory

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
EXEC = SimpleNamespace(
    async_scheduling=False, multi_stream=True, static_buffers=False, pad_to_power_of_two=False, cuda_graphs=False,
    cuda_graph_memory_reserve_bytes=1 << 30,
)


def test_ouro_page_is_three_mebibytes():
    # One page of K+V at every layer: 2 x 24 x 16 x 16 x 128 x 2 bytes.
    assert memory.bytes_per_block(OURO, 16, 2) == 3 * 1024 * 1024


def test_overrides_and_cpu_default():
    per = memory.bytes_per_block(OURO, 16, 2)
    assert memory.plan_cache(OURO, cache_config(num_blocks=77), SCHED, EXEC, dtype=torch.bfloat16, device="cpu")[0] == 77
    blocks, info = memory.plan_cache(
        OURO, cache_config(kv_cache_memory_bytes=10 * per + per - 1), SCHED, EXEC, dtype=torch.bfloat16, device="cpu"
    )
    assert blocks == 10 and info == {"source": "bytes", "bytes_per_block": per}
    assert memory.plan_cache(OURO, cache_config(), SCHED, EXEC, dtype=torch.bfloat16, device="cpu")[0] == 256
    with pytest.raises(ValueError, match="no memory remains"):
        memory.budget_blocks(per - 1, per)


def test_execution_buffers_follow_the_enabled_features():
    cfg = cache_config()
    none = memory.execution_buffer_bytes(OURO, SCHED, cfg, EXEC, 2)
    static = memory.execution_buffer_bytes(OURO, SCHED, cfg, SimpleNamespace(**{**vars(EXEC), "static_buffers": True}), 2)
    both = memory.execution_buffer_bytes(
        OURO, SCHED, cfg, SimpleNamespace(**{**vars(EXEC), "static_buffers": True, "async_scheduling": True}), 2
    )
    assert none == 0 < static < both
    # Padding rounds the batch rows up to a power of two.
    odd = SimpleNamespace(max_num_seqs=8, max_num_batched_tokens=100)
    padded = SimpleNamespace(**{**vars(EXEC), "static_buffers": True, "pad_to_power_of_two": True})
    assert memory.execution_buffer_bytes(OURO, odd, cfg, padded, 2) == memory.execution_buffer_bytes(
        OURO, SCHED, cfg, padded, 2
    )
