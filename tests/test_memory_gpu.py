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
    base_blocks, base = memory.plan_cache(CONFIG, CACHE, SCHED, execution(), activation_bytes=0, **plan)
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

    # The state below reads descriptors through UVA (no per-bank staging copy).
    ex = execution(async_scheduling=True, use_uva=True)
    _, info = memory.plan_cache(CONFIG, CACHE, SCHED, ex, dtype=torch.bfloat16, device="cuda", activation_bytes=0)
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
    blocks, info = memory.plan_cache(
        big, cache, sched, execution(), dtype=torch.bfloat16, device="cuda", activation_bytes=0
    )
    assert info["source"] == "device_profile" and blocks > 1000
    manager = KVCacheManager(4, 4, 64, blocks, 16, 4, device="cuda", dtype=torch.bfloat16)
    assert manager.num_free_blocks == blocks
    del manager
    torch.cuda.empty_cache()


def test_workspace_growth_releases_what_it_outgrows():
    """Eager batches of growing size keep one workspace: the device holds no more
    than the planned workspace for the largest batch."""
    from vllm_rlt_amd import KVCacheManager

    cache = KVCacheManager(4, 4, 64, 64, 16, 4, device="cuda", dtype=torch.bfloat16)
    attention = cache.attention
    planned = memory.execution_bytes(
        CONFIG, SimpleNamespace(max_num_seqs=4, max_num_batched_tokens=4096), CACHE, execution(), 2
    )["attention_workspace"]
    import gc

    gc.collect()  # earlier tests' garbage must not be freed inside the measurement
    gc.disable()
    try:
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        for rows in (16, 64, 300, 1000, 4096):
            attention.reserve_decode(rows, CONFIG.num_attention_heads, CONFIG.num_key_value_heads)
            torch.cuda.synchronize()
            held = torch.cuda.memory_allocated() - before
            assert held == attention.workspace_bytes, (rows, held, attention.workspace_bytes)
    finally:
        gc.enable()
    assert attention.held_bytes == 0
    assert attention.workspace_bytes <= planned


def test_graphs_captured_at_growing_sizes_stay_within_the_planned_items():
    """Workspaces that captured graphs read stay alive; together with the final one
    they fit attention_workspace + graph_held_workspaces, and every graph still
    replays to the eager result."""
    from vllm_rlt_amd import KVCacheManager
    from vllm_rlt_amd.graphs import GraphCache

    torch.manual_seed(3)
    hq, hkv, d, page = CONFIG.num_attention_heads, CONFIG.num_key_value_heads, 64, 16
    cache = KVCacheManager(4, hkv, d, 64, page, 4, device="cuda", dtype=torch.bfloat16)
    cache.key_cache.normal_()
    cache.value_cache.normal_()
    attention = cache.attention
    graph_rows = (8, 64, 200)
    planned = memory.execution_bytes(
        CONFIG, SimpleNamespace(max_num_seqs=4, max_num_batched_tokens=256), CACHE,
        execution(cuda_graphs=True, cuda_graph_max_batch_size=max(graph_rows)), 2,
    )
    graphs = GraphCache("cuda")
    inputs = {}
    for rows in graph_rows:
        q = torch.randn(rows, hq, d, device="cuda", dtype=torch.bfloat16)
        tables = torch.randint(0, 64, (rows, 4), device="cuda", dtype=torch.int32)
        lengths = torch.randint(1, 4 * page + 1, (rows,), device="cuda", dtype=torch.int32)
        inputs[rows] = (q, tables, lengths)
        graphs.capture(rows, lambda q=q, t=tables, n=lengths: attention(q, cache.key_cache[:, 0], cache.value_cache[:, 0], t, n))
    total = attention.workspace_bytes + attention.held_bytes
    assert attention.held_bytes > 0
    assert total <= planned["attention_workspace"] + planned["graph_held_workspaces"]
    for rows, (q, tables, lengths) in inputs.items():
        graph, output = graphs.get(rows)
        expect = attention(q, cache.key_cache[:, 0], cache.value_cache[:, 0], tables, lengths)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(output, expect)


class _ToyLoopedModel(torch.nn.Module):
    """prelude / recurrent / coda over the paged cache, the surface plan_cache profiles."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
        self.embed = torch.nn.Embedding(16, config.hidden_size)
        self.qkv = torch.nn.Linear(config.hidden_size, (hq + 2 * hkv) * d, bias=False)
        self.out = torch.nn.Linear(hq * d, config.hidden_size, bias=False)
        self.depths = []

    def prelude(self, tokens):
        return self.embed(tokens)

    def recurrent(self, hidden, ids, depths, positions, cache):
        c = self.config
        hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        batch = cache._prepare_batch(ids, depths, positions)
        for layer in range(c.num_hidden_layers):
            q, k, v = self.qkv(hidden).split([hq * d, hkv * d, hkv * d], dim=-1)
            n = hidden.shape[0]
            cache._write_prepared(layer, batch, k.reshape(n, hkv, d), v.reshape(n, hkv, d))
            hidden = hidden + self.out(cache._attend_prepared(layer, batch, q.reshape(n, hq, d)).reshape(n, hq * d))
        self.depths.append(depths[0])
        return hidden, None

    def coda(self, hidden):
        return hidden.float().sum(-1)


def test_a_model_without_a_probe_runs_the_profiling_pass():
    """The engine-style call plan_cache(model, cache, scheduler, execution, backend)
    profiles prelude, the recurrent pass at every depth and coda, and budgets the peak."""
    model = _ToyLoopedModel(CONFIG).to(device="cuda", dtype=torch.bfloat16)
    blocks, info = memory.plan_cache(model, CACHE, SCHED, execution(), "hip", memory_info=(8 << 30, 16 << 30))
    assert model.depths == [0, 1, 2, 3]
    # At least the temporary pool of 64 tokens x 4 depths (4 pages per depth here).
    pool = 4 * 4 * memory.bytes_per_block(CONFIG, 16, 2)
    assert info["costs"]["activation_peak"] >= pool > 0
    assert blocks >= 1


def test_bf16_per_token_prefill_fits_the_planned_workspace():
    """bf16 at head_dim 256 takes the per-token prefill path; its workspace is the planned one."""
    from vllm_rlt_amd import KVCacheManager

    wide = SimpleNamespace(**{**vars(CONFIG), "head_dim": 256})
    sched = SimpleNamespace(max_num_seqs=2, max_num_batched_tokens=32)
    planned = memory.execution_bytes(wide, sched, CACHE, execution(), 2, dtype=torch.bfloat16)["attention_workspace"]
    cache = KVCacheManager(2, 4, 256, 64, 16, 4, device="cuda", dtype=torch.bfloat16)
    cache.key_cache.normal_()
    cache.value_cache.normal_()
    q = torch.randn(32, 8, 256, device="cuda", dtype=torch.bfloat16)
    width = -(-wide.max_position_embeddings // 16)
    tables = torch.randint(0, 64, (2, width), device="cuda", dtype=torch.int32)
    lengths = torch.tensor([40, 100], device="cuda", dtype=torch.int32)
    cu = torch.tensor([0, 16, 32], device="cuda", dtype=torch.int32)
    cache.attention.prefill(q, cache.key_cache[:, 0], cache.value_cache[:, 0], tables, lengths, cu, 16)
    torch.cuda.synchronize()
    assert 0 < cache.attention.workspace_bytes <= planned
