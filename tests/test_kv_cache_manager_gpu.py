"""KVCacheManager(backend="hip") end to end on the GPU.

Scenarios follow the reference's manager tests (cited per test); attention is
compared with the dense SDPA oracle, KV movement with exact equality.
"""

import pytest
import torch

from oracle.paged_attention import dense_attention, paged_attention_cpu

pytestmark = pytest.mark.gpu

DEV = "cuda"


def manager(**overrides):
    from vllm_rlt_amd import KVCacheManager

    values = dict(
        num_layers=2, num_kv_heads=1, head_dim=4, num_blocks=18, block_size=2, max_loops=3, device=DEV,
        dtype=torch.float32,
    )
    values.update(overrides)
    return KVCacheManager(**values)


def full(shape, value, dtype=torch.float32):
    return torch.full(shape, float(value), device=DEV, dtype=dtype)


def test_backend_and_device_are_explicit():
    from vllm_rlt_amd import KVCacheManager

    with pytest.raises(ValueError, match="backend"):
        manager(backend="automatic")
    with pytest.raises(ValueError, match="ROCm"):
        KVCacheManager(1, 1, 4, 4, 2, 2, device="cpu")
    cache = manager()
    assert cache.attention_info["backend"] == "hip"
    assert cache.bytes_per_block == 2 * 2 * 2 * 1 * 4 * 4


def test_last_exited_copies_every_layer_and_preserves_executed_depths():
    # tests/test_kv_cache.py:38-59
    cache = manager()
    assert cache.allocate("a", 4)
    for layer in range(2):
        for depth in range(2):
            keys = full((1, 1, 4), 10 * layer + depth)
            cache.write(layer, ["a"], [depth], [0], keys, keys + 100)
    cache.finalize_token("a", 0, exit_depth=1)
    for layer in range(2):
        k0, v0 = cache.read(layer, "a", 0, 1)
        k1, v1 = cache.read(layer, "a", 1, 1)
        k2, v2 = cache.read(layer, "a", 2, 1)
        assert torch.equal(k0, full((1, 1, 4), 10 * layer)) and torch.equal(v0, full((1, 1, 4), 10 * layer + 100))
        assert torch.equal(k2, k1) and torch.equal(v2, v1)
    # Physical copies: a later write at depth 1 leaves depth 2 alone.
    cache.write(0, ["a"], [1], [0], full((1, 1, 4), 0), full((1, 1, 4), 0))
    assert torch.equal(cache.read(0, "a", 2, 1)[0], full((1, 1, 4), 1))


def test_early_exit_then_later_token_loops_deeper_across_block_boundary():
    # tests/test_kv_cache.py:61-78: q = 0 reads the mean of 100 + 10p + min(p, depth) + layer.
    cache = manager()
    assert cache.allocate("a", 3)
    for position, exit_depth in [(0, 0), (1, 1), (2, 2)]:
        for depth in range(exit_depth + 1):
            for layer in range(2):
                keys = full((1, 1, 4), position * 10 + depth + layer)
                cache.write(layer, ["a"], [depth], [position], keys, keys + 100)
                attended = cache.attend(layer, ["a"], [depth], [position], torch.zeros(1, 2, 4, device=DEV))
                mean = sum(100 + p * 10 + min(p, depth) + layer for p in range(position + 1)) / (position + 1)
                torch.testing.assert_close(attended, full((1, 2, 4), mean), atol=1e-5, rtol=1e-5)
        cache.finalize_token("a", position, exit_depth)
    assert cache.read(0, "a", 2)[0].shape == (3, 1, 4)


def test_block_reuse_never_exposes_stale_request_history():
    # tests/test_kv_cache.py:80-95
    cache = manager(num_blocks=6)
    assert cache.allocate("old", 4)
    cache.write(0, ["old"] * 4, [0] * 4, list(range(4)), full((4, 1, 4), 7), full((4, 1, 4), 7))
    cache.free("old")
    assert cache.allocate("new", 4)
    with pytest.raises(RuntimeError, match="uninitialized"):
        cache.attend(0, ["new"], [0], [0], torch.ones(1, 1, 4, device=DEV))
    cache.write(0, ["new"], [0], [0], full((1, 1, 4), 0), full((1, 1, 4), 1))
    torch.testing.assert_close(cache.attend(0, ["new"], [0], [0], full((1, 1, 4), 0)), full((1, 1, 4), 1))
    with pytest.raises(RuntimeError, match="uninitialized"):
        cache.read(0, "new", 0, 2)


def test_validation_happens_before_mutation():
    # tests/test_kv_cache.py:97-114
    cache = manager()
    cache.allocate("a", 3)
    k = torch.ones(2, 1, 4, device=DEV)
    with pytest.raises(ValueError, match="position"):
        cache.write(0, ["a", "a"], [0, 0], [0, 3], k, k)
    assert cache.read(0, "a", 0)[0].shape[0] == 0
    with pytest.raises(ValueError, match="duplicate"):
        cache.write(0, ["a", "a"], [0, 0], [0, 0], k, k)
    with pytest.raises(RuntimeError, match="every layer"):
        cache.finalize_token("a", 0, 0)
    with pytest.raises(ValueError, match="one-dimensional integer"):
        cache.write(0, ["a"], [0], torch.tensor([0.5]), k[:1], k[:1])
    with pytest.raises(ValueError, match="depth"):
        cache.get_block_table("a", 3)
    with pytest.raises(ValueError, match="dtype"):
        cache.write(0, ["a"], [0], [0], k[:1].half(), k[:1].half())


def test_out_of_order_writes_only_expose_complete_prefix():
    # tests/test_kv_cache.py:116-128
    cache = manager()
    cache.allocate("a", 4)
    k = torch.arange(16, dtype=torch.float32, device=DEV).reshape(4, 1, 4)
    cache.write(0, ["a", "a"], [0, 0], [3, 1], k[[3, 1]], k[[3, 1]])
    assert cache.read(0, "a", 0)[0].shape[0] == 0
    cache.write(0, ["a"], [0], [0], k[:1], k[:1])
    assert torch.equal(cache.read(0, "a", 0)[0], k[:2])
    with pytest.raises(RuntimeError, match="uninitialized"):
        cache.attend(0, ["a"], [0], [3], torch.zeros(1, 1, 4, device=DEV))
    cache.write(0, ["a"], [0], [2], k[2:3], k[2:3])
    assert torch.equal(cache.read(0, "a", 0)[0], k)


def mixed_batch_case(dtype, head_dim):
    # tests/test_attention.py:30-55: fragmented tables, two requests, three depths, GQA 3.
    torch.manual_seed(48)
    cache = manager(num_layers=2, num_kv_heads=2, head_dim=head_dim, num_blocks=48, block_size=3, max_loops=3, dtype=dtype)
    cache.allocate("retained", 4)
    cache.allocate("hole", 8)
    cache.allocate("a", 7)
    cache.free("hole")
    cache.allocate("b", 6)
    histories = {}
    for request_id, length in [("a", 7), ("b", 6)]:
        for depth in range(3):
            k = torch.randn(length, 2, head_dim, device=DEV, dtype=dtype) + depth * 0.5
            v = torch.randn_like(k) + (4 if request_id == "a" else -4)
            cache.write(1, [request_id] * length, [depth] * length, list(range(length)), k, v)
            histories[request_id, depth] = k, v
    ids, depths, positions = ["a", "b", "a", "b"], [2, 0, 1, 2], [6, 4, 2, 5]
    q = torch.randn(4, 6, head_dim, device=DEV, dtype=dtype)
    actual = cache.attend(1, ids, depths, positions, q)
    expected = torch.stack(
        [
            dense_attention(q[r].cpu(), histories[i, d][0][: p + 1].cpu(), histories[i, d][1][: p + 1].cpu())
            for r, (i, d, p) in enumerate(zip(ids, depths, positions))
        ]
    )
    return actual.cpu(), expected


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [7, 32, 64, 128])
def test_mixed_depth_and_request_batch_matches_dense(dtype, head_dim):
    actual, expected = mixed_batch_case(dtype, head_dim)
    tol = {torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float32: 2e-5}[dtype]
    torch.testing.assert_close(actual, expected, atol=tol, rtol=tol)


def test_empty_batch_and_invalid_gqa():
    # tests/test_attention.py:99-107
    cache = manager(num_layers=1, num_kv_heads=2, head_dim=4, num_blocks=6, block_size=2, max_loops=2)
    empty = torch.empty(0, 2, 4, device=DEV)
    cache.write(0, [], [], [], empty, empty)
    assert cache.attend(0, [], [], [], torch.empty(0, 4, 4, device=DEV)).shape == (0, 4, 4)
    cache.allocate("a", 1)
    cache.write(0, ["a"], [0], [0], torch.ones(1, 2, 4, device=DEV), torch.ones(1, 2, 4, device=DEV))
    with pytest.raises(ValueError, match="positive multiple"):
        cache.attend(0, ["a"], [0], [0], torch.ones(1, 3, 4, device=DEV))


def test_fragmented_mixed_depth_rows_and_untouched_pages():
    # tests/test_prepared_kv.py:30-81: prepared once, used by every layer; other pages bit-identical.
    torch.manual_seed(71)
    cache = manager(num_layers=3, num_kv_heads=1, head_dim=4, num_blocks=36, block_size=2, max_loops=4)
    for name, size in (("left", 4), ("protected", 2), ("right", 4)):
        assert cache.allocate(name, size)
    cache.key_cache.fill_(-99)
    cache.value_cache.fill_(-98)
    cache.free("left")
    cache.free("right")
    assert cache.allocate("a", 5) and cache.allocate("b", 3)
    ids = ["a"] * 10 + ["b"] * 3
    depths = [0] * 5 + [3] * 5 + [1] * 3
    positions = list(range(5)) * 2 + list(range(3))
    batch = cache._prepare_batch(ids, depths, positions)
    keys = torch.randn(13, 1, 4, device=DEV)
    values = torch.randn(13, 1, 4, device=DEV)
    query = torch.randn(13, 2, 4, device=DEV)
    protected = [p for t in cache._allocations["protected"].block_tables for p in t]
    before = cache.key_cache[protected].clone(), cache.value_cache[protected].clone()
    for layer in range(cache.num_layers):
        layer_values = values + layer
        cache._write_prepared(layer, batch, keys, layer_values)
        actual = cache._attend_prepared(layer, batch, query)
        for row, (name, depth, position) in enumerate(zip(ids, depths, positions)):
            sel = [i for i, addr in enumerate(zip(ids, depths, positions)) if addr[:2] == (name, depth) and addr[2] <= position]
            expect = dense_attention(query[row].cpu(), keys[sel].cpu(), layer_values[sel].cpu())
            torch.testing.assert_close(actual[row].cpu(), expect, atol=1e-5, rtol=1e-5)
    assert torch.equal(cache.key_cache[protected], before[0])
    assert torch.equal(cache.value_cache[protected], before[1])


@pytest.mark.parametrize("operation", ["write", "attend"])
@pytest.mark.parametrize("stale_kind", ["free", "same_id_reallocation", "wrong_manager"])
def test_stale_batches_cannot_access_recycled_pages(operation, stale_kind):
    # tests/test_prepared_kv.py:100-130
    cache = manager(num_layers=3, num_blocks=8, max_loops=4)
    cache.allocate("a", 4)
    batch = cache._prepare_batch(["a"], [0], [0])
    if stale_kind == "wrong_manager":
        target = manager(num_layers=3, num_blocks=8, max_loops=4)
        target.allocate("a", 4)
    else:
        target = cache
        cache.free("a")
        if stale_kind == "same_id_reallocation":
            cache.allocate("a", 4)
    target.key_cache.fill_(17)
    target.value_cache.fill_(19)
    before = target.key_cache.clone(), target.value_cache.clone()
    tensor = torch.ones(1, 1, 4, device=DEV)
    with pytest.raises((ValueError, RuntimeError), match="different cache|stale"):
        if operation == "write":
            target._write_prepared(0, batch, tensor, tensor)
        else:
            target._attend_prepared(0, batch, tensor)
    torch.cuda.synchronize()
    assert torch.equal(target.key_cache, before[0]) and torch.equal(target.value_cache, before[1])


def test_duplicate_query_rows_remain_valid_but_never_authorize_writes():
    # tests/test_prepared_kv.py:165-179
    cache = manager(num_layers=3, num_blocks=36, max_loops=4)
    cache.allocate("a", 2)
    k, v = torch.ones(1, 1, 4, device=DEV), full((1, 1, 4), 3)
    cache.write(0, ["a"], [0], [0], k, v)
    q = torch.zeros(2, 2, 4, device=DEV)
    batch = cache._prepare_batch(["a", "a"], [0, 0], [0, 0], for_write=False)
    torch.testing.assert_close(cache._attend_prepared(0, batch, q), full((2, 2, 4), 3))
    with pytest.raises(ValueError, match="read-only"):
        cache._write_prepared(0, batch, k.expand(2, -1, -1), v.expand(2, -1, -1))
    with pytest.raises(ValueError, match="duplicate"):
        cache.write(0, ["a", "a"], [0, 0], [0, 0], k.expand(2, -1, -1), v.expand(2, -1, -1))


def test_shared_overwrites_one_plane():
    # tests/test_cdb_runtime.py:152-177: each depth reads [1, 13, 20].
    cache = manager(num_layers=2, num_kv_heads=1, head_dim=4, num_blocks=4, block_size=2, max_loops=4, layout="shared")
    cache.allocate("a", 3)
    for pos, exit_depth in [(0, 1), (1, 3), (2, 0)]:
        for depth in range(exit_depth + 1):
            for layer in range(2):
                value = full((1, 1, 4), pos * 10 + depth + layer)
                cache.write(layer, ["a"], [depth], [pos], value, value + 100)
        cache.finalize_token("a", pos, exit_depth)
    for depth in range(4):
        assert cache.read(0, "a", depth)[0][:, 0, 0].tolist() == [1, 13, 20]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_packed_prefill_through_the_manager(dtype):
    # tests/test_flash_attention.py:148-190: ragged prefixes, unequal depths, fragmented pages.
    torch.manual_seed(712)
    cache = manager(num_layers=2, num_kv_heads=2, head_dim=64, num_blocks=80, block_size=16, max_loops=4, dtype=dtype)
    for rid in ["hole", "a", "b", "c"]:
        cache.allocate(rid, 65)
    cache.free("hole")
    ids, depths, positions = [], [], []
    for rid, depth, prefix, count in [("a", 0, 0, 19), ("b", 2, 17, 7), ("c", 3, 31, 18)]:
        for layer in range(2):
            if prefix:
                kv = torch.randn(prefix, 2, 64, device=DEV, dtype=dtype)
                cache.write(layer, [rid] * prefix, [depth] * prefix, list(range(prefix)), kv, -kv)
        ids.extend([rid] * count)
        depths.extend([depth] * count)
        positions.extend(range(prefix, prefix + count))
    batch = cache._prepare_batch(ids, depths, positions, packed_prefill=True)
    flat = cache._prepare_batch(ids, depths, positions)
    assert batch.block_tables.shape[0] == 3 and flat.block_tables.shape[0] == len(ids)
    for layer in range(2):
        k = torch.randn(len(ids), 2, 64, device=DEV, dtype=dtype)
        v = torch.randn_like(k)
        q = torch.randn(len(ids), 4, 64, device=DEV, dtype=dtype)
        cache._write_prepared(layer, batch, k, v)
        expected = paged_attention_cpu(
            q.cpu(), cache.key_cache[:, layer].cpu(), cache.value_cache[:, layer].cpu(),
            flat.block_tables.cpu(), flat.context_lengths.cpu(),
        )
        actual = cache._attend_prepared(layer, batch, q)
        atol = 0.015 if dtype == torch.bfloat16 else 0.002
        torch.testing.assert_close(actual.cpu(), expected, atol=atol, rtol=0.02)


def test_prefix_aliased_pages_are_shared_and_never_written():
    # Aliased prefix pages (tests/test_prefix_growth.py:47-64) are read by both
    # requests and stay bit-identical while the suffixes are appended.
    from vllm_rlt_amd import KVCacheManager

    cache = KVCacheManager(2, 2, 64, 64, 16, 2, device=DEV, dtype=torch.bfloat16, enable_prefix_caching=True)
    prompt = list(range(100, 150))
    assert cache.allocate("a", 64)
    torch.manual_seed(5)
    for layer in range(2):
        for depth in range(2):
            kv = torch.randn(50, 2, 64, device=DEV, dtype=torch.bfloat16)
            cache.write(layer, ["a"] * 50, [depth] * 50, list(range(50)), kv, kv * 0.5)
    cache.publish_prefix("a", prompt, 50)
    hit = cache.lookup_prefix(prompt)
    assert len(hit) == 3  # 48 tokens: full pages of tokens[:49]
    assert cache.allocate("b", 64, prefix=hit)
    shared = [p for group in hit for p in group]
    before = cache.key_cache[shared].clone(), cache.value_cache[shared].clone()
    for layer in range(2):
        for depth in range(2):
            kv = torch.randn(4, 2, 64, device=DEV, dtype=torch.bfloat16)
            cache.write(layer, ["b"] * 4, [depth] * 4, list(range(48, 52)), kv, kv)
    q = torch.randn(2, 2, 64, device=DEV, dtype=torch.bfloat16)
    out = cache.attend(1, ["a", "b"], [1, 1], [47, 47], q)
    # Both requests see the same 48-token prefix through different tables.
    torch.testing.assert_close(out[0], cache.attend(1, ["b"], [1], [47], q[:1])[0], atol=0, rtol=0)
    torch.testing.assert_close(out[1], cache.attend(1, ["a"], [1], [47], q[1:])[0], atol=0, rtol=0)
    assert torch.equal(cache.key_cache[shared], before[0]) and torch.equal(cache.value_cache[shared], before[1])


def test_device_cache_graph_replays_match_eager():
    # worker/cuda_graph.py:105-121 contract: a captured 2-layer write+attend
    # replays to the eager result every time (several replays, eager work between).
    from vllm_rlt_amd import DeviceCache, KVCacheManager

    cache = KVCacheManager(2, 4, 128, 96, 16, 2, device=DEV, dtype=torch.bfloat16)
    for rid in ("a", "b", "c"):
        assert cache.allocate(rid, 200)
    torch.manual_seed(9)
    for layer in range(2):
        for rid, n in (("a", 37), ("b", 120), ("c", 5)):
            kv = torch.randn(n, 4, 128, device=DEV, dtype=torch.bfloat16)
            cache.write(layer, [rid] * n, [1] * n, list(range(n)), kv, -kv)
    batch = cache._prepare_batch(["a", "b", "c"], [1, 1, 1], [37, 120, 5])
    k = torch.randn(3, 4, 128, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(3, 8, 128, device=DEV, dtype=torch.bfloat16)
    proxy = DeviceCache(cache)

    def core():
        outs = []
        for layer in range(2):
            proxy._write_prepared(layer, batch, k + layer, k - layer)
            outs.append(proxy._attend_prepared(layer, batch, q))
        return torch.stack(outs)

    eager = core().clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        core()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = core()
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(captured, eager, atol=0, rtol=0)
        _ = (q * 2).sum().item()  # unrelated eager work between replays
