"""AsyncState / RoutingBank / RecurrentGraphs over the HIP path (GPU).

Scenarios follow the reference's tests/test_async_state.py and
tests/test_cuda_graph.py at the level this package owns (no engine): each
asynchronously routed step must write the same pages and produce the same
attention bits as the synchronous manager path; banks are not reused before
their last GPU reader finished; graph replays match eager execution bitwise
across replays with eager work in between.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import rope

pytestmark = pytest.mark.gpu

BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32, torch.int64: torch.int64}


def bits(t):
    return t.contiguous().view(BITS[t.dtype]).cpu()


def random_bits(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    info = torch.iinfo(BITS[dtype])
    return torch.randint(info.min, info.max, shape, generator=g, dtype=torch.int64).to(BITS[dtype]).view(dtype)


# ---------------------------------------------------------------- gather / scatter
@pytest.mark.parametrize(
    "dtype,width", [(torch.bfloat16, 2048), (torch.bfloat16, 6), (torch.int64, 1), (torch.uint8, 5)]
)
def test_gather_scatter_rows_are_byte_exact(dtype, width):
    """routing.py:45-76: gather zero-fills rows >= count and out-of-range slots; scatter skips them."""
    from vllm_rlt_amd import ops

    slots_n, size, count = 11, 8, 6
    if dtype == torch.uint8:
        pool = torch.randint(0, 255, (slots_n, width), dtype=torch.uint8)
    else:
        pool = random_bits((slots_n, width), dtype, 1)
    slots = torch.tensor([3, 0, 10, 42, -1, 7, 5, 2], dtype=torch.int64)
    gpool = pool.cuda()
    out = torch.full((size, width), 99, dtype=dtype).cuda() if dtype != torch.bfloat16 else random_bits(
        (size, width), dtype, 2
    ).cuda()
    ops.gather_rows(gpool, slots.cuda(), out, count)
    torch.cuda.synchronize()
    expect = torch.zeros(size, width, dtype=dtype)
    for r in range(count):
        if 0 <= slots[r] < slots_n:
            expect[r] = pool[slots[r]]
    view = torch.int16 if dtype == torch.bfloat16 else dtype
    assert torch.equal(out.cpu().view(view), expect.view(view))
    # Scatter the gathered rows back shifted by one slot.
    values = out.clone()
    target = torch.tensor([4, 1, 9, 99, -3, 8, 0, 0], dtype=torch.int64)
    ops.scatter_rows(values, target.cuda(), gpool, count)
    torch.cuda.synchronize()
    expect_pool = pool.clone()
    for r in range(count):
        if 0 <= target[r] < slots_n:
            expect_pool[target[r]] = expect[r]
    assert torch.equal(gpool.cpu().view(view), expect_pool.view(view))


# ---------------------------------------------------------------- async routing
def manager():
    from vllm_rlt_amd import KVCacheManager

    return KVCacheManager(
        num_layers=2, num_kv_heads=2, head_dim=64, num_blocks=64, block_size=16, max_loops=4, device="cuda",
        dtype=torch.bfloat16,
    )


CONFIG = SimpleNamespace(max_position_embeddings=256, total_ut_steps=4, hidden_size=128)
SCHEDULER = SimpleNamespace(max_num_seqs=3)


class Request:
    def __init__(self, rid, hidden=None):
        self.request_id, self.hidden_state = rid, hidden


@pytest.mark.parametrize("use_uva", [True, False])
def test_async_routed_steps_match_synchronous_path(use_uva):
    from vllm_rlt_amd.async_state import AsyncState

    routed, plain = manager(), manager()
    for cache in (routed, plain):
        cache.key_cache.zero_()
        cache.value_cache.zero_()
        assert cache.allocate("a", 64, initial_tokens=20) and cache.allocate("b", 64, initial_tokens=3)
    state = AsyncState(routed, CONFIG, SCHEDULER, rows=4, use_uva=use_uva)
    hidden_a = torch.randn(CONFIG.hidden_size, dtype=torch.bfloat16, device="cuda")
    requests = [Request("a", hidden_a.clone()), Request("b")]
    g = torch.Generator().manual_seed(0)
    size = 4  # padded batch: rows 2..3 are padding
    for step in range(26):
        positions = [step, step]
        if positions[1] >= 3:  # "b" grows one page at a time (incremental allocation)
            for cache in (routed, plain):
                cache.ensure_capacity("b", positions[1] + 1)
        if step == 18:  # "a" leaves and a new request takes its slot
            state.release("a")
            for cache in (routed, plain):
                cache.free("a")
                assert cache.allocate("c", 64, initial_tokens=19)
            requests[0] = Request("c")
        ids = [r.request_id for r in requests]
        pos = [p if r.request_id != "c" else p - 18 for r, p in zip(requests, positions)]
        bank, batch = state.prepare(requests, [0, 0], pos, size, recurrent=True)
        batch = bank.transfer(batch)
        ref = plain._prepare_batch(ids, [0, 0], pos)
        for layer in range(2):
            q = torch.randn(size, 4, 64, generator=g).to(torch.bfloat16).cuda()
            k = torch.randn(size, 2, 64, generator=g).to(torch.bfloat16).cuda()
            v = torch.randn(size, 2, 64, generator=g).to(torch.bfloat16).cuda()
            routed._write_prepared(layer, batch, k, v)
            plain._write_prepared(layer, ref, k[:2], v[:2])
            out = routed._attend_prepared(layer, batch, q)
            expect = plain._attend_prepared(layer, ref, q[:2])
            assert torch.equal(bits(out[:2]), bits(expect)), (step, layer)
            assert not out[2:].any()  # padding rows read nothing
        bank.record_done()
    torch.cuda.synchronize()
    assert torch.equal(bits(routed.key_cache), bits(plain.key_cache))
    assert torch.equal(bits(routed.value_cache), bits(plain.value_cache))
    # "c" took the slot "a" released; the third slot was never used.
    assert state.slots == {"b": 1, "c": 0} and state.free == [2] and set(state.owners) == {"b", "c"}
    # Batch-order gather of the slot pool and the scatter back.
    bank, _ = state.prepare(requests, [0, 0], [0, 0], size)
    bank.transfer()
    hidden = bank.gather().clone()
    torch.cuda.synchronize()
    assert torch.equal(bits(hidden[0]), bits(state.hidden[0])) and torch.equal(bits(hidden[1]), bits(state.hidden[1]))
    assert not hidden[2:].any()
    values = torch.randn(size, CONFIG.hidden_size, generator=g).to(torch.bfloat16).cuda()
    bank.scatter(values)
    tokens = torch.arange(size, dtype=torch.int64, device="cuda") + 40
    bank.scatter(tokens, tokens=True)
    gathered = bank.gather(tokens=True)
    bank.record_done()
    torch.cuda.synchronize()
    assert torch.equal(bits(state.hidden[0]), bits(values[0])) and torch.equal(bits(state.hidden[1]), bits(values[1]))
    assert gathered.tolist() == [40, 41, 0, 0]


def test_imported_hidden_state_lands_in_its_slot():
    from vllm_rlt_amd.async_state import AsyncState

    cache = manager()
    assert cache.allocate("a", 32) and cache.allocate("b", 32)
    state = AsyncState(cache, CONFIG, SCHEDULER, rows=4)
    ha = torch.randn(CONFIG.hidden_size, dtype=torch.bfloat16, device="cuda")
    hb = torch.randn(CONFIG.hidden_size, dtype=torch.bfloat16, device="cuda")
    requests = [Request("b", hb.clone()), Request("a", ha.clone())]
    bank, _ = state.prepare(requests, [0, 0], [0, 0], 3)
    bank.transfer()
    hidden = bank.gather()
    torch.cuda.synchronize()
    assert torch.equal(bits(hidden[0]), bits(hb)) and torch.equal(bits(hidden[1]), bits(ha))
    assert not hidden[2].any()
    assert requests[0].hidden_state.data_ptr() == state.hidden[state.slots["b"]].data_ptr()
    bank.scatter(hidden[:2] * 2)
    bank.record_done()
    torch.cuda.synchronize()
    assert torch.equal(bits(state.hidden[state.slots["a"]]), bits(ha * 2))


def test_bank_is_not_reused_until_its_final_gpu_reader_finishes():
    """tests/test_async_state.py:69-97: prepare() on a wrapped-around bank waits for its readers."""
    from vllm_rlt_amd import ops
    from vllm_rlt_amd.async_state import AsyncState

    cache = manager()
    assert cache.allocate("a", 32)
    state = AsyncState(cache, CONFIG, SCHEDULER, rows=4, banks=1)
    request = Request("a")
    bank, _ = state.prepare([request], [0], [5], 1)
    bank.transfer()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(100_000_000)
        # A reader of the pinned descriptors that runs only after the delay.
        ops.build_decode_metadata(
            bank.host[:1], 1, 1, state.tables, cache.block_size, bank.slots, bank.positions, bank.lengths,
            bank.blocks, bank.offsets, bank.tables, bank.width,
        )
        bank.record_done()
    assert not bank.done.query()
    reused, _ = state.prepare([request], [0], [9], 1)  # rewrites the same pinned descriptors
    assert reused is bank and bank.done.query()
    assert int(bank.positions[0]) == 5  # the delayed reader saw the old descriptor


# ---------------------------------------------------------------- graphs
def core_fn(num_layers):
    """A recurrent core over the cache interface: per layer rotate + write, attend, update hidden."""

    def core(hidden, batch, cache):
        n = hidden.shape[0]
        for layer in range(num_layers):
            q = (hidden[:, :256].reshape(n, 4, 64) * (layer + 1)).contiguous()
            k = hidden[:, 256:384].reshape(n, 2, 64).contiguous()
            v = hidden[:, 384:512].reshape(n, 2, 64).contiguous()
            cos, sin = EMB[:n, 0], EMB[:n, 1]
            q_rot = cache._write_prepared_rotary(layer, batch, q, k, v, (cos, sin))
            out = cache._attend_prepared(layer, batch, q_rot)
            hidden = hidden + torch.cat([out.reshape(n, 256)] * 2, dim=1)
        return hidden

    return core


EMB = None


def test_graph_replay_matches_eager_bitwise():
    """tests/test_cuda_graph.py:29-72: replays equal eager execution; limits fall back."""
    global EMB
    from vllm_rlt_amd import KVCacheManager
    from vllm_rlt_amd.graphs import RecurrentGraphs

    def fresh():
        cache = KVCacheManager(
            num_layers=3, num_kv_heads=2, head_dim=64, num_blocks=96, block_size=16, max_loops=4, device="cuda",
            dtype=torch.bfloat16,
        )
        cache.key_cache.zero_()
        cache.value_cache.zero_()
        for rid in ("a", "b", "c"):
            assert cache.allocate(rid, 100)
        return cache

    cos, sin = rope.rotary_cos_sin(torch.arange(8), 64, 1_000_000.0, torch.bfloat16)
    EMB = torch.stack([cos, sin], dim=1).cuda()  # [8, 2, 64]
    graphed, eager = fresh(), fresh()
    graphs = RecurrentGraphs(core_fn(3), graphed, max_batch_size=2, max_graphs=2, max_positions=128)
    core = core_fn(3)
    g = torch.Generator().manual_seed(1)
    for step in range(6):
        ids = ["a", "b"] if step % 3 != 2 else ["a", "b", "c"]  # 3 rows exceed the graph batch limit
        pos = [step, step] if len(ids) == 2 else [step, step, 0]
        if step > 2 and len(ids) == 3:
            pos = [step, step, 1]
        hidden = torch.randn(len(ids), 512, generator=g).to(torch.bfloat16).cuda()
        gb = graphed._prepare_batch(ids, [0] * len(ids), pos)
        eb = eager._prepare_batch(ids, [0] * len(ids), pos)
        got = graphs.run(hidden, gb)
        with torch.inference_mode():
            expect = core(hidden, eb, eager)
        torch.cuda.synchronize()
        assert torch.equal(bits(got), bits(expect)), step
        # Eager work between replays (a different batch shape on the same cache) must not disturb them.
        scratch = torch.randn(64, 64, device="cuda").sum()
        assert torch.isfinite(scratch)
    assert graphs.captures == 1 and graphs.replays == 4 and graphs.fallbacks == 2
    assert torch.equal(bits(graphed.key_cache), bits(eager.key_cache))
    assert torch.equal(bits(graphed.value_cache), bits(eager.value_cache))


# ---------------------------------------------------------------- device tables
@pytest.mark.parametrize("use_uva", [True, False])
def test_device_tables_follow_growth_and_slot_reuse(use_uva):
    """The device tables hold every leased request's pages; a step ships only entries the device lacks."""
    from vllm_rlt_amd import KVCacheManager
    from vllm_rlt_amd.async_state import AsyncState

    cache = KVCacheManager(
        num_layers=1, num_kv_heads=2, head_dim=64, num_blocks=200, block_size=16, max_loops=4, device="cuda",
        dtype=torch.bfloat16, incremental_allocation=True,
    )
    state = AsyncState(cache, CONFIG, SCHEDULER, rows=4, use_uva=use_uva)
    assert cache.allocate("a", 200, initial_tokens=40) and cache.allocate("b", 200, initial_tokens=1)
    requests = {"a": Request("a"), "b": Request("b")}

    def check():
        torch.cuda.synchronize()
        for rid, slot in state.slots.items():
            for plane, table in enumerate(cache._get_allocation(rid).block_tables):
                assert state.tables[slot, plane, : len(table)].tolist() == list(table), (rid, plane)

    bank, _ = state.prepare([requests["a"], requests["b"]], [0, 1], [39, 0], 2, recurrent=True)
    assert bank.n_patches == 4 * (3 + 1)  # every plane of both tables, once
    bank.transfer()
    bank.record_done()
    check()
    for step, position in enumerate(range(1, 60, 7)):
        grew = -(-(position + 1) // 16) - len(cache._get_allocation("b").block_tables[0])
        assert cache.ensure_capacity("b", position + 1)
        bank, _ = state.prepare([requests["a"], requests["b"]], [2, 3], [39, position], 2, recurrent=True)
        assert bank.n_patches == 4 * max(grew, 0)  # only the new pages of "b"
        bank.transfer()
        bank.record_done()
        check()
    # "a" leaves; "c" takes its slot and ships its whole table.
    state.release("a")
    cache.free("a")
    assert cache.allocate("c", 100, initial_tokens=33)
    requests["c"] = Request("c")
    bank, _ = state.prepare([requests["c"], requests["b"]], [0, 0], [32, 5], 2, recurrent=True)
    assert state.slots["c"] == 0 and bank.n_patches == 4 * 3
    bank.transfer()
    bank.record_done()
    check()
    # A stale owner is refused: the same id from another request object.
    with pytest.raises(RuntimeError, match="earlier owner"):
        state.prepare([Request("c")], [0], [0], 1)


# ---------------------------------------------------------------- graphs across layouts
@pytest.mark.parametrize("layout", ["last_exited", "shared"])
def test_routed_graph_replays_match_eager_across_layouts_and_depths(layout):
    """tests/test_cuda_graph.py:29-72 (backend x async x layout): routed, padded batches at depths above 0."""
    global EMB
    from vllm_rlt_amd import KVCacheManager
    from vllm_rlt_amd.async_state import AsyncState
    from vllm_rlt_amd.graphs import RecurrentGraphs

    def fresh():
        cache = KVCacheManager(
            num_layers=3, num_kv_heads=2, head_dim=64, num_blocks=96, block_size=16, max_loops=4, device="cuda",
            dtype=torch.bfloat16, layout=layout,
        )
        cache.key_cache.zero_()
        cache.value_cache.zero_()
        for rid in ("a", "b"):
            assert cache.allocate(rid, 64)
        return cache

    cos, sin = rope.rotary_cos_sin(torch.arange(8), 64, 1_000_000.0, torch.bfloat16)
    EMB = torch.stack([cos, sin], dim=1).cuda()
    graphed, eager = fresh(), fresh()
    state = AsyncState(graphed, CONFIG, SimpleNamespace(max_num_seqs=2), rows=4)
    graphs = RecurrentGraphs(core_fn(3), graphed, max_batch_size=2, max_graphs=1, max_positions=64)
    core = core_fn(3)
    requests = [Request("a"), Request("b")]
    g = torch.Generator().manual_seed(5)
    # LAST-EXITED rows keep their own depth (their plane holds the history);
    # SHARED rows loop 1..exit on one position, then move on.
    depth = [1, 3] if layout == "last_exited" else [0, 0]
    exits, position = [2, 4], [0, 0]
    for step in range(10):
        hidden = torch.randn(2, 512, generator=g).to(torch.bfloat16).cuda()
        bank, batch = state.prepare(requests, list(depth), list(position), 4, recurrent=True)
        routed = bank.transfer(batch)  # padded to 4 rows
        got = graphs.run(hidden, routed)
        bank.record_done()
        with torch.inference_mode():
            expect = core(hidden, eager._prepare_batch(["a", "b"], list(depth), list(position)), eager)
        torch.cuda.synchronize()
        assert torch.equal(bits(got), bits(expect)), (layout, step, depth, position)
        _ = torch.randn(64, 64, device="cuda").sum().item()  # eager work between replays
        for r in range(2):
            if layout == "last_exited":
                position[r] += 1
            else:
                depth[r] += 1
                if depth[r] == exits[r]:
                    depth[r], position[r] = 0, position[r] + 1
    assert graphs.captures == 1 and graphs.replays == 10 and graphs.fallbacks == 0
    assert torch.equal(bits(graphed.key_cache), bits(eager.key_cache))
    assert torch.equal(bits(graphed.value_cache), bits(eager.value_cache))
