"""Workspace and PrefillMetadataBank on the GPU.

The bank's metadata must equal the manager's own packed-prefill batch field
by field for every depth (the reference's test,
tests/test_prefix_growth.py:189-224), and a Workspace batch must write and
attend exactly like the manager's prepared batch, with zero rows for padding.
"""

import random

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
FIELDS = ("position_ids", "write_blocks", "write_offsets", "block_tables", "context_lengths", "cu_seqlens_q")


def manager(*args, **kwargs):
    from vllm_rlt_amd import KVCacheManager

    return KVCacheManager(*args, device=DEV, **kwargs)


def assert_same_batch(actual, expected):
    for name in FIELDS:
        a, e = getattr(actual, name), getattr(expected, name)
        assert a.dtype == e.dtype and a.shape == e.shape, name
        assert torch.equal(a, e), name
    assert actual.max_seqlen_q == expected.max_seqlen_q
    assert [(id(a), d, p) for a, d, p in actual.rows] == [(id(a), d, p) for a, d, p in expected.rows]


def test_prefill_bank_matches_prepare_batch_and_waits_for_consumer():
    # tests/test_prefix_growth.py:189-224
    from vllm_rlt_amd import PrefillMetadataBank

    c = manager(2, 2, 64, 64, 16, 4, dtype=torch.bfloat16)
    assert c.allocate("a", 16) and c.allocate("b", 32)
    bank = PrefillMetadataBank(c)
    ids = ["a"] * 3 + ["b"] * 4
    positions = [0, 1, 2, 16, 17, 18, 19]
    tokens = [1, 2, 3, 4, 5, 6, 7]
    assert bank.prepare(ids, positions, tokens).tolist() == tokens
    for depth in range(4):
        expected = c._prepare_batch(ids, [depth] * len(ids), positions, packed_prefill=True)
        assert_same_batch(bank.metadata(depth), expected)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    saved = torch.empty_like(bank.tokens)
    with torch.cuda.stream(stream):
        torch.cuda._sleep(20_000_000)
        saved.copy_(bank.tokens)
        bank.release()
    bank.prepare(ids, positions, [9] * 7)
    assert saved.tolist() == tokens
    assert bank.tokens.tolist() == [9] * 7
    bank.release()
    torch.cuda.synchronize()


@pytest.mark.parametrize("seed", range(4))
def test_prefill_bank_random_chunks_and_buffer_growth(seed):
    from vllm_rlt_amd import PrefillMetadataBank

    rng = random.Random(seed)
    c = manager(1, 2, 128, 2048, 16, 4, dtype=torch.bfloat16)
    bank = PrefillMetadataBank(c)
    for round_ in range(3):
        ids, positions = [], []
        for s in range(rng.randint(1, 3 + 2 * round_)):
            rid = f"r{round_}.{s}"
            size = rng.randint(1, 200)
            assert c.allocate(rid, size)
            chunk = rng.randint(1, min(size, 40))
            start = rng.randint(0, size - chunk)
            ids += [rid] * chunk
            positions += list(range(start, start + chunk))
        tokens = [rng.randrange(1 << 40) for _ in ids]
        assert bank.prepare(ids, positions, torch.tensor(tokens)).tolist() == tokens
        for depth in range(4):
            expected = c._prepare_batch(ids, [depth] * len(ids), positions, packed_prefill=True)
            assert_same_batch(bank.metadata(depth), expected)
        bank.release()
    assert bank.capacity >= bank.n * 3 and bank.row_capacity >= bank.n
    torch.cuda.synchronize()


def test_prefill_bank_on_a_shared_pool_uses_the_one_plane():
    from vllm_rlt_amd import PrefillMetadataBank

    c = manager(1, 1, 64, 64, 16, 3, dtype=torch.bfloat16, layout="shared")
    assert c.allocate("a", 40)
    bank = PrefillMetadataBank(c)
    positions = list(range(5, 37))
    bank.prepare(["a"] * len(positions), positions, positions)
    expected = c._prepare_batch(["a"] * len(positions), [0] * len(positions), positions)
    for depth in range(3):
        batch = bank.metadata(depth)
        assert torch.equal(batch.write_blocks, expected.write_blocks)
        assert torch.equal(batch.write_offsets, expected.write_offsets)
        assert batch.block_tables.tolist() == [expected.block_tables[-1].tolist()]
        assert batch.context_lengths.tolist() == [37] and batch.cu_seqlens_q.tolist() == [0, 32]
    bank.release()
    torch.cuda.synchronize()


@pytest.mark.parametrize("layout", ["last_exited", "shared"])
def test_workspace_batch_writes_and_attends_like_the_manager(layout):
    from vllm_rlt_amd import Workspace

    torch.manual_seed(3)
    hkv, hq, d, page, layers = 2, 4, 128, 16, 2
    lengths = {"a": 37, "b": 70, "c": 5}
    caches = []
    for _ in range(2):
        c = manager(layers, hkv, d, 64, page, 3, dtype=torch.bfloat16, layout=layout)
        c.key_cache.zero_()  # pools start uninitialised; compare written slots only
        c.value_cache.zero_()
        for rid, n in lengths.items():
            assert c.allocate(rid, n + 1)
        caches.append(c)
    ids, depths = ["a", "b", "c"], [2, 0, 1]
    history = {rid: torch.randn(layers, n, hkv, d, device=DEV).to(torch.bfloat16) for rid, n in lengths.items()}
    for c in caches:
        for layer in range(layers):
            for rid, depth in zip(ids, depths):
                n = lengths[rid]
                h = history[rid][layer]
                c.write(layer, [rid] * n, [depth] * n, list(range(n)), h, -h)
    size = 5
    k = torch.randn(size, hkv, d, device=DEV).to(torch.bfloat16)
    v = torch.randn(size, hkv, d, device=DEV).to(torch.bfloat16)
    q = torch.randn(size, hq, d, device=DEV).to(torch.bfloat16)
    positions = [lengths[rid] for rid in ids]
    ws = Workspace(8, 16, 64, DEV, torch.bfloat16)
    ws.acquire()
    batch = ws.prepare(caches[0], ids, depths, positions, size)
    reference = caches[1]._prepare_batch(ids, depths, positions)
    for layer in range(layers):
        caches[0]._write_prepared(layer, batch, k, v)
        caches[1]._write_prepared(layer, reference, k[:3].contiguous(), v[:3].contiguous())
    assert torch.equal(caches[0].key_cache, caches[1].key_cache)
    assert torch.equal(caches[0].value_cache, caches[1].value_cache)
    for layer in range(layers):
        out = caches[0]._attend_prepared(layer, batch, q)
        expected = caches[1]._attend_prepared(layer, reference, q[:3].contiguous())
        assert torch.equal(out[:3], expected)
        assert out[3:].eq(0).all()
    ws.release()
    ws.acquire()
    assert ws.event is not None and ws.event.query()
