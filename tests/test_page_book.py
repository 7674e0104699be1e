"""Host bookkeeping of the paged pool (CPU only): allocation, prefix sharing, batch plans.

Scenarios and golden values follow the reference's own tests (cited per test).
"""

import hashlib
import struct

import pytest
import torch

from vllm_rlt_amd.page_book import KVPageBook, WrittenPrefix


def book(**overrides):
    values = dict(num_layers=2, num_kv_heads=1, head_dim=4, num_blocks=18, block_size=2, max_loops=3)
    values.update(overrides)
    return KVPageBook(**values)


class PackedBook(KVPageBook):
    """A book whose attention backend accepts packed prefill."""

    def _supports_packed_prefill(self):
        return True


def test_admission_is_atomic_and_counts_all_depths():
    # tests/test_kv_cache.py:15-36
    cache = book(num_blocks=12)
    assert cache.required_blocks(3) == 6
    assert cache.allocate("a", 3)
    assert cache.num_used_blocks == 6
    assert not cache.allocate("b", 5)
    assert cache.num_used_blocks == 6
    with pytest.raises(ValueError, match="pool has"):
        cache.allocate("impossible", 9)
    with pytest.raises(ValueError, match="already owns"):
        cache.allocate("a", 3)
    assert cache.allocate("b", 4)
    assert cache.num_free_blocks == 0
    cache.free("never-admitted")
    cache.free("a")
    cache.free("a")
    assert cache.num_free_blocks == 6
    assert cache.allocate("c", 4)
    c_pages = {p for d in range(3) for p in cache.get_block_table("c", d)}
    b_pages = {p for d in range(3) for p in cache.get_block_table("b", d)}
    assert c_pages.isdisjoint(b_pages)


def test_first_pages_come_in_order_and_planes_split_the_claim():
    # The free stack pops 0, 1, 2, ... and plane d gets claimed[d*tail:(d+1)*tail] (:137, :278-281).
    cache = book(num_blocks=18)
    assert cache.allocate("a", 3)
    assert [cache.get_block_table("a", d) for d in range(3)] == [(0, 1), (2, 3), (4, 5)]
    cache.free("a")
    # Freed pages are pushed table by table, each table reversed (1, 0, 3, 2, 5, 4), so the
    # next claim pops 4, 5, 2.
    assert cache.allocate("b", 1)
    assert [cache.get_block_table("b", d) for d in range(3)] == [(4,), (5,), (2,)]


def test_shared_layout_uses_one_plane_and_reclaims_it_once():
    # tests/test_cdb_runtime.py:152-177 (bookkeeping part)
    cache = book(num_blocks=4, max_loops=4, layout="shared")
    assert cache.required_blocks(3) == 2
    cache.allocate("a", 3)
    assert cache.get_block_table("a", 0) == cache.get_block_table("a", 3)
    cache.free("a")
    cache.free("a")
    assert cache.num_free_blocks == 4
    assert len(set(cache._free_blocks)) == 4


def test_prefix_refcounts_and_eviction():
    # tests/test_prefix_growth.py:47-64
    c = KVPageBook(1, 1, 4, 12, 2, 2, enable_prefix_caching=True)
    assert c.allocate("a", 5)
    c.mark_imported_prefix("a", 5)
    c.publish_prefix("a", [1, 2, 3, 4, 5], 5)
    hit = c.lookup_prefix([1, 2, 3, 4, 9])
    assert c.allocate("b", 5, prefix=hit)
    a = c._get_allocation("a").block_tables
    b = c._get_allocation("b").block_tables
    assert a[0][:2] == b[0][:2]
    c.free("a")
    assert c._refs[b[0][0]] == 2  # the cache entry and the live request
    c.free("b")
    assert c.num_free_blocks == 12
    assert c.allocate("all", 12)
    assert not c.lookup_prefix([1, 2, 3, 4, 5])
    c.free("all")
    assert c.num_free_blocks == 12


def test_prefix_keys_are_chained_sha256_of_full_pages():
    # kv_cache_manager.py:194-199: digest_i = sha256(digest_{i-1} || int64le(page_i tokens)).
    c = KVPageBook(1, 1, 4, 12, 4, 2, enable_prefix_caching=True)
    tokens = [5, 6, 7, 8, 9, 10, 11, 12, 13]
    first = hashlib.sha256(struct.pack("<4q", 5, 6, 7, 8)).digest()
    second = hashlib.sha256(first + struct.pack("<4q", 9, 10, 11, 12)).digest()
    assert list(c._index.keys(tokens)) == [first, second]
    # A partial last page has no key; a prefix of the tokens shares its keys.
    assert list(c._index.keys(tokens[:7])) == [first]
    assert list(c._index.keys(tokens[:3])) == []


def test_prefix_publication_needs_every_plane_and_layer_written():
    c = KVPageBook(2, 1, 4, 16, 2, 2, enable_prefix_caching=True)
    c.allocate("a", 6)
    alloc = c._get_allocation("a")
    for plane in alloc.written:
        for w in plane:
            for p in range(4):
                w.add(p)
    alloc.written[1][1] = WrittenPrefix(prefix=2)  # one (plane, layer) only has the first page
    c.publish_prefix("a", [1, 2, 3, 4, 5, 6], 6)
    assert len(c.lookup_prefix([1, 2, 3, 4, 5, 6])) == 1
    # Aliased prefix pages are shared by reference in the new request's tables, per plane.
    hit = c.lookup_prefix([1, 2, 3, 4, 5, 6])
    c.allocate("b", 6, prefix=hit)
    assert [t[0] for t in c._get_allocation("b").block_tables] == [t[0] for t in alloc.block_tables]
    assert c._get_allocation("b").written[0][0].prefix == 2


def test_incremental_growth_and_transfer_leases():
    c = book(num_blocks=18)
    assert c.allocate("a", 8, initial_tokens=2)
    assert [len(c.get_block_table("a", d)) for d in range(3)] == [1, 1, 1]
    assert c.ensure_capacity("a", 5)
    assert [len(c.get_block_table("a", d)) for d in range(3)] == [3, 3, 3]
    with pytest.raises(ValueError, match="logical capacity"):
        c.ensure_capacity("a", 9)
    c.pin_transfer("a", "t1")
    c.free("a")
    assert "a" in c._allocations  # deferred while the transfer holds the pages
    with pytest.raises(RuntimeError, match="scheduled for release"):
        c.pin_transfer("a", "t2")
    c.unpin_transfer("a", "t1")
    assert "a" not in c._allocations and c.num_free_blocks == 18


def test_written_prefix_exposes_only_the_contiguous_run():
    w = WrittenPrefix()
    for p in (3, 1):
        w.add(p)
    assert w.prefix == 0 and 3 in w and 2 not in w
    w.add(0)
    assert w.prefix == 2
    w.add(2)
    assert w.prefix == 4 and not w.pending


def test_prepared_metadata_shapes_dtypes_and_padding():
    # tests/test_prepared_kv.py:30-53
    cache = book(num_layers=3, num_blocks=36, max_loops=4)
    for name, size in (("left", 4), ("protected", 2), ("right", 4)):
        assert cache.allocate(name, size)
    cache.free("left")
    cache.free("right")
    assert cache.allocate("a", 5) and cache.allocate("b", 3)
    assert any(t != tuple(range(t[0], t[0] + len(t))) for t in cache._allocations["a"].block_tables)
    ids = ["a"] * 10 + ["b"] * 3
    depths = [0] * 5 + [3] * 5 + [1] * 3
    positions = list(range(5)) * 2 + list(range(3))
    batch = cache._prepare_batch(ids, depths, positions)
    assert len(batch.allocations) == 2
    assert batch.block_tables.shape == (13, 3)
    assert batch.block_tables.dtype == batch.context_lengths.dtype == torch.int32
    assert batch.position_ids.dtype == batch.write_blocks.dtype == batch.write_offsets.dtype == torch.int64
    assert batch.block_tables[-1, -1].item() == -1
    expected = [cache.get_block_table(i, d)[p // 2] for i, d, p in zip(ids, depths, positions)]
    assert batch.write_blocks.tolist() == expected
    assert batch.write_offsets.tolist() == [p % 2 for p in positions]
    assert batch.context_lengths.tolist() == [p + 1 for p in positions]


def test_packed_prefill_metadata_groups_queries_and_rejects_gaps():
    # tests/test_flash_attention.py:122-142
    cache = PackedBook(1, 1, 8, 32, 4, 2)
    cache.allocate("a", 20)
    cache.allocate("b", 20)
    batch = cache._prepare_batch(["a"] * 3 + ["b"] * 2, [0] * 3 + [1] * 2, [7, 8, 9, 3, 4], packed_prefill=True)
    assert batch.block_tables.shape == (2, 3)
    assert batch.context_lengths.tolist() == [10, 5]
    assert batch.cu_seqlens_q.tolist() == [0, 3, 5]
    assert batch.max_seqlen_q == 3
    assert batch.position_ids.tolist() == [7, 8, 9, 3, 4]
    assert len(batch.write_blocks) == 5
    with pytest.raises(ValueError, match="contiguous"):
        cache._prepare_batch(["a", "a"], [0, 0], [1, 3], packed_prefill=True)
    with pytest.raises(ValueError, match="one sequence"):
        cache._prepare_batch(["a", "b", "a"], [0, 0, 0], [1, 1, 2], packed_prefill=True)
    with pytest.raises(ValueError, match="packed prefill requires"):
        book()._prepare_batch([], [], [], packed_prefill=True)


@pytest.mark.parametrize(
    "ids,depths,positions,exception",
    [
        (["a"], [0], [True], ValueError),
        (["a"], [0], [0.5], ValueError),
        (["a"], [0], [2], ValueError),
        (["a"], [3], [0], ValueError),
        (["a"], [], [0], ValueError),
        (["missing"], [0], [0], KeyError),
        (["a"], [0], torch.tensor([[0]]), ValueError),
        (["a"], [0], torch.tensor([0.0]), ValueError),
    ],
)
def test_invalid_rows_are_rejected(ids, depths, positions, exception):
    # tests/test_prepared_kv.py:182-206 (the host half)
    cache = book()
    cache.allocate("a", 2)
    with pytest.raises(exception):
        cache._prepare_batch(ids, depths, positions)


def test_duplicate_write_addresses_and_read_only_duplicates():
    cache = book()
    cache.allocate("a", 3)
    with pytest.raises(ValueError, match="duplicate"):
        cache._prepare_batch(["a", "a"], [0, 0], [0, 0])
    batch = cache._prepare_batch(["a", "a"], [0, 0], [0, 0], for_write=False)
    assert not batch.writable and len(batch.rows) == 2


@pytest.mark.parametrize("stale_kind", ["free", "same_id_reallocation", "wrong_manager"])
def test_stale_batches_are_detected(stale_kind):
    # tests/test_prepared_kv.py:100-130 (the ownership check)
    cache = book(num_blocks=9)
    cache.allocate("a", 4)
    batch = cache._prepare_batch(["a"], [0], [0])
    target = cache
    if stale_kind == "wrong_manager":
        target = book(num_blocks=9)
        target.allocate("a", 4)
    else:
        cache.free("a")
        if stale_kind == "same_id_reallocation":
            cache.allocate("a", 4)
    with pytest.raises((ValueError, RuntimeError), match="different cache|stale"):
        target._require_live_batch(batch)


def test_other_requests_do_not_invalidate_a_live_batch():
    # tests/test_prepared_kv.py:133-142 (the ownership check)
    cache = book()
    cache.allocate("a", 2)
    cache.allocate("b", 2)
    batch = cache._prepare_batch(["a"], [0], [0])
    cache.free("b")
    cache.allocate("replacement", 2)
    cache._require_live_batch(batch)


def test_imported_prefix_marks_every_plane_and_layer():
    c = book()
    c.allocate("a", 6)
    c.mark_imported_prefix("a", 4)
    assert all(w.prefix == 4 for plane in c._get_allocation("a").written for w in plane)
    with pytest.raises(RuntimeError, match="already initialized"):
        c.mark_imported_prefix("a", 4)
    with pytest.raises(ValueError, match="imported prefix"):
        c.mark_imported_prefix("a", 7, start=4)
