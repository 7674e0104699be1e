"""Workspace host logic on the CPU: row padding, addresses, tables, reuse.

The reference's Workspace (vllm_rlt/worker/buffers.py:29-96) also runs with a
CPU device (no pinned memory, plain copies), so its whole contract is
checkable here.  Write addresses and table contents are checked against the
page book's own batch plan and block tables, an independent code path.
"""

import pytest
import torch

from vllm_rlt_amd.buffers import Workspace
from vllm_rlt_amd.page_book import KVPageBook


def book(**overrides):
    values = dict(num_layers=2, num_kv_heads=1, head_dim=4, num_blocks=40, block_size=2, max_loops=3)
    values.update(overrides)
    return KVPageBook(**values)


def workspace(rows=6, width=8):
    return Workspace(rows, width, 8, "cpu", torch.float32)


def test_prepare_fills_rows_and_zero_pads_to_size():
    cache = book()
    assert cache.allocate("a", 7) and cache.allocate("b", 4)
    ws = workspace()
    ids, depths, positions = ["a", "b", "a"], [2, 0, 0], [6, 3, 1]
    batch = ws.prepare(cache, ids, depths, positions, 5)
    plan = cache._plan_batch(ids, depths, positions)
    assert batch.position_ids.tolist() == [6, 3, 1, 0, 0]
    assert batch.context_lengths.tolist() == [7, 4, 2, 0, 0]
    assert batch.write_blocks.tolist() == plan.write_blocks.tolist()
    assert batch.write_offsets.tolist() == plan.write_offsets.tolist()
    assert batch.position_ids.dtype == batch.write_blocks.dtype == batch.write_offsets.dtype == torch.int64
    assert batch.block_tables.dtype == batch.context_lengths.dtype == torch.int32
    assert batch.block_tables.shape == (5, 8)
    for i, (rid, depth) in enumerate(zip(ids, depths)):
        table = list(cache.get_block_table(rid, depth))
        assert batch.block_tables[i].tolist() == table + [0] * (8 - len(table))
    assert batch.block_tables[3:].eq(0).all()
    assert batch.writable and batch.cu_seqlens_q is None and batch.max_seqlen_q == 1
    assert [r[1:] for r in batch.rows] == [(2, 6), (0, 3), (0, 1)]
    assert dict(batch.allocations).keys() == {"a", "b"}
    cache._require_live_batch(batch)


def test_rows_of_a_larger_previous_batch_are_cleared():
    cache = book()
    assert cache.allocate("a", 7) and cache.allocate("b", 7)
    ws = workspace()
    ws.prepare(cache, ["a", "b", "a"], [0, 1, 1], [5, 6, 2], 4)
    batch = ws.prepare(cache, ["b"], [2], [0], 4)
    assert batch.position_ids.tolist() == [0, 0, 0, 0]
    assert batch.context_lengths.tolist() == [1, 0, 0, 0]
    assert batch.write_blocks.shape == (1,)
    assert batch.block_tables[1:].eq(0).all()
    table = list(cache.get_block_table("b", 2))
    assert batch.block_tables[0].tolist() == table + [0] * (8 - len(table))


def test_device_buffers_keep_their_addresses():
    cache = book()
    assert cache.allocate("a", 7)
    ws = workspace()
    first = ws.prepare(cache, ["a"], [0], [3], 2)
    second = ws.prepare(cache, ["a", "a"], [0, 1], [4, 4], 3)
    for name in ("position_ids", "write_blocks", "write_offsets", "block_tables", "context_lengths"):
        assert getattr(first, name).data_ptr() == getattr(second, name).data_ptr(), name


def test_duplicate_write_addresses_are_rejected():
    cache = book()
    assert cache.allocate("a", 7)
    ws = workspace()
    with pytest.raises(ValueError, match="duplicate KV write addresses"):
        ws.prepare(cache, ["a", "a"], [1, 1], [3, 3], 2)
    shared = book(layout="shared")
    assert shared.allocate("a", 7)
    # Every depth of a SHARED pool writes the same slot.
    with pytest.raises(ValueError, match="duplicate KV write addresses"):
        ws.prepare(shared, ["a", "a"], [0, 2], [3, 3], 2)
    batch = ws.prepare(shared, ["a", "a"], [0, 2], [3, 4], 2)
    assert batch.write_blocks.tolist() == [shared.get_block_table("a", 0)[1], shared.get_block_table("a", 0)[2]]


def test_rows_are_validated_like_the_manager():
    cache = book()
    assert cache.allocate("a", 4)
    ws = workspace()
    with pytest.raises(KeyError, match="no KV allocation"):
        ws.prepare(cache, ["zz"], [0], [0], 1)
    with pytest.raises(ValueError, match="position must be in"):
        ws.prepare(cache, ["a"], [0], [4], 1)
    with pytest.raises(ValueError, match="depth must be in"):
        ws.prepare(cache, ["a"], [3], [0], 1)
    with pytest.raises(ValueError, match="size must be in"):
        ws.prepare(cache, ["a", "a"], [0, 1], [0, 0], 1)
    with pytest.raises(ValueError, match="size must be in"):
        ws.prepare(cache, ["a"], [0], [0], 7)
    narrow = Workspace(2, 1, 8, "cpu", torch.float32)
    with pytest.raises(ValueError, match="wider than the workspace"):
        narrow.prepare(cache, ["a"], [0], [0], 1)


def test_tokens_are_zero_padded():
    ws = workspace()
    assert ws.tokens([7, 8, 9], 5).tolist() == [7, 8, 9, 0, 0]
    out = ws.tokens([4], 3)
    assert out.tolist() == [4, 0, 0] and out.dtype == torch.int64


def test_cpu_workspace_has_no_event():
    ws = workspace()
    ws.release()
    ws.acquire()
    assert ws.event is None and not ws.host["tables"].is_pinned()
