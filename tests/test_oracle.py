"""Pin the CPU oracle before trusting it (CPU only).

Attention is checked against textbook SDPA, an independent float64 numpy
evaluation and the reference's own known answers; the byte/integer
restatements against the golden vectors the reference's tests hold.  The
mutation tests at the end plant plausible mistakes in copies of the oracle
and show that these checks catch them.
"""

import math

import numpy as np
import pytest
import torch

from oracle import kv_ops
from oracle.paged_attention import dense_attention, paged_attention_cpu, paged_attention_f64
from paged_cases import random_decode_case


def single_page_case(keys, values, query, page=16):
    """One row, scalar head (d=1, so the 1/sqrt(d) scale is 1), one page per 16 tokens."""
    n = len(keys)
    blocks = (n + page - 1) // page
    kc = torch.zeros(blocks, page, 1, 1, dtype=torch.float64)
    vc = torch.zeros_like(kc)
    for t in range(n):
        kc[t // page, t % page, 0, 0] = keys[t]
        vc[t // page, t % page, 0, 0] = values[t]
    q = torch.tensor([[[query]]], dtype=torch.float64)
    tables = torch.arange(blocks, dtype=torch.int32)[None]
    return q.float(), kc.float(), vc.float(), tables, torch.tensor([n], dtype=torch.int32)


def test_worked_examples_from_kv_layout_note():
    # docs/kv_layout_computation.md:62-85: LAST_EXITED loop 1 reads A(1,10), B(1,30) -> 20.
    out = paged_attention_cpu(*single_page_case([1, 1], [10, 30], 1.0))
    assert out.item() == pytest.approx(20.0, abs=1e-5)
    # :90-109: SHARED loop 1 reads A(2,20), B(1,30) -> 22.6894.
    out = paged_attention_cpu(*single_page_case([2, 1], [20, 30], 1.0))
    assert out.item() == pytest.approx(22.6894, abs=1e-4)
    # :152-178: SHARED loop 2, q = k_B = h/20, v_B = h with h the previous output -> 20.73.
    h = out.item()
    out2 = paged_attention_cpu(*single_page_case([2, h / 20], [20, h], h / 20))
    assert out2.item() == pytest.approx(20.73, abs=5e-3)


def test_uniform_query_reads_the_mean_of_values():
    # tests/test_kv_cache.py:61-78: q = 0 gives uniform weights, i.e. the mean of V.
    case = random_decode_case([1, 5, 17, 33, 64], hq=4, hkv=2, d=8, page=4, dtype=torch.float32, seed=3)
    q = torch.zeros_like(case.q)
    out = paged_attention_cpu(q, case.key_slice, case.value_slice, case.tables, case.lengths)
    for row, n in enumerate(case.lengths.tolist()):
        t = torch.arange(n)
        vals = case.value_slice[case.tables[row, t // 4].long(), t % 4]  # [n, hkv, d]
        mean = vals.double().mean(0).repeat_interleave(2, dim=0)
        torch.testing.assert_close(out[row].double(), mean, atol=1e-6, rtol=1e-6)


def test_empty_rows_are_zero():
    # vllm_rlt/kernels/paged_attention.py:25-27 and tests/test_flash_attention.py:70.
    case = random_decode_case([0, 3, 0], hq=2, hkv=2, d=4, page=2, dtype=torch.float32, seed=1)
    out = paged_attention_cpu(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0
    assert torch.isfinite(out[1]).all()


@pytest.mark.parametrize("d", [7, 32])
@pytest.mark.parametrize("group", [1, 3])
def test_matches_dense_sdpa_and_float64(d, group):
    # Fragmented tables, ragged lengths, GQA (tests/test_attention.py:30-55 geometry).
    case = random_decode_case([7, 1, 6, 3, 16, 9], hq=2 * group, hkv=2, d=d, page=3, dtype=torch.float32, seed=48)
    out = paged_attention_cpu(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    f64 = paged_attention_f64(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    np.testing.assert_allclose(out.double().numpy(), f64, atol=2e-6, rtol=2e-5)
    for row, n in enumerate(case.lengths.tolist()):
        t = torch.arange(n)
        pages = case.tables[row, t // 3].long()
        expected = dense_attention(case.q[row], case.key_slice[pages, t % 3], case.value_slice[pages, t % 3])
        torch.testing.assert_close(out[row], expected, atol=2e-5, rtol=2e-5)


def test_online_softmax_geometry_scaled_inputs():
    # tests/test_attention.py:63-79: x8-scaled q/k, 71 tokens, page 5, several lengths.
    g = torch.Generator().manual_seed(89)
    k = torch.randn(71, 1, 32, generator=g) * 8
    v = torch.randn(71, 1, 32, generator=g)
    q = torch.randn(4, 2, 32, generator=g) * 8
    blocks = torch.randperm(15, generator=g)
    kc = torch.zeros(15, 5, 1, 32)
    vc = torch.zeros(15, 5, 1, 32)
    t = torch.arange(71)
    kc[blocks[t // 5], t % 5] = k
    vc[blocks[t // 5], t % 5] = v
    positions = [0, 31, 32, 70]
    tables = blocks.to(torch.int32).repeat(4, 1)
    out = paged_attention_cpu(q, kc, vc, tables, torch.tensor([p + 1 for p in positions], dtype=torch.int32))
    for row, p in enumerate(positions):
        torch.testing.assert_close(out[row], dense_attention(q[row], k[: p + 1], v[: p + 1]), atol=2e-4, rtol=2e-4)


def test_bf16_rounding_of_the_output():
    # The oracle rounds fp32 results to the storage dtype once, at the end.
    case = random_decode_case([40, 17], hq=4, hkv=4, d=16, page=16, dtype=torch.bfloat16, seed=5)
    out = paged_attention_cpu(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    f64 = paged_attention_f64(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    assert out.dtype == torch.bfloat16
    rounded = torch.from_numpy(f64).float().to(torch.bfloat16)
    # fp32 accumulation may flip a rounding boundary, never more than one bf16 ulp.
    ulp = (rounded.float().abs() * 2**-7).clamp_min(2**-133)
    assert ((out.float() - rounded.float()).abs() <= ulp + 1e-6).all()


# ---------------------------------------------------------------------------
# Byte/integer restatements.


def test_append_then_gather_shared_plane_golden():
    # tests/test_cdb_runtime.py:152-177: SHARED, page 2, 4 loops; (pos, exit) = (0,1), (1,3), (2,0);
    # every depth writes the same plane, so each depth reads [1, 13, 20] at layer 0, head 0, dim 0.
    layers, page = 2, 2
    key_pool = np.zeros((4, layers, page, 1, 4), dtype=np.float32)
    value_pool = np.zeros_like(key_pool)
    table = [2, 3]  # one plane; the same table for every depth
    for pos, exit_depth in [(0, 1), (1, 3), (2, 0)]:
        for depth in range(exit_depth + 1):
            for layer in range(layers):
                value = np.full((1, 1, 4), float(pos * 10 + depth + layer), dtype=np.float32)
                kv_ops.append(key_pool, value_pool, layer, [table[pos // page]], [pos % page], value, value + 100)
    got = kv_ops.gather(key_pool, 0, table, 3, page)
    assert got[:, 0, 0].tolist() == [1, 13, 20]


def test_exit_copies_keep_executed_depths_golden():
    # tests/test_kv_cache.py:38-59: 2 layers, 3 depths, exit at depth 1 copies depth 1 into depth 2
    # at every layer; depth 0 keeps its own values.
    layers, page = 2, 2
    key_pool = np.zeros((6, layers, page, 1, 4), dtype=np.float32)
    value_pool = np.zeros_like(key_pool)
    tables = np.array([[[0, 1], [2, 3], [4, 5]]], dtype=np.int32)  # [slot, plane, page]
    for layer in range(layers):
        for depth in range(2):
            keys = np.full((1, 1, 4), float(10 * layer + depth), dtype=np.float32)
            kv_ops.append(key_pool, value_pool, layer, [tables[0, depth, 0]], [0], keys, keys + 100)
    kv_ops.finalize_batched([[0, 1, 0]], tables, key_pool, value_pool, max_loops=3, page=page)
    for layer in range(layers):
        assert (kv_ops.gather(key_pool, layer, tables[0, 0], 1, page) == 10 * layer).all()
        assert (kv_ops.gather(value_pool, layer, tables[0, 0], 1, page) == 10 * layer + 100).all()
        np.testing.assert_array_equal(
            kv_ops.gather(key_pool, layer, tables[0, 2], 1, page), kv_ops.gather(key_pool, layer, tables[0, 1], 1, page)
        )


def test_finalize_touches_only_target_positions_and_depths():
    # tests/test_async_state.py:131-166: whole-pool equality except the copied slots.
    rng = np.random.default_rng(11)
    layers, page, planes, width = 3, 4, 4, 3
    pool_k = rng.integers(0, 2**16, size=(40, layers, page, 2, 8), dtype=np.uint16)
    pool_v = rng.integers(0, 2**16, size=pool_k.shape, dtype=np.uint16)
    tables = rng.permutation(40)[: 3 * planes * width].reshape(3, planes, width).astype(np.int32)
    desc = np.array([[0, 0, 5], [1, 1, 1], [2, 2, 11], [1, 3, 7]], dtype=np.int64)
    before_k, before_v = pool_k.copy(), pool_v.copy()
    kv_ops.finalize_batched(desc, tables, pool_k, pool_v, max_loops=planes, page=page)
    changed = np.argwhere((pool_k != before_k).any(axis=(1, 3, 4)) | (pool_v != before_v).any(axis=(1, 3, 4)))
    allowed = set()
    for slot, depth, pos in desc:
        for target in range(depth + 1, planes):
            allowed.add((tables[slot, target, pos // page], pos % page))
            src = tables[slot, depth, pos // page]
            dst = tables[slot, target, pos // page]
            assert (pool_k[dst, :, pos % page] == before_k[src, :, pos % page]).all()
            assert (pool_v[dst, :, pos % page] == before_v[src, :, pos % page]).all()
    assert {tuple(x) for x in changed} <= allowed


def test_packed_prefill_metadata_golden():
    # tests/test_flash_attention.py:122-142: page 4; a@depth0 positions 7,8,9 and b@depth1 positions 3,4.
    positions = [7, 8, 9, 3, 4]
    keys = [("a", 0)] * 3 + [("b", 1)] * 2
    cumulative, ends, max_q = kv_ops.packed_prefill_groups(keys, positions)
    table_a, table_b = (0, 1, 2, 3, 4), (5, 6, 7, 8, 9)
    rows = [table_a if k[0] == "a" else table_b for k in keys]
    blocks, offsets, tables, lengths = kv_ops.prepare_addresses([rows[i] for i in ends], [positions[i] for i in ends], 4)
    assert tables.shape == (2, 3)
    assert lengths.tolist() == [10, 5]
    assert cumulative == [0, 3, 5]
    assert max_q == 3
    with pytest.raises(ValueError, match="contiguous"):
        kv_ops.packed_prefill_groups([("a", 0)] * 2, [1, 3])
    with pytest.raises(ValueError, match="one sequence"):
        kv_ops.packed_prefill_groups([("a", 0), ("b", 0), ("a", 0)], [1, 1, 2])


def test_prepared_tables_are_cut_to_the_batch_width_and_padded():
    # tests/test_prepared_kv.py:44-53: 13 rows, page 2, positions 0..4 / 0..2 -> width 3, pad -1.
    positions = list(range(5)) * 2 + list(range(3))
    tables = [(7, 3, 9)] * 5 + [(1, 4, 8)] * 5 + [(5, 6)] * 3
    blocks, offsets, padded, lengths = kv_ops.prepare_addresses(tables, positions, 2)
    assert padded.shape == (13, 3) and padded.dtype == np.int32 and lengths.dtype == np.int32
    assert blocks.dtype == offsets.dtype == np.int64
    assert padded[-1, -1] == -1
    assert blocks.tolist()[:5] == [7, 7, 3, 3, 9] and offsets.tolist()[:5] == [0, 1, 0, 1, 0]


def test_decode_metadata_hand_example():
    # kernels/routing.py:8-41 by hand: tables[slot, plane, col] = 100*slot + 10*plane + col.
    tables = np.array([[[100 * s + 10 * p + c for c in range(4)] for p in range(2)] for s in range(2)], np.int32)
    desc = np.array([[1, 1, 5], [0, 0, 2]], dtype=np.int64)
    meta = kv_ops.decode_metadata(desc, count=2, size=3, tables=tables, page=4, out_width=2)
    assert meta["slots"].tolist() == [1, 0, 0]
    assert meta["positions"].tolist() == [5, 2, 0]
    assert meta["lengths"].tolist() == [6, 3, 0]
    assert meta["blocks"].tolist() == [111, 0]
    assert meta["offsets"].tolist() == [1, 2]
    assert meta["tables"][:, :2].tolist() == [[110, 111], [0, 1], [0, 0]]


def test_prefill_stage_and_expand_hand_example():
    src = np.array([3, -1, 2**33 + 7], dtype=np.int64)
    wide, narrow = kv_ops.stage_prefill(src)
    assert wide.tolist() == src.tolist() and narrow.tolist() == [3, -1, 7]
    tables = np.array([[9, 8, 7], [6, 5, 4]], dtype=np.int32)
    blocks, offsets = kv_ops.expand_prefill([0, 5, 9, 4], [0, 0, 1, 1], tables, 4)
    assert blocks.tolist() == [9, 8, 4, 5] and offsets.tolist() == [0, 1, 1, 0]


# ---------------------------------------------------------------------------
# Planted mistakes: each would pass a check that merely retyped the formula,
# but fails the pins above.


def _mutated_attention(mistake):
    def attention(q, key_cache, value_cache, block_tables, context_lengths):
        page = key_cache.shape[1]
        group = q.shape[1] // key_cache.shape[2]
        out = torch.empty_like(q)
        for row, n in enumerate(context_lengths.tolist()):
            n_used = n - 1 if mistake == "drop_last_token" and n > 1 else n
            pos = torch.arange(n_used)
            pages = block_tables[row, pos // page].long()
            keys = key_cache[pages, pos % page]
            vals = value_cache[pages, pos % page]
            if mistake == "head_modulo":
                idx = torch.arange(q.shape[1]) % key_cache.shape[2]
            else:
                idx = torch.arange(q.shape[1]) // group
            keys, vals = keys[:, idx], vals[:, idx]
            scale = 1.0 if mistake == "no_scale" else 1.0 / math.sqrt(q.shape[-1])
            logits = torch.einsum("hd,nhd->hn", q[row].float(), keys.float()) * scale
            out[row] = torch.einsum("hn,nhd->hd", logits.softmax(-1), vals.float()).to(q.dtype)
        return out

    return attention


@pytest.mark.parametrize("mistake", ["drop_last_token", "head_modulo", "no_scale"])
def test_planted_attention_mistakes_are_caught(mistake):
    case = random_decode_case([7, 1, 6, 3, 16, 9], hq=6, hkv=2, d=7, page=3, dtype=torch.float32, seed=48)
    wrong = _mutated_attention(mistake)(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    f64 = paged_attention_f64(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    assert not np.allclose(wrong.double().numpy(), f64, atol=2e-6, rtol=2e-5)
    right = _mutated_attention(None)(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    np.testing.assert_allclose(right.double().numpy(), f64, atol=2e-6, rtol=2e-5)


def _exit_copy_golden(copy_token, finalize_batched):
    """tests/test_kv_cache.py:38-59 run through both exit-copy restatements.

    2 layers, 3 depths, page 2; the token at position 0 writes depths 0 and 1
    with keys 10*layer + depth (values +100) and exits at depth 1.  Depth 2
    must then equal depth 1 at every layer, depth 0 keeps its own values, and
    the copies are physical: a later write at depth 1 leaves depth 2 at the
    old value.  Returns the list of failed checks (empty when the golden holds).
    """
    layers, page = 2, 2
    tables = np.array([[[0, 1], [2, 3], [4, 5]]], dtype=np.int32)  # [slot, plane, page]
    failed = []
    for route in ("copy_token", "finalize_batched"):
        # Distinct negative sentinels in every element, so any stray copy shows.
        key_pool = -1.0 - np.arange(6 * layers * page * 4, dtype=np.float32).reshape(6, layers, page, 1, 4)
        value_pool = key_pool - 1000.0
        for layer in range(layers):
            for depth in range(2):
                keys = np.full((1, 1, 4), float(10 * layer + depth), dtype=np.float32)
                kv_ops.append(key_pool, value_pool, layer, [tables[0, depth, 0]], [0], keys, keys + 100)
        before_k, before_v = key_pool.copy(), value_pool.copy()
        if route == "copy_token":
            copy_token(key_pool, value_pool, int(tables[0, 1, 0]), [int(tables[0, 2, 0])], 0)
        else:
            finalize_batched([[0, 1, 0]], tables, key_pool, value_pool, max_loops=3, page=page)
        for layer in range(layers):
            read = {d: (kv_ops.gather(key_pool, layer, tables[0, d], 1, page),
                        kv_ops.gather(value_pool, layer, tables[0, d], 1, page)) for d in range(3)}
            if not ((read[0][0] == 10 * layer).all() and (read[0][1] == 10 * layer + 100).all()):
                failed.append((route, layer, "depth 0 changed"))
            if not ((read[2][0] == 10 * layer + 1).all() and (read[2][1] == 10 * layer + 101).all()):
                failed.append((route, layer, "depth 2 is not depth 1"))
        # Only the (page 4, offset 0) slot of every layer may change.
        changed = (key_pool != before_k) | (value_pool != before_v)
        changed[4, :, 0] = False
        if changed.any():
            failed.append((route, "a slot other than the target changed"))
        # Physical copies: overwrite depth 1 at layer 0, depth 2 keeps the old keys (ones).
        kv_ops.append(key_pool, value_pool, 0, [tables[0, 1, 0]], [0],
                      np.zeros((1, 1, 4), np.float32), np.zeros((1, 1, 4), np.float32))
        if not (kv_ops.gather(key_pool, 0, tables[0, 2], 1, page) == 1.0).all():
            failed.append((route, "depth 2 aliases depth 1"))
    return failed


def test_exit_copy_restatements_pass_the_golden():
    assert _exit_copy_golden(kv_ops.copy_token, kv_ops.finalize_batched) == []


def _copy_token_mistake(mistake):
    def copy_token(key_pool, value_pool, src_block, dst_blocks, offset):
        for dst in dst_blocks:
            if mistake == "reversed":
                key_pool[src_block, :, offset] = key_pool[dst, :, offset]
                value_pool[src_block, :, offset] = value_pool[dst, :, offset]
            elif mistake == "first_layer_only":
                key_pool[dst, 0, offset] = key_pool[src_block, 0, offset]
                value_pool[dst, 0, offset] = value_pool[src_block, 0, offset]
            elif mistake == "keys_into_values":
                key_pool[dst, :, offset] = key_pool[src_block, :, offset]
                value_pool[dst, :, offset] = key_pool[src_block, :, offset]
            elif mistake == "whole_page":
                key_pool[dst] = key_pool[src_block]
                value_pool[dst] = value_pool[src_block]

    return copy_token


def _finalize_mistake(mistake):
    def finalize_batched(descriptors, tables, key_pool, value_pool, max_loops, page):
        for slot, depth, pos in np.asarray(descriptors).reshape(-1, 3):
            # wrong_source: copy from plane 0 instead of the exit plane.
            src = tables[slot, 0 if mistake == "wrong_source" else depth, pos // page]
            first = depth if mistake == "includes_exit_plane" else depth + 1
            for target in range(first, max_loops - (mistake == "stops_short")):
                dst = tables[slot, target, pos // page]
                key_pool[dst, :, pos % page] = key_pool[src, :, pos % page]
                value_pool[dst, :, pos % page] = value_pool[src, :, pos % page]

    return finalize_batched


@pytest.mark.parametrize("mistake", ["reversed", "first_layer_only", "keys_into_values", "whole_page"])
def test_planted_copy_token_mistakes_are_caught(mistake):
    assert _exit_copy_golden(_copy_token_mistake(mistake), kv_ops.finalize_batched) != []


@pytest.mark.parametrize("mistake", ["wrong_source", "stops_short"])
def test_planted_finalize_mistakes_are_caught(mistake):
    assert _exit_copy_golden(kv_ops.copy_token, _finalize_mistake(mistake)) != []
    assert _exit_copy_golden(kv_ops.copy_token, _finalize_mistake(None)) == []
