"""Fused KV append + decode attention (rlt_paged_decode_append) on the GPU.

The fused launch must leave the pages and produce the output bit for bit as
the two-step sequence it replaces (vllm_rlt/core/kv_cache_manager.py:520-534
then 559-586: kv_append, then paged_decode), on batches where no row reads a
slot another row writes.  Both are checked against the CPU oracle's append
and attention.  Shapes the fused kernel does not cover (KV heads not a
multiple of 4, strided new tokens, other head sizes) take the append-first
path and must agree the same way.
"""

import pytest
import torch

from oracle import kv_ops
from oracle.paged_attention import paged_attention_cpu
from paged_cases import random_decode_case

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-3, 2e-3), torch.float32: (1e-5, 1e-5)}
BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}


def bits(t):
    return t.contiguous().view(BITS[t.dtype]).cpu()


def decode_batch(lengths, *, hq, hkv, d, dtype, seed, n_write=None, page=16, layers=2, layer=1):
    """A random paged case whose rows append their last token (length - 1) before attending."""
    case = random_decode_case(lengths, hq=hq, hkv=hkv, d=d, page=page, dtype=dtype, seed=seed, layers=layers,
                              layer=layer, fill_unused=0.0)
    g = torch.Generator().manual_seed(seed + 1)
    rows = len(lengths)
    n = rows if n_write is None else n_write
    k_new = torch.randn(rows, hkv, d, generator=g).to(dtype)
    v_new = torch.randn(rows, hkv, d, generator=g).to(dtype)
    blocks = torch.tensor([int(case.tables[r, (n_ - 1) // page]) if n_ else 0 for r, n_ in enumerate(lengths)],
                          dtype=torch.int64)
    offsets = torch.tensor([(n_ - 1) % page if n_ else 0 for n_ in lengths], dtype=torch.int64)
    return case, k_new, v_new, blocks[:n], offsets[:n], n


def two_step(case, k_new, v_new, blocks, offsets, n):
    from vllm_rlt_amd import ops

    dev = case.to("cuda")
    ops.kv_append(dev.key_pool, dev.value_pool, case.layer, blocks.cuda(), offsets.cuda(), k_new.cuda(), v_new.cuda(),
                  n_rows=n)
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths)
    torch.cuda.synchronize()
    return out.cpu(), dev.key_pool.cpu(), dev.value_pool.cpu()


def fused(case, k_new, v_new, blocks, offsets, n):
    from vllm_rlt_amd import ops

    dev = case.to("cuda")
    out = ops.paged_decode_append(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, k_new.cuda(),
                                  v_new.cuda(), blocks.cuda(), offsets.cuda(), n_write=n)
    torch.cuda.synchronize()
    return out.cpu(), dev.key_pool.cpu(), dev.value_pool.cpu()


def check_against_oracle(case, k_new, v_new, blocks, offsets, n, out, key_pool, value_pool):
    exp_k = case.key_pool.view(BITS[case.q.dtype]).numpy().copy()
    exp_v = case.value_pool.view(BITS[case.q.dtype]).numpy().copy()
    kv_ops.append(exp_k, exp_v, case.layer, blocks.tolist(), offsets.tolist(),
                  k_new.view(BITS[case.q.dtype]).numpy(), v_new.view(BITS[case.q.dtype]).numpy(), n_rows=n)
    assert (key_pool.view(BITS[case.q.dtype]).numpy() == exp_k).all()
    assert (value_pool.view(BITS[case.q.dtype]).numpy() == exp_v).all()
    expect = paged_attention_cpu(case.q, key_pool[:, case.layer], value_pool[:, case.layer], case.tables, case.lengths)
    atol, rtol = TOL[case.q.dtype]
    torch.testing.assert_close(out, expect, atol=atol, rtol=rtol)


LENGTHS = [1, 15, 16, 17, 255, 256, 257, 300, 600, 1029, 4100, 9000]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hq,hkv,d", [(16, 16, 128), (32, 16, 128), (16, 4, 128), (8, 8, 64), (4, 4, 256), (4, 2, 128),
                                     (32, 4, 128), (64, 8, 64)])
def test_fused_append_equals_two_steps_and_the_oracle(dtype, hq, hkv, d):
    case, k_new, v_new, blocks, offsets, n = decode_batch(LENGTHS, hq=hq, hkv=hkv, d=d, dtype=dtype, seed=hq + d)
    print(f"[decode_append] {dtype} hq={hq} hkv={hkv} d={d}", flush=True)
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    got = fused(case, k_new, v_new, blocks, offsets, n)
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))
    check_against_oracle(case, k_new, v_new, blocks, offsets, n, *got)


SHORT = [1, 15, 16, 17, 120, 200, 255, 256]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hq,hkv,d", [(16, 16, 128), (16, 4, 128), (8, 8, 64), (4, 2, 128), (32, 4, 128)])
def test_tables_of_one_split_store_the_token_in_the_split_pass(dtype, hq, hkv, d):
    # Tables of at most 256 tokens: every row is one split, the split pass
    # writes the outputs and stores the new tokens itself, and no merge runs.
    case, k_new, v_new, blocks, offsets, n = decode_batch(SHORT, hq=hq, hkv=hkv, d=d, dtype=dtype, seed=hq + d + 3)
    assert case.tables.shape[1] * 16 <= 256
    print(f"[decode_append] one split {dtype} hq={hq} hkv={hkv} d={d}", flush=True)
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    got = fused(case, k_new, v_new, blocks, offsets, n)
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))
    check_against_oracle(case, k_new, v_new, blocks, offsets, n, *got)


def test_one_split_tables_with_empty_rows_and_a_slot_nobody_reads():
    # An empty row that appends (to a page no table reads) and pad rows past
    # n_write, in a launch where every row is one split.
    lengths = [40, 0, 90, 256, 0, 0]
    case, k_new, v_new, blocks, offsets, n = decode_batch(lengths, hq=16, hkv=16, d=128, dtype=torch.bfloat16,
                                                          seed=17, n_write=4)
    spare = sorted(set(range(case.key_pool.shape[0])) - set(case.tables.flatten().tolist()))[0]
    blocks[1], offsets[1] = spare, 5
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    got = fused(case, k_new, v_new, blocks, offsets, n)
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))
    assert torch.count_nonzero(got[0][[1, 4, 5]]) == 0
    check_against_oracle(case, k_new, v_new, blocks, offsets, n, *got)


def test_fused_append_with_a_stale_workspace():
    # The merge kernel reads the new token from a clamped row and every split slot
    # before it knows the row's split count; a NaN-filled workspace (what earlier
    # launches leave) and pad rows past n_write must still give the two-step bits.
    from vllm_rlt_amd import ops

    case, k_new, v_new, blocks, offsets, n = decode_batch(LENGTHS, hq=16, hkv=16, d=128, dtype=torch.bfloat16,
                                                          seed=404, n_write=len(LENGTHS) - 3)
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    dev = case.to("cuda")
    nbytes = ops.decode_workspace_bytes(len(LENGTHS), 16, 16, 128)
    workspace = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")
    out = ops.paged_decode_append(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, k_new.cuda(),
                                  v_new.cuda(), blocks.cuda(), offsets.cuda(), n_write=n, workspace=workspace)
    torch.cuda.synchronize()
    got = (out.cpu(), dev.key_pool.cpu(), dev.value_pool.cpu())
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))


def test_fused_append_pad_rows_and_empty_rows():
    # Rows past n_write are padding (no write; length 0 reads nothing), and an
    # empty row inside the written range attends to nothing.
    lengths = [300, 40, 2000, 17, 0, 0]
    case, k_new, v_new, blocks, offsets, n = decode_batch(lengths, hq=16, hkv=16, d=128, dtype=torch.bfloat16,
                                                          seed=5, n_write=4)
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    got = fused(case, k_new, v_new, blocks, offsets, n)
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))
    assert torch.count_nonzero(got[0][4:]) == 0


def test_fused_append_to_a_slot_nobody_reads():
    # A row whose write slot is not its own last token's slot reads its last
    # token from the page, as the two steps do when no row reads the slot written.
    case, k_new, v_new, blocks, offsets, n = decode_batch([40, 90, 513], hq=16, hkv=16, d=128, dtype=torch.bfloat16,
                                                          seed=6)
    # random_decode_case keeps spare blocks that no table uses.
    spare = sorted(set(range(case.key_pool.shape[0])) - set(case.tables.flatten().tolist()))[0]
    blocks[1], offsets[1] = spare, 3
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    got = fused(case, k_new, v_new, blocks, offsets, n)
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))


def test_fused_append_strided_new_tokens_take_the_append_first_path():
    case, k_new, v_new, blocks, offsets, n = decode_batch([70, 300, 1500], hq=16, hkv=16, d=128,
                                                          dtype=torch.bfloat16, seed=7)
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    from vllm_rlt_amd import ops

    dev = case.to("cuda")
    wide_k = torch.zeros(3, 16, 256, dtype=torch.bfloat16, device="cuda")
    wide_v = torch.zeros_like(wide_k)
    wide_k[:, :, ::2] = k_new.cuda()
    wide_v[:, :, ::2] = v_new.cuda()
    out = ops.paged_decode_append(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, wide_k[:, :, ::2],
                                  wide_v[:, :, ::2], blocks.cuda(), offsets.cuda())
    torch.cuda.synchronize()
    assert torch.equal(bits(out), bits(ref[0]))
    assert torch.equal(bits(dev.key_pool), bits(ref[1])) and torch.equal(bits(dev.value_pool), bits(ref[2]))


def test_fused_append_more_than_8192_rows():
    # Two launches; the writes of rows past 8192 belong to the second.
    g = torch.Generator().manual_seed(8301)
    lengths = torch.randint(1, 41, (8300,), generator=g).tolist()
    case, k_new, v_new, blocks, offsets, n = decode_batch(lengths, hq=8, hkv=4, d=64, dtype=torch.bfloat16, seed=8,
                                                          n_write=8250, layers=1, layer=0)
    ref = two_step(case, k_new, v_new, blocks, offsets, n)
    got = fused(case, k_new, v_new, blocks, offsets, n)
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))


# ---------------------------------------------------------------- the manager
def _manager(layout):
    from vllm_rlt_amd import KVCacheManager

    return KVCacheManager(num_layers=2, num_kv_heads=4, head_dim=128, num_blocks=320, block_size=16, max_loops=4,
                          device="cuda", dtype=torch.bfloat16, layout=layout)


@pytest.mark.parametrize("layout", ["last_exited", "shared"])
def test_manager_write_attend_equals_write_then_attend(layout):
    fused_cache, plain = _manager(layout), _manager(layout)
    g = torch.Generator().manual_seed(11)
    for cache in (fused_cache, plain):
        cache.key_cache.zero_()
        cache.value_cache.zero_()
        for rid in ("a", "b", "c"):
            assert cache.allocate(rid, 300)
    depths = [0, 2, 3] if layout == "last_exited" else [0, 1, 3]
    for pos in range(40):
        batch_f = fused_cache._prepare_batch(["a", "b", "c"], depths, [pos, pos, pos])
        batch_p = plain._prepare_batch(["a", "b", "c"], depths, [pos, pos, pos])
        assert fused_cache._rows_independent(batch_f)
        for layer in range(2):
            q = torch.randn(3, 8, 128, generator=g).to(torch.bfloat16).cuda()
            k = torch.randn(3, 4, 128, generator=g).to(torch.bfloat16).cuda()
            v = torch.randn(3, 4, 128, generator=g).to(torch.bfloat16).cuda()
            out_f = fused_cache._write_attend_prepared(layer, batch_f, q, k, v)
            plain._write_prepared(layer, batch_p, k, v)
            out_p = plain._attend_prepared(layer, batch_p, q)
            assert torch.equal(bits(out_f), bits(out_p)), (pos, layer)
    assert torch.equal(bits(fused_cache.key_cache), bits(plain.key_cache))
    assert torch.equal(bits(fused_cache.value_cache), bits(plain.value_cache))
    assert fused_cache.read(1, "b", depths[1]) is not None


def test_manager_dependent_rows_take_the_two_steps():
    # One request twice on one plane: the second row reads the first row's new
    # token, so the manager must not fuse.
    fused_cache, plain = _manager("last_exited"), _manager("last_exited")
    for cache in (fused_cache, plain):
        cache.key_cache.zero_()
        cache.value_cache.zero_()
        assert cache.allocate("a", 300)
    g = torch.Generator().manual_seed(12)
    for pos in range(0, 30, 2):
        ids, depths, positions = ["a", "a"], [1, 1], [pos, pos + 1]
        batch_f = fused_cache._prepare_batch(ids, depths, positions)
        batch_p = plain._prepare_batch(ids, depths, positions)
        assert not fused_cache._rows_independent(batch_f)
        q = torch.randn(2, 8, 128, generator=g).to(torch.bfloat16).cuda()
        k = torch.randn(2, 4, 128, generator=g).to(torch.bfloat16).cuda()
        v = torch.randn(2, 4, 128, generator=g).to(torch.bfloat16).cuda()
        out_f = fused_cache._write_attend_prepared(0, batch_f, q, k, v)
        plain._write_prepared(0, batch_p, k, v)
        out_p = plain._attend_prepared(0, batch_p, q)
        assert torch.equal(bits(out_f), bits(out_p))


def test_graph_replays_of_the_fused_core_match_eager():
    from vllm_rlt_amd.graphs import RecurrentGraphs

    def core(hidden, batch, cache):
        n = hidden.shape[0]
        for layer in range(2):
            q = (hidden[:, :1024].reshape(n, 8, 128) * (layer + 1)).contiguous()
            k = hidden[:, 1024:1536].reshape(n, 4, 128).contiguous()
            v = hidden[:, 1536:2048].reshape(n, 4, 128).contiguous()
            out = cache._write_attend_prepared(layer, batch, q, k, v)
            hidden = hidden + torch.cat([out.reshape(n, 1024)] * 2, dim=1)
        return hidden

    graphed, eager = _manager("last_exited"), _manager("last_exited")
    for cache in (graphed, eager):
        cache.key_cache.zero_()
        cache.value_cache.zero_()
        for rid in ("a", "b"):
            assert cache.allocate(rid, 200)
    graphs = RecurrentGraphs(core, graphed, max_batch_size=4, max_graphs=2, max_positions=256)
    g = torch.Generator().manual_seed(13)
    for pos in range(12):
        hidden = torch.randn(2, 2048, generator=g).to(torch.bfloat16).cuda()
        got = graphs.run(hidden, graphed._prepare_batch(["a", "b"], [1, 3], [pos, pos]))
        with torch.inference_mode():
            expect = core(hidden, eager._prepare_batch(["a", "b"], [1, 3], [pos, pos]), eager)
        torch.cuda.synchronize()
        assert torch.equal(bits(got), bits(expect)), pos
        _ = torch.randn(32, 32, device="cuda").sum().item()
    assert graphs.captures == 1 and graphs.replays == 12
    assert torch.equal(bits(graphed.key_cache), bits(eager.key_cache))
