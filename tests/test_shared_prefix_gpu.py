"""Decode with a shared-prefix hint (rlt_paged_decode_shared_prefix) on the GPU.

Rows listed in the hint begin their tables with the same pages, as
prefix-cache aliasing makes them (vllm_rlt/core/kv_cache_manager.py:240-293).
The result must be the attention the reference computes (the CPU oracle,
tolerances of the decode tests), whatever the hint says: rows the prefix pass
serves, rows it cannot serve (another split length, too short), a listed row
whose table does not hold the shared pages, and rows outside the hint, which
must match the plain decode bit for bit.
"""

import pytest
import torch

from oracle.paged_attention import paged_attention_cpu
from paged_cases import DecodeCase

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-3, 2e-3), torch.float32: (1e-5, 1e-5)}
PAGE = 16


def prefix_case(lengths, members, prefix_pages, *, hq, hkv, d=128, dtype=torch.bfloat16, seed=0, liars=()):
    """Members' tables start with `prefix_pages` shared pages; liars are listed but own theirs."""
    g = torch.Generator().manual_seed(seed)
    pages = [(n + PAGE - 1) // PAGE for n in lengths]
    own = [max(p - prefix_pages, 0) if r in members and r not in liars else p for r, p in enumerate(pages)]
    width = max(pages + [prefix_pages, 1])
    blocks = prefix_pages + sum(own) + 3
    perm = torch.randperm(blocks, generator=g).to(torch.int32)
    shared = perm[:prefix_pages]
    key_pool = torch.randn((blocks, 1, PAGE, hkv, d), generator=g)
    value_pool = torch.randn((blocks, 1, PAGE, hkv, d), generator=g)
    tables = torch.full((len(lengths), width), -1, dtype=torch.int32)
    live = torch.zeros(blocks, PAGE, dtype=torch.bool)
    live[shared.long()] = True
    used = prefix_pages
    for r, (n, p) in enumerate(zip(lengths, pages)):
        ids = perm[used : used + own[r]]
        used += own[r]
        if r in members and r not in liars:
            tables[r, :prefix_pages] = shared
            tables[r, prefix_pages : prefix_pages + own[r]] = ids
        else:
            tables[r, :p] = ids
            if p:
                live[ids[:-1].long()] = True
                live[ids[-1].long(), : n - (p - 1) * PAGE] = True
        if r in members and r not in liars and own[r]:
            live[ids[:-1].long()] = True
            live[ids[-1].long(), : n - (p - 1) * PAGE] = True
    key_pool.transpose(1, 2)[~live] = float("nan")
    value_pool.transpose(1, 2)[~live] = float("nan")
    q = torch.randn(len(lengths), hq, d, generator=g)
    case = DecodeCase(q.to(dtype), key_pool.to(dtype), value_pool.to(dtype), 0, tables,
                      torch.tensor(lengths, dtype=torch.int32))
    return case, shared


def run(case, hint_rows=None, shared=None, split_lengths=None):
    from vllm_rlt_amd import ops

    dev = case.to("cuda")
    hint = None
    if hint_rows is not None:
        lengths = split_lengths if split_lengths is not None else [int(case.lengths[r]) for r in hint_rows]
        hint = ops.shared_prefix(hint_rows, shared, case.q.shape[0], lengths, "cuda")
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, shared_prefix=hint)
    torch.cuda.synchronize()
    return out.cpu()


def check(case, actual):
    atol, rtol = TOL[case.q.dtype]
    expected = paged_attention_cpu(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    torch.testing.assert_close(actual, expected, atol=atol, rtol=rtol)
    assert torch.isfinite(actual).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(16, 16), (8, 4), (16, 4), (16, 2)])
def test_shared_prefix_with_256_token_splits(dtype, hq, hkv):
    # 40 shared pages (640 tokens, two whole 256-token splits).  Members: longer
    # than the prefix, shorter than it, a single split (not served), empty; row
    # 6 is listed but owns its pages; rows 7-8 are outside the hint.
    lengths = [2000, 700, 520, 300, 256, 0, 1500, 900, 640]
    members, liars = [0, 1, 2, 3, 4, 5, 6], [6]
    case, shared = prefix_case(lengths, members, 40, hq=hq, hkv=hkv, dtype=dtype, seed=hq + 7 * hkv, liars=liars)
    hinted = run(case, members, shared)
    check(case, hinted)
    plain = run(case)
    assert torch.equal(hinted[7:], plain[7:])
    assert torch.equal(hinted[4:7], plain[4:7])  # served by nothing but the split pass


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 4)])
def test_shared_prefix_with_512_token_splits(hq, hkv):
    # Rows past 16384 tokens use 512-token splits.  600 shared pages (9600
    # tokens) give 18 whole 512-token splits.  Row 3 (9000 tokens) uses
    # 256-token splits, so the prefix pass (512) leaves it to the split pass.
    lengths = [17000, 20000, 16500, 9000, 17500]
    members = [0, 1, 2, 3]
    case, shared = prefix_case(lengths, members, 600, hq=hq, hkv=hkv, seed=hq + hkv)
    hinted = run(case, members, shared)
    check(case, hinted)
    plain = run(case)
    assert torch.equal(hinted[3:], plain[3:])


def test_shared_prefix_hint_for_a_split_length_no_member_uses():
    lengths = [3000, 4000, 2500]
    case, shared = prefix_case(lengths, [0, 1, 2], 100, hq=8, hkv=8, seed=3)
    hinted = run(case, [0, 1, 2], shared, split_lengths=[20000, 20000, 20000])  # asks for 512-token splits
    assert torch.equal(hinted, run(case))


@pytest.mark.parametrize("dtype,d", [(torch.float32, 128), (torch.bfloat16, 64)])
def test_shared_prefix_hint_is_ignored_where_the_pass_does_not_exist(dtype, d):
    lengths = [1000, 1300, 800]
    case, shared = prefix_case(lengths, [0, 1, 2], 40, hq=4, hkv=4, d=d, dtype=dtype, seed=11)
    hinted = run(case, [0, 1, 2], shared)
    assert torch.equal(hinted, run(case))
    check(case, hinted)


def test_shared_prefix_ouro_shape():
    # Ouro-1.4B heads over the prefix-stress shape: rows of 16-32K tokens
    # sharing an 8192-token prefix.
    g = torch.Generator().manual_seed(5)
    lengths = torch.randint(16384, 32769, (8,), generator=g).tolist()
    case, shared = prefix_case(lengths, list(range(8)), 512, hq=16, hkv=16, seed=5)
    check(case, run(case, list(range(8)), shared))


def test_shared_prefix_arguments_are_checked():
    from vllm_rlt_amd import ops

    case, shared = prefix_case([1000, 900], [0, 1], 40, hq=4, hkv=4, seed=2)
    dev = case.to("cuda")
    with pytest.raises(ValueError, match="distinct batch rows"):
        ops.shared_prefix([0, 0], shared, 2, [1000, 900], "cuda")
    with pytest.raises(ValueError, match="distinct batch rows"):
        ops.shared_prefix([2], shared, 2, [1000], "cuda")
    hint = ops.shared_prefix([0, 1], shared, 2, [1000, 900], "cuda")
    bad = ops.SharedPrefix(hint.member, hint.rows, hint.table, 300)
    with pytest.raises(ValueError, match="prefix_split_len"):
        ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, shared_prefix=bad)
    wide = ops.SharedPrefix(hint.member, hint.rows, torch.zeros(999, dtype=torch.int32, device="cuda"), 256)
    with pytest.raises(ValueError, match="wider than the block tables"):
        ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, shared_prefix=wide)
    short = ops.SharedPrefix(hint.member[:1], hint.rows, hint.table, 256)
    with pytest.raises(ValueError, match=r"member must be contiguous int32 \[rows\]"):
        ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, shared_prefix=short)


@pytest.mark.parametrize("share", [False, True])
def test_manager_shares_the_prefix_reads_of_aliasing_rows(share):
    # Requests b, c, d reuse a's published 800-token prefix (50 pages per
    # depth, tests/test_prefix_growth.py:47-64); a decode batch of all four
    # at depth 1 then reads those pages once when share_prefix_reads is set.
    from dataclasses import replace

    from vllm_rlt_amd import KVCacheManager

    cache = KVCacheManager(1, 2, 128, 1024, 16, 2, device="cuda", dtype=torch.bfloat16,
                           enable_prefix_caching=True, share_prefix_reads=share)
    torch.manual_seed(21)
    prompt = list(range(1000, 1801))
    assert cache.allocate("a", 1400)
    for depth in range(2):
        kv = torch.randn(800, 2, 128, device="cuda", dtype=torch.bfloat16)
        cache.write(0, ["a"] * 800, [depth] * 800, list(range(800)), kv, -kv)
    cache.publish_prefix("a", prompt, 800)
    hit = cache.lookup_prefix(prompt)
    assert len(hit) == 50
    ends = {"a": 1100, "b": 1000, "c": 1290, "d": 900}
    for rid in ("b", "c", "d"):
        assert cache.allocate(rid, 1400, prefix=hit)
    for rid, end in ends.items():
        for depth in range(2):
            n = end - 800
            kv = torch.randn(n, 2, 128, device="cuda", dtype=torch.bfloat16)
            cache.write(0, [rid] * n, [depth] * n, list(range(800, end)), kv, kv * 0.5)
    ids = list(ends)
    batch = cache._prepare_batch(ids, [1] * 4, [ends[r] - 1 for r in ids], for_write=False)
    q = torch.randn(4, 4, 128, device="cuda", dtype=torch.bfloat16)
    out = cache._attend_prepared(0, batch, q)
    if not share:
        assert batch.shared_prefix is None
        return
    hint = batch.shared_prefix
    assert hint.rows.tolist() == [0, 1, 2, 3] and hint.member.tolist() == [1, 1, 1, 1]
    assert hint.table.tolist() == list(cache.get_block_table("b", 1)[:50]) and hint.split_len == 256
    plain = cache._attend_prepared(0, replace(batch, shared_prefix=None), q)
    torch.testing.assert_close(out, plain, atol=2e-2, rtol=1e-2)
    expected = paged_attention_cpu(
        q.cpu(), cache.key_cache[:, 0].cpu(), cache.value_cache[:, 0].cpu(), batch.block_tables.cpu(),
        batch.context_lengths.cpu(),
    )
    torch.testing.assert_close(out.cpu(), expected, atol=2e-2, rtol=1e-2)


def test_shared_prefix_decode_replays_in_a_graph():
    # A captured write+attend over rows that alias a published prefix (with
    # the hint) replays to the eager result every time, eager work between.
    from vllm_rlt_amd import DeviceCache, KVCacheManager

    cache = KVCacheManager(2, 2, 128, 512, 16, 2, device="cuda", dtype=torch.bfloat16,
                           enable_prefix_caching=True, share_prefix_reads=True)
    torch.manual_seed(4)
    prompt = list(range(2000, 2641))
    assert cache.allocate("a", 1200)
    for layer in range(2):
        for depth in range(2):
            kv = torch.randn(640, 2, 128, device="cuda", dtype=torch.bfloat16)
            cache.write(layer, ["a"] * 640, [depth] * 640, list(range(640)), kv, -kv)
    cache.publish_prefix("a", prompt, 640)
    hit = cache.lookup_prefix(prompt)
    ends = {"a": 1000, "b": 900, "c": 1100}
    for rid in ("b", "c"):
        assert cache.allocate(rid, 1200, prefix=hit)
    for layer in range(2):
        for rid, end in ends.items():
            n = end - 640
            kv = torch.randn(n, 2, 128, device="cuda", dtype=torch.bfloat16)
            cache.write(layer, [rid] * n, [0] * n, list(range(640, end)), kv, kv)
    ids = list(ends)
    batch = cache._prepare_batch(ids, [0, 0, 0], [ends[r] for r in ids])
    assert batch.shared_prefix is not None and batch.shared_prefix.rows.numel() == 3
    k = torch.randn(3, 2, 128, device="cuda", dtype=torch.bfloat16)
    q = torch.randn(3, 4, 128, device="cuda", dtype=torch.bfloat16)
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
