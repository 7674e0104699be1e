"""Decode with prefix groups (rlt_paged_decode_shared_prefix) on the GPU.

Rows whose tables begin with prefix-cache pages alias those pages read-only
(vllm_rlt/core/kv_cache_manager.py:211-293); under LAST-EXITED every plane has
its own prefix pages, so a mixed-depth batch holds one group per plane and per
prefix.  The result must be the attention the reference computes (the CPU
oracle, tolerances of the decode tests), whatever the hint says: rows the
prefix pass serves, rows it cannot serve (another split length, too short), a
row whose hint names pages its table does not hold, and rows outside every
group, which must match the plain decode bit for bit.  A row's bits must not
depend on the rest of its batch (the reference pins decode bits across batch
compositions, tests/test_flash_attention.py:193-208).
"""

import pytest
import torch

from oracle import kv_ops
from oracle.paged_attention import paged_attention_cpu
from paged_cases import DecodeCase

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-3, 2e-3), torch.float32: (1e-5, 1e-5)}
PAGE = 16


def groups_case(lengths, row_group, group_pages, *, hq, hkv, d=128, dtype=torch.bfloat16, seed=0, liars=()):
    """Rows r with row_group[r] = g >= 0 start their tables with group g's
    group_pages[g] shared pages; liars are given the group's pages as their hint
    but own all of theirs.  Returns (case, shared page ids per group, hint pages per row)."""
    g = torch.Generator().manual_seed(seed)
    pages = [(n + PAGE - 1) // PAGE for n in lengths]
    shares = [row_group[r] >= 0 and r not in liars for r in range(len(lengths))]
    own = [max(p - group_pages[row_group[r]], 0) if shares[r] else p for r, p in enumerate(pages)]
    width = max(pages + list(group_pages) + [1])
    blocks = sum(group_pages) + sum(own) + 3
    perm = torch.randperm(blocks, generator=g).to(torch.int32)
    shared, used = [], 0
    for n in group_pages:
        shared.append(perm[used : used + n])
        used += n
    key_pool = torch.randn((blocks, 1, PAGE, hkv, d), generator=g)
    value_pool = torch.randn((blocks, 1, PAGE, hkv, d), generator=g)
    tables = torch.full((len(lengths), width), -1, dtype=torch.int32)
    live = torch.zeros(blocks, PAGE, dtype=torch.bool)
    for ids in shared:
        live[ids.long()] = True
    hint_pages = []
    for r, (n, p) in enumerate(zip(lengths, pages)):
        ids = perm[used : used + own[r]]
        used += own[r]
        grp = row_group[r]
        hint_pages.append(shared[grp].tolist() if grp >= 0 else [])
        if shares[r]:
            k = group_pages[grp]
            tables[r, :k] = shared[grp]
            tables[r, k : k + own[r]] = ids
        else:
            tables[r, :p] = ids
        if own[r]:
            live[ids[:-1].long()] = True
            live[ids[-1].long(), : n - (p - 1) * PAGE] = True
    key_pool.transpose(1, 2)[~live] = float("nan")
    value_pool.transpose(1, 2)[~live] = float("nan")
    q = torch.randn(len(lengths), hq, d, generator=g)
    case = DecodeCase(q.to(dtype), key_pool.to(dtype), value_pool.to(dtype), 0, tables,
                      torch.tensor(lengths, dtype=torch.int32))
    return case, shared, hint_pages


def hint_for(case, hint_pages, lengths=None):
    from vllm_rlt_amd import ops

    lengths = [int(n) for n in case.lengths] if lengths is None else lengths
    return ops.prefix_groups(hint_pages, lengths, PAGE, case.q.shape[1] // case.key_pool.shape[3], "cuda")


def run(case, hint_pages=None, split_lengths=None):
    from vllm_rlt_amd import ops

    dev = case.to("cuda")
    hint = None if hint_pages is None else hint_for(case, hint_pages, split_lengths)
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, shared_prefix=hint)
    torch.cuda.synchronize()
    return out.cpu()


def check(case, actual):
    atol, rtol = TOL[case.q.dtype]
    expected = paged_attention_cpu(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    torch.testing.assert_close(actual, expected, atol=atol, rtol=rtol)
    assert torch.isfinite(actual).all()


def bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(16, 16), (8, 4), (16, 4), (16, 2), (32, 4)])
def test_one_group_with_256_token_splits(dtype, hq, hkv):
    # 40 shared pages (640 tokens, two whole 256-token splits).  Members: longer
    # than the prefix, shorter than it, a single split (not served), empty; row
    # 6 is hinted but owns its pages; rows 7-8 are outside the hint.
    lengths = [2000, 700, 520, 300, 256, 0, 1500, 900, 640]
    row_group = [0, 0, 0, 0, 0, 0, 0, -1, -1]
    case, _, hint_pages = groups_case(lengths, row_group, [40], hq=hq, hkv=hkv, dtype=dtype, seed=hq + 7 * hkv,
                                      liars=[6])
    print(f"[prefix groups] one group {dtype} hq={hq} hkv={hkv}", flush=True)
    hinted = run(case, hint_pages)
    check(case, hinted)
    plain = run(case)
    assert torch.equal(hinted[7:], plain[7:])
    assert torch.equal(hinted[4:7], plain[4:7])  # served by nothing but the split pass


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 4)])
def test_four_planes_of_prefixes_in_one_launch(hq, hkv):
    # A LAST-EXITED mixed-depth batch: rows at depths 0..3 read plane d's own
    # prefix (48, 40, 64, 33 pages), two rows read none, one row's hint is false.
    g = torch.Generator().manual_seed(hq * 3 + hkv)
    n = 24
    depth = torch.randint(0, 4, (n,), generator=g).tolist()
    depth[5] = depth[17] = -1
    lengths = torch.randint(900, 2600, (n,), generator=g).tolist()
    case, _, hint_pages = groups_case(lengths, depth, [48, 40, 64, 33], hq=hq, hkv=hkv, seed=hq + hkv, liars=[9])
    print(f"[prefix groups] four planes hq={hq} hkv={hkv}", flush=True)
    hint = hint_for(case, hint_pages)
    assert hint.n_groups == len({d for d in depth if d >= 0})
    hinted = run(case, hint_pages)
    check(case, hinted)
    plain = run(case)
    assert torch.equal(hinted[[5, 17, 9]], plain[[5, 17, 9]])


@pytest.mark.parametrize("hq,hkv", [(16, 4), (8, 8), (32, 4)])
def test_many_groups_in_one_launch(hq, hkv):
    # 72 groups of two rows (prefixes of 16-40 pages, one row with no group per
    # eight): the item -> group search walks many groups, and each of the
    # launch's prefix workers computes several items in turn.
    g = torch.Generator().manual_seed(hq + 5 * hkv)
    groups = 72
    group_pages = torch.randint(16, 41, (groups,), generator=g).tolist()
    row_group = [r // 2 if r % 8 != 7 else -1 for r in range(2 * groups)]
    lengths = [int(group_pages[grp] * PAGE + torch.randint(1, 700, (1,), generator=g)) if grp >= 0
               else int(torch.randint(300, 1500, (1,), generator=g)) for grp in row_group]
    case, _, hint_pages = groups_case(lengths, row_group, group_pages, hq=hq, hkv=hkv, seed=hq * 7 + hkv)
    print(f"[prefix groups] {groups} groups hq={hq} hkv={hkv}", flush=True)
    hint = hint_for(case, hint_pages)
    assert hint.n_groups == len({grp for grp in row_group if grp >= 0})
    assert hint.n_items * hkv > 128  # more items than prefix workers
    hinted = run(case, hint_pages)
    check(case, hinted)
    plain = run(case)
    ungrouped = [r for r, grp in enumerate(row_group) if grp < 0]
    assert torch.equal(bits(hinted[ungrouped]), bits(plain[ungrouped]))


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 4)])
def test_512_token_splits_beside_256_token_splits(hq, hkv):
    # Rows past 16384 tokens use 512-token splits: the same 600 shared pages
    # form one group per split length.
    lengths = [17000, 20000, 16500, 9000, 17500, 12000]
    case, _, hint_pages = groups_case(lengths, [0] * 6, [600], hq=hq, hkv=hkv, seed=hq + hkv)
    print(f"[prefix groups] 512-token splits hq={hq} hkv={hkv}", flush=True)
    assert hint_for(case, hint_pages).n_groups == 2
    hinted = run(case, hint_pages)
    check(case, hinted)


def test_a_hint_for_a_split_length_no_member_uses_changes_nothing():
    lengths = [3000, 4000, 2500]
    case, _, hint_pages = groups_case(lengths, [0, 0, 0], [100], hq=8, hkv=8, seed=3)
    hinted = run(case, hint_pages, split_lengths=[20000, 20000, 20000])  # groups at 512-token splits
    assert torch.equal(hinted, run(case))


@pytest.mark.parametrize("dtype,d", [(torch.float32, 128), (torch.bfloat16, 64)])
def test_the_hint_is_ignored_where_the_pass_does_not_exist(dtype, d):
    lengths = [1000, 1300, 800]
    case, _, hint_pages = groups_case(lengths, [0, 0, 0], [40], hq=4, hkv=4, d=d, dtype=dtype, seed=11)
    hinted = run(case, hint_pages)
    assert torch.equal(hinted, run(case))
    check(case, hinted)


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 4)])
def test_a_rows_bits_do_not_depend_on_its_batch(hq, hkv):
    # Row 0 decoded alone (a group of one), in a batch of 40 members of its
    # group, and at another batch position among other groups' rows: the same
    # bits each time.
    lengths = torch.randint(700, 3000, (40,), generator=torch.Generator().manual_seed(8)).tolist()
    case, _, hint_pages = groups_case(lengths, [0] * 40, [44], hq=hq, hkv=hkv, seed=21)
    print(f"[prefix groups] batch invariance hq={hq} hkv={hkv}", flush=True)
    full = run(case, hint_pages)
    check(case, full)
    for rows in ([0], [0, 7, 30], list(range(39, -1, -1)), [12, 0, 3]):
        sub = DecodeCase(case.q[rows], case.key_pool, case.value_pool, 0, case.tables[rows], case.lengths[rows])
        out = run(sub, [hint_pages[r] for r in rows])
        for i, r in enumerate(rows):
            assert torch.equal(bits(out[i]), bits(full[r])), (rows, r)


@pytest.mark.parametrize("hq,hkv", [(16, 16), (32, 16)])
def test_fused_append_with_prefix_groups(hq, hkv):
    # rlt_paged_decode_shared_prefix with its append: the same pages and output
    # bits as kv_append followed by the hinted decode, the new tokens in place,
    # the shared pages untouched, and the oracle's attention.
    from vllm_rlt_amd import ops

    g = torch.Generator().manual_seed(hq)
    n = 20
    depth = torch.randint(0, 3, (n,), generator=g).tolist()
    depth[4] = -1
    contexts = torch.randint(800, 2000, (n,), generator=g).tolist()
    lengths = [c + 1 for c in contexts]
    case, shared, hint_pages = groups_case(lengths, depth, [32, 40, 48], hq=hq, hkv=hkv, seed=hq + 1)
    # The new token's slot holds NaN until the append writes it.
    blocks = torch.tensor([int(case.tables[r, c // PAGE]) for r, c in enumerate(contexts)])
    offsets = torch.tensor([c % PAGE for c in contexts])
    k_new = torch.randn(n, hkv, 128, generator=g).to(torch.bfloat16)
    v_new = torch.randn(n, hkv, 128, generator=g).to(torch.bfloat16)
    print(f"[prefix groups] fused append hq={hq} hkv={hkv}", flush=True)
    dev = case.to("cuda")
    hint = hint_for(case, hint_pages)
    fused = ops.paged_decode_append(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, k_new.cuda(),
                                    v_new.cuda(), blocks.cuda(), offsets.cuda(), shared_prefix=hint)
    torch.cuda.synchronize()
    two = case.to("cuda")
    ops.kv_append(two.key_pool, two.value_pool, 0, blocks.cuda(), offsets.cuda(), k_new.cuda(), v_new.cuda())
    split = ops.paged_decode(two.q, two.key_slice, two.value_slice, two.tables, two.lengths, shared_prefix=hint)
    torch.cuda.synchronize()
    assert torch.equal(bits(fused.cpu()), bits(split.cpu()))
    assert torch.equal(bits(dev.key_pool.cpu()), bits(two.key_pool.cpu()))
    assert torch.equal(bits(dev.value_pool.cpu()), bits(two.value_pool.cpu()))
    exp_k, exp_v = case.key_pool.clone(), case.value_pool.clone()
    kv_ops.append(exp_k, exp_v, 0, blocks.tolist(), offsets.tolist(), k_new, v_new)
    assert torch.equal(bits(dev.key_pool.cpu()), bits(exp_k)) and torch.equal(bits(dev.value_pool.cpu()), bits(exp_v))
    for ids in shared:
        assert torch.equal(bits(dev.key_pool.cpu()[ids.long()]), bits(case.key_pool[ids.long()]))
    expect = paged_attention_cpu(case.q, exp_k[:, 0], exp_v[:, 0], case.tables, case.lengths)
    torch.testing.assert_close(fused.cpu(), expect, atol=2e-2, rtol=1e-2)


def test_ouro_shape_with_a_long_prefix():
    # Ouro-1.4B heads over the prefix-stress shape: rows of 16-32K tokens
    # sharing an 8192-token prefix.
    g = torch.Generator().manual_seed(5)
    lengths = torch.randint(16384, 32769, (8,), generator=g).tolist()
    case, _, hint_pages = groups_case(lengths, [0] * 8, [512], hq=16, hkv=16, seed=5)
    check(case, run(case, hint_pages))


def test_prefix_group_arguments_are_checked():
    from dataclasses import replace

    from vllm_rlt_amd import ops

    case, _, hint_pages = groups_case([1000, 900], [0, 0], [40], hq=4, hkv=4, seed=2)
    dev = case.to("cuda")
    hint = hint_for(case, hint_pages)
    args = (dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths)
    with pytest.raises(ValueError, match="contiguous int32 hint for 2 rows"):
        ops.paged_decode(*args, shared_prefix=replace(hint, hint=hint.hint[:-1]))
    with pytest.raises(ValueError, match="contiguous int32 hint for 2 rows"):
        ops.paged_decode(*args, shared_prefix=replace(hint, n_rows=3))
    with pytest.raises(ValueError, match="wider than the block tables"):
        ops.paged_decode(*args, shared_prefix=replace(hint, n_pages=999, hint=torch.zeros(
            2 + 6 + 1 + 2 + 999, dtype=torch.int32, device="cuda")))
    # A hint sized for fewer q heads per KV head than the call has is not used.
    narrow = replace(hint, group_size=0)
    with pytest.raises(ValueError, match="group size"):
        ops._prefix_call(narrow, 2, dev.tables)


def test_a_corrupt_hint_is_bounds_checked_on_the_device():
    # Group records pointing past the member and page sections, a row group past
    # the group count, and an item count larger than the groups': the pass
    # ignores them and every row equals the plain decode.
    from dataclasses import replace

    from vllm_rlt_amd import ops

    case, _, hint_pages = groups_case([1000, 900, 1200], [0, 0, 0], [40], hq=4, hkv=4, seed=12)
    dev = case.to("cuda")
    hint = hint_for(case, hint_pages)
    plain = run(case)
    host = hint.hint.cpu()
    bad = host.clone()
    bad[3 + 0] = 50  # first member past the members section
    bad[3 + 2] = 1000  # first page past the pages section
    bad[0] = 7  # row 0 in a group that does not exist
    broken = replace(hint, hint=bad.cuda(), n_items=hint.n_items + 5)
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths, shared_prefix=broken)
    torch.cuda.synchronize()
    assert torch.equal(bits(out.cpu()), bits(plain))


def _published_prefix_cache(share, layers=1, planes=2, seed=21):
    """Request a publishes an 800-token prefix (50 pages per plane); b, c, d reuse it
    (tests/test_prefix_growth.py:47-64) and grow past it at every depth."""
    from vllm_rlt_amd import KVCacheManager

    cache = KVCacheManager(layers, 2, 128, 1024, 16, planes, device="cuda", dtype=torch.bfloat16,
                           enable_prefix_caching=True, share_prefix_reads=share)
    torch.manual_seed(seed)
    prompt = list(range(1000, 1801))
    assert cache.allocate("a", 1400)
    for layer in range(layers):
        for depth in range(planes):
            kv = torch.randn(800, 2, 128, device="cuda", dtype=torch.bfloat16)
            cache.write(layer, ["a"] * 800, [depth] * 800, list(range(800)), kv, -kv)
    cache.publish_prefix("a", prompt, 800)
    hit = cache.lookup_prefix(prompt)
    assert len(hit) == 50
    ends = {"a": 1100, "b": 1000, "c": 1290, "d": 900}
    for rid in ("b", "c", "d"):
        assert cache.allocate(rid, 1400, prefix=hit)
    for layer in range(layers):
        for rid, end in ends.items():
            for depth in range(planes):
                n = end - 800
                kv = torch.randn(n, 2, 128, device="cuda", dtype=torch.bfloat16)
                cache.write(layer, [rid] * n, [depth] * n, list(range(800, end)), kv, kv * 0.5)
    return cache, ends


@pytest.mark.parametrize("share", [False, True])
def test_manager_groups_rows_by_their_planes_prefix(share):
    # b, c, d took a's published prefix from the cache (50 pages per plane); a
    # batch of all four at mixed depths reads each plane's prefix once for the
    # rows that took it (a itself owns the pages it published).
    from dataclasses import replace

    cache, ends = _published_prefix_cache(share)
    ids = list(ends)
    depths = [1, 1, 0, 1]
    batch = cache._prepare_batch(ids, depths, [ends[r] - 1 for r in ids], for_write=False)
    q = torch.randn(4, 4, 128, device="cuda", dtype=torch.bfloat16)
    out = cache._attend_prepared(0, batch, q)
    expected = paged_attention_cpu(
        q.cpu(), cache.key_cache[:, 0].cpu(), cache.value_cache[:, 0].cpu(), batch.block_tables.cpu(),
        batch.context_lengths.cpu(),
    )
    torch.testing.assert_close(out.cpu(), expected, atol=2e-2, rtol=1e-2)
    if not share:
        assert batch.shared_prefix is None
        return
    hint = batch.shared_prefix
    assert hint.n_groups == 2 and hint.n_members == 3
    host = hint.hint.cpu().tolist()
    assert host[:4] == [-1, 0, 1, 0]  # b, d at plane 1; c at plane 0
    # Pages cut to whole 256-token splits: 48 of the 50 prefix pages.
    assert host[4:9] == [0, 2, 0, 48, 256] and host[9:14] == [2, 1, 48, 48, 256]
    pages = host[-96:]
    assert pages[:48] == list(cache.get_block_table("b", 1)[:48])
    assert pages[48:] == list(cache.get_block_table("c", 0)[:48])
    plain = cache._attend_prepared(0, replace(batch, shared_prefix=None), q)
    torch.testing.assert_close(out, plain, atol=2e-2, rtol=1e-2)


def test_manager_fused_write_attend_with_prefix_groups():
    # _write_attend_prepared takes the fused launch with the groups: same bits
    # as the two steps, every plane's prefix pages unchanged.
    cache, ends = _published_prefix_cache(True, planes=3, seed=31)
    ids = list(ends)
    depths = [2, 0, 1, 2]
    positions = [ends[r] for r in ids]
    prefix_ids = [cache.get_block_table("b", d)[:50] for d in range(3)]
    before = [cache.key_cache[list(p)].clone() for p in prefix_ids]
    q = torch.randn(4, 4, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(4, 2, 128, device="cuda", dtype=torch.bfloat16)
    v = torch.randn(4, 2, 128, device="cuda", dtype=torch.bfloat16)
    snapshot = cache.key_cache.clone(), cache.value_cache.clone()
    batch = cache._prepare_batch(ids, depths, positions)
    assert batch.shared_prefix is not None and batch.shared_prefix.n_groups == 3
    fused = cache._write_attend_prepared(0, batch, q, k, v)
    torch.cuda.synchronize()
    pools = cache.key_cache.clone(), cache.value_cache.clone()
    cache.key_cache.copy_(snapshot[0])
    cache.value_cache.copy_(snapshot[1])
    batch2 = cache._prepare_batch(ids, depths, positions)
    cache._write_prepared(0, batch2, k, v)
    two = cache._attend_prepared(0, batch2, q)
    torch.cuda.synchronize()
    assert torch.equal(bits(fused), bits(two))
    assert torch.equal(bits(pools[0]), bits(cache.key_cache)) and torch.equal(bits(pools[1]), bits(cache.value_cache))
    for p, b in zip(prefix_ids, before):
        assert torch.equal(bits(cache.key_cache[list(p)]), bits(b))


def test_prefix_group_decode_replays_in_a_graph():
    # A captured write+attend over rows that alias a published prefix (with
    # the groups) replays to the eager result every time, eager work between.
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
    assert batch.shared_prefix is not None and batch.shared_prefix.n_members == 2
    k = torch.randn(3, 2, 128, device="cuda", dtype=torch.bfloat16)
    q = torch.randn(3, 4, 128, device="cuda", dtype=torch.bfloat16)
    proxy = DeviceCache(cache, fused_append=True)

    def core():
        outs = []
        for layer in range(2):
            outs.append(proxy._write_attend_prepared(layer, batch, q, k + layer, k - layer))
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
