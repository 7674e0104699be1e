"""Full-size parity of the chunked-prefill and aliased-prefix workloads, and the
launch paths only large inputs reach (GPU).

* Chunked prefill at Ouro shape: 8 sequences x 512 new tokens over paged
  prefixes U[0, 16384], 16/16 heads x 128, page 16, bf16: the chunk's K/V are
  appended, then attended with bottom-right causal masking
  (tests/test_flash_attention.py:148-190 geometry at full size).  Sampled
  query rows (the first, a middle and the last row of every 128-row tile) are
  checked against the per-token CPU oracle.
* Aliased-prefix decode: 64 rows with contexts U[16384, 32768], an 8192-token
  prefix (512 pages) shared read-only by every table, page ids placed past
  element 2**32 of the pool (tests/test_attention_64bit.py:16-30,
  tests/test_prefix_growth.py:47-64), through the shared-prefix entry point.
* Prefix caching under LAST-EXITED (every plane its own 2048-token prefix,
  contexts U[4096, 8192], mixed depths): one fused append + decode launch with
  the step's prefix groups; all four planes' prefix pages stay bit-identical.
* More than 8192 decode rows (the entry point's per-launch row chunking) and
  a prefill whose block tables are wider than 4096 pages (the MFMA variant
  that reads page ids from the table instead of staging them in LDS).

Tolerances: bf16 max-abs 2e-2 / rel 1e-2.  Page contents: bit-exact.
"""

import math

import pytest
import torch

from oracle import kv_ops
from oracle.paged_attention import paged_attention_cpu
from paged_cases import random_decode_case

pytestmark = pytest.mark.gpu

BF16_TOL = dict(atol=2e-2, rtol=1e-2)
HEADS, HEAD_DIM, PAGE = 16, 128, 16


def _need_free(gib):
    if torch.cuda.mem_get_info()[0] < gib * 2**30:
        pytest.skip(f"needs {gib} GiB free device memory")


def _fp32_reference(q, key_slice, value_slice, table, length, scale):
    """Dense fp32 attention of one row on the device (gather, scores, softmax, values)."""
    t = torch.arange(length, device=q.device)
    pages = table[t // PAGE].long()
    k = key_slice[pages, t % PAGE].float()  # [n, hkv, d]
    v = value_slice[pages, t % PAGE].float()
    group = q.shape[0] // k.shape[1]
    k = k.repeat_interleave(group, dim=1).transpose(0, 1).contiguous()  # [h, n, d]
    v = v.repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
    scores = torch.matmul(k, q.float()[:, :, None])[..., 0] * scale  # [h, n]
    return torch.matmul(scores.softmax(-1)[:, None, :], v)[:, 0]  # [h, d]


def _host_pages(key_slice, value_slice, tables, lengths):
    """Host copies of the pages the given rows read, with the tables remapped onto them."""
    used = sorted({int(b) for row, n in enumerate(lengths) for b in tables[row, : -(-int(n) // PAGE)].tolist()})
    index = torch.tensor(used, dtype=torch.long, device=key_slice.device)
    remap = {b: i for i, b in enumerate(used)}
    small = torch.zeros(tables.shape, dtype=torch.int32)
    for row, n in enumerate(lengths):
        for col, b in enumerate(tables[row, : -(-int(n) // PAGE)].tolist()):
            small[row, col] = remap[int(b)]
    return key_slice[index].cpu(), value_slice[index].cpu(), small


# ---------------------------------------------------------------------------
# Chunked prefill at full size.


def test_chunked_prefill_ouro_full_size():
    from vllm_rlt_amd import ops

    _need_free(4)
    g = torch.Generator().manual_seed(4040)
    seqs, chunk = 8, 512
    prefixes = torch.randint(0, 16385, (seqs,), generator=g).tolist()
    prefixes[0] = 0  # one chunk over an empty prefix
    lens = [p + chunk for p in prefixes]
    pages = [math.ceil(n / PAGE) for n in lens]
    nb = sum(pages) + 8
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    tables = torch.full((seqs, max(pages)), -1, dtype=torch.int32)
    used = 0
    for s, p in enumerate(pages):
        tables[s, :p] = perm[used : used + p]
        used += p
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(4041)
    # Two layers; the chunk is written into and read from layer 1 (a strided slice).
    key_cache = torch.randn((nb, 2, PAGE, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    value_cache = torch.randn((nb, 2, PAGE, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    total = seqs * chunk
    q = torch.randn((total, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    k_new = torch.randn((total, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((total, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    positions = [p + i for p in prefixes for i in range(chunk)]
    rows_seq = [s for s in range(seqs) for _ in range(chunk)]
    blocks = torch.tensor([int(tables[s, pos // PAGE]) for s, pos in zip(rows_seq, positions)], dtype=torch.int64)
    offsets = torch.tensor([pos % PAGE for pos in positions], dtype=torch.int64)
    cu = torch.tensor([s * chunk for s in range(seqs + 1)], dtype=torch.int32)
    print(f"[prefill full size] prefixes={prefixes}", flush=True)

    touched = sorted(set(blocks.tolist()))
    before_k = key_cache[touched].cpu()
    before_v = value_cache[touched].cpu()
    ops.kv_append(key_cache, value_cache, 1, blocks.to(dev), offsets.to(dev), k_new, v_new)
    out = ops.paged_prefill(
        q, key_cache[:, 1], value_cache[:, 1], tables.to(dev), torch.tensor(lens, dtype=torch.int32, device=dev),
        cu.to(dev), chunk,
    )
    torch.cuda.synchronize()

    # The append, bit for bit against the oracle on host copies of the touched pages.
    remap = {b: i for i, b in enumerate(touched)}
    exp_k = before_k.view(torch.int16).numpy().copy()
    exp_v = before_v.view(torch.int16).numpy().copy()
    kv_ops.append(
        exp_k, exp_v, 1, [remap[b] for b in blocks.tolist()], offsets.tolist(),
        k_new.cpu().view(torch.int16).numpy(), v_new.cpu().view(torch.int16).numpy(),
    )
    assert (key_cache[touched].cpu().view(torch.int16).numpy() == exp_k).all()
    assert (value_cache[touched].cpu().view(torch.int16).numpy() == exp_v).all()

    # Attention: first, middle and last row of every 128-row query tile.
    sample = []
    for s in range(seqs):
        for t0 in range(0, chunk, 128):
            sample += [s * chunk + t0, s * chunk + t0 + 61, s * chunk + t0 + 127]
    row_tables = torch.stack([tables[rows_seq[r]] for r in sample])
    row_lengths = [positions[r] + 1 for r in sample]
    hk, hv, small = _host_pages(key_cache[:, 1], value_cache[:, 1], row_tables, row_lengths)
    expect = paged_attention_cpu(q[sample].cpu(), hk, hv, small, torch.tensor(row_lengths, dtype=torch.int32))
    torch.testing.assert_close(out[sample].cpu(), expect, **BF16_TOL)
    assert torch.isfinite(out).all()
    # Every row against a dense fp32 reference on the device.
    scale = HEAD_DIM**-0.5
    tables_dev = tables.to(dev)
    for r in range(0, total, 7):
        ref = _fp32_reference(q[r], key_cache[:, 1], value_cache[:, 1], tables_dev[rows_seq[r]], positions[r] + 1, scale)
        torch.testing.assert_close(out[r].float(), ref, **BF16_TOL)


def test_prefill_tables_wider_than_4096_pages():
    # One sequence of 65,600 keys needs 4,100 pages: the MFMA kernel then reads
    # page ids from the block table rather than staging the key range's ids in LDS.
    from vllm_rlt_amd import ops

    _need_free(2)
    g = torch.Generator().manual_seed(4100)
    hq = hkv = 4
    prefixes, chunks = [65400, 10, 0], [200, 70, 129]
    lens = [p + c for p, c in zip(prefixes, chunks)]
    pages = [math.ceil(n / PAGE) for n in lens]
    assert max(pages) > 4096
    nb = sum(pages) + 3
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    tables = torch.full((3, max(pages)), -1, dtype=torch.int32)
    used = 0
    for s, p in enumerate(pages):
        tables[s, :p] = perm[used : used + p]
        used += p
    key_pool = torch.randn(nb, PAGE, hkv, HEAD_DIM, generator=g).to(torch.bfloat16)
    value_pool = torch.randn(nb, PAGE, hkv, HEAD_DIM, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(chunks), hq, HEAD_DIM, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0] + torch.tensor(chunks).cumsum(0).tolist(), dtype=torch.int32)
    out = ops.paged_prefill(
        q.cuda(), key_pool.cuda(), value_pool.cuda(), tables.cuda(), torch.tensor(lens, dtype=torch.int32).cuda(),
        cu.cuda(), max(chunks),
    )
    torch.cuda.synchronize()
    row_seq = [s for s, c in enumerate(chunks) for _ in range(c)]
    row_len = [p + i + 1 for p, c in zip(prefixes, chunks) for i in range(c)]
    sample = list(range(0, 200, 9)) + [199] + list(range(200, len(row_seq)))
    expect = paged_attention_cpu(
        q[sample], key_pool, value_pool, torch.stack([tables[row_seq[r]] for r in sample]),
        torch.tensor([row_len[r] for r in sample], dtype=torch.int32),
    )
    torch.testing.assert_close(out.cpu()[sample], expect, **BF16_TOL)
    # The short sequences through tables cut to their own width (the LDS-staged
    # variant) agree with the wide-table launch.
    short = ops.paged_prefill(
        q[200:].cuda(), key_pool.cuda(), value_pool.cuda(), tables[1:, : max(pages[1:])].contiguous().cuda(),
        torch.tensor(lens[1:], dtype=torch.int32).cuda(), (cu[1:] - 200).cuda(), max(chunks[1:]),
    )
    torch.testing.assert_close(short.cpu(), out.cpu()[200:], **BF16_TOL)


# ---------------------------------------------------------------------------
# Decode row chunking.


def test_decode_more_than_8192_rows():
    # 8,300 rows: two launches of the split pass and merge, each chunk's q,
    # out, tables and lengths offset by the rows before it.
    from vllm_rlt_amd import ops

    g = torch.Generator().manual_seed(8300)
    lengths = torch.randint(0, 41, (8300,), generator=g).tolist()
    lengths[8191], lengths[8192], lengths[8299] = 40, 33, 17
    case = random_decode_case(lengths, hq=4, hkv=2, d=64, layers=1, layer=0, seed=8300)
    dev = case.to("cuda")
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths)
    torch.cuda.synchronize()
    expect = paged_attention_cpu(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    torch.testing.assert_close(out.cpu(), expect, **BF16_TOL)
    zero = case.lengths == 0
    assert torch.count_nonzero(out.cpu()[zero]) == 0
    # Rows past 8192 give the bits they give in a batch of their own.
    tail = ops.paged_decode(dev.q[8192:], dev.key_slice, dev.value_slice, dev.tables[8192:], dev.lengths[8192:])
    torch.testing.assert_close(tail, out[8192:], atol=0, rtol=0)


# ---------------------------------------------------------------------------
# Aliased-prefix decode at full size, page ids past element 2**32.


def test_aliased_prefix_decode_full_size_64bit_pages():
    from vllm_rlt_amd import ops

    _need_free(24)
    g = torch.Generator().manual_seed(5005)
    rows, prefix_tokens = 64, 8192
    prefix_pages = prefix_tokens // PAGE
    contexts = torch.randint(16384, 32769, (rows,), generator=g).tolist()
    lengths = [c + 1 for c in contexts]  # the appended token included
    own = [math.ceil(n / PAGE) - prefix_pages for n in lengths]
    # One layer: a block is 2**15 elements, so blocks >= 2**17 start past element 2**32.
    high = 1 << 17
    nb = high + prefix_pages + 64
    prefix = (high + torch.randperm(prefix_pages + 64, generator=g)[:prefix_pages]).to(torch.int32)
    private = torch.randperm(high, generator=g)[: sum(own)].to(torch.int32)
    width = max(own) + prefix_pages
    tables = torch.full((rows, width), -1, dtype=torch.int32)
    used = 0
    for r in range(rows):
        tables[r, :prefix_pages] = prefix
        tables[r, prefix_pages : prefix_pages + own[r]] = private[used : used + own[r]]
        used += own[r]
    dev = torch.device("cuda")
    shape = (nb, 1, PAGE, HEADS, HEAD_DIM)
    key_cache = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    value_cache = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(5006)
    for pool in (key_cache, value_cache):
        flat = pool.view(-1)
        for start in range(0, flat.numel(), 1 << 28):
            flat[start : start + (1 << 28)].normal_(generator=gen)
    q = torch.randn((rows, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    k_new = torch.randn((rows, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((rows, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    blocks = torch.tensor([int(tables[r, c // PAGE]) for r, c in enumerate(contexts)], dtype=torch.int64)
    offsets = torch.tensor([c % PAGE for c in contexts], dtype=torch.int64)
    prefix_dev = prefix.to(dev).long()
    snapshot = key_cache[prefix_dev].clone(), value_cache[prefix_dev].clone()
    print(f"[aliased prefix full size] max page id {int(tables.max())}, blocks >= {high} past element 2**32", flush=True)

    ops.kv_append(key_cache, value_cache, 0, blocks.to(dev), offsets.to(dev), k_new, v_new)
    tables_dev, lengths_dev = tables.to(dev), torch.tensor(lengths, dtype=torch.int32, device=dev)
    hint = ops.prefix_groups([prefix.tolist()] * rows, lengths, PAGE, 1, dev)
    assert hint.n_groups >= 1 and hint.n_members == rows
    out = ops.paged_decode(q, key_cache[:, 0], value_cache[:, 0], tables_dev, lengths_dev, shared_prefix=hint)
    plain = ops.paged_decode(q, key_cache[:, 0], value_cache[:, 0], tables_dev, lengths_dev)
    torch.cuda.synchronize()

    # The aliased pages are read-only: bit-identical after the append and both decodes.
    assert torch.equal(key_cache[prefix_dev], snapshot[0]) and torch.equal(value_cache[prefix_dev], snapshot[1])
    # The appended slots hold the new tokens exactly.
    assert torch.equal(key_cache[blocks.to(dev), 0, offsets.to(dev)], k_new)
    assert torch.equal(value_cache[blocks.to(dev), 0, offsets.to(dev)], v_new)
    # Sampled rows against the CPU oracle on host copies of their pages.
    sample = [0, 21, 42, 63]
    hk, hv, small = _host_pages(key_cache[:, 0], value_cache[:, 0], tables[sample], [lengths[r] for r in sample])
    expect = paged_attention_cpu(q[sample].cpu(), hk, hv, small, torch.tensor([lengths[r] for r in sample], dtype=torch.int32))
    torch.testing.assert_close(out[sample].cpu(), expect, **BF16_TOL)
    # Every row against a dense fp32 device reference, and the hinted launch
    # against the plain one.
    scale = HEAD_DIM**-0.5
    for r in range(rows):
        ref = _fp32_reference(q[r], key_cache[:, 0], value_cache[:, 0], tables_dev[r], lengths[r], scale)
        torch.testing.assert_close(out[r].float(), ref, **BF16_TOL)
    torch.testing.assert_close(out, plain, **BF16_TOL)


def test_last_exited_prefix_groups_full_size():
    """Prefix caching under the reference's own semantics at the bench shape: 64
    requests, contexts U[4096, 8192], four LAST-EXITED planes, each plane's tables
    beginning with that plane's 2048-token prefix, every request at a depth drawn
    from U{1..4}; the fused append with the step's prefix groups."""
    from vllm_rlt_amd import ops

    _need_free(12)
    g = torch.Generator().manual_seed(7007)
    rows, planes, prefix_pages = 64, 4, 2048 // PAGE
    contexts = torch.randint(4096, 8193, (rows,), generator=g).tolist()
    depths = torch.randint(0, planes, (rows,), generator=g).tolist()
    lengths = [c + 1 for c in contexts]
    own = [math.ceil(n / PAGE) - prefix_pages for n in lengths]
    nb = planes * prefix_pages + planes * sum(own) + 8
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    prefixes = perm[: planes * prefix_pages].view(planes, prefix_pages)
    used = planes * prefix_pages
    width = max(own) + prefix_pages
    plane_tables = torch.full((rows, planes, width), -1, dtype=torch.int32)
    for r in range(rows):
        for p in range(planes):
            plane_tables[r, p, :prefix_pages] = prefixes[p]
            plane_tables[r, p, prefix_pages : prefix_pages + own[r]] = perm[used : used + own[r]]
            used += own[r]
    tables = plane_tables[torch.arange(rows), torch.tensor(depths)].contiguous()  # depth-resolved rows
    dev = torch.device("cuda")
    shape = (nb, 1, PAGE, HEADS, HEAD_DIM)
    key_cache = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    value_cache = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(7008)
    for pool in (key_cache, value_cache):
        flat = pool.view(-1)
        for start in range(0, flat.numel(), 1 << 28):
            flat[start : start + (1 << 28)].normal_(generator=gen)
    q = torch.randn((rows, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    k_new = torch.randn((rows, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((rows, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    blocks = torch.tensor([int(tables[r, c // PAGE]) for r, c in enumerate(contexts)], dtype=torch.int64)
    offsets = torch.tensor([c % PAGE for c in contexts], dtype=torch.int64)
    prefix_dev = prefixes.reshape(-1).long().to(dev)
    snapshot = key_cache[prefix_dev].clone(), value_cache[prefix_dev].clone()
    groups = ops.prefix_groups([prefixes[d].tolist() for d in depths], lengths, PAGE, 1, dev)
    assert groups.n_groups == len(set(depths)) and groups.n_members == rows
    print(f"[LAST-EXITED prefix groups full size] {groups.n_groups} groups, {nb} pages", flush=True)

    tables_dev, lengths_dev = tables.to(dev), torch.tensor(lengths, dtype=torch.int32, device=dev)
    out = ops.paged_decode_append(
        q, key_cache[:, 0], value_cache[:, 0], tables_dev, lengths_dev, k_new, v_new, blocks.to(dev),
        offsets.to(dev), shared_prefix=groups,
    )
    torch.cuda.synchronize()
    # Every plane's prefix pages are read-only: bit-identical after the fused launch.
    assert torch.equal(key_cache[prefix_dev], snapshot[0]) and torch.equal(value_cache[prefix_dev], snapshot[1])
    # The appended slots hold the new tokens exactly.
    assert torch.equal(key_cache[blocks.to(dev), 0, offsets.to(dev)], k_new)
    assert torch.equal(value_cache[blocks.to(dev), 0, offsets.to(dev)], v_new)
    # Sampled rows (one per plane at least) against the CPU oracle on host copies of their pages.
    sample = sorted({0, rows - 1, *[depths.index(p) for p in set(depths)]})
    hk, hv, small = _host_pages(key_cache[:, 0], value_cache[:, 0], tables[sample], [lengths[r] for r in sample])
    expect = paged_attention_cpu(q[sample].cpu(), hk, hv, small, torch.tensor([lengths[r] for r in sample], dtype=torch.int32))
    torch.testing.assert_close(out[sample].cpu(), expect, **BF16_TOL)
    # Every row against a dense fp32 device reference, and against the plain decode.
    scale = HEAD_DIM**-0.5
    for r in range(rows):
        ref = _fp32_reference(q[r], key_cache[:, 0], value_cache[:, 0], tables_dev[r], lengths[r], scale)
        torch.testing.assert_close(out[r].float(), ref, **BF16_TOL)
    plain = ops.paged_decode(q, key_cache[:, 0], value_cache[:, 0], tables_dev, lengths_dev)
    torch.testing.assert_close(out, plain, **BF16_TOL)
