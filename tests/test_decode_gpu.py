"""HIP paged decode / packed prefill attention against the CPU oracle (GPU).

Tolerances: bf16 max-abs 2e-2 / rel 1e-2, fp16 2e-3, fp32 1e-5 (atol and rtol).
"""

import math

import pytest
import torch

from oracle.paged_attention import paged_attention_cpu
from paged_cases import DecodeCase, random_decode_case

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-3, 2e-3), torch.float32: (1e-5, 1e-5)}

# Ragged lengths covering: empty rows, a single token, page and split edges,
# several 256-token splits.
LENGTHS = [0, 1, 15, 16, 17, 255, 256, 257, 300, 0, 600, 1029]


def run_hip(case):
    from vllm_rlt_amd import ops

    dev = case.to("cuda")
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths)
    torch.cuda.synchronize()
    return out.cpu()


def expected(case):
    return paged_attention_cpu(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)


def assert_close(actual, case):
    atol, rtol = TOL[case.q.dtype]
    torch.testing.assert_close(actual, expected(case), atol=atol, rtol=rtol)
    assert torch.isfinite(actual).all()
    zero = case.lengths == 0
    assert torch.count_nonzero(actual[zero]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hq,hkv", [(16, 16), (8, 4), (16, 4), (16, 2), (32, 8), (32, 4), (64, 8)])
def test_tiled_decode_matches_oracle(dtype, hq, hkv):
    case = random_decode_case(LENGTHS, hq=hq, hkv=hkv, d=128, dtype=dtype, seed=hq * 31 + hkv)
    assert_close(run_hip(case), case)


@pytest.mark.parametrize("d", [128, 256])
def test_tiled_decode_long_rows_many_splits(d):
    # 33 to 65 splits per row: the merge's further load batches (beyond the first
    # 64 / (d / 64) splits) and the doubled split length past 64 splits.
    case = random_decode_case([8449, 12000, 16640, 300, 0], hq=4, hkv=4, d=d, dtype=torch.bfloat16, seed=d + 5)
    assert_close(run_hip(case), case)


# Split counts at the merge's load-batch edges: the first batch holds 16 splits,
# later batches 48 (head_dim 64 and 128) or 24 (head_dim 256).
MERGE_EDGE_SPLITS = [1, 2, 15, 16, 17, 40, 47, 48, 49, 63, 64]


@pytest.mark.parametrize(
    "d,dtype,hq,hkv",
    [(64, torch.bfloat16, 4, 4), (128, torch.bfloat16, 4, 4), (256, torch.bfloat16, 4, 4),
     (64, torch.float32, 4, 4), (128, torch.float32, 2, 2), (128, torch.bfloat16, 16, 4)],
)
def test_merge_batch_edges(d, dtype, hq, hkv):
    lengths = [200 if ns == 1 else ns * 256 - 7 * ns % 256 for ns in MERGE_EDGE_SPLITS]
    case = random_decode_case(lengths, hq=hq, hkv=hkv, d=d, dtype=dtype, seed=d + hq)
    print(f"[merge edges] d={d} dtype={dtype} hq={hq} hkv={hkv}", flush=True)
    assert_close(run_hip(case), case)


@pytest.mark.parametrize("hq,hkv", [(16, 4), (32, 4)])
def test_grouped_query_rows_past_65536_tokens(hq, hkv):
    # Rows past 65536 tokens get 2048-token splits, which the grouped-query
    # items on the matrix cores walk in several 64-page table chunks.
    case = random_decode_case([70000, 131072, 5000, 0], hq=hq, hkv=hkv, d=128, dtype=torch.bfloat16, seed=hq + hkv)
    print(f"[decode long gqa] hq={hq} hkv={hkv}", flush=True)
    assert_close(run_hip(case), case)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 256])
def test_tiled_decode_other_head_dims(dtype, d):
    if dtype == torch.float32 and d == 256:
        d = 128
    case = random_decode_case(LENGTHS[:9], hq=4, hkv=4, d=d, dtype=dtype, seed=d)
    assert_close(run_hip(case), case)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d,page,hq,hkv", [(7, 3, 6, 2), (32, 5, 2, 1), (128, 8, 6, 2), (100, 16, 3, 3)])
def test_generic_decode_matches_oracle(dtype, d, page, hq, hkv):
    # Shapes outside the tiled kernel (odd head_dim, page != 16, group 3) use the generic kernel.
    case = random_decode_case([0, 1, 7, 40, 71], hq=hq, hkv=hkv, d=d, page=page, dtype=dtype, seed=d + page)
    assert_close(run_hip(case), case)


def test_online_softmax_scaled_inputs():
    # x8-scaled q/k (tests/test_attention.py:63-79), long rows: large score ranges.
    for dtype in (torch.bfloat16, torch.float32):
        case = random_decode_case([71, 513, 2000], hq=16, hkv=16, d=128, dtype=dtype, seed=89, scale=8.0)
        assert_close(run_hip(case), case)


def test_poisoned_slots_never_reach_the_output():
    # Page tails and unused blocks hold NaN; padding may be -1 or 0.
    for pad in (-1, 0):
        case = random_decode_case(LENGTHS, d=128, seed=7, pad=pad, fill_unused=float("nan"))
        assert_close(run_hip(case), case)


def test_stale_workspace_slots_never_reach_the_output():
    # The merge loads every split slot of a (row, head) before it knows the row's
    # split count and discards the slots past it: a workspace full of NaN from
    # earlier launches must not leak into rows of 1, 2 or 5 splits, or 33+.
    from vllm_rlt_amd import ops

    lengths = [1, 200, 256, 257, 300, 1029, 0, 8449, 40]
    case = random_decode_case(lengths, hq=8, hkv=4, d=128, dtype=torch.bfloat16, seed=77).to("cuda")
    nbytes = ops.decode_workspace_bytes(len(lengths), 8, 4, 128)
    workspace = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")  # every float slot is NaN
    out = ops.paged_decode(case.q, case.key_slice, case.value_slice, case.tables, case.lengths, workspace=workspace)
    torch.cuda.synchronize()
    assert_close(out.cpu(), case.to("cpu"))


@pytest.mark.parametrize("hq,hkv", [(16, 16), (32, 4)])
def test_rows_are_batch_invariant(hq, hkv):
    # tests/test_flash_attention.py:193-208: a row's bits do not depend on the batch around it
    # (also for the grouped-query items on the matrix cores).
    from vllm_rlt_amd import ops

    case = random_decode_case([1025, 1029, 1025, 1031, 3, 4000], hq=hq, hkv=hkv, d=128, seed=1234).to("cuda")
    together = ops.paged_decode(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    for rows in ([2, 3], [3, 0], [1], [5, 4, 0]):
        idx = torch.tensor(rows, device="cuda")
        separate = ops.paged_decode(case.q[idx], case.key_slice, case.value_slice, case.tables[idx], case.lengths[idx])
        torch.testing.assert_close(separate, together[idx], rtol=0, atol=0)


def test_strided_query_and_output_views():
    from vllm_rlt_amd import ops

    case = random_decode_case([33, 300], hq=16, hkv=16, d=128, seed=3).to("cuda")
    wide = torch.zeros(2, 32, 128, dtype=case.q.dtype, device="cuda")
    wide[:, ::2] = case.q
    out_wide = torch.zeros_like(wide)
    ops.paged_decode(wide[:, ::2], case.key_slice, case.value_slice, case.tables, case.lengths, out=out_wide[:, 1::2])
    plain = ops.paged_decode(case.q, case.key_slice, case.value_slice, case.tables, case.lengths)
    torch.testing.assert_close(out_wide[:, 1::2], plain, rtol=0, atol=0)
    assert torch.count_nonzero(out_wide[:, ::2]) == 0


def test_64bit_offsets_exact_answer():
    # tests/test_attention_64bit.py:16-30: block 2048 x stride 2**20 = 2**31 elements.
    from vllm_rlt_amd import ops

    if torch.cuda.mem_get_info()[0] < 9 * 2**30:
        pytest.skip("needs 9 GiB free device memory")
    shape, strides = (2049, 1, 1, 16), (2**20, 16, 16, 1)
    key = torch.empty_strided(shape, strides, device="cuda", dtype=torch.float16)
    value = torch.empty_strided(shape, strides, device="cuda", dtype=torch.float16)
    key[0].zero_()
    value[0].fill_(-3)
    key[2048].fill_(1)
    expect = torch.arange(16, device="cuda", dtype=torch.float16).view(1, 1, 16)
    value[2048].copy_(expect)
    q = torch.ones((1, 1, 16), device="cuda", dtype=torch.float16)
    table = torch.tensor([[2048]], device="cuda", dtype=torch.int32)
    out = ops.paged_decode(q, key, value, table, torch.tensor([1], device="cuda", dtype=torch.int32))
    torch.cuda.synchronize()
    torch.testing.assert_close(out, expect, rtol=0, atol=0)


def test_64bit_offsets_tiled_kernel():
    # Ouro-shaped bf16 pages at a 2**21-element block stride: block 2048 starts at
    # element 2**32 (8 GiB), beyond both int32 element and byte offsets.
    from vllm_rlt_amd import ops

    if torch.cuda.mem_get_info()[0] < 18 * 2**30:
        pytest.skip("needs 18 GiB free device memory")
    shape, strides = (2049, 16, 16, 128), (2**21, 2048, 128, 1)
    key = torch.empty_strided(shape, strides, device="cuda", dtype=torch.bfloat16)
    value = torch.empty_strided(shape, strides, device="cuda", dtype=torch.bfloat16)
    used = [2048, 3, 1500, 0]
    g = torch.Generator().manual_seed(64)
    small_k = torch.randn(len(used), 16, 16, 128, generator=g).to(torch.bfloat16)
    small_v = torch.randn(len(used), 16, 16, 128, generator=g).to(torch.bfloat16)
    for i, b in enumerate(used):
        key[b].copy_(small_k[i])
        value[b].copy_(small_v[i])
    q = torch.randn(2, 16, 128, generator=g).to(torch.bfloat16)
    tables = torch.tensor([[2048, 3, 1500, 0], [1500, 2048, 0, 0]], dtype=torch.int32)
    lengths = torch.tensor([61, 20], dtype=torch.int32)
    out = ops.paged_decode(q.cuda(), key, value, tables.cuda(), lengths.cuda())
    torch.cuda.synchronize()
    remap = {b: i for i, b in enumerate(used)}
    small_tables = tables.clone().apply_(lambda b: remap[b])
    expect = paged_attention_cpu(q, small_k, small_v, small_tables, lengths)
    torch.testing.assert_close(out.cpu(), expect, atol=2e-2, rtol=1e-2)


def test_config1_append_then_decode():
    # Batch 4, 16/16 heads, head_dim 128, page 16, contexts U[1,256], one token
    # appended per row before attention, bf16 N(0,1), random free-page permutation.
    from oracle import kv_ops
    from vllm_rlt_amd import ops

    g = torch.Generator().manual_seed(2024)
    contexts = torch.randint(1, 257, (4,), generator=g).tolist()
    lengths = [c + 1 for c in contexts]
    case = random_decode_case(lengths, d=128, layers=1, layer=0, seed=2024)
    k_new = torch.randn(4, 16, 128, generator=g).to(torch.bfloat16)
    v_new = torch.randn(4, 16, 128, generator=g).to(torch.bfloat16)
    blocks = torch.tensor([int(case.tables[r, c // 16]) for r, c in enumerate(contexts)], dtype=torch.int64)
    offsets = torch.tensor([c % 16 for c in contexts], dtype=torch.int64)
    key_pool, value_pool = case.key_pool.clone(), case.value_pool.clone()
    kv_ops.append(key_pool, value_pool, 0, blocks, offsets, k_new, v_new)
    expect = paged_attention_cpu(case.q, key_pool[:, 0], value_pool[:, 0], case.tables, case.lengths)
    dev = case.to("cuda")
    ops.kv_append(dev.key_pool, dev.value_pool, 0, blocks.cuda(), offsets.cuda(), k_new.cuda(), v_new.cuda())
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths)
    torch.cuda.synchronize()
    # Compare raw bits: the pools hold NaN poison in unused slots.
    assert torch.equal(dev.key_pool.cpu().view(torch.int16), key_pool.view(torch.int16))
    assert torch.equal(dev.value_pool.cpu().view(torch.int16), value_pool.view(torch.int16))
    torch.testing.assert_close(out.cpu(), expect, atol=2e-2, rtol=1e-2)


def test_ouro_shape_sampled_rows_and_uniform_query():
    # Config-2 geometry (64 rows, contexts U[512, 4096]); oracle on a sample of rows,
    # and the size-independent property q = 0 -> mean(V) on every row.
    from vllm_rlt_amd import ops

    g = torch.Generator().manual_seed(77)
    lengths = torch.randint(512, 4097, (64,), generator=g).tolist()
    case = random_decode_case(lengths, d=128, layers=1, layer=0, seed=77, spare_blocks=0)
    dev = case.to("cuda")
    out = ops.paged_decode(dev.q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths).cpu()
    sample = [0, 17, 40, 63]
    sub = DecodeCase(case.q[sample], case.key_pool, case.value_pool, 0, case.tables[sample], case.lengths[sample])
    torch.testing.assert_close(out[sample], expected(sub), atol=2e-2, rtol=1e-2)
    zero_q = torch.zeros_like(dev.q)
    mean = ops.paged_decode(zero_q, dev.key_slice, dev.value_slice, dev.tables, dev.lengths).float()
    for row in range(64):
        n = lengths[row]
        t = torch.arange(n, device="cuda")
        vals = dev.value_slice[dev.tables[row, t // 16].long(), t % 16].float().mean(0)
        torch.testing.assert_close(mean[row], vals, atol=2e-2, rtol=1e-2)


def prefill_case(dtype, seed=712):
    """3 packed sequences over ragged prefixes (tests/test_flash_attention.py:148-190 geometry)."""
    g = torch.Generator().manual_seed(seed)
    page, hkv, hq, d = 16, 2, 4, 64
    specs = [(0, 19), (17, 7), (31, 18)]  # (prefix, chunk)
    pages = [math.ceil((p + c) / page) for p, c in specs]
    nb = sum(pages) + 4
    perm = torch.randperm(nb, generator=g)
    key_pool = torch.randn(nb, 2, page, hkv, d, generator=g).to(dtype)
    value_pool = torch.randn(nb, 2, page, hkv, d, generator=g).to(dtype)
    width = max(pages)
    tables = torch.full((3, width), -1, dtype=torch.int32)
    used = 0
    for s, p in enumerate(pages):
        tables[s, :p] = perm[used : used + p].to(torch.int32)
        used += p
    q = torch.randn(sum(c for _, c in specs), hq, d, generator=g).to(dtype)
    cu = torch.tensor([0, 19, 26, 44], dtype=torch.int32)
    lengths = torch.tensor([p + c for p, c in specs], dtype=torch.int32)
    # The per-token oracle: every chunk row is its own decode row.
    row_tables = torch.cat([tables[s].repeat(c, 1) for s, (_, c) in enumerate(specs)])
    row_lengths = torch.tensor([p + i + 1 for p, c in specs for i in range(c)], dtype=torch.int32)
    return q, key_pool, value_pool, tables, lengths, cu, row_tables, row_lengths


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mfma_prefill_empty_and_single_token_sequences(dtype):
    # Sequences with no new token (equal cu_seqlens entries) between others,
    # a one-token chunk over an empty prefix (one key) and one over a long
    # prefix: the empty sequences own no rows, and every row of the others
    # matches the per-token oracle.
    from vllm_rlt_amd import ops

    prefixes, chunks = [40, 0, 700, 0, 1500, 33], [0, 1, 0, 130, 1, 0]
    lens = [p + c for p, c in zip(prefixes, chunks)]
    live = [i for i, c in enumerate(chunks) if c > 0]
    q, kp, vp, tables, _, cu, row_tables, row_lengths = ragged_prefill_case(
        dtype, 16, 16, 128, [prefixes[i] for i in live], [chunks[i] for i in live], 11
    )
    # Re-pack with the empty sequences in place: their tables point at valid pages, their q rows are none.
    full_tables = torch.full((len(chunks), tables.shape[1]), -1, dtype=torch.int32)
    for k, i in enumerate(live):
        full_tables[i] = tables[k]
    for i, c in enumerate(chunks):
        if c == 0:
            pages = -(-lens[i] // 16)
            full_tables[i, :pages] = tables[0, 0]
    full_cu = torch.tensor([0] + torch.tensor(chunks).cumsum(0).tolist(), dtype=torch.int32)
    print(f"[prefill empty] chunks={chunks} prefixes={prefixes} {dtype}", flush=True)
    out = torch.full_like(q, 7.0).cuda()
    ops.paged_prefill(
        q.cuda(), kp.cuda(), vp.cuda(), full_tables.cuda(), torch.tensor(lens, dtype=torch.int32).cuda(),
        full_cu.cuda(), max(chunks), out=out,
    )
    torch.cuda.synchronize()
    expect = paged_attention_cpu(q, kp, vp, row_tables, row_lengths)
    atol, rtol = TOL[dtype]
    torch.testing.assert_close(out.cpu(), expect, atol=atol, rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,d", [(16, 16, 128), (4, 2, 64)])
def test_mfma_prefill_context_shorter_than_chunk(dtype, hq, hkv, d):
    # Query row i of a chunk sees context_length - (chunk - 1 - i) keys, none
    # when that is not positive: such rows are zeros, like the per-token
    # oracle's zero-length rows -- including whole 128-row query tiles that see
    # nothing (chunk 300 over 20 keys: rows 0-279), and a sequence with no keys.
    from vllm_rlt_amd import ops

    chunks, contexts = [300, 200, 5, 40], [20, 0, 3, 40]
    q, kp, vp, tables, _, cu, row_tables, _ = ragged_prefill_case(dtype, hq, hkv, d, [0] * 4, chunks, 31)
    row_lengths = torch.tensor(
        [max(0, n - (c - 1 - i)) for n, c in zip(contexts, chunks) for i in range(c)], dtype=torch.int32
    )
    print(f"[prefill short context] chunks={chunks} contexts={contexts} hq={hq} d={d} {dtype}", flush=True)
    out = torch.full_like(q, 7.0).cuda()
    ops.paged_prefill(
        q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), torch.tensor(contexts, dtype=torch.int32).cuda(),
        cu.cuda(), max(chunks), out=out,
    )
    torch.cuda.synchronize()
    expect = paged_attention_cpu(q, kp, vp, row_tables, row_lengths)
    assert torch.count_nonzero(out.cpu()[row_lengths == 0]) == 0
    atol, rtol = TOL[dtype]
    torch.testing.assert_close(out.cpu(), expect, atol=atol, rtol=rtol)


@pytest.mark.parametrize("num_seqs", [137, 512, 513])
def test_mfma_prefill_many_sequences(num_seqs):
    # The ranked work list sorts and scans the sequences in the workgroup (up to
    # 512 of them: 137 and 512 are ranked, 513 falls back to the direct list),
    # with short chunks over short prefixes so that most query tiles are alone.
    from vllm_rlt_amd import ops

    g = torch.Generator().manual_seed(7000 + num_seqs)
    prefixes = [int(x) for x in torch.randint(0, 80, (num_seqs,), generator=g)]
    chunks = [int(x) for x in torch.randint(1, 5, (num_seqs,), generator=g)]
    q, kp, vp, tables, lens, cu, row_tables, row_lengths = ragged_prefill_case(
        torch.bfloat16, 8, 8, 128, prefixes, chunks, num_seqs
    )
    print(f"[prefill many] num_seqs={num_seqs} rows={sum(chunks)}", flush=True)
    out = ops.paged_prefill(q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), lens.cuda(), cu.cuda(), max(chunks))
    torch.cuda.synchronize()
    expect = paged_attention_cpu(q, kp, vp, row_tables, row_lengths)
    atol, rtol = TOL[torch.bfloat16]
    torch.testing.assert_close(out.cpu(), expect, atol=atol, rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_packed_prefill_matches_per_token_oracle(dtype):
    from vllm_rlt_amd.paged_attention import HipPagedAttention

    q, kp, vp, tables, lengths, cu, row_tables, row_lengths = prefill_case(dtype)
    attention = HipPagedAttention(torch.device("cuda"), dtype, 64, 16)
    for layer in range(2):
        out = attention.prefill(
            q.cuda(), kp[:, layer].cuda(), vp[:, layer].cuda(), tables.cuda(), lengths.cuda(), cu.cuda(), 19
        )
        torch.cuda.synchronize()
        expect = paged_attention_cpu(q, kp[:, layer], vp[:, layer], row_tables, row_lengths)
        atol, rtol = TOL[dtype]
        torch.testing.assert_close(out.cpu(), expect, atol=atol, rtol=rtol)


def ragged_prefill_case(dtype, hq, hkv, d, prefixes, chunks, seed):
    """Packed chunks over paged prefixes with random page permutations, plus its per-token oracle rows."""
    g = torch.Generator().manual_seed(seed)
    page = 16
    lens = [p + c for p, c in zip(prefixes, chunks)]
    pages = [math.ceil(n / page) for n in lens]
    nb = sum(pages) + 3
    perm = torch.randperm(nb, generator=g)
    key_pool = torch.randn(nb, page, hkv, d, generator=g).to(dtype)
    value_pool = torch.randn(nb, page, hkv, d, generator=g).to(dtype)
    width = max(pages)
    tables = torch.full((len(lens), width), -1, dtype=torch.int32)
    used = 0
    for s, p in enumerate(pages):
        tables[s, :p] = perm[used : used + p].to(torch.int32)
        used += p
    # Slots past each sequence's last key hold NaN: the kernels must not read them.
    for s, n in enumerate(lens):
        if n % page:
            key_pool[int(tables[s, pages[s] - 1]), n % page :] = float("nan")
            value_pool[int(tables[s, pages[s] - 1]), n % page :] = float("nan")
    q = torch.randn(sum(chunks), hq, d, generator=g).to(dtype)
    cu = torch.tensor([0] + list(torch.tensor(chunks).cumsum(0).tolist()), dtype=torch.int32)
    row_tables = torch.cat([tables[s].repeat(c, 1) for s, c in enumerate(chunks)])
    row_lengths = torch.tensor([p + i + 1 for p, c in zip(prefixes, chunks) for i in range(c)], dtype=torch.int32)
    return q, key_pool, value_pool, tables, torch.tensor(lens, dtype=torch.int32), cu, row_tables, row_lengths


@pytest.mark.parametrize(
    "dtype,hq,hkv,d",
    [
        (torch.bfloat16, 16, 16, 128),
        (torch.float16, 16, 16, 128),
        (torch.bfloat16, 8, 4, 128),
        (torch.bfloat16, 4, 4, 64),
        (torch.float32, 4, 4, 128),
    ],
)
def test_mfma_prefill_ragged_chunks_over_long_prefixes(dtype, hq, hkv, d):
    # Chunks that end mid-tile, a one-token chunk, prefixes past several key tiles.
    from vllm_rlt_amd import ops

    prefixes, chunks = [0, 300, 1000, 2900, 17], [256, 130, 65, 1, 200]
    q, kp, vp, tables, lens, cu, row_tables, row_lengths = ragged_prefill_case(dtype, hq, hkv, d, prefixes, chunks, 4)
    out = ops.paged_prefill(q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), lens.cuda(), cu.cuda(), max(chunks))
    torch.cuda.synchronize()
    expect = paged_attention_cpu(q, kp, vp, row_tables, row_lengths)
    atol, rtol = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-3, 2e-3), torch.float32: (1e-5, 1e-5)}[dtype]
    torch.testing.assert_close(out.cpu(), expect, atol=atol, rtol=rtol)


@pytest.mark.parametrize("d", [64, 128])
def test_mfma_prefill_negative_scale_negates_scores(d):
    # scale -1/sqrt(d) over q equals the reference's 1/sqrt(d) over -q (sign flips are exact).
    from vllm_rlt_amd import ops

    prefixes, chunks = [70, 0, 513], [129, 64, 33]
    q, kp, vp, tables, lens, cu, row_tables, row_lengths = ragged_prefill_case(
        torch.bfloat16, 8, 8, d, prefixes, chunks, 9
    )
    out = ops.paged_prefill(
        q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), lens.cuda(), cu.cuda(), max(chunks), scale=-(d**-0.5)
    )
    torch.cuda.synchronize()
    expect = paged_attention_cpu(-q, kp, vp, row_tables, row_lengths)
    torch.testing.assert_close(out.cpu(), expect, atol=2e-2, rtol=1e-2)
    with pytest.raises(ValueError, match="scale"):
        ops.paged_prefill(q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), lens.cuda(), cu.cuda(), 129, scale=0.0)


@pytest.mark.parametrize("seed", range(8))
def test_mfma_prefill_random_shapes(seed):
    # Seeded random packed batches: odd and even key-tile counts (the second key
    # group's last tile may not exist), one-tile workgroups, chunks shorter
    # than a wave's rows (waves wholly past the chunk), diagonal tiles at every
    # offset, GQA, both dtypes and head sizes, ranked and direct work lists.
    from vllm_rlt_amd import ops

    g = torch.Generator().manual_seed(1000 + seed)
    n = int(torch.randint(1, 6, (1,), generator=g))
    prefixes = [int(x) for x in torch.randint(0, 700, (n,), generator=g)]
    chunks = [int(x) for x in torch.randint(1, 300, (n,), generator=g)]
    if seed % 3 == 0:
        prefixes[0] = 0  # a chunk over an empty prefix
    if seed % 4 == 1:
        chunks[-1] = 64 * int(torch.randint(1, 4, (1,), generator=g))  # chunk ending on a tile edge
    hq, hkv = [(16, 16), (8, 2), (4, 4), (16, 4)][seed % 4]
    d = 64 if seed % 5 == 4 else 128
    dtype = torch.float16 if seed % 2 else torch.bfloat16
    q, kp, vp, tables, lens, cu, row_tables, row_lengths = ragged_prefill_case(
        dtype, hq, hkv, d, prefixes, chunks, seed
    )
    print(f"[prefill random] seed={seed} prefixes={prefixes} chunks={chunks} hq={hq} hkv={hkv} d={d} {dtype}", flush=True)
    out = ops.paged_prefill(q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), lens.cuda(), cu.cuda(), max(chunks))
    torch.cuda.synchronize()
    expect = paged_attention_cpu(q, kp, vp, row_tables, row_lengths)
    atol, rtol = TOL[dtype]
    torch.testing.assert_close(out.cpu(), expect, atol=atol, rtol=rtol)
