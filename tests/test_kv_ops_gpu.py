"""HIP KV movement kernels are bit-exact against the numpy oracle (GPU)."""

import numpy as np
import pytest
import torch

from oracle import kv_ops

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]
BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw storage bits of a tensor on the host (bf16 has no numpy dtype)."""
    return t.contiguous().view(BITS[t.dtype]).cpu().numpy()


def random_bits(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    info = torch.iinfo(BITS[dtype])
    raw = torch.randint(info.min, info.max, shape, generator=g, dtype=torch.int64).to(BITS[dtype])
    return raw.view(dtype)


def pool(shape, dtype, seed):
    return random_bits(shape, dtype, seed).cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("contiguous", [True, False])
def test_append_is_bit_exact_and_touches_only_its_slots(dtype, contiguous):
    from vllm_rlt_amd import ops

    nb, layers, page, hkv, d = 23, 3, 16, 4, 64
    kc, vc = pool((nb, layers, page, hkv, d), dtype, 1), pool((nb, layers, page, hkv, d), dtype, 2)
    rows = 9
    if contiguous:
        k, v = pool((rows, hkv, d), dtype, 3), pool((rows, hkv, d), dtype, 4)
    else:  # head-major source: [rows, hkv, d] view with a non-standard head stride
        k = pool((hkv, rows, d), dtype, 3).transpose(0, 1)
        v = pool((hkv, rows, d), dtype, 4).transpose(0, 1)
    g = torch.Generator().manual_seed(5)
    slots = torch.randperm(nb * page, generator=g)[:rows]
    blocks = (slots // page).cuda()
    offsets = (slots % page).cuda()
    expect_k, expect_v = bits(kc), bits(vc)
    n_rows = rows - 2  # trailing padding rows must not be written
    kv_ops.append(expect_k, expect_v, 2, blocks.cpu().numpy(), offsets.cpu().numpy(), bits(k), bits(v), n_rows)
    ops.kv_append(kc, vc, 2, blocks, offsets, k, v, n_rows=n_rows)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(kc), expect_k)
    np.testing.assert_array_equal(bits(vc), expect_v)


def test_append_skips_out_of_range_addresses():
    from vllm_rlt_amd import ops

    kc, vc = pool((4, 1, 16, 2, 64), torch.bfloat16, 1), pool((4, 1, 16, 2, 64), torch.bfloat16, 2)
    before_k, before_v = bits(kc), bits(vc)
    k = pool((3, 2, 64), torch.bfloat16, 3)
    blocks = torch.tensor([-1, 4, 1], device="cuda")
    offsets = torch.tensor([0, 0, 16], device="cuda")
    ops.kv_append(kc, vc, 0, blocks, offsets, k, k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(kc), before_k)
    np.testing.assert_array_equal(bits(vc), before_v)


@pytest.mark.parametrize("dtype", DTYPES)
def test_copy_token_matches_oracle(dtype):
    from vllm_rlt_amd import ops

    kc, vc = pool((12, 5, 4, 2, 32), dtype, 7), pool((12, 5, 4, 2, 32), dtype, 8)
    expect_k, expect_v = bits(kc), bits(vc)
    kv_ops.copy_token(expect_k, expect_v, 3, [7, 1, 10], 2)
    ops.kv_copy_token(kc, vc, 3, [7, 1, 10], 2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(kc), expect_k)
    np.testing.assert_array_equal(bits(vc), expect_v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_batched_finalize_matches_oracle(dtype):
    from vllm_rlt_amd import ops

    layers, page, planes, width, slots = 3, 16, 4, 5, 6
    nb = slots * planes * width + 3
    kc, vc = pool((nb, layers, page, 2, 64), dtype, 9), pool((nb, layers, page, 2, 64), dtype, 10)
    g = torch.Generator().manual_seed(12)
    tables = torch.randperm(nb, generator=g)[: slots * planes * width].reshape(slots, planes, width).to(torch.int32)
    desc = torch.tensor([[0, 0, 5], [1, 1, 17], [2, 3, 70], [4, 2, 33], [5, 0, 79]], dtype=torch.int64)
    expect_k, expect_v = bits(kc), bits(vc)
    kv_ops.finalize_batched(desc.numpy(), tables.numpy(), expect_k, expect_v, max_loops=planes, page=page)
    ops.kv_finalize(desc.cuda(), tables.cuda(), kc, vc, max_loops=planes)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(kc), expect_k)
    np.testing.assert_array_equal(bits(vc), expect_v)


def test_batched_finalize_reads_pinned_host_descriptors():
    from vllm_rlt_amd import ops

    kc, vc = pool((40, 2, 16, 2, 64), torch.bfloat16, 13), pool((40, 2, 16, 2, 64), torch.bfloat16, 14)
    tables = torch.arange(40, dtype=torch.int32)[:32].reshape(2, 4, 4)
    desc = torch.tensor([[1, 0, 20], [0, 2, 3]], dtype=torch.int64).pin_memory()
    expect_k, expect_v = bits(kc), bits(vc)
    kv_ops.finalize_batched(desc.numpy(), tables.numpy(), expect_k, expect_v, max_loops=4, page=16)
    ops.kv_finalize(desc, tables.cuda(), kc, vc, max_loops=4)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(kc), expect_k)
    np.testing.assert_array_equal(bits(vc), expect_v)


@pytest.mark.parametrize("dtype", DTYPES)
def test_gather_matches_oracle(dtype):
    from vllm_rlt_amd import ops

    kc, vc = pool((20, 3, 16, 4, 32), dtype, 15), pool((20, 3, 16, 4, 32), dtype, 16)
    table = torch.tensor([13, 2, 19, 7], dtype=torch.int32)
    out_k, out_v = ops.kv_gather(kc, vc, 1, table.cuda(), 53)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out_k), kv_ops.gather(bits(kc), 1, table.numpy(), 53, 16))
    np.testing.assert_array_equal(bits(out_v), kv_ops.gather(bits(vc), 1, table.numpy(), 53, 16))


@pytest.mark.parametrize("planes", [1, 4])
def test_decode_metadata_matches_oracle(planes):
    from vllm_rlt_amd import ops

    slots, width, page = 5, 40, 16
    g = torch.Generator().manual_seed(21)
    tables = torch.randint(0, 10_000, (slots, planes, width), generator=g, dtype=torch.int32)
    count, size, out_width = 7, 10, 23
    desc = torch.stack(
        [
            torch.randint(0, slots, (count,), generator=g),
            torch.randint(0, planes, (count,), generator=g),
            torch.randint(0, out_width * page, (count,), generator=g),
        ],
        dim=1,
    ).to(torch.int64)
    expect = kv_ops.decode_metadata(desc.numpy(), count, size, tables.numpy(), page, out_width)
    dev = lambda shape, dt: torch.full(shape, -7, dtype=dt, device="cuda")  # noqa: E731
    out = dict(
        slots=dev((size,), torch.int64),
        positions=dev((size,), torch.int64),
        lengths=dev((size,), torch.int32),
        blocks=dev((size,), torch.int64),
        offsets=dev((size,), torch.int64),
        tables=dev((size, width), torch.int32),
    )
    ops.build_decode_metadata(
        desc.cuda(), count, size, tables.cuda(), page, out["slots"], out["positions"], out["lengths"],
        out["blocks"], out["offsets"], out["tables"], out_width,
    )
    torch.cuda.synchronize()
    for name in ("slots", "positions", "lengths"):
        np.testing.assert_array_equal(out[name].cpu().numpy(), expect[name])
    np.testing.assert_array_equal(out["blocks"][:count].cpu().numpy(), expect["blocks"])
    np.testing.assert_array_equal(out["offsets"][:count].cpu().numpy(), expect["offsets"])
    assert (out["blocks"][count:] == -7).all()  # padding rows get no write address
    np.testing.assert_array_equal(out["tables"][:, :out_width].cpu().numpy(), expect["tables"][:, :out_width])
    assert (out["tables"][:, out_width:] == -7).all()


def test_prefill_stage_and_expand_match_oracle():
    from vllm_rlt_amd import ops

    src = torch.tensor([3, -1, 2**33 + 7, 12, 0], dtype=torch.int64).pin_memory()
    wide = torch.empty(5, dtype=torch.int64, device="cuda")
    narrow = torch.empty(5, dtype=torch.int32, device="cuda")
    ops.stage_prefill(src, wide, narrow, 5)
    expect_wide, expect_narrow = kv_ops.stage_prefill(src.numpy())
    tables = torch.tensor([[9, 8, 7], [6, 5, 4]], dtype=torch.int32)
    positions = torch.tensor([0, 5, 9, 4, 47], dtype=torch.int64)
    sequences = torch.tensor([0, 0, 1, 1, 1], dtype=torch.int64)
    blocks = torch.empty(5, dtype=torch.int64, device="cuda")
    offsets = torch.empty(5, dtype=torch.int64, device="cuda")
    ops.expand_prefill(positions.cuda(), sequences.cuda(), tables.cuda(), 16, blocks, offsets, 5)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(wide.cpu().numpy(), expect_wide)
    np.testing.assert_array_equal(narrow.cpu().numpy(), expect_narrow)
    expect_blocks, expect_offsets = kv_ops.expand_prefill(positions.numpy(), sequences.numpy(), tables.numpy(), 16)
    np.testing.assert_array_equal(blocks.cpu().numpy(), expect_blocks)
    np.testing.assert_array_equal(offsets.cpu().numpy(), expect_offsets)
