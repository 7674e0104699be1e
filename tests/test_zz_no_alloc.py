"""rlt_paged_decode_no_alloc against rlt_paged_decode, both through the C ABI (GPU).

The allocation-free entry point keeps the split-K partials in the library's
static per-device array instead of a caller workspace.  Its output must equal
rlt_paged_decode's bit for bit (a row's bits depend only on that row), over
two calls in a row (the second smaller, so stale partials of the first are in
the array), a batch longer than one of its row chunks, and a graph capture,
where no allocation may happen.
"""

import pytest
import torch

from paged_cases import random_decode_case

pytestmark = pytest.mark.gpu


def _args(dev, rows):
    from vllm_rlt_amd import _native

    i64 = _native.int64_array
    nb, page, hkv, d = dev.key_slice.shape
    return [
        dev.q.data_ptr(), i64(dev.q.stride()), dev.key_slice.data_ptr(), dev.value_slice.data_ptr(),
        i64(dev.key_slice.stride()), dev.tables.data_ptr(), dev.tables.stride(0), dev.tables.shape[1],
        dev.lengths.data_ptr(), None, None, rows, dev.q.shape[1], hkv, d, page, nb, d**-0.5,
        _native.dtype_code(dev.q.dtype),
    ]


def with_workspace(dev):
    from vllm_rlt_amd import _native

    lib = _native.load()
    rows = dev.q.shape[0]
    out = torch.empty_like(dev.q)
    need = lib.rlt_paged_decode_workspace_bytes(rows, dev.q.shape[1], dev.key_slice.shape[2], dev.q.shape[2])
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev.q.device)
    args = _args(dev, rows)
    args[9], args[10] = out.data_ptr(), _native.int64_array(out.stride())
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(lib.rlt_paged_decode(*args, ws.data_ptr(), need, stream), "rlt_paged_decode")
    return out


def no_alloc(dev, out=None):
    from vllm_rlt_amd import _native

    lib = _native.load()
    out = torch.empty_like(dev.q) if out is None else out
    args = _args(dev, dev.q.shape[0])
    args[9], args[10] = out.data_ptr(), _native.int64_array(out.stride())
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(lib.rlt_paged_decode_no_alloc(*args, stream), "rlt_paged_decode_no_alloc")
    return out


def _same_bits(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_no_alloc_decode_equals_workspace_decode_twice_in_a_row():
    # Ouro heads; contexts spanning one to many splits, an empty row.
    first = random_decode_case([700, 0, 4100, 1, 2333, 256, 257, 9000], seed=71).to("cuda")
    second = random_decode_case([3000, 17, 600], seed=72).to("cuda")
    for case in (first, second):
        expect = with_workspace(case)
        got = no_alloc(case)
        torch.cuda.synchronize()
        print(f"[no_alloc] rows={case.q.shape[0]} max_abs_diff={float((got.float() - expect.float()).abs().max())}",
              flush=True)
        assert _same_bits(got, expect)


def test_no_alloc_decode_walks_row_chunks():
    from vllm_rlt_amd import _native

    per = _native.load().rlt_paged_decode_no_alloc_rows_per_launch(16, 16, 128)
    assert 64 <= per < 300
    g = torch.Generator().manual_seed(73)
    lengths = torch.randint(1, 2000, (300,), generator=g).tolist()
    case = random_decode_case(lengths, layers=1, layer=0, seed=73).to("cuda")
    expect = with_workspace(case)
    got = no_alloc(case)
    torch.cuda.synchronize()
    assert _same_bits(got, expect)


def test_no_alloc_decode_replays_in_a_graph():
    case = random_decode_case([900, 40, 3000], hq=8, hkv=4, seed=74).to("cuda")
    expect = with_workspace(case)
    out = torch.empty_like(case.q)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        no_alloc(case, out)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        no_alloc(case, out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert _same_bits(out, expect)
        _ = with_workspace(random_decode_case([50, 60], seed=75).to("cuda"))  # eager work between replays


def test_no_alloc_decode_rejects_rows_larger_than_the_scratch():
    from vllm_rlt_amd import _native

    lib = _native.load()
    # 64 query heads x head_dim 4096: one row needs just over 64 MiB of partials.
    assert lib.rlt_paged_decode_no_alloc_rows_per_launch(64, 64, 4096) == 0
    # Real device buffers of the declared shapes (one row of one token over one
    # page), so that even a launch past a broken size check reads and writes
    # valid memory and the assert, not the device, reports the regression.
    hq, d, page = 64, 4096, 16
    q = torch.zeros(1, hq, d, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros_like(q)
    kc = torch.zeros(1, page, hq, d, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    tables = torch.zeros(1, 1, dtype=torch.int32, device="cuda")
    lengths = torch.ones(1, dtype=torch.int32, device="cuda")
    qs = _native.int64_array(q.stride())
    kvs = _native.int64_array(kc.stride())
    rc = lib.rlt_paged_decode_no_alloc(
        q.data_ptr(), qs, kc.data_ptr(), vc.data_ptr(), kvs, tables.data_ptr(), 1, 1, lengths.data_ptr(),
        out.data_ptr(), _native.int64_array(out.stride()), 1, hq, hq, d, page, 1, 1.0, _native.RLT_BFLOAT16,
        torch.cuda.current_stream().cuda_stream,
    )
    torch.cuda.synchronize()
    assert rc == _native.RLT_EUNSUPPORTED and "static scratch" in _native.last_error()
