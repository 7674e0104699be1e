"""The ctypes binding's stream and stride-array helpers (GPU)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_stream_handle_is_torchs_current_stream():
    from vllm_rlt_amd import _native

    dev = torch.device("cuda:0")
    assert _native.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    side = torch.cuda.Stream(device=dev)  # default priority
    with torch.cuda.stream(side):
        assert _native.stream_handle(dev) == side.cuda_stream
        assert _native.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    assert _native.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    torch.cuda.synchronize()


def test_launch_on_a_side_stream_orders_with_that_stream():
    from vllm_rlt_amd import ops

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    blocks, page, hkv, d = 8, 16, 2, 64
    kc = torch.zeros(blocks, 1, page, hkv, d, dtype=torch.float32, device=dev)
    vc = torch.zeros_like(kc)
    k = torch.randn(4, hkv, d, generator=g).to(dev)
    v = torch.randn(4, hkv, d, generator=g).to(dev)
    b = torch.tensor([1, 3, 5, 7], dtype=torch.int64, device=dev)
    o = torch.tensor([0, 2, 15, 9], dtype=torch.int64, device=dev)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        ops.kv_append(kc, vc, 0, b, o, k, v)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    for i in range(4):
        assert torch.equal(kc[b[i], 0, o[i]], k[i])
        assert torch.equal(vc[b[i], 0, o[i]], v[i])

