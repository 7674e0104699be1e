"""The C-ABI library loads, exports every declared symbol and validates arguments (CPU only)."""

import ctypes
import re

import pytest

from conftest import REPO


def _library():
    from vllm_rlt_amd import _native

    if not _native.LIBRARY_PATH.exists():
        from vllm_rlt_amd._build import build

        build()
    return _native.load(), _native


def declared_functions():
    text = (REPO / "include" / "rlt_kv.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rlt_\w+)\s*\(", text)))


def test_header_declares_the_bound_api():
    from vllm_rlt_amd import _native

    assert declared_functions() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib, _ = _library()
    raw = ctypes.CDLL(str(lib._name))
    missing = [name for name in declared_functions() if not hasattr(raw, name)]
    assert not missing, f"librlt_kv.so lacks {missing}"
    assert lib.rlt_version().decode().endswith("gfx950")


def test_invalid_arguments_are_rejected_before_any_launch():
    lib, native = _library()
    strides = native.int64_array([1, 1, 1, 1, 1])
    # Unknown dtype: nothing is enqueued, a message is recorded.
    rc = lib.rlt_kv_append(None, None, strides, None, strides, None, strides, None, None, 1, 0, 1, 1, 1, 1, 1, 99, None)
    assert rc == native.RLT_EINVAL
    assert "dtype" in native.last_error()
    # Layer out of range.
    rc = lib.rlt_kv_append(None, None, strides, None, strides, None, strides, None, None, 1, 5, 2, 4, 16, 1, 8, 2, None)
    assert rc == native.RLT_EINVAL and "layer" in native.last_error()
    # Query heads must be a multiple of KV heads (kv_cache_manager.py:491-492 wording).
    rc = lib.rlt_paged_decode(
        None, strides, None, None, strides, None, 1, 1, None, None, strides, 1, 3, 2, 8, 16, 4, 1.0, 2, None, 0, None
    )
    assert rc == native.RLT_EINVAL and "positive multiple" in native.last_error()
    # Too small a workspace is its own status.
    rc = lib.rlt_paged_decode(
        1, strides, 1, 1, strides, 1, 1, 1, 1, 1, strides, 4, 16, 16, 128, 16, 4, 1.0, 2, 16, 0, None
    )
    assert rc == native.RLT_EWORKSPACE
    with pytest.raises(ValueError, match="workspace"):
        native.check(rc, "rlt_paged_decode")
    # Fused rotary append: odd head_dim and n_write > n_rows are refused on the host.
    s3 = native.int64_array([1, 1, 1])
    s2 = native.int64_array([1, 1])
    rc = lib.rlt_rope_kv_append(
        1, 1, strides, 1, s3, 1, s3, 1, s3, 1, 1, s2, 1, s3, 1, 1, 2, 2, 0, 1, 4, 16, 2, 2, 7, 2, None
    )
    assert rc == native.RLT_EINVAL and "even" in native.last_error()
    rc = lib.rlt_rope_kv_append(
        1, 1, strides, 1, s3, 1, s3, 1, s3, 1, 1, s2, 1, s3, 1, 1, 2, 3, 0, 1, 4, 16, 2, 2, 8, 2, None
    )
    assert rc == native.RLT_EINVAL and "n_write" in native.last_error()
    # Exit-copy targets are validated on the host.
    dst = native.int64_array([3])
    rc = lib.rlt_kv_copy_token(1, 1, strides, 3, dst, 1, 0, 1, 8, 4, 1, 8, 2, None)
    assert rc == native.RLT_EINVAL and "source" in native.last_error()
    # Prefix groups: missing buffer, group, member and page counts.
    decode = (1, strides, 1, 1, strides, 1, 64, 64, 1, 1, strides, 4, 16, 16, 128, 16, 4096, 1.0, 2)
    append = (None, None, None, None, None, None, 0)
    tail = (16, 1 << 30, None)
    rc = lib.rlt_paged_decode_shared_prefix(*decode, *append, None, 1, 2, 32, 32, *tail)
    assert rc == native.RLT_EINVAL and "NULL prefix_groups" in native.last_error()
    rc = lib.rlt_paged_decode_shared_prefix(*decode, *append, 1, 0, 2, 32, 32, *tail)
    assert rc == native.RLT_EINVAL and "n_groups" in native.last_error()
    rc = lib.rlt_paged_decode_shared_prefix(*decode, *append, 1, 1, 5, 32, 32, *tail)
    assert rc == native.RLT_EINVAL and "n_members" in native.last_error()
    rc = lib.rlt_paged_decode_shared_prefix(*decode, *append, 1, 1, 2, 0, 32, *tail)
    assert rc == native.RLT_EINVAL and "n_pages" in native.last_error()
    rc = lib.rlt_paged_decode_shared_prefix(*decode, *append, 1, 1, 2, 65, 32, *tail)
    assert rc == native.RLT_EINVAL and "n_pages" in native.last_error()
    rc = lib.rlt_paged_decode_shared_prefix(*decode, *append, 1, 1, 2, 32, -1, *tail)
    assert rc == native.RLT_EINVAL and "n_items" in native.last_error()
    # Items x KV heads (16 here) must fit the workers' 32-bit item indices.
    rc = lib.rlt_paged_decode_shared_prefix(*decode, *append, 1, 1, 2, 32, (1 << 31) // 16, *tail)
    assert rc == native.RLT_EINVAL and "n_items x num_kv_heads" in native.last_error()


def test_workspace_sizes_depend_only_on_shape():
    lib, _ = _library()
    one = lib.rlt_paged_decode_workspace_bytes(64, 16, 16, 128)
    assert one > 0
    assert lib.rlt_paged_decode_workspace_bytes(64, 16, 16, 128) == one
    assert lib.rlt_paged_decode_workspace_bytes(128, 16, 16, 128) > one
    assert lib.rlt_paged_decode_workspace_bytes(0, 16, 16, 128) == 0
    # bf16, head_dim 128, page 16: the MFMA path needs no workspace; fp32 takes the decode-row path.
    assert lib.rlt_paged_prefill_workspace_bytes(4096, 8, 1057, 16, 16, 128, 16, 2) == 0
    assert lib.rlt_paged_prefill_workspace_bytes(4096, 8, 1057, 16, 16, 128, 16, 0) > 0


def test_ops_refuse_cpu_tensors():
    import torch

    from vllm_rlt_amd import ops
    from vllm_rlt_amd.paged_attention import HipPagedAttention, hip_paged_attention

    q = torch.zeros(1, 2, 8)
    cache = torch.zeros(4, 16, 2, 8)
    tables = torch.zeros(1, 1, dtype=torch.int32)
    lengths = torch.ones(1, dtype=torch.int32)
    with pytest.raises(ValueError, match="ROCm"):
        ops.paged_decode(q, cache, cache, tables, lengths)
    with pytest.raises(ValueError, match="ROCm"):
        hip_paged_attention(q, cache, cache, tables, lengths)
    with pytest.raises(ValueError, match="ROCm"):
        HipPagedAttention(torch.device("cpu"), torch.bfloat16, 128, 16)


def test_int64_arrays_are_shared_by_value():
    from vllm_rlt_amd import _native

    strides = _native.int64_array((2048, 128, 1))
    assert _native.int64_array([2048, 128, 1]) is strides
    assert list(strides) == [2048, 128, 1]
    assert list(_native.int64_array(list(range(20)))) == list(range(20))
    assert list(_native.int64_array([])) == []
