"""The "hip" attention backend: decode and packed-prefill paged attention on gfx950.

HipPagedAttention has the surface the reference's cache manager and runner
use on an attention backend object (vllm_rlt/kernels/flash_attention.py:34-130):
a decode __call__, a packed-prefill .prefill(...) and an .info dict.  Instead
of impersonating FlashAttention-4 through `.generation == 4`, it advertises
packed prefill with its own capability flag, `supports_packed_prefill`.
"""

from __future__ import annotations

import torch

from . import _native, ops

SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def hip_paged_attention(
    q: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lengths: torch.Tensor,
) -> torch.Tensor:
    """Explicit HIP dispatch with no fallback (cf. triton_paged_attention, paged_attention.py:39-54)."""
    if q.device.type != "cuda" or not torch.version.hip:
        raise ValueError("the hip attention backend requires a ROCm device")
    return ops.paged_decode(q, key_cache, value_cache, block_tables, context_lengths)


class HipPagedAttention:
    """Attention backend object for KVCacheManager(backend="hip")."""

    generation = None
    supports_packed_prefill = True

    def __init__(self, device, dtype, head_dim, block_size):
        device = torch.device(device)
        if device.type != "cuda" or not torch.version.hip:
            raise ValueError("the hip attention backend requires a ROCm device")
        if dtype not in SUPPORTED_DTYPES:
            raise ValueError("KV dtype must be float32, float16, or bfloat16")
        if head_dim <= 0 or head_dim > 512:
            raise ValueError("the hip attention backend supports head_dim <= 512")
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        lib = _native.load()
        self.head_dim = head_dim
        self.block_size = block_size
        self.info = dict(
            backend="hip",
            arch="gfx950",
            library=str(_native.LIBRARY_PATH.name),
            version=lib.rlt_version().decode(),
        )

    def __call__(self, q, key_cache, value_cache, block_tables, context_lengths, shared_prefix=None):
        """Decode attention; `shared_prefix` (an ops.SharedPrefix, beyond the
        reference's signature) reads rows' aliased prefix pages once."""
        return ops.paged_decode(q, key_cache, value_cache, block_tables, context_lengths, shared_prefix=shared_prefix)

    def prefill(self, q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q, max_seqlen_q):
        """Packed ragged chunks over paged prefixes, bottom-right causal.

        Sequence s owns query rows cu_seqlens_q[s]:cu_seqlens_q[s+1]; its keys
        end at its last query, so query i of an n_q-token chunk sees
        context_lengths[s] - (n_q - 1 - i) keys (flash_attention.py:76-80).
        """
        return ops.paged_prefill(q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q, max_seqlen_q)
