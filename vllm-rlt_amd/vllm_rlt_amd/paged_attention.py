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
    """Attention backend object for KVCacheManager(backend="hip").

    The object owns one grow-only device workspace for the decode split
    partials and the per-token prefill path, so steady-state calls allocate
    nothing.  It grows to the next power of two when a batch needs more
    (reserve() grows it ahead of a graph capture).  A buffer it outgrows is
    released, unless a graph was captured while it was the workspace: such a
    graph keeps reading that address, so the buffer stays alive with the
    object.  Graphs captured at growing sizes therefore hold less than the
    final workspace again (powers of two below it).  Calls on one object are
    meant to run on one stream, in order: two streams sharing the object at
    once would share the workspace.
    """

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
        self.device = device
        self.head_dim = head_dim
        self.block_size = block_size
        self._workspace = None
        self._captured = False  # a graph was captured reading the current workspace
        self._held = []  # outgrown workspaces a captured graph still reads
        self.info = dict(
            backend="hip",
            arch="gfx950",
            library=str(_native.LIBRARY_PATH.name),
            version=lib.rlt_version().decode(),
        )

    @property
    def workspace_bytes(self) -> int:
        return 0 if self._workspace is None else self._workspace.numel()

    @property
    def held_bytes(self) -> int:
        """Bytes of outgrown workspaces kept alive for captured graphs."""
        return sum(t.numel() for t in self._held)

    @staticmethod
    def workspace_size_for(nbytes: int) -> int:
        """Size the workspace grows to for a need of nbytes: a power of two, 1 MiB or more."""
        return 1 << max(20, (max(int(nbytes), 1) - 1).bit_length())

    def reserve(self, nbytes: int) -> torch.Tensor:
        """The workspace, grown to at least nbytes."""
        if self._workspace is None or self._workspace.numel() < int(nbytes):
            if self._workspace is not None and self._captured:
                self._held.append(self._workspace)
            elif self._workspace is not None:
                # Back to the caching allocator, reusable only once the work
                # queued on this stream (the object's stream) has finished.
                self._workspace.record_stream(torch.cuda.current_stream(self.device))
            self._workspace = None
            size = self.workspace_size_for(nbytes)
            self._workspace = torch.empty(size, dtype=torch.uint8, device=self.device)
            self._captured = False
        if torch.cuda.is_current_stream_capturing():
            self._captured = True
        return self._workspace

    def reserve_decode(self, rows: int, num_q_heads: int, num_kv_heads: int) -> torch.Tensor:
        """Grow the workspace for decode batches of up to `rows` rows."""
        return self.reserve(ops.decode_workspace_bytes(rows, num_q_heads, num_kv_heads, self.head_dim))

    def __call__(self, q, key_cache, value_cache, block_tables, context_lengths, shared_prefix=None):
        """Decode attention; `shared_prefix` (an ops.PrefixGroups, beyond the
        reference's signature) reads each group's aliased prefix pages once."""
        workspace = self.reserve_decode(q.shape[0], q.shape[1], key_cache.shape[2]) if q.shape[0] else None
        return ops.paged_decode(
            q, key_cache, value_cache, block_tables, context_lengths, workspace=workspace, shared_prefix=shared_prefix
        )

    def decode_append(self, q, key_cache, value_cache, block_tables, context_lengths, k_new, v_new, write_blocks,
                      write_offsets, n_write=None, shared_prefix=None):
        """Append rows' new K/V, then decode attention, in one launch (beyond the reference's interface).

        The caller guarantees that no row reads a slot another row writes.
        `shared_prefix` as for __call__.
        """
        workspace = self.reserve_decode(q.shape[0], q.shape[1], key_cache.shape[2]) if q.shape[0] else None
        return ops.paged_decode_append(
            q, key_cache, value_cache, block_tables, context_lengths, k_new, v_new, write_blocks, write_offsets,
            n_write=n_write, workspace=workspace, shared_prefix=shared_prefix,
        )

    def prefill(self, q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q, max_seqlen_q):
        """Packed ragged chunks over paged prefixes, bottom-right causal.

        Sequence s owns query rows cu_seqlens_q[s]:cu_seqlens_q[s+1]; its keys
        end at its last query, so query i of an n_q-token chunk sees
        context_lengths[s] - (n_q - 1 - i) keys (flash_attention.py:76-80).
        """
        need = ops.prefill_workspace_bytes(
            q.shape[0], block_tables.shape[0], block_tables.shape[1], q.shape[1], key_cache.shape[2], self.head_dim,
            self.block_size, q.dtype if ops.rows_aligned16(q, key_cache, value_cache) else torch.float32,
        )
        workspace = self.reserve(need) if need else None
        return ops.paged_prefill(
            q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q, max_seqlen_q, workspace=workspace
        )
