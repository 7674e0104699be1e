"""Rotary position embedding of Ouro's attention, restated on the CPU (test infrastructure only).

The reference computes the rotary angles once per traversal and applies them
to q and k of every layer before the KV write:

* angles, cos, sin: OuroRotaryEmbedding (vllm_rlt/models/ouro.py:39-70).
  inv_freq = 1 / theta ** (arange(0, D, 2) / D) in float32; angles =
  positions.float()[:, None] * inv_freq, duplicated to D columns; cos and sin
  are taken in float32 and rounded to the activation dtype.
* apply: q * cos + rotate_half(q) * sin (vllm_rlt/models/ouro.py:73-75,
  108-109), with rotate_half(x) = cat(-x[D/2:], x[:D/2]).  Each product and
  the sum round to the activation dtype (torch elementwise semantics).
* the rotated k (and the unrotated v) are then written to the pages
  (vllm_rlt/models/ouro.py:110 -> kv_cache_manager.py:531-532).

Pinned by the reference's own output bits on seeded inputs
(tests/golden/rotary_cpu.npz, written by tests/golden/make_reference_goldens.py),
by position 0 being the identity, and by an independent float64 complex-number
rotation (tests/test_rope_oracle.py).
"""

from __future__ import annotations

import torch


def rotary_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype: torch.dtype):
    """(cos, sin), each [N, head_dim] in `dtype`, for int positions [N] (ouro.py:45-70)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    angles = positions.float().unsqueeze(-1) * inv_freq.float()
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos().to(dtype), angles.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """cat(-second half, first half) along the last dim (ouro.py:73-75)."""
    first, second = x.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [N, H, D] rotated by per-row cos/sin [N, D] (ouro.py:108-109)."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    return x * cos + rotate_half(x) * sin


def rope_append(key_pool, value_pool, layer, write_blocks, write_offsets, q, k, v, cos, sin, n_rows=None):
    """Rotate q and k, write rotated k and v to the pages; returns rotated q.

    The first n_rows rows are written (kv_cache_manager.py:531); q is rotated
    for every row.  Pools are torch tensors [blocks, layers, page, hkv, d].
    """
    q_rot = apply_rotary(q, cos, sin)
    k_rot = apply_rotary(k, cos, sin)
    n = len(write_blocks) if n_rows is None else n_rows
    for i in range(n):
        key_pool[int(write_blocks[i]), layer, int(write_offsets[i])] = k_rot[i]
        value_pool[int(write_blocks[i]), layer, int(write_offsets[i])] = v[i]
    return q_rot
