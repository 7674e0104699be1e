"""CPU restatements of paged decode attention (test infrastructure only).

paged_attention_cpu follows the reference CPU path step for step
(vllm_rlt/kernels/paged_attention.py:12-36): for each row, gather the row's
tokens through its block table, widen KV heads to query heads, take fp32
products scaled by 1/sqrt(head_dim), softmax in fp32, weight the values in
fp32 and round the result to the query dtype.  It is the tolerance oracle for
the HIP kernel and the timed CPU baseline.
"""

from __future__ import annotations

import math

import numpy as np
import torch
from torch.nn import functional as F


def paged_attention_cpu(
    q: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lengths: torch.Tensor,
) -> torch.Tensor:
    """q [rows, hq, d]; caches [blocks, page, hkv, d] (layer slices); tables int32 [rows, W]."""
    page = key_cache.shape[1]
    group = q.shape[1] // key_cache.shape[2]
    inv_sqrt_d = 1.0 / math.sqrt(q.shape[-1])
    result = torch.empty_like(q)
    lengths = [int(x) for x in context_lengths.tolist()]
    for row, n in enumerate(lengths):
        if n == 0:
            result[row] = 0
            continue
        pos = torch.arange(n, device=q.device)
        pages = block_tables[row, pos // page].long()
        slots = pos % page
        keys = key_cache[pages, slots]  # [n, hkv, d]
        vals = value_cache[pages, slots]
        if group > 1:
            keys = keys.repeat_interleave(group, dim=1)
            vals = vals.repeat_interleave(group, dim=1)
        logits = torch.einsum("hd,nhd->hn", q[row].float(), keys.float()) * inv_sqrt_d
        weights = torch.softmax(logits, dim=-1)
        result[row] = torch.einsum("hn,nhd->hd", weights, vals.float()).to(q.dtype)
    return result


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Dense SDPA of one query row q [hq, d] over k, v [n, hkv, d] (tests/test_attention.py:8-15)."""
    group = q.shape[0] // k.shape[1]
    kk = k.float().repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
    vv = v.float().repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
    out = F.scaled_dot_product_attention(q.float()[None, :, None], kk[None], vv[None])
    return out[0, :, 0].to(q.dtype)


def paged_attention_f64(q, key_cache, value_cache, block_tables, context_lengths) -> np.ndarray:
    """Independent float64 evaluation (numpy, explicit max-shifted exponentials)."""
    q = np.asarray(torch.as_tensor(q).float(), dtype=np.float64)
    kc = np.asarray(torch.as_tensor(key_cache).float(), dtype=np.float64)
    vc = np.asarray(torch.as_tensor(value_cache).float(), dtype=np.float64)
    tables = np.asarray(torch.as_tensor(block_tables), dtype=np.int64)
    lengths = np.asarray(torch.as_tensor(context_lengths), dtype=np.int64)
    rows, hq, d = q.shape
    page, hkv = kc.shape[1], kc.shape[2]
    group = hq // hkv
    out = np.zeros((rows, hq, d))
    for r in range(rows):
        n = int(lengths[r])
        if n == 0:
            continue
        t = np.arange(n)
        keys = kc[tables[r, t // page], t % page]  # [n, hkv, d]
        vals = vc[tables[r, t // page], t % page]
        for h in range(hq):
            kv = h // group
            s = keys[:, kv, :] @ q[r, h] / math.sqrt(d)
            w = np.exp(s - s.max())
            out[r, h] = (w / w.sum()) @ vals[:, kv, :]
    return out
