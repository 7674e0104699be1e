"""numpy restatements of the byte/integer work on the paged pool (test infrastructure only).

Pools are numpy arrays [blocks, layers, page, kv_heads, head_dim] of any
element type; bf16 pools are handled as their raw uint16 bits so every copy is
byte-exact.  Each function names the reference lines it restates.
"""

from __future__ import annotations

import numpy as np


def append(key_pool, value_pool, layer, write_blocks, write_offsets, k, v, n_rows=None):
    """pool[block_i, layer, offset_i] = k_i / v_i for i < n_rows.

    vllm_rlt/core/kv_cache_manager.py:531-532 (only the first len(rows) rows
    are written, :531).
    """
    n = len(write_blocks) if n_rows is None else n_rows
    for i in range(n):
        key_pool[write_blocks[i], layer, write_offsets[i]] = k[i]
        value_pool[write_blocks[i], layer, write_offsets[i]] = v[i]


def copy_token(key_pool, value_pool, src_block, dst_blocks, offset):
    """pool[dst, :, offset] = pool[src, :, offset] for all layers (kv_cache_manager.py:609-611)."""
    for dst in dst_blocks:
        key_pool[dst, :, offset] = key_pool[src_block, :, offset]
        value_pool[dst, :, offset] = value_pool[src_block, :, offset]


def finalize_batched(descriptors, tables, key_pool, value_pool, max_loops, page):
    """Exit copies from (slot, depth, pos) descriptors and [slots, planes, W] tables.

    vllm_rlt/kernels/routing.py:80-109: for target in (depth, max_loops), copy the
    token's K/V at every layer from plane `depth` to plane `target`.
    """
    for slot, depth, pos in np.asarray(descriptors).reshape(-1, 3):
        src = tables[slot, depth, pos // page]
        for target in range(depth + 1, max_loops):
            dst = tables[slot, target, pos // page]
            key_pool[dst, :, pos % page] = key_pool[src, :, pos % page]
            value_pool[dst, :, pos % page] = value_pool[src, :, pos % page]


def gather(pool, layer, table, length, page):
    """[length, kv_heads, head_dim] history in position order (kv_cache_manager.py:631-637)."""
    t = np.arange(length)
    return pool[np.asarray(table)[t // page], layer, t % page]


def decode_metadata(descriptors, count, size, tables, page, out_width):
    """Per-row routing metadata (vllm_rlt/kernels/routing.py:8-41).

    tables: [slots, planes, W].  Rows >= count are padding: slot = pos = 0,
    length 0, no write address, zero table row.  Returns a dict of arrays;
    blocks/offsets have `count` entries.
    """
    planes, width = tables.shape[1], tables.shape[2]
    desc = np.zeros((size, 3), dtype=np.int64)
    desc[:count] = np.asarray(descriptors).reshape(-1, 3)[:count]
    out = {
        "slots": desc[:, 0].copy(),
        "positions": desc[:, 2].copy(),
        "lengths": np.where(np.arange(size) < count, desc[:, 2] + 1, 0).astype(np.int32),
        "blocks": np.zeros(count, dtype=np.int64),
        "offsets": np.zeros(count, dtype=np.int64),
        "tables": np.zeros((size, width), dtype=np.int32),
    }
    for row in range(size):
        slot, depth, pos = desc[row]
        plane = depth if planes > 1 else 0
        if row < count:
            out["blocks"][row] = tables[slot, plane, pos // page]
            out["offsets"][row] = pos % page
            out["tables"][row, :out_width] = tables[slot, plane, :out_width]
    return out


def stage_prefill(source):
    """int64 values staged to int64 and (truncated) int32 (kernels/prefill_metadata.py:8-12)."""
    src = np.asarray(source, dtype=np.int64)
    return src.copy(), src.astype(np.int32)


def expand_prefill(positions, sequences, tables, page):
    """blocks = tables[seq, pos // page], offsets = pos % page (kernels/prefill_metadata.py:16-32)."""
    positions = np.asarray(positions, dtype=np.int64)
    sequences = np.asarray(sequences, dtype=np.int64)
    return np.asarray(tables)[sequences, positions // page].astype(np.int64), positions % page


def prepare_addresses(block_tables_by_row, positions, page):
    """Write address, padded table and length of each row (kv_cache_manager.py:409-415,420,445-448,466-470).

    block_tables_by_row[i] is row i's depth-resolved table (tuple of page ids).
    Tables are cut to width = max(pos // page + 1) and padded with -1.
    """
    width = max((p // page + 1 for p in positions), default=0)
    blocks = np.array([t[p // page] for t, p in zip(block_tables_by_row, positions)], dtype=np.int64)
    offsets = np.array([p % page for p in positions], dtype=np.int64)
    tables = np.full((len(positions), width), -1, dtype=np.int32)
    for i, t in enumerate(block_tables_by_row):
        cut = list(t[:width])
        tables[i, : len(cut)] = cut
    lengths = np.array([p + 1 for p in positions], dtype=np.int32)
    return blocks, offsets, tables, lengths


def packed_prefill_groups(keys, positions):
    """cu_seqlens_q, per-sequence last row and max_seqlen_q of a packed chunk.

    kv_cache_manager.py:424-444: consecutive rows with the same (request, depth)
    key and contiguous positions form one sequence; a key may not reappear
    after its run ends, and positions inside a run must be contiguous.
    """
    cumulative, ends, seen = [0], [], set()
    for i, (key, pos) in enumerate(zip(keys, positions)):
        if i and key == keys[i - 1]:
            if pos != positions[i - 1] + 1:
                raise ValueError("packed prefill positions must be contiguous")
            ends[-1] = i
            cumulative[-1] = i + 1
        else:
            if key in seen:
                raise ValueError("packed prefill request/depth must form one sequence")
            seen.add(key)
            ends.append(i)
            cumulative.append(i + 1)
    max_q = max((b - a for a, b in zip(cumulative, cumulative[1:])), default=1)
    return cumulative, ends, max_q
