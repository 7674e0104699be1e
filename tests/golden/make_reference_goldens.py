"""Write golden vectors by running the reference implementation on the CPU.

Run in the build container only (the reference tree is not shipped):

    python tests/golden/make_reference_goldens.py /root/reference

Three fixtures pin what the reference's own tests leave open:
  allocator_trace.json -- exact physical page ids, refcounts and free counts of
      KVCacheManager (vllm_rlt/core/kv_cache_manager.py:137-344) after every
      step of a scripted sequence of allocate / ensure_capacity / free /
      prefix publish / lookup / eviction / transfer leases, plus the host
      metadata of _prepare_batch (:398-478) for a few batches.
  paged_attention_cpu.npz -- inputs and exact output bits of
      torch_paged_attention (vllm_rlt/kernels/paged_attention.py:12-36) on
      seeded bf16 / fp16 / fp32 cases.
  rotary_cpu.npz -- positions, inputs and exact output bits of the
      reference's rotary embedding (OuroRotaryEmbedding, vllm_rlt/models/
      ouro.py:39-70) and of the q/k rotation q * cos + _rotate_half(q) * sin
      (ouro.py:73-75, 108-109) in bf16 / fp16 / fp32.
  pd_segments.json -- the exact, ordered output lists of the reference's
      kv_segments and partition_segments (vllm_rlt/pd/transport.py:18-68) for
      several pool geometries, multi-depth tables and token ranges (whole
      pages, partial first/last pages, single tokens), and its error messages
      for invalid ranges.
The fixture files hold data only (inputs and outputs).

Fixture names given after the reference path select which files are
rewritten (default: all), so one fixture can be added without touching the
bytes of the others.

The reference tree is read-only: bytecode writing is switched off before the
reference is put on sys.path, so importing it leaves no __pycache__ there.
"""

import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent

# Scripted bookkeeping steps.  Each step is [op, *args]; the replay in
# tests/test_golden_reference.py interprets the same list.
STEPS = [
    ["allocate", "r0", 9, None],
    ["allocate", "r1", 20, 5],
    ["allocate", "r2", 6, None],
    ["write_all", "r1", 8],
    ["ensure", "r1", 13],
    ["free", "r0"],
    ["allocate", "r3", 17, 3],
    ["mark_imported", "r2", 6],
    ["publish", "r2", [7, 7, 1, 2, 3, 4, 5], 6],
    ["lookup", [7, 7, 1, 2, 3, 4, 9, 9]],
    ["allocate_prefix", "r4", 12, None, [7, 7, 1, 2, 3, 4, 9, 9]],
    ["free", "r2"],
    ["ensure", "r3", 17],
    ["pin", "r3", "t0"],
    ["free", "r3"],
    ["allocate", "r5", 8, None],
    ["unpin", "r3", "t0"],
    ["allocate", "big", 30, None],
    ["lookup", [7, 7, 1, 2, 3, 4, 9, 9]],
    ["free", "r4"],
    ["free", "r1"],
    ["allocate", "r6", 4, 1],
    ["free", "big"],
    ["allocate", "r7", 33, 10],
]

# Batches planned after the last step: (request ids, depths, positions).
BATCHES = [
    (["r6", "r7", "r7", "r5"], [2, 0, 1, 1], [0, 9, 3, 7]),
    (["r7"] * 3 + ["r5"] * 2, [1, 1, 1, 2, 2], [4, 5, 6, 0, 1]),
]


def snapshot(cache):
    return {
        "tables": {rid: [list(t) for t in a.block_tables] for rid, a in sorted(cache._allocations.items())},
        "free": list(cache._free_blocks),
        "refs": list(cache._refs),
        "num_free": cache.num_free_blocks,
        "prefixes": [list(blocks) for blocks in cache._prefixes.values()],
    }


def allocator_trace():
    from vllm_rlt.core.kv_cache_manager import KVCacheManager

    cache = KVCacheManager(2, 1, 2, 64, 4, 3, enable_prefix_caching=True)
    results = []
    for step in STEPS:
        op, args = step[0], step[1:]
        out = None
        if op == "allocate":
            rid, max_tokens, initial = args
            out = cache.allocate(rid, max_tokens, initial_tokens=initial)
        elif op == "allocate_prefix":
            rid, max_tokens, initial, tokens = args
            out = cache.allocate(rid, max_tokens, initial_tokens=initial, prefix=cache.lookup_prefix(tokens))
        elif op == "ensure":
            out = cache.ensure_capacity(*args)
        elif op == "free":
            cache.free(*args)
        elif op == "write_all":
            rid, n = args
            for plane in cache._allocations[rid].written:
                for w in plane:
                    for p in range(n):
                        w.add(p)
        elif op == "mark_imported":
            cache.mark_imported_prefix(*args)
        elif op == "publish":
            cache.publish_prefix(*args)
        elif op == "lookup":
            out = [list(b) for b in cache.lookup_prefix(args[0])]
        elif op == "pin":
            cache.pin_transfer(*args)
        elif op == "unpin":
            cache.unpin_transfer(*args)
        else:
            raise ValueError(op)
        results.append({"step": step, "result": out, "state": snapshot(cache)})
    batches = []
    for ids, depths, positions in BATCHES:
        b = cache._prepare_batch(ids, depths, positions)
        batches.append(
            {
                "ids": ids,
                "depths": depths,
                "positions": positions,
                "write_blocks": b.write_blocks.tolist(),
                "write_offsets": b.write_offsets.tolist(),
                "block_tables": b.block_tables.tolist(),
                "context_lengths": b.context_lengths.tolist(),
            }
        )
    config = dict(num_layers=2, num_kv_heads=1, head_dim=2, num_blocks=64, block_size=4, max_loops=3)
    return {"config": config, "steps": results, "batches": batches}


def attention_cases():
    from vllm_rlt.kernels.paged_attention import torch_paged_attention

    arrays = {}
    cases = [
        ("bf16_g1", torch.bfloat16, 4, 4, 32, 16, [0, 1, 37, 100]),
        ("fp16_g2", torch.float16, 4, 2, 16, 5, [12, 3, 0, 64]),
        ("fp32_g3", torch.float32, 6, 2, 8, 3, [7, 1, 19, 30]),
        ("bf16_d128", torch.bfloat16, 2, 2, 128, 16, [300, 17]),
    ]
    for name, dtype, hq, hkv, d, page, lengths in cases:
        g = torch.Generator().manual_seed(len(name) * 7919 + d)
        pages = [(n + page - 1) // page for n in lengths]
        nb = sum(pages) + 2
        perm = torch.randperm(nb, generator=g)
        tables = torch.full((len(lengths), max(pages + [1])), -1, dtype=torch.int32)
        used = 0
        for r, p in enumerate(pages):
            tables[r, :p] = perm[used : used + p].to(torch.int32)
            used += p
        key_cache = (torch.randn(nb, page, hkv, d, generator=g) * 2).to(dtype)
        value_cache = torch.randn(nb, page, hkv, d, generator=g).to(dtype)
        q = torch.randn(len(lengths), hq, d, generator=g).to(dtype)
        lens = torch.tensor(lengths, dtype=torch.int32)
        out = torch_paged_attention(q, key_cache, value_cache, tables, lens)
        bits = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}[dtype]
        for field, t in (("q", q), ("k", key_cache), ("v", value_cache), ("out", out)):
            arrays[f"{name}/{field}"] = t.view(bits).numpy()
        arrays[f"{name}/tables"] = tables.numpy()
        arrays[f"{name}/lengths"] = lens.numpy()
        arrays[f"{name}/dtype"] = np.array(str(dtype).split(".")[-1])
    return arrays


def rotary_cases():
    """Reference rotary angles and q/k rotation (vllm_rlt/models/ouro.py:39-75, 104-109)."""
    from vllm_rlt.models.config import OuroConfig
    from vllm_rlt.models.ouro import OuroRotaryEmbedding, _rotate_half

    arrays = {}
    cases = [
        ("bf16_ouro", torch.bfloat16, OuroConfig(), 16, [0, 1, 2, 15, 16, 511, 4095, 16383, 32767, 65535]),
        ("fp16_ouro", torch.float16, OuroConfig(), 4, [0, 3, 1000, 40000]),
        ("fp32_ouro", torch.float32, OuroConfig(), 2, [0, 7, 20000, 65535]),
        ("bf16_tiny", torch.bfloat16, OuroConfig.tiny(), 4, [0, 1, 5, 127]),
    ]
    for name, dtype, config, heads, positions in cases:
        g = torch.Generator().manual_seed(len(name) * 131 + config.head_dim)
        rotary = OuroRotaryEmbedding(config)
        pos = torch.tensor(positions, dtype=torch.int64)
        x = (torch.randn(len(positions), heads, config.head_dim, generator=g) * 3).to(dtype)
        cos, sin = rotary(x, pos)  # [N, 1, D] each, in x's dtype
        out = x * cos + _rotate_half(x) * sin
        bits = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}[dtype]
        arrays[f"{name}/positions"] = pos.numpy()
        arrays[f"{name}/theta"] = np.array(config.rope_theta, dtype=np.float64)
        arrays[f"{name}/dtype"] = np.array(str(dtype).split(".")[-1])
        for field, t in (("x", x), ("cos", cos[:, 0]), ("sin", sin[:, 0]), ("out", out)):
            arrays[f"{name}/{field}"] = t.contiguous().view(bits).numpy()
    return arrays


# Segment cases: pool geometry, tables (one per storage depth), [start, end)
# ranges, and (byte_limit, descriptor_limit) pairs for partition_segments.
SEGMENT_GEOMETRIES = [
    # block_size, num_layers, token_bytes, num_blocks, key_ptr, value_ptr, tables
    (4, 3, 64, 24, 0, 10**9, [[5, 2, 9], [11, 0, 7], [3, 4, 8]]),
    (16, 24, 4096, 4096, 1 << 40, (1 << 40) + (1 << 36), [[4095, 17, 1024, 3], [8, 9, 10, 11]]),
    (1, 2, 32, 6, 4096, 8192, [[5, 0, 3, 1]]),
    (8, 1, 16, 10, 0, 1 << 20, [[9, 1], [2, 3], [4, 5], [6, 7]]),
]
SEGMENT_RANGES = {
    4: [(2, 9), (0, 8), (4, 5), (0, 1), (3, 12), (0, 12), (11, 12), (1, 3)],
    16: [(0, 64), (5, 6), (15, 17), (16, 48), (3, 61), (0, 1), (63, 64)],
    1: [(0, 4), (2, 3), (1, 4)],
    8: [(0, 16), (7, 9), (8, 16), (1, 15)],
}
PARTITION_LIMITS = [(333, 3), (1 << 30, 1), (64, 1000), (4096 * 16 + 5, 4), (7, 2), (1 << 20, 7)]
MAX_PIECES = 400  # limits that would cut a case into more pieces are skipped


def segment_cases():
    from vllm_rlt.pd.transport import kv_segments, partition_segments

    cases = []
    for page, layers, token, blocks, key_ptr, value_ptr, tables in SEGMENT_GEOMETRIES:
        info = dict(
            block_size=page,
            num_layers=layers,
            token_bytes=token,
            layer_bytes=page * token,
            block_bytes=layers * page * token,
            num_blocks=blocks,
            key_ptr=key_ptr,
            value_ptr=value_ptr,
            device=0,
        )
        for start, end in SEGMENT_RANGES[page]:
            segments = [list(s) for s in kv_segments(info, tables, start, end)]
            partitions = []
            total = sum(n for _, n, _ in segments)
            for byte_limit, descriptor_limit in PARTITION_LIMITS:
                if total // byte_limit + len(segments) > MAX_PIECES:
                    continue
                # The reference test pairs a list with itself; shift the target so the
                # pairing of source and target pieces is visible in the fixture.
                target = [(a + 12345, n, 1) for a, n, _ in segments]
                parts = partition_segments([tuple(s) for s in segments], target, byte_limit, descriptor_limit)
                partitions.append(
                    {
                        "byte_limit": byte_limit,
                        "descriptor_limit": descriptor_limit,
                        "parts": [[[list(x) for x in src], [list(x) for x in dst], n] for src, dst, n in parts],
                    }
                )
            cases.append(
                {"info": info, "tables": tables, "start": start, "end": end, "segments": segments, "partitions": partitions}
            )
    errors = []
    page, layers, token, blocks, key_ptr, value_ptr, tables = SEGMENT_GEOMETRIES[0]
    info = dict(cases[0]["info"])
    for name, use_info, use_tables, start, end in [
        ("empty", info, tables, 5, 5),
        ("negative", info, tables, -1, 3),
        ("past_allocation", info, tables, 0, 13),
        ("block_outside_pool", dict(info, num_blocks=9), tables, 0, 12),
        ("second_table_short", info, [tables[0] + [1], [2]], 0, 13),
    ]:
        try:
            list(kv_segments(use_info, use_tables, start, end))
            message = None
        except ValueError as e:
            message = str(e)
        errors.append({"case": name, "info": use_info, "tables": use_tables, "start": start, "end": end, "error": message})
    try:
        list(partition_segments([(0, 8, 0), (64, 8, 0)], [(0, 8, 0)], 100, 4))
        mismatch = None
    except ValueError as e:
        mismatch = str(e)
    return {"cases": cases, "errors": errors, "partition_mismatch_error": mismatch}


FIXTURES = {
    "allocator_trace.json": lambda path: path.write_text(json.dumps(allocator_trace(), indent=1)),
    "paged_attention_cpu.npz": lambda path: np.savez_compressed(path, **attention_cases()),
    "rotary_cpu.npz": lambda path: np.savez_compressed(path, **rotary_cases()),
    "pd_segments.json": lambda path: path.write_text(json.dumps(segment_cases())),
}


def main():
    reference = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    names = sys.argv[2:] or list(FIXTURES)
    sys.dont_write_bytecode = True  # never write .pyc files into the reference tree
    sys.path.insert(0, reference)
    torch.set_num_threads(1)
    for name in names:
        FIXTURES[name](OUT / name)
        print("wrote", OUT / name)


if __name__ == "__main__":
    main()
