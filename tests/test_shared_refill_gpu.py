"""SHARED-layout decode with refill through KVCacheManager(layout="shared") (GPU).

The workload: 256 request slots, contexts U[1024, 8192], 16/16 heads x 128,
page 16, bf16.  Each request runs loops 1..e on one position with the exit
depth e drawn from P(1, 2, 3, 4) = (0.1, 0.2, 0.3, 0.4); every loop writes
the one SHARED plane (a later depth overwrites the slot,
tests/test_cdb_runtime.py:152-177) before attending.  After U{1..8} tokens a
request finishes, its pages return to the free list, which is shuffled, and
a new request with a fresh context takes its place one step later, so some
steps run with padded batches (pad rows: length 0, no write address,
tests/test_cdb_runtime.py:274-292).  A new request's history is declared
valid with mark_imported_prefix, as after a page import.

Each step checks:
* the written slots bit-exact against the oracle's append on host copies of
  the touched pages, and every other slot of the pool unchanged (free pages
  and other requests' pages included);
* pad rows return zeros;
* sampled rows against the CPU oracle and every row against a dense fp32
  reference on the device (bf16 max-abs 2e-2 / rel 1e-2).
"""

import random

import numpy as np
import pytest
import torch

from oracle import kv_ops
from oracle.paged_attention import paged_attention_cpu

pytestmark = pytest.mark.gpu

ROWS, CTX, EXIT_P = 256, (1024, 8192), (0.1, 0.2, 0.3, 0.4)
LAYERS, HEADS, HEAD_DIM, PAGE, LOOPS = 2, 16, 128, 16, 4
STEPS = 6
TOL = dict(atol=2e-2, rtol=1e-2)


def _fill(pool, pages, gen):
    idx = torch.as_tensor(pages, dtype=torch.long, device=pool.device)
    pool[idx] = torch.randn((len(pages),) + pool.shape[1:], generator=gen, device=pool.device).to(pool.dtype)


def _changed_slots(after, before, chunk=4096):
    """(block, layer, offset) triples whose bytes differ between the two pools."""
    out = []
    for b0 in range(0, after.shape[0], chunk):
        diff = (after[b0 : b0 + chunk].view(torch.int16) != before[b0 : b0 + chunk].view(torch.int16))
        hit = diff.flatten(3).any(-1).nonzero()
        hit[:, 0] += b0
        out += [tuple(x) for x in hit.tolist()]
    return set(out)


def _dense_row(q, key_slice, value_slice, table, length):
    t = torch.arange(length, device=q.device)
    pages = table[t // PAGE].long()
    k = key_slice[pages, t % PAGE].float().transpose(0, 1).contiguous()  # [h, n, d]
    v = value_slice[pages, t % PAGE].float().transpose(0, 1).contiguous()
    scores = torch.matmul(k, q.float()[:, :, None])[..., 0] * HEAD_DIM**-0.5
    return torch.matmul(scores.softmax(-1)[:, None, :], v)[:, 0]


def test_shared_decode_with_refill_and_random_page_reuse():
    from vllm_rlt_amd import KVCacheManager
    from vllm_rlt_amd.buffers import Workspace

    if torch.cuda.mem_get_info()[0] < 80 * 2**30:
        pytest.skip("needs 80 GiB free device memory")
    rng = random.Random(303)
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(304)
    # Enough pages for every slot's largest request (a refill follows a free).
    width = (CTX[1] + 8 + PAGE - 1) // PAGE
    num_blocks = ROWS * width + 1024
    cache = KVCacheManager(
        num_layers=LAYERS, num_kv_heads=HEADS, head_dim=HEAD_DIM, num_blocks=num_blocks, block_size=PAGE,
        max_loops=LOOPS, device=dev, dtype=torch.bfloat16, layout="shared",
    )
    for pool in (cache.key_cache, cache.value_cache):
        flat = pool.view(-1)
        for start in range(0, flat.numel(), 1 << 28):
            flat[start : start + (1 << 28)].normal_(generator=gen)
    rng.shuffle(cache._free_blocks)  # the first requests draw random pages

    serial = iter(range(10**6))
    slots = [None] * ROWS  # [request id, position, loops done, exit depth, tokens left]

    def admit(slot):
        rid = f"r{next(serial)}"
        ctx, gen_tokens = rng.randint(*CTX), rng.randint(1, 8)
        assert cache.allocate(rid, ctx + gen_tokens)
        pages = list(cache.get_block_table(rid, 0))
        _fill(cache.key_cache, pages, gen)
        _fill(cache.value_cache, pages, gen)
        cache.mark_imported_prefix(rid, ctx)
        exit_depth = rng.choices(range(1, LOOPS + 1), weights=EXIT_P)[0]
        slots[slot] = [rid, ctx, 0, exit_depth, gen_tokens]

    for slot in range(ROWS):
        admit(slot)
    workspace = Workspace(ROWS, width, 8, dev, torch.bfloat16)
    padded_steps = finished = 0
    for step in range(STEPS):
        live = [s for s in range(ROWS) if slots[s] is not None]
        ids = [slots[s][0] for s in live]
        depths = [slots[s][2] for s in live]
        positions = [slots[s][1] for s in live]
        n = len(live)
        padded_steps += n < ROWS
        # Full batches go through the manager's own upload; padded ones through
        # the runner's fixed-size workspace.
        if n == ROWS:
            batch = cache._prepare_batch(ids, depths, positions)
        else:
            batch = workspace.prepare(cache, ids, depths, positions, ROWS)
        blocks = [cache.get_block_table(i, 0)[p // PAGE] for i, p in zip(ids, positions)]
        offsets = [p % PAGE for p in positions]
        print(f"[shared refill] step {step}: {n} live rows, depths {np.bincount(depths, minlength=4).tolist()}", flush=True)
        for layer in range(LAYERS):
            q = torch.randn((ROWS, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
            k = torch.randn((ROWS, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((ROWS, HEADS, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
            before_k, before_v = cache.key_cache.clone(), cache.value_cache.clone()
            cache._write_prepared(layer, batch, k, v)
            out = cache._attend_prepared(layer, batch, q)
            torch.cuda.synchronize()
            # Only the n written slots changed, and they hold the oracle's append.
            touched = {(b, layer, o) for b, o in zip(blocks, offsets)}
            changed = _changed_slots(cache.key_cache, before_k) | _changed_slots(cache.value_cache, before_v)
            assert changed <= touched
            pages = sorted({b for b in blocks})
            remap = {b: i for i, b in enumerate(pages)}
            exp_k = before_k[pages].cpu().view(torch.int16).numpy().copy()
            exp_v = before_v[pages].cpu().view(torch.int16).numpy().copy()
            kv_ops.append(
                exp_k, exp_v, layer, [remap[b] for b in blocks], offsets,
                k.cpu().view(torch.int16).numpy(), v.cpu().view(torch.int16).numpy(), n_rows=n,
            )
            assert (cache.key_cache[pages].cpu().view(torch.int16).numpy() == exp_k).all()
            assert (cache.value_cache[pages].cpu().view(torch.int16).numpy() == exp_v).all()
            del before_k, before_v
            # Pad rows attend to nothing.
            assert torch.count_nonzero(out[n:]) == 0
            # Sampled rows against the CPU oracle on host copies of their pages.
            sample = sorted(rng.sample(range(n), 3))
            tables = [cache.get_block_table(ids[r], 0)[: positions[r] // PAGE + 1] for r in sample]
            used = sorted({b for t in tables for b in t})
            where = {b: i for i, b in enumerate(used)}
            small = torch.full((len(sample), max(map(len, tables))), -1, dtype=torch.int32)
            for i, t in enumerate(tables):
                small[i, : len(t)] = torch.tensor([where[b] for b in t], dtype=torch.int32)
            hk = cache.key_cache[used, layer].cpu()
            hv = cache.value_cache[used, layer].cpu()
            lengths = torch.tensor([positions[r] + 1 for r in sample], dtype=torch.int32)
            expect = paged_attention_cpu(q[sample].cpu(), hk, hv, small, lengths)
            torch.testing.assert_close(out[sample].cpu(), expect, **TOL)
            # Every live row against a dense fp32 device reference.
            for r in range(n):
                table = batch.block_tables[r]
                ref = _dense_row(q[r], cache.key_cache[:, layer], cache.value_cache[:, layer], table, positions[r] + 1)
                torch.testing.assert_close(out[r].float(), ref, **TOL)
        # Advance: loop to the exit depth, then the next position; finished
        # requests free their pages (shuffled back into the free list) and are
        # replaced on the next step.
        for s in range(ROWS):
            if slots[s] is None:
                admit(s)
                continue
            st = slots[s]
            st[2] += 1
            if st[2] < st[3]:
                continue
            cache.finalize_token(st[0], st[1], st[3] - 1)  # SHARED: validates, copies nothing
            st[1], st[2], st[4] = st[1] + 1, 0, st[4] - 1
            st[3] = rng.choices(range(1, LOOPS + 1), weights=EXIT_P)[0]
            if st[4] == 0:
                cache.free(st[0])
                slots[s] = None
                finished += 1
        rng.shuffle(cache._free_blocks)
    assert finished > 0 and padded_steps > 0
    # Every page is either free or held by a live request, each exactly once.
    held = [b for st in slots if st is not None for b in cache.get_block_table(st[0], 0)]
    assert sorted(held + list(cache._free_blocks)) == list(range(num_blocks))
