"""Paged decode attention + KV append on Ouro-1.4B-shaped synthetic data (one MI355X).

Workload (default, "ouro-last-exited"): 24 layers x 4 loop depths (LAST-EXITED:
one storage plane per depth), 16 query / 16 KV heads, head_dim 128, page 16,
bf16.  Batch 64; request contexts uniform in [512, 4096]; every step each
request sits at a depth drawn uniformly from {1..4} (planes 0..3), appends one
token's K/V at that depth for all 24 layers and runs decode attention over the
depth-resolved pages.  Block tables are random page permutations.

One "loop-step" = one recurrent pass of the whole batch: the device-side
routing metadata build, then 24 x (KV append + paged decode attention).
Positions advance by one per step.  Inputs live in HBM before timing starts.

Prints one JSON line (bench contract) with loop-steps/s as `value`, the
step's algorithmic HBM GB/s, the decode launch's roofline (algorithmic bytes /
HIP-event-timed duration), and the CPU oracle's throughput on a bounded
sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _path in (REPO, REPO / "vllm-rlt_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
LAYERS, HQ, HKV, HEAD_DIM, PAGE, LOOPS = 24, 16, 16, 128, 16, 4

MFMA_BF16_PEAK_TFLOPS = 2500.0
# Decode workloads.  ctx: initial context lengths U[lo, hi]; planes: KV storage
# planes (LAST-EXITED = one per loop depth, SHARED = 1); depth_probs: exit-depth
# distribution (None: every step each request sits at a depth drawn uniformly);
# refill: requests run their loops to the exit depth, finish after a few tokens
# and are replaced, their pages freed and handed out again in random order;
# prefix: tokens of a common prefix whose pages are aliased in every table.
WORKLOADS = {
    "ouro-last-exited": dict(batch=64, ctx=(512, 4096), planes=LOOPS, depth_probs=None, refill=False, prefix=0),
    "ouro-shared": dict(
        batch=256, ctx=(1024, 8192), planes=1, depth_probs=(0.1, 0.2, 0.3, 0.4), refill=True, prefix=0
    ),
    "ouro-prefix-stress": dict(
        batch=64, ctx=(16384, 32768), planes=1, depth_probs=None, refill=False, prefix=8192
    ),
    # Prefix caching under the reference's own semantics (LAST-EXITED only,
    # a published prefix holds one page per plane): 4 planes, each with its
    # own 2048-token prefix aliased by every row at that depth; contexts are
    # the prefix-stress ones scaled by 1/4 so the 4 planes fit one GPU.
    "ouro-prefix-last-exited": dict(
        batch=64, ctx=(4096, 8192), planes=LOOPS, depth_probs=None, refill=False, prefix=2048
    ),
    # The reference CPU case's shape (batch 4, contexts U[1, 256]) over all 24
    # layers and 4 planes: launch-bound, where graph replay matters.
    "ouro-small-batch": dict(batch=4, ctx=(1, 256), planes=LOOPS, depth_probs=None, refill=False, prefix=0),
}
# The headline workload (the bench line) and the configs measured after it in
# the same run, each reported under the line's `workloads` key.
HEADLINE = "ouro-last-exited"
SECONDARY = ("ouro-shared", "ouro-prefix-stress", "ouro-prefix-last-exited", "ouro-prefill")
# CPU baseline row sampling of the large decode workloads: every n-th row,
# scaled back to the whole batch (keeps each CPU sample to seconds).
CPU_ROW_SAMPLE = {"ouro-shared": 4, "ouro-prefix-stress": 4, "ouro-prefix-last-exited": 2}
# SHARED refill: a request finishes after U{1..8} generated tokens.
REFILL_TOKENS = (1, 8)
# Chunked prefill: 8 sequences x 512 new tokens over prefixes U[0, 16384], the
# full 4-loop prefill (4 depths x 24 layers of append + packed attention).
PREFILL = dict(seqs=8, chunk=512, prefix=(0, 16384))


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", choices=sorted(WORKLOADS) + ["ouro-prefill"], default="ouro-last-exited")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--cpu-reps", type=int, default=5, help="timed repetitions of each CPU baseline sample")
    p.add_argument(
        "--only", action="store_true", help="run only --workload (the default run adds the other configs)"
    )
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-check", action="store_true", help="skip the pre-timing parity spot check")
    p.add_argument(
        "--graph",
        action="store_true",
        help="decode workloads: capture one loop-step in a HIP graph and time its replays",
    )
    p.add_argument(
        "--append",
        choices=["fused", "separate"],
        default="fused",
        help="decode workloads: KV append fused into the decode launch, or its own launch before it",
    )
    p.add_argument(
        "--calibrate-counters",
        action="store_true",
        help="only run one 1 GiB device-to-device copy (known-size kernel for scaling HBM counters)",
    )
    return p.parse_args()


def calibrate_counters(device):
    """One plain 1 GiB copy: rocprofv3 FETCH_SIZE / WRITE_SIZE of this dispatch give the counter scale."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": src.numel()}), flush=True)


def _profile_figure(key, workload):
    """The number on a committed profile summary line `<key>[<workload>] = <number>`, if any."""
    import re

    pattern = re.compile(rf"{re.escape(key)}\[{re.escape(workload)}\]\s*=\s*([0-9.eE+]+)")
    for path in sorted((REPO / "profiles").glob("*.md")):
        match = pattern.search(path.read_text())
        if match:
            return float(match.group(1))
    return None


def profiled_traffic(workload):
    """HBM bytes per launch of the workload's kernel from the committed rocprofv3 --pmc summary, if any.

    The summary carries a line `traffic_bytes_per_launch[<workload>] = <bytes>`
    computed from FETCH_SIZE and WRITE_SIZE scaled by the calibration copy.
    """
    value = _profile_figure("traffic_bytes_per_launch", workload)
    return None if value is None else int(value)


def profiled_launch_ms(workload):
    """The launch's average kernel time (ms) in the committed rocprofv3 --kernel-trace summary, if any.

    The summary carries `rocprof_avg_launch_us[<workload>] = <us>`: the traced
    average of the kernels one launch runs (for the decode, split pass plus
    merge), reported beside the live HIP-event average, which also holds the
    gap between those kernels.
    """
    value = _profile_figure("rocprof_avg_launch_us", workload)
    return None if value is None else round(value / 1e3, 5)


def describe(name):
    cfg = WORKLOADS[name]
    lo, hi = cfg["ctx"]
    text = (
        f"{name}: Ouro-1.4B decode, 24 layers, {cfg['planes']} KV plane(s), 16/16 heads, head_dim 128, page 16, "
        f"bf16, batch {cfg['batch']}, contexts U[{lo},{hi}]"
    )
    if cfg["refill"]:
        text += (
            f", exit depth P(1..4)={list(cfg['depth_probs'])} with loops run to the exit depth, requests "
            f"replaced after U{{{REFILL_TOKENS[0]}..{REFILL_TOKENS[1]}}} tokens, freed pages reused in random order"
        )
    elif cfg["planes"] > 1:
        text += ", each step every request at a depth drawn from U{1..4}"
    if cfg["prefix"]:
        where = "every table" if cfg["planes"] == 1 else "every plane's table (one prefix per plane)"
        text += f", a {cfg['prefix']}-token prefix aliased read-only in {where}"
    return text + "; loop-step = metadata build + 24 x (KV append + decode)"


def make_schedule(name, total_steps, seed):
    """Host-side page tables and per-step (slot, plane, position) descriptors of a decode workload.

    Returns (descriptors [steps, batch, 3] int64, tables [slots, planes, width]
    int32, num_blocks, contexts, shared_pages [planes, prefix pages]).  Without
    refill, every request keeps one slot, appends at context + step, and its
    table covers every position the run touches; with a prefix, each plane's
    table begins with that plane's prefix pages.  With refill (SHARED), a request runs loops
    0 .. exit-1 on one position, then moves to the next; after its generated
    tokens it leaves, its pages return to the free list, and a new request
    with a fresh context takes a new slot, drawing pages at random positions
    of the free list.
    """
    import random

    cfg = WORKLOADS[name]
    batch, planes = cfg["batch"], cfg["planes"]
    lo, hi = cfg["ctx"]
    g = torch.Generator().manual_seed(seed)
    contexts = torch.randint(lo, hi + 1, (batch,), generator=g)
    if not cfg["refill"]:
        prefix_pages = cfg["prefix"] // PAGE
        pages = (contexts + total_steps + PAGE - 1) // PAGE
        width = int(pages.max())
        own = [int(n) - prefix_pages for n in pages]
        num_blocks = (prefix_pages + sum(own)) * planes
        perm = torch.randperm(num_blocks, generator=g).to(torch.int32)
        shared = perm[: prefix_pages * planes].view(planes, prefix_pages)
        used = prefix_pages * planes
        tables = torch.zeros(batch, planes, width, dtype=torch.int32)
        for r in range(batch):
            for plane in range(planes):
                tables[r, plane, :prefix_pages] = shared[plane]
                tables[r, plane, prefix_pages : prefix_pages + own[r]] = perm[used : used + own[r]]
                used += own[r]
        if cfg["depth_probs"] is None:
            depths = torch.randint(0, LOOPS, (total_steps, batch), generator=g)
        else:
            probs = torch.tensor(cfg["depth_probs"])
            depths = torch.multinomial(probs, total_steps * batch, replacement=True, generator=g)
            depths = depths.view(total_steps, batch)
        steps = torch.arange(total_steps)[:, None]
        desc = torch.stack(
            [
                torch.arange(batch).expand(total_steps, -1),
                depths if planes > 1 else torch.zeros_like(depths),
                contexts[None, :] + steps,
            ],
            dim=-1,
        ).to(torch.int64)
        return desc, tables, num_blocks, contexts, shared.long()

    rng = random.Random(seed)
    probs = cfg["depth_probs"]
    tok_lo, tok_hi = REFILL_TOKENS

    def draw_exit():
        return rng.choices(range(1, LOOPS + 1), weights=probs)[0]

    def need(ctx, gen):
        return (ctx + gen + PAGE - 1) // PAGE

    gens = [rng.randint(tok_lo, tok_hi) for _ in range(batch)]
    first = [need(int(contexts[r]), gens[r]) for r in range(batch)]
    num_blocks = int(sum(first) * 1.02) + 64
    free = list(range(num_blocks))
    slot_pages = []

    def admit(ctx, gen):
        n = need(ctx, gen)
        got = []
        for _ in range(n):  # a random free page, O(1) per page
            i = rng.randrange(len(free))
            free[i], free[-1] = free[-1], free[i]
            got.append(free.pop())
        slot_pages.append(got)
        return len(slot_pages) - 1

    state = []  # [slot, position, depth, exit, tokens left]
    for r in range(batch):
        state.append([admit(int(contexts[r]), gens[r]), int(contexts[r]), 0, draw_exit(), gens[r]])
    desc = torch.empty(total_steps, batch, 3, dtype=torch.int64)
    for step in range(total_steps):
        for r, st in enumerate(state):
            desc[step, r, 0], desc[step, r, 1], desc[step, r, 2] = st[0], 0, st[1]
        for st in state:
            st[2] += 1
            if st[2] < st[3]:
                continue
            st[1], st[2], st[3], st[4] = st[1] + 1, 0, draw_exit(), st[4] - 1
            if st[4] > 0:
                continue
            free.extend(slot_pages[st[0]])
            gen = rng.randint(tok_lo, tok_hi)
            ctx = rng.randint(lo, hi)
            ctx = max(1, min(ctx, len(free) * PAGE - gen))
            st[:] = [admit(ctx, gen), ctx, 0, draw_exit(), gen]
    width = max(len(pg) for pg in slot_pages)
    tables = torch.zeros(len(slot_pages), 1, width, dtype=torch.int32)
    for slot, pg in enumerate(slot_pages):
        tables[slot, 0, : len(pg)] = torch.tensor(pg, dtype=torch.int32)
    return desc, tables, num_blocks, contexts, torch.empty(1, 0, dtype=torch.int64)


class Workload:
    """Device-resident pool, page tables, per-step descriptors and per-layer inputs."""

    def __init__(self, name, total_steps, seed, device):
        cfg = WORKLOADS[name]
        self.name = name
        self.batch = cfg["batch"]
        self.planes = cfg["planes"]
        self.device = device
        desc, tables, self.num_blocks, self.contexts, self.shared_pages = make_schedule(name, total_steps, seed)
        self.width = tables.shape[2]
        self.tables_host = tables
        self.tables = tables.to(device)
        self.descriptors_host = desc
        self.descriptors = desc.to(device)  # [steps, batch, 3]
        self.prefix_tokens = cfg["prefix"]
        # Pool [blocks, layers, page, kv_heads, head_dim], filled with N(0,1) bf16.
        shape = (self.num_blocks, LAYERS, PAGE, HKV, HEAD_DIM)
        self.key_cache = torch.empty(shape, dtype=torch.bfloat16, device=device)
        self.value_cache = torch.empty(shape, dtype=torch.bfloat16, device=device)
        gen = torch.Generator(device=device).manual_seed(seed + 1)
        for pool in (self.key_cache, self.value_cache):
            flat = pool.view(-1)
            chunk = 1 << 28
            for start in range(0, flat.numel(), chunk):
                flat[start : start + chunk].normal_(generator=gen)
        # Per-layer synthetic projections (q, new k, new v).
        self.q = torch.randn((LAYERS, self.batch, HQ, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        self.k_new = torch.randn((LAYERS, self.batch, HKV, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        self.v_new = torch.randn((LAYERS, self.batch, HKV, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        self.out = torch.empty_like(self.q)
        # Routing outputs of the metadata build (one set, rebuilt every step).
        n = self.batch
        self.slots = torch.empty(n, dtype=torch.int64, device=device)
        self.positions = torch.empty(n, dtype=torch.int64, device=device)
        self.lengths = torch.empty(n, dtype=torch.int32, device=device)
        self.blocks = torch.empty(n, dtype=torch.int64, device=device)
        self.offsets = torch.empty(n, dtype=torch.int64, device=device)
        self.row_tables = torch.zeros((n, self.width), dtype=torch.int32, device=device)
        from vllm_rlt_amd import ops

        self.workspace = torch.empty(
            ops.decode_workspace_bytes(n, HQ, HKV, HEAD_DIM), dtype=torch.uint8, device=device
        )
        # Every row's table begins with its plane's aliased prefix pages: the
        # decode reads each plane's once per launch for all rows at that plane
        # (rlt_paged_decode_shared_prefix).  The step's prefix groups follow the
        # rows' depths; like the descriptors they are built before timing and
        # live on the device.
        self.fused_append = True  # KV append inside the decode launch
        self.prefix_hints = None
        if self.shared_pages.numel():
            self.prefix_hints = []
            for step in range(total_steps):
                planes_now = desc[step, :, 1].tolist()
                rows_pages = [tables[r, p, : self.shared_pages.shape[1]].tolist() for r, p in enumerate(planes_now)]
                self.prefix_hints.append(
                    ops.prefix_groups(rows_pages, self.lengths_at(step), PAGE, HQ // HKV, device)
                )
        self.prefix_hint = None  # the current step's groups

    def lengths_at(self, step):
        """Attention length of every row at a step (context incl. the appended token)."""
        return (self.descriptors_host[step, :, 2] + 1).tolist()

    def pool_bytes(self):
        return 2 * self.key_cache.numel() * self.key_cache.element_size()

    def shared_snapshot(self):
        """Copies of every plane's aliased prefix pages (all layers), to prove they stay read-only."""
        if self.shared_pages.numel() == 0:
            return None
        idx = self.shared_pages.reshape(-1).to(self.device)
        return self.key_cache[idx].clone(), self.value_cache[idx].clone()

    def shared_unchanged(self, snapshot):
        idx = self.shared_pages.reshape(-1).to(self.device)
        return torch.equal(self.key_cache[idx], snapshot[0]) and torch.equal(self.value_cache[idx], snapshot[1])

    def rows_per_plane(self, step):
        """Rows of each storage plane at a step."""
        return torch.bincount(self.descriptors_host[step, :, 1], minlength=self.planes).tolist()


def build_metadata(w, step, descriptors=None):
    from vllm_rlt_amd import ops

    if w.prefix_hints is not None:
        w.prefix_hint = w.prefix_hints[step]
    ops.build_decode_metadata(
        w.descriptors[step] if descriptors is None else descriptors, w.batch, w.batch, w.tables, PAGE, w.slots,
        w.positions, w.lengths, w.blocks, w.offsets, w.row_tables, w.width,
    )


def layer_step(w, layer):
    """KV append then decode attention of one layer.

    Every row is a different request (or a request at one depth), so no row
    reads a slot another row writes: one fused launch (with the step's prefix
    groups when the tables alias prefix pages).
    """
    from vllm_rlt_amd import ops

    if w.fused_append:
        ops.paged_decode_append(
            w.q[layer], w.key_cache[:, layer], w.value_cache[:, layer], w.row_tables, w.lengths, w.k_new[layer],
            w.v_new[layer], w.blocks, w.offsets, out=w.out[layer], workspace=w.workspace,
            shared_prefix=w.prefix_hint,
        )
        return
    ops.kv_append(w.key_cache, w.value_cache, layer, w.blocks, w.offsets, w.k_new[layer], w.v_new[layer])
    ops.paged_decode(
        w.q[layer], w.key_cache[:, layer], w.value_cache[:, layer], w.row_tables, w.lengths,
        out=w.out[layer], workspace=w.workspace, shared_prefix=w.prefix_hint,
    )


def loop_step(w, step, descriptors=None):
    build_metadata(w, step, descriptors)
    for layer in range(LAYERS):
        layer_step(w, layer)


def capture_loop_step(w):
    """One loop-step captured in a HIP graph; its descriptors are read from a static buffer."""
    from vllm_rlt_amd.graphs import GraphCache

    static = torch.empty_like(w.descriptors[0])
    static.copy_(w.descriptors[0])
    graph, _ = GraphCache(w.device).capture("loop-step", lambda: loop_step(w, 0, static))
    torch.cuda.synchronize()
    return graph, static


def step_bytes(lengths, shared_tokens=0, plane_rows=None):
    """Algorithmic HBM bytes of one loop-step (24 layer-steps) and of one decode launch.

    Returns (loop-step bytes, decode-launch bytes, decode-launch unique bytes):
    the unique figure counts the K/V of `shared_tokens` aliased prefix tokens
    once per launch and plane instead of once per row that reads them, and so
    does the loop-step figure (the decode reads each plane's shared pages once
    per launch).  plane_rows: rows at each plane (default: all at one).
    """
    kv_token = 2 * HKV * HEAD_DIM * 2  # K+V of one token in one layer (8 KiB)
    qo = 2 * HQ * HEAD_DIM * 2  # q read + out write
    new_kv = 2 * HKV * HEAD_DIM * 2
    decode = sum(kv_token * n + qo + 4 * math.ceil(n / PAGE) + 4 for n in lengths)
    append = len(lengths) * (2 * new_kv + 16)  # read new k/v, write the page slots, block+offset
    plane_rows = [len(lengths)] if plane_rows is None else plane_rows
    repeats = sum(n - 1 for n in plane_rows if n > 0)
    unique = decode - kv_token * shared_tokens * repeats
    return LAYERS * (unique + append), decode, unique


def spot_check(w):
    """Parity of the first step's layer 0 against the CPU oracle on a row sample (untimed)."""
    from oracle.paged_attention import paged_attention_cpu

    sample = [0, w.batch // 2, w.batch - 1]
    torch.cuda.synchronize()
    rows = torch.tensor(sample)
    tables = w.row_tables[rows].cpu()
    lengths = w.lengths[rows].cpu()
    need = sorted({int(b) for r in range(len(sample)) for b in tables[r, : math.ceil(int(lengths[r]) / PAGE)]})
    remap = {b: i for i, b in enumerate(need)}
    idx = torch.tensor(need, device=w.device)
    kc = w.key_cache[idx, 0].cpu()
    vc = w.value_cache[idx, 0].cpu()
    local = torch.full_like(tables, -1)
    for r in range(len(sample)):
        for c in range(math.ceil(int(lengths[r]) / PAGE)):
            local[r, c] = remap[int(tables[r, c])]
    expect = paged_attention_cpu(w.q[0][rows].cpu(), kc, vc, local, lengths)
    got = w.out[0][rows].cpu()
    err = (got.float() - expect.float()).abs().max().item()
    if not torch.allclose(got.float(), expect.float(), atol=2e-2, rtol=1e-2):
        raise SystemExit(f"parity spot check failed: max-abs error {err}")
    return err


def iqr(values):
    """[25th, 75th] percentile of the values (ms), rounded."""
    q = statistics.quantiles(values, n=4) if len(values) > 1 else [values[0]] * 3
    return [round(q[0], 5), round(q[2], 5)]


def usable_cpus():
    """Cores this process may run on: its affinity mask, limited by a cgroup CPU quota if one is set."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if quota != "max":
            n = min(n, max(1, int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    return n


def cpu_description(threads):
    """Host facts reported beside a CPU baseline."""
    model = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "cpu_model": model,
        "os_cpu_count": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "torch_threads": threads,
    }


def median_time(fn, reps):
    """Median wall time of `reps` runs of fn() after one untimed warmup run."""
    fn()
    times = []
    for _ in range(max(reps, 1)):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(w, step, reps, rows_sample=None):
    """The CPU oracle (op-for-op restatement of the reference CPU path) on one loop-step.

    Sample: the workload's rows at `step` (every `rows_sample`-th row when
    given, scaled back to the batch).  The host metadata build of the loop-step
    (_prepare_batch: write addresses, -1-padded tables, lengths,
    kv_cache_manager.py:398-478) once, then one layer-step: index_put-style KV
    append plus paged attention over a 1-layer host copy of exactly the pages
    those rows reference.  loop-steps/s = 1 / (metadata + 24 * layer-step),
    medians of `reps` runs after one warmup, on every core the process may use
    and on one thread.
    """
    from oracle import kv_ops
    from oracle.paged_attention import paged_attention_cpu

    threads = usable_cpus()
    torch.set_num_threads(threads)
    torch.cuda.synchronize()
    stride = rows_sample or 1
    picked = list(range(0, w.batch, stride))
    scale = w.batch / len(picked)
    desc = [w.descriptors_host[step].tolist()[r] for r in picked]
    host_tables = [tuple(w.tables_host[slot, plane].tolist()) for slot, plane, _ in desc]
    host_positions = [pos for _, _, pos in desc]
    sel = torch.tensor(picked)
    lengths = w.lengths.cpu()[sel]
    tables = w.row_tables.cpu()[sel]
    need = sorted({int(b) for r in range(len(picked)) for b in tables[r, : math.ceil(int(lengths[r]) / PAGE)]})
    remap = torch.full((w.num_blocks,), -1, dtype=torch.int64)
    remap[torch.tensor(need)] = torch.arange(len(need))
    idx = torch.tensor(need, device=w.device)
    kc = w.key_cache[idx, 0:1].cpu()  # [used blocks, 1 layer, page, hkv, d]
    vc = w.value_cache[idx, 0:1].cpu()
    local = torch.where(tables >= 0, remap[tables.clamp_min(0).long()], -1).to(torch.int32)
    blocks = remap[w.blocks.cpu()[sel]]
    offsets = w.offsets.cpu()[sel]
    q, k_new, v_new = w.q[0].cpu()[sel], w.k_new[0].cpu()[sel], w.v_new[0].cpu()[sel]

    def metadata():
        b, o, t, n = kv_ops.prepare_addresses(host_tables, host_positions, PAGE)
        return torch.from_numpy(b), torch.from_numpy(o), torch.from_numpy(t), torch.from_numpy(n)

    def layer():
        kv_ops.append(kc, vc, 0, blocks, offsets, k_new, v_new)
        paged_attention_cpu(q, kc[:, 0], vc[:, 0], local, lengths)

    meta_s = median_time(metadata, reps) * scale
    layer_s = median_time(layer, reps) * scale
    torch.set_num_threads(1)
    single_s = median_time(layer, reps) * scale
    torch.set_num_threads(threads)
    loop_s = meta_s + LAYERS * layer_s
    rows_text = f"all {w.batch} rows" if stride == 1 else f"every {stride}th row ({len(picked)} of {w.batch}, x{scale:g})"
    return {
        "value": 1.0 / loop_s,
        "unit": "loop-steps/s",
        "cores": threads,
        "kind": "port",
        "single_thread_value": 1.0 / (meta_s + LAYERS * single_s),
        **cpu_description(threads),
        "sample": f"one loop-step of {rows_text}: the host metadata build ({meta_s * 1e3:.2f} ms) plus "
        f"one layer-step (append + attention, 1-layer pool) extrapolated x{LAYERS} layers; "
        f"{layer_s * 1e3:.1f} ms/layer-step on {threads} threads, {single_s * 1e3:.1f} ms on 1 thread "
        f"(medians of {reps} after 1 warmup)",
    }


def config1_exact(seed, device, reps):
    """The reference CPU case timed exactly: batch 4, 16/16 heads, head_dim 128, page 16,
    contexts U[1, 256], one layer, one depth, one appended token per sequence, then
    decode attention.  CPU: host metadata + index_put append + the oracle's
    attention; GPU: the fused append + decode launch on the same inputs (events
    around 100 launches).  Microseconds per step, medians."""
    from oracle import kv_ops
    from oracle.paged_attention import paged_attention_cpu
    from vllm_rlt_amd import ops

    g = torch.Generator().manual_seed(seed)
    rows = 4
    contexts = torch.randint(1, 257, (rows,), generator=g)
    pages = [(int(c) + 1 + PAGE - 1) // PAGE for c in contexts]
    nb = sum(pages) + 2
    perm = torch.randperm(nb, generator=g)
    tables = torch.full((rows, max(pages)), -1, dtype=torch.int32)
    used = 0
    for r, n in enumerate(pages):
        tables[r, :n] = perm[used : used + n].to(torch.int32)
        used += n
    kc = torch.randn(nb, 1, PAGE, HKV, HEAD_DIM, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, 1, PAGE, HKV, HEAD_DIM, generator=g).to(torch.bfloat16)
    q = torch.randn(rows, HQ, HEAD_DIM, generator=g).to(torch.bfloat16)
    k_new = torch.randn(rows, HKV, HEAD_DIM, generator=g).to(torch.bfloat16)
    v_new = torch.randn(rows, HKV, HEAD_DIM, generator=g).to(torch.bfloat16)
    table_rows = [tuple(int(x) for x in tables[r, : pages[r]]) for r in range(rows)]
    positions = [int(c) for c in contexts]

    def cpu_step():
        b, o, t, n = kv_ops.prepare_addresses(table_rows, positions, PAGE)
        kv_ops.append(kc, vc, 0, torch.from_numpy(b), torch.from_numpy(o), k_new, v_new)
        return paged_attention_cpu(q, kc[:, 0], vc[:, 0], torch.from_numpy(t), torch.from_numpy(n))

    threads = usable_cpus()
    torch.set_num_threads(threads)
    cpu_s = median_time(cpu_step, reps)
    torch.set_num_threads(1)
    single_s = median_time(cpu_step, reps)
    torch.set_num_threads(threads)
    expect = cpu_step()
    # GPU: same inputs; appending the same token again rewrites the same bits.
    b, o, t, n = (torch.from_numpy(x).to(device) for x in kv_ops.prepare_addresses(table_rows, positions, PAGE))
    dk, dv = kc.to(device), vc.to(device)
    dq, dkn, dvn = q.to(device), k_new.to(device), v_new.to(device)
    out = torch.empty_like(dq)
    ws = torch.empty(ops.decode_workspace_bytes(rows, HQ, HKV, HEAD_DIM), dtype=torch.uint8, device=device)

    def gpu_step():
        ops.paged_decode_append(dq, dk[:, 0], dv[:, 0], t, n, dkn, dvn, b, o, out=out, workspace=ws)

    gpu_step()
    torch.cuda.synchronize()
    if not torch.allclose(out.cpu().float(), expect.float(), atol=2e-2, rtol=1e-2):
        raise SystemExit("config-1 parity check failed")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(100):
        gpu_step()
    end.record()
    torch.cuda.synchronize()
    gpu_us = start.elapsed_time(end) * 10.0
    lengths = [p + 1 for p in positions]
    step_bytes_1 = sum(2 * HKV * HEAD_DIM * 2 * n + 4 * HQ * HEAD_DIM * 2 + 4 * HKV * HEAD_DIM * 2 for n in lengths)
    return {
        "workload": "batch 4, 16/16 heads, head_dim 128, page 16, bf16, contexts U[1,256] "
        f"({positions}), 1 layer, 1 depth: append 1 token per sequence, then decode attention",
        "cpu_us_per_step": round(cpu_s * 1e6, 1),
        "cpu_single_thread_us_per_step": round(single_s * 1e6, 1),
        "cpu_threads": threads,
        "gpu_us_per_step": round(gpu_us, 2),
        "algorithmic_bytes_per_step": step_bytes_1,
        "gpu_gb_per_s": round(step_bytes_1 / (gpu_us * 1e-6) / 1e9, 1),
        "reps": f"CPU medians of {reps} after 1 warmup; GPU mean of 100 launches between two events",
    }


class PrefillWorkload:
    """LAST-EXITED pool, per-depth packed-prefill metadata and per-layer chunk projections."""

    def __init__(self, seed, device):
        g = torch.Generator().manual_seed(seed)
        n, chunk = PREFILL["seqs"], PREFILL["chunk"]
        lo, hi = PREFILL["prefix"]
        self.prefixes = torch.randint(lo, hi + 1, (n,), generator=g)
        self.lens = self.prefixes + chunk
        pages = (self.lens + PAGE - 1) // PAGE
        self.width = int(pages.max())
        self.num_blocks = int(pages.sum()) * LOOPS
        perm = torch.randperm(self.num_blocks, generator=g)
        tables = torch.zeros(n, LOOPS, self.width, dtype=torch.int32)
        used = 0
        for s in range(n):
            for plane in range(LOOPS):
                k = int(pages[s])
                tables[s, plane, :k] = perm[used : used + k].to(torch.int32)
                used += k
        rows = torch.arange(n).repeat_interleave(chunk)
        pos = (self.prefixes[rows] + torch.arange(chunk).repeat(n)).long()
        self.depth_blocks = [tables[rows, d, pos // PAGE].long().to(device) for d in range(LOOPS)]
        self.offsets = (pos % PAGE).to(device)
        self.depth_tables = [tables[:, d].contiguous().to(device) for d in range(LOOPS)]
        self.context_lengths = self.lens.to(torch.int32).to(device)
        self.cu = torch.arange(0, (n + 1) * chunk, chunk, dtype=torch.int32).to(device)
        shape = (self.num_blocks, LAYERS, PAGE, HKV, HEAD_DIM)
        self.key_cache = torch.empty(shape, dtype=torch.bfloat16, device=device)
        self.value_cache = torch.empty(shape, dtype=torch.bfloat16, device=device)
        gen = torch.Generator(device=device).manual_seed(seed + 1)
        for pool in (self.key_cache, self.value_cache):
            flat = pool.view(-1)
            for start in range(0, flat.numel(), 1 << 28):
                flat[start : start + (1 << 28)].normal_(generator=gen)
        total = n * chunk
        self.q = torch.randn((LAYERS, total, HQ, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        self.k_new = torch.randn((LAYERS, total, HKV, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        self.v_new = torch.randn((LAYERS, total, HKV, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        self.out = torch.empty_like(self.q)

    def flops(self):
        """Visible (query, key) pairs x 4 * Hq * D over 4 depths x 24 layers (QK^T and PV)."""
        chunk = PREFILL["chunk"]
        pairs = sum(chunk * int(p) + chunk * (chunk + 1) // 2 for p in self.prefixes)
        return 4 * HQ * HEAD_DIM * pairs * LOOPS * LAYERS

    def layer(self, depth, layer, events=None):
        from vllm_rlt_amd import ops

        ops.kv_append(
            self.key_cache, self.value_cache, layer, self.depth_blocks[depth], self.offsets,
            self.k_new[layer], self.v_new[layer],
        )
        if events is not None:
            events[0].record()
        ops.paged_prefill(
            self.q[layer], self.key_cache[:, layer], self.value_cache[:, layer], self.depth_tables[depth],
            self.context_lengths, self.cu, PREFILL["chunk"], out=self.out[layer],
        )
        if events is not None:
            events[1].record()

    def step(self):
        for depth in range(LOOPS):
            for layer in range(LAYERS):
                self.layer(depth, layer)


def prefill_spot_check(w):
    """Parity of the last (depth 3, layer 23) prefill on a few query rows against the CPU oracle."""
    from oracle.paged_attention import paged_attention_cpu

    torch.cuda.synchronize()
    chunk = PREFILL["chunk"]
    picks = [(0, 0), (0, chunk - 1), (PREFILL["seqs"] - 1, chunk // 2)]
    tables = w.depth_tables[LOOPS - 1].cpu()
    worst = 0.0
    for s, i in picks:
        n = int(w.prefixes[s]) + i + 1
        pages = [int(b) for b in tables[s, : (n + PAGE - 1) // PAGE]]
        idx = torch.tensor(pages, device=w.key_cache.device)
        kc = w.key_cache[idx, LAYERS - 1].cpu()
        vc = w.value_cache[idx, LAYERS - 1].cpu()
        local = torch.arange(len(pages), dtype=torch.int32)[None]
        row = s * chunk + i
        expect = paged_attention_cpu(w.q[LAYERS - 1][row : row + 1].cpu(), kc, vc, local, torch.tensor([n], dtype=torch.int32))
        got = w.out[LAYERS - 1][row : row + 1].cpu()
        err = (got.float() - expect.float()).abs().max().item()
        if not torch.allclose(got.float(), expect.float(), atol=2e-2, rtol=1e-2):
            raise SystemExit(f"prefill parity spot check failed at seq {s} row {i}: max-abs {err}")
        worst = max(worst, err)
    return worst


def prefill_cpu_baseline(w, reps, stride=32):
    """The per-token CPU oracle on a bounded sample of the prefill launch.

    Sample: every `stride`-th query row of every chunk at depth 0, layer 0 (each
    row attends over its own causal length), against a 1-layer host copy of the
    pages those sequences reference.  TFLOP/s = the sampled rows' algorithmic
    FLOPs / median time, comparable with the kernel's per-launch rate.
    """
    from oracle.paged_attention import paged_attention_cpu

    threads = usable_cpus()
    torch.set_num_threads(threads)
    chunk = PREFILL["chunk"]
    tables = w.depth_tables[0].cpu()
    lens = w.lens
    need = sorted({int(b) for s in range(len(lens)) for b in tables[s, : math.ceil(int(lens[s]) / PAGE)]})
    remap = torch.full((w.num_blocks,), -1, dtype=torch.int64)
    remap[torch.tensor(need)] = torch.arange(len(need))
    idx = torch.tensor(need, device=w.key_cache.device)
    kc = w.key_cache[idx, 0].cpu()  # [used blocks, page, hkv, d]
    vc = w.value_cache[idx, 0].cpu()
    rows, row_lens, row_seq = [], [], []
    for s in range(len(lens)):
        for i in range(0, chunk, stride):
            rows.append(s * chunk + i)
            row_lens.append(int(w.prefixes[s]) + i + 1)
            row_seq.append(s)
    local = torch.where(tables >= 0, remap[tables.clamp_min(0).long()], -1).to(torch.int32)[row_seq]
    q = w.q[0][rows].cpu()
    lengths = torch.tensor(row_lens, dtype=torch.int32)

    def attend():
        paged_attention_cpu(q, kc, vc, local, lengths)

    t_multi = median_time(attend, reps)
    torch.set_num_threads(1)
    t_single = median_time(attend, reps)
    torch.set_num_threads(threads)
    flops = 4 * HQ * HEAD_DIM * sum(row_lens)
    return {
        "value": flops / t_multi / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "single_thread_value": flops / t_single / 1e12,
        **cpu_description(threads),
        "sample": f"{len(rows)} query rows (1 in {stride} of each 512-token chunk, depth 0, layer 0, "
        f"{sum(row_lens)} visible keys), medians of {reps} after 1 warmup: {t_multi * 1e3:.1f} ms on {threads} "
        f"threads, {t_single * 1e3:.1f} ms on 1 thread",
    }


def run_prefill(args, device):
    t_setup = time.perf_counter()
    w = PrefillWorkload(args.seed, device)
    torch.cuda.synchronize()
    print(
        f"[bench] workload ouro-prefill: {PREFILL['seqs']} x {PREFILL['chunk']} tokens, prefixes "
        f"{w.prefixes.tolist()}, pool {2 * w.key_cache.numel() * 2 / 1e9:.1f} GB, setup "
        f"{time.perf_counter() - t_setup:.1f}s",
        file=sys.stderr,
        flush=True,
    )
    err = None
    for step in range(args.warmup):
        w.step()
        if step == 0 and not args.no_check:
            err = prefill_spot_check(w)
            print(f"[bench] ouro-prefill: parity spot check ok (max-abs {err:.3g})", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        w.step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # Events are created before the pass, so no event creation sits between launches.
    pairs = [
        (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        for _ in range(args.steps * LOOPS * LAYERS)
    ]
    events = iter(pairs)
    for _ in range(args.steps):
        for depth in range(LOOPS):
            for layer in range(LAYERS):
                w.layer(depth, layer, next(events))
    torch.cuda.synchronize()
    launch_list = [a.elapsed_time(b) for a, b in pairs]
    launch_ms = statistics.fmean(launch_list)
    flops = w.flops()
    launch_tflops = flops / (LOOPS * LAYERS) / (launch_ms * 1e-3) / 1e12
    step_tflops = flops * args.steps / elapsed / 1e12
    line = {
        "metric": "chunked prefill attention: bf16 MFMA TFLOP/s (% of dense peak)",
        "value": round(step_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "parity_max_abs": err,
        "config": {
            "workload": f"ouro-prefill: {PREFILL['seqs']} sequences x {PREFILL['chunk']} new tokens over prefixes "
            f"U{list(PREFILL['prefix'])}, 16/16 heads, head_dim 128, page 16, LAST-EXITED, step = 4 depths x 24 "
            "layers x (chunk KV append + packed causal prefill attention)",
            "global_batch": PREFILL["seqs"],
            "seq_len": PREFILL["chunk"],
            "parallelism": "single-gpu",
        },
        "roofline": {
            "kernel": "rlt_paged_prefill (paged_prefill_mfma_kernel)",
            "bound": "mfma",
            "achieved": round(launch_tflops, 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(launch_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": profiled_traffic("ouro-prefill"),
            "rocprof_avg_launch_ms": profiled_launch_ms("ouro-prefill"),
            "avg_launch_ms": round(launch_ms, 5),
            "median_launch_ms": round(statistics.median(launch_list), 5),
            "launch_ms_iqr": iqr(launch_list),
            "algorithmic_flops_per_launch": int(flops / (LOOPS * LAYERS)),
        },
    }
    if not args.no_cpu_baseline:
        print("[bench] ouro-prefill: timing the CPU oracle baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = prefill_cpu_baseline(w, args.cpu_reps)
    release(w)
    return line


def release(*objects):
    """Drop a workload's device memory before the next one is set up."""
    for obj in objects:
        del obj
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def run_decode(args, name, device, with_cpu=True):
    """One decode workload: timed loop-steps, the per-step launch window, parity, CPU baseline."""
    total = args.warmup + args.steps
    t_setup = time.perf_counter()
    w = Workload(name, total, args.seed, device)
    w.fused_append = args.append == "fused"
    torch.cuda.synchronize()
    print(
        f"[bench] workload {name}: batch {w.batch}, planes {w.planes}, pool "
        f"{w.pool_bytes() / 1e9:.1f} GB ({w.num_blocks} pages), setup {time.perf_counter() - t_setup:.1f}s",
        file=sys.stderr,
        flush=True,
    )

    snapshot = w.shared_snapshot()
    # Warmup (also the parity spot check on step 0).
    spot = None
    for step in range(args.warmup):
        loop_step(w, step)
        if step == 0 and not args.no_check:
            spot = spot_check(w)
            print(f"[bench] {name}: parity spot check ok (max-abs {spot:.3g})", file=sys.stderr, flush=True)
    torch.cuda.synchronize()

    # Timed region: exactly `steps` loop-steps.
    total_bytes = 0
    decode_bytes, unique_bytes = [], []
    for step in range(args.warmup, total):
        b, d, u = step_bytes(w.lengths_at(step), w.prefix_tokens, w.rows_per_plane(step))
        total_bytes += b
        decode_bytes.append(d)
        unique_bytes.append(u)
    graph = None
    if args.graph:
        if w.prefix_hints is not None:
            raise SystemExit("--graph replays one step's metadata; the prefix workloads change their groups per step")
        graph, static = capture_loop_step(w)
        for step in range(args.warmup):  # warm the replay path too
            static.copy_(w.descriptors[step])
            graph.replay()
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    # Eager steps also mark the end of their metadata build: the window from
    # there to the step's end holds exactly its 24 layer launches.
    launched = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    t0 = time.perf_counter()
    marks[0].record()
    if graph is None:
        for i, step in enumerate(range(args.warmup, total)):
            build_metadata(w, step)
            launched[i].record()
            for layer in range(LAYERS):
                layer_step(w, layer)
            marks[i + 1].record()
    else:
        for i, step in enumerate(range(args.warmup, total)):
            static.copy_(w.descriptors[step])
            graph.replay()
            marks[i + 1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_ms = [marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps)]
    if graph is not None:
        # The replayed steps must leave the same outputs as eager steps.
        last = w.out.clone()
        loop_step(w, total - 1)
        torch.cuda.synchronize()
        if not torch.equal(last.view(torch.int16), w.out.view(torch.int16)):
            raise SystemExit("graph replay differs from eager execution")

    # Launch timing, from the timed steps themselves (all work is on the
    # current stream): a launch's time is its step's launch window / 24, gaps
    # between launches included, so 24 launches never add up to more than a
    # step.  No event sits between two launches of a window.  Graph replays
    # have no such mark; their step window (metadata build included) is used.
    if graph is None:
        windows = [launched[i].elapsed_time(marks[i + 1]) for i in range(args.steps)]
    else:
        windows = step_ms
    launch_ms = [t / LAYERS for t in windows]
    decode_ms = statistics.fmean(launch_ms)
    # The fused launch also moves the new tokens: 8 KiB read + 8 KiB written + 16 B of address per row;
    # with a separate append launch, the window holds the append too.
    append_bytes = w.batch * (4 * HKV * HEAD_DIM * 2 + 16)
    decode_avg_bytes = statistics.fmean(decode_bytes) + append_bytes
    unique_avg_bytes = statistics.fmean(unique_bytes) + append_bytes
    # Aliased prefix pages are read by every row but fetched from HBM about
    # once per launch: the roofline uses the unique bytes.
    achieved = unique_avg_bytes / (decode_ms * 1e-3) / 1e9
    if snapshot is not None:
        if not w.shared_unchanged(snapshot):
            raise SystemExit("aliased prefix pages changed during the run")
        print(f"[bench] {name}: aliased prefix pages unchanged (bitwise)", file=sys.stderr, flush=True)
        del snapshot

    steps_per_s = args.steps / elapsed
    gbs = total_bytes / elapsed / 1e9
    prefix = w.prefix_hints is not None
    if w.fused_append and prefix:
        kernel = (
            "rlt_paged_decode_shared_prefix with its append (paged_decode_prefix_kernel: prefix workers over "
            "every plane's prefix beside the split pass reading each row's new token in place; "
            "paged_decode_merge_kernel storing it)"
        )
    elif w.fused_append:
        kernel = (
            "rlt_paged_decode_append (paged_decode_kernel split pass reading each row's new token in place + "
            "paged_decode_merge_kernel storing it)"
        )
    elif not prefix:
        kernel = "rlt_kv_append + rlt_paged_decode (paged_decode_kernel split pass + paged_decode_merge_kernel)"
    else:
        kernel = (
            "rlt_kv_append + rlt_paged_decode_shared_prefix (paged_decode_prefix_kernel: prefix workers + "
            "split pass; paged_decode_merge_kernel)"
        )
    line = {
        "metric": "paged decode attn+KV append: HBM GB/s (% peak), loop-steps/s at Ouro-1.4B",
        "value": round(steps_per_s, 3),
        "unit": "loop-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": describe(name),
            "global_batch": w.batch,
            "seq_len": int(w.contexts.float().mean().item()),
            "parallelism": "single-gpu",
            "launch": "hip-graph replay" if graph is not None else "eager",
            "append": "fused into the decode launch" if w.fused_append else "own launch before the decode",
        },
        "hbm_gb_per_s": round(gbs, 1),
        "hbm_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "step_ms_median": round(statistics.median(step_ms), 4),
        "step_ms_iqr": iqr(step_ms),
        "parity_max_abs": spot,
        "roofline": {
            "kernel": kernel,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(name),
            "rocprof_avg_launch_ms": profiled_launch_ms(name),
            "avg_launch_ms": round(decode_ms, 5),
            "median_launch_ms": round(statistics.median(launch_ms), 5),
            "launch_ms_iqr": iqr(launch_ms),
            "launch_timing": "timed loop-steps: event after the metadata build to the step's end event, / 24 "
            "(gaps between launches included)",
            "algorithmic_bytes_per_launch": int(unique_avg_bytes),
        },
    }
    if w.prefix_tokens:
        line["roofline"]["per_request_bytes_per_launch"] = int(decode_avg_bytes)
        line["roofline"]["per_request_gb_per_s"] = round(decode_avg_bytes / (decode_ms * 1e-3) / 1e9, 1)
    if with_cpu and not args.no_cpu_baseline:
        print(f"[bench] {name}: timing the CPU oracle baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(w, total - 1, args.cpu_reps, rows_sample=CPU_ROW_SAMPLE.get(name))
    release(w)
    return line


def compact(line):
    """A secondary workload's figures for the headline line's `workloads` key."""
    keep = ("metric", "value", "unit", "ms_per_step", "steps", "warmup", "hbm_gb_per_s", "hbm_frac_of_peak",
            "step_ms_median", "step_ms_iqr", "parity_max_abs", "config", "roofline", "cpu_baseline")
    return {k: line[k] for k in keep if k in line}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on one GPU: --gpus {args.gpus} is not supported; decode shards by request or "
            "KV head with no cross-GPU exchange, so one GPU's throughput is the per-GPU figure",
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm device")
    from vllm_rlt_amd import _native

    if not _native.LIBRARY_PATH.exists():
        import __graft_entry__

        __graft_entry__.build()
    _native.load()

    device = torch.device("cuda:0")
    if args.calibrate_counters:
        calibrate_counters(device)
        return
    if args.workload == "ouro-prefill":
        print(json.dumps(run_prefill(args, device)), flush=True)
        return
    line = run_decode(args, args.workload, device)
    if args.workload == HEADLINE and not args.only:
        # The other measured configs, each after the previous pool is freed.
        extra = {}
        for name in SECONDARY:
            t0 = time.perf_counter()
            extra[name] = compact(run_prefill(args, device) if name == "ouro-prefill" else run_decode(args, name, device))
            print(f"[bench] {name} done in {time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)
        line["workloads"] = extra
        if not args.no_cpu_baseline and "cpu_baseline" in line:
            line["cpu_baseline"]["config1_exact"] = config1_exact(args.seed, device, args.cpu_reps)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
