"""The bench's byte accounting and synthetic workloads (CPU only).

The roofline figures rest on two things checked here: the algorithmic bytes of
a decode launch follow the per-row formula the metric is defined by (K+V page
reads, the appended token's read and write, q and out, table entries, length
and write address), and the synthetic schedules have the layout each workload
claims (every plane's prefix aliased by every row, private pages never shared,
page ids inside the pool).
"""

import math

import pytest
import torch

import bench

KV_TOKEN = 2 * 16 * 128 * 2  # K+V of one token in one layer at Ouro heads (8 KiB)


def by_hand(lengths):
    """The per-row formula spelled out: 8192 n + 8192 (new K/V read) + 8192 (page write)
    + 8192 (q read + out write) + 4 ceil(n / 16) + 20."""
    return sum(8192 * n + 8192 + 8192 + 8192 + 4 * math.ceil(n / 16) + 20 for n in lengths)


def test_launch_and_step_bytes_follow_the_per_row_formula():
    lengths = [1, 16, 17, 4096, 2437]
    step, decode, unique = bench.step_bytes(lengths)
    assert decode == unique
    append = len(lengths) * (2 * KV_TOKEN + 16)
    assert decode + append == by_hand(lengths)
    assert step == bench.LAYERS * by_hand(lengths)


def test_aliased_prefix_bytes_count_once_per_plane():
    lengths = [5000, 6000, 7000, 8000, 4500, 4700]
    shared = 2048
    # Rows per plane: 2 at plane 0, 1 at plane 1, none at plane 2, 3 at plane 3.
    step, decode, unique = bench.step_bytes(lengths, shared, [2, 1, 0, 3])
    assert decode - unique == KV_TOKEN * shared * (1 + 0 + 2)
    # One plane holding every row: the prefix is read once instead of six times.
    _, _, one_plane = bench.step_bytes(lengths, shared)
    assert decode - one_plane == KV_TOKEN * shared * 5
    assert step == bench.LAYERS * (unique + len(lengths) * (2 * KV_TOKEN + 16))


@pytest.mark.parametrize("name", ["ouro-prefix-last-exited", "ouro-prefix-stress", "ouro-last-exited"])
def test_schedules_alias_exactly_each_planes_prefix(name):
    steps = 3
    desc, tables, num_blocks, contexts, shared = bench.make_schedule(name, steps, seed=0)
    cfg = bench.WORKLOADS[name]
    planes, prefix_pages = cfg["planes"], cfg["prefix"] // bench.PAGE
    assert tables.shape[:2] == (cfg["batch"], planes)
    assert shared.shape == (planes, prefix_pages)
    if prefix_pages:
        # Every row's plane-p table begins with plane p's prefix; the planes' prefixes differ.
        for p in range(planes):
            assert torch.equal(tables[:, p, :prefix_pages], shared[p].to(torch.int32).expand(cfg["batch"], -1))
        assert len(set(shared.reshape(-1).tolist())) == planes * prefix_pages
    # Pages each row needs for every position the run touches; private pages appear once in the pool.
    private = []
    for r in range(cfg["batch"]):
        need = -(-(int(contexts[r]) + steps) // bench.PAGE)
        for p in range(planes):
            row = tables[r, p, :need].tolist()
            assert all(0 <= b < num_blocks for b in row)
            private += row[prefix_pages:]
    assert len(private) == len(set(private))
    assert not set(private) & set(shared.reshape(-1).tolist())
    # Descriptors: one row per request, the depth's plane, positions advancing by one per step.
    assert desc.shape == (steps, cfg["batch"], 3)
    assert torch.equal(desc[1, :, 2] - desc[0, :, 2], torch.ones(cfg["batch"], dtype=torch.int64))
    assert int(desc[:, :, 1].max()) < planes
