"""Prefill ordering on the host (worker/model_runner.py:247-320), with a recording cache (CPU only)."""

from types import SimpleNamespace

import pytest
import torch

from vllm_rlt_amd.prefill_order import PrefillItem, PrefillOrder


class RecordingCache:
    def __init__(self, layout, packed):
        self.layout = layout
        self.attention = SimpleNamespace(supports_packed_prefill=packed)
        self.calls = []

    def _prepare_batch(self, ids, depths, positions, packed_prefill=False):
        self.calls.append(("prepare", tuple(ids), tuple(depths), tuple(positions), packed_prefill))
        return SimpleNamespace(depth=depths[0], positions=list(positions))


def order(cache, loops=3):
    def prelude(tokens):
        cache.calls.append(("prelude", tuple(tokens.tolist())))
        return tokens.to(torch.float32)

    def core(hidden, batch, c):
        assert c is cache
        c.calls.append(("core", batch.depth, tuple(batch.positions)))
        return hidden + 1000, None  # tuple results take their first element

    return PrefillOrder(cache, prelude, core, loops, "cpu", prefill_uva=False)


def test_last_exited_packed_is_depth_major_over_the_whole_chunk():
    cache = RecordingCache("last_exited", packed=True)
    items = [PrefillItem("a", 2, 3, list(range(10, 20))), PrefillItem("b", 0, 2, [7, 8, 9])]
    saved = order(cache).prefill(items)
    ids, positions = ("a", "a", "a", "b", "b"), (2, 3, 4, 0, 1)
    assert cache.calls == [
        ("prelude", (12, 13, 14, 7, 8)),
        *[
            call
            for depth in range(3)
            for call in (("prepare", ids, (depth,) * 5, positions, True), ("core", depth, positions))
        ],
    ]
    # Each item saves its last row after every loop.
    assert [float(h) for h in saved] == [14 + 3000, 8 + 3000]


def test_without_packed_prefill_every_token_is_a_decode_row():
    cache = RecordingCache("last_exited", packed=False)
    order(cache, loops=2).prefill([PrefillItem("a", 0, 3, [4, 5, 6])])
    assert [c[4] for c in cache.calls if c[0] == "prepare"] == [False, False]


def test_shared_runs_every_loop_of_a_position_before_the_next():
    cache = RecordingCache("shared", packed=True)
    items = [PrefillItem("a", 1, 3, [9, 10, 11, 12]), PrefillItem("b", 0, 1, [5])]
    saved = order(cache, loops=2).prefill(items)
    cores = [(c[1], c[2]) for c in cache.calls if c[0] == "core"]
    assert cores == [(0, (1, 0)), (1, (1, 0)), (0, (2,)), (1, (2,)), (0, (3,)), (1, (3,))]
    assert all(not c[4] for c in cache.calls if c[0] == "prepare")
    assert [float(h) for h in saved] == [12 + 2000, 5 + 2000]


def test_bad_arguments():
    cache = RecordingCache("last_exited", packed=True)
    with pytest.raises(ValueError, match="loops"):
        order(cache, loops=0)
    with pytest.raises(ValueError, match="equal length"):
        order(cache).prefill_tokens(["a"], [0, 1], [3])
    assert order(cache).prefill([]) == []
