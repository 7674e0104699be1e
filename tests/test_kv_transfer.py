"""Segment format of page transfers (CPU): kv_segments and partition_segments.

The exact, ordered output of both functions is pinned by
tests/golden/pd_segments.json, recorded from the reference's own
kv_segments / partition_segments (vllm_rlt/pd/transport.py:18-68): the order
is part of the format, since a peer pairs its segments with ours one by one.
Beyond that, the byte ranges are pinned the way the reference's own test pins
them (tests/test_pd.py:47-82): the union of the segments must be exactly the
bytes of tokens [start, end) at every layer, depth and K/V plane, computed by
brute force from the closed-form address (block, layer, token); partitions must
conserve bytes and respect both limits.  Known page ids come from the host
page book, which reproduces the reference's allocator page for page.
"""

import json
from pathlib import Path

import pytest

from vllm_rlt_amd.kv_transfer import kv_segments, partition_segments
from vllm_rlt_amd.page_book import KVPageBook


def layout_info(num_layers=3, block_size=4, num_blocks=24, heads=2, head_dim=8, element=4):
    token = heads * head_dim * element
    layer = block_size * token
    return dict(
        block_size=block_size,
        num_blocks=num_blocks,
        num_layers=num_layers,
        device=0,
        block_bytes=num_layers * layer,
        layer_bytes=layer,
        token_bytes=token,
        key_ptr=0,
        value_ptr=10**9,
    )


def brute_force(info, tables, start, end):
    expected = set()
    for table in tables:
        for token in range(start, end):
            for layer in range(info["num_layers"]):
                for base in (info["key_ptr"], info["value_ptr"]):
                    pos = (
                        base
                        + table[token // info["block_size"]] * info["block_bytes"]
                        + layer * info["layer_bytes"]
                        + (token % info["block_size"]) * info["token_bytes"]
                    )
                    expected.update(range(pos, pos + info["token_bytes"]))
    return expected


@pytest.mark.parametrize("start,end", [(2, 9), (0, 8), (4, 5), (0, 1), (3, 12)])
def test_segments_cover_exactly_the_valid_tokens_of_every_layer_and_depth(start, end):
    book = KVPageBook(3, 2, 8, 24, 4, 4)
    assert book.allocate("a", 12)
    info = layout_info()
    tables = book._get_allocation("a").block_tables
    segments = list(kv_segments(info, tables, start, end))
    actual = set()
    for address, size, device in segments:
        assert device == 0 and size > 0
        actual.update(range(address, address + size))
    assert actual == brute_force(info, tables, start, end)
    # Segments never overlap, so the byte count is the set size.
    assert sum(size for _, size, _ in segments) == len(actual)
    # A fully valid page is one segment of the whole block.
    full_pages = [p for p in range(start // 4, (end - 1) // 4 + 1) if p * 4 >= start and p * 4 + 4 <= end]
    assert sum(size == info["block_bytes"] for _, size, _ in segments) == 2 * len(tables) * len(full_pages)


def test_partitions_conserve_bytes_and_respect_limits():
    book = KVPageBook(3, 2, 8, 24, 4, 4)
    assert book.allocate("a", 9)
    info = layout_info()
    segments = list(kv_segments(info, book._get_allocation("a").block_tables, 2, 9))
    parts = list(partition_segments(segments, segments, 333, 3))
    assert sum(n for _, _, n in parts) == sum(s for _, s, _ in segments)
    assert all(n <= 333 and len(src) <= 3 and src == dst for src, dst, n in parts)
    # Splitting preserves address order within the original segments.
    flat = [(a, s) for src, _, _ in parts for a, s, _ in src]
    joined, i = [], 0
    for address, size, _ in segments:
        covered = 0
        while covered < size:
            a, s = flat[i]
            assert a == address + covered
            covered += s
            i += 1
    assert i == len(flat)


def test_invalid_ranges_and_mismatched_geometry_raise():
    book = KVPageBook(3, 2, 8, 24, 4, 4)
    assert book.allocate("a", 8)
    info = layout_info()
    tables = book._get_allocation("a").block_tables
    with pytest.raises(ValueError, match="invalid KV range"):
        list(kv_segments(info, tables, 5, 5))
    with pytest.raises(ValueError, match="exceeds allocation"):
        list(kv_segments(info, tables, 0, 9))
    with pytest.raises(ValueError, match="outside registered pool"):
        list(kv_segments(dict(info, num_blocks=1), tables, 0, 8))
    segs = list(kv_segments(info, tables, 0, 6))
    with pytest.raises(ValueError, match="incompatible"):
        list(partition_segments(segs, segs[:-1], 1000, 10))


GOLDEN = json.loads((Path(__file__).parent / "golden" / "pd_segments.json").read_text())


@pytest.mark.parametrize("case", range(len(GOLDEN["cases"])))
def test_segment_lists_equal_the_reference_recording(case):
    c = GOLDEN["cases"][case]
    segments = kv_segments(c["info"], c["tables"], c["start"], c["end"])
    assert [list(s) for s in segments] == c["segments"]
    # Union of the recorded segments is exactly the brute-force byte set, so the
    # fixture itself agrees with the closed-form address map.
    if sum(n for _, n, _ in segments) <= 1 << 16:
        covered = set()
        for address, size, _ in segments:
            covered.update(range(address, address + size))
        assert covered == brute_force(c["info"], c["tables"], c["start"], c["end"])
    assert c["partitions"], "every case carries at least one partition recording"
    for p in c["partitions"]:
        target = [(a + 12345, n, 1) for a, n, _ in segments]
        parts = partition_segments(segments, target, p["byte_limit"], p["descriptor_limit"])
        got = [[[list(x) for x in src], [list(x) for x in dst], n] for src, dst, n in parts]
        assert got == p["parts"]


@pytest.mark.parametrize("entry", GOLDEN["errors"], ids=lambda e: e["case"])
def test_segment_errors_match_the_reference(entry):
    if entry["error"] is None:
        kv_segments(entry["info"], entry["tables"], entry["start"], entry["end"])
    else:
        with pytest.raises(ValueError) as err:
            kv_segments(entry["info"], entry["tables"], entry["start"], entry["end"])
        assert str(err.value) == entry["error"]


def test_partition_mismatch_message_matches_the_reference():
    with pytest.raises(ValueError) as err:
        partition_segments([(0, 8, 0), (64, 8, 0)], [(0, 8, 0)], 100, 4)
    assert str(err.value) == GOLDEN["partition_mismatch_error"]


def test_planted_order_mistakes_fail_the_golden():
    """Orders a plausible rewrite could produce (V before K, layers outermost,
    tables innermost) cover the same bytes but fail the recorded list."""
    c = next(c for c in GOLDEN["cases"] if len(c["tables"]) > 1 and c["start"] % c["info"]["block_size"])
    segs = [tuple(s) for s in c["segments"]]
    info = c["info"]
    v_first = sorted(segs, key=lambda s: (s[0] < info["value_ptr"], s[0]))
    by_address = sorted(segs)
    for wrong in (v_first, by_address, segs[::-1]):
        assert sorted(wrong) == sorted(segs)
        assert [list(s) for s in wrong] != c["segments"]
