"""Host side of the prefix-group decode hint (CPU only)."""

import numpy as np
import pytest

from vllm_rlt_amd import ops

FIELDS = ops.GROUP_FIELDS


def test_split_length_follows_the_decode_plan():
    # 256-token splits up to 64 of them, then the length doubles until 64 cover the row.
    assert ops.decode_split_len(0) == 256
    assert ops.decode_split_len(1) == 256
    assert ops.decode_split_len(64 * 256) == 256
    assert ops.decode_split_len(64 * 256 + 1) == 512
    assert ops.decode_split_len(64 * 512) == 512
    assert ops.decode_split_len(64 * 512 + 1) == 1024
    for n in (1, 300, 16384, 16385, 40000, 1 << 20):
        per = ops.decode_split_len(n)
        assert -(-n // per) <= 64 and (per == 256 or -(-n // (per // 2)) > 64)


def sections(layout, n_rows):
    """Split a hint into its sections (row_group, records, item_start, members, pages)."""
    hint, n_groups, n_members, n_pages, n_items, group_size = layout
    assert hint.dtype == np.int32
    assert len(hint) == n_rows + (FIELDS + 1) * n_groups + 1 + n_members + n_pages
    row_group = hint[:n_rows]
    records = hint[n_rows : n_rows + FIELDS * n_groups].reshape(n_groups, FIELDS)
    at = n_rows + FIELDS * n_groups
    item_start = hint[at : at + n_groups + 1]
    members = hint[at + n_groups + 1 : at + n_groups + 1 + n_members]
    pages = hint[at + n_groups + 1 + n_members :]
    assert item_start[-1] == n_items and len(pages) == n_pages
    return row_group, records, item_start, members, pages


def test_one_group_per_plane_prefix_and_split_length():
    # Planes 0 and 1 of a LAST-EXITED pool each have their own prefix pages;
    # rows 0, 2 read plane 0's, rows 1, 4 plane 1's (row 4 at 512-token splits),
    # row 3 has no prefix, row 5 a prefix shorter than one split.
    p0, p1 = list(range(100, 140)), list(range(200, 240))  # 40 pages = 640 tokens
    row_pages = [p0, p1, p0, (), p1, p0[:10]]
    lengths = [1000, 900, 700, 500, 20000, 400]
    layout = ops.prefix_group_layout(row_pages, lengths, 16, 1)
    row_group, records, item_start, members, pages = sections(layout, 6)
    assert row_group.tolist() == [0, 1, 0, -1, 2, -1]
    # (first member, members, first page, pages, split length); pages cut to whole splits.
    assert records[0].tolist() == [0, 2, 0, 32, 256]
    assert records[1].tolist() == [2, 1, 32, 32, 256]
    # Row 4 at 512-token splits: 640 tokens hold one whole split of 512 (32 pages).
    assert records[2].tolist() == [3, 1, 64, 32, 512]
    assert members.tolist() == [0, 2, 1, 4]
    assert pages.tolist() == p0[:32] + p1[:32] + p1[:32]
    # Items: whole splits x ceil(members x G / 64).
    assert item_start.tolist() == [0, 2, 4, 5]


def test_items_cover_every_query_block_and_cap_at_63_splits():
    shared = list(range(1000, 1000 + 4096))  # 65536 tokens: 256 splits of 256 (capped at 63)
    row_pages = [shared] * 70
    layout = ops.prefix_group_layout(row_pages, [16000] * 70, 16, 1)
    _, records, item_start, members, _ = sections(layout, 70)
    # 16000 tokens use 256-token splits: 4096 pages hold 256 of them; the pass takes at most 63.
    assert records[0, 4] == 256 and item_start[-1] == 63 * 2  # 70 queries: two 64-query blocks
    layout8 = ops.prefix_group_layout(row_pages, [16000] * 70, 16, 8)
    assert sections(layout8, 70)[2][-1] == 63 * 9  # 560 queries: nine blocks
    assert members.tolist() == list(range(70))


def test_the_layout_depends_on_the_rows_alone():
    # The same rows in another batch order give the same groups, relabelled.
    p = list(range(50, 90))
    rows = [(p, 1000), ((), 300), (p, 600), (list(range(7, 47)), 800)]
    a = ops.prefix_group_layout([r[0] for r in rows], [r[1] for r in rows], 16, 1)
    b = ops.prefix_group_layout([r[0] for r in rows[::-1]], [r[1] for r in rows[::-1]], 16, 1)
    ga, ra, _, _, pa = sections(a, 4)
    gb, rb, _, _, pb = sections(b, 4)
    for i in range(4):
        j = 3 - i
        if ga[i] < 0:
            assert gb[j] < 0
            continue
        ia, ib = ra[ga[i]], rb[gb[j]]
        assert pa[ia[2] : ia[2] + ia[3]].tolist() == pb[ib[2] : ib[2] + ib[3]].tolist()
        assert ia[4] == ib[4]


def test_no_groups_without_a_whole_split_of_shared_pages():
    assert ops.prefix_group_layout([(), ()], [100, 200], 16, 1) is None
    assert ops.prefix_group_layout([list(range(10))], [1000], 16, 1) is None  # 160 tokens < 256
    assert ops.prefix_group_layout([list(range(20))], [0], 16, 1) is None  # empty row
    with pytest.raises(ValueError, match="one length per row"):
        ops.prefix_group_layout([()], [1, 2], 16, 1)


def test_rows_join_a_group_by_its_first_and_last_page_and_count():
    # Grouping costs O(1) per row: a row whose pages agree with the group's at
    # the ends joins it (the device compares every page before taking a split,
    # so a differing middle page only sends that split to the split pass).
    a = list(range(100, 140))
    b = a[:10] + [999] + a[11:]
    c = a[:31] + [7] + a[32:]  # differs at the last page of the 32-page cut
    layout = ops.prefix_group_layout([a, b, c], [1000, 1000, 1000], 16, 1)
    row_group, records, _, members, pages = sections(layout, 3)
    assert row_group.tolist() == [0, 0, 1]
    assert pages[:32].tolist() == a[:32]  # the first member's list
    assert members.tolist() == [0, 1, 2]
