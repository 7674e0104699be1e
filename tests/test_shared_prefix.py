"""Host side of the shared-prefix decode hint (CPU only)."""

import numpy as np
import pytest
import torch

from vllm_rlt_amd import ops


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


def test_hint_lists_members_and_takes_the_common_split_length():
    hint = ops.shared_prefix([4, 1, 2], [7, 8, 9], 6, [20000, 17000, 9000], "cpu")
    assert hint.member.tolist() == [0, 1, 1, 0, 1, 0]
    assert hint.rows.tolist() == [4, 1, 2]
    assert hint.table.tolist() == [7, 8, 9]
    assert hint.split_len == 512
    assert hint.member.dtype == hint.rows.dtype == hint.table.dtype == torch.int32


def test_hint_rows_must_be_distinct_batch_rows():
    with pytest.raises(ValueError, match="distinct batch rows"):
        ops.shared_prefix([], [1], 4, [], "cpu")
    with pytest.raises(ValueError, match="distinct batch rows"):
        ops.shared_prefix([1, 1], [1], 4, [5, 5], "cpu")
    with pytest.raises(ValueError, match="distinct batch rows"):
        ops.shared_prefix([-1], [1], 4, [5], "cpu")


def table_rows(prefix, owns, width):
    rows = []
    for own in owns:
        row = list(prefix) + list(own)
        rows.append(row + [-1] * (width - len(row)))
    return np.array(rows, dtype=np.int32)


def test_detector_finds_the_largest_group_and_its_common_pages():
    shared = list(range(100, 120))  # 20 pages = 320 tokens >= one 256-token split
    tables = np.concatenate(
        [
            table_rows(shared, [[1, 2], [3], [4, 5, 6]], 24),
            table_rows([7, 8], [[9]], 24),  # a row of its own
            table_rows(shared[:5], [[10]], 24),  # shares only 5 pages (80 tokens, no whole split)
        ]
    )
    lengths = np.array([350, 330, 360, 40, 90])
    rows, pages, split_len = ops.find_shared_prefix(tables, lengths, 16)
    assert rows == [0, 1, 2] and pages == shared and split_len == 256


def test_detector_stops_at_padding_and_needs_a_whole_split():
    shared = list(range(50, 70))
    tables = table_rows(shared, [[], []], 30)  # both rows end with the prefix, then -1 padding
    rows, pages, split_len = ops.find_shared_prefix(tables, np.array([320, 300]), 16)
    assert rows == [0, 1] and pages == shared and split_len == 256
    assert ops.find_shared_prefix(table_rows(shared[:10], [[1], [2]], 12), np.array([170, 170]), 16) is None


def test_detector_ignores_empty_rows_and_unshared_batches():
    assert ops.find_shared_prefix(table_rows([], [[1, 2], [3, 4]], 2), np.array([20, 20]), 16) is None
    shared = list(range(20))
    tables = table_rows(shared, [[], []], 20)
    assert ops.find_shared_prefix(tables, np.array([320, 0]), 16) is None  # one live member
    assert ops.find_shared_prefix(tables[:1], np.array([320]), 16) is None
