"""Host side of the shared-prefix decode hint (CPU only)."""

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
