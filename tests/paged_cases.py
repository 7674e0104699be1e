"""Seeded synthetic paged-KV layouts shared by the CPU and GPU tests."""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class DecodeCase:
    q: torch.Tensor  # [rows, hq, d]
    key_pool: torch.Tensor  # [blocks, layers, page, hkv, d]
    value_pool: torch.Tensor
    layer: int
    tables: torch.Tensor  # int32 [rows, width], padded with `pad`
    lengths: torch.Tensor  # int32 [rows]

    @property
    def key_slice(self):
        return self.key_pool[:, self.layer]

    @property
    def value_slice(self):
        return self.value_pool[:, self.layer]

    def to(self, device):
        return DecodeCase(
            self.q.to(device),
            self.key_pool.to(device),
            self.value_pool.to(device),
            self.layer,
            self.tables.to(device),
            self.lengths.to(device),
        )


def random_decode_case(
    lengths,
    *,
    hq=16,
    hkv=16,
    d=128,
    page=16,
    layers=2,
    layer=1,
    dtype=torch.bfloat16,
    seed=0,
    spare_blocks=3,
    pad=-1,
    scale=1.0,
    fill_unused=float("nan"),
) -> DecodeCase:
    """Rows with independent random page permutations; unused pool slots hold `fill_unused`."""
    g = torch.Generator().manual_seed(seed)
    lengths = [int(x) for x in lengths]
    pages = [(n + page - 1) // page for n in lengths]
    width = max(pages + [1])
    blocks = sum(pages) + spare_blocks
    perm = torch.randperm(blocks, generator=g)
    key_pool = torch.randn((blocks, layers, page, hkv, d), generator=g) * scale
    value_pool = torch.randn((blocks, layers, page, hkv, d), generator=g)
    tables = torch.full((len(lengths), width), pad, dtype=torch.int32)
    live = torch.zeros(blocks, page, dtype=torch.bool)
    used = 0
    for row, (n, p) in enumerate(zip(lengths, pages)):
        ids = perm[used : used + p]
        used += p
        tables[row, :p] = ids.to(torch.int32)
        if p:
            live[ids[:-1]] = True
            live[ids[-1], : n - (p - 1) * page] = True
    # Slots no row owns (page tails, spare blocks) hold a poison value so a
    # kernel that reads them produces a visibly wrong answer.
    key_pool.transpose(1, 2)[~live] = fill_unused
    value_pool.transpose(1, 2)[~live] = fill_unused
    q = torch.randn(len(lengths), hq, d, generator=g) * scale
    return DecodeCase(
        q.to(dtype),
        key_pool.to(dtype),
        value_pool.to(dtype),
        layer,
        tables,
        torch.tensor(lengths, dtype=torch.int32),
    )
