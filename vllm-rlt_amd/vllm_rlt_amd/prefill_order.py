"""Prefill ordering over the depth-aware KV cache (vllm_rlt/worker/model_runner.py:247-320).

The order in which a prompt chunk's loops write and read the cache is part of
the cache's semantics, so it is mirrored here with the runner's names:

- LAST-EXITED with a backend that takes packed prefill: the prelude runs once
  over the packed chunk, then depth 0 .. loops-1 each run one recurrent pass
  over the whole chunk with that depth's packed metadata (depth-major).  A
  depth's pass writes the chunk's K/V at that depth before it attends, layer by
  layer.  The metadata comes from a rotating set of PrefillMetadataBank
  (``prefill_uva``) or from ``cache._prepare_batch(..., packed_prefill=True)``.
- Otherwise every token is a decode row (length position + 1): the same
  depth-major passes over per-token metadata (``_prepare_batch`` without packing).
- SHARED: positions advance one at a time.  All loops of position p of every
  active request run before position p + 1, so a prompt's result does not
  depend on how it was cut into chunks (:248-259).

The model is the caller's: ``prelude(tokens) -> hidden`` and
``core(hidden, batch, cache) -> hidden`` (or a tuple whose first element is
hidden), the reference's ``model.prelude`` and ``model.recurrent_prepared``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable, Sequence

import torch

from .prefill_metadata import PrefillMetadataBank


@dataclass(frozen=True)
class PrefillItem:
    """The fields of a scheduled prefill item that the ordering reads."""

    request_id: Any
    token_start: int
    token_count: int
    prompt_token_ids: Sequence[int]


class PrefillOrder:
    def __init__(
        self,
        cache,
        prelude: Callable,
        core: Callable,
        loops: int,
        device,
        prefill_uva: bool = True,
        banks: int = 3,
    ):
        if loops < 1:
            raise ValueError("loops must be positive")
        self.cache = cache
        self.prelude = prelude
        self.core = core
        self.loops = int(loops)
        self.device = torch.device(device)
        self.prefill_uva = bool(prefill_uva)
        self._bank_count = int(banks)
        self._banks = None
        self._bank_index = 0

    def packed(self) -> bool:
        cache = self.cache
        return cache.layout == "last_exited" and bool(getattr(cache.attention, "supports_packed_prefill", False))

    def _run_core(self, hidden, batch):
        out = self.core(hidden, batch, self.cache)
        return out[0] if isinstance(out, tuple) else out

    def prefill_tokens(self, ids, positions, tokens) -> torch.Tensor:
        """Every loop of the given token rows; returns the final hidden rows (:271-320)."""
        ids, positions, tokens = list(ids), [int(p) for p in positions], [int(t) for t in tokens]
        if not ids or len(positions) != len(ids) or len(tokens) != len(ids):
            raise ValueError("ids, positions and tokens must be non-empty and of equal length")
        cache = self.cache
        if self.packed():
            bank = None
            if self.prefill_uva:
                if self._banks is None:
                    self._banks = [PrefillMetadataBank(cache) for _ in range(self._bank_count)]
                bank = self._banks[self._bank_index]
                self._bank_index = (self._bank_index + 1) % len(self._banks)
            tensor = (
                bank.prepare(ids, positions, tokens)
                if bank
                else torch.tensor(tokens, device=self.device, dtype=torch.long)
            )
            hidden = self.prelude(tensor)
            for depth in range(self.loops):
                metadata = (
                    bank.metadata(depth)
                    if bank
                    else cache._prepare_batch(ids, [depth] * len(ids), positions, packed_prefill=True)
                )
                hidden = self._run_core(hidden, metadata)
            if bank:
                bank.release()
            return hidden
        hidden = self.prelude(torch.tensor(tokens, device=self.device, dtype=torch.long))
        for depth in range(self.loops):
            hidden = self._run_core(hidden, cache._prepare_batch(ids, [depth] * len(ids), positions))
        return hidden

    def prefill(self, items: Sequence[PrefillItem]) -> list:
        """One scheduled prefill batch; returns each item's last hidden row, what the runner saves (:247-269)."""
        items = list(items)
        if not items:
            return []
        saved: list = [None] * len(items)
        if self.cache.layout == "shared":
            for offset in range(max(item.token_count for item in items)):
                active = [i for i, item in enumerate(items) if offset < item.token_count]
                ids = [items[i].request_id for i in active]
                positions = [items[i].token_start + offset for i in active]
                tokens = [items[i].prompt_token_ids[p] for i, p in zip(active, positions)]
                hidden = self.prefill_tokens(ids, positions, tokens)
                for row, i in enumerate(active):
                    saved[i] = hidden[row]
            return saved
        ids, positions, tokens = [], [], []
        for item in items:
            start, count = item.token_start, item.token_count
            ids.extend([item.request_id] * count)
            positions.extend(range(start, start + count))
            tokens.extend(item.prompt_token_ids[start : start + count])
        hidden = self.prefill_tokens(ids, positions, tokens)
        end = 0
        for i, item in enumerate(items):
            end += item.token_count
            saved[i] = hidden[end - 1]
        return saved
