"""Prefill ordering through KVCacheManager(backend="hip") on the GPU (worker/model_runner.py:247-320).

A toy looped model drives the cache: an embedding prelude and a core whose
per-layer projections are elementwise, so a row's arithmetic never depends on
which other rows share its batch.  The checks are properties of the ordering:
the pinned metadata bank and the manager's packed batch give the same bits, the
packed MFMA prefill agrees with per-token decode rows, and SHARED prefill does
not depend on how a prompt is cut into chunks.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
LAYERS, HEADS, D, LOOPS, VOCAB = 2, 2, 64, 3, 50


class ToyModel:
    def __init__(self, dtype, seed=3):
        g = torch.Generator().manual_seed(seed)

        def rand(*shape, s=1.0):
            return (torch.randn(*shape, generator=g) * s).to(DEV, dtype)

        self.embed = rand(VOCAB, HEADS, D)
        self.wq, self.wk, self.wv = rand(LAYERS, HEADS, D), rand(LAYERS, HEADS, D), rand(LAYERS, HEADS, D)
        self.wo = rand(LAYERS, HEADS, D, s=0.25)

    def prelude(self, tokens):
        return self.embed[tokens]

    def core(self, hidden, batch, cache):
        for layer in range(LAYERS):
            q = hidden * self.wq[layer]
            k = torch.tanh(hidden * self.wk[layer])
            v = hidden * self.wv[layer]
            cache._write_prepared(layer, batch, k, v)
            hidden = hidden + cache._attend_prepared(layer, batch, q) * self.wo[layer]
        return hidden, None


def manager(layout, dtype):
    from vllm_rlt_amd import KVCacheManager

    return KVCacheManager(
        LAYERS, HEADS, D, 96, 16, LOOPS, device=DEV, dtype=dtype, backend="hip", layout=layout
    )


def prompts():
    g = torch.Generator().manual_seed(11)
    return {rid: torch.randint(0, VOCAB, (n,), generator=g).tolist() for rid, n in [("a", 45), ("b", 20), ("c", 33)]}


def run(layout, dtype, chunks, prefill_uva=True, packed=None):
    """Prefill every prompt in the given chunks: a list of batches of (request, start, count)."""
    from vllm_rlt_amd import PrefillItem, PrefillOrder

    cache = manager(layout, dtype)
    cache.key_cache.zero_()  # pools start uninitialised; page tails are compared below
    cache.value_cache.zero_()
    tokens = prompts()
    for rid, toks in tokens.items():
        cache.allocate(rid, len(toks))
    model = ToyModel(dtype)
    order = PrefillOrder(cache, model.prelude, model.core, LOOPS, DEV, prefill_uva=prefill_uva)
    if packed is not None:
        order.packed = lambda: packed
    last = {}
    for batch in chunks:
        items = [PrefillItem(rid, start, count, tokens[rid]) for rid, start, count in batch]
        for (rid, _, _), hidden in zip(batch, order.prefill(items)):
            last[rid] = hidden.clone()
    torch.cuda.synchronize()
    return cache, last


WHOLE = [[("a", 0, 45), ("b", 0, 20), ("c", 0, 33)]]
CHUNKED = [[("a", 0, 17), ("b", 0, 20), ("c", 0, 5)], [("a", 17, 28), ("c", 5, 28)]]


def used_pages(cache):
    return sorted({b for rid in "abc" for plane in cache._allocations[rid].block_tables for b in plane})


def test_bank_and_manager_metadata_give_the_same_bits():
    bank_cache, bank = run("last_exited", torch.bfloat16, CHUNKED, prefill_uva=True)
    flat_cache, flat = run("last_exited", torch.bfloat16, CHUNKED, prefill_uva=False)
    for rid in "abc":
        assert torch.equal(bank[rid], flat[rid])
    pages = used_pages(bank_cache)
    assert pages == used_pages(flat_cache)
    assert torch.equal(bank_cache.key_cache[pages], flat_cache.key_cache[pages])
    assert torch.equal(bank_cache.value_cache[pages], flat_cache.value_cache[pages])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_packed_prefill_agrees_with_per_token_rows(dtype):
    _, packed = run("last_exited", dtype, WHOLE, packed=True)
    _, rows = run("last_exited", dtype, WHOLE, packed=False)
    # Six attention steps (2 layers x 3 loops) compose; per step the kernels agree to
    # the attention tolerance, so the final rows get a few activation ULPs of slack.
    tol = 5e-2 if dtype == torch.bfloat16 else 1e-2
    embed = ToyModel(dtype).embed
    for rid in "abc":
        assert torch.isfinite(packed[rid].float()).all()
        # The loops move the row away from its embedding: attention is not vacuous here.
        assert (packed[rid].float() - embed[prompts()[rid][-1]].float()).abs().max() > 0.1
        torch.testing.assert_close(packed[rid].float(), rows[rid].float(), atol=tol, rtol=tol)


def test_last_exited_chunks_agree_with_one_pass():
    _, whole = run("last_exited", torch.float16, WHOLE)
    _, chunked = run("last_exited", torch.float16, CHUNKED)
    for rid in "abc":
        torch.testing.assert_close(chunked[rid].float(), whole[rid].float(), atol=1e-2, rtol=1e-2)


def test_shared_prefill_does_not_depend_on_the_chunking():
    whole_cache, whole = run("shared", torch.bfloat16, WHOLE)
    chunked_cache, chunked = run("shared", torch.bfloat16, CHUNKED)
    for rid in "abc":
        assert torch.equal(chunked[rid], whole[rid])
    pages = used_pages(whole_cache)
    assert pages == used_pages(chunked_cache)
    assert torch.equal(whole_cache.key_cache[pages], chunked_cache.key_cache[pages])
    assert torch.equal(whole_cache.value_cache[pages], chunked_cache.value_cache[pages])
