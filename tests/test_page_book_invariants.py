"""Allocator and prefix-cache invariants over random operation sequences (CPU only).

The golden trace pins the page ids of one scripted sequence; these checks hold
after every step of many seeded random sequences (admissions with and without
prefix hits, partial writes, immediate and deferred publication, growth,
transfer leases, frees and evictions under pressure):

- every page's hold count equals the number of request tables plus prefix
  entries that list it (kv_cache_manager.py:175-192, 231-236, 278-281);
- the free stack holds exactly the unheld pages, each once;
- num_free_blocks counts free pages plus cached pages only the cache holds
  (kv_cache_manager.py:149-153);
- an entry holds, page for page, what a publisher's tables held at that
  index when it was published, and it never changes while it is cached;
- a prefix hit returns exactly the cached entries, and the new request's
  tables begin with them, plane by plane;
- entries leave the cache least recently used first, where a hit counts as a
  use (kv_cache_manager.py:182-186, 240-251).
"""

import random
from collections import Counter

import pytest

from vllm_rlt_amd.page_book import KVPageBook


class Event:
    """A completion event that fires after a seeded number of queries."""

    def __init__(self, polls):
        self.polls = polls

    def query(self):
        self.polls -= 1
        return self.polls < 0


def check(book, published):
    holds = Counter()
    for allocation in book._allocations.values():
        for table in allocation.block_tables:
            holds.update(table)
    for pages in book._prefixes.values():
        holds.update(pages)
    assert [book._refs[b] for b in range(book.num_blocks)] == [holds[b] for b in range(book.num_blocks)]
    free = list(book._free_blocks)
    assert len(free) == len(set(free))
    assert set(free) == {b for b in range(book.num_blocks) if book._refs[b] == 0}
    cached_only = sum(1 for pages in book._prefixes.values() for b in pages if book._refs[b] == 1)
    assert book.num_free_blocks == len(free) + cached_only
    for allocation in book._allocations.values():
        assert len({len(t) for t in allocation.block_tables}) == 1
        assert len(allocation.block_tables) == book.storage_depths
    # Every cached entry still names the pages it was published with.
    for key, pages in book._prefixes.items():
        assert published[key] == pages


def record_new_entries(book, before, publishers, published):
    """Note the pages of every index entry that appeared during an operation.

    publishers: (allocation, tokens) of the immediate publication and of every
    deferred one that could have fired (lookup_prefix polls them too).
    """
    page = book.block_size
    for key in book._prefixes.keys() - before.keys():
        # Only pages every plane and layer of the publisher has written may be published.
        found = {tuple(t[i] for t in a.block_tables) for a, tokens in publishers
                 for i, k in enumerate(book._index.keys(tokens))
                 if k == key and min(w.prefix for plane in a.written for w in plane) >= (i + 1) * page}
        assert book._prefixes[key] in found, "an index entry no fully written publisher's table holds"
        published[key] = book._prefixes[key]


def reconcile(book, order):
    """Check the index's recency order against the model, oldest first.

    Entries that left the index since the model was updated must be the
    oldest (eviction takes the least recently used first); new entries join
    at the recent end in the order they were inserted.
    """
    gone = [k for k in order if k not in book._prefixes]
    assert order[: len(gone)] == gone, "eviction skipped a less recently used entry"
    kept = order[len(gone):]
    kept += [k for k in book._prefixes if k not in set(kept)]
    assert list(book._prefixes) == kept
    order[:] = kept


def run(seed):
    rng = random.Random(seed)
    page = rng.choice([1, 2, 4])
    book = KVPageBook(rng.choice([1, 2]), 1, 4, rng.randint(6, 40), page, rng.choice([1, 2, 3]),
                      enable_prefix_caching=True)
    vocab = rng.choice([2, 3, 40])
    prompts, published, order = {}, {}, []
    for step in range(150):
        live = sorted(book._allocations)
        op = rng.random()
        before = dict(book._prefixes)
        publishers = [(item.allocation, item.tokens) for item in book._deferred]
        if op < 0.3:
            rid = f"r{rng.randint(0, 10)}"
            n = rng.randint(1, 12 * page)
            tokens = [rng.randint(0, vocab) for _ in range(n)]
            frontier = rng.randint(1, n)
            if rng.random() < 0.7:
                hit = book.lookup_prefix(tokens)
                record_new_entries(book, before, publishers, published)  # the lookup may have polled
                # A hit is the longest cached run of the prompt's pages (its last token excluded),
                # and every entry of it becomes the most recently used, in order.
                # Entries the lookup's poll inserted came before its touches.
                order += [k for k in book._prefixes if k not in set(order)]
                keys = list(book._index.keys(tokens[:-1]))
                run = 0
                while run < len(keys) and keys[run] in published and keys[run] in book._prefixes:
                    run += 1
                assert len(hit) == run
                for key, pages in zip(keys, hit):
                    assert published[key] == pages
                    order.remove(key) if key in order else None
                    order.append(key)
                reconcile(book, order)
            else:
                hit = ()
            hit = hit[: -(-frontier // page)]
            try:
                admitted = book.allocate(rid, n, initial_tokens=frontier, prefix=hit)
            except ValueError:
                admitted = False
            if admitted:
                prompts[rid] = tokens
                tables = book._allocations[rid].block_tables
                assert all(table[: len(hit)] == tuple(p[d] for p in hit) for d, table in enumerate(tables))
        elif op < 0.45 and live:
            book.free(rng.choice(live))
        elif op < 0.6 and live:
            # Writes only land on allocated pages (the manager addresses them through the tables).
            allocation = book._allocations[rng.choice(live)]
            upto = rng.randint(0, len(allocation.block_tables[0]) * page)
            for plane in allocation.written:
                for w in plane:
                    for p in range(upto):
                        if rng.random() < 0.95:
                            w.add(p)
        elif op < 0.75 and live:
            rid = rng.choice(live)
            tokens = prompts.get(rid, [])
            publishers.append((book._allocations[rid], tokens))
            event = Event(rng.randint(0, 3)) if rng.random() < 0.3 else None
            book.publish_prefix(rid, tokens, rng.randint(0, len(tokens) + 1), event)
        elif op < 0.85 and live:
            rid = rng.choice(live)
            book.ensure_capacity(rid, rng.randint(1, book._allocations[rid].max_tokens))
        elif op < 0.9:
            book.poll_prefixes()
        elif live:
            rid = rng.choice(live)
            if rng.random() < 0.5:
                if book._allocations[rid].release_requested:
                    with pytest.raises(RuntimeError, match="scheduled for release"):
                        book.pin_transfer(rid, "t")
                else:
                    book.pin_transfer(rid, "t")
            else:
                book.unpin_transfer(rid, "t")
        record_new_entries(book, before, publishers, published)
        reconcile(book, order)
        check(book, published)
    # Releasing every request and evicting every prefix returns the whole pool.
    for rid in sorted(book._allocations):
        book._allocations[rid].transfer_leases.clear()
        book.free(rid)
    assert book.num_free_blocks == book.num_blocks
    while (pages := book._index.evict_oldest()) is not None:
        book._pool.release(pages)
    assert sorted(book._free_blocks) == list(range(book.num_blocks))


@pytest.mark.parametrize("seed", range(60))
def test_invariants_hold_after_every_step(seed):
    run(seed)
