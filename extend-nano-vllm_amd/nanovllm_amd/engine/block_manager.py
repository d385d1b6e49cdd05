"""KV-cache page accounting with a prefix cache.

Behaviour follows nanovllm/engine/block_manager.py:8-205.  Its observable
state is pinned step by step by traces of the reference's own classes
(tests/golden/scheduler_traces.json): the free list's order, reference
counts, page keys and the key index.  The attribute names the traces read
(``blocks``, ``free_block_ids``, ``used_block_ids``, ``hash_to_block_id``,
``stats`` and the per-page fields) are kept for that reason.

Model:
  * a *page* is one physical block of ``block_size`` token slots;
  * the *pool* hands out pages from the head of an ordered free list and
    takes released pages back at its tail; a page's reference count is the
    number of block tables holding it;
  * a full page gets a *key*: xxhash64 chained over the previous page's key
    (8 little-endian bytes) and its token ids (int64).  Once its K/V are
    computed (``ready``) the key is *published* in the prefix index, and a
    new sequence whose leading pages have the same keys and tokens reuses
    them.  A released page keeps its key and content until the pool hands
    it out again, so it can still be reused meanwhile.
  * speculative decoding reserves pages for every draft position before the
    draft writes K/V (``ensure_num_blocks_for_length``) and releases the
    pages past the accepted length afterwards (``truncate``): the logical
    rollback that the device-side rollback kernel mirrors.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import numpy as np
import xxhash

from nanovllm_amd.engine.sequence import Sequence

NO_KEY = -1


def page_key(token_ids: list[int], prev_key: int = NO_KEY) -> int:
    """xxhash64 of [prev_key as 8 little-endian bytes] + token ids as int64
    (the prefix-cache key format, shared with the reference)."""
    h = xxhash.xxh64()
    if prev_key != NO_KEY:
        h.update(prev_key.to_bytes(8, "little"))
    h.update(np.asarray(token_ids, dtype=np.int64).tobytes())
    return h.intdigest()


@dataclass(slots=True)
class Page:
    block_id: int
    ref_count: int = 0
    hash: int = NO_KEY                     # the page key, once full
    token_ids: list = field(default_factory=list)
    ready: bool = False                    # K/V computed: reusable through the index


class BlockManager:

    compute_hash = staticmethod(page_key)

    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = True):
        self.block_size = block_size
        self.enable_prefix_caching = enable_prefix_caching
        self.blocks = [Page(i) for i in range(num_blocks)]
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        self.hash_to_block_id: dict[int, int] = {}
        self.stats = dict.fromkeys(("prefix_cache_hits", "prefix_cache_misses",
                                    "reused_tokens"), 0)

    # ------------------------------------------------------------ pool

    def _new_page(self, block_id: int | None = None) -> Page:
        """The head of the free list (or the free page ``block_id``), emptied,
        with one reference.  Its old key stops pointing at it."""
        if block_id is None:
            page = self.blocks[self.free_block_ids.popleft()]
        else:
            self.free_block_ids.remove(block_id)
            page = self.blocks[block_id]
        assert page.ref_count == 0
        if page.hash != NO_KEY and self.hash_to_block_id.get(page.hash) == page.block_id:
            del self.hash_to_block_id[page.hash]
        page.ref_count, page.hash, page.token_ids, page.ready = 1, NO_KEY, [], False
        self.used_block_ids.add(page.block_id)
        return page

    def _share(self, page: Page) -> None:
        """One more table holds a cached page (taken off the free list if it
        was released, content kept)."""
        if page.block_id in self.used_block_ids:
            page.ref_count += 1
            return
        self.free_block_ids.remove(page.block_id)
        self.used_block_ids.add(page.block_id)
        page.ref_count = 1

    def _release(self, block_ids: list[int]) -> None:
        """Drop one reference to each page, last page first; pages left with
        none go to the tail of the free list."""
        for block_id in reversed(block_ids):
            page = self.blocks[block_id]
            page.ref_count -= 1
            if page.ref_count == 0:
                self.used_block_ids.remove(block_id)
                self.free_block_ids.append(block_id)

    # ------------------------------------------------------------ keys

    def _publish(self, page: Page) -> None:
        if self.enable_prefix_caching and page.ready:
            self.hash_to_block_id[page.hash] = page.block_id

    def _seal(self, seq: Sequence, index: int) -> None:
        """Give page ``index`` of ``seq`` its key, chained on the previous
        page's key."""
        page = self.blocks[seq.block_table[index]]
        prev = self.blocks[seq.block_table[index - 1]].hash if index else NO_KEY
        page.token_ids = seq.page_tokens(index)
        page.hash = page_key(page.token_ids, prev)

    def _cached_prefix(self, pages: list[tuple[int, list[int]]]) -> int:
        """Number of leading (key, tokens) pages of a new sequence that ready
        cached pages hold exactly."""
        if not self.enable_prefix_caching:
            return 0
        n = 0
        for key, tokens in pages:
            block_id = self.hash_to_block_id.get(key) if key != NO_KEY else None
            page = self.blocks[block_id] if block_id is not None else None
            if page is None or not page.ready or page.hash != key or page.token_ids != tokens:
                break
            n += 1
        return n

    # ------------------------------------------------------------ prefill

    def can_allocate(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= seq.num_blocks

    def allocate(self, seq: Sequence) -> None:
        """Lay out a new sequence's block table: the longest run of leading
        pages found in the prefix index is shared, every later page is new.
        At least the last prompt token stays uncomputed (its logits are
        needed), even when every page was cached."""
        assert not seq.block_table
        pages, key = [], NO_KEY
        for i in range(seq.num_blocks):
            tokens = seq.page_tokens(i)
            key = page_key(tokens, key) if len(tokens) == self.block_size else NO_KEY
            pages.append((key, tokens))
        hits = self._cached_prefix(pages)
        for i, (key, tokens) in enumerate(pages):
            if i < hits:
                page = self.blocks[self.hash_to_block_id[key]]
                self._share(page)
            else:
                page = self._new_page()
                if key != NO_KEY:
                    self.stats["prefix_cache_misses"] += 1
                    page.hash, page.token_ids = key, tokens
            seq.block_table.append(page.block_id)
        self.stats["prefix_cache_hits"] += hits
        self.stats["reused_tokens"] += hits * self.block_size
        seq.num_cached_tokens += hits * self.block_size
        seq.num_computed_tokens = min(seq.num_cached_tokens, max(len(seq) - 1, 0))

    def mark_computed(self, seq: Sequence) -> None:
        """Pages wholly covered by computed tokens become ready (keyed first
        if they are not yet) and are published."""
        full = min(seq.num_computed_tokens // self.block_size, len(seq.block_table))
        for index in range(full):
            page = self.blocks[seq.block_table[index]]
            if page.ready:
                continue
            if page.hash == NO_KEY:
                self._seal(seq, index)
            page.ready = True
            self._publish(page)

    def deallocate(self, seq: Sequence) -> None:
        self._release(seq.block_table)
        seq.block_table.clear()
        seq.num_cached_tokens = seq.num_computed_tokens = seq.num_scheduled_tokens = 0

    # ------------------------------------------------------------ decode

    def can_append(self, seq: Sequence) -> bool:
        """Room for the token just appended: a length of k*block_size + 1
        opens a page."""
        opens_page = len(seq) % self.block_size == 1
        return len(self.free_block_ids) >= int(opens_page)

    def may_append(self, seq: Sequence) -> None:
        """Keep the table in step with a sequence that just grew by one token.
        Both cases are idempotent, because speculation may have reserved the
        next page or sealed the last one already:
          length % block_size == 1: the new token opens a page;
          length % block_size == 0: the last page is full and gets its key."""
        last = self.blocks[seq.block_table[-1]]
        offset = len(seq) % self.block_size
        if offset == 1:
            if len(seq.block_table) < seq.num_blocks:
                assert last.hash != NO_KEY
                seq.block_table.append(self._new_page().block_id)
        elif offset == 0:
            if last.hash == NO_KEY:
                table = seq.block_table
                prev = self.blocks[table[-2]].hash if len(table) > 1 else NO_KEY
                last.token_ids = seq.page_tokens(seq.num_blocks - 1)
                last.hash = page_key(last.token_ids, prev)
                self._publish(last)
        else:
            assert last.hash == NO_KEY

    # ------------------------------------------------------------ speculation

    # pages the look-ahead reservation searches at the free list's tail
    LOOKAHEAD_SCAN = 64

    def _lookahead_page_id(self) -> int | None:
        """A free page for a look-ahead reservation: the newest page without
        a key among the last LOOKAHEAD_SCAN of the free list (a truncate
        returns the rejected positions' unkeyed pages there), so keyed
        pages waiting for prefix reuse keep their place; None (the head)
        when there is none."""
        free = self.free_block_ids
        for i, block_id in enumerate(reversed(free)):
            if i == self.LOOKAHEAD_SCAN:
                break
            if self.blocks[block_id].hash == NO_KEY:
                return block_id
        return None

    def ensure_num_blocks_for_length(self, seq: Sequence, num_tokens: int,
                                     lookahead: bool = False) -> None:
        """Reserve pages for ``num_tokens`` tokens before the draft writes K/V
        for positions not yet committed.  ``lookahead`` pages (one step
        further than the reference reserves, held only until the step's
        truncate) come from the free list's tail, see _lookahead_page_id."""
        missing = -(-num_tokens // self.block_size) - len(seq.block_table)
        for _ in range(missing):
            if not self.free_block_ids:
                raise RuntimeError("not enough KV-cache blocks for speculative proposal")
            block_id = self._lookahead_page_id() if lookahead else None
            seq.block_table.append(self._new_page(block_id).block_id)

    def truncate(self, seq: Sequence) -> None:
        """Release the pages past the sequence's current length (rejected
        draft positions)."""
        keep = seq.num_blocks
        self._release(seq.block_table[keep:])
        del seq.block_table[keep:]
