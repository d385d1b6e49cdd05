"""Paged KV-cache block accounting with prefix caching
(nanovllm/engine/block_manager.py:8-205).

Blocks hold ``block_size`` tokens.  A full block is identified by a chained
xxhash64 of (previous block hash, its token ids) so identical prefixes can
share physical blocks (reference-counted).  Speculative decoding adds
``ensure_num_blocks_for_length`` (reserve draft positions before the draft
writes K/V) and ``truncate`` (free the tail after rejection) -- the logical
rollback that the device-side rollback kernel mirrors.
"""
from collections import deque

import numpy as np
import xxhash

from nanovllm_amd.engine.sequence import Sequence


class Block:

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1
        self.token_ids: list[int] = []
        self.ready = False

    def update(self, h: int, token_ids: list[int]) -> None:
        self.hash = h
        self.token_ids = token_ids

    def reset(self) -> None:
        self.ref_count = 1
        self.hash = -1
        self.token_ids = []
        self.ready = False


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = True):
        self.block_size = block_size
        self.enable_prefix_caching = enable_prefix_caching
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        self.stats = {"prefix_cache_hits": 0, "prefix_cache_misses": 0, "reused_tokens": 0}

    @classmethod
    def compute_hash(cls, token_ids: list[int], prefix: int = -1) -> int:
        """xxhash64 over the 8-byte little-endian prefix hash (when chained)
        followed by the token ids as a native int64 array."""
        h = xxhash.xxh64()
        if prefix != -1:
            h.update(prefix.to_bytes(8, "little"))
        h.update(np.array(token_ids).tobytes())
        return h.intdigest()

    # ------------------------------------------------------------ internals

    def _take(self, block_id: int) -> Block:
        """Move a free block to the used set with a fresh single reference."""
        block = self.blocks[block_id]
        assert block.ref_count == 0
        if block.hash != -1 and self.hash_to_block_id.get(block.hash) == block_id:
            del self.hash_to_block_id[block.hash]
        block.reset()
        self.free_block_ids.remove(block_id)
        self.used_block_ids.add(block_id)
        return block

    def _release(self, block_id: int) -> None:
        assert self.blocks[block_id].ref_count == 0
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)

    def _drop_ref(self, block_id: int) -> None:
        block = self.blocks[block_id]
        block.ref_count -= 1
        if block.ref_count == 0:
            self._release(block_id)

    def _cached_block(self, h: int, token_ids: list[int]) -> int:
        """Physical id of a ready block holding exactly these tokens, else -1."""
        if not self.enable_prefix_caching or h == -1:
            return -1
        block_id = self.hash_to_block_id.get(h, -1)
        if block_id == -1:
            return -1
        block = self.blocks[block_id]
        if not block.ready or block.hash != h or block.token_ids != token_ids:
            return -1
        return block_id

    # ------------------------------------------------------------ prefill

    def can_allocate(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= seq.num_blocks

    def allocate(self, seq: Sequence) -> None:
        """Give a new sequence its block table, reusing cached prefix blocks
        until the first miss."""
        assert not seq.block_table
        h = -1
        missed = False
        for i in range(seq.num_blocks):
            token_ids = seq.block(i)
            full = len(token_ids) == self.block_size
            h = self.compute_hash(token_ids, h) if full else -1
            block_id = -1 if missed else self._cached_block(h, token_ids)
            if block_id == -1:
                missed = True
                if h != -1:
                    self.stats["prefix_cache_misses"] += 1
                block_id = self.free_block_ids[0]
                block = self._take(block_id)
            else:
                seq.num_cached_tokens += self.block_size
                self.stats["prefix_cache_hits"] += 1
                self.stats["reused_tokens"] += self.block_size
                block = self.blocks[block_id]
                if block_id in self.used_block_ids:
                    block.ref_count += 1
                else:
                    self.free_block_ids.remove(block_id)
                    self.used_block_ids.add(block_id)
                    block.ref_count = 1
            if h != -1:
                block.update(h, token_ids)
                if self.enable_prefix_caching and block.ready:
                    self.hash_to_block_id[h] = block_id
            seq.block_table.append(block_id)
        # at least the last prompt token is recomputed to produce logits
        seq.num_computed_tokens = min(seq.num_cached_tokens, max(seq.num_tokens - 1, 0))

    def mark_computed(self, seq: Sequence) -> None:
        """Blocks fully covered by computed tokens become reusable."""
        full = min(seq.num_computed_tokens // self.block_size, len(seq.block_table))
        for index in range(full):
            block = self.blocks[seq.block_table[index]]
            if block.ready:
                continue
            if block.hash == -1:
                prefix = self.blocks[seq.block_table[index - 1]].hash if index > 0 else -1
                token_ids = seq.block(index)
                block.update(self.compute_hash(token_ids, prefix), token_ids)
            block.ready = True
            if self.enable_prefix_caching:
                self.hash_to_block_id[block.hash] = block.block_id

    def deallocate(self, seq: Sequence) -> None:
        for block_id in reversed(seq.block_table):
            self._drop_ref(block_id)
        seq.num_cached_tokens = 0
        seq.num_computed_tokens = 0
        seq.num_scheduled_tokens = 0
        seq.block_table.clear()

    # ------------------------------------------------------------ decode

    def can_append(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= (len(seq) % self.block_size == 1)

    def may_append(self, seq: Sequence) -> None:
        """Keep the block table consistent after one token was appended.

        A length of k*block_size + 1 needs a new block (unless speculation
        already reserved it); a length of k*block_size finalises (hashes) the
        last block unless that already happened."""
        table = seq.block_table
        last = self.blocks[table[-1]]
        rem = len(seq) % self.block_size
        if rem == 1:
            if len(table) >= seq.num_blocks:
                return
            assert last.hash != -1
            block = self._take(self.free_block_ids[0])
            table.append(block.block_id)
        elif rem == 0:
            if last.hash != -1:
                return
            token_ids = seq.block(seq.num_blocks - 1)
            prefix = self.blocks[table[-2]].hash if len(table) > 1 else -1
            h = self.compute_hash(token_ids, prefix)
            last.update(h, token_ids)
            if self.enable_prefix_caching and last.ready:
                self.hash_to_block_id[h] = last.block_id
        else:
            assert last.hash == -1

    # ------------------------------------------------------------ speculation

    def ensure_num_blocks_for_length(self, seq: Sequence, num_tokens: int) -> None:
        """Reserve blocks for ``num_tokens`` tokens before draft K/V is written."""
        need = -(-num_tokens // self.block_size)
        while len(seq.block_table) < need:
            if not self.free_block_ids:
                raise RuntimeError("not enough KV-cache blocks for speculative proposal")
            seq.block_table.append(self._take(self.free_block_ids[0]).block_id)

    def truncate(self, seq: Sequence) -> None:
        """Release blocks beyond the sequence's current length."""
        keep = seq.num_blocks
        for block_id in reversed(seq.block_table[keep:]):
            self._drop_ref(block_id)
        del seq.block_table[keep:]
