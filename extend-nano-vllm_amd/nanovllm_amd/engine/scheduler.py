"""Step scheduling (prefill or decode) and the bookkeeping of a speculative
step.

Behaviour follows nanovllm/engine/scheduler.py:10-191; the traces of the
reference's own classes in tests/golden/scheduler_traces.json pin it step by
step (queues, block tables, counters, statistics and error messages).

Policy:
  * prefill goes first, but never twice in a row while sequences are
    running, so decode keeps moving; without prefill batching one request
    is admitted per step, and a long prompt is chunked by the token budget;
  * a decode step takes running sequences from the front; when one needs a
    page and none is free, sequences are preempted from the back (the
    newest first) and return to the front of the waiting queue;
  * a speculative step reserves pages for every draft position, appends the
    drafts, and afterwards keeps the accepted prefix (clipped to the token
    budget and at the first EOS) plus the replacement token.
"""
from __future__ import annotations

from collections import deque

from nanovllm_amd.engine.block_manager import BlockManager
from nanovllm_amd.engine.sequence import Sequence, SequenceStatus


class Scheduler:

    def __init__(self, config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.enable_prefill_batching = bool(getattr(config, "enable_prefill_batching", False))
        spec = getattr(config, "speculative_config", None)
        self.num_speculative_tokens = spec.num_speculative_tokens if spec is not None else 0
        self.eos = config.eos
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size,
                                          config.enable_prefix_caching)
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self.last_step_was_prefill = False
        self.stats = {"prefill_steps": 0, "max_prefill_tokens_per_step": 0}

    def is_finished(self) -> bool:
        return not (self.waiting or self.running)

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    # ------------------------------------------------------------ scheduling

    def schedule(self) -> tuple[list[Sequence], bool]:
        """(sequences, is_prefill) of the next step."""
        if self.waiting and not (self.running and self.last_step_was_prefill):
            admitted = self._admit()
            if admitted:
                self.last_step_was_prefill = True
                return admitted, True
        batch = self._decode_batch()
        self.last_step_was_prefill = False
        return batch, False

    def _admit(self) -> list[Sequence]:
        """Waiting sequences to prefill this step, in queue order, each
        given as many of its remaining tokens as the budget allows."""
        bm = self.block_manager
        budget = self.max_num_batched_tokens
        admitted: list[Sequence] = []
        for seq in self.waiting:
            full = (len(admitted) == self.max_num_seqs or budget == 0
                    or (admitted and not self.enable_prefill_batching))
            if full:
                break
            if not seq.block_table:
                if not bm.can_allocate(seq):
                    if not (self.running or admitted):
                        raise RuntimeError("not enough KV-cache blocks for request")
                    break
                bm.allocate(seq)
            seq.num_scheduled_tokens = min(len(seq) - seq.num_computed_tokens, budget)
            budget -= seq.num_scheduled_tokens
            admitted.append(seq)
        if admitted:
            used = self.max_num_batched_tokens - budget
            self.stats["prefill_steps"] += 1
            self.stats["max_prefill_tokens_per_step"] = max(
                self.stats["max_prefill_tokens_per_step"], used)
        return admitted

    def _decode_batch(self) -> list[Sequence]:
        """Running sequences for a decode step, front first, each with room
        for its next token."""
        batch: list[Sequence] = []
        while self.running and len(batch) < self.max_num_seqs:
            seq = self.running.popleft()
            if self._make_room(seq):
                self.block_manager.may_append(seq)
                batch.append(seq)
        assert batch
        self.running.extendleft(reversed(batch))
        return batch

    def _make_room(self, seq: Sequence) -> bool:
        """Preempt running sequences from the back until ``seq`` can take its
        next token; preempt ``seq`` itself when none is left.  True when
        ``seq`` stays scheduled."""
        while not self.block_manager.can_append(seq):
            if not self.running:
                self.preempt(seq)
                return False
            self.preempt(self.running.pop())
        return True

    def preempt(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.WAITING
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    # ------------------------------------------------------------ results

    def _stops_at(self, seq: Sequence, token_id: int) -> bool:
        """Non-speculative stop rule: EOS (unless ignored) or the token budget."""
        return ((not seq.ignore_eos and token_id == self.eos)
                or seq.num_completion_tokens == seq.max_tokens)

    def _finish(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.FINISHED
        self.block_manager.deallocate(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        """Record one model step's sampled tokens."""
        bm = self.block_manager
        for seq, token_id in zip(seqs, token_ids):
            if is_prefill:
                seq.num_computed_tokens += seq.num_scheduled_tokens
                seq.num_scheduled_tokens = 0
            else:
                seq.num_computed_tokens = len(seq)
            bm.mark_computed(seq)
            if is_prefill:
                if not seq.is_prefill_complete:
                    continue                       # the next chunk comes later
                self.waiting.remove(seq)
                seq.status = SequenceStatus.RUNNING
            seq.append_token(token_id)
            if self._stops_at(seq, token_id):
                self._finish(seq)
                if not is_prefill:
                    self.running.remove(seq)
            elif is_prefill:
                self.running.append(seq)

    # ------------------------------------------------------------ speculation

    def reserve_speculation(self, seq: Sequence) -> None:
        """Pages for every draft position, before the draft writes their K/V
        (the token budget caps the positions)."""
        limit = min(seq.max_tokens + seq.num_prompt_tokens, len(seq) + self.num_speculative_tokens)
        self.block_manager.ensure_num_blocks_for_length(seq, limit)

    def reserve_lookahead(self, seqs: list[Sequence]) -> bool:
        """Pages one step further than reserve_speculation for every
        sequence (len + 2k tokens, within the token budget), so that the next
        step's draft can be queued before this step's results are read.
        False, with nothing reserved, when the pool is short of pages.
        postprocess_speculation releases what the step does not keep.  The
        extra pages are unkeyed ones from the free list's tail (where the
        step's truncate returns them), so the per-step churn leaves pages
        that wait for prefix reuse alone."""
        bm = self.block_manager
        k = self.num_speculative_tokens
        limits = [min(seq.max_tokens + seq.num_prompt_tokens, len(seq) + 2 * k) for seq in seqs]
        need = sum(max(-(-n // bm.block_size) - len(seq.block_table), 0)
                   for seq, n in zip(seqs, limits))
        if need > len(bm.free_block_ids):
            return False
        for seq, n in zip(seqs, limits):
            bm.ensure_num_blocks_for_length(seq, n, lookahead=True)
        return True

    def begin_speculation(self, seq: Sequence, proposal_tokens: list[int]) -> int:
        """Append the drafts (their pages are reserved) and return the length
        before them, ``base``."""
        if seq not in self.running:
            raise RuntimeError("speculative decode requires a running sequence")
        base = len(seq)
        seq.token_ids.extend(proposal_tokens)
        return base

    def postprocess_speculation(self, seq: Sequence, base_num_tokens: int,
                                accepted_tokens: list[int],
                                replacement_token: int | None) -> int:
        """Keep ``base`` tokens, the accepted drafts and the replacement.
        Returns the number of drafts kept."""
        kept, replacement_token = self._settle(seq, base_num_tokens, accepted_tokens,
                                               replacement_token)
        bm = self.block_manager
        # roll the drafts back to the kept prefix: tokens, then pages; the
        # target has evaluated everything up to it
        seq.truncate_tokens(base_num_tokens + len(kept))
        bm.truncate(seq)
        seq.num_computed_tokens = base_num_tokens + len(kept)
        bm.mark_computed(seq)
        # a sequence ending on a page boundary gets its last page keyed
        # before anything is appended
        if len(seq) % bm.block_size == 0:
            bm.may_append(seq)
        # the replacement is an output: its K/V is written by the next step,
        # so only its page is reserved now
        if replacement_token is not None and seq.num_completion_tokens < seq.max_tokens:
            seq.append_token(replacement_token)
            bm.may_append(seq)
        if ((not seq.ignore_eos and seq.last_token == self.eos)
                or seq.num_completion_tokens >= seq.max_tokens):
            self._finish(seq)
            self.running.remove(seq)
        return len(kept)

    def _settle(self, seq: Sequence, base: int, accepted: list[int],
                replacement: int | None) -> tuple[list[int], int | None]:
        """The drafts to keep and the replacement to append: the accepted
        drafts within the token budget, up to and including the first EOS;
        no replacement once the budget or an EOS cut the accepted drafts."""
        room = max(seq.max_tokens - (base - seq.num_prompt_tokens), 0)
        kept = accepted[:room]
        if not seq.ignore_eos and self.eos in kept:
            return kept[:kept.index(self.eos) + 1], None
        if len(kept) < len(accepted):
            return kept, None
        return kept, replacement
