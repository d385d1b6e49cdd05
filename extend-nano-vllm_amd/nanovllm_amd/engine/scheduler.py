"""Prefill/decode scheduling and the speculation bookkeeping
(nanovllm/engine/scheduler.py:10-191)."""
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
        return not self.waiting and not self.running

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def _finished(self, seq: Sequence, token_id: int) -> bool:
        return ((not seq.ignore_eos and token_id == self.eos)
                or seq.num_completion_tokens >= seq.max_tokens)

    def schedule(self) -> tuple[list[Sequence], bool]:
        """Return (sequences, is_prefill).

        Prefill has priority, but never twice in a row while sequences are
        running, so decode keeps progressing.  Without prefill batching one
        request is prefilled per step; long prompts are chunked by the token
        budget."""
        if self.waiting and not (self.running and self.last_step_was_prefill):
            picked: list[Sequence] = []
            budget = self.max_num_batched_tokens
            for seq in self.waiting:
                if (len(picked) == self.max_num_seqs or budget == 0
                        or (picked and not self.enable_prefill_batching)):
                    break
                if not seq.block_table:
                    if not self.block_manager.can_allocate(seq):
                        if not self.running and not picked:
                            raise RuntimeError("not enough KV-cache blocks for request")
                        break
                    self.block_manager.allocate(seq)
                seq.num_scheduled_tokens = min(seq.num_tokens - seq.num_computed_tokens, budget)
                budget -= seq.num_scheduled_tokens
                picked.append(seq)
            if picked:
                self.last_step_was_prefill = True
                self.stats["prefill_steps"] += 1
                self.stats["max_prefill_tokens_per_step"] = max(
                    self.stats["max_prefill_tokens_per_step"],
                    self.max_num_batched_tokens - budget)
                return picked, True

        picked = []
        while self.running and len(picked) < self.max_num_seqs:
            seq = self.running.popleft()
            while not self.block_manager.can_append(seq):
                if self.running:
                    self.preempt(self.running.pop())
                else:
                    self.preempt(seq)
                    break
            else:
                self.block_manager.may_append(seq)
                picked.append(seq)
        assert picked
        self.running.extendleft(reversed(picked))
        self.last_step_was_prefill = False
        return picked, False

    def preempt(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.WAITING
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        if is_prefill:
            for seq, token_id in zip(seqs, token_ids):
                seq.num_computed_tokens += seq.num_scheduled_tokens
                seq.num_scheduled_tokens = 0
                self.block_manager.mark_computed(seq)
                if not seq.is_prefill_complete:
                    continue
                self.waiting.remove(seq)
                seq.status = SequenceStatus.RUNNING
                seq.append_token(token_id)
                if self._finished(seq, token_id):
                    seq.status = SequenceStatus.FINISHED
                    self.block_manager.deallocate(seq)
                else:
                    self.running.append(seq)
            return
        for seq, token_id in zip(seqs, token_ids):
            seq.num_computed_tokens = len(seq)
            self.block_manager.mark_computed(seq)
            seq.append_token(token_id)
            if self._finished(seq, token_id):
                seq.status = SequenceStatus.FINISHED
                self.block_manager.deallocate(seq)
                self.running.remove(seq)

    # ------------------------------------------------------------ speculation

    def begin_speculation(self, seq: Sequence, proposal_tokens: list[int]) -> int:
        """Append the drafts (their blocks were reserved); return the length
        before them (``base``)."""
        if seq not in self.running:
            raise RuntimeError("speculative decode requires a running sequence")
        base = len(seq)
        seq.append_tokens(proposal_tokens)
        return base

    def reserve_speculation(self, seq: Sequence) -> None:
        """Reserve blocks for every draft position before the draft model
        writes K/V for them."""
        max_tokens = min(seq.max_tokens + seq.num_prompt_tokens,
                         len(seq) + self.num_speculative_tokens)
        self.block_manager.ensure_num_blocks_for_length(seq, max_tokens)

    def postprocess_speculation(self, seq: Sequence, base_num_tokens: int,
                                accepted_tokens: list[int],
                                replacement_token: int | None) -> int:
        """Commit the accepted drafts plus the replacement/bonus token.

        Accepted drafts are clipped to max_tokens and at the first EOS (no
        replacement then); the sequence and its block table are rolled back
        to base + committed drafts, the replacement is appended if there is
        room, and the sequence finishes on EOS or max_tokens.  Returns the
        number of committed drafts."""
        remaining = seq.max_tokens - (base_num_tokens - seq.num_prompt_tokens)
        committed = accepted_tokens[:max(remaining, 0)]
        if not seq.ignore_eos and self.eos in committed:
            committed = committed[:committed.index(self.eos) + 1]
            replacement_token = None
        elif len(committed) < len(accepted_tokens):
            replacement_token = None

        seq.truncate_tokens(base_num_tokens + len(committed))
        self.block_manager.truncate(seq)
        # the target has evaluated the tail and the committed drafts; the
        # replacement is an output whose K/V is not in the cache yet
        seq.num_computed_tokens = base_num_tokens + len(committed)
        self.block_manager.mark_computed(seq)

        bs = self.block_manager.block_size
        if replacement_token is not None and seq.num_completion_tokens < seq.max_tokens:
            if len(seq) % bs == 0:
                self.block_manager.may_append(seq)     # finalise the full page first
            seq.append_token(replacement_token)
            self.block_manager.may_append(seq)         # reserve a new page if needed
        elif len(seq) % bs == 0:
            self.block_manager.may_append(seq)

        if ((not seq.ignore_eos and seq.last_token == self.eos)
                or seq.num_completion_tokens >= seq.max_tokens):
            seq.status = SequenceStatus.FINISHED
            self.block_manager.deallocate(seq)
            self.running.remove(seq)
        return len(committed)
