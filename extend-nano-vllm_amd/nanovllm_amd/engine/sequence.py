"""One generation request: its tokens, its KV pages and how far the target
model has processed it.

Behaviour follows nanovllm/engine/sequence.py:8-120 (the attribute names are
the engine's interface: the scheduler, the model runner and the reference's
benchmarks read them).  The token list is the single source of truth: its
length, last token, prompt and completion views are derived from it.
"""
from __future__ import annotations

from enum import Enum, auto
from itertools import count

from nanovllm_amd.sampling_params import SamplingParams

_ids = count()


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    """A request: ``token_ids`` (prompt followed by completions) and the
    physical KV pages holding them (``block_table``, page size
    ``block_size``).

    Progress counters, all in tokens:
      num_cached_tokens     prompt tokens whose pages came from the prefix cache
      num_computed_tokens   tokens whose K/V are in the target cache
      num_scheduled_tokens  tokens the current step feeds the model
    """

    block_size = 256

    def __init__(self, token_ids: list[int], sampling_params: SamplingParams | None = None):
        if not token_ids:
            raise ValueError("a sequence needs at least one token")
        sp = sampling_params if sampling_params is not None else SamplingParams()
        self.seq_id = next(_ids)
        self.status = SequenceStatus.WAITING
        self.token_ids = list(token_ids)
        self.num_prompt_tokens = len(self.token_ids)
        self.block_table: list[int] = []
        self.num_cached_tokens = 0
        self.num_computed_tokens = 0
        self.num_scheduled_tokens = 0
        self.temperature = sp.temperature
        self.max_tokens = sp.max_tokens
        self.ignore_eos = sp.ignore_eos

    # ---- sizes and views
    def __len__(self) -> int:
        return len(self.token_ids)

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def last_token(self) -> int:
        return self.token_ids[-1]

    @property
    def num_completion_tokens(self) -> int:
        return len(self.token_ids) - self.num_prompt_tokens

    @property
    def prompt_token_ids(self) -> list[int]:
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    @property
    def is_prefill_complete(self) -> bool:
        return self.num_computed_tokens >= len(self.token_ids)

    # ---- pages
    @property
    def num_blocks(self) -> int:
        """Pages needed for the current tokens."""
        return -(-len(self.token_ids) // self.block_size)

    def page_tokens(self, page: int) -> list[int]:
        """Tokens of logical page ``page`` (the last one may be partial)."""
        if not 0 <= page < self.num_blocks:
            raise IndexError(f"page {page} out of range")
        start = page * self.block_size
        return self.token_ids[start:start + self.block_size]

    # ---- edits
    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)

    def truncate_tokens(self, num_tokens: int) -> None:
        """Cut the sequence back to ``num_tokens`` tokens (speculative
        rollback; the prompt is never cut).  Counters past the new end are
        clamped to it."""
        if not self.num_prompt_tokens <= num_tokens <= len(self.token_ids):
            raise ValueError("cannot truncate outside the sequence token range")
        del self.token_ids[num_tokens:]
        self.num_computed_tokens = min(self.num_computed_tokens, num_tokens)
        self.num_scheduled_tokens = min(self.num_scheduled_tokens, num_tokens)
