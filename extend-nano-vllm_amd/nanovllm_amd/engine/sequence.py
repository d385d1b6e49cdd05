"""Request state: token list, paged block table and progress counters
(nanovllm/engine/sequence.py:8-120)."""
from copy import copy
from enum import Enum, auto
from itertools import count

from nanovllm_amd.sampling_params import SamplingParams


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    """One request.

    ``num_computed_tokens`` counts tokens whose K/V are in the target cache;
    ``num_scheduled_tokens`` is the slice the current step feeds the model;
    ``block_table`` lists the physical KV blocks (block_size tokens each)."""

    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], sampling_params: SamplingParams = SamplingParams()):
        if not token_ids:
            raise ValueError("a sequence needs at least one token")
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.token_ids = copy(token_ids)
        self.last_token = token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = len(token_ids)
        self.num_cached_tokens = 0
        self.num_computed_tokens = 0
        self.num_scheduled_tokens = 0
        self.block_table: list[int] = []
        self.temperature = sampling_params.temperature
        self.max_tokens = sampling_params.max_tokens
        self.ignore_eos = sampling_params.ignore_eos

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self) -> bool:
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self) -> int:
        return self.num_tokens - self.num_prompt_tokens

    @property
    def prompt_token_ids(self) -> list[int]:
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_cached_blocks(self) -> int:
        return self.num_cached_tokens // self.block_size

    @property
    def is_prefill_complete(self) -> bool:
        return self.num_computed_tokens >= self.num_tokens

    @property
    def num_blocks(self) -> int:
        return -(-self.num_tokens // self.block_size)

    @property
    def last_block_num_tokens(self) -> int:
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def block(self, i: int) -> list[int]:
        if not 0 <= i < self.num_blocks:
            raise IndexError(f"block {i} out of range")
        return self.token_ids[i * self.block_size:(i + 1) * self.block_size]

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1

    def append_tokens(self, token_ids: list[int]) -> None:
        for token_id in token_ids:
            self.append_token(token_id)

    def truncate_tokens(self, num_tokens: int) -> None:
        """Drop tokens beyond ``num_tokens`` (never into the prompt)."""
        if not self.num_prompt_tokens <= num_tokens <= self.num_tokens:
            raise ValueError("cannot truncate outside the sequence token range")
        del self.token_ids[num_tokens:]
        self.num_tokens = num_tokens
        self.last_token = self.token_ids[-1]
        self.num_computed_tokens = min(self.num_computed_tokens, num_tokens)
        self.num_scheduled_tokens = min(self.num_scheduled_tokens, num_tokens)

    def __getstate__(self):
        return (self.seq_id, self.status, self.num_tokens, self.num_prompt_tokens,
                self.num_cached_tokens, self.num_computed_tokens, self.num_scheduled_tokens,
                self.block_table, self.temperature, self.max_tokens, self.ignore_eos,
                self.token_ids)

    def __setstate__(self, state):
        (self.seq_id, self.status, self.num_tokens, self.num_prompt_tokens,
         self.num_cached_tokens, self.num_computed_tokens, self.num_scheduled_tokens,
         self.block_table, self.temperature, self.max_tokens, self.ignore_eos,
         self.token_ids) = state
        self.last_token = self.token_ids[-1]
