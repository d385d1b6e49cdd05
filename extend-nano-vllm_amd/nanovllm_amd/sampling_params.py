"""Per-request sampling knobs (nanovllm/sampling_params.py:4-11)."""
from dataclasses import dataclass


@dataclass
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False

    def __post_init__(self):
        # the reference asserts (sampling_params.py:11); raised explicitly so
        # the check survives python -O
        if not self.temperature >= 0:
            raise AssertionError("temperature must be non-negative")
        # not in the reference: a budget of 0 tokens never reaches its
        # stopping test (num_completion_tokens == max_tokens after a token is
        # appended, scheduler.py:184-190) and would run to max_model_len
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be at least 1")
