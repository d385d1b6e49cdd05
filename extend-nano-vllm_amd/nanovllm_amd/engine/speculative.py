"""Greedy acceptance of draft proposals (nanovllm/engine/speculative.py:4-30).

``verify_greedy_proposals`` is the host-side statement of the rule; the
engine's hot path computes the same result on the GPU for a whole batch
(``kernels.argmax_accept``) and builds ``GreedyVerification`` objects from
it with ``from_device``.
"""
from dataclasses import dataclass


@dataclass(frozen=True)
class GreedyVerification:
    accepted_count: int
    accepted_tokens: list[int]
    replacement_token: int | None


def verify_greedy_proposals(proposal_tokens: list[int],
                            target_tokens: list[int]) -> GreedyVerification:
    """Accept the longest prefix on which the draft agrees with the target.

    The first disagreeing target token replaces the rejected draft; when every
    draft is accepted the next target token (if any) is the bonus token.
    Raises ValueError when the target does not cover every proposal."""
    if len(target_tokens) < len(proposal_tokens):
        raise ValueError("target verification must cover every proposal")
    n = 0
    while n < len(proposal_tokens) and proposal_tokens[n] == target_tokens[n]:
        n += 1
    replacement = target_tokens[n] if n < len(target_tokens) else None
    return GreedyVerification(n, list(proposal_tokens[:n]), replacement)


def from_device(proposal_tokens: list[int], accept_len: int, bonus: int) -> GreedyVerification:
    """GreedyVerification from the fused GPU scan (accept_len, bonus token).

    The verify batch always holds len(proposal) + 1 target rows, so a
    replacement/bonus token always exists."""
    if not 0 <= accept_len <= len(proposal_tokens):
        raise RuntimeError(
            f"device acceptance out of range: {accept_len} for {len(proposal_tokens)} proposals")
    return GreedyVerification(accept_len, list(proposal_tokens[:accept_len]), int(bonus))
