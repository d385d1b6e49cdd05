"""LLMEngine: request intake, the step loop and generate()
(nanovllm/engine/llm_engine.py:20-228, single GPU).

The speculative step keeps the reference's order of operations
(llm_engine.py:124-178) -- reserve blocks, propose, begin speculation,
verify, accept, postprocess, commit -- with two batched stages: acceptance
comes from the fused GPU scan (one device->host copy per step) and the draft
replays every sequence's committed tail in one forward.
"""
from __future__ import annotations

import atexit
from dataclasses import fields
from time import perf_counter

from nanovllm_amd.config import Config
from nanovllm_amd.engine.model_runner import ModelRunner
from nanovllm_amd.engine.scheduler import Scheduler
from nanovllm_amd.engine.sequence import Sequence
from nanovllm_amd.engine.speculative import verify_greedy_proposals
from nanovllm_amd.sampling_params import SamplingParams


def _load_tokenizer(path: str):
    """The checkpoint's tokenizer, or None when the directory has none
    (random-weight checkpoints; prompts must then be token ids)."""
    try:
        from transformers import AutoTokenizer

        return AutoTokenizer.from_pretrained(path, use_fast=True)
    except Exception:
        return None


class LLMEngine:

    def __init__(self, model, **kwargs):
        names = {f.name for f in fields(Config)}
        config = Config(model, **{k: v for k, v in kwargs.items() if k in names})
        self.config = config
        self._exited = False
        self.model_runner = ModelRunner(config, 0, None)
        self.tokenizer = _load_tokenizer(config.model)
        if self.tokenizer is not None and self.tokenizer.eos_token_id is not None:
            config.eos = self.tokenizer.eos_token_id
        else:
            eos = getattr(config.hf_config, "eos_token_id", None)
            config.eos = eos[0] if isinstance(eos, (list, tuple)) else (eos if eos is not None else -1)
        self.scheduler = Scheduler(config)
        self.spec_stats = {"steps": 0, "drafted": 0, "accepted": 0, "committed": 0}
        # comparison runs: execute speculative steps with the reference's
        # structure (see _reference_speculative_step)
        self.reference_pipeline = False
        # queue each step's successor draft behind its verify (see
        # _speculative_step); off, every step drafts after the host's
        # bookkeeping, as before
        self.prelaunch_draft = True
        atexit.register(self.exit)

    def exit(self):
        if self._exited:
            return
        self._exited = True
        try:
            self.model_runner.call("exit")
        finally:
            atexit.unregister(self.exit)

    @property
    def cache_stats(self):
        return self.scheduler.block_manager.stats.copy()

    def add_request(self, prompt: str | list[int], sampling_params: SamplingParams):
        if self.config.speculative_config is not None and sampling_params.temperature != 0:
            raise ValueError("EAGLE3 speculative decoding currently requires temperature=0")
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("this checkpoint has no tokenizer: pass token ids")
            prompt = self.tokenizer.encode(prompt)
        if not prompt:
            raise ValueError("prompt must contain at least one token")
        if len(prompt) + sampling_params.max_tokens > self.config.max_model_len:
            raise ValueError("prompt and completion exceed max_model_len: "
                             f"{len(prompt)} + {sampling_params.max_tokens} > "
                             f"{self.config.max_model_len}")
        self.scheduler.add(Sequence(prompt, sampling_params))

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        scheduled = sum(seq.num_scheduled_tokens for seq in seqs)
        if self.config.speculative_config is not None and not is_prefill:
            step = self._reference_speculative_step if self.reference_pipeline else self._speculative_step
            num_tokens = -step(seqs)
        else:
            token_ids = self.model_runner.call("run", seqs, is_prefill)
            self.scheduler.postprocess(seqs, token_ids, is_prefill)
            num_tokens = scheduled if is_prefill else -len(seqs)
        outputs = [(seq.seq_id, seq.completion_token_ids) for seq in seqs if seq.is_finished]
        return outputs, num_tokens

    def _speculative_step(self, seqs: list[Sequence]) -> int:
        """One EAGLE3 decode step over ``seqs``; returns the committed count."""
        for seq in seqs:
            self.scheduler.reserve_speculation(seq)
        # the runner may enqueue the verify right behind the draft, so that
        # the host's bookkeeping below overlaps the target forward, and the
        # next step's draft behind both (prelaunch) when the batch will stay
        # as it is: nothing waiting, every sequence two steps from its budget
        k = self.scheduler.num_speculative_tokens
        prelaunch = (self.prelaunch_draft and not self.scheduler.waiting
                     and all(seq.max_tokens - seq.num_completion_tokens > 2 * k + 1
                             for seq in seqs)
                     and self.scheduler.reserve_lookahead(seqs))
        proposals = self.model_runner.call("propose_verify_eagle3_batch", seqs, prelaunch)
        pipelined = proposals is not None
        if not pipelined:
            proposals = self.model_runner.call("propose_eagle3_batch", seqs)
        bases = []
        for seq, proposal in zip(seqs, proposals):
            bases.append(self.scheduler.begin_speculation(seq, proposal))
            # the tail token (the previous target output) is verified with the drafts
            seq.num_computed_tokens = bases[-1] - 1
        targets, accept_len, bonus = self.model_runner.call(
            "collect_verify_eagle3_batch" if pipelined else "verify_eagle3_batch_fused",
            seqs, [len(p) + 1 for p in proposals])
        commit_seqs, commit_tokens, commit_starts = [], [], []
        for seq, proposal, base, target, a, b in zip(seqs, proposals, bases, targets,
                                                     accept_len, bonus):
            if len(target) != len(proposal) + 1:
                raise RuntimeError("EAGLE3 target verification returned an incomplete batch: "
                                   f"proposals={len(proposal)}, target_tokens={len(target)}")
            # the host rule (hookable, as in the reference engine) must agree
            # with the fused GPU scan
            v = verify_greedy_proposals(proposal, target)
            if (v.accepted_count, v.replacement_token) != (a, b):
                raise RuntimeError(f"device acceptance ({a}, {b}) disagrees with greedy "
                                   f"verification ({v.accepted_count}, {v.replacement_token})")
            self.spec_stats["drafted"] += len(proposal)
            self.spec_stats["accepted"] += v.accepted_count
            self.scheduler.postprocess_speculation(seq, base, v.accepted_tokens,
                                                   v.replacement_token)
            tail = seq.token_ids[base:]
            if tail and not seq.is_finished:
                commit_seqs.append(seq)
                commit_tokens.append(tail)
                commit_starts.append(base - 1)
            if seq.is_finished:
                self.model_runner.call("release_eagle3_state", seq.seq_id)
        if commit_seqs:
            self.model_runner.call("commit_eagle3_batch", commit_seqs, commit_tokens,
                                   commit_starts)
        committed = sum(len(seq) - base for seq, base in zip(seqs, bases))
        self.spec_stats["steps"] += 1
        self.spec_stats["committed"] += committed
        return committed

    def _reference_speculative_step(self, seqs: list[Sequence]) -> int:
        """One EAGLE3 step in the reference's structure (llm_engine.py:124-178):
        proposals with a host sync per draft step, per-sequence argmax and
        host rule, and a serial single-token draft replay per committed token.
        Same kernels as the engine's own step; used to time the reference's
        pipeline shape on this hardware."""
        runner = self.model_runner
        for seq in seqs:
            self.scheduler.reserve_speculation(seq)
        proposals = runner.call("propose_eagle3_batch_reference", seqs)
        bases = []
        for seq, proposal in zip(seqs, proposals):
            bases.append(self.scheduler.begin_speculation(seq, proposal))
            seq.num_computed_tokens = bases[-1] - 1
        targets, aux = runner.call("verify_eagle3_batch_reference", seqs,
                                   [len(p) + 1 for p in proposals])
        for seq, proposal, base, target, rows in zip(seqs, proposals, bases, targets, aux):
            v = verify_greedy_proposals(proposal, target)
            self.spec_stats["drafted"] += len(proposal)
            self.spec_stats["accepted"] += v.accepted_count
            self.scheduler.postprocess_speculation(seq, base, v.accepted_tokens,
                                                   v.replacement_token)
            tail = seq.token_ids[base:]
            if tail and not seq.is_finished:
                runner.call("commit_eagle3_serial", seq, tail, rows, base - 1)
            if seq.is_finished:
                runner.call("release_eagle3_state", seq.seq_id)
        committed = sum(len(seq) - base for seq, base in zip(seqs, bases))
        self.spec_stats["steps"] += 1
        self.spec_stats["committed"] += committed
        return committed

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    def generate(self, prompts, sampling_params, use_tqdm: bool = True):
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        pbar = None
        if use_tqdm:
            from tqdm.auto import tqdm

            pbar = tqdm(total=len(prompts), desc="Generating", dynamic_ncols=True)
        for prompt, sp in zip(prompts, sampling_params):
            self.add_request(prompt, sp)
        outputs = {}
        prefill_tps = decode_tps = 0.0
        while not self.is_finished():
            t = perf_counter()
            output, num_tokens = self.step()
            if pbar is not None:
                dt = perf_counter() - t
                if num_tokens > 0:
                    prefill_tps = num_tokens / dt
                else:
                    decode_tps = -num_tokens / dt
                pbar.set_postfix({"Prefill": f"{int(prefill_tps)}tok/s",
                                  "Decode": f"{int(decode_tps)}tok/s"})
            for seq_id, token_ids in output:
                outputs[seq_id] = token_ids
                if pbar is not None:
                    pbar.update(1)
        if pbar is not None:
            pbar.close()
        ordered = [outputs[i] for i in sorted(outputs)]
        decode = (lambda ids: self.tokenizer.decode(ids)) if self.tokenizer is not None else (lambda ids: "")
        return [{"text": decode(ids), "token_ids": ids} for ids in ordered]

