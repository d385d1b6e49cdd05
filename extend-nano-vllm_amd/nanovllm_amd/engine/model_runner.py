"""Runs the target and EAGLE3 draft models on one GPU
(nanovllm/engine/model_runner.py, the single-process EAGLE3 subset).

Method names and return values follow the reference so the engine-level
orchestration is unchanged: ``run``, ``propose_eagle3_batch``,
``verify_eagle3_batch``, ``commit_eagle3``, ``release_eagle3_state``,
``get_eagle3_runtime_capabilities``, ``run_eagle3_graph``, ``call``.
The engine's hot path uses the batched forms ``verify_eagle3_batch_fused``
(argmax + accept fused on the GPU, one device->host copy per step) and
``commit_eagle3_batch`` (one ragged draft forward for every sequence's
committed tail instead of one forward per token per sequence).

Draft KV slots.  The draft consumes the pair (token[p+1], target aux state
at p) at RoPE position p and stores its K/V at the slot of position p, in
prefill, proposal and commit alike.  (The reference stores decode- and
commit-time draft K/V one slot later than prefill, model_runner.py:
1087-1096 / :1143-1149 vs :784-789, leaving one slot unwritten but read;
emitted tokens do not depend on it because the target verifies every
token.)
"""
from __future__ import annotations

import numpy as np
import torch

from nanovllm_amd import _native
from nanovllm_amd import kernels as K
from nanovllm_amd.context import get_context, reset_context, set_context
from nanovllm_amd.eagle3 import Eagle3KVCache, load_eagle3_model
from nanovllm_amd.engine.graphs import (BUCKETS, ChainedProposeGraph, CommitGraph,
                                        DeviceCommitGraph, ProposeGraph, VerifyGraph,
                                        block_table_array, bucket_for)
from nanovllm_amd.engine.sequence import Sequence
from nanovllm_amd.layers import Attention, init_random_, param_bytes
from nanovllm_amd.loader import load_model
from nanovllm_amd.qwen3 import Qwen3ForCausalLM, aux_concat


def _use_gemm_tuning(path: str) -> None:
    """Dispatch the projection GEMMs through the solutions recorded in
    ``path`` (PyTorch TunableOp results for this GPU and library versions).
    Lookup only: no tuning runs, so HIP graph capture is unaffected; shapes
    not in the file keep the library's default choice."""
    import torch.cuda.tunable as tunable

    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    if not tunable.read_file(path):
        raise RuntimeError(f"cannot read GEMM tuning results {path}")


def _pinned(values, dtype) -> torch.Tensor:
    if isinstance(values, np.ndarray):
        out = torch.empty(values.shape, dtype=dtype, pin_memory=True)
        out.copy_(torch.from_numpy(values))
        return out
    return torch.tensor(values, dtype=dtype, pin_memory=True)


class ModelRunner:

    def __init__(self, config, rank: int = 0, event=None):
        if rank != 0:
            raise ValueError("this build runs one process per GPU (rank 0 only)")
        _native.load()   # fail loudly without the HIP library
        self.config = config
        hf = config.hf_config
        self.block_size = config.kvcache_block_size
        self.enforce_eager = config.enforce_eager
        self.rank = rank
        self.device = torch.device("cuda", config.device_offset)
        torch.cuda.set_device(self.device)
        if config.gemm_tuning_file is not None:
            _use_gemm_tuning(config.gemm_tuning_file)
        self._exited = False
        self.decode_graph_replay_count = 0
        default_dtype = torch.get_default_dtype()
        dtype = getattr(hf, "torch_dtype", None) or getattr(hf, "dtype", None) or torch.bfloat16
        if isinstance(dtype, str):
            dtype = getattr(torch, dtype)
        self.dtype = dtype
        torch.set_default_dtype(dtype)
        torch.set_default_device(self.device)
        try:
            self.model = Qwen3ForCausalLM(hf)
            if config.load_format == "dummy":
                init_random_(self.model, config.seed)
            else:
                load_model(self.model, config.model)
            self.model.eval()
            self.speculative_config = config.speculative_config
            self.eagle3_model = None
            self.eagle_graphs: dict = {}
            self.eagle_graph_vars: dict = {}
            self.graphs: dict = {}
            self.graph_pool = None
            self._verify_graphs: dict[int, VerifyGraph] = {}
            self._propose_graphs: dict[int, ProposeGraph] = {}
            self._commit_graphs: dict[tuple[int, int], CommitGraph] = {}
            self._device_commit_graphs: dict[int, DeviceCommitGraph] = {}
            self._chained_graphs: dict[int, ChainedProposeGraph] = {}
            self._proposal_buffers: dict[int, torch.Tensor] = {}
            self._device_committed = None
            self._pending_verify = None
            self._pending_graph = None
            if self.speculative_config is not None:
                self.eagle3_model = load_eagle3_model(self.speculative_config.model, self.device,
                                                      config.load_format, config.seed + 1)
                ec = self.eagle3_model.config
                if ec.target_hidden_size != hf.hidden_size or ec.target_vocab_size != hf.vocab_size:
                    raise ValueError("EAGLE3 checkpoint is incompatible with the target Qwen3")
                if ec.num_aux_hidden_states != len(self.speculative_config.aux_hidden_state_layers):
                    raise ValueError("EAGLE3 aux state count does not match aux_hidden_state_layers")
            self.warmup_model()
            self.allocate_kv_cache()
            k = self.speculative_config.num_speculative_tokens if self.speculative_config else 0
            # upper bounds of one sequence's keys and block-table width
            self.max_seqlen_k = config.max_model_len + k + 1
            self.max_blocks_per_seq = -(-self.max_seqlen_k // self.block_size)
            if self.eagle3_model is not None:
                # recurrent draft state of every running sequence, one row each
                h = self.eagle3_model.config.hidden_size
                # plus one scratch row that padded graph rows write into
                rows = config.max_num_seqs + 1
                self.scratch_state_row = rows
                self.state_hidden = torch.zeros(rows + 1, h, dtype=self.dtype, device=self.device)
                self.state_feedback = torch.zeros(rows + 1, h, dtype=self.dtype, device=self.device)
                self._state_slot: dict[int, int] = {}
                self._free_state = list(range(rows - 1, -1, -1))
        finally:
            torch.set_default_device("cpu")
            torch.set_default_dtype(default_dtype)
        # benchmarks may ask to keep the last verify's logits and inputs, or to
        # run the verify forward eagerly (kernel-level timing)
        self.keep_verify_inputs = False
        self.use_verify_graph = True
        self.last_verify_inputs = None
        # propose and verify enqueued back to back (propose_verify_eagle3_batch),
        # and the draft commit right behind the verify (DeviceCommitGraph)
        self.pipeline_verify = True
        self.device_commit = True
        # tests and benchmarks: draft_override(seqs, tokens) may rewrite the
        # device proposals in place before they are verified (tokens [k,
        # bucket] from a draft graph, [steps, len(seqs)] from the eager loop;
        # column i is seqs[i])
        self.draft_override = None
        self._inflight_verify = None
        # the next step's draft queued behind a verify (propose_verify_eagle3_batch
        # with prelaunch): (graph, seq id per draft column, lengths before the
        # step, lengths after it once collect has the results)
        self._prelaunched = None
        self.prelaunch_stats = {"queued": 0, "used": 0}
        # pipelined steps, and those among them with a sequence proposing
        # fewer than k drafts (close to its budget)
        self.pipeline_stats = {"steps": 0, "ragged": 0}
        self._proposal_host = torch.empty(0, dtype=torch.int64)
        # one pinned host buffer receives argmax + accept results each verify
        self._verify_host = torch.empty(1 << 16, dtype=torch.int32, pin_memory=True)
        self._verify_dev = torch.empty(1 << 16, dtype=torch.int32, device=self.device)
        if self.eagle3_model is not None and self._use_graphs():
            self.capture_eagle3_graphs()

    def eagle3_graph_batch_sizes(self) -> list[int]:
        """The padded batch sizes (buckets) whose step graphs are captured at
        initialisation: every bucket below max_num_seqs (at most 512) and the
        one that holds max_num_seqs, as the reference captures its draft
        step for 1, 2, 4, 8 and multiples of 16 up to max_num_seqs
        (model_runner.py:1472-1481)."""
        max_bs = min(self.config.max_num_seqs, BUCKETS[-1])
        return [b for b in BUCKETS if b < max_bs] + [bucket_for(max_bs)]

    @torch.inference_mode()
    def capture_eagle3_graphs(self) -> None:
        """Capture the speculative step's graphs for every batch bucket
        before serving (model_runner.py:195, :1472-1523): the verify (target
        forward, LM head, fused argmax + accept), the k-step draft, the
        device commit behind the verify and the next step's draft behind
        both.  Largest bucket first, so the shared attention and argmax
        workspaces reach their final size before the smaller captures.
        Buckets a step needs later (a batch above max_num_seqs cannot occur)
        are captured on first use."""
        k = self.speculative_config.num_speculative_tokens
        for bs in reversed(self.eagle3_graph_batch_sizes()):
            vgraph = self._verify_graphs.get(bs)
            if vgraph is None:
                vgraph = self._verify_graphs[bs] = VerifyGraph(self, bs, k + 1)
            if bs not in self._propose_graphs:
                self._propose_graphs[bs] = ProposeGraph(self, bs, k)
            if bs not in self._device_commit_graphs:
                self._device_commit_graphs[bs] = DeviceCommitGraph(self, vgraph)
            if bs not in self._chained_graphs:
                self._chained_graphs[bs] = ChainedProposeGraph(self, bs, k, vgraph)

    # ------------------------------------------------------------ RPC surface

    def call(self, method_name: str, *args):
        method = getattr(self, method_name, None)
        if method is None:
            raise AttributeError(f"ModelRunner has no method {method_name!r}")
        return method(*args)

    @property
    def eagle3_states(self) -> dict[int, Eagle3KVCache]:
        """Per-sequence draft state (views into the state table)."""
        return {sid: Eagle3KVCache(self.state_hidden[r:r + 1], self.state_feedback[r:r + 1])
                for sid, r in self._state_slot.items()}

    def proposal_buffer(self, bs: int) -> torch.Tensor:
        """The [k, bs] int64 proposals of bucket bs: every draft graph of the
        bucket writes its tokens here and the bucket's verify graph composes
        its input ids from here, so the captured graphs share one address."""
        buf = self._proposal_buffers.get(bs)
        if buf is None:
            k = self.speculative_config.num_speculative_tokens
            buf = self._proposal_buffers[bs] = torch.zeros(k, bs, dtype=torch.int64,
                                                           device=self.device)
        return buf

    def _state_rows(self, seqs) -> list[int]:
        rows = []
        for seq in seqs:
            r = self._state_slot.get(seq.seq_id)
            if r is None:
                if not self._free_state:
                    raise RuntimeError("no free EAGLE3 draft-state rows")
                r = self._free_state.pop()
                self._state_slot[seq.seq_id] = r
            rows.append(r)
        return rows

    def _store_states(self, seqs, hidden, feedback, last_rows: list[int]) -> None:
        dst = _pinned(self._state_rows(seqs), torch.int64).to(self.device, non_blocking=True)
        src = _pinned(last_rows, torch.int64).to(self.device, non_blocking=True)
        self.state_hidden.index_copy_(0, dst, hidden.index_select(0, src))
        self.state_feedback.index_copy_(0, dst, feedback.index_select(0, src))

    def exit(self):
        if self._exited:
            return
        self._exited = True
        torch.cuda.synchronize(self.device)
        self.graphs.clear()
        self.eagle_graphs.clear()
        self.eagle_graph_vars.clear()
        self._pending_graph = None
        self._commit_graphs.clear()
        self._device_commit_graphs.clear()
        self._verify_graphs.clear()
        self._propose_graphs.clear()
        self._chained_graphs.clear()
        self._proposal_buffers.clear()
        self._prelaunched = None
        self._inflight_verify = None
        self._device_committed = None

    # ------------------------------------------------------------ memory

    @torch.inference_mode()
    def warmup_model(self):
        """One dummy prefill (attention returns zeros) at the largest batch to
        measure peak activation memory before sizing the KV cache."""
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(self.device)
        n = max(1, min(self.config.max_num_batched_tokens, self.config.max_model_len))
        ids = torch.zeros(n, dtype=torch.int64, device=self.device)
        pos = torch.arange(n, dtype=torch.int64, device=self.device)
        set_context(True)
        get_context().is_dummy = True
        try:
            if self.speculative_config is not None:
                hidden, aux = self.model.forward_with_aux_hidden_states(
                    ids, pos, self.speculative_config.aux_hidden_state_layers)
                combined = self.eagle3_model.combine_hidden_states(aux_concat(aux))
                self.eagle3_model.forward_with_cache(ids, pos, combined)
            else:
                hidden = self.model(ids, pos)
            self.model.compute_logits(hidden[-1:])
        finally:
            reset_context()
        torch.cuda.synchronize(self.device)
        torch.cuda.empty_cache()

    def _kv_dtype(self):
        return torch.float8_e4m3fn if self.config.kv_cache_dtype == "fp8" else self.dtype

    def _kv_pages(self, kinds, layers, num_blocks, num_kv_heads, head_dim, dtype):
        """KV pages with the reference's logical shape [2, layers, blocks,
        block_size, Hkv, D] (model_runner.py:285-364 of the reference).  With
        the head-major layout the storage is [layers, blocks, Hkv, 2,
        block_size, D] -- one kv head's K rows and then its V rows, each a
        contiguous run -- and this is a permuted view of it: every consumer
        (store, attention) addresses pages through their strides, and a
        layer's K and V views share them."""
        if self.config.kv_cache_layout == "head_major":
            pages = torch.empty(layers, num_blocks, num_kv_heads, kinds, self.block_size, head_dim,
                                dtype=dtype, device=self.device)
            return pages.permute(3, 0, 1, 4, 2, 5)
        return torch.empty(kinds, layers, num_blocks, self.block_size, num_kv_heads, head_dim,
                           dtype=dtype, device=self.device)

    def allocate_kv_cache(self):
        config = self.config
        hf = config.hf_config
        kv_dtype = self._kv_dtype()
        head_dim = getattr(hf, "head_dim", None) or hf.hidden_size // hf.num_attention_heads
        layers = hf.num_hidden_layers
        block_bytes = 2 * layers * self.block_size * hf.num_key_value_heads * head_dim * kv_dtype.itemsize
        if self.eagle3_model is not None:
            ec = self.eagle3_model.config
            block_bytes += 2 * self.block_size * ec.num_key_value_heads * ec.head_dim * ec.torch_dtype.itemsize
        free, total = torch.cuda.mem_get_info(self.device)
        used = total - free
        stats = torch.cuda.memory_stats(self.device)
        peak = stats["allocated_bytes.all.peak"]
        current = stats["allocated_bytes.all.current"]
        budget = int(total * config.gpu_memory_utilization - used - peak + current)
        num_blocks = budget // block_bytes
        if config.num_kvcache_blocks > 0:
            num_blocks = min(num_blocks, config.num_kvcache_blocks)
        if num_blocks <= 0:
            raise RuntimeError("not enough GPU memory for the KV cache")
        config.num_kvcache_blocks = int(num_blocks)
        self.kv_cache = self._kv_pages(2, layers, num_blocks, hf.num_key_value_heads, head_dim,
                                       kv_dtype)
        attns = [m for m in self.model.modules() if isinstance(m, Attention)]
        assert len(attns) == layers
        for i, m in enumerate(attns):
            m.k_cache = self.kv_cache[0, i]
            m.v_cache = self.kv_cache[1, i]
        self.eagle_kv_cache = None
        if self.eagle3_model is not None:
            # same block ids as the target: the scheduler's block table and its
            # logical rollback govern both caches
            ec = self.eagle3_model.config
            d_attns = [m for m in self.eagle3_model.modules() if isinstance(m, Attention)]
            self.eagle_kv_cache = self._kv_pages(2, len(d_attns), num_blocks,
                                                 ec.num_key_value_heads, ec.head_dim,
                                                 ec.torch_dtype)
            for i, m in enumerate(d_attns):
                m.k_cache = self.eagle_kv_cache[0, i]
                m.v_cache = self.eagle_kv_cache[1, i]

    # ------------------------------------------------------------ metadata

    def _slot(self, seq: Sequence, position: int) -> int:
        return seq.block_table[position // self.block_size] * self.block_size + position % self.block_size

    def prepare_block_tables(self, seqs: list[Sequence]) -> torch.Tensor:
        width = max(len(seq.block_table) for seq in seqs)
        rows = [seq.block_table + [-1] * (width - len(seq.block_table)) for seq in seqs]
        return _pinned(rows, torch.int32).to(self.device, non_blocking=True)

    def prepare_prefill(self, seqs: list[Sequence]):
        """Varlen metadata for rows [num_computed, num_computed + scheduled)
        of each sequence (model_runner.py:761-800).  Also used by verify."""
        input_ids, positions, slots = [], [], []
        cu_q, cu_k = [0], [0]
        max_q = max_k = 0
        for seq in seqs:
            start = seq.num_computed_tokens
            scheduled = seq.num_scheduled_tokens or seq.num_tokens
            end = min(start + scheduled, seq.num_tokens)
            input_ids.extend(seq.token_ids[start:end])
            positions.extend(range(start, end))
            cu_q.append(cu_q[-1] + end - start)
            cu_k.append(cu_k[-1] + end)
            max_q = max(max_q, end - start)
            max_k = max(max_k, end)
            if seq.block_table:
                slots.extend(self._slot(seq, p) for p in range(start, end))
        block_tables = None
        if any(seq.block_table for seq in seqs):
            if not all(seq.block_table for seq in seqs):
                raise RuntimeError("mixed allocated and unallocated KV-cache batches")
            block_tables = self.prepare_block_tables(seqs)
        dev = self.device
        ids_t = _pinned(input_ids, torch.int64).to(dev, non_blocking=True)
        pos_t = _pinned(positions, torch.int64).to(dev, non_blocking=True)
        set_context(True, _pinned(cu_q, torch.int32).to(dev, non_blocking=True),
                    _pinned(cu_k, torch.int32).to(dev, non_blocking=True), max_q, max_k,
                    _pinned(slots, torch.int32).to(dev, non_blocking=True), None, block_tables)
        self._host_prefill = (input_ids, cu_q)
        return ids_t, pos_t

    def prepare_decode(self, seqs: list[Sequence]):
        """One row per sequence at its last token (model_runner.py:802-836)."""
        input_ids = [seq.last_token for seq in seqs]
        positions = [len(seq) - 1 for seq in seqs]
        context_lens = [len(seq) for seq in seqs]
        slots = [self._slot(seq, p) for seq, p in zip(seqs, positions)]
        dev = self.device
        cu_q = list(range(len(seqs) + 1))
        cu_k = [0]
        for n in context_lens:
            cu_k.append(cu_k[-1] + n)
        set_context(False, _pinned(cu_q, torch.int32).to(dev, non_blocking=True),
                    _pinned(cu_k, torch.int32).to(dev, non_blocking=True), 1, max(context_lens),
                    _pinned(slots, torch.int32).to(dev, non_blocking=True),
                    _pinned(context_lens, torch.int32).to(dev, non_blocking=True),
                    self.prepare_block_tables(seqs))
        return (_pinned(input_ids, torch.int64).to(dev, non_blocking=True),
                _pinned(positions, torch.int64).to(dev, non_blocking=True))

    def prepare_sample(self, seqs: list[Sequence]) -> torch.Tensor:
        return _pinned([seq.temperature for seq in seqs], torch.float32).to(self.device,
                                                                             non_blocking=True)

    # ------------------------------------------------------------ sampling

    def sample(self, logits: torch.Tensor, temperatures: torch.Tensor) -> torch.Tensor:
        """Greedy rows use the argmax kernel; temperature rows the
        exponential-race sampler of layers/sampler.py:10-19."""
        greedy = K.argmax_rows(logits)
        if not bool((temperatures > 0).any()):
            return greedy
        probs = torch.softmax(logits.float() / temperatures.clamp_min(1e-10).unsqueeze(1), dim=-1)
        sampled = probs.div_(torch.empty_like(probs).exponential_(1).clamp_min_(1e-10)).argmax(-1)
        return torch.where(temperatures == 0, greedy, sampled)

    # ------------------------------------------------------------ plain steps

    @torch.inference_mode()
    def run(self, seqs: list[Sequence], is_prefill: bool) -> list[int]:
        if not seqs:
            raise ValueError("empty batch")
        try:
            if is_prefill:
                input_ids, positions = self.prepare_prefill(seqs)
            else:
                if self.speculative_config is not None:
                    raise RuntimeError("EAGLE3 target runner received an unsupported decode")
                input_ids, positions = self.prepare_decode(seqs)
            temperatures = self.prepare_sample(seqs)
            if self.speculative_config is not None:
                return self._run_prefill_eagle3(seqs, input_ids, positions, temperatures)
            hidden = self.model(input_ids, positions)
            if is_prefill:
                last = get_context().cu_seqlens_q[1:].long() - 1
                hidden = hidden[last]
            logits = self.model.compute_logits(hidden)
            return self.sample(logits, temperatures).tolist()
        finally:
            reset_context()

    def _run_prefill_eagle3(self, seqs, input_ids, positions, temperatures) -> list[int]:
        """Target prefill with aux states, then the draft over the same rows
        (its K/V at the same slots) to seed each sequence's recurrent state
        (model_runner.py:1020-1044, :1369-1391)."""
        ctx = get_context()
        hidden, aux = self.model.forward_with_aux_hidden_states(
            input_ids, positions, self.speculative_config.aux_hidden_state_layers)
        last = ctx.cu_seqlens_q[1:].long() - 1
        next_tokens = self.sample(self.model.compute_logits(hidden[last]), temperatures)
        host_ids, cu = self._host_prefill
        # draft input at row p is token p+1; the last row takes the sampled
        # token (or the next prompt token when the prompt continues)
        shifted = list(host_ids[1:]) + [0]
        next_host = next_tokens.tolist()
        for i, seq in enumerate(seqs):
            end_pos = seq.num_computed_tokens + (cu[i + 1] - cu[i])
            shifted[cu[i + 1] - 1] = (next_host[i] if end_pos >= seq.num_tokens
                                      else seq.token_ids[end_pos])
        eagle_ids = _pinned(shifted, torch.int64).to(self.device, non_blocking=True)
        combined = self.eagle3_model.combine_hidden_states(aux_concat(aux))
        d_hidden, d_feedback = self.eagle3_model.forward_with_cache(eagle_ids, positions, combined)
        self._store_states(seqs, d_hidden, d_feedback, [cu[i + 1] - 1 for i in range(len(seqs))])
        return next_host

    # ------------------------------------------------------------ EAGLE3

    def get_eagle3_runtime_capabilities(self):
        """The reference's report (model_runner.py:982-990): a paged draft
        cache, and the batch sizes with captured draft-step graphs (here the
        k-step draft graphs, captured at initialisation unless
        enforce_eager)."""
        return {
            "paged_kv_cache": bool(getattr(self, "eagle3_model", None) is not None
                                   and getattr(self, "eagle_kv_cache", None) is not None),
            "cuda_graph": bool(getattr(self, "eagle_graphs", {})
                               or getattr(self, "_propose_graphs", {})),
            "graph_batch_sizes": sorted(set(getattr(self, "eagle_graphs", {}))
                                        | set(getattr(self, "_propose_graphs", {}))),
        }

    def _draft_step_metadata(self, seqs: list[Sequence], limits: list[int], steps: int):
        """Per draft step s < steps - 1 and sequence i: the RoPE position
        len_i - 1 + s, the slot its K/V goes to, and the keys it sees.  A
        sequence that needs fewer proposals (limits[i] < steps, near its
        max_tokens) gets slot -1 in the steps past its own last one: those
        steps' tokens are discarded, and their positions may lie beyond the
        pages reserved for it (reserve_speculation stops at max_tokens).
        Arrays [steps - 1, len(seqs)] (int64 positions, int32 slots and
        lengths); a slot whose page is not in the block table raises
        IndexError, as the block-table lookup does."""
        b = len(seqs)
        lens = np.fromiter((len(seq) for seq in seqs), dtype=np.int64, count=b)
        s = np.arange(max(steps - 1, 0), dtype=np.int64)[:, None]
        pos = lens[None, :] - 1 + s
        need = s < np.asarray(limits, dtype=np.int64)[None, :] - 1
        bt, nblk = block_table_array([seq.block_table for seq in seqs])
        blk = pos // self.block_size
        if np.any(need & (blk >= nblk[None, :])):
            raise IndexError("a draft position has no page in its block table")
        ids = bt[np.arange(b)[None, :], np.minimum(blk, bt.shape[1] - 1)].astype(np.int64)
        slots = np.where(need, ids * self.block_size + pos % self.block_size, -1).astype(np.int32)
        return pos, slots, (pos + 1).astype(np.int32)

    def _use_graphs(self) -> bool:
        return not self.enforce_eager

    @torch.inference_mode()
    def propose_eagle3_batch(self, seqs: list[Sequence]) -> list[list[int]]:
        """k greedy draft tokens per sequence (fewer near max_tokens) from the
        recurrent states (model_runner.py:1159-1213).  Draft step s consumes
        the previous token at RoPE position len-1+s and writes its K/V at that
        position's slot; every step's metadata goes to the device in one copy
        and all proposals come back in one."""
        assert self.eagle3_model is not None
        k = self.speculative_config.num_speculative_tokens
        limits = [min(k, seq.max_tokens - seq.num_completion_tokens) for seq in seqs]
        steps = max(limits, default=0)
        if steps <= 0:
            return [[] for _ in seqs]
        lens = [len(seq) for seq in seqs]
        pos, slots, ctx_lens = self._draft_step_metadata(seqs, limits, steps)
        rows = self._state_rows(seqs)
        bs = bucket_for(len(seqs))
        if self._use_graphs() and steps == k and bs is not None:
            graph = self._propose_graphs.get(bs)
            if graph is None:
                graph = self._propose_graphs[bs] = ProposeGraph(self, bs, k)
            # columns longest sequence first (the attention's work order)
            order = sorted(range(len(seqs)), key=lambda i: -lens[i])
            dseqs = [seqs[i] for i in order]
            tokens = graph.run([rows[i] for i in order], pos[:, order], slots[:, order],
                               ctx_lens[:, order], [seq.block_table for seq in dseqs])
            if self.draft_override is not None:
                self.draft_override(dseqs, tokens)
            sorted_table = tokens[:, :len(seqs)].cpu().tolist()
            table = [[0] * len(seqs) for _ in range(k)]
            for p, i in enumerate(order):
                for s_ in range(k):
                    table[s_][i] = sorted_table[s_][p]
        else:
            state_rows = _pinned(rows, torch.int64).to(self.device, non_blocking=True)
            table = self._propose_eager(seqs, state_rows, steps, pos, slots, ctx_lens, lens)
        return [[table[s][i] for s in range(limits[i])] for i in range(len(seqs))]

    def _propose_eager(self, seqs, state_rows, steps, pos, slots, ctx_lens, lens,
                       sync_each_step: bool = False):
        try:
            hidden = self.state_hidden.index_select(0, state_rows)
            feedback = self.state_feedback.index_select(0, state_rows)
            tokens = [self.eagle3_model.sample_greedy(hidden)]
            if sync_each_step:
                tokens[-1].tolist()
            if steps > 1:
                pos_d = _pinned(pos, torch.int64).to(self.device, non_blocking=True)
                slot_d = _pinned(slots, torch.int32).to(self.device, non_blocking=True)
                ctx_d = _pinned(ctx_lens, torch.int32).to(self.device, non_blocking=True)
                block_tables = self.prepare_block_tables(seqs)
                for s in range(steps - 1):
                    set_context(False, slot_mapping=slot_d[s], context_lens=ctx_d[s],
                                block_tables=block_tables, max_seqlen_k=max(lens) + s)
                    hidden, feedback = self.eagle3_model.forward_with_cache(tokens[-1], pos_d[s],
                                                                            feedback)
                    tokens.append(self.eagle3_model.sample_greedy(hidden))
                    if sync_each_step:
                        tokens[-1].tolist()
            stacked = torch.stack(tokens)
            if self.draft_override is not None:
                self.draft_override(seqs, stacked)
            return stacked.cpu().tolist()
        finally:
            reset_context()

    # ------------------------------------------------------------ reference-structured step
    # The reference's step structure (model_runner.py:1047-1078, 1127-1156,
    # 1159-1249) on this build's kernels, for comparison runs: a host sync
    # after every draft step, one argmax and one device->host copy per
    # sequence in verify, and one single-token draft forward per committed
    # token.  The engine's own step does not use these.

    @torch.inference_mode()
    def propose_eagle3_batch_reference(self, seqs: list[Sequence]) -> list[list[int]]:
        k = self.speculative_config.num_speculative_tokens
        limits = [min(k, seq.max_tokens - seq.num_completion_tokens) for seq in seqs]
        steps = max(limits, default=0)
        if steps <= 0:
            return [[] for _ in seqs]
        lens = [len(seq) for seq in seqs]
        pos, slots, ctx_lens = self._draft_step_metadata(seqs, limits, steps)
        state_rows = _pinned(self._state_rows(seqs), torch.int64).to(self.device, non_blocking=True)
        table = self._propose_eager(seqs, state_rows, steps, pos, slots, ctx_lens, lens,
                                    sync_each_step=True)
        return [[table[s][i] for s in range(limits[i])] for i in range(len(seqs))]

    @torch.inference_mode()
    def verify_eagle3_batch_reference(self, seqs: list[Sequence], num_input_tokens: list[int]):
        try:
            for seq, n in zip(seqs, num_input_tokens):
                seq.num_scheduled_tokens = n
            input_ids, positions = self.prepare_prefill(seqs)
            hidden, aux = self.model.forward_with_aux_hidden_states(
                input_ids, positions, self.speculative_config.aux_hidden_state_layers)
            logits = self.model.compute_all_logits(hidden)
            _, cu = self._host_prefill
            full = aux_concat(aux)
            targets = [logits[cu[i]:cu[i + 1]].argmax(dim=-1).tolist() for i in range(len(seqs))]
            return targets, [full[cu[i]:cu[i + 1]] for i in range(len(seqs))]
        finally:
            for seq in seqs:
                seq.num_scheduled_tokens = 0
            reset_context()

    @torch.inference_mode()
    def commit_eagle3_serial(self, seq: Sequence, output_tokens: list[int],
                             target_aux_hidden_states: torch.Tensor, start_position: int) -> None:
        if not output_tokens or seq.is_finished:
            return
        combined = self.eagle3_model.combine_hidden_states(
            target_aux_hidden_states[:len(output_tokens)])
        for i, tok in enumerate(output_tokens):
            self._draft_commit([seq], [[tok]], [start_position + i], combined[i:i + 1])

    @torch.inference_mode()
    def verify_eagle3_batch_fused(self, seqs: list[Sequence], num_input_tokens: list[int]):
        """Target forward over [previous token, drafts] of every sequence, then
        the fused argmax + accept kernel.  Returns host lists
        (target_tokens per sequence, accept_len, bonus) in the caller's
        order; the aux hidden-state pairs stay on the device for
        ``commit_eagle3_batch``.

        The forward runs the batch longest sequence first: the verify
        attention hands its workgroups out in batch order, and longest-first
        lets every CU pair a long key range with a shorter one (measured on
        the Qwen3-8B verify shape: 69.6 -> 61.3 us per attention call)."""
        if len(seqs) != len(num_input_tokens):
            raise ValueError("EAGLE3 verification metadata does not match requests")
        order = sorted(range(len(seqs)), key=lambda i: -len(seqs[i]))
        targets, acc, bonus = self._verify_fused([seqs[i] for i in order],
                                                 [num_input_tokens[i] for i in order])
        out_t, out_a, out_b = [None] * len(seqs), [0] * len(seqs), [0] * len(seqs)
        for pos, i in enumerate(order):
            out_t[i], out_a[i], out_b[i] = targets[pos], acc[pos], bonus[pos]
        return out_t, out_a, out_b

    @torch.inference_mode()
    def propose_verify_eagle3_batch(self, seqs: list[Sequence], prelaunch: bool = False):
        """Proposals and verification in one pass over the stream: the draft
        graph runs, its tokens are copied to the host, and the verify graph
        is enqueued behind them with its input ids composed on the device
        (previous token, then the k proposals of each sequence), so the
        target forward runs while the host records the proposals.  Returns
        the proposals (as propose_eagle3_batch) and leaves the verify in
        flight for collect_verify_eagle3_batch; returns None when the graphs
        do not cover the step (no bucket, or graphs off), and the caller then
        proposes and verifies in turn.  The block tables must not change in
        between (the drafts' blocks are reserved before proposing, as in the
        reference).

        A sequence close to its budget proposes only min(k, max_tokens -
        completion) tokens (model_runner.py:1169-1176); the graphs still run
        k draft steps and k + 1 verify rows for it.  Its draft steps past its
        own limit write no K/V (slot -1), the verify rows past it are
        ignored (row j's target depends on the tokens up to j only), and
        collect_verify_eagle3_batch caps its accepted count at the limit.

        prelaunch: also queue the next step's draft (ChainedProposeGraph)
        behind this step's verify and device commit, so that it runs while
        the host works through the results; the caller has reserved pages
        for it (Scheduler.reserve_lookahead).  The next call uses those
        proposals if its batch and lengths are the ones the results imply,
        and drafts again otherwise."""
        assert self.eagle3_model is not None
        k = self.speculative_config.num_speculative_tokens
        b = len(seqs)
        bs = bucket_for(b)
        pre, self._prelaunched = self._prelaunched, None
        if (not self.pipeline_verify or not self._use_graphs() or not self.use_verify_graph
                or self.keep_verify_inputs or bs is None or k < 1 or b == 0):
            return None
        limits = [min(k, seq.max_tokens - seq.num_completion_tokens) for seq in seqs]
        if min(limits) < 1:
            return None
        lens = [len(seq) for seq in seqs]
        vgraph = self._verify_graphs.get(bs)
        if vgraph is None:
            vgraph = self._verify_graphs[bs] = VerifyGraph(self, bs, k + 1)
        # the verify batch runs longest sequence first (verify_eagle3_batch_fused),
        # and so does a fresh draft's: col[i] is sequence i's draft column
        order = sorted(range(b), key=lambda i: -lens[i])
        tokens = None
        if pre is not None:
            graph, col_ids, _, col_lens_after = pre
            col_of = {sid: p for p, sid in enumerate(col_ids)}
            col = [col_of.get(seq.seq_id, -1) for seq in seqs]
            if (graph.bs == bs and len(col_ids) == b and min(col) >= 0
                    and all(col_lens_after[c] == n for c, n in zip(col, lens))):
                tokens = graph.tokens
                self.prelaunch_stats["used"] += 1
        if tokens is None:
            col = [0] * b
            for p, i in enumerate(order):
                col[i] = p
            dseqs = [seqs[i] for i in order]
            pos, slots, ctx_lens = self._draft_step_metadata(dseqs, [limits[i] for i in order], k)
            pgraph = self._propose_graphs.get(bs)
            if pgraph is None:
                pgraph = self._propose_graphs[bs] = ProposeGraph(self, bs, k)
            tokens = pgraph.run(self._state_rows(dseqs), pos, slots, ctx_lens,
                                [seq.block_table for seq in dseqs])
        if self.draft_override is not None:
            by_col = [None] * b
            for i, c in enumerate(col):
                by_col[c] = seqs[i]
            self.draft_override(by_col, tokens)
        if self._proposal_host.numel() < k * bs:
            self._proposal_host = torch.empty(k * bs, dtype=torch.int64, pin_memory=True)
        host = self._proposal_host[:k * bs]
        host.copy_(tokens.reshape(-1), non_blocking=True)
        proposed = torch.cuda.Event()
        proposed.record()
        # the verify's input ids are composed inside the graph from the proposals
        q = k + 1
        vgraph.run_composed([seqs[i].token_ids[-1] for i in order], [col[i] for i in order],
                            [lens[i] - 1 for i in order], [q] * b,
                            [seqs[i].block_table for i in order])
        t_pad = vgraph.T
        self._verify_host[:t_pad + 2 * bs].copy_(vgraph.out, non_blocking=True)
        verified = torch.cuda.Event()
        verified.record()
        self._device_committed = None
        if self.device_commit:
            # the draft commit follows on the device while the host works
            # through the results (commit_eagle3_batch then has nothing to do)
            cgraph = self._device_commit_graphs.get(bs)
            if cgraph is None:
                cgraph = self._device_commit_graphs[bs] = DeviceCommitGraph(self, vgraph)
            state_rows = self._state_rows(seqs)
            cgraph.run([state_rows[i] for i in order])
            self._device_committed = vgraph
            if prelaunch:
                # the next step's draft, its columns in this verify's order
                # (longest first), column p reading verify row p's results
                chained = self._chained_graphs.get(bs)
                if chained is None:
                    chained = self._chained_graphs[bs] = ChainedProposeGraph(self, bs, k, vgraph)
                chained.launch([state_rows[i] for i in order], [lens[i] for i in order],
                               list(range(b)), [seqs[i].block_table for i in order])
                self._prelaunched = (chained, [seqs[i].seq_id for i in order],
                                     [lens[i] for i in order], None)
                self.prelaunch_stats["queued"] += 1
        self._inflight_verify = (order, vgraph, verified, [seqs[i].seq_id for i in range(b)],
                                 limits)
        self.pipeline_stats["steps"] += 1
        self.pipeline_stats["ragged"] += min(limits) < k
        proposed.synchronize()
        table = host.view(k, bs)[:, :b].tolist()
        return [[table[s][col[i]] for s in range(limits[i])] for i in range(b)]

    @torch.inference_mode()
    def collect_verify_eagle3_batch(self, seqs: list[Sequence], num_input_tokens: list[int]):
        """Results of the verify propose_verify_eagle3_batch enqueued, in the
        form of verify_eagle3_batch_fused (the same sequences, in the same
        order, each verifying its k proposals)."""
        if self._inflight_verify is None:
            raise RuntimeError("collect_verify_eagle3_batch needs propose_verify_eagle3_batch first")
        order, vgraph, verified, ids, limits = self._inflight_verify
        self._inflight_verify = None
        b = len(seqs)
        if [seq.seq_id for seq in seqs] != ids or \
                list(num_input_tokens) != [n + 1 for n in limits]:
            raise RuntimeError("EAGLE3 verification metadata does not match the proposed batch")
        verified.synchronize()
        bs, q, t_pad = vgraph.bs, vgraph.q, vgraph.T
        res = self._verify_host[:t_pad + 2 * bs].tolist()
        cu = [i * q for i in range(b + 1)]
        out_t, out_a, out_b = [None] * b, [0] * b, [0] * b
        for p, i in enumerate(order):
            # the first limit + 1 rows are the sequence's verify window; the
            # scan over all k drafts is capped at its limit (a sequence whose
            # cap bites reaches its budget this step)
            n = limits[i]
            out_t[i] = res[cu[p]:cu[p] + n + 1]
            a = res[t_pad + p]
            if a > n:
                out_a[i], out_b[i] = n, out_t[i][n]
            else:
                out_a[i], out_b[i] = a, res[t_pad + bs + p]
        self._pending_verify = (vgraph.aux, cu, {seqs[i].seq_id: p for p, i in enumerate(order)})
        self._pending_graph = vgraph
        if self._prelaunched is not None:
            # the lengths the queued draft assumed, per column (column p is
            # verify row p, sequence order[p]): len + accepted + 1
            graph, col_ids, col_lens, _ = self._prelaunched
            self._prelaunched = (graph, col_ids, col_lens,
                                 [n + out_a[i] + 1 for n, i in zip(col_lens, order)])
        return out_t, out_a, out_b

    def _verify_fused(self, seqs: list[Sequence], num_input_tokens: list[int]):
        k = self.speculative_config.num_speculative_tokens
        b = len(seqs)
        bs = bucket_for(b)
        self._device_committed = None
        try:
            for seq, n in zip(seqs, num_input_tokens):
                seq.num_scheduled_tokens = n
            if (self._use_graphs() and self.use_verify_graph and bs is not None
                    and not self.keep_verify_inputs
                    and all(n == k + 1 for n in num_input_tokens)):
                ids, starts, qlens, cu = [], [], [], [0]
                for seq in seqs:
                    start = seq.num_computed_tokens
                    end = min(start + seq.num_scheduled_tokens, seq.num_tokens)
                    ids.extend(seq.token_ids[start:end])
                    starts.append(start)
                    qlens.append(end - start)
                    cu.append(cu[-1] + end - start)
                graph = self._verify_graphs.get(bs)
                if graph is None:
                    graph = self._verify_graphs[bs] = VerifyGraph(self, bs, k + 1)
                graph.run(ids, starts, qlens, [seq.block_table for seq in seqs])
                t_pad = graph.T
                self._verify_host[:t_pad + 2 * bs].copy_(graph.out, non_blocking=True)
                torch.cuda.current_stream().synchronize()
                res = self._verify_host[:t_pad + 2 * bs].tolist()
                argmax = res[:cu[-1]]
                acc = res[t_pad:t_pad + b]
                bonus = res[t_pad + bs:t_pad + bs + b]
                aux = graph.aux
                self._pending_graph = graph
            else:
                input_ids, positions = self.prepare_prefill(seqs)
                ctx = get_context()
                hidden, aux = self.model.forward_with_aux_hidden_states(
                    input_ids, positions, self.speculative_config.aux_hidden_state_layers)
                logits = self.model.compute_all_logits(hidden)
                t = logits.shape[0]
                n = t + 2 * b
                if n > self._verify_dev.numel():
                    self._verify_dev = torch.empty(2 * n, dtype=torch.int32, device=self.device)
                    self._verify_host = torch.empty(2 * n, dtype=torch.int32, pin_memory=True)
                K.argmax_accept(logits, ctx.cu_seqlens_q, input_ids, out=self._verify_dev[:n])
                self._verify_host[:n].copy_(self._verify_dev[:n], non_blocking=True)
                torch.cuda.current_stream().synchronize()
                res = self._verify_host[:n].tolist()
                _, cu = self._host_prefill
                if self.keep_verify_inputs:
                    self.last_verify_inputs = (logits, list(cu), input_ids)
                argmax, acc, bonus = res[:t], res[t:t + b], res[t + b:n]
                self._pending_graph = None
            targets = [argmax[cu[i]:cu[i + 1]] for i in range(b)]
            self._pending_verify = (aux, cu, {seq.seq_id: i for i, seq in enumerate(seqs)})
            return targets, acc, bonus
        finally:
            for seq in seqs:
                seq.num_scheduled_tokens = 0
            reset_context()

    @torch.inference_mode()
    def verify_eagle3_batch(self, seqs: list[Sequence], num_input_tokens: list[int]):
        """Reference-shaped result (model_runner.py:1047-1078): per-sequence
        target argmax lists and aux hidden-state rows [q_i, 3H]."""
        targets, _, _ = self.verify_eagle3_batch_fused(seqs, num_input_tokens)
        aux, cu, index = self._pending_verify
        full = aux_concat(aux)
        rows = [index[seq.seq_id] for seq in seqs]
        return targets, [full[cu[i]:cu[i + 1]] for i in rows]

    @torch.inference_mode()
    def commit_eagle3_batch(self, seqs: list[Sequence], output_tokens: list[list[int]],
                            start_positions: list[int]) -> None:
        """Replay every sequence's committed tail into the draft cache in one
        ragged forward.  Sequence i's verify rows cu[i] .. cu[i] + n_i - 1 hold
        the aux states of positions start_i .. start_i + n_i - 1, paired with
        its committed tokens (model_runner.py:1216-1249 does this one token
        and one sequence at a time)."""
        if self._pending_verify is None:
            raise RuntimeError("commit_eagle3_batch needs a preceding verify")
        if self._device_committed is not None and self._device_committed is self._pending_graph:
            # DeviceCommitGraph already replayed every tail of this verify
            self._device_committed = None
            return
        aux, cu, index = self._pending_verify
        rows = []
        for seq, toks in zip(seqs, output_tokens):
            i = index[seq.seq_id]
            if len(toks) > cu[i + 1] - cu[i]:
                raise RuntimeError("committed tail longer than the verify window")
            rows.extend(range(cu[i], cu[i] + len(toks)))
        if not rows:
            return
        lens = {len(t) for t in output_tokens}
        graph = self._pending_graph
        if graph is not None and len(lens) == 1 and len(seqs) <= graph.bs:
            n = lens.pop()
            key = (graph.bs, n)
            cg = self._commit_graphs.get(key)
            if cg is None:
                cg = self._commit_graphs[key] = CommitGraph(self, graph, n)
            ids, pos, slots, cq, ck = [], [], [], [0], [0]
            for seq, toks, start in zip(seqs, output_tokens, start_positions):
                ids.extend(toks)
                pos.extend(range(start, start + n))
                slots.extend(self._slot(seq, p) for p in range(start, start + n))
                cq.append(cq[-1] + n)
                ck.append(ck[-1] + start + n)
            cg.run(rows, ids, pos, cq, ck, slots, [seq.block_table for seq in seqs])
            self._store_states(seqs, cg.hidden, cg.feedback, [cq[i + 1] - 1 for i in range(len(seqs))])
            return
        rows_d = _pinned(rows, torch.int32).to(self.device, non_blocking=True)
        combined = self.eagle3_model.combine_hidden_states(aux_concat(aux, rows_d))
        self._draft_commit(seqs, output_tokens, start_positions, combined)

    @torch.inference_mode()
    def commit_eagle3(self, seq: Sequence, output_tokens: list[int],
                      target_aux_hidden_states: torch.Tensor, start_position: int) -> None:
        """Single-sequence form of the reference (model_runner.py:1216-1249)."""
        if not output_tokens or seq.is_finished:
            return
        combined = self.eagle3_model.combine_hidden_states(
            target_aux_hidden_states[:len(output_tokens)])
        self._draft_commit([seq], [output_tokens], [start_position], combined)

    def _draft_commit(self, seqs, output_tokens, start_positions, combined) -> None:
        ids, pos, slots = [], [], []
        cu_q, cu_k = [0], [0]
        for seq, toks, start in zip(seqs, output_tokens, start_positions):
            n = len(toks)
            ids.extend(toks)
            pos.extend(range(start, start + n))
            slots.extend(self._slot(seq, p) for p in range(start, start + n))
            cu_q.append(cu_q[-1] + n)
            cu_k.append(cu_k[-1] + start + n)
        dev = self.device
        try:
            set_context(True, _pinned(cu_q, torch.int32).to(dev, non_blocking=True),
                        _pinned(cu_k, torch.int32).to(dev, non_blocking=True),
                        max(len(t) for t in output_tokens),
                        max(s + len(t) for s, t in zip(start_positions, output_tokens)),
                        _pinned(slots, torch.int32).to(dev, non_blocking=True), None,
                        self.prepare_block_tables(seqs))
            hidden, feedback = self.eagle3_model.forward_with_cache(
                _pinned(ids, torch.int64).to(dev, non_blocking=True),
                _pinned(pos, torch.int64).to(dev, non_blocking=True), combined)
            self._store_states(seqs, hidden, feedback, [cu_q[i + 1] - 1 for i in range(len(seqs))])
        finally:
            reset_context()

    def release_eagle3_state(self, seq_id: int) -> None:
        r = self._state_slot.pop(seq_id, None)
        if r is not None:
            self._free_state.append(r)

    @torch.inference_mode()
    def run_eagle3_graph(self, input_ids, positions, feedback, seqs):
        """Replay the captured draft step of the smallest batch bucket >= len(seqs)
        after copying inputs and the current paged metadata into its static
        buffers (model_runner.py:1526-1548)."""
        bs = len(seqs)
        graph_bs = next(size for size in sorted(self.eagle_graphs) if size >= bs)
        graph = self.eagle_graphs[graph_bs]
        v = self.eagle_graph_vars[graph_bs]
        v["input_ids"].zero_()
        v["positions"].zero_()
        v["feedback"].zero_()
        v["slot_mapping"].fill_(-1)
        v["context_lens"].fill_(1)
        v["block_tables"].zero_()
        v["input_ids"][:bs].copy_(input_ids)
        v["positions"][:bs].copy_(positions)
        v["feedback"][:bs].copy_(feedback)
        ctx = get_context()
        v["slot_mapping"][:bs].copy_(ctx.slot_mapping)
        v["context_lens"][:bs].copy_(ctx.context_lens)
        v["block_tables"][:bs, :ctx.block_tables.size(1)].copy_(ctx.block_tables)
        graph.replay()
        hidden, next_feedback = v["outputs"]
        return hidden[:bs], next_feedback[:bs]

    # ------------------------------------------------------------ diagnostics

    def get_diagnostics(self):
        return {
            "device": str(self.device),
            "parameter_bytes": param_bytes(self.model),
            "draft_parameter_bytes": param_bytes(self.eagle3_model) if self.eagle3_model else 0,
            "kv_cache_dtype": str(self.kv_cache.dtype),
            "kv_cache_blocks": self.kv_cache.size(2),
            "kv_cache_bytes": self.kv_cache.numel() * self.kv_cache.element_size(),
            "decode_graph_replay_count": self.decode_graph_replay_count,
            "eagle3_runtime": self.get_eagle3_runtime_capabilities(),
        }
