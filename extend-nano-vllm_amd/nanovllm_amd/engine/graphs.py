"""HIP-graph captures of the three device stages of a speculative step.

Each graph is captured once per padded batch size (bucket) -- every bucket
up to max_num_seqs when the runner is built, any other on first use -- and
replayed with its static metadata buffers refreshed by one host->device copy
per dtype.  Padded sequences have slot -1 (no K/V write) and block id -1 (no
K/V read), so they cost compute but touch no cache state.  Sequences close
to their token budget propose fewer drafts; the graphs still run k draft
steps and k + 1 verify rows for them, with slot -1 past their own limit.
Steps the graphs do not cover (no bucket, graphs off, ragged commits off the
device-commit path) run eagerly; results are identical either way.

  VerifyGraph   target forward over q = k+1 rows per sequence, all-row LM
                head, fused argmax + accept      (model_runner.py:1047-1078)
  ProposeGraph  k greedy draft tokens: sample, then k-1 draft decode steps
                                                  (model_runner.py:1159-1213)
  CommitGraph   draft replay of n committed tokens per sequence, aux rows
                gathered from the VerifyGraph's static aux states
                                                  (model_runner.py:1216-1249)
  DeviceCommitGraph
                the same replay with every sequence's committed tail read
                from the VerifyGraph's own accept results on the device, so
                it can run right behind the verify, before the host has
                seen the results
"""
from __future__ import annotations

import gc
import itertools
import sys

import numpy as np
import torch

from nanovllm_amd import kernels as K
from nanovllm_amd.context import reset_context, set_context
from nanovllm_amd.qwen3 import aux_concat

BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 192, 256, 384, 512)


def bucket_for(n: int) -> int | None:
    for b in BUCKETS:
        if b >= n:
            return b
    return None


def block_table_array(rows, nrows: int | None = None,
                      width: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Block-table rows as one int32 array [nrows, width], each row padded
    with -1 (and -1 rows past len(rows)), plus the rows' lengths.  width
    defaults to the longest row (at least 1); a longer row raises
    ValueError.  Built from one flat pass over the ids: the per-step graph
    metadata of a 64-sequence batch took ~50 us as nested Python lists."""
    n = len(rows)
    lens = np.fromiter((len(r) for r in rows), dtype=np.int64, count=n)
    longest = int(lens.max()) if n else 0
    width = max(longest, 1) if width is None else width
    if longest > width:
        raise ValueError(f"a block table of {longest} blocks exceeds the width {width}")
    out = np.full((n if nrows is None else nrows, width), -1, dtype=np.int32)
    total = int(lens.sum())
    if total:
        flat = np.fromiter(itertools.chain.from_iterable(rows), dtype=np.int32, count=total)
        out[:n][np.arange(width)[None, :] < lens[:, None]] = flat
    return out, lens


class _Staging:
    """A device buffer plus a pinned host twin of the same dtype; fields are
    contiguous slices of both.

    upload() only queues the copy: the DMA reads the pinned buffer when the
    stream reaches it, which for the graphs queued behind a verify (the
    device commit, the next step's draft) can be after the host has started
    the next step.  So upload() records an event behind its copy, and the
    first fill() after it waits for that event before writing: a queued
    copy never reads values meant for the next one.  The wait precedes
    waits the host makes anyway (each step reads the proposals that the
    queued graphs produce after their copies), so it costs no step time."""

    def __init__(self, sizes: dict[str, int], dtype: torch.dtype, device: torch.device):
        total = sum(sizes.values())
        self.host = torch.zeros(max(total, 1), dtype=dtype, pin_memory=True)
        # fields are written through a numpy view of the pinned buffer: a
        # torch tensor built from a list plus a copy_ per field cost the
        # host ~30 us each, on the path between two verify graphs
        self.host_np = self.host.numpy()
        self.dev = torch.zeros(max(total, 1), dtype=dtype, device=device)
        self.fields: dict[str, tuple[int, int]] = {}
        off = 0
        for name, n in sizes.items():
            self.fields[name] = (off, n)
            off += n
        self.total = total
        self._copied = torch.cuda.Event()
        self._in_flight = False
        self.waits = 0      # fills that found the previous copy still queued

    def dev_view(self, name: str) -> torch.Tensor:
        off, n = self.fields[name]
        return self.dev[off:off + n]

    def _writable(self) -> None:
        if self._in_flight:
            if not self._copied.query():
                self.waits += 1
                self._copied.synchronize()
            self._in_flight = False

    def fill(self, name: str, values) -> None:
        off, n = self.fields[name]
        a = np.asarray(values, dtype=self.host_np.dtype).reshape(-1)
        if a.size != n:
            raise ValueError(f"{name}: {a.size} values for {n} slots")
        self._writable()
        self.host_np[off:off + n] = a

    def upload(self) -> None:
        self._writable()
        self.dev[:self.total].copy_(self.host[:self.total], non_blocking=True)
        self._copied.record()
        self._in_flight = True


class _GraphBase:

    def __init__(self, runner):
        self.runner = runner
        self.device = runner.device
        self.graph = torch.cuda.CUDAGraph()

    def _capture(self, body) -> None:
        """Eager run (allocates workspaces, compiles nothing), then capture.

        The capture begins outside inference mode: the first capture of a
        process registers torch's CUDA generator and allocates its graph-safe
        seed/offset tensors.  Allocated under inference mode they would be
        inference tensors, and every later capture outside inference mode
        (the caller's own graphs) would fail on their in-place update.

        Python's cyclic garbage collector is off during the capture: a
        collection there can free objects of an engine that is gone (pinned
        host buffers, graphs), and their release is not allowed while the
        stream captures."""
        body()
        torch.cuda.synchronize(self.device)
        ctx = torch.cuda.graph(self.graph, pool=self.runner.graph_pool)
        with torch.inference_mode(False):
            ctx.__enter__()
        collecting = gc.isenabled()
        gc.disable()
        try:
            body()
        except BaseException:
            if collecting:
                gc.enable()
            ctx.__exit__(*sys.exc_info())
            raise
        if collecting:
            gc.enable()
        ctx.__exit__(None, None, None)
        if self.runner.graph_pool is None:
            self.runner.graph_pool = self.graph.pool()
        torch.cuda.synchronize(self.device)


class VerifyGraph(_GraphBase):
    """The host uploads per-sequence first positions and query lengths, the
    block tables and either the input ids (run) or each sequence's last
    token and column in the draft's proposals (run_composed: the ids are
    composed inside the graph, nva_verify_input_ids, from the bucket's
    proposal buffer that every draft graph writes); positions, slot
    mapping and cu_seqlens are derived on the device inside the graph
    (nva_verify_metadata)."""

    def __init__(self, runner, bs: int, q: int):
        super().__init__(runner)
        self.bs, self.q, self.T = bs, q, bs * q
        T = self.T
        self.max_blocks = runner.max_blocks_per_seq
        self.i64 = _Staging({"ids": T}, torch.int64, self.device)
        self.i32 = _Staging({"compose": 1, "last": bs, "order": bs, "start": bs, "qlen": bs,
                             "bt": bs * self.max_blocks}, torch.int32, self.device)
        self.proposals = runner.proposal_buffer(bs)
        if self.proposals.shape[0] != q - 1:
            raise ValueError(f"verify rows per sequence ({q}) must be the proposals ({self.proposals.shape[0]}) + 1")
        self.pos = torch.zeros(T, dtype=torch.int64, device=self.device)
        self.slots = torch.zeros(T, dtype=torch.int32, device=self.device)
        self.cu_q = torch.zeros(bs + 1, dtype=torch.int32, device=self.device)
        self.cu_k = torch.zeros(bs + 1, dtype=torch.int32, device=self.device)
        self.out = torch.zeros(T + 2 * bs, dtype=torch.int32, device=self.device)
        self.aux = None
        # valid dummy metadata for the capture run
        self._fill_dummy()
        self._capture(self._body)

    def _fill_dummy(self):
        bs, q = self.bs, self.q
        self.i64.fill("ids", [0] * self.T)
        self.i32.fill("compose", [0])
        self.i32.fill("last", [0] * bs)
        self.i32.fill("order", [-1] * bs)
        self.i32.fill("start", [0] * bs)
        self.i32.fill("qlen", [q] * bs)
        self.i32.fill("bt", [-1] * (bs * self.max_blocks))
        self.i64.upload()
        self.i32.upload()

    def _body(self):
        r = self.runner
        ids = self.i64.dev_view("ids")
        bt = self.i32.dev_view("bt").view(self.bs, self.max_blocks)
        K.verify_input_ids(self.i32.dev_view("compose"), self.i32.dev_view("last"),
                           self.i32.dev_view("order"), self.proposals, self.q, ids)
        K.verify_metadata(self.i32.dev_view("start"), self.i32.dev_view("qlen"), bt,
                          r.block_size, self.T, self.cu_q, self.cu_k, self.pos, self.slots)
        set_context(True, self.cu_q, self.cu_k, self.q, r.max_seqlen_k, self.slots, None, bt)
        try:
            hidden, aux = r.model.forward_with_aux_hidden_states(
                ids, self.pos, r.speculative_config.aux_hidden_state_layers)
            logits = r.model.compute_all_logits(hidden)
            K.argmax_accept(logits, self.cu_q, ids, out=self.out)
            self.aux = aux
        finally:
            reset_context()

    def run(self, ids, starts, qlens, bt_rows) -> None:
        """Host lists for the real sequences (token ids, first position and
        query length per sequence, block tables); the rest of the bucket is
        padding: q rows at positions 0.. with no cache blocks."""
        n = len(ids)
        self.i64.fill("ids", list(ids) + [0] * (self.T - n))
        self.i64.upload()
        self.i32.fill("compose", [0])
        self._run_staged(starts, qlens, bt_rows)

    def run_composed(self, last_tokens, columns, starts, qlens, bt_rows) -> None:
        """As run(), for sequences that verify the bucket's proposals in
        full (q = k + 1 rows each): row p's ids are last_tokens[p] and then
        the proposals of draft column columns[p], composed inside the graph
        from whatever the draft graphs last wrote to the proposal buffer."""
        bs = self.bs
        b = len(columns)
        if b > bs or any(not 0 <= c < bs for c in columns) or any(n != self.q for n in qlens):
            raise ValueError("composed verify rows need draft columns within the bucket and q rows")
        self.i32.fill("compose", [1])
        self.i32.fill("last", list(last_tokens) + [0] * (bs - b))
        self.i32.fill("order", list(columns) + [-1] * (bs - b))
        self._run_staged(starts, qlens, bt_rows)

    def _run_staged(self, starts, qlens, bt_rows) -> None:
        bs, q = self.bs, self.q
        b = len(starts)
        self.i32.fill("start", list(starts) + [0] * (bs - b))
        self.i32.fill("qlen", list(qlens) + [q] * (bs - b))
        self.i32.fill("bt", block_table_array(bt_rows, bs, self.max_blocks)[0])
        self.i32.upload()
        self.graph.replay()


class ProposeGraph(_GraphBase):

    def __init__(self, runner, bs: int, k: int):
        super().__init__(runner)
        self.bs, self.k = bs, k
        r = runner
        h = r.eagle3_model.config.hidden_size
        self.max_blocks = r.max_blocks_per_seq
        steps = max(k - 1, 1)
        self.hidden = torch.zeros(bs, h, dtype=r.dtype, device=self.device)
        self.feedback = torch.zeros(bs, h, dtype=r.dtype, device=self.device)
        self.tokens = r.proposal_buffer(bs)
        if self.tokens.shape[0] != k:
            raise ValueError(f"draft steps ({k}) must match the proposal buffer ({self.tokens.shape[0]})")
        # the draft-state rows of the batch (gathered inside the graph) and
        # the draft steps' metadata, one host->device copy per dtype
        self.i64 = _Staging({"state": bs, "pos": steps * bs}, torch.int64, self.device)
        self.i32 = _Staging({"slots": steps * bs, "ctx": steps * bs, "bt": bs * self.max_blocks},
                            torch.int32, self.device)
        self.i64.fill("state", [0] * bs)
        self.i64.fill("pos", [0] * (steps * bs))
        self.i32.fill("slots", [-1] * (steps * bs))
        self.i32.fill("ctx", [1] * (steps * bs))
        self.i32.fill("bt", [-1] * (bs * self.max_blocks))
        self.i64.upload()
        self.i32.upload()
        self._capture(self._body)

    def _body(self):
        bs = self.bs
        self._draft_loop(self.i64.dev_view("state"), self.i64.dev_view("pos").view(-1, bs),
                         self.i32.dev_view("slots").view(-1, bs),
                         self.i32.dev_view("ctx").view(-1, bs),
                         self.i32.dev_view("bt").view(bs, self.max_blocks))

    def _draft_loop(self, state, pos, slots, ctx, bt):
        r = self.runner
        draft = r.eagle3_model
        torch.index_select(r.state_hidden, 0, state, out=self.hidden)
        torch.index_select(r.state_feedback, 0, state, out=self.feedback)
        draft.sample_greedy(self.hidden, out=self.tokens[0])
        feedback = self.feedback
        try:
            for s in range(self.k - 1):
                set_context(False, slot_mapping=slots[s], context_lens=ctx[s], block_tables=bt,
                            max_seqlen_k=r.max_seqlen_k)
                hidden, feedback = draft.forward_with_cache(self.tokens[s], pos[s], feedback)
                draft.sample_greedy(hidden, out=self.tokens[s + 1])
        finally:
            reset_context()

    def run(self, state_rows, pos, slots, ctx, bt_rows) -> torch.Tensor:
        """state_rows: host list of the sequences' rows in the runner's
        draft-state table (the padding rows read row 0 and are discarded).
        pos/slots/ctx: host [k-1][b] (arrays or nested lists).  Returns tokens
        [k, bs] (device)."""
        b = len(state_rows)
        bs = self.bs
        self.i64.fill("state", list(state_rows) + [0] * (bs - b))

        def padded(values, dtype, fill):
            a = np.asarray(values, dtype=dtype).reshape(-1, b)
            out = np.full((a.shape[0], bs), fill, dtype=dtype)
            out[:, :b] = a
            return out

        self.i64.fill("pos", padded(pos, np.int64, 0))
        self.i32.fill("slots", padded(slots, np.int32, -1))
        self.i32.fill("ctx", padded(ctx, np.int32, 1))
        self.i32.fill("bt", block_table_array(bt_rows, bs, self.max_blocks)[0])
        self.i64.upload()
        self.i32.upload()
        self.graph.replay()
        return self.tokens


class ChainedProposeGraph(ProposeGraph):
    """The next step's draft, queued right behind a VerifyGraph and its
    DeviceCommitGraph, before the host has read the results: each
    sequence's length after the step, len + accepted + 1, comes from the
    verify's accept results on the device, and with it the draft steps'
    positions, slots (through block tables the host reserved one step
    ahead) and context lengths.  The draft states it starts from are the
    ones the device commit just wrote.  The host checks the lengths once it
    has the results and drafts again if they differ (a sequence finished,
    or left the batch); positions this draft wrote K/V for are written
    again before anything reads them (model_runner.py:1159-1213)."""

    def __init__(self, runner, bs: int, k: int, vgraph: "VerifyGraph"):
        self.vgraph = vgraph
        super().__init__(runner, bs, k)

    def _body(self):
        r = self.runner
        bs, k, mb = self.bs, self.k, self.max_blocks
        steps = max(k - 1, 1)
        dev = self.device
        if not hasattr(self, "lens"):
            # static inputs (host copies, one entry per column) and outputs
            self.meta = _Staging({"state": bs, "lens": bs, "vrow": bs}, torch.int64, dev)
            self.meta32 = _Staging({"bt": bs * mb}, torch.int32, dev)
            self.meta.fill("state", [0] * bs)
            self.meta.fill("lens", [0] * bs)
            self.meta.fill("vrow", [0] * bs)
            self.meta32.fill("bt", [-1] * (bs * mb))
            self.meta.upload()
            self.meta32.upload()
            self.lens = self.meta.dev_view("lens")
            self.cpos = torch.zeros(steps, bs, dtype=torch.int64, device=dev)
            self.cslots = torch.zeros(steps, bs, dtype=torch.int32, device=dev)
            self.cctx = torch.zeros(steps, bs, dtype=torch.int32, device=dev)
        bt = self.meta32.dev_view("bt").view(bs, mb)
        v = self.vgraph
        # one launch: each column's length after the verified step (its
        # accepted count read from the verify's accept output), then every
        # draft step's position, slot and context; padding columns have an
        # empty block-table row, so their slots are -1
        K.draft_metadata(self.lens, self.meta.dev_view("vrow"), v.out[v.T:v.T + bs], bs, bt,
                         r.block_size, self.cpos, self.cslots, self.cctx)
        self._draft_loop(self.meta.dev_view("state"), self.cpos, self.cslots, self.cctx, bt)

    def launch(self, state_rows, lens, vrows, bt_rows) -> torch.Tensor:
        """Host lists, one entry per draft column (the engine passes the
        verify's order, longest sequence first, so the draft's attention
        works through its sequences in the order that balances best):
        draft-state rows, the lengths before the verified step, each
        column's row in the verify batch, block tables (reserved one step
        ahead).  Padding columns get length 0 (no K/V written).  Returns
        tokens [k, bs] (device)."""
        b, bs = len(state_rows), self.bs
        self.meta.fill("state", list(state_rows) + [0] * (bs - b))
        self.meta.fill("lens", list(lens) + [0] * (bs - b))
        self.meta.fill("vrow", list(vrows) + [0] * (bs - b))
        self.meta32.fill("bt", block_table_array(bt_rows, bs, self.max_blocks)[0])
        self.meta.upload()
        self.meta32.upload()
        self.graph.replay()
        return self.tokens


class CommitGraph(_GraphBase):
    """n committed tokens for each of bs sequences whose aux rows live in
    ``verify.aux`` (the verify graph of the same bucket)."""

    def __init__(self, runner, verify: VerifyGraph, n: int):
        super().__init__(runner)
        self.verify = verify
        self.bs, self.n = verify.bs, n
        R = self.bs * n
        self.R = R
        self.max_blocks = runner.max_blocks_per_seq
        self.i64 = _Staging({"ids": R, "pos": R}, torch.int64, self.device)
        self.i32 = _Staging({"rows": R, "cu_q": self.bs + 1, "cu_k": self.bs + 1, "slots": R,
                             "bt": self.bs * self.max_blocks}, torch.int32, self.device)
        self.i64.fill("ids", [0] * R)
        self.i64.fill("pos", [j for _ in range(self.bs) for j in range(n)])
        self.i32.fill("rows", [-1] * R)
        self.i32.fill("cu_q", [i * n for i in range(self.bs + 1)])
        self.i32.fill("cu_k", [i * n for i in range(self.bs + 1)])
        self.i32.fill("slots", [-1] * R)
        self.i32.fill("bt", [-1] * (self.bs * self.max_blocks))
        self.i64.upload()
        self.i32.upload()
        self.hidden = self.feedback = None
        self._capture(self._body)

    def _body(self):
        r = self.runner
        draft = r.eagle3_model
        combined = draft.combine_hidden_states(aux_concat(self.verify.aux,
                                                          self.i32.dev_view("rows")))
        set_context(True, self.i32.dev_view("cu_q"), self.i32.dev_view("cu_k"), self.n,
                    r.max_seqlen_k, self.i32.dev_view("slots"), None,
                    self.i32.dev_view("bt").view(self.bs, self.max_blocks))
        try:
            self.hidden, self.feedback = draft.forward_with_cache(
                self.i64.dev_view("ids"), self.i64.dev_view("pos"), combined)
        finally:
            reset_context()

    def run(self, rows, ids, pos, cu_q, cu_k, slots, bt_rows) -> None:
        R, bs, n = self.R, self.bs, self.n
        m = len(ids)
        b = len(cu_q) - 1
        self.i32.fill("rows", list(rows) + [-1] * (R - m))
        self.i64.fill("ids", list(ids) + [0] * (R - m))
        self.i64.fill("pos", list(pos) + [0] * (R - m))
        self.i32.fill("cu_q", list(cu_q) + [cu_q[-1] + n * (i + 1) for i in range(bs - b)])
        self.i32.fill("cu_k", list(cu_k) + [cu_k[-1] + n * (i + 1) for i in range(bs - b)])
        self.i32.fill("slots", list(slots) + [-1] * (R - m))
        flat = []
        for row in bt_rows:
            flat.extend(row + [-1] * (self.max_blocks - len(row)))
        flat.extend([-1] * (self.max_blocks * (bs - b)))
        self.i32.fill("bt", flat)
        self.i64.upload()
        self.i32.upload()
        self.graph.replay()


class DeviceCommitGraph(_GraphBase):
    """Draft replay of the committed tails of a VerifyGraph's batch, derived
    on the device from that graph's results.  Sequence i (in the verify
    batch's order) accepted a_i drafts, so it commits its verify rows
    i*q .. i*q + a_i: the accepted drafts and then the bonus token, whose
    ids are the target argmax of those rows (an accepted draft equals it),
    at the rows' positions and slots.  Those are verify_metadata's outputs
    for the verify starts and query lengths a_i + 1.  Every sequence of the
    bucket commits, padding included (slot -1: no cache write; its state
    goes to the runner's scratch state row), and finished sequences too
    (their state row is released afterwards, their blocks were reserved),
    so the graph needs nothing from the host but the state rows.  The draft
    forward runs over all T = bs*q rows; rows past the committed ones have
    position 0 and slot -1, and attention never reads them."""

    def __init__(self, runner, verify: VerifyGraph):
        super().__init__(runner)
        self.verify = verify
        self.bs, self.q, self.T = verify.bs, verify.q, verify.T
        dev = self.device
        self.i64 = _Staging({"state": self.bs}, torch.int64, dev)
        self.i64.fill("state", [runner.scratch_state_row] * self.bs)
        self.i64.upload()
        self.cu_q = torch.zeros(self.bs + 1, dtype=torch.int32, device=dev)
        self.cu_k = torch.zeros(self.bs + 1, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(self.T, dtype=torch.int64, device=dev)
        self.slots = torch.zeros(self.T, dtype=torch.int32, device=dev)
        self.rows = torch.zeros(self.T, dtype=torch.int32, device=dev)
        self.ids = torch.zeros(self.T, dtype=torch.int64, device=dev)
        self.last = torch.zeros(self.bs, dtype=torch.int64, device=dev)
        self._capture(self._body)

    def _body(self):
        r = self.runner
        v = self.verify
        draft = r.eagle3_model
        bs, q, T = self.bs, self.q, self.T
        bt = v.i32.dev_view("bt").view(bs, v.max_blocks)
        start = v.i32.dev_view("start")
        # one launch: the commit rows' positions, slots, verify rows and
        # tokens, and each sequence's last commit row, from the accept scan
        K.commit_metadata(start, v.out[T:T + bs], q, v.out[:T], bt, r.block_size, T, self.cu_q,
                          self.cu_k, self.pos, self.slots, self.rows, self.ids, self.last)
        combined = draft.combine_hidden_states(aux_concat(v.aux, self.rows))
        set_context(True, self.cu_q, self.cu_k, q, r.max_seqlen_k, self.slots, None, bt)
        try:
            hidden, feedback = draft.forward_with_cache(self.ids, self.pos, combined)
        finally:
            reset_context()
        state = self.i64.dev_view("state")
        r.state_hidden.index_copy_(0, state, hidden.index_select(0, self.last))
        r.state_feedback.index_copy_(0, state, feedback.index_select(0, self.last))

    def run(self, state_rows) -> None:
        """state_rows: the draft-state row of each sequence of the verify
        batch, in its order."""
        pad = self.bs - len(state_rows)
        self.i64.fill("state", list(state_rows) + [self.runner.scratch_state_row] * pad)
        self.i64.upload()
        self.graph.replay()
