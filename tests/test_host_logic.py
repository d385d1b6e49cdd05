"""Host-side logic of the speculative step on the CPU: acceptance rule,
speculation bookkeeping of Scheduler / BlockManager, decode metadata and the
runner's graph-metadata copy.  Expected values are hand-worked from the
reference's code or taken from its own tests (cited per test)."""
import json
import os
import random
from types import SimpleNamespace

import pytest
import torch

from nanovllm_amd.engine import model_runner as mr
from nanovllm_amd.engine.graphs import BUCKETS, bucket_for
from nanovllm_amd.engine.scheduler import Scheduler
from nanovllm_amd.engine.sequence import Sequence, SequenceStatus
from nanovllm_amd.engine.speculative import verify_greedy_proposals
from nanovllm_amd.context import get_context, reset_context, set_context
from nanovllm_amd.sampling_params import SamplingParams

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
BS = 256


# ---------------------------------------------------------------- acceptance rule

def test_engine_acceptance_rule_on_golden_vectors():
    """speculative.py:11-30 of the reference, through the engine's own symbol."""
    cases = json.load(open(os.path.join(GOLDEN, "accept_cases.json")))["cases"]
    for c in cases:
        if "error" in c:
            with pytest.raises(ValueError):
                verify_greedy_proposals(c["proposal"], c["target"])
            continue
        v = verify_greedy_proposals(c["proposal"], c["target"])
        assert v.accepted_count == c["accepted"]
        assert v.accepted_tokens == c["tokens"]
        assert v.replacement_token == c["replacement"]


# ---------------------------------------------------------------- scheduler / blocks

def _scheduler(num_blocks=16, k=5, eos=7, max_num_seqs=8):
    cfg = SimpleNamespace(max_num_seqs=max_num_seqs, max_num_batched_tokens=1 << 16,
                          enable_prefill_batching=True,
                          speculative_config=SimpleNamespace(num_speculative_tokens=k),
                          eos=eos, num_kvcache_blocks=num_blocks, kvcache_block_size=BS,
                          enable_prefix_caching=True)
    return Scheduler(cfg)


def _prefilled(sched, prompt, first_token, **sp):
    """Admit and prefill one sequence (scheduler.py prefill branch + postprocess)."""
    seq = Sequence(list(prompt), SamplingParams(temperature=0.0, **sp))
    sched.add(seq)
    seqs, is_prefill = sched.schedule()
    assert is_prefill and seqs == [seq]
    sched.postprocess(seqs, [first_token], True)
    return seq


def _spec_step(sched, seq, proposal, target):
    """One speculative step in the engine's order (llm_engine.py:124-178)."""
    seqs, is_prefill = sched.schedule()
    assert not is_prefill and seq in seqs
    sched.reserve_speculation(seq)
    base = sched.begin_speculation(seq, proposal)
    seq.num_computed_tokens = base - 1
    v = verify_greedy_proposals(proposal, target)
    committed = sched.postprocess_speculation(seq, base, v.accepted_tokens, v.replacement_token)
    return base, committed


def _check_invariants(sched, live):
    bm = sched.block_manager
    assert len(bm.free_block_ids) + len(bm.used_block_ids) == len(bm.blocks)
    refs = {}
    for seq in live:
        if seq.is_finished:
            continue
        assert len(seq.block_table) == seq.num_blocks
        for b in seq.block_table:
            refs[b] = refs.get(b, 0) + 1
    assert set(refs) == bm.used_block_ids
    for b, n in refs.items():
        assert bm.blocks[b].ref_count == n


def test_full_acceptance_across_a_page_boundary():
    """250-token prompt: the five drafts fill page 0 exactly, the bonus opens
    page 1 (scheduler.py:172-182 page finalisation)."""
    sched = _scheduler()
    seq = _prefilled(sched, range(100, 350), 1, max_tokens=64, ignore_eos=True)
    assert len(seq) == 251 and len(seq.block_table) == 1
    base, committed = _spec_step(sched, seq, [11, 12, 13, 14, 15], [11, 12, 13, 14, 15, 16])
    assert (base, committed) == (251, 5)
    assert seq.token_ids[250:] == [1, 11, 12, 13, 14, 15, 16]
    assert len(seq) == 257 and len(seq.block_table) == 2
    assert seq.num_computed_tokens == 256
    first = sched.block_manager.blocks[seq.block_table[0]]
    assert first.ready and first.hash != -1
    _check_invariants(sched, [seq])


def test_rejection_frees_the_reserved_page():
    """254-token prompt: the reservation takes page 1 for the drafts; rejecting
    all of them truncates it away (block_manager.py:197-205)."""
    sched = _scheduler()
    seq = _prefilled(sched, range(254), 1, max_tokens=64, ignore_eos=True)
    seqs, _ = sched.schedule()
    sched.reserve_speculation(seq)
    assert len(seq.block_table) == 2                      # ceil((255 + 5) / 256)
    reserved = seq.block_table[1]
    base = sched.begin_speculation(seq, [5, 6, 7, 8, 9])
    seq.num_computed_tokens = base - 1
    v = verify_greedy_proposals([5, 6, 7, 8, 9], [4, 6, 7, 8, 9, 10])
    assert sched.postprocess_speculation(seq, base, v.accepted_tokens, v.replacement_token) == 0
    assert seq.token_ids[254:] == [1, 4] and len(seq) == 256
    assert len(seq.block_table) == 1
    assert reserved in sched.block_manager.free_block_ids
    assert seq.num_computed_tokens == 255
    _check_invariants(sched, [seq])


def test_reserve_lookahead_takes_two_steps_of_pages():
    """Scheduler.reserve_lookahead: pages for len + 2k tokens (the next
    step's draft is queued before this step's results are read), capped by
    the token budget; what the step does not keep goes back in
    postprocess_speculation."""
    sched = _scheduler(num_blocks=4)
    seq = Sequence(list(range(250)), SamplingParams(temperature=0.0, max_tokens=64,
                                                    ignore_eos=True))
    capped = Sequence(list(range(500, 750)), SamplingParams(temperature=0.0, max_tokens=3,
                                                            ignore_eos=True))
    sched.add(seq)
    sched.add(capped)
    seqs, is_prefill = sched.schedule()
    assert is_prefill and seqs == [seq, capped]
    sched.postprocess(seqs, [1, 2], True)
    seqs, is_prefill = sched.schedule()
    assert not is_prefill and seqs == [seq, capped]
    sched.reserve_speculation(seq)
    assert len(seq) == 251 and len(seq.block_table) == 1      # 251 + 5 tokens
    assert sched.reserve_lookahead([seq, capped])
    assert len(seq.block_table) == 2                          # 251 + 10 tokens
    assert len(capped.block_table) == 1                       # budget: 250 + 3 tokens
    free = len(sched.block_manager.free_block_ids)
    base = sched.begin_speculation(seq, [5, 6, 7, 8, 9])
    seq.num_computed_tokens = base - 1
    v = verify_greedy_proposals([5, 6, 7, 8, 9], [4, 6, 7, 8, 9, 10])
    assert sched.postprocess_speculation(seq, base, v.accepted_tokens, v.replacement_token) == 0
    assert len(seq) == 252 and len(seq.block_table) == 1      # the look-ahead page went back
    assert len(sched.block_manager.free_block_ids) == free + 1
    _check_invariants(sched, [seq, capped])


def test_reserve_lookahead_is_all_or_nothing():
    """Short of pages for every sequence's look-ahead, nothing is reserved."""
    sched = _scheduler(num_blocks=3)
    a = Sequence(list(range(250)), SamplingParams(temperature=0.0, max_tokens=64, ignore_eos=True))
    b = Sequence(list(range(300, 550)), SamplingParams(temperature=0.0, max_tokens=64,
                                                       ignore_eos=True))
    sched.add(a)
    sched.add(b)
    seqs, is_prefill = sched.schedule()
    assert is_prefill and seqs == [a, b]
    sched.postprocess(seqs, [1, 2], True)
    assert len(a.block_table) == len(b.block_table) == 1
    free = list(sched.block_manager.free_block_ids)
    assert len(free) == 1                                  # each needs a second page
    assert not sched.reserve_lookahead([a, b])
    assert len(a.block_table) == len(b.block_table) == 1
    assert list(sched.block_manager.free_block_ids) == free
    assert sched.reserve_lookahead([a])
    bm = sched.block_manager
    assert len(a.block_table) == 2 and not bm.free_block_ids
    # mid-step a holds one page beyond its length; the pool still adds up
    assert bm.used_block_ids == set(a.block_table) | set(b.block_table)
    assert len(bm.used_block_ids) == len(bm.blocks)


def test_block_table_array_pads_rows_and_rejects_wide_ones():
    """The graphs' block-table staging: rows padded with -1 to the width,
    -1 rows past the given ones, the rows' lengths returned; a row wider
    than the width is an error, not a silent clip."""
    from nanovllm_amd.engine.graphs import block_table_array
    out, lens = block_table_array([[4, 9], [7], []], nrows=4, width=3)
    assert out.dtype.name == "int32" and out.tolist() == [[4, 9, -1], [7, -1, -1],
                                                          [-1, -1, -1], [-1, -1, -1]]
    assert lens.tolist() == [2, 1, 0]
    out, _ = block_table_array([[1, 2, 3], [5]])
    assert out.tolist() == [[1, 2, 3], [5, -1, -1]]
    assert block_table_array([])[0].shape == (0, 1)
    with pytest.raises(ValueError):
        block_table_array([[1, 2, 3]], nrows=1, width=2)


def test_eos_inside_accepted_drafts_ends_the_sequence():
    """EOS truncation drops the replacement and finishes (scheduler.py:158-163)."""
    sched = _scheduler(eos=7)
    seq = _prefilled(sched, range(10, 40), 1, max_tokens=64)
    base, committed = _spec_step(sched, seq, [3, 7, 9, 9, 9], [3, 7, 9, 9, 9, 5])
    assert committed == 2
    assert seq.completion_token_ids == [1, 3, 7]
    assert seq.status == SequenceStatus.FINISHED and not seq.block_table
    assert not sched.running
    assert len(sched.block_manager.free_block_ids) == 16


def test_max_tokens_clips_the_accepted_drafts():
    """Accepted drafts are clipped to the remaining budget, with no replacement
    (scheduler.py:156-157)."""
    sched = _scheduler()
    seq = _prefilled(sched, range(30), 1, max_tokens=3, ignore_eos=True)
    sched.schedule()
    sched.reserve_speculation(seq)
    # reserve covers min(prompt + max_tokens, len + k) = min(33, 36) tokens
    assert len(seq.block_table) == 1
    base = sched.begin_speculation(seq, [4, 5, 6])
    v = verify_greedy_proposals([4, 5, 6], [4, 5, 6, 8])
    assert sched.postprocess_speculation(seq, base, v.accepted_tokens, v.replacement_token) == 2
    assert seq.completion_token_ids == [1, 4, 5]
    assert seq.is_finished


def test_replacement_only_when_budget_remains():
    sched = _scheduler()
    seq = _prefilled(sched, range(30), 1, max_tokens=2, ignore_eos=True)
    base, committed = _spec_step(sched, seq, [4], [9, 9])
    assert committed == 0
    assert seq.completion_token_ids == [1, 9]
    assert seq.is_finished


def test_random_speculation_keeps_block_accounting_consistent():
    """Many steps over several sequences with random acceptance: the block
    table always covers ceil(len/256) pages, reference counts match the
    tables, and freed pages return to the pool."""
    rng = random.Random(0)
    sched = _scheduler(num_blocks=64, k=5, eos=-1)
    live = []
    for i in range(4):
        prompt = [rng.randrange(1000) for _ in range(rng.randrange(200, 700))]
        live.append(Sequence(prompt, SamplingParams(temperature=0.0, max_tokens=300,
                                                    ignore_eos=True)))
        sched.add(live[-1])
    seqs, is_prefill = sched.schedule()                   # prefill batching: all four
    assert is_prefill and seqs == live
    sched.postprocess(seqs, [rng.randrange(1000) for _ in seqs], True)
    steps = 0
    while sched.running and steps < 400:
        seqs, is_prefill = sched.schedule()
        assert not is_prefill
        for seq in seqs:
            sched.reserve_speculation(seq)
            k = min(5, seq.max_tokens - seq.num_completion_tokens)
            proposal = [rng.randrange(1000) for _ in range(k)]
            a = rng.randrange(k + 1)
            target = proposal[:a] + [rng.randrange(1000, 2000)] + \
                [rng.randrange(1000) for _ in range(k - a)]
            base = sched.begin_speculation(seq, proposal)
            seq.num_computed_tokens = base - 1
            before = seq.token_ids[:base]
            v = verify_greedy_proposals(proposal, target)
            assert v.accepted_count == a
            c = sched.postprocess_speculation(seq, base, v.accepted_tokens, v.replacement_token)
            assert seq.token_ids[:base] == before
            assert seq.token_ids[base:base + c] == proposal[:c]
            if not seq.is_finished:
                assert seq.num_computed_tokens == base + c
        _check_invariants(sched, live)
        steps += 1
    assert all(s.is_finished for s in live)
    assert all(s.num_completion_tokens == 300 for s in live)
    assert len(sched.block_manager.free_block_ids) == 64


def test_prefix_cache_hash_is_chained_xxhash64():
    """Block hashes chain the previous hash as 8 little-endian bytes before
    the int64 token ids (block_manager.py compute_hash)."""
    import numpy as np
    import xxhash

    from nanovllm_amd.engine.block_manager import BlockManager

    toks = list(range(256))
    h0 = xxhash.xxh64(np.array(toks, dtype=np.int64).tobytes()).intdigest()
    assert BlockManager.compute_hash(toks) == h0
    h1 = xxhash.xxh64(h0.to_bytes(8, "little") + np.array(toks, dtype=np.int64).tobytes())
    assert BlockManager.compute_hash(toks, h0) == h1.intdigest()


# ---------------------------------------------------------------- runner metadata

@pytest.fixture
def cpu_runner(monkeypatch):
    monkeypatch.setattr(mr, "_pinned", lambda values, dtype: torch.tensor(values, dtype=dtype))
    runner = mr.ModelRunner.__new__(mr.ModelRunner)
    runner.block_size = BS
    runner.device = torch.device("cpu")
    yield runner
    reset_context()


def test_prepare_decode_slots_match_reference_vector(cpu_runner):
    """tests/test_decode_context.py:26-32 of the reference."""
    cpu_runner.prepare_block_tables = lambda seqs: torch.tensor(
        [[seq.block_table[0]] for seq in seqs], dtype=torch.int32)
    first = Sequence([11] * 16)
    second = Sequence([12] * 17)
    first.block_table = [3]
    second.block_table = [5]
    input_ids, positions = cpu_runner.prepare_decode([first, second])
    ctx = get_context()
    assert not ctx.is_prefill
    assert input_ids.tolist() == [11, 12]
    assert positions.tolist() == [15, 16]
    assert ctx.context_lens.tolist() == [16, 17]
    assert ctx.slot_mapping.tolist() == [3 * 256 + 15, 5 * 256 + 16]


def test_runtime_capabilities(cpu_runner):
    """tests/test_eagle3_runtime.py:24-50 of the reference."""
    cpu_runner.eagle3_model = object()
    cpu_runner.eagle_kv_cache = torch.empty(2, 1, 2, 4, 1, 8)
    cpu_runner.eagle_graphs = {1: object()}
    caps = cpu_runner.get_eagle3_runtime_capabilities()
    assert caps["paged_kv_cache"] is True
    assert caps["cuda_graph"] is True
    assert caps["graph_batch_sizes"] == [1]
    cpu_runner.eagle3_model = None
    cpu_runner.eagle_kv_cache = None
    cpu_runner.eagle_graphs = {}
    cpu_runner._propose_graphs = {}
    assert cpu_runner.get_eagle3_runtime_capabilities() == {
        "paged_kv_cache": False, "cuda_graph": False, "graph_batch_sizes": []}


def test_graph_replay_copies_paged_metadata(cpu_runner):
    """tests/test_eagle3_runtime.py:53-91 of the reference."""
    class FakeGraph:
        def replay(self):
            return None

    cpu_runner.eagle_graphs = {1: FakeGraph()}
    cpu_runner.eagle_graph_vars = {1: {
        "input_ids": torch.zeros(1, dtype=torch.int64),
        "positions": torch.zeros(1, dtype=torch.int64),
        "feedback": torch.zeros(1, 2),
        "slot_mapping": torch.full((1,), -1, dtype=torch.int32),
        "context_lens": torch.ones(1, dtype=torch.int32),
        "block_tables": torch.zeros(1, 2, dtype=torch.int32),
        "outputs": (torch.ones(1, 2), torch.full((1, 2), 2.0)),
    }}
    set_context(False, slot_mapping=torch.tensor([7], dtype=torch.int32),
                context_lens=torch.tensor([9], dtype=torch.int32),
                block_tables=torch.tensor([[3, 4]], dtype=torch.int32))
    hidden, feedback = cpu_runner.run_eagle3_graph(torch.tensor([5]), torch.tensor([8]),
                                                   torch.zeros(1, 2), [object()])
    v = cpu_runner.eagle_graph_vars[1]
    assert v["slot_mapping"].tolist() == [7]
    assert v["context_lens"].tolist() == [9]
    assert v["block_tables"].tolist() == [[3, 4]]
    assert hidden.tolist() == [[1.0, 1.0]]
    assert feedback.tolist() == [[2.0, 2.0]]


def test_bucket_for_picks_the_smallest_covering_bucket():
    assert bucket_for(1) == 1
    assert bucket_for(3) == 4
    assert bucket_for(64) == 64
    assert bucket_for(65) == 96
    assert bucket_for(BUCKETS[-1]) == BUCKETS[-1]
    assert bucket_for(BUCKETS[-1] + 1) is None


def test_config_rejects_multi_gpu_and_bad_kv_dtype(tmp_path):
    from nanovllm_amd.config import Config
    from nanovllm_amd.synthetic import write_qwen3_config

    path = write_qwen3_config(str(tmp_path / "m"), "tiny")
    with pytest.raises(ValueError, match="one GPU"):
        Config(path, tensor_parallel_size=2)
    with pytest.raises(ValueError, match="kv_cache_dtype"):
        Config(path, kv_cache_dtype="int8")
    with pytest.raises(ValueError):
        Config(str(tmp_path / "missing"))


def test_gemm_tuning_file_is_well_formed(tmp_path):
    """The packaged TunableOp results name one solution per projection GEMM
    shape of the Qwen3-8B EAGLE3 step, and Config rejects a missing file."""
    import csv

    from nanovllm_amd.config import Config
    from nanovllm_amd.synthetic import write_qwen3_config

    path = os.path.join(os.path.dirname(__file__), "..", "extend-nano-vllm_amd", "nanovllm_amd",
                        "tuning", "gemm_mi355x_qwen3_8b_eagle3.csv")
    rows = list(csv.reader(open(path)))
    validators = {r[1] for r in rows if r[0] == "Validator"}
    assert {"PT_VERSION", "GCN_ARCH_NAME", "HIPBLASLT_VERSION"} <= validators
    gemms = [r for r in rows if r[0].startswith("GemmTunableOp")]
    shapes = {r[1].split("_ld_")[0] for r in gemms}
    assert len(shapes) == len(gemms)                 # one solution per shape
    # verify (384 rows) and draft (64 rows) projections of the 8B geometry
    for shape in ("tn_6144_384_4096", "tn_4096_384_4096", "tn_24576_384_4096",
                  "tn_4096_384_12288", "tn_151936_64_4096"):
        assert shape in shapes
    model = write_qwen3_config(str(tmp_path / "m"), "tiny")
    with pytest.raises(ValueError, match="gemm_tuning_file"):
        Config(model, gemm_tuning_file=str(tmp_path / "missing.csv"))


# ---------------------------------------------------------------- reference traces

def _traces():
    import json
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "scheduler_traces.json")
    with open(path) as f:
        return json.load(f)


@pytest.mark.parametrize("index", range(7))
def test_scheduler_matches_reference_traces(index):
    """Step-by-step states of the reference's own Scheduler / BlockManager /
    Sequence (recorded by tests/golden/gen_scheduler_traces.py from
    nanovllm/engine/{scheduler,block_manager,sequence}.py) driven through
    chunked and batched prefill, speculative steps with accepted prefixes,
    bonus tokens, EOS and max_tokens clipping, page crossings, prefix-cache
    hits, decode preemption and pool exhaustion: this build's classes,
    replaying the same inputs, must reach identical block tables, free-list
    order, reference counts, block hashes, queues and errors after every
    step."""
    from helpers import scheduler_trace
    from nanovllm_amd.engine.scheduler import Scheduler
    from nanovllm_amd.engine.sequence import Sequence
    from nanovllm_amd.sampling_params import SamplingParams

    trace = _traces()[index]
    _, snaps, final = scheduler_trace(Scheduler, Sequence, SamplingParams, trace["scenario"],
                                      inputs=trace["inputs"])
    assert len(snaps) == len(trace["snapshots"]), trace["scenario"]["name"]
    for step, (got, want) in enumerate(zip(snaps, trace["snapshots"])):
        assert got == want, f"{trace['scenario']['name']} step {step}"
    assert final == trace["final_tokens"]


@pytest.mark.parametrize("prefill", [True, False])
def test_bench_torch_attention_matches_oracle(prefill):
    """bench.py's torch stand-in for FlashAttention-2 (the comparator's
    attention backend) computes the paged causal attention of the oracle:
    bottom-right aligned verify rows, GQA, shuffled pages, ragged lengths;
    and one row per sequence for the decode form.  Run on the CPU."""
    from types import SimpleNamespace

    import numpy as np

    import bench
    from helpers import bits, paged_case
    from oracle import oracle

    case = paged_case(seed=21, batch=4, q_len=[3, 1, 5, 2] if prefill else 1, ctx_lo=5,
                      ctx_hi=700, hq=8, hkv=2)
    layer = SimpleNamespace(k_cache=case["k_cache"], v_cache=case["v_cache"], scale=128 ** -0.5)
    if prefill:
        set_context(True, case["cu_q"], case["cu_k"], max(case["q_lens"]), int(case["lens"].max()),
                    None, None, case["block_tables"])
    else:
        set_context(False, context_lens=case["lens"], block_tables=case["block_tables"])
    try:
        got = bench.TorchAttention().attend(layer, case["q"]).float().numpy()
    finally:
        reset_context()
    ref = oracle.paged_attention(bits(case["q"]), bits(case["k_cache"]), bits(case["v_cache"]),
                                 case["cu_q"].numpy(), case["lens"].numpy(),
                                 case["block_tables"].numpy(), 128 ** -0.5)
    assert np.abs(got - ref).max() <= 2e-2


def test_draft_steps_past_a_sequence_limit_write_nowhere(cpu_runner):
    """A batch mixing a sequence near max_tokens (one proposal left, its
    pages reserved only up to prompt + max_tokens) with one that drafts k:
    the draft steps past the short sequence's own last step get slot -1 (no
    K/V write, no page lookup past its table), the others their slots."""
    sched = _scheduler(k=5)
    near = Sequence(list(range(253)), SamplingParams(temperature=0.0, max_tokens=2,
                                                     ignore_eos=True))
    far = Sequence(list(range(1000, 1040)), SamplingParams(temperature=0.0, max_tokens=64,
                                                           ignore_eos=True))
    sched.add(near)
    sched.add(far)
    seqs, is_prefill = sched.schedule()                   # prefill batching: both
    assert is_prefill and seqs == [near, far]
    sched.postprocess(seqs, [1, 1], True)                 # near: len 254, one token left
    sched.schedule()
    for seq in (near, far):
        sched.reserve_speculation(seq)
    assert len(near.block_table) == 1          # 253 + 2 tokens fit page 0
    with pytest.raises(IndexError):            # position 256 has no page
        cpu_runner._slot(near, 256)
    limits = [min(5, s.max_tokens - s.num_completion_tokens) for s in (near, far)]
    assert limits == [1, 5]
    pos, slots, ctx = cpu_runner._draft_step_metadata([near, far], limits, 5)
    assert [row[0] for row in pos] == [253, 254, 255, 256]
    assert [row[0] for row in slots] == [-1, -1, -1, -1]
    assert [row[1] for row in slots] == [far.block_table[0] * BS + p for p in (40, 41, 42, 43)]
    assert [row[1] for row in ctx] == [41, 42, 43, 44]


def test_sampling_params_errors_follow_the_reference():
    """A negative temperature fails the reference's assert
    (sampling_params.py:11), so it raises AssertionError here too; a zero
    token budget (which the reference does not check) is refused up front."""
    with pytest.raises(AssertionError, match="temperature must be non-negative"):
        SamplingParams(temperature=-0.5)
    with pytest.raises(AssertionError):
        SamplingParams(temperature=float("nan"))
    with pytest.raises(ValueError, match="max_tokens"):
        SamplingParams(max_tokens=0)
    assert SamplingParams(temperature=0.0, max_tokens=1).max_tokens == 1


def test_lookahead_churn_leaves_cached_prefix_pages_alone():
    """reserve_lookahead's extra pages are unkeyed pages from the free
    list's tail (where the step's truncate returns them), so a finished
    sequence's keyed prefix pages, waiting in the free list, survive
    several look-ahead steps and a new request with the same prompt reuses
    them.  Taking them from the head instead cycles the six-page pool in
    five steps and evicts both."""
    sched = _scheduler(num_blocks=6, k=5)
    bm = sched.block_manager
    a = _prefilled(sched, list(range(1000, 1512)), 3, max_tokens=64, ignore_eos=True)
    keyed = list(a.block_table)
    assert len(keyed) == 2 and all(bm.blocks[b].hash != -1 for b in keyed)
    sched.running.remove(a)
    bm.deallocate(a)                          # both pages wait, keyed, in the free list
    b = _prefilled(sched, list(range(245)), 1, max_tokens=64, ignore_eos=True)
    looked_ahead = 0
    for step in range(8):
        seqs, is_prefill = sched.schedule()
        assert not is_prefill and seqs == [b]
        sched.reserve_speculation(b)
        before = len(b.block_table)
        assert sched.reserve_lookahead([b])
        looked_ahead += len(b.block_table) > before
        base = sched.begin_speculation(b, [7, 7, 7, 7, 7])
        b.num_computed_tokens = base - 1
        v = verify_greedy_proposals([7, 7, 7, 7, 7], [9, 9, 9, 9, 9, 9])   # nothing accepted
        sched.postprocess_speculation(b, base, v.accepted_tokens, v.replacement_token)
        _check_invariants(sched, [b])
    assert looked_ahead >= 5
    for block_id in keyed:
        assert block_id in bm.free_block_ids and bm.hash_to_block_id[bm.blocks[block_id].hash] == block_id
    c = Sequence(list(range(1000, 1512)), SamplingParams(temperature=0.0, max_tokens=8))
    hits = bm.stats["prefix_cache_hits"]
    bm.allocate(c)
    assert bm.stats["prefix_cache_hits"] == hits + 2 and c.block_table == keyed
