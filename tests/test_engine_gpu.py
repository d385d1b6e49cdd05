"""End-to-end EAGLE3 engine on the GPU with random-weight tiny models.

The emitted tokens must be the target's greedy tokens: every generated token
equals the argmax of the target's logits given the generated prefix
(teacher-forced), except where the top-2 logit margin is below 2e-2, and the
speculative and non-speculative engines agree up to such a near tie.
Acceptance paths (accepted drafts, bonus tokens, page crossings, max_tokens
clipping) are exercised with proposals taken from the target's own greedy
continuation, partly corrupted.
"""
import pytest
import torch

from nanovllm_amd import LLM, SamplingParams
from nanovllm_amd.engine.sequence import Sequence
from nanovllm_amd.synthetic import write_eagle3_config, write_qwen3_config

pytestmark = pytest.mark.gpu

MARGIN_TOL = 2e-2
AUX = (1, 2, 4)


@pytest.fixture(scope="module")
def dirs(tmp_path_factory):
    root = tmp_path_factory.mktemp("ckpt")
    target = write_qwen3_config(str(root / "target"), "tiny")
    draft = write_eagle3_config(str(root / "draft"), "tiny", aux_layers=AUX)
    return target, draft


def make_llm(dirs, spec=True, k=4, blocks=96, eager=True, kv_cache_dtype="auto"):
    target, draft = dirs
    kw = dict(load_format="dummy", seed=0, max_model_len=2048, num_kvcache_blocks=blocks,
              enforce_eager=eager, max_num_batched_tokens=4096, kv_cache_dtype=kv_cache_dtype,
              max_num_seqs=16)
    if spec:
        kw["speculative_config"] = {"method": "eagle3", "model": draft,
                                    "num_speculative_tokens": k, "aux_hidden_state_layers": AUX}
    return LLM(target, **kw)


def prompts(n, seed=0, lo=5, hi=300):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi, (n,), generator=g).tolist()
    return [torch.randint(0, 2048, (L,), generator=g).tolist() for L in lens]


@torch.inference_mode()
def teacher_forced_logits(llm, tokens):
    """Target logits at every position of ``tokens`` (a fresh prefill)."""
    runner = llm.model_runner
    bm = llm.scheduler.block_manager
    seq = Sequence(tokens)
    bm.allocate(seq)
    seq.num_computed_tokens = 0
    seq.num_scheduled_tokens = len(tokens)
    try:
        ids, pos = runner.prepare_prefill([seq])
        hidden = runner.model(ids, pos)
        return runner.model.compute_all_logits(hidden).float().cpu()
    finally:
        from nanovllm_amd.context import reset_context
        reset_context()
        bm.deallocate(seq)


def check_greedy(llm, prompt, out):
    logits = teacher_forced_logits(llm, prompt + out)
    full = prompt + out
    bad = []
    for p in range(len(prompt), len(full)):
        row = logits[p - 1]
        top2 = row.topk(2).values
        if int(row.argmax()) != full[p] and float(top2[0] - top2[1]) >= MARGIN_TOL:
            bad.append(p)
    return bad


def assert_same_greedy_path(llm, prompt, got, ref):
    """``got`` is a valid greedy path of the target and equals ``ref`` up to
    their first difference, which must sit at a near tie."""
    assert len(got) == len(ref)
    assert check_greedy(llm, prompt, got) == []
    n = next((i for i, (x, y) in enumerate(zip(got, ref)) if x != y), None)
    if n is not None:
        row = teacher_forced_logits(llm, prompt + got[:n])[-1]
        top2 = row.topk(2).values
        assert float(top2[0] - top2[1]) < MARGIN_TOL, (n, float(top2[0] - top2[1]))


def test_spec_equals_target_greedy(dirs):
    ps = prompts(6, seed=1)
    sp = SamplingParams(temperature=0.0, max_tokens=40, ignore_eos=True)
    spec = make_llm(dirs, spec=True)
    try:
        outs = [o["token_ids"] for o in spec.generate(ps, sp, use_tqdm=False)]
        assert all(len(o) == 40 for o in outs)
        for p, o in zip(ps, outs):
            assert check_greedy(spec, p, o) == []
        assert spec.spec_stats["steps"] > 0
        assert spec.model_runner.get_eagle3_runtime_capabilities()["paged_kv_cache"]
    finally:
        spec.exit()
    plain = make_llm(dirs, spec=False)
    try:
        ref = [o["token_ids"] for o in plain.generate(ps, sp, use_tqdm=False)]
        for p, a, b in zip(ps, outs, ref):
            # identical up to the first near tie (then both are valid greedy paths)
            n = next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), None)
            if n is not None:
                row = teacher_forced_logits(plain, p + a[:n])[-1]
                top2 = row.topk(2).values
                assert float(top2[0] - top2[1]) < MARGIN_TOL
    finally:
        plain.exit()


def test_acceptance_paths_with_oracle_drafts(dirs):
    """Proposals = the target's own greedy continuation, corrupted at a few
    positions: exercises accepted prefixes, bonus tokens, multi-token commits,
    page crossings (prompts near 256) and max_tokens clipping."""
    ps = [prompts(1, seed=7, lo=240, hi=250)[0], prompts(1, seed=8, lo=20, hi=30)[0],
          prompts(1, seed=9, lo=500, hi=510)[0]]
    max_tokens = [37, 23, 30]
    plain = make_llm(dirs, spec=False)
    try:
        ref = [plain.generate([p], SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True),
                              use_tqdm=False)[0]["token_ids"] for p, m in zip(ps, max_tokens)]
    finally:
        plain.exit()
    spec = make_llm(dirs, spec=True, k=5)
    runner = spec.model_runner
    original = runner.propose_eagle3_batch
    calls = {"n": 0}
    full = {tuple(p): p + r for p, r in zip(ps, ref)}

    def oracle_propose(seqs):
        drafted = original(seqs)        # keeps the draft model's own K/V and state path
        out = []
        for seq, d in zip(seqs, drafted):
            seqfull = full[tuple(seq.prompt_token_ids)]
            want = seqfull[len(seq):len(seq) + len(d)]
            want = want + d[len(want):]
            calls["n"] += 1
            if calls["n"] % 3 == 0 and len(want) > 2:
                want = list(want)
                want[2] = (want[2] + 1) % 2048     # reject from the third draft on
            out.append(want)
        return out

    runner.propose_eagle3_batch = oracle_propose
    try:
        for p, m, r in zip(ps, max_tokens, ref):
            spec.add_request(p, SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True))
        outs = {}
        while not spec.is_finished():
            for seq_id, toks in spec.step()[0]:
                outs[seq_id] = toks
        got = [outs[i] for i in sorted(outs)]
        for p, a, b in zip(ps, got, ref):
            assert_same_greedy_path(spec, p, a, b)
        stats = spec.spec_stats
        assert stats["accepted"] > stats["steps"]          # multi-token commits happened
        assert stats["committed"] == sum(max_tokens) - len(ps)   # first token comes from prefill
    finally:
        spec.exit()


def test_errors_match_reference(dirs):
    spec = make_llm(dirs, spec=True)
    try:
        with pytest.raises(ValueError):
            spec.add_request([1, 2, 3], SamplingParams(temperature=0.7))
        with pytest.raises(ValueError):
            spec.add_request([], SamplingParams(temperature=0.0))
        with pytest.raises(ValueError):
            spec.add_request([1] * 2040, SamplingParams(temperature=0.0, max_tokens=64))
        with pytest.raises(ValueError):
            spec.add_request("text prompt", SamplingParams(temperature=0.0))
    finally:
        spec.exit()


def test_hip_graph_steps_are_greedy(dirs):
    """The captured verify / propose / commit graphs (padded buckets) produce
    the same greedy paths as the eager engine."""
    ps = prompts(6, seed=3)
    sp = SamplingParams(temperature=0.0, max_tokens=33, ignore_eos=True)
    eager = make_llm(dirs, spec=True, eager=True)
    try:
        assert eager.model_runner.get_eagle3_runtime_capabilities() == {
            "paged_kv_cache": True, "cuda_graph": False, "graph_batch_sizes": []}
        ref = [o["token_ids"] for o in eager.generate(ps, sp, use_tqdm=False)]
    finally:
        eager.exit()
    graphed = make_llm(dirs, spec=True, eager=False)
    try:
        # captured at initialisation, as the reference reports at engine-up
        # (model_runner.py:195, :982-990): every bucket up to max_num_seqs
        runner = graphed.model_runner
        assert runner.get_eagle3_runtime_capabilities() == {
            "paged_kv_cache": True, "cuda_graph": True, "graph_batch_sizes": [1, 2, 4, 8, 16]}
        captured = {b: (runner._verify_graphs[b], runner._propose_graphs[b])
                    for b in (1, 2, 4, 8, 16)}
        got = [o["token_ids"] for o in graphed.generate(ps, sp, use_tqdm=False)]
        # the steps replayed the graphs captured at initialisation
        for b, (v, p) in captured.items():
            assert runner._verify_graphs[b] is v and runner._propose_graphs[b] is p
        assert sorted(runner._verify_graphs) == [1, 2, 4, 8, 16]
        for p, a, b in zip(ps, got, ref):
            assert_same_greedy_path(graphed, p, a, b)
        # the engine's captures leave torch's generator usable by a caller's
        # own capture outside inference mode while the engine's graphs live
        x = torch.arange(8, dtype=torch.float32, device="cuda")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = x * 2
        for rep in range(3):
            x.fill_(rep)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y.cpu(), torch.full((8,), 2.0 * rep))
    finally:
        graphed.exit()


def test_reference_structured_step_is_greedy(dirs):
    """The reference-shaped step (host sync per draft step, per-sequence
    argmax, serial single-token draft replay) emits the same greedy paths as
    the engine's batched step."""
    ps = prompts(4, seed=11)
    sp = SamplingParams(temperature=0.0, max_tokens=21, ignore_eos=True)
    fast = make_llm(dirs, spec=True)
    try:
        ref = [o["token_ids"] for o in fast.generate(ps, sp, use_tqdm=False)]
    finally:
        fast.exit()
    slow = make_llm(dirs, spec=True)
    slow.reference_pipeline = True
    try:
        got = [o["token_ids"] for o in slow.generate(ps, sp, use_tqdm=False)]
        assert slow.spec_stats["steps"] > 0
        for p, a, b in zip(ps, got, ref):
            assert_same_greedy_path(slow, p, a, b)
    finally:
        slow.exit()


def test_fp8_kv_cache_spec_equals_target_greedy(dirs):
    """EAGLE3 over an FP8 E4M3 KV cache (which the reference does not allow):
    the speculative engine emits the greedy path of the FP8-cache target,
    including prompts that prefill several query tiles."""
    ps = prompts(4, seed=12, lo=200, hi=600)
    sp = SamplingParams(temperature=0.0, max_tokens=25, ignore_eos=True)
    spec = make_llm(dirs, spec=True, kv_cache_dtype="fp8")
    try:
        assert spec.model_runner.kv_cache.dtype == torch.float8_e4m3fn
        outs = [o["token_ids"] for o in spec.generate(ps, sp, use_tqdm=False)]
        for p, o in zip(ps, outs):
            assert len(o) == 25
            assert check_greedy(spec, p, o) == []
    finally:
        spec.exit()
    plain = make_llm(dirs, spec=False, kv_cache_dtype="fp8")
    try:
        ref = [o["token_ids"] for o in plain.generate(ps, sp, use_tqdm=False)]
        for p, a, b in zip(ps, outs, ref):
            assert_same_greedy_path(plain, p, a, b)
    finally:
        plain.exit()


def test_pipelined_verify_with_oracle_drafts(dirs):
    """Graph steps with the verify enqueued behind the draft (input ids
    composed on the device): proposals rewritten on the device to the
    target's own greedy continuation, corrupted at a few positions, must give
    the target's greedy path with multi-token commits, as the sequential
    propose-then-verify path does; the budgets differ per sequence, so the
    last steps verify ragged proposal counts on the same path."""
    ps = [prompts(1, seed=17, lo=240, hi=250)[0], prompts(1, seed=18, lo=20, hi=30)[0],
          prompts(1, seed=19, lo=500, hi=510)[0], prompts(1, seed=20, lo=60, hi=70)[0]]
    max_tokens = [41, 29, 33, 26]
    plain = make_llm(dirs, spec=False)
    try:
        ref = [plain.generate([p], SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True),
                              use_tqdm=False)[0]["token_ids"] for p, m in zip(ps, max_tokens)]
    finally:
        plain.exit()
    full = {tuple(p): p + r for p, r in zip(ps, ref)}
    calls = {"n": 0, "pipelined": 0}

    def override(seqs, tokens):
        calls["pipelined"] += 1
        k = tokens.shape[0]
        host = tokens.cpu()
        for i, seq in enumerate(seqs):
            seqfull = full[tuple(seq.prompt_token_ids)]
            want = seqfull[len(seq):len(seq) + k]
            calls["n"] += 1
            for s_, tok in enumerate(want):
                host[s_, i] = tok
            if calls["n"] % 3 == 0 and k > 2:
                host[2, i] = (int(host[2, i]) + 1) % 2048   # reject from the third draft on
        tokens.copy_(host.to(tokens.device))

    spec = make_llm(dirs, spec=True, k=5, eager=False)
    spec.model_runner.draft_override = override
    try:
        for p, m in zip(ps, max_tokens):
            spec.add_request(p, SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True))
        outs = {}
        while not spec.is_finished():
            for seq_id, toks in spec.step()[0]:
                outs[seq_id] = toks
        got = [outs[i] for i in sorted(outs)]
        for p, a, b in zip(ps, got, ref):
            assert_same_greedy_path(spec, p, a, b)
        stats = spec.spec_stats
        assert calls["pipelined"] > 0
        assert stats["accepted"] > stats["steps"]          # multi-token commits happened
        assert stats["committed"] == sum(max_tokens) - len(ps)
        # the steps where a sequence is within k tokens of its budget (it
        # proposes fewer drafts) stay on the pipelined graph path too
        pipe = spec.model_runner.pipeline_stats
        assert pipe["steps"] == stats["steps"] and pipe["ragged"] > 0, pipe
    finally:
        spec.exit()


def test_device_commit_matches_host_commit(dirs):
    """The draft commit derived on the device from the verify results (run
    right behind the verify) leaves the same draft state as the commit built
    from the host's accepted tails: after every step, each live sequence's
    recurrent draft state agrees (the two replays run their GEMMs over
    different row counts, so agreement is to bf16 rounding).  Drafts agree
    with the target's greedy continuation for a varying number of steps, so
    the committed tails have different lengths."""
    ps = [prompts(1, seed=31 + i, lo=20 + 40 * i, hi=30 + 40 * i)[0] for i in range(5)]
    sp = SamplingParams(temperature=0.0, max_tokens=24, ignore_eos=True)
    plain = make_llm(dirs, spec=False)
    try:
        ref = [o["token_ids"] for o in plain.generate(ps, sp, use_tqdm=False)]
    finally:
        plain.exit()
    full = {tuple(p): p + r for p, r in zip(ps, ref)}

    def override(seqs, tokens):
        # every proposal fixed: the target's next tokens for (len % 3 + 1)
        # positions, then wrong ones, so acceptance does not depend on the
        # draft state the two runs compute
        host = tokens.cpu()
        for i, seq in enumerate(seqs):
            want = full[tuple(seq.prompt_token_ids)]
            n = len(seq)
            for s_ in range(tokens.shape[0]):
                tok = want[n + s_] if n + s_ < len(want) else 0
                host[s_, i] = tok if s_ <= n % 3 else (tok + 1) % 2048
        tokens.copy_(host.to(tokens.device))

    runs = {}
    for device_commit in (True, False):
        llm = make_llm(dirs, spec=True, k=4, eager=False)
        llm.model_runner.device_commit = device_commit
        llm.model_runner.draft_override = override
        try:
            for p in ps:
                llm.add_request(p, sp)
            states, outs = [], {}
            while not llm.is_finished():
                for seq_id, toks in llm.step()[0]:
                    outs[seq_id] = toks
                runner = llm.model_runner
                snap = {}
                for seq in llm.scheduler.running:
                    row = runner._state_slot.get(seq.seq_id)
                    if row is not None:
                        snap[tuple(seq.prompt_token_ids)] = (
                            len(seq), runner.state_hidden[row].float().cpu(),
                            runner.state_feedback[row].float().cpu())
                states.append(snap)
            got = [outs[i] for i in sorted(outs)]
            for p, g, r in zip(ps, got, ref):
                assert_same_greedy_path(llm, p, g, r)
            runs[device_commit] = (states, got, dict(llm.spec_stats))
        finally:
            llm.exit()
    (sa_all, out_a, st_a), (sb_all, out_b, st_b) = runs[True], runs[False]
    assert out_a == out_b
    assert st_a["accepted"] == st_b["accepted"] > st_a["steps"]
    assert len(sa_all) == len(sb_all) > 2
    compared = 0
    for sa, sb in zip(sa_all, sb_all):
        assert sa.keys() == sb.keys()
        for key in sa:
            la, ha, fa = sa[key]
            lb, hb, fb = sb[key]
            assert la == lb
            torch.testing.assert_close(ha, hb, atol=3e-2, rtol=3e-2)
            torch.testing.assert_close(fa, fb, atol=3e-2, rtol=3e-2)
            compared += 1
    assert compared > 10


def test_prelaunched_drafts_equal_fresh_drafts(dirs):
    """A step's draft queued behind the previous step's verify and device
    commit (lengths, positions and slots derived on the device from the
    accept results) proposes exactly what a draft launched after the host's
    bookkeeping proposes: with acceptance forced by oracle drafts (so the
    lengths grow by varying amounts), the raw draft tokens of every step,
    the outputs and the acceptance counts agree between the two engines,
    and the queued drafts were used."""
    ps = [prompts(1, seed=31, lo=250, hi=258)[0], prompts(1, seed=32, lo=20, hi=30)[0],
          prompts(1, seed=33, lo=500, hi=510)[0]]
    max_tokens = [70, 64, 58]
    plain = make_llm(dirs, spec=False)
    try:
        ref = [plain.generate([p], SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True),
                              use_tqdm=False)[0]["token_ids"] for p, m in zip(ps, max_tokens)]
    finally:
        plain.exit()
    full = {tuple(p): p + r for p, r in zip(ps, ref)}

    def run(prelaunch):
        raw, calls = [], {"n": 0}

        def override(seqs, tokens):
            k = tokens.shape[0]
            host = tokens.cpu()
            # per sequence: the two engines may order the draft columns
            # differently (a queued draft keeps the previous verify's order)
            raw.append({tuple(seq.prompt_token_ids): host[:, i].clone()
                        for i, seq in enumerate(seqs)})
            for i, seq in enumerate(seqs):
                want = full[tuple(seq.prompt_token_ids)][len(seq):len(seq) + k]
                calls["n"] += 1
                for s_, tok in enumerate(want):
                    host[s_, i] = tok
                if calls["n"] % 4 == 0:
                    host[calls["n"] % k, i] = (int(host[calls["n"] % k, i]) + 1) % 2048
            tokens.copy_(host.to(tokens.device))

        llm = make_llm(dirs, spec=True, k=5, eager=False)
        llm.prelaunch_draft = prelaunch
        llm.model_runner.draft_override = override
        try:
            for p, m in zip(ps, max_tokens):
                llm.add_request(p, SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True))
            outs = {}
            while not llm.is_finished():
                for seq_id, toks in llm.step()[0]:
                    outs[seq_id] = toks
            return ([outs[i] for i in sorted(outs)], raw, dict(llm.spec_stats),
                    dict(llm.model_runner.prelaunch_stats))
        finally:
            llm.exit()

    got_on, raw_on, stats_on, pre_on = run(True)
    got_off, raw_off, stats_off, pre_off = run(False)
    assert pre_on["used"] >= 5 and pre_on["used"] <= pre_on["queued"], pre_on
    assert pre_off == {"queued": 0, "used": 0}
    assert stats_on == stats_off and stats_on["accepted"] > stats_on["steps"]
    assert got_on == got_off
    assert len(raw_on) == len(raw_off)
    for step, (a, b) in enumerate(zip(raw_on, raw_off)):
        assert a.keys() == b.keys(), step
        for key in a:
            assert torch.equal(a[key], b[key]), step


def test_prelaunched_drafts_with_the_device_running_behind(dirs, monkeypatch):
    """The queued device commit and next-step draft take their metadata from
    pinned staging buffers the host refills every step.  Here the draft
    override rewrites the proposals with device work only (no host sync),
    and a spin kernel is queued ahead of every device commit, so the host
    reaches the next step's refill while the previous step's copies are
    still queued.  The raw draft tokens of every step must equal those of
    an engine that drafts after the host's bookkeeping, and the refills
    must have found copies still queued (the case the staging's wait
    covers)."""
    from nanovllm_amd.engine import graphs

    ps = [prompts(1, seed=41, lo=250, hi=258)[0], prompts(1, seed=42, lo=20, hi=30)[0],
          prompts(1, seed=43, lo=500, hi=510)[0]]
    max_tokens = [60, 54, 48]
    plain = make_llm(dirs, spec=False)
    try:
        ref = [plain.generate([p], SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True),
                              use_tqdm=False)[0]["token_ids"] for p, m in zip(ps, max_tokens)]
    finally:
        plain.exit()
    full = {tuple(p): p + r for p, r in zip(ps, ref)}

    orig_run = graphs.DeviceCommitGraph.run

    def run_behind(self, state_rows):
        torch.cuda._sleep(3_000_000)        # a few ms of spinning ahead of the copy
        orig_run(self, state_rows)

    def run(prelaunch, slow):
        raw, calls = [], {"n": 0}

        def override(seqs, tokens):
            k, bs = tokens.shape
            # stays on the device; keyed per sequence (column orders may differ)
            raw.append(([tuple(seq.prompt_token_ids) for seq in seqs],
                        tokens[:, :len(seqs)].clone()))
            want = torch.zeros(k, bs, dtype=torch.int64, pin_memory=True)
            for i, seq in enumerate(seqs):
                cont = full[tuple(seq.prompt_token_ids)][len(seq):len(seq) + k]
                calls["n"] += 1
                for s_, tok in enumerate(cont):
                    want[s_, i] = tok
                if calls["n"] % 4 == 0:
                    want[calls["n"] % k, i] = (int(want[calls["n"] % k, i]) + 1) % 2048
            tokens.copy_(want.to(tokens.device, non_blocking=True))

        if slow:
            monkeypatch.setattr(graphs.DeviceCommitGraph, "run", run_behind)
        else:
            monkeypatch.setattr(graphs.DeviceCommitGraph, "run", orig_run)
        llm = make_llm(dirs, spec=True, k=5, eager=False)
        llm.prelaunch_draft = prelaunch
        llm.model_runner.draft_override = override
        try:
            for p, m in zip(ps, max_tokens):
                llm.add_request(p, SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True))
            outs = {}
            while not llm.is_finished():
                for seq_id, toks in llm.step()[0]:
                    outs[seq_id] = toks
            runner = llm.model_runner
            waits = sum(g.i64.waits for g in runner._device_commit_graphs.values())
            waits += sum(g.meta.waits + g.meta32.waits for g in runner._chained_graphs.values())
            per_seq = [{key: t[:, i].cpu() for i, key in enumerate(keys)} for keys, t in raw]
            return ([outs[i] for i in sorted(outs)], per_seq,
                    dict(llm.spec_stats), dict(runner.prelaunch_stats), waits)
        finally:
            llm.exit()

    got_on, raw_on, stats_on, pre_on, waits_on = run(True, slow=True)
    got_off, raw_off, stats_off, pre_off, _ = run(False, slow=False)
    print(f"prelaunch {pre_on}, refills that waited for a queued copy: {waits_on}", flush=True)
    assert pre_on["used"] >= 5, pre_on
    assert waits_on > 0
    assert stats_on == stats_off and stats_on["accepted"] > stats_on["steps"]
    assert got_on == got_off
    assert len(raw_on) == len(raw_off)
    for step, (a, b) in enumerate(zip(raw_on, raw_off)):
        assert a.keys() == b.keys(), step
        for key in a:
            assert torch.equal(a[key], b[key]), step
