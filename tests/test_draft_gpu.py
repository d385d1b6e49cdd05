"""The EAGLE3 draft step on the GPU against the CPU float32 restatement
(oracle/draft_oracle.py), through the engine's own step.

After the prefill, the draft's recurrent states and its paged K/V history
are copied to the host.  One speculative step then runs: the proposal loop
(ProposeGraph, or the eager loop), the target verify, and the batched draft
commit (DeviceCommitGraph on the pipelined path, commit_eagle3_batch
otherwise).  The restatement replays, per sequence:

* the proposals from the stored states, fed with the device's own tokens so
  that a near tie does not compound: every device proposal must be the
  restatement's argmax or within MARGIN_TOL of its top logit
  (eagle3.py:294-296, model_runner.py:1159-1213);
* the commit of the accepted tail from the verify's aux rows, one token
  after the other (model_runner.py:1127-1156, :1216-1249): the new
  recurrent states and the draft K/V rows written at the committed
  positions must agree within bf16 tolerance.

The batched commit is also compared with commit_eagle3_serial, the
reference's one-token-at-a-time structure on the same kernels.

The draft's norm weights are moved away from one and d2t permutes the
vocabulary, so that a swapped norm or a skipped id map would show.
Target verification is exact, so the engine's greedy-equality tests cannot
see a wrong draft; these can.
"""
import pytest
import torch

from nanovllm_amd import LLM, SamplingParams
from nanovllm_amd.synthetic import write_eagle3_config, write_qwen3_config
from oracle import draft_oracle as D

pytestmark = pytest.mark.gpu

AUX = (1, 2, 4)
K_SPEC = 4
MARGIN_TOL = 2e-2
# relative L2 error of a state or K/V block against the float32 restatement
# (the device rounds to bf16 after every op, as the reference does)
STATE_RTOL = 3e-2


@pytest.fixture(scope="module")
def dirs(tmp_path_factory):
    root = tmp_path_factory.mktemp("draft_ckpt")
    return (write_qwen3_config(str(root / "target"), "tiny"),
            write_eagle3_config(str(root / "draft"), "tiny", aux_layers=AUX))


def _perturb(model, seed=7):
    """Norm weights 1 + 0.2 N(0, 1) and d2t = a permutation of the ids
    (target id = perm[draft id]); returns the inverse permutation."""
    g = torch.Generator().manual_seed(seed)
    layer = model.layers[0]
    for norm in (layer.hidden_norm, layer.input_layernorm, layer.post_attention_layernorm,
                 model.norm):
        w = 1 + 0.2 * torch.randn(norm.weight.shape, generator=g)
        norm.weight.data.copy_(w.to(norm.weight.dtype))
    v = model.d2t.numel()
    perm = torch.randperm(v, generator=g)
    model.d2t.copy_((perm - torch.arange(v)).to(model.d2t.device))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(v)
    return inv


def _history(runner, block_table, n):
    """Draft K/V of positions [0, n) of one sequence, float32 [n, Hkv, D]."""
    pos = torch.arange(n)
    blocks = torch.tensor(block_table, dtype=torch.long)[pos // runner.block_size]
    off = pos % runner.block_size
    kc, vc = runner.eagle_kv_cache[0, 0], runner.eagle_kv_cache[1, 0]
    dev = kc.device
    return (kc[blocks.to(dev), off.to(dev)].float().cpu(),
            vc[blocks.to(dev), off.to(dev)].float().cpu())


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30))


@pytest.mark.parametrize("eager", [False, True])
def test_draft_step_matches_restatement(dirs, eager):
    target, draft = dirs
    llm = LLM(target, load_format="dummy", seed=0, max_model_len=2048, num_kvcache_blocks=96,
              enforce_eager=eager, max_num_batched_tokens=4096,
              speculative_config={"method": "eagle3", "model": draft,
                                  "num_speculative_tokens": K_SPEC,
                                  "aux_hidden_state_layers": AUX})
    try:
        runner = llm.model_runner
        inv = _perturb(runner.eagle3_model)
        w = D.DraftWeights.from_module(runner.eagle3_model)
        g = torch.Generator().manual_seed(11)
        # prompt lengths put some proposal / commit positions across a page
        lens = [40, 254, 255, 300, 511]
        sp = SamplingParams(temperature=0.0, max_tokens=64, ignore_eos=True)
        for n in lens:
            llm.add_request(torch.randint(0, 2048, (n,), generator=g).tolist(), sp)
        while llm.scheduler.waiting:                          # prefills, one per step
            llm.step()
        seqs = list(llm.scheduler.running)
        assert len(seqs) == len(lens)
        snap = {}
        for seq in seqs:
            row = runner._state_slot[seq.seq_id]
            kh, vh = _history(runner, seq.block_table, len(seq) - 1)
            snap[seq.seq_id] = dict(base=len(seq), hidden=runner.state_hidden[row].float().cpu(),
                                    feedback=runner.state_feedback[row].float().cpu(),
                                    k=kh, v=vh)
        seen = {}

        def recorder(name):
            inner = getattr(runner, name)

            def wrapped(step_seqs, *rest):
                props = inner(step_seqs, *rest)
                if props is not None:
                    seen.update({s.seq_id: list(p) for s, p in zip(step_seqs, props)})
                return props
            return wrapped

        runner.propose_verify_eagle3_batch = recorder("propose_verify_eagle3_batch")
        runner.propose_eagle3_batch = recorder("propose_eagle3_batch")
        llm.step()                                            # one speculative step
        torch.cuda.synchronize()
        assert sorted(seen) == sorted(snap)

        # ---- proposals
        exact = total = 0
        for sid, s in snap.items():
            props = seen[sid]
            toks, rows, _, _ = D.propose(w, s["hidden"], s["feedback"], s["base"] - 1,
                                         len(props), s["k"], s["v"], forced=props)
            for j, (got, want) in enumerate(zip(props, toks)):
                total += 1
                exact += got == want
                row = rows[j]
                gap = float(row.max() - row[int(inv[got])])
                assert gap < MARGIN_TOL, (sid, j, got, want, gap)
        assert exact >= 0.8 * total, (exact, total)

        # ---- batched commit: recurrent states and the K/V rows it wrote
        aux_pairs, cu, index = runner._pending_verify
        from nanovllm_amd.qwen3 import aux_concat

        aux = aux_concat(aux_pairs)
        by_id = {seq.seq_id: seq for seq in seqs}
        committed = []
        for sid, s in snap.items():
            seq = by_id[sid]
            tail = seq.token_ids[s["base"]:]
            assert 1 <= len(tail) <= K_SPEC + 1
            p = index[sid]
            rows_aux = aux[cu[p]:cu[p] + len(tail)]
            start = s["base"] - 1
            normed, pre, ks, vs = D.commit(w, tail, rows_aux.float().cpu(), start, s["k"],
                                           s["v"])
            row = runner._state_slot[sid]
            got_k, got_v = _history(runner, seq.block_table, start + len(tail))
            assert _rel(runner.state_hidden[row].cpu(), normed) < STATE_RTOL, sid
            assert _rel(runner.state_feedback[row].cpu(), pre) < STATE_RTOL, sid
            assert _rel(got_k[start:], ks) < STATE_RTOL, sid
            assert _rel(got_v[start:], vs) < STATE_RTOL, sid
            # the positions before the commit are untouched
            assert torch.equal(got_k[:start], s["k"][:start])
            committed.append((seq, tail, rows_aux, start, row))

        # ---- batched commit == the reference's serial structure
        batched = {row: (runner.state_hidden[row].clone(), runner.state_feedback[row].clone())
                   for _, _, _, _, row in committed}
        for seq, tail, rows_aux, start, row in committed:
            runner.commit_eagle3_serial(seq, tail, rows_aux, start)
        torch.cuda.synchronize()
        for seq, tail, rows_aux, start, row in committed:
            bh, bf = batched[row]
            assert _rel(runner.state_hidden[row], bh) < 1e-2, seq.seq_id
            assert _rel(runner.state_feedback[row], bf) < 1e-2, seq.seq_id
    finally:
        llm.exit()
