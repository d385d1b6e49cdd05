"""Input generators shared by the tests (seeded, generated on the CPU so the
GPU kernels and the CPU oracle consume byte-identical data)."""
from __future__ import annotations

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """Storage bits of a CPU bf16 / fp8 tensor as a numpy array."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    raise TypeError(t.dtype)


def from_bits(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.bfloat16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    if dtype == torch.float8_e4m3fn:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8)).view(torch.float8_e4m3fn)
    raise TypeError(dtype)


def acceptance_logits(batch: int, k: int, vocab: int, p_accept: float, seed: int):
    """Config-1 style verify batch: bf16 logits [B*(k+1), V] ~ N(0,1); for
    each (sequence, draft position j < k), with probability p_accept the
    draft token's logit is raised to the row max + 1.0 (in fp32, then cast).

    Returns (logits bf16 CPU, cu_q int32, input_ids int64, proposals [B, k])."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(batch, k + 1, vocab, generator=g)
    proposals = torch.randint(0, vocab, (batch, k), generator=g)
    raise_mask = torch.rand(batch, k, generator=g) < p_accept
    for s in range(batch):
        for j in range(k):
            if raise_mask[s, j]:
                row = logits[s, j]
                row[proposals[s, j]] = row.max() + 1.0
    logits = logits.to(torch.bfloat16).reshape(batch * (k + 1), vocab)
    cu_q = torch.arange(0, batch * (k + 1) + 1, k + 1, dtype=torch.int32)
    input_ids = torch.zeros(batch, k + 1, dtype=torch.int64)
    input_ids[:, 0] = torch.randint(0, vocab, (batch,), generator=g)
    input_ids[:, 1:] = proposals
    return logits, cu_q, input_ids.reshape(-1), proposals


def paged_case(seed: int, batch: int, q_len, ctx_lo: int, ctx_hi: int, hq: int, hkv: int,
               head_dim: int = 128, block_size: int = 256, spare_blocks: int = 3,
               scale: float = 0.5):
    """A shuffled paged KV layout plus new rows to verify.

    q_len: int or list per sequence.  Context lengths L_i ~ U[ctx_lo, ctx_hi]
    include the q_i new rows.  Returns a dict of CPU tensors: q [T,Hq,D],
    k_new/v_new [T,Hkv,D], k_cache/v_cache [NB,bs,Hkv,D] (random old
    content), block_tables [B, max_blocks] (-1 padded), cu_q, cu_k, lens,
    slot_mapping [T]."""
    g = torch.Generator().manual_seed(seed)
    qs = [q_len] * batch if isinstance(q_len, int) else list(q_len)
    lens = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=g).tolist()
    lens = [max(L, q) for L, q in zip(lens, qs)]
    nblk = [(L + block_size - 1) // block_size for L in lens]
    total = sum(nblk) + spare_blocks
    perm = torch.randperm(total, generator=g).tolist()
    max_blocks = max(nblk) + 1
    bt = torch.full((batch, max_blocks), -1, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = torch.tensor(perm[pos:pos + n], dtype=torch.int32)
        pos += n
    t = sum(qs)
    k_cache = (torch.randn(total, block_size, hkv, head_dim, generator=g) * scale).to(torch.bfloat16)
    v_cache = (torch.randn(total, block_size, hkv, head_dim, generator=g) * scale).to(torch.bfloat16)
    q = (torch.randn(t, hq, head_dim, generator=g) * scale).to(torch.bfloat16)
    k_new = (torch.randn(t, hkv, head_dim, generator=g) * scale).to(torch.bfloat16)
    v_new = (torch.randn(t, hkv, head_dim, generator=g) * scale).to(torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum(qs).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    slots = []
    for i, (L, qn) in enumerate(zip(lens, qs)):
        for p in range(L - qn, L):
            slots.append(int(bt[i, p // block_size]) * block_size + p % block_size)
    return dict(q=q, k_new=k_new, v_new=v_new, k_cache=k_cache, v_cache=v_cache,
                block_tables=bt, cu_q=cu_q, cu_k=cu_k, lens=torch.tensor(lens, dtype=torch.int32),
                slot_mapping=torch.tensor(slots, dtype=torch.int32), q_lens=qs,
                block_size=block_size)


# ---------------------------------------------------------------- scheduler traces

def scheduler_trace(Scheduler, Sequence, SamplingParams, scenario, inputs=None, seed=0):
    """Drive a Scheduler through prefill and speculative (or plain) decode
    steps in the order LLMEngine.step uses them (llm_engine.py:118-186 of the
    reference): reserve_speculation for every sequence, begin_speculation
    with k' = min(k, max_tokens - completion) proposals, num_computed =
    base - 1, then postprocess_speculation with the accepted prefix and the
    replacement token.  With ``inputs=None`` the tokens, proposals and
    acceptance lengths are drawn from ``random.Random(seed)`` and recorded;
    otherwise the recorded ones are replayed.  Returns (inputs, snapshots):
    one snapshot of every sequence, the block manager and the queues after
    each step.  Implementation-agnostic: the classes are passed in."""
    import random
    from types import SimpleNamespace

    sc = scenario
    spec = SimpleNamespace(num_speculative_tokens=sc["k"]) if sc["k"] else None
    cfg = SimpleNamespace(max_num_seqs=sc["max_num_seqs"],
                          max_num_batched_tokens=sc["max_num_batched_tokens"],
                          enable_prefill_batching=sc["enable_prefill_batching"],
                          speculative_config=spec, eos=sc["eos"],
                          num_kvcache_blocks=sc["num_blocks"], kvcache_block_size=256,
                          enable_prefix_caching=sc["prefix_caching"])
    sched = Scheduler(cfg)
    seqs = []
    for req in sc["requests"]:
        sp = SamplingParams(temperature=0.0 if sc["k"] else 1.0, max_tokens=req["max_tokens"],
                            ignore_eos=req["ignore_eos"])
        seq = Sequence(list(req["prompt"]), sp)
        seqs.append(seq)
        sched.add(seq)
    index = {id(s): i for i, s in enumerate(seqs)}
    rng = random.Random(seed)
    record = inputs is None
    inputs = [] if record else list(inputs)
    eos, k = sc["eos"], sc["k"]

    def tok():
        return eos if rng.random() < sc["p_eos"] else rng.randrange(1000)

    def snapshot(step_seqs, is_prefill):
        bm = sched.block_manager
        return {
            "scheduled": [index[id(s)] for s in step_seqs],
            "is_prefill": bool(is_prefill),
            "seqs": [[s.status.name, len(s), s.num_computed_tokens, s.num_cached_tokens,
                      list(s.block_table), s.num_completion_tokens, s.last_token] for s in seqs],
            "waiting": [index[id(s)] for s in sched.waiting],
            "running": [index[id(s)] for s in sched.running],
            "free": list(bm.free_block_ids),
            "used": sorted(bm.used_block_ids),
            "blocks": [[b.block_id, b.ref_count, b.hash, bool(b.ready), len(b.token_ids)]
                       for b in bm.blocks if b.ref_count],
            "hash_to_block": sorted([h, i] for h, i in bm.hash_to_block_id.items()),
            "bm_stats": dict(bm.stats),
            "stats": dict(sched.stats),
        }

    snaps = []
    step = 0
    while not sched.is_finished() and step < sc["max_steps"]:
        try:
            step_seqs, is_prefill = _trace_step(sched, step, record, inputs, tok, rng, k)
        except (RuntimeError, ValueError, AssertionError) as exc:
            # the reference's own failure (e.g. blocks exhausted by a
            # speculative reservation) ends the trace; the message is part
            # of the contract
            snaps.append({"error": f"{type(exc).__name__}: {exc}"})
            break
        snaps.append(snapshot(step_seqs, is_prefill))
        step += 1
    final = [list(s.token_ids) for s in seqs]
    return inputs, snaps, final


def _trace_step(sched, step, record, inputs, tok, rng, k):
    """One engine step of scheduler_trace (see there)."""
    step_seqs, is_prefill = sched.schedule()
    if is_prefill or not k:
        if record:
            toks = [tok() for _ in step_seqs]
            inputs.append({"tokens": toks})
        else:
            toks = inputs[step]["tokens"]
        sched.postprocess(step_seqs, toks, is_prefill)
    else:
        for s in step_seqs:
            sched.reserve_speculation(s)
        if record:
            props, acc, repl = [], [], []
            for s in step_seqs:
                n = min(k, s.max_tokens - s.num_completion_tokens)
                props.append([tok() for _ in range(n)])
                acc.append(rng.randint(0, n))
                repl.append(tok())
            inputs.append({"proposals": props, "accept": acc, "replacement": repl})
        else:
            props = inputs[step]["proposals"]
            acc = inputs[step]["accept"]
            repl = inputs[step]["replacement"]
        bases = []
        for s, p in zip(step_seqs, props):
            base = sched.begin_speculation(s, list(p))
            bases.append(base)
            s.num_computed_tokens = base - 1
        for s, p, base, a, r in zip(step_seqs, props, bases, acc, repl):
            sched.postprocess_speculation(s, base, list(p[:a]), r)
    return step_seqs, is_prefill


# ---------------------------------------------------------------- full-size device cases

def device_paged_case(dev, seed, batch, q_len, ctx_lo, ctx_hi, hq, hkv, fp8=False,
                      shared_frac=0.0, head_dim=128, block_size=256):
    """A BASELINE-sized verify batch built on the device (too large for the
    CPU oracle): lengths L_i ~ U[ctx_lo, ctx_hi] (the q_len new rows
    included), shuffled physical blocks in the engine's page order
    ([blocks, Hkv, 2, block_size, D]: a head's K rows then its V rows, seen
    as [blocks, block_size, Hkv, D] views), and the first ``shared_frac`` of
    every sequence's blocks taken from one shared prefix (the same physical
    ids for every sequence).  Returns a dict of device tensors."""
    import torch

    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=g).tolist()
    nblk = [-(-L // block_size) for L in lens]
    nshared = [int(n * shared_frac) for n in nblk]
    prefix = max(nshared)
    total = prefix + sum(n - s for n, s in zip(nblk, nshared))
    perm = torch.randperm(total, generator=g)
    shared_ids, own_ids = perm[:prefix], perm[prefix:]
    bt = torch.full((batch, max(nblk)), -1, dtype=torch.int32)
    off = 0
    for i, (n, s) in enumerate(zip(nblk, nshared)):
        bt[i, :s] = shared_ids[:s].to(torch.int32)
        bt[i, s:n] = own_ids[off:off + n - s].to(torch.int32)
        off += n - s
    gd = torch.Generator(device=dev).manual_seed(seed)
    pages = torch.empty(total, hkv, 2, block_size, head_dim, dtype=torch.bfloat16, device=dev)
    pages.normal_(0.0, 0.5, generator=gd)
    if fp8:
        pages = pages.to(torch.float8_e4m3fn)
    view = pages.permute(2, 0, 3, 1, 4)
    t = batch * q_len
    q = (torch.randn(t, hq, head_dim, generator=gd, device=dev) * 0.5).to(torch.bfloat16)
    cu_q = torch.arange(0, t + 1, q_len, dtype=torch.int32)
    cu_k = torch.tensor([0] + lens, dtype=torch.int64).cumsum(0).to(torch.int32)
    return {"pages": pages, "k_cache": view[0], "v_cache": view[1], "q": q,
            "cu_q": cu_q.to(dev), "cu_k": cu_k.to(dev), "lens": lens, "q_len": q_len,
            "block_tables": bt.to(dev), "max_k": max(lens)}
