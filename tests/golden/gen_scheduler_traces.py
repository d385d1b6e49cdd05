"""Writes tests/golden/scheduler_traces.json: step-by-step traces of the
reference's own Scheduler / BlockManager / Sequence (nanovllm/engine/
scheduler.py, block_manager.py, sequence.py) driven through prefill and
speculative decode by tests/helpers.scheduler_trace.

Run in the build container, where the reference is mounted read-only:
    python tests/golden/gen_scheduler_traces.py
The reference does not travel: the JSON holds only inputs (prompts, drawn
tokens, proposals, acceptance lengths) and the reference's resulting states.
"""
import json
import os
import random
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))            # tests/ (helpers)
sys.path.insert(0, "/root/reference")

from helpers import scheduler_trace  # noqa: E402
from nanovllm.engine.scheduler import Scheduler  # noqa: E402
from nanovllm.engine.sequence import Sequence  # noqa: E402
from nanovllm.sampling_params import SamplingParams  # noqa: E402


def prompts(rng, lens, shared=()):
    out = [[rng.randrange(1000) for _ in range(n)] for n in lens]
    for dst, src, n in shared:          # dst starts with src's first n tokens
        out[dst][:n] = out[src][:n]
    return out


def scenarios():
    rng = random.Random(1234)
    base = dict(eos=7, p_eos=0.02, prefix_caching=True, max_steps=400)
    sc = []
    # speculative k=5, batched chunked prefill, shared 512-token prefixes,
    # prompt lengths at and around page boundaries
    lens = [300, 512, 700, 255, 256, 900, 513]
    ps = prompts(rng, lens, shared=[(5, 2, 512), (6, 1, 512)])
    sc.append(dict(base, name="spec_k5_prefix_sharing", k=5, max_num_seqs=8,
                   max_num_batched_tokens=1024, enable_prefill_batching=True, num_blocks=64,
                   requests=[dict(prompt=p, max_tokens=m, ignore_eos=ie) for p, m, ie in
                             zip(ps, [40, 31, 64, 5, 17, 50, 23],
                                 [False, True, False, False, True, False, False])]))
    # speculative k=8, one prefill per step, long outputs crossing pages
    lens = [250, 10, 480, 1000]
    ps = prompts(rng, lens)
    sc.append(dict(base, name="spec_k8_page_crossings", k=8, max_num_seqs=4,
                   max_num_batched_tokens=4096, enable_prefill_batching=False, num_blocks=24,
                   p_eos=0.01,
                   requests=[dict(prompt=p, max_tokens=m, ignore_eos=False) for p, m in
                             zip(ps, [300, 270, 90, 33])]))
    # speculative k=3 under block pressure (preemption and re-prefill)
    lens = [700, 650, 600, 520, 400]
    ps = prompts(rng, lens, shared=[(1, 0, 256)])
    sc.append(dict(base, name="spec_k3_block_pressure", k=3, max_num_seqs=5,
                   max_num_batched_tokens=2048, enable_prefill_batching=True, num_blocks=16,
                   p_eos=0.0,
                   requests=[dict(prompt=p, max_tokens=m, ignore_eos=True) for p, m in
                             zip(ps, [200, 150, 180, 120, 90])]))
    # plain decode (no speculation) for the same bookkeeping
    lens = [260, 511, 33]
    ps = prompts(rng, lens)
    sc.append(dict(base, name="plain_decode", k=0, max_num_seqs=3,
                   max_num_batched_tokens=512, enable_prefill_batching=True, num_blocks=12,
                   requests=[dict(prompt=p, max_tokens=m, ignore_eos=False) for p, m in
                             zip(ps, [30, 20, 300])]))
    # speculation landing exactly on page boundaries: prompts just below a
    # page, k=4, long outputs, so truncations, bonus tokens and page
    # finalisation meet at len % 256 == 0 again and again
    lens = [250, 251, 252, 253, 254, 255]
    ps = prompts(rng, lens)
    sc.append(dict(base, name="spec_k4_page_boundaries", k=4, max_num_seqs=6,
                   max_num_batched_tokens=4096, enable_prefill_batching=True, num_blocks=20,
                   p_eos=0.0, max_steps=300,
                   requests=[dict(prompt=p, max_tokens=m, ignore_eos=True) for p, m in
                             zip(ps, [520, 300, 400, 280, 310, 530])]))
    # plain decode under block pressure: decode preempts the newest running
    # sequence when a page boundary finds no free block, then re-prefills it
    lens = [500, 490, 250]
    ps = prompts(rng, lens)
    sc.append(dict(base, name="plain_decode_preemption", k=0, max_num_seqs=3,
                   max_num_batched_tokens=2048, enable_prefill_batching=True, num_blocks=7,
                   p_eos=0.0,
                   requests=[dict(prompt=p, max_tokens=m, ignore_eos=True) for p, m in
                             zip(ps, [40, 30, 60])]))
    # speculative reservation with the pool exhausted: the reference raises
    lens = [500, 490]
    ps = prompts(rng, lens)
    sc.append(dict(base, name="spec_k4_pool_exhausted", k=4, max_num_seqs=2,
                   max_num_batched_tokens=2048, enable_prefill_batching=True, num_blocks=5,
                   p_eos=0.0,
                   requests=[dict(prompt=p, max_tokens=m, ignore_eos=True) for p, m in
                             zip(ps, [300, 300])]))
    return sc


def main():
    out = []
    for i, sc in enumerate(scenarios()):
        inputs, snaps, final = scheduler_trace(Scheduler, Sequence, SamplingParams, sc,
                                               seed=100 + i)
        out.append({"scenario": sc, "inputs": inputs, "snapshots": snaps, "final_tokens": final})
        print(f"{sc['name']}: {len(snaps)} steps", flush=True)
    path = os.path.join(HERE, "scheduler_traces.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
