"""Benchmark: EAGLE3 speculative decode steps, Qwen3-8B geometry, k=5, batch 64
random-init weights, synthetic prompts.

One "step" is one speculative decode step of LLMEngine over the whole batch
(propose k drafts, verify k+1 rows per sequence, accept, commit).  ``value``
is accepted tok/s = tokens committed in the K timed steps / their wall time
(the reference's definition, llm_engine.py:175-185), with every sequence
already prefilled (prefill is not timed).

The same JSON line carries
  roofline:      the verify attention kernel (K1), timed with HIP events on
                 its stream around every verify-attention launch of
                 --roofline-steps further steps of the same workload (the
                 timed steps replay HIP graphs, inside which ROCm torch cannot
                 record timing events, so these steps launch the verify
                 forward eagerly); achieved = algorithmic bytes per launch /
                 mean launch time, algorithmic bytes = sum_i L_i*Hkv*D*2B*2
                 (K and V read once) + T*Hq*D*2B*2 (Q in, O out);
  cpu_baseline:  the reference's host acceptance logic (per-sequence bf16
                 argmax + .tolist() + verify_greedy_proposals) timed on this
                 host's cores over verify batches copied from the run.
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "extend-nano-vllm_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "accepted tok/s, Qwen3-8B EAGLE3 k=5 bs64; verify-attn HBM GB/s % of peak"


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--k", type=int, default=5)
    ap.add_argument("--preset", default="qwen3-8b")
    ap.add_argument("--prompt-min", type=int, default=256)
    ap.add_argument("--prompt-max", type=int, default=2048)
    ap.add_argument("--max-tokens", type=int, default=256)
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--eager", action="store_true", help="disable HIP graphs")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bound on the CPU-baseline sample's run time")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--roofline-steps", type=int, default=5,
                    help="extra steps with the verify forward run eagerly so that every "
                         "verify-attention launch is bracketed by HIP events")
    return ap.parse_args()


class AttnTimer:
    """Brackets each verify-attention launch with HIP events on the current
    stream (the stream the kernels are enqueued on) and records its
    algorithmic bytes from the host-side metadata."""

    def __init__(self):
        self.enabled = False
        self.events = []
        self.bytes = []

    def wrap(self, kernels):
        import torch

        orig = kernels.paged_attention_varlen
        timer = self

        def timed(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                  softmax_scale, block_table, causal=True, k_scale=None, v_scale=None, out=None):
            if not timer.enabled or timer.current_lens is None:
                return orig(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                            max_seqlen_k, softmax_scale, block_table, causal, k_scale, v_scale, out)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            o = orig(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                     softmax_scale, block_table, causal, k_scale, v_scale, out)
            e.record()
            hkv, d = k_cache.shape[2], k_cache.shape[3]
            esz = k_cache.element_size()
            kv = sum(timer.current_lens) * hkv * d * esz * 2
            qo = q.shape[0] * q.shape[1] * d * 2 * 2
            timer.events.append((s, e))
            timer.bytes.append(kv + qo)
            return o

        self.current_lens = None
        kernels.paged_attention_varlen = timed
        import nanovllm_amd.layers as layers
        layers.K.paged_attention_varlen = timed

    def result(self):
        import torch

        torch.cuda.synchronize()
        ms = [s.elapsed_time(e) for s, e in self.events]
        if not ms:
            return None
        mean_ms = sum(ms) / len(ms)
        mean_bytes = sum(self.bytes) / len(self.bytes)
        gbs = mean_bytes / (mean_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "paged_attention_kernel (+ split combine)",
                "launches": len(ms), "mean_us": round(mean_ms * 1e3, 2),
                "bytes_per_launch": int(mean_bytes)}


def cpu_baseline(batches, seconds):
    """Reference host acceptance on CPU torch, bounded to ~``seconds``."""
    import torch
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    logits, cu, ids = batches[0]
    for _ in range(2):
        oracle.reference_cpu_acceptance(logits, cu, ids)
    times, committed = [], 0
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end or len(times) < 3:
        logits, cu, ids = batches[i % len(batches)]
        t0 = time.perf_counter()
        _, _, c = oracle.reference_cpu_acceptance(logits, cu, ids)
        times.append(time.perf_counter() - t0)
        committed += c
        i += 1
    total = sum(times)
    return {"value": round(committed / total, 1), "unit": "accepted tok/s (acceptance logic only)",
            "cores": cores, "kind": "port",
            "sample": f"{len(times)} verify batches of [{logits.shape[0]}, {logits.shape[1]}] bf16 "
                      f"logits from this run ({len(cu) - 1} sequences each), per-sequence "
                      f"argmax+tolist+verify_greedy_proposals, torch CPU with {cores} threads on "
                      f"{model}; {total / len(times) * 1e3:.1f} ms per batch"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported by this build "
              "(single-GPU hot path; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)
    import torch

    from nanovllm_amd import LLM, SamplingParams
    from nanovllm_amd import kernels
    from nanovllm_amd.synthetic import default_aux_layers, write_eagle3_config, write_qwen3_config

    timer = AttnTimer()
    timer.wrap(kernels)

    tmp = tempfile.mkdtemp(prefix="nva_bench_")
    target = write_qwen3_config(os.path.join(tmp, "target"), args.preset)
    aux = default_aux_layers(args.preset)
    draft = write_eagle3_config(os.path.join(tmp, "draft"), args.preset, aux_layers=aux)
    max_len = args.prompt_max + args.max_tokens
    blocks_per_seq = -(-(max_len + args.k + 1) // 256)
    llm = LLM(target, load_format="dummy", seed=0, max_num_seqs=args.batch,
              max_model_len=max_len, num_kvcache_blocks=args.batch * blocks_per_seq + 8,
              max_num_batched_tokens=16384, enable_prefill_batching=True,
              enforce_eager=args.eager,
              speculative_config={"method": "eagle3", "model": draft,
                                  "num_speculative_tokens": args.k,
                                  "aux_hidden_state_layers": aux})
    runner = llm.model_runner
    log(f"engine up: {runner.get_diagnostics()}")
    vocab = llm.config.hf_config.vocab_size
    g = torch.Generator().manual_seed(args.seed)
    lens = torch.randint(args.prompt_min, args.prompt_max + 1, (args.batch,), generator=g).tolist()
    sp = SamplingParams(temperature=0.0, max_tokens=args.max_tokens, ignore_eos=True)
    for L in lens:
        llm.add_request(torch.randint(0, vocab, (L,), generator=g).tolist(), sp)

    t_setup = time.perf_counter()
    while llm.scheduler.waiting:
        llm.step()
    log(f"prefill done in {time.perf_counter() - t_setup:.1f}s")
    for _ in range(args.warmup):
        llm.step()
    log("warmup done")
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    # capture verify batches for the CPU baseline (outside the timed region)
    cpu_batches = []
    runner.keep_verify_inputs = True

    orig_verify = runner.verify_eagle3_batch_fused

    def verify_with_lens(seqs, n):
        timer.current_lens = [len(s) for s in seqs]
        try:
            return orig_verify(seqs, n)
        finally:
            timer.current_lens = None

    runner.verify_eagle3_batch_fused = verify_with_lens
    if not args.no_cpu_baseline:
        llm.step()
        logits, cu, ids = runner.last_verify_inputs
        cpu_batches.append((logits.cpu(), list(cu), ids.cpu().tolist()))
    runner.keep_verify_inputs = False
    runner.last_verify_inputs = None

    n_active = len(llm.scheduler.running)
    before = dict(llm.spec_stats)
    committed = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        _, num_tokens = llm.step()
        committed += -num_tokens
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    elapsed = t1 - t0
    stats = {k: llm.spec_stats[k] - before[k] for k in before}

    # roofline: the same workload for a few more steps with the verify forward
    # launched eagerly (events cannot be recorded inside a captured HIP graph
    # on ROCm); the kernels and their inputs are those of the timed steps
    runner.use_verify_graph = False
    timer.enabled = True
    for _ in range(args.roofline_steps):
        llm.step()
    torch.cuda.synchronize()
    timer.enabled = False
    runner.use_verify_graph = True
    roof = timer.result()

    log(f"timed {args.steps} steps in {elapsed:.3f}s")
    cpu = None
    if cpu_batches:
        cpu = cpu_baseline(cpu_batches, args.cpu_seconds)
    llm.exit()

    result = {
        "metric": METRIC,
        "value": round(committed / elapsed, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random prompt ids)",
        "config": {"workload": "EAGLE3 speculative decode step, Qwen3-8B geometry (36 layers, "
                               "H4096, 32q/8kv, D128, MLP12288, V151936), draft 1 layer + fc 3H->H "
                               "on aux layers 2/18/33",
                   "preset": args.preset, "batch": args.batch, "k": args.k,
                   "prompt_len": [args.prompt_min, args.prompt_max],
                   "max_tokens": args.max_tokens, "active_seqs": n_active,
                   "hip_graphs": not args.eager},
        "roofline": roof,
        "cpu_baseline": cpu,
        "committed_tokens": committed,
        "accepted_drafts_per_seq_step": round(stats["accepted"] / max(stats["steps"] * n_active, 1), 4),
        "committed_per_seq_step": round(stats["committed"] / max(stats["steps"] * n_active, 1), 4),
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
