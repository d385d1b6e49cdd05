"""Benchmark: EAGLE3 speculative decode steps, Qwen3-8B geometry, k=5, batch 64
random-init weights, synthetic prompts.

One "step" is one speculative decode step of LLMEngine over the whole batch
(propose k drafts, verify k+1 rows per sequence, accept, commit).  ``value``
is accepted tok/s = tokens committed in the K timed steps / their wall time
(the reference's definition, llm_engine.py:175-185), with every sequence
already prefilled (prefill is not timed).

The same JSON line carries
  roofline:      the verify attention call (K1: attention kernel + split
                 combine), timed with HIP events on its stream: one further
                 step of the same workload runs its verify forward eagerly
                 (the timed steps replay HIP graphs, inside which ROCm torch
                 cannot record timing events), and its 36 verify-attention
                 launches are re-issued back to back --roofline-repeats times
                 between two events; achieved = algorithmic bytes per launch /
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
DEFAULT_GEMM_TUNING = os.path.join(ROOT, "extend-nano-vllm_amd", "nanovllm_amd", "tuning",
                                   "gemm_mi355x_qwen3_8b_eagle3.csv")

# HBM bytes per verify-attention call on this workload, from two rocprofv3
# --pmc runs of `bench.py --attention-only` (FETCH_SIZE, then WRITE_SIZE;
# KiB per dispatch, averaged over the 75 calls of `--attention-only
# --roofline-repeats 2`), scaled by what the same counters read for a 1 GiB
# device copy in the same runs: FETCH_SIZE 524301 KiB (x2.0 to bytes read),
# WRITE_SIZE 1048576 KiB (x1.0).  attention kernel: FETCH 158667.1, WRITE
# 3072.0 (no sequence of this workload needs a second split, so no combine
# kernel runs).  Only quoted for the default workload, whose shapes it was
# measured on.
PMC_TRAFFIC_BYTES = int((158667.1 * 2.0 + 3072.0 * 1.0) * 1024)
PMC_WORKLOAD = dict(preset="qwen3-8b", batch=64, k=5, prompt_min=256, prompt_max=2048,
                    max_tokens=256, seed=2)
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
    ap.add_argument("--roofline-repeats", type=int, default=10,
                    help="times the verify-attention launches of one step are re-issued "
                         "between HIP events for the roofline figure")
    ap.add_argument("--reference-steps", type=int, default=3,
                    help="steps timed with the reference's step structure for comparison "
                         "(0 to skip)")
    ap.add_argument("--gemm-tuning", default=DEFAULT_GEMM_TUNING,
                    help="TunableOp results for the projection GEMMs ('' for library defaults)")
    ap.add_argument("--kv-layout", default="head_major", choices=["head_major", "token_major"],
                    help="physical order inside a KV page (the engine's kv_cache_layout)")
    ap.add_argument("--kernels", action="store_true",
                    help="time each hot-path kernel alone on the seeded synthetic inputs of "
                         "BASELINE configs 1, 2, 4 and 5 (and config 3's shapes); one JSON line "
                         "per kernel and config")
    ap.add_argument("--batch-order", default="longest_first", choices=["longest_first", "drawn"],
                    help="--kernels: sequences longest first (the engine's verify order) or "
                         "in the order drawn")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the verify-attention launches of the workload and a "
                         "1 GiB copy (for hardware-counter runs); prints their own JSON")
    return ap.parse_args()


class AttnTimer:
    """Times the verify-attention launches of one speculative step.

    While ``capture`` is set, every verify-attention call made by the verify
    forward (launched eagerly) is recorded with its arguments and its
    algorithmic bytes, computed from the host-side metadata.  ``measure``
    then re-issues those exact launches back to back, ``repeats`` times, on
    the current stream (the one the kernels are enqueued on), between two HIP
    events, so that the mean launch time is the kernels' own time and not the
    host's launch latency.  The re-issued launches only read the K/V cache
    and write fresh output buffers."""

    def __init__(self):
        self.capture = False
        self.calls = []
        self.bytes = []
        self.current_lens = None
        self.orig = None

    def wrap(self, kernels):
        orig = kernels.paged_attention_varlen
        self.orig = orig
        timer = self

        def recorded(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                     softmax_scale, block_table, causal=True, k_scale=None, v_scale=None, out=None):
            o = orig(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                     softmax_scale, block_table, causal, k_scale, v_scale, out)
            if timer.capture and timer.current_lens is not None:
                hkv, d = k_cache.shape[2], k_cache.shape[3]
                kv = sum(timer.current_lens) * hkv * d * k_cache.element_size() * 2
                qo = q.shape[0] * q.shape[1] * d * 2 * 2
                timer.calls.append((q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                    max_seqlen_k, softmax_scale, block_table, causal, k_scale,
                                    v_scale))
                timer.bytes.append(kv + qo)
            return o

        kernels.paged_attention_varlen = recorded
        import nanovllm_amd.layers as layers
        layers.K.paged_attention_varlen = recorded

    def measure(self, repeats: int, traffic):
        import torch

        if not self.calls:
            return None
        for args in self.calls:  # warm the workspace cache
            self.orig(*args)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(repeats):
            for args in self.calls:
                self.orig(*args)
        e.record(stream)
        torch.cuda.synchronize()
        launches = repeats * len(self.calls)
        mean_ms = s.elapsed_time(e) / launches
        mean_bytes = sum(self.bytes) / len(self.bytes)
        gbs = mean_bytes / (mean_ms * 1e-3) / 1e9
        self.calls = []
        return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "paged_attention_kernel (+ combine_kernel when a sequence is split): one "
                          "verify-attention call",
                "launches": launches, "mean_us": round(mean_ms * 1e3, 2),
                "bytes_per_launch": int(mean_bytes)}


def cpu_baseline(batches, seconds, one_thread_seconds=5.0):
    """Reference host acceptance on CPU torch, bounded to ~``seconds`` with
    every core the process may use, then ~``one_thread_seconds`` on one."""
    import statistics

    import torch
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass

    def timed(threads, budget):
        torch.set_num_threads(threads)
        logits, cu, ids = batches[0]
        for _ in range(3):
            oracle.reference_cpu_acceptance(logits, cu, ids)
        times, committed = [], 0
        t_end = time.perf_counter() + budget
        i = 0
        while time.perf_counter() < t_end or len(times) < 3:
            logits, cu, ids = batches[i % len(batches)]
            t0 = time.perf_counter()
            _, _, c = oracle.reference_cpu_acceptance(logits, cu, ids)
            times.append(time.perf_counter() - t0)
            committed += c
            i += 1
        return times, committed

    times, committed = timed(cores, seconds)
    times1, committed1 = timed(1, one_thread_seconds)
    torch.set_num_threads(cores)
    logits, cu, _ = batches[0]
    rows = logits.shape[0]
    med, med1 = statistics.median(times), statistics.median(times1)
    return {"value": round(committed / sum(times), 1), "unit": "accepted tok/s (acceptance logic only)",
            "cores": cores, "kind": "port",
            "sample": f"{len(times)} verify batches of [{rows}, {logits.shape[1]}] bf16 "
                      f"logits from this run ({len(cu) - 1} sequences each), per-sequence "
                      f"argmax+tolist+verify_greedy_proposals, torch CPU with {cores} threads on "
                      f"{model}; median {med * 1e3:.1f} ms per batch",
            "median_ms_per_batch": round(med * 1e3, 2), "rows_per_s": round(rows / med, 1),
            "one_thread": {"value": round(committed1 / sum(times1), 1), "batches": len(times1),
                           "median_ms_per_batch": round(med1 * 1e3, 2),
                           "rows_per_s": round(rows / med1, 1)}}


def attention_only(args) -> None:
    """Verify attention alone on the bench workload's shapes, for counter runs.

    The sequences are the bench's (same seeded prompt lengths, longest
    first as the engine orders them) at the point the roofline step verifies
    them: prompt + committed tokens + k+1 verify rows, with random bf16 K/V
    in one cache per layer (block ids shuffled), so that consecutive calls
    read different pages as the step's layers do.  Launches
    ``--roofline-repeats`` x 36 verify-attention calls (one step's worth per
    repeat, layer by layer), then a plain device copy of 1 GiB as often, for
    scaling FETCH_SIZE / WRITE_SIZE counter readings to bytes."""
    import torch

    from nanovllm_amd import kernels
    from nanovllm_amd.synthetic import QWEN3_PRESETS

    dev = torch.device("cuda", 0)
    cfg = QWEN3_PRESETS[args.preset]
    hq, hkv, d, layers = (cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"],
                          cfg["num_hidden_layers"])
    g = torch.Generator().manual_seed(args.seed)
    lens = torch.randint(args.prompt_min, args.prompt_max + 1, (args.batch,), generator=g).tolist()
    lens = sorted(lens, reverse=True)  # the engine verifies its batch longest sequence first
    done = args.warmup + args.steps + 2  # tokens each sequence holds when the roofline step runs
    q_len = args.k + 1
    seqlens = [L + done + q_len for L in lens]
    block = 256
    nblk = [-(-L // block) for L in seqlens]
    total = sum(nblk)
    perm = torch.randperm(total, generator=g)
    width = max(nblk)
    bt = torch.full((args.batch, width), -1, dtype=torch.int32)
    off = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    gd = torch.Generator(device=dev).manual_seed(args.seed)
    if args.kv_layout == "head_major":  # the engine's page order, same logical view
        pages = torch.empty(layers, total, hkv, 2, block, d, dtype=torch.bfloat16, device=dev)
        pages = pages.permute(3, 0, 1, 4, 2, 5)
    else:
        pages = torch.empty(2, layers, total, block, hkv, d, dtype=torch.bfloat16, device=dev)
    pages.normal_(generator=gd)
    T = args.batch * q_len
    q = torch.randn(T, hq, d, generator=g).to(torch.bfloat16).to(dev)
    cu_q = torch.arange(0, T + 1, q_len, dtype=torch.int32).to(dev)
    cu_k = torch.tensor([0] + seqlens, dtype=torch.int64).cumsum(0).to(torch.int32).to(dev)
    bt = bt.to(dev)
    out = torch.empty_like(q)
    max_k = args.prompt_max + args.max_tokens + q_len  # the engine's max_seqlen_k
    scale = d ** -0.5

    layer = [0]

    def attn():
        l = layer[0]
        layer[0] = (l + 1) % layers
        kernels.paged_attention_varlen(q, pages[0, l], pages[1, l], cu_q, cu_k, q_len, max_k, scale,
                                       bt, out=out)

    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)

    def timed(fn, n):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(n):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / n * 1e3

    n_attn = args.roofline_repeats * layers
    attn_us = timed(attn, n_attn)
    copy_us = timed(lambda: dst.copy_(src), args.roofline_repeats)
    byts = sum(seqlens) * hkv * d * 2 * 2 + T * hq * d * 2 * 2
    print(json.dumps({"workload": "verify attention only", "batch": args.batch, "q_len": q_len,
                      "kv_layout": args.kv_layout,
                      "sum_seqlen_k": sum(seqlens), "longest_seq": max(seqlens),
                      "attention_calls": n_attn + 3, "attention_us": round(attn_us, 2),
                      "bytes_per_call": byts,
                      "achieved_GBs": round(byts / attn_us / 1e3, 1),
                      "copy_bytes": src.numel(), "copy_calls": args.roofline_repeats + 3,
                      "copy_us": round(copy_us, 1),
                      "copy_GBs": round(2 * src.numel() / copy_us / 1e3, 1)}), flush=True)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kernel_configs(args) -> None:
    """Each hot-path kernel alone, at the BASELINE configs' shapes.

    Seeds follow the configs' order (config 1: 0 ... config 5: 4).  Inputs
    are device-resident before timing.  ``iters`` launches are captured in a
    HIP graph, so that the host's launch latency does not pace the small
    kernels, and each figure is one replay between two HIP events on the
    replay stream, divided by ``iters``.
    Algorithmic bytes per launch:
      K1 attention: sum_i L_i*Hkv*D*esz*2 + T*Hq*D*2*2 (config 5: logical
                    bytes; its prefix-shared pages are read once per sharer);
      K2 store:     T*Hkv*D*(2 + esz)*2 (read bf16 rows, write cache rows);
      K3 aux:       R*3H*2*2 read + R*3H*2 written;
      K4 argmax:    rows*V*2 read."""
    import torch

    from nanovllm_amd import kernels
    from nanovllm_amd.synthetic import QWEN3_PRESETS

    dev = torch.device("cuda", 0)
    V = QWEN3_PRESETS["qwen3-8b"]["vocab_size"]
    D, BS = 128, 256

    def timed(fn, iters=30):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(iters):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        graph.replay()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters * 1e3

    def emit(kernel, config, us, byts, **extra):
        gbs = byts / us / 1e3
        print(json.dumps({"bench": "kernels", "kernel": kernel, "config": config,
                          "us": round(us, 2), "bytes": int(byts), "GBs": round(gbs, 1),
                          "frac": round(gbs / HBM_PEAK_GBS, 4), **extra}), flush=True)

    def pages(seed, batch, q_len, lo, hi, hq, hkv, fp8=False, shared_frac=0.0, copies=1):
        g = torch.Generator().manual_seed(seed)
        lens = torch.randint(lo, hi + 1, (batch,), generator=g).tolist()
        if args.batch_order == "longest_first":  # the engine's verify order
            lens = sorted(lens, reverse=True)
        nblk = [-(-L // BS) for L in lens]
        n_shared = [int(shared_frac * n) for n in nblk]
        pool = max(n_shared) if n_shared else 0
        unique = sum(n - s for n, s in zip(nblk, n_shared))
        total = pool + unique
        perm = torch.randperm(total, generator=g)
        bt = torch.full((batch, max(nblk)), -1, dtype=torch.int32)
        off = pool
        for i, (n, sh) in enumerate(zip(nblk, n_shared)):
            bt[i, :sh] = perm[:sh].to(torch.int32)        # the shared prefix pages
            bt[i, sh:n] = perm[off:off + n - sh].to(torch.int32)
            off += n - sh
        gd = torch.Generator(device=dev).manual_seed(seed)
        dt = torch.float8_e4m3fn if fp8 else torch.bfloat16
        # `copies` caches of the same content layout, used in turn, so that
        # caches smaller than the 256 MB last-level cache are not re-read from it
        if args.kv_layout == "head_major":
            kv = torch.empty(copies, total, hkv, 2, BS, D, dtype=dt, device=dev)
            kv = kv.permute(0, 3, 1, 4, 2, 5)
        else:
            kv = torch.empty(copies, 2, total, BS, hkv, D, dtype=dt, device=dev)
        if fp8:
            for cp in range(copies):
                for kind in range(2):
                    kv[cp, kind].copy_(torch.empty(total, BS, hkv, D, device=dev)
                                       .normal_(0.0, 0.5, generator=gd))
        else:
            kv.normal_(0.0, 0.5, generator=gd)
        kc, vc = kv[0, 0], kv[0, 1]
        T = batch * q_len
        q = torch.empty(T, hq, D, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.5, generator=gd)
        cu_q = torch.arange(0, T + 1, q_len, dtype=torch.int32, device=dev)
        cu_k = torch.tensor([0] + lens, dtype=torch.int64).cumsum(0).to(torch.int32).to(dev)
        slots = torch.tensor([int(bt[i, p // BS]) * BS + p % BS
                              for i, L in enumerate(lens) for p in range(L - q_len, L)],
                             dtype=torch.int32, device=dev)
        phys = (pool + unique) * BS * hkv * D * (1 if fp8 else 2) * 2
        return dict(lens=lens, kc=kc, vc=vc, kv=kv, q=q, cu_q=cu_q, cu_k=cu_k, bt=bt.to(dev),
                    slots=slots, T=T, q_len=q_len, hq=hq, hkv=hkv, fp8=fp8, phys=phys)

    def attention(name, c):
        esz = 1 if c["fp8"] else 2
        one = torch.ones(1, device=dev) if c["fp8"] else None
        out = torch.empty_like(c["q"])
        turn = [0]

        def call():
            cp = turn[0] % c["kv"].shape[0]
            turn[0] += 1
            kernels.paged_attention_varlen(c["q"], c["kv"][cp, 0], c["kv"][cp, 1], c["cu_q"],
                                           c["cu_k"], c["q_len"], max(c["lens"]), D ** -0.5,
                                           c["bt"], k_scale=one, v_scale=one, out=out)

        us = timed(call)
        byts = sum(c["lens"]) * c["hkv"] * D * esz * 2 + c["T"] * c["hq"] * D * 2 * 2
        extra = {}
        if c["phys"] < sum(c["lens"]) * c["hkv"] * D * esz * 2:
            extra["unique_kv_bytes"] = int(c["phys"])
        emit("K1 paged_attention_varlen", name, us, byts, batch=len(c["lens"]), q_len=c["q_len"],
             heads=f"{c['hq']}/{c['hkv']}", kv="fp8" if c["fp8"] else "bf16",
             sum_seqlen_k=sum(c["lens"]), kv_layout=args.kv_layout,
             batch_order=args.batch_order, **extra)

    def store(name, c):
        esz = 1 if c["fp8"] else 2
        one = torch.ones(1, device=dev) if c["fp8"] else None
        hkv, T = c["hkv"], c["T"]
        qkv = torch.randn(T, (c["hq"] + 2 * hkv) * D, device=dev).to(torch.bfloat16)
        key = qkv[:, c["hq"] * D:(c["hq"] + hkv) * D].view(T, hkv, D)
        value = qkv[:, (c["hq"] + hkv) * D:].view(T, hkv, D)
        us = timed(lambda: kernels.store_kvcache(key, value, c["kc"], c["vc"], c["slots"], one,
                                                 one))
        emit("K2 store_kvcache", name, us, T * hkv * D * (2 + esz) * 2, rows=T)

    def rollback(name, c):
        g = torch.Generator().manual_seed(7)
        b = len(c["lens"])
        acc = torch.randint(0, c["q_len"], (b,), generator=g).to(torch.int32).to(dev)
        slots = c["slots"].clone()
        seqlens = torch.tensor(c["lens"], dtype=torch.int32, device=dev)
        us = timed(lambda: kernels.rollback(c["cu_q"], acc, slots, seqlens))
        emit("K2 rollback (slots only)", name, us, b * 4 * 3 + c["T"] * 4, seqs=b)

    # config 1: greedy acceptance, [8, 5, V] logits, drafts raised with p = 0.7
    def acceptance(name, seed, batch, k):
        g = torch.Generator().manual_seed(seed)
        q_len = k + 1
        logits = torch.randn(batch, q_len, V, generator=g)
        prop = torch.randint(0, V, (batch, k), generator=g)
        hit = torch.rand(batch, k, generator=g) < 0.7
        for s_ in range(batch):
            for j in range(k):
                if hit[s_, j]:
                    logits[s_, j, prop[s_, j]] = logits[s_, j].max() + 1.0
        lg = logits.view(batch * q_len, V).to(torch.bfloat16).to(dev)
        ids = torch.cat([torch.randint(0, V, (batch, 1), generator=g), prop], 1)
        ids = ids.reshape(-1).to(dev)
        cu = torch.arange(0, batch * q_len + 1, q_len, dtype=torch.int32, device=dev)
        us = timed(lambda: kernels.argmax_accept(lg, cu, ids))
        emit("K4 argmax_accept", name, us, batch * q_len * V * 2, rows=batch * q_len, vocab=V)

    acceptance("config1 B8 k4", 0, 8, 4)
    acceptance("config3 verify rows B64 k5", 2, 64, 5)

    c2 = pages(1, 32, 5, 512, 4096, 16, 8, copies=4)
    store("config2 B32 q5", c2)
    attention("config2 B32 q5 Qwen3-0.6B", c2)
    rollback("config2 B32 q5", c2)
    del c2

    c3 = pages(2, 64, 6, 256, 2304, 32, 8, copies=4)
    store("config3 B64 q6", c3)
    attention("config3 B64 q6 Qwen3-8B", c3)
    H = QWEN3_PRESETS["qwen3-8b"]["hidden_size"]
    hid = [torch.randn(c3["T"], H, device=dev).to(torch.bfloat16) for _ in range(3)]
    res = [torch.randn(c3["T"], H, device=dev).to(torch.bfloat16) for _ in range(3)]
    src = torch.arange(c3["T"], dtype=torch.int32, device=dev)
    us = timed(lambda: kernels.aux_gather(hid, res, src))
    emit("K3 aux_gather", "config3 R=384 H=4096 3 layers", us, c3["T"] * 3 * H * 2 * 3)
    dec = pages(5, 64, 1, 256, 2304, 32, 8, copies=4)
    attention("config3 draft decode B64 q1", dec)
    del c3, dec, hid, res

    c4 = pages(3, 128, 5, 4096, 16384, 16, 8, fp8=True)
    store("config4 B128 q5 fp8", c4)
    attention("config4 B128 q5 fp8", c4)
    del c4

    c5 = pages(4, 128, 8, 2048, 8192, 64, 8, shared_frac=0.3)
    attention("config5 B128 q8 Qwen3-32B (30% shared prefix pages)", c5)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported by this build "
              "(the hot path runs on one GPU)", file=sys.stderr)
        sys.exit(2)
    if args.attention_only:
        attention_only(args)
        return
    if args.kernels:
        kernel_configs(args)
        return
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
              enforce_eager=args.eager, kv_cache_layout=args.kv_layout,
              gemm_tuning_file=(args.gemm_tuning or None) if args.preset == "qwen3-8b" else None,
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

    # roofline: one more step of the same workload with the verify forward
    # launched eagerly (events cannot be recorded inside a captured HIP graph
    # on ROCm); its verify-attention launches, with the timed steps' kernels
    # and shapes, are then re-issued back to back between HIP events
    runner.use_verify_graph = False
    timer.capture = True
    llm.step()
    timer.capture = False
    runner.use_verify_graph = True
    default_workload = all(getattr(args, key) == val for key, val in PMC_WORKLOAD.items())
    roof = timer.measure(args.roofline_repeats, PMC_TRAFFIC_BYTES if default_workload else None)

    log(f"timed {args.steps} steps in {elapsed:.3f}s")
    ref = None
    if args.reference_steps > 0 and llm.scheduler.running:
        # the reference's step structure on the same kernels and sequences:
        # one warm-up step, then the timed ones
        llm.reference_pipeline = True
        llm.step()
        torch.cuda.synchronize()
        r0 = time.perf_counter()
        ref_committed = 0
        for _ in range(args.reference_steps):
            _, num_tokens = llm.step()
            ref_committed += -num_tokens
        torch.cuda.synchronize()
        r_el = time.perf_counter() - r0
        llm.reference_pipeline = False
        ref = {"value": round(ref_committed / r_el, 1), "unit": "tok/s",
               "ms_per_step": round(r_el / args.reference_steps * 1e3, 2),
               "steps": args.reference_steps,
               "structure": "reference llm_engine.py:124-178 step shape on this build's kernels: "
                            "eager draft loop with a host sync per draft step, eager target "
                            "verify with one torch argmax + .tolist() per sequence, host "
                            "acceptance per sequence, serial single-token draft replay per "
                            "committed token (model_runner.py:1127-1156)"}
        log(f"reference-structured steps: {ref['ms_per_step']} ms/step")
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
                   "hip_graphs": not args.eager, "kv_layout": args.kv_layout,
                   "gemm_tuning": os.path.basename(args.gemm_tuning) if args.gemm_tuning else None},
        "roofline": roof,
        "cpu_baseline": cpu,
        "reference_pipeline": ref,
        "committed_tokens": committed,
        "accepted_drafts_per_seq_step": round(stats["accepted"] / max(stats["steps"] * n_active, 1), 4),
        "committed_per_seq_step": round(stats["committed"] / max(stats["steps"] * n_active, 1), 4),
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
