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
                 launches, --roofline-repeats times over, are captured in a
                 HIP graph whose replays are timed between events (so the
                 host's launch rate cannot pace them; the median of three
                 replays); achieved = algorithmic bytes per launch / mean
                 launch time, algorithmic bytes = sum_i L_i*Hkv*D*2B*2
                 (K and V read once) + T*Hq*D*2B*2 (Q in, O out);
  cpu_baseline:  the reference's host acceptance logic (per-sequence bf16
                 argmax + .tolist() + verify_greedy_proposals) timed on this
                 host's cores over verify batches copied from the run.
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
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
# --pmc runs of `bench.py --attention-only --roofline-repeats 2` (FETCH_SIZE,
# then WRITE_SIZE; KiB per dispatch, mean of the 75 calls), scaled by what
# the same counters read for a 1 GiB device copy and a 1 GiB read in the same
# runs: FETCH_SIZE 524303 / 524348 KiB (x2.0 to bytes read), WRITE_SIZE
# 1048576 KiB for the copy (x1.0).  Attention kernel (paired mode, one
# split per sequence, so no combine kernel runs; K and V staged through LDS)
# on the sequences of the default run's roofline step (sum L = 77 172):
# FETCH 155978.2, WRITE 3072.5.  A recorded constant, quoted only for the
# default workload, whose shapes it was measured on, and only while the
# kernel source is the one it was measured on.
PMC_TRAFFIC_BYTES = int((155978.2 * 2.0 + 3072.5 * 1.0) * 1024)
PMC_WORKLOAD = dict(preset="qwen3-8b", batch=64, k=5, prompt_min=256, prompt_max=2048,
                    max_tokens=256, seed=2, kv_layout="head_major")
# the kernel source the counters were read on (sha256 of csrc/paged_attention.hip
# then csrc/common.h, first 16 hex digits): the constant is quoted only while
# the source is unchanged, since a change of the kernel's loads changes it
PMC_ATTENTION_SOURCE = "5ff53aaca177830c"
ATTENTION_SOURCES = ("paged_attention.hip", "common.h")


def attention_source_hash() -> str:
    import hashlib

    h = hashlib.sha256()
    for name in ATTENTION_SOURCES:
        with open(os.path.join(ROOT, "extend-nano-vllm_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def pmc_traffic_reason(args) -> str | None:
    """Why the recorded traffic constant does not apply (None when it does)."""
    if not all(getattr(args, key) == val for key, val in PMC_WORKLOAD.items()):
        return "the counters were read on the default workload only"
    if attention_source_hash() != PMC_ATTENTION_SOURCE:
        return (f"the attention kernel's source ({attention_source_hash()}) is not the one the "
                f"counters were read on ({PMC_ATTENTION_SOURCE})")
    return None


def pmc_traffic_bytes(args) -> int | None:
    return PMC_TRAFFIC_BYTES if pmc_traffic_reason(args) is None else None
METRIC = "accepted tok/s, Qwen3-8B EAGLE3 k=5 bs64; verify-attn HBM GB/s % of peak"


def workload_label(args) -> tuple:
    """(metric, workload) of the bench line for the chosen preset, batch and
    k; the default workload keeps METRIC."""
    from nanovllm_amd.synthetic import QWEN3_PRESETS, default_aux_layers

    p = QWEN3_PRESETS[args.preset]
    name = {"qwen3-8b": "Qwen3-8B", "qwen3-0.6b": "Qwen3-0.6B",
            "qwen3-32b": "Qwen3-32B"}.get(args.preset, args.preset)
    aux = "/".join(str(a) for a in default_aux_layers(args.preset))
    workload = (f"EAGLE3 speculative decode step, {name} geometry ({p['num_hidden_layers']} "
                f"layers, H{p['hidden_size']}, {p['num_attention_heads']}q/"
                f"{p['num_key_value_heads']}kv, D{p['head_dim']}, MLP{p['intermediate_size']}, "
                f"V{p['vocab_size']}), draft 1 layer + fc 3H->H on aux layers {aux}")
    if (args.preset, args.k, args.batch) == ("qwen3-8b", 5, 64):
        return METRIC, workload
    return (f"accepted tok/s, {name} EAGLE3 k={args.k} bs{args.batch}; verify-attn HBM GB/s % "
            f"of peak", workload)


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
                         "(captured in one HIP graph, replayed between HIP events) for the "
                         "roofline figure")
    ap.add_argument("--reference-steps", type=int, default=5,
                    help="steps timed with the reference's step structure for comparison, on "
                         "this build's kernels and on torch attention (0 to skip)")
    ap.add_argument("--acceptance-steps", type=int, default=20,
                    help="steps of the forced-acceptance run (0 to skip)")
    ap.add_argument("--draft-keep", type=float, default=0.7,
                    help="forced-acceptance run: probability that a draft position carries "
                         "the target's greedy token")
    ap.add_argument("--no-per-config", action="store_true",
                    help="skip the per-config kernel figures of the JSON line")
    ap.add_argument("--profile-steps", type=int, default=0,
                    help="after the timed steps, run this many more steps between two marker "
                         "kernels (torch spin_kernel), to cut a rocprofv3 kernel trace to "
                         "steady-state steps")
    ap.add_argument("--workload", default="config3", choices=["config3", "config5"],
                    help="config3: the default bench line (BASELINE config 3); config5: the "
                         "Qwen3-32B-geometry engine run of BASELINE config 5 (k=7, B128, "
                         "contexts U[2048, 8192], shuffled pages), its own JSON line")
    ap.add_argument("--gemm-tuning", default=DEFAULT_GEMM_TUNING,
                    help="TunableOp results for the projection GEMMs ('' for library defaults)")
    ap.add_argument("--kv-layout", default="head_major", choices=["head_major", "token_major"],
                    help="physical order inside a KV page (the engine's kv_cache_layout)")
    ap.add_argument("--kernels", action="store_true",
                    help="time each hot-path kernel alone on the seeded synthetic inputs of "
                         "BASELINE configs 1, 2, 4 and 5 (and config 3's shapes); one JSON line "
                         "per kernel and config")
    ap.add_argument("--kernel-filter", default="",
                    help="--kernels: only the records whose config name contains this text")
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
    then captures those exact launches, ``repeats`` times over, in a HIP
    graph and times three replays on the current stream (the one the kernels
    are enqueued on) between HIP events, so that the mean launch time (of the
    median replay) is the kernels' own time and not the host's launch rate.
    The re-issued launches only read the K/V cache and write fresh output
    buffers."""

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
        # the launches are captured in a HIP graph and one replay is timed,
        # so that the host's launch rate (the Python wrapper per call) cannot
        # pace the kernels: eager re-issue read 66.7 us per call on a box
        # whose trace showed 58 us of kernel time
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(repeats):
                for args in self.calls:
                    self.orig(*args)
        graph.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        # the median of three replays: the same launches run a few percent
        # slower through some stretches of a few ms
        replay_ms = []
        for _ in range(3):
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record(stream)
            graph.replay()
            e.record(stream)
            torch.cuda.synchronize()
            replay_ms.append(s.elapsed_time(e))
        del graph
        launches = repeats * len(self.calls)
        mean_ms = sorted(replay_ms)[1] / launches
        mean_bytes = sum(self.bytes) / len(self.bytes)
        gbs = mean_bytes / (mean_ms * 1e-3) / 1e9
        self.calls = []
        return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "paged_attention_kernel (+ combine_kernel when a sequence is split): one "
                          "verify-attention call",
                "launches": launches, "replays": 3, "mean_us": round(mean_ms * 1e3, 2),
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
    repeat, layer by layer), then a plain device copy of 1 GiB and a 1 GiB
    read (a sum) as often, for scaling FETCH_SIZE / WRITE_SIZE counter
    readings to bytes."""
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
    # the roofline step's position: the prompts prefilled again (one token),
    # the warm-up steps, the profiled steps and the CPU baseline's step
    # commit one token each (nothing is accepted), and the step verifies
    # from the last of them: its keys are prompt + done + k + 1
    done = args.warmup + args.profile_steps + (0 if args.no_cpu_baseline else 1)
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
    # a read-only reference (1 GiB read, 4 bytes written): the FETCH_SIZE
    # scale for a kernel that reads with wide vector loads and writes little
    total = torch.empty((), dtype=torch.float32, device=dev)
    flat = src.view(torch.float32)
    read_us = timed(lambda: torch.sum(flat, 0, out=total), args.roofline_repeats)
    byts = sum(seqlens) * hkv * d * 2 * 2 + T * hq * d * 2 * 2
    print(json.dumps({"workload": "verify attention only", "batch": args.batch, "q_len": q_len,
                      "kv_layout": args.kv_layout,
                      "sum_seqlen_k": sum(seqlens), "longest_seq": max(seqlens),
                      "attention_calls": n_attn + 3, "attention_us": round(attn_us, 2),
                      "bytes_per_call": byts,
                      "achieved_GBs": round(byts / attn_us / 1e3, 1),
                      "copy_bytes": src.numel(), "copy_calls": args.roofline_repeats + 3,
                      "copy_us": round(copy_us, 1),
                      "copy_GBs": round(2 * src.numel() / copy_us / 1e3, 1),
                      "read_calls": args.roofline_repeats + 3, "read_us": round(read_us, 1),
                      "read_GBs": round(src.numel() / read_us / 1e3, 1)}), flush=True)


class TorchAttention:
    """Paged attention in plain torch ops, standing in for FlashAttention-2
    in the reference-structured comparator (the reference calls
    flash_attn_varlen_func / flash_attn_with_kvcache, layers/attention.py:
    385-399; flash-attn is not installed on this box).  Replaces
    Attention.attend while installed: every sequence's pages are gathered
    through the block table into one padded [B, Hkv, L, D] tensor, then a
    bf16 batched QK^T, the bottom-right causal mask and an fp32 softmax,
    and a bf16 batched PV -- a few launches per layer whatever the batch,
    as one FA2 call would be.  Both right-hand operands are made contiguous
    before the batched products: bf16 batched products with a transposed
    right operand are a documented fault hazard of this GPU pool (this
    build has not run them in that form).  The per-forward metadata is read
    to the host once and shared by all layers (FA2 would read it on the
    device)."""

    def __init__(self):
        self.saved = None
        self.meta_key = None
        self.meta = None

    def install(self):
        import nanovllm_amd.layers as layers

        self.saved = layers.Attention.attend
        backend = self

        def attend(layer, q):
            return backend.attend(layer, q)

        layers.Attention.attend = attend

    def uninstall(self):
        import nanovllm_amd.layers as layers

        layers.Attention.attend = self.saved
        self.meta_key = self.meta = None

    def _host_meta(self, ctx):
        # the key holds the metadata tensors themselves (compared by
        # identity), so none is freed and replaced by a new one at the same id
        key = (ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.context_lens, ctx.block_tables)
        if self.meta_key is None or any(a is not b for a, b in zip(key, self.meta_key)):
            if ctx.is_prefill:
                cu_q = ctx.cu_seqlens_q.tolist()
                cu_k = ctx.cu_seqlens_k.tolist()
                qn = [b - a for a, b in zip(cu_q, cu_q[1:])]
                lens = [b - a for a, b in zip(cu_k, cu_k[1:])]
            else:
                lens = ctx.context_lens.tolist()
                qn = [1] * len(lens)
                cu_q = list(range(len(lens) + 1))
            self.meta_key, self.meta = key, (cu_q, qn, lens)
        return self.meta

    def attend(self, layer, q):
        import torch

        from nanovllm_amd.context import get_context

        ctx = get_context()
        cu_q, qn, lens = self._host_meta(ctx)
        kc, vc = layer.k_cache, layer.v_cache                 # [blocks, bs, Hkv, D] views
        b, bs, hkv, d = len(lens), kc.shape[1], kc.shape[2], kc.shape[3]
        hq = q.shape[1]
        g = hq // hkv
        lmax, qmax = max(lens), max(qn)
        nblk = -(-lmax // bs)
        dev = q.device
        idx = ctx.block_tables[:b, :nblk].long().clamp_min(0)
        k = kc[idx].reshape(b, nblk * bs, hkv, d)[:, :lmax]   # gather: [B, L, Hkv, D]
        v = vc[idx].reshape(b, nblk * bs, hkv, d)[:, :lmax]
        kt = k.permute(0, 2, 3, 1).contiguous()                # [B, Hkv, D, L]
        vv = v.permute(0, 2, 1, 3).contiguous()                # [B, Hkv, L, D]
        # query rows padded to [B, qmax]
        rows = torch.tensor([cu_q[i] + j for i in range(b) for j in range(qmax)], device=dev)
        valid = torch.tensor([j < qn[i] for i in range(b) for j in range(qmax)], device=dev)
        qp = q.index_select(0, rows.clamp_max(q.shape[0] - 1)).view(b, qmax, hkv, g, d)
        qq = qp.permute(0, 2, 3, 1, 4).reshape(b, hkv, g * qmax, d)
        s = torch.matmul(qq, kt).float().view(b, hkv, g, qmax, lmax) * layer.scale
        last = (torch.tensor(lens, device=dev) - torch.tensor(qn, device=dev))[:, None] + \
            torch.arange(qmax, device=dev)[None, :]           # last visible key per row
        vis = torch.arange(lmax, device=dev)[None, None, :] <= last[:, :, None]
        s = s.masked_fill(~vis[:, None, None], float("-inf"))
        p = torch.softmax(s, -1).nan_to_num_(0.0).to(q.dtype).view(b, hkv, g * qmax, lmax)
        o = torch.matmul(p, vv).view(b, hkv, g, qmax, d).permute(0, 3, 1, 2, 4)
        o = o.reshape(b * qmax, hq, d)[valid]
        if o.shape[0] == q.shape[0]:
            return o
        out = torch.zeros_like(q)                              # rows past the batch
        out[:o.shape[0]] = o
        return out


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kernel_configs(args, cpu_seconds: float = 0.0) -> list:
    """Each hot-path kernel alone, at the BASELINE configs' shapes; returns
    one record per (kernel, config).

    Seeds follow the configs' order (config 1: 0 ... config 5: 4).  Inputs
    are device-resident before timing.  Each kernel's launches are captured
    in a HIP graph, so that the host's launch latency does not pace the small
    kernels, as many as make one replay last >= 20 ms (30 to 2000 launches),
    and each figure is the median of three replays between HIP events on the
    replay stream, divided by the launches per replay.
    Algorithmic bytes per launch:
      K1 attention: sum_i L_i*Hkv*D*esz*2 + T*Hq*D*2*2 (config 5: logical
                    bytes; its prefix-shared pages are read once per sharer);
      K2 store:     T*Hkv*D*(2 + esz)*2 (read bf16 rows, write cache rows);
      K3 aux:       R*3H*2*2 read + R*3H*2 written;
      K4 argmax:    rows*V*2 read.
    With cpu_seconds > 0, the acceptance configs also time the reference's
    host acceptance logic (oracle.reference_cpu_acceptance) on the same
    seeded bf16 bytes the kernel reads, with every host core and with one,
    and the attention records of configs 2 and 4 time the CPU oracle's
    textbook attention on their own pages (config 2 whole, config 4 every
    32nd sequence; one thread) as context."""
    import statistics

    import torch

    from nanovllm_amd import kernels
    from nanovllm_amd.synthetic import QWEN3_PRESETS

    dev = torch.device("cuda", 0)
    V = QWEN3_PRESETS["qwen3-8b"]["vocab_size"]
    D, BS = 128, 256

    stream = torch.cuda.current_stream()

    def capture(fn, iters):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(iters):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        return graph

    def replay_us(graph, iters):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        graph.replay()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters * 1e3

    def timed(fn, min_ms=20.0, max_iters=2000, replays=3):
        """(mean launch time in us, launches per replay).  The burst is sized
        from a 30-launch replay so that one replay runs >= min_ms: on MI355X
        the same launches run a few percent slower through some stretches of
        a few ms (a 300-launch trace of config 3's attention: 58-59 us, then
        70 launches at 62.2, then 59.5; the next replay 58.05 throughout), so
        a 2 ms window reads 60-63 us where 20 ms windows read 57.7-57.9.
        The median of ``replays`` replays is returned."""
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        iters = 30
        graph = capture(fn, iters)
        want = min(max_iters, max(iters, math.ceil(min_ms * 1e3 / replay_us(graph, iters))))
        if want > iters:
            del graph
            iters = want
            graph = capture(fn, iters)
        us = statistics.median(replay_us(graph, iters) for _ in range(replays))
        del graph
        return us, iters

    records = []

    def wanted(config):
        return args.kernel_filter in config

    def emit(kernel, config, timing, byts, **extra):
        us, launches = timing
        gbs = byts / us / 1e3
        records.append({"kernel": kernel, "config": config, "us": round(us, 2),
                        "bytes": int(byts), "GBs": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "launches": launches, **extra})
        log(f"kernel {kernel} / {config}: {us:.2f} us ({launches} launches per replay)")

    def cpu_acceptance(lg_cpu, q_len, batch, ids_cpu):
        """The reference's per-sequence argmax + verify on the host, timed
        as the median of >= 20 runs after 3 warm-ups, all cores then one."""
        from oracle import oracle

        cu = list(range(0, batch * q_len + 1, q_len))
        ids = ids_cpu.tolist()
        cores = len(os.sched_getaffinity(0))
        out = {"cores": cores, "kind": "port"}
        for key, threads in (("all_cores", cores), ("one_thread", 1)):
            torch.set_num_threads(threads)
            for _ in range(3):
                oracle.reference_cpu_acceptance(lg_cpu, cu, ids)
            times = []
            t_end = time.perf_counter() + cpu_seconds / 2
            while len(times) < 20 or time.perf_counter() < t_end:
                t0 = time.perf_counter()
                oracle.reference_cpu_acceptance(lg_cpu, cu, ids)
                times.append(time.perf_counter() - t0)
                if len(times) >= 2000:
                    break
            med = statistics.median(times)
            out[key] = {"threads": threads, "us_per_batch": round(med * 1e6, 1),
                        "rows_per_s": round(batch * q_len / med, 1), "runs": len(times)}
        torch.set_num_threads(cores)
        return out

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

    def cpu_attention(c, every):
        """The CPU oracle's textbook paged attention (double accumulation,
        one thread) on every `every`-th sequence of the config's own pages
        and queries, for context beside K1 (BASELINE configs 2 and 4; not a
        target).  The copies to host memory are not timed."""
        import numpy as np
        from oracle import oracle

        sel = list(range(0, len(c["lens"]), every))
        q_len = c["q_len"]
        if c["fp8"]:
            def bits(x):
                return x.contiguous().view(torch.uint8).numpy()
        else:
            def bits(x):
                return x.contiguous().view(torch.int16).numpy().view(np.uint16)
        kc, vc = bits(c["kv"][0, 0].cpu()), bits(c["kv"][0, 1].cpu())
        rows = [i * q_len + j for i in sel for j in range(q_len)]
        q = c["q"].cpu()[rows].contiguous().view(torch.int16).numpy().view(np.uint16)
        lens = [c["lens"][i] for i in sel]
        bt = c["bt"].cpu()[sel].numpy()
        cu = np.arange(0, len(sel) * q_len + 1, q_len, dtype=np.int32)
        t0 = time.perf_counter()
        oracle.paged_attention(q, kc, vc, cu, lens, bt, D ** -0.5)
        dt = time.perf_counter() - t0
        keys, total = sum(lens), sum(c["lens"])
        return {"kind": "port", "threads": 1, "seconds": round(dt, 3),
                "sample": f"sequences 0, {every}, {2 * every}, ...: {len(sel)} of "
                          f"{len(c['lens'])}, {keys} of {total} keys",
                "us_per_call_scaled_to_batch": round(dt * 1e6 * total / keys, 1),
                "keys_per_s": round(keys / dt, 1)}

    def attention(name, c, cpu_every=0):
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

        timing = timed(call)
        byts = sum(c["lens"]) * c["hkv"] * D * esz * 2 + c["T"] * c["hq"] * D * 2 * 2
        extra = {}
        if c["phys"] < sum(c["lens"]) * c["hkv"] * D * esz * 2:
            extra["unique_kv_bytes"] = int(c["phys"])
        if cpu_every and cpu_seconds > 0:
            extra["cpu_oracle"] = cpu_attention(c, cpu_every)
        emit("K1 paged_attention_varlen", name, timing, byts, batch=len(c["lens"]), q_len=c["q_len"],
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
        timing = timed(lambda: kernels.store_kvcache(key, value, c["kc"], c["vc"], c["slots"], one,
                                                 one))
        emit("K2 store_kvcache", name, timing, T * hkv * D * (2 + esz) * 2, rows=T)

    def rollback(name, c):
        g = torch.Generator().manual_seed(7)
        b = len(c["lens"])
        acc = torch.randint(0, c["q_len"], (b,), generator=g).to(torch.int32).to(dev)
        slots = c["slots"].clone()
        seqlens = torch.tensor(c["lens"], dtype=torch.int32, device=dev)
        timing = timed(lambda: kernels.rollback(c["cu_q"], acc, slots, seqlens))
        emit("K2 rollback (slots only)", name, timing, b * 4 * 3 + c["T"] * 4, seqs=b,
             on_step=False)

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
        lg_cpu = logits.view(batch * q_len, V).to(torch.bfloat16)
        lg = lg_cpu.to(dev)
        ids_cpu = torch.cat([torch.randint(0, V, (batch, 1), generator=g), prop], 1).reshape(-1)
        ids = ids_cpu.to(dev)
        cu = torch.arange(0, batch * q_len + 1, q_len, dtype=torch.int32, device=dev)
        timing = timed(lambda: kernels.argmax_accept(lg, cu, ids))
        extra = {}
        if cpu_seconds > 0:
            extra["cpu_baseline"] = cpu_acceptance(lg_cpu, q_len, batch, ids_cpu)
        emit("K4 argmax_accept", name, timing, batch * q_len * V * 2, rows=batch * q_len, vocab=V,
             **extra)

    if wanted("config1 B8 k4"):
        acceptance("config1 B8 k4", 0, 8, 4)
    if wanted("config3 verify rows B64 k5"):
        acceptance("config3 verify rows B64 k5", 2, 64, 5)

    if wanted("config2 B32 q5"):
        c2 = pages(1, 32, 5, 512, 4096, 16, 8, copies=4)
        store("config2 B32 q5", c2)
        attention("config2 B32 q5 Qwen3-0.6B", c2, cpu_every=1)
        rollback("config2 B32 q5", c2)
        del c2

    if wanted("config3 B64 q6"):
        c3 = pages(2, 64, 6, 256, 2304, 32, 8, copies=4)
        store("config3 B64 q6", c3)
        attention("config3 B64 q6 Qwen3-8B", c3)
        H = QWEN3_PRESETS["qwen3-8b"]["hidden_size"]
        hid = [torch.randn(c3["T"], H, device=dev).to(torch.bfloat16) for _ in range(3)]
        res = [torch.randn(c3["T"], H, device=dev).to(torch.bfloat16) for _ in range(3)]
        src = torch.arange(c3["T"], dtype=torch.int32, device=dev)
        timing = timed(lambda: kernels.aux_gather(hid, res, src))
        emit("K3 aux_gather", "config3 B64 q6 R=384 H=4096 3 layers", timing, c3["T"] * 3 * H * 2 * 3)
        del c3, hid, res
    if wanted("config3 draft decode B64 q1"):
        dec = pages(5, 64, 1, 256, 2304, 32, 8, copies=4)
        attention("config3 draft decode B64 q1", dec)
        del dec

    if wanted("config4 B128 q5 fp8"):
        c4 = pages(3, 128, 5, 4096, 16384, 16, 8, fp8=True)
        store("config4 B128 q5 fp8", c4)
        attention("config4 B128 q5 fp8", c4, cpu_every=32)
        del c4

    if wanted("config5 B128 q8"):
        c5 = pages(4, 128, 8, 2048, 8192, 64, 8, shared_frac=0.3)
        attention("config5 B128 q8 Qwen3-32B (30% shared prefix pages)", c5)
        del c5
    if wanted("config5 draft decode B128 q1"):
        # the draft's one-layer cache: one query row per sequence, 64 q heads
        d5 = pages(6, 128, 1, 2048, 8192, 64, 8)
        attention("config5 draft decode B128 q1 Qwen3-32B", d5)
        del d5
    torch.cuda.empty_cache()
    return records


def make_engine(args, tmp: str):
    """The bench workload's engine (random weights, seeded)."""
    from nanovllm_amd import LLM
    from nanovllm_amd.synthetic import default_aux_layers, write_eagle3_config, write_qwen3_config

    target = write_qwen3_config(os.path.join(tmp, "target"), args.preset)
    aux = default_aux_layers(args.preset)
    draft = write_eagle3_config(os.path.join(tmp, "draft"), args.preset, aux_layers=aux)
    max_len = args.prompt_max + args.max_tokens
    blocks_per_seq = -(-(max_len + args.k + 1) // 256)
    return LLM(target, load_format="dummy", seed=0, max_num_seqs=args.batch,
               max_model_len=max_len, num_kvcache_blocks=args.batch * blocks_per_seq + 8,
               max_num_batched_tokens=16384, enable_prefill_batching=True,
               enforce_eager=args.eager, kv_cache_layout=args.kv_layout,
               gemm_tuning_file=(args.gemm_tuning or None) if args.preset == "qwen3-8b" else None,
               speculative_config={"method": "eagle3", "model": draft,
                                   "num_speculative_tokens": args.k,
                                   "aux_hidden_state_layers": aux})


def add_prompts(llm, args, seq_row: dict | None = None):
    """The seeded prompts (lengths U[prompt_min, prompt_max], random ids);
    returns the prompt token lists in request order.  seq_row (optional)
    receives each new sequence's id -> its row in that order."""
    import torch

    from nanovllm_amd import SamplingParams

    vocab = llm.config.hf_config.vocab_size
    g = torch.Generator().manual_seed(args.seed)
    lens = torch.randint(args.prompt_min, args.prompt_max + 1, (args.batch,), generator=g).tolist()
    sp = SamplingParams(temperature=0.0, max_tokens=args.max_tokens, ignore_eos=True)
    prompts = []
    for L in lens:
        prompts.append(torch.randint(0, vocab, (L,), generator=g).tolist())
        llm.add_request(prompts[-1], sp)
        if seq_row is not None:
            seq_row[llm.scheduler.waiting[-1].seq_id] = len(prompts) - 1
    return prompts


def release(llm) -> None:
    import gc

    import torch

    llm.exit()
    del llm
    gc.collect()
    torch.cuda.empty_cache()


def profiled_steps(llm, steps: int) -> None:
    """``steps`` more engine steps between two marker kernels (torch's
    spin_kernel, launched only here), so that a `rocprofv3 --kernel-trace`
    record can be cut to exactly these steady-state steps."""
    import torch

    if steps <= 0:
        return
    torch.cuda.synchronize()
    torch.cuda._sleep(1000)
    torch.cuda.synchronize()
    for _ in range(steps):
        llm.step()
    torch.cuda.synchronize()
    torch.cuda._sleep(1000)
    torch.cuda.synchronize()
    log(f"{steps} profiled steps done (between two spin_kernel markers)")


def timed_steps(llm, steps: int):
    """Wall time and committed tokens of ``steps`` engine steps (synchronised
    on both sides), plus the engine's speculation counters over them."""
    import torch

    before = dict(llm.spec_stats)
    pre_before = dict(llm.model_runner.prelaunch_stats)
    committed = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        _, num_tokens = llm.step()
        committed += -num_tokens
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    stats = {k: llm.spec_stats[k] - before[k] for k in before}
    stats["prelaunch"] = {k: llm.model_runner.prelaunch_stats[k] - pre_before[k] for k in pre_before}
    return elapsed, committed, stats


def generation(llm, warmup: int, steps: int, seq_row: dict):
    """Every decode step of the batch, from the first one after prefill to the
    last sequence's finish (the reference's decode throughput covers the
    whole generate(), llm_engine.py:175-185, :200-219), with the bench
    line's window inside it: after ``warmup`` steps, ``steps`` steps
    bracketed by synchronisations (the window's two synchronisations are
    the only ones the generation adds).  Returns (whole, window, outputs):
    whole / window = dicts of seconds, engine steps, committed tokens,
    speculation counters, mean keys per sequence at the start and end;
    outputs = {request row: completion token ids}."""
    import torch

    def mean_keys():
        run = llm.scheduler.running
        return round(sum(len(x) for x in run) / max(len(run), 1), 1)

    before = dict(llm.spec_stats)
    pre_before = dict(llm.model_runner.prelaunch_stats)
    outputs, n, committed = {}, 0, 0
    window = None
    keys0 = mean_keys()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    while not llm.is_finished():
        if n == warmup:
            torch.cuda.synchronize()
            w0, w_committed, w_keys = time.perf_counter(), committed, mean_keys()
            w_stats = dict(llm.spec_stats)
            w_pre = dict(llm.model_runner.prelaunch_stats)
        out, num_tokens = llm.step()
        if num_tokens > 0:
            raise RuntimeError("a prefill step inside the decode generation")
        committed += -num_tokens
        n += 1
        for seq_id, toks in out:
            outputs[seq_row[seq_id]] = toks
        if n == warmup + steps:
            torch.cuda.synchronize()
            w1 = time.perf_counter()
            window = {"seconds": w1 - w0, "steps": steps, "committed": committed - w_committed,
                      "keys_start": w_keys, "keys_end": mean_keys(),
                      "stats": {k: llm.spec_stats[k] - w_stats[k] for k in w_stats},
                      "prelaunch": {k: llm.model_runner.prelaunch_stats[k] - w_pre[k]
                                    for k in w_pre}}
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t_start
    whole = {"seconds": seconds, "steps": n, "committed": committed, "keys_start": keys0,
             "stats": {k: llm.spec_stats[k] - before[k] for k in before},
             "prelaunch": {k: llm.model_runner.prelaunch_stats[k] - pre_before[k]
                           for k in pre_before}}
    return whole, window, outputs


def generation_record(whole: dict, n_seqs: int, note: str) -> dict:
    st = whole["stats"]
    seq_steps = max(st["steps"], 1) * n_seqs
    return {"value": round(whole["committed"] / whole["seconds"], 1), "unit": "tok/s",
            "seconds": round(whole["seconds"], 3), "steps": whole["steps"],
            "ms_per_step": round(whole["seconds"] / max(whole["steps"], 1) * 1e3, 3),
            "committed_tokens": whole["committed"], "sequences": n_seqs,
            "mean_keys_per_seq_at_start": whole["keys_start"],
            "accepted_drafts": st["accepted"], "drafted": st["drafted"],
            "prelaunched_drafts": whole["prelaunch"], "note": note}


def reference_steps(llm, steps: int, torch_attention: bool):
    """The reference's step structure (llm_engine.py:124-178): one warm-up
    step, then ``steps`` timed ones; on this build's attention kernel or on
    the torch stand-in for FA2."""
    backend = TorchAttention() if torch_attention else None
    if backend:
        backend.install()
    llm.reference_pipeline = True
    try:
        llm.step()
        elapsed, committed, _ = timed_steps(llm, steps)
    finally:
        llm.reference_pipeline = False
        if backend:
            backend.uninstall()
    return {"value": round(committed / elapsed, 1), "unit": "tok/s",
            "ms_per_step": round(elapsed / steps * 1e3, 2), "steps": steps,
            "attention": ("torch paged gather + batched bf16 matmul / fp32 softmax (stand-in for "
                          "FlashAttention-2, flash_attn_varlen_func / flash_attn_with_kvcache at "
                          "layers/attention.py:385-399)") if torch_attention else
                         "this build's K1",
            "structure": "reference llm_engine.py:124-178 step shape: eager draft loop with a "
                         "host sync per draft step, eager target verify with one torch argmax + "
                         ".tolist() per sequence, host acceptance per sequence, serial "
                         "single-token draft replay per committed token "
                         "(model_runner.py:1127-1156)"}


def forced_acceptance(args, tmp: str, continuations):
    """The workload with accepted drafts: a fresh engine (same seeded
    weights and prompts) whose proposals are rewritten on the device, right
    after the draft graph, to the target's greedy continuation recorded by
    the main run, each draft position keeping the target's token with
    probability args.draft_keep (a seeded choice per sequence and position)
    and otherwise a different id.  The rewrite is one small host-to-device
    copy and one gather per step inside the timed region.  Timed like the
    main run: the whole generation, with a window of 3 + args.acceptance_steps
    steps at its start."""
    import torch

    llm = make_engine(args, tmp)
    runner = llm.model_runner
    prompts = add_prompts(llm, args)
    vocab = llm.config.hf_config.vocab_size
    width = max(len(c) for c in continuations.values()) + args.k + 1
    rng = torch.Generator().manual_seed(args.seed + 100)
    table = torch.zeros(len(prompts), width, dtype=torch.int64)
    for i, p in enumerate(prompts):
        cont = torch.tensor(continuations[tuple(p)], dtype=torch.int64)
        keep = torch.rand(cont.numel(), generator=rng) < args.draft_keep
        table[i, :cont.numel()] = torch.where(keep, cont, (cont + 1) % vocab)
    table = table.to(runner.device)
    row_of = {seq.seq_id: i for i, seq in enumerate(llm.scheduler.waiting)}
    pinned = torch.empty(2 * args.batch, dtype=torch.int64, pin_memory=True)

    def override(seqs, tokens):
        b, k = len(seqs), tokens.shape[0]
        pinned[:b] = torch.tensor([row_of[s.seq_id] for s in seqs])
        pinned[b:2 * b] = torch.tensor([len(s) for s in seqs])
        info = pinned[:2 * b].to(tokens.device, non_blocking=True)
        pos = info[b:][None, :] + torch.arange(k, device=tokens.device)[:, None]
        tokens[:, :b] = table[info[:b][None, :].expand(k, b), pos]

    seq_row = dict(row_of)
    try:
        while llm.scheduler.waiting:
            llm.step()
        runner.draft_override = override
        n_active = len(llm.scheduler.running)
        whole, window, outputs = generation(llm, 3, args.acceptance_steps, seq_row)
    finally:
        runner.draft_override = None
        release(llm)
    if window is None:
        raise RuntimeError("the forced-acceptance generation ended inside its timed window")
    stats = window["stats"]
    seq_steps = max(stats["steps"] * n_active, 1)
    # the forced drafts only reorder how the target's tokens are committed:
    # every sequence must end with the main run's greedy continuation
    same = sum(outputs[i] == continuations[tuple(p)][len(p):] for i, p in enumerate(prompts))
    wst = whole["stats"]
    return {"value": round(window["committed"] / window["seconds"], 1), "unit": "tok/s",
            "ms_per_step": round(window["seconds"] / args.acceptance_steps * 1e3, 3),
            "steps": args.acceptance_steps, "warmup": 3, "active_seqs": n_active,
            "draft_keep": args.draft_keep,
            "accepted_drafts_per_seq_step": round(stats["accepted"] / seq_steps, 4),
            "mean_acceptance_length": round(stats["committed"] / seq_steps, 4),
            "position_accept_rate": round(stats["accepted"] / max(stats["drafted"], 1), 4),
            "whole_generation": dict(generation_record(
                whole, n_active, "every decode step from the first after prefill to the last "
                "finished sequence, forced drafts (the window above is its steps 4-23)"),
                mean_acceptance_length=round(wst["committed"] / max(wst["steps"] * n_active, 1),
                                             4)),
            "outputs_equal_main_run": f"{same} of {len(prompts)}",
            "outputs_equal_note": (
                "the forced run's batch shrinks as its sequences finish, so its later verify "
                "steps run with other GEMM row counts and, below 33 sequences, another verify-"
                "attention decomposition (eight waves per split instead of paired mode), whose "
                "last-bit rounding differs; sequences that part from the main run do so where "
                "that rounding flips a near tie (with either decomposition forced for every "
                "batch size, 63 of 64 sequences equal)"),
            "drafts": "target-greedy continuation of each sequence (recorded by the main run, "
                      "whose steps commit exactly the target's argmax), kept per position with "
                      "probability draft_keep"}


def config5(args) -> None:
    """BASELINE config 5 through the engine: Qwen3-32B geometry (64 layers,
    H5120, 64 q / 8 kv heads, MLP 25600, V151936, random weights), an EAGLE3
    draft with k = 7 (8 verify rows per sequence, 64-row attention tiles),
    128 sequences with prompts of U[2048, 8192] random tokens (seed 4).  The
    pool's free list is shuffled (seeded), so block tables are fragmented.
    The config's 30% prefix-shared pages are a kernel-level property (the
    per-config K1 figure reads them): the engine, like the reference
    (config.py:150), turns prefix caching off with EAGLE3, because the
    draft's K/V at a page's last position depends on the next page's first
    token.  Without sharing the pages take ~198 GB next to 70 GB of weights.
    Prints one JSON line: step time and accepted tok/s over the timed steps
    (zero acceptance with random weights), the verify attention of one step
    re-issued between HIP events, and a greedy check of 4 sequences
    (teacher-forced prefill of prompt + output: the largest gap between an
    output token's logit and its row's top, in bf16 ulps; the GPU test of
    this geometry holds it to the plain engine's own gap)."""
    from collections import deque

    import torch

    from nanovllm_amd import LLM, SamplingParams
    from nanovllm_amd import kernels
    from nanovllm_amd.context import reset_context
    from nanovllm_amd.engine.sequence import Sequence
    from nanovllm_amd.synthetic import default_aux_layers, write_eagle3_config, write_qwen3_config

    preset, batch, k, block = "qwen3-32b", 128, 7, 256
    lo, hi, seed = 2048, 8192, 4
    timer = AttnTimer()
    timer.wrap(kernels)
    tmp = tempfile.mkdtemp(prefix="nva_c5_")
    target = write_qwen3_config(os.path.join(tmp, "target"), preset)
    aux = default_aux_layers(preset)
    draft = write_eagle3_config(os.path.join(tmp, "draft"), preset, aux_layers=aux)
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g).tolist()
    prompts = [torch.randint(0, 151936, (L,), generator=g).tolist() for L in lens]
    # one token per step at zero acceptance: the decode steps that alternate
    # with the ~40 prefill steps (16k tokens each), warm-up, timed and
    # roofline steps, and the k draft positions reserved ahead; the pool
    # also holds the greedy check's probe (its own full table)
    gen = 48 + args.warmup + args.steps + args.profile_steps + 2 + k + 1
    max_len = hi + gen
    pages = sum(-(-(L + gen) // block) for L in lens) + -(-max_len // block) + 8
    t0 = time.perf_counter()
    llm = LLM(target, load_format="dummy", seed=0, max_num_seqs=batch, max_model_len=max_len,
              num_kvcache_blocks=pages, max_num_batched_tokens=16384,
              enable_prefill_batching=True, gpu_memory_utilization=0.97,
              kv_cache_layout=args.kv_layout,
              speculative_config={"method": "eagle3", "model": draft,
                                  "num_speculative_tokens": k, "aux_hidden_state_layers": aux})
    runner = llm.model_runner
    bm = llm.scheduler.block_manager
    total = len(bm.blocks)
    bm.free_block_ids = deque(torch.randperm(total, generator=g).tolist())
    log(f"config5 engine up in {time.perf_counter() - t0:.1f}s ({total} of {pages} pages): "
        f"{runner.get_diagnostics()}")
    sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
    t0 = time.perf_counter()
    for p in prompts:
        llm.add_request(p, sp)
    steps = 0
    while llm.scheduler.waiting:
        llm.step()
        steps += 1
        if steps % 8 == 0:
            log(f"config5 prefill: {len(llm.scheduler.waiting)} waiting after {steps} steps")
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"config5 prefill done in {prefill_s:.1f}s ({steps} steps)")
    for _ in range(args.warmup):
        llm.step()
    n_active = len(llm.scheduler.running)
    elapsed, committed, stats = timed_steps(llm, args.steps)
    ctx = [len(s) + k + 1 for s in llm.scheduler.running]
    log(f"config5 timed {args.steps} steps in {elapsed:.3f}s")
    profiled_steps(llm, args.profile_steps)
    # the verify attention of one more step, re-issued between HIP events
    orig_verify = runner.verify_eagle3_batch_fused

    def verify_with_lens(seqs, n):
        timer.current_lens = [len(x) for x in seqs]
        try:
            return orig_verify(seqs, n)
        finally:
            timer.current_lens = None

    runner.verify_eagle3_batch_fused = verify_with_lens
    runner.use_verify_graph = False
    timer.capture = True
    llm.step()
    timer.capture = False
    runner.use_verify_graph = True
    runner.verify_eagle3_batch_fused = orig_verify
    roof = timer.measure(2, None)
    # greedy check of 4 sequences (the longest among them) by teacher forcing
    running = list(llm.scheduler.running)
    picks = sorted(running, key=lambda x: -len(x))[:1] + running[:3]
    worst, checked = 0.0, 0
    for seq in picks:
        toks = list(seq.token_ids)
        start = seq.num_prompt_tokens
        probe = Sequence(toks)
        bm.allocate(probe)
        probe.num_computed_tokens = 0
        probe.num_scheduled_tokens = len(toks)
        try:
            with torch.inference_mode():
                ids, pos = runner.prepare_prefill([probe])
                hidden = runner.model(ids, pos)
                rows = runner.model.compute_all_logits(hidden[start - 1:len(toks) - 1]).float()
        finally:
            reset_context()
            bm.deallocate(probe)
        top = rows.max(-1).values
        got = rows.gather(1, torch.tensor(toks[start:], device=rows.device)[:, None])[:, 0]
        ulp = torch.exp2(torch.floor(torch.log2(top.abs())) - 7)
        gaps = ((top - got) / ulp).cpu()
        worst = max(worst, float(gaps.max()))
        checked += gaps.numel()
    release(llm)
    seq_steps = max(stats["steps"] * n_active, 1)
    print(json.dumps({
        "workload": "BASELINE config 5 through LLM: Qwen3-32B geometry (64 layers, H5120, "
                    "64q/8kv, D128, MLP25600, V151936), EAGLE3 draft k=7, random weights, "
                    "shuffled pages (no prefix sharing with EAGLE3, as in the reference)",
        "batch": n_active, "k": k, "steps": args.steps, "warmup": args.warmup,
        "value": round(committed / elapsed, 1), "unit": "tok/s",
        "ms_per_step": round(elapsed / args.steps * 1e3, 2),
        "committed_per_seq_step": round(stats["committed"] / seq_steps, 4),
        "context_len": [min(ctx), max(ctx), round(sum(ctx) / len(ctx))],
        "prefill_s": round(prefill_s, 1), "pages": total,
        "verify_attention": roof,
        "greedy_check": {"sequences": len(picks), "tokens": checked,
                         "max_gap_ulps": round(worst, 1),
                         "note": "informational: the largest gap, in bf16 ulps of the row's top "
                                 "logit, between an emitted token's logit and the top of its "
                                 "teacher-forced prefill row; tests/test_engine_32b_gpu.py holds "
                                 "the speculative engine at this geometry to bounds measured "
                                 "from the plain engine in the same run (tests/greedy_e2e.py)"},
    }), flush=True)


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
        for rec in kernel_configs(args, 0.0 if args.no_cpu_baseline else 4.0):
            print(json.dumps({"bench": "kernels", **rec}), flush=True)
        return
    if args.workload == "config5":
        config5(args)
        return
    import torch

    from nanovllm_amd import kernels

    # Each hot-path kernel alone, first while the process is fresh: after an
    # engine has been built, run and released in the same process, the
    # streaming kernels read slower on memory allocated afterwards (K4 at
    # config 3's verify rows 20.9-21.2 -> 23.1-23.9 us, K1 at config 3
    # 61.1-61.3 -> 63.1-67.1 us, same code and shapes).  The engine's own
    # buffers are allocated in a fresh process, so the fresh figures are the
    # kernels'; the same records after the engines are kept beside them.
    per_config = None
    if not args.no_per_config:
        per_config = kernel_configs(args, 0.0 if args.no_cpu_baseline else 4.0)
        torch.cuda.empty_cache()

    timer = AttnTimer()
    timer.wrap(kernels)

    tmp = tempfile.mkdtemp(prefix="nva_bench_")
    llm = make_engine(args, tmp)
    runner = llm.model_runner
    log(f"engine up: {runner.get_diagnostics()}")
    seq_row = {}
    prompts = add_prompts(llm, args, seq_row)

    t_setup = time.perf_counter()
    while llm.scheduler.waiting:
        llm.step()
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    log(f"prefill done in {setup_s:.1f}s")
    n_active = len(llm.scheduler.running)

    # the whole generation, first decode step to last finished sequence, with
    # the line's window (W warm-up steps, then the K timed steps) at its start
    whole, window, outputs = generation(llm, args.warmup, args.steps, seq_row)
    if window is None:
        raise RuntimeError(f"the generation ended within {args.warmup} + {args.steps} steps")
    elapsed, committed, stats = window["seconds"], window["committed"], window["stats"]
    stats["prelaunch"] = window["prelaunch"]
    log(f"timed {args.steps} steps in {elapsed:.3f}s; whole generation: {whole['steps']} steps "
        f"in {whole['seconds']:.3f}s")
    # zero acceptance (random draft): every committed token is the target's
    # argmax, so the outputs are the target-greedy continuations the
    # forced-acceptance run replays as drafts
    continuations = {tuple(p): p + outputs[i] for i, p in enumerate(prompts)}

    # the same prompts again, for the measurements that need live sequences
    # and perturb a step (eager verify launches, host syncs): the CPU
    # baseline's logits, the roofline's attention launches, the
    # reference-structured steps
    add_prompts(llm, args, {})
    while llm.scheduler.waiting:
        llm.step()
    for _ in range(args.warmup):
        llm.step()
    profiled_steps(llm, args.profile_steps)

    orig_verify = runner.verify_eagle3_batch_fused

    def verify_with_lens(seqs, n):
        timer.current_lens = [len(s) for s in seqs]
        try:
            return orig_verify(seqs, n)
        finally:
            timer.current_lens = None

    runner.verify_eagle3_batch_fused = verify_with_lens
    cpu_batches = []
    if not args.no_cpu_baseline:
        runner.keep_verify_inputs = True
        llm.step()
        logits, cu, ids = runner.last_verify_inputs
        cpu_batches.append((logits.cpu(), list(cu), ids.cpu().tolist()))
        runner.keep_verify_inputs = False
        runner.last_verify_inputs = None

    # roofline: one more step of the same workload with the verify forward
    # launched eagerly (events cannot be recorded inside a captured HIP graph
    # on ROCm); its verify-attention launches, with the timed steps' kernels
    # and shapes, are then re-issued back to back between HIP events
    runner.use_verify_graph = False
    timer.capture = True
    llm.step()
    timer.capture = False
    runner.use_verify_graph = True
    traffic = pmc_traffic_bytes(args)
    roof = timer.measure(args.roofline_repeats, traffic)
    if roof is not None:
        roof["traffic_source"] = (
            "recorded constant (not measured by this run): rocprofv3 --pmc FETCH_SIZE then "
            "WRITE_SIZE over `bench.py --attention-only` on this workload, scaled by the same "
            "counters' readings for a 1 GiB device copy and a 1 GiB read, measured on "
            f"paged_attention.hip sha256[:16] {PMC_ATTENTION_SOURCE}; "
            "profiles/verify_attention_traffic_qwen3_8b_bs64.md" if traffic is not None else
            "null: " + pmc_traffic_reason(args))

    ref = ref_torch = None
    if args.reference_steps > 0 and llm.scheduler.running:
        ref = reference_steps(llm, args.reference_steps, torch_attention=False)
        log(f"reference-structured steps: {ref['ms_per_step']} ms/step")
        ref_torch = reference_steps(llm, args.reference_steps, torch_attention=True)
        log(f"reference-structured steps, torch attention: {ref_torch['ms_per_step']} ms/step")
    cpu = None
    if cpu_batches:
        cpu = cpu_baseline(cpu_batches, args.cpu_seconds)
    release(llm)

    forced = None
    if args.acceptance_steps > 0:
        forced = forced_acceptance(args, tmp, continuations)
        log(f"forced acceptance: {forced['value']} tok/s, {forced['ms_per_step']} ms/step, "
            f"mean acceptance length {forced['mean_acceptance_length']}; whole generation "
            f"{forced['whole_generation']['value']} tok/s")
    per_config_after = None
    if not args.no_per_config:
        per_config_after = [{k: v for k, v in rec.items() if k != "cpu_baseline"}
                            for rec in kernel_configs(args, 0.0)]

    metric, workload = workload_label(args)
    result = {
        "metric": metric,
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
        "config": {"workload": workload,
                   "preset": args.preset, "batch": args.batch, "k": args.k,
                   "prompt_len": [args.prompt_min, args.prompt_max],
                   "max_tokens": args.max_tokens, "active_seqs": n_active,
                   "hip_graphs": not args.eager, "kv_layout": args.kv_layout,
                   "gemm_tuning": os.path.basename(args.gemm_tuning) if args.gemm_tuning else None},
        "roofline": roof,
        "cpu_baseline": cpu,
        "committed_tokens": committed,
        "window": {"position": f"decode steps {args.warmup + 1}-{args.warmup + args.steps} of "
                               f"{whole['steps']}",
                   "mean_keys_per_seq": [window["keys_start"], window["keys_end"]]},
        "whole_generation": generation_record(
            whole, n_active, "every decode step from the first after prefill to the last "
            "finished sequence, in the run that holds the timed window (its only extra "
            "synchronisations are the window's two)"),
        "accepted_drafts_per_seq_step": round(stats["accepted"] / max(stats["steps"] * n_active, 1), 4),
        "committed_per_seq_step": round(stats["committed"] / max(stats["steps"] * n_active, 1), 4),
        "prelaunched_drafts": dict(stats["prelaunch"], note=(
            "timed steps whose draft was queued behind the previous step's verify "
            "(used) and next-step drafts queued (queued)")),
        "forced_acceptance": forced,
        "reference_pipeline": ref,
        "reference_pipeline_torch_attention": ref_torch,
        "per_config": per_config,
        "per_config_after_engines": per_config_after,
        "per_config_note": "per_config: each kernel alone at the BASELINE configs' shapes, timed "
                           "before any engine ran in this process; per_config_after_engines: the "
                           "same records after the engines were built, run and released (memory "
                           "allocated after that reads slower)" if per_config else None,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
