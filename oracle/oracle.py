"""Python face of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import this module, and only to check or to time the reference
algorithm.  The product package never imports it.

The numeric restatements live in spec_oracle.c (built into liboracle.so by
oracle/Makefile); this module loads it with ctypes and wraps each entry point
for numpy arrays.  It also holds the pure-Python restatements of the
reference's host-side acceptance logic:

* ``verify_greedy_proposals`` restates nanovllm/engine/speculative.py:11-30.
* ``verify_metadata`` restates the per-token loops of prepare_prefill
  (nanovllm/engine/model_runner.py:761-800) for verify rows.
* ``commit_metadata`` and ``draft_metadata`` restate the draft's commit
  replay and draft-step contexts (model_runner.py:1087-1096, :1127-1156,
  :1216-1249) in either draft slot convention (slot_offset 0 or 1).
* ``reference_cpu_acceptance`` restates the per-sequence
  ``logits[start:end].argmax(dim=-1).tolist()`` loop of
  nanovllm/engine/model_runner.py:1066-1074 followed by
  ``verify_greedy_proposals`` per sequence (nanovllm/engine/llm_engine.py:154-156);
  bench.py times it as the CPU baseline.

Pinning of each function is covered by tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so from spec_oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_F64 = ctypes.c_double


def _declare(l: ctypes.CDLL) -> None:
    l.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
    l.oracle_bf16_to_f32.restype = _F32
    l.oracle_f32_to_bf16.argtypes = [_F32]
    l.oracle_f32_to_bf16.restype = ctypes.c_uint16
    l.oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
    l.oracle_e4m3_to_f32.restype = _F32
    l.oracle_f32_to_e4m3.argtypes = [_F32]
    l.oracle_f32_to_e4m3.restype = ctypes.c_uint8
    l.oracle_argmax_bf16.argtypes = [_P, _I64, _I64, _I64, _P]
    l.oracle_argmax_bf16.restype = None
    l.oracle_accept.argtypes = [_P, _I32, _P, _P, _P, _P]
    l.oracle_accept.restype = None
    l.oracle_store_kv.argtypes = [_P, _I64, _P, _I64, _P, _P, _I32, _P, _I32, _I32,
                                  _I64, _F32, _F32]
    l.oracle_store_kv.restype = None
    l.oracle_rollback.argtypes = [_P, _P, _I32, _P, _P, _P, _P, _I32, _I32, _I64, _I32]
    l.oracle_rollback.restype = None
    l.oracle_aux_gather.argtypes = [_P, _P, _I32, _I64, _I32, _P, _I32, _P, _I64]
    l.oracle_aux_gather.restype = None
    l.oracle_paged_attention.argtypes = [_P, _I64, _I64, _P, _P, _I32, _I64, _I64, _I64,
                                         _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32,
                                         _F64, _F64, _F64, _P]
    l.oracle_paged_attention.restype = None
    l.oracle_fp8_paged_decode.argtypes = [_P, _I64, _I64, _P, _P, _I64, _I64, _I64,
                                          _P, _P, _I64, _I32, _I32, _I32, _I32, _I32,
                                          _F32, _F32, _F32, _P]
    l.oracle_fp8_paged_decode.restype = None


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


# ---------------------------------------------------------------- scalars

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    f = np.vectorize(lambda v: lib().oracle_f32_to_bf16(float(v)), otypes=[np.uint16])
    return f(np.asarray(x, np.float32))


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    table = np.array([lib().oracle_e4m3_to_f32(c) for c in range(256)], np.float32)
    return table[np.asarray(codes, np.uint8)]


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    f = np.vectorize(lambda v: lib().oracle_f32_to_e4m3(float(v)), otypes=[np.uint8])
    return f(np.asarray(x, np.float32))


# ---------------------------------------------------------------- K4

def argmax_bf16(logits_bits: np.ndarray) -> np.ndarray:
    """Row argmax of a [rows, vocab] uint16 (bfloat16 bit pattern) array."""
    x = _c(logits_bits, np.uint16)
    rows, vocab = x.shape
    out = np.empty(rows, np.int32)
    lib().oracle_argmax_bf16(_ptr(x), rows, vocab, vocab, _ptr(out))
    return out


def accept(cu_q, argmax, input_ids):
    """Accepted-prefix length and bonus token per sequence (int32 arrays)."""
    cu = _c(cu_q, np.int32)
    am = _c(argmax, np.int32)
    ids = _c(input_ids, np.int64)
    b = cu.size - 1
    acc = np.empty(b, np.int32)
    bonus = np.empty(b, np.int32)
    lib().oracle_accept(_ptr(cu), b, _ptr(am), _ptr(ids), _ptr(acc), _ptr(bonus))
    return acc, bonus


# ---------------------------------------------------------------- K2

def store_kv(key_bits, value_bits, k_cache, v_cache, slot_mapping, k_scale=1.0, v_scale=1.0):
    """In-place store into caches shaped [num_blocks, block_size, Hkv, D].

    key/value: uint16 [T, Hkv, D]; caches uint16 (bf16) or uint8 (e4m3)."""
    k = _c(key_bits, np.uint16)
    v = _c(value_bits, np.uint16)
    slots = _c(slot_mapping, np.int32)
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    kv_dtype = 0 if k_cache.dtype == np.uint16 else 1
    t = k.shape[0]
    row = int(np.prod(k.shape[1:]))
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    lib().oracle_store_kv(_ptr(k), row, _ptr(v), row, _ptr(k_cache), _ptr(v_cache), kv_dtype,
                          _ptr(slots), t, row, num_slots, float(k_scale), float(v_scale))


def rollback(cu_q, accept_len, slot_mapping, seqlens_k, k_cache, v_cache, poison=False):
    """Returns (slot_mapping, seqlens_k) after rollback; caches edited in place."""
    cu = _c(cu_q, np.int32)
    acc = _c(accept_len, np.int32)
    slots = _c(slot_mapping, np.int32).copy()
    lens = _c(seqlens_k, np.int32).copy()
    kv_dtype = 0 if k_cache.dtype == np.uint16 else 1
    row = int(np.prod(k_cache.shape[2:]))
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    lib().oracle_rollback(_ptr(cu), _ptr(acc), cu.size - 1, _ptr(slots), _ptr(lens),
                          _ptr(k_cache), _ptr(v_cache), kv_dtype, row, num_slots, int(poison))
    return slots, lens


# ---------------------------------------------------------------- K3

def aux_gather(hidden, residual, src_rows):
    """hidden/residual: lists of uint16 [T, H]; returns uint16 [R, L*H]."""
    hs = [_c(h, np.uint16) for h in hidden]
    rs = [_c(r, np.uint16) for r in residual]
    n = len(hs)
    t, h = hs[0].shape
    src = _c(src_rows, np.int32)
    out = np.empty((src.size, n * h), np.uint16)
    hp = (ctypes.c_void_p * n)(*[_ptr(a) for a in hs])
    rp = (ctypes.c_void_p * n)(*[_ptr(a) for a in rs])
    lib().oracle_aux_gather(hp, rp, n, h, h, _ptr(src), src.size, _ptr(out), n * h)
    return out


# ---------------------------------------------------------------- K1

def paged_attention(q_bits, k_cache, v_cache, cu_q, seqlens_k, block_tables, softmax_scale,
                    k_scale=1.0, v_scale=1.0):
    """Textbook paged causal attention (double accumulation).

    q_bits: uint16 [T, Hq, D]; caches [num_blocks, block_size, Hkv, D] uint16
    (bf16) or uint8 (e4m3); block_tables int32 [B, max_blocks]. Returns float32
    [T, Hq, D]."""
    q = _c(q_bits, np.uint16)
    t, hq, d = q.shape
    kc = np.ascontiguousarray(k_cache)
    vc = np.ascontiguousarray(v_cache)
    nb, bs, hkv, d2 = kc.shape
    assert d2 == d
    kv_dtype = 0 if kc.dtype == np.uint16 else 1
    cu = _c(cu_q, np.int32)
    lens = _c(seqlens_k, np.int32)
    bt = _c(block_tables, np.int32)
    out = np.zeros((t, hq, d), np.float32)
    lib().oracle_paged_attention(_ptr(q), hq * d, d, _ptr(kc), _ptr(vc), kv_dtype,
                                 bs * hkv * d, hkv * d, d, _ptr(cu), _ptr(lens), _ptr(bt),
                                 bt.shape[1], cu.size - 1, hq, hkv, d, bs,
                                 float(softmax_scale), float(k_scale), float(v_scale), _ptr(out))
    return out


def fp8_paged_decode(q_bits, k_cache, v_cache, context_lens, block_tables, softmax_scale,
                     k_scale=1.0, v_scale=1.0):
    """Restatement of the reference FP8 paged decode kernel (one row per token)."""
    q = _c(q_bits, np.uint16)
    t, hq, d = q.shape
    kc = _c(k_cache, np.uint8)
    vc = _c(v_cache, np.uint8)
    nb, bs, hkv, _ = kc.shape
    ctx = _c(context_lens, np.int32)
    bt = _c(block_tables, np.int32)
    out = np.zeros((t, hq, d), np.float32)
    lib().oracle_fp8_paged_decode(_ptr(q), hq * d, d, _ptr(kc), _ptr(vc), bs * hkv * d, hkv * d, d,
                                  _ptr(ctx), _ptr(bt), bt.shape[1], t, hq, hkv, d, bs,
                                  float(softmax_scale), float(k_scale), float(v_scale), _ptr(out))
    return out


# ---------------------------------------------------------------- host logic

@dataclass(frozen=True)
class GreedyVerification:
    accepted_count: int
    accepted_tokens: list
    replacement_token: int | None


def verify_greedy_proposals(proposal_tokens, target_tokens) -> GreedyVerification:
    """Restates nanovllm/engine/speculative.py:11-30."""
    if len(target_tokens) < len(proposal_tokens):
        raise ValueError("target verification must cover every proposal")
    n = 0
    for p, t in zip(proposal_tokens, target_tokens):
        if p != t:
            return GreedyVerification(n, list(proposal_tokens[:n]), t)
        n += 1
    repl = target_tokens[n] if len(target_tokens) > n else None
    return GreedyVerification(n, list(proposal_tokens), repl)


def reference_cpu_acceptance(logits, cu_q, input_ids):
    """The reference's host acceptance path on a CPU torch tensor.

    logits: torch.bfloat16 [T, V] (CPU); cu_q: list[int]; input_ids: list[int]
    (verify inputs, proposals at rows 1..q_i-1).  Per sequence: bf16 argmax of
    its rows + .tolist() (model_runner.py:1071-1073), then
    verify_greedy_proposals (llm_engine.py:154-156).  Returns
    (accept_len list, bonus list, committed token count)."""
    accepted, bonus = [], []
    committed = 0
    for i in range(len(cu_q) - 1):
        s, e = cu_q[i], cu_q[i + 1]
        target = logits[s:e].argmax(dim=-1).tolist()
        v = verify_greedy_proposals(input_ids[s + 1:e], target)
        accepted.append(v.accepted_count)
        bonus.append(v.replacement_token)
        committed += v.accepted_count + (v.replacement_token is not None)
    return accepted, bonus, committed


def _slot_of(row, position, block_size):
    """Slot of a token position through one block-table row
    (model_runner.py:784-789): -1 for a negative block id (the reference's
    padding, :755-759) or a position past the row."""
    idx = position // block_size
    bid = int(row[idx]) if 0 <= idx < len(row) else -1
    return bid * block_size + position % block_size if bid >= 0 else -1


def verify_metadata(start_pos, q_lens, block_tables, block_size, num_tokens, slot_offset=0):
    """Restates prepare_prefill's per-sequence loop for verify rows
    (nanovllm/engine/model_runner.py:770-789): sequence i covers positions
    start .. start + q - 1, sees start + q keys, and token position p maps to
    slot block_table[p // block_size] * block_size + p % block_size.  Block
    ids of -1 (the reference's padding, :755-759) give slot -1 here, and rows
    past the last sequence get position 0 and slot -1.  slot_offset (draft
    commits only) moves every row's K/V to the slot of position
    p + slot_offset and the key count to start + q + slot_offset.  Returns
    int numpy arrays (cu_q, cu_k, positions, slots)."""
    cu_q, cu_k, positions, slots = [0], [0], [], []
    for i, (start, q) in enumerate(zip(start_pos, q_lens)):
        cu_q.append(cu_q[-1] + int(q))
        cu_k.append(cu_k[-1] + int(start) + int(q) + int(slot_offset))
        row = list(block_tables[i])
        for p in range(int(start), int(start) + int(q)):
            positions.append(p)
            slots.append(_slot_of(row, p + int(slot_offset), block_size))
    pad = num_tokens - len(positions)
    positions += [0] * pad
    slots += [-1] * pad
    return (np.array(cu_q, np.int32), np.array(cu_k, np.int32),
            np.array(positions[:num_tokens], np.int64), np.array(slots[:num_tokens], np.int32))


def commit_metadata(start_pos, accept_len, q_stride, verify_argmax, block_tables, block_size,
                    num_tokens, slot_offset=0):
    """Restates what commit_eagle3 builds for one sequence
    (nanovllm/engine/model_runner.py:1216-1249: the output tokens, their
    positions start .. start + n - 1, the first n aux rows of the
    sequence's verify block, the last row's draft state), laid end to end
    for a batch: sequence i commits n_i = min(max(a_i, 0) + 1, q_stride)
    tokens, the verify argmax of its rows i * q_stride .. + n_i - 1 (the
    accepted drafts equal the argmax of their rows; the last is the
    bonus).  Rows past the committed ones read verify row -1 -> token of
    row 0.  slot_offset = 1 is the reference's slots and contexts
    (_commit_eagle3_tokens, :1127-1156: token i at slot start + 1 + i,
    context start + 2 + i); 0 stores position p at slot p.  Returns
    (cu_q, cu_k, positions, slots, verify_rows, token_ids, last_rows) as
    numpy arrays."""
    n = [min(max(int(a), 0) + 1, int(q_stride)) for a in accept_len]
    cu_q, cu_k, positions, slots = verify_metadata(start_pos, n, block_tables, block_size,
                                                   num_tokens, slot_offset)
    rows = []
    for i, ni in enumerate(n):
        rows += [i * int(q_stride) + j for j in range(ni)]
    rows = (rows + [-1] * num_tokens)[:num_tokens]
    am = np.asarray(verify_argmax)
    ids = [int(am[r]) if 0 <= r < len(am) else (int(am[0]) if len(am) else 0) for r in rows]
    last = [int(cu_q[i + 1]) - 1 for i in range(len(n))]
    return (cu_q, cu_k, positions, slots, np.array(rows, np.int32), np.array(ids, np.int64),
            np.array(last, np.int64))


def draft_metadata(lens, verify_row, accept_len, num_seqs, bs, steps, block_tables, block_size,
                   slot_offset=0):
    """Restates the per-step loop of propose_eagle3_batch /
    _set_eagle3_decode_context (nanovllm/engine/model_runner.py:1087-1096,
    :1190-1203) for the draft queued behind a verify: column i < num_seqs
    is a sequence of length L = lens[i] + accept_len[verify_row[i]] + 1
    after the verified step; its step s queries RoPE position
    p = L - 1 + s, writes its K/V at the slot of position p + slot_offset and
    sees p + slot_offset + 1 keys (the reference: slot len + step, context
    len + step + 1, i.e. slot_offset = 1).  Padding columns get position 0,
    slot -1 and context 1.  Returns int numpy arrays [steps, bs]
    (positions int64, slots int32, contexts int32)."""
    pos = np.zeros((steps, bs), np.int64)
    slots = np.full((steps, bs), -1, np.int32)
    ctx = np.ones((steps, bs), np.int32)
    for i in range(num_seqs):
        length = int(lens[i]) + int(accept_len[int(verify_row[i])]) + 1
        row = list(block_tables[i])
        for step in range(steps):
            p = length - 1 + step
            pos[step, i] = p
            slots[step, i] = _slot_of(row, p + int(slot_offset), block_size)
            ctx[step, i] = p + int(slot_offset) + 1
    return pos, slots, ctx
