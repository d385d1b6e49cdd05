"""torch-tensor front end of the HIP kernels (libnanovllm_amd.so).

Each function mirrors the reference operator it replaces -- same argument
meaning, same errors -- and forwards raw device pointers, element strides
and the current HIP stream to the C ABI in include/nanovllm_amd.h.  All work
is enqueued on ``torch.cuda.current_stream()`` without host synchronisation,
so every call can be captured in a HIP graph (workspaces must then be
reserved before capture, see ``reserve_workspace``).

There is no CPU or PyTorch fallback: without the HIP library (or without a
GPU) these functions raise.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native
from ._native import check

BF16 = torch.bfloat16
FP8 = torch.float8_e4m3fn


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _kv_dtype(cache: torch.Tensor) -> int:
    if cache.dtype == BF16:
        return _native.KV_BF16
    if cache.dtype == FP8:
        return _native.KV_FP8_E4M3
    raise TypeError(f"KV cache dtype must be bfloat16 or float8_e4m3fn, got {cache.dtype}")


def _require_cuda(*tensors: torch.Tensor) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("nanovllm_amd kernels take device (cuda) tensors only")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")


def _i32(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous int32 tensor")


def _scale(s) -> torch.Tensor | None:
    if s is None:
        return None
    if not isinstance(s, torch.Tensor) or s.dtype != torch.float32 or s.numel() != 1:
        raise TypeError("k_scale / v_scale must be one-element float32 tensors")
    return s


# ---------------------------------------------------------------- workspaces

class _Workspaces:
    """Per-(device, kind) scratch buffers that only grow.

    Superseded buffers are kept alive because captured graphs may still point
    at them."""

    def __init__(self) -> None:
        self._bufs: dict[tuple[int, str], torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def get(self, device: torch.device, kind: str, nbytes: int) -> torch.Tensor:
        key = (device.index if device.index is not None else torch.cuda.current_device(), kind)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"{kind} workspace of {nbytes} bytes was not reserved before graph capture")
            size = max(int(nbytes), 4096)
            if buf is not None:
                self._retired.append(buf)
                size = max(size, 2 * buf.numel())
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


_WS = _Workspaces()


def reserve_workspace(device: torch.device, kind: str, nbytes: int) -> None:
    """Grow a workspace ahead of HIP-graph capture ('argmax' or 'attention')."""
    _WS.get(device, kind, nbytes)


def argmax_workspace_bytes(num_rows: int, num_seqs: int, vocab: int) -> int:
    return int(_native.load().nva_argmax_workspace_size(num_rows, num_seqs, vocab))


def attention_workspace_bytes(num_seqs: int, num_tokens: int, num_q_heads: int, num_kv_heads: int,
                              head_dim: int, max_seqlen_q: int, max_seqlen_k: int) -> int:
    return int(_native.load().nva_paged_attention_workspace_size(
        num_seqs, num_tokens, num_q_heads, num_kv_heads, head_dim, max_seqlen_q, max_seqlen_k))


# ---------------------------------------------------------------- K2

def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                  k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> None:
    """Write key/value rows into the paged caches at ``slot_mapping``.

    Mirrors nanovllm.layers.attention.store_kvcache (attention.py:189-217):
    key/value [N, Hkv, D] with unit element stride and head stride D, caches
    [num_blocks, block_size, Hkv, D] (any block / token / head strides with a
    contiguous head_dim, so head-major pages seen through a permuted view
    work too), slot -1 skipped; FP8 caches store e4m3(x / scale)."""
    lib = _native.load()
    _require_cuda(key, value, k_cache, v_cache, slot_mapping)
    n, hkv, d = key.shape
    if key.dtype != BF16 or value.dtype != BF16:
        raise TypeError("key/value must be bfloat16")
    if not (key.stride(-1) == 1 and value.stride(-1) == 1):
        raise ValueError("key/value must have unit stride in the last dim")
    if not (key.stride(1) == d and value.stride(1) == d):
        raise ValueError("key/value head stride must equal head_dim")
    kvd, bstr, tstr, hstr, nb, bs, c_hkv, c_d = _cache_args(k_cache, v_cache)
    if (c_hkv, c_d) != (hkv, d):
        raise ValueError("cache heads / head_dim do not match key")
    if slot_mapping.numel() != n:
        raise ValueError("slot_mapping must have one entry per token")
    _i32(slot_mapping, "slot_mapping")
    check(lib.nva_store_kvcache_paged(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_cache.data_ptr(),
        v_cache.data_ptr(), kvd, bstr, tstr, hstr, nb, bs, slot_mapping.data_ptr(), n, hkv, d,
        _ptr(_scale(k_scale)), _ptr(_scale(v_scale)), _stream()), "store_kvcache")


def store_kvcache_rows(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                       k_scale: torch.Tensor | None = None,
                       v_scale: torch.Tensor | None = None) -> None:
    """store_kvcache through the reference-shaped entry point
    (``nva_store_kvcache``): caches with contiguous token rows only, as the
    reference asserts (attention.py:198-203)."""
    lib = _native.load()
    _require_cuda(key, value, k_cache, v_cache, slot_mapping)
    n, hkv, d = key.shape
    row = hkv * d
    if k_cache.stride(1) != row or v_cache.stride(1) != row or k_cache.stride(-1) != 1:
        raise ValueError("cache token stride must equal num_kv_heads * head_dim")
    if k_cache.dtype != v_cache.dtype:
        raise TypeError("k_cache and v_cache must share a dtype")
    _i32(slot_mapping, "slot_mapping")
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    check(lib.nva_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_cache.data_ptr(),
        v_cache.data_ptr(), _kv_dtype(k_cache), slot_mapping.data_ptr(), n, hkv, d, num_slots,
        _ptr(_scale(k_scale)), _ptr(_scale(v_scale)), _stream()), "store_kvcache")


def rollback(cu_seqlens_q: torch.Tensor, accept_len: torch.Tensor, slot_mapping: torch.Tensor,
             seqlens_k: torch.Tensor, k_cache: torch.Tensor | None = None,
             v_cache: torch.Tensor | None = None, poison: bool = False) -> None:
    """Device-side rollback of rejected verify rows (in place).

    Rows j > accept_len[i] of sequence i get slot -1 and seqlens_k[i] drops by
    their count (the logical rollback of scheduler.py:165-170 /
    block_manager.py:197-205).  With ``poison`` the rejected slots are zeroed
    in every layer of k_cache / v_cache, given as [layers, num_blocks,
    block_size, Hkv, D] or one layer [num_blocks, block_size, Hkv, D]."""
    lib = _native.load()
    _require_cuda(cu_seqlens_q, accept_len, slot_mapping, seqlens_k, k_cache, v_cache)
    for t, name in ((cu_seqlens_q, "cu_seqlens_q"), (accept_len, "accept_len"),
                    (slot_mapping, "slot_mapping"), (seqlens_k, "seqlens_k")):
        _i32(t, name)
    b = accept_len.numel()
    if cu_seqlens_q.numel() != b + 1 or seqlens_k.numel() != b:
        raise ValueError("cu_seqlens_q must have num_seqs + 1 entries, seqlens_k num_seqs")
    kc = vc = 0
    layers = 1
    layer_stride = row = num_slots = 0
    kv_dtype = _native.KV_BF16
    if poison:
        if k_cache is None or v_cache is None:
            raise ValueError("poison needs the caches")
        if k_cache.dim() == 4:
            k_cache, v_cache = k_cache.unsqueeze(0), v_cache.unsqueeze(0)
        layers, nb, bs, hkv, d = k_cache.shape
        row = hkv * d
        num_slots = nb * bs
        layer_stride = k_cache.stride(0)
        if not (k_cache.stride(2) == row and v_cache.stride(0) == layer_stride
                and v_cache.stride(2) == row):
            raise ValueError("caches must be contiguous per layer")
        kc, vc = k_cache.data_ptr(), v_cache.data_ptr()
        kv_dtype = _kv_dtype(k_cache)
    check(lib.nva_rollback(cu_seqlens_q.data_ptr(), accept_len.data_ptr(), b,
                           slot_mapping.data_ptr(), seqlens_k.data_ptr(), kc, vc, kv_dtype,
                           layers, layer_stride, row, num_slots, int(poison), _stream()),
          "rollback")


# ---------------------------------------------------------------- K3

def aux_gather(hidden: list[torch.Tensor], residual: list[torch.Tensor], src_rows: torch.Tensor,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """out[r] = concat_l bf16(hidden[l][src_rows[r]] + residual[l][src_rows[r]]).

    Fuses models/qwen3.py:284-289 (aux add + torch.cat) with the row slicing
    of model_runner.py:1073/:1236-1242."""
    lib = _native.load()
    n = len(hidden)
    if n != len(residual) or not 1 <= n <= 4:
        raise ValueError("need 1..4 (hidden, residual) pairs")
    _require_cuda(*hidden, *residual, src_rows, out)
    _i32(src_rows, "src_rows")
    rows, h = hidden[0].shape
    stride = hidden[0].stride(0)
    for t in (*hidden, *residual):
        if t.dtype != BF16 or t.shape != (rows, h) or t.stride(1) != 1 or t.stride(0) != stride:
            raise ValueError("hidden/residual must be bf16 [rows, H] with one shared row stride")
    r = src_rows.numel()
    if out is None:
        out = torch.empty(r, n * h, dtype=BF16, device=hidden[0].device)
    if out.shape != (r, n * h) or out.stride(1) != 1 or out.dtype != BF16:
        raise ValueError("out must be bf16 [R, L*H] with unit last stride")
    hp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in hidden])
    rp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in residual])
    check(lib.nva_aux_gather(hp, rp, n, stride, h, rows, src_rows.data_ptr(), r, out.data_ptr(),
                             out.stride(0), _stream()), "aux_gather")
    return out


# ---------------------------------------------------------------- K4

def argmax_accept(logits: torch.Tensor, cu_seqlens_q: torch.Tensor, input_ids: torch.Tensor,
                  out: torch.Tensor | None = None):
    """Fused verify argmax + greedy acceptance for a whole batch.

    Replaces the per-sequence ``logits[s:e].argmax(-1).tolist()`` of
    model_runner.py:1066-1074 plus verify_greedy_proposals
    (speculative.py:11-30).  ``input_ids`` are the int64 verify inputs (the
    proposals sit at rows 1..q_i-1 of each sequence).  Returns int32
    (argmax[T], accept_len[B], bonus[B]) -- views of ``out`` (int32, T + 2B)
    when given, so one copy brings all three to the host."""
    lib = _native.load()
    _require_cuda(logits, cu_seqlens_q, input_ids, out)
    if logits.dtype != BF16 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be bf16 [T, V] with unit last stride")
    _i32(cu_seqlens_q, "cu_seqlens_q")
    if input_ids.dtype != torch.int64 or not input_ids.is_contiguous():
        raise TypeError("input_ids must be contiguous int64")
    t, v = logits.shape
    b = cu_seqlens_q.numel() - 1
    if input_ids.numel() != t:
        raise ValueError("input_ids must have one entry per logits row")
    if out is None:
        out = torch.empty(t + 2 * b, dtype=torch.int32, device=logits.device)
    if out.dtype != torch.int32 or not out.is_contiguous() or out.numel() < t + 2 * b:
        raise ValueError("out must be contiguous int32 with at least T + 2B entries")
    argmax, acc, bonus = out[:t], out[t:t + b], out[t + b:t + 2 * b]
    nbytes = argmax_workspace_bytes(t, b, v)
    ws = _WS.get(logits.device, "argmax", nbytes)
    check(lib.nva_argmax_accept(logits.data_ptr(), logits.stride(0), v, cu_seqlens_q.data_ptr(), b,
                                t, input_ids.data_ptr(), argmax.data_ptr(), acc.data_ptr(),
                                bonus.data_ptr(), ws.data_ptr(), ws.numel(), _stream()),
          "argmax_accept")
    return argmax, acc, bonus


def argmax_accept_static(logits: torch.Tensor, cu_seqlens_q: torch.Tensor,
                         input_ids: torch.Tensor, out: torch.Tensor) -> tuple:
    """``argmax_accept`` through the allocation-free entry point
    (``nva_argmax_accept_static``): the chunk keys go to the library's static
    per-device array instead of a workspace, and the caller provides ``out``
    (int32, at least T + 2B entries), so nothing is allocated on any path.
    Raises ValueError when T * ceil(V / 16384) exceeds the array
    (``_native.ARGMAX_STATIC_KEYS`` keys).  Calls that overlap on one GPU
    share the array and must be serialised."""
    lib = _native.load()
    _require_cuda(logits, cu_seqlens_q, input_ids, out)
    if logits.dtype != BF16 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be bf16 [T, V] with unit last stride")
    _i32(cu_seqlens_q, "cu_seqlens_q")
    if input_ids.dtype != torch.int64 or not input_ids.is_contiguous():
        raise TypeError("input_ids must be contiguous int64")
    t, v = logits.shape
    b = cu_seqlens_q.numel() - 1
    if input_ids.numel() != t:
        raise ValueError("input_ids must have one entry per logits row")
    if out.dtype != torch.int32 or not out.is_contiguous() or out.numel() < t + 2 * b:
        raise ValueError("out must be contiguous int32 with at least T + 2B entries")
    argmax, acc, bonus = out[:t], out[t:t + b], out[t + b:t + 2 * b]
    check(lib.nva_argmax_accept_static(logits.data_ptr(), logits.stride(0), v,
                                       cu_seqlens_q.data_ptr(), b, t, input_ids.data_ptr(),
                                       argmax.data_ptr(), acc.data_ptr(), bonus.data_ptr(),
                                       _stream()), "argmax_accept_static")
    return argmax, acc, bonus


def argmax_rows(logits: torch.Tensor, index_map: torch.Tensor | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy token per row: argmax (+ index_map[argmax]) as int64.

    Replaces Eagle3ForCausalLM.sample_greedy (eagle3.py:294-296, index_map =
    d2t) and Sampler's temperature-0 branch (sampler.py:10-19)."""
    lib = _native.load()
    _require_cuda(logits, index_map, out)
    if logits.dtype != BF16 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be bf16 [rows, V] with unit last stride")
    rows, v = logits.shape
    if index_map is not None and (index_map.dtype != torch.int64 or index_map.numel() != v
                                  or not index_map.is_contiguous()):
        raise ValueError("index_map must be contiguous int64 [V]")
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    if out.dtype != torch.int64 or not out.is_contiguous() or out.numel() < rows:
        raise ValueError("out must be contiguous int64 [rows]")
    nbytes = argmax_workspace_bytes(rows, 0, v)
    ws = _WS.get(logits.device, "argmax", nbytes)
    check(lib.nva_argmax_rows(logits.data_ptr(), logits.stride(0), v, rows, _ptr(index_map),
                              out.data_ptr(), ws.data_ptr(), ws.numel(), _stream()), "argmax_rows")
    return out[:rows]


# ---------------------------------------------------------------- K1

def _cache_args(k_cache: torch.Tensor, v_cache: torch.Tensor):
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("caches must be [num_blocks, block_size, num_kv_heads, head_dim] "
                         "with identical strides")
    if k_cache.stride(-1) != 1:
        raise ValueError("cache head_dim must be contiguous")
    if k_cache.dtype != v_cache.dtype:
        raise TypeError("k_cache and v_cache must share a dtype")
    nb, bs, hkv, d = k_cache.shape
    return (_kv_dtype(k_cache), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), nb, bs,
            hkv, d)


def _device_lengths(t, device: torch.device, name: str):
    """(device int32 tensor, host lengths or None) for a cu_seqlens / seqlens
    argument.  A device tensor passes through (its values are not read: that
    would need a synchronisation); a CPU tensor or a list is host-known, so
    its values are returned for the bound checks and it is copied to the
    device (not allowed under graph capture)."""
    if isinstance(t, torch.Tensor) and t.is_cuda:
        if t.device != device:
            raise ValueError("all tensors must be on the same device")
        return t, None
    host = torch.as_tensor(t, dtype=torch.int32)
    if host.dim() != 1:
        raise ValueError(f"{name} must be one-dimensional")
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"{name} on the host cannot be uploaded under graph capture")
    return host.contiguous().to(device), host.tolist()


def _check_bound(bound: int, lengths, what: str, name: str) -> None:
    longest = max(lengths, default=0)
    if longest > bound:
        raise ValueError(f"{name}={bound} is below the longest {what} ({longest}); the kernel "
                         f"would clip it")


def _q_out(q: torch.Tensor, out: torch.Tensor | None):
    if q.dtype != BF16 or q.dim() != 3 or q.stride(-1) != 1:
        raise ValueError("q must be bf16 [tokens, num_heads, head_dim] with unit last stride")
    if out is None:
        out = torch.empty(q.shape, dtype=BF16, device=q.device)
    if out.shape != q.shape or out.dtype != BF16 or out.stride(-1) != 1:
        raise ValueError("out must match q")
    return out


def paged_attention_varlen(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                           max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float,
                           block_table: torch.Tensor, causal: bool = True,
                           k_scale: torch.Tensor | None = None,
                           v_scale: torch.Tensor | None = None,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """Paged varlen causal attention (the EAGLE3 verify attention).

    Mirrors the reference call flash_attn_varlen_func(q, k_cache, v_cache,
    max_seqlen_q, cu_seqlens_q, max_seqlen_k, cu_seqlens_k, softmax_scale,
    causal=True, block_table) of layers/attention.py:385-395: bottom-right
    aligned causal mask, GQA by head groups, keys read through block_table.

    ``max_seqlen_q`` / ``max_seqlen_k`` size the launch; the kernel clips a
    longer sequence to them (rows past max_seqlen_q come back as zeros, keys
    past max_seqlen_k are not seen).  When cu_seqlens_q / cu_seqlens_k are
    given on the host (CPU tensors or lists) their lengths are known here and
    a bound below them raises ValueError; device tensors are not read."""
    if not causal:
        raise ValueError("only causal paged attention is supported")
    lib = _native.load()
    _require_cuda(q, k_cache, v_cache, block_table, out)
    cu_seqlens_q, host_q = _device_lengths(cu_seqlens_q, q.device, "cu_seqlens_q")
    cu_seqlens_k, host_k = _device_lengths(cu_seqlens_k, q.device, "cu_seqlens_k")
    if host_q is not None:
        _check_bound(int(max_seqlen_q), [b - a for a, b in zip(host_q, host_q[1:])],
                     "query length", "max_seqlen_q")
    if host_k is not None:
        _check_bound(int(max_seqlen_k), [b - a for a, b in zip(host_k, host_k[1:])],
                     "key length", "max_seqlen_k")
    kvd, bstr, tstr, hstr, nb, bs, hkv, d = _cache_args(k_cache, v_cache)
    t, hq, dq = q.shape
    if dq != d:
        raise ValueError("q head_dim must match the cache")
    if hq % hkv != 0:
        raise ValueError("num query heads must divide evenly by KV heads")
    _i32(cu_seqlens_q, "cu_seqlens_q")
    _i32(cu_seqlens_k, "cu_seqlens_k")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise TypeError("block_table must be int32 [num_seqs, max_blocks]")
    b = cu_seqlens_q.numel() - 1
    if cu_seqlens_k.numel() != b + 1 or block_table.shape[0] < b:
        raise ValueError("cu_seqlens_k / block_table do not match cu_seqlens_q")
    out = _q_out(q, out)
    nbytes = attention_workspace_bytes(b, t, hq, hkv, d, max_seqlen_q, max_seqlen_k)
    ws = _WS.get(q.device, "attention", nbytes) if nbytes else None
    check(lib.nva_paged_attention_varlen(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), kvd, bstr,
        tstr, hstr, nb, bs, cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], b, t,
        int(max_seqlen_q), int(max_seqlen_k),
        hq, hkv, d, float(softmax_scale), _ptr(_scale(k_scale)), _ptr(_scale(v_scale)),
        out.data_ptr(), out.stride(0), out.stride(1), _ptr(ws), 0 if ws is None else ws.numel(),
        _stream()), "paged_attention_varlen")
    return out


def paged_attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           cache_seqlens: torch.Tensor, block_table: torch.Tensor,
                           softmax_scale: float, max_seqlen_k: int | None = None,
                           k_scale: torch.Tensor | None = None,
                           v_scale: torch.Tensor | None = None,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """One query row per sequence over its paged cache.

    Mirrors flash_attn_with_kvcache(q[:, None], k_cache, v_cache,
    cache_seqlens, block_table, softmax_scale, causal=True) of
    layers/attention.py:396-399.  q: [B, Hq, D].  ``max_seqlen_k`` bounds the
    lengths (default: every cache slot of one table row); the kernel clips a
    longer length to it.  When ``cache_seqlens`` is given on the host (a CPU
    tensor or a list) a bound below its largest value raises ValueError."""
    lib = _native.load()
    _require_cuda(q, k_cache, v_cache, block_table, out)
    cache_seqlens, host_lens = _device_lengths(cache_seqlens, q.device, "cache_seqlens")
    kvd, bstr, tstr, hstr, nb, bs, hkv, d = _cache_args(k_cache, v_cache)
    b, hq, dq = q.shape
    if dq != d:
        raise ValueError("q head_dim must match the cache")
    if hq % hkv != 0:
        raise ValueError("num query heads must divide evenly by KV heads")
    _i32(cache_seqlens, "cache_seqlens")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise TypeError("block_table must be int32 [num_seqs, max_blocks]")
    if cache_seqlens.numel() != b or block_table.shape[0] < b:
        raise ValueError("cache_seqlens / block_table must have one row per query")
    if max_seqlen_k is None:
        max_seqlen_k = block_table.shape[1] * bs
    if host_lens is not None:
        _check_bound(int(max_seqlen_k), host_lens, "context length", "max_seqlen_k")
    out = _q_out(q, out)
    nbytes = attention_workspace_bytes(b, b, hq, hkv, d, 1, max_seqlen_k)
    ws = _WS.get(q.device, "attention", nbytes) if nbytes else None
    check(lib.nva_paged_attention_decode(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), kvd, bstr,
        tstr, hstr, nb, bs, cache_seqlens.data_ptr(), block_table.data_ptr(),
        block_table.stride(0), block_table.shape[1], b, int(max_seqlen_k), hq, hkv, d, float(softmax_scale),
        _ptr(_scale(k_scale)), _ptr(_scale(v_scale)), out.data_ptr(), out.stride(0),
        out.stride(1), _ptr(ws), 0 if ws is None else ws.numel(), _stream()),
        "paged_attention_decode")
    return out


def fp8_paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                               context_lens: torch.Tensor, block_tables: torch.Tensor,
                               scale: float, k_scale: torch.Tensor,
                               v_scale: torch.Tensor) -> torch.Tensor:
    """Same interface and errors as the reference's fp8_paged_decode_attention
    (layers/attention.py:249-293): one row per token, FP8 caches, head_dim 128."""
    num_tokens, num_heads, head_dim = q.shape
    if head_dim != 128:
        raise ValueError("the teaching FP8 paged kernel currently requires head_dim=128")
    if num_heads % k_cache.size(2) != 0:
        raise ValueError("num query heads must divide evenly by KV heads")
    return paged_attention_decode(q, k_cache, v_cache, context_lens, block_tables, scale,
                                  k_scale=k_scale, v_scale=v_scale)


# ---------------------------------------------------------------- forward helpers

def _rows2d(x: torch.Tensor, name: str) -> None:
    if x.dtype != BF16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"{name} must be bf16 [rows, hidden] with unit last stride")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm without residual (layers/layernorm.py:70-89)."""
    lib = _native.load()
    _require_cuda(x, weight, out)
    _rows2d(x, "x")
    rows, h = x.shape
    if weight.numel() != h:
        raise ValueError("weight must have one element per hidden column")
    if out is None:
        out = torch.empty(rows, h, dtype=BF16, device=x.device)
    elif out.dtype != BF16 or out.dim() != 2 or tuple(out.shape) != (rows, h) or out.stride(1) != 1:
        raise ValueError("out must be bf16 [rows, hidden] with unit last stride")
    check(lib.nva_rms_norm(x.data_ptr(), x.stride(0), weight.data_ptr(), out.data_ptr(),
                           out.stride(0), rows, h, float(eps), _stream()), "rms_norm")
    return out


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """RMSNorm with residual add (layers/layernorm.py:91-107).

    Returns (normed, new_residual); both are new tensors."""
    lib = _native.load()
    _require_cuda(x, residual, weight)
    _rows2d(x, "x")
    _rows2d(residual, "residual")
    if residual.shape != x.shape or weight.numel() != x.shape[1]:
        raise ValueError("residual must match x and weight its hidden size")
    rows, h = x.shape
    out = torch.empty(rows, h, dtype=BF16, device=x.device)
    res_out = torch.empty(rows, h, dtype=BF16, device=x.device)
    check(lib.nva_add_rms_norm(x.data_ptr(), x.stride(0), residual.data_ptr(), residual.stride(0),
                               weight.data_ptr(), out.data_ptr(), out.stride(0), res_out.data_ptr(),
                               res_out.stride(0), rows, h, float(eps), _stream()), "add_rms_norm")
    return out, res_out


def _qkv_rows(qkv: torch.Tensor, positions: torch.Tensor, hq: int, hkv: int, d: int) -> None:
    if positions.numel() != qkv.shape[0]:
        raise ValueError("positions must have one entry per qkv row")
    if qkv.shape[1] < (hq + 2 * hkv) * d:
        raise ValueError("qkv rows must hold [q heads | k heads | v heads]")


def add_then_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """``h = x + residual`` in bf16, then RMSNorm(h) without residual, as the
    EAGLE3 draft layer composes them (eagle3.py:141-146).  Returns
    (normed, h); both are new tensors."""
    lib = _native.load()
    _require_cuda(x, residual, weight)
    _rows2d(x, "x")
    _rows2d(residual, "residual")
    if residual.shape != x.shape or weight.numel() != x.shape[1]:
        raise ValueError("residual must match x and weight its hidden size")
    rows, h = x.shape
    out = torch.empty(rows, h, dtype=BF16, device=x.device)
    total = torch.empty(rows, h, dtype=BF16, device=x.device)
    check(lib.nva_add_then_rms_norm(x.data_ptr(), x.stride(0), residual.data_ptr(),
                                    residual.stride(0), weight.data_ptr(), out.data_ptr(),
                                    out.stride(0), total.data_ptr(), total.stride(0), rows, h,
                                    float(eps), _stream()), "add_then_rms_norm")
    return out, total


def qk_norm_rope(qkv: torch.Tensor, positions: torch.Tensor, q_norm_weight: torch.Tensor | None,
                 k_norm_weight: torch.Tensor | None, cos_sin: torch.Tensor, num_q_heads: int,
                 num_kv_heads: int, head_dim: int, eps: float):
    """Per-head q/k RMSNorm + neox RoPE on a fused QKV output
    (models/qwen3.py:77-98).  Returns contiguous q [T, Hq, D], k [T, Hkv, D]."""
    lib = _native.load()
    _require_cuda(qkv, positions, q_norm_weight, k_norm_weight, cos_sin)
    _rows2d(qkv, "qkv")
    if positions.dtype != torch.int64 or not positions.is_contiguous():
        raise TypeError("positions must be contiguous int64")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous():
        raise TypeError("cos_sin must be contiguous float32 [max_position, head_dim]")
    t = qkv.shape[0]
    _qkv_rows(qkv, positions, num_q_heads, num_kv_heads, head_dim)
    q = torch.empty(t, num_q_heads, head_dim, dtype=BF16, device=qkv.device)
    k = torch.empty(t, num_kv_heads, head_dim, dtype=BF16, device=qkv.device)
    check(lib.nva_qk_norm_rope(qkv.data_ptr(), qkv.stride(0), positions.data_ptr(),
                               _ptr(q_norm_weight), _ptr(k_norm_weight), cos_sin.data_ptr(),
                               cos_sin.shape[0], t, num_q_heads, num_kv_heads, head_dim,
                               float(eps), q.data_ptr(), k.data_ptr(), _stream()), "qk_norm_rope")
    return q, k


def qk_norm_rope_store(qkv: torch.Tensor, positions: torch.Tensor,
                       q_norm_weight: torch.Tensor | None, k_norm_weight: torch.Tensor | None,
                       cos_sin: torch.Tensor, num_q_heads: int, num_kv_heads: int, head_dim: int,
                       eps: float, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       slot_mapping: torch.Tensor, k_scale: torch.Tensor | None = None,
                       v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """qk_norm_rope, then store_kvcache of the rotated keys and the value
    heads of ``qkv`` (models/qwen3.py:77-98; attention.py:189-217), in one
    launch.  Returns q [T, Hq, D]; the cache contents are exactly those the
    two separate calls leave."""
    lib = _native.load()
    _require_cuda(qkv, positions, q_norm_weight, k_norm_weight, cos_sin, k_cache, v_cache,
                  slot_mapping)
    _rows2d(qkv, "qkv")
    if positions.dtype != torch.int64 or not positions.is_contiguous():
        raise TypeError("positions must be contiguous int64")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous():
        raise TypeError("cos_sin must be contiguous float32 [max_position, head_dim]")
    kvd, bstr, tstr, hstr, nb, bs, c_hkv, c_d = _cache_args(k_cache, v_cache)
    if (c_hkv, c_d) != (num_kv_heads, head_dim):
        raise ValueError("cache heads / head_dim do not match the projection")
    t = qkv.shape[0]
    _qkv_rows(qkv, positions, num_q_heads, num_kv_heads, head_dim)
    if slot_mapping.numel() != t:
        raise ValueError("slot_mapping must have one entry per token")
    _i32(slot_mapping, "slot_mapping")
    q = torch.empty(t, num_q_heads, head_dim, dtype=BF16, device=qkv.device)
    check(lib.nva_qk_norm_rope_store(
        qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), _ptr(q_norm_weight),
        _ptr(k_norm_weight), cos_sin.data_ptr(), cos_sin.shape[0], t, num_q_heads, num_kv_heads,
        head_dim, float(eps), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), kvd, bstr,
        tstr, hstr, nb, bs, slot_mapping.data_ptr(), _ptr(_scale(k_scale)),
        _ptr(_scale(v_scale)), _stream()), "qk_norm_rope_store")
    return q


def silu_mul(x: torch.Tensor) -> torch.Tensor:
    """SiluAndMul (layers/activation.py:11-14) on rows [a | b]."""
    lib = _native.load()
    _require_cuda(x)
    _rows2d(x, "x")
    rows, two_i = x.shape
    inter = two_i // 2
    out = torch.empty(rows, inter, dtype=BF16, device=x.device)
    check(lib.nva_silu_mul(x.data_ptr(), x.stride(0), out.data_ptr(), out.stride(0), rows, inter,
                           _stream()), "silu_mul")
    return out


# ---------------------------------------------------------------- verify metadata

def _block_table_args(block_tables: torch.Tensor, num_seqs: int):
    """(pointer, row stride, width) of an int32 [num_seqs, max_blocks] block
    table; with no sequence nothing is read, so no table is needed."""
    if num_seqs == 0:
        return None, 0, 0
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.stride(1) != 1 \
            or block_tables.shape[0] < num_seqs:
        raise TypeError("block_tables must be int32 [num_seqs, max_blocks]")
    return block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1]


def verify_metadata(start_pos: torch.Tensor, q_lens: torch.Tensor, block_tables: torch.Tensor,
                    block_size: int, num_tokens: int, cu_seqlens_q: torch.Tensor,
                    cu_seqlens_k: torch.Tensor, positions: torch.Tensor,
                    slot_mapping: torch.Tensor) -> None:
    """Device-side prepare_prefill for verify rows (model_runner.py:761-800):
    from per-sequence first positions and query lengths plus the block
    tables, write cu_seqlens_q/k [B+1], positions [T] (int64) and
    slot_mapping [T] (int32).  Rows past the last sequence get position 0
    and slot -1."""
    lib = _native.load()
    _require_cuda(start_pos, q_lens, block_tables, cu_seqlens_q, cu_seqlens_k, positions,
                  slot_mapping)
    b = start_pos.numel()
    for t, name in ((start_pos, "start_pos"), (q_lens, "q_lens"), (cu_seqlens_q, "cu_seqlens_q"),
                    (cu_seqlens_k, "cu_seqlens_k"), (slot_mapping, "slot_mapping")):
        _i32(t, name)
    if q_lens.numel() != b or cu_seqlens_q.numel() < b + 1 or cu_seqlens_k.numel() < b + 1:
        raise ValueError("start_pos / q_lens / cu_seqlens sizes do not match")
    if positions.dtype != torch.int64 or positions.numel() < num_tokens or \
            slot_mapping.numel() < num_tokens:
        raise ValueError("positions (int64) and slot_mapping need num_tokens entries")
    bt_ptr, bt_stride, bt_width = _block_table_args(block_tables, b)
    check(lib.nva_verify_metadata(start_pos.data_ptr(), q_lens.data_ptr(), b,
                                  bt_ptr, bt_stride, bt_width, int(block_size),
                                  cu_seqlens_q.data_ptr(),
                                  cu_seqlens_k.data_ptr(), positions.data_ptr(),
                                  slot_mapping.data_ptr(), int(num_tokens), _stream()),
          "verify_metadata")


def draft_metadata(lens: torch.Tensor, verify_row: torch.Tensor, accept_len: torch.Tensor,
                   num_seqs: int, block_tables: torch.Tensor, block_size: int,
                   positions: torch.Tensor, slot_mapping: torch.Tensor,
                   context_lens: torch.Tensor, slot_offset: int = 0) -> None:
    """Draft-step metadata after a verify, on the device (the host loop of
    model_runner.py:1087-1096, :1159-1213): column i < num_seqs of the
    [steps, bs] outputs is a sequence of length lens[i] +
    accept_len[verify_row[i]] + 1 after the verified step, its step s at
    RoPE position p = len - 1 + s, its K/V at the slot of position
    p + slot_offset (through block_tables row i) and its context
    p + slot_offset + 1; padding columns get position 0, slot -1, context 1.
    slot_offset 1 is the reference's decode convention (slot len + step,
    context len + step + 1), 0 this engine's (slot p, context p + 1).  lens
    and verify_row are int64 [bs], accept_len int32 (the accept scan's
    output)."""
    lib = _native.load()
    _require_cuda(lens, verify_row, accept_len, block_tables, positions, slot_mapping,
                  context_lens)
    if positions.dim() != 2 or positions.dtype != torch.int64 or not positions.is_contiguous():
        raise ValueError("positions must be contiguous int64 [steps, bs]")
    steps, bs = positions.shape
    for t, name in ((slot_mapping, "slot_mapping"), (context_lens, "context_lens")):
        _i32(t, name)
        if t.shape != positions.shape or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous int32 [steps, bs]")
    _i32(accept_len, "accept_len")
    if lens.dtype != torch.int64 or verify_row.dtype != torch.int64 or \
            lens.numel() < num_seqs or verify_row.numel() < num_seqs:
        raise ValueError("lens and verify_row must be int64 with an entry per sequence")
    if not 0 <= num_seqs <= bs:
        raise ValueError("num_seqs must be within the bs columns")
    bt_ptr, bt_stride, bt_width = _block_table_args(block_tables, num_seqs)
    check(lib.nva_draft_metadata(lens.data_ptr(), verify_row.data_ptr(), accept_len.data_ptr(),
                                 int(num_seqs), bs, steps, bt_ptr, bt_stride, bt_width,
                                 int(block_size), int(slot_offset), positions.data_ptr(),
                                 slot_mapping.data_ptr(), context_lens.data_ptr(), _stream()),
          "draft_metadata")



def verify_input_ids(compose: torch.Tensor, last_tokens: torch.Tensor, order: torch.Tensor,
                     proposals: torch.Tensor, q: int, ids: torch.Tensor) -> None:
    """The verify batch's input ids on the device (each sequence's last
    token, then its proposals: llm_engine.py:129-141 with
    model_runner.py:770-774): row p of q ids is last_tokens[p] followed by
    proposals[:, order[p]] (proposals [q-1, stride] int64, the draft's
    output); rows whose order[p] is outside [0, stride) are padding (ids 0).
    compose, last_tokens and order are int32 device tensors; when
    compose[0] == 0 the kernel leaves ids untouched."""
    lib = _native.load()
    _require_cuda(compose, last_tokens, order, proposals, ids)
    for t, name in ((compose, "compose"), (last_tokens, "last_tokens"), (order, "order")):
        _i32(t, name)
    num_rows = order.numel()
    if last_tokens.numel() != num_rows or compose.numel() < 1:
        raise ValueError("last_tokens needs an entry per row and compose one flag")
    if proposals.dim() != 2 or proposals.dtype != torch.int64 or not proposals.is_contiguous() \
            or proposals.shape[0] < q - 1 or proposals.shape[1] < 1:
        raise ValueError("proposals must be contiguous int64 [q-1, stride]")
    if ids.dtype != torch.int64 or not ids.is_contiguous() or ids.numel() < num_rows * q:
        raise ValueError("ids must be contiguous int64 with num_rows * q entries")
    check(lib.nva_verify_input_ids(compose.data_ptr(), last_tokens.data_ptr(), order.data_ptr(),
                                   proposals.data_ptr(), proposals.shape[1], num_rows, int(q),
                                   ids.data_ptr(), _stream()), "verify_input_ids")

def commit_metadata(start_pos: torch.Tensor, accept_len: torch.Tensor, q_stride: int,
                    verify_argmax: torch.Tensor, block_tables: torch.Tensor, block_size: int,
                    num_tokens: int, cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                    positions: torch.Tensor, slot_mapping: torch.Tensor,
                    verify_rows: torch.Tensor, token_ids: torch.Tensor,
                    last_rows: torch.Tensor, slot_offset: int = 0) -> None:
    """Device-side metadata of the draft's replay of the committed tails
    (commit_eagle3, model_runner.py:1216-1249): sequence i commits
    accept_len[i] + 1 rows (at most q_stride) starting at position
    start_pos[i], taken from its verify rows i * q_stride ..  Writes
    verify_metadata's outputs for those lengths, plus per commit row its
    verify row (int32, -1 past the committed rows) and its token (the verify
    argmax of that row, int64), and per sequence its last commit row
    (int64).  slot_offset shifts every row's slot and the sequence's key
    count by that many positions: 1 is the reference's commit convention
    (token i at slot start + 1 + i, context start + 2 + i,
    model_runner.py:1143-1149), 0 this engine's (position p at slot p)."""
    lib = _native.load()
    _require_cuda(start_pos, accept_len, verify_argmax, block_tables, cu_seqlens_q, cu_seqlens_k,
                  positions, slot_mapping, verify_rows, token_ids, last_rows)
    b = start_pos.numel()
    for t, name in ((start_pos, "start_pos"), (accept_len, "accept_len"),
                    (verify_argmax, "verify_argmax"), (cu_seqlens_q, "cu_seqlens_q"),
                    (cu_seqlens_k, "cu_seqlens_k"), (slot_mapping, "slot_mapping"),
                    (verify_rows, "verify_rows")):
        _i32(t, name)
    if accept_len.numel() != b or cu_seqlens_q.numel() < b + 1 or cu_seqlens_k.numel() < b + 1 \
            or last_rows.numel() < b:
        raise ValueError("start_pos / accept_len / cu_seqlens / last_rows sizes do not match")
    for t, name in ((positions, "positions"), (token_ids, "token_ids"), (last_rows, "last_rows")):
        if t.dtype != torch.int64 or not t.is_contiguous():
            raise TypeError(f"{name} must be contiguous int64")
    if positions.numel() < num_tokens or slot_mapping.numel() < num_tokens or \
            verify_rows.numel() < num_tokens or token_ids.numel() < num_tokens:
        raise ValueError("positions / slot_mapping / verify_rows / token_ids need num_tokens "
                         "entries")
    bt_ptr, bt_stride, bt_width = _block_table_args(block_tables, b)
    check(lib.nva_commit_metadata(start_pos.data_ptr(), accept_len.data_ptr(), b, int(q_stride),
                                  verify_argmax.data_ptr(), verify_argmax.numel(),
                                  bt_ptr, bt_stride, bt_width, int(block_size),
                                  int(slot_offset), cu_seqlens_q.data_ptr(),
                                  cu_seqlens_k.data_ptr(), positions.data_ptr(),
                                  slot_mapping.data_ptr(), verify_rows.data_ptr(),
                                  token_ids.data_ptr(), last_rows.data_ptr(), int(num_tokens),
                                  _stream()),
          "commit_metadata")
