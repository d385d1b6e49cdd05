"""Building blocks of the target and draft forwards.

Projection GEMMs stay on torch (hipBLASLt); norms, RoPE, SiLU-and-mul, the
KV write and the paged attention run in the HIP library.  Module and
parameter names follow the reference (nanovllm/layers/*.py) so checkpoints
load unchanged.
"""
from __future__ import annotations

from functools import lru_cache

import torch
import torch.nn.functional as F
from torch import nn

from nanovllm_amd import kernels as K
from nanovllm_amd.context import get_context


class Linear(nn.Module):
    """y = x W^T (+ b).  ``shards`` maps a checkpoint shard id to its
    (row offset, rows) inside a fused weight (QKV / gate_up packing,
    nanovllm/layers/linear.py:85-170 at TP=1)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 shards: dict | None = None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.shards = shards or {}
        self.weight = nn.Parameter(torch.empty(out_features, in_features), requires_grad=False)
        self.weight.weight_loader = self._load
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features), requires_grad=False)
            self.bias.weight_loader = self._load
        else:
            self.register_parameter("bias", None)

    def _load(self, param: nn.Parameter, loaded: torch.Tensor, shard_id=None) -> None:
        if shard_id is None:
            if param.shape != loaded.shape:
                raise ValueError(f"weight shape {tuple(loaded.shape)} != {tuple(param.shape)}")
            param.data.copy_(loaded)
            return
        offset, rows = self.shards[shard_id]
        if loaded.shape[0] != rows:
            raise ValueError(f"shard {shard_id!r} has {loaded.shape[0]} rows, expected {rows}")
        param.data[offset:offset + rows].copy_(loaded)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, self.weight, self.bias)


class Embedding(nn.Module):
    """Token embedding (VocabParallelEmbedding at TP=1, embed_head.py:15-48)."""

    def __init__(self, num_embeddings: int, embedding_dim: int):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(num_embeddings, embedding_dim), requires_grad=False)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return F.embedding(ids, self.weight)


class RMSNorm(nn.Module):
    """RMSNorm with optional fused residual add (layers/layernorm.py:39-119)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size), requires_grad=False)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return K.rms_norm(x, self.weight, self.eps)
        return K.add_rms_norm(x, residual, self.weight, self.eps)


@lru_cache(maxsize=8)
def rope_cos_sin(head_dim: int, max_position: int, base: float, device_index: int) -> torch.Tensor:
    """float32 [max_position, head_dim] table: cos | sin of position * inv_freq
    (rotary_embedding.py:28-35), built on the host in float32."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device="cpu")
                               / head_dim))
    t = torch.arange(max_position, dtype=torch.float32, device="cpu")
    freqs = torch.outer(t, inv_freq)
    table = torch.cat((freqs.cos(), freqs.sin()), dim=-1).contiguous()
    return table.to(torch.device("cuda", device_index))


class Attention(nn.Module):
    """Paged attention over this layer's slice of the KV cache.

    forward(q, k, v): writes k/v at ``context.slot_mapping`` (K2) and attends
    with the varlen entry (prefill / verify: several rows per sequence) or the
    decode entry (one row per sequence), as layers/attention.py:317-400.
    Per-layer fp32 k_scale / v_scale (1.0) apply to FP8 caches only."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.register_buffer("k_scale", torch.tensor([1.0], dtype=torch.float32))
        self.register_buffer("v_scale", torch.tensor([1.0], dtype=torch.float32))

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        ctx = get_context()
        if ctx.is_dummy:
            return torch.zeros_like(q)
        self._check_bound(ctx)
        K.store_kvcache(k, v, self.k_cache, self.v_cache, ctx.slot_mapping, self.k_scale,
                        self.v_scale)
        return self.attend(q)

    def _check_bound(self, ctx) -> None:
        if not self.k_cache.numel():
            raise RuntimeError("attention needs a bound paged KV cache")
        if ctx.slot_mapping is None or ctx.block_tables is None:
            raise RuntimeError("paged KV attention requires slot mapping and block tables")

    def attend(self, q: torch.Tensor) -> torch.Tensor:
        """The attention half of forward(): this step's K/V rows are already
        in the cache (written by forward's store or by the fused
        qk_norm_rope_store)."""
        ctx = get_context()
        if ctx.is_prefill:
            return K.paged_attention_varlen(q, self.k_cache, self.v_cache, ctx.cu_seqlens_q,
                                            ctx.cu_seqlens_k, ctx.max_seqlen_q, ctx.max_seqlen_k,
                                            self.scale, ctx.block_tables, k_scale=self.k_scale,
                                            v_scale=self.v_scale)
        return K.paged_attention_decode(q, self.k_cache, self.v_cache, ctx.context_lens,
                                        ctx.block_tables, self.scale,
                                        max_seqlen_k=ctx.max_seqlen_k or None,
                                        k_scale=self.k_scale, v_scale=self.v_scale)


class SelfAttention(nn.Module):
    """Qwen3-style attention block: fused QKV projection, per-head q/k RMSNorm
    (optional), neox RoPE, paged attention, output projection
    (models/qwen3.py:16-112)."""

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int,
                 max_position: int, rms_norm_eps: float, qkv_bias: bool, rope_theta: float,
                 qkv_input_size: int | None = None, use_qk_norm: bool | None = None):
        super().__init__()
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.q_size = num_heads * head_dim
        self.kv_size = num_kv_heads * head_dim
        self.eps = rms_norm_eps
        self.max_position = max_position
        self.rope_theta = rope_theta
        self.use_qk_norm = (not qkv_bias) if use_qk_norm is None else use_qk_norm
        self.qkv_proj = Linear(qkv_input_size or hidden_size, self.q_size + 2 * self.kv_size,
                               bias=qkv_bias,
                               shards={"q": (0, self.q_size), "k": (self.q_size, self.kv_size),
                                       "v": (self.q_size + self.kv_size, self.kv_size)})
        self.o_proj = Linear(self.q_size, hidden_size)
        self.attn = Attention(num_heads, head_dim, head_dim ** -0.5, num_kv_heads)
        if self.use_qk_norm:
            self.q_norm = RMSNorm(head_dim, rms_norm_eps)
            self.k_norm = RMSNorm(head_dim, rms_norm_eps)

    def forward(self, positions: torch.Tensor, hidden_states: torch.Tensor) -> torch.Tensor:
        qkv = self.qkv_proj(hidden_states)
        cos_sin = rope_cos_sin(self.head_dim, self.max_position, float(self.rope_theta),
                               qkv.device.index)
        ctx = get_context()
        attn = self.attn
        if not ctx.is_dummy:
            # norm + RoPE + this step's K/V write in one launch, then attention
            attn._check_bound(ctx)
            q = K.qk_norm_rope_store(qkv, positions,
                                     self.q_norm.weight if self.use_qk_norm else None,
                                     self.k_norm.weight if self.use_qk_norm else None,
                                     cos_sin, self.num_heads, self.num_kv_heads, self.head_dim,
                                     self.eps, attn.k_cache, attn.v_cache, ctx.slot_mapping,
                                     attn.k_scale, attn.v_scale)
            return self.o_proj(attn.attend(q).view(-1, self.q_size))
        q, k = K.qk_norm_rope(qkv, positions,
                              self.q_norm.weight if self.use_qk_norm else None,
                              self.k_norm.weight if self.use_qk_norm else None,
                              cos_sin, self.num_heads, self.num_kv_heads, self.head_dim, self.eps)
        v = qkv[:, self.q_size + self.kv_size:].view(-1, self.num_kv_heads, self.head_dim)
        o = self.attn(q, k, v)
        return self.o_proj(o.view(-1, self.q_size))


class MLP(nn.Module):
    """gate_up projection, SiLU-and-mul, down projection (qwen3.py:115-140)."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_up_proj = Linear(hidden_size, 2 * intermediate_size,
                                   shards={0: (0, intermediate_size),
                                           1: (intermediate_size, intermediate_size)})
        self.down_proj = Linear(intermediate_size, hidden_size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(K.silu_mul(self.gate_up_proj(x)))


def init_random_(module: nn.Module, seed: int, std: float = 0.02) -> None:
    """Random weights for checkpoint-free runs: N(0, std) for projection and
    embedding weights, zero biases, ones for RMSNorm weights (seeded,
    generated on the device in module order)."""
    device = next(module.parameters()).device
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for m in module.modules():
        if isinstance(m, RMSNorm):
            m.weight.data.fill_(1.0)
        elif isinstance(m, (Linear, Embedding)):
            m.weight.data.normal_(0.0, std, generator=gen)
            if getattr(m, "bias", None) is not None:
                m.bias.data.zero_()


def param_bytes(module: nn.Module) -> int:
    return sum(p.numel() * p.element_size() for p in module.parameters())


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)

