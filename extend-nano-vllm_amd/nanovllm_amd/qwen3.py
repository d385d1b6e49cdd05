"""Qwen3 dense target model with EAGLE3 auxiliary hidden states
(nanovllm/models/qwen3.py:16-416, PP=TP=1).

``forward_with_aux_hidden_states`` returns the final hidden states and, for
each requested (1-indexed) aux layer, the pair (hidden, residual) left by
that layer; the EAGLE3 aux state is bf16(hidden + residual) and is formed by
the aux-gather kernel only for the rows that need it.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from nanovllm_amd import kernels as K
from nanovllm_amd.layers import MLP, Embedding, Linear, RMSNorm, SelfAttention


class Qwen3DecoderLayer(nn.Module):

    def __init__(self, config):
        super().__init__()
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        self.self_attn = SelfAttention(
            hidden_size=config.hidden_size,
            num_heads=config.num_attention_heads,
            num_kv_heads=config.num_key_value_heads,
            head_dim=head_dim,
            max_position=config.max_position_embeddings,
            rms_norm_eps=config.rms_norm_eps,
            qkv_bias=getattr(config, "attention_bias", True),
            rope_theta=getattr(config, "rope_theta", 1000000),
        )
        self.mlp = MLP(config.hidden_size, config.intermediate_size)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, positions, hidden_states, residual):
        if residual is None:
            residual = hidden_states
            hidden_states = self.input_layernorm(hidden_states)
        else:
            hidden_states, residual = self.input_layernorm(hidden_states, residual)
        hidden_states = self.self_attn(positions, hidden_states)
        hidden_states, residual = self.post_attention_layernorm(hidden_states, residual)
        return self.mlp(hidden_states), residual


class Qwen3Model(nn.Module):

    def __init__(self, config):
        super().__init__()
        self.embed_tokens = Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(Qwen3DecoderLayer(config) for _ in range(config.num_hidden_layers))
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, input_ids, positions):
        hidden, _ = self.forward_with_aux_hidden_states(input_ids, positions, ())
        return hidden

    def forward_with_aux_hidden_states(self, input_ids, positions, aux_hidden_state_layers):
        hidden = self.embed_tokens(input_ids)
        residual = None
        aux = []
        for layer_id, layer in enumerate(self.layers, start=1):
            hidden, residual = layer(positions, hidden, residual)
            if layer_id in aux_hidden_state_layers:
                aux.append((hidden, residual))
        if len(aux) != len(aux_hidden_state_layers):
            raise ValueError("requested EAGLE3 auxiliary layer is unavailable")
        hidden, _ = self.norm(hidden, residual)
        return hidden, aux


class Qwen3ForCausalLM(nn.Module):
    packed_modules_mapping = {
        "q_proj": ("qkv_proj", "q"),
        "k_proj": ("qkv_proj", "k"),
        "v_proj": ("qkv_proj", "v"),
        "gate_proj": ("gate_up_proj", 0),
        "up_proj": ("gate_up_proj", 1),
    }

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.model = Qwen3Model(config)
        self.tie_word_embeddings = bool(getattr(config, "tie_word_embeddings", False))
        self.lm_head = Linear(config.hidden_size, config.vocab_size)
        if self.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids, positions):
        return self.model(input_ids, positions)

    def forward_with_aux_hidden_states(self, input_ids, positions, aux_hidden_state_layers):
        return self.model.forward_with_aux_hidden_states(input_ids, positions,
                                                         tuple(aux_hidden_state_layers))

    def compute_logits(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden_states, self.lm_head.weight)

    def compute_all_logits(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """One logit row per token (the EAGLE3 verify needs every row;
        models/qwen3.py:407-416)."""
        return F.linear(hidden_states, self.lm_head.weight)


def aux_concat(aux: list[tuple[torch.Tensor, torch.Tensor]],
               rows: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(hidden + residual) of each aux layer, concatenated on the last dim,
    for ``rows`` (int32, device) or all rows -- the aux-gather kernel."""
    hidden = [h for h, _ in aux]
    residual = [r for _, r in aux]
    if rows is None:
        rows = torch.arange(hidden[0].shape[0], dtype=torch.int32, device=hidden[0].device)
    return K.aux_gather(hidden, residual, rows)
