"""EAGLE3 draft model (speculators checkpoint format)
(nanovllm/models/eagle3.py:16-308).

One Llama-style decoder layer whose attention reads the concatenation of the
normalised token embedding and the (normalised) recurrent hidden state
(2H -> attention), an ``fc`` that fuses three target aux hidden states
(3H -> H), and a draft LM head whose argmax is mapped to target ids with
``d2t``.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn

from nanovllm_amd import kernels as K
from nanovllm_amd.layers import MLP, Embedding, Linear, RMSNorm, SelfAttention, init_random_
from nanovllm_amd.loader import load_model


@dataclass(frozen=True)
class Eagle3Config:
    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    max_position_embeddings: int
    rms_norm_eps: float
    rope_theta: float
    attention_bias: bool
    target_vocab_size: int
    draft_vocab_size: int
    target_hidden_size: int
    num_aux_hidden_states: int
    norm_before_residual: bool
    torch_dtype: torch.dtype

    @classmethod
    def from_pretrained(cls, model_path) -> "Eagle3Config":
        raw = json.loads((Path(model_path) / "config.json").read_text())
        if raw.get("speculators_model_type") != "eagle3":
            raise ValueError("expected a speculators-format EAGLE3 checkpoint")
        layer = raw.get("transformer_layer_config")
        if not isinstance(layer, dict):
            raise ValueError("EAGLE3 config must contain transformer_layer_config")
        if layer.get("model_type") != "llama":
            raise ValueError("only Llama-style EAGLE3 transformer layers are supported")
        hidden = layer["hidden_size"]
        aux_ids = raw.get("eagle_aux_hidden_state_layer_ids")
        n_aux = len(aux_ids) if aux_ids else raw.get("num_aux_hidden_states", 3)
        dtype = getattr(torch, raw.get("torch_dtype", "bfloat16"), None)
        if not isinstance(dtype, torch.dtype):
            raise ValueError(f"unsupported EAGLE3 torch_dtype: {raw.get('torch_dtype')}")
        return cls(
            hidden_size=hidden,
            intermediate_size=layer["intermediate_size"],
            num_attention_heads=layer["num_attention_heads"],
            num_key_value_heads=layer["num_key_value_heads"],
            head_dim=layer.get("head_dim", hidden // layer["num_attention_heads"]),
            max_position_embeddings=layer["max_position_embeddings"],
            rms_norm_eps=layer["rms_norm_eps"],
            rope_theta=layer.get("rope_theta", 10000.0),
            attention_bias=layer.get("attention_bias", False),
            target_vocab_size=layer["vocab_size"],
            draft_vocab_size=raw["draft_vocab_size"],
            target_hidden_size=raw.get("target_hidden_size") or hidden,
            num_aux_hidden_states=n_aux,
            norm_before_residual=raw.get("norm_before_residual", True),
            torch_dtype=dtype,
        )


@dataclass
class Eagle3KVCache:
    """Recurrent draft state of one sequence: the normalised last hidden state
    (sampled from) and the pre-norm one (fed back)."""
    last_hidden_state: torch.Tensor | None = None
    last_feedback_hidden_state: torch.Tensor | None = None

    def clone(self) -> "Eagle3KVCache":
        return Eagle3KVCache(self.last_hidden_state, self.last_feedback_hidden_state)


class Eagle3DecoderLayer(nn.Module):

    def __init__(self, config: Eagle3Config):
        super().__init__()
        self.norm_before_residual = config.norm_before_residual
        self.hidden_norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.self_attn = SelfAttention(
            hidden_size=config.hidden_size,
            num_heads=config.num_attention_heads,
            num_kv_heads=config.num_key_value_heads,
            head_dim=config.head_dim,
            max_position=config.max_position_embeddings,
            rms_norm_eps=config.rms_norm_eps,
            qkv_bias=config.attention_bias,
            rope_theta=config.rope_theta,
            qkv_input_size=2 * config.hidden_size,
            use_qk_norm=False,
        )
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.mlp = MLP(config.hidden_size, config.intermediate_size)

    def forward(self, input_embeds, hidden_states, positions):
        """eagle3.py:128-146: attention over [norm(embed) | norm(hidden)], two
        residual adds."""
        mlp_out, residual = self.forward_parts(input_embeds, hidden_states, positions)
        return residual + mlp_out

    def forward_parts(self, input_embeds, hidden_states, positions):
        """The layer up to its last residual add: returns (mlp_out, residual),
        whose bf16 sum is the layer's output.  The two norms write straight
        into the halves of the attention input (no concat), and the first
        residual add is fused with post_attention_layernorm, which normalises
        the bf16 sum exactly as the separate ops do."""
        n, h = hidden_states.shape
        attn_in = torch.empty(n, 2 * h, dtype=hidden_states.dtype, device=hidden_states.device)
        K.rms_norm(input_embeds, self.input_layernorm.weight, self.input_layernorm.eps,
                   out=attn_in[:, :h])
        normed = K.rms_norm(hidden_states, self.hidden_norm.weight, self.hidden_norm.eps,
                            out=attn_in[:, h:])
        residual = normed if self.norm_before_residual else hidden_states
        x, residual = K.add_then_rms_norm(self.self_attn(positions, attn_in), residual,
                                          self.post_attention_layernorm.weight,
                                          self.post_attention_layernorm.eps)
        return self.mlp(x), residual


class Eagle3ForCausalLM(nn.Module):
    packed_modules_mapping = {
        "q_proj": ("qkv_proj", "q"),
        "k_proj": ("qkv_proj", "k"),
        "v_proj": ("qkv_proj", "v"),
        "gate_proj": ("gate_up_proj", 0),
        "up_proj": ("gate_up_proj", 1),
    }

    def __init__(self, config: Eagle3Config):
        super().__init__()
        self.config = config
        self.embed_tokens = Embedding(config.target_vocab_size, config.hidden_size)
        self.fc = Linear(config.target_hidden_size * config.num_aux_hidden_states,
                         config.hidden_size)
        self.layers = nn.ModuleList([Eagle3DecoderLayer(config)])
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.lm_head = Linear(config.hidden_size, config.draft_vocab_size)
        self.register_buffer("d2t", torch.zeros(config.draft_vocab_size, dtype=torch.long))
        self.register_buffer("t2d", torch.zeros(config.target_vocab_size, dtype=torch.bool))
        self._loaded_weight_names: set[str] = set()

    # ---- checkpoint loading (eagle3.py:198-233)
    def load_weight(self, name: str, loaded: torch.Tensor) -> bool:
        self._loaded_weight_names.add(name)
        if name in ("d2t", "t2d"):
            self.get_buffer(name).copy_(loaded)
            return True
        return False

    def validate_loaded_weights(self) -> None:
        expected = {name for name, _ in self.named_parameters()}
        expected.update(("d2t", "t2d"))
        for packed, parts in {
            "layers.0.self_attn.qkv_proj.weight": ("layers.0.self_attn.q_proj.weight",
                                                   "layers.0.self_attn.k_proj.weight",
                                                   "layers.0.self_attn.v_proj.weight"),
            "layers.0.mlp.gate_up_proj.weight": ("layers.0.mlp.gate_proj.weight",
                                                 "layers.0.mlp.up_proj.weight"),
        }.items():
            if packed in expected:
                expected.remove(packed)
                expected.update(parts)
        missing = expected - self._loaded_weight_names
        unexpected = self._loaded_weight_names - expected
        if missing or unexpected:
            raise ValueError(f"EAGLE3 checkpoint/model mismatch: missing={sorted(missing)}, "
                             f"unexpected={sorted(unexpected)}")

    # ---- forward pieces
    def combine_hidden_states(self, target_hidden_states: torch.Tensor) -> torch.Tensor:
        want = self.config.target_hidden_size * self.config.num_aux_hidden_states
        if target_hidden_states.ndim != 2 or target_hidden_states.size(-1) != want:
            raise ValueError(f"target_hidden_states must have shape [num_tokens, {want}]")
        return self.fc(target_hidden_states)

    def forward_with_cache(self, input_ids, positions, hidden_states):
        """One draft step over the paged draft cache; returns (normalised,
        pre-norm) hidden states (eagle3.py:244-262)."""
        if input_ids.ndim != 1 or positions.ndim != 1:
            raise ValueError("EAGLE3 forward expects 1D input_ids and positions")
        if input_ids.numel() != positions.numel():
            raise ValueError("input_ids and positions must contain the same number of tokens")
        if hidden_states.ndim != 2 or hidden_states.size(-1) != self.config.hidden_size:
            raise ValueError("EAGLE3 feedback hidden_states must have shape "
                             f"[num_tokens, {self.config.hidden_size}]")
        embeds = self.embed_tokens(input_ids)
        for layer in self.layers[:-1]:
            hidden_states = layer(embeds, hidden_states, positions)
        # the last layer's residual add is fused with the final norm
        mlp_out, residual = self.layers[-1].forward_parts(embeds, hidden_states, positions)
        return K.add_then_rms_norm(mlp_out, residual, self.norm.weight, self.norm.eps)

    def forward(self, input_ids, positions, target_hidden_states):
        return self.forward_with_cache(input_ids, positions,
                                       self.combine_hidden_states(target_hidden_states))[0]

    def sample_greedy(self, hidden_states: torch.Tensor, out: torch.Tensor | None = None):
        """argmax of the draft logits mapped to target ids (eagle3.py:294-296),
        fused in the argmax kernel."""
        logits = F.linear(hidden_states, self.lm_head.weight)
        return K.argmax_rows(logits, self.d2t, out=out)


def load_eagle3_model(model_path, device="cuda", load_format: str = "auto",
                      seed: int = 1) -> Eagle3ForCausalLM:
    """Build the draft and load its checkpoint (or random weights with
    load_format="dummy")."""
    config = Eagle3Config.from_pretrained(model_path)
    model = Eagle3ForCausalLM(config).to(device=device)
    # cast parameters only: the attention layers' fp32 KV scales and the
    # d2t / t2d maps keep their dtypes
    for p in model.parameters():
        p.data = p.data.to(config.torch_dtype)
    if load_format == "dummy":
        init_random_(model, seed)
        model.t2d.fill_(True)
    else:
        load_model(model, str(model_path))
        model.validate_loaded_weights()
    return model.eval()
