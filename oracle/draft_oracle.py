"""CPU float32 restatement of the EAGLE3 draft step (TEST INFRASTRUCTURE ONLY).

Only tests/ may import this module, and only to check the product: the
product package never imports it.  It restates, in float32 torch on the CPU,
one token at a time:

* ``Eagle3DecoderLayer.forward`` (nanovllm/models/eagle3.py:128-146): the
  hidden state is RMS-normalised (``hidden_norm``; with
  ``norm_before_residual`` the normalised state is also the residual), the
  token embedding is RMS-normalised (``input_layernorm``), their
  concatenation [embed | hidden] (2H) feeds the attention, then residual
  add, ``post_attention_layernorm``, MLP, residual add;
* the attention block: ``Qwen3Attention`` without q/k norm
  (nanovllm/models/qwen3.py:77-112): fused QKV projection, neox RoPE
  (nanovllm/layers/rotary_embedding.py:6-48, theta from the config), causal
  softmax attention with scale head_dim ** -0.5 over the draft's K/V
  history plus this token's own K/V, GQA head h -> kv head h // (Hq / Hkv),
  output projection;
* the MLP: gate_up projection, SiLU(gate) * up, down projection
  (nanovllm/layers/activation.py:11-14, models/qwen3.py:115-140);
* ``forward_with_cache`` (eagle3.py:244-262): returns (final-normalised,
  pre-norm) states; ``combine_hidden_states`` = ``fc`` (:235-242);
  ``sample_greedy`` (:294-296): argmax of the LM-head logits plus d2t;
* the proposal recurrence of ``propose_eagle3_batch``
  (nanovllm/engine/model_runner.py:1159-1213): the first proposal is sampled
  from the stored normalised state; step s feeds the previous proposal at
  RoPE position start + s with the stored / previous pre-norm state;
* the commit replay of ``commit_eagle3`` / ``_commit_eagle3_tokens``
  (model_runner.py:1127-1156, :1216-1249): committed token i at position
  start + i consumes fc(aux row i), one token after the other, and the last
  token's states become the recurrent state.

Draft K/V slots follow this build's convention (draft position p is stored
at position p, also in decode and commit; the reference stores decode and
commit positions at p + 1, model_runner.py:1087-1096): the history passed
in holds the draft K/V of positions [0, start).

Pinned by tests/test_oracle.py: RMSNorm, RoPE and the MLP against the
transformers Llama modules in float32; the attention against torch's
scaled_dot_product_attention; closed forms of the layer (zero attention and
MLP outputs leave exactly the normalised / raw hidden state, one visible
key returns its V row) and of d2t sampling.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class DraftWeights:
    """Float32 CPU copies of an EAGLE3 draft's weights."""
    embed: torch.Tensor          # [V, H]
    fc: torch.Tensor             # [H, 3H]
    hidden_norm: torch.Tensor    # [H]
    input_norm: torch.Tensor     # [H]
    qkv: torch.Tensor            # [(Hq + 2 Hkv) D, 2H]
    o: torch.Tensor              # [H, Hq D]
    post_norm: torch.Tensor      # [H]
    gate_up: torch.Tensor        # [2 I, H]
    down: torch.Tensor           # [H, I]
    norm: torch.Tensor           # [H]
    lm_head: torch.Tensor        # [Vd, H]
    d2t: torch.Tensor            # [Vd] int64
    num_heads: int
    num_kv_heads: int
    head_dim: int
    eps: float
    rope_theta: float
    norm_before_residual: bool = True

    @classmethod
    def from_module(cls, m) -> "DraftWeights":
        """From an Eagle3ForCausalLM (parameter names of the reference's
        checkpoint layout, eagle3.py:149-196)."""
        layer = m.layers[0]
        cfg = m.config
        f = lambda t: t.detach().float().cpu().clone()  # noqa: E731
        return cls(embed=f(m.embed_tokens.weight), fc=f(m.fc.weight),
                   hidden_norm=f(layer.hidden_norm.weight),
                   input_norm=f(layer.input_layernorm.weight),
                   qkv=f(layer.self_attn.qkv_proj.weight), o=f(layer.self_attn.o_proj.weight),
                   post_norm=f(layer.post_attention_layernorm.weight),
                   gate_up=f(layer.mlp.gate_up_proj.weight), down=f(layer.mlp.down_proj.weight),
                   norm=f(m.norm.weight), lm_head=f(m.lm_head.weight),
                   d2t=m.d2t.detach().cpu().long().clone(), num_heads=cfg.num_attention_heads,
                   num_kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                   eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                   norm_before_residual=cfg.norm_before_residual)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * w over the last dim (layernorm.py:70-89)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rope(x: torch.Tensor, pos: int, theta: float) -> torch.Tensor:
    """Neox rotary embedding of one position: x [heads, D]; the first and
    second halves rotate together by angle pos * theta^(-2i/D)
    (rotary_embedding.py:6-35).  The angles are float32 products of float32
    inverse frequencies and positions, as in the reference's table
    (:28-35); at positions in the thousands they differ from exact angles
    by ~1e-4 rad."""
    d = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = torch.tensor(float(pos), dtype=torch.float32) * inv
    cos, sin = torch.cos(ang), torch.sin(ang)
    x1, x2 = x[..., :d // 2], x[..., d // 2:]
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1)


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T * D^-0.5) v of one query row q [Hq, D] over every key of
    k / v [n, Hkv, D] (the query is the last position, so all n keys are
    visible); query head h reads kv head h // (Hq / Hkv)."""
    hq, d = q.shape
    g = hq // k.shape[1]
    kk = k.repeat_interleave(g, dim=1)                   # [n, Hq, D]
    vv = v.repeat_interleave(g, dim=1)
    s = torch.einsum("hd,nhd->hn", q, kk) * d ** -0.5
    return torch.einsum("hn,nhd->hd", torch.softmax(s, -1), vv)


def forward_token(w: DraftWeights, token: int, pos: int, hidden_in: torch.Tensor,
                  k_hist: torch.Tensor, v_hist: torch.Tensor):
    """One draft token at RoPE position ``pos``: hidden_in [H] is the fed-back
    pre-norm state or the fc output; k_hist / v_hist [pos, Hkv, D] hold the
    draft K/V of positions [0, pos).  Returns (normed [H], prenorm [H],
    k [Hkv, D], v [Hkv, D])."""
    hq, hkv, d = w.num_heads, w.num_kv_heads, w.head_dim
    hn = rms_norm(hidden_in, w.hidden_norm, w.eps)
    residual = hn if w.norm_before_residual else hidden_in
    attn_in = torch.cat((rms_norm(w.embed[token], w.input_norm, w.eps), hn))
    qkv = w.qkv @ attn_in
    q = rope(qkv[:hq * d].view(hq, d), pos, w.rope_theta)
    k = rope(qkv[hq * d:(hq + hkv) * d].view(hkv, d), pos, w.rope_theta)
    v = qkv[(hq + hkv) * d:].view(hkv, d)
    o = attend(q, torch.cat((k_hist, k[None])), torch.cat((v_hist, v[None])))
    h1 = residual + w.o @ o.reshape(-1)
    out = h1 + mlp(w, rms_norm(h1, w.post_norm, w.eps))
    return rms_norm(out, w.norm, w.eps), out, k, v


def mlp(w: DraftWeights, x: torch.Tensor) -> torch.Tensor:
    """down(SiLU(gate x) * (up x)); gate_up holds [gate; up] row blocks."""
    gu = w.gate_up @ x
    inter = gu.shape[0] // 2
    return w.down @ (torch.nn.functional.silu(gu[:inter]) * gu[inter:])


def logits(w: DraftWeights, normed: torch.Tensor) -> torch.Tensor:
    """Draft LM-head logits over the draft vocabulary."""
    return w.lm_head @ normed


def sample_greedy(w: DraftWeights, normed: torch.Tensor) -> int:
    """argmax of the draft logits, mapped to a target id with d2t
    (eagle3.py:294-296)."""
    i = int(torch.argmax(logits(w, normed)))
    return i + int(w.d2t[i])


def propose(w: DraftWeights, hidden: torch.Tensor, feedback: torch.Tensor, start: int,
            steps: int, k_hist: torch.Tensor, v_hist: torch.Tensor, forced=None):
    """The proposal recurrence of one sequence: ``steps`` tokens from the
    stored states (hidden = normalised, feedback = pre-norm), draft step s
    at position start + s.  With ``forced`` (a token list) step s is fed
    forced[s] instead of the restatement's own token, so the comparison of a
    device run does not compound after a near tie.  Returns (tokens, logit
    rows [steps, Vd], K rows, V rows [steps - 1, Hkv, D] written at positions
    start .. start + steps - 2)."""
    toks, rows, ks, vs = [], [], [], []
    normed = hidden
    for s in range(steps):
        rows.append(logits(w, normed))
        toks.append(sample_greedy(w, normed))
        if s + 1 == steps:
            break
        fed = toks[-1] if forced is None else int(forced[s])
        normed, feedback, k, v = forward_token(w, fed, start + s, feedback,
                                               torch.cat((k_hist, *[x[None] for x in ks])),
                                               torch.cat((v_hist, *[x[None] for x in vs])))
        ks.append(k)
        vs.append(v)
    empty = k_hist.new_zeros((0,) + tuple(k_hist.shape[1:]))
    return (toks, torch.stack(rows), torch.stack(ks) if ks else empty,
            torch.stack(vs) if vs else empty)


def commit(w: DraftWeights, tokens, aux_rows: torch.Tensor, start: int, k_hist: torch.Tensor,
           v_hist: torch.Tensor):
    """The commit replay of one sequence: committed token i at position
    start + i consumes fc(aux_rows[i]) (aux_rows [n, 3H], the target aux
    states of positions start ..), one token after the other.  Returns the
    last token's (normed, prenorm) states -- the new recurrent state -- and
    the K / V rows written at positions start .. start + n - 1."""
    combined = aux_rows @ w.fc.t()
    ks, vs = [], []
    normed = pre = None
    for i, tok in enumerate(tokens):
        normed, pre, k, v = forward_token(w, int(tok), start + i, combined[i],
                                          torch.cat((k_hist, *[x[None] for x in ks])),
                                          torch.cat((v_hist, *[x[None] for x in vs])))
        ks.append(k)
        vs.append(v)
    return normed, pre, torch.stack(ks), torch.stack(vs)
