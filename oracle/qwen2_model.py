"""Eager, unbufferized Qwen2 CausalLM -- TEST INFRASTRUCTURE ONLY.

Restates the reference's model math (src/stateful_llm_compiler/qwen2.py of
Edison-Ayan/llm-compiler): RMSNorm with the Qwen2 rounding order
(model.py:44-51), fp32 RoPE inverse frequencies and cos/sin cast to the model
dtype (qwen2.py:112-149), half-rotation RoPE (qwen2.py:73-96), GQA attention
with a concatenated KV cache, scores scaled in the model dtype and softmaxed
in fp32 over ``scores + mask`` (qwen2.py:158-240), SwiGLU MLP
(qwen2.py:243-256), residual decoder layers (qwen2.py:259-297), final norm
and (tied) LM head (qwen2.py:394-452).  This is the "unbufferized program"
the compiled KV-state graphs are diffed against.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .kernels import rotate_half


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    variance = x.float().pow(2).mean(dim=-1, keepdim=True)
    normalized = x.float() * torch.rsqrt(variance + eps)
    return weight * normalized.to(x.dtype)


def rope_tables(position_ids: torch.Tensor, inv_freq: torch.Tensor, dtype: torch.dtype):
    freqs = position_ids.float().unsqueeze(-1) * inv_freq.float().view(1, 1, -1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


class EagerQwen2:
    """Functional eager model over a weights dict (Hugging Face names)."""

    def __init__(self, config, weights: dict[str, torch.Tensor]) -> None:
        self.c = config
        self.w = weights

    def _attention(self, layer, h, mask, cos, sin, past):
        c, w = self.c, self.w
        p = f"layers.{layer}.self_attn."
        B, T, _ = h.shape
        q = F.linear(h, w[p + "q_proj.weight"], w[p + "q_proj.bias"]).view(B, T, c.num_heads, c.head_dim).transpose(1, 2)
        k = F.linear(h, w[p + "k_proj.weight"], w[p + "k_proj.bias"]).view(B, T, c.num_kv_heads, c.head_dim).transpose(1, 2)
        v = F.linear(h, w[p + "v_proj.weight"], w[p + "v_proj.bias"]).view(B, T, c.num_kv_heads, c.head_dim).transpose(1, 2)
        cu, su = cos.unsqueeze(1), sin.unsqueeze(1)
        q = q * cu + rotate_half(q) * su
        k = k * cu + rotate_half(k) * su
        if past is not None:
            k = torch.cat((past[0], k), dim=2)
            v = torch.cat((past[1], v), dim=2)
        groups = c.num_heads // c.num_kv_heads
        ak = k.repeat_interleave(groups, dim=1)
        av = v.repeat_interleave(groups, dim=1)
        scores = torch.matmul(q, ak.transpose(-2, -1)) * (c.head_dim ** -0.5)
        probs = torch.softmax(scores.float() + mask.float(), dim=-1).to(q.dtype)
        ctx = torch.matmul(probs, av).transpose(1, 2).contiguous().reshape(B, T, c.hidden_size)
        return F.linear(ctx, w[p + "o_proj.weight"]), k, v

    def _layer(self, layer, h, mask, cos, sin, past):
        c, w = self.c, self.w
        p = f"layers.{layer}."
        attn, k, v = self._attention(layer, rms_norm(h, w[p + "input_layernorm.weight"], c.rms_norm_eps),
                                     mask, cos, sin, past)
        h = h + attn
        x = rms_norm(h, w[p + "post_attention_layernorm.weight"], c.rms_norm_eps)
        gate = F.silu(F.linear(x, w[p + "mlp.gate_proj.weight"]))
        mlp = F.linear(gate * F.linear(x, w[p + "mlp.up_proj.weight"]), w[p + "mlp.down_proj.weight"])
        return h + mlp, k, v

    def forward(self, input_ids, mask, position_ids, past=None):
        c, w = self.c, self.w
        h = F.embedding(input_ids, w["embed_tokens.weight"])
        cos, sin = rope_tables(position_ids, w["rotary_emb.inv_freq"], h.dtype)
        present = []
        for layer in range(c.num_layers):
            h, k, v = self._layer(layer, h, mask, cos, sin, None if past is None else past[layer])
            present.append((k, v))
        h = rms_norm(h, w["norm.weight"], c.rms_norm_eps)
        lm = w.get("lm_head.weight", w["embed_tokens.weight"])
        return F.linear(h, lm), tuple(present)

    def prefill(self, input_ids, mask, position_ids):
        """Prompt pass from an empty cache (qwen2.py:410-424)."""

        return self.forward(input_ids, mask, position_ids, None)

    def decode(self, input_ids, mask, position_ids, past):
        """One step over a concatenated past cache (qwen2.py:436-452)."""

        return self.forward(input_ids, mask, position_ids, past)


def causal_mask(batch: int, tokens: int, dtype=torch.float32) -> torch.Tensor:
    """Additive causal mask of make_qwen2_prefill_inputs (qwen2.py:540-573)."""

    future = torch.triu(torch.ones(tokens, tokens, dtype=torch.bool), diagonal=1)
    return torch.zeros(batch, 1, tokens, tokens, dtype=dtype).masked_fill(future, float("-inf"))
