"""Qwen2 CausalLM as ServeIR: configuration, seeded weights, graph builders.

The reference obtains its ServeIR by capturing its PyTorch Qwen2 with
torch.export and running its fusion passes (src/stateful_llm_compiler/
qwen2.py:73-452, optimizer.py:32-64).  Those passes sit outside this
backend's scope, so this module emits the graph those passes produce for the
Qwen2 decoder directly: per layer one serve.rms_norm (Qwen2 rounding order,
model.py:44-51), Q/K/V serve.linear, one dual-output serve.rope, the KV ops
(kv.length / kv.store / kv.advance + serve.decode_attention for decode,
kv.init / kv.prefill_store + serve.prefill_attention for prefill), the O
projection, residual adds, the post-attention norm and the SwiGLU MLP; then
the final norm and the tied LM head.  The ops the reference leaves as eager
ATen nodes appear in their fused ServeIR forms (serve.embedding, serve.add,
serve.swiglu, serve.rope_table) and views as aten.view / aten.transpose.

Decode takes its RoPE positions from the KV state (``kv.length`` of slot 0
before the step), which is what the caller passes as ``position_ids`` to the
reference's decode graph; keeping them on the device lets a whole step be
replayed as one HIP graph.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from .ir import (
    Effect,
    EffectKind,
    Function,
    IRBuilder,
    KVStateType,
    Module,
    TensorType,
    Value,
    dims,
)


@dataclass(frozen=True)
class Qwen2Config:
    """Decoder configuration (qwen2.py:15-45); defaults are Qwen2-0.5B's shape."""

    hidden_size: int = 896
    intermediate_size: int = 4864
    num_layers: int = 24
    num_heads: int = 14
    num_kv_heads: int = 2
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    vocab_size: int = 151936
    tie_word_embeddings: bool = True

    def __post_init__(self) -> None:
        if self.hidden_size % self.num_heads:
            raise ValueError("hidden_size must be divisible by num_heads")
        if self.num_heads % self.num_kv_heads:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        if self.head_dim % 2:
            raise ValueError("Qwen2 RoPE needs an even head_dim")

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def groups(self) -> int:
        return self.num_heads // self.num_kv_heads


def inverse_frequency(config: Qwen2Config, device: torch.device | str = "cpu") -> torch.Tensor:
    """fp32 RoPE inverse frequencies, 1 / theta^(2i/D) (qwen2.py:112-134)."""

    steps = torch.arange(0, config.head_dim, 2, dtype=torch.float32, device=device)
    return 1.0 / (config.rope_theta ** (steps / config.head_dim))


def causal_prefill_mask(batch: int, tokens: int, *, dtype: torch.dtype = torch.float32,
                        device: torch.device | str = "cpu") -> torch.Tensor:
    """Additive causal mask [B, 1, T, T] of a prompt (0 on and below the
    diagonal, -inf above), the prefill input of make_qwen2_prefill_inputs
    (qwen2.py:540-573)."""

    future = torch.triu(torch.ones(tokens, tokens, dtype=torch.bool, device=device), diagonal=1)
    mask = torch.zeros(batch, 1, tokens, tokens, dtype=dtype, device=device)
    return mask.masked_fill(future, float("-inf"))


def weight_names(config: Qwen2Config) -> list[str]:
    """Parameter order of the compiled functions (Hugging Face names)."""

    names = ["embed_tokens.weight", "rotary_emb.inv_freq"]
    for layer in range(config.num_layers):
        p = f"layers.{layer}."
        names += [
            p + "input_layernorm.weight",
            p + "self_attn.q_proj.weight", p + "self_attn.q_proj.bias",
            p + "self_attn.k_proj.weight", p + "self_attn.k_proj.bias",
            p + "self_attn.v_proj.weight", p + "self_attn.v_proj.bias",
            p + "self_attn.o_proj.weight",
            p + "post_attention_layernorm.weight",
            p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", p + "mlp.down_proj.weight",
        ]
    names.append("norm.weight")
    if not config.tie_word_embeddings:
        names.append("lm_head.weight")
    return names


def init_weights(
    config: Qwen2Config,
    *,
    seed: int = 0,
    dtype: torch.dtype = torch.bfloat16,
    device: torch.device | str = "cpu",
    std: float = 0.02,
    draw_on_device: bool = False,
) -> dict[str, torch.Tensor]:
    """Seeded random weights: projections, biases and embeddings N(0, std),
    norm weights 1 + N(0, std).  Generated in fp32 on the CPU, then cast and
    moved, so every device and dtype sees the same draw."""

    # Drawn on the CPU by default so every device sees the same values; a
    # CUDA ``device`` with ``draw_on_device=True`` draws there instead (much
    # faster for the 0.5B-parameter model, reproducible on that device).
    draw = torch.device(device) if draw_on_device else torch.device("cpu")
    g = torch.Generator(device=draw).manual_seed(seed)
    H, I, V = config.hidden_size, config.intermediate_size, config.vocab_size
    kv = config.num_kv_heads * config.head_dim
    shapes: dict[str, tuple[int, ...]] = {"embed_tokens.weight": (V, H)}
    for layer in range(config.num_layers):
        p = f"layers.{layer}."
        shapes.update({
            p + "input_layernorm.weight": (H,),
            p + "self_attn.q_proj.weight": (H, H), p + "self_attn.q_proj.bias": (H,),
            p + "self_attn.k_proj.weight": (kv, H), p + "self_attn.k_proj.bias": (kv,),
            p + "self_attn.v_proj.weight": (kv, H), p + "self_attn.v_proj.bias": (kv,),
            p + "self_attn.o_proj.weight": (H, H),
            p + "post_attention_layernorm.weight": (H,),
            p + "mlp.gate_proj.weight": (I, H), p + "mlp.up_proj.weight": (I, H),
            p + "mlp.down_proj.weight": (H, I),
        })
    shapes["norm.weight"] = (H,)
    if not config.tie_word_embeddings:
        shapes["lm_head.weight"] = (V, H)
    weights: dict[str, torch.Tensor] = {}
    for name, shape in shapes.items():
        t = torch.randn(*shape, generator=g, device=draw) * std
        if name.endswith("norm.weight"):
            t = t + 1.0
        weights[name] = t.to(dtype).to(device)
        del t
    weights["rotary_emb.inv_freq"] = inverse_frequency(config, device)
    return weights


def weight_arguments(config: Qwen2Config, weights: dict[str, torch.Tensor]) -> list[torch.Tensor]:
    return [weights[name] for name in weight_names(config)]


_DTYPE = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


class _GraphBuilder:
    """Shared emission helpers for the decode and prefill functions."""

    def __init__(self, config: Qwen2Config, dtype: torch.dtype, device: str) -> None:
        self.config = config
        self.dt = _DTYPE[dtype]
        self.device = device
        self.b = IRBuilder()
        self.weights: dict[str, Value] = {}

    def tensor(self, *shape: Any, dtype: str | None = None) -> TensorType:
        return TensorType(dims(*shape), dtype or self.dt, self.device)

    def add_weights(self) -> None:
        c = self.config
        kv = c.num_kv_heads * c.head_dim
        shape_of = {
            "embed_tokens.weight": (c.vocab_size, c.hidden_size),
            "rotary_emb.inv_freq": (c.head_dim // 2,),
            "norm.weight": (c.hidden_size,),
            "lm_head.weight": (c.vocab_size, c.hidden_size),
        }
        for name in weight_names(c):
            if name in shape_of:
                shape = shape_of[name]
            elif name.endswith("layernorm.weight"):
                shape = (c.hidden_size,)
            elif "q_proj.weight" in name or "o_proj.weight" in name:
                shape = (c.hidden_size, c.hidden_size)
            elif "q_proj.bias" in name:
                shape = (c.hidden_size,)
            elif "k_proj.weight" in name or "v_proj.weight" in name:
                shape = (kv, c.hidden_size)
            elif "k_proj.bias" in name or "v_proj.bias" in name:
                shape = (kv,)
            elif "gate_proj" in name or "up_proj" in name:
                shape = (c.intermediate_size, c.hidden_size)
            else:  # down_proj
                shape = (c.hidden_size, c.intermediate_size)
            dtype = "f32" if name == "rotary_emb.inv_freq" else self.dt
            self.weights[name] = self.b.argument(self.tensor(*shape, dtype=dtype), _hint(name))

    def op(self, name: str, operands, result_types, **attributes) -> list[Value]:
        effects = attributes.pop("_effects", ())
        return self.b.emit(name, operands, result_types, attributes=attributes, effects=effects).results

    def rms_norm(self, x: Value, weight: Value) -> Value:
        return self.op("serve.rms_norm", [x, weight], [x.type], epsilon=self.config.rms_norm_eps,
                       axis=-1, round_before_weight=True)[0]

    def linear(self, x: Value, weight: Value, bias: Value | None = None) -> Value:
        n, k = (d.value for d in weight.type.shape)
        out = TensorType(x.type.shape[:-1] + dims(n), self.dt, self.device)
        operands = [x, weight] + ([bias] if bias is not None else [])
        return self.op("serve.linear", operands, [out], has_bias=bias is not None,
                       input_features=k, output_features=n)[0]

    def split_heads(self, x: Value, heads: int, B: Any, T: Any) -> Value:
        """[B, T, heads*D] -> view [B, T, heads, D] -> transpose [B, heads, T, D]."""

        D = self.config.head_dim
        viewed = self.op("aten.view.default", [x], [self.tensor(B, T, heads, D)],
                         shape=[{"dim": 0}, {"dim": 1}, heads, D])[0]
        return self.op("aten.transpose.int", [viewed], [self.tensor(B, heads, T, D)], dim0=1, dim1=2)[0]

    def merge_heads(self, x: Value, B: Any, T: Any) -> Value:
        c = self.config
        t = self.op("aten.transpose.int", [x], [self.tensor(B, T, c.num_heads, c.head_dim)], dim0=1, dim1=2)[0]
        return self.op("aten.view.default", [t], [self.tensor(B, T, c.hidden_size)],
                       shape=[{"dim": 0}, {"dim": 1}, c.hidden_size])[0]

    def layer_head(self, h: Value, layer: int, B: Any, T: Any, cos: Value, sin: Value):
        """Input norm, Q/K/V projections and RoPE of one layer."""

        c = self.config
        w = self.weights
        p = f"layers.{layer}."
        x = self.rms_norm(h, w[p + "input_layernorm.weight"])
        q = self.linear(x, w[p + "self_attn.q_proj.weight"], w[p + "self_attn.q_proj.bias"])
        k = self.linear(x, w[p + "self_attn.k_proj.weight"], w[p + "self_attn.k_proj.bias"])
        v = self.linear(x, w[p + "self_attn.v_proj.weight"], w[p + "self_attn.v_proj.bias"])
        q4 = self.split_heads(q, c.num_heads, B, T)
        k4 = self.split_heads(k, c.num_kv_heads, B, T)
        v4 = self.split_heads(v, c.num_kv_heads, B, T)
        qr, kr = self.op("serve.rope", [q4, k4, cos, sin], [q4.type, k4.type],
                         head_dim=c.head_dim, variant="qwen2_half_rotation")
        return qr, kr, v4

    def layer_tail(self, h: Value, context: Value, layer: int, B: Any, T: Any) -> Value:
        """O projection, residual, post-attention norm, SwiGLU MLP, residual."""

        w = self.weights
        p = f"layers.{layer}."
        merged = self.merge_heads(context, B, T)
        o = self.linear(merged, w[p + "self_attn.o_proj.weight"])
        h2 = self.op("serve.add", [h, o], [h.type])[0]
        x2 = self.rms_norm(h2, w[p + "post_attention_layernorm.weight"])
        gate = self.linear(x2, w[p + "mlp.gate_proj.weight"])
        up = self.linear(x2, w[p + "mlp.up_proj.weight"])
        act = self.op("serve.swiglu", [gate, up], [gate.type])[0]
        down = self.linear(act, w[p + "mlp.down_proj.weight"])
        return self.op("serve.add", [h2, down], [h2.type])[0]

    def head(self, h: Value) -> Value:
        x = self.rms_norm(h, self.weights["norm.weight"])
        lm = self.weights.get("lm_head.weight", self.weights["embed_tokens.weight"])
        return self.linear(x, lm)

    def rope_table(self, positions: Value, B: Any, T: Any) -> tuple[Value, Value]:
        c = self.config
        table = self.tensor(B, T, c.head_dim)
        cos, sin = self.op("serve.rope_table", [positions, self.weights["rotary_emb.inv_freq"]],
                           [table, table], head_dim=c.head_dim, dtype=self.dt,
                           theta=c.rope_theta)
        return cos, sin


def _hint(name: str) -> str:
    return name.replace(".", "_")


def _kv_effects(resource: str = "kv", write: bool = False):
    effects = [Effect(EffectKind.READ, resource)]
    if write:
        effects.append(Effect(EffectKind.WRITE, resource))
    return tuple(effects)


def kv_state_type(dtype: str, config: "Qwen2Config", capacity: int,
                  page_tokens: int | None = None) -> KVStateType:
    """The model's KV state type: contiguous_bshd buffers, or the paged
    layout (pools of ``page_tokens``-token pages + a block table) when
    ``page_tokens`` is given."""

    return KVStateType(dtype, config.num_layers, config.num_kv_heads, config.head_dim,
                       layout="contiguous_bshd" if page_tokens is None else "paged",
                       capacity=capacity, page_tokens=page_tokens)


def build_decode_module(
    config: Qwen2Config,
    *,
    capacity: int,
    page_tokens: int | None = None,
    dtype: torch.dtype = torch.bfloat16,
    device: str = "cuda:0",
    batch: int | str = "s_batch",
) -> Module:
    """Single-token stateful decode over bufferized KV state.

    ``@decode(input_ids [B,1] i64, attention_mask [B,1,1,S], state, weights...)
    -> (logits [B,1,V], state)``
    """

    g = _GraphBuilder(config, dtype, device)
    c = config
    B, T = batch, 1
    input_ids = g.b.argument(g.tensor(B, T, dtype="i64"), "input_ids")
    mask = g.b.argument(g.tensor(B, 1, 1, "s_mask"), "attention_mask")
    state_type = kv_state_type(g.dt, c, capacity, page_tokens)
    state = g.b.argument(state_type, "kv_state")
    g.add_weights()

    h = g.op("serve.embedding", [input_ids, g.weights["embed_tokens.weight"]],
             [g.tensor(B, T, c.hidden_size)])[0]
    positions = g.op("serve.kv.length", [state], [g.tensor(B, dtype="i64")], slot=0,
                     _effects=_kv_effects())[0]
    position_ids = g.op("aten.unsqueeze.default", [positions], [g.tensor(B, 1, dtype="i64")], dim=1)[0]
    cos, sin = g.rope_table(position_ids, B, T)
    for layer in range(c.num_layers):
        qr, kr, v4 = g.layer_head(h, layer, B, T, cos, sin)
        pos = g.op("serve.kv.length", [state], [g.tensor(B, dtype="i64")], slot=layer,
                   _effects=_kv_effects())[0]
        state = g.op("serve.kv.store", [state, kr, v4, pos], [state_type], slot=layer,
                     _effects=_kv_effects(write=True))[0]
        state = g.op("serve.kv.advance", [state], [state_type], slot=layer, delta=1,
                     _effects=_kv_effects(write=True))[0]
        context = g.op("serve.decode_attention", [state, qr, mask], [qr.type], slot=layer,
                       groups=c.groups, scale=c.head_dim ** -0.5, algorithm="online_softmax",
                       _effects=_kv_effects())[0]
        h = g.layer_tail(h, context, layer, B, T)
    logits = g.head(h)
    return Module([Function("decode", g.b.block, [logits, state])])


def build_prefill_module(
    config: Qwen2Config,
    *,
    capacity: int,
    page_tokens: int | None = None,
    dtype: torch.dtype = torch.bfloat16,
    device: str = "cuda:0",
    batch: int | str = "s_batch",
    tokens: int | str = "s_tokens",
    mask_dtype: str = "f32",
) -> Module:
    """Multi-token stateful prefill that creates and fills the KV state.

    ``@prefill(input_ids [B,T] i64, attention_mask [B,1,T,T], position_ids
    [B,T] i64, weights...) -> (logits [B,T,V], state)``
    """

    g = _GraphBuilder(config, dtype, device)
    c = config
    B, T = batch, tokens
    input_ids = g.b.argument(g.tensor(B, T, dtype="i64"), "input_ids")
    mask = g.b.argument(g.tensor(B, 1, T, T, dtype=mask_dtype), "attention_mask")
    position_ids = g.b.argument(g.tensor(B, T, dtype="i64"), "position_ids")
    g.add_weights()
    state_type = kv_state_type(g.dt, c, capacity, page_tokens)

    h = g.op("serve.embedding", [input_ids, g.weights["embed_tokens.weight"]],
             [g.tensor(B, T, c.hidden_size)])[0]
    cos, sin = g.rope_table(position_ids, B, T)
    state = None
    for layer in range(c.num_layers):
        qr, kr, v4 = g.layer_head(h, layer, B, T, cos, sin)
        if state is None:
            paging = {} if page_tokens is None else {"layout": "paged", "page_tokens": page_tokens}
            state = g.op("serve.kv.init", [kr], [state_type], num_layers=c.num_layers,
                         capacity=capacity, **paging,
                         _effects=(Effect(EffectKind.ALLOCATE, "kv"), Effect(EffectKind.WRITE, "kv")))[0]
        state = g.op("serve.kv.prefill_store", [state, kr, v4], [state_type], slot=layer,
                     _effects=_kv_effects(write=True))[0]
        context = g.op("serve.prefill_attention", [qr, kr, v4, mask], [qr.type],
                       groups=c.groups, scale=c.head_dim ** -0.5, causal="mask",
                       algorithm="online_softmax")[0]
        h = g.layer_tail(h, context, layer, B, T)
    logits = g.head(h)
    return Module([Function("prefill", g.b.block, [logits, state])])
