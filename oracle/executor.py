"""CPU interpreter of ServeIR -- TEST INFRASTRUCTURE ONLY.

Restates the reference executor (src/stateful_llm_compiler/execution.py of
Edison-Ayan/llm-compiler): the preallocated KV runtime state
(execution.py:98-475: B x Capacity x H x D buffers, int64 lengths, store by
index_copy_ at positions + t, advance = lengths + delta with a capacity
check, prefill_store from position 0) and the serve.* handlers
(execution.py:498-767), plus the fused forms of the ops the reference runs as
eager ATen nodes (embedding, residual add, SwiGLU, RoPE table) with the eager
Qwen2 semantics.  It runs un-lowered ServeIR on the CPU so the graphs the HIP
backend compiles can be checked against the eager model without a GPU.
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Any, Sequence

import torch
import torch.nn.functional as F

from . import kernels as ref
from .qwen2_model import rms_norm as qwen2_rms_norm
from .qwen2_model import rope_tables

_DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


class OracleError(RuntimeError):
    pass


@dataclass(frozen=True)
class OracleKVState:
    keys: tuple[torch.Tensor, ...]
    values: tuple[torch.Tensor, ...]
    lengths: tuple[torch.Tensor, ...]
    capacity: int
    generation: int = 0

    @classmethod
    def empty(cls, key: torch.Tensor, num_layers: int, capacity: int) -> "OracleKVState":
        batch, heads, _, head_dim = key.shape
        keys = tuple(torch.zeros(batch, capacity, heads, head_dim, dtype=key.dtype) for _ in range(num_layers))
        values = tuple(torch.zeros_like(k) for k in keys)
        lengths = tuple(torch.zeros(batch, dtype=torch.int64) for _ in range(num_layers))
        return cls(keys, values, lengths, capacity)

    @classmethod
    def from_layer_tensors(cls, past, capacity: int) -> "OracleKVState":
        keys, values, lengths = [], [], []
        for key, value in past:
            batch, heads, sequence, head_dim = key.shape
            kb = torch.zeros(batch, capacity, heads, head_dim, dtype=key.dtype)
            vb = torch.zeros_like(kb)
            kb[:, :sequence] = key.transpose(1, 2)
            vb[:, :sequence] = value.transpose(1, 2)
            keys.append(kb)
            values.append(vb)
            lengths.append(torch.full((batch,), sequence, dtype=torch.int64))
        return cls(tuple(keys), tuple(values), tuple(lengths), capacity)

    def store(self, slot: int, key: torch.Tensor, value: torch.Tensor, positions: torch.Tensor) -> "OracleKVState":
        """native_kv_store (execution.py:743-781) with the capacity check."""

        batch, heads, tokens, head_dim = key.shape
        if bool((positions + tokens > self.capacity).any()):
            raise OracleError(f"KV store exceeds capacity {self.capacity}")
        rows = torch.arange(batch).view(batch, 1) * self.capacity
        index = (rows + positions.view(batch, 1) + torch.arange(tokens).view(1, tokens)).reshape(-1)
        src_k = key.transpose(1, 2).reshape(batch * tokens, heads, head_dim)
        src_v = value.transpose(1, 2).reshape(batch * tokens, heads, head_dim)
        self.keys[slot].view(-1, heads, head_dim).index_copy_(0, index, src_k)
        self.values[slot].view(-1, heads, head_dim).index_copy_(0, index, src_v)
        return self

    def advance(self, slot: int, delta: int) -> "OracleKVState":
        nxt = self.lengths[slot] + delta
        if bool((nxt > self.capacity).any()):
            raise OracleError(f"KV advance exceeds capacity {self.capacity}")
        lengths = list(self.lengths)
        lengths[slot] = nxt
        return replace(self, lengths=tuple(lengths), generation=self.generation + 1)

    def prefill_store(self, slot: int, key: torch.Tensor, value: torch.Tensor) -> "OracleKVState":
        if bool((self.lengths[slot] != 0).any()):
            raise OracleError("prefill store needs a zero-length slot")
        self.store(slot, key, value, self.lengths[slot])
        return self.advance(slot, key.shape[2])

    def decode_attention(self, slot, query, mask, groups, scale):
        return ref.decode_attention(query, self.keys[slot], self.values[slot], self.lengths[slot], mask,
                                    groups=groups, scale=scale)


def _resolve_shape(spec, tensor):
    return [int(tensor.shape[int(s["dim"])]) if isinstance(s, dict) else int(s) for s in spec]


class OracleExecutor:
    """Runs a ServeIR function (un-lowered) with eager CPU semantics."""

    def run(self, module, arguments: Sequence[Any], function_name: str | None = None):
        function = module.functions[0] if function_name is None else next(
            f for f in module.functions if f.name == function_name
        )
        env: dict[str, Any] = {a.name: v for a, v in zip(function.block.arguments, arguments)}
        for op in function.block.operations:
            args = [env[v.name] for v in op.operands]
            result = self._execute(op.name, op.attributes, args)
            if len(op.results) == 1:
                env[op.results[0].name] = result
            else:
                for value, item in zip(op.results, result):
                    env[value.name] = item
        return tuple(env[v.name] for v in function.returns)

    def _execute(self, name: str, a: dict[str, Any], args: list[Any]):
        if name == "serve.rms_norm":
            x, w = args
            if a.get("round_before_weight"):
                return qwen2_rms_norm(x, w, float(a["epsilon"]))
            return ref.rms_norm(x, w, epsilon=float(a["epsilon"]), output_dtype=a.get("output_dtype"))
        if name == "serve.linear":
            return ref.linear(*args)
        if name == "serve.rope":
            return ref.rope(*args)
        if name == "serve.embedding":
            return F.embedding(args[0], args[1])
        if name == "serve.add":
            return args[0] + args[1]
        if name == "serve.swiglu":
            return F.silu(args[0]) * args[1]
        if name == "serve.rope_table":
            return rope_tables(args[0], args[1], _DTYPES[a["dtype"]])
        if name == "aten.view.default":
            # The eager model copies here (transpose().contiguous().reshape()).
            return args[0].reshape(_resolve_shape(a["shape"], args[0]))
        if name == "aten.transpose.int":
            return args[0].transpose(int(a["dim0"]), int(a["dim1"]))
        if name == "aten.unsqueeze.default":
            return args[0].unsqueeze(int(a["dim"]))
        if name == "serve.kv.init":
            return OracleKVState.empty(args[0], int(a["num_layers"]), int(a["capacity"]))
        if name == "serve.kv.length":
            return args[0].lengths[int(a.get("slot", 0))]
        if name == "serve.kv.store":
            state, k, v, positions = args
            return state.store(int(a.get("slot", 0)), k, v, positions)
        if name == "serve.kv.advance":
            return args[0].advance(int(a.get("slot", 0)), int(a.get("delta", 1)))
        if name == "serve.kv.prefill_store":
            state, k, v = args
            return state.prefill_store(int(a.get("slot", 0)), k, v)
        if name == "serve.decode_attention":
            state, q, mask = args
            return state.decode_attention(int(a.get("slot", 0)), q, mask, int(a["groups"]), float(a["scale"]))
        if name == "serve.prefill_attention":
            q, k, v, mask = args
            return ref.prefill_attention(q, k, v, mask, groups=int(a["groups"]), scale=float(a["scale"]),
                                         causal=a.get("causal"))
        raise OracleError(f"oracle executor has no handler for {name}")
