"""ServeIR / KernelIR containers: SSA values, types, effects and the verifier.

Restates the contract of the reference's IR (src/stateful_llm_compiler/ir.py
of Edison-Ayan/llm-compiler): the same type vocabulary (tensor, scalar,
tuple, unknown, KV-state), the same effect model (read / write / allocate /
free on a named resource) and the same verifier rules for the KV, linear,
RoPE and attention ops (ir.py:220-742), extended to the ``kernel.hip.*`` op
names this backend lowers to.  Pure Python; nothing here touches a device.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Iterable


class IRType:
    def __str__(self) -> str:  # pragma: no cover - abstract
        raise NotImplementedError


@dataclass(frozen=True)
class StaticDim:
    value: int

    def __str__(self) -> str:
        return str(self.value)


@dataclass(frozen=True)
class SymbolicDim:
    name: str
    bounds: str | None = None

    def __str__(self) -> str:
        return f"{self.name}<{self.bounds}>" if self.bounds else self.name


Dimension = StaticDim | SymbolicDim


def dims(*values: int | str | Dimension) -> tuple[Dimension, ...]:
    """Build a shape: ints become static dims, strings symbolic dims."""

    out: list[Dimension] = []
    for value in values:
        if isinstance(value, (StaticDim, SymbolicDim)):
            out.append(value)
        elif isinstance(value, int):
            out.append(StaticDim(value))
        else:
            out.append(SymbolicDim(value))
    return tuple(out)


@dataclass(frozen=True)
class TensorType(IRType):
    shape: tuple[Dimension, ...]
    dtype: str
    device: str = "cpu"

    def __str__(self) -> str:
        return f"tensor<{'x'.join(str(d) for d in self.shape)}x{self.dtype}, {self.device}>"


@dataclass(frozen=True)
class ScalarType(IRType):
    dtype: str

    def __str__(self) -> str:
        return self.dtype


@dataclass(frozen=True)
class TupleType(IRType):
    elements: tuple[IRType, ...]

    def __str__(self) -> str:
        return "tuple<" + ", ".join(str(item) for item in self.elements) + ">"


@dataclass(frozen=True)
class UnknownType(IRType):
    reason: str = "unknown"

    def __str__(self) -> str:
        return f"!serve.unknown<{self.reason}>"


@dataclass(frozen=True)
class KVStateType(IRType):
    """Handle of the KV cache state that lives across inference steps."""

    dtype: str
    num_layers: int
    num_kv_heads: int
    head_dim: int
    layout: str = "blocked"
    resource: str = "kv"
    capacity: int | None = None
    # Tokens per page of the "paged" layout (pools + block table); None for
    # the contiguous layouts.
    page_tokens: int | None = None

    def __str__(self) -> str:
        capacity = f", capacity={self.capacity}" if self.capacity is not None else ""
        if self.page_tokens is not None:
            capacity += f", page_tokens={self.page_tokens}"
        return (
            f"!serve.kv_state<{self.dtype}, layers={self.num_layers}, "
            f"heads={self.num_kv_heads}, head_dim={self.head_dim}, "
            f"layout={self.layout}, resource={self.resource}{capacity}>"
        )


class EffectKind(str, Enum):
    READ = "read"
    WRITE = "write"
    ALLOCATE = "allocate"
    FREE = "free"


@dataclass(frozen=True)
class Effect:
    kind: EffectKind
    resource: str

    def __str__(self) -> str:
        return f"{self.kind.value}({self.resource})"


@dataclass(eq=False)
class Value:
    name: str
    type: IRType

    def __str__(self) -> str:
        return self.name


@dataclass
class Operation:
    name: str
    operands: list[Value]
    results: list[Value]
    attributes: dict[str, Any] = field(default_factory=dict)
    effects: tuple[Effect, ...] = ()


@dataclass
class Block:
    arguments: list[Value] = field(default_factory=list)
    operations: list[Operation] = field(default_factory=list)


@dataclass
class Function:
    name: str
    block: Block
    returns: list[Value]


@dataclass
class Module:
    functions: list[Function] = field(default_factory=list)


class IRBuilder:
    """Creates uniquely named SSA values inside one block."""

    def __init__(self, block: Block | None = None) -> None:
        self.block = block or Block()
        self._next = 0
        self._names: set[str] = set()

    def argument(self, type_: IRType, hint: str = "arg") -> Value:
        value = Value(self._unique(f"%{hint}"), type_)
        self.block.arguments.append(value)
        return value

    def emit(
        self,
        name: str,
        operands: Iterable[Value],
        result_types: Iterable[IRType],
        *,
        attributes: dict[str, Any] | None = None,
        effects: Iterable[Effect] = (),
    ) -> Operation:
        results = []
        for type_ in result_types:
            results.append(Value(self._unique(f"%v{self._next}"), type_))
            self._next += 1
        operation = Operation(
            name, list(operands), results, dict(attributes or {}), tuple(effects)
        )
        self.block.operations.append(operation)
        return operation

    def _unique(self, base: str) -> str:
        name, index = base, 1
        while name in self._names:
            name = f"{base}_{index}"
            index += 1
        self._names.add(name)
        return name


class VerificationError(ValueError):
    def __init__(self, errors: list[str]) -> None:
        super().__init__("\n".join(errors))
        self.errors = errors


# Op-name families: the high-level op and every KernelIR op it may become.
KV_OPS = {
    "serve.kv.init", "serve.kv.read", "serve.kv.append", "serve.kv.length",
    "serve.kv.store", "serve.kv.advance", "serve.kv.prefill_store",
    "serve.decode_attention",
}
LINEAR_OPS = {"serve.linear", "kernel.hip.linear", "kernel.rocm_compat.linear"}
ROPE_OPS = {"serve.rope", "kernel.hip.rope", "kernel.rocm_compat.rope"}
PREFILL_OPS = {
    "serve.prefill_attention", "kernel.hip.prefill_attention",
    "kernel.rocm_compat.prefill_attention",
}
DECODE_KERNEL_OPS = {"kernel.hip.decode_attention", "kernel.rocm_compat.decode_attention"}


def verify_module(module: Module) -> None:
    """Check SSA dominance and uniqueness and the per-op contracts."""

    errors: list[str] = []
    seen: set[str] = set()
    for function in module.functions:
        if function.name in seen:
            errors.append(f"function defined twice: @{function.name}")
        seen.add(function.name)
        _verify_function(function, errors)
    if errors:
        raise VerificationError(errors)


def _verify_function(function: Function, errors: list[str]) -> None:
    defined: set[int] = set()
    names: set[str] = set()
    for argument in function.block.arguments:
        if argument.name in names:
            errors.append(f"@{function.name}: duplicate argument {argument.name}")
        names.add(argument.name)
        defined.add(id(argument))
    for index, operation in enumerate(function.block.operations):
        for operand in operation.operands:
            if id(operand) not in defined:
                errors.append(
                    f"@{function.name} op {index} {operation.name} uses "
                    f"undefined value {operand.name}"
                )
        operand_names = {operand.name for operand in operation.operands}
        for reference in _ssa_references(operation.attributes):
            if reference not in operand_names:
                errors.append(
                    f"@{function.name} op {index} {operation.name}: attribute "
                    f"references non-operand {reference}"
                )
        for result in operation.results:
            if result.name in names:
                errors.append(f"@{function.name}: SSA name defined twice: {result.name}")
            names.add(result.name)
            defined.add(id(result))
        _verify_kv(operation, errors)
        _verify_linear(operation, errors)
        _verify_rope(operation, errors)
        _verify_prefill(operation, errors)
        if operation.name in DECODE_KERNEL_OPS:
            _verify_decode_attention(operation, errors)
    for value in function.returns:
        if id(value) not in defined:
            errors.append(f"@{function.name} returns undefined value {value.name}")


def _effects(operation: Operation) -> set[tuple[EffectKind, str]]:
    return {(effect.kind, effect.resource) for effect in operation.effects}


def _verify_kv(operation: Operation, errors: list[str]) -> None:
    """KV-op rules of the reference verifier (ir.py:282-460)."""

    name = operation.name
    if name not in KV_OPS:
        return
    if name == "serve.kv.init":
        _verify_kv_init(operation, errors)
        return
    if not operation.operands or not isinstance(operation.operands[0].type, KVStateType):
        errors.append(f"{name}: first operand must be a KVStateType")
        return
    state: KVStateType = operation.operands[0].type
    slot = operation.attributes.get("slot", 0)
    if not isinstance(slot, int) or not 0 <= slot < state.num_layers:
        errors.append(f"{name}: slot must be in [0, {state.num_layers})")
    effects = _effects(operation)
    if (EffectKind.READ, state.resource) not in effects:
        errors.append(f"{name}: missing read({state.resource}) effect")
    if name in {"serve.kv.append", "serve.kv.store", "serve.kv.advance",
                "serve.kv.prefill_store"} and (EffectKind.WRITE, state.resource) not in effects:
        errors.append(f"{name}: missing write({state.resource}) effect")
    same_state = len(operation.results) == 1 and operation.results[0].type == state
    if name == "serve.kv.append":
        if len(operation.operands) != 3:
            errors.append("serve.kv.append takes state, key and value")
        else:
            for operand in operation.operands[1:]:
                _verify_kv_tensor(operand.type, state, "serve.kv.append operand", errors)
        if not same_state:
            errors.append("serve.kv.append must return a new state of the same type")
    elif name == "serve.kv.read":
        if len(operation.results) != 2:
            errors.append("serve.kv.read returns key and value")
        else:
            for result in operation.results:
                _verify_kv_tensor(result.type, state, "serve.kv.read result", errors)
    elif name == "serve.kv.length":
        if len(operation.operands) != 1 or len(operation.results) != 1:
            errors.append("serve.kv.length takes one state and returns positions")
        elif not _is_positions(operation.results[0].type):
            errors.append("serve.kv.length must return a 1-D i64 tensor")
    elif name == "serve.kv.store":
        if len(operation.operands) != 4:
            errors.append("serve.kv.store takes state, key, value and positions")
        else:
            for operand in operation.operands[1:3]:
                _verify_kv_tensor(operand.type, state, "serve.kv.store operand", errors)
            if not _is_positions(operation.operands[3].type):
                errors.append("serve.kv.store positions must be a 1-D i64 tensor")
        if not same_state:
            errors.append("serve.kv.store must return an aliasing state of the same type")
    elif name == "serve.kv.advance":
        delta = operation.attributes.get("delta", 1)
        if not isinstance(delta, int) or delta <= 0:
            errors.append("serve.kv.advance delta must be a positive integer")
        if len(operation.operands) != 1:
            errors.append("serve.kv.advance takes one state")
        if not same_state:
            errors.append("serve.kv.advance must return a new state of the same type")
    elif name == "serve.kv.prefill_store":
        if len(operation.operands) != 3:
            errors.append("serve.kv.prefill_store takes state, key and value")
        else:
            for operand in operation.operands[1:]:
                _verify_kv_tensor(operand.type, state, "serve.kv.prefill_store operand", errors)
        if not same_state:
            errors.append("serve.kv.prefill_store must return a new state of the same type")
    elif name == "serve.decode_attention":
        _verify_decode_attention(operation, errors)


# KV layouts the runtime executes: the reference's contiguous buffers and the
# paged layout (page pools + block table) its bufferization plan names next
# (docs/kv-bufferization.md:317-323).
KV_LAYOUTS = ("contiguous_bshd", "paged")


def _verify_paging(state: KVStateType, context: str, errors: list[str]) -> None:
    if state.layout != "paged":
        if state.page_tokens is not None:
            errors.append(f"{context}: page_tokens only applies to the paged layout")
        return
    p = state.page_tokens
    if not isinstance(p, int) or p < 16 or p & (p - 1):
        errors.append(f"{context}: a paged state needs page_tokens, a power of two >= 16")
    elif state.capacity is not None and state.capacity % p:
        errors.append(f"{context}: the capacity must be a multiple of page_tokens")


def _verify_kv_init(operation: Operation, errors: list[str]) -> None:
    if len(operation.operands) != 1 or len(operation.results) != 1:
        errors.append("serve.kv.init takes a key template and returns one state")
        return
    state = operation.results[0].type
    if not isinstance(state, KVStateType):
        errors.append("serve.kv.init must return a KVStateType")
        return
    if state.layout not in KV_LAYOUTS or state.capacity is None:
        errors.append("serve.kv.init must create a contiguous_bshd or paged state with a capacity")
    _verify_paging(state, "serve.kv.init", errors)
    if operation.attributes.get("layout", "contiguous_bshd") != state.layout:
        errors.append("serve.kv.init layout does not match the state type")
    if operation.attributes.get("page_tokens") != state.page_tokens:
        errors.append("serve.kv.init page_tokens does not match the state type")
    _verify_kv_tensor(operation.operands[0].type, state, "serve.kv.init template", errors)
    if operation.attributes.get("num_layers") != state.num_layers:
        errors.append("serve.kv.init num_layers does not match the state type")
    if operation.attributes.get("capacity") != state.capacity:
        errors.append("serve.kv.init capacity does not match the state type")
    effects = _effects(operation)
    if (EffectKind.ALLOCATE, state.resource) not in effects:
        errors.append("serve.kv.init is missing its allocate effect")
    if (EffectKind.WRITE, state.resource) not in effects:
        errors.append("serve.kv.init is missing its write effect")


def _verify_kv_tensor(type_: IRType, state: KVStateType, context: str, errors: list[str]) -> None:
    if not isinstance(type_, TensorType) or len(type_.shape) != 4:
        errors.append(f"{context} must be a 4-D B x H x S x D tensor")
        return
    heads, head_dim = type_.shape[1], type_.shape[3]
    if not isinstance(heads, StaticDim) or heads.value != state.num_kv_heads:
        errors.append(f"{context} must have {state.num_kv_heads} KV heads")
    if not isinstance(head_dim, StaticDim) or head_dim.value != state.head_dim:
        errors.append(f"{context} must have head dim {state.head_dim}")
    if type_.dtype != state.dtype:
        errors.append(f"{context} must have dtype {state.dtype}")


def _is_positions(type_: IRType) -> bool:
    return isinstance(type_, TensorType) and len(type_.shape) == 1 and type_.dtype == "i64"


def _verify_linear(operation: Operation, errors: list[str]) -> None:
    """Linear rules (ir.py:463-548): N x K weight, optional N bias, static K/N."""

    if operation.name not in LINEAR_OPS:
        return
    name = operation.name
    if len(operation.operands) not in {2, 3} or len(operation.results) != 1:
        errors.append(f"{name} takes input, weight, optional bias and returns one tensor")
        return
    x, w, y = operation.operands[0].type, operation.operands[1].type, operation.results[0].type
    if not all(isinstance(t, TensorType) for t in (x, w, y)):
        errors.append(f"{name}: input, weight and result must be tensors")
        return
    if len(x.shape) not in {2, 3} or len(w.shape) != 2 or len(y.shape) != len(x.shape):
        errors.append(f"{name}: input must be 2-D/3-D, weight 2-D, result of input rank")
        return
    n, k = w.shape
    if x.shape[-1] != k:
        errors.append(f"{name}: input K must equal weight K")
    if y.shape[:-1] != x.shape[:-1] or y.shape[-1] != n:
        errors.append(f"{name}: result shape must be input leading dims x N")
    if not (x.dtype == w.dtype == y.dtype and x.device == w.device == y.device):
        errors.append(f"{name}: dtype and device must agree")
    has_bias = operation.attributes.get("has_bias")
    if has_bias is not (len(operation.operands) == 3):
        errors.append(f"{name}: has_bias does not match the operand count")
    if len(operation.operands) == 3:
        b = operation.operands[2].type
        if not isinstance(b, TensorType) or b.shape != (n,) or b.dtype != x.dtype:
            errors.append(f"{name}: bias must be a 1-D N tensor of the input dtype")
    for attribute, dimension in (("input_features", k), ("output_features", n)):
        if not isinstance(dimension, StaticDim) or operation.attributes.get(attribute) != dimension.value:
            errors.append(f"{name}: {attribute} attribute mismatch")


def _verify_rope(operation: Operation, errors: list[str]) -> None:
    """RoPE rules (ir.py:624-678): B x H x T x D q/k, B x T x D cos/sin."""

    if operation.name not in ROPE_OPS:
        return
    name = operation.name
    if len(operation.operands) != 4 or len(operation.results) != 2:
        errors.append(f"{name} takes query, key, cosine, sine and returns two tensors")
        return
    q, k, cos, sin = (o.type for o in operation.operands)
    rq, rk = (r.type for r in operation.results)
    if not all(isinstance(t, TensorType) for t in (q, k, cos, sin, rq, rk)):
        errors.append(f"{name}: operands and results must be tensors")
        return
    if len(q.shape) != 4 or len(k.shape) != 4 or len(cos.shape) != 3:
        errors.append(f"{name}: query/key must be 4-D and cosine/sine 3-D")
        return
    head_dim = q.shape[3]
    if not (q.shape[0] == k.shape[0] and q.shape[2:] == k.shape[2:]
            and cos.shape == (q.shape[0], q.shape[2], head_dim) and sin == cos):
        errors.append(f"{name}: batch, token or head-dim mismatch")
    if not (q.dtype == k.dtype == cos.dtype):
        errors.append(f"{name}: dtype mismatch")
    if rq != q or rk != k:
        errors.append(f"{name}: results must match query and key")
    if (not isinstance(head_dim, StaticDim) or head_dim.value % 2
            or operation.attributes.get("head_dim") != head_dim.value):
        errors.append(f"{name}: needs an even static head dim matching the attribute")
    if operation.attributes.get("variant") != "qwen2_half_rotation":
        errors.append(f"{name}: only the qwen2_half_rotation variant is supported")


def _verify_prefill(operation: Operation, errors: list[str]) -> None:
    """Prefill-attention rules (ir.py:551-621)."""

    if operation.name not in PREFILL_OPS:
        return
    name = operation.name
    if len(operation.operands) != 4 or len(operation.results) != 1:
        errors.append(f"{name} takes query, key, value, mask and returns context")
        return
    q, k, v, m = (o.type for o in operation.operands)
    ctx = operation.results[0].type
    if not all(isinstance(t, TensorType) and len(t.shape) == 4 for t in (q, k, v, m, ctx)):
        errors.append(f"{name}: all operands and the result must be 4-D tensors")
        return
    groups = operation.attributes.get("groups")
    qh, kvh = q.shape[1], k.shape[1]
    if (not isinstance(groups, int) or groups <= 0 or not isinstance(qh, StaticDim)
            or not isinstance(kvh, StaticDim) or qh.value != kvh.value * groups):
        errors.append(f"{name}: GQA groups do not match the head counts")
    if k != v:
        errors.append(f"{name}: key and value types must match")
    if not (q.shape[0] == k.shape[0] == m.shape[0] and q.shape[2] == k.shape[2]
            and q.shape[2] == m.shape[2] == m.shape[3] and q.shape[3] == k.shape[3]):
        errors.append(f"{name}: batch, token or head-dim mismatch")
    if not isinstance(m.shape[1], StaticDim) or m.shape[1].value != 1:
        errors.append(f"{name}: mask head dim must be 1")
    if ctx.dtype != q.dtype or ctx.shape[0] != q.shape[0] or ctx.shape[3] != q.shape[3]:
        errors.append(f"{name}: context must match the query dtype and shape")
    scale = operation.attributes.get("scale")
    if not isinstance(scale, (int, float)) or float(scale) <= 0:
        errors.append(f"{name}: scale must be positive")
    if operation.attributes.get("causal") not in {True, "mask"}:
        errors.append(f"{name}: causal must be True (kernel) or 'mask'")


def _verify_decode_attention(operation: Operation, errors: list[str]) -> None:
    """Decode-attention rules (ir.py:681-742)."""

    name = operation.name
    if len(operation.operands) != 3:
        errors.append(f"{name} takes state, query and mask")
        return
    state, q, m = (o.type for o in operation.operands)
    if not isinstance(state, KVStateType):
        return
    if state.layout not in KV_LAYOUTS:
        errors.append(f"{name}: only the contiguous_bshd and paged KV layouts are supported")
    _verify_paging(state, name, errors)
    if not isinstance(q, TensorType) or len(q.shape) != 4:
        errors.append(f"{name}: query must be 4-D")
        return
    if not isinstance(q.shape[2], StaticDim) or q.shape[2].value != 1:
        errors.append(f"{name}: query must be a single token")
    if not isinstance(m, TensorType) or len(m.shape) != 4:
        errors.append(f"{name}: mask must be 4-D")
    else:
        if not isinstance(m.shape[1], StaticDim) or m.shape[1].value != 1:
            errors.append(f"{name}: mask head dim must be 1")
        if not isinstance(m.shape[2], StaticDim) or m.shape[2].value != 1:
            errors.append(f"{name}: mask query dim must be 1")
        if m.shape[0] != q.shape[0]:
            errors.append(f"{name}: mask batch does not match the query")
    groups = operation.attributes.get("groups")
    if not isinstance(groups, int) or groups <= 0:
        errors.append(f"{name}: groups must be a positive integer")
    elif isinstance(q.shape[1], StaticDim) and q.shape[1].value != state.num_kv_heads * groups:
        errors.append(f"{name}: query heads must equal KV heads x groups")
    if isinstance(q.shape[3], StaticDim) and q.shape[3].value != state.head_dim:
        errors.append(f"{name}: head dim does not match the KV state")
    scale = operation.attributes.get("scale")
    if not isinstance(scale, (int, float)) or float(scale) <= 0:
        errors.append(f"{name}: scale must be positive")
    if len(operation.results) != 1 or operation.results[0].type != q:
        errors.append(f"{name}: result must have the query's type")


def _ssa_references(value: Any) -> list[str]:
    if isinstance(value, dict):
        if set(value) == {"ssa"} and isinstance(value["ssa"], str):
            return [value["ssa"]]
        out: list[str] = []
        for item in value.values():
            out.extend(_ssa_references(item))
        return out
    if isinstance(value, (list, tuple)):
        out = []
        for item in value:
            out.extend(_ssa_references(item))
        return out
    return []


def format_module(module: Module) -> str:
    """MLIR-like text of a module (for snapshots and debugging)."""

    lines = ["module {"]
    for function in module.functions:
        args = ", ".join(f"{a.name}: {a.type}" for a in function.block.arguments)
        rets = ", ".join(str(v.type) for v in function.returns)
        lines.append(f"  func @{function.name}({args}) -> ({rets}) {{")
        for operation in function.block.operations:
            results = ", ".join(r.name for r in operation.results)
            assign = f"{results} = " if results else ""
            operands = ", ".join(o.name for o in operation.operands)
            attrs = (
                " " + json.dumps(operation.attributes, sort_keys=True, separators=(",", ":"), default=str)
                if operation.attributes else ""
            )
            effects = (
                " effects[" + ", ".join(str(e) for e in operation.effects) + "]"
                if operation.effects else ""
            )
            in_types = ", ".join(str(o.type) for o in operation.operands)
            out_types = ", ".join(str(r.type) for r in operation.results)
            lines.append(
                f'    {assign}"{operation.name}"({operands}){attrs}{effects} : ({in_types}) -> ({out_types})'
            )
        lines.append("    return " + ", ".join(v.name for v in function.returns))
        lines.append("  }")
    lines.append("}")
    return "\n".join(lines)
