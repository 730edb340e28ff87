"""Attach profile plans of kernel variants to ServeIR ops.

``SelectRMSNormLoweringPass`` keeps the reference pass's name, its
``lowering_plan`` attribute on ``serve.rms_norm`` and its statistics keys
(src/stateful_llm_compiler/passes/lowering_selection.py:12-72); what the plan
chooses is a HIP kernel variant (``cost_model``).  ``SelectDecodeSplitPass``
does the same for the split of ``serve.decode_attention`` (``split_plan``)
and ``SelectLinearTilePass`` for the GEMM tile of ``serve.linear``
(``tile_plan``).
"""

from __future__ import annotations

from collections import Counter
from typing import Any

from ..cost_model import KernelProfile, ProfileError
from ..ir import Module, Operation, StaticDim, TensorType
from ..pass_manager import CompilerPass, PassResult


def _static_dims(value_type, *axes: int) -> list[int] | None:
    """The static sizes of ``axes`` of a tensor type (None if any is dynamic)."""

    if not isinstance(value_type, TensorType) or not value_type.shape:
        return None
    try:
        picked = [value_type.shape[axis] for axis in axes]
    except IndexError:
        return None
    if not all(isinstance(dim, StaticDim) for dim in picked):
        return None
    return [dim.value for dim in picked]


class _PlanPass(CompilerPass):
    op_name = ""
    attribute = ""

    def __init__(self, profile: KernelProfile) -> None:
        self.profile = profile

    def static_key(self, operation: Operation) -> dict[str, Any] | None:
        raise NotImplementedError

    def run(self, module: Module) -> PassResult:
        planned = missing = 0
        variants: Counter[str] = Counter()
        changed = False
        for function in module.functions:
            for operation in function.block.operations:
                if operation.name != self.op_name:
                    continue
                try:
                    key = self.static_key(operation)
                except ProfileError:
                    key = None
                plan = None if key is None else self.profile.plan(self.plan_op, **key)
                if plan is None:
                    missing += 1
                    continue
                planned += 1
                for sample in plan["samples"]:
                    variants.update(sample["latency_us"])
                if operation.attributes.get(self.attribute) != plan:
                    operation.attributes[self.attribute] = plan
                    changed = True
        return PassResult(self.name, changed, {
            "planned_operations": planned,
            "missing_profile": missing,
            "variant_backends": dict(sorted(variants.items())),
        })


class SelectRMSNormLoweringPass(_PlanPass):
    name = "select-rmsnorm-lowering"
    op_name = "serve.rms_norm"
    plan_op = "rms_norm"
    attribute = "lowering_plan"

    def static_key(self, operation: Operation) -> dict[str, Any] | None:
        hidden = _static_dims(operation.operands[0].type, -1)
        if hidden is None:
            return None
        dtype = operation.attributes.get("output_dtype") or operation.operands[0].type.dtype
        return {"hidden_size": hidden[0], "dtype": dtype}


class SelectDecodeSplitPass(_PlanPass):
    name = "select-decode-attention-split"
    op_name = "serve.decode_attention"
    plan_op = "decode_attention"
    attribute = "split_plan"

    def static_key(self, operation: Operation) -> dict[str, Any] | None:
        if len(operation.operands) < 2:
            return None
        query_type = operation.operands[1].type  # [B, QH, 1, D]
        dims = _static_dims(query_type, 1, 3) if len(getattr(query_type, "shape", ())) == 4 else None
        groups = int(operation.attributes.get("groups", 0))
        if dims is None or groups <= 0 or dims[0] % groups:
            return None
        return {"q_heads": dims[0], "kv_heads": dims[0] // groups, "head_dim": dims[1],
                "dtype": query_type.dtype}


class SelectLinearTilePass(_PlanPass):
    name = "select-linear-tile"
    op_name = "serve.linear"
    plan_op = "linear"
    attribute = "tile_plan"

    def static_key(self, operation: Operation) -> dict[str, Any] | None:
        if len(operation.operands) < 2:
            return None
        dims = _static_dims(operation.operands[1].type, 0, 1)  # weight [N, K]
        if dims is None:
            return None
        return {"out_features": dims[0], "in_features": dims[1],
                "dtype": operation.operands[0].type.dtype}
