"""Attach profile-derived lowering plans to ``serve.rms_norm`` ops.

Restates the reference's SelectRMSNormLoweringPass
(src/stateful_llm_compiler/passes/lowering_selection.py:12-72).
"""

from __future__ import annotations

from collections import Counter

from ..cost_model import RMSNormCostModel
from ..ir import Module, StaticDim, TensorType
from ..pass_manager import CompilerPass, PassResult


class SelectRMSNormLoweringPass(CompilerPass):
    name = "select-rmsnorm-lowering"

    def __init__(self, cost_model: RMSNormCostModel, *, fallback: str = "hip") -> None:
        self.cost_model = cost_model
        self.fallback = fallback

    def run(self, module: Module) -> PassResult:
        planned = missing = 0
        backends: Counter[str] = Counter()
        changed = False
        for function in module.functions:
            for operation in function.block.operations:
                if operation.name != "serve.rms_norm":
                    continue
                input_type = operation.operands[0].type
                if (not isinstance(input_type, TensorType) or not input_type.shape
                        or not isinstance(input_type.shape[-1], StaticDim)):
                    missing += 1
                    continue
                dtype = operation.attributes.get("output_dtype", input_type.dtype)
                plan = self.cost_model.plan_attribute(
                    input_type.shape[-1].value, dtype, fallback=self.fallback
                )
                if plan["variants"]:
                    planned += 1
                    backends.update(v["backend"] for v in plan["variants"])
                else:
                    missing += 1
                if operation.attributes.get("lowering_plan") != plan:
                    operation.attributes["lowering_plan"] = plan
                    changed = True
        return PassResult(self.name, changed, {
            "planned_operations": planned,
            "missing_profile": missing,
            "variant_backends": dict(sorted(backends.items())),
        })
