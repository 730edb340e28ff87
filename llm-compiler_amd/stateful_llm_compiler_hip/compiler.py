"""Compile entry point: ServeIR module -> verified, lowered KernelIR.

Mirrors the reference's ``compile_exported_program`` / ``CompileOptions``
(src/stateful_llm_compiler/compiler.py:25-79) for graphs that already are
ServeIR: optional profile-guided plans of kernel variants (RMSNorm launch
width, decode-attention split, GEMM tile), the KernelIR lowering in the chosen numerical
mode, and ``require_full_lowering`` when strict.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

from .cost_model import KernelProfile
from .ir import Module
from .lowering import LoweringCoverage, LowerToKernelIRPass, analyze_lowering_coverage, require_full_lowering
from .pass_manager import PassManager, PassResult, operation_counts
from .passes import (FuseDecodeKernelsPass, SelectDecodeSplitPass, SelectLinearTilePass,
                     SelectRMSNormLoweringPass)


@dataclass(frozen=True)
class CompileOptions:
    numerical_mode: str = "fast"
    require_full_lowering: bool = True
    # Schema-v1 profile (the reference's option name): its RMSNorm rows plan
    # serve.rms_norm, its decode_attention and linear rows (extensions) the
    # attention split and the GEMM tile.
    rmsnorm_profile: str | Path | None = None
    # Fuse decode-step op chains into single kernels (fast mode only; the
    # fused kernels are bit-identical to the chains they replace).
    fuse: bool = True
    # Softmax order of the HIP attention kernels in fast mode ("exact" or
    # "online"; see lowering.SOFTMAX_ORDERS).
    attention_softmax: str = "exact"
    # GEMM family: None follows the numerical mode; "pytorch_compatible" in
    # fast mode runs the linears on PyTorch's ROCm BLAS call.
    linear_backend: str | None = None


@dataclass
class CompileResult:
    module: Module
    passes: list[PassResult]
    coverage: LoweringCoverage
    operation_counts: dict[str, int] = field(default_factory=dict)

    def statistics(self) -> dict[str, Any]:
        return {
            "passes": [{"name": r.name, "changed": r.changed, **r.statistics} for r in self.passes],
            "coverage": self.coverage.to_dict(),
            "operation_counts": self.operation_counts,
        }


def compile_module(module: Module, options: CompileOptions | None = None) -> CompileResult:
    """Lower ``module`` in place and return it with pass statistics."""

    options = options or CompileOptions()
    manager = PassManager()
    if options.rmsnorm_profile is not None:
        profile = KernelProfile.load(options.rmsnorm_profile)
        manager.add(SelectRMSNormLoweringPass(profile))
        manager.add(SelectDecodeSplitPass(profile))
        manager.add(SelectLinearTilePass(profile))
    manager.add(LowerToKernelIRPass(numerical_mode=options.numerical_mode,
                                    attention_softmax=options.attention_softmax,
                                    linear_backend=options.linear_backend))
    if options.fuse and options.numerical_mode == "fast":
        manager.add(FuseDecodeKernelsPass())
    results = manager.run(module)
    coverage = require_full_lowering(module) if options.require_full_lowering else analyze_lowering_coverage(module)
    return CompileResult(module, results, coverage, operation_counts(module))
