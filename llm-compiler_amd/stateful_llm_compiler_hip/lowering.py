"""ServeIR -> KernelIR lowering for the gfx950 backend, and coverage checks.

Same entry points and contract as the reference's lowering layer
(src/stateful_llm_compiler/lowering.py:19-208): ``LowerToKernelIRPass``
renames every supported ServeIR op to an explicit backend op and records
``lowered_from`` / ``numerical_mode`` / ``backend_selection``;
``analyze_lowering_coverage`` counts what is left to eager execution and
``require_full_lowering`` raises ``LoweringCoverageError`` when anything is.
The lowering itself never touches a device.

Backend op families:
  kernel.hip.*         hand-written gfx950 kernels (libslc_hip.so)
  kernel.rocm_compat.* PyTorch-ROCm composites that keep PyTorch eager's
                       bf16 rounding boundaries (the ``pytorch_compatible``
                       mode, as the reference's kernel.cuda.* / cublas ops)
  kernel.metadata.*    zero-copy views (no device work)
  runtime.kv.*         KV runtime-state operations
"""

from __future__ import annotations

from collections import Counter
from dataclasses import asdict, dataclass

from .ir import Module, Operation
from .pass_manager import CompilerPass, PassResult

NUMERICAL_MODES = ("fast", "pytorch_compatible")

_KERNEL_LOWERINGS = {
    "serve.kv.store": "kernel.hip.kv_store",
    "serve.kv.prefill_store": "kernel.hip.kv_prefill_store",
    # Ops the reference leaves to eager PyTorch; fused ServeIR forms of the
    # Qwen2 embedding, residual add, SwiGLU and RoPE table.
    "serve.embedding": "kernel.hip.embedding",
    "serve.add": "kernel.hip.add",
    "serve.swiglu": "kernel.hip.swiglu",
    "serve.rope_table": "kernel.hip.rope_table",
}

_NUMERICAL_LOWERINGS = {
    "fast": {
        "serve.rms_norm": "kernel.hip.rms_norm",
        "serve.prefill_attention": "kernel.hip.prefill_attention",
        "serve.rope": "kernel.hip.rope",
        "serve.decode_attention": "kernel.hip.decode_attention",
    },
    "pytorch_compatible": {
        "serve.rms_norm": "kernel.rocm_compat.rms_norm",
        "serve.prefill_attention": "kernel.rocm_compat.prefill_attention",
        # The HIP RoPE kernel rounds each product before the add exactly as
        # the eager composite does, so it is already element-wise exact.
        "serve.rope": "kernel.hip.rope",
        "serve.decode_attention": "kernel.rocm_compat.decode_attention",
        # cos/sin and SiLU go through PyTorch's own transcendental kernels so
        # their last bit matches the eager model.
        "serve.rope_table": "kernel.rocm_compat.rope_table",
        "serve.swiglu": "kernel.rocm_compat.swiglu",
    },
}

_RUNTIME_LOWERINGS = {
    "serve.kv.init": "runtime.kv.init",
    "serve.kv.length": "runtime.kv.length",
    "serve.kv.advance": "runtime.kv.advance",
}

_METADATA_LOWERINGS = {
    "aten.view.default": "kernel.metadata.view",
    "aten.reshape.default": "kernel.metadata.reshape",
    "aten.transpose.int": "kernel.metadata.transpose",
    "aten.unsqueeze.default": "kernel.metadata.unsqueeze",
    "builtin.getitem": "kernel.metadata.getitem",
}

_LINEAR_TARGETS = {"fast": "kernel.hip.linear", "pytorch_compatible": "kernel.rocm_compat.linear"}

# Softmax orders of the HIP attention kernels: "exact" normalises the
# probabilities before rounding them for P.V, as the reference executor does
# (execution.py:319-327, 720-739) -- the default, since it keeps bf16 fast
# mode within the logits tolerance; "online" is the single-pass form of the
# reference's Triton kernels (triton_attention.py:103-119).
SOFTMAX_ORDERS = ("exact", "online")
_ATTENTION_KERNELS = frozenset({"kernel.hip.decode_attention", "kernel.hip.prefill_attention"})

# Decode-step fusions (passes/fusion.py) of the ops above.
_FUSED_OPERATIONS = frozenset({
    "kernel.hip.norm_linear_group",
    "kernel.hip.norm_linear_swiglu",
    "kernel.hip.linear_residual",
    "kernel.hip.rope_kv_store",
    "kernel.hip.rope_store_attention",
})

EXECUTABLE_OPERATIONS = (
    _FUSED_OPERATIONS
    | frozenset(_KERNEL_LOWERINGS.values())
    | frozenset(_RUNTIME_LOWERINGS.values())
    | frozenset(_METADATA_LOWERINGS.values())
    | frozenset(_LINEAR_TARGETS.values())
    | frozenset(t for table in _NUMERICAL_LOWERINGS.values() for t in table.values())
)


@dataclass(frozen=True)
class LoweringCoverage:
    """How far a graph is from zero eager fallback."""

    total_operations: int
    lowered_operations: int
    unlowered_operations: int
    coverage: float
    lowered_by_name: dict[str, int]
    unlowered_by_name: dict[str, int]

    @property
    def is_complete(self) -> bool:
        return self.unlowered_operations == 0

    def to_dict(self) -> dict[str, object]:
        return asdict(self)


class LoweringCoverageError(RuntimeError):
    """Strict compilation found operations that were not lowered."""

    def __init__(self, coverage: LoweringCoverage) -> None:
        self.coverage = coverage
        details = ", ".join(f"{name}x{count}" for name, count in coverage.unlowered_by_name.items())
        super().__init__(
            "KernelIR is not fully lowered: "
            f"{coverage.unlowered_operations}/{coverage.total_operations} "
            f"operations remain ({details})"
        )


class LowerToKernelIRPass(CompilerPass):
    """Rewrite supported ServeIR ops into explicit kernel / runtime ops."""

    name = "lower-to-kernel-ir"

    def __init__(self, *, numerical_mode: str = "fast", attention_softmax: str = "exact",
                 linear_backend: str | None = None) -> None:
        if numerical_mode not in _NUMERICAL_LOWERINGS:
            raise ValueError(
                f"unsupported numerical mode {numerical_mode}; choose one of "
                + ", ".join(sorted(_NUMERICAL_LOWERINGS))
            )
        if attention_softmax not in SOFTMAX_ORDERS:
            raise ValueError(f"attention_softmax must be one of {SOFTMAX_ORDERS}, got {attention_softmax!r}")
        if linear_backend is not None and linear_backend not in _LINEAR_TARGETS:
            raise ValueError(f"linear_backend must be one of {sorted(_LINEAR_TARGETS)}")
        self.numerical_mode = numerical_mode
        self.attention_softmax = attention_softmax
        # The GEMM family may be chosen apart from the mode (a fast-mode graph
        # with the library GEMMs isolates the hand-written GEMM's rounding).
        self.linear_backend = linear_backend or numerical_mode

    def run(self, module: Module) -> PassResult:
        lowered = Counter()
        for function in module.functions:
            for operation in function.block.operations:
                source = operation.name
                if source == "serve.linear":
                    target = _select_linear_backend(operation, self.linear_backend)
                else:
                    target = _NUMERICAL_LOWERINGS[self.numerical_mode].get(source)
                    if target is None:
                        target = (
                            _KERNEL_LOWERINGS.get(source)
                            or _RUNTIME_LOWERINGS.get(source)
                            or _METADATA_LOWERINGS.get(source)
                        )
                if target is None:
                    continue
                operation.name = target
                operation.attributes["lowered_from"] = source
                if source in _NUMERICAL_LOWERINGS["fast"]:
                    operation.attributes["numerical_mode"] = self.numerical_mode
                if target in _ATTENTION_KERNELS:
                    operation.attributes["softmax_order"] = self.attention_softmax
                lowered[f"{source}->{target}"] += 1
        coverage = analyze_lowering_coverage(module)
        return PassResult(
            name=self.name,
            changed=bool(lowered),
            statistics={
                "lowered": sum(lowered.values()),
                "lowered_rules": dict(sorted(lowered.items())),
                "coverage": coverage.to_dict(),
            },
        )


def _select_linear_backend(operation: Operation, numerical_mode: str) -> str:
    """fast: the gfx950 MFMA GEMM for every shape (it picks its tile from M at
    run time); pytorch_compatible: PyTorch's ROCm BLAS call, whose rounding the
    eager model shares (the reference routes compat mode to kernel.cublas.linear,
    lowering.py:155-171)."""

    if numerical_mode == "pytorch_compatible":
        operation.attributes["backend_selection"] = "pytorch_compatible"
    else:
        k = operation.attributes.get("input_features")
        n = operation.attributes.get("output_features")
        large = isinstance(k, int) and isinstance(n, int) and max(k, n) >= 4096
        operation.attributes["backend_selection"] = (
            "hip_mfma_large_static_gemm" if large else "hip_mfma_small_static_gemm"
        )
    return _LINEAR_TARGETS[numerical_mode]


def analyze_lowering_coverage(module: Module) -> LoweringCoverage:
    lowered = Counter()
    unlowered = Counter()
    for function in module.functions:
        for operation in function.block.operations:
            (lowered if operation.name in EXECUTABLE_OPERATIONS else unlowered)[operation.name] += 1
    n_low = sum(lowered.values())
    n_un = sum(unlowered.values())
    total = n_low + n_un
    return LoweringCoverage(
        total_operations=total,
        lowered_operations=n_low,
        unlowered_operations=n_un,
        coverage=1.0 if total == 0 else n_low / total,
        lowered_by_name=dict(sorted(lowered.items())),
        unlowered_by_name=dict(sorted(unlowered.items())),
    )


def require_full_lowering(module: Module) -> LoweringCoverage:
    """Refuse a graph that still contains eager (unlowered) operations."""

    coverage = analyze_lowering_coverage(module)
    if not coverage.is_complete:
        raise LoweringCoverageError(coverage)
    return coverage
