"""Profile-guided choice of gfx950 kernel variants.

The reference plans ``serve.rms_norm`` from a schema-v1 profile of measured
latencies (src/stateful_llm_compiler/cost_model.py:93-123 reads the format,
benchmarks/bench_rmsnorm.py:183-208 writes it) and picks a *backend*
(native / triton / inductor) per row bucket.  None of those backends exists
here: every op runs a hand-written HIP kernel.  What does vary is which HIP
kernel an op launches, so this module plans *variants*:

* ``rms_norm``: ``wave`` (one wavefront per row, the row held in registers)
  or ``block`` (a 256-thread workgroup per row); the run-time axis is the row
  count.
* ``decode_attention``: ``fixed`` (a fixed chunk per (batch, kv head), sized
  to fill the GPU), ``balanced`` (the length-balanced split) or ``chunk<N>``
  (a fixed chunk of N tokens); the run-time axis is batch x mask length.
* ``linear``: the workgroup tile of the prefill-sized MFMA GEMM
  (``t128x128``, ``t128x64``, ``t64x128``, ``t64x64``, ``t32x64``; all give
  the same bits); static key (out_features, in_features, dtype), run-time
  axis the row count M.

A profile keeps the schema-v1 layout -- ``schema_version``, ``target`` and a
``results`` list of RMSNorm rows keyed ``rows`` / ``hidden_size`` / ``dtype``,
so a reference profile loads unchanged -- and adds per-row ``hip_variants``
(variant -> microseconds) plus ``decode_attention`` and ``linear`` lists of
the same form.
A reference row without ``hip_variants`` contributes its ``hip_us`` (if any)
as the automatic variant and nothing else.

A plan is the op's measured samples, attached to the op as an attribute.  At
run time every variant's latency is interpolated linearly in log(size)
between the two samples around the actual size (outside the sampled range the
end sample stands), and the call launches the variant with the lowest
estimate.  Ties go to the variant listed first in ``VARIANTS``.
"""

from __future__ import annotations

import json
import math
import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Mapping

SCHEMA_VERSION = 1

# Variants each op can launch, in tie-break order; "auto" lets the kernel
# library decide (a reference row's hip_us stands for it).
VARIANTS: dict[str, tuple[str, ...]] = {
    "rms_norm": ("auto", "wave", "block"),
    "decode_attention": ("auto", "fixed", "balanced"),
    "linear": ("auto", "t128x128", "t128x64", "t64x128", "t64x64", "t32x64",
               "r128x128", "r256x128", "r128x64", "r64x64", "s256x128"),
}
_CHUNK = re.compile(r"chunk(\d+)$")

_DTYPES = {"f16": "fp16", "float16": "fp16", "fp16": "fp16", "half": "fp16",
           "bf16": "bf16", "bfloat16": "bf16", "f32": "fp32", "float32": "fp32",
           "fp32": "fp32", "float": "fp32"}


class ProfileError(ValueError):
    """A profile or plan that cannot be used."""


def canonical_dtype(dtype: Any) -> str:
    name = str(dtype).rsplit(".", 1)[-1].lower()
    if name not in _DTYPES:
        raise ProfileError(f"unsupported dtype {dtype!r}")
    return _DTYPES[name]


def _known_variant(op: str, variant: str) -> bool:
    return variant in VARIANTS[op] or (op == "decode_attention" and _CHUNK.match(variant) is not None)


@dataclass(frozen=True)
class VariantChoice:
    """What a call launches and why."""

    variant: str
    source: str                     # "profile" or "default"
    size: int
    estimated_us: float | None = None


@dataclass
class VariantCurve:
    """Measured latencies of one op's variants at a few sizes of its run-time
    axis, for one static configuration.  Samples of equal size (for decode
    attention: different batch / length splits of the same work) average."""

    op: str
    static: tuple[tuple[str, Any], ...]
    axis: str
    samples: dict[int, dict[str, list[float]]] = field(default_factory=dict)
    _seen: set = field(default_factory=set)

    def add(self, size: int, latencies: Mapping[str, float], *, key: Any = None) -> None:
        if size <= 0:
            raise ProfileError(f"{self.op}: sample size must be positive, got {size}")
        key = size if key is None else key
        if key in self._seen:
            raise ProfileError(f"{self.op} {dict(self.static)}: two samples of {key}")
        self._seen.add(key)
        for variant, value in latencies.items():
            if not _known_variant(self.op, variant):
                raise ProfileError(f"{self.op}: unknown variant {variant!r}")
            value = float(value)
            if not math.isfinite(value) or value <= 0:
                raise ProfileError(f"{self.op}: latency of {variant} must be finite and positive")
            self.samples.setdefault(size, {}).setdefault(variant, []).append(value)

    def to_plan(self, source: str, target: Mapping[str, Any]) -> dict[str, Any]:
        return {
            "schema_version": SCHEMA_VERSION,
            "op": self.op,
            "axis": self.axis,
            "static": dict(self.static),
            "profile_source": source,
            "target": dict(target),
            "samples": [{"size": size,
                         "latency_us": {v: sum(xs) / len(xs) for v, xs in self.samples[size].items()}}
                        for size in sorted(self.samples)],
        }


def _estimate(points: list[tuple[float, float]], x: float) -> float:
    """Piecewise-linear value at x of points sorted by their first element;
    flat beyond the ends."""

    if x <= points[0][0]:
        return points[0][1]
    for (x0, y0), (x1, y1) in zip(points, points[1:]):
        if x <= x1:
            return y0 + (y1 - y0) * (x - x0) / (x1 - x0)
    return points[-1][1]


def choose_variant(plan: Mapping[str, Any] | None, size: int, *,
                   allowed: tuple[str, ...] | None = None) -> VariantChoice:
    """The variant with the lowest interpolated latency at ``size``."""

    if size <= 0:
        raise ProfileError("run-time size must be positive")
    if not plan:
        return VariantChoice("auto", "default", size)
    op = plan.get("op")
    if op not in VARIANTS:
        raise ProfileError(f"plan for unknown op {op!r}")
    curves: dict[str, list[tuple[float, float]]] = {}
    for sample in plan.get("samples", []):
        x = math.log(float(sample["size"]))
        for variant, value in sample["latency_us"].items():
            if allowed is None or variant in allowed:
                curves.setdefault(variant, []).append((x, float(value)))
    if not curves:
        return VariantChoice("auto", "default", size)
    x = math.log(float(size))
    order = {name: i for i, name in enumerate(VARIANTS[op])}
    best = min(
        ((name, _estimate(sorted(points), x)) for name, points in curves.items()),
        key=lambda item: (item[1], order.get(item[0], len(order)), item[0]),
    )
    return VariantChoice(best[0], "profile", size, best[1])


def linear_tile(variant: str) -> str:
    """linear variant -> the tile name hip_linear takes (SLC_TILE_*)."""

    if variant not in VARIANTS["linear"]:
        raise ProfileError(f"not a linear tile variant: {variant!r}")
    return variant


def waves_per_row(variant: str) -> int:
    """rms_norm variant -> the waves_per_row argument of slc_hip_rms_norm."""

    return {"auto": 0, "wave": 1, "block": 4}[variant]


def split_tokens(variant: str) -> int:
    """decode_attention variant -> the split_tokens argument of
    slc_hip_decode_attention (SLC_SPLIT_BALANCED is -1)."""

    if variant in ("auto", "fixed"):
        return 0
    if variant == "balanced":
        return -1
    match = _CHUNK.match(variant)
    if match is None:
        raise ProfileError(f"not a decode attention variant: {variant!r}")
    return int(match.group(1))


class KernelProfile:
    """A loaded schema-v1 profile: variant curves per (op, static key)."""

    def __init__(self, target: Mapping[str, Any], curves: list[VariantCurve], *,
                 source: str = "memory") -> None:
        self.target = dict(target)
        self.source = source
        self.curves = {(curve.op, curve.static): curve for curve in curves}

    @classmethod
    def load(cls, path: str | Path) -> "KernelProfile":
        path = Path(path)
        try:
            payload = json.loads(path.read_text(encoding="utf-8"))
        except (OSError, json.JSONDecodeError) as error:
            raise ProfileError(f"cannot read profile {path}: {error}") from error
        return cls.from_dict(payload, source=str(path))

    @classmethod
    def from_dict(cls, payload: Any, *, source: str = "memory") -> "KernelProfile":
        if isinstance(payload, list):  # early profiles: the results list alone
            payload = {"schema_version": SCHEMA_VERSION, "results": payload}
        if not isinstance(payload, dict) or payload.get("schema_version") != SCHEMA_VERSION:
            raise ProfileError("a profile must be a schema_version 1 object")
        curves: dict[tuple[str, tuple], VariantCurve] = {}

        def curve(op, static, axis):
            key = (op, static)
            if key not in curves:
                curves[key] = VariantCurve(op, static, axis)
            return curves[key]

        for row in payload.get("results", []) or []:
            try:
                static = (("hidden_size", int(row["hidden_size"])),
                          ("dtype", canonical_dtype(row["dtype"])))
                size = int(row["rows"])
            except (KeyError, TypeError, ValueError) as error:
                raise ProfileError(f"illegal rms_norm row {row!r}") from error
            latencies = dict(row.get("hip_variants") or {})
            if not latencies and row.get("hip_us") is not None:
                latencies = {"auto": row["hip_us"]}
            curve("rms_norm", static, "rows").add(size, latencies)
        for row in payload.get("decode_attention", []) or []:
            try:
                static = (("q_heads", int(row["q_heads"])), ("kv_heads", int(row["kv_heads"])),
                          ("head_dim", int(row["head_dim"])), ("dtype", canonical_dtype(row["dtype"])))
                size = int(row["batch"]) * int(row["mask_len"])
            except (KeyError, TypeError, ValueError) as error:
                raise ProfileError(f"illegal decode_attention row {row!r}") from error
            curve("decode_attention", static, "batch*mask_len").add(
                size, row.get("hip_variants") or {}, key=(int(row["batch"]), int(row["mask_len"])))
        for row in payload.get("linear", []) or []:
            try:
                static = (("out_features", int(row["out_features"])),
                          ("in_features", int(row["in_features"])),
                          ("dtype", canonical_dtype(row["dtype"])))
                size = int(row["rows"])
            except (KeyError, TypeError, ValueError) as error:
                raise ProfileError(f"illegal linear row {row!r}") from error
            curve("linear", static, "rows").add(size, row.get("hip_variants") or {})
        return cls(payload.get("target") or {}, [c for c in curves.values() if c.samples],
                   source=source)

    def plan(self, op: str, **static: Any) -> dict[str, Any] | None:
        """The plan attribute of ``op`` at a static configuration, or None
        when the profile has no samples for it."""

        if "dtype" in static:
            static["dtype"] = canonical_dtype(static["dtype"])
        keys = {"rms_norm": ("hidden_size", "dtype"),
                "decode_attention": ("q_heads", "kv_heads", "head_dim", "dtype"),
                "linear": ("out_features", "in_features", "dtype")}[op]
        curve = self.curves.get((op, tuple((k, static[k]) for k in keys)))
        return None if curve is None else curve.to_plan(self.source, self.target)
