"""Profile-guided lowering plans for ``serve.rms_norm``.

Restates the reference's cost model (src/stateful_llm_compiler/cost_model.py:
1-324): a schema-v1 profile of measured latencies per (rows, hidden, dtype)
becomes row buckets split at the geometric midpoints of neighbouring
measurements; each bucket picks its cheapest backend; at run time
``resolve_lowering_plan`` maps the actual row count to a decision.  The gfx950
backend adds the ``hip`` backend name; profiles measured on MI355X list it
next to (or instead of) the reference's names.
"""

from __future__ import annotations

import json
import math
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Any, Iterable

BACKENDS = ("hip", "triton", "inductor", "native")


class ProfileError(ValueError):
    pass


@dataclass(frozen=True)
class TargetProfile:
    device_name: str = "unknown"
    compute_capability: str = "unknown"
    torch_version: str = "unknown"
    triton_version: str = "unknown"


@dataclass(frozen=True)
class RMSNormProfileEntry:
    rows: int
    hidden_size: int
    dtype: str
    native_us: float
    triton_us: float | None = None
    inductor_us: float | None = None
    hip_us: float | None = None

    def backend_costs(self) -> dict[str, float]:
        costs = {"native": self.native_us}
        for name, value in (("triton", self.triton_us), ("inductor", self.inductor_us),
                            ("hip", self.hip_us)):
            if value is not None:
                costs[name] = value
        return costs


@dataclass(frozen=True)
class LoweringVariant:
    min_rows: int
    max_rows: int | None
    profile_rows: int
    backend: str
    estimated_us: float
    num_warps: int | None = None

    def contains(self, rows: int) -> bool:
        return rows >= self.min_rows and (self.max_rows is None or rows <= self.max_rows)


@dataclass(frozen=True)
class LoweringDecision:
    backend: str
    source: str
    profile_rows: int | None = None
    estimated_us: float | None = None
    num_warps: int | None = None


class RMSNormCostModel:
    """Row-bucketed lowering plans built from discrete measurements."""

    def __init__(self, target: TargetProfile, entries: Iterable[RMSNormProfileEntry], *,
                 source: str = "memory") -> None:
        self.target = target
        self.entries = tuple(entries)
        self.source = source
        if not self.entries:
            raise ProfileError("a profile needs at least one measurement")
        _validate_entries(self.entries)

    @classmethod
    def load(cls, path: str | Path) -> "RMSNormCostModel":
        path = Path(path)
        return cls.from_dict(json.loads(path.read_text(encoding="utf-8")), source=str(path))

    @classmethod
    def from_dict(cls, payload: Any, *, source: str = "memory") -> "RMSNormCostModel":
        if isinstance(payload, list):  # legacy: bare list of rows
            target_data: dict[str, Any] = {}
            rows = payload
        elif isinstance(payload, dict):
            if payload.get("schema_version") != 1:
                raise ProfileError("unsupported profile schema_version")
            target_data = payload.get("target", {})
            rows = payload.get("results", [])
        else:
            raise ProfileError("a profile must be an object or a list")
        target = TargetProfile(
            device_name=str(target_data.get("device_name", "unknown")),
            compute_capability=str(target_data.get("compute_capability", "unknown")),
            torch_version=str(target_data.get("torch_version", "unknown")),
            triton_version=str(target_data.get("triton_version", "unknown")),
        )
        return cls(target, [_parse_entry(row) for row in rows], source=source)

    def variants(self, hidden_size: int, dtype: str, *,
                 allowed_backends: Iterable[str] = BACKENDS) -> list[LoweringVariant]:
        dtype = normalize_dtype(dtype)
        allowed = set(allowed_backends)
        candidates = sorted(
            (e for e in self.entries if e.hidden_size == hidden_size and e.dtype == dtype),
            key=lambda e: e.rows,
        )
        if not candidates:
            return []
        thresholds = [math.floor(math.sqrt(a.rows * b.rows)) for a, b in zip(candidates, candidates[1:])]
        variants = []
        minimum = 1
        for index, entry in enumerate(candidates):
            maximum = thresholds[index] if index < len(thresholds) else None
            costs = {k: v for k, v in entry.backend_costs().items() if k in allowed}
            if not costs:
                raise ProfileError(f"M={entry.rows},N={hidden_size},{dtype} has no allowed backend")
            backend = min(costs, key=costs.get)
            variants.append(LoweringVariant(
                min_rows=minimum, max_rows=maximum, profile_rows=entry.rows, backend=backend,
                estimated_us=costs[backend],
                num_warps=select_num_warps(entry.rows, hidden_size) if backend in ("triton", "hip") else None,
            ))
            minimum = maximum + 1 if maximum is not None else minimum
        return variants

    def plan_attribute(self, hidden_size: int, dtype: str, *, fallback: str = "hip",
                       allowed_backends: Iterable[str] = BACKENDS) -> dict[str, Any]:
        return {
            "schema_version": 1,
            "profile_source": self.source,
            "target": asdict(self.target),
            "hidden_size": hidden_size,
            "dtype": normalize_dtype(dtype),
            "fallback": fallback,
            "variants": [asdict(v) for v in self.variants(hidden_size, dtype, allowed_backends=allowed_backends)],
        }


def select_variant(variants: Iterable[LoweringVariant] | Iterable[dict[str, Any]], rows: int) -> LoweringVariant | None:
    for item in variants:
        variant = item if isinstance(item, LoweringVariant) else LoweringVariant(**item)
        if variant.contains(rows):
            return variant
    return None


def resolve_lowering_plan(plan: dict[str, Any] | None, rows: int, *,
                          default_backend: str = "hip") -> LoweringDecision:
    """Map the run-time row count onto a compile-time plan (cost_model.py:220-245)."""

    if rows <= 0:
        raise ProfileError("run-time rows must be positive")
    if not plan:
        return LoweringDecision(default_backend, "default")
    variant = select_variant(plan.get("variants", []), rows)
    if variant is None:
        return LoweringDecision(str(plan.get("fallback", default_backend)), "fallback")
    return LoweringDecision(
        backend=variant.backend, source="profile", profile_rows=variant.profile_rows,
        estimated_us=variant.estimated_us, num_warps=variant.num_warps,
    )


def select_num_warps(rows: int, hidden_size: int) -> int:
    block = 1 << max(0, hidden_size - 1).bit_length()
    if block < 2048:
        return 4
    if 4 <= rows <= 16:
        return 4
    return 8


def normalize_dtype(dtype: str) -> str:
    aliases = {"f16": "fp16", "float16": "fp16", "fp16": "fp16", "bf16": "bf16",
               "bfloat16": "bf16", "f32": "fp32", "float32": "fp32", "fp32": "fp32"}
    try:
        return aliases[str(dtype).lower()]
    except KeyError as error:
        raise ProfileError(f"unsupported dtype {dtype}") from error


def _parse_entry(row: dict[str, Any]) -> RMSNormProfileEntry:
    try:
        def opt(key: str) -> float | None:
            return float(row[key]) if row.get(key) is not None else None

        return RMSNormProfileEntry(
            rows=int(row["rows"]), hidden_size=int(row["hidden_size"]),
            dtype=normalize_dtype(str(row["dtype"])), native_us=float(row["native_eager_us"]),
            triton_us=opt("triton_us"), inductor_us=opt("inductor_us"), hip_us=opt("hip_us"),
        )
    except (KeyError, TypeError, ValueError) as error:
        raise ProfileError(f"illegal profile row: {row}") from error


def _validate_entries(entries: tuple[RMSNormProfileEntry, ...]) -> None:
    keys = set()
    for entry in entries:
        if entry.rows <= 0 or entry.hidden_size <= 0:
            raise ProfileError("rows and hidden size must be positive")
        if any(not math.isfinite(c) or c <= 0 for c in entry.backend_costs().values()):
            raise ProfileError("backend latencies must be finite and positive")
        key = (entry.rows, entry.hidden_size, entry.dtype)
        if key in keys:
            raise ProfileError(f"duplicate measurement {key}")
        keys.add(key)
