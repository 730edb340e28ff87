"""Compiler pass protocol and a verifying pass manager.

Same contract as the reference (src/stateful_llm_compiler/pass_manager.py:
12-53): a pass returns ``PassResult(name, changed, statistics)``; the manager
verifies the module before the first pass and after every pass.
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass, field
from typing import Any, Iterable

from .ir import Module, verify_module


@dataclass
class PassResult:
    name: str
    changed: bool
    statistics: dict[str, Any] = field(default_factory=dict)


class CompilerPass:
    name = "pass"

    def run(self, module: Module) -> PassResult:  # pragma: no cover - abstract
        raise NotImplementedError


def operation_counts(module: Module) -> dict[str, int]:
    counts = Counter(op.name for fn in module.functions for op in fn.block.operations)
    return dict(sorted(counts.items()))


class PassManager:
    def __init__(self, passes: Iterable[CompilerPass] = ()) -> None:
        self.passes = list(passes)

    def add(self, compiler_pass: CompilerPass) -> "PassManager":
        self.passes.append(compiler_pass)
        return self

    def run(self, module: Module) -> list[PassResult]:
        verify_module(module)
        results = []
        for compiler_pass in self.passes:
            before = sum(len(fn.block.operations) for fn in module.functions)
            result = compiler_pass.run(module)
            verify_module(module)
            result.statistics.setdefault("operations_before", before)
            result.statistics.setdefault(
                "operations_after", sum(len(fn.block.operations) for fn in module.functions)
            )
            results.append(result)
        return results
