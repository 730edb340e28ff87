"""CPU oracle of the KernelIR hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, from scratch and in PyTorch-eager on the CPU, the
semantics of the reference's own reference executor
(src/stateful_llm_compiler/execution.py of Edison-Ayan/llm-compiler): the KV
runtime state, the serve.* op handlers and the Qwen2 model math.  It is the
checker the HIP backend is compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package never does.

Every function cites the reference file:line it follows.  How each one is
pinned (golden vectors, closed forms, brute force) is listed in
``tests/test_oracle.py``.
"""
