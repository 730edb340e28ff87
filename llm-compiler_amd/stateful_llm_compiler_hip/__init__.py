"""MI355X (gfx950) HIP backend for the StatefulLLM-Compiler KernelIR.

The package mirrors the reference's KernelIR boundary
(src/stateful_llm_compiler/lowering.py and backends/): ServeIR ops are lowered
to ``kernel.hip.*`` names and executed by ``HipExecutor`` through the C ABI of
``libslc_hip.so`` (include/slc_hip.h).
"""

__version__ = "0.1.0"
