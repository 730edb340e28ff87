"""The decode-step fusion pass (passes/fusion.py) on the CPU: which chains it
fuses in the Qwen2 graphs, that the result verifies and stays fully lowered,
and that it leaves alone what it must not touch."""

from __future__ import annotations

import torch

from stateful_llm_compiler_hip.compiler import CompileOptions, compile_module
from stateful_llm_compiler_hip.ir import IRBuilder, Function, Module, TensorType, dims, verify_module
from stateful_llm_compiler_hip.qwen2 import Qwen2Config, build_decode_module, build_prefill_module

CONFIG = Qwen2Config(num_layers=2, vocab_size=1024)


def _counts(module):
    counts = {}
    for op in module.functions[0].block.operations:
        counts[op.name] = counts.get(op.name, 0) + 1
    return counts


def test_decode_graph_fuses_every_layer_chain():
    plain = compile_module(build_decode_module(CONFIG, capacity=64), CompileOptions(fuse=False))
    fused = compile_module(build_decode_module(CONFIG, capacity=64), CompileOptions())
    verify_module(fused.module)
    assert fused.coverage.is_complete
    c = _counts(fused.module)
    layers = CONFIG.num_layers
    assert c["kernel.hip.norm_linear_group"] == layers + 1   # Q/K/V per layer + the LM head
    assert c["kernel.hip.norm_linear_swiglu"] == layers
    assert c["kernel.hip.linear_residual"] == 2 * layers
    assert c["kernel.hip.rope_store_attention"] == layers
    for gone in ("kernel.hip.rms_norm", "kernel.hip.swiglu", "kernel.hip.add", "kernel.hip.rope",
                 "kernel.hip.kv_store", "kernel.hip.linear", "kernel.hip.rope_kv_store",
                 "kernel.hip.decode_attention"):
        assert gone not in c, gone
    before = len(plain.module.functions[0].block.operations)
    after = len(fused.module.functions[0].block.operations)
    # per layer: norm+3 linears, norm+2 linears+swiglu, 2 x linear+add,
    # rope+store, store+advance, store+attention
    assert before - after == layers * (3 + 3 + 2 + 1 + 1 + 1) + 1
    fused_ops = [op for op in fused.module.functions[0].block.operations
                 if op.name == "kernel.hip.rope_store_attention"]
    assert all(op.attributes["advance"] == 1 and op.attributes["groups"] == 7
               and len(op.operands) == 8 for op in fused_ops)
    assert "runtime.kv.advance" not in c
    stats = next(p for p in fused.passes if p.name == "fuse-decode-kernels").statistics
    assert stats["fused"]["kernel.hip.rope_kv_store"] == layers
    assert stats["fused"]["kernel.hip.rope_store_attention"] == layers


def test_store_feeding_another_reader_keeps_its_attention():
    # The first layer's rotated query is returned too: that layer's store and
    # attention stay apart, the other layer's fuse.
    result = compile_module(build_decode_module(CONFIG, capacity=64), CompileOptions(fuse=False))
    function = result.module.functions[0]
    from stateful_llm_compiler_hip.passes.fusion import FuseDecodeKernelsPass
    rope = next(op for op in function.block.operations if op.name == "kernel.hip.rope")
    function.returns.append(rope.results[0])
    FuseDecodeKernelsPass().run(result.module)
    verify_module(result.module)
    c = _counts(result.module)
    assert c["kernel.hip.rope_store_attention"] == CONFIG.num_layers - 1
    assert c["kernel.hip.decode_attention"] == 1 and c["kernel.hip.rope_kv_store"] == 1


def test_vocabulary_sized_head_fuses_with_its_norm():
    # The head's kernel (one wave per 16 features over all of K) normalises
    # the rows in its input staging, so the final norm joins the head:
    # one group for the layer's Q/K/V, one for the norm and the head.
    wide = Qwen2Config(num_layers=1, vocab_size=151936)
    fused = compile_module(build_decode_module(wide, capacity=64), CompileOptions())
    c = _counts(fused.module)
    assert c.get("kernel.hip.rms_norm", 0) == 0 and c.get("kernel.hip.linear", 0) == 0
    assert c["kernel.hip.norm_linear_group"] == 2
    # Narrower heads fuse too (on the equal-workgroup kernel).
    narrow = Qwen2Config(num_layers=1, vocab_size=16000)
    c = _counts(compile_module(build_decode_module(narrow, capacity=64), CompileOptions()).module)
    assert c.get("kernel.hip.rms_norm", 0) == 0 and c["kernel.hip.norm_linear_group"] == 2


def test_prefill_graph_fuses_and_compat_mode_does_not():
    fused = compile_module(build_prefill_module(CONFIG, capacity=64), CompileOptions())
    assert _counts(fused.module).get("kernel.hip.norm_linear_swiglu") == CONFIG.num_layers
    compat = compile_module(build_decode_module(CONFIG, capacity=64),
                            CompileOptions(numerical_mode="pytorch_compatible"))
    names = set(_counts(compat.module))
    assert not names & {"kernel.hip.norm_linear_group", "kernel.hip.norm_linear_swiglu",
                        "kernel.hip.linear_residual", "kernel.hip.rope_kv_store",
                        "kernel.hip.rope_store_attention"}


def test_value_with_another_user_is_not_fused_away():
    b = IRBuilder()
    t = lambda *s: TensorType(dims(*s), "bf16", "cuda:0")  # noqa: E731
    h = b.argument(t(2, 1, 64), "h")
    nw = b.argument(t(64), "nw")
    w = b.argument(t(32, 64), "w")
    x = b.emit("serve.rms_norm", [h, nw], [t(2, 1, 64)],
               attributes={"epsilon": 1e-6, "axis": -1, "round_before_weight": True}).results[0]
    y = b.emit("serve.linear", [x, w], [t(2, 1, 32)],
               attributes={"has_bias": False, "input_features": 64, "output_features": 32}).results[0]
    module = Module([Function("f", b.block, [y, x])])  # the normalised rows are returned too
    result = compile_module(module, CompileOptions())
    names = [op.name for op in result.module.functions[0].block.operations]
    assert names == ["kernel.hip.rms_norm", "kernel.hip.linear"]
    torch.manual_seed(0)  # keeps the import used; nothing random here
