"""Host logic: IR verifier rules, lowering tables, coverage and strict mode,
profile-guided plans.  Mirrors the reference's CPU unit tests (test_ir.py,
test_lowering.py, test_cost_model.py) for the hot-path ops."""

from __future__ import annotations

import copy

import pytest

from stateful_llm_compiler_hip.compiler import CompileOptions, compile_module
from stateful_llm_compiler_hip.cost_model import (
    ProfileError,
    RMSNormCostModel,
    resolve_lowering_plan,
    select_num_warps,
)
from stateful_llm_compiler_hip.ir import (
    Block,
    Effect,
    EffectKind,
    Function,
    IRBuilder,
    KVStateType,
    Module,
    TensorType,
    VerificationError,
    dims,
    format_module,
    verify_module,
)
from stateful_llm_compiler_hip.lowering import (
    EXECUTABLE_OPERATIONS,
    LoweringCoverageError,
    LowerToKernelIRPass,
    analyze_lowering_coverage,
    require_full_lowering,
)
from stateful_llm_compiler_hip.qwen2 import Qwen2Config, build_decode_module, build_prefill_module

SMALL = Qwen2Config(num_layers=2, vocab_size=1024)


def _kv_state(capacity=64):
    return KVStateType("bf16", 1, 2, 64, layout="contiguous_bshd", capacity=capacity)


def _decode_attention_module(groups=7, q_heads=14, tokens=1, effects=True):
    b = IRBuilder()
    state = b.argument(_kv_state(), "state")
    q = b.argument(TensorType(dims("B", q_heads, tokens, 64), "bf16"), "q")
    m = b.argument(TensorType(dims("B", 1, 1, "S"), "bf16"), "mask")
    eff = (Effect(EffectKind.READ, "kv"),) if effects else ()
    op = b.emit("serve.decode_attention", [state, q, m], [q.type],
                attributes={"slot": 0, "groups": groups, "scale": 0.125}, effects=eff)
    return Module([Function("f", b.block, op.results)])


def test_verifier_accepts_builder_graphs():
    verify_module(build_decode_module(SMALL, capacity=64, device="cpu"))
    verify_module(build_prefill_module(SMALL, capacity=64, device="cpu"))
    verify_module(_decode_attention_module())


@pytest.mark.parametrize("kwargs,needle", [
    ({"groups": 6}, "KV heads x groups"),
    ({"tokens": 2}, "single token"),
    ({"effects": False}, "missing read"),
])
def test_verifier_rejects_bad_decode_attention(kwargs, needle):
    with pytest.raises(VerificationError) as error:
        verify_module(_decode_attention_module(**kwargs))
    assert needle in str(error.value)


def test_verifier_rejects_use_before_definition_and_bad_linear():
    b = IRBuilder()
    x = b.argument(TensorType(dims(4, 896), "bf16"), "x")
    w = b.argument(TensorType(dims(128, 896), "bf16"), "w")
    op = b.emit("serve.linear", [x, w], [TensorType(dims(4, 128), "bf16")],
                attributes={"has_bias": True, "input_features": 896, "output_features": 128})
    with pytest.raises(VerificationError) as error:
        verify_module(Module([Function("f", b.block, op.results)]))
    assert "has_bias" in str(error.value)
    ghost = TensorType(dims(4), "bf16")
    block = Block()
    orphan_builder = IRBuilder(block)
    from stateful_llm_compiler_hip.ir import Value
    stray = Value("%stray", ghost)
    orphan_builder.emit("serve.add", [stray, stray], [ghost])
    with pytest.raises(VerificationError):
        verify_module(Module([Function("g", block, [])]))


def test_verifier_kv_store_and_slot_rules():
    b = IRBuilder()
    state = b.argument(_kv_state(), "state")
    k = b.argument(TensorType(dims("B", 2, 1, 64), "bf16"), "k")
    pos = b.argument(TensorType(dims("B"), "i64"), "pos")
    b.emit("serve.kv.store", [state, k, k, pos], [state.type], attributes={"slot": 3},
           effects=(Effect(EffectKind.READ, "kv"),))
    with pytest.raises(VerificationError) as error:
        verify_module(Module([Function("f", b.block, [])]))
    text = str(error.value)
    assert "slot must be in" in text and "missing write" in text


def test_format_module_is_stable_text():
    text = format_module(_decode_attention_module())
    assert '"serve.decode_attention"' in text and "!serve.kv_state<bf16" in text


@pytest.mark.parametrize("mode", ["fast", "pytorch_compatible"])
def test_full_lowering_of_24_layer_graphs(mode):
    config = Qwen2Config()
    decode = compile_module(build_decode_module(config, capacity=2048), CompileOptions(numerical_mode=mode))
    prefill = compile_module(build_prefill_module(config, capacity=2048), CompileOptions(numerical_mode=mode))
    for result in (decode, prefill):
        assert result.coverage.is_complete and result.coverage.coverage == 1.0
    counts = decode.coverage.lowered_by_name
    assert counts["runtime.kv.length"] == 25
    if mode == "fast":
        # The per-layer advance rides on the rope + store kernel.
        assert "runtime.kv.advance" not in counts
        # ... and the store, advance and attention run as one kernel.
        assert counts["kernel.hip.rope_store_attention"] == 24
        assert "kernel.hip.rope_kv_store" not in counts
        # Every layer's chains are fused; the vocabulary-sized LM head keeps
        # its own norm and linear.
        assert counts["kernel.hip.linear"] == 1 and counts["kernel.hip.rms_norm"] == 1
        assert counts["kernel.hip.norm_linear_group"] == 24
        assert counts["kernel.hip.norm_linear_swiglu"] == 24
        assert counts["kernel.hip.linear_residual"] == 48
        assert "kernel.hip.decode_attention" not in counts
        assert not any(name.startswith("kernel.rocm_compat") for name in counts)
        plain = compile_module(build_decode_module(config, capacity=2048), CompileOptions(fuse=False))
        plain_counts = plain.coverage.lowered_by_name
        assert plain_counts["kernel.hip.linear"] == 24 * 7 + 1
        assert plain_counts["kernel.hip.rms_norm"] == 49
    else:
        assert counts["runtime.kv.advance"] == 24
        assert counts["kernel.rocm_compat.linear"] == 24 * 7 + 1
        assert counts["kernel.hip.rope"] == 24  # bit-exact in both modes


def test_lowering_annotates_and_is_idempotent():
    module = build_decode_module(SMALL, capacity=64)
    LowerToKernelIRPass().run(module)
    once = format_module(module)
    result = LowerToKernelIRPass().run(module)
    assert format_module(module) == once and not result.changed
    ops = module.functions[0].block.operations
    attn = next(op for op in ops if op.name == "kernel.hip.decode_attention")
    assert attn.attributes["lowered_from"] == "serve.decode_attention"
    assert attn.attributes["numerical_mode"] == "fast"
    lin = next(op for op in ops if op.name == "kernel.hip.linear")
    assert lin.attributes["backend_selection"].startswith("hip_mfma")


def test_strict_mode_rejects_unknown_ops():
    module = build_decode_module(SMALL, capacity=64)
    ops = module.functions[0].block.operations
    ops.insert(1, copy.copy(ops[0]))
    ops[1].name = "aten.exp.default"
    ops[1].results = []
    LowerToKernelIRPass().run(module)
    coverage = analyze_lowering_coverage(module)
    assert coverage.unlowered_by_name == {"aten.exp.default": 1}
    with pytest.raises(LoweringCoverageError) as error:
        require_full_lowering(module)
    assert "aten.exp.default" in str(error.value)
    # Unknown kernel.* names are not counted as lowered either.
    assert "kernel.triton.rms_norm" not in EXECUTABLE_OPERATIONS


def test_unsupported_numerical_mode():
    with pytest.raises(ValueError):
        LowerToKernelIRPass(numerical_mode="exact")


# ------------------------------------------------------------------ cost model

PROFILE = {
    "schema_version": 1,
    "target": {"device_name": "AMD Instinct MI355X"},
    "results": [
        {"rows": 1, "hidden_size": 896, "dtype": "bf16", "native_eager_us": 9.0, "hip_us": 3.0},
        {"rows": 64, "hidden_size": 896, "dtype": "bf16", "native_eager_us": 4.0, "hip_us": 5.0},
        {"rows": 4096, "hidden_size": 896, "dtype": "bf16", "native_eager_us": 30.0, "hip_us": 12.0},
    ],
}


def test_cost_model_buckets_split_at_geometric_midpoints():
    model = RMSNormCostModel.from_dict(PROFILE)
    variants = model.variants(896, "bf16")
    assert [(v.min_rows, v.max_rows, v.backend) for v in variants] == [
        (1, 8, "hip"), (9, 512, "native"), (513, None, "hip"),
    ]
    plan = model.plan_attribute(896, "bfloat16")
    assert resolve_lowering_plan(plan, 8).profile_rows == 1
    assert resolve_lowering_plan(plan, 9).backend == "native"
    assert resolve_lowering_plan(plan, 100000).backend == "hip"
    assert resolve_lowering_plan(None, 4).source == "default"
    assert model.variants(1536, "bf16") == []


def test_cost_model_rejects_bad_profiles():
    with pytest.raises(ProfileError):
        RMSNormCostModel.from_dict({"schema_version": 2, "results": []})
    bad = copy.deepcopy(PROFILE)
    bad["results"].append(dict(bad["results"][0]))
    with pytest.raises(ProfileError):
        RMSNormCostModel.from_dict(bad)
    with pytest.raises(ProfileError):
        resolve_lowering_plan({"variants": []}, 0)
    assert select_num_warps(8, 896) == 4 and select_num_warps(64, 4096) == 8


def test_profile_plan_pass_attaches_plans(tmp_path):
    import json

    path = tmp_path / "profile.json"
    path.write_text(json.dumps(PROFILE))
    result = compile_module(build_decode_module(SMALL, capacity=64),
                            CompileOptions(rmsnorm_profile=path))
    norms = [op for op in result.module.functions[0].block.operations if op.name == "kernel.hip.rms_norm"]
    assert norms and all(op.attributes["lowering_plan"]["variants"] for op in norms)
    assert result.passes[0].statistics["planned_operations"] == len(norms)
