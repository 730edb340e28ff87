"""Host logic: IR verifier rules, lowering tables, coverage and strict mode,
profile-guided plans.  Mirrors the reference's CPU unit tests (test_ir.py,
test_lowering.py, test_cost_model.py) for the hot-path ops."""

from __future__ import annotations

import copy

import pytest

from stateful_llm_compiler_hip.compiler import CompileOptions, compile_module
from stateful_llm_compiler_hip.cost_model import (
    KernelProfile,
    ProfileError,
    choose_variant,
    split_tokens,
    waves_per_row,
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


def test_paged_layout_verifies_and_lowers():
    decode = build_decode_module(SMALL, capacity=256, page_tokens=64, device="cpu")
    prefill = build_prefill_module(SMALL, capacity=256, page_tokens=64, device="cpu")
    verify_module(decode)
    verify_module(prefill)
    state = decode.functions[0].block.arguments[2].type
    assert state.layout == "paged" and state.page_tokens == 64
    assert "layout=paged" in str(state) and "page_tokens=64" in str(state)
    init = next(op for op in prefill.functions[0].block.operations if op.name == "serve.kv.init")
    assert init.attributes["layout"] == "paged" and init.attributes["page_tokens"] == 64
    for module in (decode, prefill):
        result = compile_module(module, CompileOptions())
        assert result.coverage.is_complete
    lowered = next(op for op in prefill.functions[0].block.operations if op.name == "runtime.kv.init")
    assert lowered.attributes["page_tokens"] == 64


@pytest.mark.parametrize("layout,page_tokens,capacity,needle", [
    ("paged", None, 64, "power of two"),
    ("paged", 24, 96, "power of two"),
    ("paged", 8, 64, "power of two"),
    ("paged", 64, 96, "multiple of page_tokens"),
    ("contiguous_bshd", 64, 64, "only applies to the paged layout"),
    ("blocked", None, 64, "contiguous_bshd and paged"),
])
def test_verifier_rejects_bad_paging(layout, page_tokens, capacity, needle):
    b = IRBuilder()
    state = b.argument(KVStateType("bf16", 1, 2, 64, layout=layout, capacity=capacity,
                                   page_tokens=page_tokens), "state")
    q = b.argument(TensorType(dims("B", 14, 1, 64), "bf16"), "q")
    m = b.argument(TensorType(dims("B", 1, 1, "S"), "bf16"), "mask")
    op = b.emit("serve.decode_attention", [state, q, m], [q.type],
                attributes={"slot": 0, "groups": 7, "scale": 0.125},
                effects=(Effect(EffectKind.READ, "kv"),))
    with pytest.raises(VerificationError) as error:
        verify_module(Module([Function("f", b.block, op.results)]))
    assert needle in str(error.value)


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
        # Every layer's chains are fused, and the final norm with the
        # vocabulary-sized LM head.
        assert "kernel.hip.linear" not in counts and "kernel.hip.rms_norm" not in counts
        assert counts["kernel.hip.norm_linear_group"] == 25
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

# A profile in the reference's format (benchmarks/bench_rmsnorm.py:183-208):
# backends this build does not have, and hip_us.
REFERENCE_PROFILE = {
    "schema_version": 1,
    "target": {"device_name": "AMD Instinct MI355X"},
    "results": [
        {"rows": 1, "hidden_size": 896, "dtype": "bf16", "native_eager_us": 9.0,
         "triton_us": 4.0, "inductor_us": 8.0, "hip_us": 3.0},
        {"rows": 4096, "hidden_size": 896, "dtype": "bf16", "native_eager_us": 30.0, "hip_us": 12.0},
    ],
}

VARIANT_PROFILE = {
    "schema_version": 1,
    "target": {"device_name": "AMD Instinct MI355X"},
    "results": [
        {"rows": 1, "hidden_size": 896, "dtype": "bf16", "hip_variants": {"wave": 3.0, "block": 2.0}},
        {"rows": 64, "hidden_size": 896, "dtype": "bf16", "hip_variants": {"wave": 5.0, "block": 6.0}},
        {"rows": 4096, "hidden_size": 896, "dtype": "bf16", "hip_variants": {"wave": 12.0, "block": 30.0}},
    ],
    "decode_attention": [
        {"batch": 8, "mask_len": 1024, "q_heads": 14, "kv_heads": 2, "head_dim": 64, "dtype": "bf16",
         "hip_variants": {"fixed": 10.0, "balanced": 13.0}},
        {"batch": 64, "mask_len": 8192, "q_heads": 14, "kv_heads": 2, "head_dim": 64, "dtype": "bf16",
         "hip_variants": {"fixed": 52.0, "balanced": 46.0, "chunk1024": 60.0}},
    ],
    "linear": [
        {"rows": 128, "out_features": 128, "in_features": 896, "dtype": "bf16",
         "hip_variants": {"t128x128": 11.7, "t64x64": 9.0, "t32x64": 5.9}},
        {"rows": 32768, "out_features": 128, "in_features": 896, "dtype": "bf16",
         "hip_variants": {"t128x128": 22.0, "t64x64": 20.6, "t32x64": 28.7}},
    ],
}


def test_reference_profile_loads_and_plans_the_automatic_variant():
    profile = KernelProfile.from_dict(REFERENCE_PROFILE)
    plan = profile.plan("rms_norm", hidden_size=896, dtype="bfloat16")
    assert [s["latency_us"] for s in plan["samples"]] == [{"auto": 3.0}, {"auto": 12.0}]
    assert choose_variant(plan, 100).variant == "auto"
    assert profile.plan("rms_norm", hidden_size=1536, dtype="bf16") is None
    assert choose_variant(None, 4).source == "default"


def test_variant_latencies_interpolate_in_log_size():
    plan = KernelProfile.from_dict(VARIANT_PROFILE).plan("rms_norm", hidden_size=896, dtype="bf16")
    # rows 1: block 2 < wave 3.
    assert choose_variant(plan, 1).variant == "block"
    # rows 8 sits halfway (in log) between 1 and 64: wave 4.0 == block 4.0, a
    # tie that goes to the variant listed first.
    eight = choose_variant(plan, 8)
    assert eight.variant == "wave" and eight.estimated_us == pytest.approx(4.0)
    # rows 4: a third of the way: wave 3 + 2/3 < block 2 + 4/3?  No: 3.667 > 3.333.
    four = choose_variant(plan, 4)
    assert four.variant == "block" and four.estimated_us == pytest.approx(2.0 + 4.0 / 3.0)
    # Past the last sample the end values stand: wave 12 < block 30.
    assert choose_variant(plan, 10**6).variant == "wave"
    assert waves_per_row("wave") == 1 and waves_per_row("block") == 4 and waves_per_row("auto") == 0

    split = KernelProfile.from_dict(VARIANT_PROFILE).plan(
        "decode_attention", q_heads=14, kv_heads=2, head_dim=64, dtype="bf16")
    assert choose_variant(split, 8 * 1024).variant == "fixed"
    assert choose_variant(split, 64 * 8192).variant == "balanced"
    # chunk1024 was measured only at the large size: its flat estimate (60)
    # never wins.
    assert choose_variant(split, 100).variant == "fixed"
    assert [split_tokens(v) for v in ("fixed", "balanced", "chunk1024", "auto")] == [0, -1, 1024, 0]


def test_bad_profiles_are_rejected():
    with pytest.raises(ProfileError):
        KernelProfile.from_dict({"schema_version": 2, "results": []})
    dup = copy.deepcopy(VARIANT_PROFILE)
    dup["results"].append(dict(dup["results"][0]))
    with pytest.raises(ProfileError):
        KernelProfile.from_dict(dup)
    unknown = copy.deepcopy(VARIANT_PROFILE)
    unknown["results"][0]["hip_variants"]["warp32"] = 1.0
    with pytest.raises(ProfileError):
        KernelProfile.from_dict(unknown)
    negative = copy.deepcopy(VARIANT_PROFILE)
    negative["decode_attention"][0]["hip_variants"]["fixed"] = -1.0
    with pytest.raises(ProfileError):
        KernelProfile.from_dict(negative)
    with pytest.raises(ProfileError):
        choose_variant({"op": "rms_norm", "samples": []}, 0)
    with pytest.raises(ProfileError):
        split_tokens("wave")


def test_profile_plan_passes_attach_plans(tmp_path):
    import json

    path = tmp_path / "profile.json"
    path.write_text(json.dumps(VARIANT_PROFILE))
    result = compile_module(build_decode_module(SMALL, capacity=64),
                            CompileOptions(rmsnorm_profile=path))
    ops = result.module.functions[0].block.operations
    norms = [op for op in ops if op.name == "kernel.hip.rms_norm"]
    attention = [op for op in ops if op.name == "kernel.hip.decode_attention"]
    assert norms and all(op.attributes["lowering_plan"]["op"] == "rms_norm" for op in norms)
    assert attention and all(op.attributes["split_plan"]["op"] == "decode_attention" for op in attention)
    stats = {r.name: r.statistics for r in result.passes}
    # SMALL's K/V projections are 896 -> 128 (the profiled shape); the
    # others have no samples and stay unplanned.
    assert stats["select-linear-tile"]["planned_operations"] == 2 * SMALL.num_layers
    assert stats["select-linear-tile"]["missing_profile"] > 0
    assert stats["select-rmsnorm-lowering"]["planned_operations"] == len(norms)
    assert stats["select-decode-attention-split"]["planned_operations"] == len(attention)
    # A planned attention keeps its own launch (the fused RoPE + attention
    # kernel runs the fixed split only).
    assert not any(op.name == "kernel.hip.rope_store_attention" for op in ops)


def test_committed_mi355x_profile_plans_the_measured_winners():
    """The profile measured on MI355X (profile_variants.py) loads, and its
    plans pick what it measured fastest: one wave per RMSNorm row, and the
    fixed-chunk split at the decode-attention bench shape."""

    from pathlib import Path

    import stateful_llm_compiler_hip

    path = Path(stateful_llm_compiler_hip.__file__).parent / "profiles" / "mi355x.json"
    profile = KernelProfile.load(path)
    norm = profile.plan("rms_norm", hidden_size=896, dtype="bf16")
    for rows in (1, 8, 4096, 32768):
        assert choose_variant(norm, rows).variant == "wave"
    split = profile.plan("decode_attention", q_heads=14, kv_heads=2, head_dim=64, dtype="bf16")
    assert choose_variant(split, 32 * 8192).variant == "fixed"


def test_plan_changes_the_variant_the_executor_launches(monkeypatch):
    """The plan's choice reaches the HIP wrapper's launch argument (and from
    there the C ABI's waves_per_row / split_tokens) and the lowering trace."""

    import torch

    from stateful_llm_compiler_hip import execution

    profile = KernelProfile.from_dict(VARIANT_PROFILE)
    seen = {}

    def fake_rms_norm(tensor, weight, **kwargs):
        seen["num_warps"] = kwargs.get("num_warps")
        return tensor

    monkeypatch.setattr(execution, "hip_rms_norm", fake_rms_norm)
    executor = execution.HipExecutor()
    plan = profile.plan("rms_norm", hidden_size=896, dtype="bf16")
    attrs = {"epsilon": 1e-6, "round_before_weight": True, "lowering_plan": plan}
    executor._rms_norm([torch.zeros(1, 896), torch.ones(896)], attrs)
    assert seen["num_warps"] == 4                      # rows 1: the block variant
    executor._rms_norm([torch.zeros(4096, 896), torch.ones(896)], attrs)
    assert seen["num_warps"] == 1                      # rows 4096: one wave per row
    executor._rms_norm([torch.zeros(4096, 896), torch.ones(896)],
                       {"epsilon": 1e-6, "round_before_weight": True})
    assert seen["num_warps"] is None                   # no plan: the library decides
    assert [t["variant"] for t in executor.lowering_trace] == ["block", "wave", "auto"]

    class RecordingState(execution.PreallocatedKVCacheState):
        def decode_attention(self, slot, query, mask, **kwargs):
            seen["split_tokens"] = kwargs["split_tokens"]
            return query

    state = object.__new__(RecordingState)
    split = profile.plan("decode_attention", q_heads=14, kv_heads=2, head_dim=64, dtype="bf16")
    attrs = {"groups": 7, "scale": 0.125, "split_plan": split}
    executor._decode_attention([state, torch.zeros(64, 14, 1, 64), torch.zeros(64, 1, 1, 8192)], attrs)
    assert seen["split_tokens"] == -1                  # the balanced split
    executor._decode_attention([state, torch.zeros(8, 14, 1, 64), torch.zeros(8, 1, 1, 1024)], attrs)
    assert seen["split_tokens"] == 0                   # the fixed-chunk split
    assert executor.lowering_trace[-1]["variant"] == "fixed"




def test_linear_tile_plan_follows_rows_and_reaches_the_wrapper(monkeypatch):
    """The GEMM tile plan: static key (N, K, dtype), run-time axis M; the
    executor passes the chosen tile to hip_linear (which hands it to
    slc_hip_linear_tile) and records it in the lowering trace."""

    import torch

    from stateful_llm_compiler_hip import execution
    from stateful_llm_compiler_hip.cost_model import linear_tile

    profile = KernelProfile.from_dict(VARIANT_PROFILE)
    plan = profile.plan("linear", out_features=128, in_features=896, dtype="bfloat16")
    assert plan["axis"] == "rows"
    assert choose_variant(plan, 128).variant == "t32x64"
    assert choose_variant(plan, 32768).variant == "t64x64"
    assert profile.plan("linear", out_features=896, in_features=896, dtype="bf16") is None
    with pytest.raises(ProfileError):
        linear_tile("t16x16")
    with pytest.raises(ProfileError):
        KernelProfile.from_dict({"schema_version": 1, "linear": [
            {"rows": 128, "out_features": 128, "in_features": 896, "dtype": "bf16",
             "hip_variants": {"t256x256": 1.0}}]})

    seen = []

    def fake_linear(tensor, weight, bias=None, *, tile="auto"):
        seen.append(tile)
        return tensor

    monkeypatch.setattr(execution, "hip_linear", fake_linear)
    executor = execution.HipExecutor()
    w = torch.zeros(128, 896)
    executor._linear([torch.zeros(2, 64, 896), w], {"has_bias": False, "tile_plan": plan})
    executor._linear([torch.zeros(32768, 896), w], {"has_bias": False, "tile_plan": plan})
    executor._linear([torch.zeros(32768, 896), w], {"has_bias": False})
    assert seen == ["t32x64", "t64x64", "auto"]
    assert [(t["variant"], t["rows"]) for t in executor.lowering_trace] == [("t32x64", 128), ("t64x64", 32768)]


def test_exact_order_downgrade_is_traced():
    """A decode attention whose IR asks for the exact softmax order over a
    mask longer than the kernel's exact limit runs the online order, and the
    lowering trace says so."""

    import torch

    from stateful_llm_compiler_hip import execution

    seen = {}

    class RecordingState(execution.PreallocatedKVCacheState):
        def decode_attention(self, slot, query, mask, **kwargs):
            seen["order"] = kwargs["softmax_order"]
            return query

    state = object.__new__(RecordingState)
    executor = execution.HipExecutor()
    query = torch.zeros(2, 14, 1, 64, dtype=torch.bfloat16)
    attrs = {"groups": 7, "scale": 0.125, "softmax_order": "exact"}
    executor._decode_attention([state, query, torch.zeros(2, 1, 1, 1024)], attrs)
    assert executor.lowering_trace == []
    executor._decode_attention([state, query, torch.zeros(2, 1, 1, 8192)], attrs)
    entry = executor.lowering_trace[-1]
    assert entry["softmax_order"] == "online" and entry["requested_softmax_order"] == "exact"
    assert entry["mask_len"] == 8192
