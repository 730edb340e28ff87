"""The C-ABI library loads on a CPU-only machine and exports exactly the entry
points include/slc_hip.h declares, with the ctypes signatures the host side
binds.  No kernel is called here."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

from stateful_llm_compiler_hip import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "slc_hip.h"


def _declared() -> dict[str, int]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for match in re.finditer(r"SLC_API\s+[\w\s\*]+?\b(slc_hip_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        params = match.group(2).strip()
        out[match.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_header_declares_every_bound_symbol_with_matching_arity():
    declared = _declared()
    assert set(declared) == set(_native.SIGNATURES), (
        set(declared) ^ set(_native.SIGNATURES)
    )
    for name, (_, argtypes) in _native.SIGNATURES.items():
        assert declared[name] == len(argtypes), name


def test_library_exports_every_declared_symbol():
    if not _native.LIBRARY_PATH.exists():
        pytest.fail(f"{_native.LIBRARY_PATH} missing: run __graft_entry__.build()")
    lib = _native.library()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.slc_hip_version() >= 100
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIBRARY_PATH)],
                        capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line}
    assert {s for s in exported if s.startswith("slc_hip_")} == set(_declared())


def test_argument_checks_fail_without_touching_a_device():
    # Invalid sizes are rejected on the host before any launch.
    lib = _native.library()
    status = lib.slc_hip_linear(None, None, None, None, 99, 1, 1, 1, 1, 1, None)
    assert status == -1
    assert b"bad dtype" in lib.slc_hip_last_error()
    assert lib.slc_hip_decode_attention_workspace_size(0, 14, 64, 8192, 2, 2, 0) == 0
    # Workspace of the headline shape: B x QH x chunks x (D + 2) floats of
    # split partials (4 chunks of 2048 tokens); counters B x KVH merge + B
    # advance ints.
    size = lib.slc_hip_decode_attention_workspace_size(32, 14, 64, 8192, 2, 2, 0)
    assert size == 32 * 14 * 4 * 66 * 4
    assert lib.slc_hip_decode_attention_counter_count(32, 2) == 32 * 2 + 32
    # The exact softmax order: 4096 tokens at head_dim 64 (LDS), 2048 at 128;
    # unlimited on the generic kernel (fp32).
    assert lib.slc_hip_decode_attention_exact_max_tokens(64, 2) == 4096
    assert lib.slc_hip_decode_attention_exact_max_tokens(128, 1) == 2048
    assert lib.slc_hip_decode_attention_exact_max_tokens(64, 0) == 2**63 - 1
    # Argmax: 64 segments of (index, value) per row (counters: one per row).
    assert lib.slc_hip_argmax_workspace_size(8) == 8 * 64 * 12


def test_product_never_imports_the_oracle():
    package = ROOT / "llm-compiler_amd" / "stateful_llm_compiler_hip"
    for source in package.rglob("*.py"):
        text = source.read_text()
        assert "import oracle" not in text and "from oracle" not in text, source


def test_fused_entry_points_decline_or_reject_before_any_device_call():
    # Host-side argument logic of the fused entry points, exercised without a
    # GPU: the shape checks run before any HIP call, so dummy (never
    # dereferenced) pointers are enough.  -2 = SLC_ERR_UNSUPPORTED (the caller
    # runs the unfused ops), -1 = SLC_ERR_INVALID_ARGUMENT.
    if not _native.LIBRARY_PATH.exists():
        pytest.fail(f"{_native.LIBRARY_PATH} missing: run __graft_entry__.build()")
    lib = _native.library()
    p = 0x1000  # 4 KiB-aligned, never dereferenced on these paths
    bf16, f32 = 2, 0
    # gate/up + SwiGLU: rows <= 64, K not a multiple of 64, N not a multiple of 8
    assert lib.slc_hip_linear_swiglu(p, 896, 64, 896, 4864, p, p, p, 4864, bf16, None) == -2
    assert lib.slc_hip_linear_swiglu(p, 72, 300, 72, 4864, p, p, p, 4864, bf16, None) == -2
    assert lib.slc_hip_linear_swiglu(p, 896, 300, 896, 100, p, p, p, 100, bf16, None) == -2
    assert lib.slc_hip_linear_swiglu(None, 896, 300, 896, 4864, p, p, p, 4864, bf16, None) == -1
    assert lib.slc_hip_linear_swiglu(p, 896, 0, 896, 4864, p, p, p, 4864, bf16, None) == 0
    # grouped projections: a width that is not a multiple of 8; fp32
    assert lib.slc_hip_linear_group(p, 896, 300, 896, 2, p, None, p, 896, 896,
                                    p, None, p, 100, 100, None, None, None, 0, 0,
                                    bf16, None) == -2
    assert lib.slc_hip_linear_group(p, 896, 300, 896, 1, p, None, p, 896, 896,
                                    None, None, None, 0, 0, None, None, None, 0, 0,
                                    f32, None) == -2
    assert lib.slc_hip_linear_group(p, 896, 300, 896, 4, p, None, p, 896, 896,
                                    None, None, None, 0, 0, None, None, None, 0, 0,
                                    bf16, None) == -1
    # RoPE decode attention: fp32 and head_dim 80 are not its kernel's cases
    args = [p] * 10 + [None, 0, p, None, 0, p, 1000]
    sizes = [4, 14, 2, 64, 256, 256]
    strides = [896, 64, 128, 64, 128, 64, 64, 64, 32768, 128, 64, 0, 0, 896, 64]
    assert lib.slc_hip_rope_decode_attention(*args, f32, *sizes, *strides, 0.125, 0, None) == -2
    sizes_d80 = [4, 14, 2, 80, 256, 256]
    assert lib.slc_hip_rope_decode_attention(*args, bf16, *sizes_d80, *strides, 0.125, 0, None) == -2
    # ... nor an exact-order mask longer than its LDS holds, nor a bad order.
    sizes_long = [4, 14, 2, 64, 8192, 8192]
    assert lib.slc_hip_rope_decode_attention(*args, bf16, *sizes_long, *strides, 0.125, 1, None) == -2
    assert lib.slc_hip_rope_decode_attention(*args, bf16, *sizes, *strides, 0.125, 7, None) == -1


def test_paged_kv_store_rejects_a_grid_past_one_launch():
    # 2^43 16-byte units need 2^35 workgroups of 256, past a launch: rejected on
    # the host (the pointers are never dereferenced).
    lib = _native.library()
    fake = 1 << 20
    batch, heads, tokens, head_dim = 1 << 16, 512, 1 << 15, 64  # x 8 units per row
    status = lib.slc_hip_paged_kv_store(
        fake, fake, fake, 64, 64, 16, 16 * heads * head_dim, heads * head_dim, head_dim,
        fake, fake, fake, None, _native.SLC_BF16, batch, heads, tokens, head_dim,
        heads * tokens * head_dim, tokens * head_dim, head_dim,
        heads * tokens * head_dim, tokens * head_dim, head_dim, None)
    assert status == -1
    assert b"exceed one launch's grid" in lib.slc_hip_last_error()


def test_stream_workspaces_are_bounded(monkeypatch):
    # The per-stream workspace cache keeps the most recently used streams
    # only (no device memory is touched: workspaces allocate lazily).
    import torch

    handles = iter(range(1000, 2000))
    monkeypatch.setattr(_native, "current_stream", lambda device: next(handles))
    monkeypatch.setattr(_native, "_stream_workspaces", type(_native._stream_workspaces)())
    first = _native.stream_workspace(torch.device("cuda", 0))
    for _ in range(_native.MAX_STREAM_WORKSPACES + 10):
        _native.stream_workspace(torch.device("cuda", 0))
    assert len(_native._stream_workspaces) == _native.MAX_STREAM_WORKSPACES
    assert first not in _native._stream_workspaces.values()
