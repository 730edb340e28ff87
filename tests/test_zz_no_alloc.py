"""The allocation-free decode-attention entry point against the ordinary one.

slc_hip_decode_attention_noalloc keeps its split partials and counters in the
library's own device array; its results must equal slc_hip_decode_attention's
bit for bit (the same kernels), on consecutive calls that reuse the array, the
second with a smaller input, and the call must make no device allocation.
A fresh process makes its first no-alloc call inside a HIP graph capture and
checks every replay against the workspace entry point.
"""

from __future__ import annotations

import subprocess
import sys
import textwrap
from pathlib import Path

import pytest
import torch

from helpers import announce, generator

SPLIT_BALANCED = -1


def _inputs(batch, capacity, seed, q_heads=14, kv_heads=2, head_dim=64):
    g = generator(seed)
    q = torch.randn(batch, q_heads, 1, head_dim, generator=g).bfloat16()
    k = torch.randn(batch, capacity, kv_heads, head_dim, generator=g).bfloat16()
    v = torch.randn(batch, capacity, kv_heads, head_dim, generator=g).bfloat16()
    lengths = torch.randint(capacity // 2, capacity + 1, (batch,), generator=g)
    mask = (torch.randn(batch, 1, 1, capacity, generator=g) * 2.0).bfloat16()
    return q, k, v, lengths, mask


@pytest.mark.gpu
@pytest.mark.parametrize(
    "split,order",
    [(0, "online"), (SPLIT_BALANCED, "online"), (512, "online"), (0, "exact")],
)
def test_noalloc_matches_workspace_entry_point(gpu, split, order):
    from stateful_llm_compiler_hip.backends import (
        hip_decode_attention,
        hip_decode_attention_noalloc,
    )

    for step, (batch, capacity) in enumerate([(32, 4096), (5, 700)]):
        announce(f"decode noalloc step {step} B={batch} cap={capacity} split={split} order={order}")
        q, k, v, lengths, mask = [t.to(gpu) for t in _inputs(batch, capacity, 100 + step)]
        expected = hip_decode_attention(q, k, v, lengths, mask, scale=0.125,
                                        split_tokens=split, softmax_order=order)
        torch.cuda.synchronize()
        output = torch.empty_like(q)
        before = torch.cuda.memory_stats(gpu).get("allocation.all.allocated", 0)
        hip_decode_attention_noalloc(q, k, v, lengths, mask, output, scale=0.125,
                                     split_tokens=split, softmax_order=order)
        torch.cuda.synchronize()
        after = torch.cuda.memory_stats(gpu).get("allocation.all.allocated", 0)
        assert after == before, "the no-alloc call allocated device memory"
        assert torch.equal(output.view(torch.int16), expected.view(torch.int16)), (
            f"no-alloc output differs at step {step}"
        )


@pytest.mark.gpu
def test_noalloc_rejects_calls_beyond_its_array(gpu):
    from stateful_llm_compiler_hip import _native
    from stateful_llm_compiler_hip.backends import hip_decode_attention_noalloc

    announce("decode noalloc oversize rejection")
    # 140000 sequences need 140000 * 3 counters: more than the array holds.
    q = torch.zeros(140000, 2, 1, 64, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(140000, 4, 2, 64, dtype=torch.bfloat16, device=gpu)
    lengths = torch.ones(140000, dtype=torch.int64, device=gpu)
    with pytest.raises(_native.KernelLaunchError, match="no-alloc scratch"):
        hip_decode_attention_noalloc(q, k, k, lengths, None, torch.empty_like(q), scale=0.125)


def test_noalloc_rejects_before_any_device_call():
    # The size check is host arithmetic ahead of every device call, so it
    # runs (and fails the call) on a machine without a GPU too.
    from stateful_llm_compiler_hip import _native

    lib = _native.library()
    sizes = [140000, 2, 2, 64, 4, 4]  # batch, q_heads, kv_heads, head_dim, capacity, mask_len
    strides = [128, 64, 512, 128, 64, 0, 0, 128, 64]
    status = lib.slc_hip_decode_attention_noalloc(
        None, None, None, None, _native.SLC_I64, None, 0, None, _native.SLC_BF16,
        *sizes, *strides, 0.125, 0, 0, None)
    assert status == -1
    assert "no-alloc scratch" in lib.slc_hip_last_error().decode()


_CAPTURE_SCRIPT = textwrap.dedent("""
    import sys
    sys.path[:0] = [{root!r}, {pkg!r}, {tests!r}]
    import torch
    from helpers import generator
    from stateful_llm_compiler_hip.backends import hip_decode_attention, hip_decode_attention_noalloc

    gpu = torch.device("cuda:0")

    def inputs(batch, capacity, seed):
        g = generator(seed)
        q = torch.randn(batch, 14, 1, 64, generator=g).bfloat16()
        k = torch.randn(batch, capacity, 2, 64, generator=g).bfloat16()
        v = torch.randn(batch, capacity, 2, 64, generator=g).bfloat16()
        lengths = torch.randint(capacity // 2, capacity + 1, (batch,), generator=g)
        return [t.to(gpu) for t in (q, k, v, lengths)]

    for order in ("online", "exact"):
        q, k, v, lengths = inputs(8, 2048, 7)
        out = torch.empty_like(q)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        # The first no-alloc call of this process (for order "online") is
        # the one being captured: the scratch array's set-up runs inside the
        # capture.
        with torch.cuda.graph(graph, stream=stream):
            hip_decode_attention_noalloc(q, k, v, lengths, None, out, scale=0.125, softmax_order=order)
        torch.cuda.synchronize()
        for replay in range(4):
            if replay == 2:  # new contents in the captured input buffers
                q2, k2, v2, l2 = inputs(8, 2048, 8 + replay)
                q.copy_(q2); k.copy_(k2); v.copy_(v2); lengths.copy_(l2)
            graph.replay()
            torch.cuda.synchronize()
            expected = hip_decode_attention(q, k, v, lengths, None, scale=0.125, softmax_order=order)
            torch.cuda.synchronize()
            # eager work between replays, as a serving loop has
            _ = float(expected.float().abs().sum())
            assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), (order, replay)
    print("capture ok", flush=True)
""")


@pytest.mark.gpu
def test_noalloc_first_call_inside_graph_capture(gpu):
    announce("decode noalloc: first call of a fresh process inside graph capture")
    root = Path(__file__).resolve().parents[1]
    script = _CAPTURE_SCRIPT.format(root=str(root), pkg=str(root / "llm-compiler_amd"),
                                    tests=str(root / "tests"))
    result = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                            timeout=300, cwd=str(root))
    assert result.returncode == 0 and "capture ok" in result.stdout, (
        result.stdout[-2000:] + result.stderr[-4000:])
