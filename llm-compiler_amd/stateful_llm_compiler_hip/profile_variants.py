"""Measure the HIP kernel variants on the current GPU and write a profile.

The counterpart of the reference's ``benchmarks/bench_rmsnorm.py --output``
(which writes the schema-v1 profile ``cost_model`` reads): for each op and
size it times every variant and records the latencies as ``hip_variants``,
next to ``hip_us`` (the automatic variant) so a reference-style reader still
finds a number.  Each latency is the mean per call of a HIP graph of
back-to-back calls replayed several times (launch gaps included, host
overhead not); RMSNorm calls cycle over enough input copies to stream from
HBM.

Usage: python -m stateful_llm_compiler_hip.profile_variants --output mi355x.json
"""

from __future__ import annotations

import argparse
import itertools
import json
from pathlib import Path

import torch

from ._native import LINEAR_TILES
from .backends import hip_decode_attention, hip_linear, hip_rms_norm
from .cost_model import SCHEMA_VERSION, split_tokens, waves_per_row

RMS_ROWS = (1, 8, 64, 512, 4096, 32768)
DECODE_SHAPES = ((1, 1024), (8, 1024), (8, 2048), (8, 8192), (32, 8192), (64, 8192), (8, 32768))
DECODE_VARIANTS = ("fixed", "balanced", "chunk512", "chunk1024")
# Qwen2-0.5B projections (N, K) and prefill row counts (batch x tokens).
LINEAR_SHAPES = ((896, 896), (128, 896), (4864, 896), (896, 4864))
LINEAR_ROWS = (128, 512, 1024, 2048, 4096, 8192, 32768)
LINEAR_VARIANTS = tuple(name for name in LINEAR_TILES if name != "auto")


def _graph_us(fn, calls: int = 20, replays: int = 5) -> float:
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    begin.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return 1e3 * begin.elapsed_time(end) / (calls * replays)


def profile_rms_norm(hidden: int, dtype: torch.dtype, device) -> list[dict]:
    rows_out = []
    g = torch.Generator(device=device).manual_seed(0)
    weight = torch.rand(hidden, device=device, generator=g).to(dtype) + 0.5
    for rows in RMS_ROWS:
        copies = max(1, -(-(256 << 20) // (rows * hidden * 2 * dtype.itemsize)))
        xs = [torch.randn(rows, hidden, device=device, generator=g, dtype=dtype)
              for _ in range(min(copies, 64))]
        latencies = {}
        for variant in ("wave", "block"):
            turn = itertools.cycle(xs)
            latencies[variant] = round(_graph_us(
                lambda: hip_rms_norm(next(turn), weight, epsilon=1e-6, round_before_weight=True,
                                     num_warps=waves_per_row(variant))), 3)
        rows_out.append({"rows": rows, "hidden_size": hidden, "dtype": _name(dtype),
                         "hip_us": min(latencies.values()), "hip_variants": latencies})
        del xs
    return rows_out


def profile_decode_attention(dtype: torch.dtype, device, q_heads=14, kv_heads=2, head_dim=64) -> list[dict]:
    rows_out = []
    g = torch.Generator().manual_seed(1)
    for batch, length in DECODE_SHAPES:
        q = torch.randn(batch, q_heads, 1, head_dim, generator=g).to(dtype).to(device)
        k = torch.randn(batch, length, kv_heads, head_dim, generator=g).to(dtype).to(device)
        v = torch.randn(batch, length, kv_heads, head_dim, generator=g).to(dtype).to(device)
        lengths = torch.randint(length // 2, length + 1, (batch,), generator=g).to(device)
        mask = torch.zeros(batch, 1, 1, length, dtype=dtype, device=device)
        latencies = {}
        for variant in DECODE_VARIANTS:
            split = split_tokens(variant)
            latencies[variant] = round(_graph_us(
                lambda: hip_decode_attention(q, k, v, lengths, mask, scale=head_dim ** -0.5,
                                             split_tokens=split)), 3)
        rows_out.append({"batch": batch, "mask_len": length, "q_heads": q_heads, "kv_heads": kv_heads,
                         "head_dim": head_dim, "dtype": _name(dtype), "lengths": "U[L/2, L]",
                         "hip_variants": latencies})
        del q, k, v
    return rows_out


def profile_linear(dtype: torch.dtype, device, shapes=LINEAR_SHAPES, rows=LINEAR_ROWS,
                   variants=LINEAR_VARIANTS) -> list[dict]:
    """Every tile of the prefill-sized linear at each (rows, N, K); the
    weights rotate over copies totalling at least 256 MB so each call streams
    its operands from HBM, as in a model's prefill."""

    rows_out = []
    g = torch.Generator(device=device).manual_seed(2)
    for n, k in shapes:
        for m in rows:
            per_call = (m * k + n * k) * dtype.itemsize
            copies = max(1, min(16, -(-(256 << 20) // per_call)))
            xs = [torch.randn(m, k, device=device, generator=g, dtype=dtype) for _ in range(copies)]
            ws = [(torch.randn(n, k, device=device, generator=g, dtype=dtype) * 0.02) for _ in range(copies)]
            latencies = {}
            for variant in variants:
                turn = itertools.cycle(list(zip(xs, ws)))

                def call(variant=variant, turn=turn):
                    x, w = next(turn)
                    hip_linear(x, w, tile=variant)

                latencies[variant] = round(_graph_us(call, calls=2 * copies), 3)
            rows_out.append({"rows": m, "out_features": n, "in_features": k, "dtype": _name(dtype),
                             "hip_variants": latencies})
            del xs, ws
    return rows_out


def _name(dtype: torch.dtype) -> str:
    return {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]


def build_profile(device="cuda:0") -> dict:
    device = torch.device(device)
    props = torch.cuda.get_device_properties(device)
    return {
        "schema_version": SCHEMA_VERSION,
        "target": {
            "device_name": torch.cuda.get_device_name(device),
            "compute_capability": getattr(props, "gcnArchName", "unknown"),
            "torch_version": torch.__version__,
            "triton_version": "none",
        },
        "benchmark": {"timing": "HIP graph of 20 back-to-back calls, 5 replays, mean per call"},
        "results": profile_rms_norm(896, torch.bfloat16, device),
        "decode_attention": profile_decode_attention(torch.bfloat16, device),
        "linear": profile_linear(torch.bfloat16, device),
    }


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--output", type=Path, required=True)
    args = parser.parse_args()
    profile = build_profile()
    args.output.parent.mkdir(parents=True, exist_ok=True)
    args.output.write_text(json.dumps(profile, indent=2) + "\n", encoding="utf-8")
    print(json.dumps(profile, indent=1))


if __name__ == "__main__":
    main()
