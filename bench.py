"""Benchmark of the KernelIR hot path on one MI355X.

Headline (BASELINE.json metric): serve.decode_attention HBM GB/s at the
Qwen2-0.5B GQA shape (14 query / 2 KV heads, head_dim 64, bf16), batch 32,
per-sequence lengths uniform in [L/2, L] for L = 8192.  One step
is one decode-attention launch over that batch with all inputs resident in
HBM.  ``value`` is algorithmic bytes x steps / wall time of the timed region;
``roofline`` divides the algorithmic bytes of one launch by the launch's mean
duration measured with HIP events on the launch stream.  The CPU baseline is
the oracle (eager PyTorch restatement of the reference executor) on a bounded
sample of the same workload on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import itertools
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "llm-compiler_amd"))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "decode-attn HBM GB/s (% of peak) + decode tok/s, Qwen2-0.5B shape, 1 GPU"

BATCH, QH, KVH, D, LMAX = 32, 14, 2, 64, 8192
SEED = 2


def decode_inputs(device, batch=BATCH, lmax=LMAX, seed=SEED):
    g = torch.Generator(device="cpu").manual_seed(seed)
    lengths = torch.randint(lmax // 2, lmax + 1, (batch,), generator=g)
    query = torch.randn(batch, QH, 1, D, generator=g).bfloat16()
    key = torch.randn(batch, lmax, KVH, D, generator=g).bfloat16()
    value = torch.randn(batch, lmax, KVH, D, generator=g).bfloat16()
    mask = torch.zeros(batch, 1, 1, lmax, dtype=torch.bfloat16)
    tensors = [query, key, value, lengths, mask]
    return [t.to(device) for t in tensors]


def decode_bytes(lengths: torch.Tensor, batch=BATCH) -> int:
    """Algorithmic HBM bytes of one decode-attention launch (bf16).

    K and V rows of every attended token (2 x KVH x D x 2 B = 512 B/token), the
    mask entry of every attended token (2 B), q and the output (B x QH x D x
    2 B each) and the int64 lengths.
    """

    tokens = int(lengths.sum().item())
    return tokens * (2 * KVH * D * 2 + 2) + 2 * batch * QH * D * 2 + batch * 8


def cpu_baseline(seconds_budget: float = 20.0) -> dict:
    """Oracle decode attention on the host cores over a bounded sample."""

    sys.path.insert(0, str(ROOT))
    from oracle import kernels as ref

    sample_batch = 4
    q, k, v, lengths, mask = decode_inputs("cpu", batch=sample_batch)
    ref.decode_attention(q, k, v, lengths, mask, groups=QH // KVH, scale=D**-0.5)
    reps, start = 0, time.perf_counter()
    while True:
        ref.decode_attention(q, k, v, lengths, mask, groups=QH // KVH, scale=D**-0.5)
        reps += 1
        elapsed = time.perf_counter() - start
        if elapsed > seconds_budget / 4 or reps >= 20:
            break
    per_call = elapsed / reps
    gbs = decode_bytes(lengths, batch=sample_batch) / per_call / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "cores_affinity": len(os.sched_getaffinity(0)),
        "torch_threads": torch.get_num_threads(),
        "kind": "port",
        "sample": (
            f"oracle decode_attention (eager torch CPU, bf16), batch {sample_batch} "
            f"of the same L={LMAX} workload, {reps} reps, {per_call * 1e3:.1f} ms/call"
        ),
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_attention_b32_l8192.md"


def profiled_traffic() -> int | None:
    """HBM bytes per launch of the dominant kernel, from the committed
    FETCH_SIZE/WRITE_SIZE counter runs (calibrated against a plain copy)."""

    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def dominant_kernel_us(call, reps: int, repeats: int = 20) -> float:
    """Mean duration of one launch of the dominant kernel of ``call()``, from
    HIP events the library records around it on its launch stream.  While the
    events are armed the library launches that kernel ``repeats`` times back
    to back (it rewrites the same outputs), so the launch latency of a single
    call is amortised and the figure matches the profiler's kernel time."""

    from stateful_llm_compiler_hip import _native

    lib = _native.library()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for b, e in pairs:  # creates the underlying hipEvent_t handles
        b.record()
        e.record()
    torch.cuda.synchronize()
    try:
        lib.slc_hip_set_timing_repeats(repeats)
        for b, e in pairs:
            lib.slc_hip_set_timing_events(b.cuda_event, e.cuda_event)
            call()
    finally:
        lib.slc_hip_set_timing_events(None, None)
        lib.slc_hip_set_timing_repeats(1)
    torch.cuda.synchronize()
    return 1e3 * sum(b.elapsed_time(e) for b, e in pairs) / reps / repeats


def bench_decode_attention(steps: int, warmup: int, split_tokens: int) -> dict:
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    device = torch.device("cuda:0")
    q, k, v, lengths, mask = decode_inputs(device)
    nbytes = decode_bytes(lengths.cpu())

    def step():
        return hip_decode_attention(q, k, v, lengths, mask, scale=D**-0.5, split_tokens=split_tokens)

    # Warm the workspace and the library, then capture steps in HIP graphs so
    # host launch overhead does not throttle a ~20 us step: a graph of
    # GRAPH_STEPS back-to-back steps (how a serving loop runs decode) and a
    # one-step graph for the remainder, so the timed region runs exactly
    # `steps` steps.
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(GRAPH_STEPS):
            out = step()
    single = torch.cuda.CUDAGraph()
    with torch.cuda.graph(single):
        out = step()
    for _ in range(max(1, warmup // GRAPH_STEPS)):
        graph.replay()
    torch.cuda.synchronize()

    # Per-step duration of the graphed steps (split + merge kernels and the
    # gaps between launches) with events on the replay stream.
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
    for s, e in events:
        s.record()
        graph.replay()
        e.record()
    torch.cuda.synchronize()
    step_us = 1e3 * sum(s.elapsed_time(e) for s, e in events) / len(events) / GRAPH_STEPS

    # Duration of one launch of the dominant (split-sequence) kernel.
    kernel_us = dominant_kernel_us(step, 100)

    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps // GRAPH_STEPS):
        graph.replay()
    for _ in range(steps % GRAPH_STEPS):
        single.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    del out
    achieved = nbytes / (kernel_us * 1e-6) / 1e9
    return {
        "elapsed": elapsed,
        "bytes": nbytes,
        "kernel_us": kernel_us,
        "step_us": step_us,
        "achieved_gbs": achieved,
        "tokens": int(lengths.sum().item()),
    }


PAGE_TOKENS = 64


def bench_paged_attention(contiguous: dict) -> dict:
    """The headline decode attention over the paged KV layout: the same
    tokens in 64-token pages scattered over the pool by a random block table.
    Same timing as the contiguous leg (dominant kernel by HIP events, graph
    step time); the ratio to the contiguous kernel is the paging overhead."""

    from stateful_llm_compiler_hip.backends import hip_paged_decode_attention

    device = torch.device("cuda:0")
    q, k, v, lengths, mask = decode_inputs(device)
    pages = LMAX // PAGE_TOKENS
    g = torch.Generator(device="cpu").manual_seed(SEED + 1)
    table = torch.randperm(BATCH * pages, generator=g).view(BATCH, pages).to(torch.int32).to(device)
    index = table.view(-1).long()
    key_pool = torch.empty(BATCH * pages, PAGE_TOKENS, KVH, D, dtype=k.dtype, device=device)
    value_pool = torch.empty_like(key_pool)
    key_pool[index] = k.view(BATCH * pages, PAGE_TOKENS, KVH, D)
    value_pool[index] = v.view(BATCH * pages, PAGE_TOKENS, KVH, D)
    del k, v

    def step():
        return hip_paged_decode_attention(q, key_pool, value_pool, table, lengths, mask, scale=D**-0.5)

    step_us = _time_graph(step, reps=GRAPH_STEPS, outer=20)
    kernel_us = dominant_kernel_us(step, 100)
    return {
        "workload": f"same B/L/lengths as the headline, {PAGE_TOKENS}-token pages, random int32 block table",
        "kernel_us": round(kernel_us, 3),
        "step_us_graph": round(step_us, 3),
        "achieved_gbs": round(contiguous["bytes"] / (kernel_us * 1e-6) / 1e9, 2),
        "kernel_vs_contiguous": round(kernel_us / contiguous["kernel_us"], 4),
        "step_vs_contiguous": round(step_us / contiguous["step_us"], 4),
    }


MFMA_PEAK_TFLOPS = 2500.0  # dense bf16
GRAPH_STEPS = 10  # decode-attention steps per graph replay


def _time_graph(fn, reps: int = 20, outer: int = 5) -> float:
    """Mean microseconds per call of ``fn`` from replays of a HIP graph that
    holds ``reps`` back-to-back calls (launch gaps included, host overhead
    not)."""

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(outer):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return 1e3 * start.elapsed_time(end) / (reps * outer)


def bench_kernels() -> dict:
    """The other hot-path ops at their benchmark-config (3 and 4) shapes, each against
    the roofline that bounds it (bf16; synthetic N(0,1) data)."""

    from stateful_llm_compiler_hip.backends import (
        hip_kv_store, hip_linear, hip_prefill_attention, hip_prefill_mask_tiles, hip_rms_norm,
        hip_rope,
    )

    dev = torch.device("cuda:0")
    g = torch.Generator(device="cuda:0").manual_seed(7)
    bf = torch.bfloat16
    out: dict[str, dict] = {}

    def mfma(name, us, flops, shape):
        tf = flops / (us * 1e-6) / 1e12
        out[name] = {"shape": shape, "us": round(us, 2), "TFLOP/s": round(tf, 1),
                     "frac_of_mfma_peak": round(tf / MFMA_PEAK_TFLOPS, 4)}

    def hbm(name, us, nbytes, shape):
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"shape": shape, "us": round(us, 2), "GB/s": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}

    # prefill attention, causal, config 4's largest case (B=8, T=4096)
    B, T = 8, 4096
    q = torch.randn(B, QH, T, D, device=dev, generator=g, dtype=bf)
    k = torch.randn(B, KVH, T, D, device=dev, generator=g, dtype=bf)
    v = torch.randn(B, KVH, T, D, device=dev, generator=g, dtype=bf)
    flops = 4 * B * QH * D * T * (T + 1) // 2
    us = _time_graph(lambda: hip_prefill_attention(q, k, v, None, scale=D**-0.5, causal=True), reps=5)
    mfma("prefill_attention_causal", us, flops, "B8 QH14 KVH2 T4096 D64")
    mask = torch.zeros(T, T, device=dev, dtype=bf).masked_fill(
        torch.ones(T, T, device=dev, dtype=torch.bool).triu(1), float("-inf")).expand(B, 1, T, T).contiguous()
    # The mask's tile classes are computed once per mask (the model's 24
    # layers share one), then every attention call uses them.
    tiles = hip_prefill_mask_tiles(mask)
    us = _time_graph(lambda: hip_prefill_attention(q, k, v, mask, scale=D**-0.5, mask_tiles=tiles), reps=5)
    mfma("prefill_attention_mask", us, flops, "B8 QH14 KVH2 T4096 D64, explicit [B,1,T,T] causal mask")
    us = _time_graph(lambda: hip_prefill_mask_tiles(mask), reps=5)
    hbm("prefill_mask_tiles", us, B * T * T * 2, "B8 T4096 bf16 [B,1,T,T] mask, classes per 64x64 tile")
    del q, k, v, mask

    # linear: the four projection shapes at M = 4096 and the MLP at M = 32768
    for m, n, kk in ((4096, 896, 896), (4096, 128, 896), (4096, 4864, 896), (4096, 896, 4864),
                     (32768, 4864, 896)):
        x = torch.randn(m, kk, device=dev, generator=g, dtype=bf)
        w = torch.randn(n, kk, device=dev, generator=g, dtype=bf) * 0.02
        us = _time_graph(lambda: hip_linear(x, w), reps=10)
        mfma(f"linear_m{m}_n{n}_k{kk}", us, 2 * m * n * kk, f"M{m} N{n} K{kk}")
    # decode-shaped linears (M = 8): weight streaming.  Each graph holds 60
    # calls cycling over enough weight copies (> 256 MB, the Infinity Cache)
    # that every call streams its weights from HBM; a graph of a few calls
    # would time the graph launch instead of the kernel.
    for n, kk in ((4864, 896), (896, 4864), (151936, 896)):
        x = torch.randn(8, kk, device=dev, generator=g, dtype=bf)
        copies = max(1, -(-(300 << 20) // (n * kk * 2)))
        ws = [torch.randn(n, kk, device=dev, generator=g, dtype=bf) * 0.02 for _ in range(copies)]
        turn = itertools.cycle(range(copies))
        us = _time_graph(lambda: hip_linear(x, ws[next(turn)]), reps=60, outer=3)
        hbm(f"linear_m8_n{n}_k{kk}", us, (n * kk + 8 * kk + 8 * n) * 2, f"M8 N{n} K{kk}")
        del ws

    # the fused decode-step kernels at batch 8 (Qwen2-0.5B layer shapes), each
    # graph of 60 calls cycling over weight / KV copies past the Infinity Cache
    from stateful_llm_compiler_hip.backends import (
        hip_linear_residual, hip_norm_linear_group, hip_norm_linear_swiglu,
        hip_rope_decode_attention,
    )

    def copies_for(nbytes):
        return max(2, -(-(300 << 20) // nbytes))

    hs = torch.randn(8, 1, 896, device=dev, generator=g, dtype=bf)
    nw = torch.rand(896, device=dev, generator=g).to(bf) + 0.5
    res = torch.randn(8, 1, 896, device=dev, generator=g, dtype=bf)
    wsz = 2 * 896 * (896 + 128 + 128)
    qkv = [[torch.randn(n, 896, device=dev, generator=g, dtype=bf) * 0.02 for n in (896, 128, 128)]
           for _ in range(copies_for(wsz))]
    qkv_b = [torch.randn(n, device=dev, generator=g, dtype=bf) * 0.02 for n in (896, 128, 128)]
    turn = itertools.cycle(range(len(qkv)))
    us = _time_graph(lambda: hip_norm_linear_group(hs, nw, qkv[next(turn)], qkv_b, epsilon=1e-6),
                     reps=60, outer=3)
    hbm("decode_norm_qkv", us, wsz + 2 * 8 * 896 * 2 + 2 * 8 * 1152, "M8 norm + Q/K/V 896->896+128+128")
    del qkv
    wsz = 2 * 2 * 4864 * 896
    gu = [(torch.randn(4864, 896, device=dev, generator=g, dtype=bf) * 0.02,
           torch.randn(4864, 896, device=dev, generator=g, dtype=bf) * 0.02)
          for _ in range(copies_for(wsz))]
    turn = itertools.cycle(range(len(gu)))
    us = _time_graph(lambda: hip_norm_linear_swiglu(hs, nw, *gu[next(turn)], epsilon=1e-6),
                     reps=60, outer=3)
    hbm("decode_norm_swiglu", us, wsz + 2 * 8 * 896 + 2 * 8 * 4864, "M8 norm + gate/up 896->4864 + SwiGLU")
    del gu
    for name, n_in, n_out in (("decode_o_residual", 896, 896), ("decode_down_residual", 4864, 896)):
        wsz = 2 * n_in * n_out
        xs = torch.randn(8, 1, n_in, device=dev, generator=g, dtype=bf)
        ws = [torch.randn(n_out, n_in, device=dev, generator=g, dtype=bf) * 0.02
              for _ in range(copies_for(wsz))]
        turn = itertools.cycle(range(len(ws)))
        us = _time_graph(lambda: hip_linear_residual(xs, ws[next(turn)], None, res), reps=60, outer=3)
        hbm(name, us, wsz + 2 * 8 * (n_in + 2 * n_out), f"M8 {n_in}->{n_out} + residual")
        del ws
    # RoPE + KV store + advance + attention at the decode step's shape: batch 8,
    # 600 tokens of a 2048-long mask (lengths into a separate tensor, so every
    # call sees the same 600)
    cap, length = 2048, 600
    kv_bytes = 2 * 8 * cap * KVH * D * 2
    kvs = [(torch.randn(8, cap, KVH, D, device=dev, generator=g, dtype=bf),
            torch.randn(8, cap, KVH, D, device=dev, generator=g, dtype=bf))
           for _ in range(copies_for(kv_bytes))]
    qd = torch.randn(8, 1, QH, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
    kd = torch.randn(8, 1, KVH, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
    cs = torch.randn(8, 1, D, device=dev, generator=g, dtype=bf)
    lens = torch.full((8,), length, device=dev, dtype=torch.int64)
    lens_out = torch.empty_like(lens)
    dmask = torch.zeros(8, 1, 1, cap, device=dev, dtype=bf)
    turn = itertools.cycle(range(len(kvs)))

    def rope_attention():
        kb, vb = kvs[next(turn)]
        return hip_rope_decode_attention(qd, kd, kd, cs, cs, kb, vb, lens, lens_out, dmask,
                                         scale=D**-0.5)

    us = _time_graph(rope_attention, reps=60, outer=3)
    hbm("decode_rope_attention", us, 8 * (length + 1) * KVH * D * 2 * 2 + 8 * cap * 2,
        "B8 QH14 KVH2 D64, 600 of a 2048 mask: RoPE + KV store + advance + attention")
    del kvs

    # rms_norm 32768 x 896
    x = torch.randn(32768, 896, device=dev, generator=g, dtype=bf)
    wn = torch.randn(896, device=dev, generator=g, dtype=bf)
    us = _time_graph(lambda: hip_rms_norm(x, wn, epsilon=1e-6, round_before_weight=True))
    hbm("rms_norm", us, (2 * x.numel() + 896) * 2, "rows 32768 hidden 896")

    # rope B=64 T=512
    B, T = 64, 512
    q = torch.randn(B, QH, T, D, device=dev, generator=g, dtype=bf)
    k = torch.randn(B, KVH, T, D, device=dev, generator=g, dtype=bf)
    cos = torch.randn(B, T, D, device=dev, generator=g, dtype=bf)
    sin = torch.randn(B, T, D, device=dev, generator=g, dtype=bf)
    us = _time_graph(lambda: hip_rope(q, k, cos, sin))
    hbm("rope", us, (2 * (q.numel() + k.numel()) + 2 * B * T * D) * 2, "B64 QH14 KVH2 T512 D64")
    del q, cos, sin

    # kv_store B=64 T=512 into a [64, 8192, 2, 64] buffer pair
    kb = torch.zeros(B, 8192, KVH, D, device=dev, dtype=bf)
    vb = torch.zeros_like(kb)
    vv = torch.randn(B, KVH, T, D, device=dev, generator=g, dtype=bf)
    pos = torch.randint(0, 4096, (B,), device=dev, generator=g)
    us = _time_graph(lambda: hip_kv_store(kb, vb, k, vv, pos))
    hbm("kv_store", us, 2 * (k.numel() + vv.numel()) * 2 + B * 8, "B64 H2 T512 D64 -> cap 8192")
    return out


MODEL_BATCH, PROMPT, CAPACITY, DECODE_STEPS = 8, 512, 2048, 128


def bench_decode_tokens(seed: int = 5) -> dict:
    """Config 5: 24-layer Qwen2-0.5B-shape CausalLM (bf16, random init, tied
    embeddings), stateful prefill of 512 random tokens at batch 8 into a KV
    state of capacity 2048, then 128 greedy decode steps on the same buffers.
    The decode step (all 24 layers + LM head + argmax) is one HIP-graph replay
    of the fully lowered KernelIR function."""

    from stateful_llm_compiler_hip.qwen2 import Qwen2Config, causal_prefill_mask, init_weights
    from stateful_llm_compiler_hip.runtime import Qwen2Runtime

    device = torch.device("cuda:0")
    config = Qwen2Config()
    weights = init_weights(config, seed=seed, dtype=torch.bfloat16, device=device, draw_on_device=True)
    runtime = Qwen2Runtime(config, weights, capacity=CAPACITY, dtype=torch.bfloat16,
                           device="cuda:0", validate=False)
    g = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.randint(0, config.vocab_size, (MODEL_BATCH, PROMPT), generator=g).to(device)
    mask = causal_prefill_mask(MODEL_BATCH, PROMPT, device=device)
    pos = torch.arange(PROMPT, device=device).view(1, -1).expand(MODEL_BATCH, -1).contiguous()

    runtime.prefill(ids, mask, pos)  # warm-up (kernel loading, allocator)
    torch.cuda.synchronize()
    start = time.perf_counter()
    logits, state = runtime.prefill(ids, mask, pos)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - start

    decoder = runtime.graph_decoder(state, logits[:, -1].argmax(-1))
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(DECODE_STEPS):
        decoder.step()
    torch.cuda.synchronize()
    decode_s = time.perf_counter() - start
    lengths = state.lengths[0].tolist()
    state.check_capacity()
    return {
        "decode_tok_s": MODEL_BATCH * DECODE_STEPS / decode_s,
        "decode_ms_per_step": decode_s * 1e3 / DECODE_STEPS,
        "prefill_tok_s": MODEL_BATCH * PROMPT / prefill_s,
        "prefill_ms": prefill_s * 1e3,
        "final_lengths": sorted(set(lengths)),
        "decode_ops_per_step": len(runtime.decode_result.module.functions[0].block.operations),
        "coverage": runtime.decode_result.coverage.coverage,
    }


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=2000)
    parser.add_argument("--warmup", type=int, default=50)
    parser.add_argument("--split-tokens", type=int, default=0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-model", action="store_true", help="skip the decode tok/s leg")
    parser.add_argument("--no-paged", action="store_true", help="skip the paged-KV decode attention leg")
    parser.add_argument("--no-kernels", action="store_true", help="skip the other-op roofline table")
    parser.add_argument(
        "--model-only", action="store_true",
        help="only run the decode tok/s leg and print its numbers (for profiling the decode step)",
    )
    parser.add_argument(
        "--calibrate-copy", type=int, default=0, metavar="MIB",
        help="only run 5 plain device-to-device copies of MIB MiB (counter calibration)",
    )
    args = parser.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures the single-GPU hot path only; this build has no "
            "multi-GPU path (see the sharding paragraph of the design notes).",
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (torch.cuda.is_available() is False)", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        src = torch.ones(args.calibrate_copy << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes": src.numel()}))
        return

    if args.model_only:
        print(json.dumps(bench_decode_tokens()))
        return

    result = bench_decode_attention(args.steps, args.warmup, args.split_tokens)
    value = result["bytes"] * args.steps / result["elapsed"] / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(result["elapsed"] * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/K/V, lengths U[L/2, L])",
        "config": {
            "workload": "serve.decode_attention GQA QH14/KVH2/D64, B=32, L=8192, lengths U[4096,8192], contiguous_bshd KV, int64 lengths, zero bf16 mask",
            "global_batch": BATCH,
            "seq_len": LMAX,
            "attended_tokens": result["tokens"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(result["achieved_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(result["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "kernel": "decode_attention_mfma_kernel (split-sequence, partials merged by the last workgroup of each (batch, kv-head))",
            "kernel_us": round(result["kernel_us"], 3),
            "step_us_graph": round(result["step_us"], 3),
            "algorithmic_bytes": result["bytes"],
        },
    }
    if not args.no_paged:
        line["paged"] = bench_paged_attention(result)
    if not args.no_model:
        tok = bench_decode_tokens()
        line["decode_tok_s"] = round(tok["decode_tok_s"], 1)
        line["decode"] = {
            "workload": "24-layer Qwen2-0.5B-shape CausalLM bf16 random init, batch 8, prefill 512 into capacity 2048, 128 greedy steps, fast mode, full lowering, HIP-graph decode step",
            "ms_per_step": round(tok["decode_ms_per_step"], 4),
            "prefill_tok_s": round(tok["prefill_tok_s"], 1),
            "prefill_ms": round(tok["prefill_ms"], 2),
            "ops_per_step": tok["decode_ops_per_step"],
            "lowering_coverage": tok["coverage"],
            "final_lengths": tok["final_lengths"],
        }
    if not args.no_kernels:
        line["kernels"] = bench_kernels()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
