"""The Qwen2 ServeIR graphs, run by the CPU oracle executor, equal the eager
unbufferized model (config 1 of the plan: 2-layer Qwen2-shaped decoder, fp32,
batch 3, past 5 from a prefill, capacity 64, 4 greedy decode steps).  This pins
the graph builder and the KV-state semantics on the CPU."""

from __future__ import annotations

import torch

from helpers import generator
from oracle.executor import OracleExecutor, OracleKVState
from oracle.qwen2_model import EagerQwen2, causal_mask
from stateful_llm_compiler_hip.ir import verify_module
from stateful_llm_compiler_hip.qwen2 import (
    Qwen2Config,
    build_decode_module,
    build_prefill_module,
    init_weights,
    weight_arguments,
)

CONFIG1 = Qwen2Config(num_layers=2, vocab_size=1024)


def _setup(dtype=torch.float32, seed=0):
    weights = init_weights(CONFIG1, seed=seed, dtype=dtype)
    return weights, EagerQwen2(CONFIG1, weights)


def test_graphs_verify():
    verify_module(build_decode_module(CONFIG1, capacity=64, dtype=torch.float32, device="cpu"))
    verify_module(build_prefill_module(CONFIG1, capacity=64, dtype=torch.float32, device="cpu"))


def test_prefill_then_greedy_decode_matches_eager_fp32():
    weights, eager = _setup()
    batch, past, capacity, steps = 3, 5, 64, 4
    g = generator(1)
    ids = torch.randint(0, CONFIG1.vocab_size, (batch, past), generator=g)
    mask = causal_mask(batch, past)
    pos = torch.arange(past).view(1, -1).expand(batch, -1).clone()

    prefill = build_prefill_module(CONFIG1, capacity=capacity, dtype=torch.float32, device="cpu")
    decode = build_decode_module(CONFIG1, capacity=capacity, dtype=torch.float32, device="cpu")
    wargs = weight_arguments(CONFIG1, weights)
    logits, state = OracleExecutor().run(prefill, [ids, mask, pos] + wargs)
    e_logits, cache = eager.prefill(ids, mask, pos)
    assert torch.allclose(logits, e_logits, rtol=1e-5, atol=1e-5)
    assert [int(x) for x in state.lengths[0]] == [past] * batch

    token = logits[:, -1].argmax(-1, keepdim=True)
    for step in range(steps):
        length = past + step
        dmask = torch.zeros(batch, 1, 1, length + 1)
        logits, state = OracleExecutor().run(decode, [token, dmask, state] + wargs)
        e_logits, cache = eager.decode(token, dmask, torch.full((batch, 1), length), cache)
        torch.testing.assert_close(logits, e_logits, rtol=1e-5, atol=1e-5)
        for slot in range(CONFIG1.num_layers):
            assert [int(x) for x in state.lengths[slot]] == [length + 1] * batch
            k = state.keys[slot][:, : length + 1].transpose(1, 2)
            v = state.values[slot][:, : length + 1].transpose(1, 2)
            torch.testing.assert_close(k, cache[slot][0], rtol=1e-5, atol=1e-5)
            torch.testing.assert_close(v, cache[slot][1], rtol=1e-5, atol=1e-5)
        token = logits[:, -1].argmax(-1, keepdim=True)
    assert state.generation == steps * CONFIG1.num_layers + CONFIG1.num_layers


def test_decode_from_random_past_matches_eager():
    # The reference's differential setup: seeded random past K/V
    # (stateful_check.py:73-102), one decode step.
    weights, eager = _setup(seed=3)
    batch, past = 2, 7
    g = generator(9)
    cache = tuple(
        (torch.randn(batch, 2, past, 64, generator=g), torch.randn(batch, 2, past, 64, generator=g))
        for _ in range(CONFIG1.num_layers)
    )
    state = OracleKVState.from_layer_tensors(cache, capacity=32)
    token = torch.randint(0, CONFIG1.vocab_size, (batch, 1), generator=g)
    mask = torch.zeros(batch, 1, 1, past + 1)
    decode = build_decode_module(CONFIG1, capacity=32, dtype=torch.float32, device="cpu")
    logits, _ = OracleExecutor().run(decode, [token, mask, state] + weight_arguments(CONFIG1, weights))
    e_logits, _ = eager.decode(token, mask, torch.full((batch, 1), past), cache)
    torch.testing.assert_close(logits, e_logits, rtol=1e-5, atol=1e-5)
