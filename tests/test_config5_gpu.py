"""Config 5 end to end: the 24-layer Qwen2-0.5B-shape CausalLM (bf16, random
init, vocab 151936, tied embeddings), stateful prefill of 512 tokens at batch
8 into a KV state of capacity 2048, then teacher-forced decode steps on the
same buffers, compiled with strict full lowering (no PyTorch fallback), in
both numerical modes, against the eager unbufferized model run on the same
GPU (the reference checks its compiled Qwen2 paths the same way,
tests/test_qwen2_prefill.py:292-459, tests/test_multilayer_decode.py:211-281).

pytorch_compatible mode must be element-wise equal to eager.  fast mode is
checked per op family (see ``test_config5_fast_mode``).
"""

from __future__ import annotations

import pytest
import torch

from helpers import announce
from oracle.qwen2_model import EagerQwen2
from stateful_llm_compiler_hip.qwen2 import Qwen2Config, causal_prefill_mask, init_weights
from stateful_llm_compiler_hip.runtime import Qwen2Runtime

pytestmark = pytest.mark.gpu

CONFIG5 = Qwen2Config()
BATCH, PROMPT, CAPACITY, STEPS = 8, 512, 2048, 3
BF16_ATOL = 2e-2


@pytest.fixture(scope="module")
def config5(gpu):
    announce("config5 eager reference (24 layers, B8, prompt 512)")
    weights = init_weights(CONFIG5, seed=5, dtype=torch.bfloat16, device=gpu, draw_on_device=True)
    g = torch.Generator(device="cpu").manual_seed(5)
    ids = torch.randint(0, CONFIG5.vocab_size, (BATCH, PROMPT), generator=g).to(gpu)
    mask = causal_prefill_mask(BATCH, PROMPT, device=gpu)
    pos = torch.arange(PROMPT, device=gpu).view(1, -1).expand(BATCH, -1).contiguous()
    eager = EagerQwen2(CONFIG5, weights)
    with torch.no_grad():
        logits, cache = eager.prefill(ids, mask, pos)
        steps = [(logits[:, -1:].clone(), None)]
        tokens = []
        token = logits[:, -1].argmax(-1, keepdim=True)
        for step in range(STEPS):
            length = PROMPT + step
            tokens.append(token)
            dmask = torch.zeros(BATCH, 1, 1, length + 1, dtype=torch.bfloat16, device=gpu)
            step_logits, cache = eager.decode(token, dmask, torch.full((BATCH, 1), length, device=gpu), cache)
            steps.append((step_logits, dmask))
            token = step_logits[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    return dict(weights=weights, ids=ids, mask=mask, pos=pos, prefill_logits=logits,
                steps=steps[1:], tokens=tokens, cache=cache)


def _run(config5, gpu, **runtime_args):
    """Prefill and teacher-forced decode through the compiled runtime; yields
    (what, actual, expected) pairs of logits and, after the last step, of
    every layer's K and V."""

    rt = Qwen2Runtime(CONFIG5, config5["weights"], capacity=CAPACITY, dtype=torch.bfloat16,
                      device=str(gpu), **runtime_args)
    assert rt.prefill_result.coverage.is_complete and rt.decode_result.coverage.is_complete
    logits, state = rt.prefill(config5["ids"], config5["mask"], config5["pos"])
    pairs = [("prefill logits", logits, config5["prefill_logits"])]
    pointers = [(k.data_ptr(), v.data_ptr()) for k, v in zip(state.keys, state.values)]
    for step, (token, (expected, dmask)) in enumerate(zip(config5["tokens"], config5["steps"])):
        logits, state = rt.decode(token, dmask, state)
        pairs.append((f"step {step} logits", logits, expected))
    length = PROMPT + STEPS
    for slot, (k, v) in enumerate(config5["cache"]):
        assert state.lengths[slot].tolist() == [length] * BATCH
        pairs.append((f"layer {slot} K", state.keys[slot][:, :length].transpose(1, 2), k))
        pairs.append((f"layer {slot} V", state.values[slot][:, :length].transpose(1, 2), v))
    assert pointers == [(k.data_ptr(), v.data_ptr()) for k, v in zip(state.keys, state.values)]
    state.check_capacity()
    torch.cuda.synchronize()
    return pairs


def _errors(pairs):
    return {what: float((a.float() - e.float()).abs().max()) for what, a, e in pairs}


def test_config5_pytorch_compatible_is_exact(gpu, config5):
    announce("config5 pytorch_compatible vs eager (element-wise equal)")
    for what, actual, expected in _run(config5, gpu, numerical_mode="pytorch_compatible"):
        assert torch.equal(actual, expected), (what, float((actual.float() - expected.float()).abs().max()))


def test_config5_fast_mode(gpu, config5):
    """bf16 fast mode with full lowering and fusion.

    Over 24 layers the residual stream amplifies any last-bit difference of
    any op: the eager model itself, with only its linears rounded once from
    fp32 sums instead of by the BLAS library's accumulation order, moves its
    logits by about 0.07 and its deepest K/V by about 0.06 (printed below),
    so the 2e-2 per-element bar is met by layer 0 and not by layer 23 of any
    implementation that is not the eager model bit for bit.  The checks are
    therefore:
      * layer 0 K/V within 2e-2 of eager (one layer of HIP ops);
      * logits and K/V no farther from eager than that GEMM-rounding
        yardstick, within 1.5x;
      * the logits no farther from the model evaluated in fp32 (same bf16
        weights) than eager's own bf16 logits are, within 1.25x.
    """

    announce("config5 fast: full HIP")
    pairs = _run(config5, gpu)
    full = _errors(pairs)
    print("fast mode vs eager:", {k: round(v, 4) for k, v in full.items() if "logits" in k},
          "K/V by layer:", [round(max(full[f"layer {i} K"], full[f"layer {i} V"]), 4)
                            for i in range(CONFIG5.num_layers)])
    hip_prefill = pairs[0][1]

    announce("config5 eager with exactly rounded linears (GEMM-rounding yardstick)")
    weights = config5["weights"]
    import oracle.qwen2_model as qm

    original = qm.F.linear

    def rounded_linear(x, w, b=None):
        y = torch.matmul(x.float(), w.float().t())
        if b is not None:
            y = y + b.float()
        return y.to(x.dtype)

    qm.F.linear = rounded_linear
    try:
        with torch.no_grad():
            yard_logits, yard_cache = EagerQwen2(CONFIG5, weights).prefill(
                config5["ids"], config5["mask"], config5["pos"])
    finally:
        qm.F.linear = original
    eager_logits = config5["prefill_logits"]
    yard = {"logits": float((yard_logits.float() - eager_logits.float()).abs().max()),
            "K/V": max(float((a.float() - e.float()).abs().max())
                       for (ak, av), (ek, ev) in zip(yard_cache, config5["cache"])
                       for a, e in ((ak, ek[:, :, :PROMPT]), (av, ev[:, :, :PROMPT])))}
    del yard_logits, yard_cache
    print("yardstick vs eager:", {k: round(v, 4) for k, v in yard.items()})

    announce("config5 fp32 evaluation of the same bf16 weights")
    w32 = {k: v.float() for k, v in weights.items()}
    with torch.no_grad():
        exact, _ = EagerQwen2(CONFIG5, w32).prefill(config5["ids"], config5["mask"].float(), config5["pos"])
    eager_err = float((eager_logits.float() - exact).abs().max())
    hip_err = float((hip_prefill.float() - exact).abs().max())
    print(f"prefill logits vs fp32 model: eager {eager_err:.4f}, HIP {hip_err:.4f}")

    assert max(full["layer 0 K"], full["layer 0 V"]) <= BF16_ATOL, full
    logits = max(v for k, v in full.items() if "logits" in k)
    kv = max(v for k, v in full.items() if "logits" not in k)
    assert logits <= 1.5 * yard["logits"], (logits, yard)
    assert kv <= 1.5 * yard["K/V"], (kv, yard)
    assert hip_err <= 1.25 * eager_err, (hip_err, eager_err)
