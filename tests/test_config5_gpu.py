"""Config 5 end to end: the 24-layer Qwen2-0.5B-shape CausalLM (bf16, random
init, vocab 151936, tied embeddings), stateful prefill of 512 tokens at batch
8 into a KV state of capacity 2048, then teacher-forced decode steps on the
same buffers, compiled with strict full lowering (no PyTorch fallback), in
both numerical modes, against the eager unbufferized model run on the same
GPU (the reference checks its compiled Qwen2 paths the same way,
tests/test_qwen2_prefill.py:292-459, tests/test_multilayer_decode.py:211-281).

pytorch_compatible mode must be element-wise equal to eager.  fp32 fast
mode is held to 1e-5 relative on logits and every layer's K/V (no bf16
amplification, so all 24 HIP layers are pinned strictly).  bf16 fast mode is
checked per op family (see ``test_config5_fast_mode``) and its achieved
errors are printed as ``[record]`` lines.  The 128-step greedy run the
config names is ``test_config5_greedy_128_steps``.
"""

from __future__ import annotations

import pytest
import torch

import json

from helpers import announce, assert_fp32_close
from oracle.qwen2_model import EagerQwen2
from stateful_llm_compiler_hip.qwen2 import Qwen2Config, causal_prefill_mask, init_weights
from stateful_llm_compiler_hip.execution import PreallocatedKVCacheState
from stateful_llm_compiler_hip.runtime import Qwen2Runtime

pytestmark = pytest.mark.gpu

CONFIG5 = Qwen2Config()
BATCH, PROMPT, CAPACITY, STEPS = 8, 512, 2048, 3
GREEDY_STEPS = 128
BF16_ATOL = 2e-2


def _record(name, payload):
    """One machine-readable line per measured error set (kept in the log)."""

    print(f"[record] {name} " + json.dumps(payload, sort_keys=True), flush=True)


@pytest.fixture(scope="module")
def config5(gpu):
    announce("config5 eager reference (24 layers, B8, prompt 512)")
    weights = init_weights(CONFIG5, seed=5, dtype=torch.bfloat16, device=gpu, draw_on_device=True)
    g = torch.Generator(device="cpu").manual_seed(5)
    ids = torch.randint(0, CONFIG5.vocab_size, (BATCH, PROMPT), generator=g).to(gpu)
    mask = causal_prefill_mask(BATCH, PROMPT, device=gpu)
    pos = torch.arange(PROMPT, device=gpu).view(1, -1).expand(BATCH, -1).contiguous()
    logits, steps, tokens, cache = _eager_teacher_forced(weights, ids, mask, pos, torch.bfloat16, STEPS, gpu)
    return dict(weights=weights, ids=ids, mask=mask, pos=pos, prefill_logits=logits,
                steps=steps, tokens=tokens, cache=cache)


def _eager_teacher_forced(weights, ids, mask, pos, dtype, steps, device):
    """Eager prefill then ``steps`` greedy steps; returns what ``_run`` compares."""

    eager = EagerQwen2(CONFIG5, weights)
    with torch.no_grad():
        logits, cache = eager.prefill(ids, mask, pos)
        out, tokens = [], []
        token = logits[:, -1].argmax(-1, keepdim=True)
        for step in range(steps):
            length = PROMPT + step
            tokens.append(token)
            dmask = torch.zeros(BATCH, 1, 1, length + 1, dtype=dtype, device=device)
            step_logits, cache = eager.decode(token, dmask, torch.full((BATCH, 1), length, device=device), cache)
            out.append((step_logits, dmask))
            token = step_logits[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    return logits, out, tokens, cache


def _run(config5, gpu, **runtime_args):
    """Prefill and teacher-forced decode through the compiled runtime; yields
    (what, actual, expected) pairs of logits and, after the last step, of
    every layer's K and V."""

    dtype = config5.get("dtype", torch.bfloat16)
    rt = Qwen2Runtime(CONFIG5, config5["weights"], capacity=CAPACITY, dtype=dtype,
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
    _record("config5_bf16_fast_vs_eager", {
        "logits": {k: round(v, 5) for k, v in full.items() if "logits" in k},
        "K": [round(full[f"layer {i} K"], 5) for i in range(CONFIG5.num_layers)],
        "V": [round(full[f"layer {i} V"], 5) for i in range(CONFIG5.num_layers)]})
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
    _record("config5_bf16_gemm_rounding_yardstick", {k: round(v, 5) for k, v in yard.items()})

    announce("config5 fp32 evaluation of the same bf16 weights")
    w32 = {k: v.float() for k, v in weights.items()}
    with torch.no_grad():
        exact, _ = EagerQwen2(CONFIG5, w32).prefill(config5["ids"], config5["mask"].float(), config5["pos"])
    eager_err = float((eager_logits.float() - exact).abs().max())
    hip_err = float((hip_prefill.float() - exact).abs().max())
    _record("config5_bf16_prefill_logits_vs_fp32_model", {"eager": round(eager_err, 5), "hip": round(hip_err, 5)})

    assert max(full["layer 0 K"], full["layer 0 V"]) <= BF16_ATOL, full
    logits = max(v for k, v in full.items() if "logits" in k)
    kv = max(v for k, v in full.items() if "logits" not in k)
    assert logits <= 1.5 * yard["logits"], (logits, yard)
    assert kv <= 1.5 * yard["K/V"], (kv, yard)
    assert hip_err <= 1.25 * eager_err, (hip_err, eager_err)


def test_config5_fp32_fast_mode(gpu):
    """The config-5 model (24 layers, B8, prompt 512, capacity 2048) with the
    same random weights in fp32, fast mode, strict lowering, against the eager
    model in fp32 on the GPU: prefill logits, three teacher-forced decode
    steps' logits and every layer's K/V within 1e-5 relative (the reference
    holds its multilayer compiled decode to 3e-5 in fp32,
    tests/test_multilayer_decode.py:255-276)."""

    announce("config5 fp32 fast mode vs eager fp32 (24 layers)")
    weights = init_weights(CONFIG5, seed=5, dtype=torch.float32, device=gpu, draw_on_device=True)
    g = torch.Generator(device="cpu").manual_seed(5)
    ids = torch.randint(0, CONFIG5.vocab_size, (BATCH, PROMPT), generator=g).to(gpu)
    mask = causal_prefill_mask(BATCH, PROMPT, device=gpu)
    pos = torch.arange(PROMPT, device=gpu).view(1, -1).expand(BATCH, -1).contiguous()
    logits, steps, tokens, cache = _eager_teacher_forced(weights, ids, mask, pos, torch.float32, STEPS, gpu)
    data = dict(weights=weights, ids=ids, mask=mask, pos=pos, prefill_logits=logits, steps=steps,
                tokens=tokens, cache=cache, dtype=torch.float32)
    pairs = _run(data, gpu)
    relative = {}
    for what, actual, expected in pairs:
        scale = float(expected.float().abs().max())
        relative[what] = float((actual.float() - expected.float()).abs().max()) / max(scale, 1e-30)
    _record("config5_fp32_fast_relative", {
        "logits": {k: float(f"{v:.3e}") for k, v in relative.items() if "logits" in k},
        "KV_max_by_layer": [float(f"{max(relative[f'layer {i} K'], relative[f'layer {i} V']):.3e}")
                            for i in range(CONFIG5.num_layers)]})
    for what, actual, expected in pairs:
        try:
            assert_fp32_close(actual, expected)
        except AssertionError as error:
            raise AssertionError(f"{what}: {error}") from None


# Bars for fast mode over the full 128-step run: 1.5x the GEMM-rounding
# yardstick that test_config5_fast_mode measures on this model (eager moves
# its logits by 0.070 and its K/V by 0.0625 when only its linears' rounding
# changes).
FAST_LOGIT_BAR = 0.105
FAST_KV_BAR = 0.094


def _bf16_ulp(value):
    """Spacing of bf16 numbers at |value| (8 significant bits)."""

    _, exponent = torch.frexp(torch.tensor(abs(value)))
    return float(torch.ldexp(torch.tensor(1.0), exponent - 8))


def _margin(logits_row, first, second):
    return float(logits_row[first].float() - logits_row[second].float())


def test_config5_greedy_128_steps(gpu, config5):
    """Config 5 as named: one prefill of 512 tokens, then 128 greedy decode
    steps on the same buffers, in both numerical modes, against the eager
    model's own greedy run from the same prompt.

    * pytorch_compatible: every generated token and the final K/V of every
      layer equal eager's exactly.
    * fast (HIP graph replay per step, as the bench runs it): the logits
      stay within FAST_LOGIT_BAR of eager's until a row's tokens first
      differ; each row's first divergence is recorded with eager's top-2
      margin there.  (A flip needs eager's top-2 margin to be at most twice
      the logit error, so it happens only at near-ties; the random-init
      model's bf16 logits are flat and tie often.)
    * fast, teacher-forced on eager's 128 tokens: every step's logits within
      FAST_LOGIT_BAR, the final K/V of every layer within FAST_KV_BAR; the
      top-1 agreement and every disagreement's margin (in bf16 ulps of the
      top logit) are recorded.
    """

    weights, ids, mask, pos = (config5[k] for k in ("weights", "ids", "mask", "pos"))
    announce("config5 greedy 128: eager reference")
    eager = EagerQwen2(CONFIG5, weights)
    eager_tokens, eager_logits = [], []
    with torch.no_grad():
        logits, cache = eager.prefill(ids, mask, pos)
        token = logits[:, -1].argmax(-1, keepdim=True)
        for step in range(GREEDY_STEPS):
            length = PROMPT + step
            eager_tokens.append(token)
            dmask = torch.zeros(BATCH, 1, 1, length + 1, dtype=torch.bfloat16, device=gpu)
            logits, cache = eager.decode(token, dmask, torch.full((BATCH, 1), length, device=gpu), cache)
            eager_logits.append(logits[:, -1].clone())
            token = logits[:, -1].argmax(-1, keepdim=True)
    eager_tokens.append(token)
    eager_tokens = torch.cat(eager_tokens, dim=1)  # [B, 129]: first token + 128 generated
    final_len = PROMPT + GREEDY_STEPS

    announce("config5 greedy 128: pytorch_compatible")
    rt = Qwen2Runtime(CONFIG5, weights, capacity=CAPACITY, dtype=torch.bfloat16, device=str(gpu),
                      numerical_mode="pytorch_compatible")
    logits, state = rt.prefill(ids, mask, pos)
    token = logits[:, -1].argmax(-1, keepdim=True)
    compat_tokens = [token]
    for step in range(GREEDY_STEPS):
        dmask = torch.zeros(BATCH, 1, 1, PROMPT + step + 1, dtype=torch.bfloat16, device=gpu)
        logits, state = rt.decode(token, dmask, state)
        token = logits[:, -1].argmax(-1, keepdim=True)
        compat_tokens.append(token)
    compat_tokens = torch.cat(compat_tokens, dim=1)
    assert torch.equal(compat_tokens, eager_tokens)
    for slot, (k, v) in enumerate(cache):
        assert state.lengths[slot].tolist() == [final_len] * BATCH
        assert torch.equal(state.keys[slot][:, :final_len].transpose(1, 2), k), f"layer {slot} K"
        assert torch.equal(state.values[slot][:, :final_len].transpose(1, 2), v), f"layer {slot} V"
    state.check_capacity()
    del rt, state

    announce("config5 greedy 128: fast mode, HIP graph replay per step")
    rt = Qwen2Runtime(CONFIG5, weights, capacity=CAPACITY, dtype=torch.bfloat16, device=str(gpu))
    logits, state = rt.prefill(ids, mask, pos)
    first = logits[:, -1].argmax(-1)
    decoder = rt.graph_decoder(state, first)
    fast_tokens, fast_logits = [first.view(-1, 1).clone()], []
    for _ in range(GREEDY_STEPS):
        decoder.step()
        fast_tokens.append(decoder.tokens.clone())
        fast_logits.append(decoder.logits[:, -1].clone())
    torch.cuda.synchronize()
    fast_tokens = torch.cat(fast_tokens, dim=1)
    assert state.lengths[0].tolist() == [final_len] * BATCH

    report = {"rows": BATCH, "steps": GREEDY_STEPS}
    assert torch.equal(fast_tokens[:, 0], eager_tokens[:, 0]), "fast-mode prefill picked a different first token"
    agree, divergences, max_err = 0, [], 0.0
    for b in range(BATCH):
        row_agree = GREEDY_STEPS
        # Token t >= 1 is the argmax of decode step t-1's logits; the two runs
        # saw the same prefix up to the first divergence.
        for t in range(1, GREEDY_STEPS + 1):
            err = float((fast_logits[t - 1][b].float() - eager_logits[t - 1][b].float()).abs().max())
            max_err = max(max_err, err)
            if int(fast_tokens[b, t]) != int(eager_tokens[b, t]):
                margin = _margin(eager_logits[t - 1][b], int(eager_tokens[b, t]), int(fast_tokens[b, t]))
                divergences.append({"row": b, "step": t, "eager_top2_margin": round(margin, 5),
                                    "fast_logit_error": round(err, 5)})
                row_agree = t - 1
                break
        agree += row_agree
    report.update(tokens_agreeing=agree, of=BATCH * GREEDY_STEPS, first_divergences=divergences,
                  max_logit_error_before_divergence=round(max_err, 5))
    _record("config5_greedy128_fast_vs_eager", report)
    assert max_err <= FAST_LOGIT_BAR, max_err
    del decoder, state

    announce("config5 greedy 128: fast mode teacher-forced on eager's tokens")
    logits, state = rt.prefill(ids, mask, pos)
    step_errors, flips = [], []
    for step in range(GREEDY_STEPS):
        dmask = torch.zeros(BATCH, 1, 1, PROMPT + step + 1, dtype=torch.bfloat16, device=gpu)
        logits, state = rt.decode(eager_tokens[:, step:step + 1], dmask, state)
        row = logits[:, -1]
        step_errors.append(float((row.float() - eager_logits[step].float()).abs().max()))
        for b in torch.nonzero(row.argmax(-1) != eager_tokens[:, step + 1]).flatten().tolist():
            margin = _margin(eager_logits[step][b], int(eager_tokens[b, step + 1]), int(row[b].argmax()))
            flips.append({"row": b, "step": step + 1, "margin": round(margin, 5),
                          "margin_ulps": round(margin / _bf16_ulp(float(eager_logits[step][b].float().max())), 2)})
    kv_errors = []
    for slot, (k, v) in enumerate(cache):
        kv_errors.append(round(max(
            float((state.keys[slot][:, :final_len].transpose(1, 2).float() - k.float()).abs().max()),
            float((state.values[slot][:, :final_len].transpose(1, 2).float() - v.float()).abs().max())), 5))
    _record("config5_teacher_forced128_fast_vs_eager", {
        "logit_error_max": round(max(step_errors), 5), "logit_error_first_last": [round(step_errors[0], 5), round(step_errors[-1], 5)],
        "top1_agreement": 1 - len(flips) / (BATCH * GREEDY_STEPS), "flips": flips, "final_KV_max_by_layer": kv_errors})
    assert max(step_errors) <= FAST_LOGIT_BAR, step_errors
    assert max(kv_errors) <= FAST_KV_BAR, kv_errors
