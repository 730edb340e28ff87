"""Fused decode-step kernels on the GPU: each must equal, bit for bit, the
sequence of single-op kernels it replaces (and so inherits their parity with
the oracle), at every row count the fused path takes and on the fallback
beyond it; and the fused Qwen2 graph must equal the unfused one."""

from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_bitwise_equal, generator
from stateful_llm_compiler_hip.backends import (
    hip_add,
    hip_kv_store,
    hip_linear,
    hip_linear_residual,
    hip_norm_linear_group,
    hip_norm_linear_swiglu,
    hip_rms_norm,
    hip_rope,
    hip_rope_kv_store,
    hip_swiglu,
)

pytestmark = pytest.mark.gpu

ROWS = [1, 3, 8, 16, 17, 32, 40]  # 40 exceeds the fused limit: fallback path


def _t(g, *shape, dtype=torch.bfloat16, scale=1.0, device):
    return (torch.randn(*shape, generator=g) * scale).to(dtype).to(device)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden,ns", [(896, (896, 128, 128)), (2048, (4096, 512, 520))])
def test_norm_linear_group_matches_norm_then_linears(gpu, rows, dtype, hidden, ns):
    # The second shape: 16 waves (long K), two MFMA tiles per workgroup in the
    # fused call against one in the single linears.
    announce(f"norm_linear_group rows={rows} {dtype} hidden={hidden} ns={ns}")
    g = generator(rows)
    h = _t(g, rows, 1, hidden, dtype=dtype, device=gpu)
    nw = _t(g, hidden, dtype=dtype, scale=0.5, device=gpu) + 1
    ws = [_t(g, n, hidden, dtype=dtype, scale=0.02, device=gpu) for n in ns]
    bs = [_t(g, n, dtype=dtype, scale=0.1, device=gpu) for n in ns]
    got = hip_norm_linear_group(h, nw, ws, bs, epsilon=1e-6)
    x = hip_rms_norm(h, nw, epsilon=1e-6, round_before_weight=True)
    want = [hip_linear(x, w, b) for w, b in zip(ws, bs)]
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert_bitwise_equal(a, b)
    # one matrix, no bias, no norm
    got1 = hip_norm_linear_group(h, None, ws[:1], [None], epsilon=1e-6)
    assert_bitwise_equal(got1[0], hip_linear(h, ws[0]))


@pytest.mark.parametrize("rows", [1, 8, 16, 17, 40])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden,vocab,bias", [(896, 151936, False), (2048, 17000, True),
                                               (256, 20000, False)])
def test_norm_vocabulary_head_matches_norm_then_linear(gpu, rows, dtype, hidden, vocab, bias):
    """The final norm and a vocabulary-width head in one launch (the wide
    kernel normalises in its input staging; rows past 16 take the
    equal-workgroup kernel, past 32 the unfused pair) equal rms_norm then
    linear bit for bit."""
    announce(f"norm + vocabulary head rows={rows} {dtype} hidden={hidden} vocab={vocab}")
    g = generator(300 + rows + hidden)
    h = _t(g, rows, 1, hidden, dtype=dtype, device=gpu)
    nw = _t(g, hidden, dtype=dtype, scale=0.5, device=gpu) + 1
    w = _t(g, vocab, hidden, dtype=dtype, scale=0.02, device=gpu)
    b = _t(g, vocab, dtype=dtype, scale=0.1, device=gpu) if bias else None
    (got,) = hip_norm_linear_group(h, nw, [w], [b], epsilon=1e-6)
    want = hip_linear(hip_rms_norm(h, nw, epsilon=1e-6, round_before_weight=True), w, b)
    torch.cuda.synchronize()
    assert_bitwise_equal(got, want)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("hidden,features", [(896, 4864), (2048, 5000)])
def test_norm_linear_swiglu_matches_the_mlp_front(gpu, rows, hidden, features):
    announce(f"norm_linear_swiglu rows={rows} hidden={hidden} features={features}")
    g = generator(100 + rows)
    h = _t(g, rows, 1, hidden, device=gpu)
    nw = _t(g, hidden, scale=0.5, device=gpu) + 1
    wg = _t(g, features, hidden, scale=0.02, device=gpu)
    wu = _t(g, features, hidden, scale=0.02, device=gpu)
    got = hip_norm_linear_swiglu(h, nw, wg, wu, epsilon=1e-6)
    x = hip_rms_norm(h, nw, epsilon=1e-6, round_before_weight=True)
    want = hip_swiglu(hip_linear(x, wg), hip_linear(x, wu))
    torch.cuda.synchronize()
    assert_bitwise_equal(got, want)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("n,k", [(896, 896), (896, 4864), (100, 64), (6000, 2048)])
def test_linear_residual_matches_linear_then_add(gpu, rows, n, k):
    announce(f"linear_residual rows={rows} n={n} k={k}")
    g = generator(200 + rows + n)
    x = _t(g, rows, 1, k, device=gpu)
    w = _t(g, n, k, scale=0.02, device=gpu)
    r = _t(g, rows, 1, n, device=gpu)
    bias = _t(g, n, scale=0.1, device=gpu) if n == 100 else None
    got = hip_linear_residual(x, w, bias, r)
    want = hip_add(r, hip_linear(x, w, bias))
    torch.cuda.synchronize()
    assert_bitwise_equal(got, want)


@pytest.mark.parametrize("tokens", [1, 5])
def test_rope_kv_store_matches_rope_then_store(gpu, tokens):
    announce(f"rope_kv_store tokens={tokens}")
    g = generator(300 + tokens)
    B, QH, KVH, D, cap = 3, 14, 2, 64, 16
    # q/k/v as the decode graph makes them: views of [B, T, H*D] projections.
    q = _t(g, B, tokens, QH * D, device=gpu).view(B, tokens, QH, D).transpose(1, 2)
    k = _t(g, B, tokens, KVH * D, device=gpu).view(B, tokens, KVH, D).transpose(1, 2)
    v = _t(g, B, tokens, KVH * D, device=gpu).view(B, tokens, KVH, D).transpose(1, 2)
    cos = _t(g, B, tokens, D, device=gpu)
    sin = _t(g, B, tokens, D, device=gpu)
    positions = torch.tensor([0, 7, cap - 2], device=gpu)  # the last row runs past the capacity
    kb1 = _t(g, B, cap, KVH, D, device=gpu)
    vb1 = _t(g, B, cap, KVH, D, device=gpu)
    kb2, vb2 = kb1.clone(), vb1.clone()
    flag1 = torch.zeros(1, dtype=torch.int32, device=gpu)
    flag2 = torch.zeros(1, dtype=torch.int32, device=gpu)
    q_got = hip_rope_kv_store(q, k, v, cos, sin, kb1, vb1, positions, overflow=flag1)
    q_want, k_rot = hip_rope(q, k, cos, sin)
    hip_kv_store(kb2, vb2, k_rot, v, positions, overflow=flag2)
    torch.cuda.synchronize()
    assert_bitwise_equal(q_got, q_want)
    assert_bitwise_equal(kb1, kb2)
    assert_bitwise_equal(vb1, vb2)
    assert int(flag1.item()) == int(flag2.item()) == (1 if tokens > 2 else 0)


def test_fused_qwen2_graph_equals_unfused(gpu):
    from oracle.qwen2_model import causal_mask
    from stateful_llm_compiler_hip.qwen2 import Qwen2Config, init_weights
    from stateful_llm_compiler_hip.runtime import Qwen2Runtime

    announce("fused vs unfused Qwen2 config-1 bf16")
    config = Qwen2Config(num_layers=2, vocab_size=1024)
    weights = {k: v.to(gpu) for k, v in init_weights(config, seed=0, dtype=torch.bfloat16).items()}
    runs = []
    for fuse in (True, False):
        rt = Qwen2Runtime(config, weights, capacity=64, dtype=torch.bfloat16, device=str(gpu), fuse=fuse)
        g = generator(1)
        ids = torch.randint(0, config.vocab_size, (3, 5), generator=g).to(gpu)
        pos = torch.arange(5).view(1, -1).expand(3, -1).contiguous().to(gpu)
        logits, state = rt.prefill(ids, causal_mask(3, 5).to(gpu), pos)
        outs = [logits]
        token = logits[:, -1].argmax(-1, keepdim=True)
        for step in range(3):
            mask = torch.zeros(3, 1, 1, 6 + step, dtype=torch.bfloat16, device=gpu)
            logits, state = rt.decode(token, mask, state)
            outs.append(logits)
            token = logits[:, -1].argmax(-1, keepdim=True)
        outs += list(state.keys) + list(state.values)
        runs.append(outs)
        ops = len(rt.decode_result.module.functions[0].block.operations)
        announce(f"fuse={fuse}: {ops} decode ops")
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert_bitwise_equal(a, b)


@pytest.mark.parametrize("in_place", [True, False])
def test_rope_kv_store_advance_matches_store_then_advance(gpu, in_place):
    # The store kernel's last workgroup advances the lengths (in place or into
    # a new tensor) exactly as the kv advance launched after it would, and
    # flags an advance past the capacity; repeated calls re-arm its counter.
    from stateful_llm_compiler_hip.backends import hip_kv_advance

    announce(f"rope_kv_store + advance in_place={in_place}")
    g = generator(401)
    B, QH, KVH, D, cap = 5, 14, 2, 64, 32
    for step in range(3):
        q = _t(g, B, 1, QH * D, device=gpu).view(B, 1, QH, D).transpose(1, 2)
        k = _t(g, B, 1, KVH * D, device=gpu).view(B, 1, KVH, D).transpose(1, 2)
        v = _t(g, B, 1, KVH * D, device=gpu).view(B, 1, KVH, D).transpose(1, 2)
        cos = _t(g, B, 1, D, device=gpu)
        sin = _t(g, B, 1, D, device=gpu)
        start = torch.tensor([0, 3, 17, cap - 2, cap - 1], device=gpu) + step
        kb1 = _t(g, B, cap, KVH, D, device=gpu)
        vb1 = _t(g, B, cap, KVH, D, device=gpu)
        kb2, vb2 = kb1.clone(), vb1.clone()
        flag1 = torch.zeros(1, dtype=torch.int32, device=gpu)
        flag2 = torch.zeros(1, dtype=torch.int32, device=gpu)
        pos1 = start.clone()
        out1 = pos1 if in_place else torch.full_like(pos1, -7)
        q1 = hip_rope_kv_store(q, k, v, cos, sin, kb1, vb1, pos1, overflow=flag1, advance=1,
                               lengths_out=out1)
        pos2 = start.clone()
        q2 = hip_rope_kv_store(q, k, v, cos, sin, kb2, vb2, pos2, overflow=flag2)
        out2 = hip_kv_advance(pos2, 1, cap, overflow=flag2)
        torch.cuda.synchronize()
        assert_bitwise_equal(q1, q2)
        assert_bitwise_equal(kb1, kb2)
        assert_bitwise_equal(vb1, vb2)
        assert out1.tolist() == out2.tolist() == (start + 1).tolist()
        assert int(flag1.item()) == int(flag2.item()) == (1 if step >= 1 else 0)
        if not in_place:
            assert pos1.tolist() == start.tolist()


@pytest.mark.parametrize(
    "B,QH,KVH,D,cap,mask_len,dtype,mask_kind,in_place,starts",
    [
        # one chunk, positions up to the capacity (the last overflows from step 1)
        (5, 14, 2, 64, 64, 64, torch.bfloat16, "bf16", True, [0, 3, 17, 62, 63]),
        # split sequence (in-kernel merge), empty chunks, new row in chunk 0 / mid / last
        (3, 14, 2, 64, 2048, 2048, torch.bfloat16, "f32", False, [0, 700, 2040]),
        # D = 128, groups of 4, fp16, no mask
        (4, 8, 2, 128, 1024, 1024, torch.float16, "none", True, [5, 255, 256, 1000]),
        # groups of 1
        (2, 4, 4, 64, 600, 600, torch.bfloat16, "bf16", True, [100, 599]),
        # new row past the mask: stored by the last chunk, not attended
        (2, 14, 2, 64, 512, 300, torch.bfloat16, "bf16", False, [400, 10]),
        # a wide batch: many chunks per sequence and many workgroups per batch
        (40, 14, 2, 64, 4096, 4096, torch.bfloat16, "bf16", True, list(range(0, 4000, 100))),
    ],
)
@pytest.mark.parametrize("order", ["online", "exact"])
def test_rope_decode_attention_matches_store_then_attention(gpu, B, QH, KVH, D, cap, mask_len,
                                                            dtype, mask_kind, in_place, starts, order):
    # One kernel rotates, stores, advances and attends; the same three steps as
    # rope_kv_store(advance=1) then decode attention, bit for bit, over three
    # consecutive calls (counters re-armed each time).
    from stateful_llm_compiler_hip.backends import hip_decode_attention, hip_rope_decode_attention

    announce(f"rope_decode_attention B={B} QH={QH} KVH={KVH} D={D} cap={cap} mask={mask_len} "
             f"{dtype} {mask_kind} in_place={in_place} {order}")
    g = generator(B * 7 + D + cap)
    kb1 = _t(g, B, cap, KVH, D, dtype=dtype, device=gpu)
    vb1 = _t(g, B, cap, KVH, D, dtype=dtype, device=gpu)
    kb2, vb2 = kb1.clone(), vb1.clone()
    start = torch.tensor(starts, device=gpu)
    for step in range(3):
        q = _t(g, B, 1, QH * D, dtype=dtype, device=gpu).view(B, 1, QH, D).transpose(1, 2)
        k = _t(g, B, 1, KVH * D, dtype=dtype, device=gpu).view(B, 1, KVH, D).transpose(1, 2)
        v = _t(g, B, 1, KVH * D, dtype=dtype, device=gpu).view(B, 1, KVH, D).transpose(1, 2)
        cos = _t(g, B, 1, D, dtype=dtype, device=gpu)
        sin = _t(g, B, 1, D, dtype=dtype, device=gpu)
        if mask_kind == "none":
            mask = None
        else:
            mdt = torch.float32 if mask_kind == "f32" else dtype
            mask = (torch.randn(B, 1, 1, mask_len, generator=g) * 2).to(mdt).to(gpu)
        flag1 = torch.zeros(1, dtype=torch.int32, device=gpu)
        flag2 = torch.zeros(1, dtype=torch.int32, device=gpu)
        pos1 = (start + step).clone()
        out1 = pos1 if in_place else torch.full_like(pos1, -7)
        o1 = hip_rope_decode_attention(q, k, v, cos, sin, kb1, vb1, pos1, out1, mask,
                                       scale=D ** -0.5, overflow=flag1, softmax_order=order)
        assert o1 is not None
        pos2 = (start + step).clone()
        q2 = hip_rope_kv_store(q, k, v, cos, sin, kb2, vb2, pos2, overflow=flag2, advance=1,
                               lengths_out=pos2)
        o2 = hip_decode_attention(q2, kb2, vb2, pos2, mask, scale=D ** -0.5, softmax_order=order)
        torch.cuda.synchronize()
        assert_bitwise_equal(o1, o2)
        assert_bitwise_equal(kb1, kb2)
        assert_bitwise_equal(vb1, vb2)
        assert out1.tolist() == pos2.tolist() == (start + step + 1).tolist()
        assert int(flag1.item()) == int(flag2.item())
        if not in_place:
            assert pos1.tolist() == (start + step).tolist()


def test_rope_decode_attention_declines_unsupported(gpu):
    # fp32 (no matrix-core kernel): nothing launched, None returned, lengths untouched.
    from stateful_llm_compiler_hip.backends import hip_rope_decode_attention

    announce("rope_decode_attention fp32 declined")
    g = generator(5)
    B, QH, KVH, D, cap = 2, 4, 2, 64, 16
    q = _t(g, B, QH, 1, D, dtype=torch.float32, device=gpu)
    k = _t(g, B, KVH, 1, D, dtype=torch.float32, device=gpu)
    cos = _t(g, B, 1, D, dtype=torch.float32, device=gpu)
    kb = _t(g, B, cap, KVH, D, dtype=torch.float32, device=gpu)
    pos = torch.tensor([1, 2], device=gpu)
    before = kb.clone()
    assert hip_rope_decode_attention(q, k, k, cos, cos, kb, kb.clone(), pos, pos, None,
                                     scale=0.125) is None
    torch.cuda.synchronize()
    assert pos.tolist() == [1, 2]
    assert_bitwise_equal(kb, before)


@pytest.mark.parametrize("rows,n,k,bias", [(300, 896, 896, False), (4096, 896, 4864, False),
                                           (129, 136, 64, True), (300, 100, 64, False)])
def test_linear_residual_prefill_rows(gpu, rows, n, k, bias):
    # Prefill-sized rows: the tile kernel adds the residual in its store
    # epilogue (N = 100 is not a multiple of 8: the two-op path), bit for bit
    # the linear then the add.
    announce(f"linear_residual prefill rows={rows} n={n} k={k} bias={bias}")
    g = generator(rows + n + k)
    x = _t(g, rows, k, device=gpu)
    w = _t(g, n, k, scale=0.02, device=gpu)
    r = _t(g, rows, n, device=gpu)
    b = _t(g, n, scale=0.1, device=gpu) if bias else None
    got = hip_linear_residual(x, w, b, r)
    want = hip_add(r, hip_linear(x, w, b))
    torch.cuda.synchronize()
    assert_bitwise_equal(got, want)


def test_fused_ops_reject_host_operands(gpu):
    announce("fused ops reject host operands")
    g = generator(3)
    x = _t(g, 4, 896, device=gpu)
    w = _t(g, 896, 896, scale=0.02, device=gpu)
    with pytest.raises(ValueError):
        hip_linear_residual(x, w, None, torch.zeros(4, 896, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        hip_norm_linear_group(x, torch.ones(896, dtype=torch.bfloat16), [w], [None], epsilon=1e-6)


@pytest.mark.parametrize("rows,hidden,features,dtype", [(300, 896, 4864, torch.bfloat16),
                                                        (4096, 896, 4864, torch.bfloat16),
                                                        (2100, 896, 4864, torch.bfloat16),
                                                        (2100, 896, 4864, torch.float16),
                                                        (129, 128, 200, torch.bfloat16),
                                                        (100, 64, 100, torch.bfloat16)])
def test_norm_linear_swiglu_prefill_rows(gpu, rows, hidden, features, dtype):
    # Prefill-sized rows: the norm, then gate/up and SwiGLU in one tile kernel
    # (features = 100: not a multiple of 8, the two-linear path), bit for bit
    # the separate ops.
    announce(f"norm_linear_swiglu prefill rows={rows} hidden={hidden} features={features} {dtype}")
    g = generator(rows + features)
    h = _t(g, rows, 1, hidden, dtype=dtype, device=gpu)
    nw = _t(g, hidden, dtype=dtype, scale=0.5, device=gpu) + 1
    wg = _t(g, features, hidden, dtype=dtype, scale=0.05, device=gpu)
    wu = _t(g, features, hidden, dtype=dtype, scale=0.05, device=gpu)
    got = hip_norm_linear_swiglu(h, nw, wg, wu, epsilon=1e-6)
    x = hip_rms_norm(h, nw, epsilon=1e-6, round_before_weight=True)
    want = hip_swiglu(hip_linear(x, wg), hip_linear(x, wu))
    torch.cuda.synchronize()
    assert_bitwise_equal(got, want)


@pytest.mark.parametrize("rows,hidden,ns,bias", [(300, 896, (896, 128, 128), True),
                                                 (4096, 896, (896, 128, 128), True),
                                                 (8192, 896, (4864, 896, 128), True),
                                                 (129, 64, (200, 8), False),
                                                 (100, 64, (96, 100), True)])
def test_norm_linear_group_prefill_rows(gpu, rows, hidden, ns, bias):
    # Prefill-sized rows: the norm, then the projections in one grouped launch
    # (a width of 100 is not a multiple of 8: one launch per matrix), bit for
    # bit the single linears.
    announce(f"norm_linear_group prefill rows={rows} hidden={hidden} ns={ns} bias={bias}")
    g = generator(rows + hidden + len(ns))
    h = _t(g, rows, 1, hidden, device=gpu)
    nw = _t(g, hidden, scale=0.5, device=gpu) + 1
    ws = [_t(g, n, hidden, scale=0.05, device=gpu) for n in ns]
    bs = [_t(g, n, scale=0.1, device=gpu) if bias else None for n in ns]
    got = hip_norm_linear_group(h, nw, ws, bs, epsilon=1e-6)
    x = hip_rms_norm(h, nw, epsilon=1e-6, round_before_weight=True)
    want = [hip_linear(x, w, b) for w, b in zip(ws, bs)]
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert_bitwise_equal(a, b)
