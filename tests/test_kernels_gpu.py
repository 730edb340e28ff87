"""GPU parity of each gfx950 kernel against the CPU oracle (same seeded inputs).

Bars: kv_store bit-exact; rope bit-exact (it reproduces the eager rounding
points); fp32 within 1e-5 relative; bf16 within 2e-2 absolute.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import (
    announce,
    assert_bf16_close,
    assert_bitwise_equal,
    assert_fp32_close,
    generator,
)
from oracle import kernels as ref

# slc_split: the length-balanced split-sequence variant of decode attention.
SPLIT_BALANCED = -1

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------- kv_store


def _kv_store_case(gpu, batch, heads, tokens, head_dim, capacity, positions, dtype, seed, strided=False):
    g = generator(seed)
    key_buffer = torch.randn(batch, capacity, heads, head_dim, generator=g).to(dtype)
    value_buffer = torch.randn(batch, capacity, heads, head_dim, generator=g).to(dtype)
    if strided:
        # B x T x H x D projection output viewed as B x H x T x D (the layout the
        # model hands to kv_store).
        key = torch.randn(batch, tokens, heads, head_dim, generator=g).to(dtype).transpose(1, 2)
        value = torch.randn(batch, tokens, heads, head_dim, generator=g).to(dtype).transpose(1, 2)
    else:
        key = torch.randn(batch, heads, tokens, head_dim, generator=g).to(dtype)
        value = torch.randn(batch, heads, tokens, head_dim, generator=g).to(dtype)
    positions = torch.tensor(positions, dtype=torch.int64)

    from stateful_llm_compiler_hip.backends import hip_kv_store

    kb, vb = key_buffer.to(gpu), value_buffer.to(gpu)
    kd, vd = key.to(gpu), value.to(gpu)
    if strided:
        kd = key.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
        vd = value.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    hip_kv_store(kb, vb, kd, vd, positions.to(gpu))
    torch.cuda.synchronize()

    width = torch.int16 if dtype != torch.float32 else torch.int32
    exp_k = key_buffer.view(width).numpy().copy()
    exp_v = value_buffer.view(width).numpy().copy()
    ref.kv_store(exp_k, exp_v, key.contiguous().view(width).numpy(), value.contiguous().view(width).numpy(), positions.numpy())
    assert_bitwise_equal(kb.cpu().view(width), torch.from_numpy(exp_k))
    assert_bitwise_equal(vb.cpu().view(width), torch.from_numpy(exp_v))


def test_kv_store_reference_positions(gpu):
    # Reference KAT: positions [1, 5, 9], capacity 16 (test_triton_backend.py:436-466).
    announce("kv_store KAT positions=[1,5,9] cap=16")
    _kv_store_case(gpu, 3, 2, 1, 8, 16, [1, 5, 9], torch.float32, 1)


@pytest.mark.parametrize("batch", [1, 8, 64])
@pytest.mark.parametrize("tokens", [1, 128, 512])
def test_kv_store_config3_bitexact(gpu, batch, tokens):
    announce(f"kv_store bf16 B={batch} T={tokens} cap=8192")
    g = generator(100 + batch + tokens)
    positions = torch.randint(0, 8192 - tokens + 1, (batch,), generator=g).tolist()
    _kv_store_case(gpu, batch, 2, tokens, 64, 8192, positions, torch.bfloat16, 7 + batch, strided=True)


def test_kv_store_capacity_overflow_rows_are_dropped(gpu):
    announce("kv_store overflow rows dropped")
    _kv_store_case(gpu, 2, 2, 6, 64, 16, [13, 0], torch.bfloat16, 3)


def test_kv_store_odd_head_dim_fp16(gpu):
    announce("kv_store fp16 D=6 (2-byte units)")
    _kv_store_case(gpu, 2, 3, 4, 6, 10, [0, 5], torch.float16, 4)


# --------------------------------------------------------- decode_attention


def _decode_case(
    gpu,
    batch,
    q_heads,
    kv_heads,
    head_dim,
    capacity,
    lengths,
    dtype,
    seed,
    *,
    mask_len=None,
    mask_kind="zeros",
    layout="bshd",
    length_dtype=torch.int64,
    split_tokens=0,
    mask_dtype=None,
    softmax_order="online",
):
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    g = generator(seed)
    mask_len = capacity if mask_len is None else mask_len
    query = torch.randn(batch, q_heads, 1, head_dim, generator=g).to(dtype)
    key_buffer = torch.randn(batch, capacity, kv_heads, head_dim, generator=g).to(dtype)
    value_buffer = torch.randn(batch, capacity, kv_heads, head_dim, generator=g).to(dtype)
    mask_dtype = dtype if mask_dtype is None else mask_dtype
    if mask_kind == "zeros":
        mask = torch.zeros(batch, 1, 1, mask_len, dtype=mask_dtype)
    else:
        mask = (torch.randn(batch, 1, 1, mask_len, generator=g) * 2.0).to(mask_dtype)
    lengths_t = torch.tensor(lengths, dtype=torch.int64)
    expected = ref.decode_attention(
        query,
        key_buffer,
        value_buffer,
        lengths_t,
        mask,
        groups=q_heads // kv_heads,
        scale=head_dim**-0.5,
    )
    if layout == "bhsd":
        # Physical [B, KVH, Lmax, D] buffer presented through a BSHD view.
        kd = key_buffer.permute(0, 2, 1, 3).contiguous().to(gpu).permute(0, 2, 1, 3)
        vd = value_buffer.permute(0, 2, 1, 3).contiguous().to(gpu).permute(0, 2, 1, 3)
    else:
        kd, vd = key_buffer.to(gpu), value_buffer.to(gpu)
    actual = hip_decode_attention(
        query.to(gpu),
        kd,
        vd,
        lengths_t.to(length_dtype).to(gpu),
        mask.to(gpu),
        scale=head_dim**-0.5,
        split_tokens=split_tokens,
        softmax_order=softmax_order,
    )
    torch.cuda.synchronize()
    return actual.cpu(), expected


def test_decode_attention_reference_lengths_fp32(gpu):
    # Reference KAT: per-batch lengths [7, 31, 65], cap 65, QH4 KVH2 D16, fp32,
    # tolerance 3e-5 (test_triton_backend.py:380-434).
    announce("decode KAT fp32 lengths=[7,31,65]")
    actual, expected = _decode_case(gpu, 3, 4, 2, 16, 65, [7, 31, 65], torch.float32, 5)
    torch.testing.assert_close(actual, expected, rtol=3e-5, atol=3e-5)
    assert_fp32_close(actual, expected)


@pytest.mark.parametrize("split", [0, SPLIT_BALANCED])
@pytest.mark.parametrize("batch", [1, 8, 32, 64])
@pytest.mark.parametrize("max_len", [64, 1024, 8192])
def test_decode_attention_config2_bf16(gpu, batch, max_len, split):
    announce(f"decode bf16 B={batch} L={max_len} split_tokens={split}")
    g = generator(batch * 7 + max_len)
    lengths = torch.randint(max_len // 2, max_len + 1, (batch,), generator=g).tolist()
    actual, expected = _decode_case(gpu, batch, 14, 2, 64, max_len, lengths, torch.bfloat16, batch + max_len,
                                    split_tokens=split)
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("split", [0, SPLIT_BALANCED])
@pytest.mark.parametrize("batch", [1, 8, 32, 64])
def test_decode_attention_config2_bf16_long(gpu, batch, split):
    # Config 2's longest rows: L = 32768, lengths U[L/2, L] (B = 64 holds 1 GB
    # of K/V on the host for the oracle).
    announce(f"decode bf16 B={batch} L=32768 split_tokens={split}")
    g = generator(11 + batch)
    lengths = torch.randint(16384, 32769, (batch,), generator=g).tolist()
    actual, expected = _decode_case(gpu, batch, 14, 2, 64, 32768, lengths, torch.bfloat16, 12 + batch,
                                    split_tokens=split)
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("split", [0, SPLIT_BALANCED])
@pytest.mark.parametrize("layout", ["bshd", "bhsd"])
@pytest.mark.parametrize("length_dtype", [torch.int64, torch.int32])
def test_decode_attention_layouts_and_length_dtypes(gpu, layout, length_dtype, split):
    announce(f"decode bf16 layout={layout} lengths={length_dtype} split_tokens={split}")
    actual, expected = _decode_case(
        gpu, 4, 14, 2, 64, 1024, [1, 333, 1000, 1024], torch.bfloat16, 21,
        layout=layout, length_dtype=length_dtype, split_tokens=split,
    )
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("split", [128, 256, 2048])
def test_decode_attention_forced_split(gpu, split):
    announce(f"decode bf16 split_tokens={split}")
    actual, expected = _decode_case(
        gpu, 3, 14, 2, 64, 2048, [2048, 1, 1500], torch.bfloat16, 31, split_tokens=split, mask_kind="random",
    )
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("split", [0, 32, 64, 100, 5000, SPLIT_BALANCED])
@pytest.mark.parametrize("batch", [3, 65, 130])
def test_decode_attention_balanced_split(gpu, batch, split):
    # The length-balanced split lays every (batch, kv-head) tile range end to
    # end: short sequences put several pairs into one workgroup, long ones
    # spread over several workgroups, and a workgroup's range may start and
    # end mid-sequence.  More than 64 sequences take several scan rounds.
    announce(f"decode bf16 balanced split B={batch} split_tokens={split}")
    g = generator(batch * 13 + split)
    lengths = torch.randint(1, 200, (batch,), generator=g)
    lengths[::7] = torch.randint(1, 33, lengths[::7].shape, generator=g)
    lengths[1] = 256
    actual, expected = _decode_case(
        gpu, batch, 14, 2, 64, 256, lengths.tolist(), torch.bfloat16, batch + split,
        split_tokens=split, mask_kind="random",
    )
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize(
    "batch,q_heads,kv_heads,cap,max_len",
    [
        (1024, 14, 2, 128, 100),   # more sequences than workgroups: the grid loops
        (2049, 14, 2, 64, 64),     # past the balanced split's batch limit: fixed chunks
        (5, 8, 1, 700, 700),       # one kv head: one head per wave
        (6, 12, 4, 900, 900),      # 4 kv heads of 3 query heads: head pairs
    ],
)
def test_decode_attention_balanced_shapes(gpu, batch, q_heads, kv_heads, cap, max_len):
    announce(f"decode bf16 balanced B={batch} QH={q_heads} KVH={kv_heads} cap={cap}")
    g = generator(batch + q_heads * 31 + cap)
    lengths = torch.randint(1, max_len + 1, (batch,), generator=g).tolist()
    actual, expected = _decode_case(
        gpu, batch, q_heads, kv_heads, 64, cap, lengths, torch.bfloat16, batch + cap,
        split_tokens=SPLIT_BALANCED, mask_kind="random",
    )
    assert_bf16_close(actual, expected)


def test_decode_attention_balanced_is_deterministic(gpu):
    # The pieces of a sequence merge in a fixed order: repeated calls on the
    # same inputs are bitwise equal.
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    announce("decode bf16 balanced determinism B=32 L=8192")
    g = generator(5)
    q = torch.randn(32, 14, 1, 64, generator=g).bfloat16().to(gpu)
    k = torch.randn(32, 8192, 2, 64, generator=g).bfloat16().to(gpu)
    v = torch.randn(32, 8192, 2, 64, generator=g).bfloat16().to(gpu)
    lengths = torch.randint(4096, 8193, (32,), generator=g).to(gpu)
    outs = [hip_decode_attention(q, k, v, lengths, None, scale=0.125, split_tokens=SPLIT_BALANCED)
            for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("split", [0, 256, SPLIT_BALANCED])
def test_decode_attention_merge_reads_fresh_partials(gpu, split):
    # Back-to-back calls on one workspace alternate between two inputs whose
    # partials differ everywhere: a merge that read a partial of the previous
    # call (a stale copy in some XCD's L2) would break bitwise repeatability.
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    announce(f"decode bf16 merge freshness B=32 L=8192 split_tokens={split}")
    g = generator(6)
    lengths = torch.randint(4096, 8193, (32,), generator=g).to(gpu)
    k = torch.randn(32, 8192, 2, 64, generator=g).bfloat16().to(gpu)
    v = torch.randn(32, 8192, 2, 64, generator=g).bfloat16().to(gpu)
    queries = [torch.randn(32, 14, 1, 64, generator=g).bfloat16().to(gpu) for _ in range(2)]
    first = [hip_decode_attention(q, k, v, lengths, None, scale=0.125, split_tokens=split)
             for q in queries]
    torch.cuda.synchronize()
    assert not torch.equal(first[0], first[1])
    outs = [hip_decode_attention(queries[i % 2], k, v, lengths, None, scale=0.125, split_tokens=split)
            for i in range(40)]
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        assert torch.equal(out, first[i % 2]), f"call {i} differs from the first call on its input"


@pytest.mark.parametrize("split", [0, 64, SPLIT_BALANCED])
def test_decode_attention_empty_sequences(gpu, split):
    # A sequence with no attended token is a softmax over an empty row: NaN,
    # as in the reference; its neighbours are unaffected.
    announce(f"decode bf16 empty sequences split_tokens={split}")
    lengths = [0, 100, 0, 0, 37, 256, 0, 1]
    actual, expected = _decode_case(
        gpu, len(lengths), 14, 2, 64, 256, lengths, torch.bfloat16, 77, split_tokens=split,
        mask_kind="random",
    )
    empty = torch.tensor(lengths) == 0
    assert torch.isnan(expected[empty]).all()
    assert torch.isnan(actual[empty]).all()
    assert_bf16_close(actual[~empty], expected[~empty])


@pytest.mark.parametrize("split", [0, SPLIT_BALANCED])
@pytest.mark.parametrize("mask_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mask_len", [1000, 1001])
def test_decode_attention_mask_dtype_and_length(gpu, mask_dtype, mask_len, split):
    # A mask length that is a multiple of 4 lets the balanced split read the
    # mask 4 tokens per load; 1001 reads it per token.
    announce(f"decode bf16 mask {mask_dtype} mask_len={mask_len} split_tokens={split}")
    actual, expected = _decode_case(
        gpu, 4, 14, 2, 64, 1024, [1001, 999, 3, 640], torch.bfloat16, 43,
        mask_len=mask_len, mask_kind="random", mask_dtype=mask_dtype, split_tokens=split,
    )
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("split", [0, SPLIT_BALANCED])
def test_decode_attention_random_mask_short_mask(gpu, split):
    # Mask shorter than the capacity bounds the attended prefix (execution.py:301-327).
    announce(f"decode bf16 mask_len < capacity, random mask, split_tokens={split}")
    actual, expected = _decode_case(
        gpu, 5, 14, 2, 64, 512, [10, 300, 512, 200, 1], torch.bfloat16, 41,
        mask_len=300, mask_kind="random", split_tokens=split,
    )
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("split", [0, SPLIT_BALANCED])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_attention_head_dim_128(gpu, dtype, split):
    announce(f"decode {dtype} D=128 QH4 KVH2 split_tokens={split}")
    actual, expected = _decode_case(gpu, 8, 4, 2, 128, 1024, [1024, 513, 2, 700, 999, 64, 65, 1000], dtype, 51,
                                    split_tokens=split)
    assert_bf16_close(actual, expected)


def test_decode_attention_fp32_qwen_shape(gpu):
    announce("decode fp32 QH14 KVH2 D64 L=1024")
    actual, expected = _decode_case(gpu, 4, 14, 2, 64, 1024, [1024, 600, 17, 900], torch.float32, 61, mask_kind="random")
    assert_fp32_close(actual, expected)


def test_decode_attention_generic_group_size(gpu):
    # 32 query heads per KV head exceed one MFMA tile: generic kernel path.
    announce("decode bf16 QH32 KVH1 (generic)")
    actual, expected = _decode_case(gpu, 2, 32, 1, 64, 256, [256, 100], torch.bfloat16, 71)
    assert_bf16_close(actual, expected)


def test_decode_attention_zero_length_is_nan(gpu):
    # The reference softmax over an all -inf row is NaN; so is the kernel's.
    announce("decode bf16 zero length")
    actual, expected = _decode_case(gpu, 2, 14, 2, 64, 128, [0, 50], torch.bfloat16, 81)
    assert torch.isnan(expected[0]).all() and torch.isnan(actual[0]).all()
    assert_bf16_close(actual[1], expected[1])


def test_decode_attention_positions_past_length_are_ignored(gpu):
    # Invariance: garbage (including inf/NaN bit patterns) after the length
    # must not change the result.
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    announce("decode bf16 garbage past length")
    g = generator(91)
    batch, cap = 2, 256
    q = torch.randn(batch, 14, 1, 64, generator=g).bfloat16().to(gpu)
    k = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
    v = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
    lengths = torch.tensor([100, 37], device=gpu)
    mask = torch.zeros(batch, 1, 1, cap, dtype=torch.bfloat16, device=gpu)
    base = hip_decode_attention(q, k, v, lengths, mask, scale=0.125)
    k2, v2 = k.clone(), v.clone()
    k2[0, 100:] = float("nan")
    v2[0, 100:] = float("inf")
    k2[1, 37:] = float("inf")
    v2[1, 37:] = float("nan")
    again = hip_decode_attention(q, k2, v2, lengths, mask, scale=0.125)
    torch.cuda.synchronize()
    assert_bitwise_equal(again, base)


# ------------------------------------------------------------------ rms_norm


@pytest.mark.parametrize("waves", [None, 1, 4])
@pytest.mark.parametrize("rows", [1, 8, 64, 512, 32768])
def test_rms_norm_bf16_round_before_weight(gpu, rows, waves):
    # Both launch widths a profile plan can pick (one wave per row, a
    # 256-thread workgroup per row) and the automatic one.
    from stateful_llm_compiler_hip.backends import hip_rms_norm

    announce(f"rms_norm bf16 rows={rows} waves_per_row={waves}")
    g = generator(rows)
    x = torch.randn(rows, 896, generator=g).bfloat16()
    w = (1.0 + 0.1 * torch.randn(896, generator=g)).bfloat16()
    expected = ref.rms_norm(x, w, epsilon=1e-6, round_before_weight=True)
    actual = hip_rms_norm(x.to(gpu), w.to(gpu), epsilon=1e-6, round_before_weight=True,
                          num_warps=waves)
    torch.cuda.synchronize()
    assert actual.dtype == expected.dtype
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("hidden", [896, 1536, 4096, 100])
def test_rms_norm_fp32(gpu, hidden):
    from stateful_llm_compiler_hip.backends import hip_rms_norm

    announce(f"rms_norm fp32 hidden={hidden}")
    g = generator(hidden)
    x = torch.randn(3, 5, hidden, generator=g)
    w = torch.randn(hidden, generator=g)
    expected = ref.rms_norm(x, w, epsilon=1e-6)
    actual = hip_rms_norm(x.to(gpu), w.to(gpu), epsilon=1e-6)
    torch.cuda.synchronize()
    assert_fp32_close(actual, expected)


def test_rms_norm_fp16_and_output_dtype(gpu):
    from stateful_llm_compiler_hip.backends import hip_rms_norm

    announce("rms_norm fp16 in -> f32 out")
    g = generator(5)
    x = torch.randn(16, 1536, generator=g).half()
    w = torch.randn(1536, generator=g).half()
    expected = ref.rms_norm(x, w, epsilon=1e-5, output_dtype="f32")
    actual = hip_rms_norm(x.to(gpu), w.to(gpu), epsilon=1e-5, output_dtype="f32")
    torch.cuda.synchronize()
    assert actual.dtype == torch.float32
    assert_fp32_close(actual, expected, rtol=2e-3)


# ---------------------------------------------------------------------- rope


def _rope_inputs(batch, tokens, dtype, seed, past_max=4096):
    g = generator(seed)
    q = torch.randn(batch, tokens, 14, 64, generator=g).to(dtype).transpose(1, 2)
    k = torch.randn(batch, tokens, 2, 64, generator=g).to(dtype).transpose(1, 2)
    past = torch.randint(0, past_max + 1, (batch, 1), generator=g)
    positions = past + torch.arange(tokens).view(1, -1)
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    freqs = positions.float().unsqueeze(-1) * inv_freq.view(1, 1, -1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return q, k, emb.cos().to(dtype), emb.sin().to(dtype)


@pytest.mark.parametrize("batch", [1, 8, 64])
@pytest.mark.parametrize("tokens", [1, 128, 512])
def test_rope_config3_bitexact_bf16(gpu, batch, tokens):
    from stateful_llm_compiler_hip.backends import hip_rope

    announce(f"rope bf16 B={batch} T={tokens}")
    q, k, cos, sin = _rope_inputs(batch, tokens, torch.bfloat16, batch * 1000 + tokens)
    eq, ek = ref.rope(q, k, cos, sin)
    qd = q.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    kd = k.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    aq, ak = hip_rope(qd, kd, cos.to(gpu), sin.to(gpu))
    torch.cuda.synchronize()
    assert_bitwise_equal(aq, eq)
    assert_bitwise_equal(ak, ek)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rope_other_dtypes_bitexact(gpu, dtype):
    from stateful_llm_compiler_hip.backends import hip_rope

    announce(f"rope {dtype}")
    q, k, cos, sin = _rope_inputs(2, 7, dtype, 2026)
    eq, ek = ref.rope(q, k, cos, sin)
    aq, ak = hip_rope(q.to(gpu), k.to(gpu), cos.to(gpu), sin.to(gpu))
    torch.cuda.synchronize()
    assert_bitwise_equal(aq, eq)
    assert_bitwise_equal(ak, ek)


def test_decode_attention_merge_in_kernel_over_many_streams(gpu):
    # The split kernel merges in its last workgroup per (batch, kv-head),
    # counting arrivals in the calling stream's workspace.  Every one of 20
    # streams gets its own workspace and the in-kernel merge (there is no
    # per-stream limit), and all agree bit for bit, call after call.
    from stateful_llm_compiler_hip import _native
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    announce("decode bf16 in-kernel merge over 20 streams")
    g = generator(91)
    batch, cap = 8, 2048
    q = torch.randn(batch, 14, 1, 64, generator=g).bfloat16().to(gpu)
    k = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
    v = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
    lengths = torch.randint(1, cap + 1, (batch,), generator=g).to(gpu)
    lengths[0] = 0  # an empty sequence: NaN
    mask = torch.randn(batch, 1, 1, cap, generator=g).bfloat16().to(gpu)
    outs, buffers = [], set()
    streams = [torch.cuda.Stream() for _ in range(20)]
    for stream in streams:
        with torch.cuda.stream(stream):
            for _ in range(2):
                out = hip_decode_attention(q, k, v, lengths, mask, scale=0.125)
            buffers.add(_native.stream_workspace(gpu).counters(1).data_ptr())
        stream.synchronize()
        outs.append(out.cpu())
    assert len(buffers) == 20
    for out in outs[1:]:
        assert torch.equal(out.view(torch.int16), outs[0].view(torch.int16))
    expected = ref.decode_attention(q.cpu(), k.cpu(), v.cpu(), lengths.cpu(), mask.cpu(), groups=7, scale=0.125)
    assert torch.isnan(outs[0][0]).all()
    assert_bf16_close(outs[0][1:], expected[1:])


def test_decode_attention_workspaces_replay_concurrently(gpu):
    # Two captured graphs, each with its own workspace, replayed at the same
    # time on two streams: both equal their sequential (eager) results bit for
    # bit.
    from stateful_llm_compiler_hip import _native
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    announce("decode bf16 two graphs with own workspaces replayed concurrently")
    g = generator(92)
    batch, cap = 16, 4096
    cases = []
    for _ in range(2):
        q = torch.randn(batch, 14, 1, 64, generator=g).bfloat16().to(gpu)
        k = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
        v = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
        lengths = torch.randint(cap // 2, cap + 1, (batch,), generator=g).to(gpu)
        mask = torch.zeros(batch, 1, 1, cap, dtype=torch.bfloat16, device=gpu)
        cases.append((q, k, v, lengths, mask, _native.DeviceWorkspace(gpu)))
    eager = [hip_decode_attention(*c[:5], scale=0.125, workspace=c[5]) for c in cases]
    torch.cuda.synchronize()
    graphs, outs = [], []
    for c in cases:
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
            outs.append(hip_decode_attention(*c[:5], scale=0.125, workspace=c[5]))
        torch.cuda.current_stream().wait_stream(stream)
        graphs.append(graph)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in graphs]
    for replay in range(3):
        for graph, stream in zip(graphs, streams):
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                for _ in range(4):
                    graph.replay()
        for stream in streams:
            torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        for out, ref_out in zip(outs, eager):
            assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), f"replay {replay}"


@pytest.mark.parametrize("batch,capacity,lengths,mask_kind,dtype,head_dim", [
    (3, 65, [7, 31, 65], "zeros", torch.bfloat16, 64),       # reference KAT lengths
    (8, 1024, None, "random", torch.bfloat16, 64),           # config 2, random mask
    (4, 4096, None, "zeros", torch.bfloat16, 64),            # the exact order's longest mask
    (4, 800, [1, 672, 673, 800], "random", torch.bfloat16, 64),  # either side of the LDS-kept V (672 tokens)
    (3, 700, [0, 1, 700], "random", torch.float16, 128),     # D = 128, an empty row (NaN)
    (2, 300, [150, 299], "zeros", torch.bfloat16, 80),       # generic kernel
])
def test_decode_attention_exact_softmax_order(gpu, batch, capacity, lengths, mask_kind, dtype, head_dim):
    """The exact order matches the oracle (the reference executor's order) in
    nearly every element bit for bit, and in more elements than the online
    order does."""

    announce(f"decode exact order B={batch} cap={capacity} {mask_kind} {dtype} D={head_dim}")
    g = generator(capacity + batch)
    if lengths is None:
        lengths = torch.randint(capacity // 2, capacity + 1, (batch,), generator=g).tolist()
    q_heads = 14 if head_dim != 128 else 8
    case = dict(mask_kind=mask_kind)
    exact, expected = _decode_case(gpu, batch, q_heads, 2, head_dim, capacity, lengths, dtype, 5,
                                   softmax_order="exact", **case)
    online, _ = _decode_case(gpu, batch, q_heads, 2, head_dim, capacity, lengths, dtype, 5, **case)
    empty = torch.tensor(lengths) == 0
    assert torch.isnan(exact[empty]).all()
    exact, online, expected = exact[~empty], online[~empty], expected[~empty]
    assert_bf16_close(exact, expected)
    e = float((exact.float() == expected.float()).float().mean())
    o = float((online.float() == expected.float()).float().mean())
    print(f"bitwise-equal fraction: exact {e:.4f}, online {o:.4f}")
    assert e >= 0.97 and e >= o


@pytest.mark.parametrize("mask_len", [1024, 700])
def test_marked_zero_mask_is_skipped_only_over_the_capacity(gpu, mask_len):
    """A mask marked all-zero (the graph decoder's) gives the unmarked mask's
    output bit for bit; one shorter than the capacity still bounds the
    attended range, so it is read."""
    from stateful_llm_compiler_hip.execution import PreallocatedKVCacheState, mark_zero_mask

    announce(f"marked zero mask mask_len={mask_len}")
    g = generator(77)
    batch, cap = 4, 1024
    q = torch.randn(batch, 14, 1, 64, generator=g).bfloat16().to(gpu)
    k = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
    v = torch.randn(batch, cap, 2, 64, generator=g).bfloat16().to(gpu)
    lengths = torch.tensor([1, 300, 900, 1024], dtype=torch.int64, device=gpu)
    state = PreallocatedKVCacheState((k,), (v,), (lengths,), cap,
                                     overflow=torch.zeros(1, dtype=torch.int32, device=gpu))
    plain = torch.zeros(batch, 1, 1, mask_len, dtype=torch.bfloat16, device=gpu)
    marked = mark_zero_mask(torch.zeros_like(plain))
    for order in ("exact", "online"):
        a = state.decode_attention(0, q, plain, groups=7, scale=0.125, softmax_order=order)
        b = state.decode_attention(0, q, marked, groups=7, scale=0.125, softmax_order=order)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), order


@pytest.mark.parametrize("order", ["exact", "online"])
def test_decode_attention_ignores_rows_past_the_length(gpu, order):
    """Rows past a sequence's length take no part, whatever the cache holds
    there: NaN and inf in them leave the output bit for bit as zeros do
    (lengths on either side of the exact order's LDS-kept V)."""
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    announce(f"decode attention ignores rows past the length order={order}")
    g = generator(41)
    batch, cap = 4, 1024
    lengths = torch.tensor([5, 300, 672, 900], dtype=torch.int64)
    q = torch.randn(batch, 14, 1, 64, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(batch, cap, 2, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(batch, cap, 2, 64, generator=g).to(torch.bfloat16)
    past = torch.arange(cap).view(1, cap) >= lengths.view(batch, 1)
    outs = []
    for fill in (0.0, float("nan"), float("inf")):
        kf, vf = k.clone(), v.clone()
        kf[past] = fill
        vf[past] = fill
        out = hip_decode_attention(q, kf.to(gpu), vf.to(gpu), lengths.to(gpu), None,
                                   scale=0.125, softmax_order=order)
        outs.append(out.cpu())
    assert torch.isfinite(outs[0].float()).all()
    for out in outs[1:]:
        assert torch.equal(out.view(torch.int16), outs[0].view(torch.int16))


def test_decode_attention_exact_order_rejects_long_masks(gpu):
    from stateful_llm_compiler_hip._native import KernelLaunchError
    from stateful_llm_compiler_hip.backends import hip_decode_attention

    announce("decode exact order over its longest mask is rejected")
    q = torch.zeros(1, 14, 1, 64, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(1, 4097, 2, 64, dtype=torch.bfloat16, device=gpu)
    lengths = torch.ones(1, dtype=torch.int64, device=gpu)
    with pytest.raises(KernelLaunchError, match="exact softmax order"):
        hip_decode_attention(q, k, k, lengths, None, scale=0.125, softmax_order="exact")
