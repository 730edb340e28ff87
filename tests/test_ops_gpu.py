"""GPU parity of the small device ops that complete a compiled Qwen2 step."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from helpers import announce, assert_bitwise_equal, generator
from oracle.qwen2_model import rope_tables
from stateful_llm_compiler_hip.qwen2 import Qwen2Config, inverse_frequency

pytestmark = pytest.mark.gpu


def _ulp(x, bits):
    return torch.exp2(torch.floor(torch.log2(x.abs().double().clamp_min(2.0**-120))) - (bits - 1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_embedding_bitexact(gpu, dtype):
    from stateful_llm_compiler_hip.backends import hip_embedding

    announce(f"embedding {dtype}")
    g = generator(1)
    table = torch.randn(1000, 896, generator=g).to(dtype)
    ids = torch.randint(0, 1000, (8, 33), generator=g)
    out = hip_embedding(ids.to(gpu), table.to(gpu))
    torch.cuda.synchronize()
    assert_bitwise_equal(out, F.embedding(ids, table))


def test_embedding_out_of_range_flag(gpu):
    from stateful_llm_compiler_hip.backends import hip_embedding

    announce("embedding bad index flag")
    table = torch.randn(10, 16).to(gpu)
    flag = torch.zeros(1, dtype=torch.int32, device=gpu)
    hip_embedding(torch.tensor([[3, 11]], device=gpu), table, bad_index=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_add_bitexact(gpu, dtype):
    from stateful_llm_compiler_hip.backends import hip_add

    announce(f"add {dtype}")
    g = generator(2)
    a = torch.randn(4, 7, 896, generator=g).to(dtype)
    b = torch.randn(4, 7, 896, generator=g).to(dtype)
    out = hip_add(a.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    assert_bitwise_equal(out, a + b)


@pytest.mark.parametrize("numel", [8 * 4864, 7 * 13])
def test_swiglu_within_one_ulp(gpu, numel):
    from stateful_llm_compiler_hip.backends import hip_swiglu

    announce(f"swiglu bf16 n={numel}")
    g = generator(3)
    gate = (torch.randn(numel, generator=g) * 3).bfloat16()
    up = torch.randn(numel, generator=g).bfloat16()
    out = hip_swiglu(gate.to(gpu), up.to(gpu)).cpu()
    expected = F.silu(gate) * up
    # silu is rounded to bf16 before the multiply; transcendental rounding may
    # differ by one ulp of silu, which moves the product by at most ~1 ulp.
    assert ((out.double() - expected.double()).abs() <= 2 * _ulp(expected, 8) + 1e-30).all()


@pytest.mark.parametrize("dtype,bits", [(torch.bfloat16, 8), (torch.float32, 24)])
def test_rope_table(gpu, dtype, bits):
    from stateful_llm_compiler_hip.backends import hip_rope_table

    announce(f"rope_table {dtype}")
    c = Qwen2Config()
    g = generator(4)
    past = torch.randint(0, 4097, (8, 1), generator=g)
    pos = past + torch.arange(128).view(1, -1)
    inv = inverse_frequency(c)
    cos, sin = hip_rope_table(pos.to(gpu), inv.to(gpu), dtype)
    torch.cuda.synchronize()
    ec, es = rope_tables(pos, inv, dtype)
    # cos/sin of the same fp32 argument: libm vs device math differ by at most a
    # couple of fp32 ulps, i.e. one ulp after rounding to the table dtype.
    for a, e in ((cos.cpu(), ec), (sin.cpu(), es)):
        tol = _ulp(e, bits) * (1 if bits == 8 else 4) + (1e-7 if bits == 24 else 0)
        assert ((a.double() - e.double()).abs() <= tol).all()


def test_kv_advance_and_overflow(gpu):
    from stateful_llm_compiler_hip.backends import hip_kv_advance

    announce("kv_advance")
    lengths = torch.tensor([0, 5, 62], device=gpu)
    flag = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = hip_kv_advance(lengths, 2, 64, overflow=flag)
    torch.cuda.synchronize()
    assert out.tolist() == [2, 7, 64] and int(flag.item()) == 0
    hip_kv_advance(out, 1, 64, out=out, overflow=flag)
    torch.cuda.synchronize()
    assert out.tolist() == [3, 8, 65] and int(flag.item()) == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_argmax_matches_torch(gpu, dtype):
    from stateful_llm_compiler_hip.backends import hip_argmax

    announce(f"argmax {dtype}")
    g = generator(5)
    logits = torch.randn(8, 1, 151936, generator=g).to(dtype)
    logits[0, 0, 17] = 100.0
    logits[0, 0, 99] = 100.0  # tie: the first index wins
    out = hip_argmax(logits.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), logits.argmax(-1))


@pytest.mark.parametrize("rows,cols", [(1, 151936), (8, 151936), (3, 50001), (300, 8192), (2, 100)])
def test_argmax_segments_ties_and_nan(gpu, rows, cols):
    # Wide rows are reduced by several workgroups per row (segments combined
    # in index order by the last one): ties across segment boundaries keep the
    # first index, a NaN wins like torch.argmax, odd widths end mid-vector.
    from stateful_llm_compiler_hip.backends import hip_argmax

    announce(f"argmax segments rows={rows} cols={cols}")
    g = generator(rows + cols)
    logits = torch.randn(rows, cols, generator=g).bfloat16()
    logits[0, cols - 1] = 50.0
    logits[0, cols // 2] = 50.0       # tie in a later and an earlier segment
    if rows > 1:
        logits[1, cols // 3] = float("nan")
        logits[1, cols - 2] = float("nan")
    for _ in range(3):  # the per-row counters re-arm between calls
        out = hip_argmax(logits.to(gpu))
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), logits.argmax(-1))
