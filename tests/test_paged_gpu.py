"""GPU parity of the paged KV layout (pages + block table).

Decode attention over pages must equal, bit for bit, the contiguous kernel
over the gathered buffer (same split, same softmax order), and match the
oracle's ``decode_attention`` over ``gather_pages`` within the bf16 bar
(2e-2 absolute or one bf16 ulp).  The paged KV store is bit-exact against
``oracle.kernels.paged_kv_store``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, assert_bf16_close, assert_bitwise_equal, generator
from oracle import kernels as ref

pytestmark = pytest.mark.gpu


def _paging(g, batch, pages, extra=5):
    """A block table naming distinct pool pages in a random order (the pool
    has ``extra`` pages no sequence owns)."""

    order = torch.randperm(batch * pages + extra, generator=g)[: batch * pages]
    return order.view(batch, pages).to(torch.int32), batch * pages + extra


def _scatter(buffer, table, num_pages, page_tokens):
    """The pool whose gather through ``table`` is ``buffer``; unowned pages
    hold NaN so that a wrong page read shows up."""

    batch, capacity = buffer.shape[:2]
    pool = torch.full((num_pages, page_tokens) + tuple(buffer.shape[2:]), float("nan"), dtype=buffer.dtype)
    pages = capacity // page_tokens
    pool[table.view(-1).long()] = buffer.reshape(batch * pages, page_tokens, *buffer.shape[2:])
    return pool


def _paged_case(gpu, batch, q_heads, kv_heads, head_dim, capacity, page_tokens, lengths, dtype, seed,
                *, split_tokens=0, softmax_order="online", mask_kind="zeros", length_dtype=torch.int64):
    from stateful_llm_compiler_hip.backends import hip_decode_attention, hip_paged_decode_attention

    g = generator(seed)
    query = torch.randn(batch, q_heads, 1, head_dim, generator=g).to(dtype)
    key = torch.randn(batch, capacity, kv_heads, head_dim, generator=g).to(dtype)
    value = torch.randn(batch, capacity, kv_heads, head_dim, generator=g).to(dtype)
    if mask_kind == "zeros":
        mask = torch.zeros(batch, 1, 1, capacity, dtype=dtype)
    else:
        mask = (torch.randn(batch, 1, 1, capacity, generator=g) * 2.0).to(dtype)
    lengths_t = torch.tensor(lengths, dtype=torch.int64)
    table, num_pages = _paging(g, batch, capacity // page_tokens)
    key_pool = _scatter(key, table, num_pages, page_tokens)
    value_pool = _scatter(value, table, num_pages, page_tokens)

    # The oracle reads the gathered layout.
    bits = torch.int16
    gathered_k = torch.from_numpy(ref.gather_pages(key_pool.view(bits).numpy(), table.numpy())).view(dtype)
    gathered_v = torch.from_numpy(ref.gather_pages(value_pool.view(bits).numpy(), table.numpy())).view(dtype)
    assert torch.equal(gathered_k.view(bits), key.view(bits))
    expected = ref.decode_attention(query, gathered_k, gathered_v, lengths_t, mask,
                                    groups=q_heads // kv_heads, scale=head_dim**-0.5)

    qd, md = query.to(gpu), mask.to(gpu)
    ld = lengths_t.to(length_dtype).to(gpu)
    paged = hip_paged_decode_attention(qd, key_pool.to(gpu), value_pool.to(gpu), table.to(gpu), ld, md,
                                       scale=head_dim**-0.5, split_tokens=split_tokens,
                                       softmax_order=softmax_order)
    contiguous = hip_decode_attention(qd, key.to(gpu), value.to(gpu), ld, md, scale=head_dim**-0.5,
                                      split_tokens=split_tokens, softmax_order=softmax_order)
    torch.cuda.synchronize()
    return paged.cpu(), contiguous.cpu(), expected


@pytest.mark.parametrize("page_tokens", [16, 64, 256])
@pytest.mark.parametrize("batch", [1, 8, 32])
def test_paged_decode_attention_equals_contiguous(gpu, batch, page_tokens):
    announce(f"paged decode bf16 B={batch} L=2048 page_tokens={page_tokens}")
    g = generator(500 + batch + page_tokens)
    lengths = torch.randint(1024, 2049, (batch,), generator=g).tolist()
    paged, contiguous, expected = _paged_case(gpu, batch, 14, 2, 64, 2048, page_tokens, lengths,
                                              torch.bfloat16, 501 + batch)
    assert_bitwise_equal(paged, contiguous)
    assert_bf16_close(paged, expected)


@pytest.mark.parametrize("order", ["online", "exact"])
@pytest.mark.parametrize("split", [0, 128, -1])
@pytest.mark.parametrize("length_dtype", [torch.int64, torch.int32])
def test_paged_decode_attention_orders_splits_masks(gpu, order, split, length_dtype):
    announce(f"paged decode bf16 order={order} split={split} lengths={length_dtype}")
    # -1 (the balanced split) runs the fixed split over pages: it must still
    # equal the contiguous call (the contiguous balanced split can differ in
    # rounding, so compare it with the oracle only).
    paged, contiguous, expected = _paged_case(
        gpu, 5, 14, 2, 64, 1024, 32, [0, 1, 333, 1000, 1024], torch.bfloat16, 520,
        split_tokens=split, softmax_order=order, mask_kind="random", length_dtype=length_dtype)
    if split >= 0:
        assert_bitwise_equal(paged, contiguous)
    # Sequence 0 attends to nothing: NaN, as in the reference.
    assert torch.isnan(paged[0]).all() and torch.isnan(expected[0]).all()
    assert_bf16_close(paged[1:], expected[1:])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim,q_heads,kv_heads", [(64, 14, 2), (128, 32, 8), (128, 16, 1)])
def test_paged_decode_attention_shapes(gpu, dtype, head_dim, q_heads, kv_heads):
    announce(f"paged decode {dtype} D={head_dim} QH={q_heads} KVH={kv_heads}")
    paged, contiguous, expected = _paged_case(
        gpu, 3, q_heads, kv_heads, head_dim, 512, 16, [17, 500, 512], dtype, 530, mask_kind="random")
    assert_bitwise_equal(paged, contiguous)
    assert_bf16_close(paged, expected)


def test_paged_decode_attention_headline_shape(gpu):
    # The bench shape: B = 32, L = 8192, lengths U[L/2, L], 64-token pages.
    announce("paged decode bf16 B=32 L=8192 page_tokens=64")
    g = generator(540)
    lengths = torch.randint(4096, 8193, (32,), generator=g).tolist()
    paged, contiguous, expected = _paged_case(gpu, 32, 14, 2, 64, 8192, 64, lengths, torch.bfloat16, 541)
    assert_bitwise_equal(paged, contiguous)
    assert_bf16_close(paged, expected)


@pytest.mark.parametrize("tokens,positions", [(1, [0, 31, 63]), (20, [0, 17, 60]), (64, [0, 0, 0])])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_kv_store_bitexact(gpu, tokens, positions, dtype):
    from stateful_llm_compiler_hip.backends import hip_paged_kv_store

    announce(f"paged kv_store {dtype} T={tokens} positions={positions}")
    g = generator(550 + tokens)
    batch, heads, head_dim, page_tokens, pages = 3, 2, 64, 16, 4
    table, num_pages = _paging(g, batch, pages)
    key_pool = torch.randn(num_pages, page_tokens, heads, head_dim, generator=g).to(dtype)
    value_pool = torch.randn(num_pages, page_tokens, heads, head_dim, generator=g).to(dtype)
    # B x T x H x D projections viewed as B x H x T x D, as the model hands them.
    key = torch.randn(batch, tokens, heads, head_dim, generator=g).to(dtype).transpose(1, 2)
    value = torch.randn(batch, tokens, heads, head_dim, generator=g).to(dtype).transpose(1, 2)
    pos = torch.tensor(positions, dtype=torch.int64)
    overflow = torch.zeros(1, dtype=torch.int32, device=gpu)

    kp, vp = key_pool.to(gpu), value_pool.to(gpu)
    hip_paged_kv_store(kp, vp, table.to(gpu), key.to(gpu), value.to(gpu), pos.to(gpu), overflow=overflow)
    torch.cuda.synchronize()

    bits = torch.int16 if dtype != torch.float32 else torch.int32
    exp_k = key_pool.view(bits).numpy().copy()
    exp_v = value_pool.view(bits).numpy().copy()
    ref.paged_kv_store(exp_k, exp_v, table.numpy(), key.contiguous().view(bits).numpy(),
                       value.contiguous().view(bits).numpy(), pos.numpy())
    assert_bitwise_equal(kp.cpu().view(bits), torch.from_numpy(exp_k))
    assert_bitwise_equal(vp.cpu().view(bits), torch.from_numpy(exp_v))
    capacity = pages * page_tokens
    spills = any(p + tokens > capacity for p in positions)
    assert int(overflow.item()) == int(spills)


def test_paged_store_then_attention_equals_contiguous(gpu):
    # Decode steps through the paged path (store the new row, attend) give the
    # contiguous path's outputs bit for bit.
    from stateful_llm_compiler_hip.backends import (
        hip_decode_attention, hip_kv_store, hip_paged_decode_attention, hip_paged_kv_store)

    announce("paged store+attention 4 steps B=4 L=256")
    g = generator(560)
    batch, kvh, qh, d, page_tokens, pages = 4, 2, 14, 64, 16, 16
    cap = pages * page_tokens
    table, num_pages = _paging(g, batch, pages)
    table = table.to(gpu)
    kp = torch.zeros(num_pages, page_tokens, kvh, d, dtype=torch.bfloat16, device=gpu)
    vp = torch.zeros_like(kp)
    kb = torch.zeros(batch, cap, kvh, d, dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    lengths = torch.tensor([0, 5, 100, 250], dtype=torch.int64)
    prefix_k = torch.randn(batch, kvh, 250, d, generator=g).to(torch.bfloat16).to(gpu)
    prefix_v = torch.randn(batch, kvh, 250, d, generator=g).to(torch.bfloat16).to(gpu)
    zero = torch.zeros(batch, dtype=torch.int64, device=gpu)
    hip_kv_store(kb, vb, prefix_k, prefix_v, zero)
    hip_paged_kv_store(kp, vp, table, prefix_k, prefix_v, zero)
    ld = lengths.to(gpu)
    mask = torch.zeros(batch, 1, 1, cap, dtype=torch.bfloat16, device=gpu)
    for step in range(4):
        k = torch.randn(batch, kvh, 1, d, generator=g).to(torch.bfloat16).to(gpu)
        v = torch.randn(batch, kvh, 1, d, generator=g).to(torch.bfloat16).to(gpu)
        q = torch.randn(batch, qh, 1, d, generator=g).to(torch.bfloat16).to(gpu)
        hip_kv_store(kb, vb, k, v, ld)
        hip_paged_kv_store(kp, vp, table, k, v, ld)
        ld = ld + 1
        a = hip_paged_decode_attention(q, kp, vp, table, ld, mask, scale=d**-0.5)
        b = hip_decode_attention(q, kb, vb, ld, mask, scale=d**-0.5)
        torch.cuda.synchronize()
        assert_bitwise_equal(a, b)


def test_paged_operand_checks(gpu):
    from stateful_llm_compiler_hip.backends import hip_paged_decode_attention

    q = torch.zeros(2, 14, 1, 64, dtype=torch.bfloat16, device=gpu)
    pool = torch.zeros(8, 24, 2, 64, dtype=torch.bfloat16, device=gpu)  # 24: not a power of two
    table = torch.zeros(2, 4, dtype=torch.int32, device=gpu)
    lengths = torch.zeros(2, dtype=torch.int64, device=gpu)
    with pytest.raises(ValueError, match="power of two"):
        hip_paged_decode_attention(q, pool, pool, table, lengths, None, scale=0.125)
    pool = torch.zeros(8, 16, 2, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="int32"):
        hip_paged_decode_attention(q, pool, pool, table.long(), lengths, None, scale=0.125)
    mask = torch.zeros(2, 1, 1, 65, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="capacity"):
        hip_paged_decode_attention(q, pool, pool, table, lengths, mask, scale=0.125)
    out = hip_paged_decode_attention(q, pool, pool, table, lengths + 3, None, scale=0.125)
    torch.cuda.synchronize()
    assert np.count_nonzero(out.float().cpu().numpy()) == 0


@pytest.mark.parametrize("order", ["online", "exact"])
@pytest.mark.parametrize("page_tokens", [16, 64])
def test_paged_rope_decode_attention_equals_contiguous_and_unfused(gpu, order, page_tokens):
    # One decode token: RoPE, store at lengths[b], advance, attention -- the
    # fused paged kernel against (a) the fused contiguous kernel on the
    # gathered buffers and (b) RoPE, paged store and paged attention in turn.
    from stateful_llm_compiler_hip.backends import (
        hip_paged_decode_attention, hip_paged_kv_store, hip_paged_rope_decode_attention,
        hip_rope, hip_rope_decode_attention)

    announce(f"paged rope decode attention order={order} page_tokens={page_tokens}")
    g = generator(570 + page_tokens)
    batch, qh, kvh, d, cap = 4, 14, 2, 64, 512
    pages = cap // page_tokens
    table, num_pages = _paging(g, batch, pages)
    key_buffer = torch.randn(batch, cap, kvh, d, generator=g).to(torch.bfloat16)
    value_buffer = torch.randn(batch, cap, kvh, d, generator=g).to(torch.bfloat16)
    kp = _scatter(key_buffer, table, num_pages, page_tokens).to(gpu)
    vp = _scatter(value_buffer, table, num_pages, page_tokens).to(gpu)
    kb, vb = key_buffer.to(gpu), value_buffer.to(gpu)
    table = table.to(gpu)
    lengths = torch.tensor([0, 17, 300, 511], dtype=torch.int64, device=gpu)
    q = torch.randn(batch, qh, 1, d, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(batch, kvh, 1, d, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(batch, kvh, 1, d, generator=g).to(torch.bfloat16).to(gpu)
    cos = torch.randn(batch, 1, d, generator=g).to(torch.bfloat16).to(gpu)
    sin = torch.randn(batch, 1, d, generator=g).to(torch.bfloat16).to(gpu)
    mask = torch.zeros(batch, 1, 1, cap, dtype=torch.bfloat16, device=gpu)

    kp2, vp2 = kp.clone(), vp.clone()
    out_paged = lengths.clone()
    fused = hip_paged_rope_decode_attention(q, k, v, cos, sin, kp, vp, table, lengths, out_paged,
                                            mask, scale=d**-0.5, softmax_order=order)
    assert fused is not None
    out_contig = lengths.clone()
    contiguous = hip_rope_decode_attention(q, k, v, cos, sin, kb, vb, lengths, out_contig, mask,
                                           scale=d**-0.5, softmax_order=order)
    assert contiguous is not None
    q_rot, k_rot = hip_rope(q, k, cos, sin)
    hip_paged_kv_store(kp2, vp2, table, k_rot, v, lengths)
    unfused = hip_paged_decode_attention(q_rot, kp2, vp2, table, lengths + 1, mask, scale=d**-0.5,
                                         softmax_order=order)
    torch.cuda.synchronize()
    assert torch.equal(out_paged, lengths + 1) and torch.equal(out_contig, lengths + 1)
    assert_bitwise_equal(fused, contiguous)
    assert_bitwise_equal(fused, unfused)
    gathered_k = kp.view(torch.int16)[table.long()].reshape(batch, cap, kvh, d)
    assert_bitwise_equal(gathered_k, kb.view(torch.int16))
    assert_bitwise_equal(kp.view(torch.int16), kp2.view(torch.int16))
    assert_bitwise_equal(vp.view(torch.int16), vp2.view(torch.int16))
