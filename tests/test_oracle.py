"""Pins the CPU oracle (oracle/kernels.py) -- it is trusted only after this.

Each oracle function is checked against something other than its own formula:
the reference's known-answer cases (test_triton_backend.py:380-466), float64
brute force on small inputs, library routines (torch SDPA, F.rms_norm),
closed forms (rotation norm preservation, softmax shift invariance) and
invariants chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import generator
from oracle import kernels as ref


# ------------------------------------------------------------ decode attention


def _brute_force_decode(q, kb, vb, lengths, mask, groups, scale):
    """float64 loops: out[b,h] = sum_s softmax(scale*q.k_s + mask_s) v_s."""

    B, QH, _, D = q.shape
    out = torch.zeros(B, QH, 1, D, dtype=torch.float64)
    S = mask.shape[-1]
    for b in range(B):
        for h in range(QH):
            kvh = h // groups
            logits = []
            for s in range(min(S, int(lengths[b]))):
                dot = sum(float(q[b, h, 0, d]) * float(kb[b, s, kvh, d]) for d in range(D))
                logits.append(dot * scale + float(mask[b, 0, 0, s]))
            m = max(logits)
            w = [math.exp(x - m) for x in logits]
            total = sum(w)
            for d in range(D):
                out[b, h, 0, d] = sum(wi * float(vb[b, s, kvh, d]) for s, wi in enumerate(w)) / total
    return out


def test_decode_attention_matches_float64_brute_force():
    g = generator(1)
    B, QH, KVH, D, cap = 2, 4, 2, 8, 9
    q = torch.randn(B, QH, 1, D, generator=g, dtype=torch.float64)
    kb = torch.randn(B, cap, KVH, D, generator=g, dtype=torch.float64)
    vb = torch.randn(B, cap, KVH, D, generator=g, dtype=torch.float64)
    mask = torch.randn(B, 1, 1, 8, generator=g, dtype=torch.float64)
    lengths = torch.tensor([3, 8])
    got = ref.decode_attention(q, kb, vb, lengths, mask, groups=2, scale=0.3)
    want = _brute_force_decode(q, kb, vb, lengths, mask, 2, 0.3)
    # The reference softmax runs in fp32 (scores.float()), hence fp32 accuracy.
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)


def test_decode_attention_reference_lengths_case_against_sdpa():
    # Shape of the reference KAT (lengths [7, 31, 65], cap 65, QH4 KVH2 D16),
    # checked against torch's SDPA with an explicit boolean mask.
    g = generator(2)
    B, QH, KVH, D, cap = 3, 4, 2, 16, 65
    q = torch.randn(B, QH, 1, D, generator=g)
    kb = torch.randn(B, cap, KVH, D, generator=g)
    vb = torch.randn(B, cap, KVH, D, generator=g)
    lengths = torch.tensor([7, 31, 65])
    mask = torch.zeros(B, 1, 1, cap)
    got = ref.decode_attention(q, kb, vb, lengths, mask, groups=2, scale=D**-0.5)
    k = kb.permute(0, 2, 1, 3).repeat_interleave(2, dim=1)
    v = vb.permute(0, 2, 1, 3).repeat_interleave(2, dim=1)
    allowed = (torch.arange(cap).view(1, 1, 1, cap) < lengths.view(-1, 1, 1, 1))
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=allowed, scale=D**-0.5)
    torch.testing.assert_close(got, want, rtol=3e-5, atol=3e-5)


def test_decode_attention_ignores_positions_past_length_and_shift_invariant():
    g = generator(3)
    q = torch.randn(2, 4, 1, 8, generator=g)
    kb = torch.randn(2, 10, 2, 8, generator=g)
    vb = torch.randn(2, 10, 2, 8, generator=g)
    lengths = torch.tensor([4, 10])
    mask = torch.zeros(2, 1, 1, 10)
    base = ref.decode_attention(q, kb, vb, lengths, mask, groups=2, scale=0.5)
    kb2, vb2 = kb.clone(), vb.clone()
    kb2[0, 4:] = 1e6
    vb2[0, 4:] = -1e6
    torch.testing.assert_close(ref.decode_attention(q, kb2, vb2, lengths, mask, groups=2, scale=0.5), base)
    # A constant added to every mask entry of a row does not change softmax.
    torch.testing.assert_close(
        ref.decode_attention(q, kb, vb, lengths, mask + 3.5, groups=2, scale=0.5), base, rtol=1e-5, atol=1e-6
    )


def test_decode_attention_gqa_head_mapping():
    # Query head h reads KV head h // groups: zeroing KV head 1 must only
    # change query heads 2 and 3 (groups = 2).
    g = generator(4)
    q = torch.randn(1, 4, 1, 8, generator=g)
    kb = torch.randn(1, 5, 2, 8, generator=g)
    vb = torch.randn(1, 5, 2, 8, generator=g)
    lengths = torch.tensor([5])
    mask = torch.zeros(1, 1, 1, 5)
    base = ref.decode_attention(q, kb, vb, lengths, mask, groups=2, scale=0.5)
    vb2 = vb.clone()
    vb2[:, :, 1] = 0
    changed = ref.decode_attention(q, kb, vb2, lengths, mask, groups=2, scale=0.5)
    assert torch.equal(changed[:, :2], base[:, :2])
    assert torch.equal(changed[:, 2:], torch.zeros_like(changed[:, 2:]))


# -------------------------------------------------------------------- kv_store


def test_kv_store_reference_positions_case():
    # Reference KAT: positions [1, 5, 9], capacity 16 (test_triton_backend.py:436-466).
    g = generator(5)
    kb = np.zeros((3, 16, 2, 8), dtype=np.float32)
    vb = np.zeros_like(kb)
    k = torch.randn(3, 2, 1, 8, generator=g).numpy()
    v = torch.randn(3, 2, 1, 8, generator=g).numpy()
    ref.kv_store(kb, vb, k, v, np.array([1, 5, 9]))
    for b, pos in enumerate([1, 5, 9]):
        assert np.array_equal(kb[b, pos], k[b, :, 0])
        assert np.array_equal(vb[b, pos], v[b, :, 0])
    # every other row untouched
    assert np.count_nonzero(kb) == k.size


def test_kv_store_matches_index_copy_and_drops_overflow():
    # The reference's native_kv_store is an index_copy_ at b*cap + pos + t
    # (execution.py:743-781); rows past the capacity are dropped by its kernel.
    g = generator(6)
    B, H, T, D, cap = 2, 2, 4, 3, 8
    k = torch.randn(B, H, T, D, generator=g)
    v = torch.randn(B, H, T, D, generator=g)
    pos = torch.tensor([2, 6])
    kb = np.zeros((B, cap, H, D), dtype=np.float32)
    vb = np.zeros_like(kb)
    ref.kv_store(kb, vb, k.numpy(), v.numpy(), pos.numpy())
    want = torch.zeros(B * cap, H, D)
    idx = []
    src = []
    for b in range(B):
        for t in range(T):
            if pos[b] + t < cap:
                idx.append(b * cap + int(pos[b]) + t)
                src.append(k[b, :, t])
    want.index_copy_(0, torch.tensor(idx), torch.stack(src))
    assert np.array_equal(kb.reshape(B * cap, H, D), want.numpy())


# ------------------------------------------------------------------ paged KV


def _random_paging(g, batch, pages, extra=3):
    """A block table naming distinct pages of a pool with spare pages, in a
    random order."""

    order = torch.randperm(batch * pages + extra, generator=g)[: batch * pages]
    return order.view(batch, pages).numpy().astype(np.int32), batch * pages + extra


def test_gather_pages_identity_table_is_a_reshape():
    # A table that names pages in order makes the pool a reshaped contiguous
    # buffer: gathering must give that buffer back.
    g = generator(40)
    B, pages, P, H, D = 3, 4, 16, 2, 8
    buffer = torch.randn(B, pages * P, H, D, generator=g).numpy()
    pool = buffer.reshape(B * pages, P, H, D)
    table = np.arange(B * pages, dtype=np.int32).reshape(B, pages)
    assert np.array_equal(ref.gather_pages(pool, table), buffer)


def test_gather_pages_inverts_a_page_scatter():
    g = generator(41)
    B, pages, P, H, D = 2, 5, 16, 2, 4
    buffer = torch.randn(B, pages * P, H, D, generator=g).numpy()
    table, num_pages = _random_paging(g, B, pages)
    pool = np.full((num_pages, P, H, D), np.nan, dtype=np.float32)
    for b in range(B):
        for j in range(pages):
            pool[table[b, j]] = buffer[b, j * P:(j + 1) * P]
    assert np.array_equal(ref.gather_pages(pool, table), buffer)


def test_paged_kv_store_equals_contiguous_store_after_gather():
    # Storing into pages then gathering must equal storing into the gathered
    # buffer, including dropped rows past the table's capacity.
    g = generator(42)
    B, pages, P, H, T, D = 3, 3, 16, 2, 20, 4
    table, num_pages = _random_paging(g, B, pages)
    kp = torch.randn(num_pages, P, H, D, generator=g).numpy()
    vp = torch.randn(num_pages, P, H, D, generator=g).numpy()
    k = torch.randn(B, H, T, D, generator=g).numpy()
    v = torch.randn(B, H, T, D, generator=g).numpy()
    pos = np.array([0, 17, 40])  # the last runs 12 rows past capacity 48
    kb, vb = ref.gather_pages(kp, table), ref.gather_pages(vp, table)
    ref.kv_store(kb, vb, k, v, pos)
    ref.paged_kv_store(kp, vp, table, k, v, pos)
    assert np.array_equal(ref.gather_pages(kp, table), kb)
    assert np.array_equal(ref.gather_pages(vp, table), vb)


# -------------------------------------------------------------------- rms_norm


def test_rms_norm_matches_torch_rms_norm_fp32():
    g = generator(7)
    x = torch.randn(5, 896, generator=g)
    w = torch.randn(896, generator=g)
    torch.testing.assert_close(ref.rms_norm(x, w, epsilon=1e-6), F.rms_norm(x, (896,), w, 1e-6),
                               rtol=1e-6, atol=1e-6)


def test_rms_norm_round_before_weight_order():
    # Qwen2 order (model.py:44-51): normalised value rounded to bf16 first,
    # then a bf16 multiply -- differs from rounding once at the end.
    g = generator(8)
    x = torch.randn(64, 896, generator=g).bfloat16()
    w = (1 + 0.5 * torch.randn(896, generator=g)).bfloat16()
    got = ref.rms_norm(x, w, epsilon=1e-6, round_before_weight=True)
    x64 = x.double()
    n = (x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6)).float().bfloat16()
    want = (n.double() * w.double()).float().bfloat16()
    assert torch.equal(got, want)
    once = ref.rms_norm(x, w, epsilon=1e-6, round_before_weight=False)
    assert not torch.equal(got, once)


# ------------------------------------------------------------------------ rope


def test_rope_is_a_rotation_and_matches_complex_multiply():
    g = generator(9)
    B, H, T, D = 2, 3, 5, 8
    q = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, 1, T, D, generator=g, dtype=torch.float64)
    theta = torch.rand(B, T, D // 2, generator=g, dtype=torch.float64) * 6.0
    emb = torch.cat((theta, theta), dim=-1)
    rq, rk = ref.rope(q, k, emb.cos(), emb.sin())
    # Pair (x_i, x_{i+D/2}) rotated by theta_i == complex multiply by e^{i theta}.
    z = torch.complex(q[..., : D // 2], q[..., D // 2 :]) * torch.polar(torch.ones_like(theta), theta).unsqueeze(1)
    torch.testing.assert_close(rq, torch.cat((z.real, z.imag), dim=-1))
    torch.testing.assert_close(rq.norm(dim=-1), q.norm(dim=-1))
    torch.testing.assert_close(rk.norm(dim=-1), k.norm(dim=-1))


# --------------------------------------------------------- prefill attention


def test_prefill_attention_matches_sdpa_causal_and_bidirectional():
    g = generator(10)
    B, QH, KVH, T, D = 2, 4, 2, 7, 16
    q = torch.randn(B, QH, T, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, KVH, T, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, KVH, T, D, generator=g, dtype=torch.float64)
    ke, ve = k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)
    # The reference softmax runs in fp32 (scores.float()): fp32 tolerances.
    tol = dict(rtol=1e-5, atol=1e-6)
    causal = ref.prefill_attention(q, k, v, None, groups=2, scale=0.25, causal=True)
    torch.testing.assert_close(causal, F.scaled_dot_product_attention(q, ke, ve, is_causal=True, scale=0.25), **tol)
    future = torch.triu(torch.ones(T, T, dtype=torch.bool), diagonal=1)
    mask = torch.zeros(B, 1, T, T, dtype=torch.float64).masked_fill(future, float("-inf"))
    by_mask = ref.prefill_attention(q, k, v, mask, groups=2, scale=0.25, causal="mask")
    torch.testing.assert_close(by_mask, causal)
    zeros = ref.prefill_attention(q, k, v, torch.zeros(B, 1, T, T, dtype=torch.float64), groups=2, scale=0.25)
    torch.testing.assert_close(zeros, F.scaled_dot_product_attention(q, ke, ve, scale=0.25), **tol)


def test_linear_matches_float64_matmul():
    g = generator(11)
    x = torch.randn(3, 5, 12, generator=g, dtype=torch.float64)
    w = torch.randn(7, 12, generator=g, dtype=torch.float64)
    b = torch.randn(7, generator=g, dtype=torch.float64)
    want = torch.einsum("btk,nk->btn", x, w) + b
    torch.testing.assert_close(ref.linear(x, w, b), want)
