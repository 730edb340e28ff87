"""``kernel.hip.prefill_attention``: multi-token causal GQA attention.

Drop-in for the reference's ``triton_prefill_attention``
(src/stateful_llm_compiler/backends/triton_prefill_attention.py:152-232) with
the semantics of the reference executor's ``_serve_prefill_attention``
(execution.py:707-739): ``causal=True`` removes future keys in the kernel
(tiles wholly in the future are skipped), and the additive mask, when given,
is applied to every computed score.
"""

from __future__ import annotations

import torch

from .. import _native


def hip_prefill_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor | None,
    *,
    scale: float,
    causal: bool = False,
    softmax_order: str = "online",
) -> torch.Tensor:
    """B x QH x T x D attention over B x KVH x T x D keys/values.

    ``softmax_order``: "online" (single pass, the reference Triton kernel's
    form) or "exact" (two passes: the row max and sum first, then the
    normalised probabilities rounded to the I/O dtype weigh V -- the
    reference executor's order, execution.py:720-739)."""

    order = _native.softmax_order_tag(softmax_order)
    tensors = [query, key, value] + ([attention_mask] if attention_mask is not None else [])
    if not all(tensor.is_cuda for tensor in tensors):
        raise ValueError("HIP prefill attention: all tensors must be on the GPU")
    if (
        query.ndim != 4
        or key.ndim != 4
        or key.shape != value.shape
        or (attention_mask is not None and (attention_mask.ndim != 4 or attention_mask.shape[1] != 1))
    ):
        raise ValueError("HIP prefill attention: illegal shapes")
    batch, query_heads, tokens, head_dim = query.shape
    kv_batch, kv_heads, kv_tokens, kv_head_dim = key.shape
    if (
        batch != kv_batch
        or tokens != kv_tokens
        or head_dim != kv_head_dim
        or query_heads % kv_heads
        or (attention_mask is not None and attention_mask.shape != (batch, 1, tokens, tokens))
    ):
        raise ValueError("HIP prefill attention: GQA or token shapes do not match")
    if query.dtype != key.dtype or key.dtype != value.dtype:
        raise ValueError("HIP prefill attention: Q/K/V dtypes must match")
    if query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"HIP prefill attention: unsupported dtype {query.dtype}")
    if query.stride(-1) != 1 or key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("HIP prefill attention: head dims must be contiguous")
    if scale <= 0:
        raise ValueError("HIP prefill attention: scale must be positive")
    if head_dim > 256:
        raise ValueError("HIP prefill attention: head_dim above 256")
    if attention_mask is not None and attention_mask.dtype not in (
        torch.float16, torch.bfloat16, torch.float32
    ):
        raise ValueError("HIP prefill attention: mask must be floating point")

    lib = _native.library()
    output = torch.empty_like(query)
    if attention_mask is None:
        mask_ptr, mask_dtype, ms = None, 0, (0, 0, 0)
    else:
        mask_ptr = attention_mask.data_ptr()
        mask_dtype = _native.dtype_tag(attention_mask.dtype)
        ms = (attention_mask.stride(0), attention_mask.stride(2), attention_mask.stride(3))
    status = lib.slc_hip_prefill_attention(
        query.data_ptr(),
        key.data_ptr(),
        value.data_ptr(),
        mask_ptr,
        mask_dtype,
        output.data_ptr(),
        _native.dtype_tag(query.dtype),
        batch,
        query_heads,
        kv_heads,
        tokens,
        head_dim,
        1 if causal else 0,
        *query.stride()[:3],
        *key.stride()[:3],
        *value.stride()[:3],
        *ms,
        *output.stride()[:3],
        float(scale),
        order,
        _native.current_stream(query.device),
    )
    _native.check(status, "slc_hip_prefill_attention")
    return output
