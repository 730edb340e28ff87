"""``kernel.hip.prefill_attention``: multi-token causal GQA attention.

Drop-in for the reference's ``triton_prefill_attention``
(src/stateful_llm_compiler/backends/triton_prefill_attention.py:152-232) with
the semantics of the reference executor's ``_serve_prefill_attention``
(execution.py:707-739): ``causal=True`` removes future keys in the kernel
(tiles wholly in the future are skipped), and the additive mask, when given,
is applied to every computed score.  A mask is first classified per 64 x 64
tile (``hip_prefill_mask_tiles``): tiles that are -inf throughout are not
visited at all (no K/V or mask loads), tiles that equal the causal pattern
are applied from the indices without loading the mask, and only the rest load
their mask tile.  Results are those of adding the whole mask.
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
    mask_tiles: torch.Tensor | None = None,
) -> torch.Tensor:
    """B x QH x T x D attention over B x KVH x T x D keys/values.

    ``softmax_order``: "online" (single pass, the reference Triton kernel's
    form) or "exact" (two passes: the row max and sum first, then the
    normalised probabilities rounded to the I/O dtype weigh V -- the
    reference executor's order, execution.py:720-739).

    ``mask_tiles``: the mask's tile classes from ``hip_prefill_mask_tiles``
    (a caller that applies one mask in many calls -- every layer of a model
    -- classifies it once); computed here when a mask comes without them."""

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
    classes = None
    if attention_mask is None:
        mask_ptr, mask_dtype, ms = None, 0, (0, 0, 0)
    else:
        mask_ptr = attention_mask.data_ptr()
        mask_dtype = _native.dtype_tag(attention_mask.dtype)
        ms = (attention_mask.stride(0), attention_mask.stride(2), attention_mask.stride(3))
        classes = hip_prefill_mask_tiles(attention_mask) if mask_tiles is None else mask_tiles
        tiles = -(-tokens // 64)
        if (classes.dtype != torch.uint8 or classes.device != query.device
                or classes.shape != (batch, tiles, tiles) or not classes.is_contiguous()):
            raise ValueError("HIP prefill attention: mask_tiles must be the mask's uint8 [B, T/64, T/64] classes")
    status = lib.slc_hip_prefill_attention_classes(
        query.data_ptr(),
        key.data_ptr(),
        value.data_ptr(),
        mask_ptr,
        mask_dtype,
        None if classes is None else classes.data_ptr(),
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
    _native.check(status, "slc_hip_prefill_attention_classes")
    return output


def hip_prefill_mask_tiles(attention_mask: torch.Tensor) -> torch.Tensor:
    """Classes of an additive [B, 1, T, T] mask per (batch, 64-query block,
    64-key tile), uint8 [B, ceil(T/64), ceil(T/64)]: 0 = -inf throughout,
    1 = the causal pattern (+0 where key <= query, -inf above), 2 = other."""

    if not attention_mask.is_cuda or attention_mask.ndim != 4 or attention_mask.shape[1] != 1:
        raise ValueError("HIP prefill mask tiles: a [B, 1, T, T] GPU mask is required")
    batch, _, tokens, keys = attention_mask.shape
    if keys != tokens or attention_mask.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("HIP prefill mask tiles: square floating-point mask required")
    tiles = -(-tokens // 64)
    classes = torch.empty(batch, tiles, tiles, dtype=torch.uint8, device=attention_mask.device)
    status = _native.library().slc_hip_prefill_mask_tiles(
        attention_mask.data_ptr(), _native.dtype_tag(attention_mask.dtype), batch, tokens,
        attention_mask.stride(0), attention_mask.stride(2), attention_mask.stride(3),
        classes.data_ptr(), _native.current_stream(attention_mask.device))
    _native.check(status, "slc_hip_prefill_mask_tiles")
    return classes
