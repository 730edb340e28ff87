"""``kernel.hip.decode_attention``: GQA single-token attention on gfx950.

Drop-in for the reference's ``triton_decode_attention``
(src/stateful_llm_compiler/backends/triton_attention.py:134-210): same
arguments, same validation (``ValueError`` on device/shape/stride/dtype
problems), same result (a new tensor shaped like ``query``).  The math is the
reference executor's (execution.py:281-327).
"""

from __future__ import annotations

import torch

from .. import _native
from .hip_ops import check_flag

SPLIT_BALANCED = _native.SPLIT_BALANCED


def _workspace(lib, device: torch.device, nbytes: int, batch: int, kv_heads: int,
               workspace: _native.DeviceWorkspace | None) -> tuple[torch.Tensor | None, torch.Tensor, int]:
    """Split-sequence partials and arrival counters: the caller's workspace,
    else the current stream's."""

    owner = workspace if workspace is not None else _native.stream_workspace(device)
    count = int(lib.slc_hip_decode_attention_counter_count(batch, kv_heads))
    return owner.scratch("decode_attention", nbytes), owner.counters(count), count


def exact_max_tokens(head_dim: int, dtype: torch.dtype) -> int:
    """Longest mask the exact softmax order takes for this shape."""

    return int(_native.library().slc_hip_decode_attention_exact_max_tokens(
        head_dim, _native.dtype_tag(dtype)))


def _check_decode_operands(query, key_buffer, value_buffer, lengths, attention_mask):
    """The reference wrapper's operand checks (triton_attention.py:152-180);
    returns (batch, query_heads, head_dim, capacity, kv_heads)."""

    tensors = [query, key_buffer, value_buffer, lengths]
    if attention_mask is not None:
        tensors.append(attention_mask)
    if not all(tensor.is_cuda for tensor in tensors):
        raise ValueError("HIP decode attention: all tensors must be on the GPU")
    if (
        query.ndim != 4
        or query.shape[2] != 1
        or key_buffer.ndim != 4
        or key_buffer.shape != value_buffer.shape
        or (
            attention_mask is not None
            and (
                attention_mask.ndim != 4
                or attention_mask.shape[1] != 1
                or attention_mask.shape[2] != 1
            )
        )
    ):
        raise ValueError("HIP decode attention: illegal shapes")
    batch, query_heads, _, head_dim = query.shape
    capacity = key_buffer.shape[1]
    kv_heads = key_buffer.shape[2]
    if (
        batch != key_buffer.shape[0]
        or (attention_mask is not None and batch != attention_mask.shape[0])
        or lengths.shape != (batch,)
        or query_heads % kv_heads
        or head_dim != key_buffer.shape[3]
    ):
        raise ValueError("HIP decode attention: GQA or batch shapes do not match")
    if lengths.dtype not in (torch.int64, torch.int32):
        raise ValueError("HIP decode attention: lengths must be int64 (or int32)")
    if query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"HIP decode attention: unsupported dtype {query.dtype}")
    if key_buffer.dtype != query.dtype or value_buffer.dtype != query.dtype:
        raise ValueError("HIP decode attention: Q/K/V dtypes must match")
    if key_buffer.stride() != value_buffer.stride() or key_buffer.stride(3) != 1:
        raise ValueError(
            "HIP decode attention: K/V buffers need equal strides and a "
            "contiguous head dim"
        )
    if query.stride(-1) != 1:
        raise ValueError("HIP decode attention: query head dim must be contiguous")
    if attention_mask is not None and attention_mask.dtype not in (
        torch.float16,
        torch.bfloat16,
        torch.float32,
    ):
        raise ValueError("HIP decode attention: mask must be floating point")
    if head_dim > 256:
        raise ValueError("HIP decode attention: head_dim above 256")

    return batch, query_heads, head_dim, capacity, kv_heads


def _mask_args(attention_mask, capacity):
    if attention_mask is None:
        return None, 0, 0, 0, capacity
    return (attention_mask.data_ptr(), _native.dtype_tag(attention_mask.dtype),
            attention_mask.stride(0), attention_mask.stride(3), attention_mask.shape[-1])


def hip_decode_attention(
    query: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    lengths: torch.Tensor,
    attention_mask: torch.Tensor | None,
    *,
    scale: float,
    split_tokens: int = 0,
    softmax_order: str = "online",
    workspace: _native.DeviceWorkspace | None = None,
) -> torch.Tensor:
    """B x H x 1 x D GQA decode attention over a B x Cap x KVH x D buffer.

    ``key_buffer``/``value_buffer`` are indexed ``[b, s, h, :]``; the
    reference's contiguous_bshd buffers are the normal case, and any view with
    a contiguous head dim and equal K/V strides (for example a BHSD buffer
    permuted to BSHD) is accepted.  ``lengths`` is int64 (the runtime's
    dtype) or int32.  ``attention_mask`` is B x 1 x 1 x S additive, or None
    for an all-zero mask over the whole capacity.

    ``split_tokens``: 0 picks a fixed chunk per (batch, kv head) sized to fill
    the GPU, > 0 a fixed chunk of that many tokens, ``SPLIT_BALANCED`` (-1)
    the length-balanced split (pieces sized from the device-side lengths).
    ``softmax_order``: "online" (the reference Triton kernel's single-pass
    form, the default) or "exact" (normalise, round, then P.V -- the
    reference executor's order; masks up to ``exact_max_tokens`` long).
    ``workspace``: the caller's ``DeviceWorkspace`` (else the current
    stream's); calls that may run concurrently need separate ones.
    """

    order = _native.softmax_order_tag(softmax_order)
    batch, query_heads, head_dim, capacity, kv_heads = _check_decode_operands(
        query, key_buffer, value_buffer, lengths, attention_mask)

    lib = _native.library()
    output = torch.empty_like(query)
    if batch == 0:
        return output
    dtype = _native.dtype_tag(query.dtype)
    mask_ptr, mask_dtype, mask_sb, mask_ss, mask_len = _mask_args(attention_mask, capacity)
    nbytes = lib.slc_hip_decode_attention_workspace_size(
        batch, query_heads, head_dim, mask_len, kv_heads, dtype, split_tokens
    )
    stream = _native.current_stream(query.device)
    buffer, counters, count = _workspace(lib, query.device, nbytes, batch, kv_heads, workspace)
    status = lib.slc_hip_decode_attention(
        query.data_ptr(),
        key_buffer.data_ptr(),
        value_buffer.data_ptr(),
        lengths.data_ptr(),
        _native.dtype_tag(lengths.dtype),
        mask_ptr,
        mask_dtype,
        output.data_ptr(),
        None if buffer is None else buffer.data_ptr(),
        nbytes,
        counters.data_ptr(),
        count,
        dtype,
        batch,
        query_heads,
        kv_heads,
        head_dim,
        capacity,
        mask_len,
        query.stride(0),
        query.stride(1),
        key_buffer.stride(0),
        key_buffer.stride(1),
        key_buffer.stride(2),
        mask_sb,
        mask_ss,
        output.stride(0),
        output.stride(1),
        float(scale),
        int(split_tokens),
        order,
        stream,
    )
    _native.check(status, "slc_hip_decode_attention")
    return output


def hip_decode_attention_noalloc(
    query: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    lengths: torch.Tensor,
    attention_mask: torch.Tensor | None,
    output: torch.Tensor,
    *,
    scale: float,
    split_tokens: int = 0,
    softmax_order: str = "online",
) -> torch.Tensor:
    """``hip_decode_attention`` into the caller's ``output`` through the entry
    point that allocates nothing (``slc_hip_decode_attention_noalloc``): its
    split partials and counters live in the library's own device array, so
    the call makes no device allocation at all.  Every call on one GPU shares
    that array: calls that may overlap in time -- on two streams, or two
    graphs replayed concurrently -- race, so issue them from one stream per
    GPU.  Nothing checks this at run time."""

    order = _native.softmax_order_tag(softmax_order)
    batch, query_heads, head_dim, capacity, kv_heads = _check_decode_operands(
        query, key_buffer, value_buffer, lengths, attention_mask)
    if not output.is_cuda or output.shape != query.shape or output.dtype != query.dtype:
        raise ValueError("HIP decode attention: output must be a GPU tensor shaped like the query")
    if output.stride(-1) != 1:
        raise ValueError("HIP decode attention: output head dim must be contiguous")
    lib = _native.library()
    mask_ptr, mask_dtype, mask_sb, mask_ss, mask_len = _mask_args(attention_mask, capacity)
    status = lib.slc_hip_decode_attention_noalloc(
        query.data_ptr(), key_buffer.data_ptr(), value_buffer.data_ptr(), lengths.data_ptr(),
        _native.dtype_tag(lengths.dtype), mask_ptr, mask_dtype, output.data_ptr(),
        _native.dtype_tag(query.dtype), batch, query_heads, kv_heads, head_dim, capacity,
        mask_len, query.stride(0), query.stride(1), key_buffer.stride(0), key_buffer.stride(1),
        key_buffer.stride(2), mask_sb, mask_ss, output.stride(0), output.stride(1),
        float(scale), int(split_tokens), order, _native.current_stream(query.device),
    )
    _native.check(status, "slc_hip_decode_attention_noalloc")
    return output


def hip_rope_decode_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cosine: torch.Tensor,
    sine: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    lengths: torch.Tensor,
    lengths_out: torch.Tensor,
    attention_mask: torch.Tensor | None,
    *,
    scale: float,
    overflow: torch.Tensor | None = None,
    softmax_order: str = "online",
    workspace: _native.DeviceWorkspace | None = None,
) -> torch.Tensor | None:
    """One decode token's RoPE, KV store at ``lengths``, length advance by one
    (into ``lengths_out``, which may be ``lengths``) and GQA attention, in one
    kernel; bit-identical to ``hip_rope_kv_store(..., advance=1)`` followed by
    ``hip_decode_attention`` of the rotated query over the advanced lengths.

    query [B, QH, 1, D] and key/value [B, KVH, 1, D] unrotated projections,
    cosine/sine [B, 1, D].  Returns None, having done nothing, when the fused
    kernel does not take the case (the caller then runs the two ops).
    ``softmax_order`` and ``workspace`` as in ``hip_decode_attention``.
    """

    order = _native.softmax_order_tag(softmax_order)

    tensors = [query, key, value, cosine, sine, key_buffer, value_buffer, lengths, lengths_out]
    if attention_mask is not None:
        tensors.append(attention_mask)
    check_flag(overflow, "HIP rope decode attention")
    if not all(tensor.is_cuda for tensor in tensors):
        return None
    if (
        query.ndim != 4 or key.ndim != 4 or value.ndim != 4 or query.shape[2] != 1
        or key.shape != value.shape or key.shape[2] != 1 or key_buffer.ndim != 4
        or key_buffer.shape != value_buffer.shape or key_buffer.stride() != value_buffer.stride()
        or cosine.ndim != 3 or cosine.shape != sine.shape or cosine.shape[1] != 1
    ):
        return None
    batch, query_heads, _, head_dim = query.shape
    kv_heads = key.shape[1]
    capacity = key_buffer.shape[1]
    if (
        key.shape[0] != batch or key_buffer.shape[0] != batch or key_buffer.shape[2] != kv_heads
        or key_buffer.shape[3] != head_dim or key.shape[3] != head_dim
        or cosine.shape != (batch, 1, head_dim) or query_heads % kv_heads
        or lengths.shape != (batch,) or lengths_out.shape != (batch,)
        or lengths.dtype != torch.int64 or lengths_out.dtype != torch.int64
        or any(t.dtype != query.dtype for t in (key, value, cosine, sine, key_buffer, value_buffer))
        or any(t.stride(-1) != 1 for t in (query, key, value, cosine, sine, key_buffer))
    ):
        return None
    if attention_mask is not None and (
        attention_mask.ndim != 4 or attention_mask.shape[:3] != (batch, 1, 1)
        or attention_mask.dtype not in (torch.float16, torch.bfloat16, torch.float32)
    ):
        return None
    lib = _native.library()
    output = torch.empty_like(query)
    if batch == 0:
        return output
    dtype = _native.dtype_tag(query.dtype)
    mask_len = capacity if attention_mask is None else attention_mask.shape[-1]
    if mask_len > capacity:
        return None
    nbytes = lib.slc_hip_decode_attention_workspace_size(
        batch, query_heads, head_dim, mask_len, kv_heads, dtype, 0
    )
    buffer, counters, count = _workspace(lib, query.device, nbytes, batch, kv_heads, workspace)
    if attention_mask is None:
        mask_ptr, mask_dtype, mask_sb, mask_ss = None, 0, 0, 0
    else:
        mask_ptr = attention_mask.data_ptr()
        mask_dtype = _native.dtype_tag(attention_mask.dtype)
        mask_sb, mask_ss = attention_mask.stride(0), attention_mask.stride(3)
    status = lib.slc_hip_rope_decode_attention(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), cosine.data_ptr(), sine.data_ptr(),
        key_buffer.data_ptr(), value_buffer.data_ptr(), lengths.data_ptr(),
        lengths_out.data_ptr(), None if overflow is None else overflow.data_ptr(),
        mask_ptr, mask_dtype, output.data_ptr(),
        None if buffer is None else buffer.data_ptr(), nbytes, counters.data_ptr(), count, dtype,
        batch, query_heads, kv_heads, head_dim, capacity, mask_len,
        query.stride(0), query.stride(1), key.stride(0), key.stride(1),
        value.stride(0), value.stride(1), cosine.stride(0), sine.stride(0),
        key_buffer.stride(0), key_buffer.stride(1), key_buffer.stride(2),
        mask_sb, mask_ss, output.stride(0), output.stride(1), float(scale), order,
        _native.current_stream(query.device),
    )
    if status == _UNSUPPORTED:
        return None
    _native.check(status, "slc_hip_rope_decode_attention")
    return output


_UNSUPPORTED = -2  # SLC_ERR_UNSUPPORTED
