"""Paged KV: decode attention and KV store through a block table.

The reference keeps one contiguous [B, Cap, H, D] buffer per layer and names a
paged layout with a block table as the next step
(docs/kv-bufferization.md:317-323; ``KVStateType.layout``, ir.py:87).  Here a
layer's K and V rows live in page pools ``[num_pages, page_tokens, H, D]``
and an int32 ``block_table[b, j]`` names the pool page that holds tokens
``[j * page_tokens, (j + 1) * page_tokens)`` of sequence ``b``.  Both ops
take the same arguments as their contiguous counterparts
(``hip_decode_attention``, ``hip_kv_store``) plus the pools and the table,
and give the same result bit for bit as the contiguous op over the gathered
tokens.
"""

from __future__ import annotations

import torch

from .. import _native
from .hip_attention import _mask_args, _workspace
from .hip_ops import check_flag


def _check_pools(key_pool: torch.Tensor, value_pool: torch.Tensor, block_table: torch.Tensor,
                 batch: int, what: str) -> tuple[int, int]:
    """(pages_per_seq, page_tokens) after the pool and table checks."""

    if key_pool.ndim != 4 or key_pool.shape != value_pool.shape:
        raise ValueError(f"{what}: pools must be equal-shaped [pages, page_tokens, H, D] tensors")
    if key_pool.stride() != value_pool.stride() or key_pool.stride(3) != 1:
        raise ValueError(f"{what}: pools need equal strides and a contiguous head dim")
    if key_pool.dtype != value_pool.dtype:
        raise ValueError(f"{what}: K/V pool dtypes must match")
    page_tokens = key_pool.shape[1]
    if page_tokens < 16 or page_tokens & (page_tokens - 1):
        raise ValueError(f"{what}: page_tokens must be a power of two >= 16, got {page_tokens}")
    if key_pool.stride(1) * page_tokens > key_pool.stride(0) and key_pool.shape[0] > 1:
        raise ValueError(f"{what}: pool pages overlap")
    if (block_table.ndim != 2 or block_table.shape[0] != batch
            or block_table.dtype != torch.int32 or block_table.stride(1) != 1):
        raise ValueError(f"{what}: block_table must be an int32 [batch, pages] tensor with unit row stride")
    if not block_table.is_cuda or not key_pool.is_cuda or not value_pool.is_cuda:
        raise ValueError(f"{what}: pools and block table must be on the GPU")
    return block_table.shape[1], page_tokens


def hip_paged_decode_attention(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_table: torch.Tensor,
    lengths: torch.Tensor,
    attention_mask: torch.Tensor | None,
    *,
    scale: float,
    split_tokens: int = 0,
    softmax_order: str = "online",
    workspace: _native.DeviceWorkspace | None = None,
) -> torch.Tensor:
    """``hip_decode_attention`` over paged K/V.

    ``query`` is B x QH x 1 x D (bf16 or fp16, D 64 or 128, at most 16 query
    heads per kv head); ``lengths`` int64 or int32 [B]; ``attention_mask``
    B x 1 x 1 x S additive (S at most pages_per_seq * page_tokens) or None for
    an all-zero mask over the table's capacity.  The block table entries a
    sequence's live tokens reach must name pages of the pool; the library does
    not bound-check them (as a CUDA paged kernel does not).
    """

    what = "HIP paged decode attention"
    order = _native.softmax_order_tag(softmax_order)
    if not (query.is_cuda and lengths.is_cuda and (attention_mask is None or attention_mask.is_cuda)):
        raise ValueError(f"{what}: all tensors must be on the GPU")
    if query.ndim != 4 or query.shape[2] != 1 or query.stride(-1) != 1:
        raise ValueError(f"{what}: query must be B x H x 1 x D with a contiguous head dim")
    batch, query_heads, _, head_dim = query.shape
    pages_per_seq, page_tokens = _check_pools(key_pool, value_pool, block_table, batch, what)
    kv_heads = key_pool.shape[2]
    if key_pool.shape[3] != head_dim or query_heads % kv_heads:
        raise ValueError(f"{what}: GQA or head shapes do not match")
    if query.dtype not in (torch.float16, torch.bfloat16) or key_pool.dtype != query.dtype:
        raise ValueError(f"{what}: Q/K/V must share one dtype, bf16 or fp16")
    if lengths.shape != (batch,) or lengths.dtype not in (torch.int64, torch.int32):
        raise ValueError(f"{what}: lengths must be an int64 (or int32) [batch] tensor")
    if attention_mask is not None and (
        attention_mask.ndim != 4 or attention_mask.shape[:3] != (batch, 1, 1)
        or attention_mask.dtype not in (torch.float16, torch.bfloat16, torch.float32)
    ):
        raise ValueError(f"{what}: mask must be a floating B x 1 x 1 x S tensor")
    capacity = pages_per_seq * page_tokens
    output = torch.empty_like(query)
    if batch == 0:
        return output
    lib = _native.library()
    dtype = _native.dtype_tag(query.dtype)
    mask_ptr, mask_dtype, mask_sb, mask_ss, mask_len = _mask_args(attention_mask, capacity)
    if mask_len > capacity:
        raise ValueError(f"{what}: mask is longer than the block table's capacity")
    nbytes = lib.slc_hip_decode_attention_workspace_size(
        batch, query_heads, head_dim, mask_len, kv_heads, dtype, split_tokens)
    buffer, counters, count = _workspace(lib, query.device, nbytes, batch, kv_heads, workspace)
    status = lib.slc_hip_paged_decode_attention(
        query.data_ptr(), key_pool.data_ptr(), value_pool.data_ptr(), block_table.data_ptr(),
        block_table.stride(0), pages_per_seq, page_tokens, key_pool.stride(0),
        lengths.data_ptr(), _native.dtype_tag(lengths.dtype), mask_ptr, mask_dtype,
        output.data_ptr(), None if buffer is None else buffer.data_ptr(), nbytes,
        counters.data_ptr(), count, dtype, batch, query_heads, kv_heads, head_dim, mask_len,
        query.stride(0), query.stride(1), key_pool.stride(1), key_pool.stride(2),
        mask_sb, mask_ss, output.stride(0), output.stride(1), float(scale), int(split_tokens),
        order, _native.current_stream(query.device),
    )
    _native.check(status, "slc_hip_paged_decode_attention")
    return output


def hip_paged_kv_store(
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_table: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    *,
    overflow: torch.Tensor | None = None,
) -> None:
    """``hip_kv_store`` into paged pools: row ``t`` of batch ``b`` lands at
    position ``positions[b] + t`` of sequence ``b``; positions at or beyond
    the table's capacity are skipped and set the optional ``overflow`` flag."""

    what = "HIP paged KV store"
    if not all(t.is_cuda for t in (key, value, positions)):
        raise ValueError(f"{what}: all tensors must be on the GPU")
    check_flag(overflow, what)
    if key.ndim != 4 or key.shape != value.shape or key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError(f"{what}: K/V must be equal B x H x T x D tensors with a contiguous head dim")
    batch, heads, tokens, head_dim = key.shape
    pages_per_seq, page_tokens = _check_pools(key_pool, value_pool, block_table, batch, what)
    if key_pool.shape[2] != heads or key_pool.shape[3] != head_dim:
        raise ValueError(f"{what}: pools and current K/V do not match")
    if not (key.dtype == value.dtype == key_pool.dtype):
        raise ValueError(f"{what}: dtypes must match")
    if positions.shape != (batch,) or positions.dtype != torch.int64:
        raise ValueError(f"{what}: positions must be a [batch] int64 tensor")
    if batch == 0 or tokens == 0:
        return
    positions = positions.contiguous()
    status = _native.library().slc_hip_paged_kv_store(
        key_pool.data_ptr(), value_pool.data_ptr(), block_table.data_ptr(), block_table.stride(0),
        pages_per_seq, page_tokens, key_pool.stride(0), key_pool.stride(1), key_pool.stride(2),
        key.data_ptr(), value.data_ptr(), positions.data_ptr(),
        None if overflow is None else overflow.data_ptr(), _native.dtype_tag(key.dtype),
        batch, heads, tokens, head_dim, key.stride(0), key.stride(1), key.stride(2),
        value.stride(0), value.stride(1), value.stride(2), _native.current_stream(key.device),
    )
    _native.check(status, "slc_hip_paged_kv_store")


_UNSUPPORTED = -2  # SLC_ERR_UNSUPPORTED


def hip_paged_rope_decode_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cosine: torch.Tensor,
    sine: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_table: torch.Tensor,
    lengths: torch.Tensor,
    lengths_out: torch.Tensor,
    attention_mask: torch.Tensor | None,
    *,
    scale: float,
    overflow: torch.Tensor | None = None,
    softmax_order: str = "online",
    workspace: _native.DeviceWorkspace | None = None,
) -> torch.Tensor | None:
    """``hip_rope_decode_attention`` over paged K/V: RoPE, the new row written
    at ``lengths[b]`` of sequence b (its page from ``block_table``), the
    length advance into ``lengths_out`` and the attention, in one kernel; bit
    for bit RoPE, ``hip_paged_kv_store`` and ``hip_paged_decode_attention``
    run in turn.  Returns None, having done nothing, when the fused kernel does
    not take the case (the caller then runs the three ops)."""

    what = "HIP paged rope decode attention"
    order = _native.softmax_order_tag(softmax_order)
    check_flag(overflow, what)
    tensors = [query, key, value, cosine, sine, key_pool, value_pool, block_table, lengths, lengths_out]
    if attention_mask is not None:
        tensors.append(attention_mask)
    if not all(t.is_cuda for t in tensors):
        return None
    if (query.ndim != 4 or query.shape[2] != 1 or key.ndim != 4 or key.shape != value.shape
            or key.shape[2] != 1 or cosine.ndim != 3 or cosine.shape != sine.shape):
        return None
    batch, query_heads, _, head_dim = query.shape
    try:
        pages_per_seq, page_tokens = _check_pools(key_pool, value_pool, block_table, batch, what)
    except ValueError:
        return None
    kv_heads = key.shape[1]
    if (key.shape[0] != batch or key_pool.shape[2] != kv_heads or key_pool.shape[3] != head_dim
            or key.shape[3] != head_dim or cosine.shape != (batch, 1, head_dim)
            or query_heads % kv_heads or lengths.shape != (batch,) or lengths_out.shape != (batch,)
            or lengths.dtype != torch.int64 or lengths_out.dtype != torch.int64
            or any(t.dtype != query.dtype for t in (key, value, cosine, sine, key_pool))
            or any(t.stride(-1) != 1 for t in (query, key, value, cosine, sine))):
        return None
    if attention_mask is not None and (
        attention_mask.ndim != 4 or attention_mask.shape[:3] != (batch, 1, 1)
        or attention_mask.dtype not in (torch.float16, torch.bfloat16, torch.float32)
    ):
        return None
    capacity = pages_per_seq * page_tokens
    output = torch.empty_like(query)
    if batch == 0:
        return output
    lib = _native.library()
    dtype = _native.dtype_tag(query.dtype)
    mask_ptr, mask_dtype, mask_sb, mask_ss, mask_len = _mask_args(attention_mask, capacity)
    if mask_len > capacity:
        return None
    nbytes = lib.slc_hip_decode_attention_workspace_size(
        batch, query_heads, head_dim, mask_len, kv_heads, dtype, 0)
    buffer, counters, count = _workspace(lib, query.device, nbytes, batch, kv_heads, workspace)
    status = lib.slc_hip_paged_rope_decode_attention(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), cosine.data_ptr(), sine.data_ptr(),
        key_pool.data_ptr(), value_pool.data_ptr(), block_table.data_ptr(), block_table.stride(0),
        pages_per_seq, page_tokens, key_pool.stride(0), lengths.data_ptr(), lengths_out.data_ptr(),
        None if overflow is None else overflow.data_ptr(), mask_ptr, mask_dtype, output.data_ptr(),
        None if buffer is None else buffer.data_ptr(), nbytes, counters.data_ptr(), count, dtype,
        batch, query_heads, kv_heads, head_dim, mask_len,
        query.stride(0), query.stride(1), key.stride(0), key.stride(1), value.stride(0),
        value.stride(1), cosine.stride(0), sine.stride(0), key_pool.stride(1), key_pool.stride(2),
        mask_sb, mask_ss, output.stride(0), output.stride(1), float(scale), order,
        _native.current_stream(query.device),
    )
    if status == _UNSUPPORTED:
        return None
    _native.check(status, "slc_hip_paged_rope_decode_attention")
    return output
