"""``kernel.hip.kv_store``: positional K/V row scatter into the KV buffers.

Drop-in for the reference's ``triton_kv_store``
(src/stateful_llm_compiler/backends/triton_kv.py:71-129) with the semantics of
``native_kv_store`` (execution.py:743-781).  Bit-exact copy.
"""

from __future__ import annotations

import torch

from .. import _native
from .hip_ops import check_flag


def hip_kv_store(
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    *,
    overflow: torch.Tensor | None = None,
) -> None:
    """Write B x H x T x D ``key``/``value`` rows into B x Cap x H x D buffers.

    Row ``t`` of batch ``b`` lands at buffer row ``positions[b] + t``; rows at
    or beyond the capacity are skipped, as in the reference kernel, and set
    the optional int32 ``overflow`` flag tensor.
    """

    if not all(
        tensor.is_cuda
        for tensor in (key_buffer, value_buffer, key, value, positions)
    ):
        raise ValueError("HIP KV store: all tensors must be on the GPU")
    check_flag(overflow, "HIP KV store")
    if (
        key_buffer.shape != value_buffer.shape
        or key.shape != value.shape
        or key.ndim != 4
        or key_buffer.ndim != 4
    ):
        raise ValueError("HIP KV store: illegal shapes")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("HIP KV store: K/V head dim must be contiguous")
    if not key_buffer.is_contiguous() or not value_buffer.is_contiguous():
        raise ValueError("HIP KV store: buffers must be contiguous")
    batch, heads, tokens, head_dim = key.shape
    if (
        batch != key_buffer.shape[0]
        or heads != key_buffer.shape[2]
        or head_dim != key_buffer.shape[3]
    ):
        raise ValueError("HIP KV store: buffers and current K/V do not match")
    if positions.shape != (batch,) or positions.dtype != torch.int64:
        raise ValueError("HIP KV store: positions must be a [batch] int64 tensor")
    if not (
        key.dtype == value.dtype == key_buffer.dtype == value_buffer.dtype
    ):
        raise ValueError("HIP KV store: dtypes must match")
    positions = positions.contiguous()
    status = _native.library().slc_hip_kv_store(
        key_buffer.data_ptr(),
        value_buffer.data_ptr(),
        key.data_ptr(),
        value.data_ptr(),
        positions.data_ptr(),
        None if overflow is None else overflow.data_ptr(),
        _native.dtype_tag(key.dtype),
        batch,
        heads,
        tokens,
        head_dim,
        key_buffer.shape[1],
        key.stride(0),
        key.stride(1),
        key.stride(2),
        value.stride(0),
        value.stride(1),
        value.stride(2),
        _native.current_stream(key.device),
    )
    _native.check(status, "slc_hip_kv_store")
