"""Wrappers of the small device ops that complete a compiled Qwen2 step.

The reference runs these as eager PyTorch ops through its reference executor
(src/stateful_llm_compiler/execution.py:500-528); here each is one HIP launch
so a fully lowered step contains no PyTorch compute kernel.
"""

from __future__ import annotations

import torch

from .. import _native

_FLOATS = (torch.float16, torch.bfloat16, torch.float32)


def check_flag(flag: torch.Tensor | None, what: str) -> None:
    """An optional device flag: an int32 GPU tensor of at least one element."""

    if flag is not None and (not flag.is_cuda or flag.dtype != torch.int32 or flag.numel() < 1):
        raise ValueError(f"{what}: the overflow flag must be an int32 GPU tensor")


def _require_gpu(*tensors: torch.Tensor, what: str) -> None:
    if not all(t.is_cuda for t in tensors):
        raise ValueError(f"{what}: all tensors must be on the GPU")


def hip_embedding(
    input_ids: torch.Tensor,
    table: torch.Tensor,
    *,
    bad_index: torch.Tensor | None = None,
) -> torch.Tensor:
    """Row gather ``table[input_ids]`` (qwen2.py:427-430 embed_tokens)."""

    _require_gpu(input_ids, table, what="HIP embedding")
    if input_ids.dtype != torch.int64 or table.ndim != 2 or table.dtype not in _FLOATS:
        raise ValueError("HIP embedding: int64 ids and a 2-D float table are required")
    if not table.is_contiguous():
        raise ValueError("HIP embedding: table must be contiguous")
    ids = input_ids.contiguous()
    out = torch.empty((*ids.shape, table.shape[1]), device=table.device, dtype=table.dtype)
    status = _native.library().slc_hip_embedding(
        ids.data_ptr(), table.data_ptr(), out.data_ptr(), _native.dtype_tag(table.dtype),
        ids.numel(), table.shape[1], table.shape[0],
        None if bad_index is None else bad_index.data_ptr(),
        _native.current_stream(table.device),
    )
    _native.check(status, "slc_hip_embedding")
    return out


def _binary(a: torch.Tensor, b: torch.Tensor, fn: str, what: str) -> torch.Tensor:
    _require_gpu(a, b, what=what)
    if a.shape != b.shape or a.dtype != b.dtype or a.dtype not in _FLOATS:
        raise ValueError(f"{what}: operands need one shape and a float dtype")
    a = a.contiguous()
    b = b.contiguous()
    out = torch.empty_like(a)
    status = getattr(_native.library(), fn)(
        a.data_ptr(), b.data_ptr(), out.data_ptr(), _native.dtype_tag(a.dtype), a.numel(),
        _native.current_stream(a.device),
    )
    _native.check(status, fn)
    return out


def hip_add(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Elementwise ``a + b`` rounded once to the dtype (residual adds)."""

    return _binary(a, b, "slc_hip_add", "HIP add")


def hip_swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` with silu materialised in the dtype (qwen2.py:253-256)."""

    return _binary(gate, up, "slc_hip_swiglu", "HIP swiglu")


def hip_rope_table(
    position_ids: torch.Tensor, inv_freq: torch.Tensor, dtype: torch.dtype
) -> tuple[torch.Tensor, torch.Tensor]:
    """B x T x D cos/sin tables of ``cat(f, f)``, ``f = pos * inv_freq`` (fp32 math)."""

    _require_gpu(position_ids, inv_freq, what="HIP rope table")
    if position_ids.dtype != torch.int64 or position_ids.ndim != 2:
        raise ValueError("HIP rope table: position_ids must be a B x T int64 tensor")
    if inv_freq.dtype != torch.float32 or inv_freq.ndim != 1:
        raise ValueError("HIP rope table: inv_freq must be a 1-D fp32 tensor")
    if position_ids.stride(1) != 1 and position_ids.shape[1] > 1:
        position_ids = position_ids.contiguous()
    batch, tokens = position_ids.shape
    head_dim = 2 * inv_freq.shape[0]
    cos = torch.empty(batch, tokens, head_dim, device=inv_freq.device, dtype=dtype)
    sin = torch.empty_like(cos)
    status = _native.library().slc_hip_rope_table(
        position_ids.data_ptr(), inv_freq.contiguous().data_ptr(), cos.data_ptr(), sin.data_ptr(),
        _native.dtype_tag(dtype), batch, tokens, position_ids.stride(0), head_dim,
        _native.current_stream(inv_freq.device),
    )
    _native.check(status, "slc_hip_rope_table")
    return cos, sin


def hip_kv_advance(
    lengths: torch.Tensor,
    delta: int,
    capacity: int,
    *,
    out: torch.Tensor | None = None,
    overflow: torch.Tensor | None = None,
) -> torch.Tensor:
    """``lengths + delta`` on the device; flags lengths past ``capacity``."""

    _require_gpu(lengths, what="HIP kv advance")
    if lengths.dtype != torch.int64 or lengths.ndim != 1 or not lengths.is_contiguous():
        raise ValueError("HIP kv advance: lengths must be a contiguous 1-D int64 tensor")
    if out is not None and (not out.is_cuda or out.dtype != torch.int64
                            or out.shape != lengths.shape or not out.is_contiguous()):
        raise ValueError("HIP kv advance: out must be a contiguous int64 GPU tensor like lengths")
    check_flag(overflow, "HIP kv advance")
    result = torch.empty_like(lengths) if out is None else out
    status = _native.library().slc_hip_kv_advance(
        lengths.data_ptr(), result.data_ptr(), lengths.shape[0], int(delta), int(capacity),
        None if overflow is None else overflow.data_ptr(),
        _native.current_stream(lengths.device),
    )
    _native.check(status, "slc_hip_kv_advance")
    return result


def hip_argmax(logits: torch.Tensor, *, out: torch.Tensor | None = None,
               workspace: _native.DeviceWorkspace | None = None) -> torch.Tensor:
    """Index of the first maximum along the last axis (int64).

    ``out`` (contiguous int64 with one element per row) receives the result in
    place, e.g. a decode loop's token buffer.  ``workspace`` (else the
    current stream's) lets wide rows split over several workgroups."""

    _require_gpu(logits, what="HIP argmax")
    if logits.dtype not in _FLOATS or logits.stride(-1) != 1:
        raise ValueError("HIP argmax: float logits with a contiguous last axis required")
    cols = logits.shape[-1]
    flat = logits.reshape(-1, cols)
    if out is None:
        out = torch.empty(flat.shape[0], device=logits.device, dtype=torch.int64)
    elif (not out.is_cuda or out.dtype != torch.int64 or not out.is_contiguous()
          or out.numel() != flat.shape[0]):
        raise ValueError("HIP argmax: out must be a contiguous int64 tensor with one entry per row")
    lib = _native.library()
    nbytes = lib.slc_hip_argmax_workspace_size(flat.shape[0])
    owner = workspace if workspace is not None else _native.stream_workspace(logits.device)
    buffer = owner.scratch("argmax", nbytes)
    counters = owner.counters(flat.shape[0])
    status = lib.slc_hip_argmax(
        flat.data_ptr(), out.data_ptr(), _native.dtype_tag(logits.dtype), flat.shape[0], cols,
        flat.stride(0), None if buffer is None else buffer.data_ptr(), nbytes,
        counters.data_ptr(), counters.numel(), _native.current_stream(logits.device),
    )
    _native.check(status, "slc_hip_argmax")
    return out.view(logits.shape[:-1])
