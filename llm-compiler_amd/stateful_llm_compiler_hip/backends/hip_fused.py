"""Fused decode-step ops (``kernel.hip.norm_linear_group`` and friends).

Each wrapper computes exactly what a short sequence of the single ops
computes -- the fused kernels share those kernels' arithmetic, so the results
are bit-identical -- in one launch when the input is decode-sized (at most 32
rows of bf16/fp16), and by running that sequence of single-op kernels
otherwise.  Both paths are HIP kernels; nothing runs on the host.

The sequences replaced (reference semantics):
  norm_linear_group   rms_norm (round_before_weight) -> 1..3 linears
                      (execution.py:674-692, triton_executor.py:159-176)
  norm_linear_swiglu  rms_norm -> gate/up linears -> swiglu (qwen2.py:253-256)
  linear_residual     linear -> residual add (qwen2.py:288-294)
  rope_kv_store       rope -> kv_store of the rotated keys and the values
                      (execution.py:741-767, :743-781)
"""

from __future__ import annotations

from typing import Sequence

import torch

from .. import _native
from .hip_linear import hip_linear
from .hip_ops import check_flag, hip_add, hip_swiglu
from .hip_rmsnorm import hip_rms_norm

MAX_FUSED_ROWS = 32
_UNSUPPORTED = -2  # SLC_ERR_UNSUPPORTED
_MATRICES = 3


def _fusable_rows(x: torch.Tensor, *, norm: bool) -> bool:
    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    return (
        x.is_cuda
        and x.dtype in (torch.bfloat16, torch.float16)
        and x.is_contiguous()
        and 1 <= rows <= MAX_FUSED_ROWS
        and hidden % 8 == 0
        and (not norm or hidden <= 2048)
        and x.data_ptr() % 16 == 0
    )


def _check_weight(weight: torch.Tensor, x: torch.Tensor, what: str) -> None:
    if (
        not weight.is_cuda
        or weight.ndim != 2
        or weight.shape[1] != x.shape[-1]
        or weight.dtype != x.dtype
        or not weight.is_contiguous()
    ):
        raise ValueError(f"HIP {what}: weight must be a contiguous [N, {x.shape[-1]}] {x.dtype} tensor")


def hip_norm_linear_group(
    tensor: torch.Tensor,
    norm_weight: torch.Tensor | None,
    weights: Sequence[torch.Tensor],
    biases: Sequence[torch.Tensor | None],
    *,
    epsilon: float,
) -> list[torch.Tensor]:
    """``[linear(rms_norm(tensor), w, b) for w, b in zip(weights, biases)]``
    (round_before_weight norm; no norm when ``norm_weight`` is None)."""

    if not 1 <= len(weights) <= _MATRICES or len(biases) != len(weights):
        raise ValueError("HIP norm_linear_group: 1 to 3 weights, one bias entry each")
    for weight in weights:
        _check_weight(weight, tensor, "norm_linear_group")
    if (norm_weight is not None and not norm_weight.is_cuda) or any(
            b is not None and not b.is_cuda for b in biases):
        raise ValueError("HIP norm_linear_group: norm weight and biases must be on the GPU")
    norm = norm_weight is not None
    if not _fusable_rows(tensor, norm=norm):
        x = hip_rms_norm(tensor, norm_weight, epsilon=epsilon, round_before_weight=True) if norm else tensor
        if len(weights) == 1:
            return [hip_linear(x, weights[0], biases[0])]
        grouped = _linear_group(x, weights, biases)
        if grouped is not None:
            return grouped
        return [hip_linear(x, w, b) for w, b in zip(weights, biases)]
    hidden = tensor.shape[-1]
    rows = tensor.numel() // hidden
    outputs = [
        torch.empty((*tensor.shape[:-1], w.shape[0]), device=tensor.device, dtype=tensor.dtype)
        for w in weights
    ]
    per_matrix: list[object] = []
    for i in range(_MATRICES):
        if i < len(weights):
            bias = biases[i]
            per_matrix += [weights[i].data_ptr(), None if bias is None else bias.data_ptr(),
                           outputs[i].data_ptr(), weights[i].shape[0], weights[i].shape[0]]
        else:
            per_matrix += [None, None, None, 0, 0]
    status = _native.library().slc_hip_norm_linear_group(
        tensor.data_ptr(), hidden, None if norm_weight is None else norm_weight.data_ptr(),
        float(epsilon), rows, hidden, len(weights), *per_matrix,
        _native.dtype_tag(tensor.dtype), _native.current_stream(tensor.device),
    )
    if status == _UNSUPPORTED:  # nothing launched: the norm, then the linear
        x = hip_rms_norm(tensor, norm_weight, epsilon=epsilon, round_before_weight=True) if norm else tensor
        return [hip_linear(x, w, b) for w, b in zip(weights, biases)]
    _native.check(status, "slc_hip_norm_linear_group")
    return outputs


def hip_norm_linear_swiglu(
    tensor: torch.Tensor,
    norm_weight: torch.Tensor,
    gate_weight: torch.Tensor,
    up_weight: torch.Tensor,
    *,
    epsilon: float,
) -> torch.Tensor:
    """``swiglu(linear(x_n, gate_weight), linear(x_n, up_weight))`` with
    ``x_n = rms_norm(tensor, norm_weight)`` (round_before_weight)."""

    _check_weight(gate_weight, tensor, "norm_linear_swiglu")
    _check_weight(up_weight, tensor, "norm_linear_swiglu")
    if not norm_weight.is_cuda:
        raise ValueError("HIP norm_linear_swiglu: norm weight must be on the GPU")
    if gate_weight.shape != up_weight.shape:
        raise ValueError("HIP norm_linear_swiglu: gate and up weights differ in shape")
    if not _fusable_rows(tensor, norm=True):
        x = hip_rms_norm(tensor, norm_weight, epsilon=epsilon, round_before_weight=True)
        fused = _linear_swiglu(x, gate_weight, up_weight)
        if fused is not None:
            return fused
        return hip_swiglu(hip_linear(x, gate_weight), hip_linear(x, up_weight))
    hidden = tensor.shape[-1]
    features = gate_weight.shape[0]
    out = torch.empty((*tensor.shape[:-1], features), device=tensor.device, dtype=tensor.dtype)
    status = _native.library().slc_hip_norm_linear_swiglu(
        tensor.data_ptr(), hidden, norm_weight.data_ptr(), float(epsilon),
        tensor.numel() // hidden, hidden, features, gate_weight.data_ptr(), up_weight.data_ptr(),
        out.data_ptr(), features, _native.dtype_tag(tensor.dtype),
        _native.current_stream(tensor.device),
    )
    _native.check(status, "slc_hip_norm_linear_swiglu")
    return out


def _linear_group(x: torch.Tensor, weights: Sequence[torch.Tensor],
                  biases: Sequence[torch.Tensor | None]) -> list[torch.Tensor] | None:
    """Prefill-sized ``[linear(x, w, b) ...]`` in one launch, or None (nothing
    launched) when that kernel does not take the shapes."""

    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    if (not x.is_cuda or not x.is_contiguous() or rows <= 64
            or x.dtype not in (torch.bfloat16, torch.float16)
            or any(b is not None and (b.dtype != x.dtype or not b.is_contiguous()) for b in biases)):
        return None
    outputs = [torch.empty((*x.shape[:-1], w.shape[0]), device=x.device, dtype=x.dtype)
               for w in weights]
    per_matrix: list[object] = []
    for i in range(_MATRICES):
        if i < len(weights):
            b = biases[i]
            per_matrix += [weights[i].data_ptr(), None if b is None else b.data_ptr(),
                           outputs[i].data_ptr(), weights[i].shape[0], weights[i].shape[0]]
        else:
            per_matrix += [None, None, None, 0, 0]
    status = _native.library().slc_hip_linear_group(
        x.data_ptr(), hidden, rows, hidden, len(weights), *per_matrix,
        _native.dtype_tag(x.dtype), _native.current_stream(x.device),
    )
    if status == _UNSUPPORTED:
        return None
    _native.check(status, "slc_hip_linear_group")
    return outputs


def _linear_swiglu(x: torch.Tensor, gate_weight: torch.Tensor,
                   up_weight: torch.Tensor) -> torch.Tensor | None:
    """Prefill-sized ``swiglu(linear(x, gate), linear(x, up))`` in one kernel,
    or None (nothing launched) when that kernel does not take the shape."""

    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    if (not x.is_cuda or not x.is_contiguous() or rows <= 64
            or x.dtype not in (torch.bfloat16, torch.float16)):
        return None
    features = gate_weight.shape[0]
    out = torch.empty((*x.shape[:-1], features), device=x.device, dtype=x.dtype)
    status = _native.library().slc_hip_linear_swiglu(
        x.data_ptr(), hidden, rows, hidden, features, gate_weight.data_ptr(),
        up_weight.data_ptr(), out.data_ptr(), features, _native.dtype_tag(x.dtype),
        _native.current_stream(x.device),
    )
    if status == _UNSUPPORTED:
        return None
    _native.check(status, "slc_hip_linear_swiglu")
    return out


def hip_linear_residual(
    tensor: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    residual: torch.Tensor,
) -> torch.Tensor:
    """``residual + linear(tensor, weight, bias)`` (each rounded like the
    separate ops)."""

    _check_weight(weight, tensor, "linear_residual")
    out_shape = (*tensor.shape[:-1], weight.shape[0])
    if tuple(residual.shape) != out_shape or residual.dtype != tensor.dtype:
        raise ValueError("HIP linear_residual: residual must match the linear output")
    if not residual.is_cuda or (bias is not None and not bias.is_cuda):
        raise ValueError("HIP linear_residual: residual and bias must be on the GPU")
    hidden = tensor.shape[-1]
    rows = tensor.numel() // hidden if hidden else 0
    # Decode-sized rows take the fused row kernel; prefill-sized rows the tile
    # kernel with the residual in its store epilogue, when it takes the shape.
    prefill = (rows > MAX_FUSED_ROWS and tensor.is_cuda and tensor.is_contiguous()
               and residual.is_contiguous() and tensor.dtype in (torch.bfloat16, torch.float16)
               and (bias is None or (bias.dtype == tensor.dtype and bias.is_contiguous())))
    if not prefill and (not _fusable_rows(tensor, norm=False) or not residual.is_contiguous()):
        return hip_add(residual, hip_linear(tensor, weight, bias))
    features = weight.shape[0]
    out = torch.empty(out_shape, device=tensor.device, dtype=tensor.dtype)
    status = _native.library().slc_hip_linear_residual(
        tensor.data_ptr(), hidden, tensor.numel() // hidden, hidden, features,
        weight.data_ptr(), None if bias is None else bias.data_ptr(), residual.data_ptr(),
        features, out.data_ptr(), features, _native.dtype_tag(tensor.dtype),
        _native.current_stream(tensor.device),
    )
    if status == _UNSUPPORTED:
        return hip_add(residual, hip_linear(tensor, weight, bias))
    _native.check(status, "slc_hip_linear_residual")
    return out


def hip_rope_kv_store(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cosine: torch.Tensor,
    sine: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    positions: torch.Tensor,
    *,
    overflow: torch.Tensor | None = None,
    advance: int = 0,
    lengths_out: torch.Tensor | None = None,
    workspace: _native.DeviceWorkspace | None = None,
) -> torch.Tensor:
    """``q_rot, k_rot = rope(query, key, cosine, sine)``; store ``k_rot`` and
    ``value`` rows at ``positions[b] + t`` of the [B, Cap, H, D] buffers;
    return ``q_rot``.  With ``advance > 0`` also write
    ``lengths_out = positions + advance`` (``lengths_out`` may be
    ``positions``), as the kv advance after the store would; the advance
    counts the store's workgroups in ``workspace`` (else the current
    stream's)."""

    tensors = (query, key, value, cosine, sine, key_buffer, value_buffer, positions)
    if not all(t.is_cuda for t in tensors):
        raise ValueError("HIP rope_kv_store: all tensors must be on the GPU")
    check_flag(overflow, "HIP rope_kv_store")
    if query.ndim != 4 or key.ndim != 4 or value.shape != key.shape:
        raise ValueError("HIP rope_kv_store: q/k/v must be [B, H, T, D] with matching k/v")
    if any(t.stride(-1) != 1 for t in (query, key, value, cosine, sine)):
        raise ValueError("HIP rope_kv_store: head dims must be contiguous")
    if not key_buffer.is_contiguous() or not value_buffer.is_contiguous():
        raise ValueError("HIP rope_kv_store: buffers must be contiguous")
    batch, q_heads, tokens, head_dim = query.shape
    kv_heads = key.shape[1]
    if (key_buffer.shape != value_buffer.shape or key_buffer.ndim != 4
            or key_buffer.shape[0] != batch or key_buffer.shape[2] != kv_heads
            or key_buffer.shape[3] != head_dim or key.shape[0] != batch
            or key.shape[2] != tokens or key.shape[3] != head_dim):
        raise ValueError("HIP rope_kv_store: shapes do not match the buffers")
    if positions.shape != (batch,) or positions.dtype != torch.int64:
        raise ValueError("HIP rope_kv_store: positions must be a [batch] int64 tensor")
    if cosine.shape != (batch, tokens, head_dim) or sine.shape != cosine.shape:
        raise ValueError("HIP rope_kv_store: cos/sin must be [B, T, D]")
    dtypes = {t.dtype for t in (query, key, value, cosine, sine, key_buffer, value_buffer)}
    if len(dtypes) != 1:
        raise ValueError("HIP rope_kv_store: dtypes must match")
    q_out = torch.empty((batch, q_heads, tokens, head_dim), device=query.device, dtype=query.dtype)
    if advance < 0 or (advance > 0) != (lengths_out is not None):
        raise ValueError("HIP rope_kv_store: advance > 0 needs lengths_out (and only then)")
    if lengths_out is not None and (lengths_out.shape != (batch,) or lengths_out.dtype != torch.int64
                                    or not lengths_out.is_cuda or not lengths_out.is_contiguous()):
        raise ValueError("HIP rope_kv_store: lengths_out must be a contiguous [batch] int64 GPU tensor")
    if not positions.is_contiguous():
        if lengths_out is not None and lengths_out.data_ptr() == positions.data_ptr():
            raise ValueError("HIP rope_kv_store: in-place advance needs contiguous positions")
        positions = positions.contiguous()
    counter = None
    if lengths_out is not None:
        owner = workspace if workspace is not None else _native.stream_workspace(query.device)
        counter = owner.counters(1)
    status = _native.library().slc_hip_rope_kv_store(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), cosine.data_ptr(), sine.data_ptr(),
        q_out.data_ptr(), key_buffer.data_ptr(), value_buffer.data_ptr(), positions.data_ptr(),
        None if overflow is None else overflow.data_ptr(),
        None if lengths_out is None else lengths_out.data_ptr(), int(advance),
        _native.dtype_tag(query.dtype),
        batch, q_heads, kv_heads, tokens, head_dim, key_buffer.shape[1],
        query.stride(0), query.stride(1), query.stride(2),
        key.stride(0), key.stride(1), key.stride(2),
        value.stride(0), value.stride(1), value.stride(2),
        cosine.stride(0), cosine.stride(1), sine.stride(0), sine.stride(1),
        q_out.stride(0), q_out.stride(1), q_out.stride(2),
        None if counter is None else counter.data_ptr(), 0 if counter is None else counter.numel(),
        _native.current_stream(query.device),
    )
    _native.check(status, "slc_hip_rope_kv_store")
    return q_out
