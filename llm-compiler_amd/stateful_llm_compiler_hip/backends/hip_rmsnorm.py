"""``kernel.hip.rms_norm``: RMSNorm over the last axis on gfx950.

Drop-in for the reference's ``triton_rms_norm``
(src/stateful_llm_compiler/backends/triton_rmsnorm.py:205-443); math of the
reference executor's ``_serve_rms_norm`` (execution.py:674-692), including the
Qwen2 ``round_before_weight`` order (model.py:44-51).
"""

from __future__ import annotations

import torch

from .. import _native

_DTYPE_NAMES = {
    "f16": torch.float16,
    "fp16": torch.float16,
    "float16": torch.float16,
    "bf16": torch.bfloat16,
    "bfloat16": torch.bfloat16,
    "f32": torch.float32,
    "fp32": torch.float32,
    "float32": torch.float32,
}


def resolve_dtype(
    output_dtype: str | torch.dtype | None, default: torch.dtype
) -> torch.dtype:
    if output_dtype is None:
        return default
    if isinstance(output_dtype, torch.dtype):
        return output_dtype
    try:
        return _DTYPE_NAMES[output_dtype]
    except KeyError as error:
        raise ValueError(f"unsupported output dtype {output_dtype}") from error


def hip_rms_norm(
    tensor: torch.Tensor,
    weight: torch.Tensor,
    *,
    epsilon: float,
    output_dtype: str | torch.dtype | None = None,
    num_warps: int | None = None,
    round_before_weight: bool = False,
) -> torch.Tensor:
    """RMSNorm of ``tensor`` over its last axis.

    ``num_warps`` keeps the reference's meaning of the launch width a profile
    plan picked, in gfx950 terms: wavefronts per row, 1 (the row in one wave's
    registers) or 4 (a 256-thread workgroup per row); None picks the first
    where it applies.
    """

    waves = 0 if num_warps is None else int(num_warps)
    if waves not in (0, 1, 4):
        raise ValueError(f"HIP RMSNorm: num_warps (waves per row) must be 1 or 4, got {num_warps}")
    if not tensor.is_cuda or not weight.is_cuda:
        raise ValueError("HIP RMSNorm: input and weight must be on the GPU")
    if tensor.ndim < 1:
        raise ValueError("HIP RMSNorm: input needs at least one dimension")
    hidden = tensor.shape[-1]
    if weight.ndim != 1 or weight.numel() != hidden:
        raise ValueError(
            f"HIP RMSNorm: weight must be [{hidden}], got {tuple(weight.shape)}"
        )
    if hidden > 65536:
        raise ValueError("HIP RMSNorm: hidden size above 65536")
    for t in (tensor, weight):
        if t.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f"HIP RMSNorm: unsupported dtype {t.dtype}")
    norm_dtype = resolve_dtype(output_dtype, tensor.dtype)
    if round_before_weight:
        out_dtype = torch.promote_types(weight.dtype, norm_dtype)
    else:
        out_dtype = norm_dtype
    if tensor.stride(-1) != 1:
        tensor = tensor.contiguous()
    rows = tensor.numel() // hidden if hidden else 0
    # Rows must be evenly strided; a (possibly non-contiguous) 2-D view of the
    # leading dims is all the kernel needs.
    try:
        flat = tensor.view(rows, hidden)
    except RuntimeError:
        tensor = tensor.contiguous()
        flat = tensor.view(rows, hidden)
    weight = weight.contiguous()
    output = torch.empty(tensor.shape, device=tensor.device, dtype=out_dtype)
    if rows == 0:
        return output
    status = _native.library().slc_hip_rms_norm(
        flat.data_ptr(),
        weight.data_ptr(),
        output.data_ptr(),
        _native.dtype_tag(tensor.dtype),
        _native.dtype_tag(weight.dtype),
        _native.dtype_tag(out_dtype),
        _native.dtype_tag(norm_dtype),
        rows,
        hidden,
        flat.stride(0),
        hidden,
        float(epsilon),
        1 if round_before_weight else 0,
        waves,
        _native.current_stream(tensor.device),
    )
    _native.check(status, "slc_hip_rms_norm")
    return output
