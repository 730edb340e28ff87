"""``kernel.hip.linear``: X . W^T (+ bias) on gfx950 MFMA.

Drop-in for the reference's ``triton_linear``
(src/stateful_llm_compiler/backends/triton_linear.py:87-148) and for the
library GEMM behind ``kernel.cublas.linear`` (triton_executor.py:159-176):
same arguments, same validation, a new output tensor.
"""

from __future__ import annotations

import torch

from .. import _native


def hip_linear(
    tensor: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    tile: str = "auto",
) -> torch.Tensor:
    """2-D or 3-D ``tensor`` [..., K] times ``weight`` [N, K]^T (+ ``bias`` [N]).

    ``tile`` picks the workgroup tile of the prefill-sized MFMA path (a
    profile plan's choice, ``cost_model``); every tile gives the same bits.
    """

    if not tensor.is_cuda or not weight.is_cuda or (bias is not None and not bias.is_cuda):
        raise ValueError("HIP linear: tensors must be on the GPU")
    if tensor.ndim not in {2, 3} or weight.ndim != 2:
        raise ValueError("HIP linear: input must be 2-D or 3-D and weight 2-D")
    if not tensor.is_contiguous() or not weight.is_contiguous():
        raise ValueError("HIP linear: input and weight must be contiguous")
    if tensor.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"HIP linear: unsupported dtype {tensor.dtype}")
    if tensor.dtype != weight.dtype or tensor.device != weight.device:
        raise ValueError("HIP linear: input and weight need one dtype and device")
    output_features, input_features = weight.shape
    if tensor.shape[-1] != input_features:
        raise ValueError("HIP linear: input K does not match weight K")
    if bias is not None:
        if (
            bias.shape != (output_features,)
            or bias.dtype != tensor.dtype
            or bias.device != tensor.device
            or not bias.is_contiguous()
        ):
            raise ValueError("HIP linear: bias shape, dtype or device mismatch")
    if tile not in _native.LINEAR_TILES:
        raise ValueError(f"HIP linear: unknown tile {tile!r}")
    rows = tensor.numel() // input_features
    output = torch.empty(
        (*tensor.shape[:-1], output_features), device=tensor.device, dtype=tensor.dtype
    )
    if rows == 0:
        return output
    status = _native.library().slc_hip_linear_tile(
        tensor.data_ptr(),
        weight.data_ptr(),
        None if bias is None else bias.data_ptr(),
        output.data_ptr(),
        _native.dtype_tag(tensor.dtype),
        rows,
        output_features,
        input_features,
        input_features,
        output_features,
        _native.LINEAR_TILES[tile],
        _native.current_stream(tensor.device),
    )
    _native.check(status, "slc_hip_linear_tile")
    return output
