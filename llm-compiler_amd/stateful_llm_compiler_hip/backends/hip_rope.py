"""``kernel.hip.rope``: dual-output Qwen2 rotary embedding on gfx950.

Drop-in for the reference's ``triton_rope``
(src/stateful_llm_compiler/backends/triton_rope.py:299-390); math of the
reference executor's ``_serve_rope`` (execution.py:741-767).  Each product is
rounded to the tensor dtype before the add, so the result is bit-identical to
the eager PyTorch composite.
"""

from __future__ import annotations

import torch

from .. import _native


def hip_rope(
    query: torch.Tensor,
    key: torch.Tensor,
    cosine: torch.Tensor,
    sine: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate B x QH x T x D ``query`` and B x KVH x T x D ``key``."""

    tensors = (query, key, cosine, sine)
    if not all(tensor.is_cuda for tensor in tensors):
        raise ValueError("HIP RoPE: all tensors must be on the GPU")
    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("HIP RoPE: query and key must be 4-D")
    if cosine.ndim != 3 or sine.shape != cosine.shape:
        raise ValueError("HIP RoPE: cosine and sine must be equal-shaped 3-D tensors")
    batch, _, tokens, head_dim = query.shape
    if (
        key.shape[0] != batch
        or key.shape[2:] != (tokens, head_dim)
        or cosine.shape != (batch, tokens, head_dim)
    ):
        raise ValueError("HIP RoPE: batch, token or head-dim mismatch")
    if head_dim <= 0 or head_dim % 2 or head_dim > 65536:
        raise ValueError("HIP RoPE: head dim must be a positive even number <= 65536")
    if len({tensor.dtype for tensor in tensors}) != 1:
        raise ValueError("HIP RoPE: all tensors must share one dtype")
    if query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"HIP RoPE: unsupported dtype {query.dtype}")
    if any(tensor.stride(-1) != 1 for tensor in tensors):
        raise ValueError("HIP RoPE: head dims must be contiguous")

    lib = _native.library()
    query_out = torch.empty_like(query)
    key_out = torch.empty_like(key)
    status = lib.slc_hip_rope(
        query.data_ptr(),
        key.data_ptr(),
        cosine.data_ptr(),
        sine.data_ptr(),
        query_out.data_ptr(),
        key_out.data_ptr(),
        _native.dtype_tag(query.dtype),
        batch,
        query.shape[1],
        key.shape[1],
        tokens,
        head_dim,
        *query.stride()[:3],
        *key.stride()[:3],
        cosine.stride(0),
        cosine.stride(1),
        sine.stride(0),
        sine.stride(1),
        *query_out.stride()[:3],
        *key_out.stride()[:3],
        _native.current_stream(query.device),
    )
    _native.check(status, "slc_hip_rope")
    return query_out, key_out
