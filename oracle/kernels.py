"""Per-op oracle: eager restatement of the reference executor's op semantics.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Paths below are relative
to the reference repository's src/stateful_llm_compiler/.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def decode_attention(
    query: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    lengths: torch.Tensor,
    attention_mask: torch.Tensor,
    *,
    groups: int,
    scale: float,
) -> torch.Tensor:
    """PreallocatedKVCacheState.decode_attention without a runner.

    Follows execution.py:301-327: slice the physical B x Cap x H x D buffers to
    the mask length, expand KV heads by ``head // groups``, matmul in the input
    dtype, scale, add the fp32 mask, mask positions >= length with -inf, fp32
    softmax, cast back, matmul with V.
    """

    sequence = attention_mask.shape[-1]
    key = key_buffer[:, :sequence].permute(0, 2, 1, 3)
    value = value_buffer[:, :sequence].permute(0, 2, 1, 3)
    head_indices = torch.arange(query.shape[1], device=query.device) // groups
    key = key.index_select(1, head_indices)
    value = value.index_select(1, head_indices)
    scores = torch.matmul(query, key.transpose(-2, -1)) * scale
    scores = scores.float() + attention_mask.float()
    valid = torch.arange(sequence, device=query.device).view(
        1, 1, 1, sequence
    ) < lengths.view(-1, 1, 1, 1)
    scores = scores.masked_fill(~valid, float("-inf"))
    probabilities = torch.softmax(scores, dim=-1).to(query.dtype)
    return torch.matmul(probabilities, value)


def kv_store(
    key_buffer: np.ndarray,
    value_buffer: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    positions: np.ndarray,
) -> None:
    """Positional row scatter, in place (execution.py:743-781 native_kv_store).

    Row t of batch b (key is B x H x T x D) goes to buffer row positions[b]+t
    of the B x Cap x H x D buffer.  Rows at or past the capacity are dropped,
    which is what the reference's kernel does (backends/triton_kv.py:37-38).
    Works on raw bit patterns (any dtype viewed as integers), so the check is
    bit-exact.
    """

    batch, heads, tokens, _ = key.shape
    capacity = key_buffer.shape[1]
    for b in range(batch):
        for t in range(tokens):
            position = int(positions[b]) + t
            if 0 <= position < capacity:
                key_buffer[b, position] = key[b, :, t]
                value_buffer[b, position] = value[b, :, t]


def gather_pages(pool: np.ndarray, block_table: np.ndarray) -> np.ndarray:
    """The contiguous B x Cap x H x D buffer a paged layout stands for.

    The paged layout is the one docs/kv-bufferization.md:317-323 plans next:
    ``pool`` is [pages, page_tokens, H, D] and ``block_table[b, j]`` names the
    pool page holding tokens [j * page_tokens, (j + 1) * page_tokens) of
    sequence b, so the buffer row of (b, s) is ``pool[table[b, s // P],
    s % P]``.  Decode attention over the pages is defined as
    ``decode_attention`` over this gathered buffer.
    """

    page_tokens = pool.shape[1]
    batch, pages = block_table.shape
    out = np.empty((batch, pages * page_tokens) + pool.shape[2:], dtype=pool.dtype)
    for b in range(batch):
        for j in range(pages):
            out[b, j * page_tokens:(j + 1) * page_tokens] = pool[int(block_table[b, j])]
    return out


def paged_kv_store(
    key_pool: np.ndarray,
    value_pool: np.ndarray,
    block_table: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    positions: np.ndarray,
) -> None:
    """``kv_store`` into a paged layout, in place: row t of batch b goes to
    position positions[b] + t of sequence b, i.e. row (p % P) of pool page
    block_table[b, p // P]; positions outside the table's capacity are
    dropped, as ``kv_store`` drops rows past the buffer."""

    page_tokens = key_pool.shape[1]
    batch, heads, tokens, _ = key.shape
    capacity = block_table.shape[1] * page_tokens
    for b in range(batch):
        for t in range(tokens):
            position = int(positions[b]) + t
            if 0 <= position < capacity:
                page = int(block_table[b, position // page_tokens])
                key_pool[page, position % page_tokens] = key[b, :, t]
                value_pool[page, position % page_tokens] = value[b, :, t]


_DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def rms_norm(
    tensor: torch.Tensor,
    weight: torch.Tensor,
    *,
    epsilon: float,
    output_dtype: str | torch.dtype | None = None,
    round_before_weight: bool = False,
) -> torch.Tensor:
    """ReferenceExecutor._serve_rms_norm (execution.py:674-692)."""

    variance = tensor.float().pow(2).mean(dim=-1, keepdim=True)
    normalized = tensor.float() * torch.rsqrt(variance + epsilon)
    if isinstance(output_dtype, torch.dtype):
        torch_dtype = output_dtype
    else:
        torch_dtype = _DTYPES.get(output_dtype, tensor.dtype)
    if round_before_weight:
        return weight * normalized.to(torch_dtype)
    return (normalized * weight.float()).to(torch_dtype)


def rotate_half(tensor: torch.Tensor) -> torch.Tensor:
    """Qwen2 half rotation (qwen2.py:73-80, execution.py:756-761)."""

    half = tensor.shape[-1] // 2
    return torch.cat((-tensor[..., half:], tensor[..., :half]), dim=-1)


def rope(
    query: torch.Tensor,
    key: torch.Tensor,
    cosine: torch.Tensor,
    sine: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """ReferenceExecutor._serve_rope (execution.py:741-767)."""

    cosine = cosine.unsqueeze(1)
    sine = sine.unsqueeze(1)
    return (
        query * cosine + rotate_half(query) * sine,
        key * cosine + rotate_half(key) * sine,
    )


def prefill_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor | None,
    *,
    groups: int,
    scale: float,
    causal: bool | str = "mask",
) -> torch.Tensor:
    """ReferenceExecutor._serve_prefill_attention (execution.py:707-739).

    ``attention_mask`` None stands for an all-zero additive mask (the
    compiler's ``causal=True`` form, where causality comes from the kernel).
    """

    expanded_key = key.repeat_interleave(groups, dim=1)
    expanded_value = value.repeat_interleave(groups, dim=1)
    scores = torch.matmul(query, expanded_key.transpose(-2, -1))
    scores = scores * float(scale)
    scores = scores.float()
    if attention_mask is not None:
        scores = scores + attention_mask.float()
    if causal is True:
        tokens = query.shape[2]
        future = torch.triu(
            torch.ones(tokens, tokens, dtype=torch.bool, device=query.device),
            diagonal=1,
        )
        scores = scores.masked_fill(future, float("-inf"))
    probabilities = torch.softmax(scores, dim=-1).to(query.dtype)
    return torch.matmul(probabilities, expanded_value)


def linear(
    tensor: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """ReferenceExecutor._serve_linear (execution.py:694-705): F.linear."""

    return F.linear(tensor, weight, bias)
