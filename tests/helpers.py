"""Shared helpers of the test-suite (seeded inputs and tolerance checks)."""

from __future__ import annotations

import sys

import torch

# Tolerances stated by the project's numerical contract:
BF16_ATOL = 2e-2  # bf16 fast mode: absolute, on logits / attention outputs / KV
FP32_RTOL = 1e-5  # fp32: relative (to the largest reference magnitude)


def announce(case: str) -> None:
    """Print and flush the case name before a GPU step (fault attribution)."""

    print(f"[case] {case}", flush=True)
    sys.stdout.flush()


def generator(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def assert_fp32_close(actual: torch.Tensor, expected: torch.Tensor, rtol: float = FP32_RTOL) -> None:
    actual = actual.detach().float().cpu()
    expected = expected.detach().float().cpu()
    assert actual.shape == expected.shape
    scale = expected.abs().max().item() if expected.numel() else 0.0
    error = (actual - expected).abs().max().item() if expected.numel() else 0.0
    assert error <= rtol * max(scale, 1e-30), (
        f"fp32 mismatch: max abs error {error:.3e} vs reference scale {scale:.3e}"
        f" (relative bound {rtol})"
    )


def assert_bf16_close(actual: torch.Tensor, expected: torch.Tensor, atol: float = BF16_ATOL) -> None:
    """|actual - expected| <= atol (2e-2) element-wise, or one bf16 unit in
    the last place of the expected value where that is larger: outputs of
    magnitude 4 and above have a bf16 spacing (2^-5) above 2e-2, so a result
    that rounds to the neighbouring bf16 value is within the contract."""

    actual = actual.detach().float().cpu()
    expected = expected.detach().float().cpu()
    assert actual.shape == expected.shape
    if not expected.numel():
        return
    diff = (actual - expected).abs()
    _, exponent = torch.frexp(expected.abs())
    ulp = torch.ldexp(torch.ones_like(expected), exponent - 8)  # bf16: 8 significant bits
    bound = torch.maximum(torch.full_like(expected, atol), ulp)
    excess = (diff - bound).max().item()
    worst = int(torch.argmax(diff - bound))
    assert excess <= 0, (
        f"bf16 mismatch: error {diff.flatten()[worst].item():.3e} at expected "
        f"{expected.flatten()[worst].item():.4g} exceeds max({atol}, 1 bf16 ulp); "
        f"max abs error {diff.max().item():.3e}"
    )


def assert_bitwise_equal(actual: torch.Tensor, expected: torch.Tensor) -> None:
    actual = actual.detach().cpu().contiguous()
    expected = expected.detach().cpu().contiguous()
    assert actual.shape == expected.shape and actual.dtype == expected.dtype
    width = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[
        actual.element_size()
    ]
    a = actual.view(width)
    b = expected.view(width)
    differ = (a != b).sum().item()
    assert differ == 0, f"{differ} of {a.numel()} elements differ bitwise"
