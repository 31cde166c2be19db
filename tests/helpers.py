"""Shared test helpers: seeded inputs of the BASELINE configs and bf16 <-> numpy conversions."""

from __future__ import annotations

import numpy as np
import torch


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> np.uint16 bit patterns (host copy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray) -> torch.Tensor:
    """np.uint16 bit patterns -> bf16 tensor (host)."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def bf16_float(a: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(a).astype(np.uint32) << 16).view(np.float32)


def linear_inputs(M: int, N: int, K: int, seed: int = 0, w_std: float = 0.02, b_std: float = 0.01):
    """Config 0's draws in order from one generator: X ~ N(0,1) (M, K), W ~ N(0, w_std) (N, K), bias ~ N(0, b_std)
    (N), all bf16."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * w_std).to(torch.bfloat16)
    b = (torch.randn(N, generator=g) * b_std).to(torch.bfloat16)
    return x, w, b


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / rms(want), float64."""
    got, want = got.astype(np.float64), want.astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2)) + 1e-30
    return float(np.max(np.abs(got - want)) / rms) if got.size else 0.0


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """The bf16 ulp at |v| (8 significant bits)."""
    a = np.abs(v.astype(np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1e-38)))
    return np.where(a > 0, 2.0 ** (e - 7), 2.0 ** -133)


def assert_bf16_close(got_bits: np.ndarray, want_bits: np.ndarray, max_frac: float = 0.01) -> None:
    """The numeric bar for bf16 outputs computed with a different fp32 summation order than the checker: every
    element within max-abs 1e-2 x RMS of the checker's, except where one bf16 ulp of the value itself is larger than
    that (a rounding flip at |v| > ~2.5 RMS), which may differ by that one ulp; and at most max_frac of the elements
    differ at all."""
    got, want = bf16_float(got_bits).astype(np.float64), bf16_float(want_bits).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    tol = np.maximum(1e-2 * rms, bf16_ulp(want) * 1.0001)
    diff = np.abs(got - want)
    bad = diff > tol
    assert not bad.any(), f"{int(bad.sum())} elements beyond tolerance, worst {float((diff / tol).max()):.3f} x tol"
    assert (got_bits != want_bits).mean() <= max_frac, f"{(got_bits != want_bits).mean():.4f} of elements differ"
