"""Decoder-step projections on gfx950: the int8-weight (W8A16) layout and the 64-row chunked call of the reference's
kernels/stream_decoder.py (prepare_w8 38-48, W8_CONFIGS 30-35, StreamDecoder._w8 148-158), kept as its callers use
them, over the skinny HIP GEMMs of cohere-inference_amd/csrc/dec_w8.hip.

    wq = prepare_w8(w_bf16)                          # (uint8 (N, K), fp32 (N))
    y = w8_linear(x, wq, bias, relu=False, ws=ws, counters=counters)
    y = bf16_linear(x, w_bf16, bias)                 # o / cross-q / cross-o (the reference's Triton `linear`)
"""

from __future__ import annotations

import torch

from kernels.cuda_ext import ext

# (N, K) -> {rows up to: (columns per CTA, K splits)}: the reference's A10 table, accepted for compatibility. The gfx950
# kernel checks these like the reference does and then chooses its own tiling (results never depend on it).
W8_CONFIGS = {
    (1024, 4096): {1: (64, 4), 8: (16, 4), 16: (16, 4), 24: (16, 2), 32: (32, 4), 48: (64, 4), 64: (64, 4)},
    (3072, 1024): {1: (32, 1), 8: (32, 1), 16: (32, 1), 24: (32, 1), 32: (32, 1), 48: (64, 1), 64: (64, 1)},
    (4096, 1024): {1: (32, 1), 8: (32, 1), 16: (32, 1), 24: (64, 1), 32: (64, 1), 48: (64, 1), 64: (64, 1)},
    (16384, 1024): {1: (16, 1), 8: (16, 1), 16: (32, 1), 24: (64, 1), 32: (64, 1), 48: (64, 1), 64: (64, 1)},
}
DEFAULT_CONFIG = (64, 4)

# physical byte j of every 16 along K holds logical K W8_PERM[j] (the reference's layout, stream_decoder.py:38)
W8_PERM = (0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15)


def prepare_w8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (N, K) -> (uint8 (N, K) = int8 + 128 with K permuted within every 16 by W8_PERM, fp32 per-channel
    scales). Quantization: s = max(amax|w|, 1e-12) / 127, q = clamp(round_half_even(w / s), +-127)."""
    n, k = w.shape
    assert k % 16 == 0
    wf = w.float()
    s = wf.abs().amax(1).clamp_min(1e-12) / 127
    q = (torch.round(wf / s[:, None]).clamp(-127, 127) + 128).to(torch.uint8)
    perm = torch.tensor(W8_PERM, device=w.device)
    return q.reshape(n, k // 16, 16).index_select(2, perm).reshape(n, k).contiguous(), s.contiguous()


def unprepare_w8(wq: torch.Tensor) -> torch.Tensor:
    """The int8 (N, K) weights in natural K order of a prepare_w8 layout."""
    n, k = wq.shape
    inv = torch.empty(16, dtype=torch.long, device=wq.device)
    inv[torch.tensor(W8_PERM, device=wq.device)] = torch.arange(16, device=wq.device)
    return (wq.reshape(n, k // 16, 16).index_select(2, inv).reshape(n, k).to(torch.int16) - 128).to(torch.int8)


def w8_config(n: int, k: int, rows: int) -> tuple[int, int]:
    configs = W8_CONFIGS.get((n, k))
    if configs is None:
        return DEFAULT_CONFIG if k % (128 * DEFAULT_CONFIG[1]) == 0 and n % 64 == 0 else (16, 1)
    return configs[next(c for c in sorted(configs) if c >= rows)]


def w8_linear(x: torch.Tensor, wq: tuple[torch.Tensor, torch.Tensor], bias: torch.Tensor | None, relu: bool = False,
              ws: torch.Tensor | None = None, counters: torch.Tensor | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """x @ dequant(wq)^T + bias through dec_w8_linear, 64 rows at a time (the reference's StreamDecoder._w8)."""
    (w, scale), (n, k) = wq, wq[0].shape
    y = out if out is not None else torch.empty(x.shape[0], n, device=x.device, dtype=x.dtype)
    for r in range(0, x.shape[0], 64):
        m = min(64, x.shape[0] - r)
        bn, splits = w8_config(n, k, m)
        if ws is None or counters is None:
            splits = 1
        ext.dec_w8_linear(x[r:r + m], w, scale, bias, y[r:r + m], relu, bn, splits, ws, counters)
    return y


def bf16_linear(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, relu: bool = False,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """x @ w^T + b (relu) with bf16 weights, 64 rows at a time (the reference's `linear`, stream_decoder.py:23-27)."""
    y = out if out is not None else torch.empty(x.shape[0], w.shape[0], device=x.device, dtype=x.dtype)
    for r in range(0, x.shape[0], 64):
        m = min(64, x.shape[0] - r)
        ext.linear_bf16(x[r:r + m], w, b, y[r:r + m], relu)
    return y
