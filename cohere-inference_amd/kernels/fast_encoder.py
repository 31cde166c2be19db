"""Encoder-side int8 linears on gfx950: the weight quantization, tile-config surface and W8A8 / 2:4 linear helpers of
the reference's kernels/fast_encoder.py (quantize_rows 60-63, I8_* / I8_SMALL / SP_CONFIGS 34-57, i8_config 50-57),
over the HIP GEMMs of cohere-inference_amd/csrc/gemm_q8.hip.

    q, s = quantize_rows(w_bf16)                         # int8 (N, K), fp32 (N)
    lin = Int8Linear(w_bf16, bias, sparse=True)          # pruned 2:4 before quantization, compressed
    y = lin(xq, xs, epi=EPI_BIAS)                        # bf16 (M, N)
"""

from __future__ import annotations

import torch

from kernels.cuda_ext import EPI_BIAS, EPI_GLU, EPI_RESID, EPI_SILU_Q8, ext
from kernels.sparse import compress_24, prune_24_magnitude

# The reference's int8 config ids (A10 tile choices). They are accepted and checked by the gfx950 GEMMs (each id keeps
# its meaning for the SILU_Q8 output group: configs 4, 6, 8 have 256-column groups) but the tiles are chosen for gfx950
# by shape; results never depend on the id.
I8_CFG, I8_CFG_GROUPED, I8_CFG_FF1, FF_GROUP = 0, 10, 4, 256
I8_SMALL = {"ff1": ((96, 6), (224, 8), (384, 4), (448, 8)),
            "ff2": ((256, 5), (640, 9), (896, 3), (1152, 9)),
            "qkv": ((192, 9), (256, 0), (320, 9)),
            "pw1": ((320, 9), (384, 0), (448, 9)),
            "o": ((640, 9), (896, 0), (1056, 9))}
SP_CONFIGS = ((448, 2), (2048, 0), (1 << 30, 3))


def i8_config(gemm: str, frames: int, default: int) -> int:
    for up_to, cfg in I8_SMALL[gemm]:
        if frames <= up_to:
            return cfg
    return default


def quantize_rows(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric int8 per output channel: s = max(amax|w|, 1e-12) / 127 (fp32), q = clamp(round_half_even(w / s),
    +-127). Load-time weight preparation (reference fast_encoder.py:60-63)."""
    wf = w.float()
    s = wf.abs().amax(-1).clamp_min(1e-12) / 127
    return torch.round(wf / s[:, None]).clamp(-127, 127).to(torch.int8).contiguous(), s.contiguous()


def quantize_activations(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (M, K) -> int8 (M, K) + fp32 (M, 1) per-row scales, on the GPU (the reference's ext.quantize_rows)."""
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(x.shape[0], 1, dtype=torch.float32, device=x.device)
    ext.quantize_rows(x, q, s)
    return q, s


class Int8Linear:
    """A W8A8 linear layer: int8 weights per output channel, optionally pruned 2:4 (magnitude, before
    quantization, as the reference prunes before fast_encoder.py:109 quantizes) and stored compressed."""

    def __init__(self, w: torch.Tensor, bias: torch.Tensor | None, sparse: bool = False):
        if sparse:
            w = prune_24_magnitude(w)
        self.q, self.s = quantize_rows(w)
        self.bias = None if bias is None else bias.to(torch.bfloat16).contiguous()
        self.n, self.k = self.q.shape
        self.sparse = sparse
        if sparse:
            self.wc, self.e = compress_24(self.q)

    def __call__(self, xq: torch.Tensor, xs: torch.Tensor, epi: int = EPI_BIAS, group: int | None = None,
                 out: torch.Tensor | None = None, resid: torch.Tensor | None = None, alpha: float = 1.0,
                 qs: torch.Tensor | None = None, cfg: int = -1) -> torch.Tensor:
        m = xq.shape[0]
        group = self.k if group is None else group
        if out is None:
            if epi == EPI_SILU_Q8:
                out = torch.empty(m, self.n, dtype=torch.int8, device=xq.device)
            else:
                out = torch.empty(m, self.n // 2 if epi == EPI_GLU else self.n, dtype=torch.bfloat16,
                                  device=xq.device)
        if self.sparse:
            ext.gemm_sp_epi(xq, xs, group, self.wc, self.e, self.s, self.bias, out, epi, resid, alpha, qs, cfg)
        else:
            ext.gemm_i8(xq, xs, group, self.q, self.s, self.bias, out, epi, resid, alpha, qs, cfg)
        return out


__all__ = ["EPI_BIAS", "EPI_GLU", "EPI_RESID", "EPI_SILU_Q8", "I8_CFG", "I8_CFG_GROUPED", "I8_CFG_FF1", "FF_GROUP",
           "I8_SMALL", "SP_CONFIGS", "Int8Linear", "i8_config", "quantize_activations", "quantize_rows"]
