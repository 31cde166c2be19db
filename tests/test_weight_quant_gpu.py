"""The weight quantizers' scale on the GPU (rows a1 / a10): the reference computes `amax.clamp_min(1e-12) / 127` on
the GPU, where PyTorch divides a tensor by a Python scalar as a multiplication by the scalar's fp32 reciprocal. This
pins that on this GPU's PyTorch (the same ATen code), and checks that the product's quantize_rows / prepare_w8 give
the checker's bytes and scales on either device."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_bits, linear_inputs

pytestmark = pytest.mark.gpu


def test_gpu_division_by_scalar_is_reciprocal_multiply(gpu):
    from kernels.fast_encoder import RCP127

    g = torch.Generator().manual_seed(11)
    a = torch.randn(1 << 18, generator=g).abs() * 4
    on_gpu = (a.to(gpu) / 127).cpu()
    assert torch.equal(on_gpu, a * RCP127)
    assert not torch.equal(on_gpu, a / 127)  # CPU PyTorch divides exactly: the forms differ on this input


@pytest.mark.parametrize("shape", [(4096, 1024), (1280, 5120)])
def test_weight_quantizers_same_on_both_devices(gpu, shape):
    from kernels.fast_encoder import quantize_rows
    from kernels.stream_decoder import prepare_w8

    _, w, _ = linear_inputs(4, *shape, seed=sum(shape))
    qo, so = O.quantize_weight_rows(bf16_bits(w))
    for dev in ("cpu", gpu):
        q, s = quantize_rows(w.to(dev))
        assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so), dev
        u, s8 = prepare_w8(w.to(dev))
        uo, s8o = O.prepare_w8(bf16_bits(w))
        assert np.array_equal(u.cpu().numpy(), uo) and np.array_equal(s8.cpu().numpy(), s8o), dev
