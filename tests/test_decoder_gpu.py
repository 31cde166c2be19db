"""GPU parity of the decoder-step skinny projections (W8A16 dec_w8_linear and bf16 linear), the LayerNorm int8
producer, and graph replay of the split-K kernel, through the C ABI.

Bar (helpers.assert_bf16_close): bf16 outputs within max-abs 1e-2 x RMS of the oracle's, or one bf16 ulp where the
value's own ulp is larger (the kernel sums in fp32 in its own order, the oracle in fp64, so a rounding may flip);
split-K results identical run to run."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_bf16_close, bf16_bits, bf16_float, linear_inputs

pytestmark = pytest.mark.gpu

SHAPES = [(3072, 1024), (4096, 1024), (1024, 4096), (16384, 1024), (1024, 1024)]


@pytest.fixture(scope="module")
def ws(gpu):
    return torch.empty(8 << 20, dtype=torch.float32, device="cuda"), torch.zeros(1024, dtype=torch.int32,
                                                                                   device="cuda")


def _check_close(got_bits, want_bits):
    assert_bf16_close(got_bits, want_bits)


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 16, 37, 64])
def test_dec_w8_linear(ws, N, K, M):
    from kernels.stream_decoder import prepare_w8, w8_linear

    print(f"dec_w8_linear M={M} N={N} K={K}", flush=True)
    x, w, b = linear_inputs(M, N, K, seed=M + N)
    wq = tuple(t.cuda() for t in prepare_w8(w))
    relu = N == 4096
    y = w8_linear(x.cuda(), wq, b.cuda(), relu=relu, ws=ws[0], counters=ws[1])
    want = O.dec_w8_linear(bf16_bits(x), wq[0].cpu().numpy(), wq[1].cpu().numpy(), bf16_bits(b), relu=relu)
    _check_close(bf16_bits(y), want)
    assert int(ws[1].abs().sum()) == 0  # counters left at zero


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 24, 64])
def test_linear_bf16(N, K, M, gpu):
    from kernels.stream_decoder import bf16_linear

    print(f"linear_bf16 M={M} N={N} K={K}", flush=True)
    x, w, b = linear_inputs(M, N, K, seed=M + 2 * N)
    y = bf16_linear(x.cuda(), w.cuda(), b.cuda())
    want = O.linear_bf16(bf16_bits(x), bf16_bits(w), bf16_bits(b))
    _check_close(bf16_bits(y), want)


def test_dec_w8_split_deterministic_and_graph_replay(ws):
    """Serial split-K: identical bits run to run, and inside a captured graph replayed several times with eager work
    between the replays (counters self-reset; no memset nodes)."""
    from kernels.stream_decoder import prepare_w8, w8_linear

    M, N, K = 64, 1024, 4096
    x, w, b = linear_inputs(M, N, K, seed=31)
    wq = tuple(t.cuda() for t in prepare_w8(w))
    xd, bd = x.cuda(), b.cuda()
    y0 = w8_linear(xd, wq, bd, ws=ws[0], counters=ws[1])
    for _ in range(3):
        assert torch.equal(w8_linear(xd, wq, bd, ws=ws[0], counters=ws[1]), y0)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w8_linear(xd, wq, bd, ws=ws[0], counters=ws[1], out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w8_linear(xd, wq, bd, ws=ws[0], counters=ws[1], out=out)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0), f"replay {i}"
        _ = w8_linear(xd, wq, bd, ws=ws[0], counters=ws[1])  # eager work between replays
    assert int(ws[1].abs().sum()) == 0


def test_layernorm_q8(gpu):
    from kernels.cuda_ext import ext

    M, D = 513, 1280
    g = torch.Generator().manual_seed(41)
    x = (torch.randn(M, D, generator=g) * 3 + 1).to(torch.bfloat16)
    w1, b1 = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16), (0.1 * torch.randn(D, generator=g)).to(
        torch.bfloat16)
    w2, b2 = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16), (0.1 * torch.randn(D, generator=g)).to(
        torch.bfloat16)
    for two in (False, True):
        xd = x.cuda()
        hq = torch.empty(M, D, dtype=torch.int8, device="cuda")
        hs = torch.empty(M, 1, dtype=torch.float32, device="cuda")
        ext.layernorm_q8(xd, w1.cuda(), b1.cuda(), 1e-5, w2.cuda() if two else None, b2.cuda() if two else None,
                         1e-5, hq, hs)
        ln1 = torch.nn.functional.layer_norm(x.double(), (D,), w1.double(), b1.double(), 1e-5).to(torch.bfloat16)
        h = torch.nn.functional.layer_norm(ln1.double(), (D,), w2.double(), b2.double(), 1e-5).to(
            torch.bfloat16) if two else ln1
        qo, so = O.q8_rows(bf16_bits(h))
        dq = np.abs(hq.cpu().numpy().astype(np.int32) - qo.astype(np.int32))
        assert dq.max() <= 1 and (dq != 0).mean() < 5e-3
        assert np.allclose(hs.cpu().numpy()[:, 0], so, rtol=2.0 ** -7)
        if two:  # x = LN1(x) in place, bf16: within one ulp of the float64 LayerNorm
            got = xd.cpu().float().numpy()
            ref = torch.nn.functional.layer_norm(x.double(), (D,), w1.double(), b1.double(), 1e-5).numpy()
            assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-3).all()
