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
@pytest.mark.parametrize("M", [1, 9, 16, 24, 32, 37, 64])
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
@pytest.mark.parametrize("M", [1, 16, 24, 32, 64])
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


FUSED = [(3072, 1024, True, False), (1024, 1024, False, False), (4096, 1024, True, True), (16384, 1024, True, False),
         (1024, 1024, True, False)]


@pytest.mark.parametrize("N,K,w8,relu", FUSED)
@pytest.mark.parametrize("M", [1, 9, 16, 24, 32, 37, 64])
def test_dec_linear_fused_ln_prologue(N, K, w8, relu, M, gpu):
    """LayerNorm prologue: dec_linear_fused(x, ln) has exactly the bits of dec_add_ln's LayerNorm followed by the plain
    projection (the product's own unfused path), and is within the projection bar of the oracle's LN -> linear."""
    from kernels.cuda_ext import DEC_EP_NONE, DEC_EP_RELU, ext
    from kernels.stream_decoder import prepare_w8

    print(f"dec_linear_fused LN M={M} N={N} K={K} w8={w8} relu={relu}", flush=True)
    x, w, b = linear_inputs(M, N, K, seed=3 * M + N)
    g = torch.Generator().manual_seed(M + K)
    lw = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    lb = (0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    xg, bg, lwg, lbg = x.cuda(), b.cuda(), lw.cuda(), lb.cuda()
    if w8:
        wq, sw = (t.cuda() for t in prepare_w8(w))
    else:
        wq, sw = w.cuda(), None
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ext.dec_linear_fused(xg, wq, sw, bg, y, DEC_EP_RELU if relu else DEC_EP_NONE, ln=(lwg, lbg, 1e-5))
    # the unfused path: dec_add_ln with a zero addend is LN(x)
    xs, h = xg.clone(), torch.empty_like(xg)
    ext.dec_add_ln(xs, torch.zeros_like(xg), lwg, lbg, 1e-5, h)
    y2 = torch.empty_like(y)
    if w8:
        ext.dec_w8_linear(h, wq, sw, bg, y2, relu, 64, 1, None, None)
    else:
        ext.linear_bf16(h, wq, bg, y2, relu)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    hb = O.dec_add_ln(bf16_bits(x).copy(), np.zeros((M, K), np.uint16), (bf16_bits(lw), bf16_bits(lb), 1e-5))
    _check_close(bf16_bits(h), hb)  # the LayerNorm against the oracle's (fp32 sums in another order)
    if w8:
        want = O.dec_w8_linear(hb, wq.cpu().numpy(), sw.cpu().numpy(), bf16_bits(b), relu=relu)
    else:
        want = O.linear_bf16(hb, bf16_bits(w), bf16_bits(b), relu=relu)
    _check_close(bf16_bits(y), want)


@pytest.mark.parametrize("N,K,w8", [(1024, 1024, False), (1024, 4096, True), (1024, 4096, False)])
@pytest.mark.parametrize("M", [1, 16, 24, 32, 37, 64])
def test_dec_linear_fused_residual(N, K, w8, M, gpu):
    """Residual epilogue: y = bf16(y + bf16(x @ w^T + b)) in place, bit-identical to the projection followed by
    dec_add_ln's sum, and the sum bit-exact against the oracle's add on the kernel's projection."""
    from kernels.cuda_ext import DEC_EP_RESID, ext
    from kernels.stream_decoder import prepare_w8

    print(f"dec_linear_fused resid M={M} N={N} K={K} w8={w8}", flush=True)
    x, w, b = linear_inputs(M, N, K, seed=5 * M + K)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    xg, bg = x.cuda(), b.cuda()
    if w8:
        wq, sw = (t.cuda() for t in prepare_w8(w))
    else:
        wq, sw = w.cuda(), None
    res = r.cuda()
    ext.dec_linear_fused(xg, wq, sw, bg, res, DEC_EP_RESID)
    proj = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    if w8:
        ext.dec_w8_linear(xg, wq, sw, bg, proj, False, 64, 1, None, None)
    else:
        ext.linear_bf16(xg, wq, bg, proj, False)
    torch.cuda.synchronize()
    want = bf16_bits(r).copy()
    lw, lb = np.full(N, 0x3F80, np.uint16), np.zeros(N, np.uint16)
    O.dec_add_ln(want, bf16_bits(proj.cpu()), (lw, lb, 1e-5))  # want = bf16(r + proj)
    assert np.array_equal(bf16_bits(res.cpu()), want)


def test_dec_linear_fused_rejects(gpu):
    from kernels.cuda_ext import DEC_EP_RESID, ext

    x = torch.zeros(4, 2048, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(64, 2048, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda")
    ln = (torch.ones(2048, dtype=torch.bfloat16, device="cuda"), torch.zeros(2048, dtype=torch.bfloat16, device="cuda"),
          1e-5)
    with pytest.raises(RuntimeError, match="LayerNorm prologue"):
        ext.dec_linear_fused(x, w, None, None, y, ln=ln)
    with pytest.raises(RuntimeError, match="residual"):
        ext.dec_linear_fused(x[:, :1024], w[:, :1024].contiguous(), None, None, y, DEC_EP_RESID,
                             ln=(ln[0][:1024], ln[1][:1024], 1e-5))
