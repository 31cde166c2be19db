"""GPU parity of the W8A8 dense and 2:4 sparse int8 GEMMs and the activation quantizer against the CPU checker
(oracle/), through the C ABI (kernels.cuda_ext.ext).

Bar: int32 accumulators and int8 activations bit-exact; bf16 outputs of BIAS / RESID / grouped epilogues bit-exact
(the arithmetic is the same sequence of correctly rounded fp32 operations); GLU and SILU_Q8 (whose sigmoid uses the
GPU's exp) within one bf16 ulp / one int8 step; every bf16 output within max-abs 1e-2 x RMS of the oracle's."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_bf16_close, bf16_bits, bf16_float, linear_inputs, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext(gpu):
    from kernels.cuda_ext import ext as e

    e.set_gemm_tile(-1)
    yield e
    e.set_gemm_tile(-1)


def _prep(M, N, K, seed=0, dev="cuda"):
    """Seeded bf16 inputs, quantized: x on the GPU by quantize_rows, w on the host (load-time weights)."""
    from kernels.fast_encoder import quantize_activations, quantize_rows

    x, w, b = linear_inputs(M, N, K, seed)
    xq, xs = quantize_activations(x.to(dev))
    wq, ws = quantize_rows(w)
    return x, xq, xs, wq.to(dev), ws.to(dev), b.to(dev)


def _np(t):
    return t.detach().cpu().numpy()


def _int_mm_cpu(xq, wq):
    return torch._int_mm(xq.cpu(), wq.cpu().t().contiguous()).numpy()


# ---- a2: activation quantizer ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("M,K", [(1, 1280), (5, 1280), (3000, 1280), (77, 5120), (33, 1024)])
def test_quantize_rows_bit_exact(ext, M, K):
    print(f"quantize_rows M={M} K={K}", flush=True)
    x, _, _ = linear_inputs(M, 64, K, seed=M)
    x[0, :] = 0  # a zero row: scale 1, all zeros
    xd = x.cuda()
    q = torch.empty(M, K, dtype=torch.int8, device="cuda")
    s = torch.empty(M, dtype=torch.float32, device="cuda")
    ext.quantize_rows(xd, q, s)
    qo, so = O.q8_rows(bf16_bits(x))
    assert np.array_equal(_np(q), qo) and np.array_equal(_np(s), so)


# ---- a3: int32 accumulators -----------------------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (17, 256, 192), (100, 640, 1280), (257, 1280, 5120),
                                   (3000, 5120, 1280), (3000, 1280, 5120)])
def test_gemm_i32_bit_exact(ext, M, N, K):
    from kernels.cuda_ext import EPI_I32

    print(f"gemm_i8 I32 M={M} N={N} K={K}", flush=True)
    _, xq, xs, wq, ws, b = _prep(M, N, K, seed=1)
    acc = torch.empty(M, N, dtype=torch.int32, device="cuda")
    ext.gemm_i8(xq, xs, K, wq, ws, b, acc, EPI_I32, None, 1.0, None, -1)
    assert np.array_equal(_np(acc), _int_mm_cpu(xq, wq))


def test_gemm_every_tile_same_bits(ext):
    """Batch/tile invariance (reference gemm_int8.cu:8-10): every gfx950 tile gives the same accumulators and bf16."""
    from kernels.cuda_ext import EPI_BIAS, EPI_I32

    M, N, K = 300, 512, 1280
    _, xq, xs, wq, ws, b = _prep(M, N, K, seed=2)
    ref_acc = _int_mm_cpu(xq, wq)
    ref_out = O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b), O.EPI_BIAS)
    n_tiles = ext.set_gemm_tile(-1)
    for tile in range(n_tiles):
        print(f"tile {tile}", flush=True)
        ext.set_gemm_tile(tile)
        acc = torch.zeros(M, N, dtype=torch.int32, device="cuda")
        ext.gemm_i8(xq, xs, K, wq, ws, b, acc, EPI_I32, None, 1.0, None, -1)
        out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        ext.gemm_i8(xq, xs, K, wq, ws, b, out, EPI_BIAS, None, 1.0, None, -1)
        torch.cuda.synchronize()
        assert np.array_equal(_np(acc), ref_acc), f"tile {tile}"
        assert np.array_equal(bf16_bits(out), ref_out), f"tile {tile}"
    ext.set_gemm_tile(-1)


def test_every_tile_epilogues_match_checker(ext):
    """Every gfx950 tile (tile shapes 64 to 256 channels wide, 16x16 and 32x32 instructions) stages its epilogue
    through LDS with its own row swizzle: RESID, GLU and SILU_Q8 (64-column groups, so every tile holds whole
    groups) against the checker at each tile."""
    from kernels.cuda_ext import EPI_GLU, EPI_RESID, EPI_SILU_Q8

    M, N, K = 200, 512, 640
    _, xq, xs, wq, ws, b = _prep(M, N, K, seed=41)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    args = (_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b))
    want_res = O.gemm_i8(*args, O.EPI_RESID, resid=bf16_bits(r), alpha=0.5)
    want_glu = O.gemm_i8(*args, O.EPI_GLU)
    want_q, want_qs = O.gemm_i8(*args, O.EPI_SILU_Q8, qgroup=64)
    n_tiles = ext.set_gemm_tile(-1)
    try:
        for tile in range(n_tiles):
            print(f"epilogues tile {tile}", flush=True)
            ext.set_gemm_tile(tile)
            res = r.cuda()
            ext.gemm_i8(xq, xs, K, wq, ws, b, res, EPI_RESID, res, 0.5, None, 0)
            glu = torch.empty(M, N // 2, dtype=torch.bfloat16, device="cuda")
            ext.gemm_i8(xq, xs, K, wq, ws, b, glu, EPI_GLU, None, 1.0, None, 0)
            q = torch.empty(M, N, dtype=torch.int8, device="cuda")
            qs = torch.empty(M, N // 64, dtype=torch.float32, device="cuda")
            ext.gemm_i8(xq, xs, K, wq, ws, b, q, EPI_SILU_Q8, None, 1.0, qs, 5)
            torch.cuda.synchronize()
            assert np.array_equal(bf16_bits(res), want_res), f"tile {tile}"
            assert_bf16_close(bf16_bits(glu), want_glu)
            dq = np.abs(_np(q).astype(np.int32) - want_q.astype(np.int32))
            assert dq.max() <= 1 and (dq != 0).mean() < 1e-2, f"tile {tile}"
            assert np.allclose(_np(qs), want_qs, rtol=2.0 ** -7, atol=0), f"tile {tile}"
    finally:
        ext.set_gemm_tile(-1)


# ---- a3 / a4: epilogues ---------------------------------------------------------------------------------------------

# 12032 rows: config 4's encoder call (32 clips of 376 frames in one call), the largest M the pipeline runs
@pytest.mark.parametrize("M,N,K", [(3000, 5120, 1280), (3000, 1280, 5120), (45, 3840, 1280), (12032, 5120, 1280)])
def test_gemm_bias_bit_exact(ext, M, N, K):
    from kernels.cuda_ext import EPI_BIAS

    print(f"gemm_i8 BIAS M={M} N={N} K={K}", flush=True)
    _, xq, xs, wq, ws, b = _prep(M, N, K, seed=3)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ext.gemm_i8(xq, xs, K, wq, ws, b, out, EPI_BIAS, None, 1.0, None, 0)
    want = O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b), O.EPI_BIAS)
    got = bf16_bits(out)
    assert rel_err(bf16_float(got), bf16_float(want)) <= 1e-2
    assert np.array_equal(got, want)
    # no bias: fmul instead of fmaf
    ext.gemm_i8(xq, xs, K, wq, ws, None, out, EPI_BIAS, None, 1.0, None, 0)
    assert np.array_equal(bf16_bits(out), O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), None, O.EPI_BIAS))


@pytest.mark.parametrize("alpha", [1.0, 0.5])
def test_gemm_resid_in_place(ext, alpha):
    from kernels.cuda_ext import EPI_RESID

    M, N, K = 700, 1280, 1280
    _, xq, xs, wq, ws, b = _prep(M, N, K, seed=4)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    x = r.cuda()
    ext.gemm_i8(xq, xs, K, wq, ws, b, x, EPI_RESID, x, alpha, None, 0)  # out aliases resid
    want = O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b), O.EPI_RESID, resid=bf16_bits(r), alpha=alpha)
    assert np.array_equal(bf16_bits(x), want)


def test_gemm_glu(ext):
    from kernels.cuda_ext import EPI_GLU

    M, N, K = 1000, 2560, 1280
    _, xq, xs, wq, ws, b = _prep(M, N, K, seed=6)
    out = torch.empty(M, N // 2, dtype=torch.bfloat16, device="cuda")
    ext.gemm_i8(xq, xs, K, wq, ws, b, out, EPI_GLU, None, 1.0, None, 0)
    want = O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b), O.EPI_GLU)
    assert_bf16_close(bf16_bits(out), want)  # the sigmoid's exp differs from libm's: rare one-ulp flips


@pytest.mark.parametrize("cfg,group", [(4, 256), (0, 128), (5, 64), (-1, 256)])
def test_gemm_silu_q8(ext, cfg, group):
    from kernels.cuda_ext import EPI_SILU_Q8

    M, N, K = 600, 5120, 1280
    _, xq, xs, wq, ws, b = _prep(M, N, K, seed=7)
    q = torch.empty(M, N, dtype=torch.int8, device="cuda")
    qs = torch.empty(M, N // group, dtype=torch.float32, device="cuda")
    ext.gemm_i8(xq, xs, K, wq, ws, b, q, EPI_SILU_Q8, None, 1.0, qs, cfg)
    qo, qso = O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b), O.EPI_SILU_Q8, qgroup=group)
    dq = np.abs(_np(q).astype(np.int32) - qo.astype(np.int32))
    assert dq.max() <= 1 and (dq != 0).mean() < 1e-2
    assert np.allclose(_np(qs), qso, rtol=2.0 ** -7, atol=0)


# ---- a5: grouped scales (the feed-forward's second GEMM) ----------------------------------------------------------

def test_ffn_grouped_chain(ext):
    """FF1 SILU_Q8 (256-column groups) -> FF2 grouped RESID alpha 0.5, as encoder_loop.cpp:65-71 chains them."""
    from kernels.cuda_ext import EPI_RESID, EPI_SILU_Q8

    M, D, F = 1500, 1280, 5120
    _, xq, xs, w1, s1, b1 = _prep(M, F, D, seed=8)
    _, w2_, _ = linear_inputs(1, D, F, seed=9)
    from kernels.fast_encoder import quantize_rows

    w2, s2 = (t.cuda() for t in quantize_rows(w2_))
    b2 = (torch.randn(D, generator=torch.Generator().manual_seed(10)) * 0.01).to(torch.bfloat16).cuda()
    tq = torch.empty(M, F, dtype=torch.int8, device="cuda")
    ts = torch.empty(M, F // 256, dtype=torch.float32, device="cuda")
    ext.gemm_i8(xq, xs, D, w1, s1, b1, tq, EPI_SILU_Q8, None, 1.0, ts, 4)
    r = torch.randn(M, D, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    x = r.cuda()
    ext.gemm_i8(tq, ts, 256, w2, s2, b2, x, EPI_RESID, x, 0.5, None, 10)
    # the second GEMM checked on the GPU's own int8 input (the first is checked in test_gemm_silu_q8)
    want = O.gemm_i8(_np(tq), _np(ts), 256, _np(w2), _np(s2), bf16_bits(b2), O.EPI_RESID, resid=bf16_bits(r),
                     alpha=0.5)
    assert np.array_equal(bf16_bits(x), want)


# ---- a8: 2:4 sparse -------------------------------------------------------------------------------------------------

def _sparse_weights(N, K, seed):
    from kernels.fast_encoder import quantize_rows
    from kernels.sparse import compress_24, prune_24_magnitude

    _, w, b = linear_inputs(1, N, K, seed=seed)
    wq, ws = quantize_rows(prune_24_magnitude(w))
    wc, e = compress_24(wq)
    return wq.cuda(), ws.cuda(), wc.cuda(), e.cuda(), b.cuda()


@pytest.mark.parametrize("M,N,K,group", [(3000, 5120, 1280, 1280), (3000, 1280, 5120, 5120), (3000, 1280, 5120, 256),
                                         (5, 256, 128, 128), (130, 640, 1024, 512), (12032, 1280, 5120, 256)])
def test_sparse_equals_dense_on_pruned(ext, M, N, K, group):
    from kernels.cuda_ext import EPI_BIAS, EPI_I32, EPI_RESID

    print(f"gemm_sp M={M} N={N} K={K} group={group}", flush=True)
    x, _, _ = linear_inputs(M, 64, K, seed=12)
    xq = torch.empty(M, K, dtype=torch.int8)
    xs = torch.empty(M, K // group, dtype=torch.float32)
    for g in range(K // group):  # per (row, group) scales as the FF1 epilogue writes them
        qg, sg = O.q8_rows(bf16_bits(x[:, g * group:(g + 1) * group]))
        xq[:, g * group:(g + 1) * group] = torch.from_numpy(qg)
        xs[:, g] = torch.from_numpy(sg)
    xq, xs = xq.cuda(), xs.cuda()
    wq, ws, wc, e, b = _sparse_weights(N, K, seed=13)
    if group == K:
        acc_s = torch.empty(M, N, dtype=torch.int32, device="cuda")
        ext.gemm_sp_epi(xq, xs, group, wc, e, ws, b, acc_s, EPI_I32, None, 1.0, None, -1)
        assert np.array_equal(_np(acc_s), _int_mm_cpu(xq, wq))
        out_s = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        out_d = torch.empty_like(out_s)
        ext.gemm_sp_epi(xq, xs, group, wc, e, ws, b, out_s, EPI_BIAS, None, 1.0, None, -1)
        ext.gemm_i8(xq, xs, group, wq, ws, b, out_d, EPI_BIAS, None, 1.0, None, -1)
        assert torch.equal(out_s, out_d)
        want = O.gemm_i8(_np(xq), _np(xs), group, _np(wq), _np(ws), bf16_bits(b), O.EPI_BIAS)
        assert np.array_equal(bf16_bits(out_s), want)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16).cuda()
    xs_, xd_ = r.clone(), r.clone()
    ext.gemm_sp(xq, xs, group, wc, e, ws, b, xs_, xs_, 0.5, 0)  # the reference's signature: RESID in place
    ext.gemm_i8(xq, xs, group, wq, ws, b, xd_, EPI_RESID, xd_, 0.5, None, -1)
    assert torch.equal(xs_, xd_)


@pytest.mark.parametrize("M,K", [(300, 1280), (300, 1152), (129, 128), (64, 256), (200, 384), (1000, 5120),
                                 (300, 4992)])
def test_sparse_every_tile_same_bits(ext, M, K):
    """Every gfx950 tile of the 2:4 kernel (the in-workgroup K split among them) gives the int32 sums of the dense
    product on the pruned weights, and the bias and residual epilogues' bits; K of 1 to 40 stages, odd and even."""
    from kernels.cuda_ext import EPI_BIAS, EPI_I32, EPI_RESID

    N = 256 if K > 4096 else 512
    _, xq, xs, _, _, _ = _prep(M, N, K, seed=21 + K)
    wq, ws, wc, e, b = _sparse_weights(N, K, seed=22 + M)
    ref_acc = _int_mm_cpu(xq, wq)
    ref_out = O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b.cpu()), O.EPI_BIAS)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(23)).to(torch.bfloat16).cuda()
    ref_res = O.gemm_i8(_np(xq), _np(xs), K, _np(wq), _np(ws), bf16_bits(b.cpu()), O.EPI_RESID, resid=bf16_bits(r.cpu()),
                        alpha=0.5)
    n_tiles = ext.set_gemm_tile(-1)
    try:
        for tile in range(n_tiles):
            print(f"gemm_sp tile {tile} M={M} K={K}", flush=True)
            ext.set_gemm_tile(tile)
            acc = torch.zeros(M, N, dtype=torch.int32, device="cuda")
            ext.gemm_sp_epi(xq, xs, K, wc, e, ws, b, acc, EPI_I32, None, 1.0, None, -1)
            out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
            ext.gemm_sp_epi(xq, xs, K, wc, e, ws, b, out, EPI_BIAS, None, 1.0, None, -1)
            res = r.clone()
            ext.gemm_sp_epi(xq, xs, K, wc, e, ws, b, res, EPI_RESID, res, 0.5, None, -1)
            torch.cuda.synchronize()
            assert np.array_equal(_np(acc), ref_acc), f"tile {tile}"
            assert np.array_equal(bf16_bits(out), ref_out), f"tile {tile}"
            assert np.array_equal(bf16_bits(res), ref_res), f"tile {tile}"
    finally:
        ext.set_gemm_tile(-1)


def test_sparse_silu_q8_equals_dense(ext):
    from kernels.cuda_ext import EPI_SILU_Q8

    M, N, K = 400, 5120, 1280
    _, xq, xs, _, _, _ = _prep(M, N, K, seed=15)
    wq, ws, wc, e, b = _sparse_weights(N, K, seed=16)
    outs = []
    for sparse in (True, False):
        q = torch.empty(M, N, dtype=torch.int8, device="cuda")
        qs = torch.empty(M, N // 256, dtype=torch.float32, device="cuda")
        if sparse:
            ext.gemm_sp_epi(xq, xs, K, wc, e, ws, b, q, EPI_SILU_Q8, None, 1.0, qs, -1)
        else:
            ext.gemm_i8(xq, xs, K, wq, ws, b, q, EPI_SILU_Q8, None, 1.0, qs, 4)
        outs.append((q, qs))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("M,N,K,group", [(3000, 5120, 1280, 1280), (3000, 1280, 5120, 5120), (3000, 1280, 5120, 256),
                                         (37, 512, 384, 128)])
def test_sparse_tiled_layout_same_bits(ext, M, N, K, group):
    """gemm_sp_tiled on pack_24_tiled's layout gives the bits of gemm_sp_epi on compress_24's, for every epilogue
    (int32 sums, BIAS, RESID in place, GLU, SILU_Q8) and, on the small shape, for every gfx950 tile."""
    from kernels.cuda_ext import EPI_BIAS, EPI_GLU, EPI_I32, EPI_RESID, EPI_SILU_Q8
    from kernels.sparse import pack_24_tiled

    print(f"gemm_sp_tiled M={M} N={N} K={K} group={group}", flush=True)
    _, xq, _, _, _, _ = _prep(M, 64, K, seed=31)
    xs = (torch.rand(M, K // group, generator=torch.Generator().manual_seed(32)) * 0.02 + 0.001).cuda()
    wq, ws, wc, e, b = _sparse_weights(N, K, seed=33)
    wt = pack_24_tiled(wc, e)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(34)).to(torch.bfloat16).cuda()

    def both(epi, dtype, width, qs_cols=0):
        outs = []
        for tiled in (False, True):
            out = (r[:, :width].clone() if epi == EPI_RESID else torch.empty(M, width, dtype=dtype, device="cuda"))
            qs = torch.empty(M, qs_cols, dtype=torch.float32, device="cuda") if qs_cols else None
            resid = out if epi == EPI_RESID else None
            if tiled:
                ext.gemm_sp_tiled(xq, xs, group, wt, ws, b, out, epi, resid, 0.5, qs, -1)
            else:
                ext.gemm_sp_epi(xq, xs, group, wc, e, ws, b, out, epi, resid, 0.5, qs, -1)
            outs.append((out, qs))
        torch.cuda.synchronize()
        raw = lambda t: t.view(torch.int16) if t.dtype == torch.bfloat16 else t  # noqa: E731
        assert torch.equal(raw(outs[0][0]), raw(outs[1][0])), epi
        if qs_cols:
            assert torch.equal(outs[0][1], outs[1][1]), epi

    tiles = range(ext.set_gemm_tile(-1)) if M < 100 else [-1]
    try:
        for tile in tiles:
            ext.set_gemm_tile(tile)
            if group == K:
                both(EPI_I32, torch.int32, N)
            both(EPI_BIAS, torch.bfloat16, N)
            both(EPI_RESID, torch.bfloat16, N)
            both(EPI_GLU, torch.bfloat16, N // 2)
            if N % 256 == 0:
                both(EPI_SILU_Q8, torch.int8, N, N // 256)
    finally:
        ext.set_gemm_tile(-1)


def test_empty_rows_noop(ext):
    from kernels.cuda_ext import EPI_BIAS

    xq = torch.empty(0, 128, dtype=torch.int8, device="cuda")
    xs = torch.empty(0, 1, dtype=torch.float32, device="cuda")
    wq = torch.zeros(64, 128, dtype=torch.int8, device="cuda")
    out = torch.empty(0, 64, dtype=torch.bfloat16, device="cuda")
    ext.gemm_i8(xq, xs, 128, wq, torch.ones(64, device="cuda"), None, out, EPI_BIAS, None, 1.0, None, 0)
    torch.cuda.synchronize()
