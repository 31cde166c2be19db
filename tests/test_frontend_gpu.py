"""GPU parity of the front end (bf16 GEMM, log-mel features, subsampling convolutions, FastEncoder) against the
CPU checker, through the C ABI (kernels.cuda_ext.ext) and the host mirrors (kernels.features, kernels.fast_encoder)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from frontend_helpers import (half, make_encoder, make_subsampling, oracle_stem, stem_rows, stem_weights,
                              synthetic_audio)
from helpers import assert_bf16_close, bf16_bits, bf16_float, bf16_ulp, from_bits

pytestmark = pytest.mark.gpu


def _ext():
    from kernels.cuda_ext import ext

    return ext


def _rms_close(got_bits, want_bits, rms_tol, max_tol):
    got, want = bf16_float(got_bits).astype(np.float64), bf16_float(want_bits).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    d = np.abs(got - want)
    print(f"rms diff {np.sqrt(np.mean(d ** 2)) / rms:.2e} x RMS, max {d.max() / rms:.2e} x RMS")
    assert np.sqrt(np.mean(d ** 2)) <= rms_tol * rms and d.max() <= max_tol * rms


EPIS = {"bias": 0, "silu": 1, "relu": 2, "resid": 3, "glu": 4, "conv_relu": 6}


@pytest.mark.parametrize("M,N,K", [(1000, 256, 256), (301, 1280, 4096), (77, 128, 96), (4099, 512, 256)])
@pytest.mark.parametrize("epi", list(EPIS))
def test_gemm_bf16(gpu, M, N, K, epi):
    """Every epilogue against the checker (fp32 accumulation in another order than its fp64 one: the bf16 bar of
    the other GEMMs); K % 64 == 32 exercises the half K tile; RESID runs in place (out is resid)."""
    g = torch.Generator().manual_seed(M + N + K + EPIS[epi])
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16)
    e = EPIS[epi]
    n_out = N // 2 if e == 4 else N
    ad, wd, bd = a.to(gpu), w.to(gpu), b.to(gpu)
    out = r.to(gpu).clone() if e == 3 else torch.empty(M, n_out, dtype=torch.bfloat16, device=gpu)
    _ext().gemm(ad, wd, bd, out, e, out if e == 3 else None, 0.5, 8)
    want = oracle.gemm_bf16(bf16_bits(a), bf16_bits(w), bf16_bits(b), e, resid=bf16_bits(r), alpha=0.5)
    if e in (1, 4, 6):
        # two roundings in a row: the activation reads bf16(v) (a flip of v moves t * sigmoid(t) by up to ~1.1 of
        # its own ulp near t = -1.3), CONV_RELU rounds the sum before adding the bias (a flip of the sum is an ulp of
        # the sum, larger than the result's where the bias cancels it): two ulps of the result or 1e-2 x RMS
        got_f, want_f = bf16_float(bf16_bits(out)).astype(np.float64), bf16_float(want).astype(np.float64)
        rms = np.sqrt(np.mean(want_f ** 2))
        assert (np.abs(got_f - want_f) <= np.maximum(1e-2 * rms, 2.0001 * bf16_ulp(want_f))).all()
        assert (bf16_bits(out) != want).mean() <= 0.02
    else:
        assert_bf16_close(bf16_bits(out), want, max_frac=0.02)


def test_gemm_bf16_strided_rows_and_no_bias(gpu):
    g = torch.Generator().manual_seed(3)
    big = torch.randn(200, 640, generator=g).to(torch.bfloat16)
    a = big[:, 64:64 + 256]  # row stride 640
    w = (torch.randn(128, 256, generator=g) * 0.06).to(torch.bfloat16)
    out = torch.empty(200, 128, dtype=torch.bfloat16, device=gpu)
    _ext().gemm(big.to(gpu)[:, 64:64 + 256], w.to(gpu), None, out, 0, None, 1.0, 3)
    want = oracle.gemm_bf16(bf16_bits(a.contiguous()), bf16_bits(w), None, 0)
    assert_bf16_close(bf16_bits(out), want)


def test_gemm_bf16_rejects(gpu):
    a = torch.zeros(10, 96, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(64, 96, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(10, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="unknown config"):
        _ext().gemm(a, w, None, out, 0, None, 1.0, 7)
    with pytest.raises(RuntimeError, match="N must be"):
        _ext().gemm(a, w[:48], None, out[:, :48], 0, None, 1.0, 8)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        _ext().gemm(a[:, :80], w[:, :80].contiguous(), None, out, 0, None, 1.0, 8)
    _ext().gemm(a[:0], w, None, out[:0], 0, None, 1.0, 8)  # no rows: nothing to do


@pytest.mark.parametrize("lengths", [[16000 * 3 + 77, 8000, 161, 100], [480000, 480000], [160 * 7]])
def test_logmel_features(gpu, lengths):
    """kernels.features.Features (the native call) against the checker on dithered synthetic audio: within one bf16
    step (or 1e-4 near zero) everywhere, at most 1 % of the values a step away; NaN exactly where the checker has it
    (a piece with one valid frame: the unbiased variance divides by zero, as the reference); pieces with no valid
    frame and the frames past the valid ones zero."""
    from kernels.features import Features, dither

    xs = [dither(x) for x in synthetic_audio(lengths, seed=sum(lengths) % 97)]
    fe = Features(device=gpu)
    feats, frames = fe(xs)
    assert frames == [n // 160 + 1 for n in lengths]
    got = bf16_bits(feats)
    want = oracle.logmel(np.concatenate(xs), lengths, fe.window512.cpu().numpy(), fe.mel.cpu().numpy(),
                         fe.band.cpu().numpy(), fe.preemphasis)
    assert got.shape == want.shape
    gf, wf = bf16_float(got), bf16_float(want)
    assert np.array_equal(np.isnan(gf), np.isnan(wf))
    diff = np.nan_to_num(np.abs(gf - wf))
    tol = np.maximum(np.maximum(bf16_ulp(wf), bf16_ulp(gf)) * 1.0001, 1e-4)
    assert (diff <= tol).all(), float(diff.max())
    assert (diff > 0).mean() <= 0.01
    # device-resident pieces take the same path
    feats2, _ = fe([torch.from_numpy(x).to(gpu) for x in xs])
    assert np.array_equal(bf16_bits(feats2), got)


def _stem_inputs(frames, seed):
    g = torch.Generator().manual_seed(seed)
    feats = torch.zeros(len(frames), max(frames), 128)
    for i, n in enumerate(frames):
        feats[i, :n] = torch.randn(n, 128, generator=g)
    return feats.to(torch.bfloat16)


@pytest.mark.parametrize("frames", [[301, 57, 9, 1], [3001]])
def test_subsampling_convolutions_bit_exact(gpu, frames):
    """sub_conv0_dw and sub_dw compute each output with the checker's own fp32 operation sequence: equal bit for
    bit (the dw input is the checker's own pointwise output, so the two kernels are checked on their own)."""
    sub = make_subsampling()
    W = stem_weights(sub)
    fb = _stem_inputs(frames, 11)
    C = W["channels"]
    t2 = half(half(frames))
    t3 = half(t2)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    a2 = torch.empty(sum(t2), 32, C, dtype=torch.bfloat16, device=gpu)
    _ext().sub_conv0_dw(fb.to(gpu), d(np.asarray(frames, np.int32)), d(stem_rows(t2)), d(W["w0"]), d(W["b0"]),
                        d(W["w2"]), d(W["b2"]), a2)
    want2 = oracle.sub_conv0_dw(bf16_bits(fb), np.asarray(frames, np.int32), stem_rows(t2), W["w0"], W["b0"], W["w2"],
                                W["b2"])
    assert np.array_equal(bf16_bits(a2), want2)
    a3 = oracle.gemm_bf16(want2.reshape(-1, C), W["pw3"], W["pw3_b"], oracle.EPI_CONV_RELU).reshape(-1, 32, C)
    starts = np.concatenate([[0], np.cumsum(t2)[:-1]]).astype(np.int32)
    a5 = torch.empty(sum(t3), 16, C, dtype=torch.bfloat16, device=gpu)
    _ext().sub_dw(from_bits(a3).to(gpu), d(starts), d(np.asarray(t2, np.int32)), d(stem_rows(t3)), d(W["w5"]),
                  d(W["b5"]), a5)
    want5 = oracle.sub_dw(a3, starts, np.asarray(t2, np.int32), stem_rows(t3), W["w5"], W["b5"])
    assert np.array_equal(bf16_bits(a5), want5)


def test_fast_encoder_subsample(gpu):
    """FastEncoder.subsample (native convolutions + bf16 GEMMs) against the checker's stem: the GEMMs sum in another
    order, so bf16 roundings move between the stages -- RMS 2e-3, max 2e-2 of the output RMS."""
    from kernels.fast_encoder import FastEncoder

    enc = make_encoder(1, seed=4, device="cpu")
    W = stem_weights(enc.subsampling)
    frames = [301, 57, 9, 1]
    fb = _stem_inputs(frames, 12)
    fast = FastEncoder(enc.to(device=gpu, dtype=torch.bfloat16), int8=True, sparse=True)
    x, t3 = fast.subsample(fb.to(gpu), frames)
    want, t3w = oracle_stem(W, bf16_bits(fb), frames)
    assert t3 == t3w
    _rms_close(bf16_bits(x), want, 2e-3, 2e-2)


def test_fast_encoder_rejects():
    from kernels.fast_encoder import FastEncoder

    enc = make_encoder(1, seed=4)
    with pytest.raises(ValueError, match="int8"):
        FastEncoder(enc, int8=False, sparse=True)
