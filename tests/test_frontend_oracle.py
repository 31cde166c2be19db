"""The checker's front end (log-mel features, subsampling convolutions, bf16 GEMM) pinned against transformers'
own implementations and exact cases. CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from frontend_helpers import (bands, hf_extractor, hf_stem, make_subsampling, oracle_stem, slaney_filters,
                              stem_weights, synthetic_audio, window512)
from helpers import bf16_bits, bf16_float, bf16_ulp


def test_slaney_filters_match_transformers():
    """kernels/features.py's restatement of librosa's Slaney filter bank against transformers' independent
    mel_filter_bank (same scale and normalization): equal to fp32 rounding, every band nonempty."""
    from transformers.audio_utils import mel_filter_bank

    mine = slaney_filters().numpy()
    hf = mel_filter_bank(num_frequency_bins=257, num_mel_filters=128, min_frequency=0.0, max_frequency=8000.0,
                         sampling_rate=16000, norm="slaney", mel_scale="slaney").T
    assert mine.shape == (128, 257) and mine.dtype == np.float32
    assert np.abs(mine - hf).max() <= 4 * np.finfo(np.float32).eps * np.abs(hf).max()
    assert ((mine != 0).sum(1) >= 1).all()
    # the triangles: each band rises then falls (one peak), bands in increasing frequency
    peaks = mine.argmax(1)
    assert (np.diff(peaks) >= 0).all()


def test_dither_matches_extractor():
    from kernels.features import dither

    x = np.linspace(-1, 1, 1234, dtype=np.float32)
    fe = hf_extractor()
    got = dither(x)
    want = fe._apply_dither(torch.from_numpy(x.copy())[None], torch.tensor([len(x)]))[0].numpy()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("lengths", [[16000 * 3 + 77, 8000, 1000], [480000], [160 * 7, 161, 319]])
def test_logmel_matches_transformers_extractor(lengths):
    """The checker's features against CohereAsrFeatureExtractor.__call__ (dither, pre-emphasis, torch.stft, the
    filter bank, log, per-feature normalization) on the same pieces: the valid frames within one bf16 step of the
    extractor's fp32 values rounded to bf16, at most 0.5 % of them a step away; frames past the valid ones zero."""
    from kernels.features import dither

    xs = synthetic_audio(lengths, seed=len(lengths))
    fe = hf_extractor()
    hf = fe(xs, sampling_rate=16000, return_tensors="pt")["input_features"].numpy()
    mel = fe.mel_filters.numpy()
    got = oracle.logmel(np.concatenate([dither(x) for x in xs]), lengths, window512(), mel, bands(mel), 0.97)
    gf = bf16_float(got)
    assert got.shape == (len(lengths), max(lengths) // 160 + 1, 128)
    for i, n in enumerate(lengths):
        v = n // 160
        want = hf[i, :v]
        want_b = bf16_float(oracle.f32_to_bf16(want))
        # one valid frame: the unbiased variance divides by zero, NaN in both (as the reference)
        assert np.array_equal(np.isnan(gf[i, :v]), np.isnan(want_b))
        diff = np.nan_to_num(np.abs(gf[i, :v] - want_b))
        # one bf16 step, or 1e-4 absolute where a value near zero is a difference of nearly equal logs
        tol = np.maximum(np.maximum(bf16_ulp(want), bf16_ulp(gf[i, :v])) * 1.0001, 1e-4)
        assert (diff <= tol).all(), float(diff.max())
        assert (diff > 0).mean() <= 5e-3
        assert (got[i, v:] == 0).all()


def test_stem_matches_transformers_subsampling():
    """The checker's stem (conv0 + dw, pointwise GEMM, dw, pointwise GEMM, linear) against transformers'
    ParakeetEncoderSubsamplingConv2D in float32 on ragged pieces, each run on its own: within the bf16 roundings the
    kernels make between the convolutions (RMS 1e-2, max 5e-2 of the output RMS); lengths as the model's."""
    sub = make_subsampling()
    W = stem_weights(sub)
    g = torch.Generator().manual_seed(5)
    frames = [301, 57, 9, 1]
    feats = torch.zeros(len(frames), max(frames), 128)
    for i, n in enumerate(frames):
        feats[i, :n] = torch.randn(n, 128, generator=g)
    fb = feats.to(torch.bfloat16)
    got, t3 = oracle_stem(W, bf16_bits(fb), frames)
    want = hf_stem(sub, fb.float(), frames).numpy().astype(np.float64)
    assert t3 == [38, 8, 2, 1] and got.shape == (sum(t3), 1280)
    gf = bf16_float(got).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    d = np.abs(gf - want)
    assert np.sqrt(np.mean(d ** 2)) <= 1e-2 * rms and d.max() <= 5e-2 * rms


def test_sub_dw_against_torch_conv():
    """The depthwise stride-2 convolution per sequence against torch's conv2d (groups = channels) in float64: within
    one bf16 rounding."""
    g = torch.Generator().manual_seed(9)
    C, F_in = 64, 32
    t_in = [7, 1, 12]
    x = torch.randn(sum(t_in), F_in, C, generator=g).to(torch.bfloat16)
    w = torch.randn(C, 9, generator=g) * 0.3
    b = torch.randn(C, generator=g) * 0.1
    t_out = [(t - 1) // 2 + 1 for t in t_in]
    rows = np.array([(i, t) for i, n in enumerate(t_out) for t in range(n)], np.int32)
    starts = np.concatenate([[0], np.cumsum(t_in)[:-1]]).astype(np.int32)
    got = bf16_float(oracle.sub_dw(bf16_bits(x), starts, np.asarray(t_in, np.int32), rows, w.numpy(), b.numpy()))
    want = []
    for s, n in zip(starts, t_in):
        xi = x[s:s + n].double().permute(2, 0, 1)[None]  # (1, C, T, F)
        y = torch.nn.functional.conv2d(xi, w.double().view(C, 1, 3, 3), b.double(), stride=2, padding=1, groups=C)
        want.append(y[0].permute(1, 2, 0).numpy())
    want = np.concatenate(want)
    assert np.all(np.abs(got - want) <= bf16_ulp(want) * 0.5 + 1e-6)


def test_sub_conv0_dw_against_torch_conv():
    """conv0 + bias + ReLU then the depthwise convolution, against torch's conv2d in float64 with the same two
    roundings of conv0's output (sum, then sum + bias): within one bf16 rounding of the output."""
    g = torch.Generator().manual_seed(10)
    C, frames = 64, [13, 4]
    feats = torch.randn(len(frames), max(frames), 128, generator=g).to(torch.bfloat16)
    w0, b0 = torch.randn(C, 9, generator=g) * 0.3, torch.randn(C, generator=g) * 0.1
    w2, b2 = torch.randn(C, 9, generator=g) * 0.3, torch.randn(C, generator=g) * 0.1
    t2 = [((t - 1) // 2) // 2 + 1 for t in frames]
    rows = np.array([(i, t) for i, n in enumerate(t2) for t in range(n)], np.int32)
    got = bf16_float(oracle.sub_conv0_dw(bf16_bits(feats), np.asarray(frames, np.int32), rows, w0.numpy(), b0.numpy(),
                                         w2.numpy(), b2.numpy()))
    want = []
    for i, n in enumerate(frames):
        xi = feats[i:i + 1, :n].double()[None]  # (1, 1, T, 128)
        c0 = torch.nn.functional.conv2d(xi, w0.double().view(C, 1, 3, 3), None, stride=2, padding=1)
        c0 = c0.float().to(torch.bfloat16).float()
        c0 = torch.relu((c0 + b0.view(1, C, 1, 1)).to(torch.bfloat16).float()).double()
        y = torch.nn.functional.conv2d(c0, w2.double().view(C, 1, 3, 3), b2.double(), stride=2, padding=1, groups=C)
        want.append(y[0].permute(1, 2, 0).numpy())
    want = np.concatenate(want)
    assert got.shape == want.shape
    # conv0's fp32 sum differs from the float64 one by an ulp now and then, moving its bf16 rounding: rare
    close = np.abs(got - want) <= bf16_ulp(want) * 0.5 + 1e-6
    assert close.mean() >= 0.999


@pytest.mark.parametrize("epi", [oracle.EPI_BIAS, oracle.EPI_SILU, oracle.EPI_RELU, oracle.EPI_RESID, oracle.EPI_GLU,
                                 oracle.EPI_CONV_RELU])
def test_gemm_bf16_exact_cases(epi):
    """Small-integer bf16 operands: products and sums are exact, so the accumulator is numpy's int64 matmul and
    each epilogue is its closed form on it."""
    rng = np.random.default_rng(epi)
    M, N, K = 7, 64, 96
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    w = rng.integers(-4, 5, (N, K)).astype(np.float32)
    b = (rng.integers(-8, 9, N) / 4).astype(np.float32)
    r = (rng.integers(-8, 9, (M, N)) / 8).astype(np.float32)
    h = lambda f: oracle.f32_to_bf16(f)  # noqa: E731
    got = bf16_float(oracle.gemm_bf16(h(a), h(w), h(b), epi, resid=h(r), alpha=0.5))
    acc = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.float64)
    rb = lambda v: bf16_float(oracle.f32_to_bf16(np.asarray(v, np.float32))).astype(np.float64)  # noqa: E731
    sig = lambda v: 1 / (1 + np.exp(-v))  # noqa: E731
    v = acc + b
    if epi == oracle.EPI_BIAS:
        want = rb(v)
    elif epi == oracle.EPI_SILU:
        want = rb(rb(v) * sig(rb(v)))
    elif epi == oracle.EPI_RELU:
        want = rb(np.maximum(v, 0))
    elif epi == oracle.EPI_CONV_RELU:
        want = rb(np.maximum(rb(acc) + b, 0))
    elif epi == oracle.EPI_RESID:
        want = rb(0.5 * rb(v) + r)
    else:
        want = rb(rb(v[:, 0::2]) * sig(rb(v[:, 1::2])))
    # the logistic in fp32 against float64: one bf16 step (and nothing meaningful below 1e-20, where it underflows)
    tol = np.maximum(bf16_ulp(want) * 1.0001, 1e-20) if epi in (oracle.EPI_SILU, oracle.EPI_GLU) else 0
    assert np.all(np.abs(got - want) <= tol)
