"""GPU parity of the encoder layer's kernels (LayerNorm, depthwise conv + BN + SiLU, relative-position attention) and
of the native int8 layer loop against the CPU checker, through the C ABI (kernels.cuda_ext.ext)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from encoder_helpers import oracle_layer_fields, product_layers
from helpers import assert_bf16_close, bf16_bits, bf16_float, bf16_ulp

pytestmark = pytest.mark.gpu


def _ext():
    from kernels.cuda_ext import ext

    return ext


def _bits(t):
    return bf16_bits(t)


def _close_to_checker(got_bits, want_bits, rms_tol=2e-3, max_tol=1e-2, frac_beyond=0.0):
    """Kernels that sum in another fp32 order than the checker: every element (but frac_beyond of them) within
    max-abs max_tol x RMS of the checker, or one bf16 ulp of the value where that is larger, and all within 5x that;
    RMS difference below rms_tol x RMS."""
    got, want = bf16_float(got_bits).astype(np.float64), bf16_float(want_bits).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    diff = np.abs(got - want)
    print(f"checker: rms diff {np.sqrt(np.mean(diff ** 2)) / rms:.2e} x RMS, max {diff.max() / rms:.2e} x RMS, "
          f"{(diff > 1e-2 * rms).mean():.2e} of elements beyond 1e-2 x RMS")
    tol = np.maximum(max_tol * rms, bf16_ulp(want) * 1.0001)
    assert (diff <= tol).mean() >= 1 - frac_beyond, f"{int((diff > tol).sum())} beyond tolerance"
    assert (diff <= np.maximum(5 * max_tol * rms, tol)).all(), f"worst {(diff / tol).max():.2f} x tolerance"
    assert np.sqrt(np.mean(diff ** 2)) <= rms_tol * rms, np.sqrt(np.mean(diff ** 2)) / rms


def _packed(lengths):
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    lo = np.concatenate([np.full(n, s) for s, n in zip(starts, lengths)]).astype(np.int32)
    hi = np.concatenate([np.full(n, s + n) for s, n in zip(starts, lengths)]).astype(np.int32)
    return lo, hi


@pytest.mark.parametrize("two", [False, True])
def test_layernorm_bf16(gpu, two):
    g = torch.Generator().manual_seed(21)
    rows, cols = 517, 1280
    x = (torch.randn(rows, cols, generator=g) * 2 + 0.3).to(torch.bfloat16)
    w1, b1, w2, b2 = ((1 + 0.2 * torch.randn(cols, generator=g)).to(torch.bfloat16) for _ in range(4))
    xd = x.to(gpu)
    h = torch.empty_like(xd)
    _ext().layernorm(xd, w1.to(gpu), b1.to(gpu), 1e-5, w2.to(gpu) if two else None, b2.to(gpu) if two else None,
                     1e-6, h)
    want_h, want_x = oracle.layernorm(_bits(x), _bits(w1), _bits(b1), 1e-5, _bits(w2) if two else None,
                                      _bits(b2) if two else None, 1e-6)
    assert_bf16_close(_bits(h), want_h)
    assert_bf16_close(_bits(xd), want_x)
    # in place: h is x
    xd2 = x.to(gpu)
    _ext().layernorm(xd2, w1.to(gpu), b1.to(gpu), 1e-5, None, None, 0.0, xd2)
    assert_bf16_close(_bits(xd2), oracle.layernorm(_bits(x), _bits(w1), _bits(b1), 1e-5)[0])


def _dwconv_inputs(lengths, C=1280, seed=22):
    g = torch.Generator().manual_seed(seed)
    rows = sum(lengths)
    x = torch.randn(rows, C, generator=g).to(torch.bfloat16)
    w = 0.3 * torch.randn(C, 9, generator=g)
    cb, sc, sh = 0.1 * torch.randn(C, generator=g), 1 + 0.2 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
    lo, hi = _packed(lengths)
    return x, w, cb, sc, sh, lo, hi


@pytest.mark.parametrize("lengths,C", [([375, 200, 1, 64, 97], 1280), ([3], 1280), ([8, 9], 1280),
                                      ([5, 130, 2], 2048), ([7, 1, 40], 8), ([33, 4], 520)])
def test_dwconv_bn_silu_bf16_and_q8(gpu, lengths, C):
    x, w, cb, sc, sh, lo, hi = _dwconv_inputs(lengths, C=C)
    d = lambda t: t.to(gpu).contiguous()  # noqa: E731
    lo_d, hi_d = d(torch.from_numpy(lo)), d(torch.from_numpy(hi))
    y = torch.empty_like(d(x))
    _ext().dwconv_bn_silu(d(x), d(w), d(cb), d(sc), d(sh), lo_d, hi_d, y)
    args = (_bits(x), w.numpy(), cb.numpy(), sc.numpy(), sh.numpy(), lo, hi)
    want = oracle.dwconv_bn_silu(*args)
    # the kernel's logistic uses the hardware exp/reciprocal: a rounding flip of the bf16 output now and then
    assert_bf16_close(_bits(y), want)
    hq = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    hs = torch.empty(x.shape[0], dtype=torch.float32, device=gpu)
    _ext().dwconv_bn_silu_q8(d(x), d(w), d(cb), d(sc), d(sh), lo_d, hi_d, hq, hs)
    # exactly quantize_rows of the kernel's own bf16 rows
    q_ref, s_ref = oracle.q8_rows(_bits(y))
    assert np.array_equal(hq.cpu().numpy(), q_ref) and np.array_equal(hs.cpu().numpy(), s_ref)
    # and within one step of the checker's
    q_or, s_or = oracle.q8_rows(want)
    assert np.abs(hq.cpu().numpy().astype(int) - q_or).max() <= 1
    assert np.allclose(hs.cpu().numpy(), s_or, rtol=1e-2)


def _attention_case(lengths, H, D, seed, max_len=512):
    g = torch.Generator().manual_seed(seed)
    rows = sum(lengths)
    qkv = torch.randn(rows, 3 * H * D, generator=g).to(torch.bfloat16)
    rel_rows = 2 * max_len - 1 + 64
    rk = (0.5 * torch.randn(rel_rows, H * D, generator=g)).to(torch.bfloat16)
    bu = (0.2 * torch.randn(H, D, generator=g)).to(torch.bfloat16)
    bv = (0.2 * torch.randn(H, D, generator=g)).to(torch.bfloat16)
    return qkv, rk, bu, bv


@pytest.mark.parametrize("H,D,lengths", [(8, 160, [375, 200, 64, 1, 97]), (16, 80, [375, 33, 130]),
                                         (16, 80, [512]), (8, 160, [2, 65]), (16, 80, [1, 32, 31, 64, 96, 33])])
def test_relpos_attention(gpu, H, D, lengths):
    from kernels.fast_encoder import metadata

    qkv, rk, bu, bv = _attention_case(lengths, H, D, seed=len(lengths) * 7 + D)
    meta = metadata(lengths, gpu)
    out = torch.empty(sum(lengths), H * D, dtype=torch.bfloat16, device=gpu)
    scale = D ** -0.5
    _ext().relpos_attention(qkv.to(gpu), rk.to(gpu), bu.to(gpu), bv.to(gpu), meta["tiles"], 511, meta["max_len"],
                            scale, out)
    want = oracle.relpos_attention(_bits(qkv), _bits(rk), _bits(bu), _bits(bv), lengths, 511, scale)
    _close_to_checker(_bits(out), want)


def test_relpos_attention_rejects_long_sequences(gpu):
    from kernels.fast_encoder import metadata

    qkv, rk, bu, bv = _attention_case([600], 8, 160, seed=1)
    meta = metadata([600], gpu)
    out = torch.empty(600, 1280, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="too long"):
        _ext().relpos_attention(qkv.to(gpu), rk.to(gpu), bu.to(gpu), bv.to(gpu), meta["tiles"], 511, 600, 0.1, out)


def _layers(gpu, n_layers, sparse, seed):
    return product_layers(gpu, n_layers, seed, sparse)


def _oracle_layers(layers):
    return oracle_layer_fields(layers)


def _diff_stats(got_bits, want_bits):
    got, want = bf16_float(got_bits).astype(np.float64), bf16_float(want_bits).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    d = np.abs(got - want)
    return np.sqrt(np.mean(d ** 2)) / rms, d.max() / rms


@pytest.mark.parametrize("n_layers,sparse,lengths", [(1, True, [120, 75]), (2, False, [64, 1, 90])])
def test_encoder_layers_int8(gpu, n_layers, sparse, lengths):
    """The native layer loop against the checker's restatement of it. A whole layer re-quantizes its activations to
    int8 five times, so a last-bit difference anywhere moves whole rows by 1/127 of their maximum: the checker itself
    moves by ~0.7 % RMS per layer when 1 % of its input elements change by one bf16 ulp. The bar: the kernels' result
    is closer to the checker than that perturbed checker is (RMS and max), and no more of its elements lie beyond
    1e-2 x RMS of the checker than of the perturbed checker's. (Config 2's workload, with each launch pinned
    separately and the drift per depth, is tests/test_encoder_config2_gpu.py.)"""
    layers = _layers(gpu, n_layers, sparse, seed=31)
    g = torch.Generator().manual_seed(32)
    x = torch.randn(sum(lengths), 1280, generator=g).to(torch.bfloat16)
    xd = x.to(gpu)
    layers(xd, lengths)
    fields = _oracle_layers(layers)
    eps = [layers.layer_eps[5 * i:5 * i + 5] for i in range(n_layers)]
    want = oracle.encoder_layers_int8(_bits(x), fields, eps, lengths, layers.rel_off, layers.scale)
    xb = _bits(x).copy()
    moved = np.random.default_rng(0).random(xb.shape) < 0.01
    xb[moved] += 1
    noise = oracle.encoder_layers_int8(xb, fields, eps, lengths, layers.rel_off, layers.scale)
    rms_gpu, max_gpu = _diff_stats(_bits(xd), want)
    rms_noise, max_noise = _diff_stats(noise, want)
    print(f"layers: kernels vs checker rms {rms_gpu:.2e} max {max_gpu:.2e}; perturbed checker rms {rms_noise:.2e} "
          f"max {max_noise:.2e}")
    assert rms_gpu < rms_noise and max_gpu < max_noise
    got_f, want_f, noise_f = bf16_float(_bits(xd)), bf16_float(want), bf16_float(noise)
    bar = 1e-2 * np.sqrt(np.mean(want_f.astype(np.float64) ** 2))
    beyond_gpu, beyond_noise = (np.abs(got_f - want_f) > bar).mean(), (np.abs(noise_f - want_f) > bar).mean()
    print(f"beyond 1e-2 x RMS: kernels {beyond_gpu:.4f}, perturbed checker {beyond_noise:.4f}")
    assert beyond_gpu <= beyond_noise


def test_encoder_layers_rejects_and_noops(gpu):
    from kernels.fast_encoder import metadata

    layers = _layers(gpu, 1, False, seed=40)
    x = torch.empty(0, 1280, dtype=torch.bfloat16, device=gpu)
    layers(x, [])  # no rows: nothing to do
    meta = metadata([10], gpu)
    # int8-converted layers hold no bf16 weights: the bf16 branch refuses them by name
    with pytest.raises(RuntimeError, match=r"bf16.*misses field"):
        _ext().encoder_layers(torch.zeros(10, 1280, dtype=torch.bfloat16, device=gpu), layers.layer_tensors,
                              layers.layer_eps, meta["tiles"], meta["lo"], meta["hi"], 511, 10, 0.1, False,
                              layers.configs(10))


def test_encoder_layers_bf16(gpu):
    """The native loop's bf16 branch (the reference's INT8=0 layers, encoder_loop.cpp:101-124) against the checker's
    restatement over two 16-head blocks. The only differences are the fp32 summation order of the GEMMs and the
    attention, but each is rounded to bf16 and carried through the LayerNorms of two blocks, so the bar is the chain's
    own sensitivity: RMS difference below, and largest difference within twice, what the checker moves when 1 % of its
    input elements move by one bf16 ulp (measured: 4.1e-3 / 6.2e-2 x RMS against 5.1e-3 / 6.2e-2)."""
    lengths = [200, 1, 97, 64]
    from encoder_helpers import make_block
    from kernels.fast_encoder import EncoderLayers

    blocks, inv = [], None
    for i in range(2):
        blk, inv = make_block(1280, 16, 5120, seed=51 + i)
        blocks.append(blk.to(device=gpu, dtype=torch.bfloat16))
    layers = EncoderLayers(blocks, inv, int8=False)
    assert all(ly.tensors["q_qkv_w"].numel() == 0 and ly.tensors["wqkv"].numel() for ly in layers.layers)
    g = torch.Generator().manual_seed(52)
    x = torch.randn(sum(lengths), 1280, generator=g).to(torch.bfloat16)
    xd = x.to(gpu)
    layers(xd, lengths)
    fields = _oracle_layers(layers)
    eps = [layers.layer_eps[5 * i:5 * i + 5] for i in range(2)]
    want = oracle.encoder_layers_bf16(_bits(x), fields, eps, lengths, layers.rel_off, layers.scale)
    xb = _bits(x).copy()
    xb[np.random.default_rng(0).random(xb.shape) < 0.01] += 1
    noise = oracle.encoder_layers_bf16(xb, fields, eps, lengths, layers.rel_off, layers.scale)
    rms_gpu, max_gpu = _diff_stats(_bits(xd), want)
    rms_noise, max_noise = _diff_stats(noise, want)
    print(f"bf16 layers: kernels vs checker rms {rms_gpu:.2e} max {max_gpu:.2e}; perturbed checker rms "
          f"{rms_noise:.2e} max {max_noise:.2e}")
    assert rms_gpu < rms_noise and max_gpu <= 2 * max_noise
