"""Pins the CPU checker (oracle/) against things other than itself: the reference's own compress_24 output (golden
fixture), exact library routines (numpy int64 matmul, torch._int_mm, torch.round), closed forms and hand-made cases.
CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_bits, bf16_float, linear_inputs

GOLDEN = "tests/golden/compress24_golden.npz"


@pytest.fixture(scope="module")
def golden():
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    return np.load(os.path.join(root, GOLDEN))


# ---- a6 / a7: compress_24, prune_24 ---------------------------------------------------------------------------------

def test_compress24_golden(golden):
    k, w = O.compress_24(golden["patterns_w"])
    assert (k == golden["patterns_kept"]).all() and (w == golden["patterns_words"]).all()
    k, w = O.compress_24(golden["random_q"])
    assert (k == golden["random_kept"]).all() and (w == golden["random_words"]).all()


def test_prune24_golden(golden):
    assert (O.prune_24(golden["random_w"]) == golden["random_pruned"]).all()


def test_compress24_roundtrip_and_rejects():
    rng = np.random.default_rng(1)
    w = rng.integers(-127, 128, size=(64, 512)).astype(np.int8)
    g = w.reshape(64, -1, 4)
    # zero two random positions per group (some groups get more zeros)
    for idx in range(g.shape[1]):
        z = rng.permutation(4)[: rng.integers(2, 5)]
        g[:, idx, z] = 0
    k, e = O.compress_24(w)
    assert (O.decompress_24(k, e) == w).all()
    bad = w.copy()
    bad[0, :4] = [1, 2, 3, 0]
    with pytest.raises(ValueError):
        O.compress_24(bad)


def test_compress24_six_pairs_by_hand():
    # group (a, b at i0 < i1): kept (a, b), nibble i0 | i1 << 2
    for i0 in range(4):
        for i1 in range(i0 + 1, 4):
            row = np.zeros(32, np.int8)
            row[i0], row[i1] = 11, -3
            k, e = O.compress_24(row[None])
            assert list(k[0, :2]) == [11, -3]
            assert (int(e[0, 0]) & 15) == (i0 | (i1 << 2))
    # one nonzero at p: kept with the lowest zero position, both in order
    for p in range(4):
        row = np.zeros(32, np.int8)
        row[p] = 9
        k, e = O.compress_24(row[None])
        other = 0 if p != 0 else 1
        lo, hi = sorted((p, other))
        assert (int(e[0, 0]) & 15) == (lo | (hi << 2))
        assert list(k[0, :2]) == ([9, 0] if p == lo else [0, 9])
    # all zero: positions 0 and 1 -> nibble 0b0100
    k, e = O.compress_24(np.zeros((1, 32), np.int8))
    assert (int(e[0, 0]) & 15) == 4 and not k.any()


def test_prune24_keeps_two_largest():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((32, 256)).astype(np.float32)
    p = O.prune_24(w)
    g, gp = np.abs(w.reshape(32, -1, 4)), p.reshape(32, -1, 4)
    assert ((gp != 0).sum(-1) == 2).all()
    kept = np.sort(np.where(gp != 0, g, -1), -1)[..., 2:]
    assert np.allclose(kept, np.sort(g, -1)[..., 2:])


# ---- a1 / a10: weight quantizers ------------------------------------------------------------------------------------

def test_quantize_weight_rows_matches_torch_and_bounds():
    _, w, _ = linear_inputs(4, 96, 320, seed=3)
    w[5] = 0  # zero row: scale 1e-12 / 127, q = 0
    q, s = O.quantize_weight_rows(bf16_bits(w))
    wf = w.float()
    # the scale as the reference's GPU computes `amax / 127`: times fp32(1 / 127) (pinned against PyTorch's own GPU
    # division in tests/test_quant_gpu.py); CPU PyTorch divides exactly, which differs on some rows
    rcp = float(np.float32(1.0) / np.float32(127.0))
    st = wf.abs().amax(-1).clamp_min(1e-12) * rcp
    qt = torch.round(wf / st[:, None]).clamp(-127, 127).to(torch.int8)
    assert np.array_equal(s, st.numpy()) and np.array_equal(q, qt.numpy())
    exact = wf.abs().amax(-1).clamp_min(1e-12) / 127
    assert (exact != st).any()  # the two forms are told apart by this input
    assert (np.abs(q).max(1)[np.arange(96) != 5] == 127).all() and not q[5].any()
    err = np.abs(q.astype(np.float64) * s[:, None] - bf16_float(bf16_bits(w)))
    assert (err <= s[:, None].astype(np.float64) * (0.5 + 1e-5)).all()


def test_quantize_weight_rows_half_even_ties():
    # amax 127 -> s = 1 exactly: w = k + 0.5 rounds to the even neighbour
    w = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.5, -2.5]], np.float32)
    q, s = O.quantize_weight_rows(w)
    assert s[0] == 1.0 and list(q[0]) == [127, 0, 2, 2, 0, -2, 4, -2]


def test_prepare_w8_is_permuted_quantize_rows():
    _, w, _ = linear_inputs(4, 64, 512, seed=4)
    u, s = O.prepare_w8(bf16_bits(w))
    q, s2 = O.quantize_weight_rows(bf16_bits(w))
    perm = [0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15]
    unperm = np.empty_like(u)
    for j, pj in enumerate(perm):
        unperm[:, pj::16] = u[:, j::16]
    assert np.array_equal(s, s2) and np.array_equal(unperm.astype(np.int16) - 128, q.astype(np.int16))


# ---- a2: activation quantizer ---------------------------------------------------------------------------------------

def test_q8_rows_properties():
    x, _, _ = linear_inputs(50, 16, 1280, seed=5)
    x[7] = 0
    q, s = O.q8_rows(bf16_bits(x))
    xf = x.float().numpy()
    mx = np.abs(xf).max(1)
    assert s[7] == 1.0 and not q[7].any()
    nz = np.arange(50) != 7
    assert np.array_equal(s[nz], (mx[nz] / np.float32(127)).astype(np.float32))
    assert (np.abs(q[nz]).max(1) == 127).all()
    # |q - x / s| <= 1/2 plus the reciprocal's rounding
    assert (np.abs(q - xf / s[:, None]) <= 0.5 + 1e-4).all()


def test_q8_rows_reciprocal_not_divide():
    # the reference multiplies by the rounded reciprocal (encoder_ops.cu:29-36); x * (1/s) and x / s differ on
    # these hand-found bf16 rows (row maximum first): 0.5625 / (1.125 / 127) is 63.5 by the reciprocal (-> 64) but
    # 63.499996 by the divide (-> 63); with maximum 1.171875 the two land the other way round
    for mx_bits, x_bits, want_recip, want_div in ((0x3F90, 0x3F10, 64, 63), (0x3F96, 0x3F16, 63, 64)):
        row = np.array([mx_bits, x_bits, 0x0000, 0xBF10], np.uint16)
        q, s = O.q8_rows(row[None])
        xf = bf16_float(row)
        assert int(np.rint(xf[1] / s[0])) == want_div  # the divide would give the other integer
        assert q[0, 1] == want_recip and q[0, 0] == 127 and q[0, 2] == 0
    rng = np.random.default_rng(6)
    for _ in range(200):
        row = rng.standard_normal(64).astype(np.float32)
        xb = bf16_bits(torch.from_numpy(row).to(torch.bfloat16))
        q, s = O.q8_rows(xb[None])
        xf = bf16_float(xb)
        inv = np.float32(1) / s[0]
        assert np.array_equal(q[0], np.rint(np.clip(xf * inv, -127, 127)).astype(np.int8))


# ---- a3-a5: GEMM ----------------------------------------------------------------------------------------------------

def _quantized(M, N, K, seed=0):
    x, w, b = linear_inputs(M, N, K, seed)
    xq, xs = O.q8_rows(bf16_bits(x))
    wq, ws = O.quantize_weight_rows(bf16_bits(w))
    return xq, xs, wq, ws, bf16_bits(b)


@pytest.mark.parametrize("M,N,K", [(37, 48, 320), (128, 64, 1280)])
def test_gemm_int32_acc_exact(M, N, K):
    xq, xs, wq, ws, b = _quantized(M, N, K)
    acc = O.gemm_i8(xq, xs, K, wq, ws, b, O.EPI_I32)
    ref = xq.astype(np.int64) @ wq.astype(np.int64).T
    assert np.array_equal(acc, ref)
    assert np.array_equal(acc, torch._int_mm(torch.from_numpy(xq), torch.from_numpy(wq).t().contiguous()).numpy())


def _fma_f64(a, b, c):
    """fp32 fma via float64 (the product is exact in float64; the sum rounds twice only in rare cases)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def test_gemm_bias_and_resid_epilogue_float64():
    M, N, K = 64, 96, 640
    xq, xs, wq, ws, b = _quantized(M, N, K, seed=7)
    out, acc = O.gemm_i8(xq, xs, K, wq, ws, b, O.EPI_BIAS, want_acc=True)
    x = acc.astype(np.float32) * xs[:, None]
    v = _fma_f64(x, ws[None, :], bf16_float(b)[None, :])
    want = O.f32_to_bf16(v)
    assert (out != want).mean() < 1e-3
    # residual, alpha 0.5, with out aliasing resid semantics (read before write)
    r = bf16_bits(torch.randn(M, N, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16))
    got = O.gemm_i8(xq, xs, K, wq, ws, b, O.EPI_RESID, resid=r, alpha=0.5)
    want = O.f32_to_bf16(_fma_f64(np.float32(0.5), bf16_float(O.f32_to_bf16(v)), bf16_float(r)))
    assert (got != want).mean() < 1e-3


def test_gemm_glu_silu_closed_forms():
    M, N, K = 32, 256, 256
    xq, xs, wq, ws, b = _quantized(M, N, K, seed=9)
    out, acc = O.gemm_i8(xq, xs, K, wq, ws, b, O.EPI_BIAS, want_acc=True)
    vb = bf16_float(out).astype(np.float64)
    glu = O.gemm_i8(xq, xs, K, wq, ws, b, O.EPI_GLU)
    want = vb[:, 0::2] / (1 + np.exp(-vb[:, 1::2]))
    # one bf16 rounding of the exact value: within one bf16 ulp (2^-8 relative)
    assert (np.abs(bf16_float(glu) - want) <= np.abs(want) * 2.0 ** -8 + 1e-7).all()
    q, qs = O.gemm_i8(xq, xs, K, wq, ws, b, O.EPI_SILU_Q8, qgroup=128)
    silu = vb / (1 + np.exp(-vb))
    deq = q.astype(np.float64) * np.repeat(qs, 128, axis=1)
    assert np.max(np.abs(deq - silu)) <= 0.51 * np.repeat(qs, 128, axis=1).max() + 1e-3
    assert (np.abs(q).reshape(M, -1, 128).max(-1) == 127).all()


def test_gemm_grouped_fold():
    M, N, K, G = 16, 32, 1024, 256
    xq, _, wq, ws, b = _quantized(M, N, K, seed=10)
    sa = (np.random.default_rng(11).random((M, K // G)) + 0.5).astype(np.float32) * np.float32(0.01)
    got = O.gemm_i8(xq, sa, G, wq, ws, None, O.EPI_BIAS)
    # float64 fold of the exact group sums, then one rounding: equal to the fp32 fold within a few bf16 ulps
    parts = np.stack([xq[:, g * G:(g + 1) * G].astype(np.int64) @ wq[:, g * G:(g + 1) * G].astype(np.int64).T
                      for g in range(K // G)], 0)
    v = (parts * sa.T[:, :, None]).sum(0) * ws[None, :]
    assert np.max(np.abs(bf16_float(got) - v)) <= 1e-2 * np.sqrt(np.mean(v ** 2))
    # one group: equals the per-row path exactly
    one = O.gemm_i8(xq, sa[:, :1].copy(), K, wq, ws, None, O.EPI_BIAS)
    acc = xq.astype(np.int64) @ wq.astype(np.int64).T
    assert np.array_equal(one, O.f32_to_bf16((acc.astype(np.float32) * sa[:, :1]) * ws[None, :]))


def test_gemm_sparse_is_dense_on_pruned():
    M, N, K = 24, 64, 512
    x, w, b = linear_inputs(M, N, K, seed=12)
    wp = O.prune_24(bf16_float(bf16_bits(w)))
    wq, ws = O.quantize_weight_rows(wp)
    k, e = O.compress_24(wq)
    assert np.array_equal(O.decompress_24(k, e), wq)


# ---- a11 / a12: decoder projections -----------------------------------------------------------------------------

def test_dec_w8_linear_matches_float64_matmul():
    x, w, b = linear_inputs(17, 128, 512, seed=13)
    u, s = O.prepare_w8(bf16_bits(w))
    y = O.dec_w8_linear(bf16_bits(x), u, s, bf16_bits(b), relu=True)
    q, _ = O.quantize_weight_rows(bf16_bits(w))
    ref = (x.double() @ (torch.from_numpy(q).double() * torch.from_numpy(s).double()[:, None]).t() +
           b.double()).clamp_min(0).numpy()
    assert (np.abs(bf16_float(y) - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()


def test_linear_bf16_matches_torch():
    x, w, b = linear_inputs(9, 64, 256, seed=14)
    y = O.linear_bf16(bf16_bits(x), bf16_bits(w), bf16_bits(b))
    ref = (x.double() @ w.double().t() + b.double()).numpy()
    assert (np.abs(bf16_float(y) - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()
