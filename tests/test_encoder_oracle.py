"""Pins of the CPU checker's encoder-layer functions (layernorm, dwconv_bn_silu, relpos_attention, the int8 layer
loop) against library routines: torch's layer_norm and conv1d in float64, and transformers' ParakeetEncoderAttention
/ ParakeetEncoderBlock -- the module the reference's fast_encoder.py converts."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from encoder_helpers import (dequantized_block, hf_block_forward, hf_distance_table, make_block, oracle_fields)
from helpers import bf16_bits, bf16_float, bf16_ulp

pytest.importorskip("transformers.models.parakeet.modeling_parakeet")


def _bf(t: torch.Tensor) -> np.ndarray:
    return bf16_bits(t.to(torch.bfloat16))


def test_layernorm_matches_torch_float64():
    g = torch.Generator().manual_seed(3)
    rows, cols = 37, 320
    x = _bf(torch.randn(rows, cols, generator=g) * 3 + 0.5)
    w1, b1 = _bf(1 + 0.2 * torch.randn(cols, generator=g)), _bf(0.1 * torch.randn(cols, generator=g))
    w2, b2 = _bf(1 + 0.2 * torch.randn(cols, generator=g)), _bf(0.1 * torch.randn(cols, generator=g))
    t = lambda a: torch.from_numpy(bf16_float(a)).double()  # noqa: E731
    want1 = torch.nn.functional.layer_norm(t(x), (cols,), t(w1), t(b1), 1e-5)
    h, xo = oracle.layernorm(x, w1, b1, 1e-5)
    assert np.array_equal(xo, x)
    diff = np.abs(bf16_float(h) - want1.numpy())
    assert (diff <= bf16_ulp(want1.numpy()) * 1.0001).all()
    # two in a row: x = LN1(x) in place, h = LN2(x)
    h2, x2 = oracle.layernorm(x, w1, b1, 1e-5, w2, b2, 1e-6)
    assert np.array_equal(x2, h)
    want2 = torch.nn.functional.layer_norm(t(x2), (cols,), t(w2), t(b2), 1e-6).numpy()
    assert (np.abs(bf16_float(h2) - want2) <= bf16_ulp(want2) * 1.0001).all()


def test_dwconv_matches_torch_conv1d_per_sequence():
    g = torch.Generator().manual_seed(4)
    lengths, C = [13, 1, 40, 6], 64
    rows = sum(lengths)
    x = _bf(torch.randn(rows, C, generator=g))
    w = (0.3 * torch.randn(C, 9, generator=g)).numpy().astype(np.float32)
    cb = (0.1 * torch.randn(C, generator=g)).numpy().astype(np.float32)
    sc = (1 + 0.2 * torch.randn(C, generator=g)).numpy().astype(np.float32)
    sh = (0.1 * torch.randn(C, generator=g)).numpy().astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    lo = np.concatenate([np.full(n, s) for s, n in zip(starts, lengths)]).astype(np.int32)
    hi = lo + np.concatenate([np.full(n, n) for n in lengths]).astype(np.int32)
    got = bf16_float(oracle.dwconv_bn_silu(x, w, cb, sc, sh, lo, hi))
    rb = lambda a: a.float().to(torch.bfloat16).double()  # noqa: E731
    want = []
    for s, n in zip(starts, lengths):
        seq = torch.from_numpy(bf16_float(x[s:s + n])).double().t()[None]  # (1, C, n)
        a = torch.nn.functional.conv1d(seq, torch.from_numpy(w).double()[:, None, :],
                                       torch.from_numpy(cb).double(), padding=4, groups=C)[0].t()
        a = rb(a)
        a = rb(a * torch.from_numpy(sc).double() + torch.from_numpy(sh).double())
        want.append(rb(a * torch.sigmoid(a)))
    want = torch.cat(want).numpy()
    diff = np.abs(got - want)
    # the checker sums the taps in fp32 (fmaf chain): one bf16 ulp of an intermediate at most, rarely
    assert (diff <= 2 * bf16_ulp(want) * 1.0001 + 1e-6).all()
    assert (diff > 0).mean() < 0.02
    hq, hs = oracle.dwconv_bn_silu_q8(x, w, cb, sc, sh, lo, hi)
    q_ref, s_ref = oracle.q8_rows(oracle.dwconv_bn_silu(x, w, cb, sc, sh, lo, hi))
    assert np.array_equal(hq, q_ref) and np.array_equal(hs, s_ref)


def _attention_inputs(T, H, D, seed, table_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(T, H, D, generator=g).to(torch.bfloat16).float() for _ in range(3))
    bu = (0.3 * torch.randn(H, D, generator=g)).to(torch.bfloat16).float()
    bv = (0.3 * torch.randn(H, D, generator=g)).to(torch.bfloat16).float()
    rel = (table_scale * torch.randn(2 * T - 1, H, D, generator=g)).to(torch.bfloat16).float()  # distance T-1-p at p
    return q, k, v, bu, bv, rel


def _oracle_attention(q, k, v, bu, bv, rel, lengths_one, rel_off, rel_rows, scale):
    T, H, D = q.shape
    qkv = _bf(torch.cat([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], 1))
    table = torch.zeros(rel_rows, H * D)
    for p in range(2 * T - 1):
        table[(T - 1 - p) + rel_off] = rel[p].reshape(-1)
    return bf16_float(oracle.relpos_attention(qkv, _bf(table), _bf(bu), _bf(bv), lengths_one, rel_off, scale))


def _hf_attention(q, k, v, bu, bv, rel, scale):
    """ParakeetEncoderAttention's arithmetic (modeling_parakeet.py forward) in float64, with its own _rel_shift."""
    from transformers.models.parakeet.modeling_parakeet import ParakeetEncoderAttention

    T, H, D = q.shape
    qh, kh, vh = (t.double().permute(1, 0, 2)[None] for t in (q, k, v))  # (1, H, T, D)
    qu = (q + bu[None]).to(torch.bfloat16).double().permute(1, 0, 2)[None]
    qv = (q + bv[None]).to(torch.bfloat16).double().permute(1, 0, 2)[None]
    relk = rel.double().permute(1, 2, 0)[None]  # (1, H, D, 2T-1)
    bd = ParakeetEncoderAttention._rel_shift(None, qv @ relk)[..., :T] * scale
    s = (qu @ kh.transpose(-1, -2)) * scale + bd
    out = torch.softmax(s, -1) @ vh
    return out[0].permute(1, 0, 2).reshape(T, H * D).numpy()


@pytest.mark.parametrize("T,H,D", [(70, 2, 80), (33, 1, 160)])
def test_relpos_attention_matches_transformers(T, H, D):
    q, k, v, bu, bv, rel = _attention_inputs(T, H, D, seed=T, table_scale=1.5)
    scale = D ** -0.5
    rel_off, rel_rows = T - 1, 2 * T - 1 + 64
    got = _oracle_attention(q, k, v, bu, bv, rel, [T], rel_off, rel_rows, scale)
    want = _hf_attention(q, k, v, bu, bv, rel, scale)
    # the module in float64 has none of the kernel's bf16 roundings (position term twice, probabilities, output):
    # RMS error below 1 %, max error below 6 % of the RMS
    rms = np.sqrt(np.mean(want ** 2))
    err = np.sqrt(np.mean((got - want) ** 2)) / rms
    assert err < 1e-2 and np.abs(got - want).max() / rms < 6e-2, err
    # the position term matters here: the same attention with the distance reversed (i - j -> j - i) is far off
    wrong = _hf_attention(q, k, v, bu, bv, rel.flip(0), scale)
    assert np.sqrt(np.mean((wrong - want) ** 2)) / rms > 50 * err


def test_relpos_attention_zero_table_is_softmax_attention():
    T, H, D = 45, 2, 80
    q, k, v, _, _, rel = _attention_inputs(T, H, D, seed=9)
    z = torch.zeros(H, D)
    got = _oracle_attention(q, k, v, z, z, rel * 0, [T], T - 1, 2 * T + 63, D ** -0.5)
    want = torch.nn.functional.scaled_dot_product_attention(
        *(t.double().permute(1, 0, 2) for t in (q, k, v)), scale=D ** -0.5).permute(1, 0, 2).reshape(T, -1).numpy()
    rms = np.sqrt(np.mean(want ** 2))
    assert np.sqrt(np.mean((got - want) ** 2)) / rms < 5e-3 and np.abs(got - want).max() / rms < 3e-2


def test_relpos_attention_packed_sequences_are_independent():
    H, D, lengths = 1, 80, [20, 35, 1]
    g = torch.Generator().manual_seed(11)
    rows = sum(lengths)
    qkv = _bf(torch.randn(rows, 3 * H * D, generator=g))
    table = _bf(torch.randn(2 * 64 + 63, H * D, generator=g))
    bu = _bf(0.1 * torch.randn(H, D, generator=g))
    bv = _bf(0.1 * torch.randn(H, D, generator=g))
    packed = oracle.relpos_attention(qkv, table, bu, bv, lengths, 63, 0.1)
    s = 0
    for n in lengths:
        alone = oracle.relpos_attention(qkv[s:s + n], table, bu, bv, [n], 63, 0.1)
        assert np.array_equal(packed[s:s + n], alone)
        s += n


def test_distance_table_mirror_matches_transformers():
    """The host mirror's relative_table (reference fast_encoder.py:155-162) against the table built from
    transformers' own positional-encoding module."""
    from kernels.fast_encoder import relative_table

    blk, inv_freq = make_block(160, 2, 640, seed=5)
    blk = blk.to(torch.bfloat16)
    want = hf_distance_table(blk, inv_freq, max_len=40)
    got = relative_table(inv_freq, blk.self_attn.relative_k_proj.weight, max_len=40).float()
    assert got.shape == want.shape
    assert (got - want).abs().max() <= 2 * bf16_ulp(want.numpy()).max()


@pytest.mark.parametrize("sparse", [False, True])
def test_encoder_layer_int8_follows_transformers_block(sparse):
    """One int8 layer of the checker (encoder_loop.cpp:63-99 order) against transformers' ParakeetEncoderBlock in
    float32 on the same (dequantized) weights: they differ by the int8 activation quantization and bf16 roundings
    only. A wrong composition (e.g. the feed-forward residual at 1.0 instead of 0.5) is several times further off."""
    hidden, heads, ff, lengths = 256, 2, 1024, [40, 23]
    blk, inv_freq = make_block(hidden, heads, ff, seed=7)
    table = hf_distance_table(blk, inv_freq, max_len=64)
    fields, eps = oracle_fields(blk, table, sparse)
    ref_blk = dequantized_block(blk, fields)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(sum(lengths), hidden, generator=g).to(torch.bfloat16)
    got = bf16_float(oracle.encoder_layers_int8(bf16_bits(x), [fields], [eps], lengths, 63, (hidden // heads) ** -0.5,
                                                group=128, qgroup_ff1=128))
    want = hf_block_forward(ref_blk, inv_freq, x.float(), lengths).numpy()
    rms = np.sqrt(np.mean(want ** 2))
    err = np.sqrt(np.mean((got - want) ** 2)) / rms
    assert err < 2e-2, err
    with torch.no_grad():  # the same block with the feed-forward residual weight doubled
        ref_blk.feed_forward1.linear2.weight.mul_(2)
        ref_blk.feed_forward1.linear2.bias.mul_(2)
    off = hf_block_forward(ref_blk, inv_freq, x.float(), lengths).numpy()
    assert np.sqrt(np.mean((off - want) ** 2)) / rms > 3 * err


def test_encoder_layer_bf16_follows_transformers_block():
    """One bf16 layer of the checker (encoder_loop.cpp:101-124 order) against transformers' ParakeetEncoderBlock in
    float32 on the same bf16-representable weights: they differ by the bf16 roundings of the intermediate results
    only. The same wrong composition as above is several times further off."""
    from encoder_helpers import oracle_fields_bf16

    hidden, heads, ff, lengths = 256, 2, 1024, [40, 23]
    blk, inv_freq = make_block(hidden, heads, ff, seed=9)
    table = hf_distance_table(blk, inv_freq, max_len=64)
    fields, eps = oracle_fields_bf16(blk, table)
    g = torch.Generator().manual_seed(10)
    x = torch.randn(sum(lengths), hidden, generator=g).to(torch.bfloat16)
    got = bf16_float(oracle.encoder_layers_bf16(bf16_bits(x), [fields], [eps], lengths, 63, (hidden // heads) ** -0.5))
    want = hf_block_forward(blk, inv_freq, x.float(), lengths).numpy()
    rms = np.sqrt(np.mean(want ** 2))
    err = np.sqrt(np.mean((got - want) ** 2)) / rms
    assert err < 1e-2, err
    with torch.no_grad():
        blk.feed_forward1.linear2.weight.mul_(2)
        blk.feed_forward1.linear2.bias.mul_(2)
    off = hf_block_forward(blk, inv_freq, x.float(), lengths).numpy()
    assert np.sqrt(np.mean((off - want) ** 2)) / rms > 3 * err
