"""Config 3's captured step taken apart: the fused program's launches (the ones the HIP graph records) called one at
a time through ext on config 3's own state (64 slots, 8 layers, vocab 16384, U(1..448) caches, 375 frames), each fed
the product's own output of the launch before and checked against its kernel's own bar on those same inputs
(reference kernels/stream_decoder.py:176-199 for the order, kernels/csrc/decoder_ops.cu:106-159 for the pick):

  * the embedding and every projection: within max-abs 1e-2 x RMS (one bf16 ulp where the value's own ulp is larger)
    of the checker's fp64-summed result. A launch with a LayerNorm prologue normalises its input rows exactly as
    dec_add_ln does with a zero addend (bit for bit: tests/test_decoder_gpu.py), so that LayerNorm is run once more on
    its own here, checked against the checker's LayerNorm at the same bar, and its output is the input the checker's
    projection gets;
  * the residual epilogues (x = bf16(x + bf16(y))): within 1e-2 x RMS of the projection's output y, plus one ulp of
    the sum;
  * attention: output within 1e-2 x RMS; the self-attention's writes into the int8 caches bit-exact;
  * the pick (token, position, end flag, output row) bit-exact on the product's own logits, and the next step's
    embedding it computes within the embedding's bar;
  * then the same step replayed from the graph, from the same starting state, is bit-identical to the staged run in
    every buffer it writes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_bf16_close, bf16_bits, bf16_float, bf16_ulp
from test_decoder_config3_gpu import LAYERS, config3_decoder

pytestmark = pytest.mark.gpu

WRITTEN = ("x", "hn", "qkv_out", "att", "q_out", "ffn_out", "logits", "tok", "pos", "finished", "out", "self_k",
           "self_v", "self_ks", "self_vs")


def _resid_close(got_bits, want_bits, y_bits):
    """x = bf16(x + bf16(y)): each element within 1e-2 x RMS(y) plus one ulp of the sum of the checker's."""
    got, want = bf16_float(got_bits).astype(np.float64), bf16_float(want_bits).astype(np.float64)
    y = bf16_float(y_bits).astype(np.float64)
    tol = 1e-2 * np.sqrt(np.mean(y ** 2)) + bf16_ulp(want) * 1.0001
    diff = np.abs(got - want)
    assert (diff <= tol).all(), f"{int((diff > tol).sum())} elements beyond, worst {(diff / tol).max():.3f} x tol"


def _close(what, got_bits, want_bits):
    """assert_bf16_close, printing the fraction of elements whose bits differ."""
    print(f"  {what}: {(got_bits != want_bits).mean():.4f} of elements differ", flush=True)
    got, want = bf16_float(got_bits).astype(np.float64), bf16_float(want_bits).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    ratio = np.abs(got - want) / np.maximum(1e-2 * rms, bf16_ulp(want) * 1.0001)
    w = np.unravel_index(np.argmax(ratio), ratio.shape)
    if ratio[w] > 1:
        print(f"    worst {w}: got {got[w]!r} want {want[w]!r} rms {rms:.4e} ulp(want) {bf16_ulp(want[w])!r}",
              flush=True)
    assert_bf16_close(got_bits, want_bits)


def _ln(what, x_gpu, ln_gpu, ln_bits):
    """The product's LayerNorm of x's rows (dec_add_ln with a zero addend: the prologue's arithmetic), checked against
    the checker's; returns it as bf16 bits."""
    from kernels.cuda_ext import ext

    xs, h = x_gpu.clone(), torch.empty_like(x_gpu)
    ext.dec_add_ln(xs, torch.zeros_like(x_gpu), *ln_gpu, h)
    torch.cuda.synchronize()
    x = bf16_bits(x_gpu)
    _close(what + " LayerNorm", bf16_bits(h), oracle.dec_add_ln(x.copy(), np.zeros_like(x), ln_bits))
    return h


def _unfused(what, proj, h_gpu, got_bits, relu=False):
    """The launch's projection run on its own (no prologue) from the standalone LayerNorm h: the fused launch must
    give the same bits. Returns h as bf16 bits for the checker."""
    y = torch.empty(h_gpu.shape[0], proj.n, dtype=torch.bfloat16, device=h_gpu.device)
    proj(h_gpu, y, relu=relu)
    torch.cuda.synchronize()
    same = np.array_equal(bf16_bits(y), got_bits)
    print(f"  {what}: fused launch == LayerNorm then projection: {same}", flush=True)
    assert same
    return bf16_bits(h_gpu)


def test_config3_staged_step(gpu):
    _, dec, st, W, b = config3_decoder(gpu)
    assert dec.fused and b in dec.graphs
    act = st["active"][:b]
    bits = lambda name: bf16_bits(getattr(dec, name)[:b])  # noqa: E731  (the step's rows of a bf16 buffer)
    start = {k: getattr(dec, k).clone() for k in WRITTEN}
    flags0 = dec.flags.clone()
    for k, a in (("self_k", "self_k8"), ("self_v", "self_v8"), ("self_ks", "self_ks"), ("self_vs", "self_vs")):
        st[a][...] = getattr(dec, k).cpu().numpy()
    for k in ("tok", "pos", "finished", "out", "plen", "limit", "forced", "cross_len"):
        st[k][...] = getattr(dec, k).cpu().numpy()

    def run(op):
        op()
        torch.cuda.synchronize()

    # the step's embedding (step() runs it first whenever the rows changed, as here after set_active)
    run(lambda: dec._embed(b))
    ox, oh = oracle.dec_embed(act, st["tok"], st["pos"], W["embed"], W["pos_table"], W["emb_ln"],
                              W["layers"][0]["ln1"])
    _close("embedding x", bits("x"), ox)
    _close("embedding LayerNorm", bits("hn"), oh)
    ops = iter(dec.programs[b])
    lin = lambda a, ly, name, relu=False: (  # noqa: E731
        oracle.dec_w8_linear(a, *ly[name + "_w8"], ly[name + "_b"], relu) if name + "_w8" in ly
        else oracle.linear_bf16(a, ly[name + "_w"], ly[name + "_b"], relu))
    checked = 0
    for i, ly in enumerate(W["layers"]):
        # self-attention: qkv (layer 0 from the embedding's LayerNorm, later layers normalise x in the prologue)
        blk = dec.blocks[i]
        hg = dec.hn[:b].clone() if i == 0 else _ln(f"layer {i} qkv", dec.x[:b], blk.norms[0], ly["ln1"])
        run(next(ops))
        h = _unfused(f"layer {i} qkv", blk.qkv, hg, bits("qkv_out"))
        _close(f"layer {i} qkv", bits("qkv_out"), lin(h, ly, "qkv"))
        qkv = bits("qkv_out")
        run(next(ops))
        want = oracle.dec_attention(True, act, qkv, st["pos"], W["scale"], k8=st["self_k8"][i], v8=st["self_v8"][i],
                                    ks=st["self_ks"][i], vs=st["self_vs"][i])
        _close(f"layer {i} self-attention", bits("att"), want)
        for k, a in (("self_k", "self_k8"), ("self_v", "self_v8"), ("self_ks", "self_ks"), ("self_vs", "self_vs")):
            assert np.array_equal(getattr(dec, k)[i].cpu().numpy(), st[a][i]), (i, k)
        # o with the residual add
        att, x = bits("att"), bits("x")
        run(next(ops))
        y = lin(att, ly, "o")
        xw = x.copy()
        oracle.dec_add_ln(xw, y, ly["ln2"])
        _resid_close(bits("x"), xw, y)
        # cross-attention: q with the LayerNorm prologue, attention over the slot's frames, o + residual
        hg = _ln(f"layer {i} cross q", dec.x[:b], blk.norms[1], ly["ln2"])
        run(next(ops))
        h = _unfused(f"layer {i} cross q", blk.cq, hg, bits("q_out"))
        _close(f"layer {i} cross q", bits("q_out"), lin(h, ly, "cq"))
        q = bits("q_out")
        run(next(ops))
        want = oracle.dec_attention(False, act, q, st["cross_len"], W["scale"], k8=st["cross_k8"][i],
                                    v8=st["cross_v8"][i], ks=st["cross_ks"][i], vs=st["cross_vs"][i])
        _close(f"layer {i} cross-attention", bits("att"), want)
        att, x = bits("att"), bits("x")
        run(next(ops))
        y = lin(att, ly, "co")
        xw = x.copy()
        oracle.dec_add_ln(xw, y, ly["ln3"])
        _resid_close(bits("x"), xw, y)
        # feed-forward: fc1 + ReLU with the LayerNorm prologue, fc2 + residual
        hg = _ln(f"layer {i} fc1", dec.x[:b], blk.norms[2], ly["ln3"])
        run(next(ops))
        h = _unfused(f"layer {i} fc1", blk.fc1, hg, bits("ffn_out"), relu=True)
        _close(f"layer {i} fc1", bits("ffn_out"), lin(h, ly, "fc1", relu=True))
        f, x = bits("ffn_out"), bits("x")
        run(next(ops))
        y = lin(f, ly, "fc2")
        xw = x.copy()
        oracle.dec_add_ln(xw, y, ly["ln1"])
        _resid_close(bits("x"), xw, y)
        checked += 8
    # the head with the final LayerNorm in its prologue
    hg = _ln("head", dec.x[:b], dec.final_ln, W["final_ln"])
    run(next(ops))
    h = _unfused("head", dec.head, hg, bits("logits"))
    _close("head", bits("logits"), lin(h, W, "head"))
    # the pick on the product's own logits, then the next step's embedding from the new token and position
    logits = bits("logits")
    run(next(ops))
    oracle.dec_pick(logits, act, st["dummy"], st["tok"], st["pos"], st["finished"], st["forced"], st["plen"],
                    st["limit"], st["out"], W["eos"])
    for k in ("tok", "pos", "finished", "out"):
        assert np.array_equal(getattr(dec, k).cpu().numpy(), st[k]), k
    assert np.array_equal(dec.flags.numpy()[act], st["finished"][act])
    ox, oh = oracle.dec_embed(act, st["tok"], st["pos"], W["embed"], W["pos_table"], W["emb_ln"],
                              W["layers"][0]["ln1"])
    _close("next embedding x", bits("x"), ox)
    _close("next embedding LayerNorm", bits("hn"), oh)
    assert next(ops, None) is None and checked == 8 * LAYERS
    staged = {k: getattr(dec, k).clone() for k in WRITTEN}
    staged_flags = dec.flags.clone()

    # the graph replay of the same step from the same state
    with torch.no_grad():
        for k, t in start.items():
            getattr(dec, k).copy_(t)
        dec.flags.copy_(flags0)
    torch.cuda.synchronize()
    dec._embed_stale = True
    dec.step(b)
    torch.cuda.synchronize()
    raw = lambda t: t.view(torch.int16) if t.dtype == torch.bfloat16 else t  # noqa: E731  (bitwise for bf16)
    for k in WRITTEN:
        assert torch.equal(raw(getattr(dec, k)), raw(staged[k])), k
    assert torch.equal(dec.flags, staged_flags)
    print(f"staged config-3 step: {checked + 3} launches checked against the checker, graph replay bit-identical",
          flush=True)
