"""CPU checker for the quantized-GEMM hot path (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only as the thing the
HIP kernels are compared with (or, for the baseline, timed beside them). The product path never calls it.

The arithmetic lives in cohere_oracle.c (built into liboracle.so by the Makefile here); this module wraps it for numpy
arrays. bf16 data is passed as np.uint16 bit patterns.

Function -> reference -> what pins it (tests/test_oracle.py unless noted):
  quantize_weight_rows  kernels/fast_encoder.py:60-63   torch.round/amax on the same formula; |q*s - w| <= s/2;
                                                        hand-made half-way ties; zero rows
  q8_rows               kernels/csrc/encoder_ops.cu:18-42  reciprocal-vs-divide cases built by hand; max|q| = 127;
                                                        |q - x/s| <= 1/2 + 1 ulp; zero row -> scale 1
  gemm_i8 (int32 acc)   kernels/csrc/gemm_int8.cu:62-289 numpy int64 matmul and torch._int_mm (exact library routines)
  gemm_i8 (epilogues)   kernels/csrc/gemm_int8.cu:201-288 float64 evaluation of the same expression (fma exact in
                                                        float64 but for rare double rounding); GLU/SILU closed
                                                        forms; grouped with one group == per-row scales
  compress_24           kernels/sparse.py:26-39          decompress(compress(W)) == W; the six position pairs and the
                                                        <2-nonzero groups by hand; golden fixture
                                                        tests/golden/compress24_golden.npz
  prune_24              kernels/sparse.py:42-46          exactly two zeros per group, survivors are the two largest
  prepare_w8            kernels/stream_decoder.py:38-48  un-permute + dequantize == quantize_weight_rows
  dec_w8_linear         kernels/csrc/dec_w8.cu:46-180    torch float64 matmul of the dequantized weights
  linear_bf16           kernels/decoder_kernels.py:19-34 torch float64 matmul
  layernorm             kernels/csrc/layernorm.cuh:6-43  torch.nn.functional.layer_norm in float64
  dwconv_bn_silu        kernels/csrc/encoder_ops.cu:455-498, 559-641  torch conv1d (groups = channels) per sequence
                                                        in float64, then BatchNorm and SiLU
  relpos_attention      kernels/csrc/encoder_ops.cu:82-337  transformers' ParakeetEncoderAttention (rel_shift form)
                                                        in float32; with a zero table and zero biases, softmax
                                                        attention in float64
  dec_embed, dec_add_ln kernels/csrc/decoder_ops.cu:24-83  torch float64 LayerNorm of the bf16 sums
  dec_attention         kernels/csrc/dec_attn.cuh:84-188  torch scaled_dot_product_attention in float64 over the
                                                        dequantized caches; the new key/value written at pos
  dec_pick              kernels/csrc/decoder_ops.cu:106-159  torch.argmax (first index of the maximum) + the
                                                        bookkeeping rules written out by hand in the test
  dec_scatter_kv        kernels/csrc/decoder_ops.cu:163-204  q8_rows-style absmax round trip per 128-vector
  decoder_step          kernels/stream_decoder.py:176-199  transformers' CohereAsrDecoder (float32, one token per
                                                        slot with its own cache) on the dequantized weights
  encoder_layers_int8   kernels/csrc/encoder_loop.cpp:63-99  transformers' ParakeetEncoderBlock in float32 on the
                                                        dequantized weights (within the int8 activation error)
  gemm_bf16             kernels/csrc/gemm.cu:150-212     exact small-integer operands: numpy int64 matmul and each
                                                        epilogue's closed form (tests/test_frontend_oracle.py)
  logmel                kernels/csrc/features.cu:34-102  transformers' CohereAsrFeatureExtractor.__call__ (torch.stft,
                                                        its normalization) on the same dithered pieces, the Slaney
                                                        filter bank pinned against transformers.audio_utils
  sub_conv0_dw, sub_dw  kernels/csrc/encoder_ops.cu:339-448  torch conv2d in float64 (with conv0's two roundings);
                                                        the whole stem against transformers'
                                                        ParakeetEncoderSubsamplingConv2D in float32
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_DIR, "liboracle.so")

EPI_BIAS, EPI_SILU, EPI_RELU, EPI_RESID, EPI_GLU, EPI_SILU_Q8, EPI_CONV_RELU, EPI_I32 = range(8)

_lib = None


def build() -> str:
    """Compile liboracle.so with the Makefile next to this file (gcc; seconds)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _DIR, "-B", "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        i64, p = ctypes.c_int64, ctypes.c_void_p
        _lib.orc_quantize_weight_rows.argtypes = [p, i64, i64, p, p]
        _lib.orc_q8_rows.argtypes = [p, i64, i64, i64, p, i64, p]
        _lib.orc_layernorm.argtypes = [p, i64, p, p, ctypes.c_float, p, p, ctypes.c_float, p, i64, i64, i64]
        _lib.orc_dwconv_bn_silu.argtypes = [p, p, p, p, p, p, p, p, i64, i64]
        _lib.orc_relpos_attention.argtypes = [p, p, i64, p, p, p, p, i64, i64, i64, i64, ctypes.c_float, p]
        _lib.orc_dec_embed.argtypes = [p, i64, p, p, p, p, p, p, ctypes.c_float, p, p, ctypes.c_float, p, p, i64]
        _lib.orc_dec_add_ln.argtypes = [p, p, i64, p, p, ctypes.c_float, p, i64, i64]
        _lib.orc_dec_attention.argtypes = [ctypes.c_int, ctypes.c_int, p, i64, p, i64, p, p, p, p, p, p, p, i64, i64,
                                           ctypes.c_float, p]
        _lib.orc_dec_pick.argtypes = [p, i64, i64, p, i64, p, p, p, p, i64, p, p, p, i64, i64]
        _lib.orc_dec_scatter_kv.argtypes = [ctypes.c_int, p, i64, p, p, p, p, p, p, p, p, i64, i64, i64, i64]
        _lib.orc_gemm_i8.argtypes = [p, i64, p, i64, i64, p, i64, p, p, p, i64, ctypes.c_int, p, i64, ctypes.c_float,
                                     p, i64, i64, i64, i64, i64, p, ctypes.c_int]
        _lib.orc_gemm_i8.restype = ctypes.c_int
        _lib.orc_compress_24.argtypes = [p, i64, i64, p, p]
        _lib.orc_compress_24.restype = ctypes.c_int
        _lib.orc_decompress_24.argtypes = [p, p, i64, i64, p]
        _lib.orc_prune_24.argtypes = [p, i64, i64, p]
        _lib.orc_prepare_w8.argtypes = [p, i64, i64, p, p]
        _lib.orc_dec_w8_linear.argtypes = [p, i64, p, p, p, p, i64, ctypes.c_int, i64, i64, i64, ctypes.c_int]
        _lib.orc_linear_bf16.argtypes = [p, i64, p, p, p, i64, ctypes.c_int, i64, i64, i64, ctypes.c_int]
        _lib.orc_gemm_bf16.argtypes = [p, i64, p, p, p, i64, ctypes.c_int, p, i64, ctypes.c_float, i64, i64, i64,
                                       ctypes.c_int]
        _lib.orc_logmel.argtypes = [p, p, i64, p, p, p, ctypes.c_float, p, i64, ctypes.c_int]
        _lib.orc_sub_conv0_dw.argtypes = [p, i64, p, p, i64, p, p, p, p, p, i64, ctypes.c_int]
        _lib.orc_sub_dw.argtypes = [p, p, p, p, i64, p, p, p, i64, i64, ctypes.c_int]
        _lib.orc_f32_to_bf16.argtypes = [p, p, i64]
        _lib.orc_bf16_to_f32.argtypes = [p, p, i64]
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- bf16 ------------------------------------------------------------------------------------------------------------

def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits (round to nearest even)."""
    f = _c(f, np.float32)
    h = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_bf16(_p(f), _p(h), f.size)
    return h


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp32 (exact: the bits shifted into the high half), through torch's bf16 widening for speed."""
    import torch

    h = _c(h, np.uint16)
    return torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float().numpy()


# ---- quantizers ------------------------------------------------------------------------------------------------------

def quantize_weight_rows(w_bf16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """a1 (fast_encoder.py:60-63): (int8 [N, K], fp32 [N])."""
    w = bf16_to_f32(w_bf16) if w_bf16.dtype == np.uint16 else _c(w_bf16, np.float32)
    n, k = w.shape
    q, s = np.empty((n, k), np.int8), np.empty(n, np.float32)
    lib().orc_quantize_weight_rows(_p(w), n, k, _p(q), _p(s))
    return q, s


def q8_rows(x_bf16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """a2 (encoder_ops.cu:18-42): bf16 rows -> (int8 [rows, cols], fp32 [rows])."""
    x = _c(x_bf16, np.uint16)
    rows, cols = x.shape
    q, s = np.empty((rows, cols), np.int8), np.empty(rows, np.float32)
    lib().orc_q8_rows(_p(x), cols, rows, cols, _p(q), cols, _p(s))
    return q, s


# ---- GEMM ------------------------------------------------------------------------------------------------------------

def gemm_i8(a, sa, group, w, sw, bias, epi, resid=None, alpha=1.0, qgroup=256, threads=0, want_acc=False):
    """a3-a5 (gemm_int8.cu): the reference's W8A8 linear on the CPU.

    a int8 [M, K]; sa fp32 [M, K / group]; w int8 [N, K]; sw fp32 [N]; bias bf16 bits [N] or None; resid bf16 bits
    [M, N] for EPI_RESID. Returns out (bf16 bits [M, N] / [M, N/2] for GLU / int8 for SILU_Q8 / int32 for EPI_I32),
    plus qs for SILU_Q8, plus the int32 accumulators when want_acc (per-row scales only)."""
    a, w = _c(a, np.int8), _c(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    sa = _c(sa, np.float32).reshape(M, -1)
    sw = _c(sw, np.float32)
    bias = None if bias is None else _c(bias, np.uint16)
    qs = None
    if epi == EPI_GLU:
        out = np.empty((M, N // 2), np.uint16)
    elif epi == EPI_SILU_Q8:
        out = np.empty((M, N), np.int8)
        qs = np.empty((M, N // qgroup), np.float32)
    elif epi == EPI_I32:
        out = np.empty((M, N), np.int32)
    else:
        out = np.empty((M, N), np.uint16)
    r = None
    if epi == EPI_RESID:
        r = _c(resid, np.uint16)
    acc = np.empty((M, N), np.int32) if want_acc else None
    rc = lib().orc_gemm_i8(_p(a), K, _p(sa), sa.shape[1], group, _p(w), K, _p(sw), _p(bias), _p(out), out.shape[1],
                           epi, _p(r), N if r is not None else 0, alpha, _p(qs), qs.shape[1] if qs is not None else 0,
                           qgroup, M, N, K, _p(acc), threads)
    if rc != 0:
        raise ValueError(f"orc_gemm_i8: bad arguments ({rc})")
    res = [out]
    if qs is not None:
        res.append(qs)
    if want_acc:
        res.append(acc)
    return res[0] if len(res) == 1 else tuple(res)


# ---- 2:4 sparsity ----------------------------------------------------------------------------------------------------

def compress_24(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """a6 (sparse.py:26-39): (kept int8 [N, K/2], selectors int32 [N, K/32])."""
    w = _c(w, np.int8)
    n, k = w.shape
    kept, words = np.empty((n, k // 2), np.int8), np.empty((n, k // 32), np.int32)
    rc = lib().orc_compress_24(_p(w), n, k, _p(kept), _p(words))
    if rc == -1:
        raise ValueError("compress_24: K must be a multiple of 32")
    if rc == -2:
        raise ValueError("compress_24: more than two nonzero values in a group of four")
    return kept, words


def decompress_24(kept: np.ndarray, words: np.ndarray) -> np.ndarray:
    kept, words = _c(kept, np.int8), _c(words, np.int32)
    n, k = kept.shape[0], kept.shape[1] * 2
    w = np.empty((n, k), np.int8)
    lib().orc_decompress_24(_p(kept), _p(words), n, k, _p(w))
    return w


def prune_24(w: np.ndarray) -> np.ndarray:
    """a7 (sparse.py:42-46) on fp32 values (the bf16 weights as fp32)."""
    w = _c(w, np.float32)
    out = np.empty_like(w)
    lib().orc_prune_24(_p(w), w.shape[0], w.shape[1], _p(out))
    return out


# ---- decoder projections -----------------------------------------------------------------------------------------

def prepare_w8(w_bf16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """a10 (stream_decoder.py:41-48): (uint8 [N, K] permuted, fp32 [N])."""
    w = bf16_to_f32(w_bf16) if w_bf16.dtype == np.uint16 else _c(w_bf16, np.float32)
    n, k = w.shape
    q, s = np.empty((n, k), np.uint8), np.empty(n, np.float32)
    lib().orc_prepare_w8(_p(w), n, k, _p(q), _p(s))
    return q, s


def dec_w8_linear(x, w, sw, bias, relu=False, threads=0):
    """a11 (dec_w8.cu): x bf16 bits [M, K], w uint8 [N, K] (prepare_w8 layout) -> bf16 bits [M, N]."""
    x, w, sw = _c(x, np.uint16), _c(w, np.uint8), _c(sw, np.float32)
    bias = None if bias is None else _c(bias, np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.uint16)
    lib().orc_dec_w8_linear(_p(x), K, _p(w), _p(sw), _p(bias), _p(y), N, int(relu), M, N, K, threads)
    return y


def linear_bf16(x, w, bias, relu=False, threads=0):
    """a12 (decoder_kernels.py:19-34): bf16 x [M, K] @ w [N, K]^T + bias -> bf16 bits [M, N]."""
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    bias = None if bias is None else _c(bias, np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.uint16)
    lib().orc_linear_bf16(_p(x), K, _p(w), _p(bias), _p(y), N, int(relu), M, N, K, threads)
    return y


# ---- the encoder layer's other producers and the layer loop (row a9) ------------------------------------------------

def layernorm(x, w1, b1, eps1, w2=None, b2=None, eps2=0.0):
    """layernorm.cuh:6-43: returns (h, x') as bf16 bits; x' = LN1(x) when w2 is given (else x unchanged)."""
    x = _c(x, np.uint16).copy()
    rows, cols = x.shape
    h = np.empty_like(x)
    lib().orc_layernorm(_p(x), cols, _p(_c(w1, np.uint16)), _p(_c(b1, np.uint16)), eps1,
                        _p(None if w2 is None else _c(w2, np.uint16)), _p(None if b2 is None else _c(b2, np.uint16)),
                        eps2, _p(h), cols, rows, cols)
    return h, x


def dwconv_bn_silu(x, w, cb, bn_scale, bn_shift, lo, hi):
    """encoder_ops.cu:455-498: bf16 bits [rows, C] -> bf16 bits [rows, C]."""
    x = _c(x, np.uint16)
    rows, C = x.shape
    y = np.empty_like(x)
    lib().orc_dwconv_bn_silu(_p(x), _p(_c(w, np.float32)), _p(_c(cb, np.float32)), _p(_c(bn_scale, np.float32)),
                             _p(_c(bn_shift, np.float32)), _p(_c(lo, np.int32)), _p(_c(hi, np.int32)), _p(y), rows, C)
    return y


def dwconv_bn_silu_q8(x, w, cb, bn_scale, bn_shift, lo, hi):
    """encoder_ops.cu:559-641: the rows of dwconv_bn_silu quantized (store_q8's arithmetic)."""
    return q8_rows(dwconv_bn_silu(x, w, cb, bn_scale, bn_shift, lo, hi))


def relpos_attention(qkv, rk, bu, bv, lengths, rel_off, scale):
    """encoder_ops.cu:82-337 over packed sequences of the given lengths: bf16 bits [rows, H D]."""
    qkv, rk = _c(qkv, np.uint16), _c(rk, np.uint16)
    bu, bv = _c(bu, np.uint16), _c(bv, np.uint16)
    H, D = bu.shape
    lengths = np.asarray(lengths, np.int32)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int32)
    out = np.zeros((qkv.shape[0], H * D), np.uint16)
    lib().orc_relpos_attention(_p(qkv), _p(rk), rk.shape[0], _p(bu), _p(bv), _p(starts), _p(lengths), len(lengths),
                               H, D, rel_off, scale, _p(out))
    return out


# the reference's per-layer field order (kernels/csrc/encoder_loop.cpp:34-44)
LAYER_FIELDS = (
    "ln_ff1_w", "ln_ff1_b", "ln_att_w", "ln_att_b", "ln_conv_w", "ln_conv_b", "ln_ff2_w", "ln_ff2_b", "ln_out_w",
    "ln_out_b", "ff1_w1", "ff1_b1", "ff1_w2", "ff1_b2", "ff2_w1", "ff2_b1", "ff2_w2", "ff2_b2", "wqkv", "bqkv", "wo",
    "bo", "bu", "bv", "rk", "wpw1", "bpw1", "wdw", "bdw", "bn_scale", "bn_shift", "wpw2", "bpw2", "q_ff1_w1",
    "q_ff1_s1", "q_ff1_w2", "q_ff1_s2", "q_ff2_w1", "q_ff2_s1", "q_ff2_w2", "q_ff2_s2", "q_qkv_w", "q_qkv_s",
    "q_pw1_w", "q_pw1_s", "q_o_w", "q_o_s", "q_pw2_w", "q_pw2_s", "sp_ff1_w", "sp_ff1_e", "sp_ff2_w", "sp_ff2_e",
    # the product's own extension: the first feed-forward linears in 2:4 form
    "sp_ff1_w1", "sp_ff1_e1", "sp_ff2_w1", "sp_ff2_e1")


def encoder_layers_int8(x, layers, eps, lengths, rel_off, scale, group=256, qgroup_ff1=256, threads=0):
    """encoder_loop.cpp:63-99 (the int8 branch), each step by the functions above and gemm_i8: x bf16 bits
    [rows, 1280] -> the layers' output (bf16 bits). layers: one dict per layer, LAYER_FIELDS -> numpy arrays (bf16 as
    uint16 bits; a 2:4 W2 given as sp_ff*_w/e, or W1 given as sp_ff*_w1/e1, is run as the dense GEMM on its
    decompressed weights, which is gemm_sparse.cu's result bit for bit). eps: per layer (ff1, att, conv, ff2, out)."""
    x = _c(x, np.uint16).copy()
    lengths = list(lengths)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    lo = np.concatenate([np.full(n, s) for s, n in zip(starts, lengths)]).astype(np.int32)
    hi = np.concatenate([np.full(n, s + n) for s, n in zip(starts, lengths)]).astype(np.int32)

    def ffn(ly, hq, hs, k):
        sp1 = ly.get(f"sp_ff{k}_w1")
        w1 = decompress_24(sp1, ly[f"sp_ff{k}_e1"]) if sp1 is not None and sp1.size else ly[f"q_ff{k}_w1"]
        tq, ts = gemm_i8(hq, hs, hq.shape[1], w1, ly[f"q_ff{k}_s1"], ly.get(f"ff{k}_b1"), EPI_SILU_Q8,
                         qgroup=qgroup_ff1, threads=threads)
        sp = ly.get(f"sp_ff{k}_w")
        w2 = decompress_24(sp, ly[f"sp_ff{k}_e"]) if sp is not None and sp.size else ly[f"q_ff{k}_w2"]
        return gemm_i8(tq, ts, group, w2, ly[f"q_ff{k}_s2"], ly.get(f"ff{k}_b2"), EPI_RESID, resid=x, alpha=0.5,
                       threads=threads)

    L = len(layers)
    h, _ = layernorm(x, layers[0]["ln_ff1_w"], layers[0]["ln_ff1_b"], eps[0][0])
    hq, hs = q8_rows(h)
    for i, ly in enumerate(layers):
        x = ffn(ly, hq, hs, 1)
        h, _ = layernorm(x, ly["ln_att_w"], ly["ln_att_b"], eps[i][1])
        hq, hs = q8_rows(h)
        qkv = gemm_i8(hq, hs, hq.shape[1], ly["q_qkv_w"], ly["q_qkv_s"], ly.get("bqkv"), EPI_BIAS, threads=threads)
        a = relpos_attention(qkv, ly["rk"], ly["bu"], ly["bv"], lengths, rel_off, scale)
        hq, hs = q8_rows(a)
        x = gemm_i8(hq, hs, hq.shape[1], ly["q_o_w"], ly["q_o_s"], ly.get("bo"), EPI_RESID, resid=x, alpha=1.0,
                    threads=threads)
        h, _ = layernorm(x, ly["ln_conv_w"], ly["ln_conv_b"], eps[i][2])
        hq, hs = q8_rows(h)
        a = gemm_i8(hq, hs, hq.shape[1], ly["q_pw1_w"], ly["q_pw1_s"], ly.get("bpw1"), EPI_GLU, threads=threads)
        hq, hs = dwconv_bn_silu_q8(a, ly["wdw"], ly["bdw"], ly["bn_scale"], ly["bn_shift"], lo, hi)
        x = gemm_i8(hq, hs, hq.shape[1], ly["q_pw2_w"], ly["q_pw2_s"], ly.get("bpw2"), EPI_RESID, resid=x, alpha=1.0,
                    threads=threads)
        h, _ = layernorm(x, ly["ln_ff2_w"], ly["ln_ff2_b"], eps[i][3])
        hq, hs = q8_rows(h)
        x = ffn(ly, hq, hs, 2)
        if i + 1 < L:
            h, x = layernorm(x, ly["ln_out_w"], ly["ln_out_b"], eps[i][4], layers[i + 1]["ln_ff1_w"],
                             layers[i + 1]["ln_ff1_b"], eps[i + 1][0])
            hq, hs = q8_rows(h)
        else:
            x, _ = layernorm(x, ly["ln_out_w"], ly["ln_out_b"], eps[i][4])
    return x


def encoder_layers_bf16(x, layers, eps, lengths, rel_off, scale, threads=0):
    """encoder_loop.cpp:101-124 (the bf16 branch): x bf16 bits [rows, 1280] -> the layers' output (bf16 bits), every
    linear by gemm_bf16 with its fused epilogue (SiLU, residual, GLU, bias), the LayerNorms, attention and depthwise
    convolution by the functions above. layers: one dict per layer with the bf16 weight fields ff*_w1/w2, wqkv, wo,
    wpw1 (GLU rows interleaved), wpw2 and the shared fields; eps: per layer (ff1, att, conv, ff2, out)."""
    x = _c(x, np.uint16).copy()
    lengths = list(lengths)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    lo = np.concatenate([np.full(n, s) for s, n in zip(starts, lengths)]).astype(np.int32)
    hi = np.concatenate([np.full(n, s + n) for s, n in zip(starts, lengths)]).astype(np.int32)
    lin = lambda a, ly, w, b, epi, resid=None, alpha=1.0: gemm_bf16(  # noqa: E731
        a, ly[w], ly.get(b), epi, resid=resid, alpha=alpha, threads=threads)
    L = len(layers)
    h, _ = layernorm(x, layers[0]["ln_ff1_w"], layers[0]["ln_ff1_b"], eps[0][0])
    for i, ly in enumerate(layers):
        t = lin(h, ly, "ff1_w1", "ff1_b1", EPI_SILU)
        x = lin(t, ly, "ff1_w2", "ff1_b2", EPI_RESID, resid=x, alpha=0.5)
        h, _ = layernorm(x, ly["ln_att_w"], ly["ln_att_b"], eps[i][1])
        qkv = lin(h, ly, "wqkv", "bqkv", EPI_BIAS)
        a = relpos_attention(qkv, ly["rk"], ly["bu"], ly["bv"], lengths, rel_off, scale)
        x = lin(a, ly, "wo", "bo", EPI_RESID, resid=x)
        h, _ = layernorm(x, ly["ln_conv_w"], ly["ln_conv_b"], eps[i][2])
        g = lin(h, ly, "wpw1", "bpw1", EPI_GLU)
        z = dwconv_bn_silu(g, ly["wdw"], ly["bdw"], ly["bn_scale"], ly["bn_shift"], lo, hi)
        x = lin(z, ly, "wpw2", "bpw2", EPI_RESID, resid=x)
        h, _ = layernorm(x, ly["ln_ff2_w"], ly["ln_ff2_b"], eps[i][3])
        t = lin(h, ly, "ff2_w1", "ff2_b1", EPI_SILU)
        x = lin(t, ly, "ff2_w2", "ff2_b2", EPI_RESID, resid=x, alpha=0.5)
        if i + 1 < L:
            h, x = layernorm(x, ly["ln_out_w"], ly["ln_out_b"], eps[i][4], layers[i + 1]["ln_ff1_w"],
                             layers[i + 1]["ln_ff1_b"], eps[i + 1][0])
        else:
            x, _ = layernorm(x, ly["ln_out_w"], ly["ln_out_b"], eps[i][4])
    return x


# ---- the decoder step (row a13) --------------------------------------------------------------------------------------
# Arrays are numpy, modified in place like the kernels' outputs; bf16 as uint16 bits.

def _ln_args(ln):
    w, b, eps = ln
    return _p(_c(w, np.uint16)), _p(_c(b, np.uint16)), float(eps)


def dec_embed(active, tok, pos, emb, ptab, ln0, ln1):
    """decoder_ops.cu:24-54: (x, h) bf16 bits [rows, width]."""
    rows, width = len(active), emb.shape[1]
    x, h = np.empty((rows, width), np.uint16), np.empty((rows, width), np.uint16)
    lib().orc_dec_embed(_p(_c(active, np.int32)), rows, _p(_c(tok, np.int64)), _p(_c(pos, np.int32)),
                        _p(_c(emb, np.uint16)), _p(_c(ptab, np.uint16)), *_ln_args(ln0), *_ln_args(ln1), _p(x), _p(h),
                        width)
    return x, h


def dec_add_ln(x, y, ln):
    """decoder_ops.cu:56-83: x = bf16(x + y) in place (x must be a C-contiguous uint16 array); returns h."""
    assert x.dtype == np.uint16 and x.flags.c_contiguous
    y = _c(y, np.uint16)
    h = np.empty_like(x)
    lib().orc_dec_add_ln(_p(x), _p(y), y.shape[1], *_ln_args(ln), _p(h), x.shape[0], x.shape[1])
    return h


def dec_attention(self_attn, active, q, n, scale, k=None, v=None, k8=None, v8=None, ks=None, vs=None):
    """dec_attn.cuh:84-188 over one layer's caches (slots, H, T, 128): bf16 (k, v) or int8 (k8, v8, ks, vs), updated
    in place for self-attention. Returns out bf16 bits [rows, H * 128]."""
    q = _c(q, np.uint16)
    q8 = k8 is not None
    caches = (k8, v8, ks, vs) if q8 else (k, v)
    for c in caches:
        assert c.flags.c_contiguous
    H, T = (k8 if q8 else k).shape[1:3]
    rows = q.shape[0]
    out = np.empty((rows, H * 128), np.uint16)
    lib().orc_dec_attention(int(self_attn), int(q8), _p(_c(active, np.int32)), rows, _p(q), q.shape[1],
                            _p(None if q8 else k), _p(None if q8 else v), _p(k8), _p(v8), _p(ks), _p(vs),
                            _p(_c(n, np.int32)), H, T, scale, _p(out))
    return out


def dec_pick(logits, active, dummy, tok, pos, finished, forced, plen, limit, out, eos):
    """decoder_ops.cu:106-159, the state arrays (numpy, contiguous) updated in place."""
    logits = _c(logits, np.uint16)
    for a in (tok, pos, finished, out):
        assert a.flags.c_contiguous
    lib().orc_dec_pick(_p(logits), logits.shape[0], logits.shape[1], _p(_c(active, np.int32)), dummy, _p(tok),
                       _p(pos), _p(finished), _p(_c(forced, np.int64)), forced.shape[1], _p(_c(plen, np.int32)),
                       _p(_c(limit, np.int32)), _p(out), out.shape[1], eos)


def dec_scatter_kv(kv, slot_of, frame_of, ck=None, cv=None, ck8=None, cv8=None, cks=None, cvs=None):
    """decoder_ops.cu:163-204 into caches (L, S, H, T, 128), in place."""
    kv = _c(kv, np.uint16)
    q8 = ck8 is not None
    L, S, H, T = (ck8 if q8 else ck).shape[:4]
    lib().orc_dec_scatter_kv(int(q8), _p(kv), kv.shape[0], _p(_c(slot_of, np.int32)), _p(_c(frame_of, np.int32)),
                             _p(ck), _p(cv), _p(ck8), _p(cv8), _p(cks), _p(cvs), L, S, H, T)


def decoder_step(W, st, b, int8=True):
    """kernels/stream_decoder.py:176-199 (StreamDecoder._step) for the first b rows of st["active"], every step of it
    by the functions above and the projections a11 / a12. W: weights (numpy; see tests/decoder_helpers.py); st: the
    slot state and caches (numpy, updated in place). Returns the head's logits (bf16 bits [b, V])."""
    act = st["active"][:b]
    x, hn = dec_embed(act, st["tok"], st["pos"], W["embed"], W["pos_table"], W["emb_ln"], W["layers"][0]["ln1"])
    lin = lambda a, name, ly, relu=False: (  # noqa: E731
        dec_w8_linear(a, *ly[name + "_w8"], ly[name + "_b"], relu) if int8 and name + "_w8" in ly
        else linear_bf16(a, ly[name + "_w"], ly[name + "_b"], relu))
    L = len(W["layers"])
    for i, ly in enumerate(W["layers"]):
        qkv = lin(hn, "qkv", ly)
        a = dec_attention(True, act, qkv, st["pos"], W["scale"], k8=st["self_k8"][i], v8=st["self_v8"][i],
                          ks=st["self_ks"][i], vs=st["self_vs"][i])
        hn = dec_add_ln(x, lin(a, "o", ly), ly["ln2"])
        a = dec_attention(False, act, lin(hn, "cq", ly), st["cross_len"], W["scale"], k8=st["cross_k8"][i],
                          v8=st["cross_v8"][i], ks=st["cross_ks"][i], vs=st["cross_vs"][i])
        hn = dec_add_ln(x, lin(a, "co", ly), ly["ln3"])
        f = lin(lin(hn, "fc1", ly, relu=True), "fc2", ly)
        hn = dec_add_ln(x, f, W["layers"][i + 1]["ln1"] if i + 1 < L else W["final_ln"])
    logits = lin(hn, "head", W)
    dec_pick(logits, act, st["dummy"], st["tok"], st["pos"], st["finished"], st["forced"], st["plen"], st["limit"],
             st["out"], W["eos"])
    return logits


# ---- bf16 GEMM and the encoder's front end (config 4) -----------------------------------------------------------

def gemm_bf16(a, w, bias, epi, resid=None, alpha=1.0, threads=0):
    """gemm.cu:150-212: bf16 bits a [M, K] @ w [N, K]^T with the epilogue -> bf16 bits [M, N] ([M, N/2] for GLU)."""
    a, w = _c(a, np.uint16), _c(w, np.uint16)
    M, K = a.shape
    N = w.shape[0]
    bias = None if bias is None else _c(bias, np.uint16)
    out = np.empty((M, N // 2 if epi == EPI_GLU else N), np.uint16)
    r = _c(resid, np.uint16) if epi == EPI_RESID else None
    lib().orc_gemm_bf16(_p(a), K, _p(w), _p(bias), _p(out), out.shape[1], epi, _p(r), N if r is not None else 0,
                        alpha, M, N, K, threads)
    return out


def logmel_meta(lengths) -> np.ndarray:
    """meta int64 [3 pieces + 1] of pieces with these sample counts (first sample, length, cumulative valid frames)."""
    lengths = np.asarray(lengths, np.int64)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    valid = lengths // 160
    return np.concatenate([starts, lengths, np.concatenate([[0], np.cumsum(valid)])]).astype(np.int64)


def logmel(x, lengths, window, mel, band, preemph, T=None, threads=0):
    """features.cu:34-102: normalized log-mel of the pieces (fp32 samples back to back) -> bf16 bits
    [pieces, T, 128], zero past each piece's valid frames (T defaults to max(n // 160) + 1)."""
    x = _c(x, np.float32)
    meta = logmel_meta(lengths)
    pieces = len(lengths)
    if T is None:
        T = max(n // 160 for n in lengths) + 1
    out = np.zeros((pieces, T, 128), np.uint16)
    lib().orc_logmel(_p(x), _p(meta), pieces, _p(_c(window, np.float32)), _p(_c(mel, np.float32)),
                     _p(_c(band, np.int32)), preemph, _p(out), T, threads)
    return out


def sub_conv0_dw(feats, mel_len, rows, w0, b0, w2, b2, threads=0):
    """encoder_ops.cu:339-413: feats bf16 bits [B, T, 128]; rows int32 [n, 2] (sequence, t2) -> bf16 bits
    [n, 32, C]."""
    feats = _c(feats, np.uint16)
    rows = _c(rows, np.int32).reshape(-1, 2)
    C = w0.shape[0]
    out = np.empty((rows.shape[0], 32, C), np.uint16)
    lib().orc_sub_conv0_dw(_p(feats), feats.shape[1] * 128, _p(_c(mel_len, np.int32)), _p(rows), rows.shape[0],
                           _p(_c(w0, np.float32)), _p(_c(b0, np.float32)), _p(_c(w2, np.float32)),
                           _p(_c(b2, np.float32)), _p(out), C, threads)
    return out


def sub_dw(x, in_start, in_len, rows, w, b, threads=0):
    """encoder_ops.cu:415-448: x bf16 bits [sum T_in, F_in, C] -> bf16 bits [n, F_in / 2, C]."""
    x = _c(x, np.uint16)
    _, F_in, C = x.shape
    rows = _c(rows, np.int32).reshape(-1, 2)
    out = np.empty((rows.shape[0], F_in // 2, C), np.uint16)
    lib().orc_sub_dw(_p(x), _p(_c(in_start, np.int32)), _p(_c(in_len, np.int32)), _p(rows), rows.shape[0],
                     _p(_c(w, np.float32)), _p(_c(b, np.float32)), _p(out), F_in, C, threads)
    return out
