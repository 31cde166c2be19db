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
    h = _c(h, np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


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
