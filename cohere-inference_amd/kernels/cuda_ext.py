"""The gfx950 kernels of the quantized-GEMM path behind the reference's `ext` call surface.

Drop-in for the reference's kernels/cuda_ext.py (`ext` object and `EPI_*` constants, cuda_ext.py:26-28) for the
functions of this path: the methods keep the names, argument order and meaning of the pybind11 module
(kernels/csrc/bindings.cpp:26-62), validate dtypes and strides as its TORCH_CHECKs do, launch on the current stream,
and raise RuntimeError on a rejected call. Underneath is libcohere_hip.so, the C ABI of include/cohere_hip.h, loaded
with ctypes; nothing here computes on the host.

    from kernels.cuda_ext import EPI_BIAS, EPI_RESID, ext
    ext.gemm_i8(a, sa, 1280, w, sw, bias, out, EPI_BIAS, None, 1.0, None, 0)

The library is built in-tree (cohere-inference_amd/csrc/build.py, run by __graft_entry__.build()); importing this
module without it raises ImportError -- there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os

import torch

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# COHERE_HIP_LIBRARY selects another build of the library (A/B comparisons of build options)
LIB_PATH = os.environ.get("COHERE_HIP_LIBRARY") or os.path.join(_PKG, "lib", "libcohere_hip.so")

EPI_BIAS, EPI_SILU, EPI_RELU, EPI_RESID, EPI_GLU, EPI_SILU_Q8, EPI_CONV_RELU = range(7)
DEC_EP_NONE, DEC_EP_RELU, DEC_EP_RESID = range(3)  # dec_linear_fused's epilogues
TILED_REC = 1280  # bytes per record of the stage-tiled 2:4 weight layout (kernels.sparse.pack_24_tiled)
EPI_I32 = 7  # raw int32 accumulators: a parity hook with no counterpart in the reference

# every symbol include/cohere_hip.h declares
EXPORTS = ("cohere_gemm_i8", "cohere_gemm_sp", "cohere_quantize_rows", "cohere_layernorm_q8", "cohere_dec_w8_linear",
           "cohere_linear_bf16", "cohere_last_error", "cohere_version", "cohere_set_gemm_tile",
           "cohere_set_skinny_shape", "cohere_layernorm", "cohere_dwconv_bn_silu", "cohere_dwconv_bn_silu_q8",
           "cohere_relpos_attention", "cohere_encoder_workspace_bytes", "cohere_encoder_layers", "cohere_dec_embed",
           "cohere_dec_add_ln", "cohere_dec_attention", "cohere_dec_attention_q8", "cohere_dec_pick",
           "cohere_dec_scatter_kv", "cohere_dec_scatter_kv_q8", "cohere_gemm_bf16", "cohere_logmel_workspace_bytes",
           "cohere_logmel_features", "cohere_sub_conv0_dw", "cohere_sub_dw", "cohere_encoder_branch_workspace_bytes",
           "cohere_encoder_layers_noalloc", "cohere_dec_linear_fused", "cohere_dec_pick_embed",
           "cohere_gemm_sp_tiled", "cohere_pack_24_tiled_bytes", "cohere_pack_24_tiled")


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise ImportError(f"libcohere_hip.so not built ({path}); run __graft_entry__.build() or "
                          "python cohere-inference_amd/csrc/build.py")
    lib = ctypes.CDLL(path)
    P, I64, I32, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float
    sig = {
        "cohere_gemm_i8": [P, I64, P, I64, I64, P, P, P, P, I64, I32, P, I64, F, P, I64, I64, I64, I64, I32, P],
        "cohere_gemm_sp": [P, I64, P, I64, I64, P, P, P, P, P, I64, I32, P, I64, F, P, I64, I64, I64, I64, I32, P],
        "cohere_gemm_sp_tiled": [P, I64, P, I64, I64, P, P, P, P, I64, I32, P, I64, F, P, I64, I64, I64, I64, I32, P],
        "cohere_pack_24_tiled_bytes": [I64, I64],
        "cohere_pack_24_tiled": [P, P, I64, I64, P],
        "cohere_quantize_rows": [P, I64, P, I64, P, I64, I64, P],
        "cohere_layernorm_q8": [P, I64, P, P, F, P, P, F, P, I64, P, I64, I64, P],
        "cohere_dec_w8_linear": [P, I64, P, P, P, P, I64, I32, I64, I64, P, I64, P, I64, I64, I64, I64, P],
        "cohere_linear_bf16": [P, I64, P, P, P, I64, I32, I64, I64, I64, P],
        "cohere_dec_linear_fused": [P, I64, P, P, F, P, P, P, P, I64, I32, I64, I64, I64, P],
        "cohere_set_gemm_tile": [I32],
        "cohere_set_skinny_shape": [I32, I32],
        "cohere_layernorm": [P, I64, P, P, F, P, P, F, P, I64, I64, I64, P],
        "cohere_dwconv_bn_silu": [P, P, P, P, P, P, P, P, I64, I64, I64, P],
        "cohere_dwconv_bn_silu_q8": [P, P, P, P, P, P, P, P, P, I64, I64, I64, P],
        "cohere_relpos_attention": [P, P, I64, P, P, P, I64, I64, I64, I64, I64, F, P, P],
        "cohere_dec_embed": [P, I64, P, P, P, P, P, P, F, P, P, F, P, P, I64, P],
        "cohere_dec_add_ln": [P, P, I64, P, P, F, P, I64, I64, P],
        "cohere_dec_attention": [I32, P, I64, P, I64, P, P, P, I64, I64, I64, F, I64, P, I64, P, P],
        "cohere_dec_attention_q8": [I32, P, I64, P, I64, P, P, P, P, P, I64, I64, I64, F, I64, P, I64, P, P],
        "cohere_dec_pick": [P, I64, I64, P, I64, P, P, P, P, I64, P, P, P, I64, I64, I64, P],
        "cohere_dec_pick_embed": [P, I64, I64, P, I64, P, P, P, P, I64, P, P, P, I64, I64, I64, P, P, P, P, F, P, P, F,
                                  P, P, I64, P, P],
        "cohere_dec_scatter_kv": [P, I64, P, P, P, P, I64, I64, I64, I64, P],
        "cohere_dec_scatter_kv_q8": [P, I64, P, P, P, P, P, P, I64, I64, I64, I64, P],
        "cohere_gemm_bf16": [P, I64, P, P, P, I64, I32, P, I64, F, I64, I64, I64, I32, P],
        "cohere_logmel_features": [P, P, I64, I64, P, P, P, F, P, I64, P, P],
        "cohere_sub_conv0_dw": [P, I64, P, P, I64, P, P, P, P, P, I64, P],
        "cohere_sub_dw": [P, P, P, P, I64, P, P, P, I64, I64, P],
        "cohere_encoder_layers": [P, I64, P, I64, P, P, I64, P, P, I64, I64, I64, ctypes.c_double, I32, I32, I32, P,
                                  I64, P, I64, P],
        "cohere_encoder_layers_noalloc": [P, I64, P, I64, P, P, I64, P, P, I64, I64, I64, ctypes.c_double, I32, I32,
                                          I32, P, I64, P],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.cohere_encoder_workspace_bytes.argtypes = [I64, I64]
    lib.cohere_encoder_workspace_bytes.restype = I64
    lib.cohere_encoder_branch_workspace_bytes.argtypes = [I64, I64, I32]
    lib.cohere_encoder_branch_workspace_bytes.restype = I64
    lib.cohere_logmel_workspace_bytes.argtypes = [I64]
    lib.cohere_logmel_workspace_bytes.restype = I64
    lib.cohere_last_error.restype = ctypes.c_char_p
    lib.cohere_last_error.argtypes = []
    lib.cohere_version.restype = ctypes.c_char_p
    lib.cohere_version.argtypes = []
    return lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


_EMPTY = torch.empty(0)  # an absent per-layer tensor


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class _Ext:
    """The methods of the reference's `ext` on this path, on gfx950."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib

    def _call(self, name: str, *args) -> None:
        rc = getattr(self._lib, name)(*args)
        if rc != 0:
            raise RuntimeError(self._lib.cohere_last_error().decode())

    @property
    def version(self) -> str:
        return self._lib.cohere_version().decode()

    def set_gemm_tile(self, tile: int) -> int:
        """Tuning hook: force a gfx950 GEMM tile (-1 = automatic). Results never depend on it."""
        return self._lib.cohere_set_gemm_tile(int(tile))

    def set_skinny_shape(self, strips: int, waves: int) -> None:
        """Tuning hook: force the skinny projections' workgroup shape (strips <= 0 = automatic)."""
        self._lib.cohere_set_skinny_shape(int(strips), int(waves))

    # ---- bf16 GEMM (bindings.cpp:3-4, 65) ----------------------------------------------------------------------------

    def gemm(self, a, w, bias, out, epi, resid, alpha, cfg):
        """out = epilogue(a @ w^T + bias) in bf16 with fp32 accumulation; a (M, K) unit stride along K, w (N, K)
        contiguous, out (M, N) or (M, N/2) for EPI_GLU (reference kernels/csrc/gemm.cu:246-279)."""
        _check(a.dtype == torch.bfloat16 and w.dtype == torch.bfloat16, "gemm: bf16 only")
        _check(a.dim() == 2 and w.dim() == 2 and a.stride(1) == 1 and w.is_contiguous() and out.stride(1) == 1,
               "gemm: a, out need unit column stride and w must be contiguous")
        _check(a.shape[1] == w.shape[1] and a.shape[1] % 32 == 0, "gemm: K must match and be a multiple of 32")
        _check(out.dtype == torch.bfloat16 and (bias is None or bias.dtype == torch.bfloat16), "gemm: bf16 only")
        _check(epi != EPI_RESID or (resid is not None and resid.stride(1) == 1), "gemm: residual epilogue needs resid")
        M, K = a.shape
        if M == 0:
            return
        self._call("cohere_gemm_bf16", _ptr(a), a.stride(0), _ptr(w), _ptr(bias), _ptr(out), out.stride(0), int(epi),
                   _ptr(resid), resid.stride(0) if resid is not None else 0, float(alpha), M, w.shape[0], K, int(cfg),
                   _stream())

    # ---- front end: log-mel features and the subsampling convolutions (bindings.cpp:51-53, 71-72, 79) ---------------

    def logmel_features(self, x, meta, total_frames, window, mel, band, preemph, out):
        """Normalized log-mel of packed pieces into out (pieces, T, 128) bf16 (reference kernels/csrc/features.cu:
        105-132): x fp32 samples back to back; meta int64 (3 pieces + 1); window (512); mel (128, 257); band (128, 2)
        int32. Frames past each piece's valid frames are left as they are."""
        _check(x.is_contiguous() and x.dtype == torch.float32 and window.numel() == 512 and band.is_contiguous() and
               band.numel() == 256 and band.dtype == torch.int32 and mel.shape == (128, 257) and mel.is_contiguous()
               and out.is_contiguous() and out.dim() == 3 and out.shape[2] == 128 and out.dtype == torch.bfloat16 and
               meta.dtype == torch.int64 and meta.numel() == 3 * out.shape[0] + 1 and meta.is_contiguous() and
               window.is_contiguous() and window.dtype == torch.float32 and mel.dtype == torch.float32,
               "logmel_features: bad arguments")
        total_frames = int(total_frames)
        if total_frames == 0:
            return
        work = torch.empty(self._lib.cohere_logmel_workspace_bytes(total_frames) // 4, dtype=torch.float32,
                           device=x.device)
        self._call("cohere_logmel_features", _ptr(x), _ptr(meta), out.shape[0], total_frames, _ptr(window), _ptr(mel),
                   _ptr(band), float(preemph), _ptr(out), out.shape[1], _ptr(work), _stream())

    def sub_conv0_dw(self, feats, mel_len, rows, w0, b0, w2, b2, out):
        """Subsampling conv0 + ReLU + depthwise, per sequence, channels-last: feats (B, T, 128) bf16, mel_len (B)
        int32, rows (n, 2) int32 (sequence, t2), weights fp32 (C, 9) / (C), out (n, 32, C) bf16 (reference
        kernels/csrc/encoder_ops.cu:709-719)."""
        _check(feats.is_contiguous() and feats.dim() == 3 and feats.shape[2] == 128 and out.is_contiguous() and
               feats.dtype == torch.bfloat16 and out.dtype == torch.bfloat16 and w0.shape[0] == 256 and
               rows.dtype == torch.int32 and rows.is_contiguous() and mel_len.dtype == torch.int32 and
               all(t.dtype == torch.float32 and t.is_contiguous() for t in (w0, b0, w2, b2)),
               "sub_conv0_dw: bad arguments")
        n = rows.shape[0]
        if n == 0:
            return
        self._call("cohere_sub_conv0_dw", _ptr(feats), feats.stride(0), _ptr(mel_len), _ptr(rows), n, _ptr(w0),
                   _ptr(b0), _ptr(w2), _ptr(b2), _ptr(out), w0.shape[0], _stream())

    def sub_dw(self, x, in_start, in_len, rows, w, b, out):
        """Depthwise 3x3 stride-2 + bias on channels-last sequences: x (sum T_in, F_in, C) bf16, in_start / in_len
        (B) int32, rows (n, 2) int32, out (n, F_in / 2, C) (reference kernels/csrc/encoder_ops.cu:723-734)."""
        n, F_in, C = rows.shape[0], x.shape[1], x.shape[2]
        _check(x.is_contiguous() and out.is_contiguous() and C % 8 == 0 and x.dtype == torch.bfloat16 and
               out.dtype == torch.bfloat16 and rows.dtype == torch.int32 and in_start.dtype == torch.int32 and
               in_len.dtype == torch.int32 and w.dtype == torch.float32 and b.dtype == torch.float32 and
               w.is_contiguous(), "sub_dw: bad arguments")
        if n == 0:
            return
        self._call("cohere_sub_dw", _ptr(x), _ptr(in_start), _ptr(in_len), _ptr(rows), n, _ptr(w), _ptr(b),
                   _ptr(out), F_in, C, _stream())

    # ---- int8 GEMMs (bindings.cpp:41-43, 59-61) ----------------------------------------------------------------------

    def gemm_i8(self, a, sa, group, w, sw, bias, out, epi, resid, alpha, qs, cfg):
        """out = epilogue(dequant(a @ w^T) + bias); a int8 (M, K) with sa (M, K / group) fp32, w int8 (N, K) with sw
        (N) fp32 (reference kernels/csrc/gemm_int8.cu:349-391). EPI_SILU_Q8 writes int8 out and qs."""
        _check(a.dtype == torch.int8 and w.dtype == torch.int8 and sa.dtype == torch.float32 and
               sw.dtype == torch.float32, "gemm_i8: a, w int8 and sa, sw fp32 expected")
        _check(a.dim() == 2 and a.stride(1) == 1 and w.is_contiguous() and out.stride(1) == 1 and sa.stride(1) == 1,
               "gemm_i8: a, out, sa need unit column stride and w must be contiguous")
        M, K = a.shape
        _check(w.shape[1] == K and K % 64 == 0 and group % 64 == 0 and K % group == 0,
               "gemm_i8: K must match, be a multiple of 64 and of group")
        _check(bias is None or bias.dtype == torch.bfloat16, "gemm_i8: bias must be bf16")
        if epi == EPI_SILU_Q8:
            _check(qs is not None and out.dtype == torch.int8, "gemm_i8: SILU_Q8 needs int8 out and qs")
        elif epi == EPI_I32:
            _check(out.dtype == torch.int32, "gemm_i8: EPI_I32 needs int32 out")
        else:
            _check(out.dtype == torch.bfloat16, "gemm_i8: out must be bf16")
        _check(epi != EPI_RESID or resid is not None, "gemm_i8: residual epilogue needs resid")
        if M == 0:
            return
        self._call("cohere_gemm_i8", _ptr(a), a.stride(0), _ptr(sa), sa.stride(0), int(group), _ptr(w), _ptr(sw),
                   _ptr(bias), _ptr(out), out.stride(0), int(epi), _ptr(resid),
                   resid.stride(0) if resid is not None else 0, float(alpha), _ptr(qs),
                   qs.stride(0) if qs is not None else 0, M, w.shape[0], K, int(cfg), _stream())

    def gemm_sp(self, x, sx, group, wc, e, sw, bias, r, out, alpha, cfg):
        """out = r + alpha * bf16(dequant(x @ w^T) + bias) with w 2:4 sparse as compress_24 stores it (wc (N, K/2)
        int8, e (N, K/32) int32); reference kernels/csrc/gemm_sparse.cu:211-253."""
        self.gemm_sp_epi(x, sx, group, wc, e, sw, bias, out, EPI_RESID, r, alpha, None, cfg)

    def gemm_sp_epi(self, x, sx, group, wc, e, sw, bias, out, epi, resid, alpha, qs, cfg):
        """The sparse GEMM with gemm_i8's epilogues (BIAS, RESID, GLU, SILU_Q8, I32): the reference's gemm_sp widened
        (its kernel has the residual epilogue only). Same results as gemm_i8 on the decompressed weights."""
        _check(x.dtype == torch.int8 and wc.dtype == torch.int8 and e.dtype == torch.int32 and
               sx.dtype == torch.float32 and sw.dtype == torch.float32, "gemm_sp: dtypes")
        _check(x.stride(1) == 1 and wc.is_contiguous() and e.is_contiguous() and sx.stride(1) == 1 and
               out.stride(1) == 1 and (resid is None or resid.stride(1) == 1), "gemm_sp: strides")
        M, K = x.shape
        _check(wc.shape[1] * 2 == K and e.shape[1] * 32 == K and K % 128 == 0 and group % 128 == 0 and
               K % group == 0, "gemm_sp: K must be a multiple of 128 and of group, wc (N, K/2), e (N, K/32)")
        _check(epi != EPI_RESID or resid is not None, "gemm_sp: residual epilogue needs r")
        _check(epi != EPI_SILU_Q8 or (qs is not None and out.dtype == torch.int8), "gemm_sp: SILU_Q8 needs qs")
        if M == 0:
            return
        self._call("cohere_gemm_sp", _ptr(x), x.stride(0), _ptr(sx), sx.stride(0), int(group), _ptr(wc), _ptr(e),
                   _ptr(sw), _ptr(bias), _ptr(out), out.stride(0), int(epi), _ptr(resid),
                   resid.stride(0) if resid is not None else 0, float(alpha), _ptr(qs),
                   qs.stride(0) if qs is not None else 0, M, wc.shape[0], K, int(cfg), _stream())

    def gemm_sp_tiled(self, x, sx, group, wt, sw, bias, out, epi, resid, alpha, qs, cfg):
        """gemm_sp_epi with the weight in the stage-tiled layout of pack_24_tiled (wt uint8 (N/16, K/128, 1280)):
        the same results bit for bit, each DMA instruction reading one contiguous kilobyte."""
        _check(x.dtype == torch.int8 and wt.dtype == torch.uint8 and sx.dtype == torch.float32 and
               sw.dtype == torch.float32, "gemm_sp_tiled: dtypes")
        _check(x.stride(1) == 1 and wt.is_contiguous() and wt.dim() == 3 and wt.shape[2] == TILED_REC and
               sx.stride(1) == 1 and out.stride(1) == 1 and (resid is None or resid.stride(1) == 1),
               "gemm_sp_tiled: strides / layout")
        M, K = x.shape
        N = wt.shape[0] * 16
        _check(wt.shape[1] * 128 == K and group % 128 == 0 and K % group == 0,
               "gemm_sp_tiled: wt (N/16, K/128, 1280), group a multiple of 128 dividing K")
        _check(epi != EPI_RESID or resid is not None, "gemm_sp_tiled: residual epilogue needs resid")
        _check(epi != EPI_SILU_Q8 or (qs is not None and out.dtype == torch.int8), "gemm_sp_tiled: SILU_Q8 needs qs")
        if M == 0:
            return
        self._call("cohere_gemm_sp_tiled", _ptr(x), x.stride(0), _ptr(sx), sx.stride(0), int(group), _ptr(wt),
                   _ptr(sw), _ptr(bias), _ptr(out), out.stride(0), int(epi), _ptr(resid),
                   resid.stride(0) if resid is not None else 0, float(alpha), _ptr(qs),
                   qs.stride(0) if qs is not None else 0, M, N, K, int(cfg), _stream())

    # ---- int8 activation producers (bindings.cpp:44-46, 73-75) --------------------------------------------------

    def quantize_rows(self, x, q, s):
        """bf16 rows -> int8 with one fp32 scale per row (reference encoder_ops.cu:545-553)."""
        _check(x.dtype == torch.bfloat16 and x.stride(1) == 1 and q.is_contiguous() and q.dtype == torch.int8 and
               s.dtype == torch.float32, "quantize_rows: bf16 x, int8 contiguous q, fp32 s")
        rows, cols = x.shape
        _check(tuple(q.shape) == (rows, cols) and s.numel() >= rows, "quantize_rows: shapes")
        self._call("cohere_quantize_rows", _ptr(x), x.stride(0), _ptr(q), cols, _ptr(s), rows, cols, _stream())

    def layernorm_q8(self, x, w1, b1, eps1, w2, b2, eps2, hq, hs):
        """h = LN(x) as int8 hq + per-row scale hs; with w2: x = LN1(x) in place, h = LN2(x) (encoder_ops.cu:522)."""
        _check(x.dtype == torch.bfloat16 and x.stride(1) == 1 and hq.is_contiguous() and hq.dtype == torch.int8 and
               hs.dtype == torch.float32, "layernorm_q8: dtypes/strides")
        rows, cols = x.shape
        _check(hq.shape[1] == cols and hs.numel() >= rows, "layernorm_q8: shapes")
        self._call("cohere_layernorm_q8", _ptr(x), x.stride(0), _ptr(w1), _ptr(b1), float(eps1), _ptr(w2), _ptr(b2),
                   float(eps2), _ptr(hq), cols, _ptr(hs), rows, cols, _stream())

    def layernorm(self, x, w1, b1, eps1, w2, b2, eps2, h):
        """h = LN(x) in bf16; with w2: x = LN1(x) in place, h = LN2(x); h may be x (encoder_ops.cu:501-520)."""
        _check(x.dtype == torch.bfloat16 and h.dtype == torch.bfloat16 and x.stride(1) == 1 and h.stride(1) == 1,
               "layernorm: bf16 rows with unit column stride")
        rows, cols = x.shape
        _check(tuple(h.shape) == (rows, cols), "layernorm: shapes")
        self._call("cohere_layernorm", _ptr(x), x.stride(0), _ptr(w1), _ptr(b1), float(eps1), _ptr(w2), _ptr(b2),
                   float(eps2), _ptr(h), h.stride(0), rows, cols, _stream())

    def _dwconv_checks(self, x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi):
        _check(x.dtype == torch.bfloat16 and x.is_contiguous() and w.dtype == torch.float32 and w.is_contiguous() and
               w.dim() == 2 and w.shape[1] == 9, "dwconv_bn_silu: contiguous bf16 x and fp32 (C, 9) weights")
        _check(all(t.dtype == torch.float32 for t in (cb, bn_scale, bn_shift)) and
               seq_lo.dtype == torch.int32 and seq_hi.dtype == torch.int32, "dwconv_bn_silu: dtypes")
        _check(seq_lo.numel() >= x.shape[0] and seq_hi.numel() >= x.shape[0], "dwconv_bn_silu: lo/hi per row")

    def dwconv_bn_silu(self, x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi, y):
        """y = silu(bn(depthwise conv(x))) per packed sequence, bf16 (encoder_ops.cu:643-656)."""
        self._dwconv_checks(x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi)
        _check(y.dtype == torch.bfloat16 and y.is_contiguous() and y.shape == x.shape, "dwconv_bn_silu: y")
        self._call("cohere_dwconv_bn_silu", _ptr(x), _ptr(w), _ptr(cb), _ptr(bn_scale), _ptr(bn_shift), _ptr(seq_lo),
                   _ptr(seq_hi), _ptr(y), x.shape[0], x.shape[1], w.shape[1], _stream())

    def dwconv_bn_silu_q8(self, x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi, hq, hs):
        """dwconv_bn_silu with int8 rows hq and per-row scales hs (encoder_ops.cu:658-674)."""
        self._dwconv_checks(x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi)
        _check(hq.dtype == torch.int8 and hq.is_contiguous() and hq.shape == x.shape and hs.dtype == torch.float32 and
               hs.numel() >= x.shape[0], "dwconv_bn_silu_q8: hq, hs")
        self._call("cohere_dwconv_bn_silu_q8", _ptr(x), _ptr(w), _ptr(cb), _ptr(bn_scale), _ptr(bn_shift),
                   _ptr(seq_lo), _ptr(seq_hi), _ptr(hq), _ptr(hs), x.shape[0], x.shape[1], w.shape[1], _stream())

    # ---- encoder attention and layer loop (bindings.cpp:66, 85) ---------------------------------------------------

    def relpos_attention(self, qkv, rk, bu, bv, tiles, rel_off, max_len, scale, out):
        """out = relative-position self-attention of qkv per packed sequence; tiles (n, 4) int32 (sequence start,
        length, first query row, 0) per 64-query tile (encoder_ops.cu:676-707). Head size 80 or 160."""
        _check(qkv.is_contiguous() and out.is_contiguous() and rk.is_contiguous() and tiles.is_contiguous(),
               "relpos_attention: contiguous tensors expected")
        H, D = bu.shape
        _check(bu.dtype == bv.dtype == qkv.dtype == rk.dtype == out.dtype == torch.bfloat16 and
               tiles.dtype == torch.int32, "relpos_attention: bf16 tensors and int32 tiles")
        _check(qkv.shape[1] == 3 * H * D and rk.shape[1] == H * D and out.shape[1] == H * D,
               "relpos_attention: shapes")
        self._call("cohere_relpos_attention", _ptr(qkv), _ptr(rk), rk.shape[0], _ptr(bu.contiguous()),
                   _ptr(bv.contiguous()), _ptr(tiles), tiles.shape[0], H, D, int(rel_off), int(max_len),
                   float(scale), _ptr(out), _stream())

    def encoder_workspace_bytes(self, rows: int, group: int) -> int:
        return int(self._lib.cohere_encoder_workspace_bytes(int(rows), int(group)))

    def _encoder_args(self, x, layers, eps, tiles, lo, hi, rel_off, max_len, scale, int8, cfg):
        """The checked C arguments of an encoder_layers call (None when there is nothing to do)."""
        _check(x.dtype == torch.bfloat16 and x.is_contiguous() and x.dim() == 2 and x.shape[1] == 1280,
               "encoder_layers: x (N, 1280) contiguous bf16")
        n_ref, n_fields = 53, 57
        _check(all(len(ly) in (n_ref, n_fields) for ly in layers),
               f"encoder_layers: {n_ref} or {n_fields} tensors per layer")
        _check(len(eps) == 5 * len(layers), "encoder_layers: 5 epsilons per layer")
        for ly in layers:
            for t in ly:
                _check(t.numel() == 0 or t.is_contiguous(), "encoder_layers: layer tensors must be contiguous")
        rows = x.shape[0]
        cfg = [int(c) for c in cfg]
        _check(len(cfg) >= 5, "encoder_layers: cfg needs at least 5 entries")
        if rows == 0 or not layers:
            return None
        H, D = layers[0][22].shape  # bias_u: (heads, head size)
        ptrs = (ctypes.c_void_p * (n_fields * len(layers)))(
            *[t.data_ptr() if t.numel() > 0 else None for ly in layers
              for t in (*ly, *([_EMPTY] * (n_fields - len(ly))))])
        eps_arr = (ctypes.c_double * len(eps))(*[float(e) for e in eps])
        cfg_arr = (ctypes.c_int64 * len(cfg))(*cfg)
        return (_ptr(x), rows, ptrs, len(layers), eps_arr, _ptr(tiles), tiles.shape[0], _ptr(lo), _ptr(hi),
                int(rel_off), int(max_len), layers[0][24].shape[0], float(scale), H, D, int(bool(int8)), cfg_arr,
                len(cfg)), cfg

    def encoder_layers(self, x, layers, eps, tiles, lo, hi, rel_off, max_len, scale, int8, cfg):
        """Every layer on packed frames x (N, 1280) bf16, in place, launched from native code
        (kernels/csrc/encoder_loop.cpp:50-124). layers: per layer the tensors in the reference's field order
        (fast_encoder.py:121-130), 53 of them, optionally followed by 4 more (the feed-forwards' first linears in
        2:4 form: ff1 kept, ff1 selectors, ff2 kept, ff2 selectors); empty tensors stand for absent ones. int8: the
        W8A8 branch on the quantized fields, else the bf16 branch on the bf16 weights (encoder_loop.cpp:101-124).
        The workspace is allocated here, through torch's caching allocator."""
        packed = self._encoder_args(x, layers, eps, tiles, lo, hi, rel_off, max_len, scale, int8, cfg)
        if packed is None:
            return
        args, cfg = packed
        nbytes = int(self._lib.cohere_encoder_branch_workspace_bytes(x.shape[0], cfg[4], int(bool(int8))))
        _check(nbytes >= 0, "encoder_layers: bad feed-forward group")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        self._call("cohere_encoder_layers", *args, _ptr(ws), nbytes, _stream())

    def encoder_layers_noalloc(self, x, layers, eps, tiles, lo, hi, rel_off, max_len, scale, int8, cfg):
        """encoder_layers with the library's own per-GPU scratch array in place of a workspace: allocates nothing
        (no counterpart in the reference; for callers that cannot allocate). At most ~3900 int8-layer rows; calls
        that overlap on one GPU race."""
        packed = self._encoder_args(x, layers, eps, tiles, lo, hi, rel_off, max_len, scale, int8, cfg)
        if packed is None:
            return
        self._call("cohere_encoder_layers_noalloc", *packed[0], _stream())

    # ---- decoder projections (bindings.cpp:55-56) -----------------------------------------------------------

    def dec_w8_linear(self, x, w, sw, bias, y, relu, bn, splits, ws, counters):
        """y = x @ dequant(w)^T + bias (relu), M <= 64, w in prepare_w8's layout (reference dec_w8.cu:205-234)."""
        _check(x.dtype == torch.bfloat16 and w.dtype == torch.uint8 and sw.dtype == torch.float32 and
               y.dtype == torch.bfloat16, "dec_w8_linear: dtypes")
        M, K = x.shape
        N = w.shape[0]
        _check(M <= 64 and x.stride(1) == 1 and w.is_contiguous() and w.shape[1] == K and y.stride(1) == 1,
               "dec_w8_linear: M <= 64, unit column strides, contiguous w")
        if M == 0:
            return
        self._call("cohere_dec_w8_linear", _ptr(x), x.stride(0), _ptr(w), _ptr(sw), _ptr(bias), _ptr(y), y.stride(0),
                   int(bool(relu)), int(bn), int(splits), _ptr(ws), ws.numel() if ws is not None else 0,
                   _ptr(counters), counters.numel() if counters is not None else 0, M, N, K, _stream())

    def linear_bf16(self, x, w, bias, y, relu=False):
        """y = x @ w^T + bias (relu) for bf16 weights, M <= 64: the decoder's o / cross-q / cross-o projections
        (the reference runs them in Triton, kernels/decoder_kernels.py:55-66)."""
        _check(x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and y.dtype == torch.bfloat16,
               "linear_bf16: bf16 expected")
        M, K = x.shape
        _check(M <= 64 and x.stride(1) == 1 and w.is_contiguous() and w.shape[1] == K and y.stride(1) == 1,
               "linear_bf16: M <= 64, unit column strides, contiguous w")
        if M == 0:
            return
        self._call("cohere_linear_bf16", _ptr(x), x.stride(0), _ptr(w), _ptr(bias), _ptr(y), y.stride(0),
                   int(bool(relu)), M, w.shape[0], K, _stream())

    def dec_linear_fused(self, x, w, sw, bias, y, epilogue=DEC_EP_NONE, ln=None):
        """A decoder projection with dec_add_ln folded in (no single counterpart in the reference, whose step runs
        dec_add_ln between the projections, stream_decoder.py:176-199): ln = (weight, bias, eps) normalises x's rows
        in the kernel first (512 <= K <= 1024); epilogue DEC_EP_RELU applies ReLU, DEC_EP_RESID adds the result into
        y in place (y = bf16(y + bf16(r))). sw None: bf16 weights w; else int8 weights in prepare_w8's layout."""
        _check(x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16 and
               (w.dtype == torch.uint8 if sw is not None else w.dtype == torch.bfloat16), "dec_linear_fused: dtypes")
        M, K = x.shape
        _check(M <= 64 and x.stride(1) == 1 and w.is_contiguous() and w.shape[1] == K and y.stride(1) == 1 and
               y.shape[0] == M and y.shape[1] == w.shape[0], "dec_linear_fused: M <= 64, unit column strides, "
               "contiguous w, y (M, N)")
        if M == 0:
            return
        lw, lb, eps = ln if ln is not None else (None, None, 0.0)
        self._call("cohere_dec_linear_fused", _ptr(x), x.stride(0), _ptr(lw), _ptr(lb), float(eps), _ptr(w),
                   _ptr(sw), _ptr(bias), _ptr(y), y.stride(0), int(epilogue), M, w.shape[0], K, _stream())

    # ---- decoder step (bindings.cpp:77-84) -------------------------------------------------------------------------

    def dec_embed(self, active, tok, pos, emb, ptab, w0, b0, eps0, w1, b1, eps1, x, h):
        """x = LN0(embed[tok[s]] + pos_table[pos[s]]), h = LN1(x) for s = active[r] (decoder_ops.cu:208-219)."""
        _check(x.is_contiguous() and h.is_contiguous() and x.dtype == h.dtype == emb.dtype == torch.bfloat16,
               "dec_embed: contiguous bf16 x, h")
        _check(active.dtype == torch.int32 and tok.dtype == torch.int64 and pos.dtype == torch.int32,
               "dec_embed: int32 active/pos, int64 tok")
        rows, width = x.shape
        _check(emb.shape[1] == width and ptab.shape[1] == width, "dec_embed: widths")
        self._call("cohere_dec_embed", _ptr(active), rows, _ptr(tok), _ptr(pos), _ptr(emb), _ptr(ptab), _ptr(w0),
                   _ptr(b0), float(eps0), _ptr(w1), _ptr(b1), float(eps1), _ptr(x), _ptr(h), width, _stream())

    def dec_add_ln(self, x, y, w, b, eps, h):
        """x = bf16(x + y) in place, h = LN(x) (decoder_ops.cu:221-233)."""
        _check(x.is_contiguous() and h.is_contiguous() and y.stride(1) == 1, "dec_add_ln: contiguous x, h")
        rows, width = x.shape
        self._call("cohere_dec_add_ln", _ptr(x), _ptr(y), y.stride(0), _ptr(w), _ptr(b), float(eps), _ptr(h), rows,
                   width, _stream())

    def _att_checks(self, q, k, out, part, splits):
        _check(k.dim() == 4 and k.shape[3] == 128 and k.is_contiguous() and q.stride(1) == 1 and out.is_contiguous(),
               "dec_attention: caches (slots, H, T, 128) contiguous, q with unit column stride")
        rows, H = q.shape[0], k.shape[1]
        _check(splits == 1 or (part is not None and part.numel() >= rows * H * splits * 130),
               "dec_attention: splits > 1 needs part")
        return rows, H

    def dec_attention(self, self_attn, active, q, k, v, n, scale, splits, part, out):
        """softmax(q k^T scale) v of one new token per row over its slot's bf16 cache (decoder_ops.cu:235-262)."""
        rows, H = self._att_checks(q, k, out, part, splits)
        self._call("cohere_dec_attention", int(bool(self_attn)), _ptr(active), rows, _ptr(q), q.stride(0), _ptr(k),
                   _ptr(v), _ptr(n), k.shape[0], H, k.shape[2], float(scale), int(splits), _ptr(part),
                   part.numel() if part is not None else 0, _ptr(out), _stream())

    def dec_attention_q8(self, self_attn, active, q, k8, v8, ks, vs, n, scale, splits, part, out):
        """dec_attention over int8 caches with one scale per 128-vector (decoder_ops.cu:264-290)."""
        rows, H = self._att_checks(q, k8, out, part, splits)
        _check(k8.dtype == torch.int8 and ks.dtype == torch.float32 and ks.is_contiguous() and vs.is_contiguous(),
               "dec_attention_q8: int8 caches, fp32 scales")
        self._call("cohere_dec_attention_q8", int(bool(self_attn)), _ptr(active), rows, _ptr(q), q.stride(0),
                   _ptr(k8), _ptr(v8), _ptr(ks), _ptr(vs), _ptr(n), k8.shape[0], H, k8.shape[2], float(scale), int(splits),
                   _ptr(part), part.numel() if part is not None else 0, _ptr(out), _stream())

    def dec_pick(self, logits, active, dummy, tok, pos, finished, forced, plen, limit, out, pad, eos):
        """Greedy choice, forced prompt and end bookkeeping per active slot (decoder_ops.cu:304-314)."""
        _check(logits.is_contiguous() and logits.shape[1] % 8 == 0, "dec_pick: contiguous logits, V % 8 == 0")
        _check(tok.dtype == torch.int64 and forced.dtype == torch.int64 and out.dtype == torch.int64 and
               finished.dtype == torch.uint8, "dec_pick: dtypes")
        rows, V = logits.shape
        self._call("cohere_dec_pick", _ptr(logits), rows, V, _ptr(active), int(dummy), _ptr(tok), _ptr(pos),
                   _ptr(finished), _ptr(forced), forced.shape[1], _ptr(plen), _ptr(limit), _ptr(out), out.shape[1],
                   int(pad), int(eos), _stream())

    def dec_pick_embed(self, logits, active, dummy, tok, pos, finished, forced, plen, limit, out, pad, eos, emb, ptab,
                       w0, b0, eps0, w1, b1, eps1, x, h, flags=None):
        """dec_pick, then each row's next embedding as dec_embed computes it (x, h), and, with flags (pinned uint8 per
        slot on the host), the stepped slots' end flags written there (no single counterpart in the reference: its
        step ends with dec_pick and a copy of the flags, and the next one starts with dec_embed)."""
        _check(logits.is_contiguous() and logits.shape[1] % 8 == 0, "dec_pick_embed: contiguous logits, V % 8 == 0")
        _check(tok.dtype == torch.int64 and forced.dtype == torch.int64 and out.dtype == torch.int64 and
               finished.dtype == torch.uint8, "dec_pick_embed: dtypes")
        _check(x.is_contiguous() and h.is_contiguous() and x.dtype == h.dtype == emb.dtype == torch.bfloat16 and
               x.shape[0] == logits.shape[0], "dec_pick_embed: contiguous bf16 x, h, a row per logits row")
        _check(flags is None or (flags.device.type == "cpu" and flags.is_pinned() and flags.dtype == torch.uint8 and
                                 flags.numel() >= finished.numel()), "dec_pick_embed: flags pinned uint8, one per slot")
        rows, V = logits.shape
        width = x.shape[1]
        _check(emb.shape[1] == width and ptab.shape[1] == width, "dec_pick_embed: widths")
        self._call("cohere_dec_pick_embed", _ptr(logits), rows, V, _ptr(active), int(dummy), _ptr(tok), _ptr(pos),
                   _ptr(finished), _ptr(forced), forced.shape[1], _ptr(plen), _ptr(limit), _ptr(out), out.shape[1],
                   int(pad), int(eos), _ptr(emb), _ptr(ptab), _ptr(w0), _ptr(b0), float(eps0), _ptr(w1), _ptr(b1),
                   float(eps1), _ptr(x), _ptr(h), width, _ptr(flags), _stream())

    def dec_scatter_kv(self, kv, slot_of, frame_of, ck, cv):
        """Cross-attention keys/values of packed frames into their slots (decoder_ops.cu:316-327)."""
        L, S, H, T = ck.shape[:4]
        _check(kv.is_contiguous() and kv.shape[1] == L * 2 * H * 128 and ck.is_contiguous() and cv.is_contiguous(),
               "dec_scatter_kv: shapes")
        self._call("cohere_dec_scatter_kv", _ptr(kv), kv.shape[0], _ptr(slot_of), _ptr(frame_of), _ptr(ck),
                   _ptr(cv), L, S, H, T, _stream())

    def dec_scatter_kv_q8(self, kv, slot_of, frame_of, ck, cv, cks, cvs):
        """The same into int8 caches with one scale per 128-vector (decoder_ops.cu:292-302)."""
        L, S, H, T = ck.shape[:4]
        _check(kv.is_contiguous() and kv.shape[1] == L * 2 * H * 128 and ck.dtype == torch.int8,
               "dec_scatter_kv_q8: shapes")
        self._call("cohere_dec_scatter_kv_q8", _ptr(kv), kv.shape[0], _ptr(slot_of), _ptr(frame_of), _ptr(ck),
                   _ptr(cv), _ptr(cks), _ptr(cvs), L, S, H, T, _stream())


_lib = load_library()
ext = _Ext(_lib)
