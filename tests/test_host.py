"""Host side, CPU only: the C-ABI library loads and exports every declared symbol, rejects bad arguments with a clear
error before touching the GPU, and the host mirrors of the reference interface (kernels/sparse.py, prepare_w8,
quantize_rows) produce the oracle's bytes."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_bits, linear_inputs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    from kernels import cuda_ext

    header = open(os.path.join(ROOT, "include", "cohere_hip.h")).read()
    declared = set(re.findall(r"\b(cohere_[a-z0-9_]+)\s*\(", header))
    assert declared == set(cuda_ext.EXPORTS)
    lib = ctypes.CDLL(cuda_ext.LIB_PATH)
    for name in declared:
        assert hasattr(lib, name), name
    assert b"gfx950" in cuda_ext._lib.cohere_version()


def test_epi_constants_match_reference_surface():
    from kernels import cuda_ext as ce

    assert (ce.EPI_BIAS, ce.EPI_SILU, ce.EPI_RELU, ce.EPI_RESID, ce.EPI_GLU, ce.EPI_SILU_Q8, ce.EPI_CONV_RELU) == \
        tuple(range(7))


def _raw(lib, name, *args):
    rc = getattr(lib, name)(*args)
    return rc, lib.cohere_last_error().decode()


def test_c_abi_rejects_bad_arguments_without_launching():
    from kernels.cuda_ext import _lib as lib

    fake = 1 << 20  # never dereferenced: every call below is rejected by argument checks first
    # K not a multiple of 64
    rc, msg = _raw(lib, "cohere_gemm_i8", fake, 96, fake, 1, 96, fake, fake, None, fake, 64, 0, None, 0, 1.0, None, 0,
                   16, 64, 96, 0, None)
    assert rc != 0 and "K=96" in msg
    # unknown reference config id
    rc, msg = _raw(lib, "cohere_gemm_i8", fake, 128, fake, 1, 128, fake, fake, None, fake, 64, 0, None, 0, 1.0, None,
                   0, 16, 64, 128, 2, None)
    assert rc != 0 and "unknown config 2" in msg
    # residual epilogue without resid
    rc, msg = _raw(lib, "cohere_gemm_i8", fake, 128, fake, 1, 128, fake, fake, None, fake, 64, 3, None, 0, 1.0, None,
                   0, 16, 64, 128, 0, None)
    assert rc != 0 and "resid" in msg
    # sparse K not a multiple of 128
    rc, msg = _raw(lib, "cohere_gemm_sp", fake, 192, fake, 1, 192, fake, fake, fake, None, fake, 64, 0, None, 0, 1.0,
                   None, 0, 16, 64, 192, 0, None)
    assert rc != 0 and "multiple of 128" in msg
    # more than 64 rows for the skinny GEMM
    rc, msg = _raw(lib, "cohere_dec_w8_linear", fake, 1024, fake, fake, None, fake, 1024, 0, 64, 1, None, 0, None, 0,
                   65, 1024, 1024, None)
    assert rc != 0 and "64 rows" in msg
    # the reference's bn / splits checks (dec_w8.cu:210-213)
    rc, msg = _raw(lib, "cohere_dec_w8_linear", fake, 1024, fake, fake, None, fake, 1024, 0, 48, 1, None, 0, None, 0,
                   8, 1024, 1024, None)
    assert rc != 0 and "bn 48" in msg
    rc, msg = _raw(lib, "cohere_dec_w8_linear", fake, 1024, fake, fake, None, fake, 1024, 0, 64, 4, None, 0, None, 0,
                   8, 1024, 1024, None)
    assert rc != 0 and "workspace" in msg
    rc, msg = _raw(lib, "cohere_quantize_rows", fake, 1284, fake, 1284, fake, 4, 1284, None)
    assert rc != 0 and "multiple of 8" in msg
    # bf16 GEMM: the reference's config ids, K % 32, N % 64
    rc, msg = _raw(lib, "cohere_gemm_bf16", fake, 96, fake, None, fake, 64, 0, None, 0, 1.0, 4, 64, 96, 7, None)
    assert rc != 0 and "unknown config 7" in msg
    rc, msg = _raw(lib, "cohere_gemm_bf16", fake, 80, fake, None, fake, 64, 0, None, 0, 1.0, 4, 64, 80, 8, None)
    assert rc != 0 and "multiple of 32" in msg
    rc, msg = _raw(lib, "cohere_gemm_bf16", fake, 96, fake, None, fake, 48, 0, None, 0, 1.0, 4, 48, 96, 8, None)
    assert rc != 0 and "N must be" in msg
    rc, msg = _raw(lib, "cohere_gemm_bf16", fake, 96, fake, None, fake, 64, 5, None, 0, 1.0, 4, 64, 96, 8, None)
    assert rc != 0 and "unknown epilogue 5" in msg  # SILU_Q8 is int8-only
    # front end: channel counts, empty batches are no-ops
    rc, msg = _raw(lib, "cohere_sub_conv0_dw", fake, 1280, fake, fake, 3, fake, fake, fake, fake, fake, 100, None)
    assert rc != 0 and "multiple of 64" in msg
    rc, msg = _raw(lib, "cohere_sub_dw", fake, fake, fake, fake, 3, fake, fake, fake, 32, 12, None)
    assert rc != 0 and "C % 8" in msg
    # decoder attention: caches of 2^32 elements or more (the kernels' offsets are 32-bit)
    rc, msg = _raw(lib, "cohere_dec_attention_q8", 1, fake, 64, fake, 3072, fake, fake, fake, fake, fake, 1 << 16, 8,
                   512, 0.1, 1, None, 0, fake, None)
    assert rc != 0 and "2^32" in msg
    rc, msg = _raw(lib, "cohere_dec_attention", 0, fake, 64, fake, 1024, fake, fake, fake, 0, 8, 512, 0.1, 1, None,
                   0, fake, None)
    assert rc != 0 and "2^32" in msg
    assert _raw(lib, "cohere_logmel_features", None, None, 0, 0, None, None, None, 0.97, None, 0, None, None)[0] == 0
    assert lib.cohere_logmel_workspace_bytes(100) == 100 * 128 * 4


def test_ext_raises_runtime_error_like_torch_check():
    from kernels.cuda_ext import EPI_BIAS, ext

    a = torch.zeros(4, 96, dtype=torch.int8)
    with pytest.raises(RuntimeError):
        ext.gemm_i8(a, torch.ones(4, 1), 96, torch.zeros(16, 96, dtype=torch.int8), torch.ones(16), None,
                    torch.empty(4, 16, dtype=torch.bfloat16), EPI_BIAS, None, 1.0, None, 0)
    with pytest.raises(RuntimeError):  # int8 a expected
        ext.gemm_i8(a.float(), torch.ones(4, 1), 128, torch.zeros(16, 128, dtype=torch.int8), torch.ones(16), None,
                    torch.empty(4, 16, dtype=torch.bfloat16), EPI_BIAS, None, 1.0, None, 0)


# ---- host mirrors of the reference interface -------------------------------------------------------------------------

def test_sparse_module_matches_golden_and_oracle():
    from kernels.sparse import compress_24, decompress_24, prune_24_magnitude

    g = np.load(os.path.join(ROOT, "tests", "golden", "compress24_golden.npz"))
    k, e = compress_24(torch.from_numpy(g["patterns_w"]))
    assert np.array_equal(k.numpy(), g["patterns_kept"]) and np.array_equal(e.numpy(), g["patterns_words"])
    k, e = compress_24(torch.from_numpy(g["random_q"]))
    assert np.array_equal(k.numpy(), g["random_kept"]) and np.array_equal(e.numpy(), g["random_words"])
    assert np.array_equal(decompress_24(k, e).numpy(), g["random_q"])
    assert np.array_equal(prune_24_magnitude(torch.from_numpy(g["random_w"])).numpy(), g["random_pruned"])
    _, w, _ = linear_inputs(4, 64, 512, seed=21)
    wp = prune_24_magnitude(w.float())
    assert np.array_equal(wp.numpy(), O.prune_24(w.float().numpy()))
    with pytest.raises(AssertionError):
        compress_24(torch.ones(2, 32, dtype=torch.int8))


def test_weight_quantizers_match_oracle():
    from kernels.fast_encoder import quantize_rows
    from kernels.stream_decoder import prepare_w8, unprepare_w8

    _, w, _ = linear_inputs(4, 128, 1024, seed=22)
    q, s = quantize_rows(w)
    qo, so = O.quantize_weight_rows(bf16_bits(w))
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)
    u, s8 = prepare_w8(w)
    uo, s8o = O.prepare_w8(bf16_bits(w))
    assert np.array_equal(u.numpy(), uo) and np.array_equal(s8.numpy(), s8o)
    assert np.array_equal(unprepare_w8(u).numpy(), qo)


def test_pack_24_tiled_matches_c_abi_and_round_trips():
    """The stage-tiled 2:4 layout: kernels.sparse.pack_24_tiled (torch) and the library's cohere_pack_24_tiled (host
    loops) give the same bytes, and every record decodes back to compress_24's kept values and selectors through the
    layout's own definition (chunk i = row i // 4, logical chunk (i % 4) ^ ((i // 8) % 4); selectors at 1024 + 16 r,
    words 0-1 and 2-3 swapped in rows 8-15)."""
    from kernels.cuda_ext import _lib as lib
    from kernels.sparse import TILED_REC, compress_24, pack_24_tiled, prune_24_magnitude

    g = torch.Generator().manual_seed(5)
    N, K = 48, 384
    w = prune_24_magnitude(torch.randn(N, K, generator=g))
    q = (torch.randint(-127, 128, (N, K), generator=g) * (w != 0)).to(torch.int8)
    kept, words = compress_24(q)
    t = pack_24_tiled(kept, words)
    assert tuple(t.shape) == (N // 16, K // 128, TILED_REC)
    assert lib.cohere_pack_24_tiled_bytes(N, K) == t.numel() and lib.cohere_pack_24_tiled_bytes(40, K) == -1
    out = np.zeros(t.numel(), np.uint8)
    assert lib.cohere_pack_24_tiled(kept.numpy().ctypes.data, words.numpy().ctypes.data, N, K, out.ctypes.data) == 0
    assert np.array_equal(out, t.numpy().reshape(-1))
    tn = t.numpy()
    back_k, back_e = np.zeros_like(kept.numpy()), np.zeros_like(words.numpy())
    for rb in range(N // 16):
        for kt in range(K // 128):
            rec = tn[rb, kt]
            for i in range(64):
                r, c = rb * 16 + i // 4, (i % 4) ^ ((i // 8) % 4)
                back_k[r, kt * 64 + c * 16:kt * 64 + c * 16 + 16] = rec[16 * i:16 * i + 16].view(np.int8)
            for r in range(16):
                stored = rec[1024 + 16 * r:1040 + 16 * r].view(np.int32)
                back_e[rb * 16 + r, kt * 4:kt * 4 + 4] = stored[[2, 3, 0, 1]] if r >= 8 else stored
    assert np.array_equal(back_k, kept.numpy()) and np.array_equal(back_e, words.numpy())
