"""cohere_encoder_layers_noalloc (no counterpart in the reference: for callers that cannot allocate device memory)
against cohere_encoder_layers with a caller workspace, through the C ABI: bit-identical outputs on two calls in a
row, the second smaller (the scratch array keeps the first call's contents), no device memory taken by the call, and
a call beyond the scratch size refused before anything is launched.

"No device memory taken" is checked two ways: torch's allocator (memory_allocated) is unchanged, and the device's
free memory (hipMemGetInfo through torch.cuda.mem_get_info) does not drop by more than 2 MiB, so a hipMalloc of the
workspace (23 MB at 3000 rows for the QKV buffer alone) inside the native call would fail the test too. The runtime
places the library's static 64 MiB array in device memory when it loads the code object that holds it (lazily, on
the first launch from that file); one small warm-up call does that before anything is measured."""

from __future__ import annotations

import pytest
import torch

from encoder_helpers import product_layers

pytestmark = pytest.mark.gpu


def _run(ext, fn, layers, x, lengths, meta=None):
    from kernels.fast_encoder import metadata

    meta = metadata(lengths, x.device) if meta is None else meta
    fn(x, layers.layer_tensors, layers.layer_eps, meta["tiles"], meta["lo"], meta["hi"], layers.rel_off,
       meta["max_len"], layers.scale, layers.int8, layers.configs(x.shape[0]))


def test_noalloc_matches_workspace_entry_point(gpu):
    from kernels.cuda_ext import ext
    from kernels.fast_encoder import metadata

    layers = product_layers(gpu, 2, seed=61, sparse=True, sparse_w1=True)
    g = torch.Generator().manual_seed(62)
    warm = torch.randn(5, 1280, generator=g).to(torch.bfloat16).to(gpu)
    _run(ext, ext.encoder_layers_noalloc, layers, warm, [5])
    torch.cuda.synchronize()
    for lengths in ([375] * 8, [120, 1, 57]):  # config 2's 3000 rows, then a smaller call
        x = torch.randn(sum(lengths), 1280, generator=g).to(torch.bfloat16).to(gpu)
        want, got = x.clone(), x.clone()
        _run(ext, ext.encoder_layers, layers, want, lengths)
        meta = metadata(lengths, gpu)
        torch.cuda.synchronize()
        before, free_before = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
        _run(ext, ext.encoder_layers_noalloc, layers, got, lengths, meta)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert free_before - torch.cuda.mem_get_info()[0] <= 2 << 20
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), lengths
        assert not torch.equal(got.view(torch.int16), x.view(torch.int16))


def test_noalloc_refuses_rows_beyond_its_scratch(gpu):
    from kernels.cuda_ext import ext

    layers = product_layers(gpu, 1, seed=63)
    lengths = [500] * 9  # 4500 rows: the int8 layers' buffers exceed the 64 MiB array
    x = torch.zeros(sum(lengths), 1280, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="scratch"):
        _run(ext, ext.encoder_layers_noalloc, layers, x, lengths)
    assert torch.count_nonzero(x) == 0
