"""2:4 structured sparsity of int8 weights: pruning and the compressed storage the sparse GEMM reads.

Mirrors the reference's kernels/sparse.py call surface for this path (compress_24, prune_24_magnitude; sparse.py:26-46).
The storage format is the reference's, unchanged: per group of four along K the two kept values in increasing
position order (nonzero positions first, completed with zero positions when a group has fewer than two nonzeros),
and a 4-bit selector i0 | i1 << 2 per group, eight to an int32 word, the lowest K in the lowest nibble. On gfx950 that
is exactly the A operand and index register of v_smfmac_i32_16x16x128_i8 (a lane holds 16 kept bytes and the word of
their 32 K positions), so the weights go to the kernel as stored.

SparseGPT calibration pruning (reference sparsegpt_24 / prune_model) needs real weights and audio and is out of
scope; prune_24_magnitude is the pruning used for synthetic weights.

    wc, e = compress_24(w_int8)          # (N, K/2) int8, (N, K/32) int32
    w_dense = decompress_24(wc, e)       # back to (N, K)
"""

from __future__ import annotations

import torch

# the kept pair (i0, i1) for each 4-bit nonzero mask of a group (bit p set when position p is nonzero): nonzero
# positions first, zero positions after, both ascending; the first two, sorted. Masks with three or four bits set
# cannot be stored (marked -1).
_PAIRS = []
for _mask in range(16):
    _nz = [p for p in range(4) if _mask >> p & 1]
    if len(_nz) > 2:
        _PAIRS.append((-1, -1))
        continue
    _sel = sorted((_nz + [p for p in range(4) if not _mask >> p & 1])[:2])
    _PAIRS.append(tuple(_sel))


def compress_24(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 (N, K) with at most two nonzeros in every group of four along K -> (kept (N, K/2) int8, selectors
    (N, K/32) int32). Raises AssertionError like the reference when K % 32 != 0 or a group has more than two."""
    n, k = w.shape
    assert w.dtype == torch.int8 and k % 32 == 0
    g = w.reshape(n, k // 4, 4)
    bits = torch.tensor([1, 2, 4, 8], device=w.device, dtype=torch.int64)
    mask = ((g != 0).to(torch.int64) * bits).sum(-1)  # (n, k/4)
    pairs = torch.tensor(_PAIRS, device=w.device, dtype=torch.int64)[mask]  # (n, k/4, 2)
    assert bool((pairs[..., 0] >= 0).all()), "more than two nonzero values in a group of four"
    kept = torch.gather(g, -1, pairs).reshape(n, k // 2).contiguous()
    nib = (pairs[..., 0] | (pairs[..., 1] << 2)).reshape(n, k // 32, 8)
    shifts = torch.arange(0, 32, 4, device=w.device, dtype=torch.int64)
    words = (nib << shifts).sum(-1)
    words = (words - ((words >> 31) << 32)).to(torch.int32)  # two's complement of the 32-bit pattern
    return kept, words.contiguous()


def decompress_24(kept: torch.Tensor, words: torch.Tensor) -> torch.Tensor:
    """The dense int8 (N, K) matrix of a compressed one."""
    n, k2 = kept.shape
    k = 2 * k2
    shifts = torch.arange(0, 32, 4, device=kept.device, dtype=torch.int64)
    nib = ((words.to(torch.int64) & 0xFFFFFFFF)[..., None] >> shifts) & 15  # (n, k/32, 8)
    nib = nib.reshape(n, k // 4)
    pos = torch.stack([nib & 3, nib >> 2], -1)  # (n, k/4, 2)
    out = torch.zeros(n, k // 4, 4, dtype=torch.int8, device=kept.device)
    out.scatter_(-1, pos, kept.reshape(n, k // 4, 2))
    return out.reshape(n, k)


def prune_24_magnitude(w: torch.Tensor) -> torch.Tensor:
    """w with the two smallest-magnitude values of every four along K set to zero (reference sparse.py:42-46). Of
    equal magnitudes the lower position is kept (the reference's topk leaves that order unspecified)."""
    g = w.reshape(w.shape[0], -1, 4)
    order = torch.sort(g.float().abs(), dim=-1, descending=True, stable=True).indices
    keep = torch.zeros_like(g, dtype=torch.bool).scatter_(-1, order[..., :2], True)
    return torch.where(keep, g, torch.zeros((), dtype=g.dtype, device=g.device)).reshape(w.shape)


TILED_REC = 1280  # bytes per (16-channel block, 128-wide K stage) record of the stage-tiled layout


def pack_24_tiled(kept: torch.Tensor, words: torch.Tensor) -> torch.Tensor:
    """compress_24's storage rearranged for the gfx950 sparse GEMM's loads (ext.gemm_sp_tiled; load time, on the
    tensors' device): uint8 (N/16, K/128, 1280), one record per block of 16 channels and 128-wide K stage -- the 64
    16-byte chunks of the block's kept values of the stage (chunk i: row i // 4, its chunk (i % 4) ^ ((i // 8) % 4),
    the LDS swizzle applied ahead of time), then the 16 rows' four selector words of the stage (in rows 8-15 words 0-1
    and 2-3 swapped, so that the GEMM's selector reads from LDS are free of bank conflicts). The same bytes as the
    library's cohere_pack_24_tiled."""
    n, half = kept.shape
    assert kept.dtype == torch.int8 and words.dtype == torch.int32 and n % 16 == 0 and half % 64 == 0
    assert tuple(words.shape) == (n, half // 16)
    kt = half // 64
    blocks = kept.view(n // 16, 16, kt, 4, 16).permute(0, 2, 1, 3, 4)  # (block, stage, row, chunk, 16 bytes)
    i = torch.arange(64, device=kept.device)
    chunks = blocks[:, :, i // 4, (i % 4) ^ ((i // 8) % 4), :].reshape(n // 16, kt, 1024)
    sel = words.view(n // 16, 16, kt, 4).permute(0, 2, 1, 3)  # (block, stage, row, word)
    r = torch.arange(16, device=kept.device)[:, None]
    w = torch.arange(4, device=kept.device)[None, :]
    sel = sel[:, :, r, w ^ torch.where(r >= 8, 2, 0)]  # rows 8-15: words 0-1 and 2-3 swapped
    sel = sel.contiguous().view(torch.uint8).reshape(n // 16, kt, 256)
    return torch.cat([chunks.view(torch.uint8), sel], dim=2).contiguous()
