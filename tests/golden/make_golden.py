"""Writes tests/golden/compress24_golden.npz: input/output vectors of the reference's own compress_24 and
prune_24_magnitude (kernels/sparse.py:26-46), the only functions on the path whose exact bytes no closed form or
library routine pins (which zero positions a group with fewer than two nonzero values keeps, and the selector packing).

Run once in the build container, where the reference checkout is mounted (it needs only torch):
    python tests/golden/make_golden.py /root/reference
The fixture is data (inputs and expected outputs); nothing at test time reads the reference.
"""

from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch


def load_sparse(ref_root: str):
    path = os.path.join(ref_root, "kernels", "sparse.py")
    spec = importlib.util.spec_from_file_location("ref_sparse", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def cases(gen: torch.Generator) -> dict[str, torch.Tensor]:
    out = {}
    # every 2-of-4 pattern and every degenerate group (0 or 1 nonzero), in all positions, several rows
    groups = []
    for i0 in range(4):
        for i1 in range(i0 + 1, 4):
            g = [0, 0, 0, 0]
            g[i0], g[i1] = 5 + i0, -7 - i1
            groups.append(g)
    for i0 in range(4):
        g = [0, 0, 0, 0]
        g[i0] = 3 - 9 * i0
        groups.append(g)
    groups.append([0, 0, 0, 0])
    groups.append([127, 0, 0, -127])
    rows = []
    for shift in range(8):
        r = []
        for j in range(16):  # 64 values = 16 groups per row
            r += groups[(j + shift) % len(groups)]
        rows.append(r)
    out["patterns"] = torch.tensor(rows, dtype=torch.int8)
    # random 2:4-pruned int8 matrices (from pruned random weights) with values at the int8 extremes
    w = torch.randn(48, 256, generator=gen)
    w[0, :8] = torch.tensor([1.0, -1.0, 0.5, -0.5, 2.0, 0.0, 0.0, 3.0])
    out["random"] = w
    return out


def main(ref_root: str) -> None:
    sp = load_sparse(ref_root)
    gen = torch.Generator().manual_seed(20241201)
    cs = cases(gen)
    rec = {}
    # patterns: compress_24 directly
    kept, words = sp.compress_24(cs["patterns"])
    rec["patterns_w"] = cs["patterns"].numpy()
    rec["patterns_kept"] = kept.numpy()
    rec["patterns_words"] = words.numpy()
    # random: prune (magnitude) on fp32, quantize-like scaling to int8, compress
    w = cs["random"]
    pruned = sp.prune_24_magnitude(w)
    s = pruned.abs().amax(-1).clamp_min(1e-12) / 127
    q = torch.round(pruned / s[:, None]).clamp(-127, 127).to(torch.int8)
    kept, words = sp.compress_24(q)
    rec["random_w"] = w.numpy()
    rec["random_pruned"] = pruned.numpy()
    rec["random_q"] = q.numpy()
    rec["random_kept"] = kept.numpy()
    rec["random_words"] = words.numpy()
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "compress24_golden.npz")
    np.savez_compressed(dst, **rec)
    print("wrote", dst, {k: v.shape for k, v in rec.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
