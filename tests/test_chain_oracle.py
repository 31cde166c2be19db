"""The checker's whole chain (oracle/chain.py) on the CPU: it composes functions pinned elsewhere; here, that its
stem equals the test fixtures' composition, and that decoding forced with its own output reproduces its own picks
(the teacher-forcing path the bench's token agreement uses)."""

from __future__ import annotations

import numpy as np
import torch

import oracle
from oracle import chain
from frontend_helpers import oracle_stem, stem_weights


def _model():
    import bench

    return bench.random_asr_model("cpu", enc_layers=1, seed=2)


def test_chain_stem_and_self_forcing():
    import bench
    from kernels.features import dither

    model = _model()
    W = chain.asr_weights(model, int8=True, sparse=True)
    xs = [dither(x) for x in bench.synthetic_audio([16000, 9600], seed=3)]
    m = W["mel"]
    lengths = [len(x) for x in xs]
    feats = oracle.logmel(np.concatenate(xs), lengths, m["window"], m["mel"], m["band"], m["preemph"])
    frames = [n // 160 + 1 for n in lengths]
    got, t3 = chain.stem(W["stem"], feats, frames)
    want, t3w = oracle_stem(stem_weights(model.model.encoder.subsampling.float()), feats, frames)
    assert t3 == t3w and np.array_equal(got, want)
    hidden, lengths = chain.encode(W, xs)
    prompt = np.array([4, 5, 6, 7])
    ids = chain.decode(W, hidden, lengths, prompt, 6)
    assert all(np.array_equal(t[:4], prompt) and 4 < len(t) <= 10 for t in ids)
    ids2, picks = chain.decode(W, hidden, lengths, prompt, 6, forced_tokens=ids)
    for a, b, p in zip(ids, ids2, picks):
        assert np.array_equal(a, b) and list(p) == list(a[4:])
