"""Config 4 at its own workload, on four of its clips: 4 x 30 s of synthetic audio through the whole pipeline (log-mel,
subsampling stem, 24 int8 blocks with both feed-forward linears 2:4, projection and cross-attention fill, greedy
decoding of up to 448 tokens with config 3's decoder) against the checker's whole chain (oracle/chain.py) on the same
audio, with the weights converted by the checker's own functions.

A 24-block random-init encoder amplifies last-bit differences layer after layer, so the bar is the chain's own
sensitivity, measured on the same input: the checker run again with 1 % of its log-mel values moved by one bf16 ulp.
  * encoder output (after 24 blocks): the kernels' RMS difference from the checker is at most 1.5x the perturbed
    checker's;
  * tokens: decoding with the GPU's tokens as history (teacher forcing), the checker picks the GPU's next token at
    least as often, less two points, as it picks its own next token when decoding from the perturbed checker's
    encoder output with its own tokens as history. Both agreements are printed;
  * clear-margin picks: the checker also decodes from the perturbed encoder output with the GPU's tokens as history,
    so that both of its runs see the same history and their logits can be compared step by step. Wherever the
    checker's gap between its best and second-best logit exceeds twice that step's largest logit difference between
    its two runs, the pick is not a near-tie and the kernels' token must equal the checker's. The number of such picks
    is printed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, bf16_float

pytestmark = pytest.mark.gpu

CLIPS, SECONDS, MAX_NEW = 4, 30.0, 448


def _agreement(picks, seqs, plen):
    same = total = 0
    for pk, toks in zip(picks, seqs):
        gen = list(toks[plen:])
        same += sum(int(a == b) for a, b in zip(gen, pk))
        total += len(gen)
    return same / max(total, 1), total


def test_config4_pipeline_against_checker_chain(gpu):
    import bench
    from kernels.pipeline import Pipeline
    from oracle import chain

    model = bench.random_asr_model(gpu, enc_layers=24, seed=1)
    pipe = Pipeline(model, None, slots=CLIPS, max_new_tokens=MAX_NEW, int8=True, sparse=True, sparse_w1=True,
                    buckets=(1, 2, 4), chunk_frames=CLIPS * 376)
    xs = [Pipeline.prepare(x) for x in bench.synthetic_audio([int(SECONDS * 16000)] * CLIPS, seed=7)]
    prompt = np.array([4, 5, 6, 7])
    got = pipe.transcribe([torch.from_numpy(x).to(gpu) for x in xs], torch.from_numpy(prompt))
    assert len(got) == CLIPS and all(np.array_equal(t[:4], prompt) for t in got)
    with torch.no_grad():
        f, fr = pipe.features([torch.from_numpy(x).to(gpu) for x in xs])
        h_gpu, t3_gpu = pipe.encoder(f, fr)
    h_gpu = bf16_float(bf16_bits(h_gpu)).astype(np.float64)

    W = chain.asr_weights(model, int8=True, sparse=True, sparse_w1=True)
    feats, frames = chain.features(W, xs)
    hidden, lengths = chain.encode_features(W, feats, frames)
    assert lengths == t3_gpu
    pert = feats.copy()
    moved = (np.random.default_rng(0).random(pert.shape) < 0.01) & (pert != 0)
    pert[moved] += 1
    hidden_p, _ = chain.encode_features(W, pert, frames)
    ho, hp = bf16_float(hidden).astype(np.float64), bf16_float(hidden_p).astype(np.float64)
    rms = np.sqrt(np.mean(ho ** 2))
    d_gpu, d_noise = np.sqrt(np.mean((h_gpu - ho) ** 2)) / rms, np.sqrt(np.mean((hp - ho) ** 2)) / rms
    print(f"encoder output after 24 blocks: kernels vs checker rms {d_gpu:.3e} x RMS, perturbed checker "
          f"{d_noise:.3e}", flush=True)
    assert d_gpu <= 1.5 * d_noise

    own = chain.decode(W, hidden, lengths, prompt, MAX_NEW)
    _, picks_gpu, rows_gpu = chain.decode(W, hidden, lengths, prompt, MAX_NEW, forced_tokens=got, want_logits=True)
    _, _, rows_pert = chain.decode(W, hidden_p, lengths, prompt, MAX_NEW, forced_tokens=got, want_logits=True)
    _, picks_noise = chain.decode(W, hidden_p, lengths, prompt, MAX_NEW, forced_tokens=own)
    a_gpu, n_gpu = _agreement(picks_gpu, got, len(prompt))
    a_noise, n_noise = _agreement(picks_noise, own, len(prompt))
    free = [next((i for i, (a, b) in enumerate(zip(g[4:], o[4:])) if a != b), min(len(g), len(o)) - 4)
            for g, o in zip(got, own)]
    print(f"tokens (teacher-forced): checker agrees with the kernels on {a_gpu:.4f} of {n_gpu}, with itself from the "
          f"perturbed encoder output on {a_noise:.4f} of {n_noise}; free-running common prefixes {free}", flush=True)
    assert a_gpu >= a_noise - 0.02
    clear_n = clear_same = 0
    for s, (pk, toks, rg, rp) in enumerate(zip(picks_gpu, got, rows_gpu, rows_pert)):
        n = min(len(pk), len(toks) - len(prompt), len(rg), len(rp))
        lg, lp = bf16_float(rg[:n]).astype(np.float64), bf16_float(rp[:n]).astype(np.float64)
        top2 = np.sort(lg, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2.0 * np.abs(lp - lg).max(axis=1)
        gen = np.asarray(toks[len(prompt):len(prompt) + n])
        ok = np.asarray(pk[:n]) == gen
        clear_n, clear_same = clear_n + int(clear.sum()), clear_same + int(ok[clear].sum())
        assert ok[clear].all(), (s, np.nonzero(clear & ~ok)[0])
    print(f"clear-margin picks: {clear_same} / {clear_n} index-exact", flush=True)
