"""End-to-end parity (config 4's path at test size): Pipeline.transcribe -- GPU log-mel, subsampling stem, int8
encoder layers, cross-attention fill, captured greedy decoding -- against the CPU checker's chain of the same
stages, on synthetic audio."""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

import oracle
from decoder_helpers import oracle_state, oracle_weights
from frontend_helpers import oracle_stem, stem_weights
from helpers import bf16_bits, bf16_float

pytestmark = pytest.mark.gpu


def _oracle_fields(layers):
    from kernels.fast_encoder import LAYER_FIELDS

    out = []
    for ly in layers.layers:
        f = {}
        for k in LAYER_FIELDS:
            t = ly.tensors[k]
            if t.numel() == 0:
                continue
            t = t.detach().cpu()
            f[k] = bf16_bits(t) if t.dtype == torch.bfloat16 else t.numpy()
        out.append(f)
    return out


def test_pipeline_matches_checker_chain(gpu):
    """Three pieces (2.0 s, 3.3 s, 1.1 s) through a 1-block encoder and config 3's decoder, 10 new tokens each. The
    checker runs every stage on the CPU (features, stem, the int8 layer, the projections in fp32, the decoder step);
    the greedy tokens must agree wherever the checker's top two logits are more than 5 % of the logits' RMS apart
    (each piece compared up to its first closer call, after which the two chains may legitimately part)."""
    import bench
    from kernels.features import dither
    from kernels.pipeline import Pipeline

    model = bench.random_asr_model(gpu, enc_layers=1, seed=5)
    sub_cpu = copy.deepcopy(model.model.encoder.subsampling).float().cpu()
    pipe = Pipeline(model, slots=4, max_new_tokens=10, int8=True, sparse=True, buckets=(1, 2, 4))
    lengths = [32000, 52800, 17600]
    xs = [dither(x) for x in bench.synthetic_audio(lengths, seed=9)]
    prompt = torch.tensor([4, 5, 6, 7])
    got = pipe.transcribe([torch.from_numpy(x).to(gpu) for x in xs], prompt)
    assert len(got) == 3 and all(len(t) <= 14 for t in got)
    assert all(np.array_equal(t[:4], prompt.numpy()) for t in got)

    # ---- the checker's chain ----
    fe = pipe.features
    feats = oracle.logmel(np.concatenate(xs), lengths, fe.window512.cpu().numpy(), fe.mel.cpu().numpy(),
                          fe.band.cpu().numpy(), fe.preemphasis)
    frames = [n // 160 + 1 for n in lengths]
    hidden, t3 = oracle_stem(stem_weights(sub_cpu), feats, frames)
    enc = pipe.encoder.layers
    eps = [enc.layer_eps[5 * i:5 * i + 5] for i in range(len(enc.layers))]
    hidden = oracle.encoder_layers_int8(hidden, _oracle_fields(enc), eps, t3, enc.rel_off, enc.scale)
    # the product's own encoder output for the same pieces: within the layer chain's noise of the checker's
    with torch.no_grad():
        f_gpu, fr = pipe.features([torch.from_numpy(x).to(gpu) for x in xs])
        h_gpu, t3_gpu = pipe.encoder(f_gpu, fr)
    assert t3_gpu == t3
    hg, ho = bf16_float(bf16_bits(h_gpu)).astype(np.float64), bf16_float(hidden).astype(np.float64)
    rms = np.sqrt(np.mean(ho ** 2))
    print(f"encoder output: rms diff {np.sqrt(np.mean((hg - ho) ** 2)) / rms:.2e} x RMS")
    assert np.sqrt(np.mean((hg - ho) ** 2)) <= 2e-2 * rms
    dec = pipe.decoder
    proj_w, proj_b = (t.detach().float().cpu() for t in dec.proj)
    mem = torch.nn.functional.linear(torch.from_numpy(bf16_float(hidden)), proj_w, proj_b).to(torch.bfloat16)
    kv = torch.nn.functional.linear(mem.float(), dec.cross_w.float().cpu(), dec.cross_b.float().cpu())
    kv = bf16_bits(kv.to(torch.bfloat16))
    S, L, H = dec.slots, len(dec.layers), dec.h
    st = oracle_state(L, S, H, dec.seq, dec.frames, dec.max_prompt, dec.pad)
    slots = list(range(len(lengths)))
    slot_of = np.concatenate([np.full(n, s, np.int32) for s, n in zip(slots, t3)])
    frame_of = np.concatenate([np.arange(n, dtype=np.int32) for n in t3])
    oracle.dec_scatter_kv(kv, slot_of, frame_of, ck8=st["cross_k8"], cv8=st["cross_v8"], cks=st["cross_ks"],
                          cvs=st["cross_vs"])
    p = prompt.numpy()
    for s, n in zip(slots, t3):
        st["forced"][s, :] = dec.pad
        st["forced"][s, :len(p)] = p
        st["out"][s, :] = dec.pad
        st["out"][s, :dec.max_prompt] = st["forced"][s]
        st["tok"][s], st["pos"][s], st["plen"][s] = p[0], 0, len(p)
        st["limit"][s], st["cross_len"][s], st["finished"][s] = len(p) - 1 + 10, n, 0
    b = 4
    st["active"] = np.array(slots + [S] * (b - len(slots)), np.int32)
    W = oracle_weights(model)
    margins = {s: [] for s in slots}
    for _ in range(len(p) - 1 + 10):
        logits = bf16_float(oracle.decoder_step(W, st, b)).astype(np.float64)
        rms_l = np.sqrt(np.mean(logits[:len(slots)] ** 2))
        for r, s in enumerate(slots):
            top2 = np.sort(logits[r])[-2:]
            margins[s].append((top2[1] - top2[0]) / rms_l)
        if st["finished"][slots].all():
            break
    compared = 0
    for s, toks in zip(slots, got):
        want = st["out"][s]
        for t in range(len(p), len(toks)):
            if margins[s][t - 1] <= 0.05:
                break
            assert toks[t] == want[t], (s, t, toks[:t + 1], want[:t + 1])
            compared += 1
    print(f"compared {compared} generated tokens")
    assert compared >= 10


def test_submit_matches_transcribe(gpu):
    """The service path (reference pipeline.py:96-115 argument order: pieces, prompt, max_new -> Future) gives the
    same tokens as transcribe() for the same pieces: every stage is per piece, and one encoder chunk holds the same
    rows on both paths. Two requests in flight at once, one with per-piece limits; close() ends the threads."""
    import bench
    from kernels.pipeline import Pipeline

    model = bench.random_asr_model(gpu, enc_layers=1, seed=6)
    pipe = Pipeline(model, None, 4, 12, True, True, buckets=(1, 2, 4))
    lengths = [32000, 52800, 17600]
    xs = [Pipeline.prepare(x) for x in bench.synthetic_audio(lengths, seed=10)]
    prompt = torch.tensor([4, 5, 6, 7])
    want = pipe.transcribe([torch.from_numpy(x).to(gpu) for x in xs], prompt)
    want_short = pipe.transcribe([torch.from_numpy(x).to(gpu) for x in xs[:2]], prompt, [3, 5])
    f1 = pipe.submit(xs, prompt)
    f2 = pipe.submit(xs[:2], prompt, [3, 5])
    got, got_short = f1.result(timeout=120), f2.result(timeout=120)
    assert pipe.submit([], prompt).result() == []
    pipe.close()
    for a, b in zip(got, want):
        assert np.array_equal(a, b), (a, b)
    for a, b, n in zip(got_short, want_short, (3, 5)):
        assert np.array_equal(a, b) and len(a) <= len(prompt) + n
    with pytest.raises(RuntimeError, match="transcribe"):
        pipe.transcribe(xs, prompt)


def test_submit_from_threads_and_failed_chunk(gpu):
    """Requests submitted from four threads at once each get the tokens transcribe() gives for their pieces; a chunk
    whose encoding raises fails exactly the requests it held (their futures raise), and the service goes on."""
    import threading

    import bench
    from kernels.pipeline import Pipeline

    model = bench.random_asr_model(gpu, enc_layers=1, seed=7)
    pipe = Pipeline(model, None, 4, 8, True, True, buckets=(1, 2, 4))
    lengths = [[32000], [17600, 9600], [52800], [24000]]
    audio = [[Pipeline.prepare(x) for x in bench.synthetic_audio(ls, seed=20 + i)] for i, ls in enumerate(lengths)]
    prompt = torch.tensor([4, 5, 6, 7])
    want = [pipe.transcribe([torch.from_numpy(x).to(gpu) for x in xs], prompt) for xs in audio]
    futures = [None] * len(audio)

    def client(i):
        futures[i] = pipe.submit(audio[i], prompt)

    threads = [threading.Thread(target=client, args=(i,)) for i in range(len(audio))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for f, w in zip(futures, want):
        got = f.result(timeout=120)
        assert len(got) == len(w) and all(np.array_equal(a, b) for a, b in zip(got, w))

    # a chunk whose encoding fails: its request fails, the next request is served
    real = pipe._encode

    def flaky(pieces, slots):
        if any(p.n == 11200 for p in pieces):
            raise RuntimeError("injected encoder failure")
        return real(pieces, slots)

    pipe._encode = flaky
    bad = pipe.submit([Pipeline.prepare(x) for x in bench.synthetic_audio([11200], seed=30)], prompt)
    with pytest.raises(RuntimeError, match="injected"):
        bad.result(timeout=120)
    good = pipe.submit(audio[0], prompt).result(timeout=120)
    assert np.array_equal(good[0], want[0][0])
    pipe.close()
