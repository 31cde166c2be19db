"""The whole transcription chain on the CPU (TEST AND BASELINE INFRASTRUCTURE ONLY): the stages of the reference's
kernels/pipeline.py composed from this package's restated functions -- log-mel features (features.cu:34-132), the
subsampling stem (fast_encoder.py:176-201, encoder_ops.cu:339-448, gemm.cu), the encoder layers
(encoder_loop.cpp:63-124), the decoder's input projection and every layer's cross-attention keys and values
(stream_decoder.py fill_cross), then greedy decoding step by step (stream_decoder.py:176-199).

The weights are converted from a transformers CohereAsrForConditionalGeneration by the checker's own functions
(quantize_weight_rows, prune_24, compress_24, prepare_w8), independently of the product's conversion. Used by tests/
and by bench.py's CPU leg (the reference path's audio-sec/sec on the host, and the token agreement of the GPU path).

    W = asr_weights(model, int8=True, sparse=True)
    tokens = transcribe(W, pieces, prompt, max_new=448)   # per piece: prompt + generated ids (np.int64)
"""

from __future__ import annotations

import numpy as np

import oracle as O


def _bits(t) -> np.ndarray:
    import torch

    return t.detach().float().cpu().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def _f32(t) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float32)


def mel_settings():
    """The extractor's framing constants: 512-point frame with the 400-point symmetric Hann window in its middle,
    transformers' Slaney filter bank (128 bands over 257 bins), each band's first and end nonzero bins, 0.97
    pre-emphasis (transformers CohereAsrFeatureExtractor)."""
    import torch
    from transformers.audio_utils import mel_filter_bank

    window = np.zeros(512, np.float32)
    window[56:456] = torch.hann_window(400, periodic=False).numpy()
    mel = mel_filter_bank(num_frequency_bins=257, num_mel_filters=128, min_frequency=0.0, max_frequency=8000.0,
                          sampling_rate=16000, norm="slaney", mel_scale="slaney").T.astype(np.float32)
    band = np.zeros((128, 2), np.int32)
    for i, row in enumerate(mel):
        nz = np.flatnonzero(row)
        if nz.size:
            band[i] = (nz[0], nz[-1] + 1)
    return {"window": window, "mel": np.ascontiguousarray(mel), "band": band, "preemph": 0.97}


def _relative_table(inv_freq, rk_weight, max_len: int = 512) -> np.ndarray:
    """The layer's projected distance table, rows d = -(max_len-1) .. max_len+63 (fast_encoder.py:155-162)."""
    import torch

    d = torch.arange(-(max_len - 1), max_len + 64, dtype=torch.float)
    f = d[:, None] * inv_freq.float().cpu()
    pos = torch.stack([f.sin(), f.cos()], -1).reshape(len(d), -1).to(torch.bfloat16).float()
    return _bits(pos @ rk_weight.detach().float().cpu().t())


def _layer_fields(blk, inv_freq, int8: bool, sparse: bool, sparse_w1: bool):
    at, cv = blk.self_attn, blk.conv
    f, eps = {}, []
    for name, m in zip(("ff1", "att", "conv", "ff2", "out"), (blk.norm_feed_forward1, blk.norm_self_att,
                                                             blk.norm_conv, blk.norm_feed_forward2, blk.norm_out)):
        f[f"ln_{name}_w"], f[f"ln_{name}_b"] = _bits(m.weight), _bits(m.bias)
        eps.append(float(m.eps))
    c = cv.depthwise_conv.in_channels
    pw1 = cv.pointwise_conv1.weight[:, :, 0]
    pb1 = cv.pointwise_conv1.bias
    import torch

    lin = {"ff1_w1": blk.feed_forward1.linear1.weight, "ff1_w2": blk.feed_forward1.linear2.weight,
           "ff2_w1": blk.feed_forward2.linear1.weight, "ff2_w2": blk.feed_forward2.linear2.weight,
           "wqkv": torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]), "wo": at.o_proj.weight,
           "wpw1": torch.stack([pw1[:c], pw1[c:]], 1).reshape(2 * c, -1), "wpw2": cv.pointwise_conv2.weight[:, :, 0]}
    for k, ff in (("ff1", blk.feed_forward1), ("ff2", blk.feed_forward2)):
        f[f"{k}_b1"], f[f"{k}_b2"] = _bits(ff.linear1.bias), _bits(ff.linear2.bias)
    f["bqkv"] = _bits(torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias]))
    f["bo"], f["bu"], f["bv"] = _bits(at.o_proj.bias), _bits(at.bias_u), _bits(at.bias_v)
    f["bpw1"] = _bits(torch.stack([pb1[:c], pb1[c:]], 1).reshape(2 * c))
    f["bpw2"] = _bits(cv.pointwise_conv2.bias)
    f["rk"] = _relative_table(inv_freq, at.relative_k_proj.weight)
    f["wdw"], f["bdw"] = _f32(cv.depthwise_conv.weight[:, 0, :]), _f32(cv.depthwise_conv.bias)
    bn = cv.norm
    scale = bn.weight.detach().float() / torch.sqrt(bn.running_var.float() + bn.eps)
    f["bn_scale"] = _f32(scale)
    f["bn_shift"] = _f32(bn.bias.detach().float() - bn.running_mean.float() * scale)
    qname = {"ff1_w1": ("q_ff1_w1", "q_ff1_s1", "sp_ff1_w1", "sp_ff1_e1"),
             "ff1_w2": ("q_ff1_w2", "q_ff1_s2", "sp_ff1_w", "sp_ff1_e"),
             "ff2_w1": ("q_ff2_w1", "q_ff2_s1", "sp_ff2_w1", "sp_ff2_e1"),
             "ff2_w2": ("q_ff2_w2", "q_ff2_s2", "sp_ff2_w", "sp_ff2_e"),
             "wqkv": ("q_qkv_w", "q_qkv_s"), "wo": ("q_o_w", "q_o_s"), "wpw1": ("q_pw1_w", "q_pw1_s"),
             "wpw2": ("q_pw2_w", "q_pw2_s")}
    for name, w in lin.items():
        if not int8:
            f[name] = _bits(w)
            continue
        q = qname[name]
        pruned = len(q) == 4 and (sparse if name.endswith("w2") else sparse_w1)
        wf = _f32(w.to(torch.bfloat16))
        f[q[0]], f[q[1]] = O.quantize_weight_rows(O.prune_24(wf) if pruned else wf)
        if pruned:
            f[q[2]], f[q[3]] = O.compress_24(f[q[0]])
            del f[q[0]]
    return f, eps


def _stem(sub) -> dict:
    conv0, dw2, pw3, dw5, pw6 = (sub.layers[i] for i in (0, 2, 3, 5, 6))
    f2 = lambda t: _f32(t).reshape(t.shape[0], -1).copy()  # noqa: E731
    ch = pw6.out_channels
    out_f = sub.linear.in_features // ch
    lin = sub.linear.weight.detach().view(-1, ch, out_f).transpose(1, 2).reshape(-1, ch * out_f)
    return {"w0": f2(conv0.weight), "b0": _f32(conv0.bias), "w2": f2(dw2.weight), "b2": _f32(dw2.bias),
            "pw3": _bits(pw3.weight[:, :, 0, 0]), "pw3_b": _bits(pw3.bias), "w5": f2(dw5.weight), "b5": _f32(dw5.bias),
            "pw6": _bits(pw6.weight[:, :, 0, 0]), "pw6_b": _bits(pw6.bias), "lin": _bits(lin),
            "lin_b": _bits(sub.linear.bias), "channels": ch}


def _decoder(model, int8: bool) -> dict:
    import torch

    dec, cfg = model.model.decoder, model.config
    ln = lambda m: (_bits(m.weight), _bits(m.bias), float(m.eps))  # noqa: E731
    W = {"embed": _bits(dec.embed_tokens.weight), "pos_table": _bits(dec.pos_emb.weight),
         "emb_ln": ln(dec.embedding_layernorm), "final_ln": ln(dec.norm),
         "scale": (cfg.hidden_size // cfg.num_attention_heads) ** -0.5, "eos": cfg.eos_token_id,
         "pad": cfg.pad_token_id, "heads": cfg.num_attention_heads, "layers": []}
    for lyr in dec.layers:
        sa, ca = lyr.self_attn, lyr.encoder_attn
        ly = {"ln1": ln(lyr.input_layernorm), "ln2": ln(lyr.post_attention_layernorm), "ln3": ln(lyr.final_layernorm),
              "qkv_b": _bits(torch.cat([sa.q_proj.bias, sa.k_proj.bias, sa.v_proj.bias])),
              "o_w": _bits(sa.o_proj.weight), "o_b": _bits(sa.o_proj.bias), "cq_w": _bits(ca.q_proj.weight),
              "cq_b": _bits(ca.q_proj.bias), "co_w": _bits(ca.o_proj.weight), "co_b": _bits(ca.o_proj.bias),
              "fc1_b": _bits(lyr.mlp.fc1.bias), "fc2_b": _bits(lyr.mlp.fc2.bias)}
        for name, w in (("qkv", torch.cat([sa.q_proj.weight, sa.k_proj.weight, sa.v_proj.weight])),
                        ("fc1", lyr.mlp.fc1.weight), ("fc2", lyr.mlp.fc2.weight)):
            if int8:
                ly[name + "_w8"] = O.prepare_w8(_bits(w))
            else:
                ly[name + "_w"] = _bits(w)
        W["layers"].append(ly)
    if int8:
        W["head_w8"] = O.prepare_w8(_bits(model.proj_out.weight))
    else:
        W["head_w"] = _bits(model.proj_out.weight)
    W["head_b"] = _bits(model.proj_out.bias)
    W["proj"] = (_bits(dec.proj.weight), _bits(dec.proj.bias))
    W["cross"] = (_bits(torch.cat([t for lyr in dec.layers for t in (lyr.encoder_attn.k_proj.weight,
                                                                     lyr.encoder_attn.v_proj.weight)])),
                  _bits(torch.cat([t for lyr in dec.layers for t in (lyr.encoder_attn.k_proj.bias,
                                                                     lyr.encoder_attn.v_proj.bias)])))
    return W


def asr_weights(model, int8: bool = True, sparse: bool = False, sparse_w1: bool = False) -> dict:
    """Every weight of the chain, converted by the checker from the model (CPU copies; the model may live on the
    GPU)."""
    enc = model.model.encoder
    inv = enc.encode_positions.inv_freq
    layers, eps = [], []
    for blk in enc.layers:
        f, e = _layer_fields(blk, inv, int8, sparse, sparse_w1)
        layers.append(f)
        eps.append(e)
    heads = enc.layers[0].self_attn.bias_u.shape[0]
    return {"mel": mel_settings(), "stem": _stem(enc.subsampling), "layers": layers, "eps": eps, "int8": int8,
            "scale": (1280 // heads) ** -0.5, "rel_off": 511, "decoder": _decoder(model, int8)}


def _half(n):
    return [(t - 1) // 2 + 1 for t in n]


def _rows(ts):
    return np.array([(i, t) for i, n in enumerate(ts) for t in range(n)], np.int32).reshape(-1, 2)


def stem(S: dict, feats: np.ndarray, frames: list[int], threads: int = 0):
    """The subsampling stem over padded features (B, T, 128) bf16 bits: packed (sum t3, 1280) bf16 bits, lengths."""
    C = S["channels"]
    t2 = _half(_half(frames))
    t3 = _half(t2)
    a2 = O.sub_conv0_dw(feats, np.asarray(frames, np.int32), _rows(t2), S["w0"], S["b0"], S["w2"], S["b2"],
                        threads=threads)
    a3 = O.gemm_bf16(a2.reshape(-1, C), S["pw3"], S["pw3_b"], O.EPI_CONV_RELU, threads=threads).reshape(-1, 32, C)
    starts = np.concatenate([[0], np.cumsum(t2)[:-1]]).astype(np.int32)
    a5 = O.sub_dw(a3, starts, np.asarray(t2, np.int32), _rows(t3), S["w5"], S["b5"], threads=threads)
    a6 = O.gemm_bf16(a5.reshape(-1, C), S["pw6"], S["pw6_b"], O.EPI_CONV_RELU, threads=threads)
    return O.gemm_bf16(a6.reshape(len(a5), -1), S["lin"], S["lin_b"], O.EPI_BIAS, threads=threads), t3


def features(W: dict, pieces: list[np.ndarray], threads: int = 0):
    """Dithered pieces -> padded log-mel features (B, T, 128) bf16 bits and the frame counts (n // 160 + 1)."""
    m = W["mel"]
    lengths = [len(p) for p in pieces]
    feats = O.logmel(np.concatenate(pieces).astype(np.float32), lengths, m["window"], m["mel"], m["band"],
                     m["preemph"], threads=threads)
    return feats, [n // 160 + 1 for n in lengths]


def encode_features(W: dict, feats: np.ndarray, frames: list[int], threads: int = 0):
    """Padded features -> packed encoder output (sum of lengths, 1280) bf16 bits and the lengths."""
    hidden, t3 = stem(W["stem"], feats, frames, threads=threads)
    run = O.encoder_layers_int8 if W["int8"] else O.encoder_layers_bf16
    return run(hidden, W["layers"], W["eps"], t3, W["rel_off"], W["scale"], threads=threads), t3


def encode(W: dict, pieces: list[np.ndarray], threads: int = 0):
    """Dithered pieces -> packed encoder output (sum of lengths, 1280) bf16 bits and the lengths."""
    feats, frames = features(W, pieces, threads=threads)
    return encode_features(W, feats, frames, threads=threads)


def decode(W: dict, hidden: np.ndarray, lengths: list[int], prompt, max_new: int, forced_tokens=None,
           threads: int = 0, want_logits: bool = False):
    """Greedy decoding of every piece at once (one row per piece; rows are independent), from packed encoder output.
    forced_tokens (optional, per piece): after each step the piece's next input is this sequence's token instead of
    the checker's own pick (teacher forcing), and the checker's picks are returned beside. Returns per piece the ids
    (prompt + generated up to and including the end token) and, with forcing, the checker's pick at every step;
    want_logits (with forcing) adds per piece the logits row (bf16 bits) behind each of those picks."""
    D = W["decoder"]
    n, L, H = len(lengths), len(D["layers"]), D["heads"]
    mem = O.gemm_bf16(hidden, D["proj"][0], D["proj"][1], O.EPI_BIAS, threads=threads)
    kv = O.gemm_bf16(mem, D["cross"][0], D["cross"][1], O.EPI_BIAS, threads=threads)
    prompt = np.asarray(prompt, np.int64)
    P, frames = len(prompt), max(lengths)
    seq = P + max_new + 1
    S1 = n + 1
    st = {"self_k8": np.zeros((L, S1, H, seq, 128), np.int8), "self_ks": np.ones((L, S1, H, seq), np.float32),
          "cross_k8": np.zeros((L, S1, H, frames, 128), np.int8), "cross_ks": np.ones((L, S1, H, frames), np.float32),
          "cross_len": np.ones(S1, np.int32), "tok": np.full(S1, D["pad"], np.int64), "pos": np.zeros(S1, np.int32),
          "plen": np.ones(S1, np.int32), "limit": np.zeros(S1, np.int32), "finished": np.ones(S1, np.uint8),
          "forced": np.full((S1, P), D["pad"], np.int64), "out": np.full((S1, seq + 1), D["pad"], np.int64),
          "dummy": n, "active": np.arange(n, dtype=np.int32)}
    st["self_v8"], st["self_vs"] = np.zeros_like(st["self_k8"]), np.ones_like(st["self_ks"])
    st["cross_v8"], st["cross_vs"] = np.zeros_like(st["cross_k8"]), np.ones_like(st["cross_ks"])
    slot_of = np.concatenate([np.full(t, s, np.int32) for s, t in enumerate(lengths)])
    frame_of = np.concatenate([np.arange(t, dtype=np.int32) for t in lengths])
    O.dec_scatter_kv(kv, slot_of, frame_of, ck8=st["cross_k8"], cv8=st["cross_v8"], cks=st["cross_ks"],
                     cvs=st["cross_vs"])
    for s in range(n):
        st["forced"][s] = prompt
        st["out"][s, :P] = prompt
        st["tok"][s], st["plen"][s], st["limit"][s] = prompt[0], P, P - 1 + max_new
        st["cross_len"][s], st["finished"][s] = lengths[s], 0
    picks = [[] for _ in range(n)]
    rows = [[] for _ in range(n)]
    for _ in range(P - 1 + max_new):
        running = st["finished"][:n] == 0
        logits = O.decoder_step(D, st, n)
        if forced_tokens is not None:
            for s in np.nonzero(running)[0]:
                at = int(st["pos"][s])  # the position this step wrote (decoder_ops.cu:106-159)
                if at < P:
                    continue
                picks[s].append(int(st["tok"][s]))
                if want_logits:
                    rows[s].append(logits[s].copy())
                seq_s = forced_tokens[s]
                if at < len(seq_s):
                    t = int(seq_s[at])
                    st["tok"][s] = st["out"][s, at] = t
                    st["finished"][s] = int(t == D["eos"] or at >= st["limit"][s])
                else:
                    st["finished"][s] = 1
        if st["finished"][:n].all():
            break
    ids = []
    for s in range(n):
        gen = st["out"][s, P:]
        end = np.nonzero(gen == D["eos"])[0]
        ids.append(st["out"][s, :P + (end[0] + 1 if len(end) else min(len(gen), max_new))].copy())
    if forced_tokens is None:
        return ids
    return (ids, picks, [np.array(r).reshape(-1, logits.shape[1]) for r in rows]) if want_logits else (ids, picks)


def transcribe(W: dict, pieces: list[np.ndarray], prompt, max_new: int = 448, threads: int = 0):
    """Dithered pieces -> per piece prompt + generated ids, the whole chain on the CPU."""
    hidden, lengths = encode(W, pieces, threads=threads)
    return decode(W, hidden, lengths, prompt, max_new, threads=threads)
