"""Pins of the CPU checker's decoder-step functions (dec_embed, dec_add_ln, dec_attention, dec_pick, dec_scatter_kv,
decoder_step) against torch in float64, hand-written rules, and transformers' CohereAsrDecoder."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from decoder_helpers import cross_kv, make_decoder, oracle_state, oracle_weights
from helpers import bf16_bits, bf16_float, bf16_ulp

pytest.importorskip("transformers.models.cohere_asr.modeling_cohere_asr")


def _bf(t):
    return bf16_bits(t.to(torch.bfloat16))


def _ln64(x, w, b, eps):
    t = lambda a: torch.from_numpy(bf16_float(a)).double()  # noqa: E731
    return torch.nn.functional.layer_norm(t(x), (x.shape[-1],), t(w), t(b), eps).numpy()


def test_dec_embed_and_add_ln_match_torch_float64():
    g = torch.Generator().manual_seed(1)
    V, P, W = 50, 40, 256
    emb, ptab = _bf(torch.randn(V, W, generator=g)), _bf(torch.randn(P, W, generator=g) * 3)
    ln0 = (_bf(1 + 0.1 * torch.randn(W, generator=g)), _bf(0.1 * torch.randn(W, generator=g)), 1e-5)
    ln1 = (_bf(1 + 0.1 * torch.randn(W, generator=g)), _bf(0.1 * torch.randn(W, generator=g)), 1e-5)
    active = np.array([3, 0, 2], np.int32)
    tok = np.array([7, 11, 49, 0], np.int64)
    pos = np.array([5, 0, 39, 1], np.int32)
    x, h = oracle.dec_embed(active, tok, pos, emb, ptab, ln0, ln1)
    s = np.stack([bf16_float(emb[tok[a]]) + bf16_float(ptab[pos[a]]) for a in active])
    s = _bf(torch.from_numpy(s))
    want_x = _ln64(s, *ln0)
    assert (np.abs(bf16_float(x) - want_x) <= bf16_ulp(want_x) * 1.0001).all()
    want_h = _ln64(x, *ln1)
    assert (np.abs(bf16_float(h) - want_h) <= bf16_ulp(want_h) * 1.0001).all()
    y = _bf(torch.randn(3, W, generator=g))
    x2 = x.copy()
    h2 = oracle.dec_add_ln(x2, y, ln1)
    assert np.array_equal(x2, _bf(torch.from_numpy(bf16_float(x) + bf16_float(y))))
    want = _ln64(x2, *ln1)
    assert (np.abs(bf16_float(h2) - want) <= bf16_ulp(want) * 1.0001).all()


def _attn_setup(seed, slots=4, H=2, T=40):
    g = torch.Generator().manual_seed(seed)
    k8 = torch.randint(-127, 128, (slots, H, T, 128), generator=g).to(torch.int8).numpy()
    v8 = torch.randint(-127, 128, (slots, H, T, 128), generator=g).to(torch.int8).numpy()
    ks = (torch.rand(slots, H, T, generator=g) * 0.02 + 0.001).numpy().astype(np.float32)
    vs = (torch.rand(slots, H, T, generator=g) * 0.02 + 0.001).numpy().astype(np.float32)
    return g, k8, v8, ks, vs


def test_dec_attention_q8_matches_sdpa_float64():
    g, k8, v8, ks, vs = _attn_setup(2)
    H, T = 2, 40
    active = np.array([2, 0, 3], np.int32)
    n = np.array([17, 5, 40, 1], np.int32)
    q = _bf(torch.randn(3, H * 128, generator=g))
    scale = 128 ** -0.5
    out = bf16_float(oracle.dec_attention(False, active, q, n, scale, k8=k8, v8=v8, ks=ks, vs=vs))
    for r, s in enumerate(active):
        kk = torch.from_numpy(k8[s, :, :n[s]].astype(np.float32) * ks[s, :, :n[s], None]).double()
        vv = torch.from_numpy(v8[s, :, :n[s]].astype(np.float32) * vs[s, :, :n[s], None]).double()
        qq = torch.from_numpy(bf16_float(q[r])).double().reshape(H, 1, 128)
        want = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, scale=scale).reshape(-1).numpy()
        assert np.abs(out[r] - want).max() <= 2 * bf16_ulp(np.abs(want).max()) + 1e-6


def test_dec_attention_self_writes_and_attends_the_new_key():
    g, k8, v8, ks, vs = _attn_setup(3)
    H = 2
    active = np.array([1], np.int32)
    pos = np.array([0, 9, 0, 0], np.int32)
    qkv = _bf(torch.randn(1, 3 * H * 128, generator=g))
    k8c, v8c, ksc, vsc = k8.copy(), v8.copy(), ks.copy(), vs.copy()
    out = bf16_float(oracle.dec_attention(True, active, qkv, pos, 0.1, k8=k8c, v8=v8c, ks=ksc, vs=vsc))
    f = bf16_float(qkv[0]).reshape(3, H, 128)
    for h in range(H):
        for which, cache, sc in ((1, k8c, ksc), (2, v8c, vsc)):
            vec = f[which, h]
            s_want = np.float32(np.abs(vec).max()) / np.float32(127)
            assert sc[1, h, 9] == s_want
            assert np.array_equal(cache[1, h, 9], np.clip(np.rint(vec * (np.float32(1) / s_want)), -127, 127))
        # keys 0..8 from the cache, the 10th unquantized
        kk = np.concatenate([k8[1, h, :9].astype(np.float32) * ks[1, h, :9, None], f[1, h][None]])
        vv = np.concatenate([v8[1, h, :9].astype(np.float32) * vs[1, h, :9, None], f[2, h][None]])
        want = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(f[0, h]).double()[None, None], torch.from_numpy(kk).double()[None],
            torch.from_numpy(vv).double()[None], scale=0.1).reshape(-1).numpy()
        assert np.abs(out[0, h * 128:(h + 1) * 128] - want).max() <= 2 * bf16_ulp(np.abs(want).max()) + 1e-6
    # nothing else of the caches moved
    k8c[1, :, 9] = k8[1, :, 9]
    assert np.array_equal(k8c, k8)


def test_dec_pick_rules():
    V = 16
    logits = np.zeros((4, V), np.float32)
    logits[0, [3, 9]] = 5.0           # a tie: the first index
    logits[1, 7] = 2.0                # inside the prompt: forced token instead
    logits[2, 3] = 1.0                # the end token
    logits[3, 12] = 1.0               # already finished: nothing moves
    active = np.array([0, 1, 2, 3], np.int32)
    tok = np.zeros(5, np.int64)
    pos = np.array([4, 0, 6, 2, 0], np.int32)
    finished = np.array([0, 0, 0, 1, 1], np.uint8)
    forced = np.full((5, 4), 2, np.int64)
    forced[1, 1] = 13
    plen = np.array([1, 3, 1, 1, 1], np.int32)
    limit = np.array([100, 100, 100, 100, 0], np.int32)
    out = np.full((5, 20), 2, np.int64)
    oracle.dec_pick(_bf(torch.from_numpy(logits)), active, 4, tok, pos, finished, forced, plen, limit, out, eos=3)
    assert tok[0] == 3 and pos[0] == 5 and out[0, 5] == 3 and finished[0] == 1  # argmax 3 = eos: ends
    assert tok[1] == 13 and pos[1] == 1 and finished[1] == 0                 # forced
    assert tok[2] == 3 and finished[2] == 1
    assert tok[3] == 0 and pos[3] == 2 and finished[3] == 1                  # untouched
    # the limit ends a row outside the prompt
    pos2, fin2, tok2, out2 = np.array([99, 0, 0, 0, 0], np.int32), np.zeros(5, np.uint8), np.zeros(5, np.int64), \
        out.copy()
    logits2 = np.zeros((1, V), np.float32)
    logits2[0, 5] = 1
    oracle.dec_pick(_bf(torch.from_numpy(logits2)), np.array([0], np.int32), 4, tok2, pos2, fin2, forced, plen,
                    limit, out2, eos=3)
    assert tok2[0] == 5 and pos2[0] == 100 and fin2[0] == 1


def test_dec_scatter_kv_q8_round_trip():
    g = torch.Generator().manual_seed(5)
    L, S, H, T = 2, 3, 2, 10
    rows = 7
    kv = _bf(torch.randn(rows, L * 2 * H * 128, generator=g))
    slot_of = np.array([0, 0, 2, 2, 2, 1, 0], np.int32)
    frame_of = np.array([0, 1, 0, 1, 2, 0, 2], np.int32)
    ck8, cv8 = np.zeros((L, S, H, T, 128), np.int8), np.zeros((L, S, H, T, 128), np.int8)
    cks, cvs = np.zeros((L, S, H, T), np.float32), np.zeros((L, S, H, T), np.float32)
    oracle.dec_scatter_kv(kv, slot_of, frame_of, ck8=ck8, cv8=cv8, cks=cks, cvs=cvs)
    f = bf16_float(kv).reshape(rows, L, 2, H, 128)
    for r in range(rows):
        for l in range(L):
            for kvi, c8, cs in ((0, ck8, cks), (1, cv8, cvs)):
                for h in range(H):
                    vec, q, s = f[r, l, kvi, h], c8[l, slot_of[r], h, frame_of[r]], cs[l, slot_of[r], h, frame_of[r]]
                    assert np.abs(q).max() == 127
                    assert np.abs(q * s - vec).max() <= s / 2 * 1.0001
    ck, cv = np.zeros((L, S, H, T, 128), np.uint16), np.zeros((L, S, H, T, 128), np.uint16)
    oracle.dec_scatter_kv(kv, slot_of, frame_of, ck=ck, cv=cv)
    assert np.array_equal(ck[1, 2, 1, 2], kv.reshape(rows, L, 2, H, 128)[4, 1, 0, 1])


def _hf_logits(model, W, tokens, memory, int8=True):
    """transformers' CohereAsrDecoder + head in float32 on the oracle's (dequantized) weights: logits of the last
    position for one sequence (tokens (t,), memory (frames, width))."""
    import copy

    m = copy.deepcopy(model)
    dec = m.model.decoder

    def deq(w8):
        q, s = w8
        k = q.shape[1]
        inv = np.empty(16, np.int64)
        inv[list(oracle_perm())] = np.arange(16)
        nat = (q.reshape(-1, k // 16, 16)[:, :, inv].reshape(q.shape).astype(np.int32) - 128).astype(np.float32)
        return torch.from_numpy(nat * s[:, None])

    with torch.no_grad():
        if int8:
            for lyr, ly in zip(dec.layers, W["layers"]):
                d = lyr.self_attn.q_proj.weight.shape[0]
                wqkv = deq(ly["qkv_w8"])
                lyr.self_attn.q_proj.weight.copy_(wqkv[:d])
                lyr.self_attn.k_proj.weight.copy_(wqkv[d:2 * d])
                lyr.self_attn.v_proj.weight.copy_(wqkv[2 * d:])
                lyr.mlp.fc1.weight.copy_(deq(ly["fc1_w8"]))
                lyr.mlp.fc2.weight.copy_(deq(ly["fc2_w8"]))
            m.proj_out.weight.copy_(deq(W["head_w8"]))
        out = dec(input_ids=torch.tensor(tokens)[None], encoder_hidden_states=memory.float()[None], use_cache=False)
        return m.proj_out(out.last_hidden_state[0, -1]).numpy()


def oracle_perm():
    return (0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15)


def test_decoder_step_follows_transformers():
    """oracle.decoder_step (the reference's step order) on int8 weights and int8 KV caches against transformers'
    CohereAsrDecoder in float32 on the same dequantized weights and float caches, teacher-forced through a prompt:
    logits within 2.5 % RMS (the int8 KV quantization and bf16 roundings), while the logits of the neighbouring
    position are several times further off."""
    model = make_decoder(seed=3)
    cfg = model.config
    W = oracle_weights(model)
    g = torch.Generator().manual_seed(4)
    lengths = [9, 20, 14]
    slots, L, H = 4, cfg.num_hidden_layers, cfg.num_attention_heads
    st = oracle_state(L, slots, H, seq=40, frames=24, max_prompt=8, pad=cfg.pad_token_id)
    memories = [torch.randn(n, cfg.hidden_size, generator=g).to(torch.bfloat16) for n in lengths]
    kv = torch.cat([cross_kv(model, mem) for mem in memories])
    slot_of = np.concatenate([np.full(n, s, np.int32) for s, n in zip([1, 0, 3], lengths)])
    frame_of = np.concatenate([np.arange(n, dtype=np.int32) for n in lengths])
    oracle.dec_scatter_kv(bf16_bits(kv), slot_of, frame_of, ck8=st["cross_k8"], cv8=st["cross_v8"],
                          cks=st["cross_ks"], cvs=st["cross_vs"])
    prompts = [torch.randint(5, cfg.vocab_size, (6,), generator=g) for _ in lengths]
    for s, p, n in zip([1, 0, 3], prompts, lengths):
        st["forced"][s, :6] = p.numpy()
        st["tok"][s], st["pos"][s], st["plen"][s], st["limit"][s] = p[0], 0, 6, 30
        st["cross_len"][s], st["finished"][s] = n, 0
    st["active"] = np.array([1, 0, 3, slots], np.int32)
    errs, shifted = [], []
    for step in range(5):
        logits = bf16_float(oracle.decoder_step(W, st, 4))
        for r, (s, mem) in enumerate(zip([1, 0, 3], memories)):
            toks = prompts[r][:step + 1].tolist()
            want = _hf_logits(model, W, toks, mem)
            errs.append(np.sqrt(np.mean((logits[r] - want) ** 2)) / np.sqrt(np.mean(want ** 2)))
            if step > 0:
                prev = _hf_logits(model, W, toks[:-1], mem)
                shifted.append(np.sqrt(np.mean((logits[r] - prev) ** 2)) / np.sqrt(np.mean(prev ** 2)))
        assert all(st["tok"][s] == prompts[r][step + 1] for r, s in enumerate([1, 0, 3]))  # forced
    assert max(errs) < 2.5e-2, errs
    assert min(shifted) > 5 * max(errs), (min(shifted), max(errs))
