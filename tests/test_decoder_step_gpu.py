"""GPU parity of the decoder step's kernels (embedding, residual LayerNorm, attention over int8 / bf16 caches, greedy
pick, cross-cache scatter) and of the captured StreamDecoder step against the CPU checker, through the C ABI."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from decoder_helpers import cross_kv, make_decoder, oracle_state, oracle_weights
from helpers import assert_bf16_close, bf16_bits, bf16_float, bf16_ulp

pytestmark = pytest.mark.gpu


def _ext():
    from kernels.cuda_ext import ext

    return ext


def _bf(t):
    return bf16_bits(t.to(torch.bfloat16))


def _close(got_bits, want_bits, rms_tol=2e-3):
    got, want = bf16_float(got_bits).astype(np.float64), bf16_float(want_bits).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    diff = np.abs(got - want)
    tol = np.maximum(1e-2 * rms, bf16_ulp(want) * 1.0001)
    assert (diff <= tol).all(), f"{int((diff > tol).sum())} beyond tolerance, worst {(diff / tol).max():.2f} x"
    assert np.sqrt(np.mean(diff ** 2)) <= rms_tol * rms


def test_dec_embed_and_add_ln(gpu):
    g = torch.Generator().manual_seed(1)
    V, P, W = 300, 64, 1024
    emb, ptab = torch.randn(V, W, generator=g).to(torch.bfloat16), (torch.randn(P, W, generator=g) * 3).to(torch.bfloat16)
    ln = [((1 + 0.1 * torch.randn(W, generator=g)).to(torch.bfloat16), (0.1 * torch.randn(W, generator=g)).to(torch.bfloat16))
          for _ in range(2)]
    active = torch.tensor([5, 0, 2, 7, 7], dtype=torch.int32)
    tok = torch.randint(0, V, (8,), generator=g)
    pos = torch.randint(0, P, (8,), generator=g).to(torch.int32)
    d = lambda t: t.to(gpu)  # noqa: E731
    x = torch.empty(5, W, dtype=torch.bfloat16, device=gpu)
    h = torch.empty_like(x)
    _ext().dec_embed(d(active), d(tok), d(pos), d(emb), d(ptab), d(ln[0][0]), d(ln[0][1]), 1e-5, d(ln[1][0]),
                     d(ln[1][1]), 1e-5, x, h)
    ox, oh = oracle.dec_embed(active.numpy(), tok.numpy(), pos.numpy(), _bf(emb), _bf(ptab),
                              (_bf(ln[0][0]), _bf(ln[0][1]), 1e-5), (_bf(ln[1][0]), _bf(ln[1][1]), 1e-5))
    assert_bf16_close(bf16_bits(x), ox)
    assert_bf16_close(bf16_bits(h), oh)
    y = torch.randn(5, W, generator=g).to(torch.bfloat16)
    x_or = bf16_bits(x).copy()
    h2 = torch.empty_like(x)
    _ext().dec_add_ln(x, d(y), d(ln[1][0]), d(ln[1][1]), 1e-5, h2)
    oh2 = oracle.dec_add_ln(x_or, _bf(y), (_bf(ln[1][0]), _bf(ln[1][1]), 1e-5))
    assert np.array_equal(bf16_bits(x), x_or)  # the residual sum is one rounding
    assert_bf16_close(bf16_bits(h2), oh2)


def _caches(g, slots, H, T):
    k8 = torch.randint(-127, 128, (slots, H, T, 128), generator=g).to(torch.int8)
    v8 = torch.randint(-127, 128, (slots, H, T, 128), generator=g).to(torch.int8)
    ks = torch.rand(slots, H, T, generator=g) * 0.02 + 0.001
    vs = torch.rand(slots, H, T, generator=g) * 0.02 + 0.001
    return k8, v8, ks, vs


@pytest.mark.parametrize("self_attn,splits", [(True, 1), (False, 1), (False, 4)])
def test_dec_attention_q8(gpu, self_attn, splits):
    g = torch.Generator().manual_seed(2 + splits)
    slots, H, T, rows = 9, 8, 465, 6
    k8, v8, ks, vs = _caches(g, slots, H, T)
    active = torch.tensor([3, 0, 8, 1, 5, 8], dtype=torch.int32)
    n = torch.tensor([448, 1, 0, 37, 200, 10, 464, 3, 2], dtype=torch.int32) if self_attn else \
        torch.tensor([375, 1, 7, 100, 64, 375, 2, 9, 30], dtype=torch.int32)
    q = torch.randn(rows, (3 if self_attn else 1) * H * 128, generator=g).to(torch.bfloat16)
    out = torch.empty(rows, H * 128, dtype=torch.bfloat16, device=gpu)
    part = torch.empty(rows * H * splits * 130, device=gpu)
    gk, gv, gks, gvs = (t.to(gpu) for t in (k8, v8, ks, vs))
    # rows 2 and 5 share slot 8 (as the dummy slot does): give them one row so the cache write is deterministic
    q[5] = q[2]
    _ext().dec_attention_q8(self_attn, active.to(gpu), q.to(gpu), gk, gv, gks, gvs, n.to(gpu), 128 ** -0.5, splits,
                            part, out)
    ck, cv, cks, cvs = (t.numpy().copy() for t in (k8, v8, ks, vs))
    want = oracle.dec_attention(self_attn, active.numpy(), _bf(q), n.numpy(), 128 ** -0.5, k8=ck, v8=cv, ks=cks,
                                vs=cvs)
    _close(bf16_bits(out), want)
    if self_attn:  # the new keys and values, quantized the same way
        assert np.array_equal(gk.cpu().numpy(), ck) and np.array_equal(gv.cpu().numpy(), cv)
        assert np.array_equal(gks.cpu().numpy(), cks) and np.array_equal(gvs.cpu().numpy(), cvs)


def test_dec_attention_bf16(gpu):
    g = torch.Generator().manual_seed(7)
    slots, H, T, rows = 4, 8, 100, 3
    k = torch.randn(slots, H, T, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(slots, H, T, 128, generator=g).to(torch.bfloat16)
    active = torch.tensor([2, 0, 3], dtype=torch.int32)
    n = torch.tensor([50, 99, 1, 7], dtype=torch.int32)
    q = torch.randn(rows, 3 * H * 128, generator=g).to(torch.bfloat16)
    gk, gv = k.to(gpu), v.to(gpu)
    out = torch.empty(rows, H * 128, dtype=torch.bfloat16, device=gpu)
    _ext().dec_attention(True, active.to(gpu), q.to(gpu), gk, gv, n.to(gpu), 0.1, 1, None, out)
    ck, cv = bf16_bits(k).copy(), bf16_bits(v).copy()
    want = oracle.dec_attention(True, active.numpy(), _bf(q), n.numpy(), 0.1, k=ck, v=cv)
    _close(bf16_bits(out), want)
    assert np.array_equal(bf16_bits(gk), ck) and np.array_equal(bf16_bits(gv), cv)


@pytest.mark.parametrize("q8", [True, False])
@pytest.mark.parametrize("self_attn", [True, False])
def test_dec_attention_long_caches(gpu, q8, self_attn):
    """Caches longer than one pass of the kernel (512 int8 / 256 bf16 keys per pass): the online softmax's rescale
    across passes, with lengths on and around the pass boundaries."""
    g = torch.Generator().manual_seed(11 + 2 * q8 + self_attn)
    slots, H, T = 7, 8, 1300
    n_self = [1299, 512, 513, 1024, 256, 257, 700]
    n_cross = [1300, 512, 513, 1025, 256, 257, 1]
    n = torch.tensor(n_self if self_attn else n_cross, dtype=torch.int32)
    active = torch.tensor([0, 1, 2, 3, 4, 5, 6], dtype=torch.int32)
    rows = active.numel()
    q = torch.randn(rows, (3 if self_attn else 1) * H * 128, generator=g).to(torch.bfloat16)
    out = torch.empty(rows, H * 128, dtype=torch.bfloat16, device=gpu)
    if q8:
        k8, v8, ks, vs = _caches(g, slots, H, T)
        gk, gv, gks, gvs = (t.to(gpu) for t in (k8, v8, ks, vs))
        _ext().dec_attention_q8(self_attn, active.to(gpu), q.to(gpu), gk, gv, gks, gvs, n.to(gpu), 128 ** -0.5, 1,
                                None, out)
        ck, cv, cks, cvs = (t.numpy().copy() for t in (k8, v8, ks, vs))
        want = oracle.dec_attention(self_attn, active.numpy(), _bf(q), n.numpy(), 128 ** -0.5, k8=ck, v8=cv,
                                    ks=cks, vs=cvs)
    else:
        k = torch.randn(slots, H, T, 128, generator=g).to(torch.bfloat16)
        v = torch.randn(slots, H, T, 128, generator=g).to(torch.bfloat16)
        gk, gv = k.to(gpu), v.to(gpu)
        _ext().dec_attention(self_attn, active.to(gpu), q.to(gpu), gk, gv, n.to(gpu), 0.05, 1, None, out)
        ck, cv = bf16_bits(k).copy(), bf16_bits(v).copy()
        want = oracle.dec_attention(self_attn, active.numpy(), _bf(q), n.numpy(), 0.05, k=ck, v=cv)
    _close(bf16_bits(out), want)


@pytest.mark.parametrize("q8", [True, False])
@pytest.mark.parametrize("self_attn,splits", [(True, 1), (True, 2), (False, 1), (False, 2)])
def test_dec_attention_many_rows(gpu, q8, self_attn, splits):
    """40 rows x 8 heads: unsplit, the register form (two workgroups per CU; cross-attention with its early pass);
    split in two, more workgroups than CUs, so the LDS form (values copied into LDS); lengths on the 64-key group
    boundaries, 0 (self: the new token alone) and 448, against the checker."""
    g = torch.Generator().manual_seed(31 + 2 * q8 + self_attn + 4 * splits)
    rows, H, T = 40, 8, 465
    slots = rows + 1
    active = torch.randperm(slots, generator=g)[:rows].int()
    edge = [0, 1, 63, 64, 65, 448] if self_attn else [1, 63, 64, 65, 375, 465]
    n = torch.randint(1, 449 if self_attn else T + 1, (slots,), generator=g).int()
    n[active[:len(edge)].long()] = torch.tensor(edge, dtype=torch.int32)
    q = torch.randn(rows, (3 if self_attn else 1) * H * 128, generator=g).to(torch.bfloat16)
    out = torch.empty(rows, H * 128, dtype=torch.bfloat16, device=gpu)
    part = torch.empty(rows * H * splits * 130, device=gpu)
    print(f"dec_attention rows={rows} q8={q8} self={self_attn} splits={splits}", flush=True)
    if q8:
        k8, v8, ks, vs = _caches(g, slots, H, T)
        gk, gv, gks, gvs = (t.to(gpu) for t in (k8, v8, ks, vs))
        _ext().dec_attention_q8(self_attn, active.to(gpu), q.to(gpu), gk, gv, gks, gvs, n.to(gpu), 128 ** -0.5,
                                splits, part, out)
        ck, cv, cks, cvs = (t.numpy().copy() for t in (k8, v8, ks, vs))
        want = oracle.dec_attention(self_attn, active.numpy(), _bf(q), n.numpy(), 128 ** -0.5, k8=ck, v8=cv,
                                    ks=cks, vs=cvs)
        if self_attn:
            assert np.array_equal(gk.cpu().numpy(), ck) and np.array_equal(gv.cpu().numpy(), cv)
            assert np.array_equal(gks.cpu().numpy(), cks) and np.array_equal(gvs.cpu().numpy(), cvs)
    else:
        k = torch.randn(slots, H, T, 128, generator=g).to(torch.bfloat16)
        v = torch.randn(slots, H, T, 128, generator=g).to(torch.bfloat16)
        gk, gv = k.to(gpu), v.to(gpu)
        _ext().dec_attention(self_attn, active.to(gpu), q.to(gpu), gk, gv, n.to(gpu), 0.05, splits, part, out)
        ck, cv = bf16_bits(k).copy(), bf16_bits(v).copy()
        want = oracle.dec_attention(self_attn, active.numpy(), _bf(q), n.numpy(), 0.05, k=ck, v=cv)
        if self_attn:
            assert np.array_equal(bf16_bits(gk), ck) and np.array_equal(bf16_bits(gv), cv)
    _close(bf16_bits(out), want)


@pytest.mark.parametrize("self_attn", [True, False])
def test_dec_attention_sixteen_heads(gpu, self_attn):
    """16 heads (the kernels take any head count; the decoders here have 8): 20 rows, int8 caches, against the
    checker, with the new key and value of self-attention written bit for bit."""
    g = torch.Generator().manual_seed(41 + self_attn)
    rows, H, T = 20, 16, 200
    slots = rows + 1
    active = torch.randperm(slots, generator=g)[:rows].int()
    n = torch.randint(0, 199 if self_attn else T + 1, (slots,), generator=g).int()
    if not self_attn:
        n = n.clamp(min=1)
    q = torch.randn(rows, (3 if self_attn else 1) * H * 128, generator=g).to(torch.bfloat16)
    out = torch.empty(rows, H * 128, dtype=torch.bfloat16, device=gpu)
    k8, v8, ks, vs = _caches(g, slots, H, T)
    gk, gv, gks, gvs = (t.to(gpu) for t in (k8, v8, ks, vs))
    _ext().dec_attention_q8(self_attn, active.to(gpu), q.to(gpu), gk, gv, gks, gvs, n.to(gpu), 128 ** -0.5, 1, None,
                            out)
    ck, cv, cks, cvs = (t.numpy().copy() for t in (k8, v8, ks, vs))
    want = oracle.dec_attention(self_attn, active.numpy(), _bf(q), n.numpy(), 128 ** -0.5, k8=ck, v8=cv, ks=cks,
                                vs=cvs)
    _close(bf16_bits(out), want)
    if self_attn:
        assert np.array_equal(gk.cpu().numpy(), ck) and np.array_equal(gv.cpu().numpy(), cv)
        assert np.array_equal(gks.cpu().numpy(), cks) and np.array_equal(gvs.cpu().numpy(), cvs)


def test_dec_pick_exact(gpu):
    g = torch.Generator().manual_seed(8)
    rows, V, S = 7, 16384, 10
    logits = torch.randn(rows, V, generator=g).to(torch.bfloat16)
    logits[1, 100] = logits[1, 9000] = 50.0  # tie: the first index
    active = torch.tensor([0, 1, 2, 3, 4, 9, 6], dtype=torch.int32)  # 9 = dummy
    st = {"tok": torch.randint(0, V, (S,), generator=g), "pos": torch.randint(0, 30, (S,), generator=g).int(),
          "finished": torch.tensor([0, 0, 0, 1, 0, 0, 0, 0, 0, 1], dtype=torch.uint8),
          "forced": torch.randint(0, V, (S, 16), generator=g), "plen": torch.randint(1, 16, (S,), generator=g).int(),
          "limit": torch.randint(5, 40, (S,), generator=g).int(), "out": torch.full((S, 50), 2, dtype=torch.long)}
    logits[4, 3] = 60.0  # eos
    dev = {k: v.to(gpu) for k, v in st.items()}
    _ext().dec_pick(logits.to(gpu), active.to(gpu), 9, dev["tok"], dev["pos"], dev["finished"], dev["forced"],
                    dev["plen"], dev["limit"], dev["out"], 2, 3)
    host = {k: v.numpy().copy() for k, v in st.items()}
    oracle.dec_pick(_bf(logits), active.numpy(), 9, host["tok"], host["pos"], host["finished"], host["forced"],
                    host["plen"], host["limit"], host["out"], 3)
    for k in ("tok", "pos", "finished", "out"):
        assert np.array_equal(dev[k].cpu().numpy(), host[k]), k


def test_dec_scatter_kv_exact(gpu):
    g = torch.Generator().manual_seed(9)
    L, S, H, T, rows = 3, 5, 8, 40, 50
    kv = torch.randn(rows, L * 2 * H * 128, generator=g).to(torch.bfloat16)
    slot_of = torch.randint(0, S, (rows,), generator=g).int()
    frame_of = torch.randperm(T, generator=g)[:rows % T].int()
    frame_of = torch.cat([frame_of, torch.randint(0, T, (rows - len(frame_of),), generator=g).int()])
    # distinct (slot, frame) targets
    keys = slot_of.long() * T + frame_of.long()
    first = torch.tensor([int((keys[:i] == keys[i]).sum()) == 0 for i in range(rows)])
    kv, slot_of, frame_of = kv[first], slot_of[first], frame_of[first]
    ck8 = torch.zeros(L, S, H, T, 128, dtype=torch.int8, device=gpu)
    cv8, cks, cvs = torch.zeros_like(ck8), torch.zeros(L, S, H, T, device=gpu), torch.zeros(L, S, H, T, device=gpu)
    _ext().dec_scatter_kv_q8(kv.to(gpu), slot_of.to(gpu), frame_of.to(gpu), ck8, cv8, cks, cvs)
    h = [np.zeros(t.shape, np.int8 if t.dtype == torch.int8 else np.float32) for t in (ck8, cv8, cks, cvs)]
    oracle.dec_scatter_kv(_bf(kv), slot_of.numpy(), frame_of.numpy(), ck8=h[0], cv8=h[1], cks=h[2], cvs=h[3])
    for a, b in zip((ck8, cv8, cks, cvs), h):
        assert np.array_equal(a.cpu().numpy(), b)
    ck = torch.zeros(L, S, H, T, 128, dtype=torch.bfloat16, device=gpu)
    cv = torch.zeros_like(ck)
    _ext().dec_scatter_kv(kv.to(gpu), slot_of.to(gpu), frame_of.to(gpu), ck, cv)
    hk, hv = np.zeros(ck.shape, np.uint16), np.zeros(ck.shape, np.uint16)
    oracle.dec_scatter_kv(_bf(kv), slot_of.numpy(), frame_of.numpy(), ck=hk, cv=hv)
    assert np.array_equal(bf16_bits(ck), hk) and np.array_equal(bf16_bits(cv), hv)


def _sync_state(dec, st):
    """The product's slot state and self caches into the checker's (teacher forcing on the state)."""
    for k in ("tok", "pos", "finished", "out", "plen", "limit", "forced", "cross_len"):
        st[k][...] = getattr(dec, k).cpu().numpy()
    st["self_k8"][...] = dec.self_k.cpu().numpy()
    st["self_v8"][...] = dec.self_v.cpu().numpy()
    st["self_ks"][...] = dec.self_ks.cpu().numpy()
    st["self_vs"][...] = dec.self_vs.cpu().numpy()


def test_stream_decoder_step(gpu):
    """The captured step (graph replay per bucket) against oracle.decoder_step from the same state at every step. A
    step chains ~30 kernels through LayerNorms, so last-bit differences of the fp32 sums reach the logits as a few
    bf16 ulps: the bar is the checker's own sensitivity -- the kernels' logits differ from the checker's by at most
    1.25x (RMS) / 2x (max) what the checker itself moves when 1 % of the position-table elements move by one bf16 ulp
    (both measure the same kind of last-bit noise; each single draw of it varies by tens of percent) -- and
    the picked token equals the checker's wherever the checker's top two logits are further apart than twice the
    largest logit difference."""
    from kernels.stream_decoder import StreamDecoder

    model = make_decoder(hidden=1024, heads=8, layers=2, ffn=4096, vocab=2048, seed=11, device=gpu,
                         dtype=torch.bfloat16)
    cfg = model.config
    dec = StreamDecoder(model, slots=8, max_new_tokens=24, max_prompt=4, buckets=(1, 2, 4, 8), int8=True, frames=32)
    W = oracle_weights(model)
    st = oracle_state(2, 8, 8, dec.seq, 32, 4, cfg.pad_token_id)
    g = torch.Generator().manual_seed(12)
    slots, lengths = [3, 0, 6, 5, 1], [32, 7, 20, 1, 15]
    memories = [torch.randn(n, 1024, generator=g).to(torch.bfloat16) for n in lengths]
    kv = torch.cat([cross_kv(model, m) for m in memories])
    slot_of = np.concatenate([np.full(n, s, np.int32) for s, n in zip(slots, lengths)])
    frame_of = np.concatenate([np.arange(n, dtype=np.int32) for n in lengths])
    _ext().dec_scatter_kv_q8(kv.to(gpu), torch.from_numpy(slot_of).to(gpu), torch.from_numpy(frame_of).to(gpu),
                             dec.cross_k, dec.cross_v, dec.cross_ks, dec.cross_vs)
    oracle.dec_scatter_kv(bf16_bits(kv), slot_of, frame_of, ck8=st["cross_k8"], cv8=st["cross_v8"],
                          cks=st["cross_ks"], cvs=st["cross_vs"])
    prompts = [torch.randint(5, cfg.vocab_size, (int(torch.randint(1, 5, (1,), generator=g)),), generator=g)
               for _ in slots]
    dec.admit(slots, prompts, lengths)
    b = dec.set_active(slots)
    torch.cuda.synchronize()
    st["active"] = dec.active.cpu().numpy()
    W_pert = dict(W)
    pt = W["pos_table"].copy()
    moved = np.random.default_rng(0).random(pt.shape) < 0.01
    pt[moved] += 1
    W_pert["pos_table"] = pt
    agree = total = 0
    stats = lambda a, w: (np.sqrt(np.mean((a - w) ** 2)), np.abs(a - w).max())  # noqa: E731
    for step in range(12):
        _sync_state(dec, st)
        st_p = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in st.items()}
        dec.step(b)
        torch.cuda.synchronize()
        want = oracle.decoder_step(W, st, b)
        noise = oracle.decoder_step(W_pert, st_p, b)
        got = bf16_bits(dec.logits[:b])
        real = [r for r, s in enumerate(st["active"][:b]) if s != dec.dummy]
        gf, wf_, nf = (bf16_float(a[real]).astype(np.float64) for a in (got, want, noise))
        (rms_k, max_k), (rms_n, max_n) = stats(gf, wf_), stats(nf, wf_)
        print(f"step {step}: kernels vs checker rms {rms_k:.2e} max {max_k:.2e}; perturbed checker rms {rms_n:.2e} "
              f"max {max_n:.2e}", flush=True)
        assert rms_k <= 1.25 * rms_n and max_k <= 2 * max_n
        diff = max_k
        wf = bf16_float(want)
        for r in real:
            s = st["active"][r]
            top2 = np.sort(wf[r])[-2:]
            if top2[1] - top2[0] > 2 * diff:
                total += 1
                agree += int(dec.tok[s].item() == st["tok"][s])
        assert np.array_equal(dec.pos.cpu().numpy(), st["pos"])
    assert total > 20 and agree == total, (agree, total)


@pytest.mark.parametrize("int8", [True, False])
def test_fused_step_matches_unfused(int8, gpu):
    """The step with the residual LayerNorms folded into the projections (the default) against the step with the
    reference's separate dec_add_ln launches, from the same state for 10 steps: logits, tokens, positions, outputs
    and the self caches bit-identical (the fused kernels do the same arithmetic in the same order)."""
    from kernels.stream_decoder import StreamDecoder

    model = make_decoder(hidden=1024, heads=8, layers=2, ffn=4096, vocab=2048, seed=13, device=gpu,
                         dtype=torch.bfloat16)
    kw = dict(slots=8, max_new_tokens=24, max_prompt=4, buckets=(1, 2, 4, 8), int8=int8, frames=32)
    decs = [StreamDecoder(model, fused=True, **kw), StreamDecoder(model, fused=False, **kw)]
    assert decs[0].fused and not decs[1].fused
    g = torch.Generator().manual_seed(14)
    slots, lengths = [3, 0, 6, 5, 1], [32, 7, 20, 1, 15]
    mem = torch.randn(sum(lengths), 1024, generator=g).to(torch.bfloat16).to(gpu)
    prompts = [torch.randint(5, model.config.vocab_size, (3,), generator=g) for _ in slots]
    for d in decs:
        d.fill_cross(mem, lengths, slots)
        d.admit(slots, prompts, lengths)
    bs = [d.set_active(slots) for d in decs]
    assert bs[0] == bs[1]
    for step in range(10):
        for d in decs:
            d.step(bs[0])
        torch.cuda.synchronize()
        a, b = decs
        print(f"step {step}", flush=True)
        assert torch.equal(a.logits[:bs[0]].view(torch.int16), b.logits[:bs[0]].view(torch.int16))
        for name in ("tok", "pos", "out", "finished", "self_k", "self_v"):
            assert torch.equal(getattr(a, name), getattr(b, name)), name
        # the fused pick writes the stepped slots' end flags to the host itself; the unfused step copies them
        assert np.array_equal(a.flags.numpy()[slots], b.flags.numpy()[slots])
        assert np.array_equal(a.flags.numpy()[slots], a.finished.cpu().numpy()[slots])
