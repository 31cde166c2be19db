"""Config 3 at its own workload: the captured decoder step with 64 active slots, 8 layers (width 1024, 8 heads, FFN
4096, vocab 16384, int8 projections and int8 caches), self-attention caches of seeded lengths U(1..448), cross-attention
over 375 encoder frames of N(0, 1) memory per slot, against the CPU checker's step (oracle.decoder_step) from the same
state at every one of 32 steps.

Teacher forcing on the state: before each step the product's slot state and self caches (which the previous step
advanced) are copied into the checker's, so every step is compared from identical inputs. The bar:
  * logits: the step chains ~30 kernels whose fp32 sums run in another order than the checker's, through bf16
    activations, so last-bit differences reach the logits; at every step the RMS difference stays within 1.5x and the
    largest within 2x of what the checker itself moves when 1 % of its position-table entries move by one bf16 ulp;
  * tokens: the product's greedy tokens equal the checker's (first index of the maximum) at least as often, less one
    percentage point, as the perturbed checker's do. With this model a perturbation of that size moves the logits
    by ~1.5 % RMS, so a few percent of the picks are near-ties (often exact bf16 ties) that either side may break;
    the measured agreement of both is printed;
  * clear-margin rows: wherever the checker's gap between its best and second-best logit exceeds twice that step's
    largest logit difference of the perturbed checker, the pick is not a near-tie, and the product's token must equal
    the checker's (index-exact); the number of such rows is printed;
  * the positions advance exactly as the checker's.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from decoder_helpers import make_decoder, oracle_state, oracle_weights
from helpers import bf16_bits, bf16_float, bf16_ulp

pytestmark = pytest.mark.gpu

SLOTS, LAYERS, WIDTH, HEADS, FFN, VOCAB, FRAMES, STEPS = 64, 8, 1024, 8, 4096, 16384, 375, 32
MAX_LEN = 448  # self-attention cache lengths drawn from U(1..448)


def _to_state(dec, st):
    for k in ("tok", "pos", "finished", "out", "plen", "limit", "forced", "cross_len"):
        st[k][...] = getattr(dec, k).cpu().numpy()
    for a, b in (("self_k", "self_k8"), ("self_v", "self_v8"), ("self_ks", "self_ks"), ("self_vs", "self_vs")):
        st[b][...] = getattr(dec, a).cpu().numpy()


def config3_decoder(gpu):
    """Config 3's decoder and state on the GPU and the checker's copy: (model, dec, st, W, b). Every slot is past its
    prompt with a self cache of U(1..448) positions of seeded int8 keys/values; the cross caches hold N(0, 1) memory's
    keys and values (computed once on the GPU and scattered on both sides identically)."""
    from kernels.stream_decoder import StreamDecoder

    model = make_decoder(hidden=WIDTH, heads=HEADS, layers=LAYERS, ffn=FFN, vocab=VOCAB, seed=3, device=gpu,
                         dtype=torch.bfloat16)
    cfg = model.config
    max_prompt = 4
    dec = StreamDecoder(model, slots=SLOTS, max_new_tokens=MAX_LEN + STEPS, max_prompt=max_prompt, buckets=(SLOTS,),
                        int8=True, frames=FRAMES)
    g = torch.Generator().manual_seed(33)
    # the slot state: every slot past its prompt, its cache holding `length` positions
    lengths = torch.randint(1, MAX_LEN + 1, (SLOTS,), generator=g).int()
    tok = torch.randint(5, VOCAB, (SLOTS,), generator=g)
    with torch.no_grad():
        for name in ("self_k", "self_v"):
            getattr(dec, name).copy_(torch.randint(-127, 128, getattr(dec, name).shape, generator=g).to(torch.int8))
        for name in ("self_ks", "self_vs"):
            getattr(dec, name).copy_(torch.rand(getattr(dec, name).shape, generator=g) * 0.02 + 0.002)
        dec.tok[:SLOTS] = tok.to(gpu)
        dec.pos[:SLOTS] = lengths.to(gpu)
        dec.plen[:SLOTS] = 1
        dec.limit[:SLOTS] = MAX_LEN + STEPS
        dec.finished[:SLOTS] = 0
        dec.cross_len[:SLOTS] = FRAMES
        # cross-attention keys and values of N(0, 1) memory, computed once on the GPU; both sides scatter the same
        mem = torch.randn(SLOTS * FRAMES, WIDTH, generator=g).to(torch.bfloat16).to(gpu)
        kv = torch.nn.functional.linear(mem.float(), dec.cross_w.float(), dec.cross_b.float()).to(torch.bfloat16)
        slot_of = torch.arange(SLOTS, dtype=torch.int32).repeat_interleave(FRAMES).to(gpu)
        frame_of = torch.arange(FRAMES, dtype=torch.int32).repeat(SLOTS).to(gpu)
        from kernels.cuda_ext import ext

        ext.dec_scatter_kv_q8(kv, slot_of, frame_of, dec.cross_k, dec.cross_v, dec.cross_ks, dec.cross_vs)
    torch.cuda.synchronize()
    st = oracle_state(LAYERS, SLOTS, HEADS, dec.seq, FRAMES, max_prompt, cfg.pad_token_id)
    for a, b in (("cross_k", "cross_k8"), ("cross_v", "cross_v8"), ("cross_ks", "cross_ks"), ("cross_vs", "cross_vs")):
        st[b][...] = getattr(dec, a).cpu().numpy()
    W = oracle_weights(model)
    b = dec.set_active(list(range(SLOTS)))
    assert b == SLOTS
    torch.cuda.synchronize()
    st["active"] = dec.active.cpu().numpy()
    return model, dec, st, W, b


def test_config3_step_tokens(gpu):
    model, dec, st, W, b = config3_decoder(gpu)
    # the checker's own sensitivity: the same step from the same state with 1 % of the position-table entries moved
    # by one bf16 ulp (the size of the last-bit differences the kernels' fp32 sums make)
    W_pert = dict(W)
    pt = W["pos_table"].copy()
    pt[np.random.default_rng(0).random(pt.shape) < 0.01] += 1
    W_pert["pos_table"] = pt
    same = same_noise = total = 0
    clear_rows = clear_same = 0
    ratios_rms, ratios_max = [], []
    for step in range(STEPS):
        _to_state(dec, st)
        st_p = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in st.items()}
        dec.step(b)
        torch.cuda.synchronize()
        want = bf16_float(oracle.decoder_step(W, st, b)).astype(np.float64)
        noise = bf16_float(oracle.decoder_step(W_pert, st_p, b)).astype(np.float64)
        got = bf16_float(bf16_bits(dec.logits[:b])).astype(np.float64)
        rms = np.sqrt(np.mean(want ** 2))
        d, dn = np.abs(got - want), np.abs(noise - want)
        ratios_rms.append(np.sqrt(np.mean(d ** 2)) / np.sqrt(np.mean(dn ** 2)))
        ratios_max.append(d.max() / dn.max())
        got_tok, want_tok = dec.tok[:SLOTS].cpu().numpy(), st["tok"][:SLOTS]
        step_same, step_noise = int((got_tok == want_tok).sum()), int((st_p["tok"][:SLOTS] == want_tok).sum())
        same, same_noise, total = same + step_same, same_noise + step_noise, total + SLOTS
        top2 = np.sort(want, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2.0 * dn.max()
        clear_rows += int(clear.sum())
        clear_same += int((got_tok == want_tok)[clear].sum())
        assert np.array_equal(got_tok[clear], want_tok[clear]), (step, np.nonzero(clear & (got_tok != want_tok))[0])
        print(f"step {step}: logits rms diff {np.sqrt(np.mean(d ** 2)) / rms:.2e} max {d.max() / rms:.2e} x RMS "
              f"(perturbed checker {np.sqrt(np.mean(dn ** 2)) / rms:.2e} / {dn.max() / rms:.2e}); tokens equal: "
              f"kernels {step_same}/{SLOTS}, perturbed checker {step_noise}/{SLOTS}", flush=True)
        for r in np.nonzero(got_tok != want_tok)[0]:
            top = want[r].max()
            print(f"  slot {r}: kernels {got_tok[r]} checker {want_tok[r]}, checker's gap between them "
                  f"{top - want[r, got_tok[r]]:.3e} (bf16 ulp of the maximum {bf16_ulp(np.array([top]))[0]:.3e})")
        assert np.array_equal(dec.pos[:SLOTS].cpu().numpy(), st["pos"][:SLOTS]), step
    print(f"tokens: kernels {same} / {total} index-exact with the checker, perturbed checker {same_noise} / {total}; "
          f"logit difference vs the perturbed checker's: rms x{max(ratios_rms):.2f}, max x{max(ratios_max):.2f} "
          f"(worst step); clear-margin rows {clear_same} / {clear_rows} index-exact", flush=True)
    assert max(ratios_rms) <= 1.5 and max(ratios_max) <= 2.0
    assert same >= same_noise - 0.01 * total
