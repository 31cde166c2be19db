"""Decoder fixtures: a seeded random-init transformers CohereAsr decoder (the module the reference's StreamDecoder
converts), its weights as the oracle's decoder_step reads them, and an oracle slot state."""

from __future__ import annotations

import types

import numpy as np
import torch

import oracle
from helpers import bf16_bits


def make_decoder(hidden=256, heads=2, layers=2, ffn=512, vocab=512, seed=0, device="cpu", dtype=torch.float32):
    """A CohereAsr decoder + output head with random weights (normal 0.02 linears and embeddings, random LayerNorm
    affines and biases), every parameter bf16-representable, and `proj` the identity (so the cross-attention memory
    can be given at decoder width). Returns an object with the attributes StreamDecoder reads."""
    from transformers.models.cohere_asr.configuration_cohere_asr import CohereAsrConfig
    from transformers.models.cohere_asr.modeling_cohere_asr import CohereAsrDecoder

    cfg = CohereAsrConfig(vocab_size=vocab, hidden_size=hidden, num_hidden_layers=layers, num_attention_heads=heads,
                          intermediate_size=ffn, head_dim=hidden // heads, max_position_embeddings=1024,
                          encoder_config={"model_type": "parakeet_encoder", "hidden_size": hidden})
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    dec = CohereAsrDecoder(cfg).eval()
    head = torch.nn.Linear(hidden, vocab)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for mod in (dec, head):
            for name, p in mod.named_parameters():
                if name.startswith("proj."):
                    continue
                if "norm" in name:
                    p.copy_((1.0 if name.endswith("weight") else 0.0) + 0.1 * torch.randn(p.shape, generator=g))
                elif p.dim() >= 2:
                    p.copy_(torch.randn(p.shape, generator=g) * 0.05)
                else:
                    p.copy_(torch.randn(p.shape, generator=g) * 0.05)
        dec.pos_emb.weight.mul_(10)  # position embeddings of the same order as the token embeddings' LN input
        dec.proj.weight.copy_(torch.eye(hidden))
        dec.proj.bias.zero_()
        for mod in (dec, head):
            for p in mod.parameters():
                p.copy_(p.to(torch.bfloat16).float())
    dec, head = dec.to(device=device, dtype=dtype), head.to(device=device, dtype=dtype)
    return types.SimpleNamespace(model=types.SimpleNamespace(decoder=dec), proj_out=head, config=cfg)


def oracle_weights(model, int8=True):
    """The decoder's weights as oracle.decoder_step reads them: bf16 bits; with int8 the qkv / fc1 / fc2 / head
    projections in prepare_w8's layout (the oracle's own quantizer), o / cq / co bf16, as the reference keeps them."""
    dec, cfg = model.model.decoder, model.config
    bits = lambda t: bf16_bits(t.detach().float().cpu().to(torch.bfloat16))  # noqa: E731
    ln = lambda m: (bits(m.weight), bits(m.bias), float(m.eps))  # noqa: E731
    W = {"embed": bits(dec.embed_tokens.weight), "pos_table": bits(dec.pos_emb.weight),
         "emb_ln": ln(dec.embedding_layernorm), "final_ln": ln(dec.norm), "scale": (cfg.hidden_size //
                                                                                  cfg.num_attention_heads) ** -0.5,
         "eos": cfg.eos_token_id, "layers": []}
    for lyr in dec.layers:
        sa, ca = lyr.self_attn, lyr.encoder_attn
        ly = {"ln1": ln(lyr.input_layernorm), "ln2": ln(lyr.post_attention_layernorm), "ln3": ln(lyr.final_layernorm)}
        qkv_w = torch.cat([sa.q_proj.weight, sa.k_proj.weight, sa.v_proj.weight])
        ly["qkv_b"] = bits(torch.cat([sa.q_proj.bias, sa.k_proj.bias, sa.v_proj.bias]))
        ly["o_w"], ly["o_b"] = bits(sa.o_proj.weight), bits(sa.o_proj.bias)
        ly["cq_w"], ly["cq_b"] = bits(ca.q_proj.weight), bits(ca.q_proj.bias)
        ly["co_w"], ly["co_b"] = bits(ca.o_proj.weight), bits(ca.o_proj.bias)
        ly["fc1_b"], ly["fc2_b"] = bits(lyr.mlp.fc1.bias), bits(lyr.mlp.fc2.bias)
        for name, w in (("qkv", qkv_w), ("fc1", lyr.mlp.fc1.weight), ("fc2", lyr.mlp.fc2.weight)):
            if int8:
                ly[name + "_w8"] = oracle.prepare_w8(bits(w))
            else:
                ly[name + "_w"] = bits(w)
        W["layers"].append(ly)
    if int8:
        W["head_w8"] = oracle.prepare_w8(bits(model.proj_out.weight))
    else:
        W["head_w"] = bits(model.proj_out.weight)
    W["head_b"] = bits(model.proj_out.bias)
    return W


def oracle_state(L, slots, heads, seq, frames, max_prompt, pad):
    """An empty oracle slot state with int8 caches (the reference's StreamDecoder buffers, numpy)."""
    S1 = slots + 1
    st = {"self_k8": np.zeros((L, S1, heads, seq, 128), np.int8), "self_ks": np.ones((L, S1, heads, seq), np.float32),
          "cross_k8": np.zeros((L, S1, heads, frames, 128), np.int8),
          "cross_ks": np.ones((L, S1, heads, frames), np.float32),
          "cross_len": np.ones(S1, np.int32), "tok": np.full(S1, pad, np.int64), "pos": np.zeros(S1, np.int32),
          "plen": np.ones(S1, np.int32), "limit": np.zeros(S1, np.int32), "finished": np.ones(S1, np.uint8),
          "forced": np.full((S1, max_prompt), pad, np.int64), "out": np.full((S1, seq + 1), pad, np.int64),
          "dummy": slots}
    st["self_v8"], st["self_vs"] = np.zeros_like(st["self_k8"]), np.ones_like(st["self_ks"])
    st["cross_v8"], st["cross_vs"] = np.zeros_like(st["cross_k8"]), np.ones_like(st["cross_ks"])
    return st


def cross_kv(model, memory: torch.Tensor) -> torch.Tensor:
    """Every layer's cross-attention keys and values of memory (frames, width): (frames, L * 2 * width), bf16, in
    the reference's order (per layer k then v), computed in float32 and rounded once."""
    dec = model.model.decoder
    w = torch.cat([t for lyr in dec.layers for t in (lyr.encoder_attn.k_proj.weight, lyr.encoder_attn.v_proj.weight)])
    b = torch.cat([t for lyr in dec.layers for t in (lyr.encoder_attn.k_proj.bias, lyr.encoder_attn.v_proj.bias)])
    return torch.nn.functional.linear(memory.float().cpu(), w.float().cpu(), b.float().cpu()).to(torch.bfloat16)
