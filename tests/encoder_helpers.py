"""FastConformer block fixtures for the encoder tests: a seeded random-init transformers ParakeetEncoderBlock (the
module the reference's fast_encoder.py converts), its distance table, and its tensors for the oracle's layer loop."""

from __future__ import annotations

import numpy as np
import torch

import oracle
from helpers import bf16_bits

MAX_LEN = 512


def make_block(hidden: int, heads: int, ff: int, seed: int, device="cpu", dtype=torch.float32):
    """A ParakeetEncoderBlock with Xavier-uniform weights (seeded), random biases, LayerNorm affines, content/position
    biases and BatchNorm statistics; every parameter bf16-representable. Returns (block, inv_freq)."""
    from transformers.models.parakeet.configuration_parakeet import ParakeetEncoderConfig
    from transformers.models.parakeet.modeling_parakeet import (ParakeetEncoderBlock,
                                                                ParakeetEncoderRelPositionalEncoding)

    cfg = ParakeetEncoderConfig(hidden_size=hidden, num_attention_heads=heads, num_key_value_heads=heads,
                                intermediate_size=ff, conv_kernel_size=9, dropout=0.0, attention_dropout=0.0,
                                activation_dropout=0.0, layerdrop=0.0)
    cfg._attn_implementation = "eager"
    blk = ParakeetEncoderBlock(cfg, 0).eval()
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if name.endswith(("bias_u", "bias_v")):
                p.copy_(torch.randn(p.shape, generator=g) * 0.2)
            elif p.dim() >= 2:
                torch.nn.init.xavier_uniform_(p, generator=g)
            elif "norm" in name and name.endswith("weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
        bn = blk.conv.norm
        bn.running_mean.copy_(0.05 * torch.randn(bn.running_mean.shape, generator=g))
        bn.running_var.copy_(1.0 + 0.2 * torch.rand(bn.running_var.shape, generator=g))
        for p in blk.parameters():
            p.copy_(p.to(torch.bfloat16).float())
    inv_freq = ParakeetEncoderRelPositionalEncoding(cfg).inv_freq.clone()
    return blk.to(device=device, dtype=dtype), inv_freq


def hf_distance_table(blk, inv_freq, max_len: int = MAX_LEN) -> torch.Tensor:
    """The reference's distance table built from transformers' own positional encoding (positions T-1 .. -(T-1) of
    ParakeetEncoderRelPositionalEncoding, reversed to ascending distance), rows d = -(max_len-1) .. max_len+63 at
    row d + max_len - 1, projected by relative_k_proj and rounded to bf16 (float32 result)."""
    from transformers.models.parakeet.modeling_parakeet import ParakeetEncoderRelPositionalEncoding

    hidden = blk.self_attn.relative_k_proj.weight.shape[1]
    enc = ParakeetEncoderRelPositionalEncoding(blk.self_attn.config)
    enc.inv_freq = inv_freq.float()
    T = max_len + 64
    pos = enc(torch.zeros(1, T, hidden)).float()[0]  # (2T - 1, hidden): distance T-1-p at row p
    pos = pos.flip(0)  # distance -(T-1) + r at row r
    first = (T - 1) - (max_len - 1)
    pos = pos[first:first + 2 * max_len - 1 + 64].to(torch.bfloat16).float()
    w = blk.self_attn.relative_k_proj.weight.detach().float().cpu()
    return (pos @ w.t()).to(torch.bfloat16).float()


def oracle_fields(blk, table: torch.Tensor, sparse: bool) -> tuple[dict, list[float]]:
    """The block's tensors as the oracle's layer loop reads them (numpy; bf16 as bits), converted with the oracle's
    own weight quantizer and 2:4 compressor; W2 pruned 2:4 first when sparse."""
    f = {}
    bits = lambda t: bf16_bits(t.detach().float().cpu().to(torch.bfloat16))  # noqa: E731
    fl = lambda t: t.detach().float().cpu().numpy().astype(np.float32)  # noqa: E731
    eps = []
    for name, m in zip(("ff1", "att", "conv", "ff2", "out"), (blk.norm_feed_forward1, blk.norm_self_att,
                                                             blk.norm_conv, blk.norm_feed_forward2, blk.norm_out)):
        f[f"ln_{name}_w"], f[f"ln_{name}_b"] = bits(m.weight), bits(m.bias)
        eps.append(float(m.eps))
    for k, ff in (("ff1", blk.feed_forward1), ("ff2", blk.feed_forward2)):
        f[f"q_{k}_w1"], f[f"q_{k}_s1"] = oracle.quantize_weight_rows(bits(ff.linear1.weight))
        w2 = fl(ff.linear2.weight)
        if sparse:
            w2 = oracle.prune_24(w2)
        f[f"q_{k}_w2"], f[f"q_{k}_s2"] = oracle.quantize_weight_rows(w2)
        if sparse:
            f[f"sp_{k}_w"], f[f"sp_{k}_e"] = oracle.compress_24(f[f"q_{k}_w2"])
        f[f"{k}_b1"], f[f"{k}_b2"] = bits(ff.linear1.bias), bits(ff.linear2.bias)
    at, cv = blk.self_attn, blk.conv
    wqkv = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight])
    f["q_qkv_w"], f["q_qkv_s"] = oracle.quantize_weight_rows(bits(wqkv))
    f["bqkv"] = bits(torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias]))
    f["q_o_w"], f["q_o_s"] = oracle.quantize_weight_rows(bits(at.o_proj.weight))
    f["bo"], f["bu"], f["bv"] = bits(at.o_proj.bias), bits(at.bias_u), bits(at.bias_v)
    f["rk"] = bits(table)
    c = cv.depthwise_conv.in_channels
    w1, b1 = cv.pointwise_conv1.weight[:, :, 0], cv.pointwise_conv1.bias
    f["q_pw1_w"], f["q_pw1_s"] = oracle.quantize_weight_rows(bits(torch.stack([w1[:c], w1[c:]], 1).reshape(2 * c, -1)))
    f["bpw1"] = bits(torch.stack([b1[:c], b1[c:]], 1).reshape(2 * c))
    f["wdw"], f["bdw"] = fl(cv.depthwise_conv.weight[:, 0, :]), fl(cv.depthwise_conv.bias)
    bn = cv.norm
    scale = bn.weight.detach().float() / torch.sqrt(bn.running_var.float() + bn.eps)
    f["bn_scale"] = fl(scale)
    f["bn_shift"] = fl(bn.bias.detach().float() - bn.running_mean.float() * scale)
    f["q_pw2_w"], f["q_pw2_s"] = oracle.quantize_weight_rows(bits(cv.pointwise_conv2.weight[:, :, 0]))
    f["bpw2"] = bits(cv.pointwise_conv2.bias)
    return f, eps


def dequantized_block(blk, fields: dict):
    """A copy of the block (float32) whose linear weights are the oracle's int8 weights times their scales, so that
    it differs from the int8 layer loop only by the activation quantization and bf16 roundings."""
    import copy

    b = copy.deepcopy(blk).float()
    deq = lambda q, s: torch.from_numpy(q.astype(np.float32) * s[:, None])  # noqa: E731
    with torch.no_grad():
        for k, ff in (("ff1", b.feed_forward1), ("ff2", b.feed_forward2)):
            ff.linear1.weight.copy_(deq(fields[f"q_{k}_w1"], fields[f"q_{k}_s1"]))
            w2 = fields[f"q_{k}_w2"]
            if f"sp_{k}_w" in fields:
                w2 = oracle.decompress_24(fields[f"sp_{k}_w"], fields[f"sp_{k}_e"])
            ff.linear2.weight.copy_(deq(w2, fields[f"q_{k}_s2"]))
        at = b.self_attn
        n = at.q_proj.weight.shape[0]
        wqkv = deq(fields["q_qkv_w"], fields["q_qkv_s"])
        at.q_proj.weight.copy_(wqkv[:n])
        at.k_proj.weight.copy_(wqkv[n:2 * n])
        at.v_proj.weight.copy_(wqkv[2 * n:])
        at.o_proj.weight.copy_(deq(fields["q_o_w"], fields["q_o_s"]))
        cv = b.conv
        c = cv.depthwise_conv.in_channels
        w1 = deq(fields["q_pw1_w"], fields["q_pw1_s"]).reshape(c, 2, -1)
        cv.pointwise_conv1.weight.copy_(torch.cat([w1[:, 0], w1[:, 1]])[:, :, None])
        cv.pointwise_conv2.weight.copy_(deq(fields["q_pw2_w"], fields["q_pw2_s"])[:, :, None])
    return b


def hf_block_forward(blk, inv_freq, x: torch.Tensor, lengths: list[int]) -> torch.Tensor:
    """transformers' block on each sequence of packed x (float32, batch of one, no mask), re-packed."""
    from transformers.models.parakeet.modeling_parakeet import ParakeetEncoderRelPositionalEncoding

    enc = ParakeetEncoderRelPositionalEncoding(blk.self_attn.config)
    enc.inv_freq = inv_freq.float()
    outs, s = [], 0
    with torch.no_grad():
        for n in lengths:
            h = x[s:s + n].float()[None]
            pos = enc(h)
            outs.append(blk(h, position_embeddings=pos)[0])
            s += n
    return torch.cat(outs)


def product_layers(device, n_layers: int, seed: int, sparse: bool = False, sparse_w1: bool = False, heads: int = 16):
    """n_layers seeded random-init blocks (1280 wide, feed-forward 5120) converted by the product's EncoderLayers."""
    from kernels.fast_encoder import EncoderLayers

    blocks, inv = [], None
    for i in range(n_layers):
        blk, inv = make_block(1280, heads, 5120, seed=seed + i)
        blocks.append(blk.to(device=device, dtype=torch.bfloat16))
    return EncoderLayers(blocks, inv, sparse=sparse, sparse_w1=sparse_w1)


def oracle_layer_fields(layers) -> list[dict]:
    """The product's converted tensors (weights quantized on the host by the product, pinned against the checker's
    quantizer elsewhere) as the checker's field dicts (numpy; bf16 as bits)."""
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


def oracle_fields_bf16(blk, table: torch.Tensor) -> tuple[dict, list[float]]:
    """The block's tensors as the checker's bf16 layer loop reads them (bf16 bits; GLU rows interleaved)."""
    f, eps = oracle_fields(blk, table, False)
    bits = lambda t: bf16_bits(t.detach().float().cpu().to(torch.bfloat16))  # noqa: E731
    at, cv = blk.self_attn, blk.conv
    for k, ff in (("ff1", blk.feed_forward1), ("ff2", blk.feed_forward2)):
        f[f"{k}_w1"], f[f"{k}_w2"] = bits(ff.linear1.weight), bits(ff.linear2.weight)
    f["wqkv"] = bits(torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]))
    f["wo"] = bits(at.o_proj.weight)
    c = cv.depthwise_conv.in_channels
    w1 = cv.pointwise_conv1.weight[:, :, 0]
    f["wpw1"] = bits(torch.stack([w1[:c], w1[c:]], 1).reshape(2 * c, -1))
    f["wpw2"] = bits(cv.pointwise_conv2.weight[:, :, 0])
    for k in [k for k in f if k.startswith("q_")]:
        del f[k]
    return f, eps
