"""Encoder-side int8 path on gfx950: the weight quantization, tile-config surface and W8A8 / 2:4 linear helpers of
the reference's kernels/fast_encoder.py (quantize_rows 60-63, I8_* / I8_SMALL / SP_CONFIGS 34-57, i8_config 50-57),
and its layer loop (_Layer 66-131, the distance table 155-162, metadata 203-213, layers_forward 215-226) over the HIP
kernels of cohere-inference_amd/csrc (int8 GEMMs, attention, depthwise convolution, LayerNorms).

    q, s = quantize_rows(w_bf16)                         # int8 (N, K), fp32 (N)
    lin = Int8Linear(w_bf16, bias, sparse=True)          # pruned 2:4 before quantization, compressed
    y = lin(xq, xs, epi=EPI_BIAS)                        # bf16 (M, N)

    layers = EncoderLayers(hf_blocks, inv_freq, sparse=True)  # transformers ParakeetEncoderBlock modules, bf16 on GPU
    x = layers(x, lengths)                               # packed frames (sum(lengths), 1280) bf16, in place

    enc = FastEncoder(hf_encoder, int8=True, sparse=True)  # subsampling stem + layers (reference FastEncoder)
    hidden, lengths = enc(features, frames)              # log-mel (B, T, 128) -> packed (sum(lengths), 1280)
"""

from __future__ import annotations

import numpy as np
import torch

from kernels.cuda_ext import EPI_BIAS, EPI_CONV_RELU, EPI_GLU, EPI_RESID, EPI_SILU_Q8, ext
from kernels.sparse import compress_24, pack_24_tiled, prune_24_magnitude

# The reference's int8 config ids (A10 tile choices). They are accepted and checked by the gfx950 GEMMs (each id keeps
# its meaning for the SILU_Q8 output group: configs 4, 6, 8 have 256-column groups) but the tiles are chosen for gfx950
# by shape; results never depend on the id.
I8_CFG, I8_CFG_GROUPED, I8_CFG_FF1, FF_GROUP = 0, 10, 4, 256
I8_SMALL = {"ff1": ((96, 6), (224, 8), (384, 4), (448, 8)),
            "ff2": ((256, 5), (640, 9), (896, 3), (1152, 9)),
            "qkv": ((192, 9), (256, 0), (320, 9)),
            "pw1": ((320, 9), (384, 0), (448, 9)),
            "o": ((640, 9), (896, 0), (1056, 9))}
SP_CONFIGS = ((448, 2), (2048, 0), (1 << 30, 3))
RCP127 = float(np.float32(1.0) / np.float32(127.0))  # fp32(1 / 127): PyTorch's GPU `tensor / 127` multiplies by it


def i8_config(gemm: str, frames: int, default: int) -> int:
    for up_to, cfg in I8_SMALL[gemm]:
        if frames <= up_to:
            return cfg
    return default


def quantize_rows(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric int8 per output channel: s = max(amax|w|, 1e-12) / 127 (fp32), q = clamp(round_half_even(w / s),
    +-127). Load-time weight preparation (reference fast_encoder.py:60-63). The reference runs it on the GPU, where
    PyTorch divides a tensor by a Python scalar as a multiplication by the scalar's fp32 reciprocal; the scale is
    computed that way here on any device (RCP127), so CPU and GPU preparation give the reference's bytes."""
    wf = w.float()
    s = wf.abs().amax(-1).clamp_min(1e-12) * RCP127
    return torch.round(wf / s[:, None]).clamp(-127, 127).to(torch.int8).contiguous(), s.contiguous()


def gemm(a, w, b, epi=EPI_BIAS, out=None, resid=None, alpha=1.0, cfg=None):
    """bf16 out = epilogue(a @ w^T + b) (reference fast_encoder.py:66-71), allocating out when not given."""
    n = w.shape[0] // 2 if epi == EPI_GLU else w.shape[0]
    if out is None:
        out = torch.empty(a.shape[0], n, device=a.device, dtype=a.dtype)
    ext.gemm(a, w, b, out, epi, resid, alpha, GEMM_CFG if cfg is None else cfg)
    return out


def quantize_activations(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (M, K) -> int8 (M, K) + fp32 (M, 1) per-row scales, on the GPU (the reference's ext.quantize_rows)."""
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(x.shape[0], 1, dtype=torch.float32, device=x.device)
    ext.quantize_rows(x, q, s)
    return q, s


class Int8Linear:
    """A W8A8 linear layer: int8 weights per output channel, optionally pruned 2:4 (magnitude, before
    quantization, as the reference prunes before fast_encoder.py:109 quantizes) and stored compressed. tiled (2:4
    only): the GEMM reads the stage-tiled copy of the compressed weight (pack_24_tiled; same results, contiguous
    loads); False reads compress_24's row-major storage."""

    def __init__(self, w: torch.Tensor, bias: torch.Tensor | None, sparse: bool = False, tiled: bool = True):
        if sparse:
            w = prune_24_magnitude(w)
        self.q, self.s = quantize_rows(w)
        self.bias = None if bias is None else bias.to(torch.bfloat16).contiguous()
        self.n, self.k = self.q.shape
        self.sparse = sparse
        self.wt = None
        if sparse:
            self.wc, self.e = compress_24(self.q)
            if tiled:
                self.wt = pack_24_tiled(self.wc, self.e)

    def __call__(self, xq: torch.Tensor, xs: torch.Tensor, epi: int = EPI_BIAS, group: int | None = None,
                 out: torch.Tensor | None = None, resid: torch.Tensor | None = None, alpha: float = 1.0,
                 qs: torch.Tensor | None = None, cfg: int = -1) -> torch.Tensor:
        m = xq.shape[0]
        group = self.k if group is None else group
        if out is None:
            if epi == EPI_SILU_Q8:
                out = torch.empty(m, self.n, dtype=torch.int8, device=xq.device)
            else:
                out = torch.empty(m, self.n // 2 if epi == EPI_GLU else self.n, dtype=torch.bfloat16,
                                  device=xq.device)
        if self.wt is not None:
            ext.gemm_sp_tiled(xq, xs, group, self.wt, self.s, self.bias, out, epi, resid, alpha, qs, cfg)
        elif self.sparse:
            ext.gemm_sp_epi(xq, xs, group, self.wc, self.e, self.s, self.bias, out, epi, resid, alpha, qs, cfg)
        else:
            ext.gemm_i8(xq, xs, group, self.q, self.s, self.bias, out, epi, resid, alpha, qs, cfg)
        return out


# ---- the layer loop --------------------------------------------------------------------------------------------------

# a layer's tensors in the reference's field order (kernels/csrc/encoder_loop.cpp:34-44, fast_encoder.py:121-130)
LAYER_FIELDS = (
    "ln_ff1_w", "ln_ff1_b", "ln_att_w", "ln_att_b", "ln_conv_w", "ln_conv_b", "ln_ff2_w", "ln_ff2_b", "ln_out_w",
    "ln_out_b", "ff1_w1", "ff1_b1", "ff1_w2", "ff1_b2", "ff2_w1", "ff2_b1", "ff2_w2", "ff2_b2", "wqkv", "bqkv", "wo",
    "bo", "bu", "bv", "rk", "wpw1", "bpw1", "wdw", "bdw", "bn_scale", "bn_shift", "wpw2", "bpw2", "q_ff1_w1",
    "q_ff1_s1", "q_ff1_w2", "q_ff1_s2", "q_ff2_w1", "q_ff2_s1", "q_ff2_w2", "q_ff2_s2", "q_qkv_w", "q_qkv_s",
    "q_pw1_w", "q_pw1_s", "q_o_w", "q_o_s", "q_pw2_w", "q_pw2_s", "sp_ff1_w", "sp_ff1_e", "sp_ff2_w", "sp_ff2_e",
    # this build's own: the feed-forwards' first linears in 2:4 form (the reference keeps them dense)
    "sp_ff1_w1", "sp_ff1_e1", "sp_ff2_w1", "sp_ff2_e1")
GEMM_CFG = 8  # the reference's bf16 GEMM config id (its first cfg entry; unused on the int8 path)
MAX_LEN = 512  # encoder frames the distance table covers (reference fast_encoder.py:135)


def relative_table(inv_freq: torch.Tensor, relative_k_proj_weight: torch.Tensor, max_len: int = MAX_LEN):
    """The per-layer table of projected sinusoids of relative distances d = -(max_len-1) .. max_len+63, row
    d + max_len - 1: sin/cos interleaved as ParakeetEncoderRelPositionalEncoding, in the weights' dtype, then
    projected by the layer's relative_k_proj (reference fast_encoder.py:155-162)."""
    dev = relative_k_proj_weight.device
    d = torch.arange(-(max_len - 1), max_len + 64, device=dev, dtype=torch.float)
    freqs = d[:, None] * inv_freq.to(dev, torch.float)
    pos = torch.stack([freqs.sin(), freqs.cos()], -1).reshape(len(d), -1).to(relative_k_proj_weight.dtype)
    return torch.nn.functional.linear(pos, relative_k_proj_weight).contiguous()


class EncoderLayer:
    """One FastConformer block's tensors for the native layer loop (reference fast_encoder.py:66-131). int8: every
    linear W8A8 per output channel; with sparse, the feed-forwards' second linears pruned 2:4 by magnitude (a no-op on
    weights that already are) before quantization and stored compressed, their dense form dropped; sparse_w1 does the
    same to the feed-forwards' first linears (both feed-forward linears 2:4; the reference prunes only the second).
    Without int8 the linears keep their bf16 weights (the reference's INT8=0 layers). tiled: the layer loop reads the
    2:4 weights from stage-tiled copies (pack_24_tiled; the same results)."""

    def __init__(self, blk, rk: torch.Tensor, sparse: bool = False, sparse_w1: bool = False, int8: bool = True,
                 tiled: bool = True):
        if (sparse or sparse_w1) and not int8:
            raise ValueError("EncoderLayer: the 2:4 linears are int8 only")
        t = {}
        self.tiled: dict[str, torch.Tensor] = {}  # stage-tiled copies of the 2:4 weights (pack_24_tiled), by field
        lns = (blk.norm_feed_forward1, blk.norm_self_att, blk.norm_conv, blk.norm_feed_forward2, blk.norm_out)
        self.eps = []
        for name, m in zip(("ff1", "att", "conv", "ff2", "out"), lns):
            t[f"ln_{name}_w"], t[f"ln_{name}_b"] = m.weight.contiguous(), m.bias.contiguous()
            self.eps.append(float(m.eps))
        dev = rk.device
        none_bf = torch.empty(0, device=dev, dtype=rk.dtype)
        none_i8 = torch.empty(0, device=dev, dtype=torch.int8)
        none_f32 = torch.empty(0, device=dev, dtype=torch.float32)
        none_i32 = torch.empty(0, device=dev, dtype=torch.int32)
        at, cv = blk.self_attn, blk.conv
        c = cv.depthwise_conv.in_channels
        pw1, pb1 = cv.pointwise_conv1.weight[:, :, 0], cv.pointwise_conv1.bias
        # the GLU's value and gate rows interleaved (a_0, g_0, a_1, g_1, ...): one epilogue lane sees both
        linears = {"ff1_w1": blk.feed_forward1.linear1.weight, "ff1_w2": blk.feed_forward1.linear2.weight,
                   "ff2_w1": blk.feed_forward2.linear1.weight, "ff2_w2": blk.feed_forward2.linear2.weight,
                   "wqkv": torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]),
                   "wo": at.o_proj.weight, "wpw1": torch.stack([pw1[:c], pw1[c:]], 1).reshape(2 * c, -1),
                   "wpw2": cv.pointwise_conv2.weight[:, :, 0]}
        t["ff1_b1"], t["ff1_b2"] = blk.feed_forward1.linear1.bias.contiguous(), blk.feed_forward1.linear2.bias.contiguous()
        t["ff2_b1"], t["ff2_b2"] = blk.feed_forward2.linear1.bias.contiguous(), blk.feed_forward2.linear2.bias.contiguous()
        t["bqkv"] = torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias]).contiguous()
        t["bo"], t["bu"], t["bv"], t["rk"] = (at.o_proj.bias.contiguous(), at.bias_u.contiguous(),
                                              at.bias_v.contiguous(), rk)
        t["bpw1"] = torch.stack([pb1[:c], pb1[c:]], 1).reshape(2 * c).contiguous()
        t["bpw2"] = cv.pointwise_conv2.bias.contiguous()
        t["wdw"] = cv.depthwise_conv.weight[:, 0, :].float().contiguous()
        t["bdw"] = cv.depthwise_conv.bias.float().contiguous()
        bn = cv.norm
        bn_scale = bn.weight.float() / torch.sqrt(bn.running_var.float() + bn.eps)
        t["bn_scale"] = bn_scale.contiguous()
        t["bn_shift"] = (bn.bias.float() - bn.running_mean.float() * bn_scale).contiguous()
        # quantized names of each linear: (int8 weight, scale) fields and, for the feed-forwards, the 2:4 pair
        qnames = {"ff1_w1": ("q_ff1_w1", "q_ff1_s1", "sp_ff1_w1", "sp_ff1_e1"),
                  "ff1_w2": ("q_ff1_w2", "q_ff1_s2", "sp_ff1_w", "sp_ff1_e"),
                  "ff2_w1": ("q_ff2_w1", "q_ff2_s1", "sp_ff2_w1", "sp_ff2_e1"),
                  "ff2_w2": ("q_ff2_w2", "q_ff2_s2", "sp_ff2_w", "sp_ff2_e"),
                  "wqkv": ("q_qkv_w", "q_qkv_s"), "wo": ("q_o_w", "q_o_s"), "wpw1": ("q_pw1_w", "q_pw1_s"),
                  "wpw2": ("q_pw2_w", "q_pw2_s")}
        for name, w in linears.items():
            q = qnames[name]
            for k, empty in zip(q, (none_i8, none_f32, none_i8, none_i32)):
                t[k] = empty
            if not int8:
                t[name] = w.contiguous()
                continue
            t[name] = none_bf
            pruned = len(q) == 4 and (sparse if name.endswith("w2") else sparse_w1)
            t[q[0]], t[q[1]] = quantize_rows(prune_24_magnitude(w) if pruned else w)
            if pruned:
                t[q[2]], t[q[3]] = compress_24(t[q[0]])
                t[q[0]] = none_i8
                if tiled:
                    self.tiled[q[2]] = pack_24_tiled(t[q[2]], t[q[3]])
        self.tensors = t
        self.int8 = int8
        self.heads, self.head_dim = at.bias_u.shape

    def fields(self) -> list[torch.Tensor]:
        """This layer's tensors in the reference's field order. A 2:4 linear with a stage-tiled copy is passed as that
        copy in the kept-values field and an empty selectors field (the layer loop then runs gemm_sp_tiled)."""
        empty = torch.empty(0, device=self.tensors["rk"].device, dtype=torch.int32)
        sel_of = {"sp_ff1_w": "sp_ff1_e", "sp_ff2_w": "sp_ff2_e", "sp_ff1_w1": "sp_ff1_e1", "sp_ff2_w1": "sp_ff2_e1"}
        dropped = {sel_of[k] for k in self.tiled}
        return [self.tiled.get(k, empty if k in dropped else self.tensors[k]) for k in LAYER_FIELDS]


def metadata(lengths: list[int], device) -> dict:
    """Index tables of a packed batch (reference fast_encoder.py:203-213 defines the format):

    - tiles: int32 (n_tiles, 4), one entry per block of 64 queries of one piece: (first row of the piece, its length,
      first query of the block within the piece, 0);
    - lo, hi: int32 (rows,), each packed row's piece as the half-open row range the depthwise convolution may read;
    - max_len: the longest piece.

    Built with whole-tensor index arithmetic on the host, then copied to the device."""
    n = torch.tensor(list(lengths), dtype=torch.int64)
    end = n.cumsum(0)
    first = end - n
    blocks = (n + 63) // 64
    piece = torch.repeat_interleave(torch.arange(len(n)), blocks)
    block_in_piece = torch.arange(int(blocks.sum())) - torch.repeat_interleave(blocks.cumsum(0) - blocks, blocks)
    tiles = torch.stack([first[piece], n[piece], 64 * block_in_piece, torch.zeros_like(piece)], 1)
    return {"tiles": tiles.to(torch.int32).to(device), "lo": torch.repeat_interleave(first, n).to(torch.int32).to(device),
            "hi": torch.repeat_interleave(end, n).to(torch.int32).to(device), "max_len": int(n.max()) if len(n) else 0}


class EncoderLayers:
    """The layers of a FastConformer encoder on packed frames (reference FastEncoder.layers_forward,
    fast_encoder.py:215-226): blocks are transformers ParakeetEncoderBlock modules (1280 wide, 8 or 16 heads) whose
    weights are converted once; a call runs every layer through ext.encoder_layers, one native launch loop. sparse /
    sparse_w1 / int8 as EncoderLayer."""

    def __init__(self, blocks, inv_freq: torch.Tensor, sparse: bool = False, max_len: int = MAX_LEN,
                 sparse_w1: bool = False, int8: bool = True):
        with torch.no_grad():
            self.layers = [EncoderLayer(b, relative_table(inv_freq, b.self_attn.relative_k_proj.weight, max_len),
                                        sparse, sparse_w1, int8) for b in blocks]
        self.int8 = int8
        self.layer_tensors = [ly.fields() for ly in self.layers]
        self.layer_eps = [e for ly in self.layers for e in ly.eps]
        self.max_len, self.rel_off = max_len, max_len - 1
        self.scale = self.layers[0].head_dim ** -0.5
        self.sparse = sparse

    def configs(self, n: int) -> list[int]:
        return [GEMM_CFG, i8_config("qkv", n, I8_CFG), i8_config("ff2", n, I8_CFG_GROUPED),
                i8_config("ff1", n, I8_CFG_FF1), FF_GROUP, i8_config("pw1", n, I8_CFG), i8_config("o", n, I8_CFG),
                next(c for up_to, c in SP_CONFIGS if n <= up_to)]

    @torch.no_grad()
    def __call__(self, x: torch.Tensor, lengths: list[int], meta: dict | None = None) -> torch.Tensor:
        meta = metadata(lengths, x.device) if meta is None else meta
        if meta["max_len"] > self.max_len:
            raise RuntimeError(f"encoder_layers: sequence of {meta['max_len']} frames exceeds {self.max_len}")
        ext.encoder_layers(x, self.layer_tensors, self.layer_eps, meta["tiles"], meta["lo"], meta["hi"], self.rel_off,
                           meta["max_len"], self.scale, self.int8, self.configs(x.shape[0]))
        return x


def _halve(t: int) -> int:
    """Length after a 3-tap, stride-2 convolution padded by one on each side."""
    return (t + 1) // 2


class SubsamplingStem:
    """The encoder's 8x time-subsampling front (transformers ParakeetEncoderSubsamplingConv2D: a 3x3 convolution,
    then two depthwise + pointwise pairs, ReLU after each pointwise, then a linear to d_model), prepared once for this
    library's kernels (reference fast_encoder.py:165-200 describes the same operation sequence):

    - sub_conv0_dw fuses the first convolution and the first depthwise one; both take fp32 taps flattened to (C, 9)
      and fp32 biases;
    - each pointwise convolution is a bf16 GEMM over rows of (frame, frequency) with channels innermost, its bias
      added in fp32 before the one rounding, then ReLU (EPI_CONV_RELU);
    - the final linear reads a frame's (frequency, channel) row; the module flattens (channel, frequency), so its
      weight columns are permuted here once.

    Every piece is convolved on its own frames only: no padding rows enter the packed output."""

    def __init__(self, sub):
        convs = [m for m in sub.layers if isinstance(m, torch.nn.Conv2d)]
        if len(convs) != 5 or convs[1].groups == 1 or convs[2].kernel_size != (1, 1):
            raise ValueError("SubsamplingStem: expected conv, (depthwise, pointwise) x 2")
        full, dw1, pw1, dw2, pw2 = convs
        taps = lambda c: c.weight.detach().float().flatten(1).contiguous()  # noqa: E731
        vec = lambda t: t.detach().float().contiguous()  # noqa: E731
        self.first = (taps(full), vec(full.bias), taps(dw1), vec(dw1.bias))
        self.second_dw = (taps(dw2), vec(dw2.bias))
        self.pointwise = [(c.weight.detach().flatten(1).contiguous(), c.bias.detach().contiguous()) for c in (pw1, pw2)]
        self.c = pw2.out_channels
        self.freq = sub.linear.in_features // self.c
        lin_w = sub.linear.weight.detach().unflatten(1, (self.c, self.freq)).transpose(1, 2).flatten(1)
        self.linear = (lin_w.contiguous(), sub.linear.bias.detach().contiguous())

    @staticmethod
    def lengths(frames: list[int]) -> tuple[list[int], list[int]]:
        """Per piece, its length after the fused first stage (stride 4) and after the whole stem (stride 8)."""
        quarter = [_halve(_halve(f)) for f in frames]
        return quarter, [_halve(t) for t in quarter]

    @staticmethod
    def _row_index(counts: list[int], dev) -> torch.Tensor:
        """int32 (sum(counts), 2): (piece, row within the piece) for every output row of a stage."""
        c = torch.tensor(counts, dtype=torch.int64)
        piece = torch.repeat_interleave(torch.arange(len(c)), c)
        within = torch.arange(int(c.sum())) - torch.repeat_interleave(c.cumsum(0) - c, c)
        return torch.stack([piece, within], 1).to(torch.int32).to(dev, non_blocking=True)

    @torch.no_grad()
    def __call__(self, features: torch.Tensor, frames: list[int]) -> tuple[torch.Tensor, list[int]]:
        dev, dt, C = features.device, features.dtype, self.c
        quarter, eighth = self.lengths(frames)
        as_dev = lambda v: torch.tensor(v, dtype=torch.int32).to(dev, non_blocking=True)  # noqa: E731
        # stage 1: (rows at stride 4, 32 frequencies, C) from the log-mel frames of each piece
        h = torch.empty(sum(quarter), 32, C, device=dev, dtype=dt)
        ext.sub_conv0_dw(features.contiguous(), as_dev(frames), self._row_index(quarter, dev), *self.first, h)
        h = gemm(h.view(-1, C), *self.pointwise[0], EPI_CONV_RELU).view(-1, 32, C)
        # stage 2: depthwise at stride 2 in time and frequency, within each piece's rows of stage 1
        first_row = [0]
        for t in quarter[:-1]:
            first_row.append(first_row[-1] + t)
        g = torch.empty(sum(eighth), 16, C, device=dev, dtype=dt)
        ext.sub_dw(h, as_dev(first_row), as_dev(quarter), self._row_index(eighth, dev), *self.second_dw, g)
        g = gemm(g.view(-1, C), *self.pointwise[1], EPI_CONV_RELU)
        return gemm(g.view(-1, self.freq * C), *self.linear, EPI_BIAS), eighth


def load_pruned_feed_forwards(encoder, path: str) -> None:
    """Put a file of 2:4-pruned feed-forward second-layer weights into the module (the format kernels/sparse.py
    writes, reference sparse.py:86-120: {"<layer>.feed_forward<1|2>": weight}). Every layer's two feed-forwards must
    be present with the module's shapes; nothing is changed otherwise."""
    state = torch.load(path, weights_only=True)
    targets = {f"{i}.{ff}": getattr(blk, ff).linear2.weight
               for i, blk in enumerate(encoder.layers) for ff in ("feed_forward1", "feed_forward2")}
    if set(state) != set(targets):
        raise ValueError(f"FastEncoder: {path} must hold exactly {len(targets)} entries <layer>.feed_forward<1|2>")
    bad = [k for k, w in state.items() if w.shape != targets[k].shape]
    if bad:
        raise ValueError(f"FastEncoder: wrong shapes for {bad}")
    with torch.no_grad():
        for k, w in state.items():
            targets[k].copy_(w)


class FastEncoder:
    """A transformers ParakeetEncoder (1280 wide, bf16 on the GPU) over packed pieces: SubsamplingStem, then the
    native layer loop (EncoderLayers), W8A8 with int8 or bf16 without (the reference's FastEncoder surface,
    fast_encoder.py:133-232: the constructor arguments, subsample / metadata / layers_forward / __call__).

    sparse needs int8: a path to a pruned-weights file (load_pruned_feed_forwards), or True to prune the
    feed-forwards' second linears 2:4 by magnitude at conversion; None / False keeps them dense. sparse_w1 prunes the
    feed-forwards' first linears as well (not in the reference)."""

    MAX_LEN = MAX_LEN

    def __init__(self, encoder, int8: bool = False, sparse: str | bool | None = None, sparse_w1: bool = False):
        wants_24 = sparse_w1 or (sparse is not None and sparse is not False)
        if wants_24 and not int8:
            raise ValueError("FastEncoder: the 2:4 feed-forwards need int8")
        if encoder.config.hidden_size != 1280 or getattr(encoder.config, "scale_input", False):
            raise ValueError("FastEncoder: 1280-wide encoders without input scaling only")
        if isinstance(sparse, str):
            load_pruned_feed_forwards(encoder, sparse)
        self.encoder, self.int8 = encoder, int8
        self.sparse = sparse is not None and sparse is not False
        with torch.no_grad():
            self.stem = SubsamplingStem(encoder.subsampling)
        self.layers = EncoderLayers(encoder.layers, encoder.encode_positions.inv_freq, sparse=self.sparse,
                                    max_len=self.MAX_LEN, sparse_w1=sparse_w1, int8=int8)

    def subsample(self, features: torch.Tensor, frames: list[int]) -> tuple[torch.Tensor, list[int]]:
        """features: padded log-mel (B, T, 128); piece b uses its first frames[b] frames. Returns the packed stem
        output (sum of lengths, 1280) and the per-piece lengths."""
        return self.stem(features, frames)

    def metadata(self, lengths: list[int], device) -> dict:
        return metadata(lengths, device)

    def layers_forward(self, x: torch.Tensor, meta: dict) -> torch.Tensor:
        """All layers over the packed rows x in place; returns x."""
        return self.layers(x, None, meta)

    def __call__(self, features: torch.Tensor, frames: list[int]) -> tuple[torch.Tensor, list[int]]:
        x, lengths = self.subsample(features, frames)
        return self.layers_forward(x, metadata(lengths, x.device)), lengths


__all__ = ["EncoderLayer", "FastEncoder", "SubsamplingStem", "load_pruned_feed_forwards", "gemm", "EncoderLayers", "LAYER_FIELDS", "metadata", "relative_table", "EPI_BIAS", "EPI_GLU", "EPI_RESID", "EPI_SILU_Q8", "I8_CFG", "I8_CFG_GROUPED", "I8_CFG_FF1", "FF_GROUP",
           "I8_SMALL", "SP_CONFIGS", "Int8Linear", "i8_config", "quantize_activations", "quantize_rows"]
