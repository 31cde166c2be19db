"""Greedy decoding with continuous batching on gfx950 (the call surface of the reference's kernels/stream_decoder.py):
the int8-weight (W8A16) layout and 64-row chunked projection calls (prepare_w8 38-48, W8_CONFIGS 30-35, _w8 148-158)
over the skinny HIP GEMMs of csrc/dec_w8.hip, and StreamDecoder (73-276): per-slot state and KV caches, one step =
embedding, 8 x (self-attention over the slot's int8 cache, cross-attention, feed-forward), head and greedy pick, held
as a fixed list of launches over preallocated buffers and captured into one HIP graph per bucket of row counts
(csrc/decoder_ops.hip for the non-GEMM kernels).

    wq = prepare_w8(w_bf16)                          # (uint8 (N, K), fp32 (N))
    y = w8_linear(x, wq, bias, relu=False, ws=ws, counters=counters)
    y = bf16_linear(x, w_bf16, bias)                 # o / cross-q / cross-o (the reference's Triton `linear`)
    dec = StreamDecoder(model, slots=64, int8=True)  # model: transformers CohereAsrForConditionalGeneration
    dec.fill_cross(hidden, lengths, slots); dec.admit(slots, prompts, lengths); b = dec.set_active(slots)
    dec.step(b)                                      # one graph replay
"""

from __future__ import annotations

import torch

from kernels.cuda_ext import DEC_EP_NONE, DEC_EP_RELU, DEC_EP_RESID, ext
from kernels.fast_encoder import RCP127

# (N, K) -> {rows up to: (columns per CTA, K splits)}: the reference's A10 table, accepted for compatibility. The gfx950
# kernel checks these like the reference does and then chooses its own tiling (results never depend on it).
W8_CONFIGS = {
    (1024, 4096): {1: (64, 4), 8: (16, 4), 16: (16, 4), 24: (16, 2), 32: (32, 4), 48: (64, 4), 64: (64, 4)},
    (3072, 1024): {1: (32, 1), 8: (32, 1), 16: (32, 1), 24: (32, 1), 32: (32, 1), 48: (64, 1), 64: (64, 1)},
    (4096, 1024): {1: (32, 1), 8: (32, 1), 16: (32, 1), 24: (64, 1), 32: (64, 1), 48: (64, 1), 64: (64, 1)},
    (16384, 1024): {1: (16, 1), 8: (16, 1), 16: (32, 1), 24: (64, 1), 32: (64, 1), 48: (64, 1), 64: (64, 1)},
}
DEFAULT_CONFIG = (64, 4)

# physical byte j of every 16 along K holds logical K W8_PERM[j] (the reference's layout, stream_decoder.py:38)
W8_PERM = (0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15)


def prepare_w8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (N, K) -> (uint8 (N, K) = int8 + 128 with K permuted within every 16 by W8_PERM, fp32 per-channel
    scales). Quantization: s = max(amax|w|, 1e-12) / 127, q = clamp(round_half_even(w / s), +-127), the scale's
    division by 127 as the reference's GPU execution of it: a multiplication by fp32(1 / 127) (RCP127, see
    kernels.fast_encoder.quantize_rows), on any device."""
    n, k = w.shape
    assert k % 16 == 0
    wf = w.float()
    s = wf.abs().amax(1).clamp_min(1e-12) * RCP127
    q = (torch.round(wf / s[:, None]).clamp(-127, 127) + 128).to(torch.uint8)
    perm = torch.tensor(W8_PERM, device=w.device)
    return q.reshape(n, k // 16, 16).index_select(2, perm).reshape(n, k).contiguous(), s.contiguous()


def unprepare_w8(wq: torch.Tensor) -> torch.Tensor:
    """The int8 (N, K) weights in natural K order of a prepare_w8 layout."""
    n, k = wq.shape
    inv = torch.empty(16, dtype=torch.long, device=wq.device)
    inv[torch.tensor(W8_PERM, device=wq.device)] = torch.arange(16, device=wq.device)
    return (wq.reshape(n, k // 16, 16).index_select(2, inv).reshape(n, k).to(torch.int16) - 128).to(torch.int8)


def w8_config(n: int, k: int, rows: int) -> tuple[int, int]:
    configs = W8_CONFIGS.get((n, k))
    if configs is None:
        return DEFAULT_CONFIG if k % (128 * DEFAULT_CONFIG[1]) == 0 and n % 64 == 0 else (16, 1)
    return configs[next(c for c in sorted(configs) if c >= rows)]


def w8_linear(x: torch.Tensor, wq: tuple[torch.Tensor, torch.Tensor], bias: torch.Tensor | None, relu: bool = False,
              ws: torch.Tensor | None = None, counters: torch.Tensor | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """x @ dequant(wq)^T + bias through dec_w8_linear, 64 rows at a time (the reference's StreamDecoder._w8)."""
    (w, scale), (n, k) = wq, wq[0].shape
    y = out if out is not None else torch.empty(x.shape[0], n, device=x.device, dtype=x.dtype)
    for r in range(0, x.shape[0], 64):
        m = min(64, x.shape[0] - r)
        bn, splits = w8_config(n, k, m)
        if ws is None or counters is None:
            splits = 1
        ext.dec_w8_linear(x[r:r + m], w, scale, bias, y[r:r + m], relu, bn, splits, ws, counters)
    return y


def bf16_linear(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, relu: bool = False,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """x @ w^T + b (relu) with bf16 weights, 64 rows at a time (the reference's `linear`, stream_decoder.py:23-27)."""
    y = out if out is not None else torch.empty(x.shape[0], w.shape[0], device=x.device, dtype=x.dtype)
    for r in range(0, x.shape[0], 64):
        m = min(64, x.shape[0] - r)
        ext.linear_bf16(x[r:r + m], w, b, y[r:r + m], relu)
    return y


# ---- the decoder and its captured step ------------------------------------------------------------------------------

class _Projection:
    """One decoder linear bound to its skinny kernel: int8 weights in prepare_w8's layout through dec_w8_linear, or
    bf16 weights through linear_bf16. A call writes y (rows, N) from x (rows, K), 64 rows per launch."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, int8: bool):
        self.n, self.k = weight.shape
        self.bias = None if bias is None else bias.contiguous()
        if int8:
            self.weight, self.scale = prepare_w8(weight)
        else:
            self.weight, self.scale = weight.contiguous(), None

    @property
    def nbytes(self) -> int:
        return self.weight.numel() * self.weight.element_size()

    def __call__(self, x: torch.Tensor, y: torch.Tensor, relu: bool = False) -> None:
        for r in range(0, x.shape[0], 64):
            xr, yr = x[r:r + 64], y[r:r + 64]
            if self.scale is None:
                ext.linear_bf16(xr, self.weight, self.bias, yr, relu)
            else:
                bn, _ = w8_config(self.n, self.k, xr.shape[0])
                ext.dec_w8_linear(xr, self.weight, self.scale, self.bias, yr, relu, bn, 1, None, None)

    def fused(self, x: torch.Tensor, y: torch.Tensor, epilogue: int = DEC_EP_NONE, ln=None) -> None:
        """The projection with its neighbouring residual LayerNorm folded in (ext.dec_linear_fused): ln normalises
        x's rows first; DEC_EP_RESID adds the result into y (the residual stream) in place."""
        for r in range(0, x.shape[0], 64):
            ext.dec_linear_fused(x[r:r + 64], self.weight, self.scale, self.bias, y[r:r + 64], epilogue, ln)


class _Block:
    """One decoder layer: its three LayerNorms (weight, bias, eps) and six projections. With int8, the
    self-attention's fused q/k/v and the feed-forward's two linears hold int8 weights; the attention outputs and the
    cross-attention query stay bf16 (the reference's int8 layout, stream_decoder.py:106-113)."""

    def __init__(self, layer, int8: bool):
        sa, ca, mlp = layer.self_attn, layer.encoder_attn, layer.mlp
        self.norms = tuple((m.weight, m.bias, float(m.eps)) for m in
                           (layer.input_layernorm, layer.post_attention_layernorm, layer.final_layernorm))
        self.qkv = _Projection(torch.cat([sa.q_proj.weight, sa.k_proj.weight, sa.v_proj.weight]),
                               torch.cat([sa.q_proj.bias, sa.k_proj.bias, sa.v_proj.bias]), int8)
        self.o = _Projection(sa.o_proj.weight, sa.o_proj.bias, False)
        self.cq = _Projection(ca.q_proj.weight, ca.q_proj.bias, False)
        self.co = _Projection(ca.o_proj.weight, ca.o_proj.bias, False)
        self.fc1 = _Projection(mlp.fc1.weight, mlp.fc1.bias, int8)
        self.fc2 = _Projection(mlp.fc2.weight, mlp.fc2.bias, int8)

    def projections(self):
        return (self.qkv, self.o, self.cq, self.co, self.fc1, self.fc2)


class StreamDecoder:
    """Greedy decoding with continuous batching (reference kernels/stream_decoder.py, same constructor, attributes
    and methods). State lives in `slots` slots plus one dummy slot that padding rows point at; a step feeds one token
    per active row. The step is a fixed list of launches over buffers allocated once (no allocation inside a step),
    built per bucket of row counts and captured into one HIP graph per bucket, so a step is one graph replay whatever
    the rows' positions and audio lengths. The model is a transformers CohereAsrForConditionalGeneration (or anything
    with its decoder attributes); `frames` may be given instead of asking the encoder for its subsampled length."""

    BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96, 112, 128)

    def __init__(self, model, slots: int = 128, max_new_tokens: int = 448, max_prompt: int = 16,
                 max_audio_s: float = 36.0, buckets=None, int8: bool = False, frames: int | None = None,
                 capture: bool = True, fused: bool | None = None, chunk: int = 4):
        dec, cfg = model.model.decoder, model.config
        self.model, self.int8 = model, int8
        self.buckets = tuple(sorted(b for b in (buckets or self.BUCKETS) if b <= slots))
        if not self.buckets:
            raise ValueError("StreamDecoder: no bucket fits the slots")
        self.h, self.width = cfg.num_attention_heads, cfg.hidden_size
        self.d = getattr(cfg, "head_dim", None) or self.width // self.h
        if self.d != 128:
            raise ValueError("StreamDecoder: the decoder kernels take head size 128")
        self.eos, self.pad, self.scale = cfg.eos_token_id, cfg.pad_token_id, self.d ** -0.5
        self.slots, self.dummy = slots, slots
        self.max_new_tokens, self.max_prompt = max_new_tokens, max_prompt
        self.seq = max_prompt + max_new_tokens + 1  # cache positions per slot
        if frames is None:
            frames = int(model.model.encoder._get_subsampling_output_length(
                torch.tensor([int(max_audio_s * 100) + 1])).item())
        self.frames = frames
        # residual LayerNorms folded into the projections (ext.dec_linear_fused) where its prologue takes the width;
        # fused=False keeps the reference's separate dec_add_ln launches (the same bits)
        can_fuse = 512 <= self.width <= 1024 and self.width % 64 == 0
        if fused and not can_fuse:
            raise ValueError(f"StreamDecoder: fused projections take widths 512-1024 (got {self.width})")
        self.fused = can_fuse if fused is None else bool(fused)

        # weights
        self.embed, self.pos_table = dec.embed_tokens.weight, dec.pos_emb.weight
        self.device = dev = self.embed.device
        self.emb_ln = (dec.embedding_layernorm.weight, dec.embedding_layernorm.bias, float(dec.embedding_layernorm.eps))
        self.final_ln = (dec.norm.weight, dec.norm.bias, float(dec.norm.eps))
        self.blocks = [_Block(layer, int8) for layer in dec.layers]
        self.layers = self.blocks
        self.head = _Projection(model.proj_out.weight, model.proj_out.bias, int8)
        self.proj = (dec.proj.weight.contiguous(), None if dec.proj.bias is None else dec.proj.bias.contiguous())
        kv_w = [w for layer in dec.layers for w in (layer.encoder_attn.k_proj.weight, layer.encoder_attn.v_proj.weight)]
        kv_b = [b for layer in dec.layers for b in (layer.encoder_attn.k_proj.bias, layer.encoder_attn.v_proj.bias)]
        self.cross_w, self.cross_b = torch.cat(kv_w).contiguous(), torch.cat(kv_b).contiguous()

        # caches: (layer, slot, head, position, 128), int8 with one fp32 scale per 128-vector when int8
        L, S1 = len(self.blocks), slots + 1
        kv_dtype = torch.int8 if int8 else self.embed.dtype

        def cache(t):
            return torch.zeros(L, S1, self.h, t, self.d, device=dev, dtype=kv_dtype)

        def scales(t):
            return torch.ones(L, S1, self.h, t, device=dev, dtype=torch.float32) if int8 else None

        self.self_k, self.self_v, self.self_ks, self.self_vs = cache(self.seq), cache(self.seq), scales(self.seq), \
            scales(self.seq)
        self.cross_k, self.cross_v, self.cross_ks, self.cross_vs = cache(frames), cache(frames), scales(frames), \
            scales(frames)

        # slot state (row `slots` is the dummy, never advanced)
        i32, i64 = dict(device=dev, dtype=torch.int32), dict(device=dev, dtype=torch.long)
        self.tok = torch.full((S1,), self.pad, **i64)
        self.pos = torch.zeros(S1, **i32)
        self.plen = torch.ones(S1, **i32)
        self.limit = torch.zeros(S1, **i32)
        self.cross_len = torch.ones(S1, **i32)
        self.finished = torch.ones(S1, device=dev, dtype=torch.uint8)
        self.forced = torch.full((S1, max_prompt), self.pad, **i64)
        self.out = torch.full((S1, self.seq + 1), self.pad, **i64)
        self.flags = torch.ones(S1, dtype=torch.uint8).pin_memory()  # `finished`, copied out by every step

        # step buffers, sized for the largest bucket
        bm, bf = self.buckets[-1], dict(device=dev, dtype=self.embed.dtype)
        self.active = torch.full((bm,), self.dummy, **i32)
        self.x, self.hn, self.att = (torch.zeros(bm, self.width, **bf) for _ in range(3))
        self.qkv_out = torch.zeros(bm, 3 * self.width, **bf)
        self.q_out = torch.zeros(bm, self.width, **bf)
        self.proj_out = torch.zeros(bm, self.width, **bf)
        self.ffn_out = torch.zeros(bm, self.blocks[0].fc1.n, **bf)
        self.logits = torch.zeros(bm, self.head.n, **bf)
        self.part = torch.empty(max(b * self.h * self._splits(b) * (self.d + 2) for b in self.buckets), device=dev,
                                dtype=torch.float32)

        self.stream = torch.cuda.Stream(device=dev)
        self._embed_stale, self._embed_rows = True, 0
        self.programs = {b: self._program(b) for b in self.buckets}
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        # `chunk` consecutive steps recorded into one graph per bucket as well (step(bucket, chunk)): a graph boundary
        # costs a few microseconds of idle GPU, which one replay per step pays every step
        self.chunk = max(1, int(chunk))
        self.chunk_graphs: dict[int, torch.cuda.CUDAGraph] = {}
        if capture:
            self._capture()

    @staticmethod
    def _splits(b: int) -> int:
        """Workgroups per (row, head) of the cross-attention: one for every bucket. The reference splits the frames
        over 4 for one or two rows (stream_decoder.py:140-144); a split changes the fp32 combine order, so a piece's
        tokens would then depend on how many rows it shares a step with. One split keeps every row's result
        independent of the batch (at 375 frames a workgroup's 64 key groups cover the frames in one pass anyway)."""
        return 1

    # ---- the step as a list of launches ------------------------------------------------------------------------

    def _attention(self, i: int, self_attn: bool, act, q, splits: int, out):
        if self_attn:
            k, v, ks, vs, n = self.self_k[i], self.self_v[i], self.self_ks, self.self_vs, self.pos
        else:
            k, v, ks, vs, n = self.cross_k[i], self.cross_v[i], self.cross_ks, self.cross_vs, self.cross_len
        if self.int8:
            ks, vs = ks[i], vs[i]
            return lambda: ext.dec_attention_q8(self_attn, act, q, k, v, ks, vs, n, self.scale, splits, self.part,
                                                out)
        return lambda: ext.dec_attention(self_attn, act, q, k, v, n, self.scale, splits, self.part, out)

    def _program(self, b: int) -> list:
        """The step for the first b active rows (reference stream_decoder.py:176-199): embedding + first LayerNorm,
        per layer self-attention (qkv, attention over the slot's cache, o, residual + LayerNorm), cross-attention (q,
        attention over the slot's frames, o, residual + LayerNorm) and feed-forward (fc1 + ReLU, fc2, residual + the
        next LayerNorm), then the head, the greedy pick and the end flags' copy to the host."""
        act, x, hn, att = self.active[:b], self.x[:b], self.hn[:b], self.att[:b]
        qkv, q, proj, ffn, logits = (t[:b] for t in (self.qkv_out, self.q_out, self.proj_out, self.ffn_out,
                                                     self.logits))
        if self.fused:
            # the residual adds ride on o / cross-o / fc2's epilogues and the LayerNorms on the next projection's
            # prologue (8 launches a layer instead of 11); the pick computes the next step's embedding of its row and
            # writes the end flags to the host itself. The same bits as the unfused step. The step's own embedding
            # comes from the previous step's pick, or from step() when the rows changed.
            ops = []
            for i, blk in enumerate(self.blocks):
                first = i == 0
                ops += [(lambda blk=blk: blk.qkv.fused(hn, qkv)) if first else
                        (lambda blk=blk: blk.qkv.fused(x, qkv, ln=blk.norms[0])),
                        self._attention(i, True, act, qkv, 1, att),
                        lambda blk=blk: blk.o.fused(att, x, DEC_EP_RESID),
                        lambda blk=blk: blk.cq.fused(x, q, ln=blk.norms[1]),
                        self._attention(i, False, act, q, self._splits(b), att),
                        lambda blk=blk: blk.co.fused(att, x, DEC_EP_RESID),
                        lambda blk=blk: blk.fc1.fused(x, ffn, DEC_EP_RELU, ln=blk.norms[2]),
                        lambda blk=blk: blk.fc2.fused(ffn, x, DEC_EP_RESID)]
            ops += [lambda: self.head.fused(x, logits, ln=self.final_ln),
                    lambda: ext.dec_pick_embed(logits, act, self.dummy, self.tok, self.pos, self.finished, self.forced,
                                               self.plen, self.limit, self.out, self.pad, self.eos, self.embed,
                                               self.pos_table, *self.emb_ln, *self.blocks[0].norms[0], x, hn,
                                               self.flags)]
            return ops
        ops = [lambda: self._embed(b)]
        for i, blk in enumerate(self.blocks):
            after_ffn = self.blocks[i + 1].norms[0] if i + 1 < len(self.blocks) else self.final_ln
            ops += [lambda blk=blk: blk.qkv(hn, qkv),
                    self._attention(i, True, act, qkv, 1, att),
                    lambda blk=blk: blk.o(att, proj),
                    lambda blk=blk: ext.dec_add_ln(x, proj, *blk.norms[1], hn),
                    lambda blk=blk: blk.cq(hn, q),
                    self._attention(i, False, act, q, self._splits(b), att),
                    lambda blk=blk: blk.co(att, proj),
                    lambda blk=blk: ext.dec_add_ln(x, proj, *blk.norms[2], hn),
                    lambda blk=blk: blk.fc1(hn, ffn, relu=True),
                    lambda blk=blk: blk.fc2(ffn, proj),
                    lambda ln=after_ffn: ext.dec_add_ln(x, proj, *ln, hn)]
        ops += [lambda: self.head(hn, logits),
                lambda: ext.dec_pick(logits, act, self.dummy, self.tok, self.pos, self.finished, self.forced,
                                     self.plen, self.limit, self.out, self.pad, self.eos),
                lambda: self.flags.copy_(self.finished, non_blocking=True)]
        return ops

    def _embed(self, b: int) -> None:
        """The embedding and first LayerNorm of the first b active rows (x, hn), on the current stream."""
        ext.dec_embed(self.active[:b], self.tok, self.pos, self.embed, self.pos_table, *self.emb_ln,
                      *self.blocks[0].norms[0], self.x[:b], self.hn[:b])

    def _run(self, b: int) -> None:
        if self.fused:
            self._embed(b)
        for op in self.programs[b]:
            op()

    @torch.no_grad()
    def _capture(self) -> None:
        """One graph per bucket, on the decoder stream; each program runs once eagerly first (every launch
        validated), then is recorded. The state is reset afterwards (the runs advanced the dummy rows only)."""
        with torch.cuda.stream(self.stream):
            for b in reversed(self.buckets):
                self._run(b)
                self.stream.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.stream):
                    for op in self.programs[b]:  # the program only: step() adds the embedding when the rows change
                        op()
                self.graphs[b] = g
                if self.chunk > 1:
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g, stream=self.stream):
                        for _ in range(self.chunk):
                            for op in self.programs[b]:
                                op()
                    self.chunk_graphs[b] = g
        self.reset()
        self.stream.synchronize()

    # ---- host side -------------------------------------------------------------------------------------------------

    def reset(self) -> None:
        """Every slot free (on the decoder stream)."""
        self._embed_stale = True
        with torch.cuda.stream(self.stream):
            self.finished.fill_(1)
            self.pos.zero_()
            self.cross_len.fill_(1)
            self.active.fill_(self.dummy)

    def bucket(self, rows: int) -> int:
        """The smallest bucket of at least `rows` rows."""
        for b in self.buckets:
            if b >= rows:
                return b
        raise ValueError(f"StreamDecoder: {rows} rows exceed the largest bucket {self.buckets[-1]}")

    def _to_device(self, host: torch.Tensor) -> torch.Tensor:
        return host.pin_memory().to(self.device, non_blocking=True)

    def fill_cross(self, hidden: torch.Tensor, lengths: list[int], slots: list[int], projected: bool = False) -> None:
        """Cross-attention keys and values of packed encoder frames hidden (sum(lengths), width) into the given slots,
        on the current stream: the decoder's input projection (unless projected), every layer's key and value
        projections in one bf16 GEMM, then the scatter into the slots' caches (quantized per 128-vector with int8)."""
        from kernels.cuda_ext import EPI_BIAS

        rows = hidden.shape[0]
        if rows == 0:
            return
        mem = hidden.contiguous()
        if not projected:
            out = torch.empty(rows, self.proj[0].shape[0], device=hidden.device, dtype=hidden.dtype)
            ext.gemm(mem, self.proj[0], self.proj[1], out, EPI_BIAS, None, 1.0, 8)
            mem = out
        kv = torch.empty(rows, self.cross_w.shape[0], device=hidden.device, dtype=hidden.dtype)
        ext.gemm(mem, self.cross_w, self.cross_b, kv, EPI_BIAS, None, 1.0, 8)
        where = torch.empty(2, rows, dtype=torch.int32)
        where[0] = torch.repeat_interleave(torch.tensor(slots, dtype=torch.int32), torch.tensor(lengths))
        where[1] = torch.cat([torch.arange(n, dtype=torch.int32) for n in lengths])
        where = where.pin_memory().to(hidden.device, non_blocking=True)
        if self.int8:
            ext.dec_scatter_kv_q8(kv, where[0], where[1], self.cross_k, self.cross_v, self.cross_ks, self.cross_vs)
        else:
            ext.dec_scatter_kv(kv, where[0], where[1], self.cross_k, self.cross_v)

    def admit(self, slots: list[int], prompts: list[torch.Tensor], frames: list[int],
              max_new: list[int] | None = None) -> None:
        """Start decoding in the given slots (on the decoder stream): each slot's prompt is forced by the steps
        themselves, `frames` encoder frames attended to, at most max_new (default max_new_tokens) tokens made."""
        n = len(slots)
        if n == 0:
            return
        forced = torch.full((n, self.max_prompt), self.pad, dtype=torch.long)
        nums = torch.empty(n, 3, dtype=torch.int32)  # prompt length, position limit, frames
        for i, p in enumerate(prompts):
            p = torch.as_tensor(p, dtype=torch.long).flatten()
            if not 1 <= len(p) <= self.max_prompt:
                raise ValueError(f"StreamDecoder: a prompt of {len(p)} tokens (1..{self.max_prompt})")
            if not 1 <= frames[i] <= self.frames:
                raise ValueError(f"StreamDecoder: {frames[i]} encoder frames (1..{self.frames})")
            forced[i, :len(p)] = p
            nums[i] = torch.tensor([len(p), len(p) - 1 + (max_new[i] if max_new else self.max_new_tokens),
                                    frames[i]])
        out_rows = torch.full((n, self.seq + 1), self.pad, dtype=torch.long)
        out_rows[:, :self.max_prompt] = forced
        with torch.cuda.stream(self.stream):
            idx = self._to_device(torch.tensor(slots, dtype=torch.long))
            forced_d, nums_d, out_d = (self._to_device(t) for t in (forced, nums, out_rows))
            self.forced.index_copy_(0, idx, forced_d)
            self.out.index_copy_(0, idx, out_d)
            self.tok.index_copy_(0, idx, forced_d[:, 0].contiguous())
            self.pos.index_fill_(0, idx, 0)
            self.plen.index_copy_(0, idx, nums_d[:, 0].contiguous())
            self.limit.index_copy_(0, idx, nums_d[:, 1].contiguous())
            self.cross_len.index_copy_(0, idx, nums_d[:, 2].contiguous())
            self.finished.index_fill_(0, idx, 0)
        self.flags[torch.tensor(slots, dtype=torch.long)] = 0
        self._embed_stale = True

    def set_active(self, slots: list[int]) -> int:
        """The active rows of the next steps (on the decoder stream), padded with the dummy slot; returns the
        bucket to step."""
        b = self.bucket(max(1, len(slots)))
        host = torch.full((b,), self.dummy, dtype=torch.int32)
        host[:len(slots)] = torch.tensor(slots, dtype=torch.int32)
        with torch.cuda.stream(self.stream):
            self.active[:b].copy_(self._to_device(host))
        self._embed_stale = True
        return b

    def step(self, bucket: int, n: int = 1) -> None:
        """`n` decoding steps of the first `bucket` active rows (graph replays on the decoder stream; n == chunk is
        one replay of the chunk graph). With the fused program the rows' embeddings come from the previous step's
        pick; after admit / set_active / reset, or on a different bucket, they are computed first."""
        with torch.cuda.stream(self.stream):
            if bucket in self.graphs:
                if self.fused and (self._embed_stale or bucket != self._embed_rows):
                    self._embed(bucket)
                if n > 1 and n == self.chunk and bucket in self.chunk_graphs:
                    self.chunk_graphs[bucket].replay()
                else:
                    for _ in range(n):
                        self.graphs[bucket].replay()
            else:
                for _ in range(n):
                    self._run(bucket)
            self._embed_stale, self._embed_rows = False, bucket

    def weight_bytes(self) -> int:
        """Bytes of projection weights one step reads."""
        return sum(p.nbytes for blk in self.blocks for p in blk.projections()) + self.head.nbytes


__all__ = ["DEFAULT_CONFIG", "StreamDecoder", "W8_CONFIGS", "W8_PERM", "bf16_linear", "prepare_w8", "unprepare_w8",
           "w8_config", "w8_linear"]
