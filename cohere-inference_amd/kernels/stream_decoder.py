"""Greedy decoding with continuous batching on gfx950 (the reference's kernels/stream_decoder.py): the int8-weight
(W8A16) layout and 64-row chunked projection calls (prepare_w8 38-48, W8_CONFIGS 30-35, _w8 148-158) over the skinny
HIP GEMMs of csrc/dec_w8.hip, and the StreamDecoder itself (73-276): per-slot state and KV caches, one step = embedding,
8 x (self-attention over the slot's int8 cache, cross-attention, feed-forward), head and greedy pick, captured into one
HIP graph per bucket of row counts (csrc/decoder_ops.hip for the non-GEMM kernels).

    wq = prepare_w8(w_bf16)                          # (uint8 (N, K), fp32 (N))
    y = w8_linear(x, wq, bias, relu=False, ws=ws, counters=counters)
    y = bf16_linear(x, w_bf16, bias)                 # o / cross-q / cross-o (the reference's Triton `linear`)
    dec = StreamDecoder(model, slots=64, int8=True)  # model: transformers CohereAsrForConditionalGeneration
    dec.fill_cross(hidden, lengths, slots); dec.admit(slots, prompts, lengths); b = dec.set_active(slots)
    dec.step(b)                                      # one graph replay
"""

from __future__ import annotations

import torch

from kernels.cuda_ext import ext

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
    scales). Quantization: s = max(amax|w|, 1e-12) / 127, q = clamp(round_half_even(w / s), +-127)."""
    n, k = w.shape
    assert k % 16 == 0
    wf = w.float()
    s = wf.abs().amax(1).clamp_min(1e-12) / 127
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


# ---- the step and its graphs (reference stream_decoder.py:60-276) ----------------------------------------------------

class _Layer:
    """One decoder layer's tensors (reference stream_decoder.py:60-71)."""

    def __init__(self, layer):
        sa, ca = layer.self_attn, layer.encoder_attn
        ln = lambda m: (m.weight, m.bias, m.eps)  # noqa: E731
        self.ln1, self.ln2, self.ln3 = ln(layer.input_layernorm), ln(layer.post_attention_layernorm), \
            ln(layer.final_layernorm)
        self.qkv = (torch.cat([sa.q_proj.weight, sa.k_proj.weight, sa.v_proj.weight]).contiguous(),
                    torch.cat([sa.q_proj.bias, sa.k_proj.bias, sa.v_proj.bias]).contiguous())
        self.o = (sa.o_proj.weight, sa.o_proj.bias)
        self.cq = (ca.q_proj.weight, ca.q_proj.bias)
        self.co = (ca.o_proj.weight, ca.o_proj.bias)
        self.fc1 = (layer.mlp.fc1.weight, layer.mlp.fc1.bias)
        self.fc2 = (layer.mlp.fc2.weight, layer.mlp.fc2.bias)


class StreamDecoder:
    """Greedy decoding with continuous batching over per-slot state and KV caches, one HIP graph per bucket of row
    counts (reference kernels/stream_decoder.py:73-276, same attributes and methods). The model is a transformers
    CohereAsrForConditionalGeneration (or anything with its decoder attributes). Differences: the decoder stream has
    the default priority (stream priorities are not used on this platform), and `frames` may be given instead of
    asking the encoder for its subsampled length."""

    BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96, 112, 128)

    def __init__(self, model, slots: int = 128, max_new_tokens: int = 448, max_prompt: int = 16,
                 max_audio_s: float = 36.0, buckets=None, int8: bool = False, frames: int | None = None,
                 capture: bool = True):
        dec, cfg = model.model.decoder, model.config
        self.buckets = tuple(b for b in (buckets or self.BUCKETS) if b <= slots)
        self.model, self.max_new_tokens = model, max_new_tokens
        self.h, self.d, self.width = cfg.num_attention_heads, getattr(cfg, "head_dim", None), cfg.hidden_size
        self.d = self.d or self.width // self.h
        assert self.d == 128, "the decoder kernels take head size 128"
        self.eos, self.pad = cfg.eos_token_id, cfg.pad_token_id
        self.scale = self.d ** -0.5
        self.embed, self.pos_table = dec.embed_tokens.weight, dec.pos_emb.weight
        ln = lambda m: (m.weight, m.bias, m.eps)  # noqa: E731
        self.emb_ln, self.final_ln = ln(dec.embedding_layernorm), ln(dec.norm)
        self.head = (model.proj_out.weight, model.proj_out.bias)
        self.proj = (dec.proj.weight, dec.proj.bias)
        self.layers = [_Layer(layer) for layer in dec.layers]
        self.int8 = int8
        if int8:
            for ly in self.layers:
                ly.qkv_w8, ly.fc1_w8, ly.fc2_w8 = prepare_w8(ly.qkv[0]), prepare_w8(ly.fc1[0]), prepare_w8(ly.fc2[0])
            self.head_w8 = prepare_w8(self.head[0])
        self.cross_w = torch.cat([w for layer in dec.layers for w in (layer.encoder_attn.k_proj.weight,
                                                                       layer.encoder_attn.v_proj.weight)]).contiguous()
        self.cross_b = torch.cat([b for layer in dec.layers for b in (layer.encoder_attn.k_proj.bias,
                                                                       layer.encoder_attn.v_proj.bias)]).contiguous()
        L, S = len(self.layers), slots
        self.slots, self.dummy = S, S
        self.max_prompt = max_prompt
        self.seq = max_prompt + max_new_tokens + 1
        if frames is None:
            frames = int(model.model.encoder._get_subsampling_output_length(
                torch.tensor([int(max_audio_s * 100) + 1])).item())
        self.frames = frames
        dev, dt = self.embed.device, self.embed.dtype
        self.device = dev
        kv_dt = torch.int8 if int8 else dt
        self.self_k = torch.zeros(L, S + 1, self.h, self.seq, self.d, device=dev, dtype=kv_dt)
        self.self_v = torch.zeros_like(self.self_k)
        self.cross_k = torch.zeros(L, S + 1, self.h, self.frames, self.d, device=dev, dtype=kv_dt)
        self.cross_v = torch.zeros_like(self.cross_k)
        if int8:  # one fp32 scale per 128-vector
            self.self_ks = torch.ones(L, S + 1, self.h, self.seq, device=dev, dtype=torch.float32)
            self.self_vs = torch.ones_like(self.self_ks)
            self.cross_ks = torch.ones(L, S + 1, self.h, self.frames, device=dev, dtype=torch.float32)
            self.cross_vs = torch.ones_like(self.cross_ks)
        i32 = dict(device=dev, dtype=torch.int32)
        self.cross_len = torch.ones(S + 1, **i32)
        self.tok = torch.full((S + 1,), self.pad, device=dev, dtype=torch.long)
        self.pos = torch.zeros(S + 1, **i32)
        self.plen = torch.ones(S + 1, **i32)
        self.limit = torch.zeros(S + 1, **i32)
        self.finished = torch.ones(S + 1, device=dev, dtype=torch.uint8)
        self.forced = torch.full((S + 1, max_prompt), self.pad, device=dev, dtype=torch.long)
        self.out = torch.full((S + 1, self.seq + 1), self.pad, device=dev, dtype=torch.long)
        self.active = torch.full((max(self.buckets),), S, **i32)
        bm = max(self.buckets)
        self.x = torch.zeros(bm, self.width, device=dev, dtype=dt)
        self.hn = torch.zeros(bm, self.width, device=dev, dtype=dt)
        self.att = torch.zeros(bm, self.width, device=dev, dtype=dt)
        self.logits = torch.zeros(bm, self.head[0].shape[0], device=dev, dtype=dt)
        self.part = torch.empty(max(b * self.h * self._splits(b) * (self.d + 2) for b in self.buckets), device=dev,
                                dtype=torch.float32)
        self.w8_ws = torch.empty(8 << 20, device=dev, dtype=torch.float32)
        self.w8_counters = torch.zeros(1024, device=dev, dtype=torch.int32)
        self.flags = torch.ones(S + 1, dtype=torch.uint8).pin_memory()
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.stream = torch.cuda.Stream()
        if capture:
            self._capture()

    @staticmethod
    def _splits(b: int) -> int:
        """Workgroups per (row, head) of the cross-attention: several only for one or two rows (reference
        stream_decoder.py:140-144)."""
        return 4 if b <= 2 else 1

    # ---- the step ----------------------------------------------------------------------------------------------

    def _w8(self, x, wq, bias, relu=False):
        return w8_linear(x, wq, bias, relu, ws=self.w8_ws, counters=self.w8_counters)

    def _proj(self, x, ly, name):
        """The o, cross q or cross o projection: bf16 weights, as the reference keeps them."""
        return bf16_linear(x, *getattr(ly, name))

    def _qkv(self, hn, ly):
        return self._w8(hn, ly.qkv_w8, ly.qkv[1]) if self.int8 else bf16_linear(hn, *ly.qkv)

    def _ffn(self, hn, ly):
        if self.int8:
            return self._w8(self._w8(hn, ly.fc1_w8, ly.fc1[1], relu=True), ly.fc2_w8, ly.fc2[1])
        return bf16_linear(bf16_linear(hn, *ly.fc1, relu=True), *ly.fc2)

    def _head(self, hn, out):
        if self.int8:
            return w8_linear(hn, self.head_w8, self.head[1], ws=self.w8_ws, counters=self.w8_counters, out=out)
        return bf16_linear(hn, *self.head, out=out)

    def _attend(self, i, self_attn, act, q, splits, a):
        if self_attn:
            caches, n = (self.self_k[i], self.self_v[i]), self.pos
            scales = (self.self_ks[i], self.self_vs[i]) if self.int8 else None
        else:
            caches, n = (self.cross_k[i], self.cross_v[i]), self.cross_len
            scales = (self.cross_ks[i], self.cross_vs[i]) if self.int8 else None
        if self.int8:
            ext.dec_attention_q8(self_attn, act, q, *caches, *scales, n, self.scale, splits, self.part, a)
        else:
            ext.dec_attention(self_attn, act, q, *caches, n, self.scale, splits, self.part, a)

    def _step(self, b: int) -> None:
        act, x, hn, a, splits = self.active[:b], self.x[:b], self.hn[:b], self.att[:b], self._splits(b)
        ext.dec_embed(act, self.tok, self.pos, self.embed, self.pos_table, *self.emb_ln, *self.layers[0].ln1, x, hn)
        for i, ly in enumerate(self.layers):
            nxt = self.layers[i + 1] if i + 1 < len(self.layers) else None
            self._attend(i, True, act, self._qkv(hn, ly), 1, a)
            ext.dec_add_ln(x, self._proj(a, ly, "o"), *ly.ln2, hn)
            self._attend(i, False, act, self._proj(hn, ly, "cq"), splits, a)
            ext.dec_add_ln(x, self._proj(a, ly, "co"), *ly.ln3, hn)
            following = nxt.ln1 if nxt else self.final_ln
            ext.dec_add_ln(x, self._ffn(hn, ly), *following, hn)
        logits = self._head(hn, self.logits[:b])
        ext.dec_pick(logits, act, self.dummy, self.tok, self.pos, self.finished, self.forced, self.plen, self.limit,
                     self.out, self.pad, self.eos)
        self.flags.copy_(self.finished, non_blocking=True)

    @torch.no_grad()
    def _capture(self) -> None:
        pool = torch.cuda.graph_pool_handle()
        with torch.cuda.stream(self.stream):
            for b in reversed(self.buckets):  # largest first: the smaller graphs fit in the pool it leaves
                self._step(b)
                torch.cuda.current_stream().synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=pool, stream=self.stream):
                    self._step(b)
                self.graphs[b] = g
            self.reset()
        self.stream.synchronize()

    def reset(self) -> None:
        """All slots free (on the decoder stream)."""
        with torch.cuda.stream(self.stream):
            self.finished.fill_(1)
            self.pos.zero_()
            self.cross_len.fill_(1)
            self.active.fill_(self.dummy)

    # ---- host side -----------------------------------------------------------------------------------------------

    def bucket(self, rows: int) -> int:
        return next(b for b in self.buckets if b >= rows)

    def fill_cross(self, hidden: torch.Tensor, lengths: list[int], slots: list[int], projected: bool = False) -> None:
        """Cross-attention keys and values of packed encoder frames (sum(lengths), encoder width) into the given slots
        (projected: hidden is already the decoder-width memory after `proj`), on the current stream."""
        mem = hidden if projected else torch.nn.functional.linear(hidden, *self.proj)
        kv = torch.nn.functional.linear(mem, self.cross_w, self.cross_b).contiguous()
        slot_of = torch.repeat_interleave(torch.tensor(slots, dtype=torch.int32), torch.tensor(lengths))
        frame_of = torch.cat([torch.arange(n, dtype=torch.int32) for n in lengths])
        slot_of, frame_of = slot_of.to(self.device), frame_of.to(self.device)
        if self.int8:
            ext.dec_scatter_kv_q8(kv, slot_of, frame_of, self.cross_k, self.cross_v, self.cross_ks, self.cross_vs)
        else:
            ext.dec_scatter_kv(kv, slot_of, frame_of, self.cross_k, self.cross_v)

    def admit(self, slots: list[int], prompts: list[torch.Tensor], frames: list[int],
              max_new: list[int] | None = None) -> None:
        """Start decoding in the given slots (on the decoder stream): the prompt forced, `frames` audio frames."""
        n = len(slots)
        idx = torch.tensor(slots, dtype=torch.long)
        forced = torch.full((n, self.max_prompt), self.pad, dtype=torch.long)
        plen = torch.tensor([len(p) for p in prompts], dtype=torch.int32)
        for i, p in enumerate(prompts):
            forced[i, :len(p)] = p
        limit = plen - 1 + torch.tensor(max_new or [self.max_new_tokens] * n, dtype=torch.int32)
        with torch.cuda.stream(self.stream):
            d = lambda t: t.to(self.device, non_blocking=True)  # noqa: E731
            di = d(idx)
            self.forced[di] = d(forced)
            self.out[di] = self.pad
            self.out[di, :self.max_prompt] = d(forced)
            self.tok[di] = d(forced[:, 0])
            self.pos[di] = 0
            self.plen[di] = d(plen)
            self.limit[di] = d(limit)
            self.cross_len[di] = d(torch.tensor(frames, dtype=torch.int32))
            self.finished[di] = 0
        self.flags[idx] = 0

    def set_active(self, slots: list[int]) -> int:
        """The active list for the next steps (on the decoder stream); returns the bucket."""
        b = self.bucket(max(1, len(slots)))
        host = torch.full((b,), self.dummy, dtype=torch.int32)
        host[:len(slots)] = torch.tensor(slots, dtype=torch.int32)
        with torch.cuda.stream(self.stream):
            self.active[:b].copy_(host.pin_memory(), non_blocking=True)
        return b

    def step(self, bucket: int) -> None:
        with torch.cuda.stream(self.stream):
            self.graphs[bucket].replay()
