"""End-to-end transcription on gfx950: audio pieces -> log-mel features -> packed encoder -> cross-attention caches ->
greedy decoding with continuous batching -> token ids.

The stages and their order are those of the reference's Pipeline (kernels/pipeline.py:60-250): features of a chunk of
pieces (kernels/features.py), the packed int8 encoder over at most CHUNK_FRAMES encoder frames per call
(kernels/fast_encoder.py), the chunk's cross-attention keys and values written into its decoder slots, then captured
decoding steps (kernels/stream_decoder.py) over every admitted piece, the end flags read one step behind (LAG) so the
GPU never waits for the host. The service around it (request threads, the encoder/decoder thread pair, the wait-time
ordering of requests) is not part of this path: transcribe() runs the stages in the caller's thread, admitting as many
pieces as there are slots and refilling slots as pieces end.

    pipe = Pipeline(model, slots=32, int8=True, sparse=True)   # transformers CohereAsrForConditionalGeneration, bf16
    tokens = pipe.transcribe([dither(x1), dither(x2)], prompt)  # per piece: prompt + generated ids (np.int64)
"""

from __future__ import annotations

from collections import deque

import numpy as np
import torch

from kernels.fast_encoder import FastEncoder
from kernels.features import Features, dither
from kernels.stream_decoder import StreamDecoder


class Pipeline:
    CHUNK_FRAMES = 3000  # encoder frames per encoder call (reference pipeline.py:61)
    LAG = 1  # steps between a step's launch and the host reading its end flags (reference pipeline.py:64)

    def __init__(self, model, extractor=None, slots: int = 128, max_new_tokens: int = 448, int8: bool = True,
                 sparse: str | bool | None = None, frames: int | None = None, buckets=None,
                 chunk_frames: int | None = None):
        dev = model.proj_out.weight.device
        self.features = Features(extractor, device=dev)
        self.encoder = FastEncoder(model.model.encoder, int8=int8, sparse=sparse)
        self.decoder = StreamDecoder(model, slots=slots, max_new_tokens=max_new_tokens, int8=int8, frames=frames,
                                     buckets=buckets)
        self.stats = {"steps": 0, "chunks": 0, "frames": 0}
        if chunk_frames is not None:  # encoder frames per call (the reference's 3000 keeps a service's calls short)
            self.CHUNK_FRAMES = chunk_frames

    @staticmethod
    def prepare(samples: np.ndarray) -> np.ndarray:
        """The extractor's dither (reference pipeline.py:98-100)."""
        return dither(samples)

    def _chunks(self, order: list[int], lengths: list[int], room: int) -> list[list[int]]:
        """Consecutive pieces of `order` in chunks of at most CHUNK_FRAMES encoder frames (a piece's estimate:
        samples // 1280 + 1, as the reference), at most `room` pieces in all."""
        chunks, cur, frames = [], [], 0
        for i in order[:room]:
            f = lengths[i] // 1280 + 1
            if cur and frames + f > self.CHUNK_FRAMES:
                chunks.append(cur)
                cur, frames = [], 0
            cur.append(i)
            frames += f
        if cur:
            chunks.append(cur)
        return chunks

    @torch.no_grad()
    def _encode(self, pieces: list, idx: list[int], slots: list[int]) -> list[int]:
        """Features and encoder of pieces idx into the given decoder slots; returns their encoder lengths."""
        feats, frames = self.features([pieces[i] for i in idx])
        hidden, lengths = self.encoder(feats, frames)
        self.decoder.fill_cross(hidden, lengths, slots)
        self.stats["chunks"] += 1
        self.stats["frames"] += sum(lengths)
        return lengths

    @torch.no_grad()
    def transcribe(self, pieces: list, prompt: torch.Tensor, max_new: list[int] | None = None) -> list[np.ndarray]:
        """Token ids (prompt + generated, up to and including the end token) of each dithered piece (numpy fp32
        samples or fp32 tensors on the GPU), greedy."""
        dec = self.decoder
        n = len(pieces)
        if n == 0:
            return []
        lengths = [len(p) for p in pieces]
        result: list[np.ndarray | None] = [None] * n
        waiting = list(range(n))
        free = list(range(dec.slots))[::-1]
        piece_of: dict[int, int] = {}
        admitted_at: dict[int, int] = {}
        active: list[int] = []
        steps: deque = deque()
        step_no, bucket = 0, 1
        out_host = torch.zeros(dec.slots + 1, dec.out.shape[1], dtype=torch.long).pin_memory()
        while waiting or active:
            if waiting and free:
                # admit what fits: encode chunk by chunk on the current stream, then order the decoder after it
                room = min(len(free), len(waiting))
                for chunk in self._chunks(waiting, lengths, room):
                    slots = [free.pop() for _ in chunk]
                    enc_lengths = self._encode(pieces, chunk, slots)
                    dec.stream.wait_stream(torch.cuda.current_stream())
                    dec.admit(slots, [prompt] * len(chunk), enc_lengths,
                              [max_new[i] if max_new else dec.max_new_tokens for i in chunk])
                    for s, i in zip(slots, chunk):
                        piece_of[s] = i
                        admitted_at[s] = step_no
                    active += slots
                    waiting = waiting[len(chunk):]
                bucket = dec.set_active(active)
            dec.step(bucket)
            ev = torch.cuda.Event()
            ev.record(dec.stream)
            steps.append((step_no, ev))
            step_no += 1
            self.stats["steps"] += 1
            # the end flags of the step LAG behind (all of them once nothing else is queued)
            changed = False
            while steps and (len(steps) > self.LAG or not active):
                k, e = steps.popleft()
                e.synchronize()
                flags = dec.flags.numpy()
                ended = [s for s in active if flags[s] and admitted_at[s] <= k]
                if ended:
                    gone = set(ended)
                    active = [s for s in active if s not in gone]
                    with torch.cuda.stream(dec.stream):
                        for s in ended:
                            out_host[s].copy_(dec.out[s], non_blocking=True)
                    dec.stream.synchronize()
                    for s in ended:
                        i = piece_of.pop(s)
                        result[i] = self._tokens(out_host[s].numpy(), len(prompt), max_new[i] if max_new else None)
                        free.append(s)
                    changed = True
            if changed and active:
                bucket = dec.set_active(active)
        while steps:  # steps launched after the last piece ended
            steps.popleft()[1].synchronize()
        return result

    def _tokens(self, row: np.ndarray, plen: int, max_new: int | None) -> np.ndarray:
        """The piece's ids: the prompt, then the generated ones up to and including the first end token (reference
        pipeline.py:240-244)."""
        gen = row[plen:]
        end = np.nonzero(gen == self.decoder.eos)[0]
        limit = max_new or self.decoder.max_new_tokens
        return row[:plen + (end[0] + 1 if len(end) else min(len(gen), limit))].copy()


__all__ = ["Pipeline"]
