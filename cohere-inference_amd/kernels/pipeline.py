"""End-to-end transcription on gfx950: audio pieces -> log-mel features -> packed encoder -> cross-attention caches ->
greedy decoding with continuous batching -> token ids (the call surface of the reference's kernels/pipeline.py).

Two ways in, one decoding engine (_Decoding: the active slots, the pieces they hold, the steps in flight -- launched
in chunks of the decoder's `chunk` steps while no piece waits, one graph replay each -- and the end flags read LAG
launches behind, so the GPU never waits for the host):

  submit(pieces, prompt, max_new) -> Future   a service: an encoder thread takes waiting pieces in chunks of at most
                                              CHUNK_FRAMES encoder frames (as many as there are free decoder slots),
                                              computes features, runs the encoder and fills the chunk's slots on its
                                              own stream, and hands the chunk over; a decoder thread admits encoded
                                              chunks between steps and answers each request when its last piece ends.
                                              The next chunk encodes while the current ones decode.
  transcribe(pieces, prompt, max_new)         the same stages in the caller's thread, admitting as many pieces as there
                                              are slots and refilling slots as pieces end (no threads; for batch runs
                                              and measurement). Not usable once submit() has started the threads.

Every stage computes each piece independently of the others it is batched with (per-row kernels, per-sequence
attention and convolution, one cross-attention split for every bucket), so a piece's tokens do not depend on which
path, chunk or batch it went through, as long as its encoder chunk has the same rows.

    pipe = Pipeline(model, extractor, slots=32, int8=True, sparse=True)  # transformers CohereAsrForConditionalGeneration
    tokens = pipe.submit([pipe.prepare(x1), pipe.prepare(x2)], prompt).result()  # per piece: prompt + generated ids
"""

from __future__ import annotations

import threading
import time
from collections import deque
from concurrent.futures import Future

import numpy as np
import torch

from kernels.fast_encoder import FastEncoder
from kernels.features import Features, dither
from kernels.stream_decoder import StreamDecoder


class _Request:
    """One submit() call: its future and the token arrays of its pieces as they end."""

    def __init__(self, n: int):
        self.future: Future = Future()
        self.tokens: list = [None] * n
        self.pending = n

    def deliver(self, k: int, tokens: np.ndarray) -> None:
        self.tokens[k] = tokens
        self.pending -= 1
        if self.pending == 0 and not self.future.done():
            self.future.set_result(self.tokens)

    def fail(self, exc: BaseException) -> None:
        if not self.future.done():
            self.future.set_exception(exc)


class _Piece:
    """A piece waiting for (or in) the pipeline: its samples (on the GPU once `ready` has fired), prompt and limit."""

    def __init__(self, samples, prompt, max_new, request=None, k=0, ready=None):
        self.samples, self.prompt, self.max_new = samples, prompt, max_new
        self.request, self.k, self.ready = request, k, ready
        self.n = len(samples)
        self.arrived = time.perf_counter()
        self.tokens = None

    @property
    def frames(self) -> int:
        """The encoder frames the piece will take (samples // 1280 + 1, the chunking estimate)."""
        return self.n // 1280 + 1


class _Decoding:
    """The decoder side shared by both paths: admits encoded pieces into their slots, steps the active rows, reads the
    end flags LAG steps behind (a slot's flag only from a step launched after its admission: an earlier step may still
    copy the previous occupant's flag) and returns the pieces that ended with their tokens."""

    def __init__(self, dec: StreamDecoder, lag: int):
        self.dec, self.lag = dec, lag
        self.active: list[int] = []
        self.holder: dict[int, _Piece] = {}
        self.first_step: dict[int, int] = {}
        self.inflight: deque = deque()
        self.steps = 0
        self.limit: dict[int, int] = {}  # a slot's step (counted from its admission) that ends it by the token limit
        self.bucket, self.stale = 1, True
        self.rows_host = torch.zeros(dec.slots + 1, dec.out.shape[1], dtype=torch.long).pin_memory()

    def admit(self, slots: list[int], pieces: list[_Piece], lengths: list[int]) -> None:
        dec = self.dec
        dec.admit(slots, [p.prompt for p in pieces], lengths, [p.max_new or dec.max_new_tokens for p in pieces])
        for s, p in zip(slots, pieces):
            self.holder[s] = p
            self.first_step[s] = self.steps
            # the pick ends a row at its step `plen - 1 + max_new` after admission, if no end token came first
            self.limit[s] = len(p.prompt) - 1 + (p.max_new or dec.max_new_tokens)
        self.active += slots
        self.stale = True

    def chunk(self) -> int:
        """Steps to launch at once: the decoder's chunk, but never past the step at which an active row reaches its
        token limit, so that rows ending by the limit are seen as early as with single steps (a row ending by its end
        token is seen up to a chunk later, and it is stepped meanwhile as between any launch and its harvest)."""
        if not self.active:
            return 1
        left = min(self.limit[s] - (self.steps - self.first_step[s]) for s in self.active)
        return max(1, min(self.dec.chunk, left))

    def step(self, n: int = 1) -> None:
        if self.stale:
            self.bucket = self.dec.set_active(self.active)
            self.stale = False
        self.dec.step(self.bucket, n)
        ev = torch.cuda.Event()
        ev.record(self.dec.stream)
        self.inflight.append((self.steps + n - 1, ev))  # the flags after the last of the n steps
        self.steps += n

    def harvest(self) -> list[tuple[int, _Piece]]:
        """(slot, piece) of every piece found ended, its tokens set; the slots are free again."""
        dec, done = self.dec, []
        while self.inflight and (len(self.inflight) > self.lag or not self.active):
            k, ev = self.inflight.popleft()
            ev.synchronize()
            flags = dec.flags.numpy()
            ended = [s for s in self.active if flags[s] and self.first_step[s] <= k]
            if not ended:
                continue
            gone = set(ended)
            self.active = [s for s in self.active if s not in gone]
            self.stale = True
            with torch.cuda.stream(dec.stream):
                for s in ended:
                    self.rows_host[s].copy_(dec.out[s], non_blocking=True)
            dec.stream.synchronize()
            for s in ended:
                p = self.holder.pop(s)
                p.tokens = self._tokens(self.rows_host[s].numpy(), len(p.prompt), p.max_new)
                done.append((s, p))
        return done

    def drain(self) -> None:
        """Wait for the steps still in flight (launched after the last piece ended)."""
        while self.inflight:
            self.inflight.popleft()[1].synchronize()

    def _tokens(self, row: np.ndarray, plen: int, max_new: int | None) -> np.ndarray:
        """The prompt, then the generated ids up to and including the first end token (reference
        pipeline.py:240-244)."""
        gen = row[plen:]
        end = np.nonzero(gen == self.dec.eos)[0]
        limit = max_new or self.dec.max_new_tokens
        return row[:plen + (end[0] + 1 if len(end) else min(len(gen), limit))].copy()


class Pipeline:
    """Features, encoder and decoder of a transformers CohereAsrForConditionalGeneration on one GPU (reference
    kernels/pipeline.py:60-250, same constructor arguments and defaults; `extractor` may be None for the
    CohereAsrFeatureExtractor settings). Keyword-only extras: frames (encoder frames per decoder slot), buckets
    (decoder row buckets), chunk_frames (encoder frames per encoder call), sparse_w1 (both feed-forward linears 2:4)."""

    CHUNK_FRAMES = 3000  # encoder frames per encoder call (reference pipeline.py:61)
    LAG = 1  # steps between a step's launch and the host reading its end flags (reference pipeline.py:64)
    MAX_WAIT_S = 0.75  # a piece waiting longer than this goes first in the next chunk, whatever its length
    # the order of the pieces that have not waited that long: "short_then_long" takes the shortest third first (early
    # answers for short requests), then the rest longest first (a short decoding tail); "short" shortest first
    ORDER = "short_then_long"

    def __init__(self, model, extractor=None, slots: int = 128, max_new_tokens: int = 448, int8: bool = False,
                 sparse: str | bool | None = None, *, frames: int | None = None, buckets=None,
                 chunk_frames: int | None = None, sparse_w1: bool = False):
        dev = model.proj_out.weight.device
        self.device = dev
        self.features = Features(extractor, device=dev)
        self.encoder = FastEncoder(model.model.encoder, int8=int8, sparse=sparse, sparse_w1=sparse_w1)
        self.decoder = StreamDecoder(model, slots=slots, max_new_tokens=max_new_tokens, int8=int8, frames=frames,
                                     buckets=buckets)
        if chunk_frames is not None:
            self.CHUNK_FRAMES = chunk_frames
        self.stats = {"steps": 0, "chunks": 0, "frames": 0}
        # the service (started by the first submit())
        self._cv = threading.Condition()
        self._waiting: list[_Piece] = []
        self._free: list[int] = list(range(slots))[::-1]
        self._encoded: deque = deque()
        self._threads: list[threading.Thread] = []
        self._closed = False
        self._enc_stream = self._up_stream = None

    # ---- shared stages --------------------------------------------------------------------------------------------

    @staticmethod
    def prepare(samples: np.ndarray) -> np.ndarray:
        """The extractor's dither, added in the caller's thread (reference pipeline.py:98-100)."""
        return dither(samples)

    @torch.no_grad()
    def _encode(self, pieces: list[_Piece], slots: list[int]) -> list[int]:
        """Features and encoder of the pieces into the given decoder slots, on the current stream; returns their
        encoder lengths."""
        feats, frames = self.features([p.samples for p in pieces])
        hidden, lengths = self.encoder(feats, frames)
        self.decoder.fill_cross(hidden, lengths, slots)
        self.stats["chunks"] += 1
        self.stats["frames"] += sum(lengths)
        return lengths

    def _chunk(self, queue: list[_Piece], room: int) -> list[_Piece]:
        """The longest prefix of queue within CHUNK_FRAMES encoder frames (at least one piece) and room pieces."""
        chunk, frames = [], 0
        for p in queue[:room]:
            if chunk and frames + p.frames > self.CHUNK_FRAMES:
                break
            chunk.append(p)
            frames += p.frames
        return chunk

    # ---- in the caller's thread -----------------------------------------------------------------------------------

    @torch.no_grad()
    def transcribe(self, pieces: list, prompt: torch.Tensor, max_new: list[int] | None = None) -> list[np.ndarray]:
        """Token ids (prompt + generated, up to and including the end token) of each dithered piece (numpy fp32
        samples or fp32 tensors on the GPU), greedy, in the caller's thread."""
        if self._threads:
            raise RuntimeError("Pipeline: transcribe() cannot run beside the submit() threads")
        dec = self.decoder
        queue = [_Piece(x, prompt, max_new[i] if max_new else None, k=i) for i, x in enumerate(pieces)]
        result: list = [None] * len(queue)
        run, free = _Decoding(dec, self.LAG), list(range(dec.slots))[::-1]
        while queue or run.active:
            if queue and free:
                room = min(len(free), len(queue))
                while room:
                    chunk = self._chunk(queue, room)
                    slots = [free.pop() for _ in chunk]
                    lengths = self._encode(chunk, slots)
                    dec.stream.wait_stream(torch.cuda.current_stream())
                    run.admit(slots, chunk, lengths)
                    queue, room = queue[len(chunk):], room - len(chunk)
            n = 1 if queue and free else run.chunk()  # single steps while pieces wait for a slot
            run.step(n)
            self.stats["steps"] += n
            for s, p in run.harvest():
                result[p.k] = p.tokens
                free.append(s)
        run.drain()
        return result

    # ---- the service ----------------------------------------------------------------------------------------------

    def submit(self, pieces: list[np.ndarray], prompt: torch.Tensor, max_new: list[int] | None = None) -> Future:
        """Decode dithered pieces (prepare()) with this prompt; the future's result is one int64 array per piece,
        prompt + generated ids. max_new: tokens to generate at most per piece (default the decoder's max_new_tokens).
        The samples are copied to the GPU here, on a stream of their own."""
        self._validate(pieces, prompt)
        req = _Request(len(pieces))
        if not pieces:
            req.future.set_result([])
            return req.future
        self._start()
        with torch.cuda.stream(self._up_stream):
            gpu = [torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).pin_memory()
                   .to(self.device, non_blocking=True) for x in pieces]
            ready = torch.cuda.Event()
            ready.record(self._up_stream)
        with self._cv:
            if self._closed:
                raise RuntimeError("Pipeline: closed")
            for k, x in enumerate(gpu):
                self._waiting.append(_Piece(x, prompt, max_new[k] if max_new else None, req, k, ready))
            self._cv.notify_all()
        return req.future

    def _validate(self, pieces: list, prompt: torch.Tensor) -> None:
        """Raise ValueError in the caller for what the decoder would refuse at admission: a prompt outside
        1..max_prompt tokens, or a piece longer than the encoder frames a slot holds (samples // 1280 + 1 is the exact
        encoder length: a centred 160-sample hop, then three stride-2 halvings)."""
        dec = self.decoder
        if not 1 <= len(prompt) <= dec.max_prompt:
            raise ValueError(f"Pipeline: a prompt of {len(prompt)} tokens (1..{dec.max_prompt})")
        for x in pieces:
            frames = len(x) // 1280 + 1
            if frames > dec.frames:
                raise ValueError(f"Pipeline: a piece of {len(x)} samples needs {frames} encoder frames "
                                 f"(at most {dec.frames})")

    def close(self) -> None:
        """Stop the service threads once the work they hold is done (pending requests are answered first)."""
        with self._cv:
            self._closed = True
            self._cv.notify_all()
        for t in self._threads:
            t.join()

    def _start(self) -> None:
        with self._cv:
            if self._threads:
                return
            self._enc_stream = torch.cuda.Stream(device=self.device)
            self._up_stream = torch.cuda.Stream(device=self.device)
            self._threads = [threading.Thread(target=self._encoder_worker, name="pipeline-encoder", daemon=True),
                             threading.Thread(target=self._decoder_worker, name="pipeline-decoder", daemon=True)]
        for t in self._threads:
            t.start()

    def _next_chunk(self) -> tuple[list[_Piece], list[int]]:
        """(lock held) The next chunk and its slots: pieces that have waited longer than MAX_WAIT_S first, in
        arrival order, then the rest in ORDER (reference pipeline.py:120-131)."""
        if not self._waiting or not self._free:
            return [], []
        now = time.perf_counter()
        late = [p for p in self._waiting if now - p.arrived > self.MAX_WAIT_S]
        rest = sorted((p for p in self._waiting if now - p.arrived <= self.MAX_WAIT_S), key=lambda p: p.n)
        if self.ORDER == "short_then_long" and len(rest) > 8:
            third = len(rest) // 3
            rest = rest[:third] + rest[third:][::-1]
        chunk = self._chunk(late + rest, len(self._free))
        taken = {id(p) for p in chunk}
        self._waiting = [p for p in self._waiting if id(p) not in taken]
        return chunk, [self._free.pop() for _ in chunk]

    @torch.no_grad()
    def _encoder_worker(self) -> None:
        torch.cuda.set_device(self.device)
        while True:
            with self._cv:
                chunk, slots = self._next_chunk()
                while not chunk:
                    if self._closed and not self._waiting:
                        return
                    self._cv.wait()
                    chunk, slots = self._next_chunk()
            try:
                with torch.cuda.stream(self._enc_stream):
                    for ev in {id(p.ready): p.ready for p in chunk}.values():
                        self._enc_stream.wait_event(ev)
                    lengths = self._encode(chunk, slots)
                    done = torch.cuda.Event()
                    done.record(self._enc_stream)
                done.synchronize()
            except Exception as exc:  # noqa: BLE001 -- the chunk's requests fail with it, the service goes on
                with self._cv:
                    self._free.extend(slots)
                    self._cv.notify_all()
                for p in chunk:
                    p.request.fail(exc)
                continue
            with self._cv:
                self._encoded.append((slots, chunk, lengths))
                self._cv.notify_all()

    @torch.no_grad()
    def _decoder_worker(self) -> None:
        torch.cuda.set_device(self.device)
        run = _Decoding(self.decoder, self.LAG)
        while True:
            with self._cv:
                while not self._encoded and not run.active and not run.inflight:
                    if self._closed and not self._waiting and not any(t.is_alive() for t in self._threads[:1]):
                        return
                    self._cv.wait(timeout=0.1 if self._closed else None)
                new = list(self._encoded)
                self._encoded.clear()
            for slots, chunk, lengths in new:
                try:
                    run.admit(slots, chunk, lengths)
                except Exception as exc:  # noqa: BLE001 -- the chunk's requests fail, its slots are freed
                    self._release(slots, chunk, exc)
            try:
                if run.active:
                    with self._cv:
                        waiting = bool(self._waiting or self._encoded)
                    n = 1 if waiting else run.chunk()  # single steps while pieces are on their way in
                    run.step(n)
                    self.stats["steps"] += n
                ended = run.harvest()
                if not run.active:
                    run.drain()
            except Exception as exc:  # noqa: BLE001 -- every piece being decoded fails; the service goes on
                held = [(s, run.holder[s]) for s in run.active if s in run.holder]
                self._release([s for s, _ in held], [p for _, p in held], exc)
                run = _Decoding(self.decoder, self.LAG)
                continue
            for _, p in ended:
                p.request.deliver(p.k, p.tokens)
            if ended:
                with self._cv:
                    self._free.extend(s for s, _ in ended)
                    self._cv.notify_all()

    def _release(self, slots: list[int], pieces: list[_Piece], exc: BaseException) -> None:
        """Fail the pieces' requests and return their slots."""
        for p in pieces:
            if p.request is not None:
                p.request.fail(exc)
        with self._cv:
            self._free.extend(slots)
            self._cv.notify_all()


__all__ = ["Pipeline"]
