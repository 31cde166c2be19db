"""Host-side scheduling of the pipeline service (no GPU): how the encoder thread cuts chunks from the waiting pieces
(reference kernels/pipeline.py:144-183 -- as many pieces as there are free slots, within CHUNK_FRAMES encoder frames,
at least one piece) and in which order it takes them (pieces that waited longer than MAX_WAIT_S first, in arrival
order, then the rest in ORDER: the shortest third, then the others longest first), how submit() refuses what the
decoder would refuse, and how a request's future completes."""

from __future__ import annotations

import types

import numpy as np
import pytest

from kernels.pipeline import Pipeline, _Piece, _Request


def _piece(n: int, arrived: float = 0.0) -> _Piece:
    p = _Piece(np.zeros(n, np.float32), None, None)
    p.arrived = arrived
    return p


def _stub(chunk_frames=3000, waiting=(), free=(), max_wait=0.75, order="short_then_long"):
    st = types.SimpleNamespace(CHUNK_FRAMES=chunk_frames, MAX_WAIT_S=max_wait, ORDER=order, _waiting=list(waiting),
                               _free=list(free))
    st._chunk = lambda queue, room: Pipeline._chunk(st, queue, room)
    return st


def test_piece_frames_estimate():
    # samples // 1280 + 1 encoder frames: 30 s at 16 kHz -> 376
    assert _piece(480000).frames == 376
    assert _piece(0).frames == 1


def test_chunk_respects_frames_and_room():
    st = _stub(chunk_frames=1000)
    q = [_piece(1280 * 399) for _ in range(4)]  # 400 frames each
    assert len(Pipeline._chunk(st, q, 10)) == 2  # 800 <= 1000 < 1200
    assert len(Pipeline._chunk(st, q, 1)) == 1
    big = [_piece(1280 * 5000)]
    assert len(Pipeline._chunk(st, big, 4)) == 1  # one piece always goes, whatever its length
    assert Pipeline._chunk(st, [], 4) == []


def test_next_chunk_order_late_first_then_shortest(monkeypatch):
    import kernels.pipeline as pl

    now = 100.0
    monkeypatch.setattr(pl.time, "perf_counter", lambda: now)
    late_long = _piece(1280 * 300, arrived=now - 2.0)
    late_short = _piece(1280 * 10, arrived=now - 1.0)
    fresh_long = _piece(1280 * 200, arrived=now)
    fresh_short = _piece(1280 * 50, arrived=now)
    st = _stub(waiting=[fresh_long, late_long, fresh_short, late_short], free=[7, 6, 5, 4, 3])
    chunk, slots = Pipeline._next_chunk(st)
    assert chunk == [late_long, late_short, fresh_short, fresh_long]
    assert slots == [3, 4, 5, 6] and st._free == [7]
    assert st._waiting == []


def test_next_chunk_short_then_long_over_eight(monkeypatch):
    """With more than 8 fresh pieces: the shortest third first, then the remaining ones longest first (reference
    pipeline.py:126-128); with 8 or fewer, or ORDER "short", plain shortest first."""
    import kernels.pipeline as pl

    monkeypatch.setattr(pl.time, "perf_counter", lambda: 0.0)
    ps = [_piece(1280 * (10 * i + 9)) for i in (3, 7, 0, 9, 1, 5, 8, 2, 6, 4, 10)]  # 11 fresh pieces, shuffled
    by_len = sorted(ps, key=lambda p: p.n)
    st = _stub(waiting=ps, free=list(range(20)))
    chunk, _ = Pipeline._next_chunk(st)
    assert chunk == by_len[:3] + by_len[3:][::-1]
    st = _stub(waiting=ps, free=list(range(20)), order="short")
    assert Pipeline._next_chunk(st)[0] == by_len
    st = _stub(waiting=ps[:8], free=list(range(20)))
    assert Pipeline._next_chunk(st)[0] == sorted(ps[:8], key=lambda p: p.n)


def test_submit_validates_in_the_caller():
    """A prompt outside 1..max_prompt or a piece beyond the slot's encoder frames raises ValueError in submit()
    (before any thread starts), instead of killing the decoder thread at admission."""
    import torch

    st = types.SimpleNamespace(decoder=types.SimpleNamespace(max_prompt=4, frames=376))
    ok = np.zeros(480000, np.float32)  # 376 frames
    Pipeline._validate(st, [ok], torch.tensor([1, 2]))
    with pytest.raises(ValueError, match="prompt"):
        Pipeline._validate(st, [ok], torch.tensor([], dtype=torch.long))
    with pytest.raises(ValueError, match="prompt"):
        Pipeline._validate(st, [ok], torch.arange(5))
    with pytest.raises(ValueError, match="encoder frames"):
        Pipeline._validate(st, [ok, np.zeros(480000 + 1280, np.float32)], torch.tensor([1]))


def test_next_chunk_bounded_by_free_slots_and_frames(monkeypatch):
    import kernels.pipeline as pl

    monkeypatch.setattr(pl.time, "perf_counter", lambda: 0.0)
    ps = [_piece(1280 * (100 + i)) for i in range(6)]
    st = _stub(chunk_frames=350, waiting=ps, free=[1, 0])
    chunk, slots = Pipeline._next_chunk(st)
    assert chunk == ps[:2] and slots == [0, 1]  # shortest first, two free slots
    assert st._waiting == ps[2:] and st._free == []
    assert Pipeline._next_chunk(st) == ([], [])  # no free slot: nothing taken
    st._free = [5, 4, 3]
    chunk, _ = Pipeline._next_chunk(st)
    assert chunk == ps[2:5]  # three free slots; 103 + 104 + 105 frames fit the 350
    assert Pipeline._next_chunk(_stub(waiting=[], free=[0])) == ([], [])


def test_request_future():
    r = _Request(2)
    r.deliver(1, np.array([1]))
    assert not r.future.done()
    r.deliver(0, np.array([0]))
    assert [t.tolist() for t in r.future.result()] == [[0], [1]]
    f = _Request(1)
    f.fail(RuntimeError("boom"))
    with pytest.raises(RuntimeError, match="boom"):
        f.future.result()
    f.deliver(0, np.array([0]))  # a late piece of a failed request changes nothing
    with pytest.raises(RuntimeError):
        f.future.result()
