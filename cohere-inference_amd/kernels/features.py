"""Normalized log-mel features of a batch of audio pieces on the GPU (drop-in for the reference's kernels/features.py).

Same call surface as the reference (Features(extractor)(pieces) -> (B, T, 128) bf16, frame counts; dither(x)); the
work is one native call, ext.logmel_features, whose kernels (cohere-inference_amd/csrc/frontend.hip) frame, FFT,
take the mel bands and log of every valid frame in LDS and normalize per piece and band.

The extractor's settings (transformers' CohereAsrFeatureExtractor: n_fft 512, hop 160, window 400, pre-emphasis
0.97, 128 Slaney mel bands) are read from the extractor object given; `default_extractor()` builds an object with
those settings and the filter bank computed by `slaney_mel_filters` (librosa's published algorithm restated), for
environments where the transformers extractor cannot be constructed (it needs librosa for its filter bank).

    x = dither(samples)                                   # in the request's thread
    feats, frames = Features(extractor)([x1, x2, ...])    # (B, T, 128) bf16 on the GPU, frame counts
"""

from __future__ import annotations

import types

import numpy as np
import torch

from kernels.cuda_ext import ext

LOG_GUARD = 2 ** -24
EPS = 1e-5


def dither(x: np.ndarray, amount: float = 1e-5) -> np.ndarray:
    """x + amount * the extractor's noise for a piece of this length: torch's CPU generator seeded with the piece's
    length, one normal draw per sample (reference features.py:29-38; transformers CohereAsrFeatureExtractor
    _apply_dither)."""
    n = len(x)
    if amount <= 0 or n == 0:
        return np.asarray(x, dtype=np.float32)
    g = torch.Generator()
    g.manual_seed(n)
    noise = torch.randn(n, dtype=torch.float32, generator=g)
    return (torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)) + amount * noise).numpy()


def _hz_to_mel(f):
    """Slaney's mel scale: linear below 1 kHz (3 mels per 200 Hz), logarithmic above (27 steps per factor 6.4)."""
    f = np.asarray(f, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    lin = f / f_sp
    return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-10) / min_log_hz) / logstep, lin)


def _mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)


def slaney_mel_filters(sr: int = 16000, n_fft: int = 512, n_mels: int = 128, fmin: float = 0.0,
                       fmax: float | None = None) -> torch.Tensor:
    """(n_mels, n_fft // 2 + 1) fp32 triangular filters on Slaney's mel scale with Slaney area normalization --
    librosa.filters.mel(sr, n_fft, n_mels, fmin, fmax, htk=False, norm="slaney"), the extractor's filter bank,
    restated from its published algorithm: band edges at n_mels + 2 points evenly spaced in mel, each filter the
    minimum of its rising and falling ramps over the FFT bin frequencies clipped at zero (stored in fp32), then scaled
    by 2 / (upper edge - lower edge) in Hz."""
    fmax = sr / 2 if fmax is None else fmax
    fftfreqs = np.linspace(0, sr / 2, 1 + n_fft // 2)
    mel_f = _mel_to_hz(np.linspace(_hz_to_mel(fmin), _hz_to_mel(fmax), n_mels + 2))
    fdiff = np.diff(mel_f)
    ramps = mel_f[:, None] - fftfreqs[None, :]
    weights = np.zeros((n_mels, 1 + n_fft // 2), dtype=np.float32)
    for i in range(n_mels):
        lower = -ramps[i] / fdiff[i]
        upper = ramps[i + 2] / fdiff[i + 1]
        weights[i] = np.maximum(0, np.minimum(lower, upper))
    enorm = 2.0 / (mel_f[2:n_mels + 2] - mel_f[:n_mels])
    weights *= enorm[:, None]
    return torch.from_numpy(weights)


def default_extractor():
    """The settings Features reads from transformers' CohereAsrFeatureExtractor, with its default values."""
    return types.SimpleNamespace(n_fft=512, hop_length=160, win_length=400, preemphasis=0.97, sampling_rate=16000,
                                 dither=1e-5, mel_filters=slaney_mel_filters())


class _Staging:
    """Pinned host buffers for the samples of numpy pieces, used in turn (two, so that one call's upload can still be
    in flight while the next call fills the other); each is reused only after the upload that last read it."""

    def __init__(self, count: int = 2):
        self.slots = [[torch.empty(0, dtype=torch.float32).pin_memory(), None] for _ in range(count)]
        self.turn = 0

    def upload(self, pieces: list, total: int, device) -> torch.Tensor:
        slot = self.slots[self.turn]
        self.turn = (self.turn + 1) % len(self.slots)
        if slot[1] is not None:
            slot[1].synchronize()
        if slot[0].numel() < total:
            slot[0] = torch.empty(max(total, 2 * slot[0].numel()), dtype=torch.float32).pin_memory()
        host = slot[0][:total].numpy()
        at = 0
        for p in pieces:
            n = len(p)
            host[at:at + n] = np.asarray(p, dtype=np.float32)
            at += n
        dev = slot[0][:total].to(device, non_blocking=True)
        slot[1] = torch.cuda.Event()
        slot[1].record()
        return dev


class Features:
    """Normalised log-mel features of a batch of pieces (reference kernels/features.py:41-88, same call surface):
    the extractor's Hann window (centred in the 512-point frame) and filter bank are prepared once, with each mel
    band's first and end nonzero bins, in the layout the log-mel kernel reads; a call is one native launch sequence
    over the valid frames of every piece."""

    def __init__(self, extractor=None, device="cuda"):
        fe = default_extractor() if extractor is None else extractor
        if (fe.n_fft, fe.hop_length, fe.win_length) != (512, 160, 400):
            raise ValueError("Features: the kernels take n_fft 512, hop 160, window 400")
        self.n_fft, self.hop, self.win = fe.n_fft, fe.hop_length, fe.win_length
        self.preemphasis = float(fe.preemphasis)
        self.device = torch.device(device)
        mel = torch.as_tensor(fe.mel_filters, dtype=torch.float32).cpu()
        if tuple(mel.shape) != (128, 257):
            raise ValueError("Features: the kernels take 128 mel bands over 257 bins")
        self.mels = mel.shape[0]
        self.mel = mel.contiguous().to(self.device)
        # torch.stft places the 400-point window in the middle of the 512-point frame
        self.window = torch.hann_window(self.win, periodic=False)
        frame_window = torch.zeros(self.n_fft)
        first = (self.n_fft - self.win) // 2
        frame_window[first:first + self.win] = self.window
        self.window512 = frame_window.to(self.device)
        self.window = self.window.to(self.device)
        edges = []
        for row in mel.numpy():
            nz = np.flatnonzero(row)
            edges.append((nz[0], nz[-1] + 1) if nz.size else (0, 0))
        self.band = torch.tensor(edges, dtype=torch.int32).to(self.device)
        self._staging = _Staging()

    @torch.no_grad()
    def __call__(self, pieces: list) -> tuple[torch.Tensor, list[int]]:
        """(B, T, 128) bf16 normalised log-mel frames of dithered pieces (numpy arrays, or fp32 tensors on the GPU),
        zero past each piece's frames, and the frame counts: a piece of n samples has n // 160 + 1 frames, the last
        one zero, as the service always fed the model."""
        sizes = [len(p) for p in pieces]
        if all(isinstance(p, torch.Tensor) for p in pieces):
            samples = torch.cat([p.reshape(-1).to(self.device, torch.float32) for p in pieces])
        else:
            samples = self._staging.upload(pieces, sum(sizes), self.device)
        valid = np.asarray(sizes, dtype=np.int64) // self.hop
        meta = np.concatenate([np.cumsum([0] + sizes[:-1]), sizes, np.concatenate([[0], np.cumsum(valid)])])
        meta = torch.from_numpy(meta.astype(np.int64)).pin_memory().to(self.device, non_blocking=True)
        out = torch.zeros(len(pieces), max(sizes) // self.hop + 1, self.mels, device=self.device,
                          dtype=torch.bfloat16)
        ext.logmel_features(samples, meta, int(valid.sum()), self.window512, self.mel, self.band, self.preemphasis,
                            out)
        return out, [int(v) + 1 for v in valid]


__all__ = ["EPS", "LOG_GUARD", "Features", "default_extractor", "dither", "slaney_mel_filters"]
