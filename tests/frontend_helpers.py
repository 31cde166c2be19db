"""Front-end fixtures: transformers' CohereAsrFeatureExtractor (constructed without librosa, with the Slaney filter
bank), a seeded random-init ParakeetEncoderSubsamplingConv2D / ParakeetEncoder, synthetic audio, and the checker's
composition of the subsampling stem (the same steps as FastEncoder.subsample)."""

from __future__ import annotations

import numpy as np
import torch

import oracle
from bench import synthetic_audio  # noqa: F401  (config 4's audio, shared with the bench)
from helpers import bf16_bits


def slaney_filters() -> torch.Tensor:
    from kernels.features import slaney_mel_filters

    return slaney_mel_filters()


def hf_extractor(dither: float = 1e-5):
    """transformers' CohereAsrFeatureExtractor with its default settings. Its __init__ builds the filter bank with
    librosa, which this image lacks: the object is made without it and given the same filter bank (Slaney mel, pinned
    against transformers.audio_utils.mel_filter_bank in the tests)."""
    from transformers.feature_extraction_sequence_utils import SequenceFeatureExtractor
    from transformers.models.cohere_asr.feature_extraction_cohere_asr import CohereAsrFeatureExtractor

    fe = object.__new__(CohereAsrFeatureExtractor)
    SequenceFeatureExtractor.__init__(fe, feature_size=128, sampling_rate=16000, padding_value=0.0)
    for k, v in dict(hop_length=160, n_fft=512, win_length=400, preemphasis=0.97, dither=dither, max_audio_clip_s=35.0,
                     overlap_chunk_second=5.0, min_energy_window_samples=1600).items():
        setattr(fe, k, v)
    fe.mel_filters = slaney_filters()
    return fe


def window512() -> np.ndarray:
    w = np.zeros(512, np.float32)
    w[56:456] = torch.hann_window(400, periodic=False).numpy()
    return w


def bands(mel: np.ndarray) -> np.ndarray:
    nz = mel != 0
    first = nz.argmax(1)
    end = mel.shape[1] - nz[:, ::-1].argmax(1)
    return np.stack([first, np.where(nz.any(1), end, first)], 1).astype(np.int32)


def make_subsampling(seed: int = 3, channels: int = 256, hidden: int = 1280):
    """transformers' ParakeetEncoderSubsamplingConv2D (8x, 128 mel bins) with seeded weights, bf16-representable,
    float32 on the CPU."""
    from transformers.models.parakeet.configuration_parakeet import ParakeetEncoderConfig
    from transformers.models.parakeet.modeling_parakeet import ParakeetEncoderSubsamplingConv2D

    cfg = ParakeetEncoderConfig(hidden_size=hidden, subsampling_conv_channels=channels, num_mel_bins=128,
                                subsampling_factor=8, subsampling_conv_kernel_size=3, subsampling_conv_stride=2)
    sub = ParakeetEncoderSubsamplingConv2D(cfg).eval()
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sub.named_parameters():
            fan_in = p[0].numel() if p.dim() > 1 else 1
            scale = (1.0 / fan_in) ** 0.5 if p.dim() > 1 else 0.05
            p.copy_((torch.randn(p.shape, generator=g) * scale).to(torch.bfloat16).float())
    return sub


def stem_weights(sub):
    """The subsampling's weights as FastEncoder prepares them (fp32 convolution taps, bf16 pointwise / linear
    weights with the linear's input columns in channels-last order), as numpy (bf16 as bits)."""
    conv0, dw2, pw3, dw5, pw6 = (sub.layers[i] for i in (0, 2, 3, 5, 6))
    f32 = lambda t: t.detach().float().reshape(t.shape[0], -1).numpy().copy()  # noqa: E731
    bits = lambda t: bf16_bits(t.detach().to(torch.bfloat16))  # noqa: E731
    ch = pw6.out_channels
    out_f = sub.linear.in_features // ch
    lin = sub.linear.weight.detach().view(-1, ch, out_f).transpose(1, 2).reshape(-1, ch * out_f)
    vec = lambda t: t.detach().float().numpy().copy()  # noqa: E731
    return {"w0": f32(conv0.weight), "b0": vec(conv0.bias), "w2": f32(dw2.weight), "b2": vec(dw2.bias),
            "pw3": bits(pw3.weight[:, :, 0, 0]), "pw3_b": bits(pw3.bias),
            "w5": f32(dw5.weight), "b5": vec(dw5.bias), "pw6": bits(pw6.weight[:, :, 0, 0]),
            "pw6_b": bits(pw6.bias), "lin": bits(lin), "lin_b": bits(sub.linear.bias), "channels": ch}


def half(n):
    return [(t - 1) // 2 + 1 for t in n]


def stem_rows(ts):
    return np.array([(i, t) for i, n in enumerate(ts) for t in range(n)], np.int32).reshape(-1, 2)


def oracle_stem(W, feats_bits: np.ndarray, frames):
    """The checker's subsampling stem over padded features (B, T, 128) bf16 bits: packed (sum t3, hidden) bf16 bits
    and the lengths."""
    C = W["channels"]
    t2 = half(half(frames))
    t3 = half(t2)
    a2 = oracle.sub_conv0_dw(feats_bits, np.asarray(frames, np.int32), stem_rows(t2), W["w0"], W["b0"], W["w2"],
                             W["b2"])
    a3 = oracle.gemm_bf16(a2.reshape(-1, C), W["pw3"], W["pw3_b"], oracle.EPI_CONV_RELU).reshape(-1, 32, C)
    starts = np.concatenate([[0], np.cumsum(t2)[:-1]]).astype(np.int32)
    a5 = oracle.sub_dw(a3, starts, np.asarray(t2, np.int32), stem_rows(t3), W["w5"], W["b5"])
    a6 = oracle.gemm_bf16(a5.reshape(-1, C), W["pw6"], W["pw6_b"], oracle.EPI_CONV_RELU)
    return oracle.gemm_bf16(a6.reshape(len(a5), -1), W["lin"], W["lin_b"], oracle.EPI_BIAS), t3


def hf_stem(sub, feats: torch.Tensor, frames) -> torch.Tensor:
    """transformers' subsampling in float32, each piece on its own (its first frames[i] frames): packed output."""
    outs = []
    for i, n in enumerate(frames):
        x = feats[i:i + 1, :n].float()
        with torch.no_grad():
            outs.append(sub(x, torch.ones(1, n, dtype=torch.long))[0])
    return torch.cat(outs)


def make_encoder(layers: int, heads: int = 16, seed: int = 1, device="cpu", dtype=torch.float32):
    """transformers' ParakeetEncoder at config 2's width (1280, FFN 5120, depthwise kernel 9, 256 subsampling
    channels, no input scaling) with `layers` blocks: Xavier-uniform matrices, random biases / norms / BatchNorm
    statistics (as encoder_helpers.make_block), seeded, bf16-representable."""
    from transformers.models.parakeet.configuration_parakeet import ParakeetEncoderConfig
    from transformers.models.parakeet.modeling_parakeet import ParakeetEncoder

    cfg = ParakeetEncoderConfig(hidden_size=1280, num_attention_heads=heads, num_key_value_heads=heads,
                                intermediate_size=5120, num_hidden_layers=layers, conv_kernel_size=9,
                                subsampling_conv_channels=256, num_mel_bins=128, subsampling_factor=8,
                                scale_input=False, dropout=0.0, attention_dropout=0.0, activation_dropout=0.0,
                                dropout_positions=0.0, layerdrop=0.0)
    cfg._attn_implementation = "eager"
    with torch.device(device):
        enc = ParakeetEncoder(cfg).eval()
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in enc.named_parameters():
            if name.endswith(("bias_u", "bias_v")):
                p.copy_(torch.randn(p.shape, generator=g, device=device) * 0.2)
            elif p.dim() >= 2:
                torch.nn.init.xavier_uniform_(p, generator=g)
            elif "norm" in name and name.endswith("weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g, device=device))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g, device=device))
        for blk in enc.layers:
            bn = blk.conv.norm
            bn.running_mean.copy_(0.05 * torch.randn(bn.running_mean.shape, generator=g, device=device))
            bn.running_var.copy_(1.0 + 0.2 * torch.rand(bn.running_var.shape, generator=g, device=device))
        for p in enc.parameters():
            p.copy_(p.to(torch.bfloat16).float())
    return enc.to(dtype=dtype)
