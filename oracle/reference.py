"""fp32 restatement of the reference BS-RoFormer forward (src/turbo_roformer/model.py) - test oracle.

Functional form over a state dict with the reference's keys; every function cites the reference lines
whose semantics it restates.  Used only by tests and the CPU baseline.
"""

from __future__ import annotations

import math
from collections.abc import Mapping
from typing import Any

import torch
import torch.nn.functional as F

Tensor = torch.Tensor


def rms_norm(x: Tensor, gamma: Tensor) -> Tensor:
    """x / max(|x|_2, 1e-12) * sqrt(dim) * gamma  (model.py:28-35; F.normalize eps on the norm)."""
    nrm = x.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    return x / nrm * math.sqrt(x.shape[-1]) * gamma


def rotary_angles(L: int, freqs: Tensor) -> Tensor:
    """fp32 angles [L, dim/2]: position p times frequency i (model.py:46-50, before repeat_interleave)."""
    pos = torch.arange(L, dtype=torch.float32)
    return pos[:, None] * freqs.float()[None, :]


def rotate(t: Tensor, ang: Tensor) -> Tensor:
    """Interleaved-pair rotation of the last axis by ``ang`` [L, dim/2], fp32 math (model.py:52-59).

    Pair (t[2i], t[2i+1]) -> (t[2i] cos - t[2i+1] sin, t[2i+1] cos + t[2i] sin).
    """
    tf = t.float()
    even, odd = tf[..., 0::2], tf[..., 1::2]
    c, s = ang.cos(), ang.sin()
    out = torch.empty_like(tf)
    out[..., 0::2] = even * c - odd * s
    out[..., 1::2] = odd * c + even * s
    return out.to(t.dtype)


def softmax_attention(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tensor:
    """softmax(q k^T * scale) v over the last two axes (F.scaled_dot_product_attention, model.py:107)."""
    s = (q @ k.transpose(-1, -2)) * scale
    s = s - s.amax(dim=-1, keepdim=True)
    p = s.exp()
    return (p / p.sum(dim=-1, keepdim=True)) @ v


def gelu_erf(x: Tensor) -> Tensor:
    """0.5 x (1 + erf(x / sqrt 2)): nn.GELU() default (model.py:69)."""
    return 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0)))


def attention(x: Tensor, sd: Mapping[str, Tensor], p: str, heads: int = 8, dim_head: int = 64) -> Tensor:
    """Attention.forward (model.py:99-111) for x (b, n, dim); ``p`` is the module prefix."""
    b, n, _ = x.shape
    xn = rms_norm(x, sd[f"{p}.norm.gamma"])
    qkv = xn @ sd[f"{p}.to_qkv.weight"].t()
    qkv = qkv.view(b, n, 3, heads, dim_head).permute(2, 0, 3, 1, 4)  # (3, b, h, n, d)
    ang = rotary_angles(n, sd[f"{p}.rotary_embed.freqs"])
    q, k, v = rotate(qkv[0], ang), rotate(qkv[1], ang), qkv[2]
    out = softmax_attention(q, k, v, dim_head**-0.5)  # (b, h, n, d)
    gates = xn @ sd[f"{p}.to_gates.weight"].t() + sd[f"{p}.to_gates.bias"]  # (b, n, h)
    out = out * gates.permute(0, 2, 1).unsqueeze(-1).sigmoid()
    out = out.permute(0, 2, 1, 3).reshape(b, n, heads * dim_head)
    return out @ sd[f"{p}.to_out.0.weight"].t()


def feed_forward(x: Tensor, sd: Mapping[str, Tensor], p: str) -> Tensor:
    """FeedForward.net (model.py:62-76): RMSNorm, Linear, GELU, Linear."""
    h = rms_norm(x, sd[f"{p}.net.0.gamma"]) @ sd[f"{p}.net.1.weight"].t() + sd[f"{p}.net.1.bias"]
    return gelu_erf(h) @ sd[f"{p}.net.4.weight"].t() + sd[f"{p}.net.4.bias"]


def transformer(x: Tensor, sd: Mapping[str, Tensor], p: str, depth: int = 1) -> Tensor:
    """Transformer.forward with norm_output=False (model.py:140-144): x = attn(x)+x; x = ff(x)+x."""
    for li in range(depth):
        x = attention(x, sd, f"{p}.layers.{li}.0") + x
        x = feed_forward(x, sd, f"{p}.layers.{li}.1") + x
    return x


def stack(x: Tensor, sd: Mapping[str, Tensor], depth: int) -> Tensor:
    """The axial loop of BSRoformer.forward (model.py:262-268) on x (b, t, bands, dim)."""
    b, nt, nb, d = x.shape
    for i in range(depth):
        x = x.transpose(1, 2).reshape(b * nb, nt, d)  # "b t f d -> (b f) t d"
        x = transformer(x, sd, f"layers.{i}.0")
        x = x.view(b, nb, nt, d).transpose(1, 2).reshape(b * nt, nb, d)  # "-> (b t) f d"
        x = transformer(x, sd, f"layers.{i}.1")
        x = x.view(b, nt, nb, d)
    return x


def _window(cfg: Mapping[str, Any]) -> Tensor:
    return torch.hann_window(cfg["stft_win_length"])


def _stft_kwargs(cfg: Mapping[str, Any]) -> dict[str, Any]:
    return dict(
        n_fft=cfg["stft_n_fft"],
        hop_length=cfg["stft_hop_length"],
        win_length=cfg["stft_win_length"],
        normalized=cfg.get("stft_normalized", False),
    )


def spectrogram(raw: Tensor, cfg: Mapping[str, Any]) -> Tensor:
    """STFT of (b, s, samples) -> real view (b, bins*s, frames, 2), bins outer (model.py:253-260)."""
    b, s, n = raw.shape
    spec = torch.view_as_real(
        torch.stft(raw.reshape(b * s, n), **_stft_kwargs(cfg), window=_window(cfg), return_complex=True)
    )
    _, nf, nt, _ = spec.shape
    return spec.view(b, s, nf, nt, 2).permute(0, 2, 1, 3, 4).reshape(b, nf * s, nt, 2)


def band_split(spec: Tensor, sd: Mapping[str, Tensor], dims: tuple[int, ...]) -> Tensor:
    """Per band RMSNorm + Linear on the (bin, channel, re/im) features of a frame (model.py:147-155, 260-261)."""
    b, fs, nt, _ = spec.shape
    x = spec.permute(0, 2, 1, 3).reshape(b, nt, fs * 2)
    out = []
    for i, part in enumerate(x.split(dims, dim=-1)):
        pn = rms_norm(part, sd[f"band_split.to_features.{i}.0.gamma"])
        out.append(pn @ sd[f"band_split.to_features.{i}.1.weight"].t() + sd[f"band_split.to_features.{i}.1.bias"])
    return torch.stack(out, dim=-2)


def mask_head(x: Tensor, sd: Mapping[str, Tensor], dims: tuple[int, ...], stem: int = 0) -> Tensor:
    """MaskEstimator (model.py:158-178): per band Linear, Tanh, Linear, GLU; concatenated -> (b, t, sum dims)."""
    outs = []
    for i, band in enumerate(x.unbind(dim=-2)):
        p = f"mask_estimators.{stem}.to_freqs.{i}.0"
        h = torch.tanh(band @ sd[f"{p}.0.weight"].t() + sd[f"{p}.0.bias"])
        o = h @ sd[f"{p}.2.weight"].t() + sd[f"{p}.2.bias"]
        a, g = o.chunk(2, dim=-1)
        outs.append(a * g.sigmoid())
    return torch.cat(outs, dim=-1)


def band_dims(cfg: Mapping[str, Any]) -> tuple[int, ...]:
    ch = 2 if cfg.get("stereo", False) else 1
    return tuple(2 * f * ch for f in cfg["freqs_per_bands"])


@torch.no_grad()
def stack_input(raw: Tensor, sd: Mapping[str, Tensor], cfg: Mapping[str, Any]) -> Tensor:
    """Band-split tokens (b, t, bands, dim) that enter the stack."""
    return band_split(spectrogram(raw.float(), cfg), sd, band_dims(cfg))


@torch.no_grad()
def mask_from_stack(x: Tensor, sd: Mapping[str, Tensor], cfg: Mapping[str, Any]) -> Tensor:
    """final_norm + mask estimator on stack output x (b, t, bands, dim) -> mask (b, t, bins*s*2) (model.py:269-271)."""
    x = rms_norm(x, sd["final_norm.gamma"])
    return mask_head(x, sd, band_dims(cfg))


@torch.no_grad()
def complex_mask(raw: Tensor, sd: Mapping[str, Tensor], cfg: Mapping[str, Any]) -> Tensor:
    """The mask the stack feeds: (b, frames, bins*channels*2) fp32 for input audio (b, 2, samples)."""
    x = stack(stack_input(raw, sd, cfg), sd, cfg["depth"])
    return mask_from_stack(x, sd, cfg)


@torch.no_grad()
def apply_mask(raw: Tensor, mask: Tensor, cfg: Mapping[str, Any]) -> Tensor:
    """Complex multiply with the spectrogram and iSTFT (model.py:272-278): (b, s, hop*(frames-1))."""
    b, s, _ = raw.shape
    spec = spectrogram(raw.float(), cfg)  # (b, f*s, t, 2)
    nfs, nt = spec.shape[1], spec.shape[2]
    m = mask.view(b, nt, nfs, 2).permute(0, 2, 1, 3)
    out = torch.view_as_complex(spec.contiguous()) * torch.view_as_complex(m.contiguous())
    out = out.view(b, nfs // s, s, nt).permute(0, 2, 1, 3).reshape(b * s, nfs // s, nt)
    audio = torch.istft(out, **_stft_kwargs(cfg), window=_window(cfg), return_complex=False)
    return audio.view(b, s, -1)


@torch.no_grad()
def forward(raw: Tensor, sd: Mapping[str, Tensor], cfg: Mapping[str, Any]) -> Tensor:
    """BSRoformer.forward (model.py:247-278) for one stem: (b, 2, samples) -> (b, 2, hop*(samples//hop))."""
    if raw.ndim == 2:
        raw = raw.unsqueeze(1)
    return apply_mask(raw, complex_mask(raw, sd, cfg), cfg)
