"""Host path around the stack: STFT, band split, iSTFT (and a torch mask head).

These stay in PyTorch (CPU by default, any torch device works), as in ``FastBSRoformer.forward``
(src/turbo_roformer/fast.py:363-394).  Everything is computed from a state dict with the reference's keys,
in fp32.  ``HostPath.mask`` is the reference's grouped-``baddbmm`` mask head in torch; the ``Separator``
runs the mask head on the gfx950 kernels instead (``HipMaskHead``).
"""

from __future__ import annotations

import math
from collections.abc import Mapping
from typing import Any

import torch

from .weights import band_dims

Tensor = torch.Tensor


class HostPath:
    """fp32 STFT / band split / mask head of one single-stem stereo BS-RoFormer."""

    def __init__(self, state_dict: Mapping[str, Tensor], cfg: Mapping[str, Any], device: str | torch.device = "cpu"):
        if not (cfg.get("stereo") and cfg.get("num_stems", 1) == 1):
            raise NotImplementedError("only single-stem stereo BS-RoFormer models are supported")
        self.cfg = dict(cfg)
        self.device = torch.device(device)
        self.dim = cfg["dim"]
        self.dims = band_dims(cfg)
        sd = {k: v.detach().float().to(self.device) for k, v in state_dict.items()}
        self.stft_kw = dict(
            n_fft=cfg["stft_n_fft"], hop_length=cfg["stft_hop_length"], win_length=cfg["stft_win_length"],
            normalized=cfg.get("stft_normalized", False),
        )
        self.window = torch.hann_window(cfg["stft_win_length"], device=self.device)
        scale = math.sqrt(self.dim)
        # band split: 16*gamma of each band's RMSNorm folded into that band's Linear (norm scale sqrt(din))
        self.split = []
        for i, d in enumerate(self.dims):
            g = sd[f"band_split.to_features.{i}.0.gamma"] * math.sqrt(d)
            self.split.append(
                (sd[f"band_split.to_features.{i}.1.weight"] * g[None, :], sd[f"band_split.to_features.{i}.1.bias"])
            )
        self.final_g = sd["final_norm.gamma"] * scale
        # mask head: consecutive bands of equal width share one batched MLP (fast.py:139-160)
        self.groups = []
        i, off = 0, 0
        while i < len(self.dims):
            j = i
            while j < len(self.dims) and self.dims[j] == self.dims[i]:
                j += 1
            p = [f"mask_estimators.0.to_freqs.{k}.0" for k in range(i, j)]
            self.groups.append(
                dict(
                    i0=i, i1=j, din=self.dims[i], off=off,
                    W1=torch.stack([sd[f"{q}.0.weight"].t() for q in p]).contiguous(),
                    b1=torch.stack([sd[f"{q}.0.bias"] for q in p]).unsqueeze(1).contiguous(),
                    W2=torch.stack([sd[f"{q}.2.weight"].t() for q in p]).contiguous(),
                    b2=torch.stack([sd[f"{q}.2.bias"] for q in p]).unsqueeze(1).contiguous(),
                )
            )
            off += self.dims[i] * (j - i)
            i = j
        self.mask_width = off

    # -------------------------------------------------------------------------------------- forward parts
    @torch.no_grad()
    def stft(self, raw: Tensor) -> Tensor:
        """(b, 2, n) -> complex STFT (b*2, bins, frames) of the mixture."""
        b, s, n = raw.shape
        return torch.stft(raw.reshape(b * s, n).float().to(self.device), **self.stft_kw, window=self.window,
                          return_complex=True)

    @staticmethod
    def features(st: Tensor, b: int) -> Tensor:
        """Complex STFT (b*2, bins, frames) -> real features (b, frames, bins*2*2), ordered (bin, channel,
        re/im) per frame."""
        r = torch.view_as_real(st)  # (b*s, bins, T, 2)
        bs, nb, T = r.shape[0], r.shape[1], r.shape[2]
        s = bs // b
        return r.view(b, s, nb, T, 2).permute(0, 3, 2, 1, 4).reshape(b, T, nb * s * 2)

    @torch.no_grad()
    def spectrogram(self, raw: Tensor) -> Tensor:
        """(b, 2, n) -> real STFT (b, frames, bins*2*2) with per-frame features ordered (bin, channel, re/im)."""
        return self.features(self.stft(raw), raw.shape[0])

    @torch.no_grad()
    def band_split(self, feats: Tensor) -> Tensor:
        """(b, T, features) -> stack input tokens (b, T, bands, dim), fp32 (model.py:147-155)."""
        out = []
        for part, (W, bias) in zip(feats.split(self.dims, dim=-1), self.split):
            pn = part / part.norm(dim=-1, keepdim=True).clamp_min(1e-12)
            out.append(torch.addmm(bias, pn.reshape(-1, pn.shape[-1]), W.t()).view(*pn.shape[:-1], self.dim))
        return torch.stack(out, dim=-2)

    @torch.no_grad()
    def mask(self, X: Tensor) -> Tensor:
        """Stack output (b, T, bands, dim) -> mask (b, T, mask width) fp32 (fast.py:349-360, 385-387)."""
        b, T, nbands, d = X.shape
        Xn = X.to(self.device) / X.norm(dim=-1, keepdim=True).clamp_min(1e-12).to(self.device) * self.final_g
        Xt = Xn.permute(2, 0, 1, 3).reshape(nbands, b * T, d)  # (bands, b*T, d)
        mask = torch.empty(b * T, self.mask_width, dtype=torch.float32, device=self.device)
        for g in self.groups:
            h = torch.baddbmm(g["b1"], Xt[g["i0"] : g["i1"]], g["W1"]).tanh_()
            o = torch.baddbmm(g["b2"], h, g["W2"])
            din = g["din"]
            o = o[..., :din] * o[..., din:].sigmoid()
            nb = g["i1"] - g["i0"]
            mask[:, g["off"] : g["off"] + nb * din] = o.transpose(0, 1).reshape(b * T, nb * din)
        return mask.view(b, T, self.mask_width)

    @torch.no_grad()
    def apply(self, raw: Tensor, mask: Tensor, st: Tensor | None = None) -> Tensor:
        """Complex-multiply the mask into the mixture STFT and invert: (b, 2, hop*(frames-1)).  ``st``: the
        mixture's complex STFT if already computed (``stft(raw)``)."""
        b, s, n = raw.shape
        if st is None:
            st = self.stft(raw)  # (b*s, bins, T)
        nb, T = st.shape[1], st.shape[2]
        m = torch.view_as_complex(mask.reshape(b, T, nb, s, 2).permute(0, 3, 2, 1, 4).contiguous())  # (b, s, bins, T)
        out = torch.istft(st * m.reshape(b * s, nb, T), **self.stft_kw, window=self.window, return_complex=False)
        return out.view(b, s, -1)
