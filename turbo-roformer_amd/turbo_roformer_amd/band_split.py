"""The band split before the stack on the gfx950 kernels: per band, RMSNorm + Linear into 256-d tokens.

``HipBandSplit`` is the counterpart of ``BandSplit`` (model.py:147-155) as ``FastBSRoformer.forward`` applies
it to a chunk's STFT features (fast.py:372-380). Instead of one norm and one Linear per band, all bands run
in one ``trf_band_split`` launch, which writes the tokens straight into the stack's order. The norm's
gain and scale, ``gamma * sqrt(din)``, are folded into each band's weights at packing. The arithmetic is
fp32 (fp32 MFMA), as in the reference. There is no CPU fallback: construction raises ``HipUnavailable``
without the HIP library or a gfx950 GPU.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

import torch

from . import _hip
from .weights import band_dims

Tensor = torch.Tensor


class HipBandSplit:
    """Band split of a BS-RoFormer: spectral features [frames, sum(dins)] -> tokens [frames * bands, 256]."""

    def __init__(self, state_dict: Mapping[str, Tensor], cfg: Mapping[str, Any], device: str | torch.device = "cuda"):
        if cfg["dim"] != _hip.DIM:
            raise NotImplementedError(f"the kernels are built for dim {_hip.DIM}, got {cfg['dim']}")
        _hip.load()
        self.device = torch.device(device)
        self.dims = band_dims(cfg)
        self.width = sum(self.dims)

        def dev(key: str) -> Tensor:
            return state_dict[key].detach().to(self.device, torch.float32).contiguous()

        bands = [
            (dev(f"band_split.to_features.{i}.1.weight"), dev(f"band_split.to_features.{i}.1.bias"),
             dev(f"band_split.to_features.{i}.0.gamma"))
            for i in range(len(self.dims))
        ]
        self.packed = torch.empty(_hip.band_split_packed_bytes(self.dims), dtype=torch.uint8, device=self.device)
        _hip.pack_band_split(bands, self.dims, self.packed)

    @torch.no_grad()
    def __call__(self, feats: Tensor, out: Tensor | None = None) -> Tensor:
        """feats [..., frames, sum(dins)] fp32 on the device (the per-frame (bin, channel, re/im) features of
        the STFT) -> tokens [n_frames * bands, 256] fp32, token n * bands + f."""
        if feats.shape[-1] != self.width:
            raise ValueError(f"feats have {feats.shape[-1]} features per frame, the model {self.width}")
        feats = feats.reshape(-1, self.width)
        n_frames = feats.shape[0]
        X = out if out is not None else torch.empty(n_frames * len(self.dims), _hip.DIM, dtype=torch.float32,
                                                    device=feats.device)
        _hip.band_split(feats, n_frames, self.dims, self.packed, X)
        return X
