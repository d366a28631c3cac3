"""The mask head after the stack on the gfx950 kernels: final RMSNorm, per-band MLP, GLU.

``HipMaskHead`` is the counterpart of the mask step of ``FastBSRoformer``: the weight grouping of its
constructor (src/turbo_roformer/fast.py:139-160), ``_mask`` (fast.py:349-360) and the final norm before it
(fast.py:385-387), i.e. ``MaskEstimator`` (model.py:158-178) with ``mask_estimator_depth`` 2.  Instead of
one batched ``baddbmm`` per group of equal-width bands, every band runs in one ``trf_mask_head`` launch;
the final norm's gamma is folded into the first Linear of every band when the weights are packed.

``precision``: ``"split"`` (default) forms each product from fp16 hi/lo parts (three MFMAs), which keeps
the mask within ~1e-6 of the reference's fp32 computation (its default ``mask_dtype``, fast.py:94);
``"fp16"`` uses one fp16 MFMA per product (~68 dB mask SNR against fp32), like the reference's reduced
``mask_dtype`` option.  There is no CPU fallback: construction raises ``HipUnavailable`` without the HIP
library or a gfx950 GPU.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

import torch

from . import _hip
from .weights import band_dims

Tensor = torch.Tensor


class HipMaskHead:
    """Final norm + mask estimator of a single-stem BS-RoFormer, one kernel launch per call."""

    def __init__(self, state_dict: Mapping[str, Tensor], cfg: Mapping[str, Any], device: str | torch.device = "cuda",
                 precision: str = "split"):
        if precision not in _hip.MASK_PRECISIONS:
            raise ValueError(f"precision must be one of {tuple(_hip.MASK_PRECISIONS)}, got {precision!r}")
        if cfg["dim"] != _hip.DIM:
            raise NotImplementedError(f"the kernels are built for dim {_hip.DIM}, got {cfg['dim']}")
        if cfg.get("mask_estimator_depth", 2) != 2:
            raise NotImplementedError("only mask_estimator_depth=2 is supported")  # as fast.py:150-151
        if cfg.get("num_stems", 1) != 1:
            raise NotImplementedError("only single-stem models are supported")
        _hip.load()
        self.device = torch.device(device)
        self.precision = precision
        self.dims = band_dims(cfg)
        self.hidden = cfg["dim"] * cfg.get("mlp_expansion_factor", 4)
        self.width = sum(self.dims)

        def dev(key: str) -> Tensor:
            return state_dict[key].detach().to(self.device, torch.float32).contiguous()

        bands = []
        for i in range(len(self.dims)):
            p = f"mask_estimators.0.to_freqs.{i}.0"
            bands.append((dev(f"{p}.0.weight"), dev(f"{p}.0.bias"), dev(f"{p}.2.weight"), dev(f"{p}.2.bias")))
        self.packed = torch.empty(_hip.mask_head_packed_bytes(self.dims, self.hidden), dtype=torch.uint8,
                                  device=self.device)
        _hip.pack_mask_head(bands, self.dims, self.hidden, dev("final_norm.gamma"), self.packed)

    @torch.no_grad()
    def __call__(self, X: Tensor, n_frames: int | None = None, out: Tensor | None = None) -> Tensor:
        """Stack output X [n_frames * bands, 256] (or [..., bands, 256]) fp32 on the device -> mask
        [n_frames, sum(dins)] fp32, band f at columns sum(dins[:f]) .. + dins[f]."""
        F = len(self.dims)
        if X.dim() > 2:
            if X.shape[-2] != F:
                raise ValueError(f"X has {X.shape[-2]} bands, the model {F}")
            X = X.reshape(-1, X.shape[-1])
        if n_frames is None:
            n_frames = X.shape[0] // F
        mask = out if out is not None else torch.empty(n_frames, self.width, dtype=torch.float32, device=X.device)
        _hip.mask_head(X, n_frames, self.dims, self.hidden, self.packed, mask, self.precision)
        return mask
