"""Song separation with the transformer stack on the GPU: the ``Separator`` of the reference, hip backend.

Mirrors ``turbo_roformer.Separator.separate`` (src/turbo_roformer/separator.py:182-232): the mix is made
stereo, short inputs are padded to whole hops, loud mixes are scaled to a 0.9 peak and back, and the song
is cut into chunks of hop * (dim_t - 1) samples at ``overlap`` predictions per sample and recombined
with a Hamming-windowed overlap-add (on the GPU, ``trf_overlap_add``: bitwise the reference's sums).  The difference is where a chunk's forward runs: STFT and iSTFT
stay in PyTorch (``HostPath``, on the same device); for a whole batch of chunks, the band split is one
``trf_band_split`` launch, the 24-sub-layer stack one ``trf_stack_forward`` call and the mask head one
``trf_mask_head`` launch on the gfx950 kernels, the tokens staying on the device throughout.  There is no CPU fallback: if the HIP library or the GPU is missing, construction raises
``HipUnavailable``.

Out of scope here: audio files, resampling (the reference uses soxr, absent from this image) and
surround downmix; ``separate`` takes mono or stereo float arrays at 44.1 kHz.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from typing import Any

import numpy as np
import torch

from . import _hip
from .chunking import chunk_starts, overlap_add_device, step_for
from .band_split import HipBandSplit
from .host import HostPath
from .mask import HipMaskHead
from .stack import HipStack

SR = 44100
PEAK = 0.9  # louder mixes are scaled to this peak before the model and back after (separator.py:25)
BACKENDS = ("auto", "hip")


def as_stereo(mix) -> np.ndarray:
    """(samples,) or (channels, samples) float -> (2, samples) float32; mono is duplicated."""
    a = np.asarray(mix)
    if a.dtype.kind != "f":
        raise ValueError(f"expected a floating point array (got dtype {a.dtype}); scale integer PCM to [-1, 1] first")
    if a.ndim == 1:
        a = a[None, :]
    elif a.ndim != 2:
        raise ValueError(f"expected (channels, samples) or (samples,), got shape {a.shape}")
    if a.shape[0] == 0 or a.shape[1] == 0:
        raise ValueError("empty input")
    if a.shape[0] > 2:
        raise ValueError(f"got {a.shape[0]} channels: only mono or stereo input is supported here")
    a = a.astype(np.float32, copy=False)
    if not np.isfinite(a).all():
        raise ValueError("input contains NaN or inf samples")
    return np.ascontiguousarray(np.repeat(a, 2, axis=0) if a.shape[0] == 1 else a)


class Separator:
    """Instrumental separation of single-stem stereo BS-RoFormer models, stack on the GPU.

    ``state_dict``/``cfg``: the model's weights (reference key names) and hyper-parameters; ``dim_t``:
    frames per chunk (chunk = hop * (dim_t - 1)); ``precision``: ``"ff_fp16"``, ``"ff_split"`` or ``"bf16"`` (see
    ``HipStack``); ``mask_precision``: ``"split"`` or ``"fp16"`` (see ``HipMaskHead``); ``batch_chunks``:
    chunks per batched stack forward (0 = the whole song at once).
    ``backend``: ``"hip"``, or ``"auto"`` which is the same here (both raise ``HipUnavailable`` when the
    kernels cannot run, like the reference's explicit ``backend="kernels"``, separator.py:147-149).
    """

    def __init__(self, state_dict: Mapping[str, torch.Tensor], cfg: Mapping[str, Any], dim_t: int,
                 device: str | torch.device = "cuda", precision: str = "ff_fp16", backend: str = "auto",
                 batch_chunks: int = 0, mask_precision: str = "split"):
        if backend not in BACKENDS:
            raise ValueError(f"backend must be one of {BACKENDS}")
        ok, why = _hip.support()
        if not ok:
            raise _hip.HipUnavailable(why)
        self.backend, self.precision = "hip", precision
        self.device = torch.device(device)
        self.hop = int(cfg["stft_hop_length"])
        self.chunk = self.hop * (int(dim_t) - 1)
        self.batch_chunks = int(batch_chunks)
        self.host = HostPath(state_dict, cfg, self.device)
        self.band_split = HipBandSplit(state_dict, cfg, self.device)
        self.stack = HipStack(state_dict, self.device, precision)
        self.mask_head = HipMaskHead(state_dict, cfg, self.device, mask_precision)

    def n_chunks(self, n_samples: int, overlap: float = 2.0) -> int:
        """Number of chunks the song is cut into (separator.py:182-186)."""
        C = min(self.chunk, n_samples)
        return len(chunk_starts(n_samples, C, step_for(C, overlap)))

    @torch.inference_mode()
    def forward_chunks(self, chunks: torch.Tensor) -> torch.Tensor:
        """(b, 2, C) chunks -> (b, 2, hop * (frames - 1)) instrumental predictions, b chunks batched."""
        raw = chunks.to(self.device, torch.float32)
        st = self.host.stft(raw)  # (b * 2, bins, T) complex, reused for the mask multiply
        feats = self.host.features(st, raw.shape[0])  # (b, T, bins * 2 * 2)
        b, T = feats.shape[:2]
        F = len(self.band_split.dims)
        Xd = self.band_split(feats.contiguous())  # (b * T * F, 256)
        self.stack(Xd, b, T, F)
        mask = self.mask_head(Xd, b * T).view(b, T, -1)
        return self.host.apply(raw, mask, st)

    @torch.inference_mode()
    def separate(self, mix, sr: int = SR, overlap: float = 2.0,
                 progress: Callable[[int, int], None] | None = None) -> np.ndarray:
        """Instrumental (2, samples) float32 of a mono or stereo mix at 44.1 kHz (separator.py:203-232)."""
        if not overlap >= 1.0:
            raise ValueError("overlap must be >= 1")
        if int(sr) != SR:
            raise NotImplementedError("only 44.1 kHz input is supported (resampling needs soxr)")
        x = as_stereo(mix)
        n0 = x.shape[1]
        if n0 < self.chunk and (n0 % self.hop or n0 < 3 * self.hop):
            # the iSTFT returns hop * (n // hop) samples: pad to whole hops, and to 3 hops at least
            target = max(-(-n0 // self.hop) * self.hop, 3 * self.hop)
            x = np.pad(x, ((0, 0), (0, target - n0)))
        peak = float(np.abs(x).max())
        gain = PEAK / peak if peak > PEAK else 1.0
        xt = torch.from_numpy(np.ascontiguousarray(x * np.float32(gain) if gain != 1.0 else x))
        # the song goes to the GPU once; chunks, predictions and the windowed sums stay there
        xd = xt.pin_memory().to(self.device, non_blocking=True)
        inst = overlap_add_device(xd, self.chunk, overlap, self.forward_chunks, self.batch_chunks, progress, gain)
        out = torch.empty(2, n0, dtype=torch.float32, pin_memory=True)
        out.copy_(inst[:, :n0])
        return out.numpy()
