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

import logging
import threading
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

log = logging.getLogger("turbo_roformer_amd")

SR = 44100
PEAK = 0.9  # louder mixes are scaled to this peak before the model and back after (separator.py:25)
BACKENDS = ("auto", "hip")
# The reference's precision names (separator.py:27) and the stack arithmetic (a ``HipStack`` precision)
# each one selects here: "bf16", its fast kernels, is the fast mode (bf16 operands, fp16 ones in the two FF
# GEMMs: the speed of all-bf16 and >= 55 dB mask SNR); "fp32", its exact path, is the most accurate mode
# (split-bf16 FF operands).  ``Separator(stack_precision=...)`` picks any stack mode directly, including
# "bf16" (every operand bf16, the reference kernels' own arithmetic).
REFERENCE_PRECISIONS = {"bf16": "ff_fp16", "fp32": "ff_split"}
# Device memory a batch of chunks may take, as a fraction of what is free when the batch is planned.
BATCH_MEMORY_FRACTION = 0.5


def resolve_backend(backend: str = "auto") -> str | None:
    """``"hip"`` when the gfx950 kernels can run here.  When they cannot: ``backend="hip"`` raises
    ``HipUnavailable`` (like the reference's explicit ``backend="kernels"``, separator.py:147-149), and
    ``backend="auto"`` logs a warning and returns None, so that a caller with CPU backends of its own falls
    back to them (the reference's ``auto``, separator.py:150-151)."""
    if backend not in BACKENDS:
        raise ValueError(f"backend must be one of {BACKENDS}")
    ok, why = _hip.support()
    if ok:
        return "hip"
    if backend == "hip":
        raise _hip.HipUnavailable(why)
    log.warning("gfx950 HIP backend unavailable (%s)", why)
    return None


def resolve_precision(precision: str, override: str | None = None) -> str:
    """The stack arithmetic for the reference precision name ``precision`` ("bf16" or "fp32"), or
    ``override`` (a ``HipStack`` precision) when given."""
    if precision not in REFERENCE_PRECISIONS:
        raise ValueError(f"precision must be one of {tuple(REFERENCE_PRECISIONS)}, got {precision!r}")
    mode = REFERENCE_PRECISIONS[precision] if override is None else override
    _hip.precision_code(mode)  # ValueError for an unknown stack precision
    return mode


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
    frames per chunk (chunk = hop * (dim_t - 1)); ``precision``: the reference's ``"bf16"`` (default) or
    ``"fp32"``, mapped to a stack arithmetic by ``REFERENCE_PRECISIONS``; ``stack_precision``: a
    ``HipStack`` precision (``"ff_fp16"``, ``"ff_split"``, ``"bf16"``) that overrides the mapping;
    ``mask_precision``: ``"split"`` or ``"fp16"`` (see ``HipMaskHead``); ``batch_chunks``:
    chunks per batched stack forward: None (default) sizes batches to the free device memory (about 0.9 GB
    per 17 s chunk), 0 runs the whole song at once, k > 0 runs k at a time.
    ``backend``: ``"hip"`` or ``"auto"``; both raise ``HipUnavailable`` when the kernels cannot run, ``"auto"``
    after a warning (this package has no CPU path; ``resolve_backend`` is the non-raising check).

    ``separate`` and ``forward_chunks`` are serialised by a per-instance lock, as in the reference
    (separator.py:101,226): an instance owns one workspace, so concurrent calls wait for each other.  Work
    runs on the calling thread's current stream; a call also waits for the previous call's work on the
    device, so callers on different streams never share the workspace at the same time.
    """

    def __init__(self, state_dict: Mapping[str, torch.Tensor], cfg: Mapping[str, Any], dim_t: int,
                 device: str | torch.device = "cuda", precision: str = "bf16", backend: str = "auto",
                 batch_chunks: int | None = None, mask_precision: str = "split",
                 stack_precision: str | None = None):
        mode = resolve_precision(precision, stack_precision)
        if batch_chunks is not None and int(batch_chunks) < 0:
            raise ValueError("batch_chunks must be None, 0 or positive")
        if resolve_backend(backend) is None:
            raise _hip.HipUnavailable(_hip.support()[1])
        self.backend = "hip"
        self.precision = precision
        self.stack_precision = mode
        self.device = torch.device(device)
        self.hop = int(cfg["stft_hop_length"])
        self.chunk = self.hop * (int(dim_t) - 1)
        self.batch_chunks = None if batch_chunks is None else int(batch_chunks)
        self.host = HostPath(state_dict, cfg, self.device)
        self.band_split = HipBandSplit(state_dict, cfg, self.device)
        self.stack = HipStack(state_dict, self.device, self.stack_precision)
        self.mask_head = HipMaskHead(state_dict, cfg, self.device, mask_precision)
        self._lock = threading.Lock()
        self._last_done: torch.cuda.Event | None = None

    def n_chunks(self, n_samples: int, overlap: float = 2.0) -> int:
        """Number of chunks the song is cut into (separator.py:182-186)."""
        C = min(self.chunk, n_samples)
        return len(chunk_starts(n_samples, C, step_for(C, overlap)))

    def chunk_bytes(self, n_samples: int | None = None) -> int:
        """Device memory one chunk of ``n_samples`` (default: a whole chunk) takes in a batched forward:
        the stack workspace and residual stream, features, mask, spectrogram and audio buffers."""
        C = self.chunk if n_samples is None else min(self.chunk, int(n_samples))
        T = C // self.hop + 1
        F = len(self.band_split.dims)
        width = self.mask_head.width
        bins = self.host.stft_kw["n_fft"] // 2 + 1
        return (_hip.workspace_bytes(1, T, F) + 2 * T * F * _hip.DIM * 4 + 2 * T * width * 4
                + 3 * 2 * bins * T * 8 + 4 * 2 * C * 4)

    def batch_size(self, n_samples: int) -> int:
        """Chunks per batched forward for a song of ``n_samples`` (see ``batch_chunks``)."""
        if self.batch_chunks is not None:
            return self.batch_chunks
        free, _ = torch.cuda.mem_get_info(self.device)
        free += torch.cuda.memory_reserved(self.device) - torch.cuda.memory_allocated(self.device)
        return max(1, int(BATCH_MEMORY_FRACTION * free) // self.chunk_bytes(n_samples))

    @torch.inference_mode()
    def forward_chunks(self, chunks: torch.Tensor) -> torch.Tensor:
        """(b, 2, C) chunks -> (b, 2, hop * (frames - 1)) instrumental predictions, b chunks batched."""
        with self._lock:
            self._wait_previous()
            out = self._forward_chunks(chunks)
            self._mark_done()
            return out

    def _wait_previous(self) -> None:
        if self._last_done is not None:
            torch.cuda.current_stream(self.device).wait_event(self._last_done)

    def _mark_done(self) -> None:
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self._last_done = ev

    def _forward_chunks(self, chunks: torch.Tensor) -> torch.Tensor:
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
        with self._lock:
            self._wait_previous()
            out = self._separate_44k(x, float(overlap), progress)
            self._mark_done()
        return out

    def _separate_44k(self, x: np.ndarray, overlap: float, progress) -> np.ndarray:
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
        inst = overlap_add_device(xd, self.chunk, overlap, self._forward_chunks, self.batch_size(x.shape[1]),
                                  progress, gain)
        out = torch.empty(2, n0, dtype=torch.float32, pin_memory=True)
        out.copy_(inst[:, :n0])  # synchronous: the song is done when this returns
        return out.numpy()
