"""Chunk schedule and Hamming-windowed overlap-add of a song, batched for the GPU stack.

The schedule and the window are the reference's (src/turbo_roformer/chunking.py:11-36): chunk starts at
multiples of step = floor(chunk / overlap), the last chunk aligned to the end of the signal, a
symmetric Hamming window, and the weighted sum normalised by the summed weights.  They have to be the
same, sample for sample, for a song to be split and recombined the way the reference does it.  What
differs is the execution: ``overlap_add`` hands every chunk of the song to ``run`` in batches (one
batched stack forward per batch) instead of one model call per chunk, and ``overlap_add_device`` does
the same with the song, the chunks, the predictions and the windowed sums on the GPU (``trf_overlap_add``,
bitwise the same sums as the host loop).
"""

from __future__ import annotations

from collections.abc import Callable

import numpy as np
import torch


def step_for(chunk: int, overlap: float) -> int:
    """Hop between chunk starts: floor(chunk / overlap), clamped to [1, chunk] (chunking.py:30-32)."""
    return max(1, min(chunk, int(chunk / overlap)))


def chunk_starts(n: int, chunk: int, step: int) -> list[int]:
    """Starts k*step while a chunk fits strictly inside the signal, then one chunk ending at n
    (never a zero-padded tail chunk; chunking.py:11-21)."""
    starts: list[int] = []
    for off in range(0, n, step):
        if off + chunk < n:
            starts.append(off)
            continue
        tail = max(n - chunk, 0)
        if not starts or starts[-1] != tail:
            starts.append(tail)
        break
    return starts


def hamming(n: int) -> np.ndarray:
    """Symmetric Hamming window 0.54 - 0.46 cos(2 pi k / (n-1)), float32; ones(1) for n = 1."""
    if n == 1:
        return np.ones(1, np.float32)
    k = np.arange(n, dtype=np.float64)
    return (0.54 - 0.46 * np.cos(2.0 * np.pi * k / (n - 1))).astype(np.float32)


def overlap_add(
    x: torch.Tensor,
    chunk: int,
    overlap: float,
    run: Callable[[torch.Tensor], torch.Tensor],
    batch: int = 0,
    progress: Callable[[int, int], None] | None = None,
) -> torch.Tensor:
    """x (2, n) -> (2, n) fp32 on the CPU.

    ``run`` maps a batch of chunks (b, 2, C) to predictions (b, 2, L) with L <= C.  ``batch`` chunks go to
    each call (0: all of them in one call).  Each prediction is weighted by the Hamming window and the sum
    is divided by the summed weights, so any overlap >= 1 crossfades chunks without seams.
    ``progress(k, n)`` is called after each chunk, with k counting up to the number of chunks n.
    """
    n = x.shape[1]
    C = min(chunk, n)
    starts = chunk_starts(n, C, step_for(C, overlap))
    w = torch.from_numpy(hamming(C))
    out = torch.zeros(2, n, dtype=torch.float32)
    wsum = torch.zeros(n, dtype=torch.float32)
    per = len(starts) if batch <= 0 else batch
    done = 0
    for b0 in range(0, len(starts), per):
        group = starts[b0 : b0 + per]
        y = run(torch.stack([x[:, s : s + C] for s in group]).contiguous()).float().cpu()
        L = min(C, y.shape[-1])
        for i, s in enumerate(group):
            out[:, s : s + L] += y[i, :, :L] * w[:L]
            wsum[s : s + L] += w[:L]
            done += 1
            if progress is not None:
                progress(done, len(starts))
    return out.div_(wsum.clamp_(min=1e-10))


def overlap_add_device(
    x: torch.Tensor,
    chunk: int,
    overlap: float,
    run: Callable[[torch.Tensor], torch.Tensor],
    batch: int = 0,
    progress: Callable[[int, int], None] | None = None,
    gain: float = 1.0,
) -> torch.Tensor:
    """``overlap_add`` with everything on the GPU: x (2, n) device -> (2, n) device, divided by ``gain``.

    The chunks are cut on the device, ``run`` returns device predictions, and ``trf_overlap_add``
    accumulates each batch in ascending chunk order with the host loop's fp32 roundings, so the result is
    bitwise that of ``overlap_add`` followed by ``div_(gain)``.
    """
    from . import _hip

    n = x.shape[1]
    C = min(chunk, n)
    starts = chunk_starts(n, C, step_for(C, overlap))
    dev = x.device
    w = torch.from_numpy(hamming(C)).to(dev)
    acc = torch.zeros(2, n, dtype=torch.float32, device=dev)
    wsum = torch.zeros(n, dtype=torch.float32, device=dev)
    per = len(starts) if batch <= 0 else batch
    for b0 in range(0, len(starts), per):
        group = starts[b0 : b0 + per]
        y = run(torch.stack([x[:, s : s + C] for s in group]).contiguous()).float().contiguous()
        L = min(C, y.shape[-1])
        _hip.overlap_add(y, L, group, w, acc, wsum)
        if progress is not None:
            for k in range(len(group)):
                progress(b0 + k + 1, len(starts))
    _hip.overlap_finish(acc, wsum, gain, acc)
    return acc
