"""Song assembly on the GPU (``overlap_add_device``, trf_overlap_add / trf_overlap_finish) against the host
overlap-add, which restates the reference's loop (chunking.py:39-61) and whose schedule the reference's
known answers pin (tests/test_chunking.py): the device sums must be bitwise the host's.

``run`` is a deterministic function whose GPU and CPU results are identical (exact scalings and one fp32
add), and which shortens its output like the iSTFT does, so the two paths see the same predictions."""

from __future__ import annotations

import pytest
import torch

from turbo_roformer_amd import signals
from turbo_roformer_amd.chunking import chunk_starts, overlap_add, overlap_add_device, step_for

pytestmark = pytest.mark.gpu


def _run(short: int):
    def run(chunks: torch.Tensor) -> torch.Tensor:
        y = chunks * 0.5 + chunks.flip(-1) * 0.25
        return y[..., : y.shape[-1] - short] if short else y
    return run


@pytest.mark.parametrize("n,chunk,overlap,batch,short,gain", [
    (200_000, 30_000, 2.0, 0, 441, 1.0),      # many chunks, one batch, iSTFT-like shortening
    (200_000, 30_000, 4.0, 3, 0, 1.37),       # overlap 4, batches of 3, peak gain
    (200_000, 30_000, 1.0, 1, 100, 1.0),      # no overlap except the tail chunk
    (61_000, 30_000, 2.5, 2, 7, 2.5),
    (20_000, 30_000, 2.0, 0, 128, 1.0),       # shorter than one chunk: a single chunk of the whole song
], ids=["ov2", "ov4-b3-gain", "ov1-b1", "ov2.5-b2", "short-song"])
def test_device_overlap_add_is_bitwise_the_host_loop(hip, n, chunk, overlap, batch, short, gain):
    x = torch.from_numpy(signals.noise_mix(n, seed=n % 97))
    C = min(chunk, n)
    print(f"overlap-add n={n} chunk={chunk} overlap={overlap}: {len(chunk_starts(n, C, step_for(C, overlap)))} chunks",
          flush=True)
    want = overlap_add(x, chunk, overlap, _run(short), batch)
    if gain != 1.0:
        want.div_(gain)
    got = overlap_add_device(x.cuda(), chunk, overlap, _run(short), batch, gain=gain).cpu()
    assert got.shape == want.shape == (2, n)
    assert torch.equal(got, want)


def test_progress_counts_every_chunk(hip):
    x = torch.from_numpy(signals.noise_mix(100_000, seed=1)).cuda()
    seen = []
    overlap_add_device(x, 20_000, 2.0, _run(0), 3, progress=lambda k, m: seen.append((k, m)))
    m = len(chunk_starts(100_000, 20_000, step_for(20_000, 2.0)))
    assert seen == [(k, m) for k in range(1, m + 1)]
