"""Chunk schedule and windowed overlap-add of the song path: the reference's known answers
(tests/test_chunking.py of LoggeL/turbo-roformer) plus batching invariants."""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from turbo_roformer_amd.chunking import chunk_starts, hamming, overlap_add, step_for
from turbo_roformer_amd.separator import as_stereo


def test_schedule_of_a_4min12_song():
    # 4:12 at 44.1 kHz with the 749,259-sample chunk and overlap 2 (the reference's example)
    n, chunk = 11130532, 749259
    starts = chunk_starts(n, chunk, step_for(chunk, 2))
    assert step_for(chunk, 2) == 374629
    assert len(starts) == 29
    assert starts[:3] == [0, 374629, 749258]
    assert starts[-1] == n - chunk
    # the benchmark song: 252 s, 17 s chunks of 749,700 samples -> also 29 chunks
    assert len(chunk_starts(252 * 44100, 749700, step_for(749700, 2))) == 29


def test_schedule_against_brute_force():
    """Every start k*step whose chunk ends before n, then the chunk that ends at n."""
    for n in (1, 5, 999, 1000, 1001, 5000, 12345):
        for chunk in (7, 1000):
            for overlap in (1.0, 1.5, 2.0, 3.0):
                C = min(chunk, n)
                step = step_for(C, overlap)
                want = [k * step for k in range(n) if k * step + C < n]
                if not want or want[-1] != n - C:
                    want.append(n - C)
                assert chunk_starts(n, C, step) == want


@pytest.mark.parametrize("n", [1, 100, 999, 1000, 1001, 5000, 12345])
@pytest.mark.parametrize("overlap", [1.0, 1.5, 2.0, 3.0])
def test_schedule_covers_signal(n, overlap):
    """Chunks lie inside the signal, starts strictly increase, and the per-sample chunk count (a
    difference array summed up) is at least one everywhere."""
    C = min(1000, n)
    starts = np.asarray(chunk_starts(n, C, step_for(C, overlap)))
    assert (starts >= 0).all() and (starts + C <= n).all()
    assert (np.diff(starts) > 0).all()
    delta = np.zeros(n + 1, np.int64)
    np.add.at(delta, starts, 1)
    np.add.at(delta, starts + C, -1)
    assert np.cumsum(delta)[:n].min() >= 1


def test_hamming_matches_numpy():
    for n in (1, 2, 7, 1000):
        np.testing.assert_allclose(hamming(n), np.hamming(n), rtol=0, atol=1e-6)
    assert hamming(1000).min() > 0.07


@pytest.mark.parametrize("n", [700, 1000, 4321, 10007])
@pytest.mark.parametrize("overlap", [1.0, 1.5, 2.0, 3.0])
@pytest.mark.parametrize("batch", [0, 1, 3])
def test_identity_model_reconstructs_input(n, overlap, batch):
    x = torch.randn(2, n, generator=torch.Generator().manual_seed(n))
    y = overlap_add(x, 1000, overlap, lambda c: c, batch)
    torch.testing.assert_close(y, x, rtol=0, atol=1e-5)


def test_batches_see_every_chunk_once_in_order():
    seen = []

    def run(c):
        seen.append(c.shape[0])
        return c

    x = torch.randn(2, 10007)
    n = len(chunk_starts(10007, 1000, 500))
    overlap_add(x, 1000, 2.0, run, batch=4)
    assert sum(seen) == n and all(b <= 4 for b in seen)
    calls = []
    overlap_add(x, 1000, 2.0, lambda c: c, batch=3, progress=lambda k, m: calls.append((k, m)))
    assert calls == [(k, n) for k in range(1, n + 1)]


def _alternating_gain_model():
    """A 'model' that scales chunk k by 0.8 (k even) or 1.2 (k odd): neighbouring chunks disagree by 0.4."""
    k = itertools.count()
    return lambda c: c * (0.8 if next(k) % 2 == 0 else 1.2)


@pytest.mark.parametrize("overlap", [1.5, 2.0, 3.0])
def test_disagreeing_chunks_are_crossfaded(overlap):
    """On a constant input the windowed sum glides between the two gains; without overlap the output
    jumps by their whole difference at each seam."""
    n, chunk = 100_000, 16000
    ones = torch.ones(2, n)
    y = overlap_add(ones, chunk, overlap, _alternating_gain_model(), batch=1).numpy()
    assert y.min() >= 0.8 - 1e-6 and y.max() <= 1.2 + 1e-6
    hard = overlap_add(ones, chunk, 1.0, _alternating_gain_model(), batch=1).numpy()
    hard_jump = np.abs(np.diff(hard, axis=1)).max()
    assert hard_jump == pytest.approx(0.4, abs=0.01)
    assert np.abs(np.diff(y, axis=1)).max() < hard_jump / 4


def test_device_overlap_add_checks_starts_on_the_host():
    """The GPU overlap-add finds a sample's chunks by binary search over the starts: its wrapper rejects
    starts that are unsorted, repeated or reach outside the song before anything is uploaded."""
    from turbo_roformer_amd._hip import check_chunk_starts

    assert check_chunk_starts([0, 5, 9], 3, 4, 13) == [0, 5, 9]
    assert check_chunk_starts(torch.tensor([0, 5]), 2, 4, 9) == [0, 5]
    for starts, nc, L, n in (([5, 0, 9], 3, 4, 13), ([0, 0], 2, 4, 13), ([0, 5], 3, 4, 13), ([-1, 5], 2, 4, 13),
                             ([0, 10], 2, 4, 13)):
        with pytest.raises(ValueError):
            check_chunk_starts(starts, nc, L, n)


def test_as_stereo():
    mono = np.linspace(-1, 1, 11, dtype=np.float32)
    assert np.array_equal(as_stereo(mono), np.stack([mono, mono]))
    st = np.random.default_rng(0).standard_normal((2, 9)).astype(np.float64)
    out = as_stereo(st)
    assert out.dtype == np.float32 and out.shape == (2, 9)
    for bad in (np.zeros((2, 4), np.int16), np.zeros((0, 4), np.float32), np.full((2, 3), np.nan, np.float32),
                np.zeros((3, 4), np.float32), np.zeros((2, 2, 2), np.float32)):
        with pytest.raises(ValueError):
            as_stereo(bad)
