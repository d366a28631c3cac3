"""Chunk schedule and windowed overlap-add of the song path: the reference's known answers
(tests/test_chunking.py of LoggeL/turbo-roformer) plus batching invariants."""

from __future__ import annotations

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
    C = min(1000, n)
    starts = chunk_starts(n, C, step_for(C, overlap))
    covered = np.zeros(n, bool)
    for s in starts:
        assert 0 <= s <= n - C
        covered[s : s + C] = True
    assert covered.all()
    assert starts == sorted(set(starts))


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


@pytest.mark.parametrize("overlap", [1.5, 2.0, 3.0])
def test_no_click_with_chunk_dependent_model(overlap):
    """Chunks that disagree (+-20 % gain) are crossfaded: with a DC input the output is the blend
    envelope, whose steps stay far below the 0.4 jump of a hard switch."""
    n, chunk = 100_000, 16000
    x = torch.ones(2, n)
    gains = iter([0.8, 1.2] * 100)
    y = overlap_add(x, chunk, overlap, lambda c: c * next(gains), batch=1).numpy()
    assert y.min() >= 0.8 - 1e-6 and y.max() <= 1.2 + 1e-6
    assert np.abs(np.diff(y, axis=1)).max() < 0.25 * 0.4
    hard = overlap_add(x, chunk, 1.0, lambda c: c * next(gains), batch=1).numpy()
    assert np.abs(np.diff(hard, axis=1)).max() > 0.39


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
