"""Seeded synthetic audio for benchmarks and parity runs, and the SNR metric.

No audio files are available offline, so every workload is synthesised: a Gaussian + pink-noise mix
for single 17 s chunks, and pink noise plus a sine-sweep "vocal" for whole songs.
"""

from __future__ import annotations

import numpy as np


def pink_noise(n: int, rng: np.random.Generator) -> np.ndarray:
    """Unit-variance noise with a 1/f power spectrum (white noise shaped by 1/sqrt(f) in the FFT domain)."""
    if n < 2:
        return rng.standard_normal(n)
    spec = np.fft.rfft(rng.standard_normal(n))
    f = np.arange(spec.shape[0], dtype=np.float64)
    f[0] = 1.0
    x = np.fft.irfft(spec / np.sqrt(f), n)
    return x / (x.std() + 1e-12)


def _peak(x: np.ndarray, peak: float) -> np.ndarray:
    return (x * (peak / max(float(np.abs(x).max()), 1e-9))).astype(np.float32)


def noise_mix(n: int, seed: int = 0, channels: int = 2, peak: float = 0.5) -> np.ndarray:
    """(channels, n) float32: Gaussian + pink noise, scaled to ``peak`` (a 17 s benchmark chunk)."""
    rng = np.random.default_rng(seed)
    out = np.stack([0.3 * rng.standard_normal(n) + pink_noise(n, rng) for _ in range(channels)])
    return _peak(out, peak)


def song(seconds: float, sr: int = 44100, seed: int = 0, peak: float = 0.5) -> np.ndarray:
    """(2, n) float32: stereo pink noise plus a centre-panned sine sweep with vibrato (a synthetic song)."""
    rng = np.random.default_rng(seed)
    n = int(round(seconds * sr))
    t = np.arange(n, dtype=np.float64) / sr
    f = 220.0 * 2.0 ** (2.0 * np.sin(2 * np.pi * t / max(seconds, 1e-3)))  # sweeps 55 Hz .. 880 Hz
    phase = 2 * np.pi * np.cumsum(f) / sr + 0.02 * np.sin(2 * np.pi * 5.5 * t)
    voice = 0.6 * np.sin(phase) * (0.6 + 0.4 * np.sin(2 * np.pi * 0.3 * t))
    out = np.stack([0.5 * pink_noise(n, rng) + voice, 0.5 * pink_noise(n, rng) + voice])
    return _peak(out, peak)


def snr_db(ref, est) -> float:
    """10 log10(sum ref^2 / sum (ref - est)^2) in fp64 (the reference's metric, tests/conftest.py:97-100)."""
    ref = np.asarray(ref, np.float64)
    est = np.asarray(est, np.float64)
    return float(10 * np.log10((ref**2).sum() / max(((ref - est) ** 2).sum(), 1e-300)))
