"""Shared test setup: import paths, the ``gpu`` marker, seeded models and inputs."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "turbo-roformer_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

from turbo_roformer_amd import weights  # noqa: E402
from turbo_roformer_amd.signals import snr_db  # noqa: E402,F401


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libtrf_hip.so")


@pytest.fixture(scope="session")
def tiny_sd():
    """Tiny structurally complete model (dim 256, 8x64 heads, depth 2), perturbed gains/biases."""
    return weights.init_state_dict(weights.TINY_CFG, seed=0)


@pytest.fixture(scope="session")
def hip():
    """The loaded library; GPU tests fail loudly (no skip) when it cannot be used."""
    from turbo_roformer_amd import _hip

    return _hip.load()


def rand_x(n: int, seed: int, scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return scale * torch.randn(n, 256, generator=g)


def assert_bf16_close(ref: torch.Tensor, out: torch.Tensor, what: str, rtol_steps: float = 2.0, min_snr: float = 50.0):
    """Elementwise within ``rtol_steps`` bf16 steps (2^-8 relative) of the reference plus one bf16 step of
    the reference's RMS (outputs that nearly cancel carry the error of their terms, not of their value),
    at most 1e-4 of the elements outside, plus an SNR floor."""
    r = ref.double().cpu()
    o = out.double().cpu()
    tol = rtol_steps * 2.0**-8 * r.abs() + 2.0**-8 * r.pow(2).mean().sqrt() + 1e-30
    bad = (o - r).abs() > tol
    s = snr_db(r.numpy(), o.numpy())
    assert int(bad.sum()) <= max(0, int(1e-4 * r.numel())), f"{what}: {int(bad.sum())} of {r.numel()} out of tolerance (snr {s:.1f} dB)"
    assert s >= min_snr, f"{what}: snr {s:.1f} dB < {min_snr}"


def np_ref(t: torch.Tensor) -> np.ndarray:
    return t.detach().double().cpu().numpy()
