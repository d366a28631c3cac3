"""Oracle and host path against golden vectors written by the reference module itself.

The fixtures in tests/golden/ were produced by make_golden.py from LoggeL/turbo-roformer's
``BSRoformer`` (model.py) and ``FastBSRoformer`` (fast.py, fp32 torch path) with this repository's seeded
tiny-model weights.  Threshold: the reference's own fp32 parity bar, 100 dB (tests/test_parity.py:25).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle import folded, reference
from turbo_roformer_amd import weights
from turbo_roformer_amd.host import HostPath

from .conftest import snr_db

GOLD = Path(__file__).resolve().parent / "golden"
CFG = weights.TINY_CFG


def _load(name):
    return np.load(GOLD / name, allow_pickle=False)


def test_seeded_weights_unchanged(tiny_sd):
    g = _load("tiny_weights_checksum.npz")
    keys = list(g["keys"])
    assert keys == sorted(tiny_sd)
    sums = np.array([float(tiny_sd[k].double().sum()) for k in keys])
    sumsq = np.array([float(tiny_sd[k].double().pow(2).sum()) for k in keys])
    np.testing.assert_allclose(sums, g["sums"], rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(sumsq, g["sumsq"], rtol=1e-9, atol=1e-9)
    assert int(g["n_params"]) == weights.param_count(CFG)


def test_reference_forward_and_mask(tiny_sd):
    g = _load("tiny_forward.npz")
    raw = torch.from_numpy(g["audio"])
    out = reference.forward(raw, tiny_sd, CFG)
    assert out.shape == g["output"].shape
    assert snr_db(g["output"], out.numpy()) >= 100.0
    mask = reference.complex_mask(raw, tiny_sd, CFG)[0]
    assert mask.shape == g["mask"].shape
    assert snr_db(g["mask"], mask.numpy()) >= 100.0


def test_stack_oracles(tiny_sd):
    g = _load("tiny_stack.npz")
    T, F = int(g["frames"]), int(g["bands"])
    x = torch.from_numpy(g["tokens_in"]).view(1, T, F, 256)
    ref = g["tokens_out"]
    assert snr_db(ref, reference.stack(x, tiny_sd, CFG["depth"]).reshape(-1, 256).numpy()) >= 100.0
    assert snr_db(ref, folded.stack(x, folded.fold(tiny_sd, CFG["depth"])).reshape(-1, 256).numpy()) >= 100.0


def test_host_band_split_matches_reference(tiny_sd):
    g = _load("tiny_stack.npz")
    host = HostPath(tiny_sd, CFG)
    x = host.band_split(host.spectrogram(torch.from_numpy(g["audio"])))
    assert snr_db(g["tokens_in"], x.reshape(-1, 256).numpy()) >= 100.0
