"""The product's host path (STFT, band split, mask head, iSTFT) against the oracle's reference forward."""

from __future__ import annotations

import torch

from oracle import reference
from turbo_roformer_amd import signals, weights
from turbo_roformer_amd.host import HostPath

from .conftest import snr_db

CFG = weights.TINY_CFG


def test_host_path_matches_reference(tiny_sd):
    raw = torch.stack([torch.from_numpy(signals.noise_mix(5000, seed=s)) for s in (1, 2)])
    host = HostPath(tiny_sd, CFG)
    X = host.band_split(host.spectrogram(raw))
    Xr = reference.stack_input(raw, tiny_sd, CFG)
    assert X.shape == Xr.shape == (2, 5000 // 128 + 1, 29, 256)
    assert snr_db(Xr.numpy(), X.numpy()) >= 110
    m = host.mask(Xr)
    mr = reference.mask_from_stack(Xr, tiny_sd, CFG)
    assert snr_db(mr.numpy(), m.numpy()) >= 110
    audio = host.apply(raw, mr)
    ar = reference.apply_mask(raw, mr, CFG)
    assert audio.shape == ar.shape == (2, 2, 128 * (5000 // 128))
    assert snr_db(ar.numpy(), audio.numpy()) >= 110
