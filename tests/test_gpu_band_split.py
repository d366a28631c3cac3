"""Band split on the GPU (trf_band_split through HipBandSplit) against the oracle.

* the reference's golden stack input (tests/golden/tiny_stack.npz, written by the reference's ``BandSplit``
  on its STFT features): the STFT features of the same audio, then the HIP band split, at 100 dB, the
  reference's fp32 parity bar (tests/test_parity.py:25);
* tiny model (29 bands of width 16..260) at frame counts 1, 33, 129 and 300 (partial 32-frame columns and
  128-frame workgroups), and the full-size model (62 bands of width 8..516) over one 17 s chunk of
  frames: against the fp64 oracle (``reference.band_split``) at >= 120 dB (fp32 arithmetic);
* an all-zero frame gives the bias exactly (the norm's max(|x|, 1e-12));
* the output is deterministic, and a frame's tokens do not depend on the other frames of the launch.
"""

from __future__ import annotations

import pytest
import torch

from oracle import reference
from turbo_roformer_amd import weights
from turbo_roformer_amd.band_split import HipBandSplit
from turbo_roformer_amd.host import HostPath

from .conftest import snr_db

pytestmark = pytest.mark.gpu

TINY = weights.TINY_CFG
FULL = weights.RESURRECTION_CFG


def _feats(n_frames: int, width: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    # spectra: a few large bins, most small, as STFT magnitudes are
    return torch.randn(n_frames, width, generator=g) * torch.rand(n_frames, width, generator=g).pow(4) * 50


def _oracle(feats: torch.Tensor, sd, cfg) -> torch.Tensor:
    """reference.band_split in fp64 on [frames, width] features -> [frames * bands, 256]."""
    dims = reference.band_dims(cfg)
    sdd = {k: v.double() for k, v in sd.items() if k.startswith("band_split")}
    out = []
    for i, part in enumerate(feats.double().split(dims, dim=-1)):
        pn = reference.rms_norm(part, sdd[f"band_split.to_features.{i}.0.gamma"])
        out.append(pn @ sdd[f"band_split.to_features.{i}.1.weight"].t() + sdd[f"band_split.to_features.{i}.1.bias"])
    return torch.stack(out, dim=-2).reshape(-1, 256)


def test_golden_stack_input(hip, tiny_sd):
    from .test_golden import _load

    g = _load("tiny_stack.npz")
    host = HostPath(tiny_sd, TINY)
    feats = host.spectrogram(torch.from_numpy(g["audio"]))  # (1, T, 1028), CPU torch STFT
    x = HipBandSplit(tiny_sd, TINY, "cuda")(feats.contiguous().cuda()).cpu()
    s = snr_db(g["tokens_in"], x.numpy())
    print(f"golden stack input (reference BandSplit): {s:.1f} dB")
    assert x.shape == g["tokens_in"].shape
    assert s >= 100.0


@pytest.mark.parametrize("n_frames", [1, 33, 129, 300])
def test_tiny_band_split_matches_oracle(hip, tiny_sd, n_frames):
    dims = weights.band_dims(TINY)
    feats = _feats(n_frames, sum(dims), seed=n_frames)
    print(f"tiny band split, {n_frames} frames", flush=True)
    got = HipBandSplit(tiny_sd, TINY, "cuda")(feats.cuda()).cpu()
    ref = _oracle(feats, tiny_sd, TINY)
    s = snr_db(ref.numpy(), got.numpy())
    print(f"  {s:.1f} dB")
    assert got.shape == (n_frames * len(dims), 256)
    assert s >= 120.0


@pytest.fixture(scope="module")
def full_sd():
    return weights.init_state_dict(FULL, seed=3, init="default", perturb=True)


def test_full_chunk_matches_oracle(hip, full_sd):
    dims = weights.band_dims(FULL)
    T = 1701
    feats = _feats(T, sum(dims), seed=5)
    feats[7] = 0.0  # a silent frame: every band's norm is 0, the output is the bias
    print(f"full-size band split, {T} frames", flush=True)
    bs = HipBandSplit(full_sd, FULL, "cuda")
    fd = feats.cuda()
    got = bs(fd).cpu()
    assert torch.equal(bs(fd).cpu(), got), "not deterministic"
    ref = _oracle(feats, full_sd, FULL)
    s = snr_db(ref.numpy(), got.numpy())
    print(f"  {s:.1f} dB")
    assert s >= 120.0
    F = len(dims)
    bias = torch.stack([full_sd[f"band_split.to_features.{i}.1.bias"] for i in range(F)])
    assert torch.equal(got.view(T, F, 256)[7], bias)
    for f in range(F):  # every band on its own
        assert snr_db(ref.view(T, F, 256)[:, f].numpy(), got.view(T, F, 256)[:, f].numpy()) >= 115.0, f"band {f}"
    part = bs(fd[1600:].contiguous()).cpu()
    assert torch.equal(part, got.view(T, F, 256)[1600:].reshape(-1, 256)), "depends on the other frames"


def test_shape_errors(hip, tiny_sd):
    bs = HipBandSplit(tiny_sd, TINY, "cuda")
    with pytest.raises(ValueError):
        bs(torch.zeros(10, 1000, device="cuda"))
    assert bs(torch.zeros(0, bs.width, device="cuda")).shape == (0, 256)
