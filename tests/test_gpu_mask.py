"""Mask head on the GPU (trf_mask_head through HipMaskHead) against the oracle.

* tiny model (29 bands of width 16..260, hidden 512), frame counts 1, 31, 33 and 200 (partial 32-frame
  columns and 128-frame workgroups): ``split`` against the fp64 oracle (final norm + mask estimator,
  model.py:158-178) at >= 100 dB, the reference's own fp32 parity bar (tests/test_parity.py:25);
  ``fp16`` against the fp64 oracle at >= 60 dB and against the emulation of its rounding points
  (oracle.kernels.mask_head) at >= 85 dB;
* the reference's golden mask (tests/golden/tiny_forward.npz, written by the reference's
  ``FastBSRoformer._mask``): oracle stack on the CPU, then the HIP mask head, at 100 dB;
* the full-size model (62 bands of width 8..516, hidden 1024; the 516 and 512 bands are split over
  three jobs each) at 150 frames against the fp64 oracle, and one full 17 s chunk (1701 frames): a frame's
  mask depends on that frame only, so rows of the full launch are checked against the oracle on those
  frames, and two batched chunks give the same rows as one;
* the output is deterministic, and n_frames = 0 writes nothing.
"""

from __future__ import annotations

import pytest
import torch

from oracle import kernels, reference
from turbo_roformer_amd import signals, weights
from turbo_roformer_amd.mask import HipMaskHead

from .conftest import snr_db

pytestmark = pytest.mark.gpu

TINY = weights.TINY_CFG
FULL = weights.RESURRECTION_CFG


def _x(n_frames: int, bands: int, seed: int, scale: float = 3.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return scale * torch.randn(1, n_frames, bands, 256, generator=g)


def _oracle(x: torch.Tensor, sd, cfg) -> torch.Tensor:
    return reference.mask_from_stack(x.double(), {k: v.double() for k, v in sd.items()}, cfg)[0]


@pytest.fixture(scope="module")
def tiny_heads(hip, tiny_sd):
    return {p: HipMaskHead(tiny_sd, TINY, "cuda", precision=p) for p in ("split", "fp16")}


@pytest.mark.parametrize("n_frames", [1, 31, 33, 200])
def test_tiny_mask_matches_oracle(tiny_heads, tiny_sd, n_frames):
    dims = weights.band_dims(TINY)
    x = _x(n_frames, len(dims), seed=n_frames)
    print(f"tiny mask head, {n_frames} frames", flush=True)
    ref = _oracle(x, tiny_sd, TINY).numpy()
    xd = x.reshape(-1, 256).cuda()
    got = {p: h(xd).cpu().numpy() for p, h in tiny_heads.items()}
    assert got["split"].shape == ref.shape == (n_frames, sum(dims))
    s_split, s_fp16 = snr_db(ref, got["split"]), snr_db(ref, got["fp16"])
    emu = kernels.mask_head(x[0], tiny_sd, dims, precision="fp16").numpy()
    s_emu = snr_db(emu, got["fp16"])
    print(f"  split {s_split:.1f} dB, fp16 {s_fp16:.1f} dB (vs its emulation {s_emu:.1f} dB)")
    assert s_split >= 100.0
    assert s_fp16 >= 60.0
    assert s_emu >= 85.0


def test_tiny_golden_mask(tiny_heads, tiny_sd):
    from .test_golden import _load

    g = _load("tiny_forward.npz")
    raw = torch.from_numpy(g["audio"])
    x = reference.stack(reference.stack_input(raw, tiny_sd, TINY), tiny_sd, TINY["depth"])  # (1, T, F, 256)
    got = tiny_heads["split"](x.reshape(-1, 256).contiguous().cuda()).cpu().numpy()
    assert got.shape == g["mask"].shape
    s = snr_db(g["mask"], got)
    print(f"golden mask (reference FastBSRoformer._mask): {s:.1f} dB")
    assert s >= 100.0


@pytest.fixture(scope="module")
def full_sd():
    return weights.init_state_dict(FULL, seed=3, init="default", perturb=True)


@pytest.fixture(scope="module")
def full_head(hip, full_sd):
    return HipMaskHead(full_sd, FULL, "cuda")


def test_full_model_mask_matches_oracle(full_head, full_sd):
    dims = weights.band_dims(FULL)
    x = _x(150, len(dims), seed=7)
    print("full-size mask head, 150 frames", flush=True)
    got = full_head(x.reshape(-1, 256).cuda()).cpu().numpy()
    ref = _oracle(x, full_sd, FULL).numpy()
    s = snr_db(ref, got)
    print(f"  split {s:.1f} dB")
    assert got.shape == (150, 4100)
    assert s >= 100.0
    lo = 0
    for f, d in enumerate(dims):  # every band (and every job of the split bands) on its own
        assert snr_db(ref[:, lo : lo + d], got[:, lo : lo + d]) >= 95.0, f"band {f}"
        lo += d


def test_full_chunk_rows_and_batching(full_head, full_sd):
    dims = weights.band_dims(FULL)
    T = 1701
    x = _x(2 * T, len(dims), seed=11)
    print("full-size mask head, two 1701-frame chunks", flush=True)
    xd = x.reshape(-1, 256).cuda()
    one = full_head(xd[: T * len(dims)]).cpu()
    both = full_head(xd).cpu()
    assert torch.isfinite(both).all()
    assert torch.equal(both[:T], one), "a frame's mask must not depend on the other frames of the launch"
    assert torch.equal(full_head(xd).cpu(), both), "not deterministic"
    rows = list(range(0, 40)) + list(range(T - 41, T + 3)) + list(range(2 * T - 30, 2 * T))
    ref = _oracle(x[:, rows], full_sd, FULL).numpy()
    s = snr_db(ref, both[rows].numpy())
    print(f"  {len(rows)} rows of the launch vs oracle: {s:.1f} dB")
    assert s >= 100.0


def test_zero_frames_and_errors(full_head):
    mask = torch.full((0, 4100), 7.0, device="cuda")
    full_head(torch.empty(0, 256, device="cuda"), 0, out=mask)
    torch.cuda.synchronize()
    with pytest.raises(ValueError):
        full_head(torch.empty(10, 256, device="cuda"), 10)  # 10 frames need 620 rows
    with pytest.raises(ValueError):
        HipMaskHead(weights.init_state_dict(TINY, seed=0), TINY, "cuda", precision="bf16")


def test_separator_uses_hip_mask_head(hip, tiny_sd):
    from turbo_roformer_amd.separator import Separator

    sep = Separator(tiny_sd, TINY, weights.TINY_DIM_T, "cuda")
    assert isinstance(sep.mask_head, HipMaskHead)
    raw = torch.from_numpy(signals.noise_mix(3000, seed=4))[None]
    out = sep.forward_chunks(raw)
    ref = reference.forward(raw, tiny_sd, TINY)
    s = snr_db(ref.numpy(), out.cpu().numpy())
    print(f"tiny chunk forward (HIP stack + HIP mask head) vs fp32 oracle: {s:.1f} dB")
    assert s >= 50.0
