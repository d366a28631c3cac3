"""Model hyper-parameters and seeded synthetic weights in the reference's state-dict layout.

The parameter names and shapes are those of the lucidrains / python-audio-separator BS-RoFormer
module tree that LoggeL/turbo-roformer keeps loadable with ``strict=True``
(src/turbo_roformer/model.py:79-245, key list in tests/test_model.py:12-28).  Nothing here
downloads weights: the generators below stand in for the real checkpoint, which is unavailable
offline.
"""

from __future__ import annotations

import math
from typing import Any

import torch

# Band layout of the reference model (model.py:25): 62 bands over 1025 STFT bins.
DEFAULT_FREQS_PER_BANDS: tuple[int, ...] = (2,) * 24 + (4,) * 12 + (12,) * 8 + (24,) * 8 + (48,) * 8 + (128, 129)

# Hyper-parameters of "BS Roformer Instrumental Resurrection" (registry.py:49-69).
RESURRECTION_CFG: dict[str, Any] = dict(
    dim=256,
    depth=12,
    stereo=True,
    num_stems=1,
    time_transformer_depth=1,
    freq_transformer_depth=1,
    linear_transformer_depth=0,
    freqs_per_bands=DEFAULT_FREQS_PER_BANDS,
    dim_head=64,
    heads=8,
    dim_freqs_in=1025,
    stft_n_fft=2048,
    stft_hop_length=441,
    stft_win_length=2048,
    stft_normalized=False,
    mask_estimator_depth=2,
    mlp_expansion_factor=4,
)
RESURRECTION_HOP = 441
RESURRECTION_DIM_T = 1700  # chunk = hop * (dim_t - 1) = 749,259 samples (registry.py:84-85)

# Small but structurally complete model of the reference test-suite (tests/conftest.py:14-33).
TINY_CFG: dict[str, Any] = dict(
    dim=256,
    depth=2,
    stereo=True,
    num_stems=1,
    time_transformer_depth=1,
    freq_transformer_depth=1,
    freqs_per_bands=(4,) * 16 + (8,) * 8 + (16,) * 4 + (65,),
    dim_head=64,
    heads=8,
    dim_freqs_in=257,
    stft_n_fft=512,
    stft_hop_length=128,
    stft_win_length=512,
    mask_estimator_depth=2,
    mlp_expansion_factor=2,
)
TINY_HOP = 128
TINY_DIM_T = 128


def band_dims(cfg: dict[str, Any]) -> tuple[int, ...]:
    """Input width of each band: bins x channels x (re, im) (model.py:239)."""
    ch = 2 if cfg.get("stereo", False) else 1
    return tuple(2 * f * ch for f in cfg.get("freqs_per_bands", DEFAULT_FREQS_PER_BANDS))


def rotary_freqs(dim_head: int = 64, theta: float = 10000.0) -> torch.Tensor:
    """fp32 rotary frequencies theta^(-2i/dim), i < dim/2 (model.py:41-44)."""
    return 1.0 / (theta ** (torch.arange(0, dim_head, 2)[: dim_head // 2].float() / dim_head))


def param_shapes(cfg: dict[str, Any]) -> dict[str, tuple[int, ...]]:
    """Every state-dict key of the model with its shape (shared rotary freqs listed per layer)."""
    dim, heads, dh = cfg["dim"], cfg.get("heads", 8), cfg.get("dim_head", 64)
    inner = heads * dh
    ff = dim * 4
    shapes: dict[str, tuple[int, ...]] = {}
    for i in range(cfg["depth"]):
        for m, depth_key in ((0, "time_transformer_depth"), (1, "freq_transformer_depth")):
            for li in range(cfg.get(depth_key, 2)):
                p = f"layers.{i}.{m}.layers.{li}"
                shapes[f"{p}.0.rotary_embed.freqs"] = (dh // 2,)
                shapes[f"{p}.0.norm.gamma"] = (dim,)
                shapes[f"{p}.0.to_qkv.weight"] = (3 * inner, dim)
                shapes[f"{p}.0.to_gates.weight"] = (heads, dim)
                shapes[f"{p}.0.to_gates.bias"] = (heads,)
                shapes[f"{p}.0.to_out.0.weight"] = (dim, inner)
                shapes[f"{p}.1.net.0.gamma"] = (dim,)
                shapes[f"{p}.1.net.1.weight"] = (ff, dim)
                shapes[f"{p}.1.net.1.bias"] = (ff,)
                shapes[f"{p}.1.net.4.weight"] = (dim, ff)
                shapes[f"{p}.1.net.4.bias"] = (dim,)
    shapes["final_norm.gamma"] = (dim,)
    dims = band_dims(cfg)
    for b, d in enumerate(dims):
        shapes[f"band_split.to_features.{b}.0.gamma"] = (d,)
        shapes[f"band_split.to_features.{b}.1.weight"] = (dim, d)
        shapes[f"band_split.to_features.{b}.1.bias"] = (dim,)
    hidden = dim * cfg.get("mlp_expansion_factor", 4)
    if cfg.get("mask_estimator_depth", 2) != 2:
        raise NotImplementedError("only mask_estimator_depth=2 is supported")
    for s in range(cfg.get("num_stems", 1)):
        for b, d in enumerate(dims):
            p = f"mask_estimators.{s}.to_freqs.{b}.0"
            shapes[f"{p}.0.weight"] = (hidden, dim)
            shapes[f"{p}.0.bias"] = (hidden,)
            shapes[f"{p}.2.weight"] = (2 * d, hidden)
            shapes[f"{p}.2.bias"] = (2 * d,)
    return shapes


def init_state_dict(
    cfg: dict[str, Any], seed: int = 0, init: str = "default", perturb: bool = True
) -> dict[str, torch.Tensor]:
    """Seeded fp32 weights for every key of ``param_shapes(cfg)``.

    ``init="default"``: nn.Linear's default bounds U(+-1/sqrt(fan_in)) for weights and biases, unit norm gains.
    ``init="normal"``: Linear weights ~ N(0, 0.02), zero biases, unit gains.
    ``perturb``: gains := 1 + 0.25 N(0,1) and biases := 0.05 N(0,1) so that weight folding is exercised
    (the reference's test fixture does the same, tests/conftest.py:49-58).
    Rotary frequencies are always the fixed theta=10000 values.
    """
    if init not in ("default", "normal"):
        raise ValueError("init must be 'default' or 'normal'")
    g = torch.Generator().manual_seed(int(seed))
    freqs = rotary_freqs(cfg.get("dim_head", 64))
    sd: dict[str, torch.Tensor] = {}
    for key, shape in param_shapes(cfg).items():
        if key.endswith("rotary_embed.freqs"):
            sd[key] = freqs.clone()
        elif key.endswith("gamma"):
            t = torch.ones(shape)
            if perturb:
                t = 1.0 + 0.25 * torch.randn(shape, generator=g)
            sd[key] = t
        elif key.endswith("bias"):
            if perturb:
                t = 0.05 * torch.randn(shape, generator=g)
            elif init == "default":
                fan_in = _fan_in(key, cfg)
                t = (torch.rand(shape, generator=g) * 2 - 1) / math.sqrt(fan_in)
            else:
                t = torch.zeros(shape)
            sd[key] = t
        else:  # Linear weight (out, in)
            if init == "default":
                sd[key] = (torch.rand(shape, generator=g) * 2 - 1) / math.sqrt(shape[1])
            else:
                sd[key] = 0.02 * torch.randn(shape, generator=g)
    return sd


def _fan_in(bias_key: str, cfg: dict[str, Any]) -> int:
    return param_shapes(cfg)[bias_key[: -len("bias")] + "weight"][1]


def param_count(cfg: dict[str, Any]) -> int:
    """Number of distinct parameters (the shared rotary freqs counted once per axis)."""
    n = 0
    for key, shape in param_shapes(cfg).items():
        if key.endswith("rotary_embed.freqs"):
            continue
        n += math.prod(shape)
    return n + 2 * (cfg.get("dim_head", 64) // 2)
