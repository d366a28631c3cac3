"""The Separator's backend and precision selection on a host with no usable GPU (this suite's CPU run):
the reference's rules (separator.py:26-27,134-158) restated for the hip backend."""

from __future__ import annotations

import logging

import pytest

from turbo_roformer_amd import _hip
from turbo_roformer_amd.separator import (
    REFERENCE_PRECISIONS,
    Separator,
    resolve_backend,
    resolve_precision,
)

no_gpu = pytest.mark.skipif(_hip.support()[0], reason="the fallback rules are checked where HIP cannot run")


@no_gpu
def test_auto_warns_and_leaves_the_fallback_to_the_caller(caplog):
    with caplog.at_level(logging.WARNING, logger="turbo_roformer_amd"):
        assert resolve_backend("auto") is None
    assert any("HIP backend unavailable" in r.getMessage() for r in caplog.records)


@no_gpu
def test_explicit_hip_raises():
    with pytest.raises(_hip.HipUnavailable):
        resolve_backend("hip")


@no_gpu
@pytest.mark.parametrize("backend", ["auto", "hip"])
def test_separator_has_no_cpu_path(tiny_sd, backend):
    from turbo_roformer_amd import weights

    with pytest.raises(_hip.HipUnavailable):
        Separator(tiny_sd, weights.TINY_CFG, weights.TINY_DIM_T, backend=backend)


def test_disabled_by_environment(monkeypatch):
    monkeypatch.setenv("TURBO_ROFORMER_DISABLE_HIP", "1")
    assert resolve_backend("auto") is None
    with pytest.raises(_hip.HipUnavailable, match="TURBO_ROFORMER_DISABLE_HIP"):
        resolve_backend("hip")


def test_unknown_backend_is_a_value_error():
    for bad in ("kernels", "torch", "cuda", ""):
        with pytest.raises(ValueError):
            resolve_backend(bad)


def test_reference_precisions_map_onto_stack_modes():
    assert set(REFERENCE_PRECISIONS) == {"bf16", "fp32"}  # the reference's PRECISIONS
    assert resolve_precision("bf16") == "ff_fp16"
    assert resolve_precision("fp32") == "ff_split"
    for mode in _hip.PRECISIONS:  # any stack arithmetic, the all-bf16 one included, by override
        assert resolve_precision("bf16", mode) == mode
    for bad in (("fp16", None), ("ff_fp16", None), ("bf16", "fp32")):
        with pytest.raises(ValueError):
            resolve_precision(*bad)
