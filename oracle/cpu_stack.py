"""AVX512-BF16 CPU stack (oracle/cpu_stack.cpp) through ctypes - TEST INFRASTRUCTURE and the CPU baseline.

A kernel-class CPU restatement of the restructured stack (src/turbo_roformer/fast.py:222-266) in the
reference's CPU kernel numerics (bf16 operands, fp32 accumulators and residual, docs/how-it-works.md:164-170),
built after the reference's published kernel design (docs/how-it-works.md:120-151) in this repository's own
C++.  ``bench.py`` times it as the same-host CPU baseline; ``tests/test_cpu_stack.py`` checks it against
``folded.stack`` (fp32).  Needs an x86-64 CPU with AVX512-BF16 (``avx512_bf16`` in /proc/cpuinfo).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import torch

Tensor = torch.Tensor
_DIR = Path(__file__).resolve().parent
LIB = _DIR / "libtrf_cpu_stack.so"
_lib = None


class CpuStackUnavailable(RuntimeError):
    pass


def cpu_flags() -> set[str]:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def supported() -> bool:
    return {"avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512_bf16"} <= cpu_flags()


def build() -> Path:
    """Compile the library with oracle/Makefile (g++, a few seconds)."""
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return LIB


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not supported():
        raise CpuStackUnavailable("this CPU has no AVX512-BF16")
    if not LIB.exists():
        build()
    lib = ctypes.CDLL(str(LIB))
    fp = ctypes.POINTER(ctypes.c_float)
    lib.trfc_new.argtypes = [ctypes.c_int]
    lib.trfc_new.restype = ctypes.c_void_p
    lib.trfc_free.argtypes = [ctypes.c_void_p]
    lib.trfc_free.restype = None
    lib.trfc_set_layer.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int] + [fp] * 8
    lib.trfc_set_layer.restype = ctypes.c_int
    lib.trfc_forward.argtypes = [ctypes.c_void_p, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.trfc_forward.restype = ctypes.c_int
    lib.trfc_phase_seconds.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double)]
    lib.trfc_phase_seconds.restype = ctypes.c_int
    _lib = lib
    return lib


def _fp(t: Tensor):
    return ctypes.cast(t.data_ptr(), ctypes.POINTER(ctypes.c_float))


PHASES = ("norm", "qkv", "attention", "out_proj", "ff1", "ff2")

_SHAPES = {"W": (1544, 256), "b": (1544,), "Wo": (256, 512), "W1": (1024, 256), "b1": (1024,), "W2": (256, 1024),
           "b2": (256,), "freqs": (32,)}


class CpuStack:
    """The stack over folded sub-layers (``folded.fold``): X (b, T, F, 256) fp32 -> a new tensor."""

    def __init__(self, layers: list[dict], threads: int | None = None):
        self.lib = load()
        self.threads = int(threads or torch.get_num_threads() or os.cpu_count() or 1)
        self.h = self.lib.trfc_new(len(layers))
        if not self.h:
            raise ValueError(f"bad sub-layer count {len(layers)}")
        for i, P in enumerate(layers):
            ts = {}
            for key, shape in _SHAPES.items():
                t = P[key].detach().to("cpu", torch.float32).contiguous()
                if tuple(t.shape) != shape:
                    raise ValueError(f"sub-layer {i} {key}: shape {tuple(t.shape)}, expected {shape}")
                ts[key] = t
            rc = self.lib.trfc_set_layer(self.h, i, int(P["mode"]), *(_fp(ts[k]) for k in _SHAPES))
            if rc:
                raise ValueError(f"sub-layer {i}: trfc_set_layer returned {rc}")

    def __del__(self):
        h, self.h = getattr(self, "h", None), None
        if h:
            self.lib.trfc_free(h)

    def phase_seconds(self) -> dict[str, float]:
        """Wall seconds per phase, summed over every forward of this stack."""
        out = (ctypes.c_double * len(PHASES))()
        self.lib.trfc_phase_seconds(self.h, out)
        return dict(zip(PHASES, out))

    def __call__(self, X: Tensor, threads: int | None = None) -> Tensor:
        if X.ndim != 4 or X.shape[-1] != 256:
            raise ValueError(f"X must be (b, T, F, 256), got {tuple(X.shape)}")
        out = X.detach().to("cpu", torch.float32).contiguous().clone()
        b, T, F, _ = out.shape
        if out.numel() == 0:
            return out
        rc = self.lib.trfc_forward(self.h, _fp(out), b, T, F, int(threads or self.threads))
        if rc:
            raise RuntimeError(f"trfc_forward returned {rc}")
        return out
