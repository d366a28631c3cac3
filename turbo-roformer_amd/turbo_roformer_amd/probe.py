"""Measurement probes (libtrf_probe.so, include/trf_probe.h): the sustained MFMA rate and HBM stream
bandwidth that the kernels' roofline figures are read against, and how much VALU work a SIMD issues beside
its MFMAs.  The counterpart of the reference's instruction-throughput benchmark
(benchmarks/dpbf16_peak.cpp); ``bench.py --mfma-peak --hbm-probe --coissue-probe`` runs them.  Not on the
stack's path."""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from ._hip import HipUnavailable, header_functions

LIB_PATH = Path(__file__).with_name("libtrf_probe.so")
HEADER_PATH = Path(__file__).resolve().parents[2] / "include" / "trf_probe.h"

_P, _I32, _I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
SIGNATURES: dict[str, tuple] = {
    "trf_probe_mfma_peak": (ctypes.c_int, [_I32, _I32, _I32, _P, _P]),
    "trf_probe_store": (ctypes.c_int, [_P, _I64, _I32, _I32, _I32, _P]),
    "trf_probe_load": (ctypes.c_int, [_P, _I64, _I32, _I32, _P, _P]),
    "trf_probe_coissue": (ctypes.c_int, [_I32, _I32, _I32, _I32, _P, _P]),
}
MFMA_FLOPS = 2 * 32 * 32 * 16  # one v_mfma_f32_32x32x16_bf16


def probe_functions() -> list[str]:
    return header_functions(HEADER_PATH)


def open_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    if not path.exists():
        raise HipUnavailable(f"{path.name} is not built (run `make -C turbo-roformer_amd/csrc`)")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def _time(fn, reps: int, warmup: int) -> float:
    """Mean ms of fn() over reps launches after warmup ones, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with code {rc}")


def mfma_peak(iters: int = 20000, reps: int = 5, warmup: int = 20) -> dict:
    """TFLOP/s of v_mfma_f32_32x32x16_bf16 on every SIMD: 1 or 2 waves per SIMD, 1-8 independent chains
    per wave, register operands (no LDS or memory traffic)."""
    lib = open_library()
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(2 * ncu * 4, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    res = {"cus": ncu, "iters": iters, "tflops": {}}
    for waves_per_simd in (1, 2):
        wg = waves_per_simd * ncu  # workgroups of 4 waves: one wave per SIMD each
        for chains in (1, 2, 4, 8):
            ms = _time(lambda: _check(lib.trf_probe_mfma_peak(chains, iters, wg, out.data_ptr(), st), "mfma probe"),
                       reps, warmup)
            flops = wg * 4 * chains * iters * MFMA_FLOPS
            res["tflops"][f"{waves_per_simd}w_{chains}c"] = round(flops / (ms * 1e-3) / 1e12, 1)
    res["best_tflops"] = max(res["tflops"].values())
    return res


def hbm_stream(nbytes: int = 1 << 30, reps: int = 10, warmup: int = 3) -> dict:
    """GB/s of load and store streams over nbytes (16-byte loads; 16- and 8-byte stores): contiguous and
    scattered 64-byte runs."""
    lib = open_library()
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    buf = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    wg = 16 * ncu
    res = {"bytes": nbytes, "gbs": {}}
    for scattered, name in ((0, "contiguous"), (1, "scattered_64B")):
        for width in (16, 8):
            ms = _time(lambda: _check(lib.trf_probe_store(buf.data_ptr(), nbytes, scattered, width, wg, st),
                                      "store probe"), reps, warmup)
            res["gbs"][f"store{width}_{name}"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        ms = _time(lambda: _check(lib.trf_probe_load(buf.data_ptr(), nbytes, scattered, wg, sink.data_ptr(), st),
                                  "load probe"), reps, warmup)
        res["gbs"][f"load_{name}"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    del buf
    return res


# trf_probe_coissue variants: (name, MFMAs per iteration, matrix-pipe cycles per iteration alone,
# VALU issue cycles per iteration alone: 4 per v_fma_f32)
COISSUE_STREAMS = (
    (0, "32x32x16, no VALU", 8, 256, 0),
    (1, "32x32x16 + 4 FMA each", 8, 256, 128),
    (2, "32x32x16 + 8 FMA each", 8, 256, 256),
    (3, "16x16x32, no VALU", 16, 256, 0),
    (4, "16x16x32 + 2 FMA each", 16, 256, 128),
    (5, "16x16x32 + 4 FMA each", 16, 256, 256),
)
SOFTMAX_TILE = (
    (6, "tile, row sum as fp32 adds"),
    (7, "tile, row sum on 16x16x32 MFMA (kernel)"),
    (8, "tile, MFMAs only"),
    (9, "tile, VALU only"),
    (10, "tile, exp2 replaced by a multiply"),
)
LDS_STREAM = (
    (11, "LDS 8 x 1 KB reads only"),
    (12, "LDS 8 x 1 KB reads, 1 MFMA each"),
    (13, "LDS 8 x 1 KB reads, 2 MFMAs each"),
)


def coissue(iters: int = 2000, reps: int = 3, warmup: int = 2) -> dict:
    """Cycles per iteration of the slowest wave (s_memtime in every wave; one workgroup per CU, so with
    two waves per SIMD this is the time the SIMD takes for one iteration of each) with one and two waves
    per SIMD: independent MFMA and v_fma_f32 streams in a fixed order, and one 64-key tile of the
    time-attention loop in five variants (1,024 cycles of matrix pipe per tile and wave)."""
    lib = open_library()
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.zeros(2 * 8 * ncu, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    res = {"cus": ncu, "cycles_per_iteration": {}}
    variants = [(v, n) for v, n, *_ in COISSUE_STREAMS] + list(SOFTMAX_TILE) + list(LDS_STREAM)
    for waves_per_simd in (1, 2):
        for v, name in variants:
            it = iters * 4 if v < 6 or v > 10 else iters
            for _ in range(reps + warmup):
                _check(lib.trf_probe_coissue(v, it, waves_per_simd, ncu, out.data_ptr(), st), "co-issue probe")
            torch.cuda.synchronize()
            cyc = out[: 2 * 4 * waves_per_simd * ncu].view(-1, 2)[:, 0].double()
            # the SIMD's time is its slower wave's: the pair is not served evenly (one wave runs ahead)
            res["cycles_per_iteration"][f"{waves_per_simd}w {name}"] = round(float(cyc.max()) / it, 1)
            res.setdefault("mean_over_waves", {})[f"{waves_per_simd}w {name}"] = round(float(cyc.mean()) / it, 1)
    # Two waves per SIMD run concurrently, so a wave's cycles per iteration are the SIMD's time for two
    # iterations.  In the heaviest streams the VALU is the bottleneck: that time is then two iterations'
    # VALU cycles plus the VALU issue time each MFMA takes away, (T - 2 valu) / (2 MFMAs).
    c = res["cycles_per_iteration"]
    res["valu_issue_cycles_per_mfma"] = {
        name: round((c[f"2w {name}"] - 2 * valu) / (2 * nmfma), 1)
        for v, name, nmfma, pipe, valu in COISSUE_STREAMS if v in (2, 5)}
    # LDS operand reads: 8 KB per wave and iteration, 4 or 8 waves per CU
    res["lds_bytes_per_cycle_per_cu"] = {
        f"{w}w {name}": round(8192 * 4 * w / c[f"{w}w {name}"], 1) for w in (1, 2) for v, name in LDS_STREAM}
    return res
