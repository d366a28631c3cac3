"""The measurement probes of libtrf_probe.so on the GPU: they run, and the co-issue harness (one workgroup
per CU, cycle counts from s_memtime) reads what the instructions take on their own."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def plib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from turbo_roformer_amd import probe

    return probe.open_library()


def _cycles(plib, variant: int, iters: int, waves_per_simd: int) -> torch.Tensor:
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.zeros(2 * 4 * waves_per_simd * ncu, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for _ in range(2):  # the second launch is the measured one
        assert plib.trf_probe_coissue(variant, iters, waves_per_simd, ncu, out.data_ptr(), st) == 0
    torch.cuda.synchronize()
    pairs = out.view(-1, 2).cpu()  # (cycles, checksum) per wave; checksums only keep the work alive
    assert torch.isfinite(pairs[:, 0]).all() and (pairs[:, 0] > 0).all()
    return pairs[:, 0].double() / iters


def test_mfma_stream_takes_its_pipe_cycles(plib):
    """8 v_mfma_f32_32x32x16_bf16 per iteration on four chains are 256 cycles of matrix pipe: one wave per
    SIMD takes about that, two waves (the SIMD's time for one iteration of each) about twice that."""
    print("co-issue probe: MFMA stream, 1 and 2 waves per SIMD", flush=True)
    one = _cycles(plib, 0, 2000, 1)
    two = _cycles(plib, 0, 2000, 2)
    assert (one > 0).all() and (two > 0).all()
    assert 240.0 <= float(one.max()) <= 320.0, float(one.max())
    assert 480.0 <= float(two.max()) <= 640.0, float(two.max())


def test_valu_beside_mfma_costs_issue_cycles(plib):
    """Eight FMAs after each MFMA do not fit beside it with one wave per SIMD (it takes longer than the MFMAs
    alone), four nearly do; the attention tile with its MFMAs alone is faster than with its softmax."""
    print("co-issue probe: FMAs beside MFMAs, attention tile", flush=True)
    base = float(_cycles(plib, 0, 2000, 1).max())
    four = float(_cycles(plib, 1, 2000, 1).max())
    eight = float(_cycles(plib, 2, 2000, 1).max())
    assert base <= four < eight, (base, four, eight)
    mfma_only = float(_cycles(plib, 8, 500, 2).max())
    kernel_form = float(_cycles(plib, 7, 500, 2).max())
    assert 2048.0 <= mfma_only < kernel_form, (mfma_only, kernel_form)


def test_lds_reads_stream(plib):
    """Reading 8 KB per wave and iteration from LDS with 8 waves per CU takes at least 64 KB / 256 B = 256
    cycles, and feeding the reads to MFMAs takes at least the MFMAs' 512 cycles."""
    print("probe: LDS operand streaming", flush=True)
    reads = float(_cycles(plib, 11, 2000, 2).max())
    with_mfma = float(_cycles(plib, 12, 2000, 2).max())
    assert 250.0 <= reads < with_mfma, (reads, with_mfma)
    assert with_mfma >= 500.0, with_mfma
