"""The C-ABI library loads without a GPU, exports every declared symbol, and validates arguments
before touching the device."""

from __future__ import annotations

import ctypes

import pytest

from turbo_roformer_amd import _hip


@pytest.fixture(scope="module")
def lib():
    return _hip.open_library()


def test_exports_every_declared_function(lib):
    names = _hip.header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_hip._SIGNATURES), "ctypes signatures out of sync with trf_hip.h"


def test_probe_library_exports_every_declared_function():
    from turbo_roformer_amd import probe

    plib = probe.open_library()
    names = probe.probe_functions()
    assert names and all(hasattr(plib, n) for n in names)
    assert set(names) == set(probe.SIGNATURES), "ctypes signatures out of sync with trf_probe.h"
    p = ctypes.c_void_p(256)
    assert plib.trf_probe_mfma_peak(3, 10, 1, p, None) == 1  # chains 1, 2, 4 or 8
    assert plib.trf_probe_store(p, 1000, 0, 16, 1, None) == 1  # not a multiple of 1 KB
    assert plib.trf_probe_store(p, 1024, 0, 4, 1, None) == 1  # 16- or 8-byte stores
    assert plib.trf_probe_load(p, 1024, 2, 1, p, None) == 1  # pattern 0 or 1
    assert plib.trf_probe_coissue(14, 10, 1, 1, p, None) == 1  # variants 0..13
    assert plib.trf_probe_coissue(0, 0, 1, 1, p, None) == 1  # at least one iteration
    assert plib.trf_probe_coissue(0, 10, 3, 1, p, None) == 1  # one or two waves per SIMD


def test_version_and_sizes(lib):
    assert lib.trf_abi_version() == _hip.ABI_VERSION
    assert [lib.trf_seq_pad(L) for L in (1, 62, 64, 65, 1700, 1701)] == [64, 64, 64, 128, 1728, 1728]
    assert lib.trf_layer_packed_bytes() % 256 == 0
    # bf16 W_qkvg (49 tiles of 32 rows), W_out, W1, W2 in 32x32 tiles, W_out and the hi and lo parts of
    # W1 and W2 in 16x16 tiles, fp16 W1 and W2 in 32x32 tiles, and the biases
    assert lib.trf_layer_packed_bytes() == (49 * 32 * 256 + 2 * 256 * 512 + 8 * 1024 * 256) * 2 + 256 + (1024 + 256) * 4
    # Q/K/Vt elements: time 62 bands x 8 heads x 1728 x 64; freq 1701 frames x 8 x 64 x 64
    assert lib.trf_seq_buffer_elems(0, 1, 1701, 62) == 62 * 8 * 1728 * 64
    assert lib.trf_seq_buffer_elems(1, 1, 1701, 62) == 1701 * 8 * 64 * 64
    ws = lib.trf_stack_workspace_bytes(1, 1701, 62)
    n = 1701 * 62
    # xn, O, G per token plus Q, K, Vt of the larger mode; the FF hidden activation needs no buffer
    assert ws >= n * (256 * 2 + 512 * 2 + 8 * 4) + 3 * 1701 * 8 * 64 * 64 * 2
    assert ws < n * (256 * 2 + 512 * 2 + 1024 * 2)  + 3 * 1701 * 8 * 64 * 64 * 2
    assert lib.trf_stack_workspace_bytes(29, 1701, 62) > 28 * ws


def test_argument_errors_need_no_device(lib):
    p = ctypes.c_void_p(256)  # aligned dummy pointer; argument checks reject before any launch
    assert lib.trf_attention(p, p, p, p, p, 5, 1, 8, 2, None) == 1
    assert b"mode" in lib.trf_last_error()
    assert lib.trf_attention(p, p, p, p, None, 0, 1, 8, 2, None) == 1
    assert b"O must not be NULL" in lib.trf_last_error()
    assert lib.trf_qkv_rope_gemm(p, p, p, 0, 0, 8, 2, p, p, p, p, None) == 1
    assert b"batch" in lib.trf_last_error()
    assert lib.trf_gemm_res_norm(p, 500, p, None, p, p, 10, 1e-12, None) == 1
    assert b"multiple of 16" in lib.trf_last_error()
    assert lib.trf_gemm_gelu(p, p, p, 100, p, 10, None) == 1
    assert b"multiple of 32" in lib.trf_last_error()
    assert lib.trf_pack_weight(p, 256, 24, p, None) == 1
    assert lib.trf_weight_packed_bytes(256, 512) == 8 * 32 * 1024
    assert lib.trf_weight_packed_bytes(96, 256) == 3 * 16 * 1024
    assert lib.trf_weight_packed_bytes(256, 24) == 0
    assert lib.trf_stack_forward(p, 1, 8, 2, None, None, 0, 0, None, None, p, 0, None) == 2
    assert b"workspace" in lib.trf_last_error()
    assert lib.trf_stack_forward(p, 1, 8, 2, None, None, 0, 7, None, None, p, 1 << 30, None) == 1
    assert b"precision" in lib.trf_last_error()
    assert lib.trf_ff_block(p, 1, 8, 2, p, 3, p, 1 << 30, None) == 1
    assert b"precision" in lib.trf_last_error()
    assert lib.trf_seq_buffer_elems(2, 1, 8, 2) == -1
    assert lib.trf_stack_workspace_bytes(0, 8, 2) == 0


def _dins(*d):
    return (ctypes.c_int32 * len(d))(*d)


def test_mask_head_packed_bytes(lib):
    from turbo_roformer_amd import weights

    def expect(dims, hidden):
        w = sum((hidden // 32) * (32 + 8 * ((d + 31) // 32)) * 1024 for d in dims)
        b1 = -(-(w + len(dims) * hidden * 4) // 256) * 256
        return b1 + sum(-(-(2 * 32 * ((d + 31) // 32) * 4) // 256) * 256 for d in dims)

    for cfg in (weights.RESURRECTION_CFG, weights.TINY_CFG):
        dims = weights.band_dims(cfg)
        hidden = cfg["dim"] * cfg["mlp_expansion_factor"]
        n = lib.trf_mask_head_packed_bytes(_dins(*dims), len(dims), hidden)
        assert n == expect(dims, hidden)
    # full-size model: W1 hi+lo (62 x 1 MB) and W2 hi+lo for 157 output pairs of 64 columns
    assert lib.trf_mask_head_packed_bytes(_dins(*weights.band_dims(weights.RESURRECTION_CFG)), 62, 1024) > 100 << 20


def test_mask_head_argument_errors_need_no_device(lib):
    p = ctypes.c_void_p(256)
    d = _dins(8, 16, 516)
    assert lib.trf_mask_head_packed_bytes(d, 3, 1000) == 0  # hidden not a multiple of 64
    assert b"hidden" in lib.trf_last_error()
    assert lib.trf_mask_head_packed_bytes(_dins(8, 18), 2, 1024) == 0  # width not a multiple of 4
    assert b"dins[1]" in lib.trf_last_error()
    assert lib.trf_mask_head_packed_bytes(d, 0, 1024) == 0
    assert lib.trf_mask_head_packed_bytes(_dins(*([16384] * 64)), 64, 1024) == 0  # 64 x 86 jobs > 192
    assert b"jobs" in lib.trf_last_error()
    assert lib.trf_mask_head(p, 10, 3, d, 1024, p, 2, p, None) == 1
    assert b"precision" in lib.trf_last_error()
    assert lib.trf_mask_head(p, -1, 3, d, 1024, p, 0, p, None) == 1
    assert lib.trf_mask_head(p, 10, 3, d, 1024, None, 0, p, None) == 1
    assert b"packed must not be NULL" in lib.trf_last_error()
    assert lib.trf_mask_head(None, 0, 3, d, 1024, None, 0, None, None) == 0  # nothing to do
    assert lib.trf_pack_mask_head(None, d, 3, 1024, p, p, None) == 1
    assert b"bands" in lib.trf_last_error()


def test_band_split_packed_bytes_and_errors(lib):
    from turbo_roformer_amd import weights

    dims = weights.band_dims(weights.RESURRECTION_CFG)
    # fp32 W' as (din / 2) k-pairs x 8 tiles x 64 lanes (= 256 x din floats) plus the bias per band
    assert lib.trf_band_split_packed_bytes(_dins(*dims), len(dims)) == 4 * 256 * (sum(dims) + len(dims))
    p = ctypes.c_void_p(256)
    assert lib.trf_band_split_packed_bytes(_dins(8, 18), 2) == 0
    assert b"dins[1]" in lib.trf_last_error()
    assert lib.trf_band_split_packed_bytes(_dins(8), 65) == 0
    assert b"n_bands" in lib.trf_last_error()
    assert lib.trf_band_split(p, -1, 1, _dins(8), p, p, None) == 1
    assert lib.trf_band_split(p, 4, 1, _dins(8), None, p, None) == 1
    assert b"packed must not be NULL" in lib.trf_last_error()
    assert lib.trf_band_split(None, 0, 1, _dins(8), None, None, None) == 0  # nothing to do
    assert lib.trf_pack_band_split(None, _dins(8), 1, p, None) == 1


def test_overlap_add_argument_errors_need_no_device(lib):
    p = ctypes.c_void_p(256)
    assert lib.trf_overlap_add(p, 3, 100, 0, p, p, 1000, p, p, None) == 1
    assert b"L must be" in lib.trf_last_error()
    assert lib.trf_overlap_add(p, 3, 100, 101, p, p, 1000, p, p, None) == 1
    assert lib.trf_overlap_add(p, 3, 100, 50, None, p, 1000, p, p, None) == 1
    assert lib.trf_overlap_add(None, 0, 100, 50, None, None, 1000, None, None, None) == 0  # nothing to do
    assert lib.trf_overlap_finish(p, p, 1000, 0.0, p, None) == 1
    assert b"gain" in lib.trf_last_error()
    assert lib.trf_overlap_finish(None, None, 0, 1.0, None, None) == 0
