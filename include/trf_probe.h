/*
 * trf_probe.h - measurement probes of libtrf_probe.so (not on the stack's path).
 *
 * No counterpart in the C ABI of the reference's ops.  They play the part of the reference's
 * instruction-throughput benchmark (benchmarks/dpbf16_peak.cpp: the sustained vdpbf16ps rate of one
 * core), for the roofline figures of the MI355X kernels: the sustained rate of the MFMA the kernels use,
 * HBM stream bandwidth in the access patterns they use, and how much VALU work issues beside the MFMAs.
 * bench.py --mfma-peak / --hbm-probe / --coissue-probe run them.  Return 0 on success, 1 for a bad
 * argument, 3 for a launch error.
 */
#ifndef TRF_PROBE_H
#define TRF_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* `workgroups` workgroups of 4 waves; every wave runs `chains` (1, 2, 4 or 8) independent accumulator
 * chains of `iters` v_mfma_f32_32x32x16_bf16 each (32x32x16 = 32,768 flops), operands in registers.  out
 * (device fp32, 4 * workgroups) receives one checksum per wave. */
int trf_probe_mfma_peak(int32_t chains, int32_t iters, int32_t workgroups, float* out, void* stream);

/* Writes `bytes` (a multiple of 1024) at dst with stores of `width` bytes per lane (16 or 8):
 * scattered = 0 as one stream (each wave instruction 64 x width contiguous bytes), 1 as 64-byte runs
 * spread across the buffer (an instruction's runs bytes / 16 apart). */
int trf_probe_store(void* dst, int64_t bytes, int32_t scattered, int32_t width, int32_t workgroups,
                    void* stream);

/* Reads `bytes` at src with 16-byte loads in the same two patterns; out (device, 4 bytes) is only
 * written for one impossible checksum, so the loads are kept. */
int trf_probe_load(const void* src, int64_t bytes, int32_t scattered, int32_t workgroups, uint32_t* out,
                   void* stream);

/* `workgroups` workgroups (one per CU: each holds 96 KB of LDS) of 4 * waves_per_simd waves, so every
 * SIMD runs exactly waves_per_simd (1 or 2) waves; each wave runs `iters` iterations of one of these loops
 * and writes its cycle count (s_memtime) to out[2w] and a checksum to out[2w + 1] (device fp32,
 * 8 * waves_per_simd * workgroups; the checksum only keeps the work alive and need not be finite):
 *   0, 1, 2: 8 v_mfma_f32_32x32x16_bf16 on four accumulator chains, each followed by 0, 4 or 8
 *            independent v_fma_f32, in that exact order (256 cycles of matrix pipe per iteration);
 *   3, 4, 5: 16 v_mfma_f32_16x16x32_bf16, each followed by 0, 2 or 4 v_fma_f32 (256 cycles as well);
 *   6 .. 10: one 64-key tile of the time-attention loop (two 32-query tiles, K and V^T operands from
 *            LDS): 6 with the row sum as fp32 adds of e, 7 with it on v_mfma_f32_16x16x32_bf16 (the
 *            kernel's form), 8 MFMAs only, 9 VALU only (exp2, adds, packs), 10 as 6 with exp2 replaced by
 *            a multiply;
 *   11, 12, 13: 8 operand blocks of 1 KB read from LDS (ds_read_b128) per iteration: 11 reads only,
 *            12 each the A operand of one v_mfma_f32_32x32x16_bf16, 13 of two (two B operands). */
int trf_probe_coissue(int32_t variant, int32_t iters, int32_t waves_per_simd, int32_t workgroups, float* out,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif
