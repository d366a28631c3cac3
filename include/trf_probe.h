/*
 * trf_probe.h - measurement probes of libtrf_probe.so (not on the stack's path).
 *
 * No counterpart in the C ABI of the reference's ops.  They play the part of the reference's
 * instruction-throughput benchmark (benchmarks/dpbf16_peak.cpp: the sustained vdpbf16ps rate of one
 * core), for the roofline figures of the MI355X kernels: the sustained rate of the MFMA the kernels use,
 * and HBM stream bandwidth in the access patterns they use.  bench.py --mfma-peak / --hbm-probe time them
 * with HIP events.  Return 0 on success, 1 for a bad argument, 3 for a launch error.
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

#ifdef __cplusplus
}
#endif

#endif
