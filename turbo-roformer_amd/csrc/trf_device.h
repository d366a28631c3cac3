// Device helpers shared by the kernel translation units (trf_kernels.hip, trf_mask.hip): operand
// vector types, the MFMA wrappers, fp16/bf16 packing and the direct-to-LDS weight streaming.
#pragma once

#include "trf_internal.h"

namespace trf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.44269504088896341f;

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma32h(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

// Two fp32 -> packed fp16 pair, round to nearest even.
__device__ __forceinline__ uint32_t pk_f16(float lo, float hi) {
  f16x2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }

// A zero splat: as the first accumulator of an MFMA chain it folds into the inline constant 0.
__device__ __forceinline__ f32x16 zero16() {
  f32x16 z = {};
  return z;
}

__device__ __forceinline__ u32x4 zero4() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return z;
}

// Feature offset of accumulator register group g (registers 4g..4g+3) of a 32-row tile.
__device__ __forceinline__ int row_of_group(int g, int hh) { return 8 * g + 4 * hh; }

// Token index of position p in sequence s (see the token-order contract in trf_hip.h).
__device__ __forceinline__ int64_t token_of(int mode, int s, int p, int T, int F) {
  if (mode == 0) {
    const int c = s / F, f = s - c * F;
    return (int64_t(c) * T + p) * F + f;
  }
  return int64_t(s) * F + p;
}

// max of x over lanes l and l ^ 32: v_permlane32_swap exchanges the half-waves, so of its two results
// one is x and the other the partner's value, in either order.
__device__ __forceinline__ float halfwave_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Index of this wave in the workgroup, as a scalar (uniform) value so that addresses derived from it
// stay in scalar registers.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ============================================================ LDS weight streaming
// Weights are packed as 1 KB operand blocks (one MFMA A operand: 64 lanes x 16 B).  A workgroup
// streams the blocks of one stage into LDS with direct global->LDS loads, double-buffered: while the
// waves compute on stage s from one buffer, the blocks of stage s+1 land in the other.
//
// The direct loads are buffer loads with an LDS destination (buffer_load_dwordx4 ... lds).  The compiler
// counts global_load_lds among the LDS operations, so after one it can only wait lgkmcnt(0) before an
// LDS read; after buffer loads it keeps exact lgkmcnt(n) waits for reads issued ahead of their use.
// Buffer loads are also bounds-checked against the resource's size (reads past it return zeros).
constexpr int kBufferRsrcWord3 = 0x00020000;  // word 3 of a gfx9 raw buffer descriptor

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferRsrcWord3);
}

// 16 bytes per lane from byte offset voff of buffer r into LDS at lds_base + 16 * lane (lds_base
// wave-uniform).
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, int voff, u32x4* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, voff, 0, 0,
                                           0);
}

// One operand block (src_block wave-uniform) into LDS.
__device__ __forceinline__ void lds_load_block(const u32x4* __restrict__ src_block, u32x4* lds_block, int lane) {
  buffer_load_lds16(buffer_rsrc(src_block, kTileBytes), lane * 16, lds_block);
}

// All of this thread's outstanding global loads (direct-to-LDS ones included) have landed, and every
// wave of the workgroup has reached this point.
__device__ __forceinline__ void stage_barrier() {
  // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15), as the builtin so that the compiler's own waitcnt
  // insertion knows every earlier global load has landed (an inline-asm wait is opaque to it, and it
  // would then wait again, for the next stage's loads too, at the first use of such a value).
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
}

// This thread's vector memory operations have completed except the N most recent, then all waves
// meet.  On gfx9 loads, direct-to-LDS loads and stores share the one vmcnt counter and complete in
// issue order, so a stage can leave its stores in flight and still wait for exactly the loads issued
// before them.  The barrier is the bare s_barrier: __syncthreads' release fence would wait for the N
// younger operations too.  The empty asm statements keep the compiler from moving LDS accesses across.
template <int N>
__device__ __forceinline__ void vmcnt_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);  // vmcnt(N) expcnt(7) lgkmcnt(15)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace trf
