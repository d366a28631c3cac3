// Measurement probes for the roofline figures of the stack's kernels (libtrf_probe.so, include/trf_probe.h):
// the sustained rate of v_mfma_f32_32x32x16_bf16 with register operands, the HBM bandwidth of plain
// streams of 16-byte loads or stores in two access patterns (whole 1 KB runs per instruction, and 64-byte
// runs scattered across the buffer, the shape of the QKV kernel's V^T stores), and how much VALU work a
// SIMD issues beside its MFMAs (independent streams, and the time-attention tile loop).  Nothing here is
// on the stack's path.
#include "trf_device.h"
#include "trf_probe.h"

namespace {

using trf::f32x16;
using trf::u32x4;

// Each wave runs `chains` independent accumulator chains of `iters` MFMAs each, operands in registers.
// The accumulators' sum leaves through out[wave] so the work cannot be dropped.
template <int CHAINS>
__global__ __launch_bounds__(256) void k_mfma_peak(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  u32x4 a = {0x3f803f80u ^ uint32_t(lane), 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  u32x4 b = {0x3c003c00u, 0x3c003c00u ^ uint32_t(lane), 0x3c003c00u, 0x3c003c00u};
  f32x16 c[CHAINS];
#pragma unroll
  for (int i = 0; i < CHAINS; ++i) c[i] = trf::zero16();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < CHAINS; ++i) c[i] = trf::mfma32(a, b, c[i]);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CHAINS; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c[i][r];
  if (lane == 0) out[blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)] = s;
}

// Element e (16 bytes) of a stream in pattern `scattered`: 0 keeps it in place (each wave instruction
// covers 1 KB contiguous); 1 moves its 64-byte run r to run (r % 16) * (runs / 16) + r / 16, so the 16 runs
// of one instruction land runs / 16 * 64 bytes apart (runs is a multiple of 16).
__device__ __forceinline__ int64_t probe_element(int64_t e, int64_t runs, int scattered) {
  if (!scattered) return e;
  const int64_t r = e >> 2, rr = (r & 15) * (runs >> 4) + (r >> 4);
  return (rr << 2) | (e & 3);
}

__global__ __launch_bounds__(256) void k_store_stream(u32x4* __restrict__ dst, int64_t n16, int scattered) {
  const int64_t runs = n16 >> 2;
  const u32x4 v = {uint32_t(threadIdx.x), 0u, 0u, 0u};
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n16; e += int64_t(gridDim.x) * blockDim.x)
    dst[probe_element(e, runs, scattered)] = v;
}

// The same streams with 8-byte stores: each wave instruction writes 512 contiguous bytes (pattern 0) or
// eight 64-byte runs (pattern 1), the store width of the QKV kernel's outputs.
__global__ __launch_bounds__(256) void k_store_stream8(trf::u32x2* __restrict__ dst, int64_t n8, int scattered) {
  const int64_t runs = n8 >> 3;
  const trf::u32x2 v = {uint32_t(threadIdx.x), 0u};
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n8; e += int64_t(gridDim.x) * blockDim.x) {
    int64_t el = e;
    if (scattered) {
      const int64_t r = e >> 3, rr = (r & 15) * (runs >> 4) + (r >> 4);
      el = (rr << 3) | (e & 7);
    }
    dst[el] = v;
  }
}

__global__ __launch_bounds__(256) void k_load_stream(const u32x4* __restrict__ src, int64_t n16, int scattered,
                                                     uint32_t* __restrict__ out) {
  const int64_t runs = n16 >> 2;
  uint32_t acc = 0;
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n16; e += int64_t(gridDim.x) * blockDim.x) {
    const u32x4 v = src[probe_element(e, runs, scattered)];
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == 0x9e3779b9u) out[0] = acc;  // keeps the loads; never true for the probe's data
}


// ------------------------------------------------------------------ MFMA / VALU co-issue
// Each wave records its own cycle count (s_memtime, shader clock) over the loop into out[2w] and a
// checksum into out[2w + 1].

// Every probe workgroup holds 96 KB of LDS, so a CU runs exactly one: with 4 or 8 waves each SIMD then
// holds exactly one or two of them.
constexpr int kCoissuePadFloats = 24 * 1024;

__device__ __forceinline__ void record(float* __restrict__ out, uint64_t t0, float sink) {
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const int w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if ((threadIdx.x & 63) == 0) {
    out[2 * w] = float(t1 - t0);
    out[2 * w + 1] = sink;
  }
}

// One MFMA followed by NF independent v_fma_f32 (on registers the MFMAs do not touch), in exactly that
// order: 8 v_mfma_f32_32x32x16_bf16 per iteration on four accumulator chains (a chain's next MFMA is four
// MFMAs later), or 16 v_mfma_f32_16x16x32_bf16.  Alone, one iteration is 256 cycles of matrix pipe (8 x 32
// or 16 x 16) and NF x 8 x 4 or NF x 16 x 4 cycles of VALU issue.
#define TRF_FMA2 "v_fma_f32 %1, %1, %11, 0.5\n v_fma_f32 %2, %2, %11, 0.5\n"
#define TRF_FMA4 TRF_FMA2 "v_fma_f32 %3, %3, %11, 0.5\n v_fma_f32 %4, %4, %11, 0.5\n"
#define TRF_FMA8 TRF_FMA4 "v_fma_f32 %5, %5, %11, 0.5\n v_fma_f32 %6, %6, %11, 0.5\n v_fma_f32 %7, %7, %11, 0.5\n v_fma_f32 %8, %8, %11, 0.5\n"
#define TRF_XOPS "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7])
#define TRF_ABK "v"(a), "v"(b), "v"(k)

template <bool BIG, int NF>
__global__ __launch_bounds__(512) void k_coissue(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  __shared__ float pad[kCoissuePadFloats];
  pad[threadIdx.x] = 1.0f;
  __syncthreads();
  const u32x4 a = {0x3c003c00u ^ uint32_t(lane), 0x3c003c00u, 0x3c00bc00u, 0x3c003c00u};
  const u32x4 b = {0x3c003c00u, 0x3c003c00u ^ uint32_t(lane), 0x3c003c00u, 0xbc003c00u};
  f32x16 c[4];
  trf::f32x4 d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = trf::zero16();
    d[i] = trf::f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = 0.001f * (lane + i);
  const float k = 0.99f;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < (BIG ? 8 : 16); ++m) {
      if (BIG) {
        f32x16& C = c[m & 3];
        if (NF == 8)
          asm volatile("v_mfma_f32_32x32x16_bf16 %0, %9, %10, %0\n" TRF_FMA8 : "+v"(C), TRF_XOPS : TRF_ABK);
        else if (NF == 4)
          asm volatile("v_mfma_f32_32x32x16_bf16 %0, %9, %10, %0\n" TRF_FMA4 : "+v"(C), TRF_XOPS : TRF_ABK);
        else
          asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n" : "+v"(C) : "v"(a), "v"(b));
      } else {
        trf::f32x4& D = d[m & 3];
        if (NF == 4)
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %9, %10, %0\n" TRF_FMA4 : "+v"(D), TRF_XOPS : TRF_ABK);
        else if (NF == 2)
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %9, %10, %0\n" TRF_FMA2 : "+v"(D), TRF_XOPS : TRF_ABK);
        else
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0\n" : "+v"(D) : "v"(a), "v"(b));
      }
    }
  }
  // the last MFMAs' results are read below: let them retire first
  asm volatile("s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7" ::: "memory");
  float sink = pad[threadIdx.x];
#pragma unroll
  for (int i = 0; i < 8; ++i) sink += x[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sink += c[i][r];
#pragma unroll
    for (int r = 0; r < 4; ++r) sink += d[i][r];
  }
  record(out, t0, sink);
}

// One 64-key tile of the time-attention loop per iteration, per wave (two 32-query tiles, K and V^T
// operands read from LDS, scores in registers): 32 v_mfma_f32_32x32x16_bf16 (1,024 cycles of matrix pipe)
// beside 64 exp2, the row sum and 32 bf16 packs.  V = 0: as the kernel did before (fp32 adds of e);
// 1: the row sum on v_mfma_f32_16x16x32_bf16 (the kernel now); 2: MFMAs only (P taken from the scores'
// bits, no VALU); 3: VALU only (exp2, adds, packs on values carried between iterations, no MFMA);
// 4: as 0 with exp2 replaced by a multiply.
template <int V>
__global__ __launch_bounds__(512) void k_softmax_tile(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  __shared__ u32x4 lds[2][12][64];
  __shared__ float pad[kCoissuePadFloats];
  pad[threadIdx.x] = 1.0f;
  for (int i = threadIdx.x; i < 2 * 12 * 64; i += blockDim.x)
    (&lds[0][0][0])[i] = u32x4{0x3c003c00u ^ uint32_t(i & 0xff), 0x3c003c00u, 0x3c00bc00u, 0x3c003c00u ^ uint32_t(i >> 8)};
  __syncthreads();
  u32x4 qb[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k)
      qb[i][k] = u32x4{0x3c003c00u ^ uint32_t(i), 0x3c003c00u ^ uint32_t(lane), 0x3c003c00u, 0xbc003c00u ^ uint32_t(k)};
  f32x16 negc[2], o[2][2], xs[2][2];
  float lsum[2] = {0.f, 0.f};
  trf::f32x4 psum[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  const uint32_t one = ((lane & 15) == 0 && !(lane & 16)) || ((lane & 15) == 1 && (lane & 16)) ? 0x3f803f80u : 0u;
  const u32x4 ones = {one, one, one, one};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      negc[q][r] = -40.0f + 0.01f * r + q;
      xs[0][q][r] = xs[1][q][r] = -0.5f - 0.001f * (r + lane);
    }
    o[q][0] = o[q][1] = trf::zero16();
  }
  uint32_t bits = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    const u32x4 (*T)[64] = lds[it & 1];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      u32x4 ka[4], v0 = trf::zero4(), v1 = trf::zero4();
      if (V != 3) {
#pragma unroll
        for (int k = 0; k < 4; ++k) ka[k] = T[4 * kh + k][lane];
        v0 = T[8 + 2 * kh][lane];
        v1 = T[9 + 2 * kh][lane];
      }
      u32x4 p0[2], p1[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        f32x16 sc = negc[qt];
        if (V == 3) {
          sc = xs[kh][qt];
        } else {
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) sc = trf::mfma32(ka[ks], qb[qt][ks], sc);
        }
        if (V == 2) {
          p0[qt] = u32x4{__float_as_uint(sc[0]), __float_as_uint(sc[1]), __float_as_uint(sc[2]), __float_as_uint(sc[3])};
          p1[qt] = u32x4{__float_as_uint(sc[4]), __float_as_uint(sc[5]), __float_as_uint(sc[6]), __float_as_uint(sc[7])};
          bits ^= __float_as_uint(sc[8]) ^ __float_as_uint(sc[15]);
          continue;
        }
        float e[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) e[r] = V == 4 ? sc[r] * 1.0001f : __builtin_amdgcn_exp2f(sc[r]);
        if (V == 3) {
#pragma unroll
          for (int r = 0; r < 16; ++r) xs[kh][qt][r] = -e[r];
        }
        p0[qt] = u32x4{trf::pk_bf16(e[0], e[1]), trf::pk_bf16(e[2], e[3]), trf::pk_bf16(e[4], e[5]), trf::pk_bf16(e[6], e[7])};
        p1[qt] = u32x4{trf::pk_bf16(e[8], e[9]), trf::pk_bf16(e[10], e[11]), trf::pk_bf16(e[12], e[13]), trf::pk_bf16(e[14], e[15])};
        if (V == 1) {
          psum[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(trf::bf16x8, ones),
                                                             __builtin_bit_cast(trf::bf16x8, p0[qt]), psum[qt], 0, 0, 0);
          psum[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(trf::bf16x8, ones),
                                                             __builtin_bit_cast(trf::bf16x8, p1[qt]), psum[qt], 0, 0, 0);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) lsum[qt] += e[r];
        }
      }
      if (V == 3) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) bits ^= p0[qt][0] ^ p0[qt][1] ^ p0[qt][2] ^ p0[qt][3] ^ p1[qt][0] ^ p1[qt][1] ^ p1[qt][2] ^ p1[qt][3];
        continue;
      }
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          o[qt][dt] = trf::mfma32(dt ? v1 : v0, p0[qt], o[qt][dt]);
          o[qt][dt] = trf::mfma32(dt ? v0 : v1, p1[qt], o[qt][dt]);
        }
    }
  }
  float sink = lsum[0] + lsum[1] + psum[0][0] + psum[1][1] + __uint_as_float(bits & 0x3f7fffffu) + pad[threadIdx.x];
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int r = 0; r < 16; ++r) sink += o[q][0][r] + o[q][1][r] + xs[0][q][r] + xs[1][q][r];
  record(out, t0, sink);
}

// LDS operand streaming: per iteration every wave reads 8 operand blocks of 1 KB (ds_read_b128, 64 lanes
// x 16 B, conflict-free) from a 32 KB table.  M = 0: reads only (one v_xor per block keeps them);
// 1: each block is the A operand of one v_mfma_f32_32x32x16_bf16 (a GEMM whose waves hold one 32-column
// tile); 2: of two MFMAs with different B operands (two column tiles per wave).
template <int M>
__global__ __launch_bounds__(512) void k_lds_stream(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  __shared__ u32x4 tab[32 * 64];
  __shared__ float pad[kCoissuePadFloats - 32 * 64 * 4];
  for (int i = threadIdx.x; i < 32 * 64; i += blockDim.x)
    tab[i] = u32x4{0x3c003c00u ^ uint32_t(i & 0xff), 0x3c003c00u, 0x3c00bc00u, 0x3c003c00u ^ uint32_t(i >> 8)};
  pad[threadIdx.x] = 1.0f;
  __syncthreads();
  const u32x4 b0 = {0x3c003c00u, 0x3c003c00u ^ uint32_t(lane), 0x3c003c00u, 0xbc003c00u};
  const u32x4 b1 = {0x3c003c00u ^ uint32_t(lane), 0x3c003c00u, 0xbc003c00u, 0x3c003c00u};
  f32x16 c[4], d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = d[i] = trf::zero16();
  uint32_t bits = 0;
  const int w = threadIdx.x >> 6;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    const int base = ((it + w) & 3) * 8;  // 8 consecutive blocks of the table, rotating
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const u32x4 a = tab[(base + m) * 64 + lane];
      if (M == 0) {
        bits ^= a[0] ^ a[3];
      } else {
        c[m & 3] = trf::mfma32(a, b0, c[m & 3]);
        if (M == 2) d[m & 3] = trf::mfma32(a, b1, d[m & 3]);
      }
    }
  }
  float sink = __uint_as_float(bits & 0x3f7fffffu) + pad[threadIdx.x];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) sink += c[i][r] + d[i][r];
  record(out, t0, sink);
}

int fail_hip(hipError_t e) { return e == hipSuccess ? 0 : 3; }

}  // namespace

extern "C" {

int trf_probe_mfma_peak(int32_t chains, int32_t iters, int32_t workgroups, float* out, void* stream) {
  if (iters < 1 || workgroups < 1 || !out) return 1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  switch (chains) {
    case 1: hipLaunchKernelGGL(k_mfma_peak<1>, dim3(workgroups), dim3(256), 0, st, iters, out); break;
    case 2: hipLaunchKernelGGL(k_mfma_peak<2>, dim3(workgroups), dim3(256), 0, st, iters, out); break;
    case 4: hipLaunchKernelGGL(k_mfma_peak<4>, dim3(workgroups), dim3(256), 0, st, iters, out); break;
    case 8: hipLaunchKernelGGL(k_mfma_peak<8>, dim3(workgroups), dim3(256), 0, st, iters, out); break;
    default: return 1;
  }
  return fail_hip(hipGetLastError());
}

int trf_probe_store(void* dst, int64_t bytes, int32_t scattered, int32_t width, int32_t workgroups, void* stream) {
  if (!dst || bytes <= 0 || bytes % 1024 != 0 || workgroups < 1 || (scattered != 0 && scattered != 1) ||
      (width != 8 && width != 16))
    return 1;
  if (width == 16)
    hipLaunchKernelGGL(k_store_stream, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<u32x4*>(dst), bytes / 16, scattered);
  else
    hipLaunchKernelGGL(k_store_stream8, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<trf::u32x2*>(dst), bytes / 8, scattered);
  return fail_hip(hipGetLastError());
}

int trf_probe_load(const void* src, int64_t bytes, int32_t scattered, int32_t workgroups, uint32_t* out,
                   void* stream) {
  if (!src || !out || bytes <= 0 || bytes % 1024 != 0 || workgroups < 1 || (scattered != 0 && scattered != 1))
    return 1;
  hipLaunchKernelGGL(k_load_stream, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), bytes / 16, scattered, out);
  return fail_hip(hipGetLastError());
}

int trf_probe_coissue(int32_t variant, int32_t iters, int32_t waves_per_simd, int32_t workgroups, float* out,
                      void* stream) {
  if (iters < 1 || workgroups < 1 || !out || (waves_per_simd != 1 && waves_per_simd != 2)) return 1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g(workgroups), b(256 * waves_per_simd);
  switch (variant) {
    case 0: hipLaunchKernelGGL((k_coissue<true, 0>), g, b, 0, st, iters, out); break;
    case 1: hipLaunchKernelGGL((k_coissue<true, 4>), g, b, 0, st, iters, out); break;
    case 2: hipLaunchKernelGGL((k_coissue<true, 8>), g, b, 0, st, iters, out); break;
    case 3: hipLaunchKernelGGL((k_coissue<false, 0>), g, b, 0, st, iters, out); break;
    case 4: hipLaunchKernelGGL((k_coissue<false, 2>), g, b, 0, st, iters, out); break;
    case 5: hipLaunchKernelGGL((k_coissue<false, 4>), g, b, 0, st, iters, out); break;
    case 6: hipLaunchKernelGGL(k_softmax_tile<0>, g, b, 0, st, iters, out); break;
    case 7: hipLaunchKernelGGL(k_softmax_tile<1>, g, b, 0, st, iters, out); break;
    case 8: hipLaunchKernelGGL(k_softmax_tile<2>, g, b, 0, st, iters, out); break;
    case 9: hipLaunchKernelGGL(k_softmax_tile<3>, g, b, 0, st, iters, out); break;
    case 10: hipLaunchKernelGGL(k_softmax_tile<4>, g, b, 0, st, iters, out); break;
    case 11: hipLaunchKernelGGL(k_lds_stream<0>, g, b, 0, st, iters, out); break;
    case 12: hipLaunchKernelGGL(k_lds_stream<1>, g, b, 0, st, iters, out); break;
    case 13: hipLaunchKernelGGL(k_lds_stream<2>, g, b, 0, st, iters, out); break;
    default: return 1;
  }
  return fail_hip(hipGetLastError());
}

}  // extern "C"
