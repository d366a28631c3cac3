// Band split of BS-RoFormer on gfx950: per band f, the RMSNorm of the frame's din_f spectral features and
// a Linear din_f -> 256 (BandSplit, model.py:147-155; called at fast.py:377-380), written straight into the
// stack's token order.
//
// Arithmetic: fp32 throughout, on v_mfma_f32_32x32x2_f32 (fp32 products and sums, as the reference's fp32
// Linear).  The norm is linear in the output, so the kernel computes W' . x on the raw features, with
// W' = W * gamma * sqrt(din) folded at packing, and scales the accumulators by 1 / max(|x|, 1e-12).
//
// Shape: C^T = W' . x^T: MFMA rows are the 256 output features (8 tiles of 32), columns are 32 frames.
// A workgroup is 4 waves on the same 32 frames of one band; wave w computes output tiles 2w and 2w+1
// (2 accumulator tiles), so the longest band (din 516) costs one wave 516 MFMAs rather than 2064, and a
// chunk makes 62 x 54 workgroups.  Per pair of input features each wave runs one MFMA per tile, its A
// operands (256-byte slices of W') read from L2/global one step (two k-pairs) ahead and its B operand one
// feature of the lane's frame; every wave sums the frame's squared features for the norm itself.  The
// workgroups of the widest bands go first.
#include "trf_device.h"

namespace trf {

constexpr int kBandWaves = 4;
constexpr int kBandTilesPerWave = 8 / kBandWaves;

__device__ __forceinline__ f32x16 mfma32f(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(64 * kBandWaves) void k_band_split(const float* __restrict__ feats,
                                                                const float* __restrict__ packed,
                                                                float* __restrict__ X, const BandPlan p) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int band = p.order[blockIdx.x / p.ngroups];
  const int group = blockIdx.x - (blockIdx.x / p.ngroups) * p.ngroups;
  const int din = p.din[band];
  const float* W = packed + p.wofs[band];  // [din/2 k-pairs][8 tiles][64 lanes], then the bias [256]
  const int n = group * kBandFrames + j;
  // Lanes past the last frame read the last frame (their column of the MFMAs only) and store nothing.
  const bool valid = n < p.n_frames;
  const float* xr = feats + int64_t(valid ? n : p.n_frames - 1) * p.width + p.col[band];
  const int t0 = kBandTilesPerWave * wave;  // this wave's first output tile

  f32x16 acc[kBandTilesPerWave];
#pragma unroll
  for (int t = 0; t < kBandTilesPerWave; ++t) acc[t] = zero16();
  float ss = 0.f;
  // A operands of this wave's tiles for k-pairs 2q and 2q+1, loaded one step ahead.
  constexpr int NA = 2 * kBandTilesPerWave;
  float a[NA];
  auto load_a = [&](int q) {
    const float* w = W + int64_t(q) * 2 * 8 * 64 + t0 * 64 + lane;
#pragma unroll
    for (int i = 0; i < NA; ++i) a[i] = w[((i / kBandTilesPerWave) * 8 + i % kBandTilesPerWave) * 64];
  };
  const int nq = din >> 2;  // float4 groups of features: k-pairs 2q (k = 4q + hh) and 2q+1 (k = 4q + 2 + hh)
  load_a(0);
  f32x4 xv = *reinterpret_cast<const f32x4*>(xr);
  for (int q = 0; q < nq; ++q) {
    float cur[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) cur[i] = a[i];
    if (q + 1 < nq) load_a(q + 1);
    const float b0 = hh ? xv[1] : xv[0], b1 = hh ? xv[3] : xv[2];
    if (q + 1 < nq) xv = *reinterpret_cast<const f32x4*>(xr + 4 * (q + 1));
    ss = fmaf(b0, b0, fmaf(b1, b1, ss));
#pragma unroll
    for (int t = 0; t < kBandTilesPerWave; ++t) acc[t] = mfma32f(cur[t], b0, acc[t]);
#pragma unroll
    for (int t = 0; t < kBandTilesPerWave; ++t) acc[t] = mfma32f(cur[kBandTilesPerWave + t], b1, acc[t]);
  }
  ss += __shfl_xor(ss, 32);  // lanes j and j + 32 hold the frame's even and odd features
  const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
  if (!valid) return;
  const float* bias = W + int64_t(din >> 1) * 8 * 64;
  float* xo = X + (int64_t(n) * p.n_bands + band) * kDim;
#pragma unroll
  for (int t = 0; t < kBandTilesPerWave; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int o = 32 * (t0 + t) + row_of_group(g, hh);
      const f32x4 b = *reinterpret_cast<const f32x4*>(bias + o);
      f32x4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = fmaf(acc[t][4 * g + r], inv, b[r]);
      *reinterpret_cast<f32x4*>(xo + o) = v;
    }
}

// Packing of one band: W'[o][k] = w[o][k] * (gamma[k] * sqrt(din)) as A operands of v_mfma_f32_32x32x2_f32:
// dst[(p * 8 + t) * 64 + lane] = W'[32t + lane%32][2p + lane/32], then the bias [256].
__global__ void k_pack_band_split(const float* __restrict__ w, const float* __restrict__ b,
                                  const float* __restrict__ gamma, int din, float sqrt_din, float* __restrict__ dst) {
  const int n_items = (din / 2) * 8 * 64;
  for (int it = blockIdx.x * blockDim.x + threadIdx.x; it < n_items + kDim; it += gridDim.x * blockDim.x) {
    if (it >= n_items) {
      dst[it] = b[it - n_items];
      continue;
    }
    const int lane = it & 63, t = (it >> 6) & 7, pk = it >> 9;
    const int o = 32 * t + (lane & 31), k = 2 * pk + (lane >> 5);
    dst[it] = w[int64_t(o) * din + k] * (gamma[k] * sqrt_din);
  }
}

void launch_pack_band_split(const float* w, const float* b, const float* gamma, int din, float sqrt_din, float* dst,
                            hipStream_t st) {
  const int n = (din / 2) * 8 * 64 + kDim;
  hipLaunchKernelGGL(k_pack_band_split, dim3((n + 255) / 256), dim3(256), 0, st, w, b, gamma, din, sqrt_din, dst);
}

void launch_band_split(const float* feats, const float* packed, float* X, const BandPlan& plan, hipStream_t st) {
  hipLaunchKernelGGL(k_band_split, dim3(unsigned(plan.n_bands) * unsigned(plan.ngroups)), dim3(64 * kBandWaves), 0,
                     st, feats, packed, X, plan);
}

}  // namespace trf
