// Hamming-windowed overlap-add of chunk predictions into a song on gfx950 (chunking.py:39-61 of the
// reference: result[:, s:s+L] += y * w; weight[s:s+L] += w, chunk by chunk in ascending order, then
// result / max(weight, 1e-10)).
//
// One thread per (channel, sample), in gather form: it finds the chunks that cover its sample (chunk
// starts are sorted; the Python wrapper checks that before uploading them) and adds their terms in
// ascending chunk order with the same two fp32 roundings per term (product, then sum; no fused
// multiply-add) as the reference's elementwise ops, so the result is bitwise that of the reference's
// loop.  A song whose chunks run in several batches accumulates batch
// after batch into the same sums, which keeps the order.
#include "trf_device.h"

// The accumulation must round the product and the sum separately, as the reference's elementwise ops do:
// no contraction of a * b + c into one fused multiply-add in this file.
#pragma clang fp contract(off)

namespace trf {

// First index c in [0, n) with starts[c] > v (starts ascending).
__device__ __forceinline__ int upper_bound(const int64_t* __restrict__ starts, int n, int64_t v) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (starts[mid] <= v)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// acc[ch][i] += sum over chunks c covering i (ascending) of y[c][ch][i - s_c] * w[i - s_c]; wsum[i] += the
// same sum of w (channel 0's threads only).  y is [nc][2][ystride], L <= ystride samples of each are used.
__global__ __launch_bounds__(256) void k_overlap_add(const float* __restrict__ y, int nc, int64_t ystride, int L,
                                                     const int64_t* __restrict__ starts,
                                                     const float* __restrict__ w, int64_t n,
                                                     float* __restrict__ acc, float* __restrict__ wsum) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= 2 * n) return;
  const int ch = int(t / n);
  const int64_t i = t - int64_t(ch) * n;
  // chunks with i - L < s_c <= i
  const int c1 = upper_bound(starts, nc, i);
  int c0 = upper_bound(starts, nc, i - L);
  float a = acc[t];
  float ws = ch == 0 ? wsum[i] : 0.f;
  for (int c = c0; c < c1; ++c) {
    const int64_t k = i - starts[c];
    // Always true for ascending starts; with starts out of order the binary searches can return chunks
    // that do not cover sample i, and their terms are skipped instead of read out of bounds.
    if (k < 0 || k >= L) continue;
    const float wk = w[k];
    const float term = y[(int64_t(c) * 2 + ch) * ystride + k] * wk;  // rounded on its own (contract off)
    a = a + term;
    if (ch == 0) ws = ws + wk;
  }
  acc[t] = a;
  if (ch == 0) wsum[i] = ws;
}

// out[ch][i] = acc[ch][i] / max(wsum[i], 1e-10) / gain (in place allowed): the reference's
// result.div_(weight.clamp_(min=1e-10)) and then inst.div_(gain) of the peak normalisation, as two
// correctly rounded fp32 divisions (torch's CPU division by a scalar divides; it does not multiply by the
// reciprocal).
__global__ __launch_bounds__(256) void k_overlap_finish(const float* acc, const float* __restrict__ wsum,
                                                        int64_t n, float gain, float* out) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= 2 * n) return;
  const int64_t i = t - (t >= n ? n : 0);
  out[t] = (acc[t] / fmaxf(wsum[i], 1e-10f)) / gain;  // correctly rounded divisions (HIP's default)
}

void launch_overlap_add(const float* y, int nc, int64_t ystride, int L, const int64_t* starts, const float* w,
                        int64_t n, float* acc, float* wsum, hipStream_t st) {
  const int64_t threads = 2 * n;
  hipLaunchKernelGGL(k_overlap_add, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, st, y, nc, ystride, L,
                     starts, w, n, acc, wsum);
}

void launch_overlap_finish(const float* acc, const float* wsum, int64_t n, float gain, float* out, hipStream_t st) {
  const int64_t threads = 2 * n;
  hipLaunchKernelGGL(k_overlap_finish, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, st, acc, wsum, n, gain,
                     out);
}

}  // namespace trf
