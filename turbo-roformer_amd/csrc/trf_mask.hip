// Mask head of BS-RoFormer on gfx950: the final RMSNorm of the stack output and, per band, the mask
// estimator MLP  mask = GLU(W2 . tanh(W1 . xn + b1) + b2)  (model.py:158-178; batched over the bands of
// equal width in fast.py:139-160 and 349-360, applied after the stack at fast.py:385-387).
//
// Arithmetic.  Both GEMMs run on v_mfma_f32_32x32x16_f16 with fp32 accumulation.  kMaskSplit splits every
// operand v into fp16 hi = f16(v) and lo = f16(v - hi) and forms hi.hi + hi.lo + lo.hi (three MFMAs per
// product; the dropped lo.lo term is ~2^-22 relative), which keeps the mask within ~1e-6 of the fp32
// computation of the reference.  kMaskFp16 uses hi alone (one MFMA per product).
//
// Shape.  C^T = W . A^T as in the stack kernels: MFMA rows are hidden units (GEMM1) or mask columns
// (GEMM2), MFMA columns are 32 frames of one band.  A workgroup is 4 waves, one per SIMD (512 registers
// each), and 128 frames of one band; each wave keeps its 32 frames' normalised inputs in registers (hi
// and lo: 128 registers) and the GEMM2 accumulators of up to kMaskPairs output pairs (a and g tiles of 32
// mask columns: 32 registers per pair).  A band wider than kMaskPairs pairs is split over several jobs,
// each recomputing the hidden layer.  The weights stream through LDS one hidden tile (32 units) per
// stage, double-buffered: stage u holds W1 of tile u and W2 of tile u-1, and runs
//   tanh of tile u-1's pre-activation, spread between GEMM1(u)'s MFMAs (one value per k-step),
//   GEMM1(u): hidden tile u = W1(u) . xn  (two accumulator chains, interleaved),
//   GEMM2(u-1): acc += W2(u-1) . tanh(tile u-1), its B operands straight from the tanh registers in
//               accumulator order (W2 is packed with its k order permuted to match).
// Stage 0 multiplies its W2 blocks (tile 0) by tanh(0) = 0 exactly; a last stage runs tanh and GEMM2 of
// the last tile.  b1 is added with the tanh; the GEMM2 accumulators start at b2; the GLU is the epilogue.
#include "trf_device.h"

namespace trf {

constexpr int kMaskWaves = kMaskFrames / 32;
constexpr int kMaskStageBlocks = kMaskW1Blocks + 8 * kMaskPairs;  // LDS blocks of the largest stage
constexpr float kMaskNormScale = 16.0f;                           // sqrt(dim) of the RMSNorm

// hi = f16(a), f16(b) and lo = f16(a - hi), f16(b - hi) as packed pairs.
__device__ __forceinline__ void split_f16(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pk_f16(a, b);
  const f16x2 h = __builtin_bit_cast(f16x2, hi);
  lo = pk_f16(a - float(h[0]), b - float(h[1]));
}

// tanh x = 1 - 2 / (e^(2x) + 1): exact 0 at x = 0, saturates to +-1 through e = inf / 0, absolute error
// ~1e-7 (v_exp_f32 and v_rcp_f32 are ~1 ulp).
__device__ __forceinline__ float tanh_f32(float x) {
  const float e = __builtin_amdgcn_exp2f(x * (2.0f * kLog2e));
  return fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
}

// The work of a stage in units, each reading its LDS operand blocks once:
//   unit k < 16: GEMM1 k-step s = k; split: blocks W1 hi(s), lo(s) and MFMAs hi.xh, hi.xl, lo.xh into
//     accumulator chains s, s+1, s (mod 2), so that consecutive MFMAs alternate chains; fp16: hi(s) . xh.
//   unit 16 + 2i + t: GEMM2 of output pair i, hidden k-step t (units 16t..16t+15 of the tile); split:
//     blocks a hi, a lo, g hi, g lo and MFMAs a.hh, g.hh, a.hl, g.hl, a_lo.hh, g_lo.hh (a and g chains
//     alternate); fp16: a.hh, g.hh.
// LDS blocks of a stage: split = the packed tile's order (W1 blocks 0..31, W2 of pair i at 32 + 8i + ...);
// fp16 = hi blocks only (W1 s at s, W2 of pair i, ag, t at 16 + 4i + 2ag + t).
template <bool SPLIT, int NP>
struct MaskOps {
  static constexpr int U1 = 16;               // GEMM1 units
  static constexpr int U = U1 + 2 * NP;       // all units of a stage
  static constexpr int R = SPLIT ? 4 : 2;     // LDS reads of a GEMM2 unit (a GEMM1 unit reads R / 2)
  static constexpr int W1B = SPLIT ? kMaskW1Blocks : kMaskW1Blocks / 2;  // LDS blocks of W1
  static constexpr int NB = W1B + (SPLIT ? 8 : 4) * NP;                  // LDS blocks of a stage
  __host__ __device__ static constexpr int reads(int k) { return k < U1 ? R / 2 : R; }
  // LDS block of read r of unit k (GEMM2 reads: split a hi, a lo, g hi, g lo; fp16 a, g).
  __host__ __device__ static constexpr int block(int k, int r) {
    if (k < U1) return SPLIT ? 2 * k + r : k;
    const int i = (k - U1) >> 1, t = (k - U1) & 1;
    return SPLIT ? W1B + 8 * i + 4 * (r >> 1) + 2 * t + (r & 1) : W1B + 4 * i + 2 * r + t;
  }
};

// One stage.  LAST: tanh and GEMM2 of the last hidden tile only.  Otherwise: pre := tile u-1 (+ b1),
// tanh(pre) into the GEMM2 B operands, one value after each GEMM1 unit, then GEMM2(u-1); b1 of tile u is
// loaded for the next stage, and dma(q) issues this wave's q-th direct-to-LDS block of the next stage
// after unit q.  (Issued all at once, the next stage's 40-80 KB per workgroup outrun what a CU keeps in
// flight and the wave stalls in issue before its MFMAs; spread over the first units, they stream under
// them and land before the stage ends.)  Each unit's operand blocks are read one unit ahead.
template <bool SPLIT, int NP, bool LAST, typename Dma>
__device__ __forceinline__ void mask_stage(const u32x4* L, int u, const float* b1, const u32x4 (&xh)[16],
                                           const u32x4 (&xl)[16], f32x16& hA, f32x16& hB, f32x4 (&b1v)[4],
                                           f32x16 (&acc)[2 * NP], int lane, int hh, Dma&& dma) {
  using O = MaskOps<SPLIT, NP>;
  constexpr int K0 = LAST ? O::U1 : 0;  // first unit of the stage
  static_assert(O::NB / kMaskWaves <= O::U, "one DMA block per unit");
  float pre[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) pre[r] = hA[r] + hB[r] + b1v[r >> 2][r & 3];
  if (!LAST) {
#pragma unroll
    for (int g = 0; g < 4; ++g) b1v[g] = *reinterpret_cast<const f32x4*>(b1 + 32 * u + 8 * g + 4 * hh);
  }
  u32x4 hbh[2], hbl[2];  // tanh(pre) as GEMM2 B operands (hidden k-steps 0 and 1 of the tile), hi and lo
  float tv[16];
  auto tanh_value = [&](int s) {
    tv[s] = tanh_f32(pre[s]);
    if (s & 1) {
      uint32_t h, l;
      split_f16(tv[s - 1], tv[s], h, l);
      hbh[s >> 3][(s & 7) >> 1] = h;
      hbl[s >> 3][(s & 7) >> 1] = l;
    }
  };
  if (LAST) {
#pragma unroll
    for (int s = 0; s < 16; ++s) tanh_value(s);
  }
  u32x4 cur[O::R], nxt[O::R];
#pragma unroll
  for (int r = 0; r < O::reads(K0); ++r) nxt[r] = L[O::block(K0, r) * 64 + lane];
  auto unit = [&](int k) {
#pragma unroll
    for (int r = 0; r < O::R; ++r) cur[r] = nxt[r];
    if (k + 1 < O::U) {
#pragma unroll
      for (int r = 0; r < O::reads(k + 1); ++r) nxt[r] = L[O::block(k + 1, r) * 64 + lane];
    }
    if (k < O::U1) {
      f32x16& c0 = (k & 1) ? hB : hA;  // chain of the hi.hi and lo.hi products
      f32x16& c1 = (k & 1) ? hA : hB;  // chain of hi.lo
      // First products of the chains start from zero: hA at k-step 0; hB at k-step 0 (split, its hi.lo)
      // or 1 (fp16).
      c0 = mfma32h(cur[0], xh[k], (k == 0 || (!SPLIT && k == 1)) ? zero16() : c0);
      if (SPLIT) {
        c1 = mfma32h(cur[0], xl[k], k == 0 ? zero16() : c1);
        c0 = mfma32h(cur[1], xh[k], c0);
      }
      if (!LAST) tanh_value(k);
    } else {
      const int i = (k - O::U1) >> 1, t = (k - O::U1) & 1;
      f32x16& a = acc[2 * i];
      f32x16& g = acc[2 * i + 1];
      a = mfma32h(cur[0], hbh[t], a);
      g = mfma32h(cur[SPLIT ? 2 : 1], hbh[t], g);
      if (SPLIT) {
        a = mfma32h(cur[0], hbl[t], a);
        g = mfma32h(cur[2], hbl[t], g);
        a = mfma32h(cur[1], hbh[t], a);
        g = mfma32h(cur[3], hbh[t], g);
      }
    }
    if (!LAST && k < O::NB / kMaskWaves) dma(k);
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int k = K0; k < O::U1; ++k) unit(k);
#pragma unroll
  for (int k = O::U1; k < O::U; ++k) unit(k);
}

template <bool SPLIT, int NP>
__device__ __forceinline__ void mask_job(const MaskPlan& p, const float* __restrict__ X,
                                         const uint8_t* __restrict__ packed, float* __restrict__ mask, int band,
                                         int p0, int tb, u32x4* smem) {
  using O = MaskOps<SPLIT, NP>;
  u32x4* lds0 = smem;
  u32x4* lds1 = smem + kMaskStageBlocks * 64;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int din = p.din[band];
  const int npairs = (din + 31) >> 5;
  const int tstride = (kMaskW1Blocks + 8 * npairs) * 64;  // u32x4 per hidden tile
  const int nht = p.hidden >> 5;
  const float* b1 = reinterpret_cast<const float*>(packed + p.b1_off) + size_t(band) * p.hidden;

  // Block q of this wave (block b = wave + kMaskWaves q) of stage u into LDS buffer dst: W1 of tile u (for
  // u = nht tile nht-1 again, unused: no branch) and W2 of tile max(u-1, 0), pairs p0..p0+NP-1.  A buffer load over the band's weights:
  // the block's offset is scalar and the lane offset one register for all blocks (reads past the band's
  // weights would return zeros).
  const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(packed + size_t(p.wofs_kb[band]) * 1024, nht * tstride * 16);
  const int voff = lane * 16;
  auto issue = [&](int u, u32x4* dst, int q) {
    const int b = wave + kMaskWaves * q;
    const int blk = b < O::W1B ? (u < nht ? u : nht - 1) * (tstride / 64) + (SPLIT ? b : 2 * b)
                               : (u > 0 ? u - 1 : 0) * (tstride / 64) + kMaskW1Blocks + 8 * p0 +
                                     (SPLIT ? b - O::W1B : 2 * (b - O::W1B));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, (__attribute__((address_space(3))) void*)(dst + b * 64), 16,
                                             voff, blk * 1024, 0, 0);
  };
  const int n = tb * kMaskFrames + wave * 32 + j;
  // Lanes past the last frame work on a copy of the last frame (a column of their own) and store nothing.
  const bool valid = n < p.n_frames;
  const float* xr = X + (int64_t(valid ? n : p.n_frames - 1) * p.F + band) * kDim;
#pragma unroll
  for (int q = 0; q < O::NB / kMaskWaves; ++q) issue(0, lds0, q);
  // This lane's half of the frame's 256 features: k = 16s + 8hh + e, the B-operand order of k-step s.
  f32x4 xv[32];
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    xv[2 * s] = *reinterpret_cast<const f32x4*>(xr + 16 * s + 8 * hh);
    xv[2 * s + 1] = *reinterpret_cast<const f32x4*>(xr + 16 * s + 8 * hh + 4);
  }
  // The GEMM2 accumulators start at b2: a tile of pair i at b2[c], its g tile at b2[pad + c] for the
  // lane's columns c (every c < pad: the packed b2 is zero past din, so no guard is needed).
  const float* b2 = reinterpret_cast<const float*>(packed + p.b2_off[band]);
  const int pad = 32 * npairs;
  f32x16 acc[2 * NP];
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 32 * (p0 + i) + 8 * g + 4 * hh;
      const f32x4 ba = *reinterpret_cast<const f32x4*>(b2 + c);
      const f32x4 bg = *reinterpret_cast<const f32x4*>(b2 + pad + c);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[2 * i][4 * g + r] = ba[r];
        acc[2 * i + 1][4 * g + r] = bg[r];
      }
    }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) ss = fmaf(xv[i][e], xv[i][e], ss);
  ss += __shfl_xor(ss, 32);
  const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);  // RMSNorm: x / max(|x|, eps) * sqrt(dim) * gamma
  u32x4 xh[16], xl[16];                                // (gamma is folded into W1)
#pragma unroll
  for (int s = 0; s < 16; ++s)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4& v = xv[2 * s + (q >> 1)];
      uint32_t h, l;
      split_f16(v[2 * (q & 1)] * inv * kMaskNormScale, v[2 * (q & 1) + 1] * inv * kMaskNormScale, h, l);
      xh[s][q] = h;
      xl[s][q] = l;
    }

  f32x16 hA = zero16(), hB = zero16();
  f32x4 b1v[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) b1v[g] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Stages go in pairs so that each one's LDS buffer is a compile-time constant (the compiler then tells
  // operand reads from the direct-to-LDS loads into the other buffer and does not wait for those).
#pragma clang loop unroll(disable)
  for (int u = 0; u < nht; u += 2) {
    stage_barrier();
    mask_stage<SPLIT, NP, false>(lds0, u, b1, xh, xl, hA, hB, b1v, acc, lane, hh,
                                 [&](int q) { issue(u + 1, lds1, q); });
    stage_barrier();
    mask_stage<SPLIT, NP, false>(lds1, u + 1, b1, xh, xl, hA, hB, b1v, acc, lane, hh,
                                 [&](int q) { issue(u + 2, lds0, q); });
  }
  stage_barrier();
  mask_stage<SPLIT, NP, true>(lds0, nht, b1, xh, xl, hA, hB, b1v, acc, lane, hh, [](int) {});

  if (!valid) return;
  float* mrow = mask + int64_t(n) * p.width + p.col[band];
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 32 * (p0 + i) + 8 * g + 4 * hh;  // mask columns c..c+3 of the band
      if (c >= din) continue;
      f32x4 m;
#pragma unroll
      for (int r = 0; r < 4; ++r) m[r] = acc[2 * i][4 * g + r] / (1.0f + __expf(-acc[2 * i + 1][4 * g + r]));
      *reinterpret_cast<f32x4*>(mrow + c) = m;
    }
}

template <bool SPLIT>
__global__ __launch_bounds__(64 * kMaskWaves) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_mask_head(
    const float* __restrict__ X, const uint8_t* __restrict__ packed, float* __restrict__ mask, const MaskPlan p) {
  // One LDS object: two stage buffers of kMaskStageBlocks operand blocks.
  __shared__ u32x4 smem[2 * kMaskStageBlocks * 64];
  const int xcd = blockIdx.x % kXcds, k = blockIdx.x / kXcds;
  const int slot = k / p.ntb, tb = k - slot * p.ntb;
  const int first = p.xcd_start[xcd];
  if (slot >= int(p.xcd_start[xcd + 1]) - first) return;
  const uint32_t job = p.job[first + slot];
  const int band = job & 0xff, np = (job >> 8) & 0xff, p0 = job >> 16;
  switch (np) {
    case 1: mask_job<SPLIT, 1>(p, X, packed, mask, band, p0, tb, smem); break;
    case 2: mask_job<SPLIT, 2>(p, X, packed, mask, band, p0, tb, smem); break;
    case 3: mask_job<SPLIT, 3>(p, X, packed, mask, band, p0, tb, smem); break;
    case 4: mask_job<SPLIT, 4>(p, X, packed, mask, band, p0, tb, smem); break;
    case 5: mask_job<SPLIT, 5>(p, X, packed, mask, band, p0, tb, smem); break;
    default: mask_job<SPLIT, 6>(p, X, packed, mask, band, p0, tb, smem); break;
  }
  static_assert(kMaskPairs == 6, "one case per pair count");
}

// ============================================================ packing
// Items of a band: (tile j, block, lane) -> one 16-byte lane slot of the layout in trf_internal.h.
//   W1 block 2s + hl, lane l: rows 32j + l%32, inputs 16s + 8(l/32) + e, times gamma (natural k order).
//   W2 block 32 + 8i + 4ag + 2t + hl, lane l: row (ag ? din : 0) + 32i + l%32 (zero past din), hidden units
//     32j + 16t + 8(e/4) + 4(l/32) + e%4: the order in which a lane holds hidden units in its accumulator
//     (rows 8(r/4) + 4(l/32) + r%4 of register r), so tanh's registers are GEMM2's B operands as they are.
__global__ void k_pack_mask_band(const float* __restrict__ w1, const float* __restrict__ gamma,
                                 const float* __restrict__ b1, const float* __restrict__ w2,
                                 const float* __restrict__ b2, int din, int hidden, u32x4* __restrict__ wdst,
                                 float* __restrict__ b1dst, float* __restrict__ b2dst) {
  const int npairs = (din + 31) / 32, pad = 32 * npairs;
  const int tstride = kMaskW1Blocks + 8 * npairs;
  const int64_t n_items = int64_t(hidden / 32) * tstride * 64;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t it = tid; it < n_items; it += stride) {
    const int lane = int(it & 63);
    const int64_t bt = it >> 6;
    const int blk = int(bt % tstride), j = int(bt / tstride);
    const int r = lane & 31, hh = lane >> 5;
    float v[8];
    int hl;
    if (blk < kMaskW1Blocks) {
      const int s = blk >> 1, k0 = 16 * s + 8 * hh;
      hl = blk & 1;
      const float* row = w1 + int64_t(32 * j + r) * kDim;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = row[k0 + e] * gamma[k0 + e];
    } else {
      const int q = blk - kMaskW1Blocks;
      const int i = q >> 3, ag = (q >> 2) & 1, t = (q >> 1) & 1, c = 32 * i + r;
      hl = q & 1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int unit = 32 * j + 16 * t + 8 * (e >> 2) + 4 * hh + (e & 3);
        v[e] = c < din ? w2[int64_t(ag ? din + c : c) * hidden + unit] : 0.f;
      }
    }
    u32x4 out;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h, l;
      const float a = v[2 * q], b = v[2 * q + 1];
      h = pk_f16(a, b);
      const f16x2 hv = __builtin_bit_cast(f16x2, h);
      l = pk_f16(a - float(hv[0]), b - float(hv[1]));
      out[q] = hl ? l : h;
    }
    wdst[it] = out;
  }
  for (int64_t i = tid; i < hidden; i += stride) b1dst[i] = b1[i];
  for (int64_t c = tid; c < pad; c += stride) {
    b2dst[c] = c < din ? b2[c] : 0.f;
    b2dst[pad + c] = c < din ? b2[din + c] : 0.f;
  }
}

void launch_pack_mask_band(const float* w1, const float* gamma, const float* b1, const float* w2, const float* b2,
                           int din, int hidden, uint8_t* wdst, float* b1dst, float* b2dst, hipStream_t st) {
  const int64_t n_items = int64_t(hidden / 32) * (kMaskW1Blocks + 8 * ((din + 31) / 32)) * 64;
  const unsigned blocks = unsigned((n_items + 255) / 256 < 4096 ? (n_items + 255) / 256 : 4096);
  hipLaunchKernelGGL(k_pack_mask_band, dim3(blocks), dim3(256), 0, st, w1, gamma, b1, w2, b2, din, hidden,
                     reinterpret_cast<u32x4*>(wdst), b1dst, b2dst);
}

void launch_mask_head(const float* X, const uint8_t* packed, float* mask, const MaskPlan& plan, unsigned grid,
                      int precision, hipStream_t st) {
  if (precision == kMaskFp16)
    hipLaunchKernelGGL(k_mask_head<false>, dim3(grid), dim3(64 * kMaskWaves), 0, st, X, packed, mask, plan);
  else
    hipLaunchKernelGGL(k_mask_head<true>, dim3(grid), dim3(64 * kMaskWaves), 0, st, X, packed, mask, plan);
}

}  // namespace trf
