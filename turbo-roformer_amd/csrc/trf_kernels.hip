// HIP kernels of the BS-RoFormer transformer stack for gfx950 (MI355X).
//
// All matrix products run on v_mfma_f32_32x32x16_bf16 (bf16 operands, fp32 accumulation).
// The kernels compute C^T = W . A^T, i.e. the 32 MFMA rows are output features and the 32
// MFMA columns are tokens.  With the 32x32 accumulator layout
//     lane l, register r  ->  row 8*(r/4) + 4*(l/32) + (r%4), column l%32
// every lane owns one token and runs of 4 consecutive features, so interleaved rotary pairs
// (2p, 2p+1), row norms and residual updates need no cross-lane exchange beyond one swap of
// the two half-waves.
//
// Numerics follow the reference kernels (src/turbo_roformer/csrc/kernels.cpp): fp32
// accumulators, fp32 residual stream, fp32 rotary/softmax/gate math, bf16 round-to-nearest-even
// for every GEMM/attention operand (kernels.cpp:30-33).
#include "trf_device.h"

#include <atomic>

#include <type_traits>

namespace trf {

// ============================================================ weight packing
// 32x32 layouts: dst[t][ks][lane][e] = W[32t + lane%32][16ks + kperm(lane/32, e)] (kperm: natural 8hh + e,
// or register order 4hh + e / 8 + 4hh + e - 4).  16x16 layouts: dst[t][ks][lane][e] =
// W[16t + lane%16][32ks + kperm16(lane/16, e)] (natural 8g + e, register order 16(e/4) + 4g + e%4).
// Rows past `rows` are zero, and so is everything when W is null.  (See trf_internal.h.)
__global__ void k_pack(const uint16_t* __restrict__ W, int rows, int K, int layout, u32x4* __restrict__ dst) {
  const bool t16 = layout >= kPack16Natural;
  const int tr = t16 ? 16 : 32, kstep = t16 ? 32 : 16;
  const int ksteps = K / kstep;
  const int64_t total = int64_t((rows + tr - 1) / tr) * ksteps * 64;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int lane = int(i % 64);
  const int ks = int((i / 64) % ksteps);
  const int t = int(i / (64 * ksteps));
  const int row = tr * t + lane % tr;
  const int grp = lane / tr;
  u32x4 v = zero4();
  if (W && row < rows) {
    const uint16_t* src = W + int64_t(row) * K + kstep * ks;
    if (layout == kPack32Natural) {
      v = *reinterpret_cast<const u32x4*>(src + 8 * grp);
    } else if (layout == kPack32RegOrder) {
      const u32x2 lo = *reinterpret_cast<const u32x2*>(src + 4 * grp);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(src + 8 + 4 * grp);
      v = u32x4{lo[0], lo[1], hi[0], hi[1]};
    } else if (layout == kPack16Natural) {
      v = *reinterpret_cast<const u32x4*>(src + 8 * grp);
    } else {
      const u32x2 lo = *reinterpret_cast<const u32x2*>(src + 4 * grp);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(src + 16 + 4 * grp);
      v = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  }
  dst[i] = v;
}

void launch_pack(const uint16_t* W, int rows, int K, int layout, uint8_t* dst, hipStream_t st) {
  const bool t16 = layout >= kPack16Natural;
  const int tr = t16 ? 16 : 32, kstep = t16 ? 32 : 16;
  const int64_t total = int64_t((rows + tr - 1) / tr) * (K / kstep) * 64;
  hipLaunchKernelGGL(k_pack, dim3(unsigned((total + 255) / 256)), dim3(256), 0, st, W, rows, K, layout,
                     reinterpret_cast<u32x4*>(dst));
}

// fp16 operand tiles, 32x32 register order, from hi + lo bf16 parts of the fp32 weights (lo optional):
// dst = fp16(hi + lo), round to nearest even.
__global__ void k_pack_f16(const uint16_t* __restrict__ hi, const uint16_t* __restrict__ lo, int rows, int K,
                           u32x4* __restrict__ dst) {
  const int ksteps = K / 16;
  const int64_t total = int64_t((rows + 31) / 32) * ksteps * 64;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int lane = int(i % 64);
  const int ks = int((i / 64) % ksteps);
  const int t = int(i / (64 * ksteps));
  const int row = 32 * t + (lane & 31), hh = lane >> 5;
  u32x4 v = zero4();
  if (row < rows) {
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = 16 * ks + (e < 4 ? 4 * hh + e : 8 + 4 * hh + (e - 4));  // register order
      const int64_t idx = int64_t(row) * K + k;
      f[e] = bf16_to_f32(hi[idx]) + (lo ? bf16_to_f32(lo[idx]) : 0.0f);
    }
    v = u32x4{pk_f16(f[0], f[1]), pk_f16(f[2], f[3]), pk_f16(f[4], f[5]), pk_f16(f[6], f[7])};
  }
  dst[i] = v;
}

void launch_pack_f16(const uint16_t* hi, const uint16_t* lo, int rows, int K, uint8_t* dst, hipStream_t st) {
  const int64_t total = int64_t((rows + 31) / 32) * (K / 16) * 64;
  hipLaunchKernelGGL(k_pack_f16, dim3(unsigned((total + 255) / 256)), dim3(256), 0, st, hi, lo, rows, K,
                     reinterpret_cast<u32x4*>(dst));
}

__global__ void k_copy_f32(const float* __restrict__ src, int n, float* __restrict__ dst) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

void launch_copy_f32(const float* src, int n, float* dst, hipStream_t st) {
  hipLaunchKernelGGL(k_copy_f32, dim3((n + 255) / 256), dim3(256), 0, st, src, n, dst);
}

// ============================================================ add + L2 row norm
// One wave per row of 256: lane l holds columns 4l..4l+3.  (kernels.cpp:101-137)
__global__ __launch_bounds__(256) void k_add_rmsnorm(float* __restrict__ X, const void* __restrict__ Y,
                                                     int y_bf16, void* __restrict__ out, int out_bf16,
                                                     int64_t n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  float* xr = X + row * kDim + 4 * lane;
  f32x4 v = *reinterpret_cast<const f32x4*>(xr);
  if (Y) {
    if (y_bf16) {
      const u32x2 y = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(Y) + row * kDim + 4 * lane);
      v[0] += __uint_as_float(y[0] << 16);
      v[1] += __uint_as_float(y[0] & 0xFFFF0000u);
      v[2] += __uint_as_float(y[1] << 16);
      v[3] += __uint_as_float(y[1] & 0xFFFF0000u);
    } else {
      const f32x4 y = *reinterpret_cast<const f32x4*>(static_cast<const float*>(Y) + row * kDim + 4 * lane);
      v += y;
    }
    *reinterpret_cast<f32x4*>(xr) = v;
  }
  float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  const float inv = 1.0f / fmaxf(sqrtf(ss), eps);
  if (out_bf16) {
    u32x2 o = {pk_bf16(v[0] * inv, v[1] * inv), pk_bf16(v[2] * inv, v[3] * inv)};
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + row * kDim + 4 * lane) = o;
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + row * kDim + 4 * lane) = v * inv;
  }
}

void launch_add_rmsnorm(float* X, const void* Y, int y_bf16, void* out, int out_bf16, int64_t n, float eps,
                        hipStream_t st) {
  hipLaunchKernelGGL(k_add_rmsnorm, dim3(unsigned((n + 3) / 4)), dim3(256), 0, st, X, Y, y_bf16, out, out_bf16,
                     n, eps);
}

// ============================================================ fused QKV + gate GEMM, rotary epilogue
// One wave owns 32 consecutive padded positions of one sequence; its 32 tokens' xn rows stay in
// registers as B operands.  The workgroup (8 waves, 2 per SIMD) streams the 49 weight tiles through
// LDS four per stage (13 stages: q heads, k heads, v heads, then the gate tile), so every stage is of
// one kind.  The rotary cos/sin of the wave's position is loaded into registers with its xn rows.
// (kernels.cpp:439-540)
//
// A stage runs as two groups of two tiles (two interleaved MFMA chains each).  A group's outputs
// leave as 8 packed 8-byte stores per lane, issued during the NEXT group's MFMA loop, one every other
// k-step, so the write stream runs under the matrix work instead of in a burst between stages.  Stage
// barriers wait with an exact vmcnt for the weight loads issued before those stores.
//
// Work is dealt in units of (block of 256 rows, stage): workgroup b of G runs units [bU/G, (b+1)U/G) of
// the U = 13 x blocks in order, so one workgroup per CU gets an even share of stages (21 or 22 for the
// 419 blocks of a 17 s chunk's time sub-layer) instead of two rounds of whole blocks (1.64 per CU).  A
// block entered mid-way loads its xn rows and rotary table again; one left early stores its last group
// at once.
constexpr int kQkvWaves = 8;
constexpr int kQkvTps = 4;
constexpr int kQkvStages = (kQkvgTiles + kQkvTps - 1) / kQkvTps;
constexpr int kQkvGroupStores = 8;  // 2 tiles x 4 register groups

__global__ __launch_bounds__(512) void k_qkv_rope(const uint16_t* __restrict__ xn, const u32x4* __restrict__ wq,
                                                  const float* __restrict__ bgate, const float* __restrict__ rope,
                                                  int mode, int nseq, int L, int Lpad, int T, int F, int nblocks,
                                                  uint16_t* __restrict__ Q, uint16_t* __restrict__ K,
                                                  uint16_t* __restrict__ Vt, float* __restrict__ G) {
  __shared__ u32x4 lds[2][kQkvTps * 16 * 64];  // 2 stages x 4 tiles x 16 k-steps x 1 KB
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int units = nblocks * kQkvStages;
  const int u_begin = int(int64_t(blockIdx.x) * units / gridDim.x);
  const int u_end = int(int64_t(blockIdx.x + 1) * units / gridDim.x);
  const int qd = lane & 3;

  auto issue = [&](int stage, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int b = wave * 8 + i;  // 64 blocks per stage: tile 4*stage + b/16, k-step b%16
      const int t = kQkvTps * stage + (b >> 4);
      if (t < kQkvgTiles) lds_load_block(wq + (int64_t(t) * 16 + (b & 15)) * 64, &lds[buf][b * 64], lane);
    }
  };
  issue(u_begin % kQkvStages, u_begin & 1);

#pragma unroll 1
  for (int u = u_begin; u < u_end;) {
    const int blk = u / kQkvStages, st0 = u - blk * kQkvStages;
    const int st1 = min(kQkvStages, st0 + (u_end - u));  // this block's stages st0 .. st1 - 1
    const int64_t row0 = (int64_t(blk) * kQkvWaves + wave) * 32;
    const bool active = row0 < int64_t(nseq) * Lpad;  // inactive waves still stage weights and meet barriers
    const int s = active ? int(row0 / Lpad) : 0;
    const int p = active ? int(row0 % Lpad) + j : 0;
    const bool valid = active && p < L;
    const int64_t tok = valid ? token_of(mode, s, p, T, F) : 0;

    u32x4 bx[16];
    {
      const u32x4* xr = reinterpret_cast<const u32x4*>(xn + tok * kDim);
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) bx[ks] = valid ? xr[2 * ks + hh] : zero4();
    }
    // Rotary of this position: features d0 = 32 half + 8g + 4hh (+0..3) form the pairs
    // i = 16 half + 4g + 2hh + c, c = 0, 1.  rope = [cos | sin] rows of 32.
    float2 rc[2][4], rsn[2][4];
    {
      const float* cr = rope + int64_t(valid ? p : 0) * 32;
      const float* sr = cr + int64_t(L) * 32;
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          rc[half][g] = *reinterpret_cast<const float2*>(cr + 16 * half + 4 * g + 2 * hh);
          rsn[half][g] = *reinterpret_cast<const float2*>(sr + 16 * half + 4 * g + 2 * hh);
        }
    }

    // q/k rows are chunk-major: features 8c..8c+7 of position p at ((s*8 + h)*8 + c)*Lpad + p, so the 32
    // lanes of a half-wave store 32 consecutive 16-byte chunks (hh fills bytes 8hh..8hh+7).
    const int64_t qk_off = (int64_t(s) * kHeads * 8 * Lpad + p) * 8 + 4 * hh;
    // V^T rows: lane 4q + r of a half-wave stores row r of its register group at positions 4q..4q+3
    const int64_t v_off = (int64_t(s) * kHeads * kHeadDim + 4 * hh + qd) * Lpad + (p & ~3);
    u32x2 pend[kQkvGroupStores];  // the previous group's packed outputs

    // Store i of the outputs of group grp of stage ps: tile 4ps + 2grp + i/4, register group i%4.  Every
    // offset beyond the lane's own is wave-uniform.
    auto store_pending = [&](int ps, int grp, int i) __attribute__((always_inline)) {
      const int tt = 2 * grp + (i >> 2), g = i & 3, t = kQkvTps * ps + tt, half = tt & 1;
      if (ps < 8) {
        const int h = (t & 15) >> 1;
        uint16_t* base = (ps < 4 ? Q : K) + qk_off;
        const int64_t off = int64_t(__builtin_amdgcn_readfirstlane((h * 8 + 4 * half + g) * Lpad)) * 8;
        *reinterpret_cast<u32x2*>(base + off) = pend[i];
      } else {
        const int h = (t - 32) >> 1;
        const int drow = h * kHeadDim + 32 * half + 8 * g;  // row of V^T, less 4hh + r
        *reinterpret_cast<u32x2*>(Vt + v_off + int64_t(__builtin_amdgcn_readfirstlane(drow * Lpad))) = pend[i];
      }
    };
    // Everything loaded so far has landed (the block's first stage barrier waits for it anyway): stated
    // as the builtin so that the compiler's own waitcnt insertion, which cannot tell the barrier branches
    // below apart, adds no waits for the xn and rotary registers inside the stage loop.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
#pragma unroll 1
    for (int stage = st0; stage < st1; ++stage, ++u) {
      // This stage's weight loads were issued at the top of the previous unit, whose two loops then
      // issued 8 stores each (only the second loop in a block's first stage); a block's first stage
      // follows the xn and rotary loads and waits for everything.
      if (active && stage >= st0 + 2)
        vmcnt_barrier<2 * kQkvGroupStores>();
      else if (active && stage == st0 + 1)
        vmcnt_barrier<kQkvGroupStores>();
      else
        vmcnt_barrier<0>();
      if (u + 1 < u_end) issue((u + 1) % kQkvStages, (u + 1) & 1);
      if (!active) continue;
      const u32x4* Ls = lds[u & 1];
      if (stage == kQkvStages - 1) {  // the gate tile: rows 0..7 live in register group 0 of both half-waves
        f32x16 acc = zero16();
        const bool pending = stage > st0;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
          acc = mfma32(Ls[ks * 64 + lane], bx[ks], acc);
          if ((ks & 1) && pending) store_pending(stage - 1, 1, ks >> 1);
        }
        if (valid) {
          const f32x4 bg = *reinterpret_cast<const f32x4*>(bgate + 4 * hh);
          f32x4 gv;
#pragma unroll
          for (int r = 0; r < 4; ++r) gv[r] = 1.0f / (1.0f + expf(-(acc[r] + bg[r])));
          *reinterpret_cast<f32x4*>(G + tok * kHeads + 4 * hh) = gv;
        }
        continue;
      }
#pragma unroll
      for (int grp = 0; grp < 2; ++grp) {
        f32x16 acc[2];
        u32x4 a[2];
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          acc[v] = zero16();
          a[v] = Ls[(2 * grp + v) * 16 * 64 + lane];
        }
        const bool pending = grp == 1 || stage > st0;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {  // operands of k-step ks+1 are read while ks multiplies
          u32x4 an[2];
#pragma unroll
          for (int v = 0; v < 2; ++v)
            if (ks + 1 < 16) an[v] = Ls[((2 * grp + v) * 16 + ks + 1) * 64 + lane];
#pragma unroll
          for (int v = 0; v < 2; ++v) acc[v] = mfma32(a[v], bx[ks], acc[v]);
          if ((ks & 1) && pending) store_pending(grp ? stage : stage - 1, grp ^ 1, ks >> 1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int v = 0; v < 2; ++v)
            if (ks + 1 < 16) a[v] = an[v];
        }
        if (stage < 8) {  // q (stages 0-3) or k (4-7): rotate interleaved pairs in fp32, pack bf16 rows
          // q leaves in units of log2(e) (scores become base-2 exponents for the softmax); k as is
          const float sc = stage < 4 ? kLog2e : 1.0f;
#pragma unroll
          for (int v = 0; v < 2; ++v) {
            const int half = v;  // tiles 2grp and 2grp+1 are halves 0 and 1 of one head
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const float2 c = rc[half][g], sn = rsn[half][g];
              const float a0 = acc[v][4 * g], a1 = acc[v][4 * g + 1], a2 = acc[v][4 * g + 2], a3 = acc[v][4 * g + 3];
              u32x2 o = {0u, 0u};
              if (valid) {
                o[0] = pk_bf16(fmaf(a0, c.x, -(a1 * sn.x)) * sc, fmaf(a1, c.x, a0 * sn.x) * sc);
                o[1] = pk_bf16(fmaf(a2, c.y, -(a3 * sn.y)) * sc, fmaf(a3, c.y, a2 * sn.y) * sc);
              }
              pend[4 * v + g] = o;
            }
          }
        } else {  // v: register group g holds rows 8g + 4hh + r (r = 0..3) of position p; a 4 x 4
          // transpose across each lane quad (two DPP exchanges) leaves lane 4q + r with row r of
          // positions 4q..4q+3, so a half-wave's store covers 4 rows x 64 contiguous bytes.
          const bool b1 = qd & 2, b0 = qd & 1;
          // byte selectors of v_perm_b32 (bytes 0-3 from the second operand, 4-7 from the first)
          const uint32_t sel_send = b0 ? 0x05040100u : 0x07060302u;
          const uint32_t sel_f0 = b0 ? 0x03020504u : 0x05040100u;
          const uint32_t sel_f1 = b0 ? 0x03020706u : 0x07060100u;
#pragma unroll
          for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              // d0/d1: rows (0,1)/(2,3) of this position (zero past the sequence end)
              const uint32_t d0 = valid ? pk_bf16(acc[v][4 * g], acc[v][4 * g + 1]) : 0u;
              const uint32_t d1 = valid ? pk_bf16(acc[v][4 * g + 2], acc[v][4 * g + 3]) : 0u;
              // exchange with lane ^ 2: lanes 0,1 keep rows 0,1 of positions q, q+2; lanes 2,3 rows 2,3
              const uint32_t r1 = uint32_t(__builtin_amdgcn_update_dpp(0, int(b1 ? d0 : d1), 0x4E, 0xF, 0xF, true));
              const uint32_t e0 = b1 ? r1 : d0, e1 = b1 ? d1 : r1;
              // exchange halves with lane ^ 1: lane r ends with row r of positions 0..3
              const uint32_t snd = __builtin_amdgcn_perm(e1, e0, sel_send);
              const uint32_t r2 = uint32_t(__builtin_amdgcn_update_dpp(0, int(snd), 0xB1, 0xF, 0xF, true));
              pend[4 * v + g] = u32x2{__builtin_amdgcn_perm(r2, e0, sel_f0), __builtin_amdgcn_perm(r2, e1, sel_f1)};
            }
        }
      }
    }
    // a block left before its gate stage: its last group's outputs leave now
    if (active && st1 < kQkvStages) {
#pragma unroll
      for (int i = 0; i < kQkvGroupStores; ++i) store_pending(st1 - 1, 1, i);
    }
  }
}

int device_cu_count() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Workgroups of the QKV kernel: one per CU (the kernel deals its units itself), at most one per unit.
static int qkv_grid(int units) {
  const int n = device_cu_count();
  return units < n ? units : n;
}

void launch_qkv(const uint16_t* xn, const uint8_t* layer, const float* rope, const SeqShape& sh, uint16_t* Q,
                uint16_t* K, uint16_t* Vt, float* G, hipStream_t st, const LaunchEvents& ev) {
  const int64_t rows = int64_t(sh.nseq) * sh.Lpad;
  const int nblocks = int((rows / 32 + kQkvWaves - 1) / kQkvWaves);
  if (nblocks <= 0) return;
  hipExtLaunchKernelGGL(k_qkv_rope, dim3(unsigned(qkv_grid(nblocks * kQkvStages))), dim3(64 * kQkvWaves), 0, st,
                        ev.start, ev.stop, 0, xn, reinterpret_cast<const u32x4*>(layer + kOffQkvg),
                        reinterpret_cast<const float*>(layer + kOffBgate), rope, sh.mode, sh.nseq, sh.L, sh.Lpad,
                        sh.T, sh.F, nblocks, Q, K, Vt, G);
}


// ============================================================ attention
// S^T = K . Q^T puts keys on MFMA rows and queries on columns.  Key rows are loaded in the
// order pi(i) (bits 2 and 3 of i swapped) so that register r of half-wave hh holds key
//     key_of(r, hh) = (r < 8 ? 8*hh + r : 16 + 8*hh + (r - 8))
// of its 32-key block: registers 0..7 / 8..15 are then exactly the 8 consecutive keys that
// lane supplies as the B operand (P^T) of the two 16-key PV instructions O^T += V^T . P^T.
__device__ __forceinline__ int key_perm(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }
__device__ __forceinline__ int key_of(int r, int hh) { return r < 8 ? 8 * hh + r : 8 + 8 * hh + r; }

// Exact softmax of one 32-query x 32-key score block held as S^T registers.
// Returns the unnormalised bf16 probabilities as two B operands and adds the fp32 sum.
// Scores are in units of log2(e) (q is pre-scaled), so e = 2^(s - m); with shift = 0 the caller has
// already subtracted the row max inside the MFMA accumulator.
__device__ __forceinline__ void softmax_block(const f32x16& sacc, int key0, int L, int hh, float shift, float& lsum,
                                              u32x4& p0, u32x4& p1) {
  float e[16];
  if (key0 + 32 <= L) {
#pragma unroll
    for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_exp2f(sacc[r] - shift);
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      e[r] = (key0 + key_of(r, hh) < L) ? __builtin_amdgcn_exp2f(sacc[r] - shift) : 0.f;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) lsum += e[r];
  p0[0] = pk_bf16(e[0], e[1]);
  p0[1] = pk_bf16(e[2], e[3]);
  p0[2] = pk_bf16(e[4], e[5]);
  p0[3] = pk_bf16(e[6], e[7]);
  p1[0] = pk_bf16(e[8], e[9]);
  p1[1] = pk_bf16(e[10], e[11]);
  p1[2] = pk_bf16(e[12], e[13]);
  p1[3] = pk_bf16(e[14], e[15]);
}

// The same probabilities for the single-sweep kernel, whose normaliser is the sum of the bf16-rounded P
// (the weights P.V actually applies), formed on the matrix pipe instead of by 16 VALU adds per block:
// v_mfma_f32_16x16x32_bf16 with A = `ones` and B = the P^T operand.  B lane l is column n = l % 16 and
// k-group l / 16; the P^T registers of lane l belong to query l % 32 = n + 16 ((l / 16) & 1), half
// (l / 32) of the keys.  A row 0 is 1 on k-groups 0 and 2 and row 1 on k-groups 1 and 3, so D row 0,
// column n (lane n, register 0) collects query n's 16 keys and row 1 (lane n, register 1) query n + 16's;
// the other rows stay 0.
__device__ __forceinline__ u32x4 rowsum_ones(int lane) {
  const int m = lane & 15, g = (lane >> 4) & 1;
  const uint32_t one = (m == 0 && g == 0) || (m == 1 && g == 1) ? 0x3f803f80u : 0u;
  return u32x4{one, one, one, one};
}

__device__ __forceinline__ f32x4 mfma16_rowsum(u32x4 ones, u32x4 p, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ones), __builtin_bit_cast(bf16x8, p), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ void softmax_block_psum(const f32x16& sacc, int key0, int L, int hh, const u32x4& ones,
                                                   f32x4& psum, u32x4& p0, u32x4& p1) {
  float e[16];
  if (key0 + 32 <= L) {
#pragma unroll
    for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_exp2f(sacc[r]);
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) e[r] = (key0 + key_of(r, hh) < L) ? __builtin_amdgcn_exp2f(sacc[r]) : 0.f;
  }
  p0 = u32x4{pk_bf16(e[0], e[1]), pk_bf16(e[2], e[3]), pk_bf16(e[4], e[5]), pk_bf16(e[6], e[7])};
  p1 = u32x4{pk_bf16(e[8], e[9]), pk_bf16(e[10], e[11]), pk_bf16(e[12], e[13]), pk_bf16(e[14], e[15])};
  psum = mfma16_rowsum(ones, p0, psum);
  psum = mfma16_rowsum(ones, p1, psum);
}

// Query j's sum from the row-sum accumulator (j = lane % 32; both half-waves get it).
__device__ __forceinline__ float psum_of_query(const f32x4& psum, int j) {
  const float a = __shfl(psum[0], j & 15), b = __shfl(psum[1], j & 15);
  return j < 16 ? a : b;
}

__device__ __forceinline__ float block_max(const f32x16& sacc, int key0, int L, int hh, float m) {
  if (key0 + 32 <= L) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) m = fmaxf(fmaxf(m, sacc[r]), sacc[r + 1]);  // one v_max3_f32 per pair
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (key0 + key_of(r, hh) < L) m = fmaxf(m, sacc[r]);
  }
  return m;
}

// Epilogue: O[tok][h*64 + d] = bf16(acc * gate / sum), 4 consecutive features per store.
__device__ __forceinline__ void attn_store(const f32x16 (&o)[2], int q, int L, int s, int h, int hh, int mode, int T,
                                           int F, const float* __restrict__ G, float lsum,
                                           uint16_t* __restrict__ O) {
  if (q >= L) return;
  const int64_t tok = token_of(mode, s, q, T, F);
  const float sc = G[tok * kHeads + h] * (1.0f / lsum);
  uint16_t* dst = O + tok * (kHeads * kHeadDim) + h * kHeadDim;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dt + row_of_group(g, hh);
      u32x2 v = {pk_bf16(o[dt][4 * g] * sc, o[dt][4 * g + 1] * sc),
                 pk_bf16(o[dt][4 * g + 2] * sc, o[dt][4 * g + 3] * sc)};
      *reinterpret_cast<u32x2*>(dst + d0) = v;
    }
}

// Long sequences (time attention, L up to a few thousand).  The reference's exact, non-online softmax
// (kernels.cpp:286-384) first finds the row max m, then forms e = 2^(s - m) (q carries the factor
// log2(e), so scores are base-2 exponents), sums e in fp32, rounds P = e to bf16 unnormalised and
// accumulates P.V; the epilogue scales by gate/sum.  Here one sweep over the keys does the same with an
// integer shift c in place of m, fixed from the first 32 keys (see kAttHeadroomFast): a power-of-two
// shift changes neither the bf16 rounding of P nor the normalised result, QK^T is computed once instead of
// twice, and no max is taken after the first keys; a workgroup whose sums overflow redoes the sweep with
// a shift raised as scores exceed it.
// The normaliser is the fp32 sum of the rounded P (on the matrix pipe, softmax_block_psum) rather than
// of e.  With the row max the dominant key's P is exactly 1 and escapes bf16 rounding; with an integer
// shift it is rounded like the others, and dividing by the sum of the weights P.V actually applied makes
// up for that: against exact attention the result is within ~0.5 dB of the reference's arithmetic on
// peaked rows, where the sum of e leaves it 2-3 dB below.
// One workgroup = one (sequence, head) and 4 waves x 64 queries; each wave holds two 32-query column
// tiles, so every K or V^T operand read from LDS feeds two MFMAs.  Tiles of 64 keys of K and V^T stream
// through a ring of LDS buffers, loaded global->LDS directly (V^T with the XOR swizzle of its 16-byte
// chunks applied through each lane's source address, for bank-conflict-free operand reads).  Only the
// last key tile can hold keys >= L, so the masked code runs once.
constexpr int kAttWaves = 4;
constexpr int kAttQT = 2;                       // 32-query column tiles per wave
constexpr int kAttBlockQ = kAttWaves * 32 * kAttQT;  // queries per workgroup

// Physical 16-byte chunk of logical chunk c in LDS row R is c ^ chunk_swz(R).  Operand reads touch
// rows R0..R0+31 at one logical chunk; with 64 four-byte banks (two 128-byte rows per bank sweep) this
// pattern is conflict-free for every group of 16 lanes (and for groups of 8 with 32 banks).
__device__ __forceinline__ int chunk_swz(int R) { return (R & 7) ^ ((R >> 3) & 1); }

// This wave's share of staging one 8 KB K tile into LDS, chunk-major like K itself: LDS block c
// (64 rows x 16 B) holds features 8c..8c+7 of the tile's 64 keys, row R = key (R&32)|pi(R&31).  Wave w
// stages chunks 2w and 2w+1, one 1 KB instruction each (64 consecutive rows of one chunk plane).
__device__ __forceinline__ void stage_k_tile(__amdgpu_buffer_rsrc_t kres, int kt, int Lpad, u32x4* lds_tile,
                                             int wave, int lane) {
  const int key = (lane & 32) | key_perm(lane & 31);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = 2 * wave + i;
    buffer_load_lds16(kres, (c * Lpad + kt * 64 + key) * 16, lds_tile + c * 64);
  }
}

// This wave's share of staging one 8 KB V^T tile (64 rows x 8 chunks of 16 B) into LDS: rows
// 16w..16w+15 (two instructions of 8 rows).  Row R holds head feature R.
__device__ __forceinline__ void stage_v_tile(__amdgpu_buffer_rsrc_t vres, int kt, int Lpad, u32x4* lds_tile,
                                             int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int R = 16 * wave + 8 * i + (lane >> 3), pc = lane & 7;
    buffer_load_lds16(vres, (R * Lpad + kt * 64 + 8 * (pc ^ chunk_swz(R))) * 2, lds_tile + (16 * wave + 8 * i) * 8);
  }
}

// K operands of one 32-key half of a tile (chunk 2ks+hh of rows 32kh..32kh+31: 16 lanes read 256
// consecutive bytes, so the chunk-major tile needs no swizzle).
__device__ __forceinline__ void load_k_half(const u32x4* __restrict__ Kl, int kh, int j, int hh, u32x4 (&ka)[4]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ka[ks] = Kl[(2 * ks + hh) * 64 + 32 * kh + j];
}

// Softmax shift of the single pass.  Scores are base-2 exponents and the shift c of a query is an
// integer.  With an integer shift, P = bf16(2^(s-c)) = 2^-c bf16(2^s), so the normalised result does not
// depend on which integer c is (up to the fp32 rounding of s - c), as long as nothing over- or
// underflows: it is the non-online softmax of the reference with the row max m replaced by an integer,
// which only moves P's bf16 rounding by a factor 2^(m - c) that is a power of two times 2^(m - ceil m).
//
// The sweep therefore takes c once, from the first 32 keys, kAttHeadroomFast above their max, and
// computes 2^(s - c) for every later key with no max at all.  Keys far below c underflow only past
// 2^-126, i.e. more than ~94 below the first keys' max, where their weight is below fp32 resolution
// anyway.  A key far above c (more than ~60 above the first keys' max) would overflow the sums: the
// sweep checks every row's sum against kAttSafeSum (and O for finiteness) at the end, and if any row of
// the workgroup fails, the workgroup redoes the sweep with the guarded shift: c raised (never lowered)
// whenever a score exceeds it, to kAttHeadroom above the running max, with the earlier probabilities,
// their sum and the P.V accumulators scaled by 2^-d (exact).
constexpr float kAttHeadroom = 8.0f;       // guarded sweep
constexpr float kAttHeadroomFast = 32.0f;  // fixed-shift sweep
constexpr float kAttSafeSum = 1099511627776.0f;  // 2^40: fixed-shift sums at most this leave O finite

// One 32-key half of a tile for one 32-query column tile: S^T = K.Q^T accumulated onto -c, then
// P = 2^(s - c) as two B operands and the fp32 sum.  FIRST (the first half of tile 0, 32 valid keys) sets c
// from its own row max; SAFE (the guarded sweep) raises c when a score exceeds it.
template <bool FIRST, bool MASK, bool SAFE>
__device__ __forceinline__ void attn_half(const u32x4 (&ka)[4], const u32x4 (&qb)[4], int key0, int L, int hh,
                                          const u32x4& ones, f32x16& negc, f32x4& psum, f32x16 (&o)[2], u32x4& p0,
                                          u32x4& p1) {
  f32x16 sacc = FIRST ? zero16() : negc;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) sacc = mfma32(ka[ks], qb[ks], sacc);
  float hm = 0.f;
  if (FIRST || SAFE) {
    hm = MASK ? block_max(sacc, key0, L, hh, -INFINITY) : block_max(sacc, 0, 32, hh, -INFINITY);
    hm = halfwave_max(hm);  // the query's 32 keys sit in lanes j and j + 32
  }
  if (FIRST) {
    const float c = ceilf(hm) + (SAFE ? kAttHeadroom : kAttHeadroomFast);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      negc[r] = -c;
      sacc[r] -= c;
    }
  } else if (SAFE && __any(hm > 0.f)) {  // a score above the shift somewhere in the wave (rare)
    const float d = hm > 0.f ? ceilf(hm) + kAttHeadroom : 0.f;
    const int di = int(d);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      negc[r] -= d;
      sacc[r] -= d;
    }
    // the row-sum accumulator of lane n < 16 holds queries n (register 0) and n + 16 (register 1)
    const int di16 = __shfl(di, (__lane_id() & 15) + 16);
    psum[0] = ldexpf(psum[0], -di);
    psum[1] = ldexpf(psum[1], -di16);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = ldexpf(o[dt][r], -di);
  }
  softmax_block_psum(sacc, MASK ? key0 : 0, MASK ? L : 32, hh, ones, psum, p0, p1);
}

// One 64-key tile: per 32-key half, scores and probabilities for both query tiles, then P.V.
template <bool FIRST, bool MASK, bool SAFE>
__device__ __forceinline__ void attn_tile(const u32x4* __restrict__ Kl, const u32x4* __restrict__ Vl,
                                          const u32x4 (&qb)[kAttQT][4], int key0, int L, int j, int hh,
                                          const u32x4& ones, f32x16 (&negc)[kAttQT], f32x4 (&psum)[kAttQT],
                                          f32x16 (&o)[kAttQT][2]) {
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    u32x4 ka[4];
    load_k_half(Kl, kh, j, hh, ka);
    u32x4 p0[kAttQT], p1[kAttQT];
#pragma unroll
    for (int qt = 0; qt < kAttQT; ++qt) {
      if (FIRST && kh == 0)
        attn_half<true, false, SAFE>(ka, qb[qt], 0, L, hh, ones, negc[qt], psum[qt], o[qt], p0[qt], p1[qt]);
      else
        attn_half<false, MASK, SAFE>(ka, qb[qt], key0 + 32 * kh, L, hh, ones, negc[qt], psum[qt], o[qt], p0[qt],
                                     p1[qt]);
    }
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int d = 32 * dt + j;
      const u32x4 v0 = Vl[d * 8 + ((4 * kh + hh) ^ chunk_swz(d))];
      const u32x4 v1 = Vl[d * 8 + ((4 * kh + 2 + hh) ^ chunk_swz(d))];
#pragma unroll
      for (int qt = 0; qt < kAttQT; ++qt) {
        o[qt][dt] = mfma32(v0, p0[qt], o[qt][dt]);
        o[qt][dt] = mfma32(v1, p1[qt], o[qt][dt]);
      }
    }
  }
}

// K/V tiles stream through a ring of kAttBufs LDS buffers, prefetched kAttBufs-1 tiles ahead.  Tile kt
// is ready once at most the loads of the tiles issued after it are outstanding (N per tile per wave:
// 2 for a K tile, 4 for K + V), and the barrier makes every wave's share visible.
constexpr int kAttBufs = 3;

__global__ __launch_bounds__(256, 2) void k_attn_long(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                                                   const uint16_t* __restrict__ Vt, const float* __restrict__ G,
                                                   uint16_t* __restrict__ O, int mode, int L, int Lpad, int T,
                                                   int F, int nqb) {
  __shared__ u32x4 lds[kAttBufs][2][64 * 8];  // [buffer][K, V^T][64 rows x 8 chunks]
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  // XCD-aware order: workgroups are dealt round-robin to the 8 XCDs (8 L2 caches), so block b runs on
  // XCD b % 8.  Give all query blocks of one (sequence, head) consecutive slots of one XCD, so its K and
  // V^T are fetched from HBM once into that XCD's L2 (nseq * 8 heads is a multiple of 8).
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;  // grid = nseq * 8 * nqb blocks
  const int sh = xcd + 8 * (slot / nqb), qblk = slot % nqb;
  const int s = sh >> 3, h = sh & 7;
  const uint16_t* Qh = Q + int64_t(sh) * Lpad * kHeadDim;
  // K and V^T of this (sequence, head) as buffer resources for the direct-to-LDS tile loads.
  const __amdgpu_buffer_rsrc_t Kh = buffer_rsrc(K + int64_t(sh) * Lpad * kHeadDim, Lpad * kHeadDim * 2);
  const __amdgpu_buffer_rsrc_t Vh = buffer_rsrc(Vt + int64_t(sh) * kHeadDim * Lpad, Lpad * kHeadDim * 2);
  const int q0 = qblk * kAttBlockQ + wave * 32 * kAttQT;
  const bool active = q0 < L;  // idle waves still stage tiles and meet every barrier

  u32x4 qb[kAttQT][4];
#pragma unroll
  for (int qt = 0; qt < kAttQT; ++qt) {
    const int q = q0 + 32 * qt + j;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qb[qt][ks] = q < Lpad ? *reinterpret_cast<const u32x4*>(Qh + (int64_t(2 * ks + hh) * Lpad + q) * 8) : zero4();
  }

  const int nkt = Lpad / 64;  // >= 2: this kernel runs for L > 64
  const u32x4 ones = rowsum_ones(lane);
  f32x4 psum[kAttQT];
  f32x16 negc[kAttQT], o[kAttQT][2];
  auto sweep = [&](auto safe_tag) {
    constexpr bool SAFE = decltype(safe_tag)::value;
#pragma unroll
    for (int qt = 0; qt < kAttQT; ++qt) {
      psum[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
      negc[qt] = o[qt][0] = o[qt][1] = zero16();
    }
#pragma unroll
    for (int i = 0; i < kAttBufs - 1; ++i)
      if (i < nkt) {
        stage_k_tile(Kh, i, Lpad, lds[i][0], wave, lane);
        stage_v_tile(Vh, i, Lpad, lds[i][1], wave, lane);
      }
    vmcnt_barrier<4 * (kAttBufs - 2)>();  // tile 0 (nkt >= 2 >= kAttBufs - 1)
    if (kAttBufs - 1 < nkt) {
      stage_k_tile(Kh, kAttBufs - 1, Lpad, lds[kAttBufs - 1][0], wave, lane);
      stage_v_tile(Vh, kAttBufs - 1, Lpad, lds[kAttBufs - 1][1], wave, lane);
    }
    if (active) attn_tile<true, false, SAFE>(lds[0][0], lds[0][1], qb, 0, L, j, hh, ones, negc, psum, o);
    for (int kt = 1; kt < nkt - 1; ++kt) {
      if (kt + kAttBufs - 2 < nkt)  // K and V: 4 loads per younger tile in flight
        vmcnt_barrier<4 * (kAttBufs - 2)>();
      else
        vmcnt_barrier<0>();
      if (kt + kAttBufs - 1 < nkt) {
        const int b = (kt + kAttBufs - 1) % kAttBufs;
        stage_k_tile(Kh, kt + kAttBufs - 1, Lpad, lds[b][0], wave, lane);
        stage_v_tile(Vh, kt + kAttBufs - 1, Lpad, lds[b][1], wave, lane);
      }
      if (active)
        attn_tile<false, false, SAFE>(lds[kt % kAttBufs][0], lds[kt % kAttBufs][1], qb, 0, L, j, hh, ones, negc,
                                      psum, o);
    }
    vmcnt_barrier<0>();
    if (active)
      attn_tile<false, true, SAFE>(lds[(nkt - 1) % kAttBufs][0], lds[(nkt - 1) % kAttBufs][1], qb, (nkt - 1) * 64, L,
                                   j, hh, ones, negc, psum, o);
  };
  sweep(std::integral_constant<bool, false>{});
  // Overflow check of the fixed-shift sweep (a key far above the first ones): the guarded sweep again,
  // by the whole workgroup (it streams K/V through the shared LDS ring), if any of its rows failed.
  bool bad = false;
#pragma unroll
  for (int qt = 0; qt < kAttQT; ++qt) {
    bad |= !(psum_of_query(psum[qt], j) <= kAttSafeSum);
    float om = 0.f;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) om = fmaxf(om, fabsf(o[qt][dt][r]));
    bad |= !(om <= 3.0e38f);
  }
  if (__syncthreads_or(active && bad)) sweep(std::integral_constant<bool, true>{});
  if (!active) return;
#pragma unroll
  for (int qt = 0; qt < kAttQT; ++qt)
    attn_store(o[qt], q0 + 32 * qt + j, L, s, h, hh, mode, T, F, G, psum_of_query(psum[qt], j), O);
}

// Short sequences (frequency attention, L <= 64).  One wave = one (sequence, head): all
// operands come straight from global memory into registers, the whole 64x64 score block is
// computed once, so the exact softmax needs a single pass.
__global__ __launch_bounds__(256) void k_attn_short(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                                                    const uint16_t* __restrict__ Vt, const float* __restrict__ G,
                                                    uint16_t* __restrict__ O, int mode, int nsh, int L, int T,
                                                    int F) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int sh = blockIdx.x * 4 + wave;
  if (sh >= nsh) return;
  const int s = sh >> 3, h = sh & 7;
  constexpr int Lp = 64;
  const uint16_t* Qh = Q + int64_t(sh) * Lp * kHeadDim;
  const uint16_t* Kh = K + int64_t(sh) * Lp * kHeadDim;
  const uint16_t* Vh = Vt + int64_t(sh) * kHeadDim * Lp;

  u32x4 ka[2][4], va[2][4];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      ka[kh][ks] = *reinterpret_cast<const u32x4*>(Kh + (int64_t(2 * ks + hh) * Lp + 32 * kh + key_perm(j)) * 8);
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
      va[dt][kc] = reinterpret_cast<const u32x4*>(Vh + int64_t(32 * dt + j) * Lp)[2 * kc + hh];

#pragma unroll 1
  for (int qt = 0; qt < 2; ++qt) {
    const int q = 32 * qt + j;
    if (32 * qt >= L) break;
    u32x4 qb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qb[ks] = *reinterpret_cast<const u32x4*>(Qh + (int64_t(2 * ks + hh) * Lp + q) * 8);
    f32x16 sacc[2];
    float m = -INFINITY;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      sacc[kh] = zero16();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) sacc[kh] = mfma32(ka[kh][ks], qb[ks], sacc[kh]);
      m = block_max(sacc[kh], 32 * kh, L, hh, m);
    }
    m = fmaxf(m, __shfl_xor(m, 32));
    const float ml = m;  // scores are already in units of log2(e)
    float lsum = 0.f;
    f32x16 o[2] = {zero16(), zero16()};
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      u32x4 p0, p1;
      softmax_block(sacc[kh], 32 * kh, L, hh, ml, lsum, p0, p1);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        o[dt] = mfma32(va[dt][2 * kh], p0, o[dt]);
        o[dt] = mfma32(va[dt][2 * kh + 1], p1, o[dt]);
      }
    }
    lsum += __shfl_xor(lsum, 32);
    attn_store(o, q, L, s, h, hh, mode, T, F, G, lsum, O);
  }
}

void launch_attention(const uint16_t* Q, const uint16_t* K, const uint16_t* Vt, const float* G, uint16_t* O,
                      const SeqShape& sh, hipStream_t st, const LaunchEvents& ev) {
  if (sh.L <= 64) {
    const int nsh = sh.nseq * kHeads;
    hipExtLaunchKernelGGL(k_attn_short, dim3((nsh + 3) / 4), dim3(256), 0, st, ev.start, ev.stop, 0, Q, K, Vt, G, O,
                          sh.mode, nsh, sh.L,
                       sh.T, sh.F);
  } else {
    const int nqb = (sh.L + kAttBlockQ - 1) / kAttBlockQ;
    hipExtLaunchKernelGGL(k_attn_long, dim3(sh.nseq * kHeads * nqb), dim3(64 * kAttWaves), 0, st, ev.start, ev.stop,
                          0, Q, K, Vt, G, O,
                       sh.mode, sh.L, sh.Lpad, sh.T, sh.F, nqb);
  }
}

// ============================================================ GEMM + residual + next norm
// X[tok] += A[tok] . W^T (+ b); xn[tok] = X / max(|X|, eps), for any A width K (a multiple of 16) and a
// weight W [256][K] packed in natural k order (launch_pack, kPack32Natural).  Each wave owns 32 tokens
// and all 256 output features (8 accumulator tiles), so the row norm needs one half-wave swap.
// (kernels.cpp:542-586)
__global__ __launch_bounds__(256) void k_gemm_res_norm(const uint16_t* __restrict__ A, int K,
                                                       const u32x4* __restrict__ wq, const float* __restrict__ bias,
                                                       float* __restrict__ X, uint16_t* __restrict__ xn, int64_t n,
                                                       float eps) {
  const int KS = K / 16;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int64_t tok0 = (int64_t(blockIdx.x) * 4 + wave) * 32;
  if (tok0 >= n) return;
  const int64_t tok = tok0 + j;
  const bool valid = tok < n;
  const u32x4* ar = reinterpret_cast<const u32x4*>(A + (valid ? tok : 0) * K);

  f32x16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = zero16();
  for (int ks = 0; ks < KS; ++ks) {
    const u32x4 b = valid ? ar[2 * ks + hh] : zero4();  // A[tok][16ks + 8hh .. +7]
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = mfma32(wq[(int64_t(t) * KS + ks) * 64 + lane], b, acc[t]);
  }
  if (!valid) return;  // no cross-lane traffic below except the half-wave swap of valid pairs
  float* xr = X + tok * kDim;
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int f0 = 32 * t + row_of_group(g, hh);
      f32x4 x = *reinterpret_cast<const f32x4*>(xr + f0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float y = acc[t][4 * g + r] + x[r];
        if (bias) y += bias[f0 + r];
        acc[t][4 * g + r] = y;
        x[r] = y;
        ss = fmaf(y, y, ss);
      }
      *reinterpret_cast<f32x4*>(xr + f0) = x;
    }
  ss += __shfl_xor(ss, 32);
  const float inv = 1.0f / fmaxf(sqrtf(ss), eps);
  uint16_t* nr = xn + tok * kDim;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int f0 = 32 * t + row_of_group(g, hh);
      u32x2 v = {pk_bf16(acc[t][4 * g] * inv, acc[t][4 * g + 1] * inv),
                 pk_bf16(acc[t][4 * g + 2] * inv, acc[t][4 * g + 3] * inv)};
      *reinterpret_cast<u32x2*>(nr + f0) = v;
    }
}

void launch_gemm_res_norm(const uint16_t* A, int K, const uint8_t* w_packed, const float* bias, float* X,
                          uint16_t* xn, int64_t n, float eps, hipStream_t st) {
  hipLaunchKernelGGL(k_gemm_res_norm, dim3(unsigned((n + 127) / 128)), dim3(256), 0, st, A, K,
                     reinterpret_cast<const u32x4*>(w_packed), bias, X, xn, n, eps);
}

// ============================================================ FF1 GEMM + GELU
// H = 0.5 x (1 + erf(x / sqrt 2)), x = xn . W^T + b  (nn.GELU() default, model.py:69), for a weight
// W [n_out][256] packed in natural k order (n_out a multiple of 32) and H [n][n_out].
__global__ __launch_bounds__(256) void k_gemm_gelu(const uint16_t* __restrict__ xn, const u32x4* __restrict__ wq,
                                                   const float* __restrict__ b1, int n_out,
                                                   uint16_t* __restrict__ H, int64_t n) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int64_t tok0 = (int64_t(blockIdx.x) * 4 + wave) * 32;
  if (tok0 >= n) return;
  const int64_t tok = tok0 + j;
  const bool valid = tok < n;
  const u32x4* xr = reinterpret_cast<const u32x4*>(xn + (valid ? tok : 0) * kDim);
  u32x4 bx[16];
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) bx[ks] = valid ? xr[2 * ks + hh] : zero4();  // natural k order
  uint16_t* hr = H + (valid ? tok : 0) * int64_t(n_out);
  for (int t = 0; t < n_out / 32; ++t) {
    f32x16 acc = zero16();
    const u32x4* w = wq + int64_t(t) * 16 * 64 + lane;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) acc = mfma32(w[ks * 64], bx[ks], acc);
    if (valid) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int f0 = 32 * t + row_of_group(g, hh);
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = acc[4 * g + r] + b1[f0 + r];
          v[r] = 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
        }
        u32x2 o = {pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3])};
        *reinterpret_cast<u32x2*>(hr + f0) = o;
      }
    }
  }
}

void launch_gemm_gelu(const uint16_t* xn, const uint8_t* w_packed, const float* bias, int n_out, uint16_t* H,
                      int64_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_gemm_gelu, dim3(unsigned((n + 127) / 128)), dim3(256), 0, st, xn,
                     reinterpret_cast<const u32x4*>(w_packed), bias, n_out, H, n);
}

// ============================================================ fused post-attention block
// out-projection + residual + norm, then FF1 + GELU + FF2 + residual + norm, for 32 tokens per wave
// (8 waves per workgroup, two per SIMD):
//   acc  := O . Wout^T + X                     (8 stages of 4 k-steps; X joins one 32-row tile per stage)
//   xn1  := acc / |acc|                        (FF1 B operands, in registers)
//   for each of 32 hidden tiles u:  h = b1 + xn1 . W1t^T ; acc += gelu(h) . W2t^T
//   acc  += b2 ; X := acc ; xn := acc / |acc|
// xn1 and each GELU tile go from accumulator registers straight into B operands (W1, W2 are packed in
// register order), so neither xn1 nor the 1024-wide hidden activation ever leaves the chip.
// Replaces gemm_res_norm (out) + oneDNN FF1 + gemm_res_norm (FF2) (fast.py:311-331, kernels.cpp:542-642).
constexpr int kMlpWaves = 8;
constexpr int kOutStages = 8;                // 32 k-steps of W_out, 4 per stage
constexpr int kFfStages = kHidden / 32;      // one 32-wide hidden tile per stage
constexpr int kMlpPrefetch = 4;              // LDS operands read ahead of their MFMA (out-projection)
constexpr int kMlpFfPrefetch = 2;            // the same in the feed-forward stages (registers are short)

// erf-GELU x Phi(x) = max(x, 0) - 0.5|x| erfc(|x|/sqrt 2), with erfc from Abramowitz & Stegun 7.1.26
// (|error of erf| <= 1.5e-7): erfc(z) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^(-z^2),
// t = 1/(1 + p z), p = 0.3275911.  Written in y = |x| sqrt(log2(e)/2) it is
//   0.5|x| erfc(|x|/sqrt 2) = y t P(t) 2^(-y^2),  t = 1/(1 + p' y),  p' = p / sqrt(log2 e),
//   P(t) = k (a1 + a2 t + a3 t^2 + a4 t^3 + a5 t^4),  k = 0.5 / sqrt(log2(e)/2),
// 11 VALU operations and two transcendentals; |GELU error| <= 2.2e-7 over the real line.  For x < 0 the
// result is the small erfc term itself (no cancellation).
constexpr float kGeluC = 0.84932180028801904f;   // sqrt(log2(e)/2)
constexpr float kGeluP = 0.27273748087922250f;   // 0.3275911 / sqrt(log2 e)
constexpr float kGeluA1 = 0.15001945782716460f;  // k * 0.254829592
constexpr float kGeluA2 = -0.16748465416966950f; // k * -0.284496736
constexpr float kGeluA3 = 0.83679339239730750f;  // k * 1.421413741
constexpr float kGeluA4 = -0.85547788041423880f; // k * -1.453152027
constexpr float kGeluA5 = 0.62485469502846850f;  // k * 1.061405429

__device__ __forceinline__ float gelu_erf(float x) {
  const float y = fabsf(x) * kGeluC;
  const float t = __builtin_amdgcn_rcpf(fmaf(kGeluP, y, 1.0f));
  float p = fmaf(kGeluA5, t, kGeluA4);
  p = fmaf(p, t, kGeluA3);
  p = fmaf(p, t, kGeluA2);
  p = fmaf(p, t, kGeluA1);
  const float e = __builtin_amdgcn_exp2f(-(y * y));
  return fmaf(-(y * t) * p, e, fmaxf(x, 0.0f));
}

// erf-GELU of the fp16 and bf16 feed-forward, whose output is rounded to fp16 or bf16: x Phi(x) written as
// x sigmoid(z(x)), with z(x) = x P(min(x^2, 30)) and P a cubic, a minimax fit of logit Phi(x) weighted by
// how an error in z moves the GELU (x Phi (1 - Phi)).  In base 2 (the coefficients carry log2 e):
//   gelu(x) = x / (1 + 2^(-x P(x^2)))
// 8 VALU operations and two transcendentals (the A&S form above: 11 and two); |GELU error| <= 1.25e-5
// over the real line, against fp16 rounding steps of 1.2e-4 and more for |GELU| >= 0.25.  The clamp
// keeps z monotone past |x| = 5.5, where the sigmoid has saturated: large x give x, large -x give -0.
constexpr float kGeluClamp = 30.0f;
constexpr float kGeluL0 = 2.3016500915968159f;
constexpr float kGeluL1 = 0.10597803067691149f;
constexpr float kGeluL2 = -0.0007343367166309341f;
constexpr float kGeluL3 = -2.5004358251987334e-05f;

__device__ __forceinline__ float gelu_logistic(float x) {
  const float x2 = fminf(x * x, kGeluClamp);
  float p = fmaf(kGeluL3, x2, kGeluL2);
  p = fmaf(p, x2, kGeluL1);
  p = fmaf(p, x2, kGeluL0);
  const float e = __builtin_amdgcn_exp2f(-(x * p));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float acc_inv_norm(const f32x16 (&acc)[8], float eps) {
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) ss = fmaf(acc[t][r], acc[t][r], ss);
  ss += __shfl_xor(ss, 32);
  return 1.0f / fmaxf(sqrtf(ss), eps);
}

__device__ __forceinline__ void store_row(const f32x16 (&acc)[8], float inv, float* __restrict__ xr,
                                          uint16_t* __restrict__ nr, int hh) {
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int f0 = 32 * t + row_of_group(g, hh);
      f32x4 x = {acc[t][4 * g], acc[t][4 * g + 1], acc[t][4 * g + 2], acc[t][4 * g + 3]};
      *reinterpret_cast<f32x4*>(xr + f0) = x;
      u32x2 v = {pk_bf16(x[0] * inv, x[1] * inv), pk_bf16(x[2] * inv, x[3] * inv)};
      *reinterpret_cast<u32x2*>(nr + f0) = v;
    }
}

// FF1 / FF2 operand packing and product for the two feed-forward arithmetics of k_mlp.
// F16: the two FF GEMMs take fp16 operands (xn, W1, gelu(h), W2; 11-bit significands instead of bf16's
// 8) on v_mfma_f32_32x32x16_f16 with fp32 accumulation; the out-projection stays bf16.
template <bool F16>
__device__ __forceinline__ uint32_t pk_ff(float lo, float hi) {
  return F16 ? pk_f16(lo, hi) : pk_bf16(lo, hi);
}
template <bool F16>
__device__ __forceinline__ f32x16 mfma_ff(u32x4 a, u32x4 b, f32x16 c) {
  return F16 ? mfma32h(a, b, c) : mfma32(a, b, c);
}

// This wave's 4 of stage s's 32 operand blocks into LDS.  Stages 0..7: W_out k-steps 4s..4s+3 of the
// 8 tiles.  Feed-forward stage u = s - 8 (0..32): blocks 0..15 are W1 tile u (k-steps 0..15; none for
// u = 32), blocks 16..31 W2 k-steps 2(u-1), 2(u-1)+1 of the 8 output tiles (for u = 0 k-steps 0, 1,
// loaded but not read).  Nothing for s past the last stage.
__device__ __forceinline__ void mlp_issue(int s, u32x4* dst, const u32x4* wo, const u32x4* w1, const u32x4* w2,
                                          int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int b = wave * 4 + i;
    const u32x4* src;
    if (s < kOutStages) {
      src = wo + (int64_t(b >> 2) * 32 + 4 * s + (b & 3)) * 64;  // W_out tile b/4, k-step 4s + b%4
    } else {
      const int u = s - kOutStages;
      if (b < 16) {
        if (u >= kFfStages) continue;
        src = w1 + (int64_t(u) * 16 + b) * 64;  // W1 tile u, k-step b
      } else {
        if (u > kFfStages) continue;
        src = w2 + (int64_t((b - 16) >> 1) * 64 + 2 * (u > 0 ? u - 1 : 0) + (b & 1)) * 64;  // W2 tile (b-16)/2
      }
    }
    lds_load_block(src, dst + b * 64, lane);
  }
}

// One feed-forward stage u, the same in every wave.  Stage u's LDS buffer holds W1 of hidden tile u
// (blocks 0..15, k-steps 0..15) and W2 of tile u-1 (block 16 + 2t + c: output tile t, hidden half c).
//   MFMAs 0..15:   FF1(u)   h := b1(u) + xn . W1(u)^T, one accumulator chain;
//   MFMAs 16..31:  FF2(u-1) acc[t] += gelu(h(u-1))[half c] . W2(u-1, t, c)^T, step j = 16 + 8c + t.
// GELU of the previous stage's h is spread between these MFMAs, value v after MFMA 3v/2, so that
// neither wave of a SIMD runs a long VALU-only stretch: on gfx950 VALU work of one wave overlaps the
// MFMAs of the other wave on its SIMD (measured: 65-80% of it hidden), while VALU work between a wave's
// own MFMAs is barely hidden at all.  Values 0..7 (the B operand of steps 16..23) are done by MFMA 10,
// values 8..15 by MFMA 22.
// KIND 0: the first stage (FF1(0) only); KIND 1: stages 1..31; KIND 2: the last stage (FF2(31) only).
constexpr int mlp_gelu_slot(int v) { return (3 * v) / 2; }

__device__ __forceinline__ constexpr int mlp_block_of(int m) {
  return m < 16 ? m : 16 + 2 * ((m - 16) % 8) + (m - 16) / 8;
}

template <bool F16, int KIND>
__device__ __forceinline__ void mlp_ff_pstage(const u32x4* Ls, const f32x4* b1s, const u32x4 (&xb)[16], int u,
                                              int hh, int lane, f32x16& h, f32x16 (&acc)[8]) {
  constexpr int D = kMlpFfPrefetch;
  constexpr int m0 = KIND == 2 ? 16 : 0, m1 = KIND == 0 ? 16 : 32;
  const f32x16 hp = h;  // h(u-1), the GELU input (KIND 1, 2)
  if (KIND != 2) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 b = b1s[8 * u + 2 * g + hh];  // h starts at b1
#pragma unroll
      for (int r = 0; r < 4; ++r) h[4 * g + r] = b[r];
    }
  }
  u32x4 hb[2] = {zero4(), zero4()};
  float gv[2];
  auto gelu_value = [&](int v) {
    gv[v & 1] = gelu_logistic(hp[v]);
    if (v & 1) hb[v >> 3][(v & 7) >> 1] = pk_ff<F16>(gv[0], gv[1]);
  };
  if (KIND == 2) {  // nothing to hide the first half behind
#pragma unroll
    for (int v = 0; v < 8; ++v) gelu_value(v);
  }
  u32x4 a[D];
#pragma unroll
  for (int i = 0; i < D; ++i)
    if (m0 + i < m1) a[i] = Ls[mlp_block_of(m0 + i) * 64 + lane];
#pragma unroll
  for (int m = m0; m < m1; ++m) {
    const int i = m - m0;
    if (m < 16) {
      h = mfma_ff<F16>(a[i % D], xb[m], h);
    } else {
      const int j = m - 16;
      acc[j % 8] = mfma_ff<F16>(a[i % D], hb[j / 8], acc[j % 8]);
    }
    if (m + D < m1) a[i % D] = Ls[mlp_block_of(m + D) * 64 + lane];
    if (KIND == 1) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (mlp_gelu_slot(v) == m) gelu_value(v);
    } else if (KIND == 2) {
      if (m < 24) gelu_value(8 + (m - 16));  // values 8..15 beside steps 16..23 (half 0)
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// 32 out-projection MFMAs of one stage: MFMA i -> output tile i%8, k-step i/8 of the stage (block
// 4(i%8) + i/8), operands read from LDS kMlpPrefetch ahead.
__device__ __forceinline__ void mlp_out_block(const u32x4* Ls, const u32x4 (&cur)[4], int lane, f32x16 (&acc)[8]) {
  constexpr int D = kMlpPrefetch;
  u32x4 a[D];
#pragma unroll
  for (int i = 0; i < D; ++i) a[i] = Ls[(4 * (i % 8) + i / 8) * 64 + lane];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    acc[i % 8] = mfma32(a[i % D], cur[i / 8], acc[i % 8]);
    if (i + D < 32) a[i % D] = Ls[(4 * ((i + D) % 8) + (i + D) / 8) * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The 33 feed-forward stages.  Every wave runs the same sequence; before stage u all waves meet (stage
// u's operands have landed and stage u-1's buffer is free) and stage u+1's operands are issued into
// that buffer.  Stages go in pairs so that each one's buffers are compile-time constants: the compiler
// can then tell the operand reads from the direct-to-LDS loads into the other buffer, and does not wait
// for those loads before reading.
template <bool F16>
__device__ __forceinline__ void mlp_ff_stages(f32x16 (&acc)[8], const u32x4 (&xb)[16], u32x4 (*lds)[32 * 64],
                                              const f32x4* b1s, const u32x4* wo, const u32x4* w1,
                                              const u32x4* w2, int wave, int lane, int hh) {
  constexpr int s0 = kOutStages;
  static_assert(s0 % 2 == 0 && kFfStages == 32, "stage 0 in buffer 0, stages 1..30 in pairs");
  f32x16 h = zero16();
  stage_barrier();
  mlp_issue(s0 + 1, lds[1], wo, w1, w2, wave, lane);
  mlp_ff_pstage<F16, 0>(lds[0], b1s, xb, 0, hh, lane, h, acc);
#pragma clang loop unroll(disable)
  for (int u = 1; u < kFfStages - 1; u += 2) {
    stage_barrier();
    mlp_issue(s0 + u + 1, lds[0], wo, w1, w2, wave, lane);
    mlp_ff_pstage<F16, 1>(lds[1], b1s, xb, u, hh, lane, h, acc);
    stage_barrier();
    mlp_issue(s0 + u + 2, lds[1], wo, w1, w2, wave, lane);
    mlp_ff_pstage<F16, 1>(lds[0], b1s, xb, u + 1, hh, lane, h, acc);
  }
  stage_barrier();
  mlp_issue(s0 + kFfStages, lds[0], wo, w1, w2, wave, lane);
  mlp_ff_pstage<F16, 1>(lds[1], b1s, xb, kFfStages - 1, hh, lane, h, acc);
  stage_barrier();
  mlp_ff_pstage<F16, 2>(lds[0], b1s, xb, kFfStages, hh, lane, h, acc);
}

template <bool OUTPROJ, bool FF, bool F16>
__global__ __launch_bounds__(512) void k_mlp(const uint16_t* __restrict__ O, const uint8_t* __restrict__ layer,
                                             float* __restrict__ X, uint16_t* __restrict__ xn, int64_t n, float eps) {
  // One LDS object: 2 stages x 32 operand blocks of 1 KB, then b1 (4 KB) and b2 (1 KB).  (With a second
  // __shared__ object written by direct-to-LDS loads, the compiler waits for those loads before every
  // operand read.)
  __shared__ u32x4 smem[2 * 32 * 64 + (kHidden + kDim) / 4];
  u32x4 (*lds)[32 * 64] = reinterpret_cast<u32x4 (*)[32 * 64]>(smem);
  u32x4* bias = smem + 2 * 32 * 64;
  const u32x4* wo = reinterpret_cast<const u32x4*>(layer + kOffOut);
  const u32x4* w1 = reinterpret_cast<const u32x4*>(layer + (F16 ? kOffFf1F16 : kOffFf1));
  const u32x4* w2 = reinterpret_cast<const u32x4*>(layer + (F16 ? kOffFf2F16 : kOffFf2));
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int64_t tok = (int64_t(blockIdx.x) * kMlpWaves + wave) * 32 + j;
  // Lanes past the last token work on a copy of the last token's row (every MFMA column and the
  // half-wave norm swap stay within one token) and store nothing.
  const bool valid = tok < n;
  const int64_t trow = valid ? tok : n - 1;
  float* xr = X + trow * kDim;
  uint16_t* nr = xn + trow * kDim;

  // With the out-projection, X joins the accumulators one 32-row tile per stage (its loads spread over
  // the stages instead of all waves of the chip loading it at once); without it, they start at X.
  f32x16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 x = OUTPROJ ? f32x4{0.f, 0.f, 0.f, 0.f}
                              : *reinterpret_cast<const f32x4*>(xr + 32 * t + row_of_group(g, hh));
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][4 * g + r] = x[r];
    }

  constexpr int s_begin = OUTPROJ ? 0 : kOutStages;
  constexpr int s_end = FF ? kOutStages + kFfStages + 1 : kOutStages;
  if (FF && wave < 4)  // b1 (4 KB) and b2 (1 KB) into LDS; the first stage barrier waits for them
    lds_load_block(reinterpret_cast<const u32x4*>(layer + kOffBff1) + wave * 64, &bias[wave * 64], lane);
  if (FF && wave == 4) lds_load_block(reinterpret_cast<const u32x4*>(layer + kOffBff2), &bias[kHidden / 4], lane);
  mlp_issue(s_begin, lds[0], wo, w1, w2, wave, lane);
  if (OUTPROJ) {
    const uint16_t* orow = O + trow * 512;
    u32x4 ob[4];  // O operands of the next stage
    auto load_o = [&](int s) {
#pragma unroll
      for (int i = 0; i < 4; ++i) ob[i] = reinterpret_cast<const u32x4*>(orow)[2 * (4 * s + i) + hh];
    };
    f32x4 xt[4];  // X tile of the next stage
    auto load_x = [&](int t) {
#pragma unroll
      for (int g = 0; g < 4; ++g) xt[g] = *reinterpret_cast<const f32x4*>(xr + 32 * t + row_of_group(g, hh));
    };
    load_o(0);
    load_x(0);
#pragma unroll
    for (int s = 0; s < kOutStages; ++s) {
      stage_barrier();
      if (s + 1 < s_end) mlp_issue(s + 1, lds[(s + 1) & 1], wo, w1, w2, wave, lane);
      const u32x4 cur[4] = {ob[0], ob[1], ob[2], ob[3]};
      const f32x4 xs[4] = {xt[0], xt[1], xt[2], xt[3]};
      if (s + 1 < kOutStages) {
        load_o(s + 1);
        load_x(s + 1);
      }
      mlp_out_block(lds[s & 1], cur, lane, acc);
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[s][4 * g + r] += xs[g][r];
    }
  }
  const float inv = acc_inv_norm(acc, eps);
  if (!FF) {
    if (valid) store_row(acc, inv, xr, nr, hh);
    return;
  }
  u32x4 xb[16];  // FF1 B operands: xn = X / |X| in register order, bf16 or fp16
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) {
    const int t = ks >> 1, g0 = 2 * (ks & 1);
    xb[ks] = u32x4{pk_ff<F16>(acc[t][4 * g0] * inv, acc[t][4 * g0 + 1] * inv),
                   pk_ff<F16>(acc[t][4 * g0 + 2] * inv, acc[t][4 * g0 + 3] * inv),
                   pk_ff<F16>(acc[t][4 * g0 + 4] * inv, acc[t][4 * g0 + 5] * inv),
                   pk_ff<F16>(acc[t][4 * g0 + 6] * inv, acc[t][4 * g0 + 7] * inv)};
  }
  const f32x4* bf = reinterpret_cast<const f32x4*>(bias);
  mlp_ff_stages<F16>(acc, xb, lds, bf, wo, w1, w2, wave, lane, hh);
#pragma unroll
  for (int t = 0; t < 8; ++t)  // + b2
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 b = bf[kHidden / 4 + 8 * t + 2 * g + hh];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][4 * g + r] += b[r];
    }
  const float inv2 = acc_inv_norm(acc, eps);
  if (valid) store_row(acc, inv2, xr, nr, hh);
}

// ============================================================ split-bf16 feed-forward
// Both FF GEMMs take split-bf16 operands v = hi + lo (hi = bf16(v), lo = bf16(v - hi)) and form
// hi.hi + hi.lo + lo.hi on the bf16 MFMA with fp32 accumulation; the dropped lo.lo term is ~2^-16
// relative.  xn and the GELU output are split in registers, W1 and W2 carry packed lo parts, and the
// out-projection stays bf16.  These four operands (W1, W2, xn into FF1, gelu(h)) are the rounding
// points that dominate the error of the all-bf16 design.
//
// Shape: v_mfma_f32_16x16x32_bf16 with 16 tokens per wave (output features on the 16 rows, tokens on
// the 16 columns; lane l holds token l%16 and rows 4(l/16)..+3 of a tile).  The residual stream is 16
// tiles x 4 registers and the hi and lo B operands of xn 2 x 32 registers, so a wave fits in 256
// registers and two waves share each SIMD: one wave's GELU runs while the other's MFMAs do.  A
// workgroup is 4 waves (64 tokens) with 2 x 32 KB of LDS stages, two workgroups per CU.
// Stages: 0..7 out-projection (W_out k-steps 2s, 2s+1 of all 16 tiles); then for each block j of 32
// hidden units, stage A_j = W1 hi and lo of tiles 2j, 2j+1 (FF1), and stage B_j = W2 hi and lo of
// k-step j of all 16 output tiles (GELU of block j, FF2).
constexpr int kX3Waves = 4;
constexpr int kX3OutStages = 8;
constexpr int kX3Blocks = kHidden / 32;
constexpr int kX3Stages = kX3OutStages + 2 * kX3Blocks;

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4f() {
  f32x4 z = {};
  return z;
}

__device__ __forceinline__ void split_pair(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pk_bf16(a, b);
  lo = pk_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

// Register-order B operand from two 16x16 accumulator tiles (values scaled by s): element pairs
// (tile u, rows 2q', 2q'+1) in the order of kperm16 = 16(e/4) + 4g + e%4.
__device__ __forceinline__ void split_operand(const f32x4& t0, const f32x4& t1, float s, u32x4& hi, u32x4& lo) {
  uint32_t h, l;
  split_pair(t0[0] * s, t0[1] * s, h, l);
  hi[0] = h;
  lo[0] = l;
  split_pair(t0[2] * s, t0[3] * s, h, l);
  hi[1] = h;
  lo[1] = l;
  split_pair(t1[0] * s, t1[1] * s, h, l);
  hi[2] = h;
  lo[2] = l;
  split_pair(t1[2] * s, t1[3] * s, h, l);
  hi[3] = h;
  lo[3] = l;
}

struct X3Weights {
  const u32x4* wo;   // W_out, 16x16 natural: [16 tiles][16 k-steps]
  const u32x4* w1h;  // W1 hi / lo, 16x16 register order: [64 tiles][8 k-steps]
  const u32x4* w1l;
  const u32x4* w2h;  // W2 hi / lo, 16x16 register order: [16 tiles][32 k-steps]
  const u32x4* w2l;
};

// This wave's 8 of the stage's 32 blocks into LDS buffer dst.
__device__ __forceinline__ void x3_issue(const X3Weights& w, int s, u32x4* dst, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int b = wave * 8 + i;
    const u32x4* src;
    if (s < kX3OutStages) {
      src = w.wo + (int64_t(b >> 1) * 16 + 2 * s + (b & 1)) * 64;  // tile b/2, k-step 2s + b%2
    } else {
      const int u = s - kX3OutStages, j = u >> 1;
      if ((u & 1) == 0)  // A_j: part b/16 (hi, lo), tile 2j + (b/8)%2, k-step b%8
        src = ((b < 16) ? w.w1h : w.w1l) + (int64_t(2 * j + ((b >> 3) & 1)) * 8 + (b & 7)) * 64;
      else  // B_j: part b/16, output tile b%16, k-step j
        src = ((b < 16) ? w.w2h : w.w2l) + (int64_t(b & 15) * 32 + j) * 64;
    }
    lds_load_block(src, dst + b * 64, lane);
  }
}

template <bool OUTPROJ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_mlp_x3(
    const uint16_t* __restrict__ O, const uint8_t* __restrict__ layer, float* __restrict__ X,
    uint16_t* __restrict__ xn, int64_t n, float eps) {
  __shared__ u32x4 lds[2][32 * 64];  // 2 stages x 32 operand blocks of 1 KB
  X3Weights w;
  w.wo = reinterpret_cast<const u32x4*>(layer + kOffOut16);
  w.w1h = reinterpret_cast<const u32x4*>(layer + kOffFf1Hi16);
  w.w1l = reinterpret_cast<const u32x4*>(layer + kOffFf1Lo16);
  w.w2h = reinterpret_cast<const u32x4*>(layer + kOffFf2Hi16);
  w.w2l = reinterpret_cast<const u32x4*>(layer + kOffFf2Lo16);
  const float* b1 = reinterpret_cast<const float*>(layer + kOffBff1);
  const float* b2 = reinterpret_cast<const float*>(layer + kOffBff2);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int col = lane & 15, g = lane >> 4;
  const int64_t tok = (int64_t(blockIdx.x) * kX3Waves + wave) * 16 + col;
  const bool valid = tok < n;  // lanes past the end work on the last token's row and store nothing
  const int64_t trow = valid ? tok : n - 1;
  float* xr = X + trow * kDim;
  uint16_t* nr = xn + trow * kDim;

  f32x4 acc[16];  // residual stream: tile t holds features 16t + 4g + r of this lane's token
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = *reinterpret_cast<const f32x4*>(xr + 16 * t + 4 * g);

  auto inv_norm = [&]() __attribute__((always_inline)) {
    float ss = 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) ss = fmaf(acc[t][r], acc[t][r], ss);
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    return 1.0f / fmaxf(sqrtf(ss), eps);
  };

  int s0 = OUTPROJ ? 0 : kX3OutStages;
  x3_issue(w, s0, lds[0], wave, lane);
  if (OUTPROJ) {
    const u32x4* orow = reinterpret_cast<const u32x4*>(O + trow * 512);
    u32x4 ob[2] = {orow[g], orow[4 + g]};  // k-steps 0, 1: O features 32ks + 8g..+7
    for (int s = 0; s < kX3OutStages; ++s) {
      stage_barrier();
      x3_issue(w, s + 1, lds[(s + 1) & 1], wave, lane);
      const u32x4* Ls = lds[s & 1];
      const u32x4 cur[2] = {ob[0], ob[1]};
      if (s + 1 < kX3OutStages) {
        ob[0] = orow[4 * (2 * s + 2) + g];
        ob[1] = orow[4 * (2 * s + 3) + g];
      }
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[t] = mfma16(Ls[(2 * t + kk) * 64 + lane], cur[kk], acc[t]);
    }
  }
  u32x4 xb[8], xl[8];  // FF1 B operands: xn hi and lo, k-step ks = tiles 2ks, 2ks+1 in register order
  {
    const float inv = inv_norm();
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) split_operand(acc[2 * ks], acc[2 * ks + 1], inv, xb[ks], xl[ks]);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const f32x4 b = *reinterpret_cast<const f32x4*>(b2 + 16 * t + 4 * g);
      acc[t] += b;
    }
  }

  f32x4 hs[2];  // FF1 of the current hidden block (tiles 2j, 2j+1), before bias and GELU
  for (int j = 0; j < kX3Blocks; ++j) {
    const int s = kX3OutStages + 2 * j;
    // stage A_j: FF1 of hidden tiles 2j, 2j+1
    stage_barrier();
    x3_issue(w, s + 1, lds[(s + 1) & 1], wave, lane);
    {
      const u32x4* Ls = lds[s & 1];
      f32x4 h0[2] = {zero4f(), zero4f()}, h1[2] = {zero4f(), zero4f()};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const u32x4 a = Ls[(8 * u + ks) * 64 + lane], al = Ls[(16 + 8 * u + ks) * 64 + lane];
          h0[u] = mfma16(a, xb[ks], h0[u]);
          h1[u] = mfma16(a, xl[ks], h1[u]);
          h0[u] = mfma16(al, xb[ks], h0[u]);
        }
      hs[0] = h0[0] + h1[0];
      hs[1] = h0[1] + h1[1];
    }
    // stage B_j: GELU of block j, then FF2 k-step j into every output tile
    const f32x4 bb0 = *reinterpret_cast<const f32x4*>(b1 + 32 * j + 4 * g);
    const f32x4 bb1 = *reinterpret_cast<const f32x4*>(b1 + 32 * j + 16 + 4 * g);
    stage_barrier();
    if (s + 2 < kX3Stages) x3_issue(w, s + 2, lds[s & 1], wave, lane);
    {
      const u32x4* Ls = lds[(s + 1) & 1];
      f32x4 v0, v1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v0[r] = gelu_erf(hs[0][r] + bb0[r]);
        v1[r] = gelu_erf(hs[1][r] + bb1[r]);
      }
      u32x4 hb, hl;
      split_operand(v0, v1, 1.0f, hb, hl);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const u32x4 a = Ls[t * 64 + lane], al = Ls[(16 + t) * 64 + lane];
        acc[t] = mfma16(a, hb, acc[t]);
        acc[t] = mfma16(a, hl, acc[t]);
        acc[t] = mfma16(al, hb, acc[t]);
      }
    }
  }
  const float inv = inv_norm();
  if (valid) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      *reinterpret_cast<f32x4*>(xr + 16 * t + 4 * g) = acc[t];
      const u32x2 v = {pk_bf16(acc[t][0] * inv, acc[t][1] * inv), pk_bf16(acc[t][2] * inv, acc[t][3] * inv)};
      *reinterpret_cast<u32x2*>(nr + 16 * t + 4 * g) = v;
    }
  }
}

void launch_post_attn(const uint16_t* O, const uint8_t* layer, float* X, uint16_t* xn, int64_t n, bool with_ff,
                      int ff_precision, float eps, hipStream_t st, const LaunchEvents& ev) {
  if (with_ff && ff_precision == kFfSplit) {
    const unsigned blocks = unsigned((n + 16 * kX3Waves - 1) / (16 * kX3Waves));
    hipExtLaunchKernelGGL(k_mlp_x3<true>, dim3(blocks), dim3(64 * kX3Waves), 0, st, ev.start, ev.stop, 0, O, layer, X,
                          xn, n, eps);
    return;
  }
  const unsigned blocks = unsigned((n + 32 * kMlpWaves - 1) / (32 * kMlpWaves));
  if (!with_ff)
    hipExtLaunchKernelGGL((k_mlp<true, false, false>), dim3(blocks), dim3(64 * kMlpWaves), 0, st, ev.start, ev.stop, 0, O, layer,
                          X, xn, n, eps);
  else if (ff_precision == kFfFp16)
    hipExtLaunchKernelGGL((k_mlp<true, true, true>), dim3(blocks), dim3(64 * kMlpWaves), 0, st, ev.start, ev.stop, 0, O, layer,
                          X, xn, n, eps);
  else
    hipExtLaunchKernelGGL((k_mlp<true, true, false>), dim3(blocks), dim3(64 * kMlpWaves), 0, st, ev.start, ev.stop, 0, O, layer,
                          X, xn, n, eps);
}

void launch_ff(const uint8_t* layer, float* X, uint16_t* xn, int64_t n, int ff_precision, float eps, hipStream_t st) {
  const uint16_t* none = nullptr;
  if (ff_precision == kFfSplit) {
    const unsigned blocks = unsigned((n + 16 * kX3Waves - 1) / (16 * kX3Waves));
    hipLaunchKernelGGL(k_mlp_x3<false>, dim3(blocks), dim3(64 * kX3Waves), 0, st, none, layer, X, xn, n, eps);
    return;
  }
  const unsigned blocks = unsigned((n + 32 * kMlpWaves - 1) / (32 * kMlpWaves));
  if (ff_precision == kFfFp16)
    hipLaunchKernelGGL((k_mlp<false, true, true>), dim3(blocks), dim3(64 * kMlpWaves), 0, st, none, layer, X, xn, n, eps);
  else
    hipLaunchKernelGGL((k_mlp<false, true, false>), dim3(blocks), dim3(64 * kMlpWaves), 0, st, none, layer, X, xn, n, eps);
}

}  // namespace trf
