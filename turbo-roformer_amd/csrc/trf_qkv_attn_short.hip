// Fused QKV GEMM + rotary + gates + exact softmax attention for sequences of at most 64 positions
// (frequency attention: the 62 bands of one frame), so that Q, K, V and the gates never leave the chip.
// It replaces the pair qkv_rope_gemm -> attention of the reference (kernels.cpp:439-540, 250-388) for
// short sequences, with the same arithmetic: fp32 accumulators, fp32 rotary, q times log2(e) before its
// bf16 rounding, bf16 q, k, v and unnormalised P, the exact row max over the valid keys, an fp32 sum of
// e = 2^(s - m), and O = (P.V) * gate / sum rounded to bf16 in token order.
//
// One wave owns one sequence.  Its (up to) 64 positions are two 32-token column tiles whose xn rows stay
// in registers (bf16, natural k order).  The 49 weight tiles of W_qkvg stream through LDS, shared by the
// 4 waves (sequences) of a workgroup: first the gate tile, then per head h and half c (head features
// 32c..32c+31) one stage holding the q, k and v tiles of those rows.  Every operand block read from LDS
// feeds two MFMAs (the two column tiles).
//
// No data crosses lanes between the projection and the attention:
//   * q and k come out of C = W . xn^T with lane (j, hh) holding token j of a column tile and features
//     8g + 4hh + r.  Packed to bf16 in that "register order", q is the B operand (Q^T) and k the A
//     operand (K) of S^T = K . Q^T: both use the same permutation of the 16 head features of a k-step,
//     which leaves the dot products unchanged.
//   * v comes out of the swapped product C = xn . W_v^T (the xn registers are the A operand, the packed
//     W_v block the B operand), so lane (j, hh) holds feature j of tokens 8g + 4hh + r: exactly the
//     A operand (V^T) of O^T = V^T . P^T with the keys of a k-step in the register order in which the
//     S^T accumulator holds them, so P^T is the B operand straight from the accumulator.
// The row max and the row sum combine the two half-waves (the query's keys sit in lanes j and j + 32).
#include "trf_device.h"

namespace trf {

constexpr int kFsWaves = 4;             // sequences per workgroup, one wave (and SIMD) each
constexpr int kFsStageBlocks = 48;      // q, k and v tiles of one head half: 3 x 16 k-steps of 1 KB
constexpr int kFsRopePairs = 16;        // pairs of rotary pairs per position (32 pairs)
constexpr int kFsRopeVecs = 2 * kFsRopePairs * 64;  // float2 [cos, sin][pair pair][position]

// This wave's share of the operand blocks of stage `stage` into buf: stage 0 is the gate tile (the last
// tile of W_qkvg, 16 blocks), stage 1 + 2h + c the q, k and v tiles of rows 32c..32c+31 of head h (48
// blocks: block b = 16 * kind + k-step, kind 0 q, 1 k, 2 v).
__device__ __forceinline__ void fs_issue(int stage, u32x4* buf, const u32x4* wq, int wave, int lane) {
  if (stage == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * wave + i;
      lds_load_block(wq + (int64_t(kQkvgTiles - 1) * 16 + b) * 64, buf + b * 64, lane);
    }
    return;
  }
  const int h = (stage - 1) >> 1, c = (stage - 1) & 1;
#pragma unroll
  for (int i = 0; i < kFsStageBlocks / kFsWaves; ++i) {
    const int b = (kFsStageBlocks / kFsWaves) * wave + i;
    const int t = 16 * (b >> 4) + 2 * h + c;  // q tiles 0..15, k tiles 16..31, v tiles 32..47
    lds_load_block(wq + (int64_t(t) * 16 + (b & 15)) * 64, buf + b * 64, lane);
  }
}

// One head half: q and k of head features 32c..32c+31 for both column tiles, rotated in fp32 (q times
// log2 e), added into the scores S^T; v of the same features as the V^T operands vb (k-step kv = 2 tt +
// kk2 covers keys 32 tt + 16 kk2 + {4hh + e, 8 + 4hh + e - 4}).
__device__ __forceinline__ void fs_half(const u32x4* __restrict__ Ls, const float2* __restrict__ ropeL,
                                        const u32x4 (&bx)[2][16], int c, int j, int hh, int lane,
                                        f32x16 (&sacc)[2][2], u32x4 (&vb)[4]) {
  f32x16 qa[2], ka[2], va[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) qa[t] = ka[t] = va[t] = zero16();
  u32x4 aq = Ls[lane], ak = Ls[16 * 64 + lane], av = Ls[32 * 64 + lane];
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) {  // operands of k-step ks + 1 are read while ks multiplies
    u32x4 nq, nk, nv;
    if (ks + 1 < 16) {
      nq = Ls[(ks + 1) * 64 + lane];
      nk = Ls[(16 + ks + 1) * 64 + lane];
      nv = Ls[(32 + ks + 1) * 64 + lane];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) qa[t] = mfma32(aq, bx[t][ks], qa[t]);
#pragma unroll
    for (int t = 0; t < 2; ++t) ka[t] = mfma32(ak, bx[t][ks], ka[t]);
#pragma unroll
    for (int t = 0; t < 2; ++t) va[t] = mfma32(bx[t][ks], av, va[t]);  // swapped: tokens on the rows
    __builtin_amdgcn_sched_barrier(0);
    if (ks + 1 < 16) {
      aq = nq;
      ak = nk;
      av = nv;
    }
  }
  // rotary of the interleaved pairs (r, r + 1) of rows 8g + 4hh + r: pair index 16c + 4g + 2hh + r/2
  u32x4 qb[2][2], kb[2][2];  // [column tile][k-step of this half]
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int p = 32 * t + j;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int pp = 8 * c + 2 * g + hh;
      const float2 cs = ropeL[pp * 64 + p], sn = ropeL[(kFsRopePairs + pp) * 64 + p];
      const float q0 = qa[t][4 * g], q1 = qa[t][4 * g + 1], q2 = qa[t][4 * g + 2], q3 = qa[t][4 * g + 3];
      qb[t][g >> 1][2 * (g & 1)] = pk_bf16(fmaf(q0, cs.x, -(q1 * sn.x)) * kLog2e, fmaf(q1, cs.x, q0 * sn.x) * kLog2e);
      qb[t][g >> 1][2 * (g & 1) + 1] =
          pk_bf16(fmaf(q2, cs.y, -(q3 * sn.y)) * kLog2e, fmaf(q3, cs.y, q2 * sn.y) * kLog2e);
      const float k0 = ka[t][4 * g], k1 = ka[t][4 * g + 1], k2 = ka[t][4 * g + 2], k3 = ka[t][4 * g + 3];
      kb[t][g >> 1][2 * (g & 1)] = pk_bf16(fmaf(k0, cs.x, -(k1 * sn.x)), fmaf(k1, cs.x, k0 * sn.x));
      kb[t][g >> 1][2 * (g & 1) + 1] = pk_bf16(fmaf(k2, cs.y, -(k3 * sn.y)), fmaf(k3, cs.y, k2 * sn.y));
    }
  }
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) sacc[kt][qt] = mfma32(kb[kt][kk], qb[qt][kk], sacc[kt][qt]);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      vb[2 * t + kk] = u32x4{pk_bf16(va[t][8 * kk], va[t][8 * kk + 1]), pk_bf16(va[t][8 * kk + 2], va[t][8 * kk + 3]),
                             pk_bf16(va[t][8 * kk + 4], va[t][8 * kk + 5]),
                             pk_bf16(va[t][8 * kk + 6], va[t][8 * kk + 7])};
}

// Key (or token) of register R of half-wave hh in a 32-row accumulator tile: row 8(R/4) + 4hh + R%4.
__device__ __forceinline__ int acc_row(int R, int hh) { return 8 * (R >> 2) + 4 * hh + (R & 3); }

__global__ __launch_bounds__(256, 1) void k_qkv_attn_short(const uint16_t* __restrict__ xn,
                                                          const u32x4* __restrict__ wq,
                                                          const float* __restrict__ bgate,
                                                          const float* __restrict__ rope, int mode, int nseq,
                                                          int L, int T, int F, uint16_t* __restrict__ O) {
  // One LDS object: two weight stages, then the rotary table.
  __shared__ u32x4 smem[2 * kFsStageBlocks * 64 + kFsRopeVecs / 2];
  u32x4(*lds)[kFsStageBlocks * 64] = reinterpret_cast<u32x4(*)[kFsStageBlocks * 64]>(smem);
  float2* ropeL = reinterpret_cast<float2*>(smem + 2 * kFsStageBlocks * 64);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int s = blockIdx.x * kFsWaves + wave;
  const bool active = s < nseq;  // idle waves still stage weights and meet every barrier

  fs_issue(0, lds[0], wq, wave, lane);
  // rotary table [2][L][32] fp32 -> LDS float2 [cos, sin][pair pair][position] (zero past L), so that the
  // 32 lanes of a half-wave read 32 consecutive positions of one pair pair
  for (int i = threadIdx.x; i < kFsRopeVecs; i += 64 * kFsWaves) {
    const int cs = i >> 10, pp = (i >> 6) & 15, p = i & 63;
    float2 v = {0.f, 0.f};
    if (p < L) v = *reinterpret_cast<const float2*>(rope + (int64_t(cs) * L + p) * 32 + 2 * pp);
    ropeL[i] = v;
  }
  u32x4 bx[2][16];  // xn of positions 32t + j (zero past L), natural k order
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int p = 32 * t + j;
    const bool valid = active && p < L;
    const u32x4* xr = reinterpret_cast<const u32x4*>(xn + (valid ? token_of(mode, s, p, T, F) : 0) * kDim);
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) bx[t][ks] = valid ? xr[2 * ks + hh] : zero4();
  }
  stage_barrier();  // the gate tile and the rotary table
  fs_issue(1, lds[1], wq, wave, lane);
  float gv[2][4];  // sigmoid gates of heads 4hh + r for the tokens of column tile t
  if (active) {
    f32x16 ga[2] = {zero16(), zero16()};
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const u32x4 a = lds[0][ks * 64 + lane];
#pragma unroll
      for (int t = 0; t < 2; ++t) ga[t] = mfma32(a, bx[t][ks], ga[t]);
    }
    const f32x4 bg = *reinterpret_cast<const f32x4*>(bgate + 4 * hh);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) gv[t][r] = 1.0f / (1.0f + expf(-(ga[t][r] + bg[r])));
  }

#pragma unroll 1
  for (int h = 0; h < kHeads; ++h) {
    f32x16 sacc[2][2] = {{zero16(), zero16()}, {zero16(), zero16()}};
    u32x4 vb[2][4];  // V^T operands of head features 32c + j
    stage_barrier();  // stage 1 + 2h (half 0) has landed in lds[1]; lds[0] is free
    fs_issue(2 + 2 * h, lds[0], wq, wave, lane);
    if (active) fs_half(lds[1], ropeL, bx, 0, j, hh, lane, sacc, vb[0]);
    stage_barrier();  // stage 2 + 2h (half 1) has landed in lds[0]; lds[1] is free
    if (h + 1 < kHeads) fs_issue(3 + 2 * h, lds[1], wq, wave, lane);
    if (!active) continue;
    fs_half(lds[0], ropeL, bx, 1, j, hh, lane, sacc, vb[1]);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      // exact softmax over the valid keys: row max, e = 2^(s - m) (q carries log2 e), fp32 sum, bf16 P
      float m = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int R = 0; R < 16; ++R)
          if (32 * kt + acc_row(R, hh) < L) m = fmaxf(m, sacc[kt][qt][R]);
      m = halfwave_max(m);
      float lsum = 0.f;
      u32x4 pb[4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        float e[16];
#pragma unroll
        for (int R = 0; R < 16; ++R)
          e[R] = 32 * kt + acc_row(R, hh) < L ? __builtin_amdgcn_exp2f(sacc[kt][qt][R] - m) : 0.f;
#pragma unroll
        for (int R = 0; R < 16; ++R) lsum += e[R];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          pb[2 * kt + kk] = u32x4{pk_bf16(e[8 * kk], e[8 * kk + 1]), pk_bf16(e[8 * kk + 2], e[8 * kk + 3]),
                                  pk_bf16(e[8 * kk + 4], e[8 * kk + 5]), pk_bf16(e[8 * kk + 6], e[8 * kk + 7])};
      }
      lsum += __shfl_xor(lsum, 32);
      f32x16 o[2];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        o[dt] = zero16();
#pragma unroll
        for (int kv = 0; kv < 4; ++kv) o[dt] = mfma32(vb[dt][kv], pb[kv], o[dt]);
      }
      // gate of head h for this query: in this lane if h / 4 == hh, else in the partner lane
      float own = gv[qt][0];
#pragma unroll
      for (int r = 1; r < 4; ++r) own = (h & 3) == r ? gv[qt][r] : own;
      const float other = __shfl_xor(own, 32);
      const int q = 32 * qt + j;
      if (q < L) {
        const float sc = (hh == (h >> 2) ? own : other) * (1.0f / lsum);
        uint16_t* dst = O + token_of(mode, s, q, T, F) * (kHeads * kHeadDim) + h * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const u32x2 v = {pk_bf16(o[dt][4 * g] * sc, o[dt][4 * g + 1] * sc),
                             pk_bf16(o[dt][4 * g + 2] * sc, o[dt][4 * g + 3] * sc)};
            *reinterpret_cast<u32x2*>(dst + 32 * dt + row_of_group(g, hh)) = v;
          }
      }
    }
  }
}

void launch_qkv_attn_short(const uint16_t* xn, const uint8_t* layer, const float* rope, const SeqShape& sh,
                           uint16_t* O, hipStream_t st) {
  const unsigned blocks = unsigned((sh.nseq + kFsWaves - 1) / kFsWaves);
  hipLaunchKernelGGL(k_qkv_attn_short, dim3(blocks), dim3(64 * kFsWaves), 0, st, xn,
                     reinterpret_cast<const u32x4*>(layer + kOffQkvg),
                     reinterpret_cast<const float*>(layer + kOffBgate), rope, sh.mode, sh.nseq, sh.L, sh.T, sh.F, O);
}

}  // namespace trf
