// Fused QKV GEMM + rotary + gates + exact softmax attention for sequences of at most 64 positions
// (frequency attention: the 62 bands of one frame), so that Q, K, V and the gates never leave the chip.
// It replaces the pair qkv_rope_gemm -> attention of the reference (kernels.cpp:439-540, 250-388) for
// short sequences, with the same arithmetic: fp32 accumulators, fp32 rotary, q times log2(e) before its
// bf16 rounding, bf16 q, k, v and unnormalised P, the exact row max over the valid keys, an fp32 sum of
// e = 2^(s - m), and O = (P.V) * gate / sum rounded to bf16 in token order.
//
// One wave owns one sequence.  Its (up to) 64 positions are two 32-token column tiles whose xn rows stay
// in registers (bf16, natural k order).  The 49 weight tiles of W_qkvg stream through LDS, shared by the
// 4 waves (sequences) of a workgroup: the gate tile once, then per head two stages, A (the q and k tiles,
// 64 KB) and B (the v tiles, 32 KB), each in its own LDS buffer so that one loads while the other is read.
// Every operand block read from LDS feeds two MFMAs (the two column tiles).
//
// Schedule (one wave per SIMD, so VALU work hides only under the same wave's MFMAs): stage A runs the q, k
// products of head half 0, then those of half 1 with the rotary of half 0 and the scaling and stores of
// the previous head's output spread between them, then S^T; stage B runs the v products with the
// softmax of S^T spread between them, then P.V.  O is written with bounds-checked buffer stores (lanes
// past the sequence use an out-of-range offset), always 16 per wave and head, so the barrier before the
// next stage B waits for that stage's loads with an exact vmcnt and never for the stores.
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

constexpr int kFsWaves = 4;              // sequences per workgroup, one wave (and SIMD) each
constexpr int kFsBlocksA = 64;           // q and k tiles of one head: 2 kinds x 2 halves x 16 k-steps of 1 KB
constexpr int kFsBlocksB = 32;           // v tiles of one head: 2 halves x 16 k-steps
constexpr int kFsBlocksG = 16;           // the gate tile
constexpr int kFsRopePairs = 16;         // pairs of rotary pairs per position (32 pairs)
constexpr int kFsRopeVecs = 2 * kFsRopePairs * 64;  // float2 [cos, sin][pair pair][position]
constexpr int kFsStoresPerHead = 16;     // O stores per wave and head: 2 query tiles x 2 feature tiles x 4
// LDS layout, in 16-byte units: stage A, stage B, the gate tile, the rotary table (128 KB).
constexpr int kFsOffB = kFsBlocksA * 64;
constexpr int kFsOffG = kFsOffB + kFsBlocksB * 64;
constexpr int kFsOffRope = kFsOffG + kFsBlocksG * 64;
constexpr int kFsLdsVecs = kFsOffRope + kFsRopeVecs / 2;
constexpr int kFsDropped = 0x40000000;   // buffer offset past any sequence's output: the store is dropped

// This wave's share of the gate tile (the last tile of W_qkvg).
__device__ __forceinline__ void fs_issue_gate(u32x4* buf, const u32x4* wq, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < kFsBlocksG / kFsWaves; ++i) {
    const int b = (kFsBlocksG / kFsWaves) * wave + i;
    lds_load_block(wq + (int64_t(kQkvgTiles - 1) * 16 + b) * 64, buf + b * 64, lane);
  }
}

// Stage A of head h: block 32 kind + 16 c + ks is k-step ks of tile 16 kind + 2h + c (kind 0 q, 1 k).
__device__ __forceinline__ void fs_issue_a(int h, u32x4* buf, const u32x4* wq, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < kFsBlocksA / kFsWaves; ++i) {
    const int b = (kFsBlocksA / kFsWaves) * wave + i;
    const int t = 16 * (b >> 5) + 2 * h + ((b >> 4) & 1);
    lds_load_block(wq + (int64_t(t) * 16 + (b & 15)) * 64, buf + b * 64, lane);
  }
}

// Stage B of head h: block 16 c + ks is k-step ks of v tile 32 + 2h + c.
__device__ __forceinline__ void fs_issue_b(int h, u32x4* buf, const u32x4* wq, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < kFsBlocksB / kFsWaves; ++i) {
    const int b = (kFsBlocksB / kFsWaves) * wave + i;
    const int t = 32 + 2 * h + (b >> 4);
    lds_load_block(wq + (int64_t(t) * 16 + (b & 15)) * 64, buf + b * 64, lane);
  }
}

// Key (or token) of register R of half-wave hh in a 32-row accumulator tile: row 8(R/4) + 4hh + R%4.
__device__ __forceinline__ int acc_row(int R, int hh) { return 8 * (R >> 2) + 4 * hh + (R & 3); }

// q and k products of head half c (4 accumulator chains over 16 k-steps; operands read one k-step ahead);
// after(ks) runs after the MFMAs of k-step ks.
template <class After>
__device__ __forceinline__ void fs_qk_half(const u32x4* __restrict__ La, int c, const u32x4 (&bx)[2][16], int lane,
                                           f32x16 (&qa)[2], f32x16 (&ka)[2], After after) {
#pragma unroll
  for (int t = 0; t < 2; ++t) qa[t] = ka[t] = zero16();
  u32x4 aq = La[(16 * c) * 64 + lane], ak = La[(32 + 16 * c) * 64 + lane];
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) {
    u32x4 nq, nk;
    if (ks + 1 < 16) {
      nq = La[(16 * c + ks + 1) * 64 + lane];
      nk = La[(32 + 16 * c + ks + 1) * 64 + lane];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) qa[t] = mfma32(aq, bx[t][ks], qa[t]);
#pragma unroll
    for (int t = 0; t < 2; ++t) ka[t] = mfma32(ak, bx[t][ks], ka[t]);
    after(ks);
    __builtin_amdgcn_sched_barrier(0);
    if (ks + 1 < 16) {
      aq = nq;
      ak = nk;
    }
  }
}

// Rotary of register group g (rows 8g + 4hh + r) of column tile t of head half c, fp32 (q times log2 e),
// into the bf16 operands: q as the B operand Q^T, k as the A operand K, k-step g / 2 of the half.
__device__ __forceinline__ void fs_rotate(const f32x16& qa, const f32x16& ka, const float2* __restrict__ ropeL, int c,
                                          int t, int g, int j, int hh, u32x4& qb, u32x4& kb) {
  const int p = 32 * t + j, pp = 8 * c + 2 * g + hh;  // pairs 2pp, 2pp + 1 = 16c + 4g + 2hh + {0, 1}
  const float2 cs = ropeL[pp * 64 + p], sn = ropeL[(kFsRopePairs + pp) * 64 + p];
  const float q0 = qa[4 * g], q1 = qa[4 * g + 1], q2 = qa[4 * g + 2], q3 = qa[4 * g + 3];
  qb[2 * (g & 1)] = pk_bf16(fmaf(q0, cs.x, -(q1 * sn.x)) * kLog2e, fmaf(q1, cs.x, q0 * sn.x) * kLog2e);
  qb[2 * (g & 1) + 1] = pk_bf16(fmaf(q2, cs.y, -(q3 * sn.y)) * kLog2e, fmaf(q3, cs.y, q2 * sn.y) * kLog2e);
  const float k0 = ka[4 * g], k1 = ka[4 * g + 1], k2 = ka[4 * g + 2], k3 = ka[4 * g + 3];
  kb[2 * (g & 1)] = pk_bf16(fmaf(k0, cs.x, -(k1 * sn.x)), fmaf(k1, cs.x, k0 * sn.x));
  kb[2 * (g & 1) + 1] = pk_bf16(fmaf(k2, cs.y, -(k3 * sn.y)), fmaf(k3, cs.y, k2 * sn.y));
}

// The output of one head waiting to be scaled and stored: O^T accumulators [d tile][query tile], the
// per-query scale gate / sum, and the byte offset of each query tile's row (kFsDropped past the end).
struct FsPending {
  f32x16 o[2][2];
  float sc[2];
  int off[2];
};

// Unit u (0..15) of storing a pending head: query tile u / 8, feature tile (u / 4) % 2, group u % 4.
__device__ __forceinline__ void fs_store_unit(const FsPending& pd, int u, int h, int hh, __amdgpu_buffer_rsrc_t ores) {
  const int qt = u >> 3, dt = (u >> 2) & 1, g = u & 3;
  const float sc = pd.sc[qt];
  const f32x16& o = pd.o[dt][qt];
  const u32x2 v = {pk_bf16(o[4 * g] * sc, o[4 * g + 1] * sc), pk_bf16(o[4 * g + 2] * sc, o[4 * g + 3] * sc)};
  const int off = pd.off[qt] + 2 * (h * kHeadDim + 32 * dt + row_of_group(g, hh));
  __builtin_amdgcn_raw_buffer_store_b64(v, ores, off, 0, 0);
}

__global__ __launch_bounds__(256, 1) void k_qkv_attn_short(const uint16_t* __restrict__ xn,
                                                          const u32x4* __restrict__ wq,
                                                          const float* __restrict__ bgate,
                                                          const float* __restrict__ rope, int mode, int nseq,
                                                          int L, int T, int F, uint16_t* __restrict__ O) {
  __shared__ u32x4 smem[kFsLdsVecs];  // one LDS object: stage A, stage B, gate tile, rotary table
  u32x4* La = smem;
  u32x4* Lb = smem + kFsOffB;
  u32x4* Lg = smem + kFsOffG;
  float2* ropeL = reinterpret_cast<float2*>(smem + kFsOffRope);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int s = blockIdx.x * kFsWaves + wave;
  const bool active = s < nseq;  // idle waves still stage weights and meet every barrier

  fs_issue_gate(Lg, wq, wave, lane);
  fs_issue_a(0, La, wq, wave, lane);
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
  // O of this sequence as a buffer: token of position p at byte (token_of(p) - token_of(0)) * 1 KB
  const int64_t tok0 = active ? token_of(mode, s, 0, T, F) : 0;
  const int tok_stride = mode == 0 ? F : 1;
  const __amdgpu_buffer_rsrc_t ores =
      buffer_rsrc(O + tok0 * (kHeads * kHeadDim), active ? ((L - 1) * tok_stride + 1) * kHeads * kHeadDim * 2 : 0);
  int qoff[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = 32 * qt + j;
    qoff[qt] = q < L ? q * tok_stride * (kHeads * kHeadDim * 2) : kFsDropped;
  }
  __syncthreads();  // the rotary table
  vmcnt_barrier<0>();  // the gate tile and stage A of head 0
  fs_issue_b(0, Lb, wq, wave, lane);
  float gv[2][4];  // sigmoid gates of heads 4hh + r for the tokens of column tile t
  if (active) {
    f32x16 ga[2] = {zero16(), zero16()};
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const u32x4 a = Lg[ks * 64 + lane];
#pragma unroll
      for (int t = 0; t < 2; ++t) ga[t] = mfma32(a, bx[t][ks], ga[t]);
    }
    const f32x4 bg = *reinterpret_cast<const f32x4*>(bgate + 4 * hh);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) gv[t][r] = 1.0f / (1.0f + expf(-(ga[t][r] + bg[r])));
  }

  // The previous head's output, stored during the next head's stage A.  Before head 0 it is a dummy
  // whose stores are all dropped, so that every head issues the same 16 stores.
  FsPending pd;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    pd.o[0][qt] = pd.o[1][qt] = zero16();
    pd.sc[qt] = 0.f;
    pd.off[qt] = kFsDropped;
  }
#pragma unroll 1
  for (int h = 0; h < kHeads; ++h) {
    // ---- stage A: q, k of both halves, rotary, S^T
    f32x16 sacc[2][2];
    if (active) {
      f32x16 qa0[2], ka0[2], qa1[2], ka1[2];
      u32x4 qb[2][2][2], kb[2][2][2];  // [half][column tile][k-step of the half]
      fs_qk_half(La, 0, bx, lane, qa0, ka0, [&](int ks) { fs_store_unit(pd, ks, h - 1, hh, ores); });
      fs_qk_half(La, 1, bx, lane, qa1, ka1, [&](int ks) {
        if (ks & 1) {
          const int u = ks >> 1, t = u >> 2, g = u & 3;
          fs_rotate(qa0[t], ka0[t], ropeL, 0, t, g, j, hh, qb[0][t][g >> 1], kb[0][t][g >> 1]);
        }
      });
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          sacc[kt][qt] = zero16();
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) sacc[kt][qt] = mfma32(kb[0][kt][kk], qb[0][qt][kk], sacc[kt][qt]);
        }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        fs_rotate(qa1[u >> 2], ka1[u >> 2], ropeL, 1, u >> 2, u & 3, j, hh, qb[1][u >> 2][(u & 3) >> 1],
                  kb[1][u >> 2][(u & 3) >> 1]);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) sacc[kt][qt] = mfma32(kb[1][kt][kk], qb[1][qt][kk], sacc[kt][qt]);
    }
    // stage B of head h has landed (its loads are older than the 16 stores issued above)
    if (active)
      vmcnt_barrier<kFsStoresPerHead>();
    else
      vmcnt_barrier<0>();
    if (h + 1 < kHeads) fs_issue_a(h + 1, La, wq, wave, lane);
    if (active) {
      // ---- stage B: v (swapped product, tokens on the rows) with the softmax of S^T between its MFMAs
      f32x16 va[2][2];  // [head half][token tile]
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t) va[c][t] = zero16();
      float m[2], lsum[2] = {0.f, 0.f};
      u32x4 pb[2][4];  // P^T operands [query tile][key k-step]
      u32x4 av0 = Lb[lane], av1 = Lb[16 * 64 + lane];
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) {
        u32x4 n0, n1;
        if (ks + 1 < 16) {
          n0 = Lb[(ks + 1) * 64 + lane];
          n1 = Lb[(16 + ks + 1) * 64 + lane];
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) va[0][t] = mfma32(bx[t][ks], av0, va[0][t]);
#pragma unroll
        for (int t = 0; t < 2; ++t) va[1][t] = mfma32(bx[t][ks], av1, va[1][t]);
        // softmax unit: query tile qt, step st (0: row max over the valid keys; 1, 2: e = 2^(s - m) of key
        // tile st - 1, its fp32 sum and bf16 P)
        if ((ks & 1) && ks < 12) {
          const int u = ks >> 1, qt = u / 3, st = u % 3;
          if (st == 0) {
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
              if (32 * kt + 32 <= L) {  // a key tile with no padded keys (uniform): no masking
#pragma unroll
                for (int R = 0; R < 16; R += 2) mx = fmaxf(fmaxf(mx, sacc[kt][qt][R]), sacc[kt][qt][R + 1]);
              } else {
#pragma unroll
                for (int R = 0; R < 16; ++R)
                  if (32 * kt + acc_row(R, hh) < L) mx = fmaxf(mx, sacc[kt][qt][R]);
              }
            }
            m[qt] = halfwave_max(mx);
          } else {
            const int kt = st - 1;
            float e[16];
            if (32 * kt + 32 <= L) {
#pragma unroll
              for (int R = 0; R < 16; ++R) e[R] = __builtin_amdgcn_exp2f(sacc[kt][qt][R] - m[qt]);
            } else {
#pragma unroll
              for (int R = 0; R < 16; ++R)
                e[R] = 32 * kt + acc_row(R, hh) < L ? __builtin_amdgcn_exp2f(sacc[kt][qt][R] - m[qt]) : 0.f;
            }
#pragma unroll
            for (int R = 0; R < 16; ++R) lsum[qt] += e[R];
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
              pb[qt][2 * kt + kk] = u32x4{pk_bf16(e[8 * kk], e[8 * kk + 1]), pk_bf16(e[8 * kk + 2], e[8 * kk + 3]),
                                          pk_bf16(e[8 * kk + 4], e[8 * kk + 5]), pk_bf16(e[8 * kk + 6], e[8 * kk + 7])};
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 1 < 16) {
          av0 = n0;
          av1 = n1;
        }
      }
      u32x4 vb[2][4];  // V^T operands [head half = feature tile][key k-step 2 tt + kk]
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            const f32x16& v = va[c][t];
            vb[c][2 * t + kk] = u32x4{pk_bf16(v[8 * kk], v[8 * kk + 1]), pk_bf16(v[8 * kk + 2], v[8 * kk + 3]),
                                      pk_bf16(v[8 * kk + 4], v[8 * kk + 5]), pk_bf16(v[8 * kk + 6], v[8 * kk + 7])};
          }
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          pd.o[dt][qt] = zero16();
#pragma unroll
          for (int kv = 0; kv < 4; ++kv) pd.o[dt][qt] = mfma32(vb[dt][kv], pb[qt][kv], pd.o[dt][qt]);
        }
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        // gate of head h for this query: in this lane if h / 4 == hh, else in the partner lane
        float own = gv[qt][0];
#pragma unroll
        for (int r = 1; r < 4; ++r) own = (h & 3) == r ? gv[qt][r] : own;
        const float other = __shfl_xor(own, 32);
        const float ls = lsum[qt] + __shfl_xor(lsum[qt], 32);
        pd.sc[qt] = (hh == (h >> 2) ? own : other) * (1.0f / ls);
        pd.off[qt] = qoff[qt];
      }
    }
    // stage A of head h + 1 has landed (the stores of head h - 1 went out during stage A of head h)
    vmcnt_barrier<0>();
    if (h + 1 < kHeads) fs_issue_b(h + 1, Lb, wq, wave, lane);
  }
  if (active) {
#pragma unroll
    for (int u = 0; u < kFsStoresPerHead; ++u) fs_store_unit(pd, u, kHeads - 1, hh, ores);
  }
}

void launch_qkv_attn_short(const uint16_t* xn, const uint8_t* layer, const float* rope, const SeqShape& sh,
                           uint16_t* O, hipStream_t st, const LaunchEvents& ev) {
  const unsigned blocks = unsigned((sh.nseq + kFsWaves - 1) / kFsWaves);
  hipExtLaunchKernelGGL(k_qkv_attn_short, dim3(blocks), dim3(64 * kFsWaves), 0, st, ev.start, ev.stop, 0, xn,
                     reinterpret_cast<const u32x4*>(layer + kOffQkvg),
                     reinterpret_cast<const float*>(layer + kOffBgate), rope, sh.mode, sh.nseq, sh.L, sh.T, sh.F, O);
}

}  // namespace trf
