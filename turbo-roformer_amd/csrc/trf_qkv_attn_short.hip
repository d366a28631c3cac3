// Fused QKV GEMM + rotary + gates + exact softmax attention for sequences of at most 64 positions
// (frequency attention: the 62 bands of one frame), so that Q, K, V and the gates never leave the chip.
// It replaces the pair qkv_rope_gemm -> attention of the reference (kernels.cpp:439-540, 250-388) for
// short sequences, with the same arithmetic: fp32 accumulators, fp32 rotary, q times log2(e) before its
// bf16 rounding, bf16 q, k, v and unnormalised P, the exact row max over the valid keys, an fp32 sum of
// e = 2^(s - m), and O = (P.V) * gate / sum rounded to bf16 in token order.
//
// A sequence is two 32-position halves, one wave each, and the two waves of a sequence share a SIMD, so
// each SIMD runs two waves and one wave's rotary, softmax and packing work can run under the other's
// MFMAs.  A wave keeps its 32 positions' xn rows in registers (bf16, natural k order) and computes q, k
// and v of its own positions; each half writes its K and V^T operand blocks to LDS and reads the other
// half's, so that every wave attends its 32 queries over all 64 keys.  A workgroup is 4 sequences (8
// waves).  The 49 weight tiles of W_qkvg stream through LDS: the gate tile, then per head stage A (the q
// and k tiles, 64 KB) and stage B (the v tiles, 32 KB), each in its own buffer so that one loads while the
// other is read (160 KB of LDS with the exchange blocks).
//
// Work is dealt in units of (group of 4 sequences, head): workgroup b of G runs units [bU/G, (b+1)U/G)
// of the U = 8 x groups in order, so one workgroup per CU gets an even share of heads (13 or 14 units
// for the 1701 frames of a 17 s chunk) instead of two rounds of whole groups (1.66 groups per CU).  A
// group entered mid-way or left early loads its xn rows and computes its gates again.
//
// Per head h:
//   A: P.V of head h - 1 (its V^T now visible from both halves) and its 8 bounds-checked O stores,
//      spread between the q products of head h; then the k products with the rotary of q between them;
//      then the rotary of k, written to LDS;
//   B: S^T = K.Q^T over both halves' keys, then the v products with the softmax of S^T between them;
//      then V^T packed and written to LDS.
// The stage barriers wait for the stage's loads with an exact vmcnt (the 8 O stores of a head are
// issued after the loads of stage B and are never waited for) and for the LDS exchange.
//
// No data crosses lanes between the projection and the attention:
//   * q and k come out of C = W . xn^T with lane (j, hh) holding token j of the column tile and features
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

constexpr int kFsSeqs = 4;                       // sequences per workgroup
constexpr int kFsWaves = 2 * kFsSeqs;            // one wave per 32-position half; waves w, w + 4 share a SIMD
constexpr int kFsBlocksA = 64;                   // q and k tiles of a head: 2 kinds x 2 halves x 16 k-steps
constexpr int kFsBlocksB = 32;                   // v tiles of a head: 2 halves x 16 k-steps
constexpr int kFsBlocksG = 16;                   // the gate tile (in stage B's buffer)
constexpr int kFsStoresPerHead = 8;              // O stores per wave and head: 2 feature tiles x 4 groups
// LDS layout, in 16-byte units: stage A, stage B, then the K and V^T operand blocks exchanged between
// the halves, [sequence][half][k-step][lane] (160 KB).
constexpr int kFsOffB = kFsBlocksA * 64;
constexpr int kFsOffKx = kFsOffB + kFsBlocksB * 64;
constexpr int kFsOffVx = kFsOffKx + kFsSeqs * 2 * 4 * 64;
constexpr int kFsLdsVecs = kFsOffVx + kFsSeqs * 2 * 4 * 64;
constexpr int kFsDropped = kFusedShortDropped;  // buffer offset past any sequence's output: the store is dropped

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

// This thread's vector memory operations have completed except the N most recent, its LDS operations
// have all completed (the K / V^T exchange), then all waves meet.
template <int N>
__device__ __forceinline__ void fs_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);  // vmcnt(N) expcnt(7) lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Key (or token) of register R of half-wave hh in a 32-row accumulator tile: row 8(R/4) + 4hh + R%4.
__device__ __forceinline__ int acc_row(int R, int hh) { return 8 * (R >> 2) + 4 * hh + (R & 3); }

// The rotary cos/sin of this lane's position: pairs 16c + 4g + 2hh + {0, 1}, the ones that register
// group g (rows 8g + 4hh + r) of head half c rotates.
struct FsRope {
  float2 cs[2][4], sn[2][4];
};

// Rotary of register group g of head half c, fp32, scaled, into the bf16 operand of k-step 2c + g/2
// (elements 2(g%2), 2(g%2) + 1).
__device__ __forceinline__ void fs_rotate(const f32x16& a, const FsRope& rp, int c, int g, float scale, u32x4& out) {
  const float2 cs = rp.cs[c][g], sn = rp.sn[c][g];
  const float a0 = a[4 * g], a1 = a[4 * g + 1], a2 = a[4 * g + 2], a3 = a[4 * g + 3];
  out[2 * (g & 1)] = pk_bf16(fmaf(a0, cs.x, -(a1 * sn.x)) * scale, fmaf(a1, cs.x, a0 * sn.x) * scale);
  out[2 * (g & 1) + 1] = pk_bf16(fmaf(a2, cs.y, -(a3 * sn.y)) * scale, fmaf(a3, cs.y, a2 * sn.y) * scale);
}

// One head's output of this wave's 32 queries, from P.V to the store: O^T accumulators [feature tile],
// the per-query scale gate / sum and the query row's byte offset (kFsDropped past the sequence end).
struct FsOut {
  f32x16 o[2];
  float sc;
  int off;
};

// Store unit u (0..7) of a head's output: feature tile u / 4, register group u % 4.
__device__ __forceinline__ void fs_store_unit(const FsOut& po, int u, int h, int hh, __amdgpu_buffer_rsrc_t ores) {
  const int dt = u >> 2, g = u & 3;
  const f32x16& o = po.o[dt];
  const u32x2 v = {pk_bf16(o[4 * g] * po.sc, o[4 * g + 1] * po.sc), pk_bf16(o[4 * g + 2] * po.sc, o[4 * g + 3] * po.sc)};
  const int off = po.off + 2 * (h * kHeadDim + 32 * dt + row_of_group(g, hh));
  __builtin_amdgcn_raw_buffer_store_b64(v, ores, off, 0, 0);
}

// What one head leaves for the next head's stage A: this half's V^T operands [feature tile][key k-step], the
// P^T operands of its queries [key k-step 2 kt + kk], and the scale and offset of its output.
struct FsCarry {
  u32x4 vb[2][2];
  u32x4 pb[4];
  float sc;
  int off;
};

// P.V of a head: the other half's V^T operands come from LDS.
__device__ __forceinline__ void fs_pv(const FsCarry& cy, const u32x4* __restrict__ vx_other, int th, int lane,
                                      FsOut& po) {
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    po.o[dt] = zero16();
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const u32x4 v = kt == th ? cy.vb[dt][kk] : vx_other[(2 * dt + kk) * 64 + lane];
        po.o[dt] = mfma32(v, cy.pb[2 * kt + kk], po.o[dt]);
      }
  }
  po.sc = cy.sc;
  po.off = cy.off;
}

struct FsCtx {
  const u32x4* wq;
  FsRope rope;
  const u32x4* kx_other;
  u32x4* kx_own;
  const u32x4* vx_other;
  u32x4* vx_own;
  __amdgpu_buffer_rsrc_t ores;
  int qoff, L, p, th, hh, lane, wave;
  bool active;
  float gv[4];  // sigmoid gates of heads 4hh + r for this lane's query
};

// One head: stage A (q and k) and stage B (v, attention).  hn is the head of the workgroup's next unit
// (its stage A is loaded during stage B), or -1.  CARRY: the previous head of the same group was run
// here, and its P.V and stores happen in this head's stage A.
template <bool CARRY>
__device__ __forceinline__ void fs_head(int h, int hn, const FsCtx& cx, u32x4* smem, const u32x4 (&bx)[16],
                                        FsCarry& cy) {
  u32x4* const La = smem;
  u32x4* const Lb = smem + kFsOffB;
  const int lane = cx.lane;

  // ---- stage A: P.V and stores of head h - 1 between the q products of head h, then the k products
  // with the rotary of q between them, then the rotary of k into LDS
  fs_barrier<0>();  // stage A landed; V^T of head h - 1 written by both halves
  fs_issue_b(h, Lb, cx.wq, cx.wave, lane);
  u32x4 qb[2][2], kb[2][2];  // [head half][k-step of the half]
  if (cx.active) {
    f32x16 qa[2];
    {
      FsOut po;
      if (CARRY) fs_pv(cy, cx.vx_other, cx.th, lane, po);
#pragma unroll
      for (int c = 0; c < 2; ++c) qa[c] = zero16();
      u32x4 a0 = La[lane], a1 = La[16 * 64 + lane];
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) {
        u32x4 n0, n1;
        if (ks + 1 < 16) {
          n0 = La[(ks + 1) * 64 + lane];
          n1 = La[(16 + ks + 1) * 64 + lane];
        }
        qa[0] = mfma32(a0, bx[ks], qa[0]);
        qa[1] = mfma32(a1, bx[ks], qa[1]);
        if (CARRY && (ks & 1)) fs_store_unit(po, ks >> 1, h - 1, cx.hh, cx.ores);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 1 < 16) {
          a0 = n0;
          a1 = n1;
        }
      }
    }
    f32x16 ka[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) ka[c] = zero16();
    const u32x4* const Lk = La + 32 * 64;
    u32x4 a0 = Lk[lane], a1 = Lk[16 * 64 + lane];
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      u32x4 n0, n1;
      if (ks + 1 < 16) {
        n0 = Lk[(ks + 1) * 64 + lane];
        n1 = Lk[(16 + ks + 1) * 64 + lane];
      }
      ka[0] = mfma32(a0, bx[ks], ka[0]);
      ka[1] = mfma32(a1, bx[ks], ka[1]);
      if (ks & 1) {
        const int u = ks >> 1, c = u >> 2, g = u & 3;
        fs_rotate(qa[c], cx.rope, c, g, kLog2e, qb[c][g >> 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < 16) {
        a0 = n0;
        a1 = n1;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) fs_rotate(ka[u >> 2], cx.rope, u >> 2, u & 3, 1.0f, kb[u >> 2][(u & 3) >> 1]);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) cx.kx_own[(2 * c + kk) * 64 + lane] = kb[c][kk];
  }

  // ---- stage B: S^T over both halves' keys, v products with the softmax between them, V^T into LDS
  if (cx.active && CARRY)
    fs_barrier<kFsStoresPerHead>();  // stage B landed (the 8 stores above are younger); K written
  else
    fs_barrier<0>();
  if (hn >= 0) fs_issue_a(hn, La, cx.wq, cx.wave, lane);
  if (cx.active) {
    f32x16 sacc[2];  // [key tile]
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      sacc[kt] = zero16();
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const u32x4 k = kt == cx.th ? kb[c][kk] : cx.kx_other[(2 * c + kk) * 64 + lane];
          sacc[kt] = mfma32(k, qb[c][kk], sacc[kt]);
        }
    }
    f32x16 va[2];  // [head half]: features 32c + j of tokens 8g + 4hh + r
#pragma unroll
    for (int c = 0; c < 2; ++c) va[c] = zero16();
    float m = 0.f, lsum = 0.f;
    const int L = cx.L, hh = cx.hh;
    u32x4 a0 = Lb[lane], a1 = Lb[16 * 64 + lane];
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      u32x4 n0, n1;
      if (ks + 1 < 16) {
        n0 = Lb[(ks + 1) * 64 + lane];
        n1 = Lb[(16 + ks + 1) * 64 + lane];
      }
      va[0] = mfma32(bx[ks], a0, va[0]);
      va[1] = mfma32(bx[ks], a1, va[1]);
      // softmax units after k-steps 1, 5, 9: the row max over the valid keys, then for each key tile
      // e = 2^(s - m), its fp32 sum and the bf16 P^T operands
      if (ks == 1) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          if (32 * kt + 32 <= L) {  // a key tile with no padded keys (uniform): no masking
#pragma unroll
            for (int R = 0; R < 16; R += 2) mx = fmaxf(fmaxf(mx, sacc[kt][R]), sacc[kt][R + 1]);
          } else {
#pragma unroll
            for (int R = 0; R < 16; ++R)
              if (32 * kt + acc_row(R, hh) < L) mx = fmaxf(mx, sacc[kt][R]);
          }
        }
        m = halfwave_max(mx);
      } else if (ks == 5 || ks == 9) {
        const int kt = ks == 5 ? 0 : 1;
        float e[16];
        if (32 * kt + 32 <= L) {
#pragma unroll
          for (int R = 0; R < 16; ++R) e[R] = __builtin_amdgcn_exp2f(sacc[kt][R] - m);
        } else {
#pragma unroll
          for (int R = 0; R < 16; ++R)
            e[R] = 32 * kt + acc_row(R, hh) < L ? __builtin_amdgcn_exp2f(sacc[kt][R] - m) : 0.f;
        }
#pragma unroll
        for (int R = 0; R < 16; ++R) lsum += e[R];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          cy.pb[2 * kt + kk] = u32x4{pk_bf16(e[8 * kk], e[8 * kk + 1]), pk_bf16(e[8 * kk + 2], e[8 * kk + 3]),
                                     pk_bf16(e[8 * kk + 4], e[8 * kk + 5]), pk_bf16(e[8 * kk + 6], e[8 * kk + 7])};
      }
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < 16) {
        a0 = n0;
        a1 = n1;
      }
    }
    // V^T operands of this half's keys [feature tile c][key k-step kk], kept and written to LDS
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const f32x16& v = va[c];
        cy.vb[c][kk] = u32x4{pk_bf16(v[8 * kk], v[8 * kk + 1]), pk_bf16(v[8 * kk + 2], v[8 * kk + 3]),
                             pk_bf16(v[8 * kk + 4], v[8 * kk + 5]), pk_bf16(v[8 * kk + 6], v[8 * kk + 7])};
        cx.vx_own[(2 * c + kk) * 64 + lane] = cy.vb[c][kk];
      }
    // gate of head h for this query: in this lane if h / 4 == hh, else in the partner lane
    float own = cx.gv[0];
#pragma unroll
    for (int r = 1; r < 4; ++r) own = (h & 3) == r ? cx.gv[r] : own;
    const float other = __shfl_xor(own, 32);
    const float ls = lsum + __shfl_xor(lsum, 32);
    cy.sc = (hh == (h >> 2) ? own : other) * (1.0f / ls);
    cy.off = cx.qoff;
  }
}

// The last head's P.V and stores of a group, once both halves have written its V^T.
__device__ __forceinline__ void fs_flush(const FsCtx& cx, const FsCarry& cy, int h) {
  fs_barrier<0>();
  if (cx.active) {
    FsOut po;
    fs_pv(cy, cx.vx_other, cx.th, cx.lane, po);
#pragma unroll
    for (int u = 0; u < kFsStoresPerHead; ++u) fs_store_unit(po, u, h, cx.hh, cx.ores);
  }
}

__global__ __launch_bounds__(64 * kFsWaves) void k_qkv_attn_short(const uint16_t* __restrict__ xn,
                                                                  const u32x4* __restrict__ wq,
                                                                  const float* __restrict__ bgate,
                                                                  const float* __restrict__ rope, int mode,
                                                                  int nseq, int L, int T, int F,
                                                                  uint16_t* __restrict__ O) {
  __shared__ u32x4 smem[kFsLdsVecs];  // one LDS object: stage A, stage B, K / V^T exchange
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int j = lane & 31, hh = lane >> 5;
  const int sl = wave & (kFsSeqs - 1), th = wave >> 2;  // sequence slot, position half
  const int units = (nseq + kFsSeqs - 1) / kFsSeqs * kHeads;
  const int u_begin = int(int64_t(blockIdx.x) * units / gridDim.x);
  const int u_end = int(int64_t(blockIdx.x + 1) * units / gridDim.x);
  FsCtx cx;
  cx.wq = wq;
  cx.kx_own = smem + kFsOffKx + (2 * sl + th) * 4 * 64;
  cx.kx_other = smem + kFsOffKx + (2 * sl + (th ^ 1)) * 4 * 64;
  cx.vx_own = smem + kFsOffVx + (2 * sl + th) * 4 * 64;
  cx.vx_other = smem + kFsOffVx + (2 * sl + (th ^ 1)) * 4 * 64;
  cx.L = L;
  cx.p = 32 * th + j;
  cx.th = th;
  cx.hh = hh;
  cx.lane = lane;
  cx.wave = wave;
  const int tok_stride = mode == 0 ? F : 1;
  // the output row of this lane's position within its sequence (kFsDropped past the sequence end)
  cx.qoff = cx.p < L ? cx.p * tok_stride * (kHeads * kHeadDim * 2) : kFsDropped;

  fs_issue_a(u_begin % kHeads, smem, wq, wave, lane);
  {  // rotary table [cos | sin][L][32] fp32, for this lane's position in every sequence (zero past L)
    const bool in = cx.p < L;
    const float* cr = rope + int64_t(in ? cx.p : 0) * 32;
    const float* sr = cr + int64_t(L) * 32;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int i = 16 * c + 4 * g + 2 * hh;
        cx.rope.cs[c][g] = in ? *reinterpret_cast<const float2*>(cr + i) : float2{0.f, 0.f};
        cx.rope.sn[c][g] = in ? *reinterpret_cast<const float2*>(sr + i) : float2{0.f, 0.f};
      }
  }
  FsCarry cy;
  int h_last = 0;
#pragma unroll 1
  for (int u = u_begin; u < u_end;) {
    const int grp = u / kHeads, h0 = u - grp * kHeads;
    const int h1 = min(kHeads, h0 + (u_end - u));  // this group's heads h0 .. h1 - 1
    if (u != u_begin) fs_flush(cx, cy, h_last);    // the previous group's last head
    fs_issue_gate(smem + kFsOffB, wq, wave, lane);
    const int s = grp * kFsSeqs + sl;
    cx.active = s < nseq;  // idle waves still stage weights and meet every barrier
    const bool valid = cx.active && cx.p < L;
    u32x4 bx[16];  // xn of this lane's position (zero past L), natural k order
    {
      const u32x4* xr = reinterpret_cast<const u32x4*>(xn + (valid ? token_of(mode, s, cx.p, T, F) : 0) * kDim);
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) bx[ks] = valid ? xr[2 * ks + hh] : zero4();
    }
    // O of this sequence as a buffer: token of position p at byte (token_of(p) - token_of(0)) * 1 KB
    const int64_t tok0 = cx.active ? token_of(mode, s, 0, T, F) : 0;
    cx.ores = buffer_rsrc(O + tok0 * (kHeads * kHeadDim),
                          cx.active ? ((L - 1) * tok_stride + 1) * kHeads * kHeadDim * 2 : 0);
    fs_barrier<0>();  // the gate tile, stage A of head h0 and xn

    // ---- the gate tile (in stage B's buffer): rows 0..7 live in register group 0 of both half-waves
    if (cx.active) {
      f32x16 ga = zero16();
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) ga = mfma32(smem[kFsOffB + ks * 64 + lane], bx[ks], ga);
      const f32x4 bg = *reinterpret_cast<const f32x4*>(bgate + 4 * hh);
#pragma unroll
      for (int r = 0; r < 4; ++r) cx.gv[r] = 1.0f / (1.0f + expf(-(ga[r] + bg[r])));
    }

    // head h0 has no previous head to finish; the others finish theirs in their stage A
    {
      const int next = grp * kHeads + h0 + 1;  // the next unit, if this workgroup has one
      fs_head<false>(h0, next < u_end ? (h0 + 1) % kHeads : -1, cx, smem, bx, cy);
    }
#pragma unroll 1
    for (int h = h0 + 1; h < h1; ++h) {
      const int next = grp * kHeads + h + 1;
      fs_head<true>(h, next < u_end ? (h + 1) % kHeads : -1, cx, smem, bx, cy);
    }
    h_last = h1 - 1;
    u += h1 - h0;
  }
  if (u_end > u_begin) fs_flush(cx, cy, h_last);
}

// Workgroups of the fused kernel: one per CU (the kernel deals its units itself), at most one per unit.
static int fs_grid(int nseq) {
  const int n = device_cu_count();
  const int units = (nseq + kFsSeqs - 1) / kFsSeqs * kHeads;
  return units < n ? units : n;
}

void launch_qkv_attn_short(const uint16_t* xn, const uint8_t* layer, const float* rope, const SeqShape& sh,
                           uint16_t* O, hipStream_t st, const LaunchEvents& ev) {
  if (sh.nseq <= 0) return;
  hipExtLaunchKernelGGL(k_qkv_attn_short, dim3(unsigned(fs_grid(sh.nseq))), dim3(64 * kFsWaves), 0, st, ev.start,
                        ev.stop, 0, xn, reinterpret_cast<const u32x4*>(layer + kOffQkvg),
                        reinterpret_cast<const float*>(layer + kOffBgate), rope, sh.mode, sh.nseq, sh.L, sh.T, sh.F,
                        O);
}

}  // namespace trf
