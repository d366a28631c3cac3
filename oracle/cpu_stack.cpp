// AVX512-BF16 CPU restatement of the 12-block axial transformer stack: test infrastructure and the
// same-host CPU baseline, never the product path.
//
// It computes what the restructured stack computes (fast.py:222-266 of the reference, folded weights as
// in fast.py:163-191: 16 * gamma in the input columns of each Linear, 1/8 in W_q, every runtime norm
// x / max(|x|, 1e-12)), with the reference's CPU kernel numerics (docs/how-it-works.md:120-170): GEMM
// and attention operands bf16 (round to nearest even), every accumulator, the residual stream, norms,
// softmax statistics and the rotary math fp32.  The design follows the published description of the
// reference's kernels (docs/how-it-works.md:120-151); the code is this file's own:
//
// * GEMMs on vdpbf16ps with a 6-row x 64-column register tile (24 zmm accumulators); weights packed at
//   set-up into panels of 64 output columns, [K/2][64][2] bf16, so one 64-byte load is 16 columns x one
//   k pair.  Every GEMM carries its elementwise work in the epilogue:
//     - QKV + gates: rotary on q and k in fp32, then q row-major, k in 64-key tiles of k pairs
//       ([32 pairs][64 keys][2], one 64-byte load = 16 keys x one pair), v in key pairs ([L/2][64][2]),
//       each in the layout the attention reads; the 8 gate columns get bias + sigmoid;
//     - output projection and FF2: X += A W^T (+ b) into the fp32 residual, then the next norm of the
//       same rows as the bf16 input of the next GEMM;
//     - FF1: bias + exact-erf GELU, bf16 out.
// * Attention per (sequence, head), 6 query rows at a time, exact softmax: pass 1 the scores of all keys
//   (64-key tiles) and the row max, pass 2 e = 2^((s - max) log2 e), summed in fp32 and stored rounded to
//   bf16, pass 3 P V with the same 6 x 64 tile; the 1/sum, the head's sigmoid gate and the head
//   merge are applied when the tile is written.
// * Work is spread over std::threads by an atomic task counter (row blocks of 48 tokens for the GEMMs,
//   (sequence, head) pairs for the attention).  A token's result does not depend on the thread count or
//   on the other tokens of its row block.
//
// exp2 is 2^n * p(f) with n = round(x), f = x - n in [-1/2, 1/2] and p the degree-6 Taylor polynomial of
// e^(f ln 2) (relative error < 2e-7); erf for the GELU is Abramowitz & Stegun 7.1.26 (absolute error
// < 1.5e-7).  Both are far below the bf16 rounding of what they feed.
//
// C ABI (ctypes, oracle/cpu_stack.py): trfc_new, trfc_set_layer, trfc_forward, trfc_free.

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <new>
#include <thread>
#include <vector>

namespace {

constexpr int kH = 8, kDh = 64, kDim = 256, kQkv = 3 * kH * kDh, kFf = 1024, kGates = kH;
constexpr int kRowBlock = 48;  // tokens per GEMM task (8 register tiles)
constexpr float kLog2e = 1.4426950408889634f;

using bf16 = uint16_t;

inline bf16 to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (no NaNs here)
  return bf16(u >> 16);
}

inline int32_t ld32(const bf16* p) {
  int32_t v;
  std::memcpy(&v, p, 4);
  return v;
}

inline __m256i ps_to_bf16x16(__m512 x) { return (__m256i)_mm512_cvtneps_pbh(x); }

// 2^x for x in [-126, 126] (clamped): 2^round(x) * e^((x - round(x)) ln 2), Taylor to degree 6.
inline __m512 exp2_ps(__m512 x) {
  x = _mm512_min_ps(_mm512_max_ps(x, _mm512_set1_ps(-126.f)), _mm512_set1_ps(126.f));
  const __m512 n = _mm512_roundscale_ps(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const __m512 y = _mm512_mul_ps(_mm512_sub_ps(x, n), _mm512_set1_ps(0.6931471805599453f));
  __m512 p = _mm512_set1_ps(1.f / 720.f);
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f / 120.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f / 24.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f / 6.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(0.5f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f));
  return _mm512_scalef_ps(p, n);
}

inline __m512 sigmoid_ps(__m512 x) {
  const __m512 e = exp2_ps(_mm512_mul_ps(x, _mm512_set1_ps(-kLog2e)));
  return _mm512_div_ps(_mm512_set1_ps(1.f), _mm512_add_ps(_mm512_set1_ps(1.f), e));
}

// 0.5 x (1 + erf(x / sqrt 2)), erf by Abramowitz & Stegun 7.1.26 on |z| with the sign restored.
inline __m512 gelu_ps(__m512 x) {
  const __m512 z = _mm512_mul_ps(_mm512_abs_ps(x), _mm512_set1_ps(0.7071067811865476f));
  const __m512 t = _mm512_div_ps(_mm512_set1_ps(1.f), _mm512_fmadd_ps(z, _mm512_set1_ps(0.3275911f), _mm512_set1_ps(1.f)));
  __m512 p = _mm512_set1_ps(1.061405429f);
  p = _mm512_fmadd_ps(p, t, _mm512_set1_ps(-1.453152027f));
  p = _mm512_fmadd_ps(p, t, _mm512_set1_ps(1.421413741f));
  p = _mm512_fmadd_ps(p, t, _mm512_set1_ps(-0.284496736f));
  p = _mm512_fmadd_ps(p, t, _mm512_set1_ps(0.254829592f));
  p = _mm512_mul_ps(p, t);
  const __m512 e = exp2_ps(_mm512_mul_ps(_mm512_mul_ps(z, z), _mm512_set1_ps(-kLog2e)));
  __m512 erf = _mm512_fnmadd_ps(p, e, _mm512_set1_ps(1.f));  // erf(|z|)
  const __m512 sign = _mm512_and_ps(x, _mm512_castsi512_ps(_mm512_set1_epi32(int32_t(0x80000000u))));
  erf = _mm512_or_ps(erf, sign);
  return _mm512_mul_ps(_mm512_mul_ps(_mm512_set1_ps(0.5f), x), _mm512_add_ps(_mm512_set1_ps(1.f), erf));
}

inline float hsum(__m512 v) { return _mm512_reduce_add_ps(v); }
inline float hmax(__m512 v) { return _mm512_reduce_max_ps(v); }

// W [O][K] fp32 -> panels of nc output columns, [panel][K/2][nc][2] bf16, zero past O.
std::vector<bf16> pack_panels(const float* W, int O, int K, int nc) {
  const int np = (O + nc - 1) / nc;
  std::vector<bf16> out(size_t(np) * K * nc, 0);
  for (int p = 0; p < np; ++p)
    for (int j = 0; j < K / 2; ++j)
      for (int c = 0; c < nc; ++c) {
        const int o = p * nc + c;
        if (o >= O) continue;
        for (int e = 0; e < 2; ++e) out[((size_t(p) * (K / 2) + j) * nc + c) * 2 + e] = to_bf16(W[size_t(o) * K + 2 * j + e]);
      }
  return out;
}

// Register tile of the GEMMs: out[r][v] = sum over k pairs j of rows[r][2j..2j+1] . panel[j][16 v + lane][0..1],
// six A rows (bf16) against one panel of NV 16-column vectors ([kp][16 NV][2] bf16), fp32 sums.
// Per k pair the six row pairs are broadcast into registers first; each panel vector is then loaded once
// and met by all six of them.  The 6 x NV sums stay in registers (a local array) and leave once at the end.
template <int NV>
inline void tile_dot(const bf16* const rows[6], const bf16* __restrict__ panel, int kp, __m512 out[6][NV]) {
  __m512 sum[NV][6];
  for (auto& col : sum)
    for (auto& x : col) x = _mm512_setzero_ps();
  const __m512i* pv = reinterpret_cast<const __m512i*>(panel);
  for (int j = 0; j < kp; ++j, pv += NV) {
    __m512bh pair[6];
#pragma GCC unroll 6
    for (int r = 0; r < 6; ++r) pair[r] = (__m512bh)_mm512_set1_epi32(ld32(rows[r] + 2 * j));
#pragma GCC unroll 4
    for (int v = 0; v < NV; ++v) {
      const __m512bh w = (__m512bh)_mm512_loadu_si512(pv + v);
#pragma GCC unroll 6
      for (int r = 0; r < 6; ++r) sum[v][r] = _mm512_dpbf16_ps(sum[v][r], pair[r], w);
    }
  }
  for (int v = 0; v < NV; ++v)
    for (int r = 0; r < 6; ++r) out[r][v] = sum[v][r];
}

template <class Fn>
void parallel_for(int n, int threads, Fn&& fn) {
  std::atomic<int> next{0};
  auto work = [&] {
    for (int i; (i = next.fetch_add(1, std::memory_order_relaxed)) < n;) fn(i);
  };
  const int nt = std::max(1, std::min(threads, n));
  std::vector<std::thread> pool;
  pool.reserve(nt - 1);
  for (int t = 1; t < nt; ++t) pool.emplace_back(work);
  work();
  for (auto& t : pool) t.join();
}

struct Layer {
  int mode = -1;                          // 0 attention over time (per band), 1 over bands (per frame)
  std::vector<bf16> wqkv, wg, wo, w1, w2;  // panels
  std::vector<float> bg, b1, b2, freqs;
};

// Token geometry of one sub-layer: sequence s, position i -> token base(s) + i * stride.
struct Axis {
  int mode, b, T, F;
  int L() const { return mode == 0 ? T : F; }
  int seqs() const { return mode == 0 ? b * F : b * T; }
  int64_t base(int s) const { return mode == 0 ? int64_t(s / F) * T * F + s % F : int64_t(s) * F; }
  int64_t stride() const { return mode == 0 ? F : 1; }
  void locate(int64_t n, int& s, int& i) const {
    if (mode == 0) {
      const int64_t bt = n / F;
      s = int((bt / T) * F + n % F);
      i = int(bt % T);
    } else {
      s = int(n / F);
      i = int(n % F);
    }
  }
};

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

enum Phase { kPhNorm, kPhQkv, kPhAttn, kPhOut, kPhFf1, kPhFf2, kPhases };

// A work buffer that is not cleared when it grows: its pages are first touched by the threads that
// write it (a serial zero fill of the ~1.5 GB of a 17 s chunk costs more than a forward).  Every element
// that is read has been written in the same forward, except the K padding keys of a sequence's last
// tile, whose scores are replaced by -inf before use.
template <class T>
struct Buffer {
  std::unique_ptr<T[]> p;
  size_t n = 0;
  void grow(size_t want) {
    if (want > n) {
      p.reset(new T[want]);  // default-initialised: not zeroed
      n = want;
    }
  }
  T* data() { return p.get(); }
  T& operator[](size_t i) { return p[i]; }
};

struct Stack {
  std::vector<Layer> layers;
  double phase_s[kPhases] = {};  // wall seconds per phase, summed over forwards
  // work buffers, grown on demand
  Buffer<bf16> xn, ao, h, q, k, v;
  Buffer<float> gates, rc, rs;

  // xn[n] = bf16(X[n] / max(|X[n]|, 1e-12)) for rows [r0, r1)
  static void norm_rows(const float* X, bf16* xn, int64_t r0, int64_t r1) {
    for (int64_t n = r0; n < r1; ++n) {
      const float* x = X + n * kDim;
      __m512 ss = _mm512_setzero_ps();
      for (int c = 0; c < kDim; c += 16) {
        const __m512 v = _mm512_loadu_ps(x + c);
        ss = _mm512_fmadd_ps(v, v, ss);
      }
      const float inv = 1.f / std::max(std::sqrt(hsum(ss)), 1e-12f);
      for (int c = 0; c < kDim; c += 16)
        _mm256_storeu_si256((__m256i*)(xn + n * kDim + c), ps_to_bf16x16(_mm512_mul_ps(_mm512_loadu_ps(x + c), _mm512_set1_ps(inv))));
    }
  }

  void forward(float* X, int b, int T, int F, int threads);
};

struct TaskRows {
  int64_t r0, rows;
};

inline TaskRows task_rows(int task, int64_t N) {
  const int64_t r0 = int64_t(task) * kRowBlock;
  return {r0, std::min<int64_t>(kRowBlock, N - r0)};
}

inline void tile_rows(const bf16* A, int64_t lda, int64_t row0, int rows, const bf16* a[6]) {
  for (int r = 0; r < 6; ++r) a[r] = A + (row0 + std::min(r, rows - 1)) * lda;
}

void Stack::forward(float* X, int b, int T, int F, int threads) {
  auto timed = [this](Phase ph, auto&& body) {
    const auto t0 = std::chrono::steady_clock::now();
    body();
    phase_s[ph] += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  };
  const int64_t N = int64_t(b) * T * F;
  const int ntask = int((N + kRowBlock - 1) / kRowBlock);
  const int64_t Lmax = std::max(T, F);
  const int64_t seq_stride = round_up(Lmax, 64) * kDh;  // elements of one (sequence, head) in q, k, v
  const int64_t max_seqs = std::max<int64_t>(int64_t(b) * F, int64_t(b) * T);
  xn.grow(size_t(N) * kDim);
  ao.grow(size_t(N) * kH * kDh);
  h.grow(size_t(N) * kFf);
  gates.grow(size_t(N) * kGates);
  q.grow(size_t(max_seqs) * kH * seq_stride);
  k.grow(size_t(max_seqs) * kH * seq_stride);
  v.grow(size_t(max_seqs) * kH * seq_stride);
  rc.grow(size_t(Lmax) * kDh);
  rs.grow(size_t(Lmax) * kDh);

  timed(kPhNorm, [&] {
    parallel_for(ntask, threads, [&](int t) {
      const TaskRows tr = task_rows(t, N);
      norm_rows(X, xn.data(), tr.r0, tr.r0 + tr.rows);
    });
  });

  for (const Layer& P : layers) {
    const Axis ax{P.mode, b, T, F};
    const int L = ax.L();
    // rotary tables: per position, per dimension d: cos(pos * freq[d / 2]) and -/+ sin for even/odd d
    for (int i = 0; i < L; ++i)
      for (int j = 0; j < kDh / 2; ++j) {
        const float ang = float(i) * P.freqs[j];
        const float c = float(std::cos(double(ang))), s = float(std::sin(double(ang)));
        rc[i * kDh + 2 * j] = c;
        rc[i * kDh + 2 * j + 1] = c;
        rs[i * kDh + 2 * j] = -s;
        rs[i * kDh + 2 * j + 1] = s;
      }

    // --- QKV + gates, written in the attention's layouts
    timed(kPhQkv, [&] {
      parallel_for(ntask, threads, [&](int t) {
        const TaskRows tr = task_rows(t, N);
        alignas(64) bf16 tmp[kDh];
        for (int p = 0; p < kQkv / 64; ++p) {
          const int which = p / kH, head = p % kH;
          const bf16* panel = P.wqkv.data() + size_t(p) * (kDim / 2) * 64 * 2;
          for (int64_t m0 = 0; m0 < tr.rows; m0 += 6) {
            const int rows = int(std::min<int64_t>(6, tr.rows - m0));
            const bf16* a[6];
            tile_rows(xn.data(), kDim, tr.r0 + m0, rows, a);
            __m512 acc[6][4];
            tile_dot<4>(a, panel, kDim / 2, acc);
            for (int r = 0; r < rows; ++r) {
              const int64_t n = tr.r0 + m0 + r;
              int s, i;
              ax.locate(n, s, i);
              const int64_t sh = (int64_t(s) * kH + head) * seq_stride;
              for (int vv = 0; vv < 4; ++vv) {
                __m512 x = acc[r][vv];
                if (which < 2) {  // rotate pairs (2j, 2j+1) by pos * freq[j]
                  const __m512 sw = _mm512_permute_ps(x, 0xB1);
                  x = _mm512_fmadd_ps(x, _mm512_loadu_ps(&rc[i * kDh + 16 * vv]), _mm512_mul_ps(sw, _mm512_loadu_ps(&rs[i * kDh + 16 * vv])));
                }
                _mm256_store_si256((__m256i*)(tmp + 16 * vv), ps_to_bf16x16(x));
              }
              if (which == 0) {
                std::memcpy(q.data() + sh + int64_t(i) * kDh, tmp, sizeof(tmp));
              } else if (which == 1) {  // k: [64-key tile][32 pairs][64 keys][2]
                bf16* kt = k.data() + sh + int64_t(i / 64) * 64 * kDh;
                for (int j = 0; j < kDh / 2; ++j) std::memcpy(kt + (j * 64 + i % 64) * 2, tmp + 2 * j, 4);
              } else {  // v: [key pair][64 dims][2]
                bf16* vp = v.data() + sh + int64_t(i / 2) * kDh * 2 + (i & 1);
                for (int d = 0; d < kDh; ++d) vp[2 * d] = tmp[d];
              }
            }
          }
        }
        // gate columns: one 16-column panel, 8 used
        for (int64_t m0 = 0; m0 < tr.rows; m0 += 6) {
          const int rows = int(std::min<int64_t>(6, tr.rows - m0));
          const bf16* a[6];
          tile_rows(xn.data(), kDim, tr.r0 + m0, rows, a);
          __m512 acc[6][1];
          tile_dot<1>(a, P.wg.data(), kDim / 2, acc);
          alignas(64) float g[16];
          for (int r = 0; r < rows; ++r) {
            _mm512_store_ps(g, sigmoid_ps(_mm512_add_ps(acc[r][0], _mm512_loadu_ps(P.bg.data()))));
            std::memcpy(gates.data() + (tr.r0 + m0 + r) * kGates, g, kGates * sizeof(float));
          }
        }
      });
    });

    // --- attention per (sequence, head)
    timed(kPhAttn, [&] {
      const int64_t stride = ax.stride();
      const int ntile = (L + 63) / 64;
      parallel_for(ax.seqs() * kH, threads, [&](int task) {
        const int s = task / kH, head = task % kH;
        const int64_t sh = (int64_t(s) * kH + head) * seq_stride;
        const bf16* qb = q.data() + sh;
        const bf16* kb = k.data() + sh;
        bf16* vb = v.data() + sh;
        if (L & 1)  // the key pair past the last key: its V half is read (times P = 0), make it 0
          for (int d = 0; d < kDh; ++d) vb[(int64_t(L / 2) * kDh + d) * 2 + 1] = 0;
        const int64_t lp = int64_t(ntile) * 64;
        thread_local std::vector<float> S;
        thread_local std::vector<bf16> Pb;
        if (S.size() < size_t(6 * lp)) S.resize(6 * lp);
        if (Pb.size() < size_t(6 * lp)) Pb.resize(6 * lp);
        const int64_t base = ax.base(s);
        for (int q0 = 0; q0 < L; q0 += 6) {
          const int rows = std::min(6, L - q0);
          const bf16* a[6];
          for (int r = 0; r < 6; ++r) a[r] = qb + int64_t(q0 + std::min(r, rows - 1)) * kDh;
          __m512 mx[6];
          for (int r = 0; r < 6; ++r) mx[r] = _mm512_set1_ps(-INFINITY);
          for (int tl = 0; tl < ntile; ++tl) {
            __m512 acc[6][4];
            tile_dot<4>(a, kb + int64_t(tl) * 64 * kDh, kDh / 2, acc);
            for (int g = 0; g < 4; ++g) {
              const int key0 = tl * 64 + 16 * g;
              const __mmask16 valid = key0 + 16 <= L ? __mmask16(0xffff) : key0 >= L ? __mmask16(0) : __mmask16((1u << (L - key0)) - 1);
              for (int r = 0; r < 6; ++r) {
                const __m512 sc = _mm512_mask_blend_ps(valid, _mm512_set1_ps(-INFINITY), acc[r][g]);
                _mm512_storeu_ps(&S[r * lp + key0], sc);
                mx[r] = _mm512_max_ps(mx[r], sc);
              }
            }
          }
          float inv[6];
          for (int r = 0; r < rows; ++r) {
            const __m512 mb = _mm512_set1_ps(hmax(mx[r]) * kLog2e);
            __m512 sum = _mm512_setzero_ps();
            for (int c = 0; c < L; c += 16) {
              const __mmask16 valid = c + 16 <= L ? __mmask16(0xffff) : __mmask16((1u << (L - c)) - 1);
              __m512 p = exp2_ps(_mm512_fmsub_ps(_mm512_loadu_ps(&S[r * lp + c]), _mm512_set1_ps(kLog2e), mb));
              p = _mm512_maskz_mov_ps(valid, p);
              _mm256_storeu_si256((__m256i*)&Pb[r * lp + c], ps_to_bf16x16(p));
              sum = _mm512_add_ps(sum, p);  // the fp32 values, before their bf16 rounding
            }
            inv[r] = 1.f / hsum(sum);
          }
          const bf16* pr[6];
          for (int r = 0; r < 6; ++r) pr[r] = &Pb[std::min(r, rows - 1) * lp];
          __m512 acc[6][4];
          tile_dot<4>(pr, vb, (L + 1) / 2, acc);
          for (int r = 0; r < rows; ++r) {
            const int64_t n = base + int64_t(q0 + r) * stride;
            const __m512 sc = _mm512_set1_ps(inv[r] * gates[n * kGates + head]);
            bf16* o = ao.data() + n * (kH * kDh) + head * kDh;
            for (int vv = 0; vv < 4; ++vv) _mm256_storeu_si256((__m256i*)(o + 16 * vv), ps_to_bf16x16(_mm512_mul_ps(acc[r][vv], sc)));
          }
        }
      });
    });

    // --- output projection: X += ao Wo^T, then the FF input norm
    timed(kPhOut, [&] {
      parallel_for(ntask, threads, [&](int t) {
        const TaskRows tr = task_rows(t, N);
        for (int p = 0; p < kDim / 64; ++p) {
          const bf16* panel = P.wo.data() + size_t(p) * (kH * kDh / 2) * 64 * 2;
          for (int64_t m0 = 0; m0 < tr.rows; m0 += 6) {
            const int rows = int(std::min<int64_t>(6, tr.rows - m0));
            const bf16* a[6];
            tile_rows(ao.data(), kH * kDh, tr.r0 + m0, rows, a);
            __m512 acc[6][4];
            tile_dot<4>(a, panel, kH * kDh / 2, acc);
            for (int r = 0; r < rows; ++r) {
              float* x = X + (tr.r0 + m0 + r) * kDim + p * 64;
              for (int vv = 0; vv < 4; ++vv) _mm512_storeu_ps(x + 16 * vv, _mm512_add_ps(_mm512_loadu_ps(x + 16 * vv), acc[r][vv]));
            }
          }
        }
        norm_rows(X, xn.data(), tr.r0, tr.r0 + tr.rows);
      });
    });

    // --- FF1 + GELU
    timed(kPhFf1, [&] {
      parallel_for(ntask, threads, [&](int t) {
        const TaskRows tr = task_rows(t, N);
        for (int p = 0; p < kFf / 64; ++p) {
          const bf16* panel = P.w1.data() + size_t(p) * (kDim / 2) * 64 * 2;
          for (int64_t m0 = 0; m0 < tr.rows; m0 += 6) {
            const int rows = int(std::min<int64_t>(6, tr.rows - m0));
            const bf16* a[6];
            tile_rows(xn.data(), kDim, tr.r0 + m0, rows, a);
            __m512 acc[6][4];
            tile_dot<4>(a, panel, kDim / 2, acc);
            for (int r = 0; r < rows; ++r) {
              bf16* o = h.data() + (tr.r0 + m0 + r) * kFf + p * 64;
              for (int vv = 0; vv < 4; ++vv)
                _mm256_storeu_si256((__m256i*)(o + 16 * vv),
                                    ps_to_bf16x16(gelu_ps(_mm512_add_ps(acc[r][vv], _mm512_loadu_ps(&P.b1[p * 64 + 16 * vv])))));
            }
          }
        }
      });
    });

    // --- FF2: X += h W2^T + b2, then the next sub-layer's input norm
    timed(kPhFf2, [&] {
      parallel_for(ntask, threads, [&](int t) {
        const TaskRows tr = task_rows(t, N);
        for (int p = 0; p < kDim / 64; ++p) {
          const bf16* panel = P.w2.data() + size_t(p) * (kFf / 2) * 64 * 2;
          for (int64_t m0 = 0; m0 < tr.rows; m0 += 6) {
            const int rows = int(std::min<int64_t>(6, tr.rows - m0));
            const bf16* a[6];
            tile_rows(h.data(), kFf, tr.r0 + m0, rows, a);
            __m512 acc[6][4];
            tile_dot<4>(a, panel, kFf / 2, acc);
            for (int r = 0; r < rows; ++r) {
              float* x = X + (tr.r0 + m0 + r) * kDim + p * 64;
              for (int vv = 0; vv < 4; ++vv)
                _mm512_storeu_ps(x + 16 * vv, _mm512_add_ps(_mm512_loadu_ps(x + 16 * vv),
                                                            _mm512_add_ps(acc[r][vv], _mm512_loadu_ps(&P.b2[p * 64 + 16 * vv]))));
            }
          }
        }
        norm_rows(X, xn.data(), tr.r0, tr.r0 + tr.rows);
      });
    });
  }
}

}  // namespace

extern "C" {

// A stack of n_layers sub-layers (block i time = 2 i, freq = 2 i + 1); NULL on a bad count.
void* trfc_new(int n_layers) {
  if (n_layers <= 0 || n_layers > 4096) return nullptr;
  auto* s = new (std::nothrow) Stack;
  if (s) s->layers.resize(n_layers);
  return s;
}

void trfc_free(void* h) { delete static_cast<Stack*>(h); }

// Wall seconds spent in each phase since the handle was made, summed over forwards: out[0] the input
// norm, out[1] QKV + gates, out[2] attention, out[3] output projection, out[4] FF1, out[5] FF2.
int trfc_phase_seconds(void* h, double* out) {
  auto* s = static_cast<Stack*>(h);
  if (!s || !out) return -1;
  for (int i = 0; i < kPhases; ++i) out[i] = s->phase_s[i];
  return 0;
}

// Folded fp32 weights of sub-layer i: W [1544][256] (q rows already scaled by 1/8, then k, v, 8 gate
// rows), b [1544] (zero for q, k, v; gate biases last), Wo [256][512], W1 [1024][256], b1 [1024],
// W2 [256][1024], b2 [256], freqs [32].  Returns 0, or -1 for a bad handle, index or mode.
int trfc_set_layer(void* h, int i, int mode, const float* W, const float* b, const float* Wo, const float* W1,
                   const float* b1, const float* W2, const float* b2, const float* freqs) {
  auto* s = static_cast<Stack*>(h);
  if (!s || i < 0 || i >= int(s->layers.size()) || (mode != 0 && mode != 1)) return -1;
  Layer& P = s->layers[i];
  P.mode = mode;
  P.wqkv = pack_panels(W, kQkv, kDim, 64);
  P.wg = pack_panels(W + size_t(kQkv) * kDim, kGates, kDim, 16);
  P.bg.assign(16, 0.f);
  std::copy(b + kQkv, b + kQkv + kGates, P.bg.begin());
  P.wo = pack_panels(Wo, kDim, kH * kDh, 64);
  P.w1 = pack_panels(W1, kFf, kDim, 64);
  P.b1.assign(b1, b1 + kFf);
  P.w2 = pack_panels(W2, kDim, kFf, 64);
  P.b2.assign(b2, b2 + kDim);
  P.freqs.assign(freqs, freqs + kDh / 2);
  return 0;
}

// X [b][T][F][256] fp32, in place, through every sub-layer on `threads` threads.  Returns 0; -1 for a
// bad handle or shape, -2 when a sub-layer was not set, -3 when the work buffers cannot be allocated.
int trfc_forward(void* h, float* X, int b, int T, int F, int threads) {
  auto* s = static_cast<Stack*>(h);
  if (!s || !X || b <= 0 || T <= 0 || F <= 0 || threads <= 0) return -1;
  for (const Layer& P : s->layers)
    if (P.mode < 0) return -2;
  try {
    s->forward(X, b, T, F, threads);
  } catch (const std::bad_alloc&) {
    return -3;
  }
  return 0;
}

}  // extern "C"
