// Internal declarations shared by the kernel and C-ABI translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trf {

constexpr int kDim = 256;
constexpr int kHeads = 8;
constexpr int kHeadDim = 64;
constexpr int kQkvgRows = 1544;
constexpr int kHidden = 1024;

// MFMA operand tiles: 32 output rows x 16 k per instruction, 64 lanes x 16 bytes.
constexpr int kTileBytes = 64 * 16;

// Packed sub-layer layout (byte offsets).  Every weight matrix W[rows][K] is stored as
// tiles[rows/32][K/16][64 lanes][8 bf16] with tile[t][ks][lane][e] = W[32t + lane%32][16ks + kperm(lane/32, e)]
// (rows past the end are zero), which is the A-operand order of v_mfma_f32_32x32x16_bf16.
// Natural order (W_qkvg, W_out): kperm(hh, e) = 8hh + e, matching B operands read as 16 contiguous
// bytes of an activation row.  Register order (W1, W2): kperm(hh, e) = 4hh + e for e < 4 and
// 8 + 4hh + (e - 4) otherwise, which is the order in which a 32x32 accumulator tile holds its rows in
// a lane (runs of 4 at 8g + 4hh), so an accumulator converted to bf16 is directly the next B operand.
constexpr int kQkvgTiles = 49;  // 1544 rows -> 49 tiles of 32 (last tile: 8 gate rows)
constexpr size_t kOffQkvg = 0;
constexpr size_t kSzQkvg = size_t(kQkvgTiles) * (kDim / 16) * kTileBytes;
constexpr size_t kOffBgate = kOffQkvg + kSzQkvg;
constexpr size_t kOffOut = kOffBgate + 256;
constexpr size_t kSzOut = size_t(kDim / 32) * (512 / 16) * kTileBytes;
constexpr size_t kOffFf1 = kOffOut + kSzOut;
constexpr size_t kSzFf1 = size_t(kHidden / 32) * (kDim / 16) * kTileBytes;
constexpr size_t kOffBff1 = kOffFf1 + kSzFf1;
constexpr size_t kOffFf2 = kOffBff1 + kHidden * 4;
constexpr size_t kSzFf2 = size_t(kDim / 32) * (kHidden / 16) * kTileBytes;
constexpr size_t kOffBff2 = kOffFf2 + kSzFf2;
// The split-bf16 feed-forward runs on 16x16x32 MFMAs, whose A operand is 16 rows x 32 k: tiles
// [rows/16][K/32][64 lanes][8 bf16], tile[t][ks][lane][e] = W[16t + lane%16][32ks + kperm16(lane/16, e)],
// natural kperm16(g, e) = 8g + e (W_out), register order kperm16(g, e) = 16(e/4) + 4g + e%4 (W1, W2: a
// 16x16 accumulator holds rows 4g..4g+3 in lane group g, so two tiles form one 32-deep B operand).
// W1 and W2 come as hi = bf16(W) and lo = bf16(W - hi).
constexpr size_t kOffOut16 = kOffBff2 + kDim * 4;
constexpr size_t kOffFf1Hi16 = kOffOut16 + kSzOut;
constexpr size_t kOffFf1Lo16 = kOffFf1Hi16 + kSzFf1;
constexpr size_t kOffFf2Hi16 = kOffFf1Lo16 + kSzFf1;
constexpr size_t kOffFf2Lo16 = kOffFf2Hi16 + kSzFf2;
// fp16 W1 and W2 (32x32 register order, fp16(hi + lo)) for the fp16 feed-forward.
constexpr size_t kOffFf1F16 = kOffFf2Lo16 + kSzFf2;
constexpr size_t kOffFf2F16 = kOffFf1F16 + kSzFf1;
constexpr size_t kLayerBytes = kOffFf2F16 + kSzFf2;

// Feed-forward arithmetic (the trf_precision values of trf_hip.h).
enum FfPrecision { kFfBf16 = 0, kFfSplit = 1, kFfFp16 = 2 };

// Operand tile layouts of launch_pack.
enum PackLayout { kPack32Natural = 0, kPack32RegOrder = 1, kPack16Natural = 2, kPack16RegOrder = 3 };

inline int32_t seq_pad(int32_t L) { return (L + 63) / 64 * 64; }

struct SeqShape {
  int mode, batch, T, F;
  int nseq, L, Lpad;
};

inline SeqShape seq_shape(int mode, int batch, int T, int F) {
  SeqShape s{mode, batch, T, F, 0, 0, 0};
  s.nseq = mode == 0 ? batch * F : batch * T;
  s.L = mode == 0 ? T : F;
  s.Lpad = seq_pad(s.L);
  return s;
}

// The fused short-sequence kernel (launch_qkv_attn_short) addresses a sequence's output rows (1 KB each,
// token stride F in time mode, 1 in frequency mode) with 32-bit buffer offsets, and drops the stores of
// padded positions by sending them to byte offset kFusedShortDropped, past every row of the sequence.  It
// therefore takes a shape only when the sequence's last row ends below that offset; larger strides go
// through the unfused pair (64-bit token indexing).
constexpr int kFusedShortDropped = 1 << 30;
inline bool fused_short_fits(const SeqShape& s) {
  const int64_t stride = s.mode == 0 ? s.F : 1;
  return s.L <= 64 && (int64_t(s.L - 1) * stride + 1) * kHeads * kHeadDim * 2 <= int64_t(kFusedShortDropped);
}

// Sets the calling thread's trf_last_error message (printf format) and returns code (trf_capi.hip).
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Optional start / stop events of a launch.  hipExtLaunchKernelGGL records them with the dispatch itself,
// which costs less than separate event-record packets around it (no events: a plain launch).
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};

// Kernel launchers (trf_kernels.hip).  They only enqueue work; the caller checks errors.
// Pack W [rows][K] bf16 into MFMA A-operand tiles (layout: PackLayout); W == nullptr packs zeros.
void launch_pack(const uint16_t* W, int rows, int K, int layout, uint8_t* dst, hipStream_t st);
// fp16(hi + lo) operand tiles in 32x32 register order (lo may be null).
void launch_pack_f16(const uint16_t* hi, const uint16_t* lo, int rows, int K, uint8_t* dst, hipStream_t st);
void launch_copy_f32(const float* src, int n, float* dst, hipStream_t st);
void launch_add_rmsnorm(float* X, const void* Y, int y_bf16, void* out, int out_bf16, int64_t n,
                        float eps, hipStream_t st);
// CUs of the current device (hipDeviceAttributeMultiprocessorCount, cached per device): the grid of the
// kernels that deal their work units themselves, one workgroup per CU.
int device_cu_count();
void launch_qkv(const uint16_t* xn, const uint8_t* layer, const float* rope, const SeqShape& sh,
                uint16_t* Q, uint16_t* K, uint16_t* Vt, float* G, hipStream_t st, const LaunchEvents& ev = {});
void launch_attention(const uint16_t* Q, const uint16_t* K, const uint16_t* Vt, const float* G,
                      uint16_t* O, const SeqShape& sh, hipStream_t st, const LaunchEvents& ev = {});
// Fused QKV + rotary + gates + attention for sequences of at most 64 positions (trf_qkv_attn_short.hip):
// xn -> O with no Q/K/V/G buffers.  Requires sh.L <= 64.
void launch_qkv_attn_short(const uint16_t* xn, const uint8_t* layer, const float* rope, const SeqShape& sh,
                           uint16_t* O, hipStream_t st, const LaunchEvents& ev = {});
// Per-op GEMMs on a standalone weight packed by launch_pack in natural k order (kPack32Natural):
// X += A [n][K] . W^T (+ bias), xn = X / max(|X|, eps) (W [256][K]); H = gelu_erf(xn . W^T + bias)
// (W [n_out][256], n_out a multiple of 32).
void launch_gemm_res_norm(const uint16_t* A, int K, const uint8_t* w_packed, const float* bias, float* X,
                          uint16_t* xn, int64_t n, float eps, hipStream_t st);
void launch_gemm_gelu(const uint16_t* xn, const uint8_t* w_packed, const float* bias, int n_out, uint16_t* H,
                      int64_t n, hipStream_t st);
// Fused out-projection + residual + norm [+ FF1 + GELU + FF2 + residual + norm]; ff_precision is a
// FfPrecision value for the two FF GEMMs.
void launch_post_attn(const uint16_t* O, const uint8_t* layer, float* X, uint16_t* xn, int64_t n, bool with_ff,
                      int ff_precision, float eps, hipStream_t st, const LaunchEvents& ev = {});
// Fused FF1 + GELU + FF2 + residual + norm on X (updated in place, its norm computed in the kernel);
// xn is written as X / |X|.
void launch_ff(const uint8_t* layer, float* X, uint16_t* xn, int64_t n, int ff_precision, float eps, hipStream_t st);

// ---------------------------------------------------------------- mask head (trf_mask.hip)
// Final norm + one MLP per band (Linear dim -> hidden, tanh, Linear hidden -> 2 din, GLU).
// Packed weights of band b, hidden tile j (32 hidden units), in 1 KB operand blocks (fp16, 64 lanes x 8):
//   W1 k-step s (16 inputs), hi/lo part hl:            block 2s + hl               (32 blocks)
//   W2 output pair i, a/g half ag, k-step t, part hl:  block 32 + 8i + 4ag + 2t + hl
// Output pair i is mask columns 32i..32i+31 of the band: its "a" tile holds W2 rows 32i+r (r < 32) and its
// "g" tile rows din + 32i + r (zero where 32i + r >= din), so a lane holds both GLU operands of a column.
// Tile j is (32 + 8 * npairs) KB; the tiles of a band follow each other.  Then b1 [n_bands][hidden] and,
// per band, b2 as [a part: pad][g part: pad] (pad = 32 * npairs, zeros past din), all fp32.
constexpr int kMaxBands = 64;
constexpr int kMaskMaxJobs = 192;
constexpr int kMaskPairs = 6;      // output pairs per job: the largest that fits the LDS stages
constexpr int kMaskFrames = 128;   // frames per workgroup (4 waves x 32)
constexpr int kMaskW1Blocks = 32;  // blocks of W1 per hidden tile
constexpr int kXcds = 8;           // workgroups are dealt round-robin over the 8 XCDs

enum MaskPrecision { kMaskSplit = 0, kMaskFp16 = 1 };

// Everything a mask-head launch needs besides the pointers, passed by value.  A job is (band, first
// output pair p0, np pairs); the workgroups of XCD x run jobs job[xcd_start[x] .. xcd_start[x+1]) one
// after the other, each over ntb blocks of kMaskFrames frames.
struct MaskPlan {
  int32_t hidden, n_frames, F, width, ntb;
  uint32_t b1_off;                  // byte offset of b1 in the packed buffer
  uint32_t xcd_start[kXcds + 1];
  uint32_t job[kMaskMaxJobs];       // band | np << 8 | p0 << 16
  uint32_t wofs_kb[kMaxBands];      // first weight block of the band, in KB from the packed start
  uint32_t b2_off[kMaxBands];       // byte offset of the band's b2
  uint32_t col[kMaxBands];          // first mask column of the band
  uint32_t din[kMaxBands];
};

// Plans go to the kernels by value and are indexed at run time (by band or job), so every array in them
// has 32-bit elements: with 16- or 8-bit elements next to 32-bit ones the compiler shared the address
// arithmetic of two arrays and issued scalar loads from bases that were not dword aligned, which read the
// wrong words for odd indices.

// ---------------------------------------------------------------- band split (trf_band_split.hip)
// Per band f: RMSNorm of the frame's din_f features, Linear din_f -> kDim.  Packed weights of a band:
// W' = W * gamma * sqrt(din) as fp32 A operands of v_mfma_f32_32x32x2_f32, [din/2 k-pairs][8 tiles][64
// lanes] (lane l: output 32t + l%32, input 2p + l/32), then the bias [kDim].
constexpr int kBandFrames = 32;  // frames per workgroup (4 waves, 2 output tiles each)

struct BandPlan {
  int32_t n_bands, n_frames, width, ngroups;  // ngroups = workgroups per band
  uint32_t col[kMaxBands];                    // first feature column of the band
  uint32_t wofs[kMaxBands];                   // first float of the band's packed weights
  uint32_t din[kMaxBands];
  uint32_t order[kMaxBands];                  // bands in launch order, widest first
};

void launch_pack_band_split(const float* w, const float* b, const float* gamma, int din, float sqrt_din, float* dst,
                            hipStream_t st);
void launch_band_split(const float* feats, const float* packed, float* X, const BandPlan& plan, hipStream_t st);

// ---------------------------------------------------------------- song assembly (trf_song.hip)
// acc [2][n] += the windowed chunk predictions y [nc][2][ystride] (first L samples) at starts[nc] (device,
// ascending), wsum [n] += the window, in ascending chunk order; then out = acc / max(wsum, 1e-10) / gain.
void launch_overlap_add(const float* y, int nc, int64_t ystride, int L, const int64_t* starts, const float* w,
                        int64_t n, float* acc, float* wsum, hipStream_t st);
void launch_overlap_finish(const float* acc, const float* wsum, int64_t n, float gain, float* out, hipStream_t st);

// Pack one band: W1 [hidden][kDim] (times gamma [kDim] per input), W2 [2 din][hidden], fp32 device.
void launch_pack_mask_band(const float* w1, const float* gamma, const float* b1, const float* w2, const float* b2,
                           int din, int hidden, uint8_t* wdst, float* b1dst, float* b2dst, hipStream_t st);
void launch_mask_head(const float* X, const uint8_t* packed, float* mask, const MaskPlan& plan, unsigned grid,
                      int precision, hipStream_t st);

}  // namespace trf
