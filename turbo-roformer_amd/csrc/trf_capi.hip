// C ABI of the stack, the band split before it and the mask head after it (declared in include/trf_hip.h):
// argument checks, workspace and packed layouts, the 24-sub-layer driver and the launch plans.  Host code
// only; the kernels live in trf_kernels.hip, trf_band_split.hip and trf_mask.hip.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "trf_hip.h"
#include "trf_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TRF_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return TRF_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_shape(int32_t batch, int32_t T, int32_t F) {
  if (batch < 1 || T < 1 || F < 1) return fail(TRF_ERR_ARG, "batch, T and F must be >= 1 (got %d, %d, %d)", batch, T, F);
  if (int64_t(batch) * T * F >= (int64_t(1) << 31))
    return fail(TRF_ERR_ARG, "batch*T*F = %lld tokens is too large", (long long)batch * T * F);
  return TRF_OK;
}

int check_precision(int32_t precision) {
  if (precision != TRF_PREC_BF16 && precision != TRF_PREC_FF_SPLIT && precision != TRF_PREC_FF_FP16)
    return fail(TRF_ERR_ARG, "precision must be 0 (bf16), 1 (ff split) or 2 (ff fp16), got %d", precision);
  return TRF_OK;
}

int check_mode(int32_t mode) {
  if (mode != TRF_MODE_TIME && mode != TRF_MODE_FREQ) return fail(TRF_ERR_ARG, "mode must be 0 (time) or 1 (freq), got %d", mode);
  return TRF_OK;
}

#define TRF_REQUIRE(ptr, name)                                                          \
  do {                                                                                  \
    if (!(ptr)) return fail(TRF_ERR_ARG, "%s must not be NULL", name);                  \
    if (!aligned((ptr), 16)) return fail(TRF_ERR_ARG, "%s must be 16-byte aligned", name); \
  } while (0)

struct Workspace {
  uint16_t* xn;
  uint16_t* O;
  float* G;
  uint16_t* Q;
  uint16_t* K;
  uint16_t* Vt;
  size_t bytes;
};

size_t round_up(size_t x) { return (x + 255) / 256 * 256; }

int64_t seq_elems(int mode, int batch, int T, int F) {
  const trf::SeqShape s = trf::seq_shape(mode, batch, T, F);
  return int64_t(s.nseq) * trf::kHeads * s.Lpad * trf::kHeadDim;
}

Workspace plan(int32_t batch, int32_t T, int32_t F, uint8_t* base) {
  const size_t n = size_t(batch) * T * F;
  const int64_t seq = seq_elems(0, batch, T, F) > seq_elems(1, batch, T, F) ? seq_elems(0, batch, T, F)
                                                                            : seq_elems(1, batch, T, F);
  Workspace w{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off += round_up(bytes);
    return p;
  };
  w.xn = reinterpret_cast<uint16_t*>(take(n * trf::kDim * 2));
  w.O = reinterpret_cast<uint16_t*>(take(n * 512 * 2));
  w.G = reinterpret_cast<float*>(take(n * trf::kHeads * 4));
  w.Q = reinterpret_cast<uint16_t*>(take(size_t(seq) * 2));
  w.K = reinterpret_cast<uint16_t*>(take(size_t(seq) * 2));
  w.Vt = reinterpret_cast<uint16_t*>(take(size_t(seq) * 2));
  w.bytes = off;
  return w;
}

hipStream_t as_hip(trf_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Optional event pair of each kernel of a layer (profiling): attached to the kernel's dispatch; events ==
// nullptr, or a NULL entry, records nothing.
struct Events {
  void* const* ev = nullptr;
  int layer = 0;
  trf::LaunchEvents of(int slot) const {
    trf::LaunchEvents e;
    if (ev) {
      e.start = reinterpret_cast<hipEvent_t>(ev[2 * (layer * TRF_SLOTS_PER_LAYER + slot)]);
      e.stop = reinterpret_cast<hipEvent_t>(ev[2 * (layer * TRF_SLOTS_PER_LAYER + slot) + 1]);
    }
    return e;
  }
  // Marks a slot with no kernel of its own as an empty interval (both events, if given, recorded here).
  int empty(int slot, hipStream_t st) const {
    const trf::LaunchEvents e = of(slot);
    for (hipEvent_t x : {e.start, e.stop}) {
      if (!x) continue;
      const hipError_t rc = hipEventRecord(x, st);
      if (rc != hipSuccess) return fail(TRF_ERR_HIP, "hipEventRecord: %s", hipGetErrorString(rc));
    }
    return TRF_OK;
  }
};

#define TRF_TRY(expr)              \
  do {                             \
    if (int rc_ = (expr)) return rc_; \
  } while (0)

// One sub-layer on an already normalised xn: qkv + rotary, attention (one fused kernel for sequences of
// at most 64 positions, whose time goes to the attention slot), then the fused out-proj + residual +
// norm, and (with_ff) FF1 + GELU + FF2 + residual + norm in the same kernel.
int run_layer(float* X, const trf::SeqShape& sh, const uint8_t* layer, const float* rope, const Workspace& w,
              int64_t n, bool with_ff, int ff_precision, hipStream_t st, const Events& ev = Events{}) {
  if (trf::fused_short_fits(sh)) {
    TRF_TRY(ev.empty(TRF_SLOT_QKV, st));
    trf::launch_qkv_attn_short(w.xn, layer, rope, sh, w.O, st, ev.of(TRF_SLOT_ATTN));
    TRF_TRY(check_launch("qkv_attention_short"));
  } else {
    trf::launch_qkv(w.xn, layer, rope, sh, w.Q, w.K, w.Vt, w.G, st, ev.of(TRF_SLOT_QKV));
    TRF_TRY(check_launch("qkv_rope_gemm"));
    trf::launch_attention(w.Q, w.K, w.Vt, w.G, w.O, sh, st, ev.of(TRF_SLOT_ATTN));
    TRF_TRY(check_launch("attention"));
  }
  trf::launch_post_attn(w.O, layer, X, w.xn, n, with_ff, ff_precision, 1e-12f, st, ev.of(TRF_SLOT_POST));
  return check_launch("post_attention");
}

int stack_impl(float* X, int32_t batch, int32_t T, int32_t F, const void* const* packed_layers, const int32_t* modes,
               int32_t n_layers, int32_t precision, const float* rope_time, const float* rope_freq,
               void* workspace, size_t workspace_bytes, void* const* events, int32_t n_events, hipStream_t st) {
  TRF_TRY(check_shape(batch, T, F));
  TRF_TRY(check_precision(precision));
  TRF_REQUIRE(X, "X");
  TRF_REQUIRE(workspace, "workspace");
  if (n_layers < 0) return fail(TRF_ERR_ARG, "n_layers must be >= 0");
  if (n_layers > 0 && (!packed_layers || !modes)) return fail(TRF_ERR_ARG, "packed_layers and modes must not be NULL");
  if (n_events != 0 && (n_events != 2 * TRF_SLOTS_PER_LAYER * n_layers || !events))
    return fail(TRF_ERR_ARG, "n_events must be 0 or 2*%d*n_layers with a non-NULL array", TRF_SLOTS_PER_LAYER);
  for (int32_t i = 0; i < n_layers; ++i) {
    TRF_TRY(check_mode(modes[i]));
    TRF_REQUIRE(packed_layers[i], "packed_layers[i]");
    if (modes[i] == TRF_MODE_TIME) TRF_REQUIRE(rope_time, "rope_time");
    if (modes[i] == TRF_MODE_FREQ) TRF_REQUIRE(rope_freq, "rope_freq");
  }
  const Workspace w = plan(batch, T, F, static_cast<uint8_t*>(workspace));
  if (workspace_bytes < w.bytes)
    return fail(TRF_ERR_WORKSPACE, "workspace is %zu bytes, need %zu", workspace_bytes, w.bytes);
  const int64_t n = int64_t(batch) * T * F;
  trf::launch_add_rmsnorm(X, nullptr, 0, w.xn, 1, n, 1e-12f, st);
  TRF_TRY(check_launch("add_rmsnorm"));
  for (int32_t i = 0; i < n_layers; ++i) {
    const uint8_t* layer = static_cast<const uint8_t*>(packed_layers[i]);
    const trf::SeqShape sh = trf::seq_shape(modes[i], batch, T, F);
    Events ev;
    ev.ev = n_events ? events : nullptr;
    ev.layer = i;
    TRF_TRY(run_layer(X, sh, layer, modes[i] == TRF_MODE_TIME ? rope_time : rope_freq, w, n, true, precision,
                      st, ev));
  }
  return TRF_OK;
}

// ---------------------------------------------------------------- mask head
// Byte layout of the packed mask head (see trf_internal.h) for a list of band widths.
struct MaskLayout {
  int n_bands = 0, hidden = 0;
  std::vector<int> din;
  std::vector<size_t> wofs, b2_off;  // bytes
  size_t b1_off = 0, total = 0;
};

int mask_npairs(int din) { return (din + 31) / 32; }
int mask_njobs(int din) { return (mask_npairs(din) + trf::kMaskPairs - 1) / trf::kMaskPairs; }

int mask_layout(const int32_t* dins, int32_t n_bands, int32_t hidden, MaskLayout& L) {
  if (!dins) return fail(TRF_ERR_ARG, "dins must not be NULL");
  if (n_bands < 1 || n_bands > trf::kMaxBands)
    return fail(TRF_ERR_ARG, "n_bands must be in [1, %d], got %d", trf::kMaxBands, n_bands);
  if (hidden < 64 || hidden > 8192 || hidden % 64)
    return fail(TRF_ERR_ARG, "hidden must be a multiple of 64 in [64, 8192], got %d", hidden);
  L = MaskLayout{};
  L.n_bands = n_bands;
  L.hidden = hidden;
  int jobs = 0;
  size_t off = 0;
  for (int f = 0; f < n_bands; ++f) {
    const int d = dins[f];
    if (d < 4 || d > 16384 || d % 4)
      return fail(TRF_ERR_ARG, "dins[%d] = %d: band widths must be multiples of 4 in [4, 16384]", f, d);
    jobs += mask_njobs(d);
    L.din.push_back(d);
    L.wofs.push_back(off);
    off += size_t(hidden / 32) * (trf::kMaskW1Blocks + 8 * mask_npairs(d)) * trf::kTileBytes;
  }
  if (jobs > trf::kMaskMaxJobs)
    return fail(TRF_ERR_ARG, "the bands make %d jobs of up to %d output pairs, more than %d", jobs,
                trf::kMaskPairs, trf::kMaskMaxJobs);
  L.b1_off = off;
  off = round_up(off + size_t(n_bands) * hidden * 4);
  for (int f = 0; f < n_bands; ++f) {
    L.b2_off.push_back(off);
    off = round_up(off + size_t(2 * 32 * mask_npairs(L.din[f])) * 4);
  }
  L.total = off;
  if (L.total >= (size_t(1) << 32)) return fail(TRF_ERR_ARG, "packed mask head would exceed 4 GiB");
  return TRF_OK;
}

// Launch plan: each band is cut into jobs of at most kMaskPairs output pairs (as even as possible), and
// the jobs are dealt to the XCDs largest first, each to the XCD with the least work so far (work of a job
// ~ its MFMAs per frame: 16 k-steps of GEMM1 + 4 per output pair of GEMM2).  A workgroup of XCD x then
// runs one job over kMaskFrames frames; the workgroups of one job on one XCD share its weights in L2.
unsigned mask_plan(const MaskLayout& L, int32_t n_frames, trf::MaskPlan& p) {
  p = trf::MaskPlan{};
  p.hidden = L.hidden;
  p.n_frames = n_frames;
  p.F = L.n_bands;
  p.ntb = (n_frames + trf::kMaskFrames - 1) / trf::kMaskFrames;
  p.b1_off = uint32_t(L.b1_off);
  struct Job {
    uint32_t code;
    int cost;
  };
  std::vector<Job> jobs;
  int col = 0;
  for (int f = 0; f < L.n_bands; ++f) {
    p.wofs_kb[f] = uint32_t(L.wofs[f] / 1024);
    p.b2_off[f] = uint32_t(L.b2_off[f]);
    p.col[f] = uint32_t(col);
    p.din[f] = uint32_t(L.din[f]);
    col += L.din[f];
    const int np = mask_npairs(L.din[f]), nj = mask_njobs(L.din[f]);
    for (int q = 0, p0 = 0; q < nj; ++q) {
      const int n = np / nj + (q < np % nj ? 1 : 0);
      jobs.push_back(Job{uint32_t(f) | uint32_t(n) << 8 | uint32_t(p0) << 16, 16 + 4 * n});
      p0 += n;
    }
  }
  p.width = col;
  std::stable_sort(jobs.begin(), jobs.end(), [](const Job& a, const Job& b) { return a.cost > b.cost; });
  std::vector<std::vector<uint32_t>> per(trf::kXcds);
  long load[trf::kXcds] = {};
  for (const Job& j : jobs) {
    int x = 0;
    for (int y = 1; y < trf::kXcds; ++y)
      if (load[y] < load[x]) x = y;
    per[x].push_back(j.code);
    load[x] += j.cost;
  }
  size_t most = 0, k = 0;
  for (int x = 0; x < trf::kXcds; ++x) {
    p.xcd_start[x] = uint32_t(k);
    for (uint32_t c : per[x]) p.job[k++] = c;
    most = per[x].size() > most ? per[x].size() : most;
  }
  p.xcd_start[trf::kXcds] = uint32_t(k);
  return unsigned(size_t(trf::kXcds) * most * p.ntb);
}

// ---------------------------------------------------------------- band split
// Packed band split: per band (din / 2) * 8 * 64 fp32 A operands and the bias [256]; offsets in floats.
int band_layout(const int32_t* dins, int32_t n_bands, std::vector<size_t>& wofs, size_t& total) {
  if (!dins) return fail(TRF_ERR_ARG, "dins must not be NULL");
  if (n_bands < 1 || n_bands > trf::kMaxBands)
    return fail(TRF_ERR_ARG, "n_bands must be in [1, %d], got %d", trf::kMaxBands, n_bands);
  wofs.clear();
  total = 0;
  for (int f = 0; f < n_bands; ++f) {
    const int d = dins[f];
    if (d < 4 || d > 16384 || d % 4)
      return fail(TRF_ERR_ARG, "dins[%d] = %d: band widths must be multiples of 4 in [4, 16384]", f, d);
    wofs.push_back(total);
    total += size_t(d / 2) * 8 * 64 + trf::kDim;
  }
  return TRF_OK;
}

}  // namespace

namespace trf {

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace trf

extern "C" {

int trf_abi_version(void) { return TRF_ABI_VERSION; }

const char* trf_last_error(void) { return g_err.c_str(); }

int32_t trf_seq_pad(int32_t L) { return trf::seq_pad(L); }

int64_t trf_seq_buffer_elems(int32_t mode, int32_t batch, int32_t T, int32_t F) {
  if (check_mode(mode) || check_shape(batch, T, F)) return -1;
  return seq_elems(mode, batch, T, F);
}

size_t trf_layer_packed_bytes(void) { return trf::kLayerBytes; }

int trf_pack_layer(const trf_layer_src* src, void* dst, trf_stream_t stream) {
  if (!src) return fail(TRF_ERR_ARG, "src must not be NULL");
  TRF_REQUIRE(dst, "dst");
  TRF_REQUIRE(src->w_qkvg, "w_qkvg");
  TRF_REQUIRE(src->w_out, "w_out");
  TRF_REQUIRE(src->w_ff1, "w_ff1");
  TRF_REQUIRE(src->w_ff2, "w_ff2");
  if ((src->w_ff1_lo && !aligned(src->w_ff1_lo, 16)) || (src->w_ff2_lo && !aligned(src->w_ff2_lo, 16)))
    return fail(TRF_ERR_ARG, "w_ff1_lo and w_ff2_lo must be 16-byte aligned");
  if (!src->b_gate || !src->b_ff1 || !src->b_ff2) return fail(TRF_ERR_ARG, "bias pointers must not be NULL");
  hipStream_t st = as_hip(stream);
  uint8_t* d = static_cast<uint8_t*>(dst);
  trf::launch_pack(src->w_qkvg, trf::kQkvgRows, trf::kDim, trf::kPack32Natural, d + trf::kOffQkvg, st);
  trf::launch_copy_f32(src->b_gate, trf::kHeads, reinterpret_cast<float*>(d + trf::kOffBgate), st);
  trf::launch_pack(src->w_out, trf::kDim, 512, trf::kPack32Natural, d + trf::kOffOut, st);
  trf::launch_pack(src->w_ff1, trf::kHidden, trf::kDim, trf::kPack32RegOrder, d + trf::kOffFf1, st);
  trf::launch_copy_f32(src->b_ff1, trf::kHidden, reinterpret_cast<float*>(d + trf::kOffBff1), st);
  trf::launch_pack(src->w_ff2, trf::kDim, trf::kHidden, trf::kPack32RegOrder, d + trf::kOffFf2, st);
  trf::launch_copy_f32(src->b_ff2, trf::kDim, reinterpret_cast<float*>(d + trf::kOffBff2), st);
  // operands of the split-bf16 feed-forward (16x16 tiles); absent lo parts pack as zeros
  trf::launch_pack(src->w_out, trf::kDim, 512, trf::kPack16Natural, d + trf::kOffOut16, st);
  trf::launch_pack(src->w_ff1, trf::kHidden, trf::kDim, trf::kPack16RegOrder, d + trf::kOffFf1Hi16, st);
  trf::launch_pack(src->w_ff1_lo, trf::kHidden, trf::kDim, trf::kPack16RegOrder, d + trf::kOffFf1Lo16, st);
  trf::launch_pack(src->w_ff2, trf::kDim, trf::kHidden, trf::kPack16RegOrder, d + trf::kOffFf2Hi16, st);
  trf::launch_pack(src->w_ff2_lo, trf::kDim, trf::kHidden, trf::kPack16RegOrder, d + trf::kOffFf2Lo16, st);
  // operands of the fp16 feed-forward: fp16(hi + lo)
  trf::launch_pack_f16(src->w_ff1, src->w_ff1_lo, trf::kHidden, trf::kDim, d + trf::kOffFf1F16, st);
  trf::launch_pack_f16(src->w_ff2, src->w_ff2_lo, trf::kDim, trf::kHidden, d + trf::kOffFf2F16, st);
  return check_launch("pack_layer");
}

int trf_add_rmsnorm(float* X, const void* Y, int32_t y_dtype, void* out, int32_t out_dtype, int64_t n_rows,
                    float eps, trf_stream_t stream) {
  TRF_REQUIRE(X, "X");
  TRF_REQUIRE(out, "out");
  if (Y && !aligned(Y, 16)) return fail(TRF_ERR_ARG, "Y must be 16-byte aligned");
  if ((y_dtype != TRF_F32 && y_dtype != TRF_BF16) || (out_dtype != TRF_F32 && out_dtype != TRF_BF16))
    return fail(TRF_ERR_ARG, "dtype must be TRF_F32 or TRF_BF16");
  if (n_rows < 0) return fail(TRF_ERR_ARG, "n_rows must be >= 0");
  if (n_rows == 0) return TRF_OK;
  trf::launch_add_rmsnorm(X, Y, y_dtype == TRF_BF16, out, out_dtype == TRF_BF16, n_rows, eps, as_hip(stream));
  return check_launch("add_rmsnorm");
}

int trf_qkv_rope_gemm(const uint16_t* xn, const void* packed_layer, const float* rope, int32_t mode, int32_t batch,
                      int32_t T, int32_t F, uint16_t* Q, uint16_t* K, uint16_t* Vt, float* G, trf_stream_t stream) {
  if (int rc = check_mode(mode)) return rc;
  if (int rc = check_shape(batch, T, F)) return rc;
  TRF_REQUIRE(xn, "xn");
  TRF_REQUIRE(packed_layer, "packed_layer");
  TRF_REQUIRE(rope, "rope");
  TRF_REQUIRE(Q, "Q");
  TRF_REQUIRE(K, "K");
  TRF_REQUIRE(Vt, "Vt");
  TRF_REQUIRE(G, "G");
  const trf::SeqShape sh = trf::seq_shape(mode, batch, T, F);
  trf::launch_qkv(xn, static_cast<const uint8_t*>(packed_layer), rope, sh, Q, K, Vt, G, as_hip(stream));
  return check_launch("qkv_rope_gemm");
}

int trf_attention(const uint16_t* Q, const uint16_t* K, const uint16_t* Vt, const float* G, uint16_t* O, int32_t mode,
                  int32_t batch, int32_t T, int32_t F, trf_stream_t stream) {
  if (int rc = check_mode(mode)) return rc;
  if (int rc = check_shape(batch, T, F)) return rc;
  TRF_REQUIRE(Q, "Q");
  TRF_REQUIRE(K, "K");
  TRF_REQUIRE(Vt, "Vt");
  TRF_REQUIRE(G, "G");
  TRF_REQUIRE(O, "O");
  const trf::SeqShape sh = trf::seq_shape(mode, batch, T, F);
  trf::launch_attention(Q, K, Vt, G, O, sh, as_hip(stream));
  return check_launch("attention");
}

int trf_qkv_attention_short(const uint16_t* xn, const void* packed_layer, const float* rope, int32_t mode,
                            int32_t batch, int32_t T, int32_t F, uint16_t* O, trf_stream_t stream) {
  if (int rc = check_mode(mode)) return rc;
  if (int rc = check_shape(batch, T, F)) return rc;
  const trf::SeqShape sh = trf::seq_shape(mode, batch, T, F);
  if (sh.L > 64) return fail(TRF_ERR_ARG, "sequences of %d positions: the fused kernel takes at most 64", sh.L);
  if (!trf::fused_short_fits(sh))
    return fail(TRF_ERR_ARG,
                "time-mode sequences of %d positions with token stride F = %d: the fused kernel's 32-bit output "
                "offsets take at most %d bytes per sequence; use trf_qkv_rope_gemm + trf_attention",
                sh.L, F, trf::kFusedShortDropped);
  TRF_REQUIRE(xn, "xn");
  TRF_REQUIRE(packed_layer, "packed_layer");
  TRF_REQUIRE(rope, "rope");
  TRF_REQUIRE(O, "O");
  trf::launch_qkv_attn_short(xn, static_cast<const uint8_t*>(packed_layer), rope, sh, O, as_hip(stream));
  return check_launch("qkv_attention_short");
}

size_t trf_weight_packed_bytes(int32_t rows, int32_t K) {
  if (rows < 1 || K < 16 || K % 16 != 0) return 0;
  return size_t((rows + 31) / 32) * size_t(K / 16) * trf::kTileBytes;
}

int trf_pack_weight(const uint16_t* W, int32_t rows, int32_t K, void* packed, trf_stream_t stream) {
  if (rows < 1 || K < 16 || K % 16 != 0)
    return fail(TRF_ERR_ARG, "rows must be >= 1 and K a positive multiple of 16 (got %d, %d)", rows, K);
  TRF_REQUIRE(W, "W");
  TRF_REQUIRE(packed, "packed");
  trf::launch_pack(W, rows, K, trf::kPack32Natural, static_cast<uint8_t*>(packed), as_hip(stream));
  return check_launch("pack_weight");
}

int trf_gemm_res_norm(const uint16_t* A, int32_t K, const void* w_packed, const float* bias, float* X, uint16_t* xn,
                      int64_t n_rows, float eps, trf_stream_t stream) {
  if (K < 16 || K % 16 != 0) return fail(TRF_ERR_ARG, "K must be a positive multiple of 16, got %d", K);
  TRF_REQUIRE(A, "A");
  TRF_REQUIRE(w_packed, "w_packed");
  if (bias && !aligned(bias, 16)) return fail(TRF_ERR_ARG, "bias must be 16-byte aligned");
  TRF_REQUIRE(X, "X");
  TRF_REQUIRE(xn, "xn");
  if (n_rows < 0) return fail(TRF_ERR_ARG, "n_rows must be >= 0");
  if (n_rows == 0) return TRF_OK;
  trf::launch_gemm_res_norm(A, K, static_cast<const uint8_t*>(w_packed), bias, X, xn, n_rows, eps, as_hip(stream));
  return check_launch("gemm_res_norm");
}

int trf_gemm_gelu(const uint16_t* xn, const void* w_packed, const float* bias, int32_t n_out, uint16_t* H,
                  int64_t n_rows, trf_stream_t stream) {
  if (n_out < 32 || n_out % 32 != 0) return fail(TRF_ERR_ARG, "n_out must be a positive multiple of 32, got %d", n_out);
  TRF_REQUIRE(xn, "xn");
  TRF_REQUIRE(w_packed, "w_packed");
  TRF_REQUIRE(bias, "bias");
  TRF_REQUIRE(H, "H");
  if (n_rows < 0) return fail(TRF_ERR_ARG, "n_rows must be >= 0");
  if (n_rows == 0) return TRF_OK;
  trf::launch_gemm_gelu(xn, static_cast<const uint8_t*>(w_packed), bias, n_out, H, n_rows, as_hip(stream));
  return check_launch("gemm_gelu");
}

size_t trf_stack_workspace_bytes(int32_t batch, int32_t T, int32_t F) {
  if (check_shape(batch, T, F)) return 0;
  return plan(batch, T, F, nullptr).bytes;
}

int trf_stack_forward(float* X, int32_t batch, int32_t T, int32_t F, const void* const* packed_layers,
                      const int32_t* modes, int32_t n_layers, int32_t precision, const float* rope_time,
                      const float* rope_freq, void* workspace, size_t workspace_bytes, trf_stream_t stream) {
  return stack_impl(X, batch, T, F, packed_layers, modes, n_layers, precision, rope_time, rope_freq, workspace,
                    workspace_bytes, nullptr, 0, as_hip(stream));
}

int trf_stack_forward_timed(float* X, int32_t batch, int32_t T, int32_t F, const void* const* packed_layers,
                            const int32_t* modes, int32_t n_layers, int32_t precision, const float* rope_time,
                            const float* rope_freq, void* workspace, size_t workspace_bytes, void* const* events,
                            int32_t n_events, trf_stream_t stream) {
  return stack_impl(X, batch, T, F, packed_layers, modes, n_layers, precision, rope_time, rope_freq, workspace,
                    workspace_bytes, events, n_events, as_hip(stream));
}

int trf_attn_block(float* X, int32_t batch, int32_t T, int32_t F, const void* packed_layer, int32_t mode,
                   const float* rope, void* workspace, size_t workspace_bytes, trf_stream_t stream) {
  if (int rc = check_mode(mode)) return rc;
  if (int rc = check_shape(batch, T, F)) return rc;
  TRF_REQUIRE(X, "X");
  TRF_REQUIRE(packed_layer, "packed_layer");
  TRF_REQUIRE(rope, "rope");
  TRF_REQUIRE(workspace, "workspace");
  const Workspace w = plan(batch, T, F, static_cast<uint8_t*>(workspace));
  if (workspace_bytes < w.bytes)
    return fail(TRF_ERR_WORKSPACE, "workspace is %zu bytes, need %zu", workspace_bytes, w.bytes);
  hipStream_t st = as_hip(stream);
  const int64_t n = int64_t(batch) * T * F;
  trf::launch_add_rmsnorm(X, nullptr, 0, w.xn, 1, n, 1e-12f, st);
  if (int rc = check_launch("add_rmsnorm")) return rc;
  return run_layer(X, trf::seq_shape(mode, batch, T, F), static_cast<const uint8_t*>(packed_layer), rope, w, n,
                   false, TRF_PREC_BF16, st);
}

int trf_ff_block(float* X, int32_t batch, int32_t T, int32_t F, const void* packed_layer, int32_t precision,
                 void* workspace, size_t workspace_bytes, trf_stream_t stream) {
  if (int rc = check_shape(batch, T, F)) return rc;
  if (int rc = check_precision(precision)) return rc;
  TRF_REQUIRE(X, "X");
  TRF_REQUIRE(packed_layer, "packed_layer");
  TRF_REQUIRE(workspace, "workspace");
  const Workspace w = plan(batch, T, F, static_cast<uint8_t*>(workspace));
  if (workspace_bytes < w.bytes)
    return fail(TRF_ERR_WORKSPACE, "workspace is %zu bytes, need %zu", workspace_bytes, w.bytes);
  hipStream_t st = as_hip(stream);
  const int64_t n = int64_t(batch) * T * F;
  trf::launch_add_rmsnorm(X, nullptr, 0, w.xn, 1, n, 1e-12f, st);
  if (int rc = check_launch("add_rmsnorm")) return rc;
  trf::launch_ff(static_cast<const uint8_t*>(packed_layer), X, w.xn, n, precision, 1e-12f, st);
  return check_launch("feed_forward");
}

size_t trf_mask_head_packed_bytes(const int32_t* dins, int32_t n_bands, int32_t hidden) {
  MaskLayout L;
  if (mask_layout(dins, n_bands, hidden, L)) return 0;
  return L.total;
}

int trf_pack_mask_head(const trf_mask_band_src* bands, const int32_t* dins, int32_t n_bands, int32_t hidden,
                       const float* final_gamma, void* packed, trf_stream_t stream) {
  MaskLayout L;
  if (int rc = mask_layout(dins, n_bands, hidden, L)) return rc;
  if (!bands) return fail(TRF_ERR_ARG, "bands must not be NULL");
  if (!final_gamma) return fail(TRF_ERR_ARG, "final_gamma must not be NULL");
  TRF_REQUIRE(packed, "packed");
  for (int f = 0; f < n_bands; ++f)
    if (!bands[f].w1 || !bands[f].b1 || !bands[f].w2 || !bands[f].b2)
      return fail(TRF_ERR_ARG, "bands[%d] has a NULL weight pointer", f);
  hipStream_t st = as_hip(stream);
  uint8_t* d = static_cast<uint8_t*>(packed);
  for (int f = 0; f < n_bands; ++f) {
    trf::launch_pack_mask_band(bands[f].w1, final_gamma, bands[f].b1, bands[f].w2, bands[f].b2, L.din[f], hidden,
                               d + L.wofs[f], reinterpret_cast<float*>(d + L.b1_off) + size_t(f) * hidden,
                               reinterpret_cast<float*>(d + L.b2_off[f]), st);
    if (int rc = check_launch("pack_mask_head")) return rc;
  }
  return TRF_OK;
}

int trf_mask_head(const float* X, int32_t n_frames, int32_t n_bands, const int32_t* dins, int32_t hidden,
                  const void* packed, int32_t precision, float* mask, trf_stream_t stream) {
  MaskLayout L;
  if (int rc = mask_layout(dins, n_bands, hidden, L)) return rc;
  if (precision != TRF_MASK_SPLIT && precision != TRF_MASK_FP16)
    return fail(TRF_ERR_ARG, "precision must be 0 (split) or 1 (fp16), got %d", precision);
  if (n_frames < 0) return fail(TRF_ERR_ARG, "n_frames must be >= 0, got %d", n_frames);
  if (int64_t(n_frames) * n_bands >= (int64_t(1) << 31))
    return fail(TRF_ERR_ARG, "n_frames * n_bands = %lld tokens is too large", (long long)n_frames * n_bands);
  if (n_frames == 0) return TRF_OK;
  TRF_REQUIRE(X, "X");
  TRF_REQUIRE(packed, "packed");
  TRF_REQUIRE(mask, "mask");
  trf::MaskPlan plan;
  const unsigned grid = mask_plan(L, n_frames, plan);
  trf::launch_mask_head(X, static_cast<const uint8_t*>(packed), mask, plan, grid, precision, as_hip(stream));
  return check_launch("mask_head");
}

size_t trf_band_split_packed_bytes(const int32_t* dins, int32_t n_bands) {
  std::vector<size_t> wofs;
  size_t total;
  if (band_layout(dins, n_bands, wofs, total)) return 0;
  return total * 4;
}

int trf_pack_band_split(const trf_band_split_src* bands, const int32_t* dins, int32_t n_bands, void* packed,
                        trf_stream_t stream) {
  std::vector<size_t> wofs;
  size_t total;
  if (int rc = band_layout(dins, n_bands, wofs, total)) return rc;
  if (!bands) return fail(TRF_ERR_ARG, "bands must not be NULL");
  TRF_REQUIRE(packed, "packed");
  for (int f = 0; f < n_bands; ++f)
    if (!bands[f].w || !bands[f].b || !bands[f].gamma) return fail(TRF_ERR_ARG, "bands[%d] has a NULL pointer", f);
  float* d = static_cast<float*>(packed);
  for (int f = 0; f < n_bands; ++f) {
    trf::launch_pack_band_split(bands[f].w, bands[f].b, bands[f].gamma, dins[f], sqrtf(float(dins[f])), d + wofs[f],
                                as_hip(stream));
    if (int rc = check_launch("pack_band_split")) return rc;
  }
  return TRF_OK;
}

int trf_band_split(const float* feats, int32_t n_frames, int32_t n_bands, const int32_t* dins, const void* packed,
                   float* X, trf_stream_t stream) {
  std::vector<size_t> wofs;
  size_t total;
  if (int rc = band_layout(dins, n_bands, wofs, total)) return rc;
  if (n_frames < 0) return fail(TRF_ERR_ARG, "n_frames must be >= 0, got %d", n_frames);
  if (int64_t(n_frames) * n_bands >= (int64_t(1) << 31))
    return fail(TRF_ERR_ARG, "n_frames * n_bands = %lld tokens is too large", (long long)n_frames * n_bands);
  if (n_frames == 0) return TRF_OK;
  TRF_REQUIRE(feats, "feats");
  TRF_REQUIRE(packed, "packed");
  TRF_REQUIRE(X, "X");
  trf::BandPlan plan{};
  plan.n_bands = n_bands;
  plan.n_frames = n_frames;
  plan.ngroups = (n_frames + trf::kBandFrames - 1) / trf::kBandFrames;
  int col = 0;
  std::vector<int> order(n_bands);
  for (int f = 0; f < n_bands; ++f) {
    plan.col[f] = uint32_t(col);
    plan.wofs[f] = uint32_t(wofs[f]);
    plan.din[f] = uint32_t(dins[f]);
    col += dins[f];
    order[f] = f;
  }
  plan.width = col;
  if (total >= (size_t(1) << 32)) return fail(TRF_ERR_ARG, "packed band split would exceed 16 GiB");
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return dins[a] > dins[b]; });  // widest first
  for (int f = 0; f < n_bands; ++f) plan.order[f] = uint32_t(order[f]);
  trf::launch_band_split(feats, static_cast<const float*>(packed), X, plan, as_hip(stream));
  return check_launch("band_split");
}

int trf_overlap_add(const float* y, int32_t n_chunks, int64_t y_stride, int32_t L, const int64_t* starts,
                    const float* window, int64_t n, float* acc, float* wsum, trf_stream_t stream) {
  if (n_chunks < 0 || n < 0) return fail(TRF_ERR_ARG, "n_chunks and n must be >= 0 (got %d, %lld)", n_chunks, (long long)n);
  if (n_chunks == 0 || n == 0) return TRF_OK;
  if (L < 1 || int64_t(L) > y_stride)
    return fail(TRF_ERR_ARG, "L must be in [1, y_stride] (got L = %d, y_stride = %lld)", L, (long long)y_stride);
  if (2 * n >= (int64_t(1) << 31) * 256) return fail(TRF_ERR_ARG, "n = %lld samples is too large", (long long)n);
  if (!y || !starts || !window || !acc || !wsum) return fail(TRF_ERR_ARG, "pointers must not be NULL");
  trf::launch_overlap_add(y, n_chunks, y_stride, L, starts, window, n, acc, wsum, as_hip(stream));
  return check_launch("overlap_add");
}

int trf_overlap_finish(const float* acc, const float* wsum, int64_t n, float gain, float* out, trf_stream_t stream) {
  if (n < 0) return fail(TRF_ERR_ARG, "n must be >= 0, got %lld", (long long)n);
  if (n == 0) return TRF_OK;
  if (!(gain > 0.f)) return fail(TRF_ERR_ARG, "gain must be > 0");
  if (2 * n >= (int64_t(1) << 31) * 256) return fail(TRF_ERR_ARG, "n = %lld samples is too large", (long long)n);
  if (!acc || !wsum || !out) return fail(TRF_ERR_ARG, "pointers must not be NULL");
  trf::launch_overlap_finish(acc, wsum, n, gain, out, as_hip(stream));
  return check_launch("overlap_finish");
}

}  // extern "C"
