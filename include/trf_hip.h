/*
 * trf_hip.h - C ABI of the MI355X (gfx950) BS-RoFormer transformer stack.
 *
 * The library replaces the AVX512-BF16 torch ops of LoggeL/turbo-roformer on the default path
 * (src/turbo_roformer/csrc/kernels.cpp:644-652: add_rmsnorm, qkv_rope_gemm, attention,
 * gemm_res_norm, gemm_gelu; the other two, rope_pack and gate_merge, serve the unfused and SDPA
 * variants, and their work is done inside trf_qkv_rope_gemm and trf_attention) and the stack loop that
 * calls them (FastBSRoformer._transformer_cpp, src/turbo_roformer/fast.py:269-341) with HIP
 * kernels, and the steps either side of it: the band split that feeds the stack and the mask head
 * that follows it (fast.py:377-387), plus the overlap-add that assembles a song from its chunks.
 * Every entry point takes plain device pointers, sizes and a HIP stream;
 * no torch type appears in a signature.  The library allocates no memory: the caller owns every
 * buffer.  Its state is a thread-local error string, each device's CU count (read once, for the
 * kernels that deal their work to one workgroup per CU) and the static workspace of
 * trf_stack_forward_static: a device array of TRF_STATIC_WORKSPACE_BYTES in the library's code
 * object, which every process that launches one of the library's kernels holds on that GPU.
 *
 * Shapes are fixed by the model: dim 256, 8 heads x 64, FF hidden 1024 (the mask head's
 * band widths and hidden size are arguments).
 *
 * Token order.  The residual stream X is fp32 [batch * T * F, 256] with token index
 *     tok = (c * T + t) * F + f        (chunk c, frame t, band f)
 * exactly as the reference keeps it (fast.py:378-380), extended by a chunk index c.
 * Time attention (mode 0) runs over frames: batch*F sequences of length T.
 * Frequency attention (mode 1) runs over bands: batch*T sequences of length F.
 *
 * Sequence buffers (written by trf_qkv_rope_gemm, read by trf_attention), bf16, with
 * Lpad = trf_seq_pad(L) and sequence s, head h, position p, head feature d:
 *     Q  [nseq][8][8][Lpad][8]  index (((s*8 + h)*8 + d/8)*Lpad + p)*8 + d%8  (rotated, times log2(e))
 *     K  [nseq][8][8][Lpad][8]  same index                                   (rotated)
 *     Vt [nseq][8][64][Lpad]    index ((s*8 + h)*64 + d)*Lpad + p             (transposed V)
 * Q and K are chunk-major: the 16-byte chunk of features 8c..8c+7 of consecutive positions is
 * contiguous, which is how the MFMA accumulators of the projection hold them.
 * Positions p >= L are written as zeros.  G is fp32 [ntok][8] = sigmoid(gate logits).
 *
 * All bf16 values are passed as uint16_t bit patterns.  Error codes: 0 = ok; otherwise
 * trf_last_error() returns a message for the calling thread.
 */
#ifndef TRF_HIP_H
#define TRF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRF_ABI_VERSION 8

#define TRF_DIM 256
#define TRF_HEADS 8
#define TRF_HEAD_DIM 64
#define TRF_QKVG_ROWS 1544 /* q(8x64) | k(8x64) | v(8x64) | gate(8) */
#define TRF_FF_HIDDEN 1024

enum trf_status {
  TRF_OK = 0,
  TRF_ERR_ARG = 1,       /* bad argument: null pointer, misalignment, unsupported size */
  TRF_ERR_WORKSPACE = 2, /* workspace smaller than trf_stack_workspace_bytes() */
  TRF_ERR_HIP = 3        /* a HIP runtime call or kernel launch failed */
};

enum trf_mode { TRF_MODE_TIME = 0, TRF_MODE_FREQ = 1 };

enum trf_dtype { TRF_F32 = 0, TRF_BF16 = 1 };

/* Arithmetic of the feed-forward GEMMs.
 * TRF_PREC_BF16: every GEMM operand is rounded to bf16, as the reference kernels do
 *   (kernels.cpp:30-33, docs/how-it-works.md:164-170).
 * TRF_PREC_FF_SPLIT: FF1 and FF2 take split-bf16 operands v = hi + lo (hi = bf16(v),
 *   lo = bf16(v - hi)) and compute hi.hi + hi.lo + lo.hi on the bf16 MFMA with fp32
 *   accumulation, which removes the four rounding points (W1, W2, xn, gelu(h)) that dominate the
 *   bf16 design's error.  It needs the lo weight parts (trf_layer_src.w_ff1_lo / w_ff2_lo).
 *   Attention, the QKV GEMM and the out-projection stay bf16 in every mode.
 * TRF_PREC_FF_FP16: FF1 and FF2 take fp16 operands (xn, W1, gelu(h), W2: 11-bit significands
 *   instead of bf16's 8) on the fp16 MFMA with fp32 accumulation, at the cost of the bf16 mode.  The
 *   fp16 weights are fp16(w_ff* + w_ff*_lo), so the lo parts make them round from fp32.  Values
 *   must stay within fp16 range (|x| < 65504), which holds for normalised inputs. */
enum trf_precision { TRF_PREC_BF16 = 0, TRF_PREC_FF_SPLIT = 1, TRF_PREC_FF_FP16 = 2 };

/* Same type as hipStream_t; NULL is the default stream. */
typedef struct ihipStream_t* trf_stream_t;

/* Plain folded weights of one sub-layer (attention + feed-forward), device pointers,
 * row-major [out][in].  This is what FastBSRoformer._prep builds (fast.py:163-191):
 *   w_qkvg = [Wq * 16*g_attn / 8 ; Wk * 16*g_attn ; Wv * 16*g_attn ; Wgate * 16*g_attn]
 *   w_ff1  = W1 * 16*g_ff
 * (g = RMSNorm gamma, 16 = sqrt(256)), so every runtime norm is x / max(|x|, 1e-12). */
typedef struct trf_layer_src {
  const uint16_t* w_qkvg; /* bf16 [1544][256] */
  const float* b_gate;    /* fp32 [8] */
  const uint16_t* w_out;  /* bf16 [256][512] */
  const uint16_t* w_ff1;  /* bf16 [1024][256] */
  const float* b_ff1;     /* fp32 [1024] */
  const uint16_t* w_ff2;  /* bf16 [256][1024] */
  const float* b_ff2;     /* fp32 [256] */
  /* Optional (NULL = zero): bf16 residuals w - bf16(w) of the fp32 folded W1 and W2, used by
   * TRF_PREC_FF_SPLIT.  Same shapes as w_ff1 / w_ff2. */
  const uint16_t* w_ff1_lo;
  const uint16_t* w_ff2_lo;
} trf_layer_src;

/* ---------------------------------------------------------------- library */

int trf_abi_version(void);
const char* trf_last_error(void);

/* Padded sequence length used by the Q/K/Vt buffers (multiple of 64). */
int32_t trf_seq_pad(int32_t L);

/* Element count (bf16) of one of Q, K or Vt for a mode and shape. */
int64_t trf_seq_buffer_elems(int32_t mode, int32_t batch, int32_t T, int32_t F);

/* ---------------------------------------------------------------- weights */

/* Bytes of one packed sub-layer (all weights in the kernels' operand order). */
size_t trf_layer_packed_bytes(void);

/* Pack plain folded weights (device) into dst (device, trf_layer_packed_bytes()).
 * Replaces the host-side VNNI packing _pack_w (fast.py:43-49) and _prep (fast.py:163-191). */
int trf_pack_layer(const trf_layer_src* src, void* dst, trf_stream_t stream);

/* ---------------------------------------------------------------- per-op entry points */

/* X += Y (Y optional, f32 or bf16); out = X / max(|X|, eps) per row of 256.
 * Replaces add_rmsnorm (kernels.cpp:101-137). */
int trf_add_rmsnorm(float* X, const void* Y, int32_t y_dtype, void* out, int32_t out_dtype,
                    int64_t n_rows, float eps, trf_stream_t stream);

/* xn [ntok][256] bf16 -> Q, K, Vt (layouts above) and G = sigmoid(xn.Wg + b_gate).
 * Rotary on q, k in fp32 from the accumulators with the caller's fp32 tables
 * rope = [2][L][32] (cos then sin, angle = p * 10000^(-2i/64)).  The 1/8 attention scale is
 * folded into the q rows of the weights; q is further multiplied by log2(e) in fp32 before its
 * single bf16 rounding, so trf_attention's scores are base-2 exponents.
 * Replaces qkv_rope_gemm (kernels.cpp:439-540). */
int trf_qkv_rope_gemm(const uint16_t* xn, const void* packed_layer, const float* rope, int32_t mode,
                      int32_t batch, int32_t T, int32_t F, uint16_t* Q, uint16_t* K, uint16_t* Vt,
                      float* G, trf_stream_t stream);

/* Exact (non-online) softmax attention per (sequence, head): with s = q.k (q as written by
 * trf_qkv_rope_gemm), a shift c, P = bf16(2^(s - c)) unnormalised and an fp32 row sum, the epilogue
 * writes
 * O[tok][h*64 + d] = gate[tok][h] / rowsum * (P V)[.][d] in token order, bf16.
 * For sequences of up to 64 positions c is the row max m and the row sum is that of 2^(s - c), as in
 * the reference.  Longer sequences are swept once with an integer c >= m (raised with exact
 * power-of-two rescales), which gives the same result as any integer shift and moves P's bf16
 * rounding by the factor 2^(m - ceil m); their row sum is that of the rounded P, which keeps the
 * result as close to exact attention as the reference's row-max arithmetic.
 * Replaces attention (kernels.cpp:250-388). */
int trf_attention(const uint16_t* Q, const uint16_t* K, const uint16_t* Vt, const float* G,
                  uint16_t* O, int32_t mode, int32_t batch, int32_t T, int32_t F,
                  trf_stream_t stream);

/* trf_qkv_rope_gemm followed by trf_attention in one kernel, for sequences of at most 64 positions
 * (L = T in mode 0, F in mode 1; the frequency attention of 62 bands): xn [ntok][256] bf16 -> O
 * [ntok][512] bf16 with the same arithmetic (shift = the row max), but Q, K, V and the gates never
 * leave the chip, so no sequence buffers are needed.  The stack uses it for every sub-layer with
 * L <= 64.  Replaces qkv_rope_gemm + attention (kernels.cpp:439-540, 250-388) for short sequences;
 * TRF_ERR_ARG when L > 64. */
int trf_qkv_attention_short(const uint16_t* xn, const void* packed_layer, const float* rope, int32_t mode,
                            int32_t batch, int32_t T, int32_t F, uint16_t* O, trf_stream_t stream);

/* Bytes of one weight matrix W [rows][K] packed by trf_pack_weight (0 for a bad shape). */
size_t trf_weight_packed_bytes(int32_t rows, int32_t K);

/* Pack a bf16 weight W [rows][K] (row-major, device; K a multiple of 16) into the MFMA operand tiles
 * that trf_gemm_res_norm and trf_gemm_gelu read (rows padded with zeros to a multiple of 32), into
 * packed (device, trf_weight_packed_bytes(rows, K)).  Replaces _pack_w (fast.py:43-49), which builds
 * the reference ops' P["Wop"], P["W1p"] and P["W2p"] (fast.py:182-189). */
int trf_pack_weight(const uint16_t* W, int32_t rows, int32_t K, void* packed, trf_stream_t stream);

/* gemm_res_norm(A, Wp, bias, X, xn, eps): X += A @ W^T (+ bias); xn = X / max(|X|, eps) as bf16.
 * A bf16 [n_rows][K] (K a multiple of 16: 512 for the out-projection, 1024 for FF2), W packed by
 * trf_pack_weight with rows = 256, bias fp32 [256] or NULL, X fp32 [n_rows][256] updated in place,
 * xn bf16 [n_rows][256].  Replaces gemm_res_norm (kernels.cpp:542-586). */
int trf_gemm_res_norm(const uint16_t* A, int32_t K, const void* w_packed, const float* bias, float* X,
                      uint16_t* xn, int64_t n_rows, float eps, trf_stream_t stream);

/* gemm_gelu(xn, Wp, bias, H): H = gelu_erf(xn @ W^T + bias) as bf16.  xn bf16 [n_rows][256], W packed by
 * trf_pack_weight with rows = n_out and K = 256 (n_out a multiple of 32), bias fp32 [n_out], H bf16
 * [n_rows][n_out].  Replaces gemm_gelu (kernels.cpp:609-642) and the oneDNN FF1 (fast.py:343-346). */
int trf_gemm_gelu(const uint16_t* xn, const void* w_packed, const float* bias, int32_t n_out, uint16_t* H,
                  int64_t n_rows, trf_stream_t stream);

/* ---------------------------------------------------------------- stack */

/* Workspace bytes for trf_stack_forward / trf_attn_block / trf_ff_block at a shape. */
size_t trf_stack_workspace_bytes(int32_t batch, int32_t T, int32_t F);

/* The whole stack: one norm, then for each layer i (mode modes[i]):
 *   qkv_rope_gemm, attention, and one fused kernel for out-proj + residual + norm, FF1 + GELU,
 *   FF2 + residual + norm (the FF hidden activation never reaches memory).
 * X fp32 [batch*T*F][256] is updated in place.  packed_layers is a host array of
 * n_layers device pointers (trf_pack_layer output); modes is a host array.
 * precision is a trf_precision value for the feed-forward GEMMs.
 * rope_time = [2][T][32], rope_freq = [2][F][32] fp32 device tables.
 * Replaces FastBSRoformer._transformer_cpp (fast.py:269-341). */
int trf_stack_forward(float* X, int32_t batch, int32_t T, int32_t F,
                      const void* const* packed_layers, const int32_t* modes, int32_t n_layers,
                      int32_t precision, const float* rope_time, const float* rope_freq,
                      void* workspace, size_t workspace_bytes, trf_stream_t stream);

/* Size of the static workspace of trf_stack_forward_static: one 17 s chunk (batch 1 at 62 bands, up to
 * T = 1826 frames; trf_stack_workspace_bytes(1, 1701, 62) is 477 MiB). */
#define TRF_STATIC_WORKSPACE_BYTES ((size_t)512 << 20)

/* No counterpart in the reference.  For callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  trf_stack_forward with the same
 * kernels and results, but with its workspace in a static device array of TRF_STATIC_WORKSPACE_BYTES
 * that the library holds on each GPU it runs on until the process ends (its device address is looked up
 * once per device, on the first call with that device current).  It allocates nothing; shapes whose
 * trf_stack_workspace_bytes exceed the array fail with TRF_ERR_WORKSPACE.  All calls on one GPU share
 * that GPU's array, which keeps the last call's contents: calls that overlap on one GPU (other streams
 * or threads) race, so the caller serialises them.  Nothing in the array has to start at zero: every
 * workspace element a call reads, the same call wrote first.  Under HIP graph capture: the first call
 * on a device (which looks the array's address up) must happen outside the capture; later calls
 * capture as plain kernel launches.  The array is part of the library's code object, so every process
 * that launches any of the library's kernels on a GPU holds it there, whether or not it calls this. */
int trf_stack_forward_static(float* X, int32_t batch, int32_t T, int32_t F,
                             const void* const* packed_layers, const int32_t* modes, int32_t n_layers,
                             int32_t precision, const float* rope_time, const float* rope_freq,
                             trf_stream_t stream);

/* Kernel slots of one layer in launch order (for trf_stack_forward_timed): the QKV GEMM, the
 * attention, and the fused post-attention kernel (out-projection + residual + norm + FF1 + GELU +
 * FF2 + residual + norm). */
enum trf_kernel_slot {
  TRF_SLOT_QKV = 0,
  TRF_SLOT_ATTN = 1,
  TRF_SLOT_POST = 2,
  TRF_SLOTS_PER_LAYER = 3
};

/* trf_stack_forward that also records caller-created hipEvent_t handles at the start and end of each
 * kernel: events[2*(i*TRF_SLOTS_PER_LAYER + k)] and events[... + 1] for kernel k of layer i, skipping
 * NULL entries; n_events must be 0 or 2*TRF_SLOTS_PER_LAYER*n_layers.  The events are part of the
 * kernel's dispatch (hipExtLaunchKernel), which costs less than separate event records; a layer with
 * sequences of at most 64 positions has one kernel for QKV and attention, reported in the attention
 * slot, and its QKV slot is an empty interval.  This is the counterpart of the reference's
 * per-section wall-clock profile (fast.py:62-80, 279-340). */
int trf_stack_forward_timed(float* X, int32_t batch, int32_t T, int32_t F,
                            const void* const* packed_layers, const int32_t* modes,
                            int32_t n_layers, int32_t precision, const float* rope_time,
                            const float* rope_freq,
                            void* workspace, size_t workspace_bytes, void* const* events,
                            int32_t n_events, trf_stream_t stream);

/* One attention sub-layer on the residual stream: xn = norm(X), qkv + rotary, attention,
 * X += O @ Wout^T.  The counterpart of "x = attn(x) + x" (model.py:141) on the folded
 * weights; rope is the table of this mode's axis. */
int trf_attn_block(float* X, int32_t batch, int32_t T, int32_t F, const void* packed_layer,
                   int32_t mode, const float* rope, void* workspace, size_t workspace_bytes,
                   trf_stream_t stream);

/* One feed-forward sub-layer: X += W2 gelu(W1 norm(X) + b1) + b2 ("x = ff(x) + x",
 * model.py:142), with the FF GEMMs in the given trf_precision. */
int trf_ff_block(float* X, int32_t batch, int32_t T, int32_t F, const void* packed_layer,
                 int32_t precision, void* workspace, size_t workspace_bytes, trf_stream_t stream);

/* ---------------------------------------------------------------- band split
 * The step before the stack: per band f of width dins[f] (2 * frequencies * channels), the RMSNorm
 * of the frame's dins[f] spectral features and a Linear dins[f] -> 256 (BandSplit, model.py:147-155;
 * called at fast.py:377-380), written as the stack's tokens X [n_frames * n_bands][256] fp32 (token
 * n * n_bands + f).  The features are the reference's per-frame layout feats [n_frames][sum(dins)]
 * fp32, (bin, channel, re/im) order (fast.py:372-376), band f at columns sum(dins[:f]) .. + dins[f].
 * Arithmetic is fp32 (fp32 MFMA).  Limits: 1 <= n_bands <= 64; each din a multiple of 4 in
 * [4, 16384]. */

/* One band's plain fp32 weights, device pointers: band_split.to_features.<f>.1.weight [256][din],
 * .1.bias [256] and the RMSNorm gain .0.gamma [din]. */
typedef struct trf_band_split_src {
  const float* w;
  const float* b;
  const float* gamma;
} trf_band_split_src;

/* Bytes of the packed band split (0 if the arguments are out of the limits above). */
size_t trf_band_split_packed_bytes(const int32_t* dins, int32_t n_bands);

/* Pack the bands (bands, dins: host arrays of n_bands) into packed (device, 16-byte aligned). */
int trf_pack_band_split(const trf_band_split_src* bands, const int32_t* dins, int32_t n_bands, void* packed,
                        trf_stream_t stream);

/* X [n_frames * n_bands][256] from feats [n_frames][sum(dins)]; n_frames = 0 does nothing. */
int trf_band_split(const float* feats, int32_t n_frames, int32_t n_bands, const int32_t* dins,
                   const void* packed, float* X, trf_stream_t stream);

/* ---------------------------------------------------------------- song assembly
 * Hamming-windowed overlap-add of chunk predictions (the reference's overlap_add, chunking.py:39-61):
 * for chunks in ascending order, acc[ch][s:s+L] += y[c][ch][:L] * window[:L] and wsum[s:s+L] += window[:L],
 * each term with the reference's two fp32 roundings (product, then sum), so the sums are bitwise those of
 * its loop; a song processed in several batches calls trf_overlap_add once per batch, in chunk order.
 * y [n_chunks][2][y_stride] fp32; starts: device int64 [n_chunks], ascending, each chunk's first sample
 * (the library cannot read them on the host: with starts out of order the sums are wrong, but every
 * access stays in bounds); window: device fp32 [>= L]; acc [2][n] and wsum [n]: device fp32, zeroed
 * before the first batch. */
int trf_overlap_add(const float* y, int32_t n_chunks, int64_t y_stride, int32_t L, const int64_t* starts,
                    const float* window, int64_t n, float* acc, float* wsum, trf_stream_t stream);

/* out [2][n] = acc / max(wsum, 1e-10) / gain, two correctly rounded divisions (out may be acc): the
 * reference's normalisation by the summed window, then by the peak gain (separator.py:187-201). */
int trf_overlap_finish(const float* acc, const float* wsum, int64_t n, float gain, float* out,
                       trf_stream_t stream);

/* ---------------------------------------------------------------- mask head
 * The step after the stack: final RMSNorm and, per band f of width dins[f] (its mask columns:
 * 2 * frequencies * channels), the mask-estimator MLP
 *     mask_f = GLU(W2_f tanh(W1_f xn + b1_f) + b2_f),   xn = x / max(|x|, 1e-12) * sqrt(256) * gamma
 * (MaskEstimator, model.py:158-178, mask_estimator_depth 2; the reference's batched form is
 * FastBSRoformer._mask, fast.py:139-160 and 349-360, called at fast.py:385-387).  The mask row of a
 * frame is the bands' outputs side by side: [n_frames][sum(dins)] fp32, band f at columns
 * sum(dins[:f]) .. + dins[f], each the GLU a * sigmoid(g) of W2's first and second dins[f] rows.
 *
 * Limits: 1 <= n_bands <= 64; hidden a multiple of 64 in [64, 8192]; each din a multiple of 4 in
 * [4, 16384]; at most 192 jobs, a job being up to 6 output pairs (64 columns: 32 of a, 32 of g) of
 * a band, i.e. sum over bands of ceil(ceil(din / 32) / 6) <= 192. */

enum trf_mask_precision {
  /* Both GEMMs on fp16 MFMA with every operand split into hi = f16(v) and lo = f16(v - hi),
   * hi.hi + hi.lo + lo.hi: fp32-level agreement with the reference's fp32 mask head (default). */
  TRF_MASK_SPLIT = 0,
  /* fp16 operands, one MFMA per product: ~3x fewer MFMAs, ~68 dB mask SNR against fp32. */
  TRF_MASK_FP16 = 1
};

/* One band's plain fp32 weights, device pointers, PyTorch Linear layout [out][in]:
 * mask_estimators.0.to_freqs.<f>.0.0.{weight,bias} and .0.2.{weight,bias}. */
typedef struct trf_mask_band_src {
  const float* w1; /* [hidden][256] */
  const float* b1; /* [hidden] */
  const float* w2; /* [2 * din][hidden] */
  const float* b2; /* [2 * din] */
} trf_mask_band_src;

/* Bytes of the packed mask head (0 if the arguments are out of the limits above). */
size_t trf_mask_head_packed_bytes(const int32_t* dins, int32_t n_bands, int32_t hidden);

/* Pack the band MLPs (bands: host array of n_bands; dins: host array) and the final norm's gamma
 * (device fp32 [256], final_norm.gamma) into packed (device, trf_mask_head_packed_bytes(),
 * 16-byte aligned).  |w1 * gamma| and |w2| must be below 65504 (fp16 range). */
int trf_pack_mask_head(const trf_mask_band_src* bands, const int32_t* dins, int32_t n_bands,
                       int32_t hidden, const float* final_gamma, void* packed, trf_stream_t stream);

/* mask [n_frames][sum(dins)] fp32 from the stack output X [n_frames][n_bands][256] fp32 (token
 * order of the stack: frame-major, band-minor), precision a trf_mask_precision value.  dins,
 * n_bands and hidden must be those of the packing.  n_frames = 0 does nothing. */
int trf_mask_head(const float* X, int32_t n_frames, int32_t n_bands, const int32_t* dins, int32_t hidden,
                  const void* packed, int32_t precision, float* mask, trf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TRF_HIP_H */
