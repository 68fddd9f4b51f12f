/*
 * tbn_hip.h -- C ABI of the MI355X (gfx950) quantized compute path of tbn.
 *
 * This is the drop-in boundary: plain pointers and sizes, int status codes,
 * one explicit HIP stream per call.  Every tensor pointer is a DEVICE pointer
 * (HBM); the library never copies through the host.  All calls are
 * asynchronous on `stream` (NULL = the default stream) unless stated.
 *
 * Status codes are the values of tbn::ErrorCode
 * (tbn-runtime/include/tbn/utils/errors.hpp:10-22).  On failure the message
 * of the most recent error on the calling thread is available from
 * tbn_hip_last_error().  Argument errors are detected on the host before any
 * work is queued.
 *
 * Packed formats (bit-exact with the reference):
 *   BINARY tensor      1 byte per weight, byte 1 = +1, any other byte = -1
 *                      (tbn-runtime/include/tbn/runtime/types.hpp:86-87;
 *                       tbn-runtime/src/operators/quantized_gemm_neon.cpp:205).
 *   BinaryMatrix       weight matrix W[K,N] packed column by column: column n
 *                      occupies K_pad/8 bytes at packed + n*K_pad/8, the value
 *                      at row k is bit (k&7) of byte (k>>3), bit 1 = -1, and
 *                      padding rows/columns are +1 (bit 0)
 *                      (GeMM/05-final/GeMM.cpp:114-151).  The runtime pads
 *                      K_pad = ceil128(K), N_pad = ceil8(N)
 *                      (tbn-runtime/src/operators/quantized_gemm_neon.cpp:38-58).
 *   Ternary 2-bit      flat element i -> byte i>>2, bits (i&3)*2..+1,
 *                      00 = -1, 01 = 0, 10 = +1, 11 decodes to 0
 *                      (tbn-runtime/include/tbn/memory/packed_weights.hpp:35-71).
 *                      For the GEMM/conv kernels the 2-bit codes are applied
 *                      to the transposed zero-padded matrix W^T[N_pad, K_pad],
 *                      so column n occupies K_pad/4 bytes at packed + n*K_pad/4.
 *
 * Arithmetic ("mode F32"): activations stay fp32, weights are the exact
 * values +-1 (or 0) times an fp32 scale, accumulation is fp32.  Every product
 * a*w is formed exactly (a is split into three bf16 parts whose sum is a, and
 * each part is multiplied by the +-1/0 weight on the bf16 matrix cores);
 * only the accumulation order differs from a sequential fp32 loop.
 */
#ifndef TBN_HIP_H
#define TBN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* tbn::ErrorCode values (tbn-runtime/include/tbn/utils/errors.hpp:10-22). */
enum tbn_status {
    TBN_SUCCESS = 0,
    TBN_INVALID_ARGUMENT = -1,
    TBN_OUT_OF_MEMORY = -2,
    TBN_NOT_IMPLEMENTED = -3,
    TBN_INVALID_MODEL = -4,
    TBN_RUNTIME_ERROR = -5,
    TBN_QUANTIZATION_ERROR = -6,
    TBN_INVALID_SHAPE = -7,
    TBN_DEVICE_NOT_SUPPORTED = -8,
    TBN_ONNX_PARSE_ERROR = -9,
    TBN_OPERATOR_NOT_SUPPORTED = -10
};

typedef void* tbn_stream_t; /* a hipStream_t */

/* Row-major layout of a weight matrix handed to the packers:
 *   TBN_LAYOUT_KN  W[K,N]  (qlinear_matmul_binary's B, Gemm's B with transB=0)
 *   TBN_LAYOUT_NK  W[N,K]  (Conv weights [M_out, C, kh, kw] seen as [M_out, C*kh*kw]) */
enum tbn_layout { TBN_LAYOUT_KN = 0, TBN_LAYOUT_NK = 1 };

/* Float -> binary sign rules (the reference uses both):
 *   TBN_SIGN_GT_THRESHOLD  +1 iff w > threshold; 0, -0.0, NaN -> -1
 *                          (quantize_to_binary, quantized_gemm_neon.cpp:553)
 *   TBN_SIGN_GE_ZERO       +1 iff w >= 0; 0, -0.0 -> +1, NaN -> -1
 *                          (Session sign extraction, model.hpp:433,803)
 *   TBN_SIGN_GEMM_SAMPLED  the Session's Gemm rule decided on the device:
 *                          GE_ZERO when the sampled elements 0, s, 2s, ... of
 *                          W in memory order (s = max(1, K*N/1000)) are all
 *                          -1, 0, +1 or +-0.999, else GT_THRESHOLD at 0
 *                          (model.hpp:765-845); threshold is ignored */
enum tbn_sign_rule { TBN_SIGN_GT_THRESHOLD = 0, TBN_SIGN_GE_ZERO = 1, TBN_SIGN_GEMM_SAMPLED = 2 };

/* Epilogue flags for the GEMM / conv entry points. */
enum tbn_epilogue {
    TBN_EPI_NONE = 0,
    TBN_EPI_RELU = 1,            /* y = max(y, 0) after scale and bias        */
    TBN_EPI_BIAS_THEN_SCALE = 2, /* y = (acc + b) * s  (Session cached conv,  */
                                 /*  model.hpp:523-557); default y = acc*s + b */
                                 /*  (conv2d_binary_with_scales, conv2d.cpp:319-369) */
    TBN_EPI_MAXPOOL2X2 = 4,      /* conv only: fused 2x2 stride-2 max pool      */
    TBN_EPI_MAXPOOL3X3S2 = 8     /* tbn_hip_conv2d_f32 with TBN_EPI_RELU, stem
                                    shape only (3 input channels, 7x7, stride 2,
                                    M <= 64): fused 3x3 stride-2 pad-1 floor max
                                    pool (the ResNet stem's, model.hpp:577-629) */
};

/* Convolution geometry (NCHW input, [M, C, kh, kw] weights, groups = 1),
 * mirroring tbn::Conv2DParams (tbn-runtime/include/tbn/operators/conv2d.hpp:12-37). */
typedef struct tbn_conv2d_desc {
    int64_t n, c, h, w;   /* input  [n, c, h, w]                 */
    int64_t m;            /* output channels                     */
    int64_t kh, kw;       /* kernel                              */
    int64_t sh, sw;       /* stride                              */
    int64_t ph, pw;       /* symmetric zero padding              */
    int64_t dh, dw;       /* dilation                            */
} tbn_conv2d_desc;

/* ---- library -------------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char* tbn_hip_last_error(void);
/* Library version, major*10000 + minor*100 + patch. */
int tbn_hip_version(void);
/* Checks that the current HIP device is a gfx950 (MI355X); returns
 * TBN_DEVICE_NOT_SUPPORTED otherwise. */
int tbn_hip_device_check(void);
/* Waits for `stream` and reports any asynchronous device error. */
int tbn_hip_synchronize(tbn_stream_t stream);

/* ---- tuning controls (no counterpart in the reference) ---------------------
 * Process-wide launch-shape choices.  Each starts from an environment variable
 * read once, at the first call that needs it (TBN_CONV_TILE, TBN_CONV_SPLITS,
 * TBN_GEMM_SPLITS, TBN_GEMM_TILE, TBN_TBN_CONV), and changes only through
 * tbn_hip_set_tuning.
 * They pick kernel variants: a forced conv tile never changes a result (every
 * tile sums in the same order); a forced split count or GEMM tile changes the
 * summation order. */
enum tbn_tuning {
    TBN_TUNE_CONV_TILE = 1,   /* patch-conv tile id, -1 = automatic (default)   */
    TBN_TUNE_CONV_SPLITS = 2, /* patch-conv K splits, 0 = automatic; pooled
                                 convs never split                               */
    TBN_TUNE_GEMM_SPLITS = 3, /* wide GEMM K splits, 0 = automatic              */
    TBN_TUNE_GEMM_TILE = 4,   /* wide GEMM tile: 0 = 128x512, 1 = 64x128,
                                 2 = 32x128 in two K groups (even K/64 only),
                                 -1 = automatic (default)                        */
    TBN_TUNE_TBN_CONV = 5     /* TBN conv kernels: 0 = automatic (default),
                                 1 = the fused kernel where a tile fits,
                                 2 = the two-pass kernels (ternarized records in
                                 the caller's scratch, then the product); both
                                 give the same bits                               */
};
int tbn_hip_set_tuning(int option, int value);
int tbn_hip_get_tuning(int option, int* value);

/* ---- quantization (north_star subsystem 1) --------------------------------- */

/* quantize_to_binary(W, threshold), FLOAT32 input: out[i] = w[i] > threshold.
 * Replaces tbn::quantize_to_binary (tbn-runtime/src/operators/quantized_gemm_neon.cpp:544-565). */
int tbn_hip_quantize_to_binary_f32(const float* w, int64_t n, float threshold,
                                   uint8_t* out, tbn_stream_t stream);
/* quantize_to_binary, INT8 input: out[i] = w[i] > 0 (same reference lines 555-559). */
int tbn_hip_quantize_to_binary_i8(const int8_t* w, int64_t n, uint8_t* out, tbn_stream_t stream);
/* quantize_to_ternary(W, lo, hi): -1 if w < lo, +1 if w > hi, else 0.
 * Replaces tbn::quantize_to_ternary (quantized_gemm_neon.cpp:570-597). */
int tbn_hip_quantize_to_ternary_f32(const float* w, int64_t n, float lo, float hi,
                                    int8_t* out, tbn_stream_t stream);
/* Session sign extraction, out[i] = w[i] >= 0 (model.hpp:423-438,797-807). */
int tbn_hip_sign_ge0_f32(const float* w, int64_t n, uint8_t* out, tbn_stream_t stream);
/* Per-channel scale = mean |w| over `per_channel` contiguous elements, summed
 * sequentially in fp32 as the Session does (model.hpp:388-394): bit-exact. */
int tbn_hip_channel_mean_abs(const float* w, int64_t channels, int64_t per_channel,
                             float* scale, tbn_stream_t stream);

/* ---- packing (north_star subsystem 1) -------------------------------------- */

/* BINARY byte tensor (layout KN or NK) -> BinaryMatrix bits [N_pad][K_pad/8].
 * Requires K_pad >= K, N_pad >= N, K_pad % 64 == 0, N_pad % 8 == 0.
 * Replaces the transpose+pad+BinaryMatrix::pack sequence of
 * quantized_gemm_neon.cpp:197-214, model.hpp:456-480 and model.hpp:809-833. */
int tbn_hip_pack_binary(const uint8_t* bin, int64_t K, int64_t N, int layout,
                        int64_t K_pad, int64_t N_pad, uint8_t* packed, tbn_stream_t stream);
/* Fused float -> sign -> BinaryMatrix bits in one pass (same layout rules);
 * `sign_rule` picks the reference rule, `threshold` applies to GT_THRESHOLD. */
int tbn_hip_quantize_pack_binary_f32(const float* w, int64_t K, int64_t N, int layout,
                                     int sign_rule, float threshold,
                                     int64_t K_pad, int64_t N_pad, uint8_t* packed,
                                     tbn_stream_t stream);
/* BinaryMatrix bits -> int8 +-1 in layout KN or NK (the sign decode). */
int tbn_hip_unpack_binary(const uint8_t* packed, int64_t K, int64_t N, int layout,
                          int64_t K_pad, int8_t* out, tbn_stream_t stream);
/* Flat 2-bit encoding of n ternary values (TernaryPackedWeights::set_weight
 * over a fresh buffer, packed_weights.hpp:52-71); values other than -1,0,+1
 * encode as 0.  packed holds ceil(n/4) bytes. */
int tbn_hip_pack_ternary2(const int8_t* t, int64_t n, uint8_t* packed, tbn_stream_t stream);
/* Flat 2-bit decode (TernaryPackedWeights::get_weight, packed_weights.hpp:35-49). */
int tbn_hip_unpack_ternary2(const uint8_t* packed, int64_t n, int8_t* out, tbn_stream_t stream);
/* Ternary weights (layout KN or NK) -> GEMM 2-bit layout W^T[N_pad][K_pad],
 * zero padded.  Requires K_pad >= K, N_pad >= N, K_pad % 32 == 0. */
int tbn_hip_pack_ternary(const int8_t* t, int64_t K, int64_t N, int layout,
                         int64_t K_pad, int64_t N_pad, uint8_t* packed, tbn_stream_t stream);
/* Fused float -> ternary (lo/hi thresholds) -> GEMM 2-bit layout. */
int tbn_hip_quantize_pack_ternary_f32(const float* w, int64_t K, int64_t N, int layout,
                                      float lo, float hi, int64_t K_pad, int64_t N_pad,
                                      uint8_t* packed, tbn_stream_t stream);

/* ---- float x binary / float x ternary GEMM (north_star subsystem 2) -------- */

/* C[m,n] = acc[m,n] * alpha * s[n] + b[n]   (optionally ReLU), with
 *   acc[m,n] = sum_k A[m,k] * w[k,n],  w = +-1 decoded from BinaryMatrix bits.
 * A: fp32 [M, K] row-major, leading dimension lda >= K.
 * scale: per-column fp32 [N] or NULL (then s = 1); alpha: scalar multiplier
 * (the reference's scalar `scale` argument); bias: [N] or NULL.
 * C: fp32 [M, N], ldc >= N.  Requires K_pad % 32 == 0, K_pad >= K, N_pad >= N.
 * Shapes whose tiles would not fill the chip split K over blocks and keep the
 * partial sums in the library's per-device stream workspace; those calls
 * return TBN_NOT_IMPLEMENTED while the stream captures.
 * Replaces tbn::qlinear_matmul_binary / _blocked_packed / _naive
 * (quantized_gemm_neon.cpp:63-90,249-309,380-430), computing the fp32-activation
 * product of qlinear_matmul_binary_naive. */
int tbn_hip_gemm_f32_binary(const float* A, int64_t lda, int64_t M, int64_t N, int64_t K,
                            const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                            const float* scale, float alpha, const float* bias, int flags,
                            float* C, int64_t ldc, tbn_stream_t stream);
/* Same with w in {-1, 0, +1} from the GEMM 2-bit layout.  Replaces
 * tbn::qlinear_matmul_ternary (quantized_gemm_neon.cpp:506-538) with the true
 * float x ternary product its own test expects (test_quantized_operators.cpp:151-155). */
int tbn_hip_gemm_f32_ternary(const float* A, int64_t lda, int64_t M, int64_t N, int64_t K,
                             const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                             const float* scale, float alpha, const float* bias, int flags,
                             float* C, int64_t ldc, tbn_stream_t stream);

/* Weight kinds of the general entry points below. */
enum tbn_weights_kind { TBN_WEIGHTS_BINARY = 0, TBN_WEIGHTS_TERNARY = 1 };

/* No counterpart in the reference (a diagnostic for profiling).  Writes into
 * name (len bytes, NUL-terminated, truncated if short) the kernel, as a
 * profiler names it, that tbn_hip_gemm_f32_binary (weights
 * TBN_WEIGHTS_BINARY) or _ternary runs for this shape in this process now
 * (tuning controls included), for 16-byte aligned A and packed weights.  No
 * GPU work. */
int tbn_hip_gemm_kernel_name(int weights, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t K_pad,
                             int64_t N_pad, char* name, size_t len);

/* General quantized GEMM used by the Session's quantized Gemm node
 * (model.hpp:763-870): weights binary or ternary as above, and
 *   C[m,n] = epi(acc[m,n]) + beta * Cin,  Cin NULL, [N] (cin_1d) or [M, N]
 * with epi as in tbn_hip_gemm_f32_binary (ReLU, if requested, applies last). */
int tbn_hip_gemm_f32_quantized(int weights, const float* A, int64_t lda, int64_t M, int64_t N,
                               int64_t K, const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                               const float* scale, float alpha, const float* bias, const float* cin,
                               int cin_1d, float beta, int flags, float* C, int64_t ldc,
                               tbn_stream_t stream);

/* ---- binary / ternary Conv2D (north_star subsystem 3) ---------------------- */

/* Implicit-GEMM convolution, im2col formed on the fly (no column buffer):
 *   y[n,m,oh,ow] = epi( sum_{c,r,s} x[n,c,ih,iw] * w[m,(c,r,s)] )
 * with w = +-1 from BinaryMatrix bits packed from the [M, C*kh*kw] weights
 * (layout NK, K_pad >= C*kh*kw, K_pad % 32 == 0, N_pad >= M).
 * epi: default acc*alpha*s[m] + b[m]; TBN_EPI_BIAS_THEN_SCALE gives
 * (acc + b[m]) * alpha*s[m]; then TBN_EPI_RELU; then TBN_EPI_MAXPOOL2X2
 * (floor mode, output [n, m, OH/2, OW/2]).
 * Replaces tbn::conv2d_binary / conv2d_binary_with_scales and the Session's
 * cached binary conv (conv2d.cpp:220-369; model.hpp:414-559). */
int tbn_hip_conv2d_f32_binary(const float* x, const tbn_conv2d_desc* desc,
                              const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                              const float* scale, float alpha, const float* bias, int flags,
                              float* y, tbn_stream_t stream);
/* Same with ternary weights in the GEMM 2-bit layout (tbn::conv2d_ternary,
 * conv2d.cpp:195-217, with true ternary values). */
int tbn_hip_conv2d_f32_ternary(const float* x, const tbn_conv2d_desc* desc,
                               const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                               const float* scale, float alpha, const float* bias, int flags,
                               float* y, tbn_stream_t stream);

/* General quantized conv used by the Session: weights binary or ternary, and
 * an optional `residual` tensor (same [n, m, OH, OW] layout as y) added after
 * scale and bias and before ReLU -- a Conv followed by a residual Add and Relu
 * (model.hpp:905-1037,1127-1174) in one pass.  residual excludes
 * TBN_EPI_MAXPOOL2X2. */
int tbn_hip_conv2d_f32_quantized(int weights, const float* x, const tbn_conv2d_desc* desc,
                                 const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                                 const float* scale, float alpha, const float* bias,
                                 const float* residual, int flags, float* y, tbn_stream_t stream);

/* ---- binary / ternary Conv2D on pre-packed conv-layout weights ------------
 * For inputs of 16 or more channels the conv kernels behind the entry points
 * above stage each block's input patch (32 channels at a time, split into the
 * three bf16 parts) in LDS and run every tap from it.  Their weights use the
 * "conv layout": for each step = (c / 32) * kh*kw + r*kw + s, one word per
 * output channel m (ceil8(M) of them) holds the 32 channels c % 32 of that
 * step, bit (or 2-bit code) c % 32 of the word, in the reference's encoding
 * (bit 1 = -1, or the 2-bit code); words are 4 bytes (binary) or 8 bytes
 * (ternary) and ordered [step][m], so that neighbouring channels' words sit
 * next to each other.  Channels >= C, and channels m >= M, are +1 / 0 and
 * meet zero activations.  The entry points above re-order the reference layout
 * into the library's per-device stream workspace on every call, and return
 * TBN_NOT_IMPLEMENTED while their stream captures (nothing is allocated into
 * a graph); a caller that runs a layer many times (the Session) packs once
 * and calls tbn_hip_conv2d_f32_prepacked, and a caller that must capture a
 * reference-layout conv uses tbn_hip_conv2d_f32_quantized_noalloc. */

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tbn_hip_conv2d_f32_quantized with the same arguments and
 * results, except that where that entry point takes a stream-ordered
 * temporary (the weight re-order and the split-K partial sums of convs with
 * >= 16 input channels) this one uses a static device buffer of the library,
 * TBN_NOALLOC_SCRATCH_BYTES per device, held until the process ends.  It
 * calls no allocator.  A conv that needs more scratch than that returns
 * TBN_INVALID_SHAPE before any work.  Every call on one device shares that
 * device's buffer, so calls that overlap on one device (other streams or
 * threads) race; calls ordered on one stream are safe. */
#define TBN_NOALLOC_SCRATCH_BYTES (16u << 20)
int tbn_hip_conv2d_f32_quantized_noalloc(int weights, const float* x, const tbn_conv2d_desc* desc,
                                         const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                                         const float* scale, float alpha, const float* bias,
                                         const float* residual, int flags, float* y, tbn_stream_t stream);

/* Bytes of the conv-layout weights for `desc` (weights: TBN_WEIGHTS_BINARY or
 * TBN_WEIGHTS_TERNARY): ceil8(M) * Kc / 8 (binary) or / 4 (ternary). */
int tbn_hip_conv_weights_bytes(int weights, const tbn_conv2d_desc* desc, int64_t* bytes);
/* Re-orders packed weights from the reference layout (BinaryMatrix bits or the
 * 2-bit GEMM layout of the [M, C*kh*kw] matrix, as tbn_hip_conv2d_f32_binary /
 * _ternary take them) into the conv layout (8-byte aligned output). */
int tbn_hip_pack_conv_weights(int weights, const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                              const tbn_conv2d_desc* desc, uint8_t* conv_weights, tbn_stream_t stream);
/* tbn_hip_conv2d_f32_quantized on conv-layout weights: same arithmetic and
 * epilogue, no weight re-order.  Returns TBN_INVALID_SHAPE for geometries
 * whose patch does not fit (very large kernels or dilations).  Geometries
 * that split K (small maps with many input channels) keep their partial sums
 * in the library's per-device stream workspace, allocated on first use;
 * such geometries return TBN_NOT_IMPLEMENTED while the stream captures. */
int tbn_hip_conv2d_f32_prepacked(int weights, const float* x, const tbn_conv2d_desc* desc,
                                 const uint8_t* conv_weights, const float* scale, float alpha, const float* bias,
                                 const float* residual, int flags, float* y, tbn_stream_t stream);
/* Same arguments as tbn_hip_conv2d_f32_prepacked (no counterpart in the
 * reference): times every conv tile that fits this geometry, a few launches
 * each, all writing y, and keeps the fastest for later calls with the same
 * geometry, epilogue flags and residual use (a process-wide cache).  Without
 * it a call uses a static rule.  Waits for `stream`; refused under stream
 * capture.  Every tile sums in the same order, so it never changes results.
 * The Session calls it once per conv layer when it compiles its plan. */
int tbn_hip_conv2d_tune_prepacked(int weights, const float* x, const tbn_conv2d_desc* desc,
                                  const uint8_t* conv_weights, const float* scale, float alpha, const float* bias,
                                  const float* residual, int flags, float* y, tbn_stream_t stream);
/* No counterpart in the reference, which runs the two Conv2D layers of a
 * ResNet downsampling block one after the other (conv2d.cpp:319-369 each).
 * One launch computes both the conv of tbn_hip_conv2d_f32_prepacked (desc:
 * 3x3, pad 1, stride s in both directions, dilation 1; flags TBN_EPI_RELU /
 * TBN_EPI_BIAS_THEN_SCALE; optional residual) and the 1x1 pad-0 stride-s
 * conv of the same x to the same desc->m channels (proj_weights in the conv
 * layout of that 1x1 desc, its own scale, alpha, bias and flags, no
 * residual; proj_y has y's shape).  The projection is summed in the order
 * the 1x1 conv uses alone, so both ways give the same bits.  mode: 0 runs,
 * 1 tunes as tbn_hip_conv2d_tune_prepacked does (its own cache entry), 2 only
 * checks that this geometry pairs (no pointer is read).  Returns
 * TBN_NOT_IMPLEMENTED when it does not (another kernel size or padding, K
 * split over blocks, no tile takes it): the caller then makes the two calls. */
int tbn_hip_conv2d_f32_prepacked_pair(int weights, const float* x, const tbn_conv2d_desc* desc,
                                      const uint8_t* conv_weights, const float* scale, float alpha, const float* bias,
                                      const float* residual, int flags, float* y, const uint8_t* proj_weights,
                                      const float* proj_scale, float proj_alpha, const float* proj_bias,
                                      int proj_flags, float* proj_y, int mode, tbn_stream_t stream);
/* No counterpart in the reference (a diagnostic for profiling).  Writes into
 * name (len bytes, NUL-terminated, truncated if short) the kernel, as a
 * profiler names it, that tbn_hip_conv2d_f32_prepacked runs for this
 * geometry, flags and residual presence in this process now: the tile the
 * tuner cached, a forced tile, else the static rule.  No GPU work. */
int tbn_hip_conv2d_kernel_name(int weights, const tbn_conv2d_desc* desc, int flags, int has_residual, char* name,
                               size_t len);

/* ---- fp32 layers and epilogue operators (Session support) ------------------ */

/* fp32 Conv2D (tbn::conv2d, conv2d.cpp:78-192), weights fp32 [M, C, kh, kw];
 * flags: TBN_EPI_RELU, TBN_EPI_MAXPOOL2X2, or TBN_EPI_RELU |
 * TBN_EPI_MAXPOOL3X3S2 (y then [N, M, (OH-1)/2+1, (OW-1)/2+1]; other shapes
 * return TBN_NOT_IMPLEMENTED). */
int tbn_hip_conv2d_f32(const float* x, const tbn_conv2d_desc* desc, const float* w,
                       const float* bias, int flags, float* y, tbn_stream_t stream);
/* TBN_SUCCESS when tbn_hip_conv2d_f32 takes this geometry and these flags
 * (TBN_NOT_IMPLEMENTED for a fused 3x3/2 pool off the stem shape).  No
 * counterpart in the reference (it has no fused pool); for a caller such as
 * the Session deciding whether to fuse a MaxPool into the conv before it. */
int tbn_hip_conv2d_f32_supported(const tbn_conv2d_desc* desc, int flags);
/* ---- grouped convolution and BatchNormalization ---------------------------
 * The reference's conv2d_grouped / depthwise_conv2d throw for groups > 1
 * (conv2d.cpp:372-393) and it has no BatchNormalization; these are new.  A
 * grouped conv with more than one input channel per group runs each group
 * through the dense entry points above on channel slices (tbn::conv2d_grouped
 * and the Session do this), gathering and scattering the slices with
 * tbn_hip_copy_channels when the batch is larger than one. */

/* Depthwise Conv2D: one input channel per group (groups = desc->c), desc->m a
 * multiple of desc->c, output channel m reading input channel m / (m/c);
 * weights fp32 [M, 1, kh, kw] (for a quantized layer the exact +-1 or
 * -1/0/+1 values).  Epilogue as tbn_hip_conv2d_f32_quantized: acc*alpha*s[m]
 * + b[m], or (acc + b[m])*alpha*s[m] with TBN_EPI_BIAS_THEN_SCALE; scale and
 * bias may be NULL; then + residual (may be NULL), then TBN_EPI_RELU.
 * Replaces tbn::depthwise_conv2d (conv2d.cpp:386-393). */
int tbn_hip_conv2d_depthwise(const float* x, const tbn_conv2d_desc* desc, const float* w,
                             const float* scale, float alpha, const float* bias, const float* residual,
                             int flags, float* y, tbn_stream_t stream);
/* dst[i, dst_c0 + j, :] = src[i, src_c0 + j, :] for i < n, j < count, over
 * rows of hw floats of src [n, src_c, hw] and dst [n, dst_c, hw]. */
int tbn_hip_copy_channels(const float* src, int64_t n, int64_t src_c, int64_t src_c0, int64_t count,
                          int64_t hw, float* dst, int64_t dst_c, int64_t dst_c0, tbn_stream_t stream);
/* y[i, j, :] = x[i, j, :] * k[j] + t[j] (one fma), then TBN_EPI_RELU, over
 * [n, c, hw]: an inference BatchNormalization with k = scale/sqrt(var + eps)
 * and t = B - mean*k. */
int tbn_hip_channel_affine(const float* x, int64_t n, int64_t c, int64_t hw, const float* k, const float* t,
                           int flags, float* y, tbn_stream_t stream);

/* fp32 GEMM (tbn::gemm, gemm.cpp:349-360): out = alpha*op(A)*op(B) + beta*C,
 * C NULL, [N] (c_is_1d) or [M, N]; flags: TBN_EPI_RELU. */
int tbn_hip_gemm_f32(const float* A, const float* B, const float* Cin, int c_is_1d,
                     int64_t M, int64_t K, int64_t N, float alpha, float beta,
                     int transA, int transB, int flags, float* out, tbn_stream_t stream);
/* MaxPool2D (tbn::maxpool2d, pooling.cpp:10-80).  out_hw (host, may be NULL)
 * receives the output height and width; y may be NULL to query only. */
int tbn_hip_maxpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                      int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                      int64_t dh, int64_t dw, int ceil_mode, float* y, int64_t* out_hw,
                      tbn_stream_t stream);
/* AvgPool2D (tbn::avgpool2d, pooling.cpp:83-148): sum of the window's taps
 * inside the image in window order, divided by their count (taps outside the
 * image also counted with count_include_pad; 0 for an empty count).  Output
 * size as tbn_hip_maxpool2d; out_hw and a NULL y work the same way. */
int tbn_hip_avgpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh,
                      int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh,
                      int64_t dw, int ceil_mode, int count_include_pad, float* y, int64_t* out_hw,
                      tbn_stream_t stream);
/* GlobalMaxPool2D (tbn::global_maxpool2d, pooling.cpp:151-181), y [n, c]:
 * -inf start, running max in memory order (NaN ignored). */
int tbn_hip_global_maxpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, float* y,
                             tbn_stream_t stream);
/* GlobalAvgPool2D (tbn::global_avgpool2d, pooling.cpp:184-216), y [n, c]. */
int tbn_hip_global_avgpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                             float* y, tbn_stream_t stream);
/* Elementwise y = a + b (+ReLU) with b broadcast over an [outer, inner, rest]
 * view: b has `outer_b * inner` elements indexed by (i_outer % outer_b, i_inner).
 * Covers the Session's Add cases (model.hpp:905-1037): same shape
 * (inner = n, rest = 1), [M,N]+[N], [N,C,H,W]+[C] / [C,1,1]. */
int tbn_hip_add(const float* a, const float* b, int64_t outer, int64_t inner, int64_t rest,
                int64_t outer_b, int flags, float* y, tbn_stream_t stream);
/* y = max(x, 0) (model.hpp:1166-1171). */
int tbn_hip_relu(const float* x, int64_t n, float* y, tbn_stream_t stream);

/* Session elementwise ops (model.hpp:1176-1300), r = b ? b[i % nb] : scalar:
 *   TBN_OP_SUB y = a - r;  TBN_OP_GREATER y = a > r;  TBN_OP_LESS y = a < r (1.0 / 0.0). */
enum tbn_elementwise_op { TBN_OP_SUB = 0, TBN_OP_GREATER = 1, TBN_OP_LESS = 2 };
int tbn_hip_elementwise(int op, const float* a, int64_t n, const float* b, int64_t nb, float scalar,
                        float* y, tbn_stream_t stream);
/* The Session's ternary replacement of Relu (model.hpp:1144-1165):
 * y = x > t ? 1 : (x < -t ? -1 : 0). */
int tbn_hip_ternary_activation(const float* x, int64_t n, float threshold, float* y,
                               tbn_stream_t stream);

/* ---- TBN mode: ternary activations x binary weights, integer arithmetic ----
 * The reference's production arithmetic for qlinear_matmul_binary and the
 * Session's cached convolutions: activations ternarized at (lo, hi) (v < lo ->
 * -1, v > hi -> +1, else 0; the reference uses -0.1 / 0.1), multiplied by the
 * +-1 BinaryMatrix weights with exact int32 accumulation.  Results are bit
 * identical to the reference's. */

/* TernaryMatrix::pack_from_float after pad_float_matrix (GeMM/05-final/
 * GeMM.cpp:71-112, quantized_gemm_neon.cpp:118-141): two row-major bit planes
 * pos / neg of rows x cols/8 bytes (bit j&7 of byte j>>3 of a row), A [M, K]
 * zero padded to [rows, cols]; rows % 8 == 0 and cols % 64 == 0 as the
 * reference requires (else TBN_INVALID_ARGUMENT). */
int tbn_hip_ternary_pack_f32(const float* A, int64_t lda, int64_t M, int64_t K, int64_t rows,
                             int64_t cols, float lo, float hi, uint8_t* pos, uint8_t* neg,
                             tbn_stream_t stream);
/* TernaryMatrix::pack (GeMM/05-final/GeMM.cpp:29-69) on the device: int8
 * values of A [M, K] (row stride lda) into the same two bit planes of rows x
 * cols/8 bytes, zero padded; a negative value sets its neg bit, a positive
 * one its pos bit (the reference accepts only -1, 0 and +1: check them first,
 * as tbn::TernaryMatrix::pack does).  rows % 8 == 0, cols % 64 == 0. */
int tbn_hip_ternary_pack_i8(const int8_t* A, int64_t lda, int64_t M, int64_t K, int64_t rows,
                            int64_t cols, uint8_t* pos, uint8_t* neg, tbn_stream_t stream);
/* impl::im2col_ternary_packed (conv2d.cpp:511-601): the im2col matrix
 * [n*OH*OW, c*kh*kw] of x, column (c*kh + r)*kw + s, ternarized into bit
 * planes of m_pad rows x k_pad/8 bytes; taps outside the image and padding
 * are 0.  k_pad % 32 == 0. */
int tbn_hip_im2col_ternary_packed(const float* x, const tbn_conv2d_desc* desc, int64_t m_pad,
                                  int64_t k_pad, float lo, float hi, uint8_t* pos, uint8_t* neg,
                                  tbn_stream_t stream);
/* GemmEngine::compute (GeMM/05-final/GeMM.cpp:303-363), reference naming:
 * C[m, k] (int32, row-major) = sum over the shared dimension n of the
 * ternary rows (pos / neg planes, m x n/8 bytes) times the BinaryMatrix
 * columns `bits` (k columns of n/8 bytes).  n % 64 == 0 (the reference needs
 * n % 128 == 0 and m, k multiples of its micro tiles; no tiling constraint
 * here), n < 2^24.  Uses the stream workspace for the fp4 operand rows:
 * m*n/2 (rounded up to 256) + k*n/2 bytes. */
int tbn_hip_tbn_gemm(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits, int64_t m,
                     int64_t n, int64_t k, int32_t* C, tbn_stream_t stream);
/* The extraction and scaling of qlinear_matmul_binary_blocked_prepacked
 * (quantized_gemm_neon.cpp:314-350) fused into tbn_hip_tbn_gemm: out[i, j] =
 * float(C[i, j]) * scale for the first m rows and `cols` (<= k) columns of C,
 * out row stride ldo. */
int tbn_hip_tbn_gemm_scaled(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits, int64_t m,
                            int64_t n, int64_t k, int64_t cols, float scale, float* out, int64_t ldo,
                            tbn_stream_t stream);
/* qlinear_matmul_binary as the reference computes it (quantized_gemm_neon.cpp:
 * 160-243,380-430): out[M, N] = float(sum_k t(A[m,k]) * w[k,n]) * scale with
 * t the ternarization at (lo, hi) and w the packed BinaryMatrix (K_pad % 64
 * == 0, K_pad < 2^24, N_pad >= N).  Uses the stream workspace for the fp4
 * operand rows: M*K_pad/2 (rounded up to 256) + N_pad*K_pad/2 bytes. */
int tbn_hip_qlinear_matmul_binary_tbn(const float* A, int64_t lda, int64_t M, int64_t K,
                                      const uint8_t* packed, int64_t K_pad, int64_t N,
                                      int64_t N_pad, float scale, float lo, float hi, float* out,
                                      int64_t ldo, tbn_stream_t stream);

/* BinaryMatrix columns (K_pad / 8 bytes each, bit 1 = -1) -> fp4 weight rows
 * w4 [N_pad, K_pad / 2] (two E2M1 codes a byte, low nibble first: +1 = 0x2,
 * -1 = 0xA), the operand layout of tbn_hip_gemm_tbn_prepacked.  K_pad % 64 ==
 * 0, packed 4-byte and w4 16-byte aligned.  The B-side half of
 * qlinear_matmul_binary_blocked_packed's per-Session cache
 * (model.hpp:809-833), done once. */
int tbn_hip_pack_f4_weights(const uint8_t* packed, int64_t K_pad, int64_t N_pad, uint8_t* w4,
                            tbn_stream_t stream);
/* The Session's quantized Gemm as the reference computes it
 * (qlinear_matmul_binary_blocked_packed, quantized_gemm_neon.cpp:249-309, then
 * model.hpp:847-870): out[m, n] = float(sum_k t(A[m, k]) * w[k, n]) * alpha,
 * then, when cin is given and beta != 0, out = fma(beta, cin, out) with cin
 * [N] (cin_1d) or [M, N] (row stride N) -- the reference's `r += beta * c`
 * as AArch64 compilers contract it; then TBN_EPI_RELU (the only flag).  t is
 * the ternarization at (lo, hi) (v < lo -> -1, v > hi -> +1, else 0); w4 from
 * tbn_hip_pack_f4_weights.  t4: caller scratch of M * K_pad / 2 bytes
 * (16-byte aligned) for the fp4 activation rows, so the call allocates
 * nothing. */
int tbn_hip_gemm_tbn_prepacked(const float* A, int64_t lda, int64_t M, int64_t K, const uint8_t* w4,
                               int64_t K_pad, int64_t N, int64_t N_pad, float alpha, const float* cin,
                               int cin_1d, float beta, float lo, float hi, int flags, uint8_t* t4,
                               float* out, int64_t ldo, tbn_stream_t stream);

/* ---- TBN-mode Conv2D (implicit GEMM, ternarized while staging) ------------ */

/* Bytes of the TBN conv weights for desc: ceil(M / 32) fragments x kh*kw*
 * ceil(C / 64) k-steps x 1024. */
int tbn_hip_tbn_conv_weights_bytes(const tbn_conv2d_desc* desc, int64_t* bytes);
/* Re-orders the reference-layout BinaryMatrix of the [M, C*kh*kw] weights
 * (layout NK, as tbn_hip_conv2d_f32_binary takes them) into the TBN conv
 * layout: for each 32-channel fragment and k-step (chunk of 64 input
 * channels x tap), 64 lanes x 16 bytes of fp4 codes, lane l holding channel
 * l % 32 and input channels 32 (l / 32) .. +31 of the chunk.  w4 16-byte
 * aligned.  The weight-side cache of the Session's conv (model.hpp:456-480). */
int tbn_hip_pack_tbn_conv_weights(const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                                  const tbn_conv2d_desc* desc, uint8_t* w4, tbn_stream_t stream);
/* Bytes of the scratch tbn_hip_conv2d_tbn_prepacked needs for desc under the
 * current tuning: 0 where the fused kernel runs (it stages the ternarized
 * input in LDS), else the input ternarized into fp4 pixel records,
 * n * ceil(C / 64) * h * w * 32. */
int tbn_hip_tbn_conv_scratch_bytes(const tbn_conv2d_desc* desc, int64_t* bytes);
/* The reference Session's quantized convolution (model.hpp:482-557 with
 * im2col_ternary_packed, conv2d.cpp:511-601; conv2d_binary, conv2d.cpp:
 * 220-316): every input tap ternarized at (lo, hi), taps outside the image 0,
 * times the +-1 weights in exact integer arithmetic (C = the reference's
 * int32), then y = float(C) * alpha*s[m] + b[m] (two roundings) or with
 * TBN_EPI_BIAS_THEN_SCALE (float(C) + b[m]) * alpha*s[m]; scale and bias may
 * be NULL.  Then `residual` (same layout as y) is added, TBN_EPI_RELU, and
 * TBN_EPI_MAXPOOL2X2 (floor mode; needs TBN_EPI_RELU and no residual).
 * C*kh*kw <= 2^24.  `scratch` (16-byte aligned, tbn_hip_tbn_conv_scratch_bytes)
 * receives the ternarized input; with scratch the call allocates nothing and
 * may be captured; NULL takes the library's stream workspace, refused
 * (TBN_NOT_IMPLEMENTED) while the stream captures. */
int tbn_hip_conv2d_tbn_prepacked(const float* x, const tbn_conv2d_desc* desc, const uint8_t* w4,
                                 const float* scale, float alpha, const float* bias, const float* residual,
                                 int flags, float lo, float hi, uint8_t* scratch, float* y,
                                 tbn_stream_t stream);
/* No counterpart in the reference, which runs the two Conv2D layers of a
 * ResNet downsampling block one after the other (model.hpp:482-557 each).
 * One launch computes both tbn_hip_conv2d_tbn_prepacked for desc (3x3, pad
 * 1, stride s in both directions, dilation 1; flags TBN_EPI_RELU /
 * TBN_EPI_BIAS_THEN_SCALE; optional residual) and the 1x1 pad-0 stride-s TBN
 * conv of the same x, ternarized at the same (lo, hi), to the same desc->m
 * channels (proj_w4 packed for that 1x1 desc, its own scale, alpha, bias and
 * flags, no residual; proj_y has y's shape).  Every product and sum is an
 * exact integer, so both outputs have the bits of the two separate calls.
 * mode: 0 runs, 2 only checks that this geometry pairs (no pointer read).
 * Returns TBN_NOT_IMPLEMENTED when it does not (another kernel size or
 * padding, or a geometry on the two-pass kernels): the caller then makes
 * the two calls.  Allocates nothing. */
int tbn_hip_conv2d_tbn_prepacked_pair(const float* x, const tbn_conv2d_desc* desc, const uint8_t* w4,
                                      const float* scale, float alpha, const float* bias, const float* residual,
                                      int flags, float lo, float hi, float* y, const uint8_t* proj_w4,
                                      const float* proj_scale, float proj_alpha, const float* proj_bias,
                                      int proj_flags, float* proj_y, int mode, tbn_stream_t stream);
/* No counterpart in the reference (a diagnostic for profiling): the conv
 * kernel tbn_hip_conv2d_tbn_prepacked runs for desc and flags, as a profiler
 * names it.  No GPU work. */
int tbn_hip_conv2d_tbn_kernel_name(const tbn_conv2d_desc* desc, int flags, char* name, size_t len);

#ifdef __cplusplus
}
#endif
#endif /* TBN_HIP_H */
