/*
 * tbn_oracle.c -- CPU oracle for the tbn quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY: a plain-C restatement of the reference
 * algorithms, used by tests/ as the parity checker and by bench.py as the
 * timed CPU baseline.  The HIP library never links or calls it.
 *
 * Each function names the reference file:line whose algorithm it restates
 * (paths relative to the Babushkin05/fast-arm-tbcnn tree).  How each one is
 * pinned (golden vectors, closed forms, brute force) is listed in the test
 * files under tests/ that exercise it.
 */
#include "tbn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================== */
/* Quantization and sign rules                                              */
/* ======================================================================== */

/* quantize_to_binary, FLOAT32 branch: byte 1 iff w > threshold, so 0, -0.0
 * and NaN all give 0 (= -1).  tbn-runtime/src/operators/quantized_gemm_neon.cpp:550-554 */
void tbo_quantize_to_binary_f32(const float* w, int64_t n, float thr, uint8_t* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = (w[i] > thr) ? 1u : 0u;
}

/* quantize_to_binary, INT8 branch: byte 1 iff w > 0.
 * tbn-runtime/src/operators/quantized_gemm_neon.cpp:555-559 */
void tbo_quantize_to_binary_i8(const int8_t* w, int64_t n, uint8_t* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = (w[i] > 0) ? 1u : 0u;
}

/* quantize_to_ternary: w < lo -> -1, w > hi -> +1, otherwise 0 (NaN -> 0).
 * tbn-runtime/src/operators/quantized_gemm_neon.cpp:570-597 */
void tbo_quantize_to_ternary_f32(const float* w, int64_t n, float lo, float hi, int8_t* out)
{
    for (int64_t i = 0; i < n; ++i) {
        const float v = w[i];
        out[i] = (v < lo) ? (int8_t)-1 : ((v > hi) ? (int8_t)1 : (int8_t)0);
    }
}

/* Session sign extraction: BINARY byte 1 iff w >= 0, so 0 and -0.0 give +1
 * and NaN gives -1.  tbn-runtime/include/tbn/runtime/model.hpp:430-435,802-804 */
void tbo_sign_ge0_f32(const float* w, int64_t n, uint8_t* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = (w[i] >= 0.0f) ? 1u : 0u;
}

/* Per-output-channel scale = mean |w|, summed sequentially in fp32 and
 * divided by the element count.  tbn-runtime/include/tbn/runtime/model.hpp:388-394 */
void tbo_channel_mean_abs(const float* w, int64_t channels, int64_t per_channel, float* scale)
{
    for (int64_t c = 0; c < channels; ++c) {
        float acc = 0.0f;
        const float* row = w + c * per_channel;
        for (int64_t i = 0; i < per_channel; ++i) acc += fabsf(row[i]);
        scale[c] = acc / (float)per_channel;
    }
}

/* "Already binary" heuristic: every channel needs at least 90% of its
 * elements within 1% of +-scale (or |w| < 0.01).
 * tbn-runtime/include/tbn/runtime/model.hpp:396-410 */
int tbo_already_binary(const float* w, int64_t channels, int64_t per_channel, const float* scale)
{
    for (int64_t c = 0; c < channels; ++c) {
        const float s = scale[c];
        int64_t near = 0;
        for (int64_t i = 0; i < per_channel; ++i) {
            const float v = w[c * per_channel + i];
            const float target = (v >= 0.0f) ? s : -s;
            if (fabsf(v - target) < 0.01f * s || fabsf(v) < 0.01f) ++near;
        }
        if ((float)near < (float)per_channel * 0.9f) return 0;
    }
    return 1;
}

/* ======================================================================== */
/* Packing                                                                  */
/* ======================================================================== */

/* BinaryMatrix::pack: int8 +-1 [rows, cols] row-major -> column-major bit
 * columns of rows/8 bytes; bit (r&7) of byte r>>3 is set iff the value is -1.
 * rows % 64 and cols % 8 are required; other values are rejected.
 * GeMM/05-final/GeMM.cpp:114-151 */
int tbo_binary_matrix_pack(const int8_t* data, uint32_t rows, uint32_t cols, uint8_t* bits)
{
    if (rows % 64u != 0u || cols % 8u != 0u) return TBO_INVALID_ARGUMENT;
    const uint32_t col_bytes = rows / 8u;
    memset(bits, 0, (size_t)cols * col_bytes);
    for (uint32_t j = 0; j < cols; ++j) {
        uint8_t* col = bits + (size_t)j * col_bytes;
        for (uint32_t r = 0; r < rows; ++r) {
            const int8_t v = data[(size_t)r * cols + j];
            if (v == -1) col[r >> 3] |= (uint8_t)(1u << (r & 7u));
            else if (v != 1) return TBO_INVALID_ARGUMENT;
        }
    }
    return TBO_OK;
}

/* Runtime weight packing for B[K,N] (qlinear_matmul_binary's B, Gemm's W):
 * BINARY bytes -> int8 (+1 iff byte == 1), padded with +1 to [K_pad, N_pad],
 * then BinaryMatrix::pack.  The fused loop below writes the same bits.
 * tbn-runtime/src/operators/quantized_gemm_neon.cpp:197-214,
 * tbn-runtime/include/tbn/runtime/model.hpp:814-830 */
int tbo_pack_binary_kn(const uint8_t* bin, int64_t K, int64_t N, int64_t K_pad, int64_t N_pad,
                       uint8_t* packed)
{
    if (K_pad < K || N_pad < N || K_pad % 64 != 0 || N_pad % 8 != 0) return TBO_INVALID_ARGUMENT;
    const int64_t col_bytes = K_pad / 8;
    memset(packed, 0, (size_t)(N_pad * col_bytes));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            if (bin[k * N + n] != 1u)
                packed[n * col_bytes + (k >> 3)] |= (uint8_t)(1u << (k & 7));
    return TBO_OK;
}

/* Conv weights [M_out, C*kh*kw] (= [N, K]) are transposed to [K, M_out] and
 * packed the same way (cache key W+"_t").
 * tbn-runtime/include/tbn/runtime/model.hpp:456-480 */
int tbo_pack_binary_nk(const uint8_t* bin, int64_t N, int64_t K, int64_t K_pad, int64_t N_pad,
                       uint8_t* packed)
{
    if (K_pad < K || N_pad < N || K_pad % 64 != 0 || N_pad % 8 != 0) return TBO_INVALID_ARGUMENT;
    const int64_t col_bytes = K_pad / 8;
    memset(packed, 0, (size_t)(N_pad * col_bytes));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            if (bin[n * K + k] != 1u)
                packed[n * col_bytes + (k >> 3)] |= (uint8_t)(1u << (k & 7));
    return TBO_OK;
}

/* 2-bit ternary codes, TernaryPackedWeights::set_weight applied to every
 * element of a fresh (zeroed) buffer: -1 -> 00, 0 -> 01, +1 -> 10, and any
 * other value is encoded as 01 (zero).
 * tbn-runtime/include/tbn/memory/packed_weights.hpp:24-27,52-71 */
static uint8_t ternary_code(int8_t t)
{
    return (t == -1) ? 0u : ((t == 1) ? 2u : 1u);
}

void tbo_ternary_pack2(const int8_t* t, int64_t n, uint8_t* packed)
{
    memset(packed, 0, (size_t)((n + 3) / 4));
    for (int64_t i = 0; i < n; ++i) {
        const int sh = (int)(i & 3) * 2;
        packed[i >> 2] = (uint8_t)((packed[i >> 2] & ~(3u << sh)) | ((unsigned)ternary_code(t[i]) << sh));
    }
}

/* TernaryPackedWeights::get_weight: 00 -> -1, 01 -> 0, 10 -> +1, 11 -> 0.
 * tbn-runtime/include/tbn/memory/packed_weights.hpp:35-49 */
int8_t tbo_ternary_get2(const uint8_t* packed, int64_t i)
{
    const unsigned code = (packed[i >> 2] >> ((i & 3) * 2)) & 3u;
    return (code == 0u) ? (int8_t)-1 : ((code == 2u) ? (int8_t)1 : (int8_t)0);
}

/* GEMM layout for ternary weights: the transposed, zero-padded matrix
 * W^T[N_pad, K_pad] flattened and encoded with the 2-bit codes above, so
 * column n occupies K_pad/4 bytes.  Padding entries are zero (code 01).
 * (The reference defines the code table only; this K-major order is the
 * GPU path's documented choice.) */
int tbo_pack_ternary_kn(const int8_t* t, int64_t K, int64_t N, int64_t K_pad, int64_t N_pad,
                        uint8_t* packed)
{
    if (K_pad < K || N_pad < N || K_pad % 4 != 0) return TBO_INVALID_ARGUMENT;
    const int64_t total = N_pad * K_pad;
    memset(packed, 0x55, (size_t)(total / 4));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            const int64_t i = n * K_pad + k;
            const int sh = (int)(i & 3) * 2;
            packed[i >> 2] = (uint8_t)((packed[i >> 2] & ~(3u << sh)) |
                                       ((unsigned)ternary_code(t[k * N + n]) << sh));
        }
    return TBO_OK;
}

int tbo_pack_ternary_nk(const int8_t* t, int64_t N, int64_t K, int64_t K_pad, int64_t N_pad,
                        uint8_t* packed)
{
    if (K_pad < K || N_pad < N || K_pad % 4 != 0) return TBO_INVALID_ARGUMENT;
    const int64_t total = N_pad * K_pad;
    memset(packed, 0x55, (size_t)(total / 4));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            const int64_t i = n * K_pad + k;
            const int sh = (int)(i & 3) * 2;
            packed[i >> 2] = (uint8_t)((packed[i >> 2] & ~(3u << sh)) |
                                       ((unsigned)ternary_code(t[n * K + k]) << sh));
        }
    return TBO_OK;
}

/* ======================================================================== */
/* Mode F32: fp32 activations x (scale * sign) weights                      */
/* ======================================================================== */

static float binary_weight(const uint8_t* packed, int64_t col_bytes, int64_t k, int64_t n)
{
    return ((packed[n * col_bytes + (k >> 3)] >> (k & 7)) & 1u) ? -1.0f : 1.0f;
}

static float ternary_weight(const uint8_t* packed, int64_t K_pad, int64_t k, int64_t n)
{
    return (float)tbo_ternary_get2(packed, n * K_pad + k);
}

static float column_multiplier(const float* scale, float alpha, int64_t n)
{
    return scale ? alpha * scale[n] : alpha;
}

/* True float x binary: sum_k a[i,k] * (+-1) accumulated sequentially over k
 * in fp32, then multiplied by the scale.  This is the only reference routine
 * that keeps the activations in fp32.
 * tbn-runtime/src/operators/quantized_gemm_neon.cpp:63-90
 * Extensions (documented on the C-ABI): the scale may be one value per
 * output column, then a per-column bias is added and ReLU applied. */
void tbo_gemm_f32_binary(const float* A, int64_t lda, int64_t M, int64_t K,
                         const uint8_t* packed, int64_t K_pad, int64_t N,
                         const float* scale, float alpha, const float* bias, int relu,
                         float* C, int64_t ldc)
{
    const int64_t col_bytes = K_pad / 8;
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (int64_t k = 0; k < K; ++k) sum += A[i * lda + k] * binary_weight(packed, col_bytes, k, j);
            float v = sum * column_multiplier(scale, alpha, j);
            if (bias) v += bias[j];
            if (relu) v = (v > 0.0f) ? v : 0.0f;
            C[i * ldc + j] = v;
        }
}

/* The same contraction with an fp64 accumulator: the "exact" reference the
 * tolerance tests measure against. */
void tbo_gemm_f64_binary(const float* A, int64_t lda, int64_t M, int64_t K,
                         const uint8_t* packed, int64_t K_pad, int64_t N,
                         const float* scale, float alpha, const float* bias, int relu,
                         double* C, int64_t ldc)
{
    const int64_t col_bytes = K_pad / 8;
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double sum = 0.0;
            for (int64_t k = 0; k < K; ++k)
                sum += (double)A[i * lda + k] * (double)binary_weight(packed, col_bytes, k, j);
            double v = sum * (double)column_multiplier(scale, alpha, j);
            if (bias) v += (double)bias[j];
            if (relu) v = (v > 0.0) ? v : 0.0;
            C[i * ldc + j] = v;
        }
}

/* True float x ternary: the semantics the reference's own operator test
 * expects (tbn-runtime/tests/test_quantized_operators.cpp:151-155), with the
 * weights decoded from the 2-bit codes above. */
void tbo_gemm_f32_ternary(const float* A, int64_t lda, int64_t M, int64_t K,
                          const uint8_t* packed, int64_t K_pad, int64_t N,
                          const float* scale, float alpha, const float* bias, int relu,
                          float* C, int64_t ldc)
{
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (int64_t k = 0; k < K; ++k) sum += A[i * lda + k] * ternary_weight(packed, K_pad, k, j);
            float v = sum * column_multiplier(scale, alpha, j);
            if (bias) v += bias[j];
            if (relu) v = (v > 0.0f) ? v : 0.0f;
            C[i * ldc + j] = v;
        }
}

void tbo_gemm_f64_ternary(const float* A, int64_t lda, int64_t M, int64_t K,
                          const uint8_t* packed, int64_t K_pad, int64_t N,
                          const float* scale, float alpha, const float* bias, int relu,
                          double* C, int64_t ldc)
{
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double sum = 0.0;
            for (int64_t k = 0; k < K; ++k)
                sum += (double)A[i * lda + k] * (double)ternary_weight(packed, K_pad, k, j);
            double v = sum * (double)column_multiplier(scale, alpha, j);
            if (bias) v += (double)bias[j];
            if (relu) v = (v > 0.0) ? v : 0.0;
            C[i * ldc + j] = v;
        }
}

/* qlinear_matmul_binary_naive on an unpacked BINARY [K,N] tensor, scalar
 * scale.  tbn-runtime/src/operators/quantized_gemm_neon.cpp:63-90 */
void tbo_qlinear_matmul_binary_naive(const float* A, int64_t M, int64_t K,
                                     const uint8_t* bin, int64_t N, float scale, float* out)
{
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float sgn = (bin[k * N + j] == 1u) ? 1.0f : -1.0f;
                sum += A[i * K + k] * sgn;
            }
            out[i * N + j] = sum * scale;
        }
}

/* ======================================================================== */
/* fp32 operators                                                           */
/* ======================================================================== */

static int64_t conv_out_dim(int64_t in, int64_t pad, int64_t dil, int64_t k, int64_t stride)
{
    return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

/* Conv2D, naive NCHW: accumulators start at the bias (or 0) and add
 * x * w over c, kh, kw in that order, skipping taps outside the image.
 * tbn-runtime/src/operators/conv2d.cpp:78-192 */
int tbo_conv2d_f32(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                   const float* w, int64_t M, int64_t kh, int64_t kw,
                   const float* bias,
                   int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                   float* y)
{
    const int64_t OH = conv_out_dim(H, ph, dh, kh, sh);
    const int64_t OW = conv_out_dim(W, pw, dw, kw, sw);
    if (OH <= 0 || OW <= 0) return TBO_INVALID_SHAPE;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m)
            for (int64_t oh = 0; oh < OH; ++oh)
                for (int64_t ow = 0; ow < OW; ++ow) {
                    float acc = bias ? bias[m] : 0.0f;
                    for (int64_t c = 0; c < C; ++c)
                        for (int64_t r = 0; r < kh; ++r)
                            for (int64_t s = 0; s < kw; ++s) {
                                const int64_t ih = oh * sh - ph + r * dh;
                                const int64_t iw = ow * sw - pw + s * dw;
                                if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                                acc += x[((n * C + c) * H + ih) * W + iw] *
                                       w[((m * C + c) * kh + r) * kw + s];
                            }
                    y[((n * M + m) * OH + oh) * OW + ow] = acc;
                }
    return TBO_OK;
}

int tbo_conv2d_f64(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                   const float* w, int64_t M, int64_t kh, int64_t kw,
                   const float* bias,
                   int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                   double* y)
{
    const int64_t OH = conv_out_dim(H, ph, dh, kh, sh);
    const int64_t OW = conv_out_dim(W, pw, dw, kw, sw);
    if (OH <= 0 || OW <= 0) return TBO_INVALID_SHAPE;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m)
            for (int64_t oh = 0; oh < OH; ++oh)
                for (int64_t ow = 0; ow < OW; ++ow) {
                    double acc = bias ? (double)bias[m] : 0.0;
                    for (int64_t c = 0; c < C; ++c)
                        for (int64_t r = 0; r < kh; ++r)
                            for (int64_t s = 0; s < kw; ++s) {
                                const int64_t ih = oh * sh - ph + r * dh;
                                const int64_t iw = ow * sw - pw + s * dw;
                                if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                                acc += (double)x[((n * C + c) * H + ih) * W + iw] *
                                       (double)w[((m * C + c) * kh + r) * kw + s];
                            }
                    y[((n * M + m) * OH + oh) * OW + ow] = acc;
                }
    return TBO_OK;
}

/* MaxPool2D: floor or ceil output size, -inf start, taps outside the image
 * skipped, running max kept with max(acc, v) (so NaN inputs are ignored).
 * tbn-runtime/src/operators/pooling.cpp:10-80 */
int tbo_maxpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                  int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                  int64_t dh, int64_t dw, int ceil_mode, float* y, int64_t* out_hw)
{
    int64_t OH, OW;
    if (ceil_mode) {
        OH = (H + 2 * ph - kh + sh - 1) / sh + 1;
        OW = (W + 2 * pw - kw + sw - 1) / sw + 1;
    } else {
        OH = (H + 2 * ph - kh) / sh + 1;
        OW = (W + 2 * pw - kw) / sw + 1;
    }
    if (out_hw) { out_hw[0] = OH; out_hw[1] = OW; }
    if (!y) return TBO_OK;
    for (int64_t nc = 0; nc < N * C; ++nc)
        for (int64_t oh = 0; oh < OH; ++oh)
            for (int64_t ow = 0; ow < OW; ++ow) {
                float mx = -INFINITY;
                for (int64_t r = 0; r < kh; ++r)
                    for (int64_t s = 0; s < kw; ++s) {
                        const int64_t ih = oh * sh - ph + r * dh;
                        const int64_t iw = ow * sw - pw + s * dw;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W) {
                            const float v = x[(nc * H + ih) * W + iw];
                            if (mx < v) mx = v;
                        }
                    }
                y[(nc * OH + oh) * OW + ow] = mx;
            }
    return TBO_OK;
}

/* AvgPool2D: output size as MaxPool2D (no dilation term); per window the
 * taps inside the image summed in window order and counted, taps outside
 * counted too with count_include_pad; sum / count, or 0 for count 0.
 * tbn-runtime/src/operators/pooling.cpp:83-148 */
int tbo_avgpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                  int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                  int64_t dh, int64_t dw, int ceil_mode, int count_include_pad, float* y,
                  int64_t* out_hw)
{
    int64_t OH, OW;
    if (ceil_mode) {
        OH = (H + 2 * ph - kh + sh - 1) / sh + 1;
        OW = (W + 2 * pw - kw + sw - 1) / sw + 1;
    } else {
        OH = (H + 2 * ph - kh) / sh + 1;
        OW = (W + 2 * pw - kw) / sw + 1;
    }
    if (out_hw) { out_hw[0] = OH; out_hw[1] = OW; }
    if (!y) return TBO_OK;
    for (int64_t nc = 0; nc < N * C; ++nc)
        for (int64_t oh = 0; oh < OH; ++oh)
            for (int64_t ow = 0; ow < OW; ++ow) {
                float sum = 0.0f;
                int count = 0;
                for (int64_t r = 0; r < kh; ++r)
                    for (int64_t s = 0; s < kw; ++s) {
                        const int64_t ih = oh * sh - ph + r * dh;
                        const int64_t iw = ow * sw - pw + s * dw;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W) {
                            sum += x[(nc * H + ih) * W + iw];
                            ++count;
                        } else if (count_include_pad) {
                            ++count;
                        }
                    }
                y[(nc * OH + oh) * OW + ow] = count > 0 ? sum / (float)count : 0.0f;
            }
    return TBO_OK;
}

/* GlobalMaxPool2D: -inf start, running max(acc, v) over the plane in memory
 * order (NaN ignored; of equal -0 / +0 the first is kept).
 * tbn-runtime/src/operators/pooling.cpp:151-181 */
void tbo_global_maxpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, float* y)
{
    const int64_t hw = H * W;
    for (int64_t nc = 0; nc < N * C; ++nc) {
        float mx = -INFINITY;
        for (int64_t i = 0; i < hw; ++i)
            if (mx < x[nc * hw + i]) mx = x[nc * hw + i];
        y[nc] = mx;
    }
}

/* GlobalAvgPool2D: sequential fp32 sum over the plane divided by H*W.
 * tbn-runtime/src/operators/pooling.cpp:184-216 */
void tbo_global_avgpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, float* y)
{
    const int64_t hw = H * W;
    for (int64_t nc = 0; nc < N * C; ++nc) {
        float sum = 0.0f;
        for (int64_t i = 0; i < hw; ++i) sum += x[nc * hw + i];
        y[nc] = sum / (float)hw;
    }
}

/* gemm (fp32, non-NEON branch): result starts at beta*C (1-D C broadcast per
 * row) or 0; 64x64x64 blocks; each block's partial dot product is summed
 * sequentially and added as alpha*partial.
 * tbn-runtime/src/operators/gemm.cpp:35-129,349-360 */
void tbo_gemm_f32_blocked(const float* A, const float* B, const float* Cin, int c_is_1d,
                          int64_t M, int64_t K, int64_t N, float alpha, float beta,
                          int transA, int transB, float* out)
{
    const int64_t BS = 64;
    if (Cin && beta != 0.0f) {
        for (int64_t i = 0; i < M; ++i)
            for (int64_t j = 0; j < N; ++j)
                out[i * N + j] = beta * (c_is_1d ? Cin[j] : Cin[i * N + j]);
    } else {
        memset(out, 0, (size_t)(M * N) * sizeof(float));
    }
    for (int64_t i0 = 0; i0 < M; i0 += BS) {
        const int64_t i1 = (i0 + BS < M) ? i0 + BS : M;
        for (int64_t j0 = 0; j0 < N; j0 += BS) {
            const int64_t j1 = (j0 + BS < N) ? j0 + BS : N;
            for (int64_t k0 = 0; k0 < K; k0 += BS) {
                const int64_t k1 = (k0 + BS < K) ? k0 + BS : K;
                for (int64_t i = i0; i < i1; ++i)
                    for (int64_t j = j0; j < j1; ++j) {
                        float part = 0.0f;
                        for (int64_t k = k0; k < k1; ++k) {
                            const float a = transA ? A[k * M + i] : A[i * K + k];
                            const float b = transB ? B[j * K + k] : B[k * N + j];
                            part += a * b;
                        }
                        out[i * N + j] += alpha * part;
                    }
            }
        }
    }
}

/* ======================================================================== */
/* Mode TBN: the reference's production path                                */
/* ======================================================================== */

/* pad_float_matrix (zero padding to [rows, cols]) followed by
 * TernaryMatrix::pack_from_float: two row-major bit planes of cols/8 bytes
 * per row; v < lo sets the negative plane, v > hi the positive plane.
 * tbn-runtime/src/operators/quantized_gemm_neon.cpp:118-141,186-195;
 * GeMM/05-final/GeMM.cpp:71-112 */
int tbo_ternary_matrix_pack_from_float(const float* a, int64_t lda, int64_t M, int64_t K,
                                       uint32_t rows, uint32_t cols, float lo, float hi,
                                       uint8_t* pos, uint8_t* neg)
{
    if (rows % 8u != 0u || cols % 64u != 0u) return TBO_INVALID_ARGUMENT;
    if ((int64_t)rows < M || (int64_t)cols < K) return TBO_INVALID_ARGUMENT;
    const uint32_t row_bytes = cols / 8u;
    memset(pos, 0, (size_t)rows * row_bytes);
    memset(neg, 0, (size_t)rows * row_bytes);
    for (uint32_t i = 0; i < rows; ++i)
        for (uint32_t j = 0; j < cols; ++j) {
            const float v = ((int64_t)i < M && (int64_t)j < K) ? a[(int64_t)i * lda + j] : 0.0f;
            const uint8_t bit = (uint8_t)(1u << (j & 7u));
            if (v < lo) neg[(size_t)i * row_bytes + (j >> 3)] |= bit;
            else if (v > hi) pos[(size_t)i * row_bytes + (j >> 3)] |= bit;
        }
    return TBO_OK;
}

static uint64_t load64(const uint8_t* p)
{
    uint64_t v;
    memcpy(&v, p, sizeof v);
    return v;
}

/* GemmEngine::compute with TilingParams::validate: C[m,k] (int32) is the
 * ternary x binary product over the shared dimension n, computed per 64-bit
 * word as popcount(pos) - popcount(neg) with
 *   pos = (ap | bc) & (am | ~bc),  neg = (ap | ~bc) & (am | bc).
 * The blocked loop order (y, x, d, r, c) and the sub-block copies are kept so
 * the CPU timing reflects the reference's portable (scalar) path.
 * GeMM/05-final/GeMM.hpp:24-37; GeMM/05-final/GeMM.cpp:160-252 (scalar
 * branch 233-247), 254-295, 303-363 */
int tbo_tbn_gemm(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits,
                 uint32_t m, uint32_t n, uint32_t k,
                 uint32_t mblk, uint32_t nblk, uint32_t kblk, uint32_t mmk, uint32_t nmk,
                 int32_t* C)
{
    if (n % 128u != 0u || kblk % 128u != 0u || mmk == 0u || nmk == 0u ||
        m % mmk != 0u || k % nmk != 0u)
        return TBO_INVALID_ARGUMENT;
    memset(C, 0, (size_t)m * k * sizeof(int32_t));
    const uint32_t row_bytes = n / 8u;
    const uint32_t sub_bytes = kblk / 8u;
    uint8_t* ap = (uint8_t*)malloc((size_t)mmk * sub_bytes);
    uint8_t* am = (uint8_t*)malloc((size_t)mmk * sub_bytes);
    uint8_t* bb = (uint8_t*)malloc((size_t)nmk * sub_bytes);
    if (!ap || !am || !bb) { free(ap); free(am); free(bb); return -2; }

    for (uint32_t y = 0; y < m; y += mblk) {
        const uint32_t my = (mblk < m - y) ? mblk : m - y;
        for (uint32_t x = 0; x < k; x += nblk) {
            const uint32_t nx = (nblk < k - x) ? nblk : k - x;
            for (uint32_t d = 0; d < n; d += kblk) {
                const uint32_t kd = (kblk < n - d) ? kblk : n - d;
                const uint32_t kbytes = kd / 8u;
                for (uint32_t r = 0; r < my; r += mmk) {
                    const uint32_t mr = (mmk < my - r) ? mmk : my - r;
                    for (uint32_t i = 0; i < mr; ++i) {
                        memcpy(ap + (size_t)i * kbytes, pos + (size_t)(y + r + i) * row_bytes + d / 8u, kbytes);
                        memcpy(am + (size_t)i * kbytes, neg + (size_t)(y + r + i) * row_bytes + d / 8u, kbytes);
                    }
                    for (uint32_t c = 0; c < nx; c += nmk) {
                        const uint32_t nc = (nmk < nx - c) ? nmk : nx - c;
                        for (uint32_t j = 0; j < nc; ++j)
                            memcpy(bb + (size_t)j * kbytes, bits + (size_t)(x + c + j) * row_bytes + d / 8u, kbytes);
                        int32_t* tile = C + (size_t)(y + r) * k + (x + c);
                        for (uint32_t i = 0; i < mr; ++i)
                            for (uint32_t j = 0; j < nc; ++j) {
                                int pc = 0, nc2 = 0;
                                for (uint32_t w = 0; w < kbytes / 8u; ++w) {
                                    const uint64_t vp = load64(ap + (size_t)i * kbytes + w * 8u);
                                    const uint64_t vm = load64(am + (size_t)i * kbytes + w * 8u);
                                    const uint64_t vb = load64(bb + (size_t)j * kbytes + w * 8u);
                                    pc += __builtin_popcountll((vp | vb) & (vm | ~vb));
                                    nc2 += __builtin_popcountll((vp | ~vb) & (vm | vb));
                                }
                                tile[(size_t)i * k + j] += pc - nc2;
                            }
                    }
                }
            }
        }
    }
    free(ap); free(am); free(bb);
    return TBO_OK;
}

/* qlinear_matmul_binary (BINARY B): PaddedDimensions (M->16, K->128, N->8),
 * activations ternarized with +-0.1, B re-packed per call, popcount GEMM,
 * out = float(int32) * scale on the unpadded region.
 * tbn-runtime/src/operators/quantized_gemm_neon.cpp:38-58,165-243,380-430 */
int tbo_qlinear_matmul_binary_tbn(const float* A, int64_t M, int64_t K,
                                  const uint8_t* bin, int64_t N, float scale,
                                  uint32_t mblk, uint32_t nblk, uint32_t kblk,
                                  uint32_t mmk, uint32_t nmk, float* out)
{
    const uint32_t m_pad = (uint32_t)((M + 15) / 16 * 16);
    const uint32_t k_pad = (uint32_t)((K + 127) / 128 * 128);
    const uint32_t n_pad = (uint32_t)((N + 7) / 8 * 8);
    const size_t abytes = (size_t)m_pad * (k_pad / 8u);
    uint8_t* pos = (uint8_t*)malloc(abytes);
    uint8_t* neg = (uint8_t*)malloc(abytes);
    uint8_t* bits = (uint8_t*)malloc((size_t)n_pad * (k_pad / 8u));
    int32_t* C = (int32_t*)malloc((size_t)m_pad * n_pad * sizeof(int32_t));
    int rc = TBO_OK;
    if (!pos || !neg || !bits || !C) { rc = -2; goto done; }
    rc = tbo_ternary_matrix_pack_from_float(A, K, M, K, m_pad, k_pad, -0.1f, 0.1f, pos, neg);
    if (rc) goto done;
    rc = tbo_pack_binary_kn(bin, K, N, k_pad, n_pad, bits);
    if (rc) goto done;
    rc = tbo_tbn_gemm(pos, neg, bits, m_pad, k_pad, n_pad, mblk, nblk, kblk, mmk, nmk, C);
    if (rc) goto done;
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j)
            out[i * N + j] = (float)C[i * n_pad + j] * scale;
done:
    free(pos); free(neg); free(bits); free(C);
    return rc;
}

/* im2col_ternary_packed: the im2col matrix [N*OH*OW, C*kh*kw] ternarized
 * straight into the two bit planes (rows padded to m_pad, cols to k_pad);
 * taps outside the image stay 0.  The reference's stride-1/pad-0 fast path
 * produces the same bits as this general form.
 * tbn-runtime/src/operators/conv2d.cpp:511-601 */
int tbo_im2col_ternary_packed(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                              int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                              int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                              uint32_t m_pad, uint32_t k_pad, float lo, float hi,
                              uint8_t* pos, uint8_t* neg)
{
    const int64_t OH = conv_out_dim(H, ph, dh, kh, sh);
    const int64_t OW = conv_out_dim(W, pw, dw, kw, sw);
    if (OH <= 0 || OW <= 0) return TBO_INVALID_SHAPE;
    if ((int64_t)m_pad < N * OH * OW || (int64_t)k_pad < C * kh * kw || k_pad % 8u != 0u)
        return TBO_INVALID_ARGUMENT;
    const uint32_t row_bytes = k_pad / 8u;
    memset(pos, 0, (size_t)m_pad * row_bytes);
    memset(neg, 0, (size_t)m_pad * row_bytes);
    for (int64_t n = 0; n < N; ++n)
        for (int64_t oh = 0; oh < OH; ++oh)
            for (int64_t ow = 0; ow < OW; ++ow) {
                const int64_t row = (n * OH + oh) * OW + ow;
                uint8_t* rp = pos + (size_t)row * row_bytes;
                uint8_t* rm = neg + (size_t)row * row_bytes;
                for (int64_t c = 0; c < C; ++c)
                    for (int64_t r = 0; r < kh; ++r)
                        for (int64_t s = 0; s < kw; ++s) {
                            const int64_t ih = oh * sh - ph + r * dh;
                            const int64_t iw = ow * sw - pw + s * dw;
                            if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                            const int64_t col = (c * kh + r) * kw + s;
                            const float v = x[((n * C + c) * H + ih) * W + iw];
                            const uint8_t bit = (uint8_t)(1u << (col & 7));
                            if (v < lo) rm[col >> 3] |= bit;
                            else if (v > hi) rp[col >> 3] |= bit;
                        }
            }
    return TBO_OK;
}
