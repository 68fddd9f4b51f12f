// Operator entry points of the tbn runtime on the MI355X.  Names, argument
// order and defaults follow the reference's operator headers
// (tbn-runtime/include/tbn/operators/{quantized_gemm,conv2d,gemm,pooling}.hpp);
// every operator runs as HIP kernels of libtbn_hip.so.
//
// Residency: an operator's result lives where its first tensor argument
// lives.  Host tensors in -> host tensor out (inputs are uploaded, the result
// is copied back: the reference's calling convention); HIP tensors in -> HIP
// tensor out, queued on the current stream with no host round trip.
//
// Arithmetic ("mode F32"): activations stay fp32 and every quantized product
// a * w (w = +-1 or -1/0/+1) is exact; accumulation is fp32.  Divergences from
// the reference's own operators are listed at each declaration.
#pragma once

#include <cstdint>
#include <vector>

#include "tensor.hpp"
#include "tiling.hpp"

namespace tbn {

// tbn::Conv2DParams (tbn-runtime/include/tbn/operators/conv2d.hpp:12-37).  The
// kernel size is taken from the weight tensor.
struct Conv2DParams {
    int64_t kernel_h = 3, kernel_w = 3;
    int64_t stride_h = 1, stride_w = 1;
    int64_t pad_h = 0, pad_w = 0;
    int64_t dilation_h = 1, dilation_w = 1;
    int64_t groups = 1;
    Conv2DParams() = default;
    Conv2DParams(int64_t kh, int64_t kw, int64_t sh = 1, int64_t sw = 1, int64_t ph = 0, int64_t pw = 0,
                 int64_t dh = 1, int64_t dw = 1, int64_t g = 1)
        : kernel_h(kh), kernel_w(kw), stride_h(sh), stride_w(sw), pad_h(ph), pad_w(pw),
          dilation_h(dh), dilation_w(dw), groups(g) {}
};

// tbn::Pool2DParams (tbn-runtime/include/tbn/operators/pooling.hpp:10-38).
struct Pool2DParams {
    int64_t kernel_h = 2, kernel_w = 2;
    int64_t stride_h = 2, stride_w = 2;
    int64_t pad_h = 0, pad_w = 0;
    int64_t dilation_h = 1, dilation_w = 1;
    bool ceil_mode = false;
    bool count_include_pad = false;
    Pool2DParams() = default;
    Pool2DParams(int64_t kh, int64_t kw, int64_t sh = 2, int64_t sw = 2, int64_t ph = 0, int64_t pw = 0)
        : kernel_h(kh), kernel_w(kw), stride_h(sh), stride_w(sw), pad_h(ph), pad_w(pw) {}
};

// ---- quantization ------------------------------------------------------------

// FLOAT32: 1 iff w > threshold (0, -0.0 and NaN give 0); INT8: 1 iff w > 0.
// (quantized_gemm_neon.cpp:544-565)
Tensor quantize_to_binary(const Tensor& weights, float threshold = 0.0f);
// FLOAT32: -1 if w < lo, +1 if w > hi, else 0.  (quantized_gemm_neon.cpp:570-597)
Tensor quantize_to_ternary(const Tensor& weights, float threshold_low = -0.1f,
                           float threshold_high = 0.1f);
// True iff every value is exactly -1, 0 or +1 (host data).
bool is_binary_float_weights(const float* data, size_t count);

// ---- pre-packed weights --------------------------------------------------------

// Device-resident packed weights: the GPU counterpart of the reference's
// BinaryMatrix (GeMM/05-final/GeMM.cpp:114-151, column n = K_pad/8 bytes,
// bit 1 = -1, padding +1) and of the 2-bit ternary code
// (tbn-runtime/include/tbn/memory/packed_weights.hpp:35-71) laid out as W^T.
struct PackedWeights {
    enum class Kind { Binary, Ternary };
    Kind kind = Kind::Binary;
    int64_t K = 0, N = 0;          // logical weight matrix W[K, N]
    int64_t K_pad = 0, N_pad = 0;  // K_pad = ceil128(K), N_pad = ceil8(N)
    Tensor bits;                   // UINT8 [N_pad * K_pad / 8] (binary) or [N_pad * K_pad / 4]
};

// Packs W[K, N] (layout "KN": a GEMM's B) or W[N, K] (layout "NK": conv
// weights [M, C, kh, kw] seen as [M, C*kh*kw]).
// BINARY bytes: byte 1 = +1.  FLOAT32: sign by `ge_zero` ? w >= 0 : w > 0.
PackedWeights pack_binary_weights(const Tensor& w, bool nk_layout, bool ge_zero = false);
// TERNARY (int8 -1/0/+1) weights.
PackedWeights pack_ternary_weights(const Tensor& w, bool nk_layout);

// ---- float x binary / float x ternary GEMM ------------------------------------

// out[M, N] = (A[M, K] . W) * b_scale with W = +-1 from B.
// B BINARY [K, N]: byte 1 = +1, else -1.  B FLOAT32 with every value in
// {-1, 0, +1}: w >= 0 -> +1 (qlinear_matmul_binary_float,
// quantized_gemm_neon.cpp:435-499).  Other FLOAT32 B is rejected
// (InvalidArgumentError); the reference reads such a B's float bytes as
// BINARY bytes.  Replaces quantized_gemm_neon.cpp:380-430; A stays fp32 (the
// reference ternarizes A at +-0.1 first, quantized_gemm_neon.cpp:160-243).
Tensor qlinear_matmul_binary(const Tensor& a, const Tensor& b_binary, float b_scale,
                             const TilingParams& params = TilingParams::default_128x128());
// out = (A . T) * b_scale with T in {-1, 0, +1} from TERNARY B [K, N]: the true
// ternary product (the reference maps 0 to +1, quantized_gemm_neon.cpp:506-538).
Tensor qlinear_matmul_ternary(const Tensor& a, const Tensor& b_ternary, float b_scale,
                              const TilingParams& params = TilingParams::default_128x128());
// B FLOAT32 with values in {-1, 0, +1}; w >= 0 -> +1.
Tensor qlinear_matmul_binary_float(const Tensor& a, const Tensor& b_binary_float, float b_scale,
                                   const TilingParams& params = TilingParams::default_128x128());
// TBN mode, the reference's own arithmetic for qlinear_matmul_binary
// (quantized_gemm_neon.cpp:160-243,380-430): A ternarized at (lo, hi) (v < lo
// -> -1, v > hi -> +1, else 0), exact integer product with the +-1 weights,
// out = float(C) * b_scale.  Bit-identical to the reference's operator;
// TilingParams is ignored (no shape is rejected for tiling reasons).
Tensor qlinear_matmul_binary_tbn(const Tensor& a, const Tensor& b_binary, float b_scale,
                                 const TilingParams& params = TilingParams::default_128x128(),
                                 float lo = -0.1f, float hi = 0.1f);
// TBN mode on pre-packed binary weights.
Tensor qlinear_matmul_packed_tbn(const Tensor& a, const PackedWeights& w, float scale, float lo = -0.1f,
                                 float hi = 0.1f);
// GEMM on pre-packed weights (qlinear_matmul_binary_blocked_packed,
// quantized_gemm_neon.cpp:249-309): out = act(acc * scale * s[n] + bias[n]),
// channel_scales and bias FLOAT32 [N] or null.
Tensor qlinear_matmul_packed(const Tensor& a, const PackedWeights& w, float scale,
                             const Tensor* channel_scales = nullptr, const Tensor* bias = nullptr,
                             bool relu = false);

// ---- convolution -----------------------------------------------------------------

// fp32 Conv2D (conv2d.cpp:78-192): y = conv(x, w) + b.  params.groups > 1 is
// conv2d_grouped.
Tensor conv2d(const Tensor& input, const Tensor& weights, const Tensor* bias = nullptr,
              const Conv2DParams& params = Conv2DParams());
// Binary Conv2D (conv2d.cpp:220-316): y = conv(x, +-1) + b, weights BINARY
// [M, C, kh, kw] (byte 1 = +1).  Implicit GEMM, no im2col buffer; any batch.
Tensor conv2d_binary(const Tensor& input, const Tensor& binary_weights, const Tensor* bias = nullptr,
                     const Conv2DParams& params = Conv2DParams());
// Ternary Conv2D with true -1/0/+1 weights (TERNARY [M, C, kh, kw]); the
// reference collapses 0 to +1 (conv2d.cpp:195-217).
Tensor conv2d_ternary(const Tensor& input, const Tensor& ternary_weights, const Tensor* bias = nullptr,
                      const Conv2DParams& params = Conv2DParams());
// y = s[m] * conv(x, +-1) + b[m] (conv2d.cpp:319-369).
Tensor conv2d_binary_with_scales(const Tensor& input, const Tensor& binary_weights, const Tensor* bias,
                                 const Conv2DParams& params, const std::vector<float>& channel_scales);

// Grouped fp32 Conv2D, weights [M, C/groups, kh, kw] (conv2d.cpp:372-384, which
// throws for groups > 1): groups == C runs the depthwise kernel, otherwise one
// dense conv per group on channel slices.
Tensor conv2d_grouped(const Tensor& input, const Tensor& weights, const Tensor* bias = nullptr,
                      int64_t groups = 1, const Conv2DParams& params = Conv2DParams());
// groups = input channels (conv2d.cpp:386-393).
Tensor depthwise_conv2d(const Tensor& input, const Tensor& weights, const Tensor* bias = nullptr,
                        const Conv2DParams& params = Conv2DParams());
// conv2d with dilation on both axes (conv2d.cpp:396-403).
Tensor dilated_conv2d(const Tensor& input, const Tensor& weights, const Tensor* bias = nullptr,
                      int64_t dilation = 1, const Conv2DParams& params = Conv2DParams());
// Inference BatchNormalization over dim 1 (not in the reference):
// y = (x - mean) / sqrt(var + eps) * scale + B, computed as x * k + t.
Tensor batch_norm(const Tensor& input, const Tensor& scale, const Tensor& B, const Tensor& mean,
                  const Tensor& var, float epsilon = 1e-5f);

// ---- fp32 GEMM, pooling, elementwise ---------------------------------------------

// out = alpha * op(A) . op(B) + beta * C, C null, [N] or [M, N] (gemm.cpp:349-360).
Tensor gemm(const Tensor& A, const Tensor& B, const Tensor* C = nullptr, float alpha = 1.0f,
            float beta = 0.0f, bool transA = false, bool transB = false);
// pooling.cpp:10-80 (floor or ceil output size, padding skipped).
Tensor maxpool2d(const Tensor& input, const Pool2DParams& params = Pool2DParams());
// pooling.cpp:83-148 (taps outside the image skipped, or counted as zeros
// with count_include_pad).
Tensor avgpool2d(const Tensor& input, const Pool2DParams& params = Pool2DParams());
// [N, C, H, W] -> [N, C, 1, 1] (pooling.cpp:151-181).
Tensor global_maxpool2d(const Tensor& input);
// [N, C, H, W] -> [N, C, 1, 1] (pooling.cpp:184-216).
Tensor global_avgpool2d(const Tensor& input);
// max(x, 0) (model.hpp:1166-1171).
Tensor relu(const Tensor& input);
// a + b with the Session's broadcasts (model.hpp:905-1037): same shape,
// [M, N] + [N], [N] + [M, N], [N, C, H, W] + [C] or [C, 1, 1].
Tensor add(const Tensor& a, const Tensor& b);

}  // namespace tbn
