// Operator entry points of the tbn runtime: argument checks in the
// reference's terms, then HIP kernels of libtbn_hip.so on the current stream.
#include <cmath>
#include <string>
#include <vector>

#include "tbn/device.hpp"
#include "internal.hpp"
#include "tbn/operators.hpp"
#include "tbn_hip.h"

namespace tbn {

namespace {

tbn_stream_t stream() { return device::current_stream(); }

// Device view of an operand (uploads host tensors).
Tensor on_device(const Tensor& t) { return t.on_device() ? t : t.to_device(DeviceType::HIP); }

// Delivers a device result where the operator's first argument lives.
Tensor deliver(const Tensor& result, const Tensor& first) {
    return first.on_device() ? result : result.to_device(DeviceType::CPU);
}

using detail::ceil_to;

void require_float(const Tensor& t, const char* what) {
    TBN_CHECK(t.dtype() == DataType::FLOAT32, InvalidArgumentError,
              std::string(what) + " must be FLOAT32");
}

// Weight matrix view: KN = W[K, N] (2-D), NK = W[N, K...] (any rank >= 2).
void weight_dims(const Tensor& w, bool nk, int64_t& K, int64_t& N) {
    const auto& d = w.shape().dims;
    TBN_CHECK(d.size() >= 2, InvalidShapeError, "weights must be at least 2-D, got " + shape_to_string(w.shape()));
    if (nk) {
        N = d[0];
        K = w.num_elements() / (N > 0 ? N : 1);
    } else {
        TBN_CHECK(d.size() == 2, InvalidShapeError, "B must be 2-D, got " + shape_to_string(w.shape()));
        K = d[0];
        N = d[1];
    }
}

struct ConvShape {
    tbn_conv2d_desc desc;
    int64_t OH, OW;
};

ConvShape conv_shape(const Tensor& input, const Tensor& weights, const Conv2DParams& p) {
    TBN_CHECK(input.shape().rank() == 4, InvalidShapeError,
              "Conv2D input must be 4D (NCHW), got " + shape_to_string(input.shape()));
    TBN_CHECK(weights.shape().rank() == 4, InvalidShapeError,
              "Conv2D weights must be 4D (MCHW), got " + shape_to_string(weights.shape()));
    require_float(input, "Conv2D input");
    const auto& x = input.shape().dims;
    const auto& w = weights.shape().dims;
    TBN_CHECK(p.groups >= 1, InvalidArgumentError, "Groups must be positive");
    TBN_CHECK(x[1] % p.groups == 0 && w[0] % p.groups == 0, InvalidShapeError,
              "Input and output channels must be divisible by groups");
    TBN_CHECK(x[1] == w[1] * p.groups, InvalidShapeError,
              "Input channels (" + std::to_string(x[1]) + ") must match weight channels (" +
                  std::to_string(w[1]) + ") times groups");
    ConvShape cs;
    cs.desc = tbn_conv2d_desc{x[0], x[1], x[2], x[3], w[0], w[2], w[3], p.stride_h, p.stride_w,
                              p.pad_h, p.pad_w, p.dilation_h, p.dilation_w};
    TBN_CHECK(p.stride_h > 0 && p.stride_w > 0 && p.dilation_h > 0 && p.dilation_w > 0 &&
                  p.pad_h >= 0 && p.pad_w >= 0,
              InvalidArgumentError, "invalid stride/padding/dilation");
    cs.OH = (x[2] + 2 * p.pad_h - p.dilation_h * (w[2] - 1) - 1) / p.stride_h + 1;
    cs.OW = (x[3] + 2 * p.pad_w - p.dilation_w * (w[3] - 1) - 1) / p.stride_w + 1;
    TBN_CHECK(cs.OH > 0 && cs.OW > 0, InvalidShapeError, "Invalid output dimensions");
    return cs;
}

void check_bias(const Tensor* bias, int64_t m) {
    if (!bias) return;
    require_float(*bias, "bias");
    TBN_CHECK(bias->num_elements() == m, InvalidShapeError,
              "bias must have " + std::to_string(m) + " elements, got " + shape_to_string(bias->shape()));
}

Tensor conv_quantized(const Tensor& input, const PackedWeights& pw, const ConvShape& cs, const Tensor* scales,
                      const Tensor* bias, int flags) {
    Tensor x = on_device(input);
    Tensor b = bias ? on_device(*bias) : Tensor();
    Tensor s = scales ? on_device(*scales) : Tensor();
    Tensor y = Tensor::empty({cs.desc.n, cs.desc.m, cs.OH, cs.OW}, DataType::FLOAT32, DeviceType::HIP);
    const auto fn = pw.kind == PackedWeights::Kind::Binary ? tbn_hip_conv2d_f32_binary : tbn_hip_conv2d_f32_ternary;
    check_status(fn(x.typed_data<float>(), &cs.desc, pw.bits.typed_data<uint8_t>(), pw.K_pad, pw.N_pad,
                    scales ? s.typed_data<float>() : nullptr, 1.0f, bias ? b.typed_data<float>() : nullptr,
                    flags, y.typed_data<float>(), stream()),
                 pw.kind == PackedWeights::Kind::Binary ? "conv2d_binary" : "conv2d_ternary");
    return deliver(y, input);
}

}  // namespace

// ---- quantization ----------------------------------------------------------------

Tensor quantize_to_binary(const Tensor& weights, float threshold) {
    Tensor w = on_device(weights);
    Tensor out = Tensor::empty(weights.shape(), DataType::BINARY, DeviceType::HIP);
    if (weights.dtype() == DataType::FLOAT32) {
        check_status(tbn_hip_quantize_to_binary_f32(w.typed_data<float>(), w.num_elements(), threshold,
                                                    out.typed_data<uint8_t>(), stream()),
                     "quantize_to_binary");
    } else if (weights.dtype() == DataType::INT8) {
        check_status(tbn_hip_quantize_to_binary_i8(w.typed_data<int8_t>(), w.num_elements(),
                                                   out.typed_data<uint8_t>(), stream()),
                     "quantize_to_binary");
    } else {
        throw InvalidArgumentError("Unsupported dtype for binary quantization");
    }
    return deliver(out, weights);
}

Tensor quantize_to_ternary(const Tensor& weights, float lo, float hi) {
    TBN_CHECK(weights.dtype() == DataType::FLOAT32, InvalidArgumentError,
              "Unsupported dtype for ternary quantization");
    Tensor w = on_device(weights);
    Tensor out = Tensor::empty(weights.shape(), DataType::TERNARY, DeviceType::HIP);
    check_status(tbn_hip_quantize_to_ternary_f32(w.typed_data<float>(), w.num_elements(), lo, hi,
                                                 out.typed_data<int8_t>(), stream()),
                 "quantize_to_ternary");
    return deliver(out, weights);
}

bool is_binary_float_weights(const float* data, size_t count) {
    for (size_t i = 0; i < count; ++i) {
        const float v = data[i];
        if (v != -1.0f && v != 1.0f && v != 0.0f) return false;
    }
    return true;
}

// ---- packing -----------------------------------------------------------------------

PackedWeights pack_binary_weights(const Tensor& weights, bool nk, bool ge_zero) {
    PackedWeights pw;
    pw.kind = PackedWeights::Kind::Binary;
    weight_dims(weights, nk, pw.K, pw.N);
    pw.K_pad = ceil_to(pw.K, 128);
    pw.N_pad = ceil_to(pw.N, 8);
    pw.bits = Tensor::empty({pw.N_pad * pw.K_pad / 8}, DataType::UINT8, DeviceType::HIP);
    Tensor w = on_device(weights);
    const int layout = nk ? TBN_LAYOUT_NK : TBN_LAYOUT_KN;
    if (weights.dtype() == DataType::BINARY || weights.dtype() == DataType::UINT8) {
        check_status(tbn_hip_pack_binary(w.typed_data<uint8_t>(), pw.K, pw.N, layout, pw.K_pad, pw.N_pad,
                                         pw.bits.typed_data<uint8_t>(), stream()),
                     "pack_binary_weights");
    } else if (weights.dtype() == DataType::FLOAT32) {
        check_status(tbn_hip_quantize_pack_binary_f32(
                         w.typed_data<float>(), pw.K, pw.N, layout,
                         ge_zero ? TBN_SIGN_GE_ZERO : TBN_SIGN_GT_THRESHOLD, 0.0f, pw.K_pad, pw.N_pad,
                         pw.bits.typed_data<uint8_t>(), stream()),
                     "pack_binary_weights");
    } else {
        throw InvalidArgumentError("binary weights must be BINARY or FLOAT32");
    }
    return pw;
}

PackedWeights pack_ternary_weights(const Tensor& weights, bool nk) {
    TBN_CHECK(weights.dtype() == DataType::TERNARY || weights.dtype() == DataType::INT8,
              InvalidArgumentError, "ternary weights must be TERNARY");
    PackedWeights pw;
    pw.kind = PackedWeights::Kind::Ternary;
    weight_dims(weights, nk, pw.K, pw.N);
    pw.K_pad = ceil_to(pw.K, 128);
    pw.N_pad = ceil_to(pw.N, 8);
    pw.bits = Tensor::empty({pw.N_pad * pw.K_pad / 4}, DataType::UINT8, DeviceType::HIP);
    Tensor w = on_device(weights);
    check_status(tbn_hip_pack_ternary(w.typed_data<int8_t>(), pw.K, pw.N, nk ? TBN_LAYOUT_NK : TBN_LAYOUT_KN,
                                      pw.K_pad, pw.N_pad, pw.bits.typed_data<uint8_t>(), stream()),
                 "pack_ternary_weights");
    return pw;
}

// ---- GEMMs ---------------------------------------------------------------------------

Tensor qlinear_matmul_packed(const Tensor& a, const PackedWeights& w, float scale, const Tensor* channel_scales,
                             const Tensor* bias, bool relu) {
    require_float(a, "Input A");
    TBN_CHECK(a.shape().rank() == 2, InvalidShapeError, "Both inputs must be 2D matrices");
    const int64_t M = a.shape().dims[0], K = a.shape().dims[1];
    TBN_CHECK(K == w.K, InvalidShapeError,
              "Matrix dimensions incompatible: A cols (" + std::to_string(K) + ") != B rows (" +
                  std::to_string(w.K) + ")");
    check_bias(channel_scales, w.N);
    check_bias(bias, w.N);
    Tensor ad = on_device(a);
    Tensor s = channel_scales ? on_device(*channel_scales) : Tensor();
    Tensor b = bias ? on_device(*bias) : Tensor();
    Tensor out = Tensor::empty({M, w.N}, DataType::FLOAT32, DeviceType::HIP);
    const auto fn = w.kind == PackedWeights::Kind::Binary ? tbn_hip_gemm_f32_binary : tbn_hip_gemm_f32_ternary;
    check_status(fn(ad.typed_data<float>(), K, M, w.N, K, w.bits.typed_data<uint8_t>(), w.K_pad, w.N_pad,
                    channel_scales ? s.typed_data<float>() : nullptr, scale,
                    bias ? b.typed_data<float>() : nullptr, relu ? TBN_EPI_RELU : 0, out.typed_data<float>(),
                    w.N, stream()),
                 w.kind == PackedWeights::Kind::Binary ? "qlinear_matmul_binary" : "qlinear_matmul_ternary");
    return deliver(out, a);
}

namespace {
void check_matmul_operands(const Tensor& a, const Tensor& b) {
    require_float(a, "Input A");
    TBN_CHECK(a.shape().rank() == 2 && b.shape().rank() == 2, InvalidShapeError,
              "Both inputs must be 2D matrices");
    TBN_CHECK(a.shape().dims[1] == b.shape().dims[0], InvalidShapeError,
              "Matrix dimensions incompatible: A cols (" + std::to_string(a.shape().dims[1]) +
                  ") != B rows (" + std::to_string(b.shape().dims[0]) + ")");
}
}  // namespace

Tensor qlinear_matmul_binary_float(const Tensor& a, const Tensor& b, float b_scale, const TilingParams&) {
    check_matmul_operands(a, b);
    require_float(b, "Input B");
    const std::vector<float> host = b.to_vector<float>();
    TBN_CHECK(is_binary_float_weights(host.data(), host.size()), InvalidArgumentError,
              "FLOAT32 B must hold only -1, 0 and +1");
    return qlinear_matmul_packed(a, pack_binary_weights(b, false, true), b_scale);
}

Tensor qlinear_matmul_binary(const Tensor& a, const Tensor& b, float b_scale, const TilingParams& params) {
    check_matmul_operands(a, b);
    if (b.dtype() == DataType::FLOAT32) return qlinear_matmul_binary_float(a, b, b_scale, params);
    TBN_CHECK(b.dtype() == DataType::BINARY, InvalidArgumentError,
              "Input B must be BINARY or FLOAT32 with binary values");
    return qlinear_matmul_packed(a, pack_binary_weights(b, false), b_scale);
}

Tensor qlinear_matmul_packed_tbn(const Tensor& a, const PackedWeights& w, float scale, float lo, float hi) {
    require_float(a, "Input A");
    TBN_CHECK(w.kind == PackedWeights::Kind::Binary, InvalidArgumentError, "TBN mode needs binary weights");
    TBN_CHECK(a.shape().rank() == 2, InvalidShapeError, "Both inputs must be 2D matrices");
    const int64_t M = a.shape().dims[0], K = a.shape().dims[1];
    TBN_CHECK(K == w.K, InvalidShapeError,
              "Matrix dimensions incompatible: A cols (" + std::to_string(K) + ") != B rows (" +
                  std::to_string(w.K) + ")");
    Tensor ad = on_device(a);
    Tensor out = Tensor::empty({M, w.N}, DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_qlinear_matmul_binary_tbn(ad.typed_data<float>(), K, M, K, w.bits.typed_data<uint8_t>(),
                                                   w.K_pad, w.N, w.N_pad, scale, lo, hi, out.typed_data<float>(),
                                                   w.N, stream()),
                 "qlinear_matmul_binary (TBN mode)");
    return deliver(out, a);
}

Tensor qlinear_matmul_binary_tbn(const Tensor& a, const Tensor& b, float b_scale, const TilingParams&, float lo,
                                 float hi) {
    check_matmul_operands(a, b);
    TBN_CHECK(b.dtype() == DataType::BINARY, InvalidArgumentError, "Input B must be BINARY");
    return qlinear_matmul_packed_tbn(a, pack_binary_weights(b, false), b_scale, lo, hi);
}

Tensor qlinear_matmul_ternary(const Tensor& a, const Tensor& b, float b_scale, const TilingParams&) {
    check_matmul_operands(a, b);
    TBN_CHECK(b.dtype() == DataType::TERNARY, InvalidArgumentError, "Input B must be TERNARY");
    return qlinear_matmul_packed(a, pack_ternary_weights(b, false), b_scale);
}

// conv2d.cpp:372-384 (which throws for groups > 1).
Tensor conv2d_grouped(const Tensor& input, const Tensor& weights, const Tensor* bias, int64_t groups,
                      const Conv2DParams& params) {
    Conv2DParams p = params;
    p.groups = groups;
    ConvShape cs = conv_shape(input, weights, p);
    require_float(weights, "Conv2D weights");
    check_bias(bias, cs.desc.m);
    if (groups == 1) return conv2d(input, weights, bias, p);
    Tensor x = on_device(input), w = on_device(weights);
    Tensor b = bias ? on_device(*bias) : Tensor();
    Tensor y = Tensor::empty({cs.desc.n, cs.desc.m, cs.OH, cs.OW}, DataType::FLOAT32, DeviceType::HIP);
    const float* wp = w.typed_data<float>();
    const float* bp = bias ? b.typed_data<float>() : nullptr;
    if (cs.desc.c == groups) {
        check_status(tbn_hip_conv2d_depthwise(x.typed_data<float>(), &cs.desc, wp, nullptr, 1.0f, bp, nullptr, 0,
                                              y.typed_data<float>(), stream()),
                     "depthwise_conv2d");
        return deliver(y, input);
    }
    const int64_t ws_floats = detail::grouped_conv_workspace(cs.desc, groups);
    Tensor ws = ws_floats ? Tensor::empty({ws_floats}, DataType::FLOAT32, DeviceType::HIP) : Tensor();
    const int64_t wpg = weights.num_elements() / groups;  // weights per group
    detail::run_grouped_conv(
        cs.desc, groups, x.typed_data<float>(), y.typed_data<float>(), ws_floats ? ws.typed_data<float>() : nullptr,
        [&](int64_t g, const float* xg, const tbn_conv2d_desc& dg, float* yg) {
            check_status(tbn_hip_conv2d_f32(xg, &dg, wp + g * wpg, bp ? bp + g * dg.m : nullptr, 0, yg, stream()),
                         "conv2d_grouped");
        },
        stream());
    return deliver(y, input);
}

// conv2d.cpp:386-393: groups = input channels.
Tensor depthwise_conv2d(const Tensor& input, const Tensor& weights, const Tensor* bias, const Conv2DParams& params) {
    TBN_CHECK(input.shape().rank() == 4, InvalidShapeError, "Conv2D input must be 4D (NCHW)");
    return conv2d_grouped(input, weights, bias, input.shape().dims[1], params);
}

// conv2d.cpp:396-403: the same dilation on both axes.
Tensor dilated_conv2d(const Tensor& input, const Tensor& weights, const Tensor* bias, int64_t dilation,
                      const Conv2DParams& params) {
    Conv2DParams p = params;
    p.dilation_h = dilation;
    p.dilation_w = dilation;
    return conv2d(input, weights, bias, p);
}

Tensor batch_norm(const Tensor& input, const Tensor& scale, const Tensor& B, const Tensor& mean, const Tensor& var,
                  float epsilon) {
    require_float(input, "BatchNormalization input");
    const auto& d = input.shape().dims;
    TBN_CHECK(d.size() >= 2, InvalidShapeError, "BatchNormalization input must be at least 2-D");
    const int64_t c = d[1];
    std::vector<float> k, t;
    detail::batch_norm_affine(scale, B, mean, var, epsilon, c, k, t);
    int64_t hw = 1;
    for (size_t i = 2; i < d.size(); ++i) hw *= d[i];
    Tensor x = on_device(input);
    Tensor kd = Tensor(Shape{c}, DataType::FLOAT32, k.data(), DeviceType::HIP);
    Tensor td = Tensor(Shape{c}, DataType::FLOAT32, t.data(), DeviceType::HIP);
    Tensor y = Tensor::empty(input.shape(), DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_channel_affine(x.typed_data<float>(), d[0], c, hw, kd.typed_data<float>(),
                                        td.typed_data<float>(), 0, y.typed_data<float>(), stream()),
                 "batch_norm");
    return deliver(y, input);
}

Tensor gemm(const Tensor& A, const Tensor& B, const Tensor* C, float alpha, float beta, bool transA,
            bool transB) {
    TBN_CHECK(A.dtype() == DataType::FLOAT32, InvalidArgumentError, "gemm requires float32 input A");
    TBN_CHECK(B.dtype() == DataType::FLOAT32, InvalidArgumentError, "gemm requires float32 input B");
    TBN_CHECK(A.shape().rank() == 2 && B.shape().rank() == 2, InvalidShapeError, "gemm inputs must be 2-D");
    const int64_t M = transA ? A.shape().dims[1] : A.shape().dims[0];
    const int64_t K = transA ? A.shape().dims[0] : A.shape().dims[1];
    const int64_t Kb = transB ? B.shape().dims[1] : B.shape().dims[0];
    const int64_t N = transB ? B.shape().dims[0] : B.shape().dims[1];
    TBN_CHECK(K == Kb, InvalidShapeError, "gemm inner dimensions differ");
    const bool use_c = C && beta != 0.0f;
    bool c_1d = false;
    if (use_c) {
        require_float(*C, "C");
        c_1d = C->shape().rank() == 1;
        TBN_CHECK(c_1d ? C->num_elements() == N : C->num_elements() == M * N, InvalidShapeError,
                  "C must be [N] or [M, N]");
    }
    Tensor a = on_device(A), b = on_device(B);
    Tensor c = use_c ? on_device(*C) : Tensor();
    Tensor out = Tensor::empty({M, N}, DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_gemm_f32(a.typed_data<float>(), b.typed_data<float>(),
                                  use_c ? c.typed_data<float>() : nullptr, c_1d ? 1 : 0, M, K, N, alpha, beta,
                                  transA, transB, 0, out.typed_data<float>(), stream()),
                 "gemm");
    return deliver(out, A);
}

// ---- convolution -------------------------------------------------------------------------

Tensor conv2d(const Tensor& input, const Tensor& weights, const Tensor* bias, const Conv2DParams& params) {
    if (params.groups != 1) return conv2d_grouped(input, weights, bias, params.groups, params);
    ConvShape cs = conv_shape(input, weights, params);
    require_float(weights, "Conv2D weights");
    check_bias(bias, cs.desc.m);
    Tensor x = on_device(input), w = on_device(weights);
    Tensor b = bias ? on_device(*bias) : Tensor();
    Tensor y = Tensor::empty({cs.desc.n, cs.desc.m, cs.OH, cs.OW}, DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_conv2d_f32(x.typed_data<float>(), &cs.desc, w.typed_data<float>(),
                                    bias ? b.typed_data<float>() : nullptr, 0, y.typed_data<float>(), stream()),
                 "conv2d");
    return deliver(y, input);
}

Tensor conv2d_binary(const Tensor& input, const Tensor& weights, const Tensor* bias, const Conv2DParams& params) {
    TBN_CHECK(params.groups == 1, NotImplementedError, "grouped binary/ternary convolution: use a Session");
    ConvShape cs = conv_shape(input, weights, params);
    TBN_CHECK(weights.dtype() == DataType::BINARY, InvalidArgumentError, "conv2d_binary needs BINARY weights");
    check_bias(bias, cs.desc.m);
    return conv_quantized(input, pack_binary_weights(weights, true), cs, nullptr, bias, 0);
}

Tensor conv2d_ternary(const Tensor& input, const Tensor& weights, const Tensor* bias, const Conv2DParams& params) {
    TBN_CHECK(params.groups == 1, NotImplementedError, "grouped binary/ternary convolution: use a Session");
    ConvShape cs = conv_shape(input, weights, params);
    TBN_CHECK(weights.dtype() == DataType::TERNARY, InvalidArgumentError, "conv2d_ternary needs TERNARY weights");
    check_bias(bias, cs.desc.m);
    return conv_quantized(input, pack_ternary_weights(weights, true), cs, nullptr, bias, 0);
}

Tensor conv2d_binary_with_scales(const Tensor& input, const Tensor& weights, const Tensor* bias,
                                 const Conv2DParams& params, const std::vector<float>& channel_scales) {
    TBN_CHECK(params.groups == 1, NotImplementedError, "grouped binary/ternary convolution: use a Session");
    ConvShape cs = conv_shape(input, weights, params);
    TBN_CHECK(weights.dtype() == DataType::BINARY, InvalidArgumentError,
              "conv2d_binary_with_scales needs BINARY weights");
    TBN_CHECK(static_cast<int64_t>(channel_scales.size()) == cs.desc.m, InvalidArgumentError,
              "channel_scales must have one value per output channel");
    check_bias(bias, cs.desc.m);
    Tensor s({cs.desc.m}, DataType::FLOAT32, channel_scales.data(), DeviceType::HIP);
    return conv_quantized(input, pack_binary_weights(weights, true), cs, &s, bias, 0);
}

// ---- pooling and elementwise -------------------------------------------------------------

Tensor maxpool2d(const Tensor& input, const Pool2DParams& p) {
    TBN_CHECK(input.shape().rank() == 4, InvalidShapeError,
              "MaxPool2D input must be 4D (NCHW), got " + shape_to_string(input.shape()));
    require_float(input, "MaxPool2D input");
    const auto& d = input.shape().dims;
    int64_t hw[2] = {0, 0};
    check_status(tbn_hip_maxpool2d(nullptr, d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w, p.stride_h,
                                   p.stride_w, p.pad_h, p.pad_w, p.dilation_h, p.dilation_w, p.ceil_mode, nullptr,
                                   hw, stream()),
                 "maxpool2d");
    Tensor x = on_device(input);
    Tensor y = Tensor::empty({d[0], d[1], hw[0], hw[1]}, DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_maxpool2d(x.typed_data<float>(), d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w,
                                   p.stride_h, p.stride_w, p.pad_h, p.pad_w, p.dilation_h, p.dilation_w,
                                   p.ceil_mode, y.typed_data<float>(), nullptr, stream()),
                 "maxpool2d");
    return deliver(y, input);
}

Tensor avgpool2d(const Tensor& input, const Pool2DParams& p) {
    TBN_CHECK(input.shape().rank() == 4, InvalidShapeError,
              "AvgPool2D input must be 4D (NCHW), got " + shape_to_string(input.shape()));
    TBN_CHECK(input.dtype() == DataType::FLOAT32, InvalidArgumentError, "AvgPool2D requires float32 input");
    const auto& d = input.shape().dims;
    int64_t hw[2] = {0, 0};
    check_status(tbn_hip_avgpool2d(nullptr, d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w, p.stride_h, p.stride_w,
                                   p.pad_h, p.pad_w, p.dilation_h, p.dilation_w, p.ceil_mode, p.count_include_pad,
                                   nullptr, hw, stream()),
                 "avgpool2d");
    Tensor x = on_device(input);
    Tensor y = Tensor::empty({d[0], d[1], hw[0], hw[1]}, DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_avgpool2d(x.typed_data<float>(), d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w, p.stride_h,
                                   p.stride_w, p.pad_h, p.pad_w, p.dilation_h, p.dilation_w, p.ceil_mode,
                                   p.count_include_pad, y.typed_data<float>(), nullptr, stream()),
                 "avgpool2d");
    return deliver(y, input);
}

Tensor global_maxpool2d(const Tensor& input) {
    TBN_CHECK(input.shape().rank() == 4, InvalidShapeError, "GlobalMaxPool2D input must be 4D (NCHW)");
    require_float(input, "GlobalMaxPool2D input");
    const auto& d = input.shape().dims;
    Tensor x = on_device(input);
    Tensor y = Tensor::empty({d[0], d[1], 1, 1}, DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_global_maxpool2d(x.typed_data<float>(), d[0], d[1], d[2], d[3], y.typed_data<float>(),
                                          stream()),
                 "global_maxpool2d");
    return deliver(y, input);
}

Tensor global_avgpool2d(const Tensor& input) {
    TBN_CHECK(input.shape().rank() == 4, InvalidShapeError, "GlobalAvgPool2D input must be 4D (NCHW)");
    require_float(input, "GlobalAvgPool2D input");
    const auto& d = input.shape().dims;
    Tensor x = on_device(input);
    Tensor y = Tensor::empty({d[0], d[1], 1, 1}, DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_global_avgpool2d(x.typed_data<float>(), d[0], d[1], d[2], d[3], y.typed_data<float>(),
                                          stream()),
                 "global_avgpool2d");
    return deliver(y, input);
}

Tensor relu(const Tensor& input) {
    require_float(input, "Relu input");
    Tensor x = on_device(input);
    Tensor y = Tensor::empty(input.shape(), DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_relu(x.typed_data<float>(), x.num_elements(), y.typed_data<float>(), stream()), "relu");
    return deliver(y, input);
}

namespace detail {

void conv_out_hw(const tbn_conv2d_desc& d, int64_t& OH, int64_t& OW) {
    OH = (d.h + 2 * d.ph - d.dh * (d.kh - 1) - 1) / d.sh + 1;
    OW = (d.w + 2 * d.pw - d.dw * (d.kw - 1) - 1) / d.sw + 1;
}

void batch_norm_affine(const Tensor& scale, const Tensor& B, const Tensor& mean, const Tensor& var, float epsilon,
                       int64_t c, std::vector<float>& k, std::vector<float>& t) {
    const Tensor* parts[4] = {&scale, &B, &mean, &var};
    for (const Tensor* p : parts)
        TBN_CHECK(p->dtype() == DataType::FLOAT32 && p->num_elements() == c, InvalidShapeError,
                  "BatchNormalization parameters must be FLOAT32 with one value per channel");
    const std::vector<float> s = scale.to_vector<float>(), b = B.to_vector<float>(), m = mean.to_vector<float>(),
                             v = var.to_vector<float>();
    k.resize(c);
    t.resize(c);
    for (int64_t i = 0; i < c; ++i) {
        const double ki = static_cast<double>(s[i]) / std::sqrt(static_cast<double>(v[i]) + static_cast<double>(epsilon));
        k[i] = static_cast<float>(ki);
        t[i] = static_cast<float>(static_cast<double>(b[i]) - static_cast<double>(m[i]) * ki);
    }
}

int64_t grouped_conv_workspace(const tbn_conv2d_desc& d, int64_t groups) {
    if (d.n <= 1) return 0;
    int64_t OH, OW;
    conv_out_hw(d, OH, OW);
    return d.n * (d.c / groups * d.h * d.w + d.m / groups * OH * OW);
}

void run_grouped_conv(const tbn_conv2d_desc& d, int64_t groups, const float* x, float* y, float* workspace,
                      const std::function<void(int64_t, const float*, const tbn_conv2d_desc&, float*)>& conv,
                      tbn_stream_t stream) {
    int64_t OH, OW;
    conv_out_hw(d, OH, OW);
    tbn_conv2d_desc dg = d;
    dg.c = d.c / groups;
    dg.m = d.m / groups;
    const int64_t hw = d.h * d.w, ohw = OH * OW;
    const bool direct = d.n == 1;
    TBN_CHECK(direct || workspace != nullptr, RuntimeError, "grouped conv: missing workspace");
    float* xg = workspace;
    float* yg = direct ? nullptr : workspace + d.n * dg.c * hw;
    for (int64_t g = 0; g < groups; ++g) {
        if (direct) {
            conv(g, x + g * dg.c * hw, dg, y + g * dg.m * ohw);
            continue;
        }
        check_status(tbn_hip_copy_channels(x, d.n, d.c, g * dg.c, dg.c, hw, xg, dg.c, 0, stream), "grouped conv gather");
        conv(g, xg, dg, yg);
        check_status(tbn_hip_copy_channels(yg, d.n, dg.m, 0, dg.m, ohw, y, d.m, g * dg.m, stream),
                     "grouped conv scatter");
    }
}

void add_view(const Shape& a, const Shape& b, int64_t& outer, int64_t& inner, int64_t& rest) {
    const auto& da = a.dims;
    const auto& db = b.dims;
    if (da.size() == 2 && db.size() == 1) {
        TBN_CHECK(db[0] == da[1], InvalidShapeError, "Broadcasting: B size must match last dim of A");
        outer = da[0]; inner = da[1]; rest = 1;
        return;
    }
    if (da.size() == 4 && ((db.size() == 3 && db[1] == 1 && db[2] == 1) || db.size() == 1)) {
        TBN_CHECK(db[0] == da[1], InvalidShapeError, "Broadcasting: B channels must match A");
        outer = da[0]; inner = da[1]; rest = da[2] * da[3];
        return;
    }
    TBN_CHECK(a == b, InvalidShapeError, "Add requires same shape tensors or broadcastable shapes");
    outer = 1; inner = a.size(); rest = 1;
}
}  // namespace detail

Tensor add(const Tensor& a_in, const Tensor& b_in) {
    require_float(a_in, "Add input A");
    require_float(b_in, "Add input B");
    // [N] + [M, N] is computed as [M, N] + [N] (float addition commutes).
    const bool swap = a_in.shape().rank() == 1 && b_in.shape().rank() == 2;
    const Tensor& a = swap ? b_in : a_in;
    const Tensor& b = swap ? a_in : b_in;
    int64_t outer, inner, rest;
    detail::add_view(a.shape(), b.shape(), outer, inner, rest);
    Tensor ad = on_device(a), bd = on_device(b);
    Tensor y = Tensor::empty(a.shape(), DataType::FLOAT32, DeviceType::HIP);
    check_status(tbn_hip_add(ad.typed_data<float>(), bd.typed_data<float>(), outer, inner, rest, 1, 0,
                             y.typed_data<float>(), stream()),
                 "add");
    return deliver(y, a_in);
}

}  // namespace tbn
