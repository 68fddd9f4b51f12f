// Pooling and elementwise operators used between the GEMM/conv layers of a
// Session (MaxPool, GlobalAveragePool, Add, Relu, Sub/Greater/Less and the
// ternary Relu replacement).  All are HBM-bound; they
// keep the reference's arithmetic order where it fixes the rounding
// (GlobalAveragePool sums each plane sequentially, as pooling.cpp:200-212).
#include <string>

#include <algorithm>

#include "common.hpp"

namespace {

constexpr int kThreads = 256;

inline int grid_for(int64_t work) {
    const int64_t blocks = tbn_hip::ceil_div(work, kThreads);
    return static_cast<int>(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

// tbn::maxpool2d (pooling.cpp:10-80): -inf start, taps outside the image are
// skipped, running max updated only when strictly greater (NaN is ignored).
__global__ void maxpool2d_kernel(const float* __restrict__ x, int64_t planes, int H, int W,
                                 int OH, int OW, int kh, int kw, int sh, int sw, int ph, int pw,
                                 int dh, int dw, float* __restrict__ y) {
    // blockIdx.y (grid-strided) walks the planes, x-threads the plane's
    // outputs: 32-bit index math only
    const int per_plane = OH * OW;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= per_plane) return;
    const int oh = i / OW;
    const int ow = i - oh * OW;
    const int ih0 = oh * sh - ph, iw0 = ow * sw - pw;
    for (int64_t plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const float* src = x + plane * H * W;
        float mx = -INFINITY;
        for (int r = 0; r < kh; ++r) {
            const int ih = ih0 + r * dh;
            if (ih < 0 || ih >= H) continue;
            for (int s = 0; s < kw; ++s) {
                const int iw = iw0 + s * dw;
                if (iw < 0 || iw >= W) continue;
                const float v = src[ih * W + iw];
                if (mx < v) mx = v;
            }
        }
        y[plane * per_plane + i] = mx;
    }
}

// tbn::global_avgpool2d (pooling.cpp:184-216): one thread per plane, summing
// in memory order so the result matches the sequential reference bit for bit.
__global__ void global_avgpool_kernel(const float* __restrict__ x, int64_t planes, int64_t hw,
                                      float* __restrict__ y) {
    const int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (p >= planes) return;
    const float* src = x + p * hw;
    float sum = 0.0f;
    for (int64_t i = 0; i < hw; ++i) sum += src[i];
    y[p] = sum / static_cast<float>(hw);
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b, int64_t outer,
                           int64_t inner, int64_t rest, int64_t outer_b, int relu,
                           float* __restrict__ y) {
    const int64_t total = outer * inner * rest;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i_in = (t / rest) % inner;
        const int64_t i_out = t / (rest * inner);
        float v = a[t] + b[(i_out % outer_b) * inner + i_in];
        if (relu) v = v > 0.0f ? v : 0.0f;
        y[t] = v;
    }
}

// std::max(0.0f, x): NaN and -0.0 give +0.0 (model.hpp:1166-1171).
__global__ void relu_kernel(const float* __restrict__ x, int64_t n, float* __restrict__ y) {
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < n;
         t += (int64_t)gridDim.x * blockDim.x) {
        const float v = x[t];
        y[t] = v > 0.0f ? v : 0.0f;
    }
}

// Sub / Greater / Less of the Session (model.hpp:1176-1300): the right
// operand is b[i % nb] when b is given, else the scalar.
__global__ void elementwise_kernel(int op, const float* __restrict__ a, int64_t n,
                                   const float* __restrict__ b, int64_t nb, float scalar,
                                   float* __restrict__ y) {
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < n;
         t += (int64_t)gridDim.x * blockDim.x) {
        const float r = b ? b[t % nb] : scalar;
        const float l = a[t];
        float v;
        if (op == TBN_OP_SUB) v = l - r;
        else if (op == TBN_OP_GREATER) v = (l > r) ? 1.0f : 0.0f;
        else v = (l < r) ? 1.0f : 0.0f;
        y[t] = v;
    }
}

// The Session's ternary Relu replacement (model.hpp:1144-1165):
// x > t -> 1, x < -t -> -1, else 0 (NaN -> 0).
__global__ void ternary_activation_kernel(const float* __restrict__ x, int64_t n, float t,
                                          float* __restrict__ y) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float v = x[i];
        y[i] = (v > t) ? 1.0f : ((v < -t) ? -1.0f : 0.0f);
    }
}

}  // namespace

extern "C" {

int tbn_hip_elementwise(int op, const float* a, int64_t n, const float* b, int64_t nb, float scalar,
                        float* y, tbn_stream_t stream) {
    TBN_REQUIRE(op == TBN_OP_SUB || op == TBN_OP_GREATER || op == TBN_OP_LESS, TBN_INVALID_ARGUMENT,
                "unknown elementwise op");
    TBN_REQUIRE(n >= 0 && (b == nullptr || nb > 0), TBN_INVALID_SHAPE, "invalid sizes");
    if (n == 0) return tbn_hip::ok();
    TBN_REQUIRE(a && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                       tbn_hip::stream_of(stream), op, a, n, b, nb, scalar, y);
    return tbn_hip::check_launch("elementwise");
}

int tbn_hip_ternary_activation(const float* x, int64_t n, float threshold, float* y,
                               tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    if (n == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipLaunchKernelGGL(ternary_activation_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                       tbn_hip::stream_of(stream), x, n, threshold, y);
    return tbn_hip::check_launch("ternary_activation");
}

int tbn_hip_maxpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh,
                      int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh,
                      int64_t dw, int ceil_mode, float* y, int64_t* out_hw, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0 && c >= 0 && h > 0 && w > 0, TBN_INVALID_SHAPE, "invalid input shape");
    TBN_REQUIRE(kh > 0 && kw > 0 && sh > 0 && sw > 0 && dh > 0 && dw > 0 && ph >= 0 && pw >= 0,
                TBN_INVALID_ARGUMENT, "invalid pooling parameters");
    int64_t OH, OW;
    if (ceil_mode) {
        OH = (h + 2 * ph - kh + sh - 1) / sh + 1;
        OW = (w + 2 * pw - kw + sw - 1) / sw + 1;
    } else {
        OH = (h + 2 * ph - kh) / sh + 1;
        OW = (w + 2 * pw - kw) / sw + 1;
    }
    TBN_REQUIRE(OH > 0 && OW > 0, TBN_INVALID_SHAPE, "invalid pooled output size");
    if (out_hw) { out_hw[0] = OH; out_hw[1] = OW; }
    if (!y || n * c == 0) return tbn_hip::ok();
    TBN_REQUIRE(x != nullptr, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    TBN_REQUIRE(h * w < (1LL << 31) && OH * OW < (1LL << 31), TBN_INVALID_SHAPE, "pooling plane too large");
    hipLaunchKernelGGL(maxpool2d_kernel,
                       dim3(static_cast<unsigned>(tbn_hip::ceil_div(OH * OW, kThreads)),
                            static_cast<unsigned>(std::min<int64_t>(n * c, 65535))),
                       dim3(kThreads), 0,
                       tbn_hip::stream_of(stream), x, n * c, int(h), int(w), int(OH), int(OW),
                       int(kh), int(kw), int(sh), int(sw), int(ph), int(pw), int(dh), int(dw), y);
    return tbn_hip::check_launch("maxpool2d");
}

int tbn_hip_global_avgpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, float* y,
                             tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0 && c >= 0 && h > 0 && w > 0, TBN_INVALID_SHAPE, "invalid input shape");
    if (n * c == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipLaunchKernelGGL(global_avgpool_kernel, dim3(tbn_hip::ceil_div(n * c, 64)), dim3(64), 0,
                       tbn_hip::stream_of(stream), x, n * c, h * w, y);
    return tbn_hip::check_launch("global_avgpool2d");
}

int tbn_hip_add(const float* a, const float* b, int64_t outer, int64_t inner, int64_t rest,
                int64_t outer_b, int flags, float* y, tbn_stream_t stream) {
    TBN_REQUIRE(outer >= 0 && inner >= 0 && rest >= 0 && outer_b >= 1, TBN_INVALID_SHAPE,
                "invalid broadcast view");
    TBN_REQUIRE((flags & ~TBN_EPI_RELU) == 0, TBN_INVALID_ARGUMENT, "unsupported flags for add");
    const int64_t total = outer * inner * rest;
    if (total == 0) return tbn_hip::ok();
    TBN_REQUIRE(a && b && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(total)), dim3(kThreads), 0,
                       tbn_hip::stream_of(stream), a, b, outer, inner, rest, outer_b,
                       (flags & TBN_EPI_RELU) ? 1 : 0, y);
    return tbn_hip::check_launch("add");
}

int tbn_hip_relu(const float* x, int64_t n, float* y, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    if (n == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipLaunchKernelGGL(relu_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                       tbn_hip::stream_of(stream), x, n, y);
    return tbn_hip::check_launch("relu");
}

}  // extern "C"
