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

// The 3x3 / stride 2 / pad 1 pool (ResNet stems): a thread walks one output
// column down a band of rows.  Each input row's 3-wide maximum (a float2 at
// 2*ow and a float at 2*ow - 1) serves the two output rows that share it.
// Taking the running maximum of the row maxima in row order, each one a
// running maximum in column order, keeps the reference's first-wins result
// (which of -0 / +0 is kept, NaN ignored).
__device__ __forceinline__ float first_max(float m, float v) { return m < v ? v : m; }

template <bool VEC2>
__global__ void __launch_bounds__(256) maxpool3x3s2_kernel(const float* __restrict__ x, int H, int W, int OH, int OW,
                                                           int band, float* __restrict__ y) {
    const int64_t plane = blockIdx.x;
    const int ow = static_cast<int>(blockIdx.y) * 64 + (threadIdx.x & 63);
    const int oh0 = (static_cast<int>(blockIdx.z) * 4 + (threadIdx.x >> 6)) * band;
    if (ow >= OW || oh0 >= OH) return;
    const int oh1 = min(OH, oh0 + band);
    const float* src = x + plane * H * W;
    float* dst = y + plane * OH * OW + ow;
    const int c = 2 * ow;
    auto row_max = [&](int ih) {
        float m = -INFINITY;
        if (ih < 0 || ih >= H) return m;
        const float* r = src + ih * W;
        if (c >= 1) m = first_max(m, r[c - 1]);
        if (VEC2 && c + 1 < W) {
            const float2 v = *reinterpret_cast<const float2*>(r + c);
            m = first_max(m, v.x);
            m = first_max(m, v.y);
        } else {
            if (c < W) m = first_max(m, r[c]);
            if (c + 1 < W) m = first_max(m, r[c + 1]);
        }
        return m;
    };
    float top = row_max(2 * oh0 - 1);
    for (int oh = oh0; oh < oh1; ++oh) {
        const float mid = row_max(2 * oh);
        const float bot = row_max(2 * oh + 1);
        float m = first_max(-INFINITY, top);
        m = first_max(m, mid);
        m = first_max(m, bot);
        dst[static_cast<int64_t>(oh) * OW] = m;
        top = bot;
    }
}

// tbn::avgpool2d (pooling.cpp:83-148): the window's taps inside the image
// summed in row-major window order; the count adds taps outside the image
// only with count_include_pad; an empty count gives 0.
__global__ void avgpool2d_kernel(const float* __restrict__ x, int64_t planes, int H, int W, int OH, int OW, int kh,
                                 int kw, int sh, int sw, int ph, int pw, int dh, int dw, int include_pad,
                                 float* __restrict__ y) {
    const int per_plane = OH * OW;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= per_plane) return;
    const int oh = i / OW;
    const int ow = i - oh * OW;
    const int ih0 = oh * sh - ph, iw0 = ow * sw - pw;
    for (int64_t plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const float* src = x + plane * H * W;
        float sum = 0.0f;
        int count = 0;
        for (int r = 0; r < kh; ++r) {
            const int ih = ih0 + r * dh;
            for (int s = 0; s < kw; ++s) {
                const int iw = iw0 + s * dw;
                if (ih >= 0 && ih < H && iw >= 0 && iw < W) {
                    sum += src[ih * W + iw];
                    ++count;
                } else if (include_pad) {
                    ++count;
                }
            }
        }
        y[plane * per_plane + i] = count > 0 ? sum / static_cast<float>(count) : 0.0f;
    }
}

// tbn::global_avgpool2d (pooling.cpp:184-216) and tbn::global_maxpool2d
// (pooling.cpp:151-181): one thread per plane, walking it in memory order so
// the result matches the sequential reference bit for bit (the sum's
// rounding; for the maximum, which of -0 / +0 is kept, NaN ignored).
template <bool MAX>
__global__ void __launch_bounds__(256) global_pool_kernel(const float* __restrict__ x, int64_t planes,
                                                          int64_t hw, float* __restrict__ y) {
    // a block owns 64 consecutive planes (contiguous in memory); each chunk
    // of 64 positions of all 64 planes is staged through LDS with coalesced
    // loads, all 16 of a thread's issued before the first store (one memory
    // latency per chunk, not 16), then thread p adds its plane's values in
    // memory order
    __shared__ float tile[64][65];
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int np = static_cast<int>(planes - p0 < 64 ? planes - p0 : 64);
    const int tid = threadIdx.x;
    float acc = MAX ? -INFINITY : 0.0f;
    for (int64_t c0 = 0; c0 < hw; c0 += 64) {
        const int cl = static_cast<int>(hw - c0 < 64 ? hw - c0 : 64);
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int idx = j * 256 + tid, pl = idx >> 6, i = idx & 63;
            v[j] = (pl < np && i < cl) ? x[(p0 + pl) * hw + c0 + i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int idx = j * 256 + tid;
            tile[idx >> 6][idx & 63] = v[j];
        }
        __syncthreads();
        if (tid < np)
            for (int i = 0; i < cl; ++i) {
                if (MAX) acc = first_max(acc, tile[tid][i]);
                else acc += tile[tid][i];
            }
        __syncthreads();
    }
    if (tid < np) y[p0 + tid] = MAX ? acc : acc / static_cast<float>(hw);
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
    if (kh == 3 && kw == 3 && sh == 2 && sw == 2 && ph == 1 && pw == 1 && dh == 1 && dw == 1 &&
        n * c < (1LL << 31) && tbn_hip::ceil_div(OW, 64) <= 65535) {
        const int64_t band = std::min<int64_t>(16, tbn_hip::ceil_div(OH, 4));
        const dim3 grid(static_cast<unsigned>(n * c), static_cast<unsigned>(tbn_hip::ceil_div(OW, 64)),
                        static_cast<unsigned>(tbn_hip::ceil_div(OH, 4 * band)));
        TBN_REQUIRE(grid.z <= 65535, TBN_INVALID_SHAPE, "pooling input too large");
        const bool vec2 = (w % 2 == 0) && (reinterpret_cast<uintptr_t>(x) % 8 == 0);
        if (vec2)
            hipLaunchKernelGGL(maxpool3x3s2_kernel<true>, grid, dim3(256), 0, tbn_hip::stream_of(stream), x, int(h),
                               int(w), int(OH), int(OW), int(band), y);
        else
            hipLaunchKernelGGL(maxpool3x3s2_kernel<false>, grid, dim3(256), 0, tbn_hip::stream_of(stream), x, int(h),
                               int(w), int(OH), int(OW), int(band), y);
        return tbn_hip::check_launch("maxpool2d");
    }
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
    hipLaunchKernelGGL(global_pool_kernel<false>, dim3(tbn_hip::ceil_div(n * c, 64)), dim3(256), 0,
                       tbn_hip::stream_of(stream), x, n * c, h * w, y);
    return tbn_hip::check_launch("global_avgpool2d");
}

int tbn_hip_global_maxpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, float* y,
                             tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0 && c >= 0 && h > 0 && w > 0, TBN_INVALID_SHAPE, "invalid input shape");
    if (n * c == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipLaunchKernelGGL(global_pool_kernel<true>, dim3(tbn_hip::ceil_div(n * c, 64)), dim3(256), 0,
                       tbn_hip::stream_of(stream), x, n * c, h * w, y);
    return tbn_hip::check_launch("global_maxpool2d");
}

int tbn_hip_avgpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t sh,
                      int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, int ceil_mode,
                      int count_include_pad, float* y, int64_t* out_hw, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0 && c >= 0 && h > 0 && w > 0, TBN_INVALID_SHAPE, "invalid input shape");
    TBN_REQUIRE(kh > 0 && kw > 0 && sh > 0 && sw > 0 && dh > 0 && dw > 0 && ph >= 0 && pw >= 0,
                TBN_INVALID_ARGUMENT, "invalid pooling parameters");
    // pooling.cpp:97-104: the output size does not involve the dilation
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
    TBN_REQUIRE(h * w < (1LL << 31) && OH * OW < (1LL << 31) && kh * kw < (1LL << 31), TBN_INVALID_SHAPE,
                "pooling plane too large");
    hipLaunchKernelGGL(avgpool2d_kernel,
                       dim3(static_cast<unsigned>(tbn_hip::ceil_div(OH * OW, kThreads)),
                            static_cast<unsigned>(std::min<int64_t>(n * c, 65535))),
                       dim3(kThreads), 0, tbn_hip::stream_of(stream), x, n * c, int(h), int(w), int(OH), int(OW),
                       int(kh), int(kw), int(sh), int(sw), int(ph), int(pw), int(dh), int(dw),
                       count_include_pad ? 1 : 0, y);
    return tbn_hip::check_launch("avgpool2d");
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
