// Grouped-convolution support: the depthwise kernel (one input channel per
// group), the channel-slice copy that lets a grouped conv run its groups
// through the dense conv kernels, and the per-channel affine map that is an
// inference BatchNormalization.  The reference has none of these: its
// conv2d_grouped and depthwise_conv2d throw for groups > 1
// (tbn-runtime/src/operators/conv2d.cpp:372-393) and BatchNorm folding is
// planned only (ADR/README.md:51).
//
// All three are HBM-bound elementwise-shaped kernels: coalesced 64-lane rows,
// fp32 FMA on the VALU, no matrix cores.
#include <type_traits>

#include "common.hpp"

namespace {

constexpr int kTileW = 64;     // output columns per block (one per lane)
constexpr int kRowsPer = 4;    // output rows per thread
constexpr int kTileH = 4 * kRowsPer;

struct DwGeom {
    int C, H, W, M, mult, OH, OW, kh, kw, sh, sw, ph, pw, dh, dw;
    int64_t planes;            // N * M
    int tiles_w, tiles;        // column tiles, column tiles * row tiles
};

// y[n, m, oh, ow] = epi(sum_{r,s} x[n, m / mult, oh*sh - ph + r*dh, ow*sw - pw + s*dw] * w[m, r, s]),
// taps summed in (r, s) order; epi as the quantized conv's: (acc + a) * alpha*s[m] + b,
// with (a, b) = (bias, 0) under TBN_EPI_BIAS_THEN_SCALE and (0, bias) otherwise,
// then + residual, then ReLU.
__global__ void __launch_bounds__(256) depthwise_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        const float* __restrict__ scale, float alpha,
                                                        const float* __restrict__ bias,
                                                        const float* __restrict__ residual, int flags,
                                                        float* __restrict__ y, DwGeom g) {
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const bool bts = (flags & TBN_EPI_BIAS_THEN_SCALE) != 0, relu = (flags & TBN_EPI_RELU) != 0;
    const int taps = g.kh * g.kw;
    for (int64_t p = blockIdx.y; p < g.planes; p += gridDim.y) {
        const int m = static_cast<int>(p % g.M);
        const int64_t n = p / g.M;
        const float* xp = x + (n * g.C + m / g.mult) * static_cast<int64_t>(g.H) * g.W;
        const float* wp = w + static_cast<int64_t>(m) * taps;
        const float mm = alpha * (scale ? scale[m] : 1.0f);
        const float bb = bias ? bias[m] : 0.0f;
        const float a = bts ? bb : 0.0f, b = bts ? 0.0f : bb;
        const int64_t ybase = p * static_cast<int64_t>(g.OH) * g.OW;
        for (int t = blockIdx.x; t < g.tiles; t += gridDim.x) {
            const int ow = (t % g.tiles_w) * kTileW + tx;
            const int oh0 = (t / g.tiles_w) * kTileH + ty * kRowsPer;
            if (ow >= g.OW) continue;
            float acc[kRowsPer] = {};
            for (int r = 0; r < g.kh; ++r) {
                for (int s = 0; s < g.kw; ++s) {
                    const float wv = wp[r * g.kw + s];
                    const int iw = ow * g.sw - g.pw + s * g.dw;
                    const bool col_in = iw >= 0 && iw < g.W;
#pragma unroll
                    for (int i = 0; i < kRowsPer; ++i) {
                        const int ih = (oh0 + i) * g.sh - g.ph + r * g.dh;
                        const float xv = (col_in && ih >= 0 && ih < g.H) ? xp[static_cast<int64_t>(ih) * g.W + iw] : 0.0f;
                        acc[i] = fmaf(xv, wv, acc[i]);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kRowsPer; ++i) {
                const int oh = oh0 + i;
                if (oh >= g.OH) break;
                const int64_t o = ybase + static_cast<int64_t>(oh) * g.OW + ow;
                float v = (acc[i] + a) * mm + b;
                if (residual) v += residual[o];
                if (relu) v = v > 0.0f ? v : 0.0f;
                y[o] = v;
            }
        }
    }
}

// 3x3 depthwise, dilation 1, stride S in {1, 2}: each thread owns a 4 x 4
// patch of outputs and reads its (3S+3) x (3S+3) input window once into
// registers (36 loads for 16 outputs at S = 1, instead of 144), so the kernel
// is bound by HBM rather than by the load pipe.  Patches are numbered across
// planes, so small planes keep every lane busy.  Each output sums its taps in
// (r, s) order, as depthwise_kernel does.
template <int S>
__global__ void __launch_bounds__(256) depthwise3x3_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ scale, float alpha,
                                                           const float* __restrict__ bias,
                                                           const float* __restrict__ residual, int flags,
                                                           float* __restrict__ y, DwGeom g, int patches_w,
                                                           int patches_plane, int patches) {
    constexpr int T = 4, WIN = 3 * S + 3;  // outputs per side, input window per side
    const bool bts = (flags & TBN_EPI_BIAS_THEN_SCALE) != 0, relu = (flags & TBN_EPI_RELU) != 0;
    const int stride = gridDim.x * blockDim.x;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < patches; idx += stride) {
        const int plane = idx / patches_plane;
        const int r0 = idx - plane * patches_plane;
        const int pr = r0 / patches_w;
        const int oh0 = pr * T, ow0 = (r0 - pr * patches_w) * T;
        const int m = plane % g.M, n = plane / g.M;
        const float* xp = x + (static_cast<int64_t>(n) * g.C + m / g.mult) * static_cast<int64_t>(g.H) * g.W;
        float wv[9];
#pragma unroll
        for (int t = 0; t < 9; ++t) wv[t] = w[m * 9 + t];
        const int ih0 = oh0 * S - g.ph, iw0 = ow0 * S - g.pw;
        bool col_ok[WIN];
#pragma unroll
        for (int j = 0; j < WIN; ++j) col_ok[j] = static_cast<unsigned>(iw0 + j) < static_cast<unsigned>(g.W);
        float acc[T][T] = {};
#pragma unroll
        for (int i = 0; i < WIN; ++i) {
            const int ih = ih0 + i;
            const bool row_ok = static_cast<unsigned>(ih) < static_cast<unsigned>(g.H);
            const float* row = xp + static_cast<int64_t>(ih) * g.W + iw0;
            float v[WIN];
#pragma unroll
            for (int j = 0; j < WIN; ++j) v[j] = (row_ok && col_ok[j]) ? row[j] : 0.0f;
#pragma unroll
            for (int a = 0; a < T; ++a) {
                const int r = i - a * S;  // kernel row this input row is for output row a
                if (r < 0 || r > 2) continue;
#pragma unroll
                for (int b = 0; b < T; ++b)
#pragma unroll
                    for (int s = 0; s < 3; ++s) acc[a][b] = fmaf(v[b * S + s], wv[r * 3 + s], acc[a][b]);
            }
        }
        const float mm = alpha * (scale ? scale[m] : 1.0f);
        const float bb = bias ? bias[m] : 0.0f;
        const float ea = bts ? bb : 0.0f, eb = bts ? 0.0f : bb;
        const int64_t ybase = static_cast<int64_t>(plane) * g.OH * g.OW;
#pragma unroll
        for (int a = 0; a < T; ++a) {
            const int oh = oh0 + a;
            if (oh >= g.OH) break;
#pragma unroll
            for (int b = 0; b < T; ++b) {
                const int ow = ow0 + b;
                if (ow >= g.OW) break;
                const int64_t o = ybase + static_cast<int64_t>(oh) * g.OW + ow;
                float val = (acc[a][b] + ea) * mm + eb;
                if (residual) val += residual[o];
                if (relu) val = val > 0.0f ? val : 0.0f;
                y[o] = val;
            }
        }
    }
}

// 3x3, padding 1, dilation 1, stride S in {1, 2}: a lane owns VEC
// consecutive output columns of kRowsTR consecutive output rows and reads the
// VEC*S input columns under them as vector loads, contiguous across the
// lanes of a row; the column to the left (and, at stride 1, to the right)
// comes from the neighbouring lane by shuffle, zero at the image edge.  So a
// wave reads whole rows once.  A wave holds 64 / (OW/VEC) row groups of the
// same or following planes.  Taps are summed in (r, s) order, as
// depthwise_kernel does.
constexpr int kRowsTR = 4;  // output rows per lane

template <int N>
struct FloatVec;
template <>
struct FloatVec<1> { using T = float; };
template <>
struct FloatVec<2> { using T = float2; };
template <>
struct FloatVec<4> { using T = float4; };

template <int VEC, int S>
__global__ void __launch_bounds__(256) depthwise3x3_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                                const float* __restrict__ scale, float alpha,
                                                                const float* __restrict__ bias,
                                                                const float* __restrict__ residual, int flags,
                                                                float* __restrict__ y, DwGeom g, int lanes_row,
                                                                int groups_per_wave, int tasks_plane,
                                                                int64_t tasks) {
    constexpr int IN = VEC * S;                 // input columns a lane loads per row
    constexpr int LV = IN < 4 ? IN : 4;         // floats per vector load
    constexpr int ROWS = (kRowsTR - 1) * S + 3;  // input rows per row group
    using V = typename FloatVec<LV>::T;
    using VO = typename FloatVec<VEC>::T;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rw = lane / lanes_row, q = lane - rw * lanes_row;
    const bool lane_ok = rw < groups_per_wave;
    const bool bts = (flags & TBN_EPI_BIAS_THEN_SCALE) != 0, relu = (flags & TBN_EPI_RELU) != 0;
    const int64_t waves_total = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t wv = static_cast<int64_t>(blockIdx.x) * 4 + wave; wv * groups_per_wave < tasks; wv += waves_total) {
        const int64_t task = wv * groups_per_wave + rw;
        const bool ok = lane_ok && task < tasks;
        const int64_t plane = ok ? task / tasks_plane : 0;
        const int oh0 = ok ? static_cast<int>(task - plane * tasks_plane) * kRowsTR : 0;
        const int m = static_cast<int>(plane % g.M);
        const int64_t n = plane / g.M;
        const float* xp = x + (n * g.C + m / g.mult) * static_cast<int64_t>(g.H) * g.W + IN * q;
        float wv9[9];
#pragma unroll
        for (int t = 0; t < 9; ++t) wv9[t] = ok ? w[m * 9 + t] : 0.0f;
        float acc[kRowsTR][VEC] = {};
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const int ih = oh0 * S - 1 + i;
            float v[IN];
#pragma unroll
            for (int e = 0; e < IN; ++e) v[e] = 0.0f;
            if (ok && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H)) {
                const V* src = reinterpret_cast<const V*>(xp + static_cast<int64_t>(ih) * g.W);
#pragma unroll
                for (int e = 0; e < IN / LV; ++e) {
                    const V t = src[e];
                    const float* f = reinterpret_cast<const float*>(&t);
#pragma unroll
                    for (int k = 0; k < LV; ++k) v[e * LV + k] = f[k];
                }
            }
            // in[0] = column IN*q - 1, in[1 + e] = column IN*q + e, in[IN + 1] = column IN*q + IN
            float in[IN + 2];
            in[0] = __shfl_up(v[IN - 1], 1);
            if (q == 0) in[0] = 0.0f;
#pragma unroll
            for (int e = 0; e < IN; ++e) in[1 + e] = v[e];
            in[IN + 1] = 0.0f;
            if (S == 1) {
                in[IN + 1] = __shfl_down(v[0], 1);
                if (q == lanes_row - 1) in[IN + 1] = 0.0f;
            }
#pragma unroll
            for (int a = 0; a < kRowsTR; ++a) {
                const int r = i - a * S;
                if (r < 0 || r > 2) continue;
#pragma unroll
                for (int c = 0; c < VEC; ++c)
#pragma unroll
                    for (int s2 = 0; s2 < 3; ++s2) acc[a][c] = fmaf(in[c * S + s2], wv9[r * 3 + s2], acc[a][c]);
            }
        }
        if (!ok) continue;
        const float mm = alpha * (scale ? scale[m] : 1.0f);
        const float bb = bias ? bias[m] : 0.0f;
        const float ea = bts ? bb : 0.0f, eb = bts ? 0.0f : bb;
        const int64_t ybase = plane * g.OH * static_cast<int64_t>(g.OW) + VEC * q;
#pragma unroll
        for (int a = 0; a < kRowsTR; ++a) {
            const int oh = oh0 + a;
            if (oh >= g.OH) break;
            const int64_t o = ybase + static_cast<int64_t>(oh) * g.OW;
            float out[VEC];
#pragma unroll
            for (int c = 0; c < VEC; ++c) out[c] = (acc[a][c] + ea) * mm + eb;
            if (residual) {
                const VO rv = *reinterpret_cast<const VO*>(residual + o);
                const float* rf = reinterpret_cast<const float*>(&rv);
#pragma unroll
                for (int c = 0; c < VEC; ++c) out[c] += rf[c];
            }
            if (relu) {
#pragma unroll
                for (int c = 0; c < VEC; ++c) out[c] = out[c] > 0.0f ? out[c] : 0.0f;
            }
            VO ov;
            float* of = reinterpret_cast<float*>(&ov);
#pragma unroll
            for (int c = 0; c < VEC; ++c) of[c] = out[c];
            *reinterpret_cast<VO*>(y + o) = ov;
        }
    }
}

template <int VEC, int S>
void launch_rows(const float* x, const float* w, const float* scale, float alpha, const float* bias,
                 const float* residual, int flags, float* y, const DwGeom& g, int lanes_row, int per_wave,
                 int tasks_plane, int64_t tasks, hipStream_t s) {
    const int64_t waves = tbn_hip::ceil_div(tasks, per_wave);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(tbn_hip::ceil_div(waves, 4), 1 << 20));
    hipLaunchKernelGGL((depthwise3x3_rows_kernel<VEC, S>), dim3(blocks), dim3(256), 0, s, x, w, scale, alpha, bias,
                       residual, flags, y, g, lanes_row, per_wave, tasks_plane, tasks);
}

// dst[n, dst_c0 + c, :] = src[n, src_c0 + c, :] for c < count; rows of `hw`
// floats, `vec` = 4 when every row start is 16-byte aligned.
template <int VEC>
__global__ void __launch_bounds__(256) copy_channels_kernel(const float* __restrict__ src, int64_t src_c,
                                                            int64_t src_c0, float* __restrict__ dst, int64_t dst_c,
                                                            int64_t dst_c0, int64_t count, int64_t hw_v,
                                                            int64_t total_v) {
    using V = typename std::conditional<VEC == 4, float4, float>::type;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total_v; i += stride) {
        const int64_t j = i % hw_v, row = i / hw_v;
        const int64_t c = row % count, n = row / count;
        const V* s = reinterpret_cast<const V*>(src) + ((n * src_c + src_c0 + c) * hw_v + j);
        V* d = reinterpret_cast<V*>(dst) + ((n * dst_c + dst_c0 + c) * hw_v + j);
        *d = *s;
    }
}

// y[n, c, i] = fma(x[n, c, i], k[c], t[c]), then ReLU: one block row per
// (n, c) plane (k, t uniform), VEC floats per lane.
template <int VEC>
__global__ void __launch_bounds__(256) channel_affine_kernel(const float* __restrict__ x, int64_t rows, int64_t c,
                                                             int64_t hw_v, const float* __restrict__ k,
                                                             const float* __restrict__ t, int relu,
                                                             float* __restrict__ y) {
    using V = typename std::conditional<VEC == 4, float4, float>::type;
    for (int64_t row = blockIdx.y; row < rows; row += gridDim.y) {
        const int64_t ch = row % c;
        const float kk = k[ch], tt = t[ch];
        const V* xr = reinterpret_cast<const V*>(x) + row * hw_v;
        V* yr = reinterpret_cast<V*>(y) + row * hw_v;
        for (int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < hw_v;
             j += static_cast<int64_t>(gridDim.x) * blockDim.x) {
            V v = xr[j];
            float* f = reinterpret_cast<float*>(&v);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                f[e] = fmaf(f[e], kk, tt);
                if (relu) f[e] = f[e] > 0.0f ? f[e] : 0.0f;
            }
            yr[j] = v;
        }
    }
}

unsigned grid_of(int64_t work, int64_t per_block) {
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(tbn_hip::ceil_div(work, per_block), 65536)));
}

}  // namespace

extern "C" {

int tbn_hip_conv2d_depthwise(const float* x, const tbn_conv2d_desc* desc, const float* w, const float* scale,
                             float alpha, const float* bias, const float* residual, int flags, float* y,
                             tbn_stream_t stream) {
    TBN_REQUIRE(desc != nullptr, TBN_INVALID_ARGUMENT, "null descriptor");
    const tbn_conv2d_desc& d = *desc;
    TBN_REQUIRE(d.n >= 0 && d.c > 0 && d.h > 0 && d.w > 0 && d.m > 0 && d.kh > 0 && d.kw > 0, TBN_INVALID_SHAPE,
                "invalid depthwise conv shape");
    TBN_REQUIRE(d.m % d.c == 0, TBN_INVALID_SHAPE, "depthwise conv: output channels must be a multiple of C");
    TBN_REQUIRE(d.sh > 0 && d.sw > 0 && d.dh > 0 && d.dw > 0 && d.ph >= 0 && d.pw >= 0, TBN_INVALID_ARGUMENT,
                "invalid stride, padding or dilation");
    TBN_REQUIRE((flags & ~(TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE)) == 0, TBN_INVALID_ARGUMENT,
                "depthwise conv: unsupported epilogue flags");
    const int64_t OH = (d.h + 2 * d.ph - d.dh * (d.kh - 1) - 1) / d.sh + 1;
    const int64_t OW = (d.w + 2 * d.pw - d.dw * (d.kw - 1) - 1) / d.sw + 1;
    TBN_REQUIRE(OH > 0 && OW > 0, TBN_INVALID_SHAPE, "depthwise conv: empty output");
    const int64_t lim = 1LL << 30;
    TBN_REQUIRE(d.h * d.w < lim && OH * OW < lim && d.kh * d.kw < lim && d.m < lim && d.c < lim &&
                    std::max({d.sh, d.sw, d.ph, d.pw, d.dh, d.dw}) < (1LL << 20) &&
                    (OH - 1) * d.sh + (d.kh - 1) * d.dh < lim && (OW - 1) * d.sw + (d.kw - 1) * d.dw < lim,
                TBN_INVALID_SHAPE, "depthwise conv: dimensions too large");
    if (d.n == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && w && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    DwGeom g;
    g.C = static_cast<int>(d.c); g.H = static_cast<int>(d.h); g.W = static_cast<int>(d.w);
    g.M = static_cast<int>(d.m); g.mult = static_cast<int>(d.m / d.c);
    g.OH = static_cast<int>(OH); g.OW = static_cast<int>(OW);
    g.kh = static_cast<int>(d.kh); g.kw = static_cast<int>(d.kw);
    g.sh = static_cast<int>(d.sh); g.sw = static_cast<int>(d.sw);
    g.ph = static_cast<int>(d.ph); g.pw = static_cast<int>(d.pw);
    g.dh = static_cast<int>(d.dh); g.dw = static_cast<int>(d.dw);
    g.planes = d.n * d.m;
    g.tiles_w = static_cast<int>(tbn_hip::ceil_div(OW, kTileW));
    const int64_t tiles = g.tiles_w * tbn_hip::ceil_div(OH, kTileH);
    TBN_REQUIRE(tiles < lim, TBN_INVALID_SHAPE, "depthwise conv: output plane too large");
    g.tiles = static_cast<int>(tiles);
    // the row kernel: 3x3, padding 1, stride 1 (OW = W) or 2 with an even W
    // (OW = W/2), VEC output columns per lane with OW / VEC lanes per row
    if (d.kh == 3 && d.kw == 3 && d.ph == 1 && d.pw == 1 && d.dh == 1 && d.dw == 1 && d.sh == d.sw &&
        (d.sh == 1 || (d.sh == 2 && d.w % 2 == 0))) {
        const int S = static_cast<int>(d.sh);
        const int vec = OW % 4 == 0 ? 4 : (OW % 2 == 0 ? 2 : 1);
        const int lv = std::min(4, vec * S);
        const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                                reinterpret_cast<uintptr_t>(residual);
        if (OW / vec <= 64 && align % (4 * static_cast<uintptr_t>(std::max(lv, vec))) == 0) {
            const int lanes_row = static_cast<int>(OW / vec);
            const int per_wave = 64 / lanes_row;
            const int64_t tasks_plane = tbn_hip::ceil_div(OH, kRowsTR);
            const int64_t tasks = g.planes * tasks_plane;
            hipStream_t st = tbn_hip::stream_of(stream);
            auto go = [&](auto vec_c, auto s_c) {
                launch_rows<decltype(vec_c)::value, decltype(s_c)::value>(x, w, scale, alpha, bias, residual, flags,
                                                                          y, g, lanes_row, per_wave,
                                                                          int(tasks_plane), tasks, st);
            };
            using I1 = std::integral_constant<int, 1>;
            using I2 = std::integral_constant<int, 2>;
            using I4 = std::integral_constant<int, 4>;
            if (S == 1) {
                if (vec == 4) go(I4{}, I1{});
                else if (vec == 2) go(I2{}, I1{});
                else go(I1{}, I1{});
            } else {
                if (vec == 4) go(I4{}, I2{});
                else if (vec == 2) go(I2{}, I2{});
                else go(I1{}, I2{});
            }
            return tbn_hip::check_launch("conv2d_depthwise");
        }
    }
    const int64_t pw4 = tbn_hip::ceil_div(OW, 4), pplane = pw4 * tbn_hip::ceil_div(OH, 4);
    const int64_t patches = g.planes * pplane;
    // stride 2 on wide planes: the generic kernel's 64-column rows coalesce
    // better than 4-column patches 8 floats apart (78 vs 95 us at 112x112)
    if (d.kh == 3 && d.kw == 3 && d.dh == 1 && d.dw == 1 && d.sh == d.sw && (d.sh == 1 || (d.sh == 2 && OW <= 32)) &&
        patches < (1LL << 31)) {
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(tbn_hip::ceil_div(patches, 256), 1 << 20));
        if (d.sh == 1)
            hipLaunchKernelGGL(depthwise3x3_kernel<1>, dim3(blocks), dim3(256), 0, tbn_hip::stream_of(stream), x, w,
                               scale, alpha, bias, residual, flags, y, g, int(pw4), int(pplane), int(patches));
        else
            hipLaunchKernelGGL(depthwise3x3_kernel<2>, dim3(blocks), dim3(256), 0, tbn_hip::stream_of(stream), x, w,
                               scale, alpha, bias, residual, flags, y, g, int(pw4), int(pplane), int(patches));
        return tbn_hip::check_launch("conv2d_depthwise");
    }
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(tiles, 65535)),
                    static_cast<unsigned>(std::min<int64_t>(g.planes, 65535)));
    hipLaunchKernelGGL(depthwise_kernel, grid, dim3(256), 0, tbn_hip::stream_of(stream), x, w, scale, alpha, bias,
                       residual, flags, y, g);
    return tbn_hip::check_launch("conv2d_depthwise");
}

int tbn_hip_copy_channels(const float* src, int64_t n, int64_t src_c, int64_t src_c0, int64_t count, int64_t hw,
                          float* dst, int64_t dst_c, int64_t dst_c0, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0 && count >= 0 && hw >= 0 && src_c0 >= 0 && dst_c0 >= 0 && src_c0 + count <= src_c &&
                    dst_c0 + count <= dst_c,
                TBN_INVALID_SHAPE, "copy_channels: channel range outside the tensor");
    const int64_t total = n * count * hw;
    if (total == 0) return tbn_hip::ok();
    TBN_REQUIRE(src && dst, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const bool vec4 = hw % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(dst) % 16 == 0;
    if (vec4)
        hipLaunchKernelGGL(copy_channels_kernel<4>, dim3(grid_of(total / 4, 256)), dim3(256), 0,
                           tbn_hip::stream_of(stream), src, src_c, src_c0, dst, dst_c, dst_c0, count, hw / 4,
                           total / 4);
    else
        hipLaunchKernelGGL(copy_channels_kernel<1>, dim3(grid_of(total, 256)), dim3(256), 0,
                           tbn_hip::stream_of(stream), src, src_c, src_c0, dst, dst_c, dst_c0, count, hw, total);
    return tbn_hip::check_launch("copy_channels");
}

int tbn_hip_channel_affine(const float* x, int64_t n, int64_t c, int64_t hw, const float* k, const float* t,
                           int flags, float* y, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0 && c > 0 && hw >= 0, TBN_INVALID_SHAPE, "channel_affine: invalid shape");
    TBN_REQUIRE((flags & ~TBN_EPI_RELU) == 0, TBN_INVALID_ARGUMENT, "channel_affine: unsupported flags");
    const int64_t total = n * c * hw;
    if (total == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && k && t && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const bool vec4 = hw % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(y) % 16 == 0;
    const int64_t hw_v = vec4 ? hw / 4 : hw, rows = n * c;
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(tbn_hip::ceil_div(hw_v, 256), 64)),
                    static_cast<unsigned>(std::min<int64_t>(rows, 65535)));
    const int relu = (flags & TBN_EPI_RELU) ? 1 : 0;
    if (vec4)
        hipLaunchKernelGGL(channel_affine_kernel<4>, grid, dim3(256), 0, tbn_hip::stream_of(stream), x, rows, c, hw_v,
                           k, t, relu, y);
    else
        hipLaunchKernelGGL(channel_affine_kernel<1>, grid, dim3(256), 0, tbn_hip::stream_of(stream), x, rows, c, hw_v,
                           k, t, relu, y);
    return tbn_hip::check_launch("channel_affine");
}

}  // extern "C"
