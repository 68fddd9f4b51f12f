// Geometry, output-position enumeration and fused epilogue shared by the
// implicit-GEMM convolution kernels (conv.hip: im2col gathered from NCHW fp32;
// conv_nhwc.hip: split bf16 NHWC activations).  Output channels are the MFMA
// rows, output positions the MFMA columns.
#pragma once

#include <string>

#include "common.hpp"
#include "mfma_core.hpp"

namespace tbnk {

struct ConvGeom {
    int C, H, W;
    int kh, kw, sh, sw, ph, pw, dh, dw;
    int K;      // C * kh * kw
    int Q;      // number of computed output positions
    int OW, OHW;  // unpooled output plane
    int pool;   // positions enumerated by 2x2 window
    int PW, PHW;  // pooled output plane
};

// Decomposes a position index into (n, oh, ow) of the conv output.
__device__ __forceinline__ void position_coords(const ConvGeom& g, int q, int& n, int& oh, int& ow) {
    if (g.pool) {
        const int per_image = g.PHW * 4;
        n = q / per_image;
        const int rem = q - n * per_image;
        const int win = rem >> 2;
        const int ph = win / g.PW;
        const int pw = win - ph * g.PW;
        oh = 2 * ph + ((rem >> 1) & 1);
        ow = 2 * pw + (rem & 1);
    } else {
        n = q / g.OHW;
        const int rem = q - n * g.OHW;
        oh = rem / g.OW;
        ow = rem - oh * g.OW;
    }
}

// y[n, m, oh, ow] = relu?( acc*alpha*s[m] + b[m] ) (or (acc + b[m])*alpha*s[m]),
// optionally max-pooled over 2x2 windows held by lanes 4t .. 4t+3.
struct ConvEpi {
    float* y;
    int M;  // output channels
    ConvGeom g;
    const float* scale;
    float alpha;
    const float* bias;
    const float* residual;  // same layout as y (unpooled only), may be null
    int flags;

    template <class Cfg>
    __device__ __forceinline__ void apply(f32x16_t (&acc)[Cfg::FR][Cfg::FC], int row0, int col0,
                                          int lane) const {
        const bool pool = g.pool != 0;
        const int plane = pool ? g.PHW : g.OHW;
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            const int q = col0 + frag_out_col(j, lane);
            const bool valid_q = q < g.Q;
            int64_t out_base = 0;
            if (valid_q) {
                if (pool) {
                    const int per_image = g.PHW * 4;
                    const int n = q / per_image;
                    const int win = (q - n * per_image) >> 2;
                    out_base = static_cast<int64_t>(n) * M * plane + win;
                } else {
                    const int n = q / g.OHW;
                    out_base = static_cast<int64_t>(n) * M * plane + (q - n * g.OHW);
                }
            }
#pragma unroll
            for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = row0 + frag_out_row(i, e, lane);
                    float v = acc[i][j][e];
                    if (m < M) {
                        const float mult = scale ? alpha * scale[m] : alpha;
                        const float b = bias ? bias[m] : 0.0f;
                        v = (flags & TBN_EPI_BIAS_THEN_SCALE) ? (v + b) * mult : v * mult + b;
                        if (residual && valid_q) v += residual[out_base + static_cast<int64_t>(m) * plane];
                        if (flags & TBN_EPI_RELU) v = v > 0.0f ? v : 0.0f;
                    }
                    if (pool) {
                        v = fmaxf(v, __shfl_xor(v, 1));
                        v = fmaxf(v, __shfl_xor(v, 2));
                    }
                    if (m < M && valid_q && (!pool || (lane & 3) == 0))
                        y[out_base + static_cast<int64_t>(m) * plane] = v;
                }
        }
    }
};

inline int make_geom(const tbn_conv2d_desc* d, int flags, ConvGeom& g) {
    TBN_REQUIRE(d != nullptr, TBN_INVALID_ARGUMENT, "conv descriptor is null");
    TBN_REQUIRE(d->n >= 0 && d->c > 0 && d->h > 0 && d->w > 0 && d->m > 0, TBN_INVALID_SHAPE,
                "conv input/output dimensions must be positive");
    TBN_REQUIRE(d->kh > 0 && d->kw > 0 && d->sh > 0 && d->sw > 0 && d->dh > 0 && d->dw > 0 &&
                    d->ph >= 0 && d->pw >= 0,
                TBN_INVALID_ARGUMENT, "invalid kernel/stride/padding/dilation");
    const int64_t OH = (d->h + 2 * d->ph - d->dh * (d->kh - 1) - 1) / d->sh + 1;
    const int64_t OW = (d->w + 2 * d->pw - d->dw * (d->kw - 1) - 1) / d->sw + 1;
    TBN_REQUIRE(OH > 0 && OW > 0, TBN_INVALID_SHAPE,
                "invalid output dimensions: " + std::to_string(OH) + "x" + std::to_string(OW));
    const int64_t K = d->c * d->kh * d->kw;
    const int64_t xsize = d->n * d->c * d->h * d->w;
    TBN_REQUIRE(K * d->kh * d->kw < (1LL << 32) && xsize < (1LL << 40) && d->h < (1 << 30) &&
                    d->w < (1 << 30),
                TBN_INVALID_SHAPE, "convolution too large");
    g.C = int(d->c); g.H = int(d->h); g.W = int(d->w);
    g.kh = int(d->kh); g.kw = int(d->kw); g.sh = int(d->sh); g.sw = int(d->sw);
    g.ph = int(d->ph); g.pw = int(d->pw); g.dh = int(d->dh); g.dw = int(d->dw);
    g.K = int(K);
    g.OW = int(OW);
    g.OHW = int(OH * OW);
    g.pool = (flags & TBN_EPI_MAXPOOL2X2) ? 1 : 0;
    if (g.pool) {
        const int64_t PH = OH / 2, PW = OW / 2;
        TBN_REQUIRE(PH > 0 && PW > 0, TBN_INVALID_SHAPE, "2x2 max pool needs an output of at least 2x2");
        g.PW = int(PW);
        g.PHW = int(PH * PW);
        TBN_REQUIRE(d->n * PH * PW * 4 < (1LL << 31), TBN_INVALID_SHAPE, "too many output positions");
        g.Q = int(d->n * PH * PW * 4);
    } else {
        g.PW = 0;
        g.PHW = 0;
        TBN_REQUIRE(d->n * OH * OW < (1LL << 31), TBN_INVALID_SHAPE, "too many output positions");
        g.Q = int(d->n * OH * OW);
    }
    return TBN_SUCCESS;
}


}  // namespace tbnk

namespace tbn_hip {
// The patch conv path (conv_patch.hip): whether it handles `desc`, and a run
// fed with reference-layout packed weights, re-ordered into the stream
// workspace for the call (a stream-ordered temporary while the stream
// captures), or, when `scratch` is given, into its first bytes with the
// split-K partial sums after them (no allocation at all).
bool conv_patch_supported(const tbn_conv2d_desc* desc);
int conv_patch_from_reference(int weights, const float* x, const tbn_conv2d_desc* desc, const uint8_t* packed,
                              int64_t K_pad, int64_t N_pad, const float* scale, float alpha, const float* bias,
                              const float* residual, int flags, float* y, hipStream_t s, void* scratch = nullptr,
                              int64_t scratch_bytes = 0);
// Scratch bytes conv_patch_from_reference needs with `scratch` given: the
// conv-layout weights (rounded up to 256 bytes) plus the split-K partial sums;
// -1 when make_patch_geom rejects the geometry.
int64_t conv_patch_scratch_bytes(int weights, const tbn_conv2d_desc* desc, int flags);
// The fp32 stem path (conv_stem.hip): few input channels, 7-wide kernels,
// stride 2 along W, <= 64 output channels, bias + optional ReLU.
bool conv_stem_supported(const tbn_conv2d_desc* desc, int flags);
int conv_stem_run(const float* x, const tbn_conv2d_desc* desc, const float* w, const float* bias, int flags,
                  float* y, hipStream_t s);
// Small layers (conv_small.hip): one image and a channel group per block,
// staged in LDS, fp32 FMAs; chosen from one image's shape only.
bool conv_small_supported(const tbn_conv2d_desc* desc);
// wmode: 0 fp32 weights [M, K], 1 binary columns, 2 ternary columns (col_bytes each).
int conv_small_run(int wmode, const float* x, const tbn_conv2d_desc* desc, const void* w, int64_t col_bytes,
                   const float* scale, float alpha, const float* bias, const float* residual, int flags, float* y,
                   hipStream_t s);
}  // namespace tbn_hip
