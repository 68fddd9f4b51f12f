// Small convolutions (LeNet-sized layers): each block stages one image, zero
// padded, and the weights of the channels it covers, decoded to fp32, in LDS;
// each thread computes one conv output with fp32 FMAs over k = (c, r, s) in
// order, then the conv epilogue (scale, bias, residual, ReLU); the optional
// 2x2 max pool reduces four neighbouring lanes.  For layers
// this small the MFMA tile engine spends its time in staging latency (LeNet's
// 6 -> 16 channel 5x5 conv took 20 us in one block); here a layer is one round
// of loads and at most a few hundred FMAs per thread, spread over
// ceil(outputs / 256) blocks per image.
//
// Which layers take this path depends only on one image's shape (input and
// output sizes), never on the batch, so a sample's result does not depend on
// the batch it runs in.
#include "common.hpp"
#include "conv_common.hpp"

namespace {

constexpr int kSmallThreads = 256;  // outputs per block (pooled outputs when pooling)
constexpr int kSmallX = 8192;       // floats of one zero-padded image staged in LDS
constexpr int kSmallW = 8192;       // floats of decoded weights staged in LDS
constexpr int kSmallK = 4096;       // taps per output channel (offset table)

struct SmallGeom {
    int C, H, W, M, K, kh, kw, sh, sw, ph, pw, dh, dw;
    int Hp, Wp;      // the zero-padded image
    int OH, OW;
    int pool;
    int plane;       // items per channel: OH*OW, or 4 per pooled output when pooling
    int PW;          // pooled width
    int Kp;          // LDS row stride of the decoded weights: ceil4(K)
    int blocks_img;  // blocks per image
};

// Weight of output channel m at k: fp32 row-major [M, K]; binary: bit k of
// column m (1 = -1, 0 = +1); ternary: 2-bit code k of column m (00 = -1,
// 01 = 0, 10 = +1, 11 = 0).
template <int WMODE>
__device__ __forceinline__ float weight_at(const void* w, int64_t col_bytes, int K, int m, int k) {
    if constexpr (WMODE == 0) {
        return static_cast<const float*>(w)[static_cast<int64_t>(m) * K + k];
    } else if constexpr (WMODE == 1) {
        const uint8_t b = static_cast<const uint8_t*>(w)[static_cast<int64_t>(m) * col_bytes + (k >> 3)];
        return ((b >> (k & 7)) & 1) ? -1.0f : 1.0f;
    } else {
        const uint8_t b = static_cast<const uint8_t*>(w)[static_cast<int64_t>(m) * col_bytes + (k >> 2)];
        const int code = (b >> (2 * (k & 3))) & 3;
        return code == 0 ? -1.0f : (code == 2 ? 1.0f : 0.0f);
    }
}

// Stages count values into LDS, four global loads in flight per thread:
// get(i) -> value i, put(i, v) stores it.
template <class Get, class Put>
__device__ __forceinline__ void stage4(int count, Get get, Put put) {
    for (int base = 0; base < count; base += 4 * kSmallThreads) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = base + j * kSmallThreads + static_cast<int>(threadIdx.x);
            v[j] = i < count ? get(i) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = base + j * kSmallThreads + static_cast<int>(threadIdx.x);
            if (i < count) put(i, v[j]);
        }
    }
}

// Decoded weights of columns [m_lo, m_lo + mb) into ws[ml * Kp + k]: fp32
// values four loads per thread at a time, packed columns one byte (8 binary
// or 4 ternary weights) per load.
template <int WMODE>
__device__ __forceinline__ void stage_weights(const void* w, int64_t col_bytes, int K, int Kp, int m_lo, int mb,
                                              float* ws) {
    if constexpr (WMODE == 0) {
        const float* wf = static_cast<const float*>(w) + static_cast<int64_t>(m_lo) * K;
        stage4(mb * K, [&](int i) { return wf[i]; },
               [&](int i, float v) {
                   const int ml = i / K;
                   ws[ml * Kp + (i - ml * K)] = v;
               });
    } else {
        constexpr int per = WMODE == 1 ? 8 : 4;
        const int bpc = (K + per - 1) / per;
        const uint8_t* wb = static_cast<const uint8_t*>(w);
        stage4(mb * bpc,
               [&](int i) {
                   const int ml = i / bpc;
                   return static_cast<float>(wb[static_cast<int64_t>(m_lo + ml) * col_bytes + (i - ml * bpc)]);
               },
               [&](int i, float v) {
                   const int ml = i / bpc, j = i - ml * bpc;
                   const unsigned byte = static_cast<unsigned>(v);
                   float* dst = ws + ml * Kp + j * per;
                   const int n = min(per, K - j * per);
                   for (int q = 0; q < n; ++q) {
                       if constexpr (WMODE == 1) {
                           dst[q] = ((byte >> q) & 1u) ? -1.0f : 1.0f;
                       } else {
                           const unsigned code = (byte >> (2 * q)) & 3u;
                           dst[q] = code == 0 ? -1.0f : (code == 2 ? 1.0f : 0.0f);
                       }
                   }
               });
    }
}

// Block b of image n computes items [256*b, 256*b + 256) of the image's
// channel-major (m, position) list, one conv output per thread; with the
// fused pool the positions run window by window, lanes 4t .. 4t+3 holding
// (oh, ow), (oh, ow+1), (oh+1, ow), (oh+1, ow+1).  The image is staged with
// its zero padding, so tap k of the output whose window starts at `base` is
// xs[base + offs[k]] with no bounds test, and padded taps contribute 0*w as
// the unfolded-patch product does.
template <int WMODE>
__global__ void __launch_bounds__(kSmallThreads)
small_conv_kernel(const float* __restrict__ x, SmallGeom g, const void* __restrict__ w, int64_t col_bytes,
                  const float* __restrict__ scale, float alpha, const float* __restrict__ bias,
                  const float* __restrict__ residual, int flags, float* __restrict__ y) {
    __shared__ float xs[kSmallX];
    __shared__ __align__(16) float ws[kSmallW];
    __shared__ __align__(16) int offs[kSmallK];
    const int n = blockIdx.x / g.blocks_img;
    const int i0 = (blockIdx.x - n * g.blocks_img) * kSmallThreads;
    const int i_end = min(i0 + kSmallThreads, g.M * g.plane);
    const int m_lo = i0 / g.plane;
    const int mb = (i_end - 1) / g.plane - m_lo + 1;

    // this thread's output and its epilogue operands, loaded ahead of staging
    const int i = i0 + static_cast<int>(threadIdx.x);
    const bool live = i < i_end;
    const int m = live ? i / g.plane : m_lo, pos = live ? i - m * g.plane : 0;
    int oh, ow;
    if (g.pool) {
        const int win = pos >> 2, q = pos & 3;
        oh = 2 * (win / g.PW) + (q >> 1);
        ow = 2 * (win % g.PW) + (q & 1);
    } else {
        oh = pos / g.OW;
        ow = pos - oh * g.OW;
    }
    const float mult = scale ? alpha * scale[m] : alpha;
    const float b = bias ? bias[m] : 0.0f;
    const float rv = residual ? residual[(static_cast<int64_t>(n) * g.M + m) * (g.OH * g.OW) + oh * g.OW + ow] : 0.0f;

    const int pp = g.Hp * g.Wp;
    const float* xn = x + static_cast<int64_t>(n) * g.C * g.H * g.W;
    stage4(g.C * pp,
           [&](int i) {
               const int c = i / pp, rem = i - c * pp;
               const int h = rem / g.Wp - g.ph, wc = rem % g.Wp - g.pw;
               return (static_cast<unsigned>(h) < static_cast<unsigned>(g.H) &&
                       static_cast<unsigned>(wc) < static_cast<unsigned>(g.W))
                          ? xn[(c * g.H + h) * g.W + wc]
                          : 0.0f;
           },
           [&](int i, float v) { xs[i] = v; });
    stage_weights<WMODE>(w, col_bytes, g.K, g.Kp, m_lo, mb, ws);
    const int taps = g.kh * g.kw;
    for (int k = threadIdx.x; k < g.K; k += kSmallThreads) {
        const int c = k / taps, rs = k - c * taps;
        const int r = rs / g.kw, sx = rs - r * g.kw;
        offs[k] = c * pp + r * g.dh * g.Wp + sx * g.dw;
    }
    __syncthreads();

    if (!live) return;  // past the block's only barrier; pooled windows leave whole
    const float* x0 = xs + oh * g.sh * g.Wp + ow * g.sw;
    const float* wr = ws + (m - m_lo) * g.Kp;
    float acc = 0.0f;
    int k = 0;
#pragma unroll 4
    for (; k + 4 <= g.K; k += 4) {
        const int4 o = *reinterpret_cast<const int4*>(offs + k);
        const float4 w4 = *reinterpret_cast<const float4*>(wr + k);
        acc = fmaf(x0[o.x], w4.x, acc);
        acc = fmaf(x0[o.y], w4.y, acc);
        acc = fmaf(x0[o.z], w4.z, acc);
        acc = fmaf(x0[o.w], w4.w, acc);
    }
    for (; k < g.K; ++k) acc = fmaf(x0[offs[k]], wr[k], acc);

    float v = (flags & TBN_EPI_BIAS_THEN_SCALE) ? (acc + b) * mult : acc * mult + b;
    if (residual) v += rv;
    if (flags & TBN_EPI_RELU) v = v > 0.0f ? v : 0.0f;
    if (g.pool) {
        // max over the window as the other conv kernels reduce it: the row
        // pairs, then their maxima
        v = fmaxf(v, __shfl_xor(v, 1));
        v = fmaxf(v, __shfl_xor(v, 2));
        if ((pos & 3) == 0) y[(static_cast<int64_t>(n) * g.M + m) * (g.plane >> 2) + (pos >> 2)] = v;
    } else {
        y[(static_cast<int64_t>(n) * g.M + m) * g.plane + pos] = v;
    }
}

struct SmallShape {
    int64_t K, Hp, Wp, OH, OW, plane;
};

SmallShape small_shape(const tbn_conv2d_desc* d, bool pool) {
    SmallShape s;
    s.K = d->c * d->kh * d->kw;
    s.Hp = d->h + 2 * d->ph;
    s.Wp = d->w + 2 * d->pw;
    s.OH = (s.Hp - d->dh * (d->kh - 1) - 1) / d->sh + 1;
    s.OW = (s.Wp - d->dw * (d->kw - 1) - 1) / d->sw + 1;
    s.plane = pool ? 4 * (s.OH / 2) * (s.OW / 2) : s.OH * s.OW;
    return s;
}

}  // namespace

namespace tbn_hip {

// The zero-padded image and the taps of the channels one block touches fit
// the LDS staging, and the layer has at most 16384 outputs per image.  Which
// layers qualify depends on one image's shape only.
bool conv_small_supported(const tbn_conv2d_desc* d) {
    if (d->n >= (1LL << 20) || d->c <= 0 || d->m <= 0) return false;
    const SmallShape s = small_shape(d, false);
    if (s.OH <= 0 || s.OW <= 0 || d->m * s.OH * s.OW > 16384) return false;
    if (d->c * s.Hp * s.Wp > kSmallX || s.K > kSmallK) return false;
    // 256 consecutive items span at most 255/plane + 2 channels (the pooled
    // plane, 4 items per pooled output, is the smaller one)
    const int64_t plane = std::max<int64_t>(1, 4 * (s.OH / 2) * (s.OW / 2));
    return std::min<int64_t>(d->m, 255 / plane + 2) * ((s.K + 3) / 4 * 4) <= kSmallW;
}

// weights: 0 fp32 [M, K], 1 binary columns, 2 ternary columns (col_bytes each).
int conv_small_run(int wmode, const float* x, const tbn_conv2d_desc* d, const void* w, int64_t col_bytes,
                   const float* scale, float alpha, const float* bias, const float* residual, int flags, float* y,
                   hipStream_t s) {
    const bool pool = (flags & TBN_EPI_MAXPOOL2X2) != 0;
    const SmallShape sh = small_shape(d, pool);
    SmallGeom g;
    g.C = int(d->c); g.H = int(d->h); g.W = int(d->w); g.M = int(d->m);
    g.kh = int(d->kh); g.kw = int(d->kw); g.sh = int(d->sh); g.sw = int(d->sw);
    g.ph = int(d->ph); g.pw = int(d->pw); g.dh = int(d->dh); g.dw = int(d->dw);
    g.K = int(sh.K);
    g.Kp = (g.K + 3) / 4 * 4;
    g.Hp = int(sh.Hp); g.Wp = int(sh.Wp);
    g.OH = int(sh.OH); g.OW = int(sh.OW);
    g.pool = pool ? 1 : 0;
    g.plane = int(sh.plane);
    g.PW = int(sh.OW / 2);
    if (g.plane == 0 || d->n == 0) return ok();
    g.blocks_img = int(ceil_div(int64_t(g.M) * g.plane, kSmallThreads));
    const int64_t blocks = d->n * g.blocks_img;
    TBN_REQUIRE(blocks < (1LL << 31), TBN_INVALID_SHAPE, "small conv: too many images");
    if (wmode == 0)
        hipLaunchKernelGGL(small_conv_kernel<0>, dim3(static_cast<unsigned>(blocks)), dim3(kSmallThreads), 0, s, x, g,
                           w, col_bytes, scale, alpha, bias, residual, flags, y);
    else if (wmode == 1)
        hipLaunchKernelGGL(small_conv_kernel<1>, dim3(static_cast<unsigned>(blocks)), dim3(kSmallThreads), 0, s, x, g,
                           w, col_bytes, scale, alpha, bias, residual, flags, y);
    else
        hipLaunchKernelGGL(small_conv_kernel<2>, dim3(static_cast<unsigned>(blocks)), dim3(kSmallThreads), 0, s, x, g,
                           w, col_bytes, scale, alpha, bias, residual, flags, y);
    return check_launch("conv2d (small)");
}

}  // namespace tbn_hip
