// TBN-mode convolution: the reference Session's quantized conv arithmetic
// (tbn-runtime/include/tbn/runtime/model.hpp:482-557 with
// impl::im2col_ternary_packed, conv2d.cpp:511-601, and conv2d_binary,
// conv2d.cpp:220-316, whose qlinear_matmul_binary ternarizes the im2col
// matrix): every input tap is ternarized at (lo, hi) -- v < lo -> -1,
// v > hi -> +1, else 0; taps outside the image are 0 -- and multiplied by
// the +-1 weights in exact integer arithmetic, then y = float(C) * alpha*s[m]
// + b[m] or (float(C) + b[m]) * alpha*s[m], then residual, ReLU, 2x2 max
// pool as the following nodes compute them.
//
// Implicit GEMM on the fp4 matrix cores: no im2col matrix and no bit planes
// are materialised.  A block owns one tile of TR x TC output pixels of one
// image and WV fragments of 32 output channels (one wave each).  K runs over
// chunks of 64 input channels; for each chunk the block stages the input
// patch the tile needs straight from NCHW fp32 into LDS, ternarized on the
// way into fp4 pixel records (64 codes, 32 bytes each), and every tap of the
// kernel is then one MFMA k-step (32 x 32 x 64) read from the same records.
// The weights are pre-packed once per layer in MFMA fragment order (1 KB per
// fragment and k-step, one 16-byte load per lane) and read from L2.
// MFMA rows are output channels and columns pixels, so a fragment's 32
// lanes store 32 consecutive pixels of a channel plane.
#include <algorithm>
#include <cstdio>
#include <string>

#include "common.hpp"
#include "tbn_f4.hpp"

namespace {

using namespace tbnk;

constexpr int kChunk = 64;             // input channels per k-step
constexpr int kRec = 32;               // LDS bytes per pixel record: 64 fp4 codes
constexpr uint32_t kOutside = 0x80000000u;
constexpr int kMaxLds = 64 * 1024;     // patch bytes a block may stage

struct TbnGeom {
    int N, C, H, W, M, kh, kw, sh, sw, ph, pw, dh, dw;
    int OH, OW;            // conv output plane
    int pool;              // fused 2x2 / 2 max pool (floor mode)
    int YH, YW;            // stored output plane
    int chunks, taps, ksteps, mfrags;
    int TR, TC;            // conv output rows / columns per tile (both even when pooled)
    int tiles_r, tiles_c;  // tiles per image
    int PR, PC;            // patch rows / columns (input pixels)
    int FC;                // pixel fragments (32 pixels) per tile
    int WV;                // waves per block, one 32-channel fragment each
    int mblocks;           // channel blocks
    int64_t blocks() const { return static_cast<int64_t>(N) * tiles_r * tiles_c * mblocks; }
    int lds() const { return PR * PC * kRec; }
};

struct TbnConvArgs {
    const float* x;
    const uint8_t* w4;
    float* y;
    const float* scale;     // per output channel, or null
    float alpha;
    const float* bias;      // per output channel, or null
    const float* residual;  // same layout as y, or null
    int flags;
    float lo, hi;
};

// v from lane (lane & ~3) | perm[lane & 3] of the same quad (DPP quad_perm).
template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// One output of the epilogue, every operation rounded on its own (no fused
// multiply-add), in the reference's order: float(C) * s + b (conv2d_binary
// and its scaled variants) or (float(C) + b) * s (the Session's cached conv),
// then + the residual (the following Add node).
__device__ __forceinline__ float epilogue_value(float acc, float mult, float bb, bool bts, const float* res) {
#pragma clang fp contract(off)
    float v = bts ? (acc + bb) * mult : acc * mult + bb;
    if (res) v = v + *res;
    return v;
}

// Tile pixel p (0 .. 32 FC) -> conv output offsets (r, c) inside the tile:
// row-major, or by 2 x 2 window when pooled (p / 4 a window, p % 4 its
// position: bit 0 the column, bit 1 the row).
__device__ __forceinline__ void tile_pixel(const TbnGeom& g, int p, int& r, int& c) {
    if (g.pool) {
        const int q = p >> 2, qc = g.TC >> 1;
        const int pr = q / qc;
        r = 2 * pr + ((p >> 1) & 1);
        c = 2 * (q - pr * qc) + (p & 1);
    } else {
        r = p / g.TC;
        c = p - r * g.TC;
    }
}

template <int FC>
__global__ void __launch_bounds__(256) tbn_conv_kernel(TbnGeom g, TbnConvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;

    // block -> (image, tile, channel block); the channel blocks of one tile
    // are consecutive in b, and consecutive b run on one XCD (blocks are
    // dealt round-robin over the 8 XCDs), so a patch is fetched into one L2
    int b = blockIdx.x;
    const int total = gridDim.x;
    if (total % 8 == 0) b = (b % 8) * (total / 8) + b / 8;
    const int mb = b % g.mblocks;
    int t = b / g.mblocks;
    const int per_image = g.tiles_r * g.tiles_c;
    const int n = t / per_image;
    t -= n * per_image;
    const int trow = t / g.tiles_c;
    const int oh0 = trow * g.TR, ow0 = (t - trow * g.tiles_c) * g.TC;
    const int ih0 = oh0 * g.sh - g.ph, iw0 = ow0 * g.sw - g.pw;
    const int mf = mb * g.WV + wave;
    const bool active = mf < g.mfrags;

    // this lane's pixel in each fragment: its record in the patch (tap 0)
    const int oh_lim = g.pool ? 2 * g.YH : g.OH, ow_lim = g.pool ? 2 * g.YW : g.OW;
    int rec[FC];
    bool ok[FC];
    int pr_[FC], pc_[FC];
#pragma unroll
    for (int j = 0; j < FC; ++j) {
        int r, c;
        tile_pixel(g, j * 32 + (lane & 31), r, c);
        ok[j] = r < g.TR && oh0 + r < oh_lim && ow0 + c < ow_lim;
        pr_[j] = r;
        pc_[j] = c;
        rec[j] = ok[j] ? (r * g.sh * g.PC + c * g.sw) * kRec + 16 * h : 16 * h;
    }

    // staging: item i = (channel group cg of 8, patch pixel), pixels fastest
    // so a load instruction reads consecutive pixels of one channel row
    const int npix = g.PR * g.PC;
    const int items = npix * 8;
    const uint32_t HW4 = static_cast<uint32_t>(g.H * g.W) * 4;
    const __amdgpu_buffer_rsrc_t x_rs =
        buffer_range(a.x + static_cast<int64_t>(n) * g.C * g.H * g.W, static_cast<uint64_t>(g.C) * HW4, 0);
    auto stage = [&](int chunk) {
        for (int i0 = tid; i0 < items; i0 += 4 * nt) {
            float v[4][8];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * nt;
                const int cg = i / npix, pix = i - (i / npix) * npix;
                const int pr = pix / g.PC, pc = pix - (pix / g.PC) * g.PC;
                const int ih = ih0 + pr, iw = iw0 + pc;
                const bool in = i < items && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                                static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
                // channels past C fall beyond the resource and read zero
                const uint32_t o =
                    in ? (static_cast<uint32_t>(chunk * kChunk + cg * 8) * g.H * g.W + ih * g.W + iw) * 4 : kOutside;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    v[u][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x_rs, o + e * HW4, 0, 0));
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * nt;
                if (i < items) {
                    const int cg = i / npix, pix = i - (i / npix) * npix;
                    uint32_t w = 0;
#pragma unroll
                    for (int e = 0; e < 8; ++e) w |= ternary_f4(v[u][e], a.lo, a.hi) << (4 * e);
                    *reinterpret_cast<uint32_t*>(lds + pix * kRec + cg * 4) = w;
                }
            }
        }
    };

    f32x16_t acc[FC];
#pragma unroll
    for (int j = 0; j < FC; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;

    // this wave's weight fragments: [mf][k-step][lane] x 16 bytes
    const i32x4_t* wp = reinterpret_cast<const i32x4_t*>(a.w4) +
                        (static_cast<int64_t>(active ? mf : 0) * g.ksteps) * 64 + lane;
    i32x4_t wcur = active ? wp[0] : i32x4_t{0, 0, 0, 0};
    for (int chunk = 0; chunk < g.chunks; ++chunk) {
        if (chunk) __syncthreads();  // every wave is done with the previous chunk's records
        stage(chunk);
        __syncthreads();
        if (active) {
            for (int tap = 0; tap < g.taps; ++tap) {
                const int ks = chunk * g.taps + tap;
                const i32x4_t wnext = ks + 1 < g.ksteps ? wp[(ks + 1) * 64] : wcur;
                const int r = tap / g.kw, s = tap - (tap / g.kw) * g.kw;
                const int toff = (r * g.dh * g.PC + s * g.dw) * kRec;
                i32x4_t bf[FC];
#pragma unroll
                for (int j = 0; j < FC; ++j) bf[j] = *reinterpret_cast<const i32x4_t*>(lds + rec[j] + toff);
#pragma unroll
                for (int j = 0; j < FC; ++j) acc[j] = mfma_f4(wcur, bf[j], acc[j]);
                wcur = wnext;
            }
        }
    }
    if (!active) return;

    // epilogue: acc is the exact integer C; rows of register e: 8 (e / 4) +
    // 4 h + e % 4 of the fragment
    const bool bts = (a.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
    const bool relu = (a.flags & TBN_EPI_RELU) != 0;
    const int64_t plane = static_cast<int64_t>(g.YH) * g.YW;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int m = mf * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        const int mc = min(m, g.M - 1);
        const float mult = a.scale ? a.alpha * a.scale[mc] : a.alpha;
        const float bb = a.bias ? a.bias[mc] : 0.0f;
        const int64_t cbase = (static_cast<int64_t>(n) * g.M + mc) * plane;
#pragma unroll
        for (int j = 0; j < FC; ++j) {
            const int oh = oh0 + pr_[j], ow = ow0 + pc_[j];
            if (g.pool) {
                float v = epilogue_value(acc[j][e], mult, bb, bts, nullptr);
                if (relu) v = v > 0.0f ? v : 0.0f;
                // the window's four values sit in lanes 4q .. 4q + 3 (after ReLU
                // every value is +0 or more and none is NaN: order-free maximum)
                v = fmaxf(v, quad_perm<0xB1>(v));
                v = fmaxf(v, quad_perm<0x4E>(v));
                if (m < g.M && ok[j] && (lane & 3) == 0)
                    a.y[cbase + static_cast<int64_t>(oh >> 1) * g.YW + (ow >> 1)] = v;
            } else if (m < g.M && ok[j]) {
                const int64_t idx = cbase + static_cast<int64_t>(oh) * g.YW + ow;
                float v = epilogue_value(acc[j][e], mult, bb, bts, a.residual ? a.residual + idx : nullptr);
                if (relu) v = v > 0.0f ? v : 0.0f;
                a.y[idx] = v;
            }
        }
    }
}

// K = 8 output dwords (8 channels) per thread: conv-layout fp4 weights from
// the reference's BinaryMatrix columns of the [M, C*kh*kw] matrix (bit
// (c*kh + r)*kw + s of column m, 1 = -1).
__global__ void pack_tbn_conv_weights_kernel(const uint8_t* __restrict__ bits, int64_t col_bytes, TbnGeom g,
                                             uint32_t* __restrict__ w4) {
    const int64_t total = static_cast<int64_t>(g.mfrags) * g.ksteps * 64 * 4;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int d = static_cast<int>(i & 3);
        const int lane = static_cast<int>((i >> 2) & 63);
        const int64_t fk = i >> 8;
        const int ks = static_cast<int>(fk % g.ksteps);
        const int mf = static_cast<int>(fk / g.ksteps);
        const int m = mf * 32 + (lane & 31);
        const int chunk = ks / g.taps, tap = ks - (ks / g.taps) * g.taps;
        const int c0 = chunk * kChunk + 32 * (lane >> 5) + 8 * d;
        uint32_t w = 0;
        if (m < g.M) {
            const uint8_t* col = bits + static_cast<int64_t>(m) * col_bytes;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int c = c0 + e;
                if (c < g.C) {
                    const int k = c * g.taps + tap;  // (c*kh + r)*kw + s
                    w |= ((col[k >> 3] >> (k & 7)) & 1u ? kF4Minus : kF4Plus) << (4 * e);
                }
            }
        }
        w4[i] = w;
    }
}

int make_tbn_geom(const tbn_conv2d_desc* d, int flags, TbnGeom& g) {
    TBN_REQUIRE(d, TBN_INVALID_ARGUMENT, "null descriptor");
    TBN_REQUIRE(d->n >= 0 && d->c > 0 && d->h > 0 && d->w > 0 && d->m > 0 && d->kh > 0 && d->kw > 0 && d->sh > 0 &&
                    d->sw > 0 && d->ph >= 0 && d->pw >= 0 && d->dh > 0 && d->dw > 0,
                TBN_INVALID_SHAPE, "invalid conv descriptor");
    TBN_REQUIRE((flags & ~(TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE | TBN_EPI_MAXPOOL2X2)) == 0, TBN_INVALID_ARGUMENT,
                "unsupported epilogue flags for a TBN conv");
    const int64_t OH = (d->h + 2 * d->ph - d->dh * (d->kh - 1) - 1) / d->sh + 1;
    const int64_t OW = (d->w + 2 * d->pw - d->dw * (d->kw - 1) - 1) / d->sw + 1;
    TBN_REQUIRE(OH > 0 && OW > 0, TBN_INVALID_SHAPE, "invalid output dimensions");
    const int64_t K = d->c * d->kh * d->kw;
    TBN_REQUIRE(K <= (1 << 24), TBN_INVALID_SHAPE, "TBN conv: C*kh*kw above 2^24 (fp32 sums inexact)");
    // 32-bit buffer offsets: channel planes up to the last chunk's end and 8
    // planes past the outside marker stay below 2^32
    const int64_t cpad = (d->c + kChunk - 1) / kChunk * kChunk;
    TBN_REQUIRE(d->c * d->h * d->w * 4 < (1LL << 31) && (cpad + 8) * d->h * d->w * 4 < (1LL << 32) &&
                    d->h * d->w * 32 < (1LL << 31) && d->m < (1 << 24) &&
                    d->n < (1LL << 31) && d->n * d->m * OH * OW < (1LL << 62),
                TBN_INVALID_SHAPE, "TBN conv: image above 2^31 bytes");
    g.N = static_cast<int>(d->n);
    g.C = static_cast<int>(d->c), g.H = static_cast<int>(d->h), g.W = static_cast<int>(d->w);
    g.M = static_cast<int>(d->m);
    g.kh = static_cast<int>(d->kh), g.kw = static_cast<int>(d->kw);
    g.sh = static_cast<int>(d->sh), g.sw = static_cast<int>(d->sw);
    g.ph = static_cast<int>(d->ph), g.pw = static_cast<int>(d->pw);
    g.dh = static_cast<int>(d->dh), g.dw = static_cast<int>(d->dw);
    g.OH = static_cast<int>(OH), g.OW = static_cast<int>(OW);
    g.pool = (flags & TBN_EPI_MAXPOOL2X2) ? 1 : 0;
    g.YH = g.pool ? g.OH / 2 : g.OH;
    g.YW = g.pool ? g.OW / 2 : g.OW;
    TBN_REQUIRE(g.YH > 0 && g.YW > 0, TBN_INVALID_SHAPE, "pooled output is empty");
    TBN_REQUIRE(!g.pool || (flags & TBN_EPI_RELU), TBN_NOT_IMPLEMENTED,
                "TBN conv: the fused 2x2 max pool needs the fused ReLU");
    g.chunks = static_cast<int>((d->c + kChunk - 1) / kChunk);
    g.taps = g.kh * g.kw;
    g.ksteps = g.chunks * g.taps;
    g.mfrags = (g.M + 31) / 32;

    // tile: the largest share of useful MFMA columns, weighed by how well the
    // grid fills the chip (512 blocks: two per CU); ties to larger tiles
    const int rows = g.pool ? 2 * g.YH : g.OH, cols = g.pool ? 2 * g.YW : g.OW;
    double best = -1.0;
    for (int wv = std::min(4, g.mfrags); wv >= 1; wv = wv == 4 ? 2 : wv - 1) {
        const int mblocks = (g.mfrags + wv - 1) / wv;
        for (int tc = cols; tc >= 1; tc = tc > 8 ? (tc + 1) / 2 : 0) {
            const int TC = g.pool ? (tc + 1) / 2 * 2 : tc;
            for (int tr = g.pool ? 2 : 1; tr <= rows; tr += g.pool ? 2 : 1) {
                const int px = tr * TC;
                if (px > 128) break;
                const int PR = (tr - 1) * g.sh + (g.kh - 1) * g.dh + 1;
                const int PC = (TC - 1) * g.sw + (g.kw - 1) * g.dw + 1;
                if (static_cast<int64_t>(PR) * PC * kRec > kMaxLds) break;
                const int fc = (px + 31) / 32;
                const int tr_n = (rows + tr - 1) / tr, tc_n = (cols + TC - 1) / TC;
                const double useful = static_cast<double>(rows) * cols / (static_cast<double>(tr_n) * tc_n * fc * 32);
                const double blocks = static_cast<double>(g.N) * tr_n * tc_n * mblocks;
                const double score = useful * std::min(1.0, blocks / 512.0) + 1e-6 * px + 1e-9 * wv;
                if (score > best) {
                    best = score;
                    g.TR = tr, g.TC = TC, g.FC = fc, g.WV = wv, g.mblocks = mblocks;
                    g.tiles_r = tr_n, g.tiles_c = tc_n, g.PR = PR, g.PC = PC;
                }
            }
        }
        if (wv == 1) break;
    }
    TBN_REQUIRE(best >= 0.0, TBN_INVALID_SHAPE, "TBN conv: no tile's input patch fits the LDS");
    TBN_REQUIRE(g.blocks() < (1LL << 31), TBN_INVALID_SHAPE, "TBN conv: grid too large");
    return TBN_SUCCESS;
}

template <int FC>
void launch_fc(const TbnGeom& g, const TbnConvArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(tbn_conv_kernel<FC>, dim3(static_cast<unsigned>(g.blocks())), dim3(64 * g.WV),
                       static_cast<size_t>(g.lds()), s, g, a);
}

}  // namespace

extern "C" {

int tbn_hip_tbn_conv_weights_bytes(const tbn_conv2d_desc* desc, int64_t* bytes) {
    TBN_REQUIRE(bytes, TBN_INVALID_ARGUMENT, "null pointer");
    TbnGeom g;
    const int rc = make_tbn_geom(desc, 0, g);
    if (rc) return rc;
    *bytes = static_cast<int64_t>(g.mfrags) * g.ksteps * 1024;
    return tbn_hip::ok();
}

int tbn_hip_pack_tbn_conv_weights(const uint8_t* packed, int64_t K_pad, int64_t N_pad, const tbn_conv2d_desc* desc,
                                  uint8_t* w4, tbn_stream_t stream) {
    TbnGeom g;
    int rc = make_tbn_geom(desc, 0, g);
    if (rc) return rc;
    TBN_REQUIRE(K_pad >= desc->c * desc->kh * desc->kw && K_pad % 8 == 0 && N_pad >= desc->m, TBN_INVALID_SHAPE,
                "K_pad / N_pad must cover the [M, C*kh*kw] weights");
    TBN_REQUIRE(packed && w4, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(w4) % 16 == 0, TBN_INVALID_ARGUMENT, "w4 must be 16-byte aligned");
    TBN_DEVICE_GUARD();
    const int64_t total = static_cast<int64_t>(g.mfrags) * g.ksteps * 256;
    const int blocks = static_cast<int>(std::min<int64_t>((total + 255) / 256, 65536));
    hipLaunchKernelGGL(pack_tbn_conv_weights_kernel, dim3(blocks), dim3(256), 0, tbn_hip::stream_of(stream), packed,
                       K_pad / 8, g, reinterpret_cast<uint32_t*>(w4));
    return tbn_hip::check_launch("pack_tbn_conv_weights");
}

int tbn_hip_conv2d_tbn_prepacked(const float* x, const tbn_conv2d_desc* desc, const uint8_t* w4, const float* scale,
                                 float alpha, const float* bias, const float* residual, int flags, float lo, float hi,
                                 float* y, tbn_stream_t stream) {
    TbnGeom g;
    int rc = make_tbn_geom(desc, flags, g);
    if (rc) return rc;
    TBN_REQUIRE(!(residual && g.pool), TBN_INVALID_ARGUMENT, "a residual excludes the fused max pool");
    if (g.N == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && w4 && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(w4) % 16 == 0, TBN_INVALID_ARGUMENT, "w4 must be 16-byte aligned");
    TBN_DEVICE_GUARD();
    const TbnConvArgs a{x, w4, y, scale, alpha, bias, residual, flags, lo, hi};
    const hipStream_t s = tbn_hip::stream_of(stream);
    switch (g.FC) {
        case 1: launch_fc<1>(g, a, s); break;
        case 2: launch_fc<2>(g, a, s); break;
        case 3: launch_fc<3>(g, a, s); break;
        default: launch_fc<4>(g, a, s); break;
    }
    return tbn_hip::check_launch("conv2d_tbn");
}

int tbn_hip_conv2d_tbn_kernel_name(const tbn_conv2d_desc* desc, int flags, char* name, size_t len) {
    TBN_REQUIRE(name && len > 0, TBN_INVALID_ARGUMENT, "null pointer");
    TbnGeom g;
    const int rc = make_tbn_geom(desc, flags, g);
    if (rc) return rc;
    std::snprintf(name, len, "tbn_conv_kernel<%d> (tile %dx%d, %d waves, %lld blocks)", g.FC, g.TR, g.TC, g.WV,
                  static_cast<long long>(g.blocks()));
    return tbn_hip::ok();
}

}  // extern "C"
