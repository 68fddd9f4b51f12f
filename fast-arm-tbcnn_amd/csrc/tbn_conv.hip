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
// No im2col matrix and no bit planes.  The fused kernel (tbn_conv_fused_
// kernel) stages each block's input patch from NCHW fp32 into LDS as fp4
// records, ternarized on the way, and runs every tap from them; it takes
// every geometry whose patch fits a tile of at most 8 staged items per
// thread.  The others (and TBN_TUNE_TBN_CONV = 2) run two passes:
//   1. tbn_records_kernel streams the fp32 NCHW input once from HBM and
//      writes it ternarized as fp4 pixel records: for each image, chunk of
//      64 input channels and pixel, 32 bytes (two E2M1 codes a byte), laid
//      out [n][chunk][ih][iw] -- an eighth of the input's bytes.
//   2. tbn_conv_kernel is an implicit GEMM on the fp4 matrix cores
//      (v_mfma_scale_f32_32x32x64_f8f6f4): MFMA rows are output channels,
//      columns output pixels (32 consecutive ones per fragment, so a
//      fragment's lanes store contiguous runs of a channel plane), and each
//      k-step is one tap of one chunk.  Every wave works alone (no LDS, no
//      barrier): it loads its weight fragments (pre-packed once per layer in
//      fragment order, 1 KB per k-step) and its pixels' records for a group
//      of k-steps with all loads in flight, straight from L2, then runs the
//      group's MFMAs; taps outside the image read zero through the buffer
//      range check.
#include <algorithm>
#include <cstdio>
#include <string>

#include "common.hpp"
#include "tbn_f4.hpp"

namespace {

using namespace tbnk;

constexpr int kChunk = 64;             // input channels per k-step
constexpr int kRec = 32;               // bytes of a pixel's chunk record: 64 fp4 codes
constexpr uint32_t kOutside = 0x80000000u;

struct TbnGeom {
    int N, C, H, W, M, kh, kw, sh, sw, ph, pw, dh, dw;
    int OH, OW;            // conv output plane
    int pool;              // fused 2x2 / 2 max pool (floor mode)
    int YH, YW;            // stored output plane
    int chunks, taps, ksteps, mfrags;
    int64_t pixels;        // computed output pixels: N*OH*OW, or N*YH*YW*4 by window when pooled
    int64_t pfrags;        // pixel fragments of 32
    int FCW;               // pixel fragments per wave
    int G;                 // k-steps per load group
    // the fused kernel: one tile of TR x TC output pixels of one image per
    // block, WV 32-channel fragments (one wave each), FC pixel fragments
    int fused;
    int TR, TC, tiles_r, tiles_c, PR, PC, FC, WV, mblocks, IPT, GF;
    FastDiv div_npix, div_pc;  // staging items -> (channel group, patch pixel) -> (row, column)
    __host__ __device__ int64_t fused_blocks() const {
        return static_cast<int64_t>(N) * tiles_r * tiles_c * mblocks;
    }
    __host__ __device__ int64_t groups() const { return (pfrags + FCW - 1) / FCW; }
    __host__ __device__ int64_t waves() const { return static_cast<int64_t>(mfrags) * groups(); }
    __host__ __device__ int64_t record_bytes() const { return static_cast<int64_t>(N) * chunks * H * W * kRec; }
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
    // the fused 1x1 projection (PROJ): its fp4 weights (the layout of the
    // 1x1 stride-s pad-0 desc: one k-step per chunk), its output (y's shape)
    // and epilogue (no residual, no pool)
    const uint8_t* proj_w4;
    float* proj_y;
    const float* proj_scale;
    float proj_alpha;
    const float* proj_bias;
    int proj_flags;
};

// Stand-ins for an absent scale (1) or bias (0), so the epilogue's loads
// are unconditional and all in flight together.
__device__ const float kUnitScale[1] = {1.0f};
__device__ const float kNoBias[1] = {0.0f};

// v from lane (lane & ~3) | perm[lane & 3] of the same quad (DPP quad_perm).
template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// One output of the epilogue, every operation rounded on its own (no fused
// multiply-add), in the reference's order: float(C) * s + b (conv2d_binary
// and its scaled variants) or (float(C) + b) * s (the Session's cached conv),
// then + the residual (the following Add node).
__device__ __forceinline__ float epilogue_value(float acc, float mult, float bb, bool bts, bool add, float res) {
#pragma clang fp contract(off)
    float v = bts ? (acc + bb) * mult : acc * mult + bb;
    if (add) v = v + res;
    return v;
}

// Output pixel p -> (n, oh, ow): row-major over [N, OH, OW], or by 2 x 2
// window when pooled (p / 4 a window of the pooled plane, p % 4 its
// position: bit 0 the column, bit 1 the row).  p < 2^31 (host-checked).
__device__ __forceinline__ void pixel_coords(const TbnGeom& g, int p, int& n, int& oh, int& ow) {
    if (g.pool) {
        const int q = p >> 2;
        const int plane = g.YH * g.YW;
        n = q / plane;
        const int rem = q - n * plane;
        const int py = rem / g.YW;
        oh = 2 * py + ((p >> 1) & 1);
        ow = 2 * (rem - py * g.YW) + (p & 1);
    } else {
        const int plane = g.OH * g.OW;
        n = p / plane;
        const int rem = p - n * plane;
        oh = rem / g.OW;
        ow = rem - oh * g.OW;
    }
}

// Pass 1: item i = (image n, chunk, input pixel, group of 8 channels), the
// group fastest, so 8 consecutive lanes write one pixel's 32-byte record and
// a wave 8 whole records; each load reads, across the wave, runs of 8 pixels
// (32 bytes) of 8 channel planes.
__global__ void __launch_bounds__(256) tbn_records_kernel(const float* __restrict__ x, TbnGeom g, float lo, float hi,
                                                          uint32_t* __restrict__ xt) {
    const int HW = g.H * g.W;
    const int64_t total = static_cast<int64_t>(g.N) * g.chunks * HW * 8;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int cg = static_cast<int>(i & 7);
        const int64_t rec = i >> 3;
        const int64_t nc = rec / HW;
        const int pix = static_cast<int>(rec - nc * HW);
        const int chunk = static_cast<int>(nc % g.chunks);
        const int64_t n = nc / g.chunks;
        const int c0 = chunk * kChunk + 8 * cg;
        const float* src = x + (n * g.C + c0) * HW + pix;
        float v[8];
        if (c0 + 8 <= g.C) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __builtin_nontemporal_load(src + e * HW);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = c0 + e < g.C ? src[e * HW] : 0.0f;
        }
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= ternary_f4(v[e], lo, hi) << (4 * e);
        xt[i] = w;
    }
}

// Pass 2.  Wave wv owns channel fragment wv % mfrags and pixel fragments
// [FCW * (wv / mfrags), +FCW): the waves of one block share their pixels'
// records through the CU's caches.
template <int FCW, int G>
__global__ void __launch_bounds__(256) tbn_conv_kernel(TbnGeom g, TbnConvArgs a, const uint8_t* __restrict__ xt) {
    const int lane = threadIdx.x & 63;
    const int64_t wv = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wv >= g.waves()) return;  // whole waves; the kernel has no barrier
    const int mf = static_cast<int>(wv % g.mfrags);
    const int pg = static_cast<int>(wv / g.mfrags);
    const int h = lane >> 5;

    // per lane and fragment: the pixel, the patch origin (ih0, iw0) and the
    // byte offset of the record of (n, chunk 0, ih0, iw0); a tap adds a
    // wave-uniform offset, and its validity is two unsigned compares
    int n_[FCW], oh_[FCW], ow_[FCW], ih0[FCW], iw0[FCW], base[FCW];
    bool ok[FCW];
#pragma unroll
    for (int j = 0; j < FCW; ++j) {
        const int p = (pg * FCW + j) * 32 + (lane & 31);
        ok[j] = p < g.pixels;
        pixel_coords(g, ok[j] ? p : 0, n_[j], oh_[j], ow_[j]);
        iw0[j] = ow_[j] * g.sw - g.pw;
        ih0[j] = oh_[j] * g.sh - g.ph;
        base[j] = ((n_[j] * g.chunks * g.H + ih0[j]) * g.W + iw0[j]) * kRec + 16 * h;
        if (!ok[j]) ih0[j] = -(1 << 30);  // a pixel past the end reads no tap
    }
    // records: host-checked below 2^31 bytes, so a 32-bit offset reaches
    // every one and kOutside none
    const __amdgpu_buffer_rsrc_t xt_rs = buffer_range(xt, static_cast<uint64_t>(g.record_bytes()), 0);

    f32x16_t acc[FCW];
#pragma unroll
    for (int j = 0; j < FCW; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;

    // the epilogue's per-channel scale and bias, loaded with the first group
    const int h4 = mf * 32 + 4 * h;
    const float* sp = a.scale ? a.scale : kUnitScale;
    const float* bp = a.bias ? a.bias : kNoBias;
    const int smask = a.scale ? -1 : 0, bmask = a.bias ? -1 : 0;
    float mults[16], biases[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int mc = min(h4 + 8 * (e >> 2) + (e & 3), g.M - 1);
        mults[e] = sp[mc & smask];  // times alpha below: alpha * 1 = alpha exactly
        biases[e] = bp[mc & bmask];
    }

    const i32x4_t* wp = reinterpret_cast<const i32x4_t*>(a.w4) + static_cast<int64_t>(mf) * g.ksteps * 64 + lane;
    const int chunk_bytes = g.H * g.W * kRec;
    // (chunk, r, s) of k-step ks0 + u, advanced by counters (no division)
    int c_ = 0, r_ = 0, s_ = 0;
    for (int ks0 = 0; ks0 < g.ksteps; ks0 += G) {
        i32x4_t wr[G];
        i32x4_t ar[G][FCW];
#pragma unroll
        for (int u = 0; u < G; ++u) {
            // k-steps past the end repeat the last one with zero activations
            const int ks = min(ks0 + u, g.ksteps - 1);
            const bool live = ks0 + u < g.ksteps;
            wr[u] = wp[ks * 64];
            const int dy = r_ * g.dh, dx = s_ * g.dw;
            const int toff = c_ * chunk_bytes + (dy * g.W + dx) * kRec;
            if (live) {
                if (++s_ == g.kw) {
                    s_ = 0;
                    if (++r_ == g.kh) r_ = 0, ++c_;
                }
            }
#pragma unroll
            for (int j = 0; j < FCW; ++j) {
                const bool in = live && static_cast<unsigned>(ih0[j] + dy) < static_cast<unsigned>(g.H) &&
                                static_cast<unsigned>(iw0[j] + dx) < static_cast<unsigned>(g.W);
                const uint32_t off = in ? static_cast<uint32_t>(base[j] + toff) : kOutside;
                ar[u][j] = __builtin_bit_cast(i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xt_rs, off, 0, 0));
            }
        }
        // every load of the group in flight before the first MFMA waits
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < G; ++u)
#pragma unroll
            for (int j = 0; j < FCW; ++j) acc[j] = mfma_f4(wr[u], ar[u][j], acc[j]);
    }

    // epilogue: acc is the exact integer C; rows of register e: 8 (e / 4) +
    // 4 h + e % 4 of the fragment
    const bool bts = (a.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
    const bool relu = (a.flags & TBN_EPI_RELU) != 0;
    const int64_t plane = static_cast<int64_t>(g.YH) * g.YW;
    // element (channel mf*32 + 4 h, this lane's pixel) of y (and residual);
    // register e adds (8 (e / 4) + e % 4) planes
    int64_t obase[FCW];
#pragma unroll
    for (int j = 0; j < FCW; ++j) {
        const int oy = g.pool ? oh_[j] >> 1 : oh_[j], ox = g.pool ? ow_[j] >> 1 : ow_[j];
        obase[j] = (static_cast<int64_t>(n_[j]) * g.M + mf * 32 + 4 * h) * plane + static_cast<int64_t>(oy) * g.YW + ox;
    }
    // the residual addends, all loads in flight together (lanes that store
    // nothing read element 0)
    const bool add = a.residual != nullptr;
    float res[FCW][16];
    if (add) {
#pragma unroll
        for (int j = 0; j < FCW; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = 8 * (e >> 2) + (e & 3);
                const bool st = ok[j] && mf * 32 + 4 * h + row < g.M;
                res[j][e] = a.residual[st ? obase[j] + row * plane : 0];
            }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int row = 8 * (e >> 2) + (e & 3);
        const int m = mf * 32 + 4 * h + row;
        const float mult = a.alpha * mults[e], bb = biases[e];
#pragma unroll
        for (int j = 0; j < FCW; ++j) {
            const int64_t idx = obase[j] + row * plane;
            if (g.pool) {
                float v = epilogue_value(acc[j][e], mult, bb, bts, false, 0.0f);
                if (relu) v = v > 0.0f ? v : 0.0f;
                // the window's four values sit in lanes 4q .. 4q + 3 (after ReLU
                // every value is +0 or more and none is NaN: order-free maximum)
                v = fmaxf(v, quad_perm<0xB1>(v));
                v = fmaxf(v, quad_perm<0x4E>(v));
                if (m < g.M && ok[j] && (lane & 3) == 0) a.y[idx] = v;
            } else if (m < g.M && ok[j]) {
                float v = epilogue_value(acc[j][e], mult, bb, bts, add, add ? res[j][e] : 0.0f);
                if (relu) v = v > 0.0f ? v : 0.0f;
                a.y[idx] = v;
            }
        }
    }
}

// Tile pixel p -> conv output offsets (r, c) inside a TR x TC tile:
// row-major, or by 2 x 2 window when pooled.
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

// The fused kernel: no record pass.  A block stages, per chunk of 64 input
// channels, the input patch of its tile (PR x PC pixels) from NCHW fp32
// straight into LDS as fp4 records, ternarized on the way: each thread issues
// its IPT items' loads (8 channels of one patch pixel each) before any
// arrives, together with its wave's weight fragments for the chunk's first
// GF taps and (once) the epilogue's scale and bias.  Every tap is then one
// MFMA k-step read from the same records.
//
// PROJ (a 3x3 pad-1 conv, GF = 9, host-checked): the 1x1 stride-s projection
// of the same input reads the centre tap's records, so the centre tap's
// pixel fragments also feed one MFMA with the projection's weights per
// chunk, into a second set of accumulators, written by a second epilogue.
// Every product and partial sum is an exact integer, so the result has the
// bits of the 1x1 conv run alone.
template <int FC, int IPT, int GF, bool PROJ>
__device__ __forceinline__ void tbn_conv_fused_body(const TbnGeom& g, const TbnConvArgs& a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x;
    const int nt = 64 * g.WV;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;

    // block -> (image, tile, channel block); the channel blocks of a tile are
    // consecutive in b, and consecutive b share an XCD (blocks are dealt
    // round-robin over the 8 XCDs), so a patch is fetched into one L2
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
    const int mfc = active ? mf : 0;

    // the epilogue's per-channel scale and bias, in flight from the start
    const int h4 = mfc * 32 + 4 * h;
    const float* sp = a.scale ? a.scale : kUnitScale;
    const float* bp = a.bias ? a.bias : kNoBias;
    const int smask = a.scale ? -1 : 0, bmask = a.bias ? -1 : 0;
    float mults[16], biases[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int mc = min(h4 + 8 * (e >> 2) + (e & 3), g.M - 1);
        mults[e] = sp[mc & smask];
        biases[e] = bp[mc & bmask];
    }

    // this lane's pixel in each fragment and its record in the patch (tap 0)
    const int oh_lim = g.pool ? 2 * g.YH : g.OH, ow_lim = g.pool ? 2 * g.YW : g.OW;
    int rec[FC], pr_[FC], pc_[FC];
    bool ok[FC];
#pragma unroll
    for (int j = 0; j < FC; ++j) {
        int r, c;
        tile_pixel(g, j * 32 + (lane & 31), r, c);
        ok[j] = r < g.TR && oh0 + r < oh_lim && ow0 + c < ow_lim;
        pr_[j] = r;
        pc_[j] = c;
        rec[j] = ok[j] ? (r * g.sh * g.PC + c * g.sw) * kRec + 16 * h : 16 * h;
    }

    const int npix = g.PR * g.PC;
    const int items = npix * 8;
    const uint32_t HW4 = static_cast<uint32_t>(g.H * g.W) * 4;
    const __amdgpu_buffer_rsrc_t x_rs =
        buffer_range(a.x + static_cast<int64_t>(n) * g.C * g.H * g.W, static_cast<uint64_t>(g.C) * HW4, 0);
    const i32x4_t* wp = reinterpret_cast<const i32x4_t*>(a.w4) + static_cast<int64_t>(mfc) * g.ksteps * 64 + lane;

    f32x16_t acc[FC], accp[PROJ ? FC : 1];
#pragma unroll
    for (int j = 0; j < FC; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
    if constexpr (PROJ) {
#pragma unroll
        for (int j = 0; j < FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) accp[j][e] = 0.0f;
    }
    // the projection's weight fragment of each chunk (one k-step per chunk)
    const i32x4_t* wpp =
        PROJ ? reinterpret_cast<const i32x4_t*>(a.proj_w4) + static_cast<int64_t>(mfc) * g.chunks * 64 + lane : nullptr;

    for (int chunk = 0; chunk < g.chunks; ++chunk) {
        // the weights of the chunk's first GF taps (taps past the end: zero)
        i32x4_t wr[GF];
#pragma unroll
        for (int u = 0; u < GF; ++u) {
            const bool live = active && u < g.taps;
            wr[u] = live ? wp[(chunk * g.taps + u) * 64] : i32x4_t{0, 0, 0, 0};
        }
        i32x4_t wpr = i32x4_t{0, 0, 0, 0};
        if constexpr (PROJ) wpr = active ? wpp[chunk * 64] : i32x4_t{0, 0, 0, 0};
        // the patch: item i = (channel group cg, patch pixel), pixels fastest
        // so one load reads consecutive pixels of a channel row; channels
        // past C fall beyond the resource and read zero
        float v[IPT][8];
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int i = tid + k * nt;
            const int cg = static_cast<int>(g.div_npix.div(i)), pix = i - cg * npix;
            const int pr = static_cast<int>(g.div_pc.div(pix)), pc = pix - pr * g.PC;
            const int ih = ih0 + pr, iw = iw0 + pc;
            const bool in = i < items && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                            static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
            const uint32_t o =
                in ? (static_cast<uint32_t>(chunk * kChunk + cg * 8) * g.H * g.W + ih * g.W + iw) * 4 : kOutside;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v[k][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x_rs, o + e * HW4, 0, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
        if (chunk) __syncthreads();  // every wave is done reading the previous chunk's records
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int i = tid + k * nt;
            if (i < items) {
                const int cg = static_cast<int>(g.div_npix.div(i)), pix = i - cg * npix;
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) w |= ternary_f4(v[k][e], a.lo, a.hi) << (4 * e);
                *reinterpret_cast<uint32_t*>(lds + pix * kRec + cg * 4) = w;
            }
        }
        __syncthreads();
        if (active) {
            int r_ = 0, s_ = 0;  // (r, s) of tap t0 + u, advanced by counters
            for (int t0 = 0; t0 < g.taps; t0 += GF) {
                if (t0) {
#pragma unroll
                    for (int u = 0; u < GF; ++u) {
                        const bool live = t0 + u < g.taps;
                        wr[u] = live ? wp[(chunk * g.taps + t0 + u) * 64] : i32x4_t{0, 0, 0, 0};
                    }
                }
#pragma unroll
                for (int u = 0; u < GF; ++u) {
                    const bool live = t0 + u < g.taps;
                    const int toff = live ? (r_ * g.dh * g.PC + s_ * g.dw) * kRec : 0;
                    if (live && ++s_ == g.kw) s_ = 0, ++r_;
                    i32x4_t bf[FC];
#pragma unroll
                    for (int j = 0; j < FC; ++j) bf[j] = *reinterpret_cast<const i32x4_t*>(lds + rec[j] + toff);
#pragma unroll
                    for (int j = 0; j < FC; ++j) acc[j] = mfma_f4(wr[u], bf[j], acc[j]);
                    if constexpr (PROJ) {
                        // tap 4 = (1, 1), the centre: the projection's input pixel
                        if (u == 4 && t0 == 0) {
#pragma unroll
                            for (int j = 0; j < FC; ++j) accp[j] = mfma_f4(wpr, bf[j], accp[j]);
                        }
                    }
                }
            }
        }
    }
    if (!active) return;

    // epilogue: buffer stores into image n's output planes (32-bit offsets,
    // host-checked): rows past M fall beyond the resource, lanes with no
    // pixel to store carry kOutside, so no store is behind a branch
    const bool bts = (a.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
    const bool relu = (a.flags & TBN_EPI_RELU) != 0;
    const uint32_t plane4 = static_cast<uint32_t>(g.YH * g.YW) * 4;
    const int64_t img = static_cast<int64_t>(n) * g.M * g.YH * g.YW;
    const __amdgpu_buffer_rsrc_t y_rs = buffer_range(a.y + img, static_cast<uint64_t>(g.M) * plane4, 0);
    uint32_t voff[FC];
#pragma unroll
    for (int j = 0; j < FC; ++j) {
        const int oh = oh0 + pr_[j], ow = ow0 + pc_[j];
        const int oy = g.pool ? oh >> 1 : oh, ox = g.pool ? ow >> 1 : ow;
        const bool st = ok[j] && (!g.pool || (lane & 3) == 0);
        voff[j] = st ? static_cast<uint32_t>(mf * 32 + 4 * h) * plane4 + static_cast<uint32_t>(oy * g.YW + ox) * 4
                     : kOutside;
    }
    const bool add = a.residual != nullptr;
    float res[FC][16];
    if (add) {
        const __amdgpu_buffer_rsrc_t r_rs = buffer_range(a.residual + img, static_cast<uint64_t>(g.M) * plane4, 0);
#pragma unroll
        for (int j = 0; j < FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                res[j][e] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(r_rs, voff[j] + (8 * (e >> 2) + (e & 3)) * plane4, 0, 0));
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t roff = (8 * (e >> 2) + (e & 3)) * plane4;
        const float mult = a.alpha * mults[e], bb = biases[e];
#pragma unroll
        for (int j = 0; j < FC; ++j) {
            float v = epilogue_value(acc[j][e], mult, bb, bts, add, add ? res[j][e] : 0.0f);
            if (relu) v = v > 0.0f ? v : 0.0f;
            if (g.pool) {
                // the window's four values sit in lanes 4q .. 4q + 3 (after ReLU
                // every value is +0 or more and none is NaN: order-free maximum)
                v = fmaxf(v, quad_perm<0xB1>(v));
                v = fmaxf(v, quad_perm<0x4E>(v));
            }
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), y_rs, voff[j] + roff, 0, 0);
        }
    }
    if constexpr (PROJ) {
        // the projection's epilogue (no residual, no pool: host-checked), its
        // factors loaded here rather than held through the K loop
        const __amdgpu_buffer_rsrc_t py_rs = buffer_range(a.proj_y + img, static_cast<uint64_t>(g.M) * plane4, 0);
        const float* psp = a.proj_scale ? a.proj_scale : kUnitScale;
        const float* pbp = a.proj_bias ? a.proj_bias : kNoBias;
        const int psmask = a.proj_scale ? -1 : 0, pbmask = a.proj_bias ? -1 : 0;
        const bool pbts = (a.proj_flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
        const bool prelu = (a.proj_flags & TBN_EPI_RELU) != 0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int mc = min(h4 + 8 * (e >> 2) + (e & 3), g.M - 1);
            const float mult = a.proj_alpha * psp[mc & psmask], bb = pbp[mc & pbmask];
            const uint32_t roff = (8 * (e >> 2) + (e & 3)) * plane4;
#pragma unroll
            for (int j = 0; j < FC; ++j) {
                float v = epilogue_value(accp[j][e], mult, bb, pbts, false, 0.0f);
                if (prelu) v = v > 0.0f ? v : 0.0f;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), py_rs, voff[j] + roff, 0, 0);
            }
        }
    }
}

// Tiles with at most four staged items per thread fit three waves per SIMD
// without spills (asked for explicitly: left alone the compiler allocates
// for two); eight items keep the compiler's choice.
template <int FC, int IPT, int GF>
__global__ void __launch_bounds__(256, (FC == 1 && IPT <= 4) ? 3 : 1) tbn_conv_fused_kernel(TbnGeom g, TbnConvArgs a) {
    tbn_conv_fused_body<FC, IPT, GF, false>(g, a);
}

// The pair (PROJ): held to two waves per SIMD, the non-pair kernel's
// occupancy; its own register demand would leave one.
template <int FC, int IPT>
__global__ void __launch_bounds__(256, 2) tbn_conv_pair_kernel(TbnGeom g, TbnConvArgs a) {
    tbn_conv_fused_body<FC, IPT, 9, true>(g, a);
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
    TBN_REQUIRE(d->c * d->kh * d->kw <= (1 << 24), TBN_INVALID_SHAPE,
                "TBN conv: C*kh*kw above 2^24 (fp32 sums inexact)");
    const int64_t chunks = (d->c + kChunk - 1) / kChunk;
    // the records of the whole input are addressed with 32-bit offsets
    TBN_REQUIRE(d->n * chunks * d->h * d->w * kRec < (1LL << 31) && d->n * OH * OW * 4 < (1LL << 31) &&
                    d->m < (1 << 24) &&
                    d->n * d->m * OH * OW < (1LL << 62) && d->h < (1 << 24) && d->w < (1 << 24),
                TBN_INVALID_SHAPE, "TBN conv: input records of 2^31 bytes or more");
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
    g.chunks = static_cast<int>(chunks);
    g.taps = g.kh * g.kw;
    g.ksteps = g.chunks * g.taps;
    g.mfrags = (g.M + 31) / 32;
    g.pixels = g.pool ? static_cast<int64_t>(g.N) * g.YH * g.YW * 4 : static_cast<int64_t>(g.N) * g.OH * g.OW;
    g.pfrags = (g.pixels + 31) / 32;
    // two pixel fragments per wave (each weight fragment serves two MFMAs)
    // while that still leaves about eight waves per CU, else one
    g.FCW = g.mfrags * ((g.pfrags + 1) / 2) >= 2048 ? 2 : 1;
    // k-steps per load group: each group costs one memory round trip, a
    // wasted (padding) step an MFMA and two cached loads
    static const int kGroups[] = {9, 8, 4, 3, 2, 1};
    double best = 0.0;
    for (int G : kGroups) {
        const int trips = (g.ksteps + G - 1) / G;
        const double cost = trips + 0.05 * (trips * G - g.ksteps);
        if (G == 9 || cost < best) best = cost, g.G = G;
    }
    TBN_REQUIRE((g.waves() + 3) / 4 < (1LL << 31), TBN_INVALID_SHAPE, "TBN conv: grid too large");

    // fused tile: staged pixels per thread bounded (IPT <= 8 items of 8
    // channels), one pixel fragment (32 output pixels); the score is the
    // share of useful MFMA columns weighed by how well the grid fills the
    // chip (512 blocks) and by the patch pixels staged per output pixel (the
    // halo).  Tiles of two to four fragments stage less halo per pixel, but
    // hold more staging registers and run fewer waves per SIMD: measured
    // slower on ResNet-18's stage-1 and stage-2 convs (26.6 -> 25.0 us and
    // 20.2 -> 17.3 us with one fragment), so they are not offered.
    const int rows = g.pool ? 2 * g.YH : g.OH, cols = g.pool ? 2 * g.YW : g.OW;
    double best_score = -1.0;
    g.fused = 0;
    for (int wv = std::min(4, g.mfrags); wv >= 1; wv = wv == 4 ? 2 : wv - 1) {
        const int mblocks = (g.mfrags + wv - 1) / wv;
        for (int tc = cols; tc >= 1; tc = tc > 8 ? (tc + 1) / 2 : 0) {
            const int TC = g.pool ? (tc + 1) / 2 * 2 : tc;
            for (int tr = g.pool ? 2 : 1; tr <= rows; tr += g.pool ? 2 : 1) {
                const int px = tr * TC;
                if (px > 32) break;
                const int PR = (tr - 1) * g.sh + (g.kh - 1) * g.dh + 1;
                const int PC = (TC - 1) * g.sw + (g.kw - 1) * g.dw + 1;
                if (static_cast<int64_t>(PR) * PC * 8 > 8LL * 64 * wv) break;
                const int fc = (px + 31) / 32;
                const int tr_n = (rows + tr - 1) / tr, tc_n = (cols + TC - 1) / TC;
                const double useful = static_cast<double>(rows) * cols / (static_cast<double>(tr_n) * tc_n * fc * 32);
                const double blocks = static_cast<double>(g.N) * tr_n * tc_n * mblocks;
                const double halo = static_cast<double>(PR) * PC / std::min(px, rows * cols);
                const double score = useful * std::min(1.0, blocks / 512.0) / (1.0 + 0.1 * halo) + 1e-9 * wv;
                if (score > best_score) {
                    best_score = score;
                    g.fused = 1;
                    g.TR = tr, g.TC = TC, g.FC = fc, g.WV = wv, g.mblocks = mblocks;
                    g.tiles_r = tr_n, g.tiles_c = tc_n, g.PR = PR, g.PC = PC;
                }
            }
        }
        if (wv == 1) break;
    }
    if (g.fused) {
        g.div_npix = make_fastdiv(static_cast<uint32_t>(g.PR * g.PC));
        g.div_pc = make_fastdiv(static_cast<uint32_t>(g.PC));
        const int ipt = (g.PR * g.PC * 8 + 64 * g.WV - 1) / (64 * g.WV);
        g.IPT = ipt <= 2 ? 2 : (ipt <= 4 ? 4 : 8);
        g.GF = g.taps == 1 ? 1 : 9;
        const int variant = tbn_hip::tuning(TBN_TUNE_TBN_CONV);
        if (variant == 2 || g.fused_blocks() >= (1LL << 31) || d->c * d->h * d->w * 4 >= (1LL << 31) ||
            (d->c + 64 + 8) * d->h * d->w * 4 >= (1LL << 32) ||
            (d->m + 32) * static_cast<int64_t>(g.YH) * g.YW * 4 >= (1LL << 31))
            g.fused = 0;  // the two-pass kernels (the forced choice, or 32-bit offsets would not reach)
    }
    return TBN_SUCCESS;
}

template <int FCW, int G>
void launch_conv(const TbnGeom& g, const TbnConvArgs& a, const uint8_t* xt, hipStream_t s) {
    hipLaunchKernelGGL((tbn_conv_kernel<FCW, G>), dim3(static_cast<unsigned>((g.waves() + 3) / 4)), dim3(256), 0, s,
                       g, a, xt);
}

template <int FCW>
void launch_conv_g(const TbnGeom& g, const TbnConvArgs& a, const uint8_t* xt, hipStream_t s) {
    switch (g.G) {
        case 9: return launch_conv<FCW, 9>(g, a, xt, s);
        case 8: return launch_conv<FCW, 8>(g, a, xt, s);
        case 4: return launch_conv<FCW, 4>(g, a, xt, s);
        case 3: return launch_conv<FCW, 3>(g, a, xt, s);
        case 2: return launch_conv<FCW, 2>(g, a, xt, s);
        default: return launch_conv<FCW, 1>(g, a, xt, s);
    }
}

// Tiles of one pixel fragment (make_tbn_geom), so FC = 1.
template <int IPT>
void launch_fused_g(const TbnGeom& g, const TbnConvArgs& a, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(g.fused_blocks())), block(64 * g.WV);
    const size_t lds = static_cast<size_t>(g.PR) * g.PC * kRec;
    if (a.proj_w4) hipLaunchKernelGGL((tbn_conv_pair_kernel<1, IPT>), grid, block, lds, s, g, a);
    else if (g.GF == 1) hipLaunchKernelGGL((tbn_conv_fused_kernel<1, IPT, 1>), grid, block, lds, s, g, a);
    else hipLaunchKernelGGL((tbn_conv_fused_kernel<1, IPT, 9>), grid, block, lds, s, g, a);
}

int run_tbn_fused(const TbnGeom& g, const TbnConvArgs& a, hipStream_t s) {
    TBN_REQUIRE(g.FC == 1, TBN_INVALID_SHAPE, "TBN conv tiles hold one pixel fragment");
    if (g.IPT == 2) launch_fused_g<2>(g, a, s);
    else if (g.IPT == 4) launch_fused_g<4>(g, a, s);
    else launch_fused_g<8>(g, a, s);
    return tbn_hip::check_launch("conv2d_tbn (fused)");
}

int run_tbn_conv(const TbnGeom& g, const TbnConvArgs& a, uint8_t* xt, hipStream_t s) {
    const int64_t items = static_cast<int64_t>(g.N) * g.chunks * 8 * g.H * g.W;
    const int blocks = static_cast<int>(std::min<int64_t>((items + 255) / 256, 1 << 20));
    hipLaunchKernelGGL(tbn_records_kernel, dim3(blocks), dim3(256), 0, s, a.x, g, a.lo, a.hi,
                       reinterpret_cast<uint32_t*>(xt));
    if (g.FCW == 2) launch_conv_g<2>(g, a, xt, s);
    else launch_conv_g<1>(g, a, xt, s);
    return tbn_hip::check_launch("conv2d_tbn");
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

int tbn_hip_tbn_conv_scratch_bytes(const tbn_conv2d_desc* desc, int64_t* bytes) {
    TBN_REQUIRE(bytes, TBN_INVALID_ARGUMENT, "null pointer");
    TbnGeom g;
    const int rc = make_tbn_geom(desc, 0, g);
    if (rc) return rc;
    *bytes = g.fused ? 0 : g.record_bytes();
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
                                 uint8_t* scratch, float* y, tbn_stream_t stream) {
    TbnGeom g;
    int rc = make_tbn_geom(desc, flags, g);
    if (rc) return rc;
    TBN_REQUIRE(!(residual && g.pool), TBN_INVALID_ARGUMENT, "a residual excludes the fused max pool");
    if (g.N == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && w4 && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(w4) % 16 == 0 && reinterpret_cast<uintptr_t>(scratch) % 16 == 0,
                TBN_INVALID_ARGUMENT, "w4 and scratch must be 16-byte aligned");
    TBN_DEVICE_GUARD();
    const TbnConvArgs a{x, w4, y, scale, alpha, bias, residual, flags, lo, hi};
    const hipStream_t s = tbn_hip::stream_of(stream);
    if (g.fused) return run_tbn_fused(g, a, s);
    if (scratch) return run_tbn_conv(g, a, scratch, s);
    // the stream workspace (refused while s captures)
    void* ws = nullptr;
    bool temporary = false;
    rc = tbn_hip::stream_workspace(s, static_cast<size_t>(g.record_bytes()), ws, temporary);
    if (rc) return rc;
    rc = run_tbn_conv(g, a, static_cast<uint8_t*>(ws), s);
    tbn_hip::release_workspace(ws, temporary, s);
    return rc;
}

int tbn_hip_conv2d_tbn_prepacked_pair(const float* x, const tbn_conv2d_desc* desc, const uint8_t* w4,
                                      const float* scale, float alpha, const float* bias, const float* residual,
                                      int flags, float lo, float hi, float* y, const uint8_t* proj_w4,
                                      const float* proj_scale, float proj_alpha, const float* proj_bias,
                                      int proj_flags, float* proj_y, int mode, tbn_stream_t stream) {
    TBN_REQUIRE(mode == 0 || mode == 2, TBN_INVALID_ARGUMENT, "mode must be 0 (run) or 2 (query)");
    constexpr int kFlags = TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE;
    TBN_REQUIRE((flags & ~kFlags) == 0 && (proj_flags & ~kFlags) == 0, TBN_INVALID_ARGUMENT,
                "a fused TBN pair takes ReLU and bias-then-scale epilogues only");
    TBN_REQUIRE(desc != nullptr, TBN_INVALID_ARGUMENT, "null pointer");
    if (desc->kh != 3 || desc->kw != 3 || desc->ph != 1 || desc->pw != 1 || desc->dh != 1 || desc->dw != 1 ||
        desc->sh != desc->sw)
        return tbn_hip::fail(TBN_NOT_IMPLEMENTED, "only a 3x3 pad-1 conv pairs with the 1x1 projection of its input");
    TbnGeom g;
    int rc = make_tbn_geom(desc, flags, g);
    if (rc) return rc;
    if (!g.fused)
        return tbn_hip::fail(TBN_NOT_IMPLEMENTED, "a TBN conv on the two-pass kernels runs apart from its projection");
    if (mode == 2 || g.N == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && w4 && y && proj_w4 && proj_y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(w4) % 16 == 0 && reinterpret_cast<uintptr_t>(proj_w4) % 16 == 0,
                TBN_INVALID_ARGUMENT, "w4 and proj_w4 must be 16-byte aligned");
    TBN_DEVICE_GUARD();
    TbnConvArgs a{x, w4, y, scale, alpha, bias, residual, flags, lo, hi};
    a.proj_w4 = proj_w4;
    a.proj_y = proj_y;
    a.proj_scale = proj_scale;
    a.proj_alpha = proj_alpha;
    a.proj_bias = proj_bias;
    a.proj_flags = proj_flags;
    return run_tbn_fused(g, a, tbn_hip::stream_of(stream));
}

int tbn_hip_conv2d_tbn_kernel_name(const tbn_conv2d_desc* desc, int flags, char* name, size_t len) {
    TBN_REQUIRE(name && len > 0, TBN_INVALID_ARGUMENT, "null pointer");
    TbnGeom g;
    const int rc = make_tbn_geom(desc, flags, g);
    if (rc) return rc;
    if (g.fused)
        std::snprintf(name, len, "tbn_conv_fused_kernel<%d, %d, %d>", g.FC, g.IPT, g.GF);
    else
        std::snprintf(name, len, "tbn_conv_kernel<%d, %d>", g.FCW, g.G);
    return tbn_hip::ok();
}

}  // extern "C"
