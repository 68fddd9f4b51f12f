// fp32 convolution for few input channels and wide kernels: the ResNet stem
// (3 -> 64 channels, 7x7, stride 2).  The im2col engine of conv.hip gathers
// every (pixel, tap) element from global memory and splits it anew; here a
// block stages the input patch of a 16 x 16 output tile in LDS once and
// builds each MFMA column fragment from it.
//
// K is ordered k = (r * C + c) * 8 + s: tap row r, channel c, tap column s
// padded from kw to 8.  A lane's 8 consecutive k of a k-slice are then 8
// consecutive input columns of one row of one channel, i.e. four float2
// reads from the patch, split into three bf16 planes in registers (hi + mid +
// lo = x exactly).  The weights are split the same way once per call into a
// [plane][64 rows][K_pad] bf16 table (zero outside M, kh, kw) that each block
// keeps in LDS for all the tiles it takes (the grid is persistent, one block
// per CU).  Products per k-slice: w_hi x_hi, w_hi x_mid, w_mid x_hi,
// w_hi x_lo, w_mid x_mid, w_lo x_hi (the terms below 2^-24 relative dropped),
// accumulated in fp32.
//
// Block: 4 waves, all 64 output channels x a 16 x 16 tile of output pixels;
// wave w owns tile rows 4w .. 4w+3 (two 32-pixel column fragments).  The next
// tile's patch is loaded into registers while the current one is computed.
#include <algorithm>
#include <mutex>
#include <string>

#include "conv_common.hpp"

namespace {

using namespace tbnk;

constexpr int kRows = 64;        // output channels per block (M <= 64)
constexpr int kTile = 16;        // output tile: 16 x 16 pixels
constexpr int kMaxPatch = 6144;  // floats of the staged input patch
constexpr int kStage = kMaxPatch / 256;
constexpr uint32_t kOutside = 0x80000000u;

struct StemGeom {
    int N, C, H, W, M;
    int kh, kw, sh, sw, ph, pw, dh;
    int OH, OW;
    int K_pad;         // 16 * slices
    int prows, pitch;  // staged patch: rows, row pitch in floats (a multiple of 4)
    int patch;         // C * prows * pitch
    int tiles_w, tiles_img, tiles;
    int relu;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

// w [M, C, kh, kw] fp32 -> [3][64][K_pad] bf16 planes in the kernel's K order.
__global__ void stem_weights_kernel(const float* __restrict__ w, StemGeom g, uint16_t* __restrict__ out) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= kRows * g.K_pad) return;
    const int m = idx / g.K_pad, k = idx - m * g.K_pad;
    const int k8 = k >> 3, s = k & 7;
    const int r = k8 / g.C, c = k8 - r * g.C;
    float v = 0.0f;
    if (m < g.M && r < g.kh && s < g.kw) v = w[((static_cast<int64_t>(m) * g.C + c) * g.kh + r) * g.kw + s];
    const uint32_t u = __float_as_uint(v);
    const float h = __uint_as_float(u & 0xFFFF0000u);
    const float r1 = (v == h) ? 0.0f : v - h;
    const uint32_t mb = __float_as_uint(r1);
    const float r2 = r1 - __uint_as_float(mb & 0xFFFF0000u);
    const int64_t plane = static_cast<int64_t>(kRows) * g.K_pad;
    out[idx] = static_cast<uint16_t>(u >> 16);
    out[plane + idx] = static_cast<uint16_t>(mb >> 16);
    out[2 * plane + idx] = static_cast<uint16_t>(__float_as_uint(r2) >> 16);
}

template <int KW, int SLICES>
__global__ void __launch_bounds__(256) stem_conv_kernel(const float* __restrict__ x, StemGeom g,
                                                        const uint16_t* __restrict__ wsplit,
                                                        const float* __restrict__ bias, float* __restrict__ y) {
    constexpr int K_PAD = 16 * SLICES;
    constexpr int KROW = K_PAD + 8;  // bf16 per LDS weight row: conflict-free 16-byte reads
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    uint16_t* wl = lds;                                             // [3][64][KROW]
    float* bl = reinterpret_cast<float*>(lds + 3 * kRows * KROW);  // [64] bias
    float* patch = bl + kRows;                                      // [C][prows][pitch]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- weights and bias, once per block ----
    constexpr int kChunks = 3 * kRows * (K_PAD / 8);  // 16-byte pieces
#pragma unroll 8
    for (int i = tid; i < kChunks; i += 256) {
        const int row = i / (K_PAD / 8), q = i - row * (K_PAD / 8);
        *reinterpret_cast<uint4*>(wl + row * KROW + q * 8) =
            *reinterpret_cast<const uint4*>(wsplit + static_cast<int64_t>(row) * K_PAD + q * 8);
    }
    if (tid < kRows) bl[tid] = (bias && tid < g.M) ? bias[tid] : 0.0f;

    // ---- patch staging: element e = tid + 256 i of [C][prows][pitch] ----
    // (c, row, col) of each element is the same for every tile: packed once
    uint32_t coord[kStage];
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int e = tid + 256 * i;
        const int c = e / (g.prows * g.pitch);
        const int rem = e - c * g.prows * g.pitch;
        const int pr = rem / g.pitch;
        const int pc = rem - pr * g.pitch;
        coord[i] = (e < g.patch) ? (static_cast<uint32_t>(c) << 24) | (static_cast<uint32_t>(pr) << 12) | pc
                                 : 0xFFFFFFFFu;
    }
    const uint32_t HW = static_cast<uint32_t>(g.H) * g.W;
    float stage[kStage];
    auto tile_origin = [&](int t, int& n, int& oh0, int& ow0) {
        n = t / g.tiles_img;
        const int r = t - n * g.tiles_img;
        const int th = r / g.tiles_w;
        oh0 = th * kTile;
        ow0 = (r - th * g.tiles_w) * kTile;
    };
    auto load_patch = [&](int t) {
        int n, oh0, ow0;
        tile_origin(t, n, oh0, ow0);
        const int ih0 = oh0 * g.sh - g.ph, iw0 = ow0 * g.sw - g.pw;
        // image n: C * H * W floats (host-checked below 2^31 bytes); outside -> 0
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(x + static_cast<int64_t>(n) * g.C * HW, g.C * HW * 4);
#pragma unroll
        for (int i = 0; i < kStage; ++i) {
            const uint32_t cd = coord[i];
            const int c = cd >> 24, pr = (cd >> 12) & 0xFFF, pc = cd & 0xFFF;
            const int ih = ih0 + pr, iw = iw0 + pc;
            const bool ok = cd != 0xFFFFFFFFu && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                            static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
            const uint32_t off = ok ? (static_cast<uint32_t>(c) * HW + ih * g.W + iw) * 4 : kOutside;
            stage[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
        }
    };
    auto store_patch = [&]() {
#pragma unroll
        for (int i = 0; i < kStage; ++i)
            if (tid + 256 * i < g.patch) patch[tid + 256 * i] = stage[i];
    };

    // ---- this lane's fragment pixels and k-slice offsets ----
    const int kg = lane >> 5;
    int pix[2];  // patch offset of the lane's pixel in fragment j (tap (0, 0), channel 0)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int tr = 4 * wave + 2 * j + ((lane & 31) >> 4);
        const int tc = lane & 15;
        pix[j] = tr * g.sh * g.pitch + tc * g.sw;
    }
    int koff[SLICES];  // patch offset of k8 = 2 t + kg: row r * dh of channel c; -1 past kh * C
#pragma unroll
    for (int t = 0; t < SLICES; ++t) {
        const int k8 = 2 * t + kg;
        const int r = k8 / g.C, c = k8 - r * g.C;
        koff[t] = (r < g.kh) ? (c * g.prows + r * g.dh) * g.pitch : -1;
    }
    const int wrow = lane & 31;

    int t = blockIdx.x;
    if (t < g.tiles) load_patch(t);
    for (; t < g.tiles; t += gridDim.x) {
        store_patch();
        __syncthreads();
        const int tn = t + gridDim.x;
        if (tn < g.tiles) load_patch(tn);

        f32x16_t acc[2][2];
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[f][j][e] = 0.0f;
#pragma unroll
        for (int sl = 0; sl < SLICES; ++sl) {
            u32x4_t a[3][2];
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int f = 0; f < 2; ++f)
                    a[p][f] = *reinterpret_cast<const u32x4_t*>(wl + (p * kRows + f * 32 + wrow) * KROW + sl * 16 +
                                                                kg * 8);
            u32x4_t b[3][2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int ko = koff[sl];
                const float* src = patch + pix[j] + (ko < 0 ? 0 : ko);
                float v[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float2 w2 = *reinterpret_cast<const float2*>(src + 2 * q);
                    v[2 * q] = w2.x;
                    v[2 * q + 1] = w2.y;
                }
                // columns past the kernel and rows past kh carry zero weights;
                // zero their inputs too so an inf there cannot make a NaN
#pragma unroll
                for (int q = KW; q < 8; ++q) v[q] = 0.0f;
                if (ko < 0) {
#pragma unroll
                    for (int q = 0; q < 8; ++q) v[q] = 0.0f;
                }
                uint4 hi, mid, lo;
                split8(v, hi, mid, lo);
                b[0][j] = u32x4_t{hi.x, hi.y, hi.z, hi.w};
                b[1][j] = u32x4_t{mid.x, mid.y, mid.z, mid.w};
                b[2][j] = u32x4_t{lo.x, lo.y, lo.z, lo.w};
            }
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[f][j] = mfma32(a[0][f], b[0][j], acc[f][j]);
                    acc[f][j] = mfma32(a[0][f], b[1][j], acc[f][j]);
                    acc[f][j] = mfma32(a[1][f], b[0][j], acc[f][j]);
                    acc[f][j] = mfma32(a[0][f], b[2][j], acc[f][j]);
                    acc[f][j] = mfma32(a[1][f], b[1][j], acc[f][j]);
                    acc[f][j] = mfma32(a[2][f], b[0][j], acc[f][j]);
                }
        }

        // ---- epilogue: + bias, ReLU; buffer stores into image n's output
        //      (rows past M and pixels past the image carry kOutside) ----
        int n, oh0, ow0;
        tile_origin(t, n, oh0, ow0);
        const uint32_t plane = static_cast<uint32_t>(g.OH) * g.OW;
        const __amdgpu_buffer_rsrc_t ys =
            make_rsrc(y + static_cast<int64_t>(n) * g.M * plane, static_cast<uint32_t>(g.M) * plane * 4);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int oh = oh0 + 4 * wave + 2 * j + ((lane & 31) >> 4);
            const int ow = ow0 + (lane & 15);
            const uint32_t base = (oh < g.OH && ow < g.OW)
                                      ? (static_cast<uint32_t>(4 * kg) * plane + oh * g.OW + ow) * 4
                                      : kOutside;
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = f * 32 + 8 * (e >> 2) + (e & 3);  // + 4 * kg in `base`
                    float v = acc[f][j][e] * 1.0f + bl[row + 4 * kg];
                    if (g.relu) v = v > 0.0f ? v : 0.0f;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ys,
                                                          base + static_cast<uint32_t>(row) * plane * 4, 0, 0);
                }
        }
        __syncthreads();
    }
}

int stem_cu_count() {
    static std::mutex mu;
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

constexpr int kStemKW = 7, kStemSlices = 11;

bool stem_geom(const tbn_conv2d_desc* d, int flags, StemGeom& g) {
    if (!d || flags & ~TBN_EPI_RELU) return false;
    if (d->kw != kStemKW || d->dw != 1 || d->m > kRows || d->sw % 2 != 0) return false;
    if ((d->kh * d->c + 1) / 2 != kStemSlices) return false;
    const int64_t OH = (d->h + 2 * d->ph - d->dh * (d->kh - 1) - 1) / d->sh + 1;
    const int64_t OW = (d->w + 2 * d->pw - (d->kw - 1) - 1) / d->sw + 1;
    if (OH <= 0 || OW <= 0) return false;
    g.N = int(d->n); g.C = int(d->c); g.H = int(d->h); g.W = int(d->w); g.M = int(d->m);
    g.kh = int(d->kh); g.kw = int(d->kw); g.sh = int(d->sh); g.sw = int(d->sw);
    g.ph = int(d->ph); g.pw = int(d->pw); g.dh = int(d->dh);
    g.OH = int(OH); g.OW = int(OW);
    g.K_pad = 16 * kStemSlices;
    g.prows = (kTile - 1) * g.sh + (g.kh - 1) * g.dh + 1;
    // a fragment reads columns tc * sw + 0..7 of each patch row
    g.pitch = ((kTile - 1) * g.sw + 8 + 3) / 4 * 4;
    g.patch = g.C * g.prows * g.pitch;
    if (g.patch > kMaxPatch || g.prows >= 4096 || g.C >= 256) return false;
    g.tiles_w = (g.OW + kTile - 1) / kTile;
    g.tiles_img = ((g.OH + kTile - 1) / kTile) * g.tiles_w;
    const int64_t tiles = static_cast<int64_t>(d->n) * g.tiles_img;
    // 32-bit offsets below 2^31: one input image, one output image (all 64
    // rows of a tile, also past M)
    if (tiles >= (1LL << 31) || d->c * d->h * d->w * 4 >= (1LL << 31) || kRows * OH * OW * 4 >= (1LL << 31))
        return false;
    g.tiles = int(tiles);
    g.relu = (flags & TBN_EPI_RELU) ? 1 : 0;
    return true;
}

}  // namespace

namespace tbn_hip {

bool conv_stem_supported(const tbn_conv2d_desc* desc, int flags) {
    StemGeom g;
    return stem_geom(desc, flags, g);
}

int conv_stem_run(const float* x, const tbn_conv2d_desc* desc, const float* w, const float* bias, int flags,
                  float* y, hipStream_t s) {
    StemGeom g;
    TBN_REQUIRE(stem_geom(desc, flags, g), TBN_INVALID_SHAPE, "shape not handled by the stem conv kernel");
    if (g.tiles == 0) return ok();
    void* wsplit = nullptr;
    const size_t wbytes = static_cast<size_t>(3) * kRows * g.K_pad * sizeof(uint16_t);
    hipError_t e = hipMallocAsync(&wsplit, wbytes, s);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(e == hipErrorOutOfMemory ? TBN_OUT_OF_MEMORY : TBN_RUNTIME_ERROR,
                    std::string("stem conv weight buffer: ") + hipGetErrorString(e));
    }
    hipLaunchKernelGGL(stem_weights_kernel, dim3(static_cast<unsigned>(ceil_div(kRows * g.K_pad, 256))), dim3(256), 0,
                       s, w, g, static_cast<uint16_t*>(wsplit));
    int rc = check_launch("conv2d_f32 (stem weights)");
    if (rc == TBN_SUCCESS) {
        constexpr int KROW = 16 * kStemSlices + 8;
        const size_t lds = static_cast<size_t>(3) * kRows * KROW * 2 + kRows * 4 + static_cast<size_t>(g.patch) * 4;
        static bool attr_set = false;
        if (!attr_set) {
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&stem_conv_kernel<kStemKW, kStemSlices>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            if (e != hipSuccess) rc = fail(TBN_RUNTIME_ERROR, std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
            else attr_set = true;
        }
        if (rc == TBN_SUCCESS) {
            const int blocks = std::min(g.tiles, stem_cu_count());
            hipLaunchKernelGGL((stem_conv_kernel<kStemKW, kStemSlices>), dim3(blocks), dim3(256), lds, s, x, g,
                               static_cast<const uint16_t*>(wsplit), bias, y);
            rc = check_launch("conv2d_f32 (stem)");
        }
    }
    (void)hipFreeAsync(wsplit, s);
    return rc;
}

}  // namespace tbn_hip
