// fp32 convolution for few input channels and wide kernels: the ResNet stem
// (3 -> 64 channels, 7x7, stride 2).  The im2col engine of conv.hip gathers
// every (pixel, tap) element from global memory and splits it anew; here each
// wave stages the input patch of its output tile in LDS once, split on the
// way into three bf16 planes (hi + mid + lo = x exactly), and reads every
// column fragment from those planes.
//
// K is ordered k = (r * C + c) * 8 + s: tap row r, channel c, tap column s
// padded from kw to 8.  A lane's 8 consecutive k of a k-slice are then 8
// consecutive input columns of one row of one channel: four dword reads per
// plane (the run starts at an even column).  Column 8 of the run (s = kw)
// and k past kh * C have zero weights; their inputs are zeroed too, so an
// infinite pixel there cannot turn into NaN.  Products per k-slice: w_hi x_hi,
// w_hi x_mid, w_mid x_hi, w_hi x_lo, w_mid x_mid, w_lo x_hi (the terms below
// 2^-24 relative dropped), accumulated in fp32.
//
// A block (persistent, one per CU) splits the weights into a [plane][64
// rows][K_pad] bf16 table in LDS once; after that its 8 waves work without
// barriers: each wave takes output tiles of all 64 channels x 4 rows x 16
// columns (two 32-pixel column fragments) with a patch buffer of its own, and
// loads its next tile's patch into registers while computing the current
// one.  Tiles are dealt wave-major across blocks (wave w of every block
// before wave w + 1 of any), so the tiles beyond a whole round land on
// different SIMDs.
//
// With the 3x3 stride-2 pad-1 max pool fused (after ReLU), a wave's tile is
// 3 x 4 pooled outputs: the 7 x 9 conv pixels their windows cover (63 of the
// 64 fragment columns), so the window rows and columns shared with the
// neighbouring tiles are computed by both.  The pool reads the tile back
// from the wave's patch buffer.  After ReLU every value is +0 or more and
// none is NaN, so the maximum does not depend on the order it is taken in
// and equals the separate pool's bit for bit; conv pixels outside the image
// count as 0, which cannot exceed a window's largest in-image value.
#include <algorithm>
#include <mutex>
#include <string>

#include "conv_common.hpp"

namespace {

using namespace tbnk;

constexpr int kRows = 64;    // output channels per tile (M <= 64)
constexpr int kWaves = 8;    // waves per block
constexpr uint32_t kOutside = 0x80000000u;
// fused pool: a wave's tile is kPoolTH x kPoolTW pooled outputs; its 64 x 32
// (pixel, channel) staging table has a pitch of 33 floats (pixels two rows
// apart, read by the two lane halves together, start 18 banks apart)
constexpr int kPoolTH = 3, kPoolTW = 4;
constexpr int kTPitch = 33;
constexpr int kTWords = 64 * kTPitch;

struct StemGeom {
    int N, H, W, M;
    int ph, pw;
    int OH, OW;
    int PH, PW;  // pooled output (fused pool only)
    int tiles_w, tiles_img, tiles;
    int relu;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

// Exact three-way bf16 split of two values, packed as (x0, x1) bf16 pairs.
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
    float x[2] = {x0, x1};
    uint32_t hb[2], mb[2], lb[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t u = __float_as_uint(x[e]);
        const float h = __uint_as_float(u & 0xFFFF0000u);
        const float r1 = (x[e] == h) ? 0.0f : x[e] - h;
        const uint32_t m = __float_as_uint(r1);
        hb[e] = u;
        mb[e] = m;
        lb[e] = __float_as_uint(r1 - __uint_as_float(m & 0xFFFF0000u));
    }
    hi = upper_halves(hb[0], hb[1]);
    mid = upper_halves(mb[0], mb[1]);
    lo = upper_halves(lb[0], lb[1]);
}

// Compile-time geometry: C channels, KH x KW taps, stride SH x SW, no
// dilation (pads, image size, batch and M <= 64 are runtime); a wave's conv
// tile is TR x TC pixels (at most 64), pixel i of the two 32-column
// fragments being tile row i / TC, column i % TC.
template <int C_, int KH_, int KW_, int SH_, int SW_, int TR_, int TC_>
struct StemShape {
    static constexpr int C = C_, KH = KH_, KW = KW_, SH = SH_, SW = SW_, TR = TR_, TC = TC_;
    static constexpr int PIX = TR * TC;
    static constexpr int SLICES = (KH * C + 1) / 2;                    // k8 groups: KH * C, two per slice
    static constexpr int K_PAD = 16 * SLICES;
    static constexpr int KROW = K_PAD + 8;                             // LDS weight row: conflict-free reads
    static constexpr int PROWS = (TR - 1) * SH + KH;                   // a wave's patch rows
    static constexpr int PITCH = ((TC - 1) * SW + 8 + 3) / 4 * 4;      // row pitch (elements)
    static constexpr int PATCH = C * PROWS * PITCH;
    static constexpr int PAIRS = PATCH / 2;                            // dwords per plane
    static constexpr int PER = (PAIRS + 63) / 64;                      // pairs staged per lane
    // a wave's LDS buffer (dwords): the patch's three planes, or the fused
    // pool's staging table after the MFMAs
    static constexpr int WBUF = 3 * PAIRS > kTWords ? 3 * PAIRS : kTWords;
    static constexpr size_t LDS = static_cast<size_t>(3) * kRows * KROW * 2 + kRows * 4 +
                                  static_cast<size_t>(kWaves) * WBUF * 4;
    static_assert(KW <= 8 && SW % 2 == 0 && PITCH % 4 == 0, "a lane's run: 8 columns from an even one");
    static_assert(PIX <= 64, "two 32-pixel fragments");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// POOL: the tile is a pooled tile (kPoolTH x kPoolTW, S::TR = 2 kPoolTH + 1,
// S::TC = 2 kPoolTW + 1) and y is the pooled output.
template <class S, bool POOL>
__global__ void __launch_bounds__(64 * kWaves) stem_conv_kernel(const float* __restrict__ x, StemGeom g,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ y) {
    constexpr int SLICES = S::SLICES, KW = S::KW, KROW = S::KROW, K_PAD = S::K_PAD;
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    uint16_t* wl = lds;                                             // [3][64][KROW]
    float* bl = reinterpret_cast<float*>(lds + 3 * kRows * KROW);  // [64] bias
    const int tid_all = threadIdx.x;
    const int lane = tid_all & 63;
    // wave-uniform (an SGPR), so the tiles, and with them the buffer
    // resources, are too: a resource in VGPRs would loop every load and store
    const int wave = __builtin_amdgcn_readfirstlane(tid_all >> 6);
    constexpr int pplane = S::PAIRS;
    uint32_t* pl = reinterpret_cast<uint32_t*>(bl + kRows) + wave * S::WBUF;  // [3 planes][C][PROWS][PITCH]

    // ---- weights, once per block: item = (row m, k8 = r * C + c), the run
    //      w[m, c, r, 0..kw) split into the three planes (zero past M, KH, KW) ----
    {
        constexpr int kGroups = K_PAD / 8;
        constexpr int kItems = kRows * kGroups;
        constexpr int kPer = (kItems + 64 * kWaves - 1) / (64 * kWaves);
        float v[kPer][8];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int item = tid_all + i * 64 * kWaves;
            const int m = item / kGroups, k8 = item - m * kGroups;
            const int r = k8 / S::C, c = k8 - r * S::C;
            const bool ok = item < kItems && m < g.M && r < S::KH;
            const float* src =
                w + ((static_cast<int64_t>(ok ? m : 0) * S::C + (ok ? c : 0)) * S::KH + (ok ? r : 0)) * KW;
#pragma unroll
            for (int q = 0; q < 8; ++q) v[i][q] = (ok && q < KW) ? src[q] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int item = tid_all + i * 64 * kWaves;
            if (item < kItems) {
                const int m = item / kGroups, k8 = item - m * kGroups;
                uint4 hi, mid, lo;
                split8(v[i], hi, mid, lo);
                uint16_t* d = wl + m * KROW + k8 * 8;
                *reinterpret_cast<uint4*>(d) = hi;
                *reinterpret_cast<uint4*>(d + kRows * KROW) = mid;
                *reinterpret_cast<uint4*>(d + 2 * kRows * KROW) = lo;
            }
        }
    }
    if (tid_all < kRows) bl[tid_all] = (bias && tid_all < g.M) ? bias[tid_all] : 0.0f;
    __syncthreads();  // the only block-wide barrier

    // ---- patch staging: pair p = lane + 64 i = elements 2p, 2p + 1 of
    //      [C][PROWS][PITCH] (the pitch is even: both in one row) ----
    const uint32_t HW = static_cast<uint32_t>(g.H) * g.W;
    float stage[S::PER][2];
    // conv pixel (oh0, ow0) is the tile's first (for a pooled tile starting at
    // pooled (pr0, pc0): conv (2 pr0 - 1, 2 pc0 - 1), the windows' first row
    // and column, possibly -1)
    auto tile_origin = [&](int t, int& n, int& oh0, int& ow0) {
        n = t / g.tiles_img;
        const int r = t - n * g.tiles_img;
        const int th = r / g.tiles_w;
        const int tw = r - th * g.tiles_w;
        if (POOL) {
            oh0 = 2 * th * kPoolTH - 1;
            ow0 = 2 * tw * kPoolTW - 1;
        } else {
            oh0 = th * S::TR;
            ow0 = tw * S::TC;
        }
    };
    auto load_patch = [&](int t) {
        int n, oh0, ow0;
        tile_origin(t, n, oh0, ow0);
        const int ih0 = oh0 * S::SH - g.ph, iw0 = ow0 * S::SW - g.pw;
        // image n: C * H * W floats (host-checked below 2^31 bytes); outside -> 0
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(x + static_cast<int64_t>(n) * S::C * HW, S::C * HW * 4);
#pragma unroll
        for (int i = 0; i < S::PER; ++i) {
            const int e = 2 * (lane + 64 * i);
            const int c = e / (S::PROWS * S::PITCH);
            const int rem = e - c * (S::PROWS * S::PITCH);
            const int pr = rem / S::PITCH;
            const int pc = rem - pr * S::PITCH;
            const int ih = ih0 + pr, iw = iw0 + pc;
            const bool row_ok = e < S::PATCH && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H);
            const uint32_t base = (static_cast<uint32_t>(c) * HW + ih * g.W + iw) * 4;
            const bool ok0 = row_ok && static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
            const bool ok1 = row_ok && static_cast<unsigned>(iw + 1) < static_cast<unsigned>(g.W);
            stage[i][0] =
                __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, ok0 ? base : kOutside, 0, 0));
            stage[i][1] =
                __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, ok1 ? base + 4 : kOutside, 0, 0));
        }
    };
    auto store_patch = [&]() {
#pragma unroll
        for (int i = 0; i < S::PER; ++i) {
            const int p = lane + 64 * i;
            if (p < S::PAIRS) {
                uint32_t hi, mid, lo;
                split2(stage[i][0], stage[i][1], hi, mid, lo);
                pl[p] = hi;
                pl[pplane + p] = mid;
                pl[2 * pplane + p] = lo;
            }
        }
    };

    // ---- this lane's fragment pixels (in dwords of a plane) ----
    const int kg = lane >> 5;
    int pix[2];  // fragment j: tile pixel i = 32 j + lane % 32 (past the tile: pixel 0)
    int prow[2], pcol[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = 32 * j + (lane & 31);
        prow[j] = i < S::PIX ? i / S::TC : 0;
        pcol[j] = i < S::PIX ? i - (i / S::TC) * S::TC : 0;
        pix[j] = (prow[j] * S::SH * S::PITCH + pcol[j] * S::SW) / 2;
    }
    // k8 = 2 sl + kg: tap row r, channel c at dword offset koff(sl, kg) of the patch
    auto koff = [&](int sl, int k) {
        const int k8 = 2 * sl + k;
        const int r = k8 / S::C, c = k8 - r * S::C;
        return (c * S::PROWS + r) * S::PITCH / 2;
    };
    const int wrow = lane & 31;

    // Fragments of slice sl: weights a[plane][f] and inputs b[plane][j]; past
    // KH * C (the last slice, kg = 1 when KH * C is odd) the inputs are zeroed.
    auto read_slice = [&](int sl, u32x4_t (&a)[3][2], u32x4_t (&b)[3][2]) {
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int f = 0; f < 2; ++f)
                a[p][f] = *reinterpret_cast<const u32x4_t*>(wl + (p * kRows + f * 32 + wrow) * KROW + sl * 16 +
                                                            kg * 8);
        const bool last_odd = (2 * sl + 1 >= S::KH * S::C);
        const int ko0 = koff(sl, 0);
        const int ko1 = last_odd ? ko0 : koff(sl, 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t* src = pl + pix[j] + (kg ? ko1 : ko0);
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                u32x4_t v;
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = src[p * pplane + q];
                if (KW == 7) v[3] &= 0x0000FFFFu;  // s = 7
                if (last_odd) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = kg ? 0u : v[q];
                }
                b[p][j] = v;
            }
        }
    };

    // tiles wave-major: wave w of block b takes w * gridDim.x + b, then steps
    // by all the waves of the grid
    const int stride = kWaves * static_cast<int>(gridDim.x);
    int t = wave * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x);
    if (t < g.tiles) load_patch(t);
    for (; t < g.tiles; t += stride) {
        store_patch();
        // a wave's own LDS operations complete in order; the fences keep the
        // compiler from moving the fragment reads above these writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (t + stride < g.tiles) load_patch(t + stride);

        f32x16_t acc[2][2];
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[f][j][e] = 0.0f;
        // per slice: 6 weight and 6 input fragments, 24 MFMAs (products
        // outermost, so consecutive MFMAs go to the four accumulators); the
        // other wave on the SIMD covers the LDS latency
#pragma unroll
        for (int sl = 0; sl < SLICES; ++sl) {
            u32x4_t a[3][2], b[3][2];
            read_slice(sl, a, b);
            constexpr int pa[6] = {0, 0, 1, 0, 1, 2}, pb[6] = {0, 1, 0, 2, 1, 0};
#pragma unroll
            for (int q = 0; q < 6; ++q)
#pragma unroll
                for (int f = 0; f < 2; ++f)
#pragma unroll
                    for (int j = 0; j < 2; ++j) acc[f][j] = mfma32(a[pa[q]][f], b[pb[q]][j], acc[f][j]);
        }
        // the next tile's store overwrites the patch: these reads come first
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        int n, oh0, ow0;
        tile_origin(t, n, oh0, ow0);
        if constexpr (!POOL) {
            // ---- epilogue: + bias, ReLU; buffer stores into image n's output
            //      (rows past M and pixels past the image carry kOutside) ----
            const uint32_t plane = static_cast<uint32_t>(g.OH) * g.OW;
            const __amdgpu_buffer_rsrc_t ys =
                make_rsrc(y + static_cast<int64_t>(n) * g.M * plane, static_cast<uint32_t>(g.M) * plane * 4);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int oh = oh0 + prow[j];
                const int ow = ow0 + pcol[j];
                const bool ok = 32 * j + (lane & 31) < S::PIX && oh < g.OH && ow < g.OW;
                const uint32_t base = ok ? (static_cast<uint32_t>(4 * kg) * plane + oh * g.OW + ow) * 4 : kOutside;
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
        } else {
            // ---- fused pool, one 32-channel half (fragment row f) at a time:
            //      + bias, ReLU (pixels outside the conv output: 0) into
            //      T[pixel][channel] (pitch kTPitch) in the wave's LDS buffer,
            //      then per (channel, pooled row) the column maxima of the
            //      window rows and the four pooled values.  Every T address is
            //      a per-lane base plus a constant offset ----
            float* tl = reinterpret_cast<float*>(pl);
            bool pv[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int oh = oh0 + prow[j], ow = ow0 + pcol[j];
                pv[j] = 32 * j + (lane & 31) < S::PIX && static_cast<unsigned>(oh) < static_cast<unsigned>(g.OH) &&
                        static_cast<unsigned>(ow) < static_cast<unsigned>(g.OW);
            }
            const int pr0 = (oh0 + 1) / 2, pc0 = (ow0 + 1) / 2;
            const uint32_t pplane_out = static_cast<uint32_t>(g.PH) * g.PW;
            const __amdgpu_buffer_rsrc_t ys =
                make_rsrc(y + static_cast<int64_t>(n) * g.M * pplane_out, static_cast<uint32_t>(g.M) * pplane_out * 4);
            const bool vec = (g.PW & 3) == 0;  // four pooled columns are one aligned 16-byte store
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                // the half's biases first: read after the table writes, each
                // would wait for the write before it (both are LDS)
                float bv[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) bv[e] = bl[f * 32 + 8 * (e >> 2) + (e & 3) + 4 * kg];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    float* trow = tl + (32 * j + (lane & 31)) * kTPitch + 4 * kg;
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int ch = 8 * (e >> 2) + (e & 3);  // + 4 kg in trow
                        float v = acc[f][j][e] * 1.0f + bv[e];
                        v = (pv[j] && v > 0.0f) ? v : 0.0f;
                        trow[ch] = v;
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                // tasks (channel, pooled row): lane, and lane + 64 for lanes 0-31
#pragma unroll
                for (int round = 0; round < 2; ++round) {
                    const int task = lane + 64 * round;
                    if (task < 32 * kPoolTH) {
                        const int ch = task & 31, pp = task >> 5;
                        const float* tcol = tl + 2 * pp * S::TC * kTPitch + ch;
                        float m[S::TC];
#pragma unroll
                        for (int b = 0; b < S::TC; ++b) {
                            const float v0 = tcol[b * kTPitch];
                            const float v1 = tcol[(S::TC + b) * kTPitch];
                            const float v2 = tcol[(2 * S::TC + b) * kTPitch];
                            m[b] = fmaxf(fmaxf(v0, v1), v2);
                        }
                        float q[kPoolTW];
#pragma unroll
                        for (int c = 0; c < kPoolTW; ++c) q[c] = fmaxf(fmaxf(m[2 * c], m[2 * c + 1]), m[2 * c + 2]);
                        const int pr = pr0 + pp, cg = f * 32 + ch;
                        const bool row_ok = pr < g.PH && cg < g.M;
                        const uint32_t base = (static_cast<uint32_t>(cg) * pplane_out + pr * g.PW + pc0) * 4;
                        if (vec) {
                            u32x4_t qv;
#pragma unroll
                            for (int c = 0; c < kPoolTW; ++c) qv[c] = __float_as_uint(q[c]);
                            __builtin_amdgcn_raw_buffer_store_b128(qv, ys, row_ok ? base : kOutside, 0, 0);
                        } else {
#pragma unroll
                            for (int c = 0; c < kPoolTW; ++c)
                                __builtin_amdgcn_raw_buffer_store_b32(
                                    __float_as_uint(q[c]), ys, row_ok && pc0 + c < g.PW ? base + 4 * c : kOutside, 0,
                                    0);
                        }
                    }
                }
                // the next half's (or tile's) writes come after these reads
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        }
    }
}

using Stem7x7 = StemShape<3, 7, 7, 2, 2, 4, 16>;  // the ResNet stem: 4 x 16 conv pixels per wave
using Stem7x7Pool = StemShape<3, 7, 7, 2, 2, 2 * kPoolTH + 1, 2 * kPoolTW + 1>;  // with the 3x3/2 pool
static_assert(Stem7x7Pool::WBUF >= kTWords, "the pool's staging table fits the wave's buffer");

// Shapes the stem kernel takes: flags RELU, or RELU | MAXPOOL3X3S2 (the
// pool: 3x3, stride 2, pad 1, floor).
bool stem_geom(const tbn_conv2d_desc* d, int flags, StemGeom& g) {
    using S = Stem7x7;
    if (!d || flags & ~(TBN_EPI_RELU | TBN_EPI_MAXPOOL3X3S2)) return false;
    const bool pool = (flags & TBN_EPI_MAXPOOL3X3S2) != 0;
    if (pool && !(flags & TBN_EPI_RELU)) return false;
    if (d->c != S::C || d->kh != S::KH || d->kw != S::KW || d->sh != S::SH || d->sw != S::SW || d->dh != 1 ||
        d->dw != 1 || d->m > kRows || d->m <= 0)
        return false;
    const int64_t OH = (d->h + 2 * d->ph - (d->kh - 1) - 1) / d->sh + 1;
    const int64_t OW = (d->w + 2 * d->pw - (d->kw - 1) - 1) / d->sw + 1;
    if (OH <= 0 || OW <= 0) return false;
    g.N = int(d->n); g.H = int(d->h); g.W = int(d->w); g.M = int(d->m);
    g.ph = int(d->ph); g.pw = int(d->pw);
    g.OH = int(OH); g.OW = int(OW);
    g.PH = pool ? (g.OH - 1) / 2 + 1 : 0;
    g.PW = pool ? (g.OW - 1) / 2 + 1 : 0;
    if (pool) {
        g.tiles_w = (g.PW + kPoolTW - 1) / kPoolTW;
        g.tiles_img = ((g.PH + kPoolTH - 1) / kPoolTH) * g.tiles_w;
    } else {
        g.tiles_w = (g.OW + S::TC - 1) / S::TC;
        g.tiles_img = ((g.OH + S::TR - 1) / S::TR) * g.tiles_w;
    }
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

template <class S, bool POOL>
int launch_stem(const float* x, const StemGeom& g, const float* w, const float* bias, float* y, hipStream_t s) {
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&stem_conv_kernel<S, POOL>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return fail(TBN_RUNTIME_ERROR, std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
        attr_set = true;
    }
    const int blocks = static_cast<int>(std::min<int64_t>(ceil_div(g.tiles, kWaves), tbn_hip::cu_count()));
    hipLaunchKernelGGL((stem_conv_kernel<S, POOL>), dim3(blocks), dim3(64 * kWaves), S::LDS, s, x, g, w, bias, y);
    return check_launch(POOL ? "conv2d_f32 (stem + 3x3/2 max pool)" : "conv2d_f32 (stem)");
}

int conv_stem_run(const float* x, const tbn_conv2d_desc* desc, const float* w, const float* bias, int flags,
                  float* y, hipStream_t s) {
    StemGeom g;
    TBN_REQUIRE(stem_geom(desc, flags, g), TBN_INVALID_SHAPE, "shape not handled by the stem conv kernel");
    if (g.tiles == 0) return ok();
    if (flags & TBN_EPI_MAXPOOL3X3S2) return launch_stem<Stem7x7Pool, true>(x, g, w, bias, y, s);
    return launch_stem<Stem7x7, false>(x, g, w, bias, y, s);
}

}  // namespace tbn_hip
