// Binary / ternary Conv2D, patch form (inputs of 16 or more channels).
//
// A block owns BM output channels x one spatial tile of TH x TW output pixels
// of one image.  The K loop runs over channel chunks of 32: for each chunk
// the block stages the input patch the tile needs -- ((TH-1)*sh + (kh-1)*dh + 1)
// x ((TW-1)*sw + (kw-1)*dw + 1) pixels x 32 channels -- from the NCHW fp32
// input into LDS, split on the way into three bf16 planes (hi + mid + lo = x
// exactly), zero outside the image.  Every tap of the chunk is then one K step
// of 32 read from the same patch, so each input element is loaded and split
// once per block instead of once per tap, and the chunk's global loads are in
// flight during the previous chunk's kh*kw K steps of MFMAs.
//
// Weights use the conv layout: one 32-bit (binary) or 64-bit (ternary) word
// per (chunk, tap, output channel) holds the 32 channels c % 32 of that
// chunk and tap, words ordered [chunk * taps + tap][channel] (taps = kh*kw),
// so the lanes of a staging load read consecutive words.  It is made once from
// the reference's packed columns by tbn_hip_pack_conv_weights; the block
// stages the chunk's words [tap][channel] into LDS next to the patch, and each
// lane decodes its channel's word to bf16 +-1 / 0 in registers.  The inner
// loop touches only LDS.  Output channels are the MFMA rows, tile pixels the columns; with
// the fused 2x2 max pool the pixels are enumerated window by window so a window
// sits in four neighbouring lanes.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <type_traits>

#include "conv_common.hpp"

namespace {

using namespace tbnk;

constexpr int kChunk = 32;               // channels per K chunk
constexpr int kPix = kChunk + 8;         // bf16 per staged pixel (80 bytes: conflict-free 16-byte reads)
constexpr int kMaxLds = 160 * 1024;      // gfx950 LDS per workgroup

struct PatchGeom {
    int N, C, H, W, M;
    int kh, kw, sh, sw, ph, pw, dh, dw;
    int OH, OW;
    int taps, chunks;      // kh*kw, ceil(C / 32)
    int PHi, PWi;          // staged patch rows / cols
    int tiles_h, tiles_w;  // 2-D tiles per image (linear == 0)
    int pool, PH, PW;      // fused 2x2 pool and its output size
    int VH, VW;            // extent of computed pixels (2*PH x 2*PW when pooling)
    // 1: a tile is QT consecutive pixels (QT/4 pool windows) of one image;
    // 2 (stacked): QT consecutive pixels of the flattened N x OH x OW output,
    // for stride 1: the images are stacked into one tall image in which input
    // row ih of image n is virtual row n * vpitch + ih (vpitch = H + ph), so
    // the ph zero rows below one image are the ph above the next, and output
    // (n, oh) reads virtual rows n * vpitch + oh - ph + r * dh.  A tile's
    // patch is virtual rows [row0, row0 + PHi) at full padded width, and its
    // output runs are whole 4*QT-byte spans of each channel plane.
    int linear;
    int vpitch;            // stacked: virtual rows per image
    int tiles_img;         // tiles per image (stacked: tiles of the whole batch)
    // the kernel's runtime divisors, as branch-free multiply-high dividers:
    // staging item -> channel group and patch pixel -> row (PHi*PWi, PWi);
    // block -> split, channel tile, image, tile row (blocks_split, channel
    // tiles, tiles_img, tiles_w); pixel -> row, window -> row, flattened pixel
    // -> image (OW, PW, OH*OW); virtual row -> image (vpitch)
    UDiv div_patch, div_pwi, div_split, div_mt, div_img, div_tw, div_ow, div_pw, div_plane, div_vpitch;
    // patch sampling: patch pixel (pr, pc) is input (ih0 + pr*psh, iw0 + pc*psw);
    // output (oh, ow) reads patch pixel ((oh-row0)*poh, (ow-col0)*pow).  1x1
    // kernels stage only the pixels they use (psh = sh, poh = 1); others stage
    // the dense rectangle (psh = 1, poh = sh)
    int psh, psw, poh, pow_;
    // split-K over blocks: split s takes chunks [s * cps, min(chunks, (s + 1) * cps))
    // and writes raw sums; blocks_split = blocks of one split
    int splits, cps, blocks_split;
    // the summation order is fixed by the shape: the chunks form groups of
    // gchunks, each summed from zero, the group sums added in group order.
    // Split-K runs one group per block; fold (splits == 1, groups > 1) runs
    // all groups in one block and adds their sums in the same order, so both
    // give the same bits and the batch may choose between them.
    int gchunks, fold;
    // 1: one LDS buffer (the next chunk waits in the staging registers and is
    // stored after a barrier), for twice the blocks per CU; 0: two buffers
    int single;
    // 1: 2-D tiles of 8-pixel rows whose 32-pixel fragments take rows
    // {0, 4, 1, 5} and {2, 6, 3, 7}: with a patch pitch of 2 mod 4 pixels
    // (80-byte records) the two rows one 16-lane group reads then sit in
    // disjoint LDS banks
    int rowperm;
    // 1: the launch also computes the 1x1 projection of the same input from
    // the centre tap (conv_patch_kernel<..., PROJ = true>)
    int proj;
};

// Buffer resource (gfx9 word 3: raw dword addressing) over `bytes` from base;
// loads at offsets past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
    const uint32_t n = bytes > 0xFFFFFFF0ull ? 0xFFFFFFF0u : static_cast<uint32_t>(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(n),
                                             0x00020000);
}

// Output pixel of the tile-local index ql and its patch index.  Linear tiles
// run along the flattened image (pool windows when pooling), so a fragment's
// 32 lanes hold 32 consecutive pixels (or 8 windows) of one channel;
// 2-D tiles are TH x TW blocks.  Pixels past the image are flagged invalid
// and mapped to patch index 0 (their results are never stored).
template <class Cfg>
__device__ __forceinline__ bool tile_pixel(const PatchGeom& g, int q0, int row0, int col0, int ql, int& oh,
                                           int& ow, int& patch_index, int& img) {
    bool valid;
    img = 0;
    if (g.linear == 2) {
        // stacked: image, row and column of flattened pixel q0 + ql
        const int plane = g.OH * g.OW;
        const int q = q0 + ql;
        valid = q < g.N * plane;
        img = valid ? udiv(q, g.div_plane) : 0;
        const int p = q - img * plane;
        oh = udiv(p, g.div_ow);
        ow = p - oh * g.OW;
        patch_index = valid ? (img * g.vpitch + oh - g.ph - row0) * g.PWi + ow : 0;
        return valid;
    }
    if (g.linear) {
        if (g.pool) {
            const int w = q0 + (ql >> 2);
            const int pr = udiv(w, g.div_pw);
            oh = 2 * pr + ((ql >> 1) & 1);
            ow = 2 * (w - pr * g.PW) + (ql & 1);
            valid = w < g.PH * g.PW;
        } else {
            const int q = q0 + ql;
            oh = udiv(q, g.div_ow);
            ow = q - oh * g.OW;
            valid = q < g.OH * g.OW;
        }
    } else {
        int i, j;
        if (g.pool) {
            const int win = ql >> 2;
            i = 2 * (win / (Cfg::TW / 2)) + ((ql >> 1) & 1);
            j = 2 * (win % (Cfg::TW / 2)) + (ql & 1);
        } else {
            i = ql / Cfg::TW;
            j = ql - i * Cfg::TW;
            if (Cfg::TW == 8 && g.rowperm) i = (i & ~3) / 2 + ((i >> 1) & 1) + 4 * (i & 1);
        }
        oh = row0 + i;
        ow = col0 + j;
        valid = oh < g.VH && ow < g.VW;
    }
    patch_index = valid ? ((oh - row0) * g.poh * g.PWi + (ow - col0) * g.pow_) : 0;
    return valid;
}

// KG = 2: two groups of waves, each summing one run of consecutive chunks
// into its own accumulators, the two sums added in group order at the end:
// the order of two folded chunk groups (conv_patch_kernel, make_patch_geom).
template <int BM_, int TH_, int TW_, int WM_, int WQ_, int KG_ = 1>
struct PatchCfg {
    static constexpr int BM = BM_, TH = TH_, TW = TW_, WM = WM_, WQ = WQ_, KG = KG_;
    static constexpr int QT = TH * TW;
    static constexpr int WAVES_M = BM / WM, WAVES_Q = QT / WQ;
    static constexpr int WAVES = WAVES_M * WAVES_Q;  // per K group
    static constexpr int NT = 64 * WAVES * KG;
    static constexpr int FR = WM / 32, FC = WQ / 32;
    static_assert(QT % WQ == 0 && BM % WM == 0 && WM % 32 == 0 && WQ % 32 == 0, "bad tile");
    static_assert(TH % 2 == 0 && TW % 2 == 0, "tiles must hold whole 2x2 pool windows");
    static_assert(NT >= BM, "one thread per channel stages the epilogue factors");
};

// 8 binary weight bits (bit e = weight e, 1 means -1) -> 8 bf16 +-1.0.  Bits
// 16 and up of x must be zero (bits 8..15 are ignored): y holds bit e at e and
// e + 15, so one shift puts bit 2d at 15 and bit 2d+1 at 31.
// `ones` is the +1.0 bf16 pair 0x3F803F80 held in a VGPR, so each dword is one
// shift and one v_and_or_b32.
__device__ __forceinline__ u32x4_t decode_binary8_fast(uint32_t x, uint32_t ones) {
    const uint32_t y = x | (x << 15);
    u32x4_t r;
    r[0] = ((y << 15) & 0x80008000u) | ones;
    r[1] = ((y << 13) & 0x80008000u) | ones;
    r[2] = ((y << 11) & 0x80008000u) | ones;
    r[3] = ((y << 9) & 0x80008000u) | ones;
    return r;
}

template <bool TERNARY>
__device__ __forceinline__ u32x4_t weight_frag(uint2 w, int kk, int kg, uint32_t ones) {
    if (TERNARY) {
        const uint32_t word = kk ? w.y : w.x;
        return decode_ternary8_x2((word >> (16 * kg)) & 0xFFFFu);  // twice the weights
    }
    return decode_binary8_fast(__builtin_amdgcn_ubfe(w.x, 8 * (2 * kk + kg), 16), ones);
}

// v from lane (lane & ~3) | perm[lane & 3] of the same quad (DPP quad_perm).
template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

struct PatchEpi {
    float* y;
    const float* scale;
    float alpha;
    const float* bias;
    const float* residual;
    int flags;
    float* partial;  // split-K: raw sums [split][N][M][OH * OW] instead of y (null: no split)
    // split-K with tile counters (zero on entry, left zero): the last block of
    // each tile adds the splits and runs the epilogue; null: a reduce kernel does
    int* counters;
    // the fused 1x1 projection (PROJ): its conv-layout words [chunk][m], its
    // output (the conv's shape) and epilogue (scale, alpha, bias, flags)
    const uint8_t* proj_w;
    float* proj_y;
    const float* proj_scale;
    float proj_alpha;
    const float* proj_bias;
    int proj_flags;
};

// bf16 elements of one LDS buffer: three planes of patch + 1 pixel records
// (the spare record takes the stores of items past the patch), the weight
// words plus a spare one; rounded to 16 bytes so both buffers stay aligned.
__host__ __device__ inline int patch_buffer_elems(int patch, int words, int word_halves) {
    return (3 * (patch + 1) * kPix + word_halves * words + 8 + 7) / 8 * 8;  // + a 16-byte spare slot
}

// TAPS = 9: 3x3 kernels, taps unrolled and the chunk's weight words held in
// registers; TAPS = 0: any kernel size, words read per tap.  MAXI bounds the
// patch items a thread stages per chunk (4 or 8, the launch picks the smaller
// that fits): the staging registers live through the whole K loop, and 8
// items (64 VGPRs) would cost a wave per SIMD on shapes that need 2.
// PROJ (3x3 taps, pad 1, one K split; host-checked): the launch also computes
// the 1x1 stride-s pad-0 projection of the same input, whose pixel is the 3x3
// window's centre: its K steps are the centre tap's pixel fragments times
// its own weight words (a table after the conv's in each chunk buffer),
// summed chunk after chunk, k-slice after k-slice, hi / mid / lo, as the 1x1
// conv sums them alone, so both give the same bits.  One K group of waves
// only: two groups would split the chunks between them.
template <class Cfg, bool TERNARY, int TAPS, int MAXI, bool FOLD = false, bool PROJ = false>
__global__ void __launch_bounds__(Cfg::NT)
conv_patch_kernel(const float* __restrict__ x, PatchGeom g, const uint8_t* __restrict__ wbits, int64_t col_bytes,
                  int m_alloc, PatchEpi epi) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    // one LDS buffer = the patch (3 planes x (pixels + 1 spare) x kPix bf16)
    // followed by the chunk's weight words [tap][channel] (uint32, or uint2 for
    // ternary) and one spare word; two buffers
    constexpr int kWordHalves = TERNARY ? 4 : 2;       // uint16 per channel word
    const int patch = g.PHi * g.PWi;
    const int plane_elems = (patch + 1) * kPix;
    const int wofs = 3 * plane_elems;                  // weight words after the planes
    // PROJ: the projection's BM words after the conv's table and its spare
    const int pofs = patch_buffer_elems(patch, Cfg::BM * g.taps, kWordHalves);
    const int buf_elems = pofs + (PROJ ? Cfg::BM * kWordHalves : 0);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kgrp = wave / Cfg::WAVES;  // K group
    const int wg = wave - kgrp * Cfg::WAVES;
    const int wm = wg / Cfg::WAVES_Q;
    const int wq = wg % Cfg::WAVES_Q;

    // block -> (channel tile, image, spatial tile); channel tiles of one pixel
    // tile are neighbours in the logical order, and blocks are dealt
    // round-robin over the 8 XCDs, so the logical order runs consecutively on
    // one XCD: the tile's patch is fetched into that XCD's L2 once
    const int tiles_m = (g.M + Cfg::BM - 1) / Cfg::BM;
    int bid = static_cast<int>(blockIdx.x);
    const int sp = udiv(bid, g.div_split);  // K split of this block
    bid -= sp * g.blocks_split;
    if ((g.blocks_split & 7) == 0) bid = (bid & 7) * (g.blocks_split >> 3) + (bid >> 3);
    const int cb = sp * g.cps;                        // the block's chunks [cb, ce)
    const int ce = min(g.chunks, cb + g.cps);
    int st = udiv(bid, g.div_mt);
    const int mt = bid - st * tiles_m;
    const int n = udiv(st, g.div_img);
    st -= n * g.tiles_img;
    const int m0 = mt * Cfg::BM;
    // first pixel / window of a linear tile; first output row / col of the
    // tile (stacked: the patch's first virtual row); the patch's first input
    // row (stacked: virtual row) and column
    int q0 = 0, oh0, ow0, ih0, iw0;
    if (g.linear == 2) {
        q0 = st * Cfg::QT;
        const int plane = g.OH * g.OW;
        const int n0 = udiv(q0, g.div_plane);
        oh0 = n0 * g.vpitch + udiv(q0 - n0 * plane, g.div_ow) - g.ph;
        ow0 = 0;
        ih0 = oh0;
        iw0 = -g.pw;
    } else {
        if (g.linear) {
            q0 = st * (g.pool ? Cfg::QT / 4 : Cfg::QT);
            oh0 = g.pool ? 2 * udiv(q0, g.div_pw) : udiv(q0, g.div_ow);
            ow0 = 0;
        } else {
            const int th = udiv(st, g.div_tw);
            oh0 = th * Cfg::TH;
            ow0 = (st - th * g.tiles_w) * Cfg::TW;
        }
        ih0 = oh0 * g.sh - g.ph;
        iw0 = ow0 * g.sw - g.pw;
    }

    // per-channel epilogue factors of the block's BM channels: loaded now (the
    // load latency hides behind the first chunk), written to LDS after the
    // patch buffers with the first chunk, read back as float4 by the epilogue
    // (buffer loads from ranges that are empty for a null pointer, read 0,
    // then select: no branch or wait lies between these loads and the
    // chunk's)
    float raw_scale, raw_bias;
    {
        const uint32_t mofs = static_cast<uint32_t>(min(m0 + tid, g.M - 1)) * 4;
        const __amdgpu_buffer_rsrc_t s_rs = make_rsrc(epi.scale, epi.scale ? static_cast<uint64_t>(g.M) * 4 : 0);
        const __amdgpu_buffer_rsrc_t b_rs = make_rsrc(epi.bias, epi.bias ? static_cast<uint64_t>(g.M) * 4 : 0);
        raw_scale = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s_rs, mofs, 0, 0));
        raw_bias = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b_rs, mofs, 0, 0));
    }

    // ---- staging of one chunk: patch items = (8-channel group, pixel) and
    //      weight items = (tap, channel) ----
    const int items = 4 * patch;
    const int per_thread = (items + Cfg::NT - 1) / Cfg::NT;  // <= kMaxItems (host-checked)
    constexpr int kMaxItems = MAXI;
    // a weight item is 16 bytes: the words of kWPI neighbouring channels of one
    // tap (one load, one LDS write)
    constexpr int kWPI = TERNARY ? 2 : 4;
    constexpr int kGroupsM = Cfg::BM / kWPI;
    const int witems = kGroupsM * g.taps;
    const int wper_thread = (witems + Cfg::NT - 1) / Cfg::NT;  // <= kMaxWItems (host-checked)
    constexpr int kMaxWItems = TAPS > 0 ? std::min(4, (kGroupsM * TAPS + Cfg::NT - 1) / Cfg::NT) : 4;
    const int64_t img = static_cast<int64_t>(n) * g.C * g.H * g.W;
    const uint32_t HW4 = static_cast<uint32_t>(g.H) * g.W * 4;
    constexpr uint32_t kWordBytes = TERNARY ? 8 : 4;
    // Staging loads are buffer loads at 32-bit byte offsets (host-checked: the
    // image with its channels padded to whole chunks, and the weight columns,
    // stay under 2^31 bytes).  An item outside the image or past the patch
    // gets an offset of at least kOutside, and a channel past C lands past the
    // image's C planes: the range check returns 0 for both, so no load waits
    // on a branch or a select.
    const uint32_t img_bytes = static_cast<uint32_t>(g.C) * HW4;  // stacked: image pitch of the offsets
    const __amdgpu_buffer_rsrc_t x_rs =
        make_rsrc(x + img, static_cast<uint64_t>(img_bytes) * (g.linear == 2 ? g.N : 1));
    const __amdgpu_buffer_rsrc_t w_rs = make_rsrc(wbits, static_cast<uint64_t>(m_alloc) * col_bytes);
    constexpr uint32_t kOutside = 0x80000000u;
    // per item, computed once: chunk-0 byte offset and LDS slot (an item past
    // the patch / the word table writes the spare record after it)
    uint32_t xoff[kMaxItems], woff[kMaxWItems];
    int xslot[kMaxItems], wslot[kMaxWItems];
#pragma unroll
    for (int it = 0; it < kMaxItems; ++it) {
        const int item = tid + it * Cfg::NT;
        const int grp = udiv(item, g.div_patch);
        const int pp = item - grp * patch;
        const int pr = udiv(pp, g.div_pwi);
        int ih = ih0 + pr * g.psh;
        const int iw = iw0 + (pp - pr * g.PWi) * g.psw;
        const bool in_patch = item < items;
        uint32_t img_ofs = 0;
        if (g.linear == 2) {
            // virtual row -> image and row (the rows past H are the zero band;
            // ih stays negative before image 0 and the image test drops the last's)
            const int nv = ih >= 0 ? udiv(ih, g.div_vpitch) : 0;
            ih = ih >= 0 && nv < g.N && ih - nv * g.vpitch < g.H ? ih - nv * g.vpitch : -1;
            img_ofs = static_cast<uint32_t>(nv) * img_bytes;
        }
        const bool ok = in_patch && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                        static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
        xoff[it] = ok ? img_ofs + static_cast<uint32_t>(grp * 8) * HW4 + static_cast<uint32_t>(ih * g.W + iw) * 4
                      : kOutside;
        xslot[it] = in_patch ? pp * kPix + grp * 8 : patch * kPix;
    }
#pragma unroll
    for (int it = 0; it < kMaxWItems; ++it) {
        const int item = tid + it * Cfg::NT;
        const int ml = (item % kGroupsM) * kWPI;
        const int tap = item / kGroupsM;
        const bool ok = item < witems && m0 + ml < m_alloc;  // m_alloc: a multiple of 8
        woff[it] = ok ? (static_cast<uint32_t>(tap) * static_cast<uint32_t>(m_alloc) + static_cast<uint32_t>(m0 + ml)) *
                            kWordBytes
                      : kOutside;
        wslot[it] = (item < witems ? tap * Cfg::BM + ml : Cfg::BM * g.taps) * kWordHalves;
    }
    // With 3x3 taps every thread stages exactly kMaxItems patch items and
    // kMaxWItems weight items (the launch picks MAXI, the smallest of 1, 2, 4,
    // 8 that covers the patch; items past it load from kOutside into the
    // spare slots), so the loads carry no branch, and no wait, between them;
    // other kernels stage per_thread / wper_thread items.
    constexpr bool kAll = TAPS > 0;
    using Stage = float[kMaxItems][8];
    // PROJ: one more 16-byte item, the projection words of kWPI channels
    // (threads below kGroupsM; a row past m_alloc loads 0)
    using WStage = u32x4_t[kMaxWItems + (PROJ ? 1 : 0)];
    Stage stage;
    WStage wstage;
    const uint32_t pchunk = static_cast<uint32_t>(m_alloc) * kWordBytes;  // projection words per chunk
    const __amdgpu_buffer_rsrc_t p_rs =
        make_rsrc(PROJ ? epi.proj_w : nullptr, PROJ ? static_cast<uint64_t>(pchunk) * g.chunks : 0);
    const uint32_t poff = tid < kGroupsM && m0 + tid * kWPI < m_alloc
                              ? static_cast<uint32_t>(m0 + tid * kWPI) * kWordBytes
                              : kOutside;
    (void)p_rs;
    (void)poff;

    auto load_chunk = [&](int ch, Stage& st_, WStage& wst_) {
        const uint32_t cofs = static_cast<uint32_t>(ch * kChunk) * HW4;
        const uint32_t wofs_ch = static_cast<uint32_t>(ch * g.taps) * static_cast<uint32_t>(m_alloc) * kWordBytes;
#pragma unroll
        for (int it = 0; it < kMaxItems; ++it) {
            if (kAll || it < per_thread) {
                const uint32_t o = xoff[it] + cofs;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    st_[it][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x_rs, o + e * HW4, 0, 0));
            }
        }
#pragma unroll
        for (int it = 0; it < kMaxWItems; ++it) {
            if (kAll || it < wper_thread) {
                wst_[it] = __builtin_bit_cast(u32x4_t,
                                              __builtin_amdgcn_raw_buffer_load_b128(w_rs, woff[it] + wofs_ch, 0, 0));
            }
        }
        if constexpr (PROJ)
            wst_[kMaxWItems] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(p_rs, poff + static_cast<uint32_t>(ch) * pchunk, 0, 0));
    };
    auto store_chunk = [&](int b, Stage& st_, WStage& wst_) {
        uint16_t* dst = lds + b * buf_elems;
#pragma unroll
        for (int it = 0; it < kMaxItems; ++it) {
            if (kAll || it < per_thread) {
                uint4 hi, mid, lo;
                split8(st_[it], hi, mid, lo);
                uint16_t* d = dst + xslot[it];
                *reinterpret_cast<uint4*>(d) = hi;
                *reinterpret_cast<uint4*>(d + plane_elems) = mid;
                *reinterpret_cast<uint4*>(d + 2 * plane_elems) = lo;
            }
        }
#pragma unroll
        for (int it = 0; it < kMaxWItems; ++it) {
            if (kAll || it < wper_thread) {
                *reinterpret_cast<u32x4_t*>(dst + wofs + wslot[it]) = wst_[it];
            }
        }
        if constexpr (PROJ) {
            if (tid < kGroupsM) *reinterpret_cast<u32x4_t*>(dst + pofs + tid * kWPI * kWordHalves) = wst_[kMaxWItems];
        }
    };

    // ---- this lane's pixels (fragment columns) inside the patch ----
    int pbase[Cfg::FC];
#pragma unroll
    for (int j = 0; j < Cfg::FC; ++j) {
        int oh, ow, pi, im;
        tile_pixel<Cfg>(g, q0, oh0, ow0, wq * Cfg::WQ + j * 32 + (lane & 31), oh, ow, pi, im);
        pbase[j] = pi * kPix;
    }
    // this lane's weight rows (fragment rows) inside the chunk's word table
    const int wrow = wm * Cfg::WM + (lane & 31);

    f32x16_t acc[Cfg::FR][Cfg::FC];
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    // PROJ: the projection's sums (one K group of waves, host-checked)
    f32x16_t accp[PROJ ? Cfg::FR : 1][PROJ ? Cfg::FC : 1];
    static_assert(!PROJ || Cfg::KG == 1, "a fused projection runs on one K group");
    if constexpr (PROJ) {
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) accp[i][j][e] = 0.0f;
    }
    (void)accp;

    // KG = 2: K group k sums the cpg chunks [cb + k * cpg, cb + (k + 1) * cpg)
    // from zero (host-checked: the block's range is a folded pair of equal
    // chunk groups).  Every thread stages both runs, run k's chunk i into
    // buffer k + 2 (i & 1), so the groups advance together between the
    // block's barriers.
    const int cpg = (ce - cb) / Cfg::KG;
    const int nbuf = g.single ? 1 : (Cfg::KG > 1 && cpg > 1 ? 4 : 2);
    Stage stage2;
    WStage wstage2;
    load_chunk(cb, stage, wstage);
    if constexpr (Cfg::KG > 1) load_chunk(cb + cpg, stage2, wstage2);
    store_chunk(0, stage, wstage);
    // [BM] multipliers, [BM] addends after the buffer(s)
    float* epi_lds = reinterpret_cast<float*>(lds + nbuf * buf_elems);
    if (tid < Cfg::BM) {
        epi_lds[tid] = epi.alpha * (epi.scale ? raw_scale : 1.0f);
        epi_lds[Cfg::BM + tid] = raw_bias;
    }
    if constexpr (Cfg::KG > 1) {
        store_chunk(1, stage2, wstage2);
        if (cpg > 1) {
            load_chunk(cb + 1, stage, wstage);
            load_chunk(cb + cpg + 1, stage2, wstage2);
        }
    } else if (cb + 1 < ce) {
        load_chunk(cb + 1, stage, wstage);
    }
    __syncthreads();

    const int kg = lane >> 5;
    uint32_t ones;
    asm volatile("v_mov_b32 %0, 0x3f803f80" : "=v"(ones));
    // FOLD: the sums of the finished chunk groups
    f32x16_t hold[FOLD ? Cfg::FR : 1][FOLD ? Cfg::FC : 1];
    bool held = false;
    int in_group = 0;
    (void)hold;
    (void)held;
    (void)in_group;
    // patch offset of tap (r, s): (r*dh*PWi + s*dw) * kPix
    const int tap_ds = g.dw * kPix;
    const int tap_dr = g.dh * g.PWi * kPix;
    for (int i = 0; i < cpg; ++i) {
        const int ch = cb + kgrp * cpg + i;
        const uint16_t* cur = lds + (g.single ? 0 : Cfg::KG > 1 ? kgrp + 2 * (i & 1) : (i & 1)) * buf_elems;
        auto read_b = [&](int toff, int kk, u32x4_t (&b)[3][Cfg::FC]) {
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
                    b[p][j] = *reinterpret_cast<const u32x4_t*>(cur + p * plane_elems + pbase[j] + toff + kk * 16 +
                                                                 kg * 8);
        };
        auto mfma_step = [&](const u32x4_t (&a)[Cfg::FR], const u32x4_t (&b)[3][Cfg::FC]) {
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j) acc[f][j] = mfma32(a[f], b[p][j], acc[f][j]);
        };
        if constexpr (TAPS > 0) {
            // the chunk's words for this lane's rows, every tap, in registers
            // (read before the first pixel fragments so no wait covers both)
            uint2 wr[Cfg::FR][TAPS];
#pragma unroll
            for (int tap = 0; tap < TAPS; ++tap)
#pragma unroll
                for (int f = 0; f < Cfg::FR; ++f) {
                    const uint16_t* src = cur + wofs + (tap * Cfg::BM + wrow + f * 32) * kWordHalves;
                    if (TERNARY) wr[f][tap] = *reinterpret_cast<const uint2*>(src);
                    else wr[f][tap] = make_uint2(*reinterpret_cast<const uint32_t*>(src), 0u);
                }
            uint2 pwr[PROJ ? Cfg::FR : 1];
            if constexpr (PROJ) {
#pragma unroll
                for (int f = 0; f < Cfg::FR; ++f) {
                    const uint16_t* src = cur + pofs + (wrow + f * 32) * kWordHalves;
                    if (TERNARY) pwr[f] = *reinterpret_cast<const uint2*>(src);
                    else pwr[f] = make_uint2(*reinterpret_cast<const uint32_t*>(src), 0u);
                }
            }
            (void)pwr;
            // software pipeline over the 2*TAPS steps (tap, kk): step t+1's
            // pixel fragments are read from LDS and its weight fragments decoded
            // while step t's MFMAs run; the scheduling barriers keep each
            // step's reads ahead of its MFMAs so no LDS wait lands in the chain
            u32x4_t bcur[3][Cfg::FC], acur[Cfg::FR];
            read_b(0, 0, bcur);
#pragma unroll
            for (int f = 0; f < Cfg::FR; ++f) acur[f] = weight_frag<TERNARY>(wr[f][0], 0, kg, ones);
#pragma unroll
            for (int t = 0; t < 2 * TAPS; ++t) {
                const int nt = (t + 1) >> 1, nk = (t + 1) & 1;
                u32x4_t bnext[3][Cfg::FC], anext[Cfg::FR];
                if (t + 1 < 2 * TAPS) read_b((nt / 3) * tap_dr + (nt % 3) * tap_ds, nk, bnext);
                __builtin_amdgcn_sched_barrier(0);
                mfma_step(acur, bcur);
                if constexpr (PROJ) {
                    // the centre tap's two k-slices (tap 4 = (1, 1)) are the
                    // projection's K steps for this chunk
                    if (t == 8 || t == 9) {
                        u32x4_t ap[Cfg::FR];
#pragma unroll
                        for (int f = 0; f < Cfg::FR; ++f) ap[f] = weight_frag<TERNARY>(pwr[f], t & 1, kg, ones);
#pragma unroll
                        for (int p = 0; p < 3; ++p)
#pragma unroll
                            for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                                for (int j = 0; j < Cfg::FC; ++j) accp[f][j] = mfma32(ap[f], bcur[p][j], accp[f][j]);
                    }
                }
                if (t + 1 < 2 * TAPS) {
#pragma unroll
                    for (int f = 0; f < Cfg::FR; ++f) anext[f] = weight_frag<TERNARY>(wr[f][nt], nk, kg, ones);
                }
#pragma unroll
                for (int q = 0; q < 3 * Cfg::FR * Cfg::FC; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1 < 2 * TAPS) {
#pragma unroll
                    for (int p = 0; p < 3; ++p)
#pragma unroll
                        for (int j = 0; j < Cfg::FC; ++j) bcur[p][j] = bnext[p][j];
#pragma unroll
                    for (int f = 0; f < Cfg::FR; ++f) acur[f] = anext[f];
                }
            }
        } else {
            // steps = (tap, kk) pairs; the B fragments of step t+1 are read from
            // LDS while the MFMAs of step t run
            u32x4_t bcur[3][Cfg::FC], bnext[3][Cfg::FC];
            read_b(0, 0, bcur);
            int toff = 0, s = 0;
            uint2 w[Cfg::FR];
            for (int tap = 0; tap < g.taps; ++tap) {
#pragma unroll
                for (int f = 0; f < Cfg::FR; ++f) {
                    const uint16_t* src = cur + wofs + (tap * Cfg::BM + wrow + f * 32) * kWordHalves;
                    if (TERNARY) w[f] = *reinterpret_cast<const uint2*>(src);
                    else w[f] = make_uint2(*reinterpret_cast<const uint32_t*>(src), 0u);
                }
                // next tap's patch offset
                int next_toff = toff + tap_ds, next_s = s + 1;
                if (next_s == g.kw) {
                    next_s = 0;
                    next_toff = toff + tap_dr - (g.kw - 1) * tap_ds;
                }
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    if (kk == 0) read_b(toff, 1, bnext);
                    else if (tap + 1 < g.taps) read_b(next_toff, 0, bnext);
                    u32x4_t a[Cfg::FR];
#pragma unroll
                    for (int f = 0; f < Cfg::FR; ++f) a[f] = weight_frag<TERNARY>(w[f], kk, kg, ones);
                    mfma_step(a, bcur);
#pragma unroll
                    for (int p = 0; p < 3; ++p)
#pragma unroll
                        for (int j = 0; j < Cfg::FC; ++j) bcur[p][j] = bnext[p][j];
                }
                toff = next_toff;
                s = next_s;
            }
        }
        if constexpr (FOLD && Cfg::KG == 1) {
            // a group ends: its sum joins the earlier groups' (in group order)
            if (++in_group == g.gchunks && ch + 1 < ce) {
                in_group = 0;
#pragma unroll
                for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            hold[f][j][e] = held ? hold[f][j][e] + acc[f][j][e] : acc[f][j][e];
                            acc[f][j][e] = 0.0f;
                        }
                held = true;
            }
        }
        if (Cfg::KG == 1 && ch + 1 < ce) {
            if (g.single) __syncthreads();  // every wave is done reading the buffer
            store_chunk(g.single ? 0 : (ch + 1 - cb) & 1, stage, wstage);
            if (ch + 2 < ce) load_chunk(ch + 2, stage, wstage);
        }
        if (Cfg::KG > 1 && i + 1 < cpg) {
            // both runs' next chunks into the buffers read one step ago
            store_chunk(2 * ((i + 1) & 1), stage, wstage);
            store_chunk(1 + 2 * ((i + 1) & 1), stage2, wstage2);
            if (i + 2 < cpg) {
                load_chunk(cb + i + 2, stage, wstage);
                load_chunk(cb + cpg + i + 2, stage2, wstage2);
            }
        }
        __syncthreads();
    }
    if constexpr (FOLD) {
        if (held) {
#pragma unroll
            for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[f][j][e] = hold[f][j][e] + acc[f][j][e];
        }
    }
    if constexpr (Cfg::KG > 1) {
        // group 1 hands its sums to group 0 through the (now free) patch
        // buffers, [wave][f][j][e][lane]; group 0 adds them after its own
        float* red = reinterpret_cast<float*>(lds);
        constexpr int kVals = Cfg::FR * Cfg::FC * 16;
        float* mine = red + wg * kVals * 64 + lane;
        if (kgrp == 1) {
#pragma unroll
            for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) mine[((f * Cfg::FC + j) * 16 + e) * 64] = acc[f][j][e];
        }
        __syncthreads();
        if (kgrp != 0) return;
#pragma unroll
        for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[f][j][e] += mine[((f * Cfg::FC + j) * 16 + e) * 64];
    }

    if constexpr (TERNARY) {
        // the ternary weights went in as twice their value (exact to undo)
#pragma unroll
        for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[f][j][e] *= 0.5f;
        if constexpr (PROJ) {
#pragma unroll
            for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) accp[f][j][e] *= 0.5f;
        }
    }

    // ---- epilogue: scale, bias, residual, ReLU, optional 2x2 max pool ----
    // Outputs go out as buffer stores at 32-bit offsets into image n's planes
    // from channel m0 on (host-checked: M + 128 planes stay under 2^31
    // bytes): rows past M fall beyond the resource and lanes without a pixel
    // to store carry kOutside, so the range check drops both with no branch.
    const bool pool = g.pool != 0;
    const uint32_t plane = pool ? static_cast<uint32_t>(g.PH * g.PW) : static_cast<uint32_t>(g.OH * g.OW);
    const uint32_t plane4 = plane * 4;
    const int64_t obase = (static_cast<int64_t>(n) * g.M + m0) * plane;
    // stacked tiles address every image's planes from channel m0 of image 0
    // (host-checked: M is a multiple of BM, so rows never pass M, and the
    // batch's output stays under 2^31 bytes)
    const uint32_t obytes = static_cast<uint32_t>((g.linear == 2 ? g.N * g.M : g.M) - m0) * plane4;
    const __amdgpu_buffer_rsrc_t y_rs = make_rsrc(epi.y + obase, obytes);
    const int rlane = wm * Cfg::WM + 4 * (lane >> 5);  // row of register 0 of fragment 0, from m0
    uint32_t voff[Cfg::FC];
#pragma unroll
    for (int j = 0; j < Cfg::FC; ++j) {
        int oh, ow, pi, im;
        const bool valid = tile_pixel<Cfg>(g, q0, oh0, ow0, wq * Cfg::WQ + j * 32 + (lane & 31), oh, ow, pi, im);
        const uint32_t pix = pool ? static_cast<uint32_t>((oh >> 1) * g.PW + (ow >> 1))
                                  : static_cast<uint32_t>(oh * g.OW + ow);
        const bool keep = valid && (!pool || (lane & 3) == 0);
        voff[j] = keep ? (static_cast<uint32_t>(im) * g.M + rlane) * plane4 + pix * 4 : kOutside;
    }
    if (epi.partial) {
        // split-K (never with the pool, host-checked): raw sums of this
        // block's chunks into split sp's plane set, stored with the
        // device-scope policy (sc1).  With tile counters, splitk_arrive
        // orders every wave's stores before the count and the count before
        // the last block's loads; that block adds the splits in split order
        // (as the reduce kernel does) and runs the epilogue below.
        constexpr int kDeviceScope = 16;
        const int64_t split_elems = static_cast<int64_t>(g.N) * g.M * plane;
        const __amdgpu_buffer_rsrc_t p_rs = make_rsrc(epi.partial + sp * split_elems + obase, obytes);
#pragma unroll
        for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    // through a VGPR: stored straight from the accumulator
                    // registers, hipcc put one register's value in all 16 stores
                    uint32_t v;
                    asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "v"(acc[f][j][e]));
                    __builtin_amdgcn_raw_buffer_store_b32(v, p_rs, voff[j] + (f * 32 + 8 * (e >> 2) + (e & 3)) * plane4,
                                                          0, kDeviceScope);
                }
        if (!epi.counters) return;
        // the flag lives in the patch buffers, free once every wave is past
        // its last MFMA (the first barrier inside splitk_arrive); no static
        // LDS: the dynamic size may be the maximum
        if (!splitk_arrive(epi.counters + bid, g.splits, reinterpret_cast<int*>(lds))) return;
        for (int s2 = 0; s2 < g.splits; ++s2) {
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(epi.partial + s2 * split_elems + obase, obytes);
#pragma unroll
            for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const float v = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(
                                       rs, voff[j] + (f * 32 + 8 * (e >> 2) + (e & 3)) * plane4, 0, kDeviceScope));
                        acc[f][j][e] = s2 == 0 ? v : acc[f][j][e] + v;
                    }
        }
        // ready for the next launch on this workspace
        if (tid == 0) __hip_atomic_store(epi.counters + bid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (PROJ) {
        // the projection's epilogue (never pooled, no residual, no split;
        // host-checked): its factors formed as the conv's are, then
        // v = (acc + a) * s + b and an optional ReLU, into the same pixels
        const __amdgpu_buffer_rsrc_t py_rs = make_rsrc(epi.proj_y + obase, obytes);
        const __amdgpu_buffer_rsrc_t ps_rs =
            make_rsrc(epi.proj_scale, epi.proj_scale ? static_cast<uint64_t>(g.M) * 4 : 0);
        const __amdgpu_buffer_rsrc_t pb_rs =
            make_rsrc(epi.proj_bias, epi.proj_bias ? static_cast<uint64_t>(g.M) * 4 : 0);
        const bool pbts = (epi.proj_flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
        const bool prelu = (epi.proj_flags & TBN_EPI_RELU) != 0;
#pragma unroll
        for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                const int r = wm * Cfg::WM + f * 32 + 8 * e4 + 4 * (lane >> 5);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t mo = static_cast<uint32_t>(min(m0 + r + i, g.M - 1)) * 4;
                    const float sc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ps_rs, mo, 0, 0));
                    const float bi = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pb_rs, mo, 0, 0));
                    const float mm = epi.proj_alpha * (epi.proj_scale ? sc : 1.0f);
                    const float a = pbts ? bi : 0.0f, b = pbts ? 0.0f : bi;
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j) {
                        float v = (accp[f][j][4 * e4 + i] + a) * mm + b;
                        if (prelu) v = v > 0.0f ? v : 0.0f;
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), py_rs,
                                                              voff[j] + (f * 32 + 8 * e4 + i) * plane4, 0, 0);
                    }
                }
            }
    }
    // v' = (v + a) * s + b with (a, b) = (bias, 0) for bias-then-scale, else (0, bias)
    const bool bts = (epi.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
    auto finish = [&](auto relu_c, auto pool_c, auto res_c) {
        constexpr bool RELU = decltype(relu_c)::value, POOL = decltype(pool_c)::value, RES = decltype(res_c)::value;
        // residual (never with the pool, host-checked): all loads issued before
        // the first store, which the compiler could not move them across
        float res[Cfg::FR][Cfg::FC][16];
        if constexpr (RES) {
            const __amdgpu_buffer_rsrc_t r_rs = make_rsrc(epi.residual + obase, obytes);
#pragma unroll
            for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        res[f][j][e] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(
                                       r_rs, voff[j] + (f * 32 + 8 * (e >> 2) + (e & 3)) * plane4, 0, 0));
        }
#pragma unroll
        for (int f = 0; f < Cfg::FR; ++f)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                // rows of registers 4*e4 .. 4*e4+3: four consecutive channels
                const int r = wm * Cfg::WM + f * 32 + 8 * e4 + 4 * (lane >> 5);
                const float4 mv = *reinterpret_cast<const float4*>(epi_lds + r);
                const float4 bv = *reinterpret_cast<const float4*>(epi_lds + Cfg::BM + r);
                const float mm[4] = {mv.x, mv.y, mv.z, mv.w};
                const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int e = 4 * e4 + i;
                        const float a = bts ? bb[i] : 0.0f, b = bts ? 0.0f : bb[i];
                        float v = (acc[f][j][e] + a) * mm[i] + b;
                        if constexpr (RES) v += res[f][j][e];
                        if constexpr (RELU) v = v > 0.0f ? v : 0.0f;
                        if constexpr (POOL) {
                            v = fmaxf(v, quad_perm<0xB1>(v));  // partner across the window's columns
                            v = fmaxf(v, quad_perm<0x4E>(v));  // and rows
                        }
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), y_rs,
                                                              voff[j] + (f * 32 + 8 * e4 + i) * plane4, 0, 0);
                    }
            }
    };
    using T = std::true_type;
    using F = std::false_type;
    const bool relu = (epi.flags & TBN_EPI_RELU) != 0;
    if (pool) {
        if (relu) finish(T{}, T{}, F{});
        else finish(F{}, T{}, F{});
    } else if (epi.residual) {
        if (relu) finish(T{}, F{}, T{});
        else finish(F{}, F{}, T{});
    } else {
        if (relu) finish(T{}, F{}, F{});
        else finish(F{}, F{}, F{});
    }
}

// Split-K sum and epilogue: y = the kernel's epilogue applied to the splits'
// raw sums added in split order (element i of the [N][M][OH * OW] output).
__global__ void __launch_bounds__(256) conv_splitk_reduce_kernel(const float* __restrict__ partial, int splits,
                                                                 int64_t total, int M, int plane, PatchEpi epi) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const bool bts = (epi.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        float v = partial[i];
        for (int sp = 1; sp < splits; ++sp) v += partial[static_cast<int64_t>(sp) * total + i];
        const int m = static_cast<int>((i / plane) % M);
        const float mm = epi.alpha * (epi.scale ? epi.scale[m] : 1.0f);
        const float bb = epi.bias ? epi.bias[m] : 0.0f;
        const float a = bts ? bb : 0.0f, b = bts ? 0.0f : bb;
        v = (v + a) * mm + b;
        if (epi.residual) v += epi.residual[i];
        if (epi.flags & TBN_EPI_RELU) v = v > 0.0f ? v : 0.0f;
        epi.y[i] = v;
    }
}

// ---------------------------------------------------------------------------
// Weight re-order: reference k = c*taps + tap  ->  k' = ((c/32)*taps + tap)*32 + c%32
// ---------------------------------------------------------------------------

struct ConvWeightDims {
    int M, C, taps, chunks;
    int64_t K_pad;   // reference layout column: K_pad/8 bytes (binary) or K_pad/4 (ternary)
    int64_t Kc;      // conv layout k' count: chunks * taps * 32
    int M_alloc;     // columns written: ceil8(M)
};

__device__ __forceinline__ bool conv_k_to_ref(const ConvWeightDims& d, int64_t kp, int64_t& k) {
    const int64_t step = kp / kChunk;
    const int cl = static_cast<int>(kp - step * kChunk);
    const int ch = static_cast<int>(step / d.taps);
    const int tap = static_cast<int>(step - static_cast<int64_t>(ch) * d.taps);
    const int c = ch * kChunk + cl;
    if (c >= d.C) return false;
    k = static_cast<int64_t>(c) * d.taps + tap;
    return true;
}

// One thread per output byte; padding channels and columns get +1 (bit 0),
// which meets zero activations.
// Output byte t of the conv layout, words of `wb` bytes ordered
// [step][channel] (step = chunk * taps + tap): its channel m and its byte kb
// within that channel's k' order (32 k' per step).
__device__ __forceinline__ void conv_layout_byte(const ConvWeightDims& d, int64_t t, int wb, int& m, int64_t& kb) {
    const int64_t word = t / wb;
    const int64_t step = word / d.M_alloc;
    m = static_cast<int>(word - step * d.M_alloc);
    kb = step * wb + (t - word * wb);
}

__global__ void reorder_conv_binary_kernel(const uint8_t* __restrict__ ref, ConvWeightDims d,
                                           uint8_t* __restrict__ out) {
    const int64_t bpc = d.Kc / 8;
    const int64_t total = static_cast<int64_t>(d.M_alloc) * bpc;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int m;
        int64_t kb;
        conv_layout_byte(d, t, 4, m, kb);
        uint32_t byte = 0;
        if (m < d.M) {
            const uint8_t* col = ref + m * (d.K_pad / 8);
            for (int e = 0; e < 8; ++e) {
                int64_t k;
                if (conv_k_to_ref(d, kb * 8 + e, k)) byte |= ((col[k >> 3] >> (k & 7)) & 1u) << e;
            }
        }
        out[t] = static_cast<uint8_t>(byte);
    }
}

// Ternary: four codes per byte; padding code 01 (0).
__global__ void reorder_conv_ternary_kernel(const uint8_t* __restrict__ ref, ConvWeightDims d,
                                            uint8_t* __restrict__ out) {
    const int64_t bpc = d.Kc / 4;
    const int64_t total = static_cast<int64_t>(d.M_alloc) * bpc;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int m;
        int64_t kb;
        conv_layout_byte(d, t, 8, m, kb);
        uint32_t byte = 0x55u;
        if (m < d.M) {
            const uint8_t* col = ref + m * (d.K_pad / 4);
            byte = 0;
            for (int e = 0; e < 4; ++e) {
                int64_t k;
                uint32_t code = 1u;
                if (conv_k_to_ref(d, kb * 4 + e, k)) code = (col[k >> 2] >> ((k & 3) * 2)) & 3u;
                byte |= code << (2 * e);
            }
        }
        out[t] = static_cast<uint8_t>(byte);
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

int64_t conv_weight_bytes(int weights, const tbn_conv2d_desc* d) {
    const int64_t Kc = (d->c + kChunk - 1) / kChunk * d->kh * d->kw * kChunk;
    return (d->m + 7) / 8 * 8 * Kc / (weights == TBN_WEIGHTS_BINARY ? 8 : 4);
}

struct TileChoice {
    int cfg;     // index into the PatchCfg menu
    int linear;  // 2: stacked linear tiles, 1: linear tiles, 0: 2-D tiles
    int TH, TW, BM, NT;
    int single;  // 1: one LDS buffer
    int kg;      // K groups of waves (PatchCfg::KG)
    int WM, WQ;  // wave tile (PatchCfg::WM, WQ)
};

size_t lds_bytes(const PatchGeom& g, int BM, bool ternary, int kg = 1) {
    // (a fused projection's words follow the conv's table)
    const size_t buf =
        static_cast<size_t>(patch_buffer_elems(g.PHi * g.PWi, BM * g.taps, ternary ? 4 : 2) + (g.proj ? BM * (ternary ? 4 : 2) : 0)) * 2;
    // two K groups over runs of more than one chunk: two buffers per run
    const int nbuf = g.single ? 1 : (kg > 1 && g.cps > kg ? 4 : 2);
    return nbuf * buf + 2 * sizeof(float) * BM;  // buffer(s) + epilogue factors
}

// Tiles of one launch (per split): stacked tiles cover the whole batch.
int64_t patch_tiles(const PatchGeom& g) { return static_cast<int64_t>(g.linear == 2 ? 1 : g.N) * g.tiles_img; }

// Stacked tiles apply to stride-1 convs whose channels fill whole chunks (a
// chunk never reads past C into the next image), whose output channels fill
// whole BM tiles, without the fused pool, with ph <= (kh-1)*dh (then a later
// pixel of a tile never sits on an earlier virtual row), and whose batch
// input and output fit 31-bit offsets.
bool stacked_ok(const PatchGeom& g, int BM) {
    const int64_t in_bytes = static_cast<int64_t>(g.N) * g.C * g.H * g.W * 4;
    const int64_t out_bytes = static_cast<int64_t>(g.N) * g.M * g.OH * g.OW * 4;
    return g.sh == 1 && g.sw == 1 && g.C % kChunk == 0 && g.M % BM == 0 && !g.pool && g.ph <= (g.kh - 1) * g.dh &&
           in_bytes < (int64_t(1) << 31) && out_bytes < (int64_t(1) << 31);
}

// The tile-dependent dividers (blocks_split and the split's divider are set
// at launch, once the channel tile is known).
void set_dividers(PatchGeom& g) {
    g.div_patch = make_udiv(static_cast<uint32_t>(g.PHi * g.PWi));
    g.div_pwi = make_udiv(static_cast<uint32_t>(g.PWi));
    g.div_img = make_udiv(static_cast<uint32_t>(std::max(1, g.tiles_img)));
    g.div_tw = make_udiv(static_cast<uint32_t>(std::max(1, g.tiles_w)));
    g.div_ow = make_udiv(static_cast<uint32_t>(std::max(1, g.OW)));
    g.div_pw = make_udiv(static_cast<uint32_t>(std::max(1, g.PW)));
    g.div_plane = make_udiv(static_cast<uint32_t>(std::max(1, g.OH * g.OW)));
    g.div_vpitch = make_udiv(static_cast<uint32_t>(std::max(1, g.vpitch)));
}

void fill_patch(PatchGeom& g, const TileChoice& c) {
    g.linear = c.linear;
    g.single = c.single;
    g.rowperm = 0;
    g.vpitch = g.H + g.ph;
    if (c.linear == 2) {
        // a run of QT pixels spans at most `rows` output rows and crosses at
        // most `bounds` image boundaries, each of which skips vpitch - OH
        // virtual rows more than a row step
        const int QT = c.TH * c.TW;
        const int plane = g.OH * g.OW;
        g.tiles_img = static_cast<int>((static_cast<int64_t>(g.N) * plane + QT - 1) / QT);
        const int rows = (g.OW - 1 + QT - 1) / g.OW + 1;
        const int bounds = (plane - 1 + QT - 1) / plane;
        g.tiles_h = g.tiles_w = 0;
        g.psh = g.psw = g.poh = g.pow_ = 1;
        g.PHi = rows - 1 + bounds * std::max(0, g.vpitch - g.OH) + (g.kh - 1) * g.dh + 1;
        g.PWi = g.W + 2 * g.pw;
        set_dividers(g);
        return;
    }
    int rows, cols;  // output rows / columns one tile's pixels span (at most)
    if (c.linear) {
        const int per = g.pool ? c.TH * c.TW / 4 : c.TH * c.TW;
        const int total = g.pool ? g.PH * g.PW : g.OH * g.OW;
        const int rowlen = g.pool ? g.PW : g.OW;
        g.tiles_img = (total + per - 1) / per;
        int span = 1;
        for (int t = 0; t < g.tiles_img; ++t) {
            const int first = t * per / rowlen;
            const int last = (std::min((t + 1) * per, total) - 1) / rowlen;
            span = std::max(span, last - first + 1);
        }
        rows = g.pool ? 2 * span : span;
        cols = g.OW;
        g.tiles_h = g.tiles_w = 0;
    } else {
        rows = c.TH;
        cols = c.TW;
        g.tiles_h = (g.VH + c.TH - 1) / c.TH;
        g.tiles_w = (g.VW + c.TW - 1) / c.TW;
        g.tiles_img = g.tiles_h * g.tiles_w;
    }
    const bool compact = g.kh == 1 && g.kw == 1;
    g.psh = compact ? g.sh : 1;
    g.psw = compact ? g.sw : 1;
    g.poh = compact ? 1 : g.sh;
    g.pow_ = compact ? 1 : g.sw;
    g.PHi = compact ? rows : (rows - 1) * g.sh + (g.kh - 1) * g.dh + 1;
    g.PWi = compact ? cols : (cols - 1) * g.sw + (g.kw - 1) * g.dw + 1;
    set_dividers(g);
    g.rowperm = (!c.linear && !g.pool && c.TH == 8 && c.TW == 8 && g.PWi % 4 == 2) ? 1 : 0;
}

// Tile menu: (BM, TH, TW, wave tile); TH x TW is also the pixel count of a
// linear tile.
using P0 = PatchCfg<128, 8, 16, 64, 64>;  // 24 MFMA per wave per K step
using P1 = PatchCfg<128, 8, 8, 64, 32>;
using P2 = PatchCfg<64, 8, 16, 32, 64>;
using P3 = PatchCfg<64, 8, 8, 32, 32>;
using P4 = PatchCfg<32, 8, 8, 32, 32>;    // <= 32 output channels
using P5 = PatchCfg<128, 4, 8, 64, 32>;   // small 2-D patches (strided / large kernels)
using P6 = PatchCfg<64, 4, 8, 32, 32>;
using P7 = PatchCfg<64, 8, 8, 64, 32>;    // 64 channels per wave: each pixel fragment feeds 2 MFMAs
using P8 = PatchCfg<64, 8, 16, 64, 32>;
using P9 = PatchCfg<128, 8, 8, 32, 32>;   // 8 waves: two per SIMD share a tile
using P10 = PatchCfg<32, 14, 16, 32, 32>; // linear: 224 pixels, a whole 14 x 14 (or smaller) image, 7 waves
// two K groups (a folded pair of chunk groups)
using P11 = PatchCfg<128, 8, 8, 64, 32, 2>;
using P12 = PatchCfg<64, 8, 8, 32, 32, 2>;
using P13 = PatchCfg<64, 8, 16, 64, 32, 2>;
using P14 = PatchCfg<32, 14, 16, 32, 32, 2>;
using P15 = PatchCfg<64, 8, 8, 64, 32, 2>;

template <class Cfg>
constexpr TileChoice choice(int cfg, int linear, int single = 0) {
    return TileChoice{cfg, linear, Cfg::TH, Cfg::TW, Cfg::BM, Cfg::NT, single, Cfg::KG, Cfg::WM, Cfg::WQ};
}

// The TBN_TUNE_CONV_TILE control forces one tile: id = cfg for linear tiles,
// 16 + cfg for 2-D tiles, plus 32 for the one-buffer variants, plus 64 for
// stacked tiles.
int tile_override() { return tbn_hip::tuning(TBN_TUNE_CONV_TILE); }
int tile_id(const TileChoice& c) {
    return (c.linear == 1 ? c.cfg : c.linear == 0 ? 16 + c.cfg : 64 + c.cfg) + 32 * c.single;
}

// In preference order (linear tiles store whole 128-byte pixel runs; larger
// tiles do more MFMA per decoded weight word), the first tile whose patch fits
// the LDS and the staging registers and that gives >= 240 blocks; otherwise
// the feasible tile with the most blocks.
constexpr TileChoice kMenu[] = {// stacked linear tiles (stride 1): output runs of whole 4*QT-byte spans
                                choice<P0>(0, 2), choice<P1>(1, 2), choice<P2>(2, 2), choice<P3>(3, 2),
                                choice<P7>(7, 2), choice<P8>(8, 2), choice<P9>(9, 2), choice<P11>(11, 2),
                                choice<P12>(12, 2), choice<P13>(13, 2), choice<P15>(15, 2), choice<P0>(0, 2, 1),
                                choice<P1>(1, 2, 1), choice<P2>(2, 2, 1), choice<P3>(3, 2, 1),
                                choice<P0>(0, 1), choice<P1>(1, 1), choice<P2>(2, 1), choice<P3>(3, 1),
                                choice<P4>(4, 1), choice<P7>(7, 1), choice<P8>(8, 1), choice<P0>(0, 0),
                                choice<P1>(1, 0), choice<P2>(2, 0), choice<P3>(3, 0), choice<P4>(4, 0),
                                choice<P5>(5, 0), choice<P6>(6, 0), choice<P7>(7, 0), choice<P8>(8, 0),
                                // one LDS buffer: twice the blocks per CU (or a
                                // patch that fits only so); considered after the
                                // two-buffer tiles, and by the measured choice
                                choice<P0>(0, 1, 1), choice<P1>(1, 1, 1), choice<P2>(2, 1, 1), choice<P3>(3, 1, 1),
                                choice<P7>(7, 1, 1), choice<P8>(8, 1, 1), choice<P0>(0, 0, 1), choice<P1>(1, 0, 1),
                                choice<P2>(2, 0, 1), choice<P3>(3, 0, 1), choice<P6>(6, 0, 1), choice<P7>(7, 0, 1),
                                choice<P8>(8, 0, 1), choice<P9>(9, 1), choice<P9>(9, 0), choice<P9>(9, 1, 1),
                                choice<P9>(9, 0, 1), choice<P10>(10, 1), choice<P10>(10, 1, 1),
                                choice<P11>(11, 1), choice<P12>(12, 1), choice<P13>(13, 1), choice<P14>(14, 1),
                                choice<P15>(15, 1), choice<P11>(11, 0), choice<P12>(12, 0), choice<P13>(13, 0),
                                choice<P15>(15, 0)};

// The tiles built with a fused projection (launch_patch_items): 8 x 8
// tiles on one K group of waves (two groups, as folded chunk pairs take,
// would sum the projection's chunks in group order, not in the 1x1 conv's),
// at most four staging items per thread.  Measured: the fused pair takes
// ResNet-18's stride-2 stage-3 / stage-4 pairs from 31.5 / 39 us to 27.2 /
// 33 us at batch 32.
bool proj_tile_ok(const PatchGeom& g, const TileChoice& c, const PatchGeom& t) {
    const bool cfg_ok = c.cfg == 1 || c.cfg == 3 || c.cfg == 9;
    return cfg_ok && c.kg == 1 && g.taps == 9 && 4 * t.PHi * t.PWi <= 4 * c.NT;
}

bool tile_fits_base(const PatchGeom& g, const TileChoice& c, PatchGeom& t);

bool tile_fits(const PatchGeom& g, const TileChoice& c, PatchGeom& t) {
    if (!tile_fits_base(g, c, t)) return false;
    return !g.proj || proj_tile_ok(g, c, t);
}

bool tile_fits_base(const PatchGeom& g, const TileChoice& c, PatchGeom& t) {
    if (g.fold) {
        // the folded K loop: 3x3 taps, at most two staging items; one K group
        // summing the groups in turn, or (exactly two equal groups) two K
        // groups of waves, one per group, whose sums are added in group order
        const bool pair = g.chunks == 2 * g.gchunks;
        if (g.taps != 9 || (c.kg != 1 && !(c.kg == 2 && pair))) return false;
        if (c.linear == 2 && !stacked_ok(g, c.BM)) return false;
        t = g;
        fill_patch(t, c);
        const size_t bufs = lds_bytes(t, c.BM, true, c.kg) - 2 * sizeof(float) * c.BM;
        const bool red_fits = c.kg == 1 || static_cast<size_t>(c.BM) * c.TH * c.TW * 4 <= bufs;
        return lds_bytes(t, c.BM, true, c.kg) <= static_cast<size_t>(kMaxLds) && 4 * t.PHi * t.PWi <= 2 * c.NT &&
               c.BM * t.taps <= 8 * c.NT && red_fits && !c.single;
    }
    // two K groups of waves take folded chunk pairs only (above): every other
    // conv sums its chunks in turn, on one K group, whatever the tile
    if (c.kg != 1) return false;
    if (c.linear == 2 && !stacked_ok(g, c.BM)) return false;
    t = g;
    fill_patch(t, c);
    return lds_bytes(t, c.BM, true) <= static_cast<size_t>(kMaxLds) && 4 * t.PHi * t.PWi <= 8 * c.NT &&
           c.BM * t.taps <= 8 * c.NT;
}

bool choose_tile(PatchGeom& g, TileChoice& out) {
    const TileChoice* best = nullptr;
    int64_t best_blocks = -1;
    const int forced = tile_override();
    for (const auto& c : kMenu) {
        const int id = tile_id(c);
        if (forced >= 0 && id != forced) continue;
        if (forced < 0) {
            if (g.M <= 32 && c.BM != 32) continue;
            if (g.M > 32 && c.BM == 32) continue;
            if (g.M <= 64 && c.BM == 128) continue;
        }
        PatchGeom t;
        if (!tile_fits(g, c, t)) continue;
        const int64_t blocks = patch_tiles(t) * ((g.M + c.BM - 1) / c.BM);
        if (forced >= 0 || blocks >= 240) {
            out = c;
            g = t;
            return true;
        }
        if (blocks > best_blocks) {
            best_blocks = blocks;
            best = &c;
        }
    }
    if (!best) return false;
    out = *best;
    fill_patch(g, out);
    return true;
}

template <class Cfg, bool TERNARY, int TAPS, int MAXI, bool FOLD = false, bool PROJ = false>
int launch_patch_taps(const float* x, const PatchGeom& g, const uint8_t* w, int64_t col_bytes, int m_alloc,
                      const PatchEpi& epi, hipStream_t s) {
    const size_t lds = lds_bytes(g, Cfg::BM, TERNARY, Cfg::KG);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_patch_kernel<Cfg, TERNARY, TAPS, MAXI, FOLD, PROJ>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
        if (e != hipSuccess) return tbn_hip::fail(TBN_RUNTIME_ERROR, std::string("hipFuncSetAttribute: ") +
                                                                         hipGetErrorString(e));
        attr_set = true;
    }
    PatchGeom gl = g;
    gl.blocks_split = static_cast<int>(patch_tiles(g) * ((g.M + Cfg::BM - 1) / Cfg::BM));
    gl.div_split = make_udiv(static_cast<uint32_t>(gl.blocks_split));
    gl.div_mt = make_udiv(static_cast<uint32_t>((g.M + Cfg::BM - 1) / Cfg::BM));
    const int64_t blocks = static_cast<int64_t>(gl.blocks_split) * g.splits;
    hipLaunchKernelGGL((conv_patch_kernel<Cfg, TERNARY, TAPS, MAXI, FOLD, PROJ>), dim3(static_cast<unsigned>(blocks)),
                       dim3(Cfg::NT), lds, s, x, gl, w, col_bytes, m_alloc, epi);
    return tbn_hip::check_launch(TERNARY ? "conv2d_f32_ternary (patch)" : "conv2d_f32_binary (patch)");
}

template <class Cfg, bool TERNARY, int TAPS>
int launch_patch_items(const float* x, const PatchGeom& g, const uint8_t* w, int64_t col_bytes, int m_alloc,
                       const PatchEpi& epi, hipStream_t s) {
    const int per_thread = (4 * g.PHi * g.PWi + Cfg::NT - 1) / Cfg::NT;
    const int wper_thread = (Cfg::BM / (TERNARY ? 2 : 4) * g.taps + Cfg::NT - 1) / Cfg::NT;
    if (per_thread > 8 || wper_thread > 4 || (Cfg::KG > 1 && per_thread > 4))
        return tbn_hip::fail(TBN_INVALID_SHAPE, "conv patch too large for the staging registers");
    if (g.proj) {
        // with the fused projection (the tiles proj_tile_ok admits)
        constexpr bool kProj =
            std::is_same<Cfg, P1>::value || std::is_same<Cfg, P3>::value || std::is_same<Cfg, P9>::value;
        if constexpr (TAPS > 0 && kProj) {
            if (g.fold) {
                if (per_thread <= 2)
                    return launch_patch_taps<Cfg, TERNARY, TAPS, 2, true, true>(x, g, w, col_bytes, m_alloc, epi, s);
            } else {
                if (per_thread <= 2)
                    return launch_patch_taps<Cfg, TERNARY, TAPS, 2, false, true>(x, g, w, col_bytes, m_alloc, epi, s);
                if (per_thread <= 4)
                    return launch_patch_taps<Cfg, TERNARY, TAPS, 4, false, true>(x, g, w, col_bytes, m_alloc, epi, s);
            }
        }
        return tbn_hip::fail(TBN_INVALID_SHAPE, "this conv tile does not take a fused projection");
    }
    if (g.fold) {
        // all chunk groups in one block (3x3, small patches): one K group of
        // waves taking the groups in turn, or two taking one group each
        if constexpr (TAPS > 0) {
            if (per_thread <= 1) return launch_patch_taps<Cfg, TERNARY, TAPS, 1, true>(x, g, w, col_bytes, m_alloc, epi, s);
            if (per_thread <= 2) return launch_patch_taps<Cfg, TERNARY, TAPS, 2, true>(x, g, w, col_bytes, m_alloc, epi, s);
        }
        return tbn_hip::fail(TBN_INVALID_SHAPE, "conv patch too large for a folded K loop");
    }
    if constexpr (TAPS > 0) {
        if (per_thread <= 1) return launch_patch_taps<Cfg, TERNARY, TAPS, 1>(x, g, w, col_bytes, m_alloc, epi, s);
        if (per_thread <= 2) return launch_patch_taps<Cfg, TERNARY, TAPS, 2>(x, g, w, col_bytes, m_alloc, epi, s);
    }
    if (per_thread <= 4) return launch_patch_taps<Cfg, TERNARY, TAPS, 4>(x, g, w, col_bytes, m_alloc, epi, s);
    if constexpr (Cfg::KG > 1) return TBN_INVALID_SHAPE;  // not reached (checked above)
    else return launch_patch_taps<Cfg, TERNARY, TAPS, 8>(x, g, w, col_bytes, m_alloc, epi, s);
}

template <class Cfg, bool TERNARY>
int launch_patch(const float* x, const PatchGeom& g, const uint8_t* w, int64_t col_bytes, int m_alloc,
                 const PatchEpi& epi, hipStream_t s) {
    if (g.kh == 3 && g.kw == 3) return launch_patch_items<Cfg, TERNARY, 9>(x, g, w, col_bytes, m_alloc, epi, s);
    if constexpr (Cfg::KG > 1) return TBN_INVALID_SHAPE;  // K groups serve 3x3 kernels only (tile_fits)
    else return launch_patch_items<Cfg, TERNARY, 0>(x, g, w, col_bytes, m_alloc, epi, s);
}

template <bool TERNARY>
int dispatch_patch(int id, const float* x, const PatchGeom& g, const uint8_t* w, int64_t col_bytes, int m_alloc,
                   const PatchEpi& epi, hipStream_t s) {
    switch (id) {
        case 0: return launch_patch<P0, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 1: return launch_patch<P1, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 2: return launch_patch<P2, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 3: return launch_patch<P3, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 4: return launch_patch<P4, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 5: return launch_patch<P5, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 6: return launch_patch<P6, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 7: return launch_patch<P7, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 8: return launch_patch<P8, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 9: return launch_patch<P9, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 10: return launch_patch<P10, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 11: return launch_patch<P11, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 12: return launch_patch<P12, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 13: return launch_patch<P13, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        case 14: return launch_patch<P14, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
        default: return launch_patch<P15, TERNARY>(x, g, w, col_bytes, m_alloc, epi, s);
    }
}

// Launches the kernel of tile choice c (g laid out for it by fill_patch).
template <bool TERNARY>
int run_choice(const TileChoice& c, const float* x, const PatchGeom& g, const uint8_t* w, int64_t col_bytes,
               int m_alloc, const PatchEpi& epi, hipStream_t s) {
    return dispatch_patch<TERNARY>(c.cfg, x, g, w, col_bytes, m_alloc, epi, s);
}

// ---- tile selection by measurement ------------------------------------------
// Which tile is fastest depends on image size, channel counts and stride in
// ways a static rule gets wrong by up to 1.6x.  tbn_hip_conv2d_tune_prepacked
// (called once per layer, e.g. by the Session at compile time) times every
// feasible tile and caches the winner for the process; the per-call path only
// reads that cache, else uses the static rule, and never times, allocates or
// waits.  Every tile accumulates each output in the same order (chunk, tap,
// k-slice, hi/mid/lo), so the choice never changes results.

struct PlanKey {
    int64_t v[17];
    bool operator<(const PlanKey& o) const { return std::lexicographical_compare(v, v + 17, o.v, o.v + 17); }
};

std::mutex& plan_mutex() {
    static std::mutex m;
    return m;
}
std::map<PlanKey, int>& plan_cache() {
    static std::map<PlanKey, int> m;
    return m;
}

PlanKey plan_key(const tbn_conv2d_desc* d, bool ternary, const PatchEpi& epi) {
    return PlanKey{{d->n, d->c, d->h, d->w, d->m, d->kh, d->kw, d->sh, d->sw, d->ph, d->pw, d->dh, d->dw,
                    ternary ? 1 : 0, epi.flags, epi.residual ? 1 : 0, epi.proj_y ? 1 : 0}};
}

template <bool TERNARY>
int dispatch_patch(int id, const float* x, const PatchGeom& g, const uint8_t* w, int64_t col_bytes, int m_alloc,
                   const PatchEpi& epi, hipStream_t s);

// The tile for this call: a forced tile, the tuned one, else the static rule.
template <bool TERNARY>
int select_tile(const tbn_conv2d_desc* d, PatchGeom& g, const PatchEpi& epi, TileChoice& out) {
    if (tile_override() < 0) {
        const PlanKey key = plan_key(d, TERNARY, epi);
        std::lock_guard<std::mutex> lock(plan_mutex());
        auto it = plan_cache().find(key);
        if (it != plan_cache().end()) {
            out = kMenu[it->second];
            fill_patch(g, out);
            return TBN_SUCCESS;
        }
    }
    if (!choose_tile(g, out)) return tbn_hip::fail(TBN_INVALID_SHAPE, "no conv tile fits this geometry");
    return TBN_SUCCESS;
}

// Times each feasible tile (all launches writing epi.y) and caches the
// fastest under the call's key.
template <bool TERNARY>
int tune_tile(const tbn_conv2d_desc* d, const PatchGeom& g0, const float* x, const uint8_t* w, int64_t col_bytes,
              int m_alloc, const PatchEpi& epi, hipStream_t s) {
    const int ceil_m = (g0.M + 31) / 32 * 32;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        (void)hipGetLastError();
        if (e0) (void)hipEventDestroy(e0);
        return tbn_hip::fail(TBN_RUNTIME_ERROR, "conv tuning: hipEventCreate failed");
    }
    // the feasible tiles, each launched once untimed; then kRounds rounds that
    // time every candidate over kLaunches back-to-back launches, candidates
    // interleaved so that clock drift meets them alike; a tile's time is its
    // best round
    constexpr int kMenuSize = static_cast<int>(sizeof(kMenu) / sizeof(kMenu[0]));
    constexpr int kRounds = 3, kLaunches = 4;
    int cand[kMenuSize];
    PatchGeom cgeom[kMenuSize];
    float cbest[kMenuSize];
    int ncand = 0;
    for (int i = 0; i < kMenuSize; ++i) {
        const TileChoice& c = kMenu[i];
        PatchGeom t;
        if (c.BM > ceil_m || !tile_fits(g0, c, t)) continue;
        if (run_choice<TERNARY>(c, x, t, w, col_bytes, m_alloc, epi, s) != TBN_SUCCESS) continue;
        cand[ncand] = i;
        cgeom[ncand] = t;
        cbest[ncand] = -1.0f;
        ++ncand;
    }
    int rc = TBN_SUCCESS;
    for (int r = 0; r < kRounds && rc == TBN_SUCCESS; ++r)
        for (int k = 0; k < ncand && rc == TBN_SUCCESS; ++k) {
            (void)hipEventRecord(e0, s);
            bool ok = true;
            for (int l = 0; l < kLaunches && ok; ++l)
                ok = run_choice<TERNARY>(kMenu[cand[k]], x, cgeom[k], w, col_bytes, m_alloc, epi, s) == TBN_SUCCESS;
            (void)hipEventRecord(e1, s);
            float ms = 0.0f;
            if (!ok) continue;
            if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
                rc = tbn_hip::fail(TBN_RUNTIME_ERROR, std::string("conv tuning: ") + hipGetErrorString(hipGetLastError()));
                break;
            }
            if (cbest[k] < 0.0f || ms < cbest[k]) cbest[k] = ms;
        }
    int best = -1;
    float best_ms = 0.0f;
    for (int k = 0; k < ncand; ++k)
        if (cbest[k] >= 0.0f && (best < 0 || cbest[k] < best_ms)) {
            best = cand[k];
            best_ms = cbest[k];
        }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc != TBN_SUCCESS) return rc;
    if (best >= 0) {
        std::lock_guard<std::mutex> lock(plan_mutex());
        plan_cache()[plan_key(d, TERNARY, epi)] = best;
    }
    return tbn_hip::ok();
}

int make_patch_geom(const tbn_conv2d_desc* d, int flags, PatchGeom& g) {
    ConvGeom cg;
    int rc = make_geom(d, flags, cg);
    if (rc) return rc;
    g.N = int(d->n); g.C = int(d->c); g.H = int(d->h); g.W = int(d->w); g.M = int(d->m);
    g.kh = int(d->kh); g.kw = int(d->kw); g.sh = int(d->sh); g.sw = int(d->sw);
    g.ph = int(d->ph); g.pw = int(d->pw); g.dh = int(d->dh); g.dw = int(d->dw);
    g.OH = cg.OHW / cg.OW;
    g.OW = cg.OW;
    g.taps = g.kh * g.kw;
    g.chunks = (g.C + kChunk - 1) / kChunk;
    g.pool = cg.pool;
    g.PH = g.pool ? g.OH / 2 : 0;
    g.PW = g.pool ? g.OW / 2 : 0;
    g.VH = g.pool ? 2 * g.PH : g.OH;
    g.VW = g.pool ? 2 * g.PW : g.OW;
    // the kernel addresses one image (channels padded to whole chunks), the
    // conv-layout weights (rows padded by a channel tile) and one image's
    // output planes (likewise) with 32-bit offsets below 2^31, the bit that
    // marks a masked element
    const int64_t image_bytes = static_cast<int64_t>(g.chunks) * kChunk * g.H * g.W * 4;
    const int64_t weight_bytes = ((d->m + 7) / 8 * 8 + 128) * static_cast<int64_t>(g.chunks) * g.taps * 8;
    const int64_t out_bytes = (d->m + 128) * static_cast<int64_t>(g.pool ? g.PH * g.PW : g.OH * g.OW) * 4;
    if (image_bytes >= (1LL << 31) || weight_bytes >= (1LL << 31) || out_bytes >= (1LL << 31))
        return tbn_hip::fail(TBN_INVALID_SHAPE, "conv image, weights or output too large for the patch kernel");
    // K splits over blocks for the smallest feature maps with many chunks
    // (ResNet's last stage, whose tiles alone leave SIMDs with one wave):
    // 2^16 outputs per image and split, at least 36 K steps of 32 per split
    // (a split's saving must pay for the reduce launch).  The
    // rule reads one image's shape, not the batch, so a sample's result does
    // not depend on the batch it runs in; the tile choice never changes it.
    const int64_t outputs_img = static_cast<int64_t>(g.M) * g.OH * g.OW;
    int splits = 1;
    if (!g.pool) {
        while (splits < 4 && outputs_img * splits * 2 <= (int64_t(1) << 16) &&
               g.chunks * g.taps / (splits * 2) >= 36)
            splits *= 2;
    }
    // a forced count (TBN_TUNE_CONV_SPLITS) applies to unpooled convs only:
    // the split partials hold unpooled planes
    const bool forced = !g.pool && tbn_hip::tuning(TBN_TUNE_CONV_SPLITS) > 0;
    if (forced) splits = tbn_hip::tuning(TBN_TUNE_CONV_SPLITS);
    g.single = 0;
    g.proj = 0;
    g.gchunks = (g.chunks + splits - 1) / splits;
    const int groups = (g.chunks + g.gchunks - 1) / g.gchunks;
    // The batch decides how the groups run: when the unsplit 8 x 8 tiles of
    // 64 channels already fill the chip, one block runs all groups (fold) and
    // no partial sums go through memory; else one block per group.  Both sum
    // in the same order, so a sample's bits do not depend on its batch.
    const int64_t unsplit = static_cast<int64_t>(g.N) * ((g.OH + 7) / 8) * ((g.OW + 7) / 8) * ((g.M + 63) / 64);
    g.fold = !forced && groups > 1 && g.taps == 9 && unsplit >= 256 ? 1 : 0;
    if (g.fold) {
        PatchGeom t = g;
        t.cps = g.chunks;
        t.splits = 1;
        TileChoice c;
        if (!choose_tile(t, c)) g.fold = 0;  // no tile takes the folded loop: split instead
    }
    g.cps = g.fold ? g.chunks : g.gchunks;
    g.splits = g.fold ? 1 : groups;
    g.blocks_split = 0;
    return TBN_SUCCESS;
}

int conv_patch_dispatch(int weights, const float* x, const tbn_conv2d_desc* desc, PatchGeom& g,
                        const uint8_t* conv_weights, int64_t col_bytes, int m_alloc, const PatchEpi& epi,
                        hipStream_t s, bool tune, bool* finished);

// Bytes of split-K partial sums a call with this geometry needs (0 when K is
// not split).
int64_t conv_patch_partial_bytes(const PatchGeom& g) {
    return g.splits > 1 ? static_cast<int64_t>(g.N) * g.M * g.OH * g.OW * g.splits * 4 : 0;
}

// One patch conv.  The split-K partial sums go to `scratch` when given (at
// least conv_patch_partial_bytes, else TBN_INVALID_ARGUMENT), else to the
// stream workspace.  With `tune`, the feasible tiles are timed instead and
// the fastest is cached for later calls (y is written by every tile).
int conv_patch_run(int weights, const float* x, const tbn_conv2d_desc* desc, const uint8_t* conv_weights,
                   const float* scale, float alpha, const float* bias, const float* residual, int flags, float* y,
                   hipStream_t s, bool tune = false, void* scratch = nullptr, int64_t scratch_bytes = 0,
                   int* counters = nullptr) {
    TBN_REQUIRE(weights == TBN_WEIGHTS_BINARY || weights == TBN_WEIGHTS_TERNARY, TBN_INVALID_ARGUMENT,
                "unknown weights kind");
    TBN_REQUIRE((flags & ~(TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE | TBN_EPI_MAXPOOL2X2)) == 0,
                TBN_INVALID_ARGUMENT, "unknown epilogue flags");
    PatchGeom g;
    int rc = make_patch_geom(desc, flags, g);
    if (rc) return rc;
    TBN_REQUIRE(!(residual && g.pool), TBN_INVALID_ARGUMENT,
                "a residual input cannot be combined with the fused max pool");
    // the split-K reduce writes unpooled planes: never split a pooled conv
    TBN_REQUIRE(!(g.splits > 1 && g.pool), TBN_INVALID_ARGUMENT, "a pooled conv cannot split K");
    TileChoice tc;
    {
        PatchGeom t = g;
        TBN_REQUIRE(choose_tile(t, tc), TBN_INVALID_SHAPE, "no conv tile fits this kernel size / stride / dilation");
    }
    if (g.VH == 0 || g.VW == 0 || g.N == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && conv_weights && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(conv_weights) % 8 == 0, TBN_INVALID_ARGUMENT,
                "conv weights must be 8-byte aligned");
    TBN_DEVICE_GUARD();
    const int64_t Kc = static_cast<int64_t>(g.chunks) * g.taps * kChunk;
    const int64_t col_bytes = Kc / (weights == TBN_WEIGHTS_BINARY ? 8 : 4);
    const int m_alloc = int((desc->m + 7) / 8 * 8);
    PatchEpi epi{y, scale, alpha, bias, residual, flags, nullptr, nullptr};
    void* part = nullptr;
    bool temporary = false;
    const int64_t part_bytes = conv_patch_partial_bytes(g);
    if (part_bytes) {
        if (scratch) {
            TBN_REQUIRE(scratch_bytes >= part_bytes, TBN_INVALID_ARGUMENT,
                        "conv scratch holds " + std::to_string(scratch_bytes) + " bytes; this geometry needs " +
                            std::to_string(part_bytes));
            part = scratch;
            epi.counters = counters;  // the scratch's owner may bring tile counters
        } else {
            // the stream workspace also brings the tile counters of the
            // in-kernel split-K finish
            rc = tbn_hip::stream_workspace(s, static_cast<size_t>(part_bytes), part, temporary, &epi.counters);
            if (rc) return rc;
        }
        epi.partial = static_cast<float*>(part);
    }
    bool finished = false;
    rc = conv_patch_dispatch(weights, x, desc, g, conv_weights, col_bytes, m_alloc, epi, s, tune, &finished);
    if (part) {
        if (rc == TBN_SUCCESS && !tune && !finished) {
            const int64_t total = static_cast<int64_t>(g.N) * g.M * g.OH * g.OW;
            const int blocks = static_cast<int>(std::min<int64_t>(tbn_hip::ceil_div(total, 256), 4096));
            PatchEpi fin = epi;
            fin.partial = nullptr;
            hipLaunchKernelGGL(conv_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s,
                               static_cast<const float*>(part), g.splits, total, g.M, g.OH * g.OW, fin);
            rc = tbn_hip::check_launch("conv2d (split-K reduce)");
        }
        if (!scratch) tbn_hip::release_workspace(part, temporary, s);
    }
    return rc;
}

// A 3x3 pad-1 conv and the 1x1 pad-0 projection of its input at the same
// stride and channel count in one launch (conv_patch_kernel<..., PROJ>).
// mode 0 runs, 1 times the tiles that take the pair and caches the fastest,
// 2 only answers whether this geometry pairs.  TBN_NOT_IMPLEMENTED: the pair
// does not fuse here (K split over blocks, no tile takes it); the caller
// then runs the two convs, which give the same bits.
int conv_patch_pair_run(int weights, const float* x, const tbn_conv2d_desc* desc, const uint8_t* conv_weights,
                        const float* scale, float alpha, const float* bias, const float* residual, int flags,
                        float* y, const uint8_t* proj_weights, const float* proj_scale, float proj_alpha,
                        const float* proj_bias, int proj_flags, float* proj_y, int mode, hipStream_t s) {
    TBN_REQUIRE(weights == TBN_WEIGHTS_BINARY || weights == TBN_WEIGHTS_TERNARY, TBN_INVALID_ARGUMENT,
                "unknown weights kind");
    TBN_REQUIRE(mode >= 0 && mode <= 2, TBN_INVALID_ARGUMENT, "mode must be 0 (run), 1 (tune) or 2 (query)");
    constexpr int kFlags = TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE;
    TBN_REQUIRE((flags & ~kFlags) == 0 && (proj_flags & ~kFlags) == 0, TBN_INVALID_ARGUMENT,
                "a fused pair takes ReLU and bias-then-scale epilogues only");
    TBN_REQUIRE(desc != nullptr, TBN_INVALID_ARGUMENT, "null pointer");
    if (desc->kh != 3 || desc->kw != 3 || desc->ph != 1 || desc->pw != 1 || desc->dh != 1 || desc->dw != 1 ||
        desc->sh != desc->sw)
        return tbn_hip::fail(TBN_NOT_IMPLEMENTED, "only a 3x3 pad-1 conv pairs with the 1x1 projection of its input");
    PatchGeom g;
    int rc = make_patch_geom(desc, flags, g);
    if (rc) return rc;
    if (g.splits != 1)
        return tbn_hip::fail(TBN_NOT_IMPLEMENTED, "a conv that splits K over blocks runs apart from its projection");
    g.proj = 1;
    TileChoice tc;
    {
        PatchGeom t = g;
        if (!choose_tile(t, tc)) return tbn_hip::fail(TBN_NOT_IMPLEMENTED, "no conv tile takes this pair");
    }
    if (mode == 2 || g.VH == 0 || g.VW == 0 || g.N == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && conv_weights && y && proj_weights && proj_y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(conv_weights) % 8 == 0 && reinterpret_cast<uintptr_t>(proj_weights) % 8 == 0,
                TBN_INVALID_ARGUMENT, "conv weights must be 8-byte aligned");
    if (mode == 1) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        TBN_REQUIRE(hipStreamIsCapturing(s, &st) == hipSuccess && st == hipStreamCaptureStatusNone,
                    TBN_INVALID_ARGUMENT, "conv tuning waits for the stream and cannot run under stream capture");
        if (tbn_hip::tuning(TBN_TUNE_CONV_TILE) >= 0) return tbn_hip::ok();  // a forced tile: nothing to choose
    }
    TBN_DEVICE_GUARD();
    const int64_t Kc = static_cast<int64_t>(g.chunks) * g.taps * kChunk;
    const int64_t col_bytes = Kc / (weights == TBN_WEIGHTS_BINARY ? 8 : 4);
    const int m_alloc = int((desc->m + 7) / 8 * 8);
    PatchEpi epi{y, scale, alpha, bias, residual, flags, nullptr, nullptr,
                 proj_weights, proj_y, proj_scale, proj_alpha, proj_bias, proj_flags};
    return conv_patch_dispatch(weights, x, desc, g, conv_weights, col_bytes, m_alloc, epi, s, mode == 1, nullptr);
}

int conv_patch_dispatch(int weights, const float* x, const tbn_conv2d_desc* desc, PatchGeom& g,
                        const uint8_t* conv_weights, int64_t col_bytes, int m_alloc, const PatchEpi& epi,
                        hipStream_t s, bool tune, bool* finished) {
    // tile timing launches without the in-kernel split-K finish
    PatchEpi e = epi;
    if (tune) e.counters = nullptr;
    if (finished) *finished = false;
    int rc;
    TileChoice tc;
    if (weights == TBN_WEIGHTS_TERNARY) {
        if (tune) return tune_tile<true>(desc, g, x, conv_weights, col_bytes, m_alloc, e, s);
        rc = select_tile<true>(desc, g, e, tc);
    } else {
        if (tune) return tune_tile<false>(desc, g, x, conv_weights, col_bytes, m_alloc, e, s);
        rc = select_tile<false>(desc, g, e, tc);
    }
    if (rc) return rc;
    // one counter per tile of a split
    const int64_t tiles = patch_tiles(g) * ((g.M + tc.BM - 1) / tc.BM);
    if (tiles > tbn_hip::kWorkspaceCounters) e.counters = nullptr;
    rc = weights == TBN_WEIGHTS_TERNARY ? run_choice<true>(tc, x, g, conv_weights, col_bytes, m_alloc, e, s)
                                        : run_choice<false>(tc, x, g, conv_weights, col_bytes, m_alloc, e, s);
    if (finished) *finished = e.partial && e.counters;
    return rc;
}

}  // namespace

namespace tbn_hip {

bool conv_patch_supported(const tbn_conv2d_desc* desc) {
    PatchGeom g;
    if (make_patch_geom(desc, 0, g) != TBN_SUCCESS) return false;
    TileChoice tc;
    return choose_tile(g, tc);
}

int64_t conv_patch_scratch_bytes(int weights, const tbn_conv2d_desc* desc, int flags) {
    PatchGeom g;
    if (make_patch_geom(desc, flags, g) != TBN_SUCCESS) return -1;
    return (conv_weight_bytes(weights, desc) + 255) / 256 * 256 + conv_patch_partial_bytes(g);
}

int conv_patch_from_reference(int weights, const float* x, const tbn_conv2d_desc* desc, const uint8_t* packed,
                              int64_t K_pad, int64_t N_pad, const float* scale, float alpha, const float* bias,
                              const float* residual, int flags, float* y, hipStream_t s, void* scratch,
                              int64_t scratch_bytes) {
    const int64_t wbytes = conv_weight_bytes(weights, desc);
    if (scratch) {
        const int64_t wspan = (wbytes + 255) / 256 * 256;
        TBN_REQUIRE(scratch_bytes >= wspan, TBN_INVALID_ARGUMENT, "conv scratch too small for the weights");
        uint8_t* cw = static_cast<uint8_t*>(scratch);
        int rc = tbn_hip_pack_conv_weights(weights, packed, K_pad, N_pad, desc, cw, s);
        if (rc == TBN_SUCCESS)
            rc = conv_patch_run(weights, x, desc, cw, scale, alpha, bias, residual, flags, y, s, false,
                                cw + wspan, scratch_bytes - wspan);
        return rc;
    }
    // the stream workspace: the re-ordered weights, the split-K sums after
    // them, and the tile counters of the in-kernel split-K finish.  While s
    // captures, stream_workspace refuses (TBN_NOT_IMPLEMENTED): nothing is
    // allocated into a graph; callers that capture use the prepacked or the
    // no-allocation entry points.
    PatchGeom g;
    int rc = make_patch_geom(desc, flags, g);
    if (rc) return rc;
    const int64_t wspan = (wbytes + 255) / 256 * 256;
    const int64_t bytes = wspan + conv_patch_partial_bytes(g);
    void* ws = nullptr;
    int* counters = nullptr;
    bool temporary = false;
    rc = stream_workspace(s, static_cast<size_t>(bytes), ws, temporary, &counters);
    if (rc) return rc;
    uint8_t* cw = static_cast<uint8_t*>(ws);
    rc = tbn_hip_pack_conv_weights(weights, packed, K_pad, N_pad, desc, cw, s);
    if (rc == TBN_SUCCESS)
        rc = conv_patch_run(weights, x, desc, cw, scale, alpha, bias, residual, flags, y, s, false, cw + wspan,
                            bytes - wspan, counters);
    release_workspace(ws, temporary, s);
    return rc;
}

}  // namespace tbn_hip

extern "C" {

int tbn_hip_conv_weights_bytes(int weights, const tbn_conv2d_desc* desc, int64_t* bytes) {
    TBN_REQUIRE(weights == TBN_WEIGHTS_BINARY || weights == TBN_WEIGHTS_TERNARY, TBN_INVALID_ARGUMENT,
                "unknown weights kind");
    PatchGeom g;
    int rc = make_patch_geom(desc, 0, g);
    if (rc) return rc;
    TileChoice tc;
    TBN_REQUIRE(choose_tile(g, tc), TBN_INVALID_SHAPE,
                "no conv tile fits this kernel size / stride / dilation (use the reference-layout entry points)");
    TBN_REQUIRE(bytes != nullptr, TBN_INVALID_ARGUMENT, "null pointer");
    *bytes = conv_weight_bytes(weights, desc);
    return tbn_hip::ok();
}

int tbn_hip_pack_conv_weights(int weights, const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                              const tbn_conv2d_desc* desc, uint8_t* conv_weights, tbn_stream_t stream) {
    TBN_REQUIRE(weights == TBN_WEIGHTS_BINARY || weights == TBN_WEIGHTS_TERNARY, TBN_INVALID_ARGUMENT,
                "unknown weights kind");
    ConvGeom g;
    int rc = make_geom(desc, 0, g);
    if (rc) return rc;
    const int64_t K = desc->c * desc->kh * desc->kw;
    TBN_REQUIRE(K_pad >= K && K_pad % 32 == 0, TBN_INVALID_SHAPE, "K_pad must be >= C*kh*kw and a multiple of 32");
    TBN_REQUIRE(N_pad >= desc->m, TBN_INVALID_SHAPE, "N_pad must be >= output channels");
    TBN_REQUIRE(packed && conv_weights, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const int chunks = int((desc->c + kChunk - 1) / kChunk);
    ConvWeightDims d{int(desc->m), int(desc->c), int(desc->kh * desc->kw), chunks, K_pad,
                     static_cast<int64_t>(chunks) * desc->kh * desc->kw * kChunk, int((desc->m + 7) / 8 * 8)};
    const int64_t bytes = conv_weight_bytes(weights, desc);
    const int blocks = static_cast<int>(std::min<int64_t>(tbn_hip::ceil_div(bytes, 256), 4096));
    if (weights == TBN_WEIGHTS_TERNARY)
        hipLaunchKernelGGL(reorder_conv_ternary_kernel, dim3(blocks), dim3(256), 0, tbn_hip::stream_of(stream),
                           packed, d, conv_weights);
    else
        hipLaunchKernelGGL(reorder_conv_binary_kernel, dim3(blocks), dim3(256), 0, tbn_hip::stream_of(stream),
                           packed, d, conv_weights);
    return tbn_hip::check_launch("pack_conv_weights");
}

int tbn_hip_conv2d_f32_prepacked(int weights, const float* x, const tbn_conv2d_desc* desc,
                                 const uint8_t* conv_weights, const float* scale, float alpha, const float* bias,
                                 const float* residual, int flags, float* y, tbn_stream_t stream) {
    return conv_patch_run(weights, x, desc, conv_weights, scale, alpha, bias, residual, flags, y,
                          tbn_hip::stream_of(stream));
}

int tbn_hip_conv2d_f32_prepacked_pair(int weights, const float* x, const tbn_conv2d_desc* desc,
                                      const uint8_t* conv_weights, const float* scale, float alpha, const float* bias,
                                      const float* residual, int flags, float* y, const uint8_t* proj_weights,
                                      const float* proj_scale, float proj_alpha, const float* proj_bias,
                                      int proj_flags, float* proj_y, int mode, tbn_stream_t stream) {
    return conv_patch_pair_run(weights, x, desc, conv_weights, scale, alpha, bias, residual, flags, y, proj_weights,
                               proj_scale, proj_alpha, proj_bias, proj_flags, proj_y, mode, tbn_hip::stream_of(stream));
}

int tbn_hip_conv2d_kernel_name(int weights, const tbn_conv2d_desc* desc, int flags, int has_residual, char* name,
                               size_t len) {
    TBN_REQUIRE(weights == TBN_WEIGHTS_BINARY || weights == TBN_WEIGHTS_TERNARY, TBN_INVALID_ARGUMENT,
                "unknown weights kind");
    TBN_REQUIRE(desc && name && len > 0, TBN_INVALID_ARGUMENT, "null pointer");
    PatchGeom g;
    int rc = make_patch_geom(desc, flags, g);
    if (rc) return rc;
    PatchEpi epi{};
    epi.flags = flags;
    epi.residual = has_residual ? reinterpret_cast<const float*>(desc) : nullptr;  // only tested for null
    TileChoice tc;
    rc = weights == TBN_WEIGHTS_TERNARY ? select_tile<true>(desc, g, epi, tc) : select_tile<false>(desc, g, epi, tc);
    if (rc) return rc;
    // the launch's template arguments, as launch_patch / launch_patch_items pick them
    const int taps = (g.kh == 3 && g.kw == 3) ? 9 : 0;
    const int per_thread = (4 * g.PHi * g.PWi + tc.NT - 1) / tc.NT;
    const int maxi = taps && per_thread <= 1 ? 1 : taps && per_thread <= 2 ? 2 : per_thread <= 4 ? 4 : 8;
    // (the last argument, PROJ, is false: this is the conv without a fused projection)
    std::snprintf(name, len, "conv_patch_kernel<PatchCfg<%d, %d, %d, %d, %d, %d>, %s, %d, %d, %s, false>", tc.BM, tc.TH,
                  tc.TW, tc.WM, tc.WQ, tc.kg, weights == TBN_WEIGHTS_TERNARY ? "true" : "false", taps, maxi,
                  g.fold ? "true" : "false");
    return tbn_hip::ok();
}

int tbn_hip_conv2d_tune_prepacked(int weights, const float* x, const tbn_conv2d_desc* desc,
                                  const uint8_t* conv_weights, const float* scale, float alpha, const float* bias,
                                  const float* residual, int flags, float* y, tbn_stream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const hipStream_t s = tbn_hip::stream_of(stream);
    TBN_REQUIRE(hipStreamIsCapturing(s, &st) == hipSuccess && st == hipStreamCaptureStatusNone,
                TBN_INVALID_ARGUMENT, "conv tuning waits for the stream and cannot run under stream capture");
    if (tbn_hip::tuning(TBN_TUNE_CONV_TILE) >= 0) return tbn_hip::ok();  // a forced tile: nothing to choose
    return conv_patch_run(weights, x, desc, conv_weights, scale, alpha, bias, residual, flags, y, s, true);
}

}  // extern "C"
