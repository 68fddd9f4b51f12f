// Implicit-GEMM Conv2D (north_star subsystem 3): the im2col matrix is never
// materialised.  Each K step gathers the [positions x 32] slice of it from the
// NCHW input straight into LDS (as three bf16 planes), so the convolution is
// the same MFMA tile engine as the GEMM with
//   MFMA rows    = output channels (packed +-1 / ternary weights, or fp32
//                  weights for the unquantized layers), and
//   MFMA columns = output positions (n, oh, ow),
// which makes every result register row 32 consecutive output pixels of one
// channel: coalesced NCHW stores.  With TBN_EPI_MAXPOOL2X2 the positions are
// enumerated window by window (n, ph, pw, dy, dx), so the four pixels of a
// 2x2 pooling window sit in four neighbouring lanes and are reduced with two
// lane shuffles before one store; pixels outside the pooled area (odd last
// row / column, floor mode) are never computed.
//
// Reference behaviour replaced: conv2d_binary (conv2d.cpp:220-316: im2col,
// weight transpose, qlinear_matmul_binary, reshape, bias),
// conv2d_binary_with_scales (conv2d.cpp:319-369), conv2d (conv2d.cpp:78-192)
// and the Session's cached binary conv (model.hpp:414-559).
#include <mutex>
#include <string>

#include "common.hpp"
#include "conv_common.hpp"
#include "mfma_core.hpp"

// Scratch of the no-allocation conv entry point: the re-ordered weights and
// the split-K partial sums of a patch conv.  One copy per device, held until
// the process ends; calls on one device share it (overlapping calls race).
// Its device address comes from hipGetSymbolAddress, once per device, on the
// first such call with that device current: in host code the array's name
// is only a stand-in, never a device address.
static __device__ __align__(256) uint8_t scratch[TBN_NOALLOC_SCRATCH_BYTES];

namespace {

using namespace tbnk;

// im2col column operand: row = output position, k = (c, r, s).  Work item =
// (position, 4 consecutive k); consecutive threads take consecutive positions
// so the gathered reads run along the image rows.
template <int ROWS, int NT>
struct Im2col {
    static constexpr int PIECES = 3;
    static constexpr int ITEMS = ROWS * (BK / 4);
    static constexpr int PER_THREAD = (ITEMS + NT - 1) / NT;
    const float* x;
    ConvGeom g;
    FastDiv div_khkw, div_kw;

    struct Regs {
        float v[PER_THREAD][4];
        int64_t base[PER_THREAD];  // n*C*H*W, or -1 for positions past the end
        int ih0[PER_THREAD], iw0[PER_THREAD];
    };

    __device__ __forceinline__ void init(Regs& rg, int c0, int tid) const {
#pragma unroll
        for (int it = 0; it < PER_THREAD; ++it) {
            const int item = tid + it * NT;
            const int q = c0 + item % ROWS;
            rg.base[it] = -1;
            rg.ih0[it] = 0;
            rg.iw0[it] = 0;
            if ((ITEMS % NT == 0 || item < ITEMS) && q < g.Q) {
                int n, oh, ow;
                position_coords(g, q, n, oh, ow);
                rg.base[it] = static_cast<int64_t>(n) * g.C * g.H * g.W;
                rg.ih0[it] = oh * g.sh - g.ph;
                rg.iw0[it] = ow * g.sw - g.pw;
            }
        }
    }

    __device__ __forceinline__ void load(Regs& rg, int, int k0, int tid) const {
#pragma unroll
        for (int it = 0; it < PER_THREAD; ++it) {
            const int item = tid + it * NT;
            const int kc = item / ROWS;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (rg.base[it] >= 0) {
                int k = k0 + kc * 4;
                uint32_t c = div_khkw.div(static_cast<uint32_t>(k));
                uint32_t rs = static_cast<uint32_t>(k) - c * div_khkw.d;
                uint32_t r = div_kw.div(rs);
                uint32_t s = rs - r * div_kw.d;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (k + e < g.K) {
                        const int ih = rg.ih0[it] + static_cast<int>(r) * g.dh;
                        const int iw = rg.iw0[it] + static_cast<int>(s) * g.dw;
                        if (static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                            static_cast<unsigned>(iw) < static_cast<unsigned>(g.W))
                            v[e] = x[rg.base[it] + (static_cast<int64_t>(c) * g.H + ih) * g.W + iw];
                    }
                    if (++s == div_kw.d) {
                        s = 0;
                        if (++r == static_cast<uint32_t>(g.kh)) { r = 0; ++c; }
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) rg.v[it][e] = v[e];
        }
    }

    __device__ __forceinline__ void store(const Regs& rg, uint16_t* lds, int tid) const {
#pragma unroll
        for (int it = 0; it < PER_THREAD; ++it) {
            const int item = tid + it * NT;
            if (ITEMS % NT == 0 || item < ITEMS) {
                const int r = item % ROWS, kc = item / ROWS;
                const Split4 s = split4(rg.v[it][0], rg.v[it][1], rg.v[it][2], rg.v[it][3]);
                uint16_t* dst = lds + r * LDS_ROW + kc * 4;
                *reinterpret_cast<uint2*>(dst) = make_uint2(s.hi[0], s.hi[1]);
                *reinterpret_cast<uint2*>(dst + ROWS * LDS_ROW) = make_uint2(s.mid[0], s.mid[1]);
                *reinterpret_cast<uint2*>(dst + 2 * ROWS * LDS_ROW) = make_uint2(s.lo[0], s.lo[1]);
            }
        }
    }
};

using CfgM128 = TileCfg<128, 64, 64, 32>;  // >= 128 output channels
using CfgM64 = TileCfg<64, 64, 32, 32>;    // 33..64 output channels, or few positions
using CfgM32 = TileCfg<32, 128, 32, 32>;   // <= 32 output channels

template <class Cfg, class RowL>
int launch_conv_impl(const RowL& rowl, const float* x, const ConvGeom& g, const ConvEpi& epi,
                     hipStream_t stream, const char* what) {
    Im2col<Cfg::BC, Cfg::NT> coll;
    coll.x = x;
    coll.g = g;
    coll.div_khkw = make_fastdiv(static_cast<uint32_t>(g.kh * g.kw));
    coll.div_kw = make_fastdiv(static_cast<uint32_t>(g.kw));
    const int tiles_r = static_cast<int>(tbn_hip::ceil_div(epi.M, Cfg::BR));
    const int tiles_c = static_cast<int>(tbn_hip::ceil_div(g.Q, Cfg::BC));
    hipLaunchKernelGGL((mfma_tile_kernel<Cfg, RowL, Im2col<Cfg::BC, Cfg::NT>, ConvEpi>),
                       dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, stream, rowl, coll, epi, g.K,
                       tiles_r, tiles_c);
    return tbn_hip::check_launch(what);
}

std::mutex g_scratch_mutex;
void* g_scratch_addr[64] = {};

int noalloc_scratch(void*& out) {
    int dev = -1;
    const hipError_t ge = hipGetDevice(&dev);
    TBN_REQUIRE(ge == hipSuccess && dev >= 0 && dev < 64, TBN_DEVICE_NOT_SUPPORTED, "no current HIP device");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return tbn_hip::fail(TBN_RUNTIME_ERROR,
                                 std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
        }
        g_scratch_addr[dev] = p;
    }
    out = g_scratch_addr[dev];
    return TBN_SUCCESS;
}

// Inputs with at least this many channels take the patch path (conv_patch.hip);
// narrower ones (LeNet) gather straight from NCHW here, where padding C to a
// chunk of 32 would waste most of the K loop.
constexpr int64_t kPatchMinChannels = 16;

template <bool TERNARY>
int conv_quant(const float* x, const tbn_conv2d_desc* desc, const uint8_t* packed, int64_t K_pad,
               int64_t N_pad, const float* scale, float alpha, const float* bias,
               const float* residual, int flags, float* y, tbn_stream_t stream, bool noalloc = false) {
    const char* what = TERNARY ? "conv2d_f32_ternary" : "conv2d_f32_binary";
    ConvGeom g;
    int rc = make_geom(desc, flags, g);
    if (rc) return rc;
    TBN_REQUIRE((flags & ~(TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE | TBN_EPI_MAXPOOL2X2)) == 0,
                TBN_INVALID_ARGUMENT, "unknown epilogue flags");
    TBN_REQUIRE(K_pad >= g.K && K_pad % 32 == 0, TBN_INVALID_SHAPE,
                "K_pad must be >= C*kh*kw and a multiple of 32");
    TBN_REQUIRE(N_pad >= desc->m, TBN_INVALID_SHAPE, "N_pad must be >= output channels");
    TBN_REQUIRE(!(residual && g.pool), TBN_INVALID_ARGUMENT,
                "a residual input cannot be combined with the fused max pool");
    if (g.Q == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && packed && y, TBN_INVALID_ARGUMENT, "null pointer");
    const int wkind = TERNARY ? TBN_WEIGHTS_TERNARY : TBN_WEIGHTS_BINARY;
    const bool patch = desc->c >= kPatchMinChannels && tbn_hip::conv_patch_supported(desc);
    int64_t need = 0;
    if (noalloc && patch) {
        need = tbn_hip::conv_patch_scratch_bytes(wkind, desc, flags);
        TBN_REQUIRE(need >= 0, TBN_INVALID_SHAPE, "conv geometry not supported");
        TBN_REQUIRE(need <= static_cast<int64_t>(TBN_NOALLOC_SCRATCH_BYTES), TBN_INVALID_SHAPE,
                    "this conv needs " + std::to_string(need) + " bytes of scratch (re-ordered weights and split-K "
                    "sums); the no-allocation entry point holds " + std::to_string(TBN_NOALLOC_SCRATCH_BYTES));
    }
    TBN_DEVICE_GUARD();
    if (patch) {
        void* scratch_ptr = nullptr;
        if (noalloc) {
            const int rc = noalloc_scratch(scratch_ptr);
            if (rc) return rc;
        }
        return tbn_hip::conv_patch_from_reference(wkind, x, desc, packed, K_pad, N_pad, scale, alpha, bias, residual,
                                                 flags, y, tbn_hip::stream_of(stream), scratch_ptr, need);
    }
    const int64_t col_bytes = TERNARY ? K_pad / 4 : K_pad / 8;
    hipStream_t s = tbn_hip::stream_of(stream);
    if (tbn_hip::conv_small_supported(desc))
        return tbn_hip::conv_small_run(TERNARY ? 2 : 1, x, desc, packed, col_bytes, scale, alpha, bias, residual,
                                       flags, y, s);
    ConvEpi epi{y, int(desc->m), g, scale, alpha, bias, residual, flags};
    const int m = int(desc->m);
    if (m <= 32) {
        SignPacked<CfgM32::BR, CfgM32::NT, TERNARY> rowl{packed, col_bytes, int(N_pad)};
        return launch_conv_impl<CfgM32>(rowl, x, g, epi, s, what);
    }
    const int64_t big_tiles = tbn_hip::ceil_div(m, 128) * tbn_hip::ceil_div(g.Q, 64);
    if (m <= 64 || big_tiles < 256) {
        SignPacked<CfgM64::BR, CfgM64::NT, TERNARY> rowl{packed, col_bytes, int(N_pad)};
        return launch_conv_impl<CfgM64>(rowl, x, g, epi, s, what);
    }
    SignPacked<CfgM128::BR, CfgM128::NT, TERNARY> rowl{packed, col_bytes, int(N_pad)};
    return launch_conv_impl<CfgM128>(rowl, x, g, epi, s, what);
}

}  // namespace

extern "C" {

int tbn_hip_conv2d_f32_binary(const float* x, const tbn_conv2d_desc* desc, const uint8_t* packed,
                              int64_t K_pad, int64_t N_pad, const float* scale, float alpha,
                              const float* bias, int flags, float* y, tbn_stream_t stream) {
    return conv_quant<false>(x, desc, packed, K_pad, N_pad, scale, alpha, bias, nullptr, flags, y,
                             stream);
}

int tbn_hip_conv2d_f32_ternary(const float* x, const tbn_conv2d_desc* desc, const uint8_t* packed,
                               int64_t K_pad, int64_t N_pad, const float* scale, float alpha,
                               const float* bias, int flags, float* y, tbn_stream_t stream) {
    return conv_quant<true>(x, desc, packed, K_pad, N_pad, scale, alpha, bias, nullptr, flags, y,
                            stream);
}

int tbn_hip_conv2d_f32_quantized(int weights, const float* x, const tbn_conv2d_desc* desc,
                                 const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                                 const float* scale, float alpha, const float* bias,
                                 const float* residual, int flags, float* y, tbn_stream_t stream) {
    if (weights == TBN_WEIGHTS_BINARY)
        return conv_quant<false>(x, desc, packed, K_pad, N_pad, scale, alpha, bias, residual, flags,
                                 y, stream);
    if (weights == TBN_WEIGHTS_TERNARY)
        return conv_quant<true>(x, desc, packed, K_pad, N_pad, scale, alpha, bias, residual, flags,
                                y, stream);
    return tbn_hip::fail(TBN_INVALID_ARGUMENT, "unknown weights kind");
}

int tbn_hip_conv2d_f32_quantized_noalloc(int weights, const float* x, const tbn_conv2d_desc* desc,
                                         const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                                         const float* scale, float alpha, const float* bias,
                                         const float* residual, int flags, float* y, tbn_stream_t stream) {
    if (weights == TBN_WEIGHTS_BINARY)
        return conv_quant<false>(x, desc, packed, K_pad, N_pad, scale, alpha, bias, residual, flags, y, stream,
                                 true);
    if (weights == TBN_WEIGHTS_TERNARY)
        return conv_quant<true>(x, desc, packed, K_pad, N_pad, scale, alpha, bias, residual, flags, y, stream,
                                true);
    return tbn_hip::fail(TBN_INVALID_ARGUMENT, "unknown weights kind");
}

int tbn_hip_conv2d_f32_supported(const tbn_conv2d_desc* desc, int flags) {
    ConvGeom g;
    const int rc = make_geom(desc, flags, g);
    if (rc) return rc;
    TBN_REQUIRE((flags & ~(TBN_EPI_RELU | TBN_EPI_MAXPOOL2X2 | TBN_EPI_MAXPOOL3X3S2)) == 0, TBN_INVALID_ARGUMENT,
                "unsupported epilogue flags for conv2d_f32");
    TBN_REQUIRE(!(flags & TBN_EPI_MAXPOOL3X3S2) || tbn_hip::conv_stem_supported(desc, flags), TBN_NOT_IMPLEMENTED,
                "the fused 3x3/2 max pool takes the stem shape (3 channels, 7x7, stride 2, M <= 64) with ReLU only");
    return tbn_hip::ok();
}

int tbn_hip_conv2d_f32(const float* x, const tbn_conv2d_desc* desc, const float* w,
                       const float* bias, int flags, float* y, tbn_stream_t stream) {
    ConvGeom g;
    int rc = make_geom(desc, flags, g);
    if (rc) return rc;
    rc = tbn_hip_conv2d_f32_supported(desc, flags);
    if (rc) return rc;
    if (g.Q == 0) return tbn_hip::ok();
    TBN_REQUIRE(x && w && y, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (tbn_hip::conv_stem_supported(desc, flags))
        return tbn_hip::conv_stem_run(x, desc, w, bias, flags, y, tbn_hip::stream_of(stream));
    if (tbn_hip::conv_small_supported(desc))
        return tbn_hip::conv_small_run(0, x, desc, w, 0, nullptr, 1.0f, bias, nullptr, flags, y,
                                       tbn_hip::stream_of(stream));
    ConvEpi epi{y, int(desc->m), g, nullptr, 1.0f, bias, nullptr, flags};
    hipStream_t s = tbn_hip::stream_of(stream);
    const int m = int(desc->m);
    auto make_rows = [&](auto& rowl) {
        rowl.base = w;
        rowl.s_row = g.K;
        rowl.s_k = 1;
        rowl.rows_valid = m;
        rowl.K = g.K;
        rowl.vec = (g.K % 4 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
        rowl.row_fast = 0;
    };
    if (m <= 32) {
        SplitMatrix<CfgM32::BR, CfgM32::NT> rowl;
        make_rows(rowl);
        return launch_conv_impl<CfgM32>(rowl, x, g, epi, s, "conv2d_f32");
    }
    SplitMatrix<CfgM64::BR, CfgM64::NT> rowl;
    make_rows(rowl);
    return launch_conv_impl<CfgM64>(rowl, x, g, epi, s, "conv2d_f32");
}

}  // extern "C"
