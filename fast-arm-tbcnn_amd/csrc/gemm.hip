// float x binary / float x ternary GEMM and the fp32 GEMM (north_star
// subsystem 2), all on the bf16-split MFMA tile engine of mfma_core.hpp.
//
// MFMA rows are the M rows of A (split operand), MFMA columns the N output
// columns (packed weights, or the fp32 B matrix for tbn::gemm), so each
// result register row is 32 consecutive columns of C: 128-byte stores.
#include <string>

#include "common.hpp"
#include "gemm_wide.hpp"
#include "mfma_core.hpp"

namespace {

using namespace tbnk;

// C[m, n] = epilogue(acc[m, n]) for the quantized and fp32 GEMMs.
struct GemmEpi {
    float* C;
    int64_t ldc;
    int M, N;
    const float* scale;  // per column, may be null
    float alpha;
    const float* bias;   // per column, may be null
    const float* cin;    // fp32 GEMM addend (null, [N] or [M, N])
    float beta;
    int cin_1d;
    int flags;

    template <class Cfg>
    __device__ __forceinline__ void apply(f32x16_t (&acc)[Cfg::FR][Cfg::FC], int row0, int col0,
                                          int lane) const {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            const int n = col0 + frag_out_col(j, lane);
            if (n >= N) continue;
            const float mult = scale ? alpha * scale[n] : alpha;
            const float b = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = row0 + frag_out_row(i, e, lane);
                    if (m >= M) continue;
                    float v = acc[i][j][e];
                    v = (flags & TBN_EPI_BIAS_THEN_SCALE) ? (v + b) * mult : v * mult + b;
                    if (cin) v += beta * (cin_1d ? cin[n] : cin[static_cast<int64_t>(m) * N + n]);
                    if (flags & TBN_EPI_RELU) v = v > 0.0f ? v : 0.0f;
                    C[static_cast<int64_t>(m) * ldc + n] = v;
                }
        }
    }
};

using CfgBig = TileCfg<128, 256, 64, 128, 2>;
using CfgSmall = TileCfg<64, 64, 32, 32>;

template <class Cfg, class ColL>
int launch_gemm(const float* A, int64_t lda, int M, int N, int K, const ColL& coll,
                const GemmEpi& epi, hipStream_t stream, const char* what) {
    SplitMatrix<Cfg::BR, Cfg::NT> rowl;
    rowl.base = A;
    rowl.s_row = lda;
    rowl.s_k = 1;
    rowl.rows_valid = M;
    rowl.K = K;
    rowl.vec = (lda % 4 == 0) && (reinterpret_cast<uintptr_t>(A) % 16 == 0);
    rowl.row_fast = 0;
    const int tiles_r = static_cast<int>(tbn_hip::ceil_div(M, Cfg::BR));
    const int tiles_c = static_cast<int>(tbn_hip::ceil_div(N, Cfg::BC));
    hipLaunchKernelGGL((mfma_tile_kernel<Cfg, SplitMatrix<Cfg::BR, Cfg::NT>, ColL, GemmEpi>),
                       dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, stream, rowl, coll, epi, K,
                       tiles_r, tiles_c);
    return tbn_hip::check_launch(what);
}

template <bool TERNARY>
int gemm_quant(const float* A, int64_t lda, int64_t M, int64_t N, int64_t K, const uint8_t* packed,
               int64_t K_pad, int64_t N_pad, const float* scale, float alpha, const float* bias,
               const float* cin, int cin_1d, float beta, int flags, float* C, int64_t ldc,
               tbn_stream_t stream) {
    const char* what = TERNARY ? "gemm_f32_ternary" : "gemm_f32_binary";
    TBN_REQUIRE(M >= 0 && N >= 0 && K >= 0, TBN_INVALID_SHAPE, "M, N, K must be non-negative");
    TBN_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), TBN_INVALID_SHAPE,
                "dimensions must be below 2^31");
    TBN_REQUIRE(M == 0 || lda >= K, TBN_INVALID_ARGUMENT, "lda must be >= K");
    TBN_REQUIRE(ldc >= N, TBN_INVALID_ARGUMENT, "ldc must be >= N");
    TBN_REQUIRE(K_pad >= K && K_pad % 32 == 0, TBN_INVALID_SHAPE,
                "K_pad must be >= K and a multiple of 32");
    TBN_REQUIRE(N_pad >= N, TBN_INVALID_SHAPE, "N_pad must be >= N");
    TBN_REQUIRE((flags & ~(TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE)) == 0, TBN_INVALID_ARGUMENT,
                "unsupported epilogue flags for a GEMM");
    if (M == 0 || N == 0) return tbn_hip::ok();
    TBN_REQUIRE(C && (K == 0 || (A && packed)), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();

    GemmEpi epi{C, ldc, static_cast<int>(M), static_cast<int>(N), scale, alpha, bias,
                (cin && beta != 0.0f) ? cin : nullptr, beta, cin_1d, flags};
    const int64_t col_bytes = TERNARY ? K_pad / 4 : K_pad / 8;
    {
        const tbn_hip::WideGemmArgs wa{A, lda, int(M), int(N), int(K), packed, col_bytes, int(N_pad), C, ldc,
                                       scale, alpha, bias, epi.cin, cin_1d, beta, flags};
        if (tbn_hip::gemm_wide_fits(wa, TERNARY)) return tbn_hip::gemm_wide(wa, TERNARY, tbn_hip::stream_of(stream));
    }
    const int64_t big_tiles = tbn_hip::ceil_div(M, CfgBig::BR) * tbn_hip::ceil_div(N, CfgBig::BC);
    if (big_tiles >= 256) {
        SignPacked<CfgBig::BC, CfgBig::NT, TERNARY> coll{packed, col_bytes, static_cast<int>(N_pad)};
        return launch_gemm<CfgBig>(A, lda, int(M), int(N), int(K), coll, epi,
                                   tbn_hip::stream_of(stream), what);
    }
    SignPacked<CfgSmall::BC, CfgSmall::NT, TERNARY> coll{packed, col_bytes, static_cast<int>(N_pad)};
    return launch_gemm<CfgSmall>(A, lda, int(M), int(N), int(K), coll, epi,
                                 tbn_hip::stream_of(stream), what);
}

}  // namespace

extern "C" {

int tbn_hip_gemm_f32_binary(const float* A, int64_t lda, int64_t M, int64_t N, int64_t K,
                            const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                            const float* scale, float alpha, const float* bias, int flags,
                            float* C, int64_t ldc, tbn_stream_t stream) {
    return gemm_quant<false>(A, lda, M, N, K, packed, K_pad, N_pad, scale, alpha, bias, nullptr, 0,
                             0.0f, flags, C, ldc, stream);
}

int tbn_hip_gemm_f32_ternary(const float* A, int64_t lda, int64_t M, int64_t N, int64_t K,
                             const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                             const float* scale, float alpha, const float* bias, int flags,
                             float* C, int64_t ldc, tbn_stream_t stream) {
    return gemm_quant<true>(A, lda, M, N, K, packed, K_pad, N_pad, scale, alpha, bias, nullptr, 0,
                            0.0f, flags, C, ldc, stream);
}

int tbn_hip_gemm_f32_quantized(int weights, const float* A, int64_t lda, int64_t M, int64_t N,
                               int64_t K, const uint8_t* packed, int64_t K_pad, int64_t N_pad,
                               const float* scale, float alpha, const float* bias, const float* cin,
                               int cin_1d, float beta, int flags, float* C, int64_t ldc,
                               tbn_stream_t stream) {
    if (weights == TBN_WEIGHTS_BINARY)
        return gemm_quant<false>(A, lda, M, N, K, packed, K_pad, N_pad, scale, alpha, bias, cin,
                                 cin_1d, beta, flags, C, ldc, stream);
    if (weights == TBN_WEIGHTS_TERNARY)
        return gemm_quant<true>(A, lda, M, N, K, packed, K_pad, N_pad, scale, alpha, bias, cin,
                                cin_1d, beta, flags, C, ldc, stream);
    return tbn_hip::fail(TBN_INVALID_ARGUMENT, "unknown weights kind");
}

int tbn_hip_gemm_f32(const float* A, const float* B, const float* Cin, int c_is_1d, int64_t M,
                     int64_t K, int64_t N, float alpha, float beta, int transA, int transB,
                     int flags, float* out, tbn_stream_t stream) {
    TBN_REQUIRE(M >= 0 && N >= 0 && K >= 0, TBN_INVALID_SHAPE, "M, N, K must be non-negative");
    TBN_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), TBN_INVALID_SHAPE,
                "dimensions must be below 2^31");
    TBN_REQUIRE((flags & ~TBN_EPI_RELU) == 0, TBN_INVALID_ARGUMENT,
                "unsupported epilogue flags for gemm_f32");
    if (M == 0 || N == 0) return tbn_hip::ok();
    TBN_REQUIRE(out && (K == 0 || (A && B)), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();

    using Cfg = CfgSmall;
    SplitMatrix<Cfg::BR, Cfg::NT> rowl;
    rowl.base = A;
    rowl.s_row = transA ? 1 : K;
    rowl.s_k = transA ? M : 1;
    rowl.rows_valid = static_cast<int>(M);
    rowl.K = static_cast<int>(K);
    rowl.vec = !transA && (K % 4 == 0) && (reinterpret_cast<uintptr_t>(A) % 16 == 0);
    rowl.row_fast = transA ? 1 : 0;
    SplitMatrix<Cfg::BC, Cfg::NT> coll;  // rows of this operand are the N columns of op(B)
    coll.base = B;
    coll.s_row = transB ? K : 1;
    coll.s_k = transB ? 1 : N;
    coll.rows_valid = static_cast<int>(N);
    coll.K = static_cast<int>(K);
    coll.vec = transB && (K % 4 == 0) && (reinterpret_cast<uintptr_t>(B) % 16 == 0);
    coll.row_fast = transB ? 0 : 1;
    GemmEpi epi{out, N, static_cast<int>(M), static_cast<int>(N), nullptr, alpha, nullptr,
                (Cin && beta != 0.0f) ? Cin : nullptr, beta, c_is_1d, flags};
    const int tiles_r = static_cast<int>(tbn_hip::ceil_div(M, Cfg::BR));
    const int tiles_c = static_cast<int>(tbn_hip::ceil_div(N, Cfg::BC));
    hipLaunchKernelGGL((mfma_tile_kernel<Cfg, SplitMatrix<Cfg::BR, Cfg::NT>,
                                         SplitMatrix<Cfg::BC, Cfg::NT>, GemmEpi>),
                       dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, tbn_hip::stream_of(stream), rowl,
                       coll, epi, static_cast<int>(K), tiles_r, tiles_c);
    return tbn_hip::check_launch("gemm_f32");
}

}  // extern "C"
