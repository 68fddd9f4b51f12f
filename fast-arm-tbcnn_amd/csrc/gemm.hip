// float x binary / float x ternary GEMM and the fp32 GEMM (north_star
// subsystem 2), all on the bf16-split MFMA tile engine of mfma_core.hpp.
//
// MFMA rows are the M rows of A (split operand), MFMA columns the N output
// columns (packed weights, or the fp32 B matrix for tbn::gemm), so each
// result register row is 32 consecutive columns of C: 128-byte stores.
#include <algorithm>
#include <cstdio>
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

// Raw sums of one K split of the fp32 GEMM: P[m, n].
struct PartialEpi {
    float* P;
    int M, N;

    template <class Cfg>
    __device__ __forceinline__ void apply(f32x16_t (&acc)[Cfg::FR][Cfg::FC], int row0, int col0,
                                          int lane) const {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            const int n = col0 + frag_out_col(j, lane);
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = row0 + frag_out_row(i, e, lane);
                    if (m < M) P[static_cast<int64_t>(m) * N + n] = acc[i][j][e];
                }
        }
    }
};

// fp32 GEMM with K split over `splits` blocks per tile (shapes with few
// tiles, e.g. a classifier layer at small batch): block = (split, tile), split
// s covers k in [s * ksplit, min(K, (s + 1) * ksplit)).
template <class Cfg>
__global__ void __launch_bounds__(Cfg::NT, Cfg::WAVES_PER_SIMD)
gemm_f32_split_kernel(SplitMatrix<Cfg::BR, Cfg::NT> rowl, SplitMatrix<Cfg::BC, Cfg::NT> coll, float* partial,
                      int M, int N, int K, int ksplit, int tiles_r, int tiles_c) {
    const int total = tiles_r * tiles_c;
    const int sp = static_cast<int>(blockIdx.x) / total;
    int tr, tc;
    tile_coords_of(static_cast<int>(blockIdx.x) - sp * total, tiles_r, tiles_c, tr, tc);
    const int k0 = sp * ksplit;
    const int klen = min(ksplit, K - k0);
    rowl.base += static_cast<int64_t>(k0) * rowl.s_k;
    rowl.K = klen;
    coll.base += static_cast<int64_t>(k0) * coll.s_k;
    coll.K = klen;
    const PartialEpi epi{partial + static_cast<int64_t>(sp) * M * N, M, N};
    mfma_tile_body<Cfg>(rowl, coll, epi, klen, tr, tc);
}

// C = epilogue(sum of the splits, in split order): the GemmEpi arithmetic
// with no scale and no bias.
__global__ void gemm_f32_reduce_kernel(const float* __restrict__ partial, int splits, int M, int N, float alpha,
                                       const float* __restrict__ cin, int cin_1d, float beta, int flags,
                                       float* __restrict__ C) {
    const int64_t total = static_cast<int64_t>(M) * N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        float v = partial[i];
        for (int s = 1; s < splits; ++s) v += partial[static_cast<int64_t>(s) * total + i];
        v = v * alpha + 0.0f;
        if (cin) v += beta * (cin_1d ? cin[i % N] : cin[i]);
        if (flags & TBN_EPI_RELU) v = v > 0.0f ? v : 0.0f;
        C[i] = v;
    }
}

// K splits of the fp32 GEMM: a function of N and K only, so a row's result
// does not depend on how many rows (the batch) the call has.
int f32_gemm_splits(int64_t N, int64_t K) {
    if (K < 512 || N > 4096) return 1;
    return static_cast<int>(std::min<int64_t>(8, K / 64));
}

// ---- small GEMMs (a classifier head: few columns, short K) ----------------
// The weight columns are decoded to fp32 in LDS once per block; each block
// then stages groups of rows of A in LDS; each output is computed by 1 to 8
// lanes, each an fp32 FMA chain over its contiguous share of k, added in a
// fixed pairwise tree.  Lanes and shares follow from N and K only, so a
// row's result does not depend on the batch.  Staging keeps four global
// loads in flight per thread; rows sit ceil4(K) + 4 floats apart so the
// 16-byte reads of different columns start on different banks.
constexpr int kSmallGemmW = 8192;  // floats of decoded weights
constexpr int kSmallGemmA = 8192;  // floats of staged rows

struct SmallGemm {
    const float* A;
    int64_t a_row, a_k;   // element (m, k) at A[m*a_row + k*a_k]
    const void* B;        // WMODE 0: fp32 element (k, n) at B[k*b_k + n*b_col]; else packed columns
    int64_t b_k, b_col;   // WMODE 0 strides; WMODE 1/2: b_col = bytes per packed column
    int M, N, K;
    int Kp;               // LDS row stride
    int lanes;            // lanes per output (a power of two, at most 8)
    int kc;               // k per lane: ceil4(ceil(K / lanes))
    int rows;             // rows of A per group: min(256 / (N * lanes), kSmallGemmA / Kp)
};

int small_gemm_stride(int64_t K) { return static_cast<int>((K + 3) / 4 * 4 + 4); }

template <class Get, class Put>
__device__ __forceinline__ void stage4_gemm(int count, Get get, Put put) {
    for (int base = 0; base < count; base += 4 * 256) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = base + j * 256 + static_cast<int>(threadIdx.x);
            v[j] = i < count ? get(i) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = base + j * 256 + static_cast<int>(threadIdx.x);
            if (i < count) put(i, v[j]);
        }
    }
}

template <int WMODE>
__global__ void __launch_bounds__(256) small_gemm_kernel(SmallGemm g, GemmEpi epi) {
    __shared__ __align__(16) float ws[kSmallGemmW];
    __shared__ __align__(16) float as[kSmallGemmA];
    const int K = g.K, Kp = g.Kp;
    if constexpr (WMODE == 0) {
        const float* B = static_cast<const float*>(g.B);
        stage4_gemm(g.N * K,
                    [&](int i) {
                        const int n = i / K, k = i - n * K;
                        return B[static_cast<int64_t>(k) * g.b_k + static_cast<int64_t>(n) * g.b_col];
                    },
                    [&](int i, float v) {
                        const int n = i / K;
                        ws[n * Kp + (i - n * K)] = v;
                    });
    } else {
        // one byte (8 binary or 4 ternary weights) per load
        constexpr int per = WMODE == 1 ? 8 : 4;
        const int bpc = (K + per - 1) / per;
        const uint8_t* B = static_cast<const uint8_t*>(g.B);
        stage4_gemm(g.N * bpc,
                    [&](int i) {
                        const int n = i / bpc;
                        return static_cast<float>(B[static_cast<int64_t>(n) * g.b_col + (i - n * bpc)]);
                    },
                    [&](int i, float v) {
                        const int n = i / bpc, j = i - n * bpc;
                        const unsigned byte = static_cast<unsigned>(v);
                        float* dst = ws + n * Kp + j * per;
                        const int cnt = min(per, K - j * per);
                        for (int q = 0; q < cnt; ++q) {
                            if constexpr (WMODE == 1) {
                                dst[q] = ((byte >> q) & 1u) ? -1.0f : 1.0f;
                            } else {
                                const unsigned code = (byte >> (2 * q)) & 3u;
                                dst[q] = code == 0 ? -1.0f : (code == 2 ? 1.0f : 0.0f);
                            }
                        }
                    });
    }
    // thread t: lane sl = t % S of output (row r, column n), (r, n) = divmod(t / S, N);
    // lane sl sums k in [sl*kc, sl*kc + kc) and the S lanes add pairwise
    const int groups = (g.M + g.rows - 1) / g.rows;
    const int S = g.lanes, kc = g.kc;
    const int t = static_cast<int>(threadIdx.x) / S, sl = static_cast<int>(threadIdx.x) % S;
    const int r = t / g.N, n = t - r * g.N;
    const int k_lo = min(sl * kc, K), k_hi = min(k_lo + kc, K);
    const float* w = ws + n * Kp;
    for (int grp = blockIdx.x; grp < groups; grp += gridDim.x) {
        const int m0 = grp * g.rows;
        const int rows = min(g.rows, g.M - m0);
        __syncthreads();  // the previous group's rows are no longer read
        stage4_gemm(rows * K,
                    [&](int i) {
                        const int rr = i / K, k = i - rr * K;
                        return g.A[static_cast<int64_t>(m0 + rr) * g.a_row + static_cast<int64_t>(k) * g.a_k];
                    },
                    [&](int i, float v) {
                        const int rr = i / K;
                        as[rr * Kp + (i - rr * K)] = v;
                    });
        __syncthreads();
        // every lane takes part in the shuffles; rows past the group's end
        // compute on row 0 and store nothing
        const bool live = r < rows;
        // the epilogue's operands, loaded before the FMA chain
        const int m = m0 + (live ? r : 0);
        const float mult = epi.scale ? epi.alpha * epi.scale[n] : epi.alpha;
        const float b = epi.bias ? epi.bias[n] : 0.0f;
        const float cv = epi.cin ? epi.beta * (epi.cin_1d ? epi.cin[n] : epi.cin[static_cast<int64_t>(m) * g.N + n])
                                 : 0.0f;
        const float* a = as + (live ? r : 0) * Kp;
        float acc = 0.0f;
        int k = k_lo;
#pragma unroll 4
        for (; k + 4 <= k_hi; k += 4) {
            const float4 a4 = *reinterpret_cast<const float4*>(a + k);
            const float4 w4 = *reinterpret_cast<const float4*>(w + k);
            acc = fmaf(a4.x, w4.x, acc);
            acc = fmaf(a4.y, w4.y, acc);
            acc = fmaf(a4.z, w4.z, acc);
            acc = fmaf(a4.w, w4.w, acc);
        }
        for (; k < k_hi; ++k) acc = fmaf(a[k], w[k], acc);
        for (int d = 1; d < S; d <<= 1) acc += __shfl_xor(acc, d);
        if (!live || sl != 0) continue;
        // GemmEpi's arithmetic for one element
        float v = (epi.flags & TBN_EPI_BIAS_THEN_SCALE) ? (acc + b) * mult : acc * mult + b;
        if (epi.cin) v += cv;
        if (epi.flags & TBN_EPI_RELU) v = v > 0.0f ? v : 0.0f;
        epi.C[static_cast<int64_t>(m) * epi.ldc + n] = v;
    }
}

bool small_gemm_fits(int64_t N, int64_t K) {
    return N >= 1 && N <= 64 && K <= kSmallGemmA - 8 && N * small_gemm_stride(K) <= kSmallGemmW;
}

template <int WMODE>
int launch_small_gemm(SmallGemm g, const GemmEpi& epi, hipStream_t s) {
    g.Kp = small_gemm_stride(g.K);
    // lanes per output from N and K only: as many as fit 256 threads with
    // one row, up to 8, keeping at least 32 k per lane
    g.lanes = 1;
    while (g.lanes < 8 && g.N * g.lanes * 2 <= 256 && g.K >= 64 * g.lanes) g.lanes *= 2;
    g.kc = (g.K + g.lanes - 1) / g.lanes;
    g.kc = (g.kc + 3) / 4 * 4;
    g.rows = std::max(1, std::min(256 / (g.N * g.lanes), kSmallGemmA / g.Kp));
    const int64_t groups = tbn_hip::ceil_div(static_cast<int64_t>(g.M), g.rows);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(groups, 2048));
    hipLaunchKernelGGL(small_gemm_kernel<WMODE>, dim3(blocks), dim3(256), 0, s, g, epi);
    return tbn_hip::check_launch("gemm (small)");
}

// ---- many columns, moderate K (a classifier over a batch: 32 x 512 -> 1000) --
// With K split over MFMA tiles such a product is mostly staging at small batch: each block
// splits a 64 x 64 tile of both operands into bf16 planes for one 64-deep
// slice of K, and a second launch adds the slices.  Here a block owns
// kRowsR rows x kRowsC columns of C in one launch.  It stages chunks of up
// to kRowsKC values of k of those rows of op(A) and columns of op(B) in LDS
// as fp32 (every load of a chunk in flight before the first store; zeros
// past the end), and kRowsS lanes compute each output: lane l runs an fp32
// FMA chain over the 4-value groups l, l + kRowsS, ... of every chunk in
// turn, and the lanes are added in a fixed butterfly.  The order depends on
// K only, so a row's result does not depend on how many rows the call has.
constexpr int kRowsR = 16, kRowsC = 4, kRowsS = 4, kRowsKC = 512;
// rows 16 floats past the chunk: a wave's 16 distinct 16-byte reads (4 rows x
// 4 lanes) fall on disjoint banks
constexpr int kRowsPitch = kRowsKC + 16;
static_assert(kRowsR * kRowsC * kRowsS == 256, "one output per kRowsS lanes of the block");

struct RowsGemm {
    const float* A;
    int64_t a_row, a_k;  // element (m, k) at A[m*a_row + k*a_k]
    const float* B;
    int64_t b_k, b_col;  // element (k, n) of op(B) at B[k*b_k + n*b_col]
    int M, N, K;
    int a_vec, b_vec;    // k contiguous and 16-byte aligned rows: float4 loads
};

// From N and K only (not M), so a row's result never depends on the batch:
// more than a small GEMM's columns, at most 4096 of them, and 256 <= K <= 4096.
bool rows_gemm_fits(int64_t N, int64_t K) { return N > 64 && N <= 4096 && K >= 256 && K <= 4096; }

// Stage a rows x kRowsKC chunk (k0 .. k0 + kl) of an operand into
// dst[rows][kRowsPitch]; values past kl or past the last row are zero.  Every
// load reads a clamped, in-range address and the value is dropped afterwards,
// so all of a thread's loads are issued before the first wait.  Strided
// operands walk the contiguous dimension across lanes.
template <int ROWS>
__device__ __forceinline__ void rows_stage(float (*dst)[kRowsPitch], const float* base, int64_t s_row, int64_t s_k,
                                           int row0, int rows_valid, int k0, int kl, bool vec) {
    const int tid = static_cast<int>(threadIdx.x);
    if (vec) {  // s_k == 1, kl a multiple of 4, 16-byte aligned rows
        constexpr int kGroups = ROWS * (kRowsKC / 4);
        constexpr int kPer = (kGroups + 255) / 256;
        float4 v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int gi = min(j * 256 + tid, kGroups - 1), rr = gi / (kRowsKC / 4), q = (gi % (kRowsKC / 4)) * 4;
            const int row = min(row0 + rr, rows_valid - 1), qc = min(q, kl - 4);
            v[j] = *reinterpret_cast<const float4*>(base + static_cast<int64_t>(row) * s_row + k0 + qc);
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int gi = j * 256 + tid, rr = gi / (kRowsKC / 4), q = (gi % (kRowsKC / 4)) * 4;
            if (gi >= kGroups) continue;
            if (row0 + rr >= rows_valid || q >= kl) v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            *reinterpret_cast<float4*>(&dst[rr][q]) = v[j];
        }
        return;
    }
    constexpr int kElems = ROWS * kRowsKC;
    constexpr int kBatch = 16;
    const bool rows_fast = s_row == 1;  // consecutive rows adjacent in memory
    for (int base_i = 0; base_i < kElems; base_i += 256 * kBatch) {
        float v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = min(base_i + j * 256 + tid, kElems - 1);
            const int rr = rows_fast ? i % ROWS : i / kRowsKC, k = rows_fast ? i / ROWS : i % kRowsKC;
            const int row = min(row0 + rr, rows_valid - 1), kk = min(k, kl - 1);
            v[j] = base[static_cast<int64_t>(row) * s_row + static_cast<int64_t>(k0 + kk) * s_k];
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = base_i + j * 256 + tid;
            if (i >= kElems) continue;
            const int rr = rows_fast ? i % ROWS : i / kRowsKC, k = rows_fast ? i / ROWS : i % kRowsKC;
            dst[rr][k] = (row0 + rr < rows_valid && k < kl) ? v[j] : 0.0f;
        }
    }
}

__global__ void __launch_bounds__(256) rows_gemm_kernel(RowsGemm g, GemmEpi epi) {
    __shared__ __align__(16) float as[kRowsR][kRowsPitch];
    __shared__ __align__(16) float bs[kRowsC][kRowsPitch];
    const int tiles_c = (g.N + kRowsC - 1) / kRowsC;
    const int m0 = static_cast<int>(blockIdx.x) / tiles_c * kRowsR;
    const int n0 = static_cast<int>(blockIdx.x) % tiles_c * kRowsC;
    const int t = static_cast<int>(threadIdx.x), sl = t % kRowsS, o = t / kRowsS;
    const int r = o / kRowsC, c = o % kRowsC;
    float acc = 0.0f;
    for (int k0 = 0; k0 < g.K; k0 += kRowsKC) {
        const int kl = min(kRowsKC, g.K - k0);
        __syncthreads();  // the previous chunk is no longer read
        rows_stage<kRowsR>(as, g.A, g.a_row, g.a_k, m0, g.M, k0, kl, g.a_vec);
        rows_stage<kRowsC>(bs, g.B, g.b_col, g.b_k, n0, g.N, k0, kl, g.b_vec);
        __syncthreads();
        const float* a = as[r];
        const float* b = bs[c];
        // every group of the chunk, zeros past kl included: fmaf(0, 0, acc)
        // is acc (acc starts at +0 and a sum is never -0), and a fixed trip
        // count lets the LDS reads of eight steps issue together
#pragma unroll 8
        for (int q = sl; q < kRowsKC / 4; q += kRowsS) {
            const float4 a4 = *reinterpret_cast<const float4*>(a + 4 * q);
            const float4 b4 = *reinterpret_cast<const float4*>(b + 4 * q);
            acc = fmaf(a4.x, b4.x, acc);
            acc = fmaf(a4.y, b4.y, acc);
            acc = fmaf(a4.z, b4.z, acc);
            acc = fmaf(a4.w, b4.w, acc);
        }
    }
    for (int d = 1; d < kRowsS; d <<= 1) acc += __shfl_xor(acc, d);
    const int m = m0 + r, n = n0 + c;
    if (sl != 0 || m >= g.M || n >= g.N) return;
    // GemmEpi's arithmetic for one element (no scale, no bias on this path)
    float v = acc * epi.alpha + 0.0f;
    if (epi.cin) v += epi.beta * (epi.cin_1d ? epi.cin[n] : epi.cin[static_cast<int64_t>(m) * g.N + n]);
    if (epi.flags & TBN_EPI_RELU) v = v > 0.0f ? v : 0.0f;
    epi.C[static_cast<int64_t>(m) * epi.ldc + n] = v;
}

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
    if (small_gemm_fits(N, K)) {
        const SmallGemm sg{A, lda, 1, packed, 0, col_bytes, int(M), int(N), int(K), 0, 0, 0, 0};
        return launch_small_gemm<TERNARY ? 2 : 1>(sg, epi, tbn_hip::stream_of(stream));
    }
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

int tbn_hip_gemm_kernel_name(int weights, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t K_pad,
                             int64_t N_pad, char* name, size_t len) {
    TBN_REQUIRE(weights == TBN_WEIGHTS_BINARY || weights == TBN_WEIGHTS_TERNARY, TBN_INVALID_ARGUMENT,
                "unknown weights kind");
    TBN_REQUIRE(name && len > 0, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31) && lda >= K &&
                    K_pad >= K && K_pad % 32 == 0 && N_pad >= N,
                TBN_INVALID_SHAPE, "no kernel runs for this shape");
    const bool ternary = weights == TBN_WEIGHTS_TERNARY;
    std::string k;
    if (small_gemm_fits(N, K)) {
        k = ternary ? "small_gemm_kernel<2>" : "small_gemm_kernel<1>";
    } else {
        // 16-byte aligned operands, as the Session and the bench allocate them
        alignas(16) static const float kAligned[4] = {};
        const tbn_hip::WideGemmArgs wa{kAligned, lda, int(M), int(N), int(K),
                                       reinterpret_cast<const uint8_t*>(kAligned), ternary ? K_pad / 4 : K_pad / 8,
                                       int(N_pad), nullptr, N, nullptr, 1.0f, nullptr, nullptr, 0, 0.0f, 0};
        if (tbn_hip::gemm_wide_fits(wa, ternary)) {
            k = tbn_hip::gemm_wide_kernel_name(wa, ternary);
        } else {
            const bool big = tbn_hip::ceil_div(M, CfgBig::BR) * tbn_hip::ceil_div(N, CfgBig::BC) >= 256;
            k = std::string("mfma_tile_kernel<TileCfg<") + (big ? "128, 256, 64, 128, 2" : "64, 64, 32, 32, 1") +
                ">, ...>";
        }
    }
    std::snprintf(name, len, "%s", k.c_str());
    return tbn_hip::ok();
}

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
    if (small_gemm_fits(N, K)) {
        const SmallGemm sg{A, transA ? 1 : K, transA ? M : 1, B, transB ? 1 : N, transB ? K : 1,
                           static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), 0, 0, 0, 0};
        return launch_small_gemm<0>(sg, epi, tbn_hip::stream_of(stream));
    }
    if (rows_gemm_fits(N, K)) {
        const bool kvec = K % 4 == 0;
        const RowsGemm rg{A, transA ? 1 : K, transA ? M : 1, B, transB ? 1 : N, transB ? K : 1,
                          static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                          !transA && kvec && reinterpret_cast<uintptr_t>(A) % 16 == 0,
                          transB && kvec && reinterpret_cast<uintptr_t>(B) % 16 == 0};
        const int64_t blocks = tbn_hip::ceil_div(M, kRowsR) * tbn_hip::ceil_div(N, kRowsC);
        TBN_REQUIRE(blocks < (1LL << 31), TBN_INVALID_SHAPE, "too many column tiles");
        hipLaunchKernelGGL(rows_gemm_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                           tbn_hip::stream_of(stream), rg, epi);
        return tbn_hip::check_launch("gemm_f32 (rows)");
    }
    const int tiles_r = static_cast<int>(tbn_hip::ceil_div(M, Cfg::BR));
    const int tiles_c = static_cast<int>(tbn_hip::ceil_div(N, Cfg::BC));
    const int splits = f32_gemm_splits(N, K);
    if (splits > 1) {
        // ksplit: a multiple of the K step; the last split may be shorter
        const int ksplit = static_cast<int>(tbn_hip::ceil_div(tbn_hip::ceil_div(K, splits), 32) * 32);
        const int used = static_cast<int>(tbn_hip::ceil_div(K, ksplit));
        hipStream_t s = tbn_hip::stream_of(stream);
        void* part = nullptr;
        bool temporary = false;
        int rc = tbn_hip::stream_workspace(s, static_cast<size_t>(used) * M * N * sizeof(float), part, temporary);
        if (rc) return rc;
        hipLaunchKernelGGL((gemm_f32_split_kernel<Cfg>), dim3(used * tiles_r * tiles_c), dim3(Cfg::NT), 0, s, rowl,
                           coll, static_cast<float*>(part), static_cast<int>(M), static_cast<int>(N),
                           static_cast<int>(K), ksplit, tiles_r, tiles_c);
        rc = tbn_hip::check_launch("gemm_f32 (split)");
        if (rc == TBN_SUCCESS) {
            const int blocks = static_cast<int>(std::min<int64_t>(tbn_hip::ceil_div(M * N, 256), 2048));
            hipLaunchKernelGGL(gemm_f32_reduce_kernel, dim3(blocks), dim3(256), 0, s,
                               static_cast<const float*>(part), used, static_cast<int>(M), static_cast<int>(N),
                               alpha, epi.cin, c_is_1d, beta, flags, out);
            rc = tbn_hip::check_launch("gemm_f32 (split reduce)");
        }
        tbn_hip::release_workspace(part, temporary, s);
        return rc;
    }
    hipLaunchKernelGGL((mfma_tile_kernel<Cfg, SplitMatrix<Cfg::BR, Cfg::NT>,
                                         SplitMatrix<Cfg::BC, Cfg::NT>, GemmEpi>),
                       dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, tbn_hip::stream_of(stream), rowl,
                       coll, epi, static_cast<int>(K), tiles_r, tiles_c);
    return tbn_hip::check_launch("gemm_f32");
}

}  // extern "C"
