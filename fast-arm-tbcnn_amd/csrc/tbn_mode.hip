// TBN mode: the reference's production arithmetic for qlinear_matmul_binary
// and the Session's cached convolutions.  Activations are ternarized at
// (lo, hi) -- v < lo -> -1, v > hi -> +1, else 0 -- and multiplied by the +-1
// BinaryMatrix weights in exact integer arithmetic.
//
//   * tbn_hip_ternary_pack_f32 / tbn_hip_im2col_ternary_packed produce the
//     reference's two row-major bit planes (TernaryMatrix::pack_from_float,
//     im2col_ternary_packed), bit for bit.
//   * The GEMM runs on v_mfma_i32_32x32x32_i8.  The ternary activations are
//     expanded once per call into int8 rows T (-1 / 0 / +1, zero padded) with
//     their row sums; the weights stay packed and each wave expands its own
//     columns' bits to 0/1 bytes b in registers (3 VALU per 4 weights).  With
//     w = 1 - 2b the exact result is C = rowsum(T) - 2 * (T . b), accumulated
//     in int32 -- the value the reference forms as popcount(pos) -
//     popcount(neg) per 64-bit word (GeMM/05-final/GeMM.cpp:160-252).
//   * Block tile 128 rows x 512 columns, 8 waves of 128 x 64 (4 x 2 fragments),
//     64 k per LDS buffer (two int8 MFMA slices), one barrier per step; rows
//     of T and packed columns are read with buffer loads (out-of-range rows /
//     columns read as zero).
#include <type_traits>

#include "common.hpp"
#include "conv_common.hpp"
#include "mfma_core.hpp"

namespace {

using namespace tbnk;

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer resource: raw dword addressing

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
    const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : static_cast<uint32_t>(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(n),
                                             kRsrcWord3);
}

// ---------------------------------------------------------------------------
// Activation packing
// ---------------------------------------------------------------------------

// Two bit planes [rows, cols / 8] of A [M, K] (zero padded): bit c of row r is
// set in neg when a < lo, in pos when a > hi.  One thread per 32-bit word.
// Float input: GeMM/05-final/GeMM.cpp:71-112 and
// tbn-runtime/src/operators/quantized_gemm_neon.cpp:118-141; int8 input (lo =
// -0.5, hi = 0.5, so the sign picks the plane): GeMM/05-final/GeMM.cpp:29-69.
template <typename T>
__global__ void ternary_planes_kernel(const T* __restrict__ A, int64_t lda, int64_t M, int64_t K,
                                      int64_t rows, int64_t wpr, float lo, float hi, uint32_t* __restrict__ pos,
                                      uint32_t* __restrict__ neg) {
    const int64_t total = rows * wpr;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = t / wpr;
        const int64_t c0 = (t - row * wpr) * 32;
        uint32_t p = 0, m = 0;
        if (row < M) {
            const T* src = A + row * lda;
#pragma unroll 8
            for (int e = 0; e < 32; ++e) {
                const float v = (c0 + e < K) ? static_cast<float>(src[c0 + e]) : 0.0f;
                m |= (v < lo ? 1u : 0u) << e;
                p |= (!(v < lo) && v > hi ? 1u : 0u) << e;
            }
        }
        pos[t] = p;
        neg[t] = m;
    }
}

// The im2col matrix [N*OH*OW, C*kh*kw] (k = (c*kh + r)*kw + s) ternarized into
// two bit planes [m_pad, k_pad / 8]; taps outside the image and padding are 0.
// tbn-runtime/src/operators/conv2d.cpp:511-601
struct Im2colDims {
    int C, H, W, kh, kw, sh, sw, ph, pw, dh, dw, OH, OW;
    int64_t positions;  // N * OH * OW
    int K;              // C * kh * kw
};

__global__ void im2col_ternary_kernel(const float* __restrict__ x, Im2colDims d, int64_t m_pad, int64_t wpr,
                                      float lo, float hi, uint32_t* __restrict__ pos, uint32_t* __restrict__ neg) {
    const int64_t total = m_pad * wpr;
    const int taps = d.kh * d.kw;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = t / wpr;
        const int c0 = static_cast<int>((t - row * wpr) * 32);
        uint32_t p = 0, m = 0;
        if (row < d.positions) {
            const int64_t plane = static_cast<int64_t>(d.OH) * d.OW;
            const int64_t n = row / plane;
            const int rem = static_cast<int>(row - n * plane);
            const int oh = rem / d.OW, ow = rem - (rem / d.OW) * d.OW;
            const float* img = x + n * d.C * static_cast<int64_t>(d.H) * d.W;
            for (int e = 0; e < 32; ++e) {
                const int col = c0 + e;
                if (col >= d.K) break;
                const int c = col / taps;
                const int tap = col - c * taps;
                const int r = tap / d.kw, s = tap - (tap / d.kw) * d.kw;
                const int ih = oh * d.sh - d.ph + r * d.dh;
                const int iw = ow * d.sw - d.pw + s * d.dw;
                if (static_cast<unsigned>(ih) >= static_cast<unsigned>(d.H) ||
                    static_cast<unsigned>(iw) >= static_cast<unsigned>(d.W))
                    continue;
                const float v = img[(static_cast<int64_t>(c) * d.H + ih) * d.W + iw];
                if (v < lo) m |= 1u << e;
                else if (v > hi) p |= 1u << e;
            }
        }
        pos[t] = p;
        neg[t] = m;
    }
}

// ---------------------------------------------------------------------------
// Expansion to int8 rows + row sums (the GEMM's activation operand)
// ---------------------------------------------------------------------------

// Block-wide int32 sum (blockDim.x a multiple of 64, at most 1024).
__device__ __forceinline__ int block_sum(int v, int* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    int s = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) s += red[w];
    return s;
}

// int8 byte of one ternary value from its plane bits.
__device__ __forceinline__ uint32_t tern_byte(bool p, bool m) { return m ? 0xFFu : (p ? 0x01u : 0x00u); }

// fp32 rows -> int8 T[row, 0..ldt) and rowsum[row]; one block per row.
__global__ void ternarize_rows_kernel(const float* __restrict__ A, int64_t lda, int M, int K, int64_t ldt, float lo,
                                      float hi, int8_t* __restrict__ T, int* __restrict__ rowsum) {
    __shared__ int red[16];
    for (int row = blockIdx.x; row < M; row += gridDim.x) {
        const float* src = A + static_cast<int64_t>(row) * lda;
        uint32_t* dst = reinterpret_cast<uint32_t*>(T + static_cast<int64_t>(row) * ldt);
        int sum = 0;
        // rows of whole float4s (K and lda multiples of 4, A 16-byte aligned):
        // one vector load per output word
        const bool vec = (K % 4 == 0) && (lda % 4 == 0) && (reinterpret_cast<uintptr_t>(A) % 16 == 0);
        for (int64_t w = threadIdx.x; w < ldt / 4; w += blockDim.x) {
            float v[4];
            if (vec) {
                const float4 f = 4 * w < K ? *reinterpret_cast<const float4*>(src + 4 * w) : make_float4(0, 0, 0, 0);
                v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = 4 * w + e < K ? src[4 * w + e] : 0.0f;
            }
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool m = v[e] < lo, p = !m && v[e] > hi;
                sum += (p ? 1 : 0) - (m ? 1 : 0);
                word |= tern_byte(p, m) << (8 * e);
            }
            dst[w] = word;
        }
        sum = block_sum(sum, red);
        if (threadIdx.x == 0) rowsum[row] = sum;
    }
}

// Bit planes [M, n / 8] -> int8 T[row, 0..n) and rowsum[row]; one block per row.
__global__ void planes_to_rows_kernel(const uint8_t* __restrict__ pos, const uint8_t* __restrict__ neg, int M,
                                      int64_t n, int8_t* __restrict__ T, int* __restrict__ rowsum) {
    __shared__ int red[16];
    for (int row = blockIdx.x; row < M; row += gridDim.x) {
        const uint8_t* rp = pos + static_cast<int64_t>(row) * (n / 8);
        const uint8_t* rm = neg + static_cast<int64_t>(row) * (n / 8);
        uint32_t* dst = reinterpret_cast<uint32_t*>(T + static_cast<int64_t>(row) * n);
        int sum = 0;
        for (int64_t w = threadIdx.x; w < n / 4; w += blockDim.x) {
            const uint32_t pb = (rp[w >> 1] >> (4 * (w & 1))) & 0xFu;
            const uint32_t mb = (rm[w >> 1] >> (4 * (w & 1))) & 0xFu;
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool p = (pb >> e) & 1u, m = (mb >> e) & 1u;
                // both bits set contributes 0 in the reference's formula
                const bool pp = p && !m, mm = m && !p;
                sum += (pp ? 1 : 0) - (mm ? 1 : 0);
                word |= tern_byte(pp, mm) << (8 * e);
            }
            dst[w] = word;
        }
        sum = block_sum(sum, red);
        if (threadIdx.x == 0) rowsum[row] = sum;
    }
}

// ---------------------------------------------------------------------------
// The int8 GEMM
// ---------------------------------------------------------------------------

struct TbnGemmArgs {
    const int8_t* T;      // [M, ldt] ternary activations, zero beyond K
    int64_t ldt;          // bytes per row (>= K, multiple of 16)
    const int* rowsum;    // [M]
    int M, N, K;          // K = shared dimension, a multiple of 64
    const uint8_t* bits;  // BinaryMatrix columns (col_bytes each, bit 1 = -1)
    int64_t col_bytes;
    int N_pad;            // columns present in bits
    void* out;            // int32 or float [M, ldo]
    int64_t ldo;
    float scale;          // float output: out = float(C) * scale
};

template <int BR_, int BC_, int WR_, int WC_, int KS_>
struct I8Cfg {
    static constexpr int BR = BR_, BC = BC_, WR = WR_, WC = WC_;
    static constexpr int KS = KS_;        // k per step (one barrier): KS / 128 16-byte weight words per column
    static constexpr int SL = KS / 32;    // MFMA slices per step
    static constexpr int WPS = KS / 32;   // 32-bit weight words per column per step
    static constexpr int KROW = KS + 16;  // bytes per LDS row: conflict-free 16-byte fragment reads
    static constexpr int WAVES_R = BR / WR, WAVES_C = BC / WC;
    static constexpr int NT = 64 * WAVES_R * WAVES_C;
    static constexpr int FR = WR / 32, FC = WC / 32;
    static constexpr int TPR = NT / BR;   // threads per A row
    static constexpr int ALD = KS / TPR / 16;  // 16-byte A loads per thread per step
    static_assert(TPR * ALD * 16 == KS && KS % 128 == 0, "a step's A tile is whole 16-byte loads per thread");
};

using I8Wide = I8Cfg<128, 512, 128, 64, 128>;

// 4 weight bits (bit i = weight k0 + i, 1 means -1) -> 4 bytes b_i in {0, 1}:
// the multiply copies bit i to bit 8i without carries.
__device__ __forceinline__ uint32_t spread4(uint32_t nib) { return __umul24(nib, 0x204081u) & 0x01010101u; }

template <class Cfg, bool FLOAT_OUT>
__global__ void __launch_bounds__(Cfg::NT)
tbn_i8_gemm_kernel(TbnGemmArgs p, int tiles_r, int tiles_c) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * Cfg::BR * Cfg::KROW];
    __shared__ __attribute__((aligned(16))) int rs_lds[Cfg::BR];
    constexpr int KS = Cfg::KS;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave / Cfg::WAVES_C;
    const int wc = wave % Cfg::WAVES_C;
    const int h = lane >> 5;

    const int total = tiles_r * tiles_c;
    int t = blockIdx.x;
    if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
    const int tr = t / tiles_c;
    const int tc = t - tr * tiles_c;
    const int r0 = tr * Cfg::BR;
    const int c0 = tc * Cfg::BC;

    if (tid < Cfg::BR) rs_lds[tid] = (r0 + tid < p.M) ? p.rowsum[r0 + tid] : 0;

    const int ar = tid / Cfg::TPR, ag = tid % Cfg::TPR;
    const __amdgpu_buffer_rsrc_t a_rs =
        make_rsrc(p.T + static_cast<int64_t>(r0) * p.ldt, static_cast<uint64_t>(p.M - r0) * p.ldt);
    const int a_voff = ar * static_cast<int>(p.ldt) + ag * 16 * Cfg::ALD;
    const __amdgpu_buffer_rsrc_t b_rs =
        make_rsrc(p.bits + static_cast<int64_t>(c0) * p.col_bytes,
                  static_cast<uint64_t>(p.N_pad - c0) * static_cast<uint64_t>(p.col_bytes));
    int b_voff[Cfg::FC];
#pragma unroll
    for (int j = 0; j < Cfg::FC; ++j)
        b_voff[j] = (wc * Cfg::WC + j * 32 + (lane & 31)) * static_cast<int>(p.col_bytes);

    // K is a multiple of 64: a last step of 64 runs two of its four slices
    // (the data loaded past K for the other two is never used)
    // K is a multiple of 64: the last step runs K % KS / 32 of its slices
    // (the data loaded past K for the others is never used)
    constexpr int SL = Cfg::SL, WPS = Cfg::WPS;
    const int steps = (p.K + KS - 1) / KS;
    const int last_slices = (p.K % KS) ? (p.K % KS) / 32 : SL;

    i32x4_t areg[Cfg::ALD];
    uint32_t bw[Cfg::FC][WPS], bwn[Cfg::FC][WPS];
    auto load_a = [&](int s) {
#pragma unroll
        for (int h2 = 0; h2 < Cfg::ALD; ++h2)
            areg[h2] = __builtin_amdgcn_raw_buffer_load_b128(a_rs, a_voff + 16 * h2, s * KS, 0);
    };
    auto load_b = [&](int s, uint32_t (&w)[Cfg::FC][WPS]) {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int q = 0; q < WPS / 4; ++q) {
                const u32x4_t x = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rs, b_voff[j], s * (KS / 8) + 16 * q, 0));
#pragma unroll
                for (int d = 0; d < 4; ++d) w[j][4 * q + d] = x[d];
            }
    };
    const int a_store = ar * Cfg::KROW + ag * 16 * Cfg::ALD;
    auto store_a = [&](int b) {
#pragma unroll
        for (int h2 = 0; h2 < Cfg::ALD; ++h2)
            *reinterpret_cast<i32x4_t*>(lds + b * Cfg::BR * Cfg::KROW + a_store + 16 * h2) = areg[h2];
    };

    i32x16_t acc[Cfg::FR][Cfg::FC];
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    const int a_frag = (wr * Cfg::WR + (lane & 31)) * Cfg::KROW + h * 16;

    // Step s: four MFMA slices of 32 k on LDS buffer s & 1; meanwhile step
    // s+1's A goes to the other buffer and step s+2's A and s+1's W words are
    // fetched.  Software pipeline across slices: slice kk+1's weight bits are
    // expanded and its A fragments read from LDS while slice kk's MFMAs run
    // (the next step's slice 0 comes from the next step's words and, after
    // the barrier, from the other LDS buffer).
    i32x4_t bfr[2][Cfg::FC];
    i32x4_t afr[2][Cfg::FR];
    auto expand_b = [&](const uint32_t (&w)[Cfg::FC][WPS], int kk, i32x4_t (&bf)[Cfg::FC]) {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            const uint32_t word = w[j][kk];
#pragma unroll
            for (int d = 0; d < 4; ++d)
                bf[j][d] = static_cast<int>(spread4(__builtin_amdgcn_ubfe(word, 16 * h + 4 * d, 4)));
        }
    };
    auto read_a = [&](int u, int kk, i32x4_t (&af)[Cfg::FR]) {
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
            af[i] = *reinterpret_cast<const i32x4_t*>(lds + u * Cfg::BR * Cfg::KROW + i * 32 * Cfg::KROW + a_frag +
                                                      kk * 32);
    };
    auto mfmas = [&](const i32x4_t (&af)[Cfg::FR], const i32x4_t (&bf)[Cfg::FC]) {
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    };

    load_a(0);
    load_b(0, bw);
    store_a(0);
    if (steps > 1) {
        load_a(1);
        load_b(1, bwn);
    }
    expand_b(bw, 0, bfr[0]);
    __syncthreads();
    int s = 0;
    // full steps that have a successor: four slices, the last one prepares the
    // next step's slice 0 weights (its A fragments follow the barrier)
    for (; s + 1 < steps; ++s) {
        const int u = s & 1;
        read_a(u, 0, afr[0]);
#pragma unroll
        for (int kk = 0; kk < SL; ++kk) {
            if (kk + 1 < SL) {
                read_a(u, kk + 1, afr[(kk + 1) & 1]);
                expand_b(bw, kk + 1, bfr[(kk + 1) & 1]);
            } else {
                expand_b(bwn, 0, bfr[0]);
            }
            mfmas(afr[kk & 1], bfr[kk & 1]);
            // per slice: the next slice's 4 fragment reads up front, then 8
            // MFMAs, each followed by 3 of the 24 expansion VALU
            if (kk + 1 < SL) __builtin_amdgcn_sched_group_barrier(0x100, Cfg::FR, 0);
#pragma unroll
            for (int q = 0; q < Cfg::FR * Cfg::FC; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
        }
        store_a(u ^ 1);
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int d = 0; d < WPS; ++d) bw[j][d] = bwn[j][d];
        if (s + 2 < steps) {
            load_a(s + 2);
            load_b(s + 2, bwn);
        }
        __syncthreads();
    }
    // the last step: an even number of slices (K is a multiple of 64)
    {
        const int u = s & 1;
        read_a(u, 0, afr[0]);
#pragma unroll
        for (int kk = 0; kk < SL; ++kk) {
            if (kk >= last_slices) break;
            if (kk + 1 < last_slices) {
                read_a(u, kk + 1, afr[(kk + 1) & 1]);
                expand_b(bw, kk + 1, bfr[(kk + 1) & 1]);
            }
            mfmas(afr[kk & 1], bfr[kk & 1]);
        }
    }

    // epilogue: C = rowsum - 2 * acc; rows of register e: i*32 + 8*(e/4) + 4*h + e%4
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i) {
        int rsum[16];
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const i32x4_t r = *reinterpret_cast<const i32x4_t*>(rs_lds + wr * Cfg::WR + i * 32 + 8 * e4 + 4 * h);
            rsum[4 * e4] = r[0], rsum[4 * e4 + 1] = r[1], rsum[4 * e4 + 2] = r[2], rsum[4 * e4 + 3] = r[3];
        }
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            const int n = c0 + wc * Cfg::WC + j * 32 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = r0 + wr * Cfg::WR + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                const int c = rsum[e] - 2 * acc[i][j][e];
                if (m < p.M && n < p.N) {
                    if (FLOAT_OUT)
                        static_cast<float*>(p.out)[static_cast<int64_t>(m) * p.ldo + n] = static_cast<float>(c) * p.scale;
                    else
                        static_cast<int*>(p.out)[static_cast<int64_t>(m) * p.ldo + n] = c;
                }
            }
        }
    }
}

int launch_i8_gemm(const TbnGemmArgs& a, bool float_out, hipStream_t stream) {
    using Cfg = I8Wide;
    const int tiles_r = static_cast<int>(tbn_hip::ceil_div(a.M, Cfg::BR));
    const int tiles_c = static_cast<int>(tbn_hip::ceil_div(a.N, Cfg::BC));
    if (float_out)
        hipLaunchKernelGGL((tbn_i8_gemm_kernel<Cfg, true>), dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, stream, a,
                           tiles_r, tiles_c);
    else
        hipLaunchKernelGGL((tbn_i8_gemm_kernel<Cfg, false>), dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, stream, a,
                           tiles_r, tiles_c);
    return tbn_hip::check_launch("tbn_gemm");
}

int grid_for(int64_t items, int threads) {
    return static_cast<int>(std::min<int64_t>(tbn_hip::ceil_div(std::max<int64_t>(items, 1), threads), 65536));
}

// Stream-ordered scratch for the int8 rows and row sums.
// Device scratch of one call (the stream workspace, see common.hpp).
struct Scratch {
    void* ptr = nullptr;
    bool temporary = false;
    hipStream_t stream = nullptr;
    int get(size_t bytes) { return tbn_hip::stream_workspace(stream, bytes, ptr, temporary); }
    ~Scratch() { tbn_hip::release_workspace(ptr, temporary, stream); }
};

}  // namespace

extern "C" {

}  // extern "C"

namespace {

template <typename T>
int ternary_pack(const T* A, int64_t lda, int64_t M, int64_t K, int64_t rows, int64_t cols, float lo, float hi,
                 uint8_t* pos, uint8_t* neg, tbn_stream_t stream, const char* what) {
    TBN_REQUIRE(M >= 0 && K >= 0 && rows >= M && cols >= K, TBN_INVALID_ARGUMENT,
                "padded dimensions must cover the matrix");
    TBN_REQUIRE(rows % 8 == 0 && cols % 64 == 0, TBN_INVALID_ARGUMENT,
                "ternary matrix rows must be a multiple of 8 and columns a multiple of 64");
    TBN_REQUIRE(M == 0 || lda >= K, TBN_INVALID_ARGUMENT, "lda must be >= K");
    if (rows == 0 || cols == 0) return tbn_hip::ok();
    TBN_REQUIRE(pos && neg && (M == 0 || K == 0 || A), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const int64_t wpr = cols / 32;
    hipLaunchKernelGGL(ternary_planes_kernel<T>, dim3(grid_for(rows * wpr, 256)), dim3(256), 0,
                       tbn_hip::stream_of(stream), A, lda, M, K, rows, wpr, lo, hi,
                       reinterpret_cast<uint32_t*>(pos), reinterpret_cast<uint32_t*>(neg));
    return tbn_hip::check_launch(what);
}

// Ternary rows (pos / neg planes, m rows of n / 8 bytes) times BinaryMatrix
// columns: int32 C, or float(C) * scale when `float_out`, into out [m, ldo]
// for the first `cols` columns.
int planes_gemm(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits, int64_t m, int64_t n, int64_t cols,
                int64_t bit_cols, bool float_out, float scale, void* out, int64_t ldo, hipStream_t s) {
    Scratch scr;
    scr.stream = s;
    const size_t tbytes = static_cast<size_t>(m) * n;
    if (int rc = scr.get(tbytes + static_cast<size_t>(m) * 4 + 16)) return rc;
    int8_t* T = static_cast<int8_t*>(scr.ptr);
    int* rowsum = reinterpret_cast<int*>(static_cast<uint8_t*>(scr.ptr) + ((tbytes + 15) / 16) * 16);
    hipLaunchKernelGGL(planes_to_rows_kernel, dim3(static_cast<int>(std::min<int64_t>(m, 65536))), dim3(256), 0, s,
                       pos, neg, static_cast<int>(m), n, T, rowsum);
    int rc = tbn_hip::check_launch("tbn_gemm (planes)");
    if (rc != TBN_SUCCESS) return rc;
    TbnGemmArgs a{T, n, rowsum, static_cast<int>(m), static_cast<int>(cols), static_cast<int>(n), bits, n / 8,
                  static_cast<int>(bit_cols), out, ldo, scale};
    return launch_i8_gemm(a, float_out, s);
}

}  // namespace

extern "C" {

int tbn_hip_ternary_pack_f32(const float* A, int64_t lda, int64_t M, int64_t K, int64_t rows, int64_t cols, float lo,
                             float hi, uint8_t* pos, uint8_t* neg, tbn_stream_t stream) {
    return ternary_pack(A, lda, M, K, rows, cols, lo, hi, pos, neg, stream, "ternary_pack_f32");
}

int tbn_hip_ternary_pack_i8(const int8_t* A, int64_t lda, int64_t M, int64_t K, int64_t rows, int64_t cols,
                            uint8_t* pos, uint8_t* neg, tbn_stream_t stream) {
    return ternary_pack(A, lda, M, K, rows, cols, -0.5f, 0.5f, pos, neg, stream, "ternary_pack_i8");
}

int tbn_hip_im2col_ternary_packed(const float* x, const tbn_conv2d_desc* desc, int64_t m_pad, int64_t k_pad,
                                  float lo, float hi, uint8_t* pos, uint8_t* neg, tbn_stream_t stream) {
    ConvGeom g;
    const int rc = make_geom(desc, 0, g);
    if (rc != TBN_SUCCESS) return rc;
    const int64_t OH = (desc->h + 2 * desc->ph - desc->dh * (desc->kh - 1) - 1) / desc->sh + 1;
    Im2colDims d{g.C, g.H, g.W, g.kh, g.kw, g.sh, g.sw, g.ph, g.pw, g.dh, g.dw, static_cast<int>(OH), g.OW,
                 desc->n * OH * g.OW, g.K};
    TBN_REQUIRE(m_pad >= d.positions && k_pad >= d.K && k_pad % 32 == 0, TBN_INVALID_ARGUMENT,
                "m_pad / k_pad must cover the im2col matrix and k_pad be a multiple of 32");
    if (m_pad == 0) return tbn_hip::ok();
    TBN_REQUIRE(pos && neg && (d.positions == 0 || x), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const int64_t wpr = k_pad / 32;
    hipLaunchKernelGGL(im2col_ternary_kernel, dim3(grid_for(m_pad * wpr, 256)), dim3(256), 0,
                       tbn_hip::stream_of(stream), x, d, m_pad, wpr, lo, hi, reinterpret_cast<uint32_t*>(pos),
                       reinterpret_cast<uint32_t*>(neg));
    return tbn_hip::check_launch("im2col_ternary_packed");
}

int tbn_hip_tbn_gemm(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits, int64_t m, int64_t n, int64_t k,
                     int32_t* C, tbn_stream_t stream) {
    TBN_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1LL << 31) && k < (1LL << 31) && n < (1LL << 24),
                TBN_INVALID_SHAPE, "m, n, k out of range");
    TBN_REQUIRE(n % 64 == 0, TBN_INVALID_ARGUMENT, "the shared dimension n must be a multiple of 64");
    if (m == 0 || k == 0) return tbn_hip::ok();
    TBN_REQUIRE(C && (n == 0 || (pos && neg && bits)), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipStream_t s = tbn_hip::stream_of(stream);
    if (n == 0) {
        if (hipMemsetAsync(C, 0, static_cast<size_t>(m) * k * sizeof(int32_t), s) != hipSuccess)
            return tbn_hip::fail(TBN_RUNTIME_ERROR, "hipMemsetAsync failed");
        return tbn_hip::ok();
    }
    return planes_gemm(pos, neg, bits, m, n, k, k, false, 1.0f, C, k, s);
}

int tbn_hip_tbn_gemm_scaled(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits, int64_t m, int64_t n,
                            int64_t k, int64_t cols, float scale, float* out, int64_t ldo, tbn_stream_t stream) {
    TBN_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1LL << 31) && k < (1LL << 31) && n < (1LL << 24),
                TBN_INVALID_SHAPE, "m, n, k out of range");
    TBN_REQUIRE(n % 64 == 0, TBN_INVALID_ARGUMENT, "the shared dimension n must be a multiple of 64");
    TBN_REQUIRE(cols >= 0 && cols <= k, TBN_INVALID_SHAPE, "cols must be in [0, k]");
    TBN_REQUIRE(ldo >= cols, TBN_INVALID_ARGUMENT, "ldo must be >= cols");
    if (m == 0 || cols == 0) return tbn_hip::ok();
    TBN_REQUIRE(out && (n == 0 || (pos && neg && bits)), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipStream_t s = tbn_hip::stream_of(stream);
    if (n == 0) {
        if (hipMemset2DAsync(out, ldo * sizeof(float), 0, cols * sizeof(float), m, s) != hipSuccess)
            return tbn_hip::fail(TBN_RUNTIME_ERROR, "hipMemset2DAsync failed");
        return tbn_hip::ok();
    }
    return planes_gemm(pos, neg, bits, m, n, cols, k, true, scale, out, ldo, s);
}

int tbn_hip_qlinear_matmul_binary_tbn(const float* A, int64_t lda, int64_t M, int64_t K, const uint8_t* packed,
                                      int64_t K_pad, int64_t N, int64_t N_pad, float scale, float lo, float hi,
                                      float* out, int64_t ldo, tbn_stream_t stream) {
    TBN_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M < (1LL << 31) && N < (1LL << 31) && K_pad < (1LL << 24),
                TBN_INVALID_SHAPE, "M, N, K out of range");
    TBN_REQUIRE(K_pad >= K && K_pad % 64 == 0, TBN_INVALID_SHAPE, "K_pad must be >= K and a multiple of 64");
    TBN_REQUIRE(N_pad >= N, TBN_INVALID_SHAPE, "N_pad must be >= N");
    TBN_REQUIRE(M == 0 || lda >= K, TBN_INVALID_ARGUMENT, "lda must be >= K");
    TBN_REQUIRE(ldo >= N, TBN_INVALID_ARGUMENT, "ldo must be >= N");
    if (M == 0 || N == 0) return tbn_hip::ok();
    TBN_REQUIRE(out && (K == 0 || (A && packed)), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    hipStream_t s = tbn_hip::stream_of(stream);
    if (K_pad == 0) {
        if (hipMemset2DAsync(out, ldo * sizeof(float), 0, N * sizeof(float), M, s) != hipSuccess)
            return tbn_hip::fail(TBN_RUNTIME_ERROR, "hipMemset2DAsync failed");
        return tbn_hip::ok();
    }
    Scratch scr;
    scr.stream = s;
    const size_t tbytes = static_cast<size_t>(M) * K_pad;
    if (int rc = scr.get(tbytes + static_cast<size_t>(M) * 4 + 16)) return rc;
    int8_t* T = static_cast<int8_t*>(scr.ptr);
    int* rowsum = reinterpret_cast<int*>(static_cast<uint8_t*>(scr.ptr) + ((tbytes + 15) / 16) * 16);
    hipLaunchKernelGGL(ternarize_rows_kernel, dim3(static_cast<int>(std::min<int64_t>(M, 65536))), dim3(256), 0, s,
                       A, lda, static_cast<int>(M), static_cast<int>(K), K_pad, lo, hi, T, rowsum);
    int rc = tbn_hip::check_launch("qlinear_matmul_binary_tbn (ternarize)");
    if (rc != TBN_SUCCESS) return rc;
    TbnGemmArgs a{T, K_pad, rowsum, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K_pad), packed,
                  K_pad / 8, static_cast<int>(N_pad), out, ldo, scale};
    return launch_i8_gemm(a, true, s);
}

}  // extern "C"
