// TBN mode: the reference's production arithmetic for qlinear_matmul_binary
// and the Session's cached convolutions.  Activations are ternarized at
// (lo, hi) -- v < lo -> -1, v > hi -> +1, else 0 -- and multiplied by the +-1
// BinaryMatrix weights in exact integer arithmetic.
//
//   * tbn_hip_ternary_pack_f32 / tbn_hip_im2col_ternary_packed produce the
//     reference's two row-major bit planes (TernaryMatrix::pack_from_float,
//     im2col_ternary_packed), bit for bit.
//   * The GEMM runs on the fp4 matrix cores
//     (v_mfma_scale_f32_32x32x64_f8f6f4, unit scales): -1, 0 and +1 are exact
//     E2M1 values, so every product is exact and every partial sum an integer
//     below 2^24, exact in the fp32 accumulators -- the value the reference
//     forms as popcount(pos) - popcount(neg) per 64-bit word
//     (GeMM/05-final/GeMM.cpp:160-252).  One pass per call turns the
//     activations (fp32 rows or bit planes) and the packed weight columns
//     into k-contiguous fp4 rows (two values a byte).
//   * Block tile 256 x 256, 8 waves of 128 x 64 (4 x 2 fragments), 256 k per
//     LDS buffer; both operands go global -> LDS by buffer_load ... lds (rows
//     past the matrix read as zero), one barrier per step.
#include <type_traits>

#include "common.hpp"
#include "conv_common.hpp"
#include "mfma_core.hpp"
#include "tbn_f4.hpp"

namespace {

using namespace tbnk;

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
// The fp4 operands of the GEMM
// ---------------------------------------------------------------------------

// Activation rows of the operand pass, one fp4 dword (8 values) per call.
// fp32 rows ternarized at (lo, hi): v < lo -> -1, v > hi -> +1, else 0 (NaN
// gives 0), zero beyond K (GeMM/05-final/GeMM.cpp:71-112 and
// tbn-runtime/src/operators/quantized_gemm_neon.cpp:118-141 form the same
// values as bit planes).
struct RowsF32 {
    const float* A;
    int64_t lda;
    int K;
    float lo, hi;
    bool vec;  // K, lda multiples of 4 and A 16-byte aligned
    __device__ __forceinline__ uint32_t word(int64_t row, int k0) const {
        const float* src = A + row * lda;
        float v[8];
        if (vec) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float4 f = k0 + 4 * q < K ? *reinterpret_cast<const float4*>(src + k0 + 4 * q)
                                                : make_float4(0, 0, 0, 0);
                v[4 * q] = f.x, v[4 * q + 1] = f.y, v[4 * q + 2] = f.z, v[4 * q + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = k0 + e < K ? src[k0 + e] : 0.0f;
        }
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool m = v[e] < lo, p = !m && v[e] > hi;
            w |= (m ? kF4Minus : (p ? kF4Plus : 0u)) << (4 * e);
        }
        return w;
    }
};

// The reference's two bit planes (row-major, n / 8 bytes a row): a value
// with both bits set is 0, as in its popcount(pos) - popcount(neg)
// (GeMM/05-final/GeMM.cpp:160-252).
struct RowsPlanes {
    const uint8_t* pos;
    const uint8_t* neg;
    int64_t row_bytes;
    __device__ __forceinline__ uint32_t word(int64_t row, int k0) const {
        const int64_t i = row * row_bytes + k0 / 8;
        const uint32_t pb = pos[i], mb = neg[i];
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool p = (pb >> e) & 1u, m = (mb >> e) & 1u;
            w |= (p && !m ? kF4Plus : (m && !p ? kF4Minus : 0u)) << (4 * e);
        }
        return w;
    }
};

// Both GEMM operands in one pass: items [0, a_items) are the activation
// dwords T4[row, 0..wpr) (8 values each), the rest the weight columns, 32
// bits of a column each (one 4-byte load, one 16-byte store into W4[col,
// 0..k / 2)).  Indices fit 32 bits (checked on the host).
template <class Act>
__global__ void f4_operands_kernel(Act act, uint32_t a_items, uint32_t wpr, uint32_t* __restrict__ T4,
                                   const uint8_t* __restrict__ bits, int64_t col_bytes, uint32_t wpc,
                                   uint32_t w_items, uint32_t* __restrict__ W4) {
    const uint32_t total = a_items + w_items;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        if (i < a_items) {
            const uint32_t row = i / wpr;
            T4[i] = act.word(row, static_cast<int>(8 * (i - row * wpr)));
        } else {
            const uint32_t j = i - a_items;
            const uint32_t c = j / wpc;
            const uint32_t b = *reinterpret_cast<const uint32_t*>(bits + c * col_bytes + 4 * (j - c * wpc));
            const u32x4_t out = {bits_word(b), bits_word(b >> 8), bits_word(b >> 16), bits_word(b >> 24)};
            *reinterpret_cast<u32x4_t*>(W4 + 4 * static_cast<int64_t>(j)) = out;
        }
    }
}

// ---------------------------------------------------------------------------
// The fp4 GEMM (the TBN product on the fp4 matrix cores)
// ---------------------------------------------------------------------------
//
// -1, 0 and +1 are exact fp4 (E2M1) values: codes 0xA, 0x0 and 0x2.  With the
// ternary activations and the +-1 weights both in fp4, every product is
// exact and every partial sum is an integer of magnitude at most K <= 2^24,
// so v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales) accumulates C exactly in
// fp32 (at twice the int8 MFMA rate).  Operands are
// k-contiguous rows of nibbles, low nibble first: a lane's MFMA operand is
// the 32 values k = 32 (lane / 32) .. +31 of its row or column, 16 bytes.

struct F4GemmArgs {
    const uint8_t* A;     // [M, lda] fp4 activations, two per byte, zero beyond K
    int64_t lda;          // bytes per row (a multiple of 16)
    const uint8_t* B;     // [n_alloc, ldb] fp4 weights (+-1), one row per output column
    int64_t ldb;
    int n_alloc;          // rows present in B
    int M, N, K;          // K = shared dimension, a multiple of 64
    void* out;            // int32 or float [M, ldo]
    int64_t ldo;
    float scale;          // float output: out = float(C) * scale
    const float* cin;     // float output with an addend: out = fma(beta, cin, float(C) * scale)
    int cin_1d;           // cin [N] (else [M, N], row stride N)
    float beta;
    int relu;             // float output: then max(out, 0) (+0 for -0 and NaN)
};

template <int BR_, int BC_, int WR_, int WC_, int KS_, int NBUF_, bool EARLY_>
struct F4Cfg {
    static constexpr int BR = BR_, BC = BC_, WR = WR_, WC = WC_;
    static constexpr int KS = KS_;                  // k per step (one barrier): KS / 64 MFMA slices
    static constexpr int NBUF = NBUF_;              // LDS buffers: loads run NBUF - 1 steps ahead
    static constexpr bool EARLY = EARLY_;           // a slice's fragment reads all issued before its MFMAs
    static constexpr int SL = KS / 64;
    static_assert(SL % 2 == 0, "fragment registers alternate by slice");
    static constexpr int RB = KS / 2;               // bytes of a row per step
    static constexpr int PARTS = RB / 16;           // 16-byte parts of a row per step
    static_assert(PARTS == 4 || PARTS == 8 || PARTS == 16, "swizzle");
    static constexpr int WAVES_R = BR / WR, WAVES_C = BC / WC;
    static constexpr int WAVES = WAVES_R * WAVES_C;
    static constexpr int NT = 64 * WAVES;
    static constexpr int FR = WR / 32, FC = WC / 32;
    static constexpr int BUF = (BR + BC) * RB;      // bytes of one LDS buffer (A rows, then B rows)
    static constexpr int LOADS = BUF / 1024 / WAVES;  // 1 KB direct-to-LDS loads per wave per step
    static_assert(LOADS * WAVES * 1024 == BUF && (BR * RB) % 1024 == 0, "tile");
    static_assert(NBUF >= 2 && NBUF <= 4 && NBUF * BUF <= 160 * 1024 && LOADS * (NBUF - 2) <= 63, "LDS / vmcnt");
};

// 256 x 256 blocks of 8 waves (2 x 4), each 128 rows x 64 columns (4 x 2
// fragments); both operands staged through LDS, so a weight row serves the
// block's two row waves and an activation row its four column waves.  256 k
// per step (four MFMA slices, 64 KB), two buffers: one LDS tile per CU.
// (Four buffers of 128 k measured 3 % slower at 4096^3.)
using F4Wide = F4Cfg<256, 256, 128, 64, 256, 2, false>;

// buffer_load_dwordx4 ... lds: lane l's 16 bytes at voffset + soffset go to
// LDS at dst + 16 l.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t rs, uint8_t* dst, int voffset, int soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16, voffset, soffset,
                                             0, 0);
}

// LDS slot (16 bytes) of part q of tile row r: rows of P parts, the part
// index XOR-swizzled so the 16-byte fragment reads of 16 consecutive rows
// (one part each) hit distinct banks.  A 256-byte bank line holds 16 / P
// rows; the rows sharing a line position differ in r / (16 / P).
template <int P>
__device__ __forceinline__ int f4_swz(int r) { return (r / (16 / P)) & (P - 1); }
template <int P>
__device__ __forceinline__ int f4_slot(int r, int q) { return r * P + (q ^ f4_swz<P>(r)); }

// Operands go global -> LDS with buffer_load_dwordx4 ... lds (no registers,
// no LDS store instructions): a wave's load writes 64 consecutive 16-byte
// slots, so each lane loads the global part that belongs in its slot.
template <class Cfg, bool FLOAT_OUT, bool SESSION = false>
__global__ void __launch_bounds__(Cfg::NT) tbn_f4_gemm_kernel(F4GemmArgs p, int tiles_r, int tiles_c) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::NBUF * Cfg::BUF];
    constexpr int RB = Cfg::RB;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave / Cfg::WAVES_C;
    const int wc = wave % Cfg::WAVES_C;
    const int h = lane >> 5;

    // the tiles of one XCD (blockIdx % 8) are consecutive in t
    const int total = tiles_r * tiles_c;
    int t = blockIdx.x;
    if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
    const int tr = t / tiles_c;
    const int tc = t - tr * tiles_c;
    const int r0 = tr * Cfg::BR;
    const int c0 = tc * Cfg::BC;

    // rows past M / columns past n_alloc read as zero (buffer range); the
    // K step's byte offset is folded into each step's resource base, so the
    // last row's bytes past the end are range-checked too
    const uint8_t* a_base = p.A + static_cast<int64_t>(r0) * p.lda;
    const uint64_t a_bytes = static_cast<uint64_t>(p.M - r0) * p.lda;
    const uint8_t* b_base = p.B + static_cast<int64_t>(c0) * p.ldb;
    const uint64_t b_bytes = c0 < p.n_alloc ? static_cast<uint64_t>(p.n_alloc - c0) * p.ldb : 0;
    // load i of this wave fills slots [64 (wave * LOADS + i), + 64) of a buffer:
    // A rows first, then B rows; lane -> (row, stored part) -> global part
    int voff[Cfg::LOADS];
    bool is_a[Cfg::LOADS];
#pragma unroll
    for (int i = 0; i < Cfg::LOADS; ++i) {
        const int slot = 64 * (wave * Cfg::LOADS + i) + lane;
        const int row_all = slot / Cfg::PARTS;  // row of the A + B tile
        const bool a = (wave * Cfg::LOADS + i) * (64 / Cfg::PARTS) < Cfg::BR;  // a load's rows lie on one side
        const int r = a ? row_all : row_all - Cfg::BR;
        const int q = (slot % Cfg::PARTS) ^ f4_swz<Cfg::PARTS>(row_all);
        is_a[i] = a;
        voff[i] = r * static_cast<int>(a ? p.lda : p.ldb) + q * 16;
    }
    auto load = [&](int s, int u) {
        const __amdgpu_buffer_rsrc_t a_rs = buffer_range(a_base, a_bytes, static_cast<uint64_t>(s) * RB);
        const __amdgpu_buffer_rsrc_t b_rs = buffer_range(b_base, b_bytes, static_cast<uint64_t>(s) * RB);
#pragma unroll
        for (int i = 0; i < Cfg::LOADS; ++i)
            load_lds16(is_a[i] ? a_rs : b_rs, lds + u * Cfg::BUF + 1024 * (wave * Cfg::LOADS + i), voff[i], 0);
    };

    f32x16_t acc[Cfg::FR][Cfg::FC];
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int arow = wr * Cfg::WR + (lane & 31);              // + 32 i
    const int brow = Cfg::BR + wc * Cfg::WC + (lane & 31);    // + 32 j
    auto read_frags = [&](int u, int sl, i32x4_t (&af)[Cfg::FR], i32x4_t (&bf)[Cfg::FC]) {
        const int q = 2 * sl + h;
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
            af[i] = *reinterpret_cast<const i32x4_t*>(lds + u * Cfg::BUF + 16 * f4_slot<Cfg::PARTS>(arow + 32 * i, q));
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
            bf[j] = *reinterpret_cast<const i32x4_t*>(lds + u * Cfg::BUF + 16 * f4_slot<Cfg::PARTS>(brow + 32 * j, q));
    };
    // MFMAs of one slice from fragment registers af / bf, with the LDS reads
    // issued just before (the next slice's fragments) spread between them
    auto mfmas = [&](const i32x4_t (&af)[Cfg::FR], const i32x4_t (&bf)[Cfg::FC], bool reads) {
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j) acc[i][j] = mfma_f4(af[i], bf[j], acc[i][j]);
        if (reads) {
            if (Cfg::EARLY) {
                __builtin_amdgcn_sched_group_barrier(0x100, Cfg::FR + Cfg::FC, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, Cfg::FR * Cfg::FC, 0);
            } else {
#pragma unroll
                for (int q = 0; q < Cfg::FR + Cfg::FC; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, Cfg::FR * Cfg::FC - Cfg::FR - Cfg::FC, 0);
            }
        }
    };

    // Step s computes from LDS buffer s % NBUF while the loads of steps up to
    // s + NBUF - 1 fly straight into the others.  The fragments of slice
    // sl + 1 are read during slice sl; the step's barrier sits before its last
    // slice's MFMAs, so the next step's first fragments are read while they
    // run.  Before the barrier a wave has waited for its loads of step s + 1
    // and for its own LDS reads of buffer s % NBUF, which the loads issued
    // after the barrier (for step s + NBUF) overwrite.
    const int steps = (p.K + Cfg::KS - 1) / Cfg::KS;
    const int last_slices = (p.K % Cfg::KS) ? (p.K % Cfg::KS) / 64 : Cfg::SL;
#pragma unroll
    for (int t = 0; t < Cfg::NBUF - 1; ++t)
        if (t < steps) load(t, t);
    // this wave's loads still allowed in flight once step t's have landed:
    // those of the newer steps t + 1 .. min(steps - 1, t + NBUF - 2)
    auto wait_step = [&](int t) {
        const int newer = min(steps - 1, t + Cfg::NBUF - 2) - t;
        if (newer >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * Cfg::LOADS) : "memory");
        else if (newer == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Cfg::LOADS) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    // The barriers are bare s_barrier: a workgroup fence would wait for every
    // load in flight, the later steps' too.
    wait_step(0);
    __builtin_amdgcn_s_barrier();
    i32x4_t af[2][Cfg::FR], bf[2][Cfg::FC];
    read_frags(0, 0, af[0], bf[0]);
    // a full step s < steps - 1; STEADY: steps s + 1 .. s + NBUF - 2 all exist
    auto full_step = [&](int s, auto steady_c) {
        constexpr bool STEADY = decltype(steady_c)::value;
        const int u = s % Cfg::NBUF;
        if (STEADY) load(s + Cfg::NBUF - 1, (s + Cfg::NBUF - 1) % Cfg::NBUF);
#pragma unroll
        for (int sl = 0; sl + 1 < Cfg::SL; ++sl) {
            read_frags(u, sl + 1, af[(sl + 1) & 1], bf[(sl + 1) & 1]);
            mfmas(af[sl & 1], bf[sl & 1], true);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (STEADY) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((Cfg::NBUF - 2) * Cfg::LOADS) : "memory");
        else wait_step(s + 1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        read_frags((s + 1) % Cfg::NBUF, 0, af[0], bf[0]);
        mfmas(af[1], bf[1], true);
        __builtin_amdgcn_sched_barrier(0);
    };
    int s = 0;
    for (; s + Cfg::NBUF - 1 < steps; ++s) full_step(s, std::true_type{});
    for (; s + 1 < steps; ++s) full_step(s, std::false_type{});
    // the last step: its first fragments are in af[0] / bf[0]
    const int u = s % Cfg::NBUF;
#pragma unroll
    for (int sl = 0; sl < Cfg::SL; ++sl) {
        if (sl >= last_slices) break;
        if (sl + 1 < last_slices) read_frags(u, sl + 1, af[(sl + 1) & 1], bf[(sl + 1) & 1]);
        mfmas(af[sl & 1], bf[sl & 1], false);
    }

    // epilogue: C (an exact integer in fp32); rows of register e: i*32 +
    // 8*(e/4) + 4*h + e%4.  Buffer stores over this block's rows [r0, M),
    // the row step of register e folded into the resource base: rows past M
    // fall outside the range and columns past N get an offset outside every
    // range, so no store is behind a branch (ldo < 2^21, host-checked, keeps
    // row * ldo * 4 below 2^31 for the 256 rows of a tile).
    const uint64_t out_bytes = static_cast<uint64_t>(p.M - r0) * p.ldo * 4;
    const uint8_t* out0 = static_cast<uint8_t*>(p.out) + static_cast<int64_t>(r0) * p.ldo * 4;
    const int ldo4 = static_cast<int>(p.ldo) * 4;
    uint32_t ooff[Cfg::FR][Cfg::FC];
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            const int n = c0 + wc * Cfg::WC + j * 32 + (lane & 31);
            const int row = wr * Cfg::WR + i * 32 + 4 * h;
            ooff[i][j] = n < p.N ? static_cast<uint32_t>(row * ldo4 + n * 4) : 0x80000000u;
        }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const __amdgpu_buffer_rsrc_t o_rs =
            buffer_range(out0, out_bytes, static_cast<uint64_t>(8 * (e >> 2) + (e & 3)) * ldo4);
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j) {
                uint32_t bits;
                if constexpr (SESSION) {
                    // the Session's quantized Gemm (model.hpp:847-870): result * alpha,
                    // then += beta * C, one fused multiply-add as AArch64 compilers
                    // contract it; then a fused Relu node
                    float v = acc[i][j][e] * p.scale;
                    if (p.cin) {
                        const int m = min(r0 + wr * Cfg::WR + i * 32 + 4 * h + 8 * (e >> 2) + (e & 3), p.M - 1);
                        const int n = min(c0 + wc * Cfg::WC + j * 32 + (lane & 31), p.N - 1);
                        const float c = p.cin_1d ? p.cin[n] : p.cin[static_cast<int64_t>(m) * p.N + n];
                        v = __builtin_fmaf(p.beta, c, v);
                    }
                    if (p.relu) v = v > 0.0f ? v : 0.0f;
                    bits = __float_as_uint(v);
                } else {
                    bits = FLOAT_OUT ? __float_as_uint(acc[i][j][e] * p.scale)
                                     : static_cast<uint32_t>(static_cast<int>(acc[i][j][e]));
                }
                __builtin_amdgcn_raw_buffer_store_b32(bits, o_rs, ooff[i][j], 0, 0);
            }
    }
}

int launch_f4_gemm(const F4GemmArgs& a, bool float_out, hipStream_t stream) {
    using Cfg = F4Wide;
    TBN_REQUIRE(a.K <= (1 << 24), TBN_INVALID_SHAPE, "TBN GEMM: shared dimension above 2^24 (fp32 sums inexact)");
    TBN_REQUIRE(a.ldo < (1 << 21), TBN_INVALID_SHAPE, "TBN GEMM: output row stride of 2^21 elements or more");
    const int tiles_r = static_cast<int>(tbn_hip::ceil_div(a.M, Cfg::BR));
    const int tiles_c = static_cast<int>(tbn_hip::ceil_div(a.N, Cfg::BC));
    if (float_out && (a.cin || a.relu))
        hipLaunchKernelGGL((tbn_f4_gemm_kernel<Cfg, true, true>), dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, stream,
                           a, tiles_r, tiles_c);
    else if (float_out)
        hipLaunchKernelGGL((tbn_f4_gemm_kernel<Cfg, true>), dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, stream, a,
                           tiles_r, tiles_c);
    else
        hipLaunchKernelGGL((tbn_f4_gemm_kernel<Cfg, false>), dim3(tiles_r * tiles_c), dim3(Cfg::NT), 0, stream, a,
                           tiles_r, tiles_c);
    return tbn_hip::check_launch("tbn_gemm (fp4)");
}

int grid_for(int64_t items, int threads) {
    return static_cast<int>(std::min<int64_t>(tbn_hip::ceil_div(std::max<int64_t>(items, 1), threads), 65536));
}

// Device scratch of one call (the stream workspace, see common.hpp).
struct Scratch {
    void* ptr = nullptr;
    bool temporary = false;
    hipStream_t stream = nullptr;
    int get(size_t bytes) { return tbn_hip::stream_workspace(stream, bytes, ptr, temporary); }
    ~Scratch() { tbn_hip::release_workspace(ptr, temporary, stream); }
};


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

// One launch of f4_operands_kernel: `rows` activation rows and `cols` weight
// columns (col_bytes apart), both over the first k (a multiple of 64) values.
template <class Act>
int launch_f4_operands(const Act& act, int64_t rows, int64_t k, uint32_t* T4, const uint8_t* bits, int64_t col_bytes,
                       int64_t cols, uint32_t* W4, hipStream_t s, const char* what) {
    const int64_t a_items = rows * (k / 8), w_items = cols * (k / 32);
    TBN_REQUIRE(a_items + w_items < (int64_t{1} << 31), TBN_INVALID_SHAPE,
                "operands beyond 2^31 fp4 dwords (8 GiB) in one call");
    hipLaunchKernelGGL(f4_operands_kernel<Act>, dim3(grid_for(a_items + w_items, 256)), dim3(256), 0, s, act,
                       static_cast<uint32_t>(a_items), static_cast<uint32_t>(k / 8), T4, bits, col_bytes,
                       static_cast<uint32_t>(k / 32), static_cast<uint32_t>(w_items), W4);
    return tbn_hip::check_launch(what);
}

// Ternary rows (pos / neg planes, m rows of n / 8 bytes) times BinaryMatrix
// columns: int32 C, or float(C) * scale when `float_out`, into out [m, ldo]
// for the first `cols` columns.
int planes_gemm(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits, int64_t m, int64_t n, int64_t cols,
                int64_t bit_cols, bool float_out, float scale, void* out, int64_t ldo, hipStream_t s) {
    Scratch scr;
    scr.stream = s;
    const size_t tbytes = (static_cast<size_t>(m) * (n / 2) + 255) / 256 * 256;
    const size_t wbytes = static_cast<size_t>(bit_cols) * (n / 2);
    if (int rc = scr.get(tbytes + wbytes)) return rc;
    uint32_t* T4 = static_cast<uint32_t*>(scr.ptr);
    uint32_t* W4 = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(scr.ptr) + tbytes);
    int rc = launch_f4_operands(RowsPlanes{pos, neg, n / 8}, m, n, T4, bits, n / 8, bit_cols, W4, s,
                                "tbn_gemm (fp4 operands)");
    if (rc != TBN_SUCCESS) return rc;
    F4GemmArgs a{reinterpret_cast<const uint8_t*>(T4), n / 2, reinterpret_cast<const uint8_t*>(W4), n / 2,
                 static_cast<int>(bit_cols), static_cast<int>(m), static_cast<int>(cols), static_cast<int>(n), out,
                 ldo, scale, nullptr, 0, 0.0f, 0};
    return launch_f4_gemm(a, float_out, s);
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

int tbn_hip_pack_f4_weights(const uint8_t* packed, int64_t K_pad, int64_t N_pad, uint8_t* w4, tbn_stream_t stream) {
    TBN_REQUIRE(K_pad >= 0 && N_pad >= 0 && K_pad % 64 == 0 && K_pad < (1LL << 24) && N_pad < (1LL << 31),
                TBN_INVALID_SHAPE, "K_pad must be a multiple of 64 below 2^24");
    if (K_pad == 0 || N_pad == 0) return tbn_hip::ok();
    TBN_REQUIRE(packed && w4, TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 4 == 0 && reinterpret_cast<uintptr_t>(w4) % 16 == 0,
                TBN_INVALID_ARGUMENT, "packed must be 4-byte and w4 16-byte aligned");
    TBN_DEVICE_GUARD();
    return launch_f4_operands(RowsF32{nullptr, 0, 0, 0.0f, 0.0f, false}, 0, K_pad, nullptr, packed, K_pad / 8, N_pad,
                              reinterpret_cast<uint32_t*>(w4), tbn_hip::stream_of(stream), "pack_f4_weights");
}

int tbn_hip_gemm_tbn_prepacked(const float* A, int64_t lda, int64_t M, int64_t K, const uint8_t* w4, int64_t K_pad,
                               int64_t N, int64_t N_pad, float alpha, const float* cin, int cin_1d, float beta,
                               float lo, float hi, int flags, uint8_t* t4, float* out, int64_t ldo,
                               tbn_stream_t stream) {
    TBN_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M < (1LL << 31) && N < (1LL << 31) && K_pad < (1LL << 24),
                TBN_INVALID_SHAPE, "M, N, K out of range");
    TBN_REQUIRE(K_pad >= K && K_pad % 64 == 0, TBN_INVALID_SHAPE, "K_pad must be >= K and a multiple of 64");
    TBN_REQUIRE(N_pad >= N, TBN_INVALID_SHAPE, "N_pad must be >= N");
    TBN_REQUIRE(M == 0 || lda >= K, TBN_INVALID_ARGUMENT, "lda must be >= K");
    TBN_REQUIRE(ldo >= N, TBN_INVALID_ARGUMENT, "ldo must be >= N");
    TBN_REQUIRE((flags & ~TBN_EPI_RELU) == 0, TBN_INVALID_ARGUMENT, "unsupported epilogue flags for a TBN Gemm");
    if (M == 0 || N == 0) return tbn_hip::ok();
    TBN_REQUIRE(out && t4 && (K == 0 || A) && (K_pad == 0 || w4), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_REQUIRE(reinterpret_cast<uintptr_t>(t4) % 16 == 0 && reinterpret_cast<uintptr_t>(w4) % 16 == 0,
                TBN_INVALID_ARGUMENT, "t4 and w4 must be 16-byte aligned");
    TBN_DEVICE_GUARD();
    hipStream_t s = tbn_hip::stream_of(stream);
    const bool add = cin && beta != 0.0f;
    if (K_pad == 0) {
        TBN_REQUIRE(!add && !flags, TBN_NOT_IMPLEMENTED, "TBN Gemm with an empty shared dimension and an epilogue");
        if (hipMemset2DAsync(out, ldo * sizeof(float), 0, N * sizeof(float), M, s) != hipSuccess)
            return tbn_hip::fail(TBN_RUNTIME_ERROR, "hipMemset2DAsync failed");
        return tbn_hip::ok();
    }
    const bool vec = K % 4 == 0 && lda % 4 == 0 && reinterpret_cast<uintptr_t>(A) % 16 == 0;
    int rc = launch_f4_operands(RowsF32{A, lda, static_cast<int>(K), lo, hi, vec}, M, K_pad,
                                reinterpret_cast<uint32_t*>(t4), nullptr, 0, 0, nullptr, s,
                                "gemm_tbn_prepacked (fp4 activations)");
    if (rc != TBN_SUCCESS) return rc;
    F4GemmArgs a{t4, K_pad / 2, w4, K_pad / 2, static_cast<int>(N_pad), static_cast<int>(M), static_cast<int>(N),
                 static_cast<int>(K_pad), out, ldo, alpha, add ? cin : nullptr, cin_1d, beta,
                 (flags & TBN_EPI_RELU) ? 1 : 0};
    return launch_f4_gemm(a, true, s);
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
    const size_t tbytes = (static_cast<size_t>(M) * (K_pad / 2) + 255) / 256 * 256;
    const size_t wbytes = static_cast<size_t>(N_pad) * (K_pad / 2);
    if (int rc = scr.get(tbytes + wbytes)) return rc;
    uint32_t* T4 = static_cast<uint32_t*>(scr.ptr);
    uint32_t* W4 = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(scr.ptr) + tbytes);
    const bool vec = K % 4 == 0 && lda % 4 == 0 && reinterpret_cast<uintptr_t>(A) % 16 == 0;
    int rc = launch_f4_operands(RowsF32{A, lda, static_cast<int>(K), lo, hi, vec}, M, K_pad, T4, packed, K_pad / 8,
                                N_pad, W4, s, "qlinear_matmul_binary_tbn (fp4 operands)");
    if (rc != TBN_SUCCESS) return rc;
    F4GemmArgs a{reinterpret_cast<const uint8_t*>(T4), K_pad / 2, reinterpret_cast<const uint8_t*>(W4), K_pad / 2,
                 static_cast<int>(N_pad), static_cast<int>(M), static_cast<int>(N), static_cast<int>(K_pad), out,
                 ldo, scale, nullptr, 0, 0.0f, 0};
    return launch_f4_gemm(a, true, s);
}

}  // extern "C"
