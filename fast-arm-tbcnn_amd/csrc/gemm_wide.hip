// Wide-tile float x binary GEMM: C = epilogue(A * W), A fp32 [M, K] row-major,
// W the reference's BinaryMatrix (column n = K_pad bits, bit 1 = -1).
//
// The large tile: a block owns BR = 128 rows of A x BC = 512 columns of W;
// its 8 waves each own all 128 rows x 64 columns (4 x 2 MFMA fragments of
// 32 x 32), so every packed weight column belongs to exactly one wave and is
// decoded once per block, in registers, straight from global memory.  The A
// tile of a K step (128 x 64 fp32) is split by the block into three bf16
// planes in LDS (hi + mid + lo = a exactly) and shared by all 8 waves; LDS
// holds two steps so one barrier per step suffices.  Per step and wave: 96
// v_mfma_f32_32x32x16_bf16 against ~330 VALU (split 16 elements, decode 8
// weight bytes per column fragment and k slice).  The mid-size tiles (64 x
// 128, and 32 x 128 in two K groups) have the same structure with fewer
// fragments per wave and load two steps ahead.
//
// Memory: A and W are read with buffer loads whose resource covers the
// block's rows / columns to the end of the matrix: rows >= M and columns >=
// N_pad read as zero, and the voffsets are fixed per lane (the K position
// moves the resource base, scalar work), so the steady-state loop issues no
// vector address arithmetic.
// A K step past K (K % 64 != 0) is zeroed before the split.
//
// Blocks are dealt round-robin over the 8 XCDs; the tile order puts the
// BC-column tiles of one BR-row band of A on the same XCD, so the band is
// fetched from HBM once into that XCD's L2 and read there by its tiles.  The
// mid-size tiles give each XCD the rectangle of tiles with the fewest A and W
// bytes to fetch (whole row bands, or e.g. 2 bands x half the columns).
#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "gemm_wide.hpp"
#include "mfma_core.hpp"

namespace {

using namespace tbnk;

template <int BR_, int BC_, int WR_, int WC_, int KS_, bool DEEP_ = false, int KG_ = 1>
struct WideCfg {
    static constexpr int BR = BR_, BC = BC_, WR = WR_, WC = WC_;
    static constexpr int KS = KS_;                 // K per step (one LDS buffer, one barrier)
    // DEEP: global loads issued two steps before their data is needed (A in
    // two register slots, W words a pair of steps at a time, three pairs
    // live), for tiles with few MFMAs per step; else one step before.
    static constexpr bool DEEP = DEEP_;
    // KG: groups of waves that each run one contiguous part of the K steps on
    // the whole tile (own LDS buffers, same barriers), their sums added in
    // group order through LDS at the end.
    static constexpr int KG = KG_;
    static constexpr int KROW = KS + 8;            // bf16 per LDS row: conflict-free 16-byte fragment reads
    static constexpr int WAVES_R = BR / WR, WAVES_C = BC / WC;
    static constexpr int NTG = 64 * WAVES_R * WAVES_C;  // threads per K group
    static constexpr int NT = NTG * KG;
    static constexpr int FR = WR / 32, FC = WC / 32;
    static constexpr int KK = KS / 16;             // MFMA k-slices per step
    static constexpr int EPT = BR * KS / NTG;      // A elements a thread stages per step
    static constexpr int TPR = KS / EPT;           // threads per A row
    static_assert(EPT % 8 == 0 && KS % EPT == 0, "a thread stages whole 8-element groups of one row");
    static_assert(WR % 32 == 0 && WC % 32 == 0 && BR % WR == 0 && BC % WC == 0, "bad tile");
    static_assert(KK % 2 == 0 && KS == 64, "two k-slice fragment buffers; 8 / 16 weight bytes per step");
    static_assert(KG == 1 || KG == 2, "one or two K groups");
    static_assert(KG == 1 || 2 * 3 * BR * KROW * 2 >= NTG * FR * FC * 16 * 4, "group sums fit the A buffers");
};

// Tile menu: 128 x 512 blocks of 8 waves for shapes whose tiles fill the chip;
// 64 x 128 blocks (4 waves of 32 x 64, two blocks per CU) for mid-size shapes,
// which split K across blocks to reach two waves per SIMD; 32 x 128 blocks of
// two K groups of 4 waves (32 x 32 each) that reach two waves per SIMD
// without a split across blocks.
using Wide = WideCfg<128, 512, 128, 64, 64>;
using WideSmall = WideCfg<64, 128, 32, 64, 64, true>;
using WideMid = WideCfg<32, 128, 32, 32, 64, true, 2>;

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x2_t __attribute__((ext_vector_type(2)));

// 8 BinaryMatrix bits (bit e = weight k0 + e, 1 means -1) -> 8 bf16 +-1.0.
// Bits 16 and up of x must be zero; bits 8..15 are ignored.  y holds bit e at
// e and at e + 15, so one shift puts bit 2d at 15 and bit 2d+1 at 31, and one
// v_and_or_b32 (mask in an SGPR, +1.0 pair in `ones`, a VGPR) finishes a dword.
__device__ __forceinline__ u32x4_t decode_binary8_y(uint32_t x, uint32_t ones) {
    const uint32_t y = x | (x << 15);
    u32x4_t r;
    r[0] = ((y << 15) & 0x80008000u) | ones;
    r[1] = ((y << 13) & 0x80008000u) | ones;
    r[2] = ((y << 11) & 0x80008000u) | ones;
    r[3] = ((y << 9) & 0x80008000u) | ones;
    return r;
}

template <bool B>
using bool_c = std::integral_constant<bool, B>;
template <int I>
using int_c = std::integral_constant<int, I>;

// One block: a BR x BC tile of C over the K steps [s0, s0 + ns).  SPLIT
// blocks (split-K) write their raw sums to `partial`; the last block of a
// tile to finish (counted in counters[tile], which it leaves zero) adds the
// splits' sums in split order and runs the epilogue, so the result is the
// same on every run whichever block finishes last.
template <class Cfg, bool TERNARY, bool SPLIT>
__global__ void __launch_bounds__(Cfg::NT)
gemm_wide_kernel(tbn_hip::WideGemmArgs p, int tiles_r, int tiles_c, int steps_per_split, float* partial,
                 int* counters) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 3 * Cfg::BR * Cfg::KROW];
    constexpr int kPlane = Cfg::BR * Cfg::KROW;  // bf16 per plane
    constexpr int KS = Cfg::KS;
    constexpr int WPS = TERNARY ? 4 : 2;        // 32-bit weight words per column per step

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave / Cfg::WAVES_C;
    const int wc = wave % Cfg::WAVES_C;
    const int h = lane >> 5;
    // +1.0 bf16 pair kept in a VGPR so each decoded dword is one v_and_or_b32
    uint32_t ones;
    asm volatile("v_mov_b32 %0, 0x3f803f80" : "=v"(ones));

    // tile order: the tiles of one XCD (blockIdx % 8) are consecutive in t,
    // and consecutive t share a row band of A; split-K blocks are split-major
    const int total = tiles_r * tiles_c;
    const int split = SPLIT ? static_cast<int>(blockIdx.x) / total : 0;
    int t = static_cast<int>(blockIdx.x) - split * total;
    if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
    const int tr = t / tiles_c;
    const int tc = t - tr * tiles_c;
    const int r0 = tr * Cfg::BR;
    const int c0 = tc * Cfg::BC;
    const int all_steps = (p.K + KS - 1) / KS;
    const int s0 = SPLIT ? split * steps_per_split : 0;
    const int ns = SPLIT ? min(steps_per_split, all_steps - s0) : all_steps;

    // A staging: thread -> row ar, EPT consecutive k from ag * EPT
    const int ar = tid / Cfg::TPR, ag = tid % Cfg::TPR;
    const float* a_base = p.A + static_cast<int64_t>(r0) * p.lda;
    const uint64_t a_bytes = static_cast<uint64_t>(p.M - r0) * p.lda * 4;
    const int a_voff = (ar * static_cast<int>(p.lda) + ag * Cfg::EPT) * 4;
    // W: lane's columns c0 + wc*WC + j*32 + lane%32
    const uint8_t* b_base = p.packed + static_cast<int64_t>(c0) * p.col_bytes;
    const uint64_t b_bytes = static_cast<uint64_t>(p.N_pad - c0) * static_cast<uint64_t>(p.col_bytes);
    int b_voff[Cfg::FC];
#pragma unroll
    for (int j = 0; j < Cfg::FC; ++j)
        b_voff[j] = (wc * Cfg::WC + j * 32 + (lane & 31)) * static_cast<int>(p.col_bytes);

    float areg[Cfg::EPT];                              // A of the next step, in flight
    uint32_t bw[Cfg::FC][WPS], bwn[Cfg::FC][WPS];      // W words of the current / next step
    u32x4_t bfr[2][Cfg::FC];                           // decoded W fragments, alternating k-slices

    // loads past the end of A / W return zeros or data of later rows / columns
    // that no result uses, so they need no guard; s is an absolute step, its
    // byte offset folded into the resource base (scalar work) so that every
    // byte past the end of A or W is range-checked
    auto load_a = [&](int s) {
        const __amdgpu_buffer_rsrc_t a_rs = buffer_range(a_base, a_bytes, static_cast<uint64_t>(s) * KS * 4);
#pragma unroll
        for (int v = 0; v < Cfg::EPT / 4; ++v) {
            const f32x4_t x =
                __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(a_rs, a_voff + 16 * v, 0, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) areg[4 * v + e] = x[e];
        }
    };
    auto load_b = [&](int s, uint32_t (&w)[Cfg::FC][WPS]) {
        const __amdgpu_buffer_rsrc_t b_rs = buffer_range(b_base, b_bytes, static_cast<uint64_t>(s) * 4 * WPS);
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            if constexpr (TERNARY) {
                const u32x4_t x = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rs, b_voff[j], 0, 0));
#pragma unroll
                for (int d = 0; d < WPS; ++d) w[j][d] = x[d];
            } else {
                const uint64_t x = __builtin_bit_cast(
                    uint64_t, __builtin_amdgcn_raw_buffer_load_b64(b_rs, b_voff[j], 0, 0));
                w[j][0] = static_cast<uint32_t>(x);
                w[j][1] = static_cast<uint32_t>(x >> 32);
            }
        }
    };
    // k-slice kk (16 k) of a step's words: binary 8 bits, ternary 16 bits per lane half
    auto decode_b = [&](const uint32_t (&w)[Cfg::FC][WPS], int kk, u32x4_t (&bf)[Cfg::FC]) {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            if constexpr (TERNARY)
                bf[j] = decode_ternary8_x2(__builtin_amdgcn_ubfe(w[j][kk], 16 * h, 16));
            else
                bf[j] = decode_binary8_y(__builtin_amdgcn_ubfe(w[j][kk / 2], 16 * (kk & 1) + 8 * h, 16), ones);
        }
    };
    // split the staged step into the three planes of LDS buffer b; with
    // MASK, values at k >= K (last step) are zeroed first
    const int a_store = ar * Cfg::KROW + ag * Cfg::EPT;
    auto store_a = [&](int b, int s, auto mask) {
        if constexpr (decltype(mask)::value) {
            const int kbase = s * KS + ag * Cfg::EPT;
#pragma unroll
            for (int e = 0; e < Cfg::EPT; ++e)
                if (kbase + e >= p.K) areg[e] = 0.0f;
        }
#pragma unroll
        for (int v = 0; v < Cfg::EPT / 8; ++v) {
            uint4 hi, mid, lo;
            split8(areg + 8 * v, hi, mid, lo);
            uint16_t* d = lds + b * 3 * kPlane + a_store + 8 * v;
            *reinterpret_cast<uint4*>(d) = hi;
            *reinterpret_cast<uint4*>(d + kPlane) = mid;
            *reinterpret_cast<uint4*>(d + 2 * kPlane) = lo;
        }
    };

    f32x16_t acc[Cfg::FR][Cfg::FC];
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // fragment read base: row wr*WR + lane%32, k offset 8*(lane/32)
    const int a_frag = (wr * Cfg::WR + (lane & 31)) * Cfg::KROW + h * 8;

    // Local step l = 2q + u on LDS buffer u: per k-slice kk, 3 planes x FR x FC
    // MFMAs with the W fragments decoded one slice ahead; meanwhile split step
    // l+1's A (in registers) into the other buffer and fetch step l+2's A and
    // W words.  FULL steps (l + 2 < ns) need no guards.
    auto step = [&](int q, auto uc, auto full) {
        constexpr int u = decltype(uc)::value;
        constexpr bool FULL = decltype(full)::value;
        const int l = 2 * q + u;
        const int s = s0 + l;
#pragma unroll
        for (int kk = 0; kk < Cfg::KK; ++kk) {
            // next slice's W fragments (the next step's first slice after the last)
            if (kk + 1 < Cfg::KK) decode_b(bw, kk + 1, bfr[(kk + 1) & 1]);
            else decode_b(bwn, 0, bfr[0]);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                u32x4_t af[Cfg::FR];
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
                    af[i] = *reinterpret_cast<const u32x4_t*>(lds + (u * 3 + pl) * kPlane + i * 32 * Cfg::KROW +
                                                             a_frag + kk * 16);
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j) acc[i][j] = mfma32(af[i], bfr[kk & 1][j], acc[i][j]);
            }
        }
        if constexpr (FULL) {
            store_a(u ^ 1, s + 1, bool_c<false>{});
            load_a(s + 2);
        } else {
            if (l + 1 < ns) store_a(u ^ 1, s + 1, bool_c<true>{});
            if (l + 2 < ns) load_a(s + 2);
        }
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int d = 0; d < WPS; ++d) bw[j][d] = bwn[j][d];
        load_b(s + 2, bwn);
        if constexpr (FULL) {
            // 4 fragment reads ahead, then per fragment: 2 MFMAs, the next read, VALU
            constexpr int kReads = Cfg::KK * 3 * Cfg::FR;
            constexpr int kPairs = Cfg::KK * 3 * Cfg::FR * Cfg::FC / 2;
            constexpr int kValu = 5;
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int r = 0; r < kReads - 4; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
            }
#pragma unroll
            for (int r = kReads - 4; r < kPairs; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
            }
        }
        __syncthreads();
        // no instruction crosses a step boundary: the scheduler would otherwise
        // hoist the next step's split of A above this step's barrier, next to
        // the loads of its data, and wait there for them (vmcnt(0) each step)
        __builtin_amdgcn_sched_barrier(0);
    };

    // prologue: step s0 split into buffer 0, step s0+1 in flight, W words of
    // steps s0 and s0+1, W fragments of step s0's first slice decoded
    load_a(s0);
    load_b(s0, bw);
    load_b(s0 + 1, bwn);
    store_a(0, s0, bool_c<true>{});
    load_a(s0 + 1);
    decode_b(bw, 0, bfr[0]);
    __syncthreads();

    const int pairs = (ns + 1) / 2;
    int q = 0;
    for (; 2 * q + 3 < ns; ++q) {
        step(q, int_c<0>{}, bool_c<true>{});
        step(q, int_c<1>{}, bool_c<true>{});
    }
    for (; q < pairs; ++q) {
        step(q, int_c<0>{}, bool_c<false>{});
        if (2 * q + 1 < ns) step(q, int_c<1>{}, bool_c<false>{});
    }

    if constexpr (SPLIT) {
        // Raw sums of this split go to partial[split][m][n]; the last block of
        // the tile to count itself in adds all splits in split order.  The
        // sums are written and read with the device-scope policy (sc1), and
        // splitk_arrive orders every wave's stores before the count and the
        // count before the last block's loads.  Buffer accesses over one
        // split's M x N sums (host-checked below 2^31 bytes): the row step of
        // register e is folded into the resource base, so rows past M are
        // dropped / read zero by the range check; lanes of columns past N
        // carry an offset beyond every range.
        constexpr int kDeviceScope = 16;  // cache policy SC1
        const int64_t MN = static_cast<int64_t>(p.M) * p.N;
        const int nsplit = static_cast<int>(gridDim.x) / total;
        int voff[Cfg::FR][Cfg::FC];
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j) {
                const int n = c0 + wc * Cfg::WC + j * 32 + (lane & 31);
                voff[i][j] = n < p.N ? ((r0 + wr * Cfg::WR + i * 32 + 4 * h) * p.N + n) * 4 : 0x7FFFFFF0;
            }
        const uint64_t split_bytes = static_cast<uint64_t>(MN) * 4;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const __amdgpu_buffer_rsrc_t rs = buffer_range(
                partial + split * MN, split_bytes, static_cast<uint64_t>(8 * (e >> 2) + (e & 3)) * p.N * 4);
#pragma unroll
            for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
                    // __float_as_uint, not __builtin_bit_cast: hipcc (ROCm 7.2) folds a bit
                    // cast of a vector element with a loop index to element 0
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][e]), rs, voff[i][j], 0,
                                                          kDeviceScope);
        }
        __shared__ int is_last;
        if (!splitk_arrive(counters + t, nsplit, &is_last)) return;
        // 0 + split 0 + split 1 + ... per output, in split order
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        for (int sp = 0; sp < nsplit; ++sp) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const __amdgpu_buffer_rsrc_t rs = buffer_range(
                    partial + sp * MN, split_bytes, static_cast<uint64_t>(8 * (e >> 2) + (e & 3)) * p.N * 4);
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j)
                        acc[i][j][e] += __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff[i][j], 0, kDeviceScope));
            }
        }
        // ready for the next launch on this workspace
        if (tid == 0) __hip_atomic_store(counters + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- epilogue: C[m, n] = relu?(acc * alpha * scale[n] + bias[n] (+ beta * cin)) ----
    float mult[Cfg::FC], badd[Cfg::FC];
    int ncol[Cfg::FC];
#pragma unroll
    for (int j = 0; j < Cfg::FC; ++j) {
        ncol[j] = c0 + wc * Cfg::WC + j * 32 + (lane & 31);
        const int nc = min(ncol[j], p.N - 1);
        mult[j] = p.alpha;
        badd[j] = 0.0f;
        if (p.scale) mult[j] = p.alpha * p.scale[nc];
        if (p.bias) badd[j] = p.bias[nc];
    }
    const bool bias_then_scale = (p.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
    const bool relu = (p.flags & TBN_EPI_RELU) != 0;
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i) {
        const int mrow = r0 + wr * Cfg::WR + i * 32 + 4 * h;
        float v[Cfg::FC][16];
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float a = TERNARY ? acc[i][j][e] * 0.5f : acc[i][j][e];  // ternary sums are doubled
                v[j][e] = bias_then_scale ? (a + badd[j]) * mult[j] : a * mult[j] + badd[j];
            }
        if (p.cin) {
            float cv[Cfg::FC][16];
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = min(mrow + 8 * (e >> 2) + (e & 3), p.M - 1);
                    const int nc = min(ncol[j], p.N - 1);
                    cv[j][e] = p.cin_1d ? p.cin[nc] : p.cin[static_cast<int64_t>(m) * p.N + nc];
                }
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) v[j][e] += p.beta * cv[j][e];
        }
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = mrow + 8 * (e >> 2) + (e & 3);
                float x = v[j][e];
                if (relu) x = x > 0.0f ? x : 0.0f;
                // non-temporal: C is not read again here (0.7 % at 4096^3, 1-2 % at the mid-size shapes)
                if (m < p.M && ncol[j] < p.N)
                    __builtin_nontemporal_store(x, &p.C[static_cast<int64_t>(m) * p.ldc + ncol[j]]);
            }
    }
}

// The mid-size kernel: the same block structure (and the same split-K
// finish) for the DEEP configurations, with two-step-ahead loads and K
// groups.  The large tile keeps its own kernel above, whose register
// allocation the extra machinery disturbs (measured 3 % slower at 4096^3 when
// both shared one kernel).
template <class Cfg, bool TERNARY, bool SPLIT>
__global__ void __launch_bounds__(Cfg::NT)
gemm_mid_kernel(tbn_hip::WideGemmArgs p, int tiles_r, int tiles_c, int steps_per_split, float* partial,
                int* counters, int xcd_cols) {
    __shared__ __attribute__((aligned(16))) uint16_t lds_all[Cfg::KG * 2 * 3 * Cfg::BR * Cfg::KROW];
    constexpr int kPlane = Cfg::BR * Cfg::KROW;  // bf16 per plane
    constexpr int KS = Cfg::KS;
    constexpr int WPS = TERNARY ? 4 : 2;        // 32-bit weight words per column per step

    const int lane = threadIdx.x & 63;
    const int kgrp = Cfg::KG == 1 ? 0 : static_cast<int>(threadIdx.x) / Cfg::NTG;
    const int tid = static_cast<int>(threadIdx.x) - kgrp * Cfg::NTG;  // thread within its K group
    const int wave = tid >> 6;
    const int wr = wave / Cfg::WAVES_C;
    const int wc = wave % Cfg::WAVES_C;
    uint16_t* const lds = lds_all + kgrp * (2 * 3 * kPlane);
    const int h = lane >> 5;
    // +1.0 bf16 pair kept in a VGPR so each decoded dword is one v_and_or_b32
    uint32_t ones;
    asm volatile("v_mov_b32 %0, 0x3f803f80" : "=v"(ones));

    // tile order (split-K blocks are split-major): XCD x = blockIdx % 8 owns a
    // rectangle of tiles -- with xcd_cols = R, the XCDs form an (8 / R) x R
    // grid over the tile grid (host-checked to divide it) -- so a row band of
    // A and a column tile of W are fetched into few XCDs' L2; with R = 1 an
    // XCD's tiles are whole row bands
    const int total = tiles_r * tiles_c;
    const int split = SPLIT ? static_cast<int>(blockIdx.x) / total : 0;
    int t = static_cast<int>(blockIdx.x) - split * total;
    int tr, tc;
    if (xcd_cols > 1) {
        const int x = t % 8, j = t / 8;
        const int rb = tiles_r * xcd_cols / 8, cb = tiles_c / xcd_cols;  // rectangle: rb row bands x cb tiles
        tr = (x / xcd_cols) * rb + j / cb;
        tc = (x % xcd_cols) * cb + j % cb;
        t = tr * tiles_c + tc;
    } else {
        if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
        tr = t / tiles_c;
        tc = t - tr * tiles_c;
    }
    const int r0 = tr * Cfg::BR;
    const int c0 = tc * Cfg::BC;
    const int all_steps = (p.K + KS - 1) / KS;
    // a K group's steps: the host gives each group the same count
    const int per_group = (SPLIT ? steps_per_split : all_steps) / Cfg::KG;
    const int s0 = (SPLIT ? split * steps_per_split : 0) + kgrp * per_group;
    const int ns = SPLIT ? min(per_group, all_steps - s0) : per_group;

    // epilogue operands: the mid-size tiles (DEEP), whose run is short, fetch
    // them now so their latency overlaps the main loop; the large tile, short
    // of registers, after it
    auto fetch_epilogue = [&](float (&mult)[Cfg::FC], float (&badd)[Cfg::FC], int (&ncol)[Cfg::FC]) {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            ncol[j] = c0 + wc * Cfg::WC + j * 32 + (lane & 31);
            const int nc = min(ncol[j], p.N - 1);
            mult[j] = p.alpha;
            badd[j] = 0.0f;
            if (p.scale) mult[j] = p.alpha * p.scale[nc];
            if (p.bias) badd[j] = p.bias[nc];
        }
    };
    float mult_e[Cfg::DEEP ? Cfg::FC : 1], badd_e[Cfg::DEEP ? Cfg::FC : 1];
    int ncol_e[Cfg::DEEP ? Cfg::FC : 1];
    if constexpr (Cfg::DEEP) fetch_epilogue(mult_e, badd_e, ncol_e);

    // A staging: thread -> row ar, EPT consecutive k from ag * EPT
    const int ar = tid / Cfg::TPR, ag = tid % Cfg::TPR;
    const float* a_base = p.A + static_cast<int64_t>(r0) * p.lda;
    const uint64_t a_bytes = static_cast<uint64_t>(p.M - r0) * p.lda * 4;
    const int a_voff = (ar * static_cast<int>(p.lda) + ag * Cfg::EPT) * 4;
    // W: lane's columns c0 + wc*WC + j*32 + lane%32
    const uint8_t* b_base = p.packed + static_cast<int64_t>(c0) * p.col_bytes;
    const uint64_t b_bytes = static_cast<uint64_t>(p.N_pad - c0) * static_cast<uint64_t>(p.col_bytes);
    int b_voff[Cfg::FC];
#pragma unroll
    for (int j = 0; j < Cfg::FC; ++j)
        b_voff[j] = (wc * Cfg::WC + j * 32 + (lane & 31)) * static_cast<int>(p.col_bytes);

    constexpr int ASLOTS = Cfg::DEEP ? 2 : 1;
    constexpr int PW = 2 * WPS;                        // W words per column per pair of steps
    float areg[ASLOTS][Cfg::EPT];                      // A of the next step(s), in flight
    uint32_t bw[Cfg::FC][WPS], bwn[Cfg::FC][WPS];      // W words of the current / next step
    uint32_t wp[3][Cfg::DEEP ? Cfg::FC : 1][Cfg::DEEP ? PW : 1];  // DEEP: W words of pairs q, q + 1, q + 2
    u32x4_t bfr[2][Cfg::FC];                           // decoded W fragments, alternating k-slices
    if constexpr (Cfg::DEEP) {
#pragma unroll
        for (int x = 0; x < 3; ++x)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int d = 0; d < PW; ++d) wp[x][j][d] = 0;
    }

    // loads past the end of A / W return zeros or data of later rows / columns
    // that no result uses, so they need no guard; s is an absolute step, its
    // byte offset folded into the resource base (scalar work) so that every
    // byte past the end of A or W is range-checked
    auto load_a = [&](int s, auto slot) {
        constexpr int sl = decltype(slot)::value;
        const __amdgpu_buffer_rsrc_t a_rs = buffer_range(a_base, a_bytes, static_cast<uint64_t>(s) * KS * 4);
#pragma unroll
        for (int v = 0; v < Cfg::EPT / 4; ++v) {
            const f32x4_t x =
                __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(a_rs, a_voff + 16 * v, 0, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) areg[sl][4 * v + e] = x[e];
        }
    };
    // DEEP: the W words of steps 2q', 2q' + 1 (one pair) into wp[x]
    auto load_pair = [&](int s, int x) {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int c = 0; c < PW / 4; ++c) {
                const __amdgpu_buffer_rsrc_t b_rs =
                    buffer_range(b_base, b_bytes, static_cast<uint64_t>(s) * 4 * WPS + 16 * c);
                const u32x4_t v = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rs, b_voff[j], 0, 0));
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    if (x == 0) wp[0][j][4 * c + d] = v[d];
                    else if (x == 1) wp[1][j][4 * c + d] = v[d];
                    else wp[2][j][4 * c + d] = v[d];
                }
            }
    };
    auto load_b = [&](int s, uint32_t (&w)[Cfg::FC][WPS]) {
        const __amdgpu_buffer_rsrc_t b_rs = buffer_range(b_base, b_bytes, static_cast<uint64_t>(s) * 4 * WPS);
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            if constexpr (TERNARY) {
                const u32x4_t x = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rs, b_voff[j], 0, 0));
#pragma unroll
                for (int d = 0; d < WPS; ++d) w[j][d] = x[d];
            } else {
                const uint64_t x = __builtin_bit_cast(
                    uint64_t, __builtin_amdgcn_raw_buffer_load_b64(b_rs, b_voff[j], 0, 0));
                w[j][0] = static_cast<uint32_t>(x);
                w[j][1] = static_cast<uint32_t>(x >> 32);
            }
        }
    };
    // k-slice kk (16 k) of a step's words: binary 8 bits, ternary 16 bits per lane half
    // (`w` may be a pair's words: `base` selects the step's first word)
    auto decode_b = [&](const auto& w, int kk, u32x4_t (&bf)[Cfg::FC], int base = 0) {
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j) {
            if constexpr (TERNARY)
                bf[j] = decode_ternary8_x2(__builtin_amdgcn_ubfe(w[j][base + kk], 16 * h, 16));
            else
                bf[j] = decode_binary8_y(__builtin_amdgcn_ubfe(w[j][base + kk / 2], 16 * (kk & 1) + 8 * h, 16),
                                         ones);
        }
    };
    // split the staged step into the three planes of LDS buffer b; with
    // MASK, values at k >= K (last step) are zeroed first
    const int a_store = ar * Cfg::KROW + ag * Cfg::EPT;
    auto store_a = [&](int b, int s, auto mask, auto slot) {
        constexpr int sl = decltype(slot)::value;
        if constexpr (decltype(mask)::value) {
            const int kbase = s * KS + ag * Cfg::EPT;
#pragma unroll
            for (int e = 0; e < Cfg::EPT; ++e)
                if (kbase + e >= p.K) areg[sl][e] = 0.0f;
        }
#pragma unroll
        for (int v = 0; v < Cfg::EPT / 8; ++v) {
            uint4 hi, mid, lo;
            split8(areg[sl] + 8 * v, hi, mid, lo);
            uint16_t* d = lds + b * 3 * kPlane + a_store + 8 * v;
            *reinterpret_cast<uint4*>(d) = hi;
            *reinterpret_cast<uint4*>(d + kPlane) = mid;
            *reinterpret_cast<uint4*>(d + 2 * kPlane) = lo;
        }
    };

    f32x16_t acc[Cfg::FR][Cfg::FC];
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // fragment read base: row wr*WR + lane%32, k offset 8*(lane/32)
    const int a_frag = (wr * Cfg::WR + (lane & 31)) * Cfg::KROW + h * 8;

    // Local step l = 2q + u on LDS buffer u: per k-slice kk, 3 planes x FR x FC
    // MFMAs with the W fragments decoded one slice ahead; meanwhile split step
    // l+1's A (in registers) into the other buffer and fetch step l+2's A and
    // W words.  FULL steps (l + 2 < ns) need no guards.
    //
    // DEEP: A of steps l + 1 and l + 2 sit in register slots (l + 1) & 1 and
    // l & 1; after step l's MFMAs, step l + 1 is split from its slot, which
    // then receives step l + 3.  The W words of pair q live in wp[0], of q + 1
    // in wp[1]; pair q + 2's are fetched into wp[2] as pair q starts and
    // rotated in as it ends.
    auto step = [&](int q, auto uc, auto full) {
        constexpr int u = decltype(uc)::value;
        constexpr bool FULL = decltype(full)::value;
        const int l = 2 * q + u;
        const int s = s0 + l;
        if constexpr (Cfg::DEEP && u == 0) {
            if (FULL || 2 * q + 4 < ns) load_pair(s + 4, 2);
        }
#pragma unroll
        for (int kk = 0; kk < Cfg::KK; ++kk) {
            // next slice's W fragments (the next step's first slice after the last)
            if constexpr (Cfg::DEEP) {
                if (kk + 1 < Cfg::KK) decode_b(wp[0], kk + 1, bfr[(kk + 1) & 1], u * WPS);
                else if (u == 0) decode_b(wp[0], 0, bfr[0], WPS);
                else decode_b(wp[1], 0, bfr[0], 0);
            } else {
                if (kk + 1 < Cfg::KK) decode_b(bw, kk + 1, bfr[(kk + 1) & 1]);
                else decode_b(bwn, 0, bfr[0]);
            }
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                u32x4_t af[Cfg::FR];
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
                    af[i] = *reinterpret_cast<const u32x4_t*>(lds + (u * 3 + pl) * kPlane + i * 32 * Cfg::KROW +
                                                             a_frag + kk * 16);
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j) acc[i][j] = mfma32(af[i], bfr[kk & 1][j], acc[i][j]);
            }
        }
        if constexpr (Cfg::DEEP) {
            if constexpr (FULL) {
                store_a(u ^ 1, s + 1, bool_c<false>{}, int_c<u ^ 1>{});
                load_a(s + 3, int_c<u ^ 1>{});
            } else {
                if (l + 1 < ns) store_a(u ^ 1, s + 1, bool_c<true>{}, int_c<u ^ 1>{});
                if (l + 3 < ns) load_a(s + 3, int_c<u ^ 1>{});
            }
            if constexpr (u == 1) {
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int d = 0; d < PW; ++d) {
                        wp[0][j][d] = wp[1][j][d];
                        wp[1][j][d] = wp[2][j][d];
                    }
            }
        } else {
            if constexpr (FULL) {
                store_a(u ^ 1, s + 1, bool_c<false>{}, int_c<0>{});
                load_a(s + 2, int_c<0>{});
            } else {
                if (l + 1 < ns) store_a(u ^ 1, s + 1, bool_c<true>{}, int_c<0>{});
                if (l + 2 < ns) load_a(s + 2, int_c<0>{});
            }
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int d = 0; d < WPS; ++d) bw[j][d] = bwn[j][d];
            load_b(s + 2, bwn);
        }
        if constexpr (FULL) {
            // 4 fragment reads ahead, then per fragment: 2 MFMAs, the next read, VALU
            constexpr int kReads = Cfg::KK * 3 * Cfg::FR;
            constexpr int kPairs = Cfg::KK * 3 * Cfg::FR * Cfg::FC / 2;
            constexpr int kValu = 5;
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int r = 0; r < kReads - 4; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
            }
#pragma unroll
            for (int r = kReads - 4; r < kPairs; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
            }
        }
        __syncthreads();
    };

    // prologue: step s0 split into buffer 0, step s0+1 (DEEP: and s0+2) in
    // flight, W words of steps s0 and s0+1 (DEEP: of pairs 0 and 1), W
    // fragments of step s0's first slice decoded
    if constexpr (Cfg::DEEP) {
        load_a(s0, int_c<0>{});
        load_pair(s0, 0);
        load_a(s0 + 1, int_c<1>{});
        load_pair(s0 + 2, 1);
        store_a(0, s0, bool_c<true>{}, int_c<0>{});
        load_a(s0 + 2, int_c<0>{});
        decode_b(wp[0], 0, bfr[0], 0);
    } else {
        load_a(s0, int_c<0>{});
        load_b(s0, bw);
        load_b(s0 + 1, bwn);
        store_a(0, s0, bool_c<true>{}, int_c<0>{});
        load_a(s0 + 1, int_c<0>{});
        decode_b(bw, 0, bfr[0]);
    }
    __syncthreads();

    const int pairs = (ns + 1) / 2;
    int q = 0;
    constexpr int kAhead = Cfg::DEEP ? 4 : 3;  // a pair is FULL when its loads stay below step ns
    for (; 2 * q + kAhead < ns; ++q) {
        step(q, int_c<0>{}, bool_c<true>{});
        step(q, int_c<1>{}, bool_c<true>{});
    }
    for (; q < pairs; ++q) {
        step(q, int_c<0>{}, bool_c<false>{});
        if (2 * q + 1 < ns) step(q, int_c<1>{}, bool_c<false>{});
    }

    if constexpr (Cfg::KG == 2) {
        // group 1's sums through LDS (the A buffers are free after the last
        // barrier) into group 0, which adds them after its own and goes on
        float* red = reinterpret_cast<float*>(lds_all);
        if (kgrp == 1) {
#pragma unroll
            for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        red[((i * Cfg::FC + j) * 16 + e) * Cfg::NTG + tid] = acc[i][j][e];
        }
        __syncthreads();
        if (kgrp == 1) return;
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] += red[((i * Cfg::FC + j) * 16 + e) * Cfg::NTG + tid];
    }

    if constexpr (SPLIT) {
        // Raw sums of this split go to partial[split][m][n]; the last block of
        // the tile to count itself in adds all splits in split order.  The
        // sums are written and read with the device-scope policy (sc1), and
        // splitk_arrive orders every wave's stores before the count and the
        // count before the last block's loads.  Buffer accesses over one
        // split's M x N sums (host-checked below 2^31 bytes): the row step of
        // register e is folded into the resource base, so rows past M are
        // dropped / read zero by the range check; lanes of columns past N
        // carry an offset beyond every range.
        constexpr int kDeviceScope = 16;  // cache policy SC1
        const int64_t MN = static_cast<int64_t>(p.M) * p.N;
        const int nsplit = static_cast<int>(gridDim.x) / total;
        int voff[Cfg::FR][Cfg::FC];
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j) {
                const int n = c0 + wc * Cfg::WC + j * 32 + (lane & 31);
                voff[i][j] = n < p.N ? ((r0 + wr * Cfg::WR + i * 32 + 4 * h) * p.N + n) * 4 : 0x7FFFFFF0;
            }
        const uint64_t split_bytes = static_cast<uint64_t>(MN) * 4;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const __amdgpu_buffer_rsrc_t rs = buffer_range(
                partial + split * MN, split_bytes, static_cast<uint64_t>(8 * (e >> 2) + (e & 3)) * p.N * 4);
#pragma unroll
            for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
                    // __float_as_uint, not __builtin_bit_cast: hipcc (ROCm 7.2) folds a bit
                    // cast of a vector element with a loop index to element 0
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][e]), rs, voff[i][j], 0,
                                                          kDeviceScope);
        }
        __shared__ int is_last;
        if (!splitk_arrive(counters + t, nsplit, &is_last)) return;
        // 0 + split 0 + split 1 + ... per output, in split order
#pragma unroll
        for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        for (int sp = 0; sp < nsplit; ++sp) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const __amdgpu_buffer_rsrc_t rs = buffer_range(
                    partial + sp * MN, split_bytes, static_cast<uint64_t>(8 * (e >> 2) + (e & 3)) * p.N * 4);
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j)
                        acc[i][j][e] += __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff[i][j], 0, kDeviceScope));
            }
        }
        // ready for the next launch on this workspace
        if (tid == 0) __hip_atomic_store(counters + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- epilogue: C[m, n] = relu?(acc * alpha * scale[n] + bias[n] (+ beta * cin)) ----
    float mult[Cfg::FC], badd[Cfg::FC];
    int ncol[Cfg::FC];
#pragma unroll
    for (int j = 0; j < Cfg::FC; ++j) {
        if constexpr (Cfg::DEEP) {
            mult[j] = mult_e[j], badd[j] = badd_e[j], ncol[j] = ncol_e[j];
        } else {
            ncol[j] = c0 + wc * Cfg::WC + j * 32 + (lane & 31);
            const int nc = min(ncol[j], p.N - 1);
            mult[j] = p.alpha;
            badd[j] = 0.0f;
            if (p.scale) mult[j] = p.alpha * p.scale[nc];
            if (p.bias) badd[j] = p.bias[nc];
        }
    }
    const bool bias_then_scale = (p.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
    const bool relu = (p.flags & TBN_EPI_RELU) != 0;
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i) {
        const int mrow = r0 + wr * Cfg::WR + i * 32 + 4 * h;
        float v[Cfg::FC][16];
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float a = TERNARY ? acc[i][j][e] * 0.5f : acc[i][j][e];  // ternary sums are doubled
                v[j][e] = bias_then_scale ? (a + badd[j]) * mult[j] : a * mult[j] + badd[j];
            }
        if (p.cin) {
            float cv[Cfg::FC][16];
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = min(mrow + 8 * (e >> 2) + (e & 3), p.M - 1);
                    const int nc = min(ncol[j], p.N - 1);
                    cv[j][e] = p.cin_1d ? p.cin[nc] : p.cin[static_cast<int64_t>(m) * p.N + nc];
                }
#pragma unroll
            for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) v[j][e] += p.beta * cv[j][e];
        }
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = mrow + 8 * (e >> 2) + (e & 3);
                float x = v[j][e];
                if (relu) x = x > 0.0f ? x : 0.0f;
                // non-temporal: C is not read again here (0.7 % at 4096^3, 1-2 % at the mid-size shapes)
                if (m < p.M && ncol[j] < p.N)
                    __builtin_nontemporal_store(x, &p.C[static_cast<int64_t>(m) * p.ldc + ncol[j]]);
            }
    }
}

// Tile and K-split choice.  Shapes whose 128 x 512 tiles fill the chip (>= 128
// blocks of 8 waves) take them whole.  Others with an even number of K steps
// whose 32 x 128 tiles number at least 256 take those, in two K groups (one
// block of 8 waves per CU, no partial sums through memory; config 2, 1024^3:
// 10.2 us kernel time against 15.2 for the 64 x 128 tile split 4 ways).  The
// rest take the 64 x 128 tile with K split over up to 8 blocks per tile,
// aiming at 512 blocks (two per CU), each split keeping at least 4 K steps
// (config 3, 256 x 4096^2 ternary: 4 splits 36.6 us, 2 splits 42.7, 8 splits
// 40.4; the 128 x 512 and 128 x 256 tiles with any split were slower).  The
// choice reads only M, N and K, so a GEMM's result does not depend on
// anything else.  TBN_TUNE_GEMM_TILE / TBN_TUNE_GEMM_SPLITS force either.
struct WidePlan {
    int cfg = 0;      // 0 Wide, 1 WideSmall, 2 WideMid
    int tiles_r = 0, tiles_c = 0, steps = 0, splits = 1, per = 0;
    int xcd_cols = 1;  // mid-size tiles: XCD grid columns (gemm_mid_kernel's tile order)
    int64_t blocks() const { return static_cast<int64_t>(tiles_r) * tiles_c * splits; }
};

template <class Cfg>
WidePlan plan_for(int cfg, int M, int N, int K, bool ternary) {
    WidePlan w;
    w.cfg = cfg;
    w.tiles_r = static_cast<int>(tbn_hip::ceil_div(M, Cfg::BR));
    w.tiles_c = static_cast<int>(tbn_hip::ceil_div(N, Cfg::BC));
    w.steps = static_cast<int>(tbn_hip::ceil_div(K, Cfg::KS));
    const int64_t tiles = static_cast<int64_t>(w.tiles_r) * w.tiles_c;
    int sp = 1;
    const int forced = tbn_hip::tuning(TBN_TUNE_GEMM_SPLITS);
    if (Cfg::KG > 1) {
        sp = 1;  // the K groups split K inside the block
    } else if (forced >= 1) {
        sp = std::min(forced, std::max(w.steps, 1));
    } else if (cfg != 0 && tiles < 512) {
        sp = static_cast<int>(std::min<int64_t>((512 + tiles - 1) / tiles, 8));
        sp = std::max(1, std::min(sp, w.steps / 4));
    }
    w.per = (w.steps + sp - 1) / sp;
    w.splits = (w.steps + w.per - 1) / w.per;  // splits that own at least one step
    if (Cfg::DEEP && tiles % 8 == 0) {
        // the XCD rectangle with the fewest A and W bytes to fetch per XCD (ties
        // to the narrower): config 3 (8 x 32 tiles) takes 2 x 16 per XCD, 3 MB
        // against 4.5 MB for whole row bands (31.0 -> 30.2 us); config 2
        // (32 x 8 tiles) keeps whole row bands
        const double a_band = static_cast<double>(Cfg::BR) * K * 4;
        const double w_tile = static_cast<double>(Cfg::BC) * K / (ternary ? 4 : 8);
        double best = 0.0;
        for (int r = 1; r <= 8; r *= 2) {
            if ((w.tiles_r * r) % 8 || w.tiles_c % r) continue;
            const double bytes = (w.tiles_r * r / 8) * a_band + (w.tiles_c / r) * w_tile;
            if (r == 1 || bytes < best) best = bytes, w.xcd_cols = r;
        }
    }
    return w;
}

// WideMid needs an even step count (its two K groups take equal halves).
bool mid_ok(int K) { return tbn_hip::ceil_div(K, WideMid::KS) % 2 == 0; }

WidePlan choose_plan(int M, int N, int K, bool ternary) {
    const int forced = tbn_hip::tuning(TBN_TUNE_GEMM_TILE);
    if (forced == 0) return plan_for<Wide>(0, M, N, K, ternary);
    if (forced == 1) return plan_for<WideSmall>(1, M, N, K, ternary);
    if (forced == 2 && mid_ok(K)) return plan_for<WideMid>(2, M, N, K, ternary);
    const WidePlan big = plan_for<Wide>(0, M, N, K, ternary);
    if (big.blocks() >= 128) return big;
    if (forced != 1 && mid_ok(K)) {
        const WidePlan mid = plan_for<WideMid>(2, M, N, K, ternary);
        if (mid.blocks() >= 256 && mid.steps >= 4) return mid;
    }
    return plan_for<WideSmall>(1, M, N, K, ternary);
}

// Kernel variants: the large tile on gemm_wide_kernel, the mid-size (DEEP)
// tiles on gemm_mid_kernel.
template <class Cfg, bool TERNARY>
void launch_wide(const tbn_hip::WideGemmArgs& a, const WidePlan& w, float* part, int* counters,
                 hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(w.blocks()));
    if constexpr (!Cfg::DEEP) {
        if (w.splits > 1)
            hipLaunchKernelGGL((gemm_wide_kernel<Cfg, TERNARY, true>), grid, dim3(Cfg::NT), 0, stream, a, w.tiles_r,
                               w.tiles_c, w.per, part, counters);
        else
            hipLaunchKernelGGL((gemm_wide_kernel<Cfg, TERNARY, false>), grid, dim3(Cfg::NT), 0, stream, a, w.tiles_r,
                               w.tiles_c, w.per, nullptr, nullptr);
    } else {
        if constexpr (Cfg::KG == 1) {
            if (w.splits > 1) {
                hipLaunchKernelGGL((gemm_mid_kernel<Cfg, TERNARY, true>), grid, dim3(Cfg::NT), 0, stream, a,
                                   w.tiles_r, w.tiles_c, w.per, part, counters, w.xcd_cols);
                return;
            }
        }
        hipLaunchKernelGGL((gemm_mid_kernel<Cfg, TERNARY, false>), grid, dim3(Cfg::NT), 0, stream, a, w.tiles_r,
                           w.tiles_c, w.per, nullptr, nullptr, w.xcd_cols);
    }
}

template <bool TERNARY>
void launch_plan(const tbn_hip::WideGemmArgs& a, const WidePlan& w, float* part, int* counters, hipStream_t s) {
    if (w.cfg == 0) launch_wide<Wide, TERNARY>(a, w, part, counters, s);
    else if (w.cfg == 1) launch_wide<WideSmall, TERNARY>(a, w, part, counters, s);
    else launch_wide<WideMid, TERNARY>(a, w, part, counters, s);
}

}  // namespace

namespace tbn_hip {

bool gemm_wide_fits(const WideGemmArgs& a, bool ternary) {
    const WidePlan w = choose_plan(a.M, a.N, a.K, ternary);
    const int waves = w.cfg == 1 ? 4 : 8;
    const int bc = w.cfg == 0 ? 512 : 128;
    // shapes that give at least half the chip one wave per SIMD
    return a.K >= 64 && w.blocks() * waves >= 512 && a.M >= 64 && a.N >= 128 && a.lda % 4 == 0 &&
           reinterpret_cast<uintptr_t>(a.A) % 16 == 0 && a.col_bytes % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.packed) % 16 == 0 && a.lda <= (1 << 22) &&
           static_cast<int64_t>(bc) * a.col_bytes < (1LL << 31) && (ternary || a.col_bytes % 16 == 0) &&
           static_cast<int64_t>(w.tiles_r) * w.tiles_c <= kWorkspaceCounters &&
           (w.splits == 1 || static_cast<int64_t>(a.M + 128) * a.N * 4 < (1LL << 31));
}

std::string gemm_wide_kernel_name(const WideGemmArgs& a, bool ternary) {
    const WidePlan w = choose_plan(a.M, a.N, a.K, ternary);
    const char* cfg = w.cfg == 0   ? "WideCfg<128, 512, 128, 64, 64, false, 1>"
                      : w.cfg == 1 ? "WideCfg<64, 128, 32, 64, 64, true, 1>"
                                   : "WideCfg<32, 128, 32, 32, 64, true, 2>";
    const bool split = w.splits > 1 && w.cfg != 2;
    return std::string(w.cfg == 0 ? "gemm_wide_kernel<" : "gemm_mid_kernel<") + cfg + ", " +
           (ternary ? "true" : "false") + ", " + (split ? "true" : "false") + ">";
}

int gemm_wide(const WideGemmArgs& a, bool ternary, hipStream_t stream) {
    const WidePlan w = choose_plan(a.M, a.N, a.K, ternary);
    const char* what = ternary ? "gemm_f32_ternary (wide)" : "gemm_f32_binary (wide)";
    void* part = nullptr;
    int* counters = nullptr;
    bool temporary = false;
    if (w.splits > 1) {
        const size_t bytes = static_cast<size_t>(w.splits) * a.M * a.N * sizeof(float);
        const int wrc = stream_workspace(stream, bytes, part, temporary, &counters);
        if (wrc) return wrc;
    }
    if (ternary) launch_plan<true>(a, w, static_cast<float*>(part), counters, stream);
    else launch_plan<false>(a, w, static_cast<float*>(part), counters, stream);
    const int rc = check_launch(what);
    if (part) release_workspace(part, temporary, stream);
    return rc;
}

}  // namespace tbn_hip
