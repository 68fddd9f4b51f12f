// MFMA tile engine shared by the GEMM and implicit-GEMM convolution kernels.
//
// One workgroup computes a BR x BC tile of D = R * C^T where the MFMA row
// operand R and column operand C are each one of
//   * a "split" operand: fp32 values v = hi + mid + lo, three bf16 numbers
//     produced by truncation, so the sum is exact (hi keeps the top 8
//     significant bits, mid the next 8, lo the last 8; each subtraction is
//     exact by Sterbenz's lemma);
//   * a "sign" operand: +-1 (binary) or -1/0/+1 (ternary) weights decoded
//     from the packed bits; these are exact in bf16.
// A split x sign product therefore needs three bf16 MFMAs, each of which
// forms exact products and accumulates in fp32.  split x split (fp32 layers)
// uses the six leading cross terms (error ~2^-24 relative per product).
//
// Pipeline per K step of BK = 32: global -> registers (prefetch of step t+1
// overlaps the MFMAs of step t) -> convert/decode -> LDS -> fragments -> MFMA
// v_mfma_f32_32x32x16_bf16.  LDS rows are BK + 8 bf16 (80 bytes) so the
// 16-byte fragment reads of 32 consecutive rows hit distinct banks.
//
// Operand lane layout of v_mfma_f32_32x32x16_bf16 (checked on gfx950):
//   row operand  lane l holds R[l%32][8*(l/32) .. +7]
//   col operand  lane l holds C[l%32][8*(l/32) .. +7]   (k-major per column)
//   result       lane l, register j holds D[8*(j/4) + 4*(l/32) + j%4][l%32]
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tbnk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int BK = 32;           // K elements staged per LDS round
constexpr int LDS_ROW = BK + 8;  // bf16 per LDS row (80 bytes)

template <int BR_, int BC_, int WR_, int WC_, int WAVES_PER_SIMD_ = 1>
struct TileCfg {
    static constexpr int BR = BR_, BC = BC_, WR = WR_, WC = WC_;
    static constexpr int WAVES_PER_SIMD = WAVES_PER_SIMD_;  // occupancy the registers must allow
    static constexpr int WAVES_R = BR / WR, WAVES_C = BC / WC;
    static constexpr int NT = 64 * WAVES_R * WAVES_C;
    static constexpr int FR = WR / 32, FC = WC / 32;
    static_assert(WR % 32 == 0 && WC % 32 == 0, "wave tile must be a multiple of 32");
    static_assert(BR % WR == 0 && BC % WC == 0, "block tile must be a multiple of the wave tile");
};

// ---------------------------------------------------------------------------
// Conversions
// ---------------------------------------------------------------------------

// Upper 16 bits of a and b packed as (bf16(a), bf16(b)) in one dword.
__device__ __forceinline__ uint32_t upper_halves(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// Exact three-way bf16 split of 8 fp32 values (hi + mid + lo = x), branch
// free: r1 = x - hi is forced to 0 where x == hi, which covers +-inf (whose
// plain difference is NaN); a NaN input keeps a NaN in hi or r1.
__device__ __forceinline__ void split8(const float* x, uint4& hi, uint4& mid, uint4& lo) {
    uint32_t hb[8], mb[8], lb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t u = __float_as_uint(x[e]);
        const float h = __uint_as_float(u & 0xFFFF0000u);
        const float r1 = (x[e] == h) ? 0.0f : x[e] - h;
        const uint32_t m = __float_as_uint(r1);
        const float r2 = r1 - __uint_as_float(m & 0xFFFF0000u);
        hb[e] = u;
        mb[e] = m;
        lb[e] = __float_as_uint(r2);
    }
    hi = make_uint4(upper_halves(hb[0], hb[1]), upper_halves(hb[2], hb[3]), upper_halves(hb[4], hb[5]),
                    upper_halves(hb[6], hb[7]));
    mid = make_uint4(upper_halves(mb[0], mb[1]), upper_halves(mb[2], mb[3]), upper_halves(mb[4], mb[5]),
                     upper_halves(mb[6], mb[7]));
    lo = make_uint4(upper_halves(lb[0], lb[1]), upper_halves(lb[2], lb[3]), upper_halves(lb[4], lb[5]),
                    upper_halves(lb[6], lb[7]));
}

struct Split4 {
    uint32_t hi[2], mid[2], lo[2];
};

// Exact three-way bf16 split of four fp32 values.  Infinity keeps hi = +-inf
// and zero mid/lo parts (the plain subtraction would give NaN); NaN inputs
// stay NaN through hi and mid.
__device__ __forceinline__ Split4 split4(float x0, float x1, float x2, float x3) {
    float x[4] = {x0, x1, x2, x3};
    uint32_t u[4], m[4], l[4];
    float r1[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        u[e] = __float_as_uint(x[e]);
        r1[e] = x[e] - __uint_as_float(u[e] & 0xFFFF0000u);
    }
    const float amax = fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3)));
    if (__builtin_expect(!(amax <= 3.40282347e38f), 0)) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (fabsf(x[e]) > 3.40282347e38f) r1[e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        m[e] = __float_as_uint(r1[e]);
        const float r2 = r1[e] - __uint_as_float(m[e] & 0xFFFF0000u);
        l[e] = __float_as_uint(r2);
    }
    Split4 s;
    s.hi[0] = upper_halves(u[0], u[1]);
    s.hi[1] = upper_halves(u[2], u[3]);
    s.mid[0] = upper_halves(m[0], m[1]);
    s.mid[1] = upper_halves(m[2], m[3]);
    s.lo[0] = upper_halves(l[0], l[1]);
    s.lo[1] = upper_halves(l[2], l[3]);
    return s;
}

// 8 BinaryMatrix bits (bit e = weight k0+e, 1 means -1) -> 8 bf16 +-1.0
// (0x3F80 = +1.0, sign bit 15 set = -1.0).
__device__ __forceinline__ u32x4_t decode_binary8(uint32_t x) {
    u32x4_t r;
    r[0] = 0x3F803F80u | ((x << 15) & 0x8000u) | ((x << 30) & 0x80000000u);
    r[1] = 0x3F803F80u | ((x << 13) & 0x8000u) | ((x << 28) & 0x80000000u);
    r[2] = 0x3F803F80u | ((x << 11) & 0x8000u) | ((x << 26) & 0x80000000u);
    r[3] = 0x3F803F80u | ((x << 9) & 0x8000u) | ((x << 24) & 0x80000000u);
    return r;
}

// One 2-bit code -> bf16 bits: 00 -> -1.0, 10 -> +1.0, 01/11 -> 0.
__device__ __forceinline__ uint32_t ternary_bf16(uint32_t code) {
    const uint32_t nonzero_mask = (code & 1u) - 1u;            // all ones iff low bit clear
    const uint32_t value = 0xBF80u ^ ((code & 2u) << 14);       // 10 -> 0x3F80, 00 -> 0xBF80
    return value & nonzero_mask & 0xFFFFu;
}

// 8 consecutive 2-bit codes (16 bits) -> 8 bf16.
__device__ __forceinline__ u32x4_t decode_ternary8(uint32_t y) {
    u32x4_t r;
#pragma unroll
    for (int d = 0; d < 4; ++d)
        r[d] = ternary_bf16((y >> (4 * d)) & 3u) | (ternary_bf16((y >> (4 * d + 2)) & 3u) << 16);
    return r;
}

// 8 two-bit ternary codes (code i in bits 2i, 2i+1: 00 -> -1, 10 -> +1, 01 and
// 11 -> 0) -> 8 bf16 of TWICE the weight.  With u = ~x, bit 2i+1 of u is the
// sign and bit 2i says "nonzero"; placed at bits 15 and 14 of a half they are
// the bf16 bits of -2 (0xC000), +2 (0x4000), -0 (0x8000) or +0.  y holds code
// i at bits 2i and 2i + 14 (bits 16 and up of x must be zero), so one shift
// puts code 2d at bits 15:14 and code 2d+1 at 31:30, and an AND of the
// inverted word finishes a dword (the inversion is done once, on y).  Kernels
// using it halve their sums before the epilogue: every product and partial
// sum is scaled by 2, which fp32 rounding commutes with (away from overflow
// and subnormals), so the result equals the sum over +-1 / 0 weights.
__device__ __forceinline__ u32x4_t decode_ternary8_x2(uint32_t x) {
    const uint32_t y = x | (x << 14);
    u32x4_t r;
#pragma unroll
    for (int d = 0; d < 4; ++d) r[d] = ~(y << (14 - 4 * d)) & 0xC000C000u;
    return r;
}

__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Fast unsigned division for n * d < 2^32 (m = ceil(2^32 / d)).
struct FastDiv {
    uint32_t d;
    uint64_t m;
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        return static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> 32);
    }
};
inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    f.m = ((uint64_t(1) << 32) + d - 1) / d;
    return f;
}

// n / d for every 0 <= n < 2^31 and d >= 1, without a branch: with
// m = floor((2^32 - 1) / d), umulhi(n, m) > n/d - n/2^32 > n/d - 1/2, so it is
// q or q - 1, and the remainder test adds the missing one (d = 1 included).
struct UDiv {
    uint32_t m, d;
};
inline UDiv make_udiv(uint32_t d) { return UDiv{0xFFFFFFFFu / (d ? d : 1u), d ? d : 1u}; }
__device__ __forceinline__ int udiv(int n, UDiv v) {
    uint32_t q = __umulhi(static_cast<uint32_t>(n), v.m);
    q += (static_cast<uint32_t>(n) - q * v.d) >= v.d ? 1u : 0u;
    return static_cast<int>(q);
}

// ---------------------------------------------------------------------------
// Buffer resources and the split-K finish
// ---------------------------------------------------------------------------

// Raw dword buffer resource over [base + skip, base + bytes): the range check
// then drops every access whose voffset reaches past `bytes - skip`, so an
// offset that would otherwise go in the (unchecked) SGPR offset field is
// folded into the base instead and stays bounds-checked.  skip >= bytes gives
// an empty range (every access dropped).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_range(const void* base, uint64_t bytes, uint64_t skip) {
    const uint64_t left = bytes > skip ? bytes - skip : 0;
    const uint32_t n = left > 0xFFFFFFFFull ? 0xFFFFFFFFu : static_cast<uint32_t>(left);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(static_cast<const char*>(base)) + skip,
                                             static_cast<short>(0), static_cast<int>(n), 0x00020000);
}

// Split-K arrival of one block at its tile's counter, after every thread has
// issued its partial-sum stores (device-scope policy).  Returns true in every
// thread of the block that arrives last; that block may then read all splits'
// partial sums.  The ordering:
//   1. each wave waits until its own stores are acknowledged (vmcnt(0)): the
//      workgroup barrier alone emits no such wait on gfx950;
//   2. the barrier then orders every wave's completed stores before thread 0;
//   3. thread 0's increment is acquire-release at agent scope: its release
//      half writes back this XCD's L2 (which covers the other waves' lines)
//      and waits before the increment, its acquire half invalidates the
//      non-coherent cache lines after it;
//   4. the last block's waves each run an agent-scope acquire fence before
//      reading the other blocks' sums.
__device__ __forceinline__ bool splitk_arrive(int* counter, int arrivals, int* flag_lds) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        *flag_lds = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == arrivals - 1;
    __syncthreads();
    const bool last = *flag_lds != 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return last;
}

// ---------------------------------------------------------------------------
// Operand loaders.  Each has a register stage (`Regs`), `load` (global ->
// registers for the K step starting at k0) and `store` (registers -> LDS in
// the [piece][row][k] bf16 layout).
// ---------------------------------------------------------------------------

// fp32 matrix operand X(row, k) = base[row * s_row + k * s_k], rows < rows_valid,
// k < K; split into three bf16 planes.  Work item = (row, 4 consecutive k).
template <int ROWS, int NT>
struct SplitMatrix {
    static constexpr int PIECES = 3;
    static constexpr int ITEMS = ROWS * (BK / 4);
    static constexpr int PER_THREAD = (ITEMS + NT - 1) / NT;
    const float* base;
    int64_t s_row, s_k;
    int rows_valid, K;
    int vec;        // s_k == 1 and 16-byte aligned rows: float4 loads
    int row_fast;   // s_row == 1: map consecutive threads to consecutive rows

    struct Regs {
        float v[PER_THREAD][4];
    };

    __device__ __forceinline__ void init(Regs&, int, int) const {}

    __device__ __forceinline__ void item_coords(int item, int& r, int& kc) const {
        if (row_fast) { r = item % ROWS; kc = item / ROWS; }
        else { r = item / (BK / 4); kc = item % (BK / 4); }
    }

    __device__ __forceinline__ void load(Regs& g, int r0, int k0, int tid) const {
#pragma unroll
        for (int it = 0; it < PER_THREAD; ++it) {
            const int item = tid + it * NT;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            if (ITEMS % NT == 0 || item < ITEMS) {
                int r, kc;
                item_coords(item, r, kc);
                const int row = r0 + r;
                const int k = k0 + kc * 4;
                if (row < rows_valid) {
                    const float* p = base + static_cast<int64_t>(row) * s_row;
                    if (vec && k + 3 < K) {
                        const float4 q = *reinterpret_cast<const float4*>(p + k);
                        a0 = q.x; a1 = q.y; a2 = q.z; a3 = q.w;
                    } else {
                        if (k + 0 < K) a0 = p[static_cast<int64_t>(k + 0) * s_k];
                        if (k + 1 < K) a1 = p[static_cast<int64_t>(k + 1) * s_k];
                        if (k + 2 < K) a2 = p[static_cast<int64_t>(k + 2) * s_k];
                        if (k + 3 < K) a3 = p[static_cast<int64_t>(k + 3) * s_k];
                    }
                }
            }
            g.v[it][0] = a0; g.v[it][1] = a1; g.v[it][2] = a2; g.v[it][3] = a3;
        }
    }

    __device__ __forceinline__ void store(const Regs& g, uint16_t* lds, int tid) const {
#pragma unroll
        for (int it = 0; it < PER_THREAD; ++it) {
            const int item = tid + it * NT;
            if (ITEMS % NT == 0 || item < ITEMS) {
                int r, kc;
                item_coords(item, r, kc);
                const Split4 s = split4(g.v[it][0], g.v[it][1], g.v[it][2], g.v[it][3]);
                uint16_t* dst = lds + r * LDS_ROW + kc * 4;
                *reinterpret_cast<uint2*>(dst) = make_uint2(s.hi[0], s.hi[1]);
                *reinterpret_cast<uint2*>(dst + ROWS * LDS_ROW) = make_uint2(s.mid[0], s.mid[1]);
                *reinterpret_cast<uint2*>(dst + 2 * ROWS * LDS_ROW) = make_uint2(s.lo[0], s.lo[1]);
            }
        }
    }
};

// Packed binary / ternary weights: row r of the operand is column r of the
// BinaryMatrix (binary, K_pad/8 bytes per column) or of the 2-bit GEMM layout
// (ternary, K_pad/4 bytes per column).  Work item = (row, 8 consecutive k).
template <int ROWS, int NT, bool TERNARY>
struct SignPacked {
    static constexpr int PIECES = 1;
    static constexpr int ITEMS = ROWS * (BK / 8);
    static constexpr int PER_THREAD = (ITEMS + NT - 1) / NT;
    const uint8_t* packed;
    int64_t col_bytes;
    int rows_valid;  // N_pad: columns present in the packed buffer

    struct Regs {
        uint32_t bits[PER_THREAD];
    };

    __device__ __forceinline__ void init(Regs&, int, int) const {}

    __device__ __forceinline__ void load(Regs& g, int r0, int k0, int tid) const {
#pragma unroll
        for (int it = 0; it < PER_THREAD; ++it) {
            const int item = tid + it * NT;
            uint32_t b = 0;
            if (ITEMS % NT == 0 || item < ITEMS) {
                const int r = item >> 2, j = item & 3;
                const int row = r0 + r;
                if (row < rows_valid) {
                    const uint8_t* col = packed + static_cast<int64_t>(row) * col_bytes;
                    if (TERNARY)
                        b = *reinterpret_cast<const uint16_t*>(col + k0 / 4 + 2 * j);
                    else
                        b = col[k0 / 8 + j];
                }
            }
            g.bits[it] = b;
        }
    }

    __device__ __forceinline__ void store(const Regs& g, uint16_t* lds, int tid) const {
#pragma unroll
        for (int it = 0; it < PER_THREAD; ++it) {
            const int item = tid + it * NT;
            if (ITEMS % NT == 0 || item < ITEMS) {
                const int r = item >> 2, j = item & 3;
                const u32x4_t v = TERNARY ? decode_ternary8(g.bits[it]) : decode_binary8(g.bits[it]);
                *reinterpret_cast<u32x4_t*>(lds + r * LDS_ROW + j * 8) = v;
            }
        }
    }
};

// ---------------------------------------------------------------------------
// The tile kernel body
// ---------------------------------------------------------------------------

template <int PR, int PC>
struct ProductSchedule;
template <>
struct ProductSchedule<3, 1> {  // split rows x sign cols
    static constexpr int N = 3;
    static constexpr int r[3] = {0, 1, 2};
    static constexpr int c[3] = {0, 0, 0};
};
template <>
struct ProductSchedule<1, 3> {  // sign rows x split cols
    static constexpr int N = 3;
    static constexpr int r[3] = {0, 0, 0};
    static constexpr int c[3] = {0, 1, 2};
};
template <>
struct ProductSchedule<3, 3> {  // split x split: hi*hi, hi*mid, mid*hi, hi*lo, mid*mid, lo*hi
    static constexpr int N = 6;
    static constexpr int r[6] = {0, 0, 1, 0, 1, 2};
    static constexpr int c[6] = {0, 1, 0, 2, 1, 0};
};

// Maps a linear workgroup id to (tile_r, tile_c): consecutive ids on one XCD
// (workgroups are dealt round-robin over the 8 XCDs) get neighbouring tiles,
// walked in groups of 8 tile-rows so operand tiles are reused from L2.
__device__ __forceinline__ void tile_coords_of(int pid, int tiles_r, int tiles_c, int& tr, int& tc) {
    const int total = tiles_r * tiles_c;
    if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
    constexpr int GROUP = 8;
    const int per_group = GROUP * tiles_c;
    const int g = pid / per_group;
    const int first = g * GROUP;
    const int rows_in_group = min(tiles_r - first, GROUP);
    const int in = pid % per_group;
    tr = first + in % rows_in_group;
    tc = in / rows_in_group;
}
__device__ __forceinline__ void tile_coords(int tiles_r, int tiles_c, int& tr, int& tc) {
    tile_coords_of(static_cast<int>(blockIdx.x), tiles_r, tiles_c, tr, tc);
}

// One block's tile (tr, tc) over K: operands staged through LDS in BK steps.
template <class Cfg, class RowL, class ColL, class Epi>
__device__ __forceinline__ void mfma_tile_body(const RowL& rowl, const ColL& coll, const Epi& epi, int K, int tr,
                                               int tc) {
    __shared__ __attribute__((aligned(16))) uint16_t lds_r[RowL::PIECES * Cfg::BR * LDS_ROW];
    __shared__ __attribute__((aligned(16))) uint16_t lds_c[ColL::PIECES * Cfg::BC * LDS_ROW];
    using Sched = ProductSchedule<RowL::PIECES, ColL::PIECES>;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave / Cfg::WAVES_C;
    const int wc = wave % Cfg::WAVES_C;
    const int r0 = tr * Cfg::BR;
    const int c0 = tc * Cfg::BC;

    f32x16_t acc[Cfg::FR][Cfg::FC];
#pragma unroll
    for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FC; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    typename RowL::Regs rg;
    typename ColL::Regs cg;
    rowl.init(rg, r0, tid);
    coll.init(cg, c0, tid);
    if (K > 0) {
        rowl.load(rg, r0, 0, tid);
        coll.load(cg, c0, 0, tid);
    }

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 8;

    for (int k0 = 0; k0 < K; k0 += BK) {
        rowl.store(rg, lds_r, tid);
        coll.store(cg, lds_c, tid);
        __syncthreads();
        if (k0 + BK < K) {
            rowl.load(rg, r0, k0 + BK, tid);
            coll.load(cg, c0, k0 + BK, tid);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            u32x4_t ra[RowL::PIECES][Cfg::FR];
            u32x4_t cb[ColL::PIECES][Cfg::FC];
#pragma unroll
            for (int p = 0; p < RowL::PIECES; ++p)
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
                    ra[p][i] = *reinterpret_cast<const u32x4_t*>(
                        lds_r + (p * Cfg::BR + wr * Cfg::WR + i * 32 + frag_row) * LDS_ROW + kk + frag_k);
#pragma unroll
            for (int p = 0; p < ColL::PIECES; ++p)
#pragma unroll
                for (int j = 0; j < Cfg::FC; ++j)
                    cb[p][j] = *reinterpret_cast<const u32x4_t*>(
                        lds_c + (p * Cfg::BC + wc * Cfg::WC + j * 32 + frag_row) * LDS_ROW + kk + frag_k);
#pragma unroll
            for (int s = 0; s < Sched::N; ++s)
#pragma unroll
                for (int i = 0; i < Cfg::FR; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::FC; ++j)
                        acc[i][j] = mfma32(ra[Sched::r[s]][i], cb[Sched::c[s]][j], acc[i][j]);
        }
        __syncthreads();
    }

    epi.template apply<Cfg>(acc, r0 + wr * Cfg::WR, c0 + wc * Cfg::WC, lane);
}

template <class Cfg, class RowL, class ColL, class Epi>
__global__ void __launch_bounds__(Cfg::NT, Cfg::WAVES_PER_SIMD)
mfma_tile_kernel(RowL rowl, ColL coll, Epi epi, int K, int tiles_r, int tiles_c) {
    int tr, tc;
    tile_coords(tiles_r, tiles_c, tr, tc);
    mfma_tile_body<Cfg>(rowl, coll, epi, K, tr, tc);
}

// Row / column of register e of fragment (i, j) relative to the wave tile.
__device__ __forceinline__ int frag_out_row(int i, int e, int lane) {
    return i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
__device__ __forceinline__ int frag_out_col(int j, int lane) { return j * 32 + (lane & 31); }

}  // namespace tbnk
