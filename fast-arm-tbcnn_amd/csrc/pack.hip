// Weight quantization and bit-packing kernels (north_star subsystem 1).
//
// Every kernel writes the reference's packed formats bit for bit:
//   BinaryMatrix   column n = K_pad/8 bytes, bit (k&7) of byte k>>3, 1 = -1,
//                  padding +1 (GeMM/05-final/GeMM.cpp:114-151)
//   ternary 2-bit  00=-1, 01=0, 10=+1, 11 decodes to 0
//                  (tbn-runtime/include/tbn/memory/packed_weights.hpp:35-71)
// The packers work on 32-bit output words (32 binary or 16 ternary weights of
// one column) so each thread issues one aligned store.  Weight packing runs
// once per Session, so these kernels favour simple coalesced reads over
// tiling.
#include <type_traits>

#include "common.hpp"

namespace {

constexpr int kThreads = 256;

inline int grid_for(int64_t work) {
    const int64_t blocks = tbn_hip::ceil_div(work, kThreads);
    return static_cast<int>(blocks < 16384 ? (blocks > 0 ? blocks : 1) : 16384);
}

// ---- elementwise quantizers ------------------------------------------------

__global__ void quantize_binary_f32_kernel(const float* __restrict__ w, int64_t n, float thr,
                                           uint8_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (w[i] > thr) ? 1 : 0;
}

__global__ void quantize_binary_i8_kernel(const int8_t* __restrict__ w, int64_t n,
                                          uint8_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (w[i] > 0) ? 1 : 0;
}

__global__ void quantize_ternary_f32_kernel(const float* __restrict__ w, int64_t n, float lo,
                                            float hi, int8_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float v = w[i];
        out[i] = (v < lo) ? int8_t(-1) : ((v > hi) ? int8_t(1) : int8_t(0));
    }
}

__global__ void sign_ge0_kernel(const float* __restrict__ w, int64_t n, uint8_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (w[i] >= 0.0f) ? 1 : 0;
}

// mean |w| per channel, summed in the same sequential order as the Session
// (model.hpp:388-394) so the scale is bit-identical: a block owns 64
// channels (contiguous rows).  Chunks of 128 positions of all 64 rows go
// through LDS (two buffers) with coalesced loads, the next chunk's loads in
// flight while thread c adds its row's values of the current one in order,
// 16 LDS reads ahead of the adds.
constexpr int kMeanChunk = 128;
__global__ void __launch_bounds__(256) channel_mean_abs_kernel(const float* __restrict__ w, int64_t channels,
                                                               int64_t per_channel, float* __restrict__ scale) {
    constexpr int kPitch = kMeanChunk + 4;  // 16-byte aligned rows
    constexpr int kPer = 64 * kMeanChunk / 256;
    __shared__ __attribute__((aligned(16))) float tile[2][64][kPitch];
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int nc = static_cast<int>(channels - c0 < 64 ? channels - c0 : 64);
    const int tid = threadIdx.x;
    float pre[kPer];
    // Every lane loads (an out-of-range slot reads element 0 and is zeroed
    // when stored), so the loads issue back to back with no branch around
    // them and the wait for them falls at the store, after the chunk's sums.
    auto in_range = [&](int j, int64_t k0) {
        const int idx = tid + 256 * j;
        return (idx / kMeanChunk < nc) & (k0 + idx % kMeanChunk < per_channel);
    };
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int idx = tid + 256 * j;
            pre[j] = w[in_range(j, k0) ? (c0 + idx / kMeanChunk) * per_channel + k0 + idx % kMeanChunk : 0];
        }
    };
    auto store = [&](int b, int64_t k0) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int idx = tid + 256 * j;
            tile[b][idx / kMeanChunk][idx % kMeanChunk] = in_range(j, k0) ? fabsf(pre[j]) : 0.0f;
        }
    };
    float acc = 0.0f;
    const int64_t chunks = (per_channel + kMeanChunk - 1) / kMeanChunk;
    load(0);
    store(0, 0);
    __syncthreads();
    for (int64_t ch = 0; ch < chunks; ++ch) {
        const int b = static_cast<int>(ch & 1);
        if (ch + 1 < chunks) load((ch + 1) * kMeanChunk);
        const int kl = static_cast<int>(per_channel - ch * kMeanChunk < kMeanChunk ? per_channel - ch * kMeanChunk
                                                                                     : kMeanChunk);
        if (tid < nc) {
            const float* row = tile[b][tid];
            int i = 0;
            for (; i + 16 <= kl; i += 16) {
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; e += 4) {
                    const float4 q = *reinterpret_cast<const float4*>(row + i + e);
                    v[e] = q.x, v[e + 1] = q.y, v[e + 2] = q.z, v[e + 3] = q.w;
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) acc += v[e];
            }
            for (; i < kl; ++i) acc += row[i];
        }
        if (ch + 1 < chunks) store(b ^ 1, (ch + 1) * kMeanChunk);
        __syncthreads();
    }
    if (tid < nc) scale[c0 + tid] = acc / static_cast<float>(per_channel);
}

// ---- BinaryMatrix packing ---------------------------------------------------

// Source of the sign of weight (k, n): a BINARY byte tensor or fp32 weights
// under one of the reference's sign rules.  Returns true when the weight is -1.
struct BinaryBytes {
    const uint8_t* p;
    __device__ bool neg(int64_t idx) const { return p[idx] != 1; }
};
struct FloatGT {
    const float* p;
    float thr;
    __device__ bool neg(int64_t idx) const { return !(p[idx] > thr); }
};
struct FloatGE0 {
    const float* p;
    __device__ bool neg(int64_t idx) const { return !(p[idx] >= 0.0f); }
};

// The Session's rule for a Gemm weight tensor it did not pack in advance
// (model.hpp:765-845): w >= 0 when every sampled value is one of -1, 0, +1,
// +-0.999, else w > 0.  `ge` is decided per block before packing.
struct FloatSampled {
    const float* p;
    bool ge;
    __device__ bool neg(int64_t idx) const { return ge ? !(p[idx] >= 0.0f) : !(p[idx] > 0.0f); }
};

// The reference's sampled check (model.hpp:773-781): elements 0, step,
// 2*step, ... of the tensor in memory order, step = max(1, elems / 1000).
__device__ bool sampled_binary_block(const float* w, int64_t elems) {
    const int64_t step = elems / 1000 > 1 ? elems / 1000 : 1;
    bool bad = false;
    for (int64_t i = threadIdx.x * step; i < elems; i += static_cast<int64_t>(blockDim.x) * step) {
        const float v = w[i];
        bad |= !(v == -1.0f || v == 1.0f || v == 0.0f || v == 0.999f || v == -0.999f);
    }
    return !__syncthreads_or(bad);
}

// Word (n, wi) holds k = 32*wi .. 32*wi+31 of column n.  For layout KN the
// thread index runs fastest over n so reads of W[k, :] coalesce; for NK it
// runs fastest over wi so each thread reads 32 contiguous weights of row n.
// FloatSampled sources decide their rule first (all threads of the block take
// part in that barrier).
template <class Src>
__global__ void pack_binary_kernel(Src src, int64_t K, int64_t N, int layout, int64_t K_pad,
                                   int64_t N_pad, uint32_t* __restrict__ packed) {
    if constexpr (std::is_same_v<Src, FloatSampled>) src.ge = sampled_binary_block(src.p, K * N);
    const int64_t words_per_col = K_pad / 32;
    const int64_t total = N_pad * words_per_col;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        int64_t n, wi;
        if (layout == TBN_LAYOUT_KN) { n = t % N_pad; wi = t / N_pad; }
        else { wi = t % words_per_col; n = t / words_per_col; }
        uint32_t word = 0;
        if (n < N) {
            const int64_t k0 = wi * 32;
#pragma unroll 4
            for (int j = 0; j < 32; ++j) {
                const int64_t k = k0 + j;
                if (k < K) {
                    const int64_t idx = (layout == TBN_LAYOUT_KN) ? k * N + n : n * K + k;
                    word |= (src.neg(idx) ? 1u : 0u) << j;
                }
            }
        }
        packed[n * words_per_col + wi] = word;
    }
}

__global__ void unpack_binary_kernel(const uint8_t* __restrict__ packed, int64_t K, int64_t N,
                                     int layout, int64_t K_pad, int8_t* __restrict__ out) {
    const int64_t total = K * N;
    const int64_t col_bytes = K_pad / 8;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        int64_t k, n;
        if (layout == TBN_LAYOUT_KN) { k = t / N; n = t % N; }
        else { n = t / K; k = t % K; }
        const uint32_t bit = (packed[n * col_bytes + (k >> 3)] >> (k & 7)) & 1u;
        out[t] = bit ? int8_t(-1) : int8_t(1);
    }
}

// ---- 2-bit ternary packing ---------------------------------------------------

__device__ __forceinline__ uint32_t ternary_code(int8_t v) {
    return (v == -1) ? 0u : ((v == 1) ? 2u : 1u);
}

__global__ void pack_ternary2_kernel(const int8_t* __restrict__ t, int64_t n,
                                     uint8_t* __restrict__ packed) {
    const int64_t bytes = (n + 3) / 4;
    for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < bytes;
         b += (int64_t)gridDim.x * blockDim.x) {
        uint32_t v = 0;  // a fresh TernaryPackedWeights buffer is zero (code 00)
        for (int j = 0; j < 4; ++j) {
            const int64_t i = b * 4 + j;
            if (i < n) v |= ternary_code(t[i]) << (2 * j);
        }
        packed[b] = static_cast<uint8_t>(v);
    }
}

__global__ void unpack_ternary2_kernel(const uint8_t* __restrict__ packed, int64_t n,
                                       int8_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t code = (packed[i >> 2] >> ((i & 3) * 2)) & 3u;
        out[i] = (code == 0u) ? int8_t(-1) : ((code == 2u) ? int8_t(1) : int8_t(0));
    }
}

struct TernaryBytes {
    const int8_t* p;
    __device__ uint32_t code(int64_t idx) const { return ternary_code(p[idx]); }
};
struct TernaryFloat {
    const float* p;
    float lo, hi;
    __device__ uint32_t code(int64_t idx) const {
        const float v = p[idx];
        return (v < lo) ? 0u : ((v > hi) ? 2u : 1u);
    }
};

// GEMM layout: flat 2-bit codes of W^T[N_pad, K_pad]; word (n, wi) holds
// k = 16*wi .. 16*wi+15 of column n, padding encodes 0 (code 01).
template <class Src>
__global__ void pack_ternary_kernel(Src src, int64_t K, int64_t N, int layout, int64_t K_pad,
                                    int64_t N_pad, uint32_t* __restrict__ packed) {
    const int64_t words_per_col = K_pad / 16;
    const int64_t total = N_pad * words_per_col;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        int64_t n, wi;
        if (layout == TBN_LAYOUT_KN) { n = t % N_pad; wi = t / N_pad; }
        else { wi = t % words_per_col; n = t / words_per_col; }
        uint32_t word = 0x55555555u;  // all zeros (code 01)
        if (n < N) {
            word = 0;
            const int64_t k0 = wi * 16;
#pragma unroll 4
            for (int j = 0; j < 16; ++j) {
                const int64_t k = k0 + j;
                uint32_t c = 1u;
                if (k < K) c = src.code((layout == TBN_LAYOUT_KN) ? k * N + n : n * K + k);
                word |= c << (2 * j);
            }
        }
        packed[n * words_per_col + wi] = word;
    }
}

int check_pack_dims(int64_t K, int64_t N, int layout, int64_t K_pad, int64_t N_pad,
                    int k_multiple) {
    TBN_REQUIRE(K >= 0 && N >= 0, TBN_INVALID_SHAPE, "K and N must be non-negative");
    TBN_REQUIRE(layout == TBN_LAYOUT_KN || layout == TBN_LAYOUT_NK, TBN_INVALID_ARGUMENT,
                "layout must be TBN_LAYOUT_KN or TBN_LAYOUT_NK");
    TBN_REQUIRE(K_pad >= K && N_pad >= N, TBN_INVALID_SHAPE, "K_pad/N_pad smaller than K/N");
    TBN_REQUIRE(K_pad % k_multiple == 0, TBN_INVALID_SHAPE,
                "K_pad must be a multiple of " + std::to_string(k_multiple));
    return TBN_SUCCESS;
}

}  // namespace

using tbn_hip::check_launch;
using tbn_hip::stream_of;

extern "C" {

int tbn_hip_quantize_to_binary_f32(const float* w, int64_t n, float threshold, uint8_t* out,
                                   tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    TBN_REQUIRE(n == 0 || (w && out), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (n == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(quantize_binary_f32_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                       stream_of(stream), w, n, threshold, out);
    return check_launch("quantize_to_binary_f32");
}

int tbn_hip_quantize_to_binary_i8(const int8_t* w, int64_t n, uint8_t* out, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    TBN_REQUIRE(n == 0 || (w && out), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (n == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(quantize_binary_i8_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                       stream_of(stream), w, n, out);
    return check_launch("quantize_to_binary_i8");
}

int tbn_hip_quantize_to_ternary_f32(const float* w, int64_t n, float lo, float hi, int8_t* out,
                                    tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    TBN_REQUIRE(n == 0 || (w && out), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (n == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(quantize_ternary_f32_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                       stream_of(stream), w, n, lo, hi, out);
    return check_launch("quantize_to_ternary_f32");
}

int tbn_hip_sign_ge0_f32(const float* w, int64_t n, uint8_t* out, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    TBN_REQUIRE(n == 0 || (w && out), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (n == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(sign_ge0_kernel, dim3(grid_for(n)), dim3(kThreads), 0, stream_of(stream),
                       w, n, out);
    return check_launch("sign_ge0_f32");
}

int tbn_hip_channel_mean_abs(const float* w, int64_t channels, int64_t per_channel, float* scale,
                             tbn_stream_t stream) {
    TBN_REQUIRE(channels >= 0 && per_channel > 0, TBN_INVALID_SHAPE,
                "channels must be >= 0 and per_channel > 0");
    TBN_REQUIRE(channels == 0 || (w && scale), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (channels == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(channel_mean_abs_kernel, dim3(tbn_hip::ceil_div(channels, 64)), dim3(256),
                       0, stream_of(stream), w, channels, per_channel, scale);
    return check_launch("channel_mean_abs");
}

int tbn_hip_pack_binary(const uint8_t* bin, int64_t K, int64_t N, int layout, int64_t K_pad,
                        int64_t N_pad, uint8_t* packed, tbn_stream_t stream) {
    int rc = check_pack_dims(K, N, layout, K_pad, N_pad, 64);
    if (rc) return rc;
    TBN_REQUIRE(N_pad % 8 == 0, TBN_INVALID_SHAPE, "N_pad must be a multiple of 8");
    TBN_REQUIRE(packed && (K * N == 0 || bin), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const int64_t words = N_pad * (K_pad / 32);
    if (words == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(pack_binary_kernel<BinaryBytes>, dim3(grid_for(words)), dim3(kThreads), 0,
                       stream_of(stream), BinaryBytes{bin}, K, N, layout, K_pad, N_pad,
                       reinterpret_cast<uint32_t*>(packed));
    return check_launch("pack_binary");
}

int tbn_hip_quantize_pack_binary_f32(const float* w, int64_t K, int64_t N, int layout,
                                     int sign_rule, float threshold, int64_t K_pad,
                                     int64_t N_pad, uint8_t* packed, tbn_stream_t stream) {
    int rc = check_pack_dims(K, N, layout, K_pad, N_pad, 64);
    if (rc) return rc;
    TBN_REQUIRE(N_pad % 8 == 0, TBN_INVALID_SHAPE, "N_pad must be a multiple of 8");
    TBN_REQUIRE(sign_rule == TBN_SIGN_GT_THRESHOLD || sign_rule == TBN_SIGN_GE_ZERO ||
                    sign_rule == TBN_SIGN_GEMM_SAMPLED,
                TBN_INVALID_ARGUMENT, "unknown sign rule");
    TBN_REQUIRE(packed && (K * N == 0 || w), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const int64_t words = N_pad * (K_pad / 32);
    if (words == 0) return tbn_hip::ok();
    uint32_t* out = reinterpret_cast<uint32_t*>(packed);
    if (sign_rule == TBN_SIGN_GT_THRESHOLD)
        hipLaunchKernelGGL(pack_binary_kernel<FloatGT>, dim3(grid_for(words)), dim3(kThreads), 0,
                           stream_of(stream), FloatGT{w, threshold}, K, N, layout, K_pad, N_pad,
                           out);
    else if (sign_rule == TBN_SIGN_GE_ZERO)
        hipLaunchKernelGGL(pack_binary_kernel<FloatGE0>, dim3(grid_for(words)), dim3(kThreads), 0,
                           stream_of(stream), FloatGE0{w}, K, N, layout, K_pad, N_pad, out);
    else
        hipLaunchKernelGGL(pack_binary_kernel<FloatSampled>, dim3(grid_for(words)), dim3(kThreads), 0,
                           stream_of(stream), FloatSampled{w, false}, K, N, layout, K_pad, N_pad, out);
    return check_launch("quantize_pack_binary_f32");
}

int tbn_hip_unpack_binary(const uint8_t* packed, int64_t K, int64_t N, int layout, int64_t K_pad,
                          int8_t* out, tbn_stream_t stream) {
    int rc = check_pack_dims(K, N, layout, K_pad, N, 8);
    if (rc) return rc;
    TBN_REQUIRE(K * N == 0 || (packed && out), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (K * N == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(unpack_binary_kernel, dim3(grid_for(K * N)), dim3(kThreads), 0,
                       stream_of(stream), packed, K, N, layout, K_pad, out);
    return check_launch("unpack_binary");
}

int tbn_hip_pack_ternary2(const int8_t* t, int64_t n, uint8_t* packed, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    TBN_REQUIRE(n == 0 || (t && packed), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (n == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(pack_ternary2_kernel, dim3(grid_for((n + 3) / 4)), dim3(kThreads), 0,
                       stream_of(stream), t, n, packed);
    return check_launch("pack_ternary2");
}

int tbn_hip_unpack_ternary2(const uint8_t* packed, int64_t n, int8_t* out, tbn_stream_t stream) {
    TBN_REQUIRE(n >= 0, TBN_INVALID_SHAPE, "n must be non-negative");
    TBN_REQUIRE(n == 0 || (packed && out), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    if (n == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(unpack_ternary2_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                       stream_of(stream), packed, n, out);
    return check_launch("unpack_ternary2");
}

int tbn_hip_pack_ternary(const int8_t* t, int64_t K, int64_t N, int layout, int64_t K_pad,
                         int64_t N_pad, uint8_t* packed, tbn_stream_t stream) {
    int rc = check_pack_dims(K, N, layout, K_pad, N_pad, 32);
    if (rc) return rc;
    TBN_REQUIRE(packed && (K * N == 0 || t), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const int64_t words = N_pad * (K_pad / 16);
    if (words == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(pack_ternary_kernel<TernaryBytes>, dim3(grid_for(words)), dim3(kThreads),
                       0, stream_of(stream), TernaryBytes{t}, K, N, layout, K_pad, N_pad,
                       reinterpret_cast<uint32_t*>(packed));
    return check_launch("pack_ternary");
}

int tbn_hip_quantize_pack_ternary_f32(const float* w, int64_t K, int64_t N, int layout, float lo,
                                      float hi, int64_t K_pad, int64_t N_pad, uint8_t* packed,
                                      tbn_stream_t stream) {
    int rc = check_pack_dims(K, N, layout, K_pad, N_pad, 32);
    if (rc) return rc;
    TBN_REQUIRE(packed && (K * N == 0 || w), TBN_INVALID_ARGUMENT, "null pointer");
    TBN_DEVICE_GUARD();
    const int64_t words = N_pad * (K_pad / 16);
    if (words == 0) return tbn_hip::ok();
    hipLaunchKernelGGL(pack_ternary_kernel<TernaryFloat>, dim3(grid_for(words)), dim3(kThreads),
                       0, stream_of(stream), TernaryFloat{w, lo, hi}, K, N, layout, K_pad, N_pad,
                       reinterpret_cast<uint32_t*>(packed));
    return check_launch("quantize_pack_ternary_f32");
}

}  // extern "C"
