// Wide-tile float x binary GEMM for large shapes (gemm_wide.hip), used by the
// quantized GEMM entry points when the shape fills the chip with its tiles.
#pragma once

#include <string>

#include "common.hpp"

namespace tbn_hip {

struct WideGemmArgs {
    const float* A;
    int64_t lda;
    int M, N, K;
    const uint8_t* packed;  // BinaryMatrix columns, col_bytes each
    int64_t col_bytes;
    int N_pad;
    float* C;
    int64_t ldc;
    const float* scale;  // per column, may be null
    float alpha;
    const float* bias;   // per column, may be null
    const float* cin;    // null, [N] (cin_1d) or [M, N]
    int cin_1d;
    float beta;
    int flags;
};

// True when the wide kernel takes this GEMM: enough tiles (with K splits) to
// fill the chip, 16-byte aligned fp32 rows and 16-byte multiple packed columns.
// `packed` holds BinaryMatrix columns, or 2-bit ternary columns when ternary.
bool gemm_wide_fits(const WideGemmArgs& a, bool ternary);
// Runs it; shapes with few tiles split K over blocks, the last block of each
// tile adding the splits in split order (stream workspace of splits * M * N
// floats).
int gemm_wide(const WideGemmArgs& a, bool ternary, hipStream_t stream);
// The kernel gemm_wide launches for this shape now (tuning controls
// included), as a profiler names it.
std::string gemm_wide_kernel_name(const WideGemmArgs& a, bool ternary);

}  // namespace tbn_hip
