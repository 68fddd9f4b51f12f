// The reference's ternary x binary GeMM engine API (GeMM/05-final/GeMM.hpp:
// 16-239) and the two operator entry points built on it
// (tbn-runtime/include/tbn/operators/quantized_gemm.hpp:69-87), so callers
// of the CPU engine (the reference's test_final.cpp, its bench, gemm.cpp)
// recompile unchanged.  Needs C++20 (std::span), as the reference's header
// does.
//
// The packed matrices stay host objects with the reference's layouts (two
// row-major bit planes for a TernaryMatrix, column-major bits with 1 = -1 for
// a BinaryMatrix); the packers and GemmEngine::compute run as HIP kernels of
// libtbn_hip.so on the current stream (operands uploaded per call, results
// copied back), with the reference's argument checks and exceptions
// (std::invalid_argument).  Results are the reference's integers, bit for bit.
#pragma once

#if __cplusplus < 202002L
#error "tbn/gemm_engine.hpp needs C++20 (std::span), like the reference's GeMM.hpp"
#endif

#include <cstdint>
#include <span>
#include <utility>
#include <vector>

#include "tensor.hpp"
#include "tiling.hpp"

namespace tbn {

// Non-owning view of a packed ternary matrix (two bit planes).
struct TernaryMatrixView {
    std::span<const std::uint8_t> positive;  // bits of +1 values
    std::span<const std::uint8_t> negative;  // bits of -1 values
    std::uint32_t rows{};
    std::uint32_t cols{};
};

// Non-owning view of a packed binary matrix (one bit plane).
struct BinaryMatrixView {
    std::span<const std::uint8_t> bits;
    std::uint32_t rows{};
    std::uint32_t cols{};
};

// Packed ternary matrix: rows x cols (rows % 8 == 0, cols % 64 == 0), row i
// holding cols/8 bytes per plane; bit j&7 of byte j>>3 is column j.
class TernaryMatrix {
public:
    TernaryMatrix() = default;

    // From int8 values in {-1, 0, +1}.
    [[nodiscard]] static TernaryMatrix pack(std::span<const std::int8_t> data, std::uint32_t rows,
                                            std::uint32_t cols);
    // From floats: v < threshold_low -> -1, v > threshold_high -> +1, else 0.
    [[nodiscard]] static TernaryMatrix pack_from_float(const float* data, std::uint32_t rows, std::uint32_t cols,
                                                       float threshold_low = -0.1f, float threshold_high = 0.1f);
    [[nodiscard]] static TernaryMatrix from_bitplanes(std::vector<std::uint8_t> positive,
                                                      std::vector<std::uint8_t> negative, std::uint32_t rows,
                                                      std::uint32_t cols) {
        return TernaryMatrix(std::move(positive), std::move(negative), rows, cols);
    }

    [[nodiscard]] std::uint32_t rows() const noexcept { return rows_; }
    [[nodiscard]] std::uint32_t cols() const noexcept { return cols_; }
    [[nodiscard]] TernaryMatrixView view() const noexcept { return {positive_, negative_, rows_, cols_}; }
    [[nodiscard]] bool empty() const noexcept { return positive_.empty(); }

private:
    TernaryMatrix(std::vector<std::uint8_t> positive, std::vector<std::uint8_t> negative, std::uint32_t rows,
                  std::uint32_t cols)
        : positive_(std::move(positive)), negative_(std::move(negative)), rows_(rows), cols_(cols) {}

    std::vector<std::uint8_t> positive_;
    std::vector<std::uint8_t> negative_;
    std::uint32_t rows_{};
    std::uint32_t cols_{};
};

// Packed binary matrix: rows x cols (rows % 64 == 0, cols % 8 == 0), column j
// holding rows/8 bytes; bit r&7 of byte r>>3 is 1 for -1.
class BinaryMatrix {
public:
    BinaryMatrix() = default;

    // From int8 values in {-1, +1}.
    [[nodiscard]] static BinaryMatrix pack(std::span<const std::int8_t> data, std::uint32_t rows,
                                           std::uint32_t cols);

    [[nodiscard]] std::uint32_t rows() const noexcept { return rows_; }
    [[nodiscard]] std::uint32_t cols() const noexcept { return cols_; }
    [[nodiscard]] BinaryMatrixView view() const noexcept { return {bits_, rows_, cols_}; }
    [[nodiscard]] bool empty() const noexcept { return bits_.empty(); }

private:
    BinaryMatrix(std::vector<std::uint8_t> bits, std::uint32_t rows, std::uint32_t cols)
        : bits_(std::move(bits)), rows_(rows), cols_(cols) {}

    std::vector<std::uint8_t> bits_;
    std::uint32_t rows_{};
    std::uint32_t cols_{};
};

// Row-major int32 result.
class Int32Matrix {
public:
    Int32Matrix() = default;
    explicit Int32Matrix(std::uint32_t rows, std::uint32_t cols)
        : data_(static_cast<std::size_t>(rows) * cols, 0), rows_(rows), cols_(cols) {}

    [[nodiscard]] std::int32_t& at(std::uint32_t row, std::uint32_t col) noexcept {
        return data_[static_cast<std::size_t>(row) * cols_ + col];
    }
    [[nodiscard]] std::int32_t at(std::uint32_t row, std::uint32_t col) const noexcept {
        return data_[static_cast<std::size_t>(row) * cols_ + col];
    }
    [[nodiscard]] std::uint32_t rows() const noexcept { return rows_; }
    [[nodiscard]] std::uint32_t cols() const noexcept { return cols_; }
    [[nodiscard]] std::span<std::int32_t> data() noexcept { return data_; }
    [[nodiscard]] std::span<const std::int32_t> data() const noexcept { return data_; }
    [[nodiscard]] std::size_t size() const noexcept { return data_.size(); }
    [[nodiscard]] bool empty() const noexcept { return data_.empty(); }
    // Sign of an entry: -1, 0 or +1.
    [[nodiscard]] std::int8_t sign_at(std::uint32_t row, std::uint32_t col) const noexcept {
        const std::int32_t v = at(row, col);
        return static_cast<std::int8_t>((v > 0) - (v < 0));
    }

private:
    std::vector<std::int32_t> data_;
    std::uint32_t rows_{};
    std::uint32_t cols_{};
};

// Weights packed once for reuse: rows padded to 64 and columns to 8 with +1.
struct PackedBinaryWeights {
    TernaryMatrix a_packed;
    BinaryMatrix b_packed;
    TilingParams tiling;
    std::uint32_t original_m{};
    std::uint32_t original_n{};
    std::uint32_t original_k{};

    [[nodiscard]] bool valid() const noexcept { return !b_packed.empty(); }
    [[nodiscard]] static PackedBinaryWeights from_int8(std::span<const std::int8_t> weights, std::uint32_t rows_raw,
                                                       std::uint32_t cols_raw, const TilingParams& tiling);
};

// C[m, k] = A[m, n] (ternary) x B[n, k] (binary), exact int32, reference
// naming (n is the shared dimension): sum over n of popcount(pos) -
// popcount(neg) per 64-bit word, on the MI355X's int8 matrix cores.
class GemmEngine {
public:
    GemmEngine() = default;
    [[nodiscard]] Int32Matrix compute(TernaryMatrixView A, BinaryMatrixView B, const TilingParams& params);
    [[nodiscard]] Int32Matrix compute(TernaryMatrixView A, BinaryMatrixView B) {
        return compute(A, B, TilingParams::default_128x128());
    }
    [[nodiscard]] std::uint64_t last_flops() const noexcept { return last_flops_; }

private:
    std::uint64_t last_flops_{};
};

// qlinear_matmul_binary's arithmetic with a pre-packed BinaryMatrix
// (quantized_gemm_neon.cpp:249-309): a [M, K] fp32 ternarized at
// (threshold_low, threshold_high), times b_packed (K <= rows), out[M, n_orig]
// = float(C) * scale.  The result lives where `a` lives (host in, host out).
// TilingParams is accepted and ignored, as by the other operators.
Tensor qlinear_matmul_binary_blocked_packed(const Tensor& a, const BinaryMatrix& b_packed, uint32_t n_orig,
                                            float scale, const TilingParams& params, float threshold_low = -0.1f,
                                            float threshold_high = 0.1f);

// Both operands pre-packed (quantized_gemm_neon.cpp:314-350): out[m_orig,
// n_orig] = float(a_packed x b_packed) * scale, a host tensor.
Tensor qlinear_matmul_binary_blocked_prepacked(const TernaryMatrix& a_packed, const BinaryMatrix& b_packed,
                                               uint32_t m_orig, uint32_t n_orig, float scale,
                                               const TilingParams& params);

}  // namespace tbn
