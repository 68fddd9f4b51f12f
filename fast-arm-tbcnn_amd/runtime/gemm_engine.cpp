// The reference's GeMM engine API (GeMM/05-final/GeMM.cpp) over libtbn_hip.so:
// argument checks and exceptions on the host, as the reference throws them;
// packing and the ternary x binary product as HIP kernels on the current
// stream, with the host-side packed matrices uploaded per call and results
// copied back.  Compiled as C++20 (std::span in the API).
#include "tbn/gemm_engine.hpp"

#include <cstring>
#include <stdexcept>
#include <string>

#include "tbn/device.hpp"
#include "tbn/errors.hpp"
#include "tbn_hip.h"

namespace tbn {

namespace {

tbn_stream_t stream() { return device::current_stream(); }

// A device copy of host bytes (empty for zero bytes).
Tensor upload(const void* data, size_t bytes) {
    return Tensor({static_cast<int64_t>(bytes)}, DataType::UINT8, data, DeviceType::HIP);
}

Tensor device_bytes(size_t bytes) {
    return Tensor::empty({static_cast<int64_t>(bytes)}, DataType::UINT8, DeviceType::HIP);
}

std::vector<std::uint8_t> download(const Tensor& t) { return t.to_vector<std::uint8_t>(); }

// Plane / column byte counts of the views the engine reads, checked against
// the dimensions so no kernel reads past a view.
void check_views(const TernaryMatrixView& A, const BinaryMatrixView& B) {
    const size_t a_bytes = static_cast<size_t>(A.rows) * (A.cols / 8);
    if (A.positive.size() < a_bytes || A.negative.size() < a_bytes)
        throw std::invalid_argument("GemmEngine: ternary view holds fewer bytes than rows x cols / 8");
    if (B.bits.size() < static_cast<size_t>(B.cols) * (B.rows / 8))
        throw std::invalid_argument("GemmEngine: binary view holds fewer bytes than rows x cols / 8");
    // The reference reads B's columns with A's row length (GeMM.cpp:303-363)
    // and so needs the shared dimension to agree.
    if (A.cols != B.rows)
        throw std::invalid_argument("GemmEngine: A cols (" + std::to_string(A.cols) + ") != B rows (" +
                                    std::to_string(B.rows) + ")");
}

// Runs the product of two views on the device: int32 C [m, k], or when
// `scaled` float(C) * scale for the first m_out rows and n_out columns.
Tensor device_product(const TernaryMatrixView& A, const BinaryMatrixView& B, bool scaled, uint32_t m_out,
                      uint32_t n_out, float scale) {
    const size_t a_bytes = static_cast<size_t>(A.rows) * (A.cols / 8);
    Tensor pos = upload(A.positive.data(), a_bytes);
    Tensor neg = upload(A.negative.data(), a_bytes);
    Tensor bits = upload(B.bits.data(), static_cast<size_t>(B.cols) * (B.rows / 8));
    if (!scaled) {
        Tensor C = Tensor::empty({static_cast<int64_t>(A.rows), static_cast<int64_t>(B.cols)}, DataType::INT32,
                                 DeviceType::HIP);
        check_status(tbn_hip_tbn_gemm(pos.typed_data<uint8_t>(), neg.typed_data<uint8_t>(),
                                      bits.typed_data<uint8_t>(), A.rows, A.cols, B.cols, C.typed_data<int32_t>(),
                                      stream()),
                     "GemmEngine::compute");
        return C;
    }
    Tensor out = Tensor::empty({static_cast<int64_t>(m_out), static_cast<int64_t>(n_out)}, DataType::FLOAT32,
                               DeviceType::HIP);
    check_status(tbn_hip_tbn_gemm_scaled(pos.typed_data<uint8_t>(), neg.typed_data<uint8_t>(),
                                         bits.typed_data<uint8_t>(), m_out, A.cols, B.cols, n_out, scale,
                                         out.typed_data<float>(), n_out, stream()),
                 "qlinear_matmul_binary_blocked_prepacked");
    return out;
}

}  // namespace

TernaryMatrix TernaryMatrix::pack(std::span<const std::int8_t> data, std::uint32_t rows, std::uint32_t cols) {
    if (rows % 8 != 0) throw std::invalid_argument("TernaryMatrix: rows must be multiple of 8");
    if (cols % 64 != 0) throw std::invalid_argument("TernaryMatrix: cols must be multiple of 64");
    if (data.size() != static_cast<size_t>(rows) * cols)
        throw std::invalid_argument("TernaryMatrix: data size doesn't match dimensions");
    for (std::int8_t v : data)
        if (v < -1 || v > 1) throw std::invalid_argument("TernaryMatrix: values must be -1, 0, or +1");
    const size_t bytes = static_cast<size_t>(rows) * (cols / 8);
    if (bytes == 0) return TernaryMatrix({}, {}, rows, cols);
    Tensor src = upload(data.data(), data.size());
    Tensor pos = device_bytes(bytes), neg = device_bytes(bytes);
    check_status(tbn_hip_ternary_pack_i8(src.typed_data<int8_t>(), cols, rows, cols, rows, cols,
                                         pos.typed_data<uint8_t>(), neg.typed_data<uint8_t>(), stream()),
                 "TernaryMatrix::pack");
    return TernaryMatrix(download(pos), download(neg), rows, cols);
}

TernaryMatrix TernaryMatrix::pack_from_float(const float* data, std::uint32_t rows, std::uint32_t cols,
                                             float threshold_low, float threshold_high) {
    if (rows % 8 != 0) throw std::invalid_argument("TernaryMatrix: rows must be multiple of 8");
    if (cols % 64 != 0) throw std::invalid_argument("TernaryMatrix: cols must be multiple of 64");
    const size_t bytes = static_cast<size_t>(rows) * (cols / 8);
    if (bytes == 0) return TernaryMatrix({}, {}, rows, cols);
    if (!data) throw std::invalid_argument("TernaryMatrix: null data");
    Tensor src = upload(data, static_cast<size_t>(rows) * cols * sizeof(float));
    Tensor pos = device_bytes(bytes), neg = device_bytes(bytes);
    check_status(tbn_hip_ternary_pack_f32(src.typed_data<float>(), cols, rows, cols, rows, cols, threshold_low,
                                          threshold_high, pos.typed_data<uint8_t>(), neg.typed_data<uint8_t>(),
                                          stream()),
                 "TernaryMatrix::pack_from_float");
    return TernaryMatrix(download(pos), download(neg), rows, cols);
}

BinaryMatrix BinaryMatrix::pack(std::span<const std::int8_t> data, std::uint32_t rows, std::uint32_t cols) {
    if (rows % 64 != 0) throw std::invalid_argument("BinaryMatrix: rows must be multiple of 64");
    if (cols % 8 != 0) throw std::invalid_argument("BinaryMatrix: cols must be multiple of 8");
    if (data.size() != static_cast<size_t>(rows) * cols)
        throw std::invalid_argument("BinaryMatrix: data size doesn't match dimensions");
    for (std::int8_t v : data)
        if (v != 1 && v != -1) throw std::invalid_argument("BinaryMatrix: values must be -1 or +1");
    const size_t bytes = static_cast<size_t>(cols) * (rows / 8);
    if (bytes == 0) return BinaryMatrix({}, rows, cols);
    // The byte packer marks every byte other than 1 as -1, so int8 +1 / -1
    // (0x01 / 0xFF) pack as they are: rows x cols row-major is layout KN.
    Tensor src = upload(data.data(), data.size());
    Tensor bits = device_bytes(bytes);
    check_status(tbn_hip_pack_binary(src.typed_data<uint8_t>(), rows, cols, TBN_LAYOUT_KN, rows, cols,
                                     bits.typed_data<uint8_t>(), stream()),
                 "BinaryMatrix::pack");
    return BinaryMatrix(download(bits), rows, cols);
}

Int32Matrix GemmEngine::compute(TernaryMatrixView A, BinaryMatrixView B, const TilingParams& params) {
    const std::uint32_t m = A.rows, n = A.cols, k = B.cols;
    params.validate(m, n, k);
    check_views(A, B);
    Int32Matrix C(m, k);
    if (C.size() > 0) {
        Tensor dc = device_product(A, B, false, 0, 0, 0.0f);
        device::copy_to_host(C.data().data(), dc.data(), C.size() * sizeof(std::int32_t));
    }
    last_flops_ = static_cast<std::uint64_t>(m) * n * k * 2;
    return C;
}

PackedBinaryWeights PackedBinaryWeights::from_int8(std::span<const std::int8_t> weights, std::uint32_t rows_raw,
                                                   std::uint32_t cols_raw, const TilingParams& tiling) {
    // GeMM.cpp:369-398: rows padded to 64 and columns to 8 with +1.
    if (weights.size() < static_cast<size_t>(rows_raw) * cols_raw)
        throw std::invalid_argument("PackedBinaryWeights: data size doesn't match dimensions");
    const std::uint32_t rows = (rows_raw + 63) / 64 * 64, cols = (cols_raw + 7) / 8 * 8;
    std::vector<std::int8_t> padded(static_cast<size_t>(rows) * cols, 1);
    for (std::uint32_t i = 0; i < rows_raw; ++i)
        std::memcpy(padded.data() + static_cast<size_t>(i) * cols, weights.data() + static_cast<size_t>(i) * cols_raw,
                    cols_raw);
    PackedBinaryWeights w;
    w.b_packed = BinaryMatrix::pack(padded, rows, cols);
    w.tiling = tiling;
    w.original_m = rows_raw;
    w.original_n = cols_raw;
    w.original_k = rows_raw;
    return w;
}

Tensor qlinear_matmul_binary_blocked_packed(const Tensor& a, const BinaryMatrix& b_packed, uint32_t n_orig,
                                            float scale, const TilingParams& params, float threshold_low,
                                            float threshold_high) {
    TBN_CHECK(a.dtype() == DataType::FLOAT32, InvalidArgumentError, "Input A must be FLOAT32");
    TBN_CHECK(a.shape().rank() == 2, InvalidShapeError, "Input A must be a 2D matrix");
    const int64_t M = a.shape().dims[0], K = a.shape().dims[1];
    const uint32_t k_pad = b_packed.rows(), n_pad = b_packed.cols();
    TBN_CHECK(K <= k_pad, InvalidShapeError,
              "A cols (" + std::to_string(K) + ") exceed the packed B rows (" + std::to_string(k_pad) + ")");
    TBN_CHECK(n_orig <= n_pad, InvalidShapeError,
              "n_orig (" + std::to_string(n_orig) + ") exceeds the packed B cols (" + std::to_string(n_pad) + ")");
    // The reference ternarizes A padded to ceil16(M) rows and runs the engine
    // on the padded shapes (quantized_gemm_neon.cpp:258-286): same checks.
    params.validate(static_cast<uint32_t>((M + 15) / 16 * 16), k_pad, n_pad);
    Tensor ad = a.on_device() ? a : a.to_device(DeviceType::HIP);
    Tensor out = Tensor::empty({M, static_cast<int64_t>(n_orig)}, DataType::FLOAT32, DeviceType::HIP);
    if (M > 0 && n_orig > 0) {
        const std::vector<std::uint8_t> bits(b_packed.view().bits.begin(), b_packed.view().bits.end());
        Tensor db = upload(bits.data(), bits.size());
        check_status(tbn_hip_qlinear_matmul_binary_tbn(ad.typed_data<float>(), K, M, K, db.typed_data<uint8_t>(),
                                                       k_pad, n_orig, n_pad, scale, threshold_low, threshold_high,
                                                       out.typed_data<float>(), n_orig, stream()),
                     "qlinear_matmul_binary_blocked_packed");
    }
    return a.on_device() ? out : out.to_device(DeviceType::CPU);
}

Tensor qlinear_matmul_binary_blocked_prepacked(const TernaryMatrix& a_packed, const BinaryMatrix& b_packed,
                                               uint32_t m_orig, uint32_t n_orig, float scale,
                                               const TilingParams& params) {
    const TernaryMatrixView A = a_packed.view();
    const BinaryMatrixView B = b_packed.view();
    params.validate(A.rows, A.cols, B.cols);
    check_views(A, B);
    TBN_CHECK(m_orig <= A.rows && n_orig <= B.cols, InvalidShapeError,
              "m_orig / n_orig exceed the packed matrices");
    if (m_orig == 0 || n_orig == 0)
        return Tensor({static_cast<int64_t>(m_orig), static_cast<int64_t>(n_orig)}, DataType::FLOAT32);
    return device_product(A, B, true, m_orig, n_orig, scale).to_device(DeviceType::CPU);
}

}  // namespace tbn
