/*
 * tbn_oracle.h -- CPU oracle for the tbn quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the C++
 * host runtime) links, loads or calls this code.  Only tests/, the smoke()
 * entry and the cpu_baseline leg of bench.py use it, and only as the checker
 * or as the timed CPU baseline.
 *
 * Every function restates an algorithm of Babushkin05/fast-arm-tbcnn; the
 * file:line it follows is cited in tbn_oracle.c.  Conventions:
 *   - BINARY byte tensors: 1 means +1, any other byte means -1
 *     (tbn-runtime/include/tbn/runtime/types.hpp:86-87,
 *      tbn-runtime/src/operators/quantized_gemm_neon.cpp:205).
 *   - BinaryMatrix packed layout: column-major along K, column n occupies
 *     K_pad/8 bytes, value at k is bit (k&7) of byte (k>>3), bit 1 means -1,
 *     padding is +1 (GeMM/05-final/GeMM.cpp:114-151).
 *   - 2-bit ternary codes: flat index i -> byte i>>2, shift (i&3)*2,
 *     00=-1, 01=0, 10=+1, 11 decodes to 0
 *     (tbn-runtime/include/tbn/memory/packed_weights.hpp:35-71).
 *
 * Return codes follow tbn::ErrorCode (tbn-runtime/include/tbn/utils/errors.hpp:10-22).
 */
#ifndef TBN_ORACLE_H
#define TBN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TBO_OK = 0,
    TBO_INVALID_ARGUMENT = -1,
    TBO_INVALID_SHAPE = -7
};

/* ---- quantization and sign rules ------------------------------------- */
void tbo_quantize_to_binary_f32(const float* w, int64_t n, float thr, uint8_t* out);
void tbo_quantize_to_binary_i8(const int8_t* w, int64_t n, uint8_t* out);
void tbo_quantize_to_ternary_f32(const float* w, int64_t n, float lo, float hi, int8_t* out);
void tbo_sign_ge0_f32(const float* w, int64_t n, uint8_t* out);
void tbo_channel_mean_abs(const float* w, int64_t channels, int64_t per_channel, float* scale);
int  tbo_already_binary(const float* w, int64_t channels, int64_t per_channel, const float* scale);

/* ---- packing ------------------------------------------------------------ */
int  tbo_binary_matrix_pack(const int8_t* data, uint32_t rows, uint32_t cols, uint8_t* bits);
int  tbo_pack_binary_kn(const uint8_t* bin, int64_t K, int64_t N, int64_t K_pad, int64_t N_pad,
                        uint8_t* packed);
int  tbo_pack_binary_nk(const uint8_t* bin, int64_t N, int64_t K, int64_t K_pad, int64_t N_pad,
                        uint8_t* packed);
void tbo_ternary_pack2(const int8_t* t, int64_t n, uint8_t* packed);
int8_t tbo_ternary_get2(const uint8_t* packed, int64_t i);
int  tbo_pack_ternary_kn(const int8_t* t, int64_t K, int64_t N, int64_t K_pad, int64_t N_pad,
                         uint8_t* packed);
int  tbo_pack_ternary_nk(const int8_t* t, int64_t N, int64_t K, int64_t K_pad, int64_t N_pad,
                         uint8_t* packed);

/* ---- float x binary / float x ternary GEMM (mode F32) ------------------- */
void tbo_gemm_f32_binary(const float* A, int64_t lda, int64_t M, int64_t K,
                         const uint8_t* packed, int64_t K_pad, int64_t N,
                         const float* scale, float alpha, const float* bias, int relu,
                         float* C, int64_t ldc);
void tbo_gemm_f64_binary(const float* A, int64_t lda, int64_t M, int64_t K,
                         const uint8_t* packed, int64_t K_pad, int64_t N,
                         const float* scale, float alpha, const float* bias, int relu,
                         double* C, int64_t ldc);
void tbo_gemm_f32_ternary(const float* A, int64_t lda, int64_t M, int64_t K,
                          const uint8_t* packed, int64_t K_pad, int64_t N,
                          const float* scale, float alpha, const float* bias, int relu,
                          float* C, int64_t ldc);
void tbo_gemm_f64_ternary(const float* A, int64_t lda, int64_t M, int64_t K,
                          const uint8_t* packed, int64_t K_pad, int64_t N,
                          const float* scale, float alpha, const float* bias, int relu,
                          double* C, int64_t ldc);
void tbo_qlinear_matmul_binary_naive(const float* A, int64_t M, int64_t K,
                                     const uint8_t* bin, int64_t N, float scale, float* out);

/* ---- fp32 operators ------------------------------------------------------ */
int  tbo_conv2d_f32(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                    const float* w, int64_t M, int64_t kh, int64_t kw,
                    const float* bias,
                    int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                    float* y);
int  tbo_conv2d_f64(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                    const float* w, int64_t M, int64_t kh, int64_t kw,
                    const float* bias,
                    int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                    double* y);
int  tbo_maxpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                   int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                   int64_t dh, int64_t dw, int ceil_mode, float* y, int64_t* out_hw);
void tbo_global_avgpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, float* y);
int  tbo_avgpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                   int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                   int64_t dh, int64_t dw, int ceil_mode, int count_include_pad, float* y,
                   int64_t* out_hw);
void tbo_global_maxpool2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, float* y);
void tbo_gemm_f32_blocked(const float* A, const float* B, const float* Cin, int c_is_1d,
                          int64_t M, int64_t K, int64_t N, float alpha, float beta,
                          int transA, int transB, float* out);

/* ---- TBN mode: ternarized activations x binary popcount GEMM ------------ */
int  tbo_ternary_matrix_pack_from_float(const float* a, int64_t lda, int64_t M, int64_t K,
                                        uint32_t rows, uint32_t cols, float lo, float hi,
                                        uint8_t* pos, uint8_t* neg);
int  tbo_tbn_gemm(const uint8_t* pos, const uint8_t* neg, const uint8_t* bits,
                  uint32_t m, uint32_t n, uint32_t k,
                  uint32_t mblk, uint32_t nblk, uint32_t kblk, uint32_t mmk, uint32_t nmk,
                  int32_t* C);
int  tbo_qlinear_matmul_binary_tbn(const float* A, int64_t M, int64_t K,
                                   const uint8_t* bin, int64_t N, float scale,
                                   uint32_t mblk, uint32_t nblk, uint32_t kblk,
                                   uint32_t mmk, uint32_t nmk, float* out);
int  tbo_im2col_ternary_packed(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                               int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                               int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                               uint32_t m_pad, uint32_t k_pad, float lo, float hi,
                               uint8_t* pos, uint8_t* neg);

#ifdef __cplusplus
}
#endif
#endif /* TBN_ORACLE_H */
