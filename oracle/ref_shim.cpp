// C entry points over the reference's own fp32 operators (tbn::conv2d,
// tbn::gemm, tbn::maxpool2d, tbn::avgpool2d, tbn::global_maxpool2d,
// tbn::global_avgpool2d), compiled from the
// reference sources by `make ref` into oracle/_ref/.  TEST INFRASTRUCTURE
// ONLY: tests/ use it to check the CPU oracle's restatements of these
// operators bit for bit.  Only the fp32 operator sources are built: the
// quantized path (GeMM/05-final/GeMM.cpp) includes <arm_neon.h>
// unconditionally and does not build on this host, so the GeMM symbols that
// conv2d.cpp / gemm.cpp reference for their binary variants stay unresolved
// and must never be called (load with RTLD_LAZY).
#include <cstdint>
#include <cstring>
#include <exception>

#include "tbn/operators/conv2d.hpp"
#include "tbn/operators/gemm.hpp"
#include "tbn/operators/pooling.hpp"

namespace {
tbn::Tensor host_tensor(const float* data, std::initializer_list<int64_t> dims) {
    return tbn::Tensor(tbn::Shape(dims), tbn::DataType::FLOAT32, data);
}
void copy_out(const tbn::Tensor& t, float* dst) { std::memcpy(dst, t.data(), t.data_size()); }
}  // namespace

extern "C" {

int ref_conv2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, const float* wt, int64_t m,
               int64_t kh, int64_t kw, const float* bias, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
               int64_t dh, int64_t dw, float* y) {
    try {
        tbn::Tensor X = host_tensor(x, {n, c, h, w});
        tbn::Tensor W = host_tensor(wt, {m, c, kh, kw});
        tbn::Tensor B = bias ? host_tensor(bias, {m}) : tbn::Tensor();
        tbn::Conv2DParams p(kh, kw, sh, sw, ph, pw, dh, dw, 1);
        copy_out(tbn::conv2d(X, W, bias ? &B : nullptr, p), y);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_gemm(const float* A, const float* B, const float* C, int c_is_1d, int64_t M, int64_t K, int64_t N,
             float alpha, float beta, int transA, int transB, float* out) {
    try {
        tbn::Tensor TA = transA ? host_tensor(A, {K, M}) : host_tensor(A, {M, K});
        tbn::Tensor TB = transB ? host_tensor(B, {N, K}) : host_tensor(B, {K, N});
        tbn::Tensor TC;
        if (C) TC = c_is_1d ? host_tensor(C, {N}) : host_tensor(C, {M, N});
        copy_out(tbn::gemm(TA, TB, C ? &TC : nullptr, alpha, beta, transA != 0, transB != 0), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_maxpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh, int64_t kw,
                  int64_t sh, int64_t sw, int64_t ph, int64_t pw, int ceil_mode, float* y, int64_t* out_hw) {
    try {
        tbn::Pool2DParams p(kh, kw, sh, sw, ph, pw);
        p.ceil_mode = ceil_mode != 0;
        tbn::Tensor r = tbn::maxpool2d(host_tensor(x, {n, c, h, w}), p);
        out_hw[0] = r.shape().dims[2];
        out_hw[1] = r.shape().dims[3];
        if (y) copy_out(r, y);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_avgpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh, int64_t kw,
                  int64_t sh, int64_t sw, int64_t ph, int64_t pw, int ceil_mode, int count_include_pad, float* y,
                  int64_t* out_hw) {
    try {
        tbn::Pool2DParams p(kh, kw, sh, sw, ph, pw);
        p.ceil_mode = ceil_mode != 0;
        p.count_include_pad = count_include_pad != 0;
        tbn::Tensor r = tbn::avgpool2d(host_tensor(x, {n, c, h, w}), p);
        out_hw[0] = r.shape().dims[2];
        out_hw[1] = r.shape().dims[3];
        if (y) copy_out(r, y);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_global_maxpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, float* y) {
    try {
        copy_out(tbn::global_maxpool2d(host_tensor(x, {n, c, h, w})), y);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_global_avgpool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, float* y) {
    try {
        copy_out(tbn::global_avgpool2d(host_tensor(x, {n, c, h, w})), y);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

}  // extern "C"
