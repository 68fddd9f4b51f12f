// Helpers shared by the operator layer and the Session compiler.
#pragma once

#include <functional>

#include <vector>

#include "tbn/tensor.hpp"
#include "tbn/types.hpp"
#include "tbn_hip.h"

namespace tbn {
namespace detail {

// Broadcast view of the Session's Add cases (model.hpp:905-1037) as
// a[outer, inner, rest] + b[inner] (b broadcast over outer and rest).  Throws
// InvalidShapeError for other shapes.  [N] + [M, N] must be swapped first.
void add_view(const Shape& a, const Shape& b, int64_t& outer, int64_t& inner, int64_t& rest);

inline int64_t ceil_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Inference BatchNormalization (ONNX: y = (x - mean) / sqrt(var + eps) * scale
// + B) as y = x * k + t per channel: k = scale / sqrt(var + eps) and
// t = B - mean * k, formed in double and rounded once.
void batch_norm_affine(const Tensor& scale, const Tensor& B, const Tensor& mean, const Tensor& var, float epsilon,
                       int64_t c, std::vector<float>& k, std::vector<float>& t);

// Output height and width of a conv descriptor (conv2d.cpp:96-101).
void conv_out_hw(const tbn_conv2d_desc& d, int64_t& OH, int64_t& OW);

// Floats of device workspace run_grouped_conv needs: none for a batch of one
// (every group's channels are contiguous), else one group's input and output
// slices.
int64_t grouped_conv_workspace(const tbn_conv2d_desc& d, int64_t groups);

// A grouped conv (groups > 1, more than one input channel per group) as one
// dense conv per group: `conv(g, xg, dg, yg)` runs group g on input slice xg
// (dg: the group's descriptor, c = C/groups, m = M/groups) into yg.  With a
// batch larger than one the slices are gathered into and scattered from
// `workspace` with tbn_hip_copy_channels.
void run_grouped_conv(const tbn_conv2d_desc& d, int64_t groups, const float* x, float* y, float* workspace,
                      const std::function<void(int64_t, const float*, const tbn_conv2d_desc&, float*)>& conv,
                      tbn_stream_t stream);

}  // namespace detail
}  // namespace tbn
