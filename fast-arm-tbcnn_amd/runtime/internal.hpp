// Helpers shared by the operator layer and the Session compiler.
#pragma once

#include "tbn/types.hpp"

namespace tbn {
namespace detail {

// Broadcast view of the Session's Add cases (model.hpp:905-1037) as
// a[outer, inner, rest] + b[inner] (b broadcast over outer and rest).  Throws
// InvalidShapeError for other shapes.  [N] + [M, N] must be swapped first.
void add_view(const Shape& a, const Shape& b, int64_t& outer, int64_t& inner, int64_t& rest);

inline int64_t ceil_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

}  // namespace detail
}  // namespace tbn
