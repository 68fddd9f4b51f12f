// tbn::TilingParams, the tiling of the reference's CPU GeMM engine
// (GeMM/05-final/GeMM.hpp:16-43).  The operator entry points accept it for
// source compatibility and ignore it (the GPU kernels choose their own tiles,
// and no shape is rejected for tiling reasons); GemmEngine::compute checks
// validate() as the reference does, so its callers see the same exceptions.
#pragma once

#include <cstdint>
#include <stdexcept>

namespace tbn {

struct TilingParams {
    uint32_t mblk = 64;  // outer block on rows
    uint32_t nblk = 64;  // outer block on columns
    uint32_t kblk = 128; // outer block on depth
    uint32_t mmk = 32;   // micro-kernel rows
    uint32_t nmk = 32;   // micro-kernel columns

    // The reference's constraints (GeMM.hpp:24-37), reference naming: m rows,
    // n shared dimension, k columns.
    void validate(uint32_t m, uint32_t n, uint32_t k) const {
        if (n % 128 != 0) throw std::invalid_argument("TilingParams: n must be multiple of 128 for NEON");
        if (kblk % 128 != 0) throw std::invalid_argument("TilingParams: kblk must be multiple of 128 for NEON");
        if (mmk == 0 || m % mmk != 0) throw std::invalid_argument("TilingParams: m must be multiple of mmk");
        if (nmk == 0 || k % nmk != 0) throw std::invalid_argument("TilingParams: k must be multiple of nmk");
    }

    static constexpr TilingParams default_128x128() noexcept { return TilingParams{}; }
};

}  // namespace tbn
