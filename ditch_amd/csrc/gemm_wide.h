// gemm_wide.h — the mid-batch Q8_0 product (gemm_wide.hip).
#pragma once
#include "gemm_common.h"

namespace ditch {

// 32 <= n <= 256 tokens on Q8_0 weights with the tiled product's side words,
// two activation terms: the wide product takes the call.
bool wide_gemm_takes(const TileView &w, int64_t n, int xt, int64_t ldk);

// out[n][rows] (row stride ldo) = A fragments (split_kernel layout,
// xs[m16][kt][term][lane], ldk k tiles per 16-token block) . W^T + epilogue.
void launch_wide_gemm(const TileView &w, float *out, int64_t ldo, const void *xs, int64_t ldk, int64_t n,
                      const MatmulEpilogue &ep, hipStream_t s);

}  // namespace ditch
