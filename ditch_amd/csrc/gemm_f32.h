// gemm_f32.h — products on f32 / f16 weights for n > 16 tokens (gemm_f32.hip).
#pragma once
#include "gemm_common.h"

namespace ditch {

bool f32_gemm_takes(const TileView &w, int64_t n);

// out[n][rows] = x . W^T + epilogue, exact products on the fp32 MFMA (plain
// products: no segments).
void launch_f32_gemm(const GemmParams &p, hipStream_t s);

}  // namespace ditch
