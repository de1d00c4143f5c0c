// attention_rope.h — the whole-prompt attention's own query rotation
// (attention.hip), for the forward (model.hip).
#pragma once
#include "internal.h"

namespace ditch {

// RoPE of the queries applied as the whole-prompt kernel loads them, in
// place of the RoPE kernel's pass over q (model.zig:4253-4295): head_dim
// 128 rotated whole in neox order (element d with d + 64), no query head
// norm; cos_t / sin_t [rope_len][64], positions past rope_len - 1 use its
// last row. The per-block kernel, which takes the rows when they are not
// dense, reads q as the RoPE kernel left it (rotated).
struct AttnRope {
    const float *cos_t = nullptr, *sin_t = nullptr;
    int64_t rope_len = 0;
};

// launch_attention_mfma with the queries' rotation in the whole-prompt
// kernel (a.dense set, a.hd == 128).
void launch_attention_mfma_rope(const AttnArgs &a, const AttnRope &rope, int64_t kv_heads, hipStream_t s);

}  // namespace ditch
