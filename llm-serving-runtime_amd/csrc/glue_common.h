// Device helpers shared by the decode-step glue kernels and the fused QKV + RoPE GEMM.
#pragma once

#include "common.h"

namespace mx {
namespace glue {

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

__device__ __forceinline__ half8v as_h8(uint4 v) { return __builtin_bit_cast(half8v, v); }
__device__ __forceinline__ uint4 as_u4(half8v v) { return __builtin_bit_cast(uint4, v); }

// Where token `pos` of row `b` lives in the pool, or -1 when its logical block is past the
// table or its physical id is outside the pool (the token is then skipped and flagged).
__device__ __forceinline__ int64_t slot_offset(const int32_t* bt, int64_t bt_sb, int max_blocks, int b, int pos,
                                               int bs, int num_pool_blocks, int64_t sblk, int64_t shead, int head,
                                               int D) {
    if (pos < 0) return -1;
    const int lb = pos / bs;
    if (lb >= max_blocks) return -1;
    const int phys = bt[(int64_t)b * bt_sb + lb];
    if (phys < 0 || phys >= num_pool_blocks) return -1;
    return (int64_t)phys * sblk + (int64_t)head * shead + (int64_t)(pos - lb * bs) * D;
}

// Rotate-half RoPE of one pair (x1 at dim i, x2 at dim i + D/2) with cs = (cos, sin) of
// frequency i at the token's position (transformers' apply_rotary_pos_emb: x * cos +
// rotate_half(x) * sin). Each output is one fp32 fma of a rounded product, rounded once
// more to fp16; pinned so that every kernel using this rounds identically.
// Returns (o1, o2).
__device__ __forceinline__ half2v rope_rotate(_Float16 x1, _Float16 x2, float2 cs) {
    const float a = (float)x1, b = (float)x2;
    return half2v{(_Float16)pin_f32(__builtin_fmaf(a, cs.x, -pin_f32(b * cs.y))),
                  (_Float16)pin_f32(__builtin_fmaf(b, cs.x, pin_f32(a * cs.y)))};
}

}  // namespace glue
}  // namespace mx
