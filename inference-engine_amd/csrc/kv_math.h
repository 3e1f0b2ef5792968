// Per-row arithmetic of the int8 KV writes, shared by the kernels that write the cache
// (kv_write.hip) and by the decode attention launch that writes the new token itself
// (decode_attention.hip), so both produce the same bits. IEEE single-precision operations in
// the stated order, no contraction into fused multiply-add.
#pragma once

#include "ie_common.h"

namespace ie {

// clamp(rint(x / s), -127, 127); x / s is an IEEE division, rint rounds half to even.
__device__ __forceinline__ int32_t quant1(float x, float s) {
    float r = rintf(x / s);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return static_cast<int32_t>(r);
}

// RMSNorm then RoPE of one head row, shared by the decode write and the prefill norm/rope
// (kernels.py:414-436 and :582-646 compute the same thing): lane i holds channels i and i + 64
// (the pair RoPE rotates); the sum of squares in the fixed butterfly order,
// rstd = 1 / sqrt(ss / 128 + eps), x * rstd * w, then the rotation with the row's cos/sin.
// IEEE single-precision operations, no contraction.
// The three parts: the row's sum of squares (every lane gets it), rstd from it, and the
// normalization and rotation of the lane's two channels.
__device__ __forceinline__ float row_sumsq(float x1, float x2) {
#pragma clang fp contract(off)
    return wave_sum_butterfly(x1 * x1) + wave_sum_butterfly(x2 * x2);
}
__device__ __forceinline__ float row_rstd(float ss, float eps) {
#pragma clang fp contract(off)
    const float var = ss / 128.0f + eps;
    return 1.0f / sqrtf(var);
}
__device__ __forceinline__ void row_norm_rope(float x1, float x2, float rstd, float w1, float w2,
                                              float cs, float sn, float& o1, float& o2) {
#pragma clang fp contract(off)
    x1 = (x1 * rstd) * w1;
    x2 = (x2 * rstd) * w2;
    o1 = (x1 * cs) - (x2 * sn);
    o2 = (x1 * sn) + (x2 * cs);
}
__device__ __forceinline__ void norm_rope_row(float x1, float x2, float w1, float w2, float cs,
                                              float sn, float eps, float& o1, float& o2) {
    row_norm_rope(x1, x2, row_rstd(row_sumsq(x1, x2), eps), w1, w2, cs, sn, o1, o2);
}

// Symmetric int8 of one head row held two channels per lane (lane i: channels i and i + 64):
// scale = max(amax, 1e-6) / 127 over the row (kernels.py:459-480), q = quant1(x, scale).
// Returns the scale; every lane gets it.
__device__ __forceinline__ float quantize_row_wave(float x1, float x2, int32_t& q1, int32_t& q2) {
#pragma clang fp contract(off)
    const float a = wave_max(fmaxf(fabsf(x1), fabsf(x2)));
    const float s = fmaxf(a, 1e-6f) / 127.0f;
    q1 = quant1(x1, s);
    q2 = quant1(x2, s);
    return s;
}

}  // namespace ie
