// ts_quant.h -- the INT4 quantizer's per-element steps, shared by the append kernel and the
// fused append in the decode kernel so both write bit-identical codes and scales.
//
// cpu_quantize (src/backend/bindless/test_int4_parity.rs:56-75): scale = max|x| / 7 (1 when
// max|x| == 0), code = clamp(round_half_away(x/scale) + 8, 1, 15); K is rotated first at its
// absolute position (src/ops/reference/rope.rs:186-196).  Every step is a separately rounded
// IEEE f32 operation (contraction is switched off inside these functions), so the including
// file's compile flags do not change the bits.
#pragma once
#include "ts_internal.h"

namespace ts {
namespace {

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Rotation of the pair (a, b) by (cos, sin) = cs, as rope.rs:193-194.  The pragma keeps the
// products rounded separately whatever -ffp-contract the including file is built with.
__device__ inline void rope_rotate(float &a, float &b, float2 cs) {
#pragma clang fp contract(off)
    // plain operators: under the pragma they carry no contraction flag (the __f*_rn library
    // wrappers do, and would be fused into FMAs)
    const float xc = a * cs.x, ys = b * cs.y;
    const float xs = a * cs.y, yc = b * cs.x;
    a = xc - ys;
    b = xs + yc;
}

__device__ inline float quant_scale(float max_abs) {
    return (max_abs == 0.0f) ? 1.0f : __fdiv_rn(max_abs, 7.0f);
}

// Rust `f32::round() as i32` followed by +8 and clamp(1, 15); NaN maps to 0 -> code 8.
__device__ inline uint32_t encode(float x, float scale) {
    float r = roundf(__fdiv_rn(x, scale));
    int q = (r != r) ? 0 : (int)fminf(fmaxf(r, -64.0f), 64.0f);
    q += 8;
    q = q < 1 ? 1 : (q > 15 ? 15 : q);
    return (uint32_t)q;
}

}  // namespace
}  // namespace ts
