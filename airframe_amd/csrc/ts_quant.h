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

// v where keep, else zeros, component by component (a conditional on the float4 objects
// themselves would select between their addresses and put both in scratch memory).
__device__ inline float4 keep4(bool keep, float4 v) {
    return make_float4(keep ? v.x : 0.f, keep ? v.y : 0.f, keep ? v.z : 0.f, keep ? v.w : 0.f);
}

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

// apply_qk_norm (src/ops/reference/attention.rs:92-108), the scale of one head vector `row`
// (hd f32): squares rounded, summed in order from 0 in f32, divided by hd, then
// 1 / sqrt(mean + eps) with correctly rounded sqrt and division.  The caller applies
// x = (x * scale) * w per element.  One thread walks the row (the order is the contract).
// The row is read in batches of 8 independent 16-byte loads (one memory latency per batch,
// not one per load) and summed in order.
__device__ inline float qk_norm_scale(const float *row, int hd, float eps) {
#pragma clang fp contract(off)
    float sum = 0.0f;
    for (int d0 = 0; d0 < hd; d0 += 32) {
        float4 x[8];
#pragma unroll
        for (int b = 0; b < 8; b++)
            x[b] = d0 + 4 * b < hd ? *reinterpret_cast<const float4 *>(row + d0 + 4 * b) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int b = 0; b < 8; b++) {
            if (d0 + 4 * b >= hd) break;  // (hd is a multiple of 8: whole float4s)
            sum = sum + x[b].x * x[b].x;
            sum = sum + x[b].y * x[b].y;
            sum = sum + x[b].z * x[b].z;
            sum = sum + x[b].w * x[b].w;
        }
    }
    const float ms = sum / (float)hd;
    return 1.0f / sqrtf(ms + eps);
}

// x * x rounded to f32 (never fused into a following add)
__device__ inline float sq_rn(float x) {
#pragma clang fp contract(off)
    return x * x;
}

// The same sum over a row spread across lanes, without touching memory: lane l holds the
// squares of dims 2l and 2l + 1 (sq0, sq1); lanes 0..n_lanes-1 are read in order and added to
// sum (a running sum over earlier dims).  Every lane gets the ordered sum (of rounded squares,
// as qk_norm_scale).
__device__ inline float ordered_sum_pairs(float sq0, float sq1, int n_lanes, float sum = 0.0f) {
#pragma clang fp contract(off)
    for (int l = 0; l < n_lanes; l++) {
        sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sq0), l));
        sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sq1), l));
    }
    return sum;
}

// Ordered sum of a 128-dim row spread over the 16 lanes of a DPP row, lane l holding the 8
// squares of dims 8l..8l+7 in order: the running sum walks the lanes with row_shr:1, so the
// additions happen in the row's order.  Every lane of the row gets the total.
__device__ inline float ordered_sum_row16(const float (&sq)[8], int l) {
#pragma clang fp contract(off)
    float run = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        // lane l receives lane l-1's running sum (0 for the row's first lane)
        float t = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(run), 0x111, 0xF, 0xF, true));
#pragma unroll
        for (int e = 0; e < 8; e++) t = t + sq[e];
        run = l == i ? t : run;
    }
    return __shfl(run, (__lane_id() & ~15) | 15, 64);
}

// 1 / sqrt(sum / hd + eps), the apply_qk_norm scale from a finished sum of squares.
__device__ inline float qk_norm_scale_from_sum(float sum, int hd, float eps) {
#pragma clang fp contract(off)
    const float ms = sum / (float)hd;
    return 1.0f / sqrtf(ms + eps);
}

__device__ inline float qk_norm_apply(float x, float scale, float w) {
#pragma clang fp contract(off)
    const float t = x * scale;
    return t * w;
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

// Max over the 64 lanes of a wave for values >= 0 (or NaN, ignored like fmaxf): DPP within each
// 16-lane row, then two permlane swaps across rows.  No LDS traffic.
template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ inline float wave_max_nonneg(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm(1,0,3,2)
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm(2,3,0,1)
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Sum over the 64 lanes of a wave, every lane getting the same value (DPP within each 16-lane
// row, then the two permlane swaps).  The additions pair lanes symmetrically, so the result is
// identical in all lanes.
__device__ inline float wave_sum(float v) {
    v = v + dpp_f<0xB1>(v);   // quad_perm(1,0,3,2)
    v = v + dpp_f<0x4E>(v);   // quad_perm(2,3,0,1)
    v = v + dpp_f<0x141>(v);  // row_half_mirror
    v = v + dpp_f<0x140>(v);  // row_mirror
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// apply_qk_norm scale of query head `mine` of the G (<= 8) consecutive head rows at q, computed
// by the whole wave: every row's squares are summed as a tree across the lanes (the query side
// only feeds the softmax, compared within tolerance, so the order of the sum is free) and no
// LDS or barrier is involved.  All lanes must call it.
// Rows of hdr floats (stride hdr), hdr <= HD.
template <int HD>
__device__ inline float q_norm_scale_wave(const float *q, int G, int mine, float eps, int hdr = HD) {
    static_assert(HD % 64 == 0, "whole float lanes per row");
    constexpr int PER = HD / 64;
    const int lane = __lane_id();
    float x[8][PER];
#pragma unroll
    for (int g = 0; g < 8; g++)
#pragma unroll
        for (int e = 0; e < PER; e++)
            x[g][e] = g < G && PER * lane + e < hdr ? q[(size_t)g * hdr + PER * lane + e] : 0.0f;
    float out = 1.0f;
#pragma unroll
    for (int g = 0; g < 8; g++) {
        if (g < G) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < PER; e++) ss += x[g][e] * x[g][e];
            const float sc = qk_norm_scale_from_sum(wave_sum(ss), hdr, eps);
            out = g == mine ? sc : out;
        }
    }
    return out;
}

// The apply_qk_norm scales of all G (<= GMAX) consecutive query head rows at q, the same in
// every lane (1 past G); computed by the whole wave like q_norm_scale_wave.
template <int HD, int GMAX>
__device__ inline void q_norm_scales_wave(const float *q, int G, float eps, int hdr, float (&out)[GMAX]) {
    static_assert(HD % 64 == 0, "whole float lanes per row");
    constexpr int PER = HD / 64;
    const int lane = __lane_id();
#pragma unroll
    for (int g = 0; g < GMAX; g++) {
        out[g] = 1.0f;
        if (g < G) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < PER; e++) {
                const float x = PER * lane + e < hdr ? q[(size_t)g * hdr + PER * lane + e] : 0.0f;
                ss += x * x;
            }
            out[g] = qk_norm_scale_from_sum(wave_sum(ss), hdr, eps);
        }
    }
}

// encode(x, scale) with the quotient taken as x * rcp(scale) wherever that cannot change the
// rounded result: |x| <= 7 scale here (scale = max|x| / 7), so the product is within ~1.3e-6
// of the correctly rounded x / scale, and only a quotient within 1e-5 of a half-integer (the
// rounding boundaries) or a scale outside [2^-126, 2^125] (denormal or overflowing reciprocal)
// takes the correctly rounded division.  Bit-identical to encode for every input.
__device__ inline uint32_t encode_fast(float x, float scale, float rinv) {
    float q = x * rinv;
    const float a = fabsf(q);
    const float f = a - floorf(a);  // exact for a < 8
    if (fabsf(f - 0.5f) < 1.0e-5f || !(scale >= 1.17549435e-38f && scale <= 4.25352959e37f))
        q = __fdiv_rn(x, scale);
    const float r = roundf(q);
    int c = (r != r) ? 0 : (int)fminf(fmaxf(r, -64.0f), 64.0f);
    c += 8;
    c = c < 1 ? 1 : (c > 15 ? 15 : c);
    return (uint32_t)c;
}

}  // namespace
}  // namespace ts
