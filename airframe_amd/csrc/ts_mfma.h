// ts_mfma.h -- device helpers shared by the decode and prefill attention kernels: INT4 -> f16
// conversion in the slot order the v_mfma_f32_16x16x32_f16 operands use, and the rotated,
// hi/lo-split query operand.
#pragma once
#include "ts_internal.h"

namespace ts {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMinit = -1.0e30f;

// 8 nibbles of w -> half8 holding (code - 8) in slot order [e0,e4,e1,e5,e2,e6,e3,e7].
__device__ inline half8 dequant8(uint32_t w) {
    const uint32_t w8 = w >> 8;
    uint32_t a = (w & 0x000F000Fu) | 0x64006400u;   // 1024 + e0 | 1024 + e4
    uint32_t b = (w & 0x00F000F0u) | 0x64006400u;   // 1024 + 16 e1 | 1024 + 16 e5
    uint32_t c = (w8 & 0x000F000Fu) | 0x64006400u;  // e2 | e6
    uint32_t d = (w8 & 0x00F000F0u) | 0x64006400u;  // e3 | e7
    half2_t ha = __builtin_bit_cast(half2_t, a), hb = __builtin_bit_cast(half2_t, b);
    half2_t hc = __builtin_bit_cast(half2_t, c), hd = __builtin_bit_cast(half2_t, d);
    const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2_t off2 = {(_Float16)-72.0f, (_Float16)-72.0f};
    ha = ha - off;
    hb = hb * sixteenth + off2;
    hc = hc - off;
    hd = hd * sixteenth + off2;
    half8 r;
    r[0] = ha[0]; r[1] = ha[1];
    r[2] = hb[0]; r[3] = hb[1];
    r[4] = hc[0]; r[5] = hc[1];
    r[6] = hd[0]; r[7] = hd[1];
    return r;
}

// dims held in slot j of a dequantized word: 8u + kPerm[j]
__device__ constexpr int kPerm[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// Rotated q for the 8 dims 8u..8u+7 of one head (rope.rs:186-196, table row qpos), split
// x = hi + lo into f16 and arranged in the slot order of dequant8.
__device__ inline void load_q8(const float *rope, int rope_pairs, const float *qrow, int u,
                               int qpos, half8 &hi, half8 &lo) {
    float x[8];
    const float4 x0 = *reinterpret_cast<const float4 *>(qrow + 8 * u);
    const float4 x1 = *reinterpret_cast<const float4 *>(qrow + 8 * u + 4);
    x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
    x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int pair = 4 * u + i;
        if (pair < rope_pairs) {
            const float2 cs = *reinterpret_cast<const float2 *>(rope + ((size_t)qpos * rope_pairs + pair) * 2);
            const float xa = x[2 * i], xb = x[2 * i + 1];
            x[2 * i] = __fsub_rn(__fmul_rn(xa, cs.x), __fmul_rn(xb, cs.y));
            x[2 * i + 1] = __fadd_rn(__fmul_rn(xa, cs.y), __fmul_rn(xb, cs.x));
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float v = x[kPerm[j]];
        const _Float16 h = (_Float16)v;
        hi[j] = h;
        lo[j] = (_Float16)(v - (float)h);
    }
}

}  // namespace
}  // namespace ts
