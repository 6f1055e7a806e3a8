// ts_mfma.h -- device helpers shared by the decode and prefill attention kernels: INT4 -> f16
// conversion in the slot order the v_mfma_f32_16x16x32_f16 operands use, and the rotated,
// hi/lo-split query operand.
#pragma once
#include "ts_quant.h"

namespace ts {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMinit = -1.0e30f;

// (w & mask) | add in one VALU op.  gfx9 VOP3 encodings take no literal constants and read at
// most one SGPR, so the masks are passed in VGPRs (see DeqConst).
//
// Inline asm is invisible to the compiler's hazard recognizer, so its result must never feed a
// matrix-core instruction directly: every use below goes through a compiler-visible packed f16
// op first, which carries the required wait states.  (Written as plain C, the compiler picks
// the same v_and_or_b32 but reschedules the decode loop into spills, ~20% slower; both builds
// give bit-identical attention outputs.)
__device__ inline uint32_t and_or(uint32_t w, uint32_t mask, uint32_t add) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "v"(mask), "v"(add));
    return r;
}

// Loop-invariant operands of dequant8, materialised once per kernel in VGPRs.
struct DeqConst {
    uint32_t lo, hi, magic;
    __device__ DeqConst() : lo(0x000F000Fu), hi(0x00F000F0u), magic(0x64006400u) {}
};
// The same, hidden from constant folding (an empty asm per value), so that plain C code
// using them keeps them in registers.
struct DeqConstV : DeqConst {
    __device__ DeqConstV() {
        asm volatile("" : "+v"(lo));
        asm volatile("" : "+v"(hi));
        asm volatile("" : "+v"(magic));
    }
};

// 8 nibbles of w -> half8 holding (code - 8) in slot order [e0,e4,e1,e5,e2,e6,e3,e7].
// 0x6400 | n is the f16 1024 + n; 0x6400 | (n << 4) is 1024 + 16 n, brought back with
// x/16 - 72 in one packed FMA.  Every step is exact.  9 VALU ops per 8 codes.
__device__ inline half8 dequant8(uint32_t w, const DeqConst &k) {
    const uint32_t w8 = w >> 8;
    const uint32_t a = and_or(w, k.lo, k.magic);   // 1024 + e0 | 1024 + e4
    const uint32_t b = and_or(w, k.hi, k.magic);   // 1024 + 16 e1 | 1024 + 16 e5
    const uint32_t c = and_or(w8, k.lo, k.magic);  // e2 | e6
    const uint32_t d = and_or(w8, k.hi, k.magic);  // e3 | e7
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

// Max of v over the four lane groups g (lanes n, n+16, n+32, n+48): two permlane swaps.
__device__ inline float group_max(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ inline float group_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// dequant8 written in plain C: the same instructions, but visible to the scheduler, so it can
// be interleaved with matrix-core work (prefill staging).
// k: the masks and the magic in VGPRs (see DeqConstV), so that each mask-and-or is one
// v_and_or_b32 (two literal operands cannot be encoded in one instruction).
__device__ inline half8 dequant8_c(uint32_t w, const DeqConst &k) {
    const uint32_t w8 = w >> 8;
    const uint32_t a = (w & k.lo) | k.magic;
    const uint32_t b = (w & k.hi) | k.magic;
    const uint32_t c = (w8 & k.lo) | k.magic;
    const uint32_t d = (w8 & k.hi) | k.magic;
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

// x as an opaque f32 register value.  Splitting v = a*b into hi = f16(v), lo = f16(v - hi)
// needs both halves taken from the same rounded v: left visible, the compiler may turn one use
// of f16(a*b) into a fused multiply-convert (one rounding of the exact product) and the other
// into a convert of the f32 product (two roundings), and the halves then disagree by an f16
// ulp.  The empty asm pins v.  (Its result only feeds VALU conversions, never an MFMA.)
__device__ inline float opaque(float x) {
    asm("" : "+v"(x));
    return x;
}

// Split of v >= 0 into hi + lo, both then converted to f16: hi = v with the low 13 mantissa
// bits cleared (exact in f16 for v in f16's normal range), lo = v - hi (exact in f32, below
// 2^-10 v, so f16 keeps it to 2^-11 of itself: ~21 bits in all).  Bit operations on one
// register: the halves cannot come from different roundings of v.
__device__ inline float split_hi(float v) { return __uint_as_float(__float_as_uint(v) & 0xFFFFE000u); }

// The 8 dims 8u..8u+7 of one head's q, normalized when nw is set (QK norm weights nw, the
// row's scale ns: attention.rs:186-189 normalizes before RoPE); zeros for the stored dims at
// or past the row length hdr (a multiple of 8).
__device__ inline void q_read8(const float *qrow, int u, const float *nw, float ns, float (&x)[8], int hdr = 1 << 30) {
    // (dims past the row: the row's first dims are loaded, unconditionally, and dropped)
    const bool in = 8 * u < hdr;
    const int uc = in ? u : 0;
    const float4 x0 = *reinterpret_cast<const float4 *>(qrow + 8 * uc);
    const float4 x1 = *reinterpret_cast<const float4 *>(qrow + 8 * uc + 4);
    x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
    x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
    if (nw) {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = qk_norm_apply(x[e], ns, nw[8 * uc + e]);
    }
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = in ? x[e] : 0.0f;
}

// Bound on |rotated q| over the 8 dims 8u..8u+7 of one head: |a cos - b sin| <= |a| + |b|.
__device__ inline float q_bound8(const float *qrow, int u, const float *nw = nullptr, float ns = 1.0f,
                                int hdr = 1 << 30) {
    float x[8];
    q_read8(qrow, u, nw, ns, x, hdr);
    return fmaxf(fmaxf(fabsf(x[0]) + fabsf(x[1]), fabsf(x[2]) + fabsf(x[3])),
                 fmaxf(fabsf(x[4]) + fabsf(x[5]), fabsf(x[6]) + fabsf(x[7])));
}

// Power-of-two scale S for q operands bounded by m: m*S lands in [2^13, 2^14), so both halves
// of the hi/lo split stay normal f16 numbers (the matrix cores flush f16 subnormals, which
// would drop the low half of every small element).  Scores come out times S; callers fold
// inv_s = 1/S into the per-key scale.
__device__ inline void q_scale(float m, float &s, float &inv_s) {
    if (!(m > 0.0f) || !(m < 3.0e38f)) {
        s = inv_s = 1.0f;
        return;
    }
    const int e = min(max(ilogbf(m), -100), 100);
    s = ldexpf(1.0f, 13 - e);
    inv_s = ldexpf(1.0f, e - 13);
}

// Rotated q for the 8 dims 8u..8u+7 of one head from its (normalized) values x and the
// rotation cs[i] of pair 4u + i (pairs at or past rope_pairs are not rotated), times `mul`,
// split x = hi + lo into f16 and arranged in the slot order of dequant8.
__device__ inline void split_q8(float (&x)[8], const float2 (&cs)[4], int u, int rope_pairs, float mul,
                                half8 &hi, half8 &lo) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (4 * u + i < rope_pairs) rope_rotate(x[2 * i], x[2 * i + 1], cs[i]);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float v = opaque(x[kPerm[j]] * mul);
        const _Float16 h = (_Float16)v;
        hi[j] = h;
        lo[j] = (_Float16)(v - (float)h);
    }
}

// The rotations split_q8 needs for dims 8u..8u+7 at table row qpos.
__device__ inline void load_rot8(const float *rope, int rope_pairs, int u, int qpos, float2 (&cs)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int pair = 4 * u + i;
        cs[i] = pair < rope_pairs ? *reinterpret_cast<const float2 *>(rope + ((size_t)qpos * rope_pairs + pair) * 2)
                                  : make_float2(1.0f, 0.0f);
    }
}

// Rotated q for the 8 dims 8u..8u+7 of one head (rope.rs:186-196, table row qpos), after the
// optional QK norm, times `mul`, split x = hi + lo into f16 and arranged in the slot order of
// dequant8.
__device__ inline void load_q8(const float *rope, int rope_pairs, const float *qrow, int u,
                               int qpos, float mul, half8 &hi, half8 &lo,
                               const float *nw = nullptr, float ns = 1.0f, int hdr = 1 << 30) {
    float x[8];
    q_read8(qrow, u, nw, ns, x, hdr);
    float2 cs[4];
    load_rot8(rope, rope_pairs, u, qpos, cs);
    split_q8(x, cs, u, rope_pairs, mul, hi, lo);
}

}  // namespace
}  // namespace ts
