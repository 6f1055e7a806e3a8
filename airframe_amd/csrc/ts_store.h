// ts_store.h -- the quantize-and-store step of the INT4 append (head_dim 128 and 64), shared
// by the append kernel (rows loaded from f32 K/V) and the fused QKV projection (rows taken
// from the projection's output tile), so both write bit-identical codes and scales.
//
// Quantiser (cpu_quantize, src/backend/bindless/test_int4_parity.rs:56-75): per head vector,
// scale = max|x| / 7 (1 when max|x| == 0), code = clamp(round_half_away(x/scale) + 8, 1, 15),
// after the optional QK norm (src/ops/reference/attention.rs:92-108) and the rotation of K at
// its position (src/ops/reference/rope.rs:186-196).  Files that include it are compiled with
// -ffp-contract=off: a product fused into a following add would change codes.
#pragma once
#include "ts_quant.h"

namespace ts {
namespace {

constexpr int kBlk = 32;

// Code of x (= clamp(round_half_away(x/scale) + 8, 1, 15)) from y = x * rcp(scale), for
// |x| <= 7 scale: t = y + 8.5 lies in [1.5, 15.5] and trunc(t) is the code unless y is within
// 1e-5 of a half-integer (|y - x/scale| <= ~1.3e-6, and the add rounds by < 1e-6), which sets
// `need` (as does NaN); the caller then recomputes with encode().
__device__ inline uint32_t code_fast(float y, bool &need) {
    const float t = y + 8.5f;
    const uint32_t c = (uint32_t)t;
    const float d = t - (float)c;
    need |= !(fabsf(d - 0.5f) <= 0.49999f);
    return c;
}

// Rotation (cos, sin) of the 4 pairs 4l..4l+3 of slot p of sequence s (identity without a
// table or past rope_pairs).
__device__ inline void rope_cs4(const KvLayerView &L, int s, int p, const float *rope, int rope_pairs,
                                int l, float2 (&cs)[4]) {
    const int pr = rot_of(L, s, p);
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const int pair = 4 * l + m;
        cs[m] = (rope && pair < rope_pairs)
                    ? *reinterpret_cast<const float2 *>(rope + ((size_t)pr * rope_pairs + pair) * 2)
                    : make_float2(1.0f, 0.0f);
    }
}

// A head row spread over LPR lanes (16 for hd 128, 8 for hd 64), lane l = lane % LPR holding
// dims 8l..8l+7.

// Max of v over the row's lanes (values >= 0): DPP inside the 16-lane row.
template <int LPR>
__device__ inline float row_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm(1,0,3,2)
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm(2,3,0,1)
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror: 8 lanes
    if (LPR == 16) v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror: 16 lanes
    return v;
}

// Sum of the row's squares in dimension order (lane 0's 8 in order, then lane 1's, ...),
// from 0, one f32 rounding per add: the running sum walks the lanes with row_shr:1.  Every
// lane of the row gets the total.
template <int LPR>
__device__ inline float row_ordered_sum(const float (&sq)[8], int l) {
#pragma clang fp contract(off)
    float run = 0.0f;
#pragma unroll
    for (int i = 0; i < LPR; i++) {
        float t = i == 0 ? 0.0f
                         : __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(run), 0x111, 0xF, 0xF, true));
#pragma unroll
        for (int e = 0; e < 8; e++) t = t + sq[e];
        run = l == i ? t : run;
    }
    return __shfl(run, (__lane_id() & ~(LPR - 1)) | (LPR - 1), 64);
}

// QK norm of a K row in place (weights kn, the row's lanes as above).
// Rows of hdr real dims (the stored dims past them are 0 and stay 0).
template <int LPR>
__device__ inline void row_qk_norm(float (&kx)[8], const float *kn, float eps, int l, int hdr) {
    float sq[8];
#pragma unroll
    for (int e = 0; e < 8; e++) sq[e] = sq_rn(kx[e]);
    const float ns = qk_norm_scale_from_sum(row_ordered_sum<LPR>(sq, l), hdr, eps);
    const int lc = 8 * l < hdr ? l : 0;  // (a lane past the row keeps its zeros: 0 * w = 0)
#pragma unroll
    for (int e = 0; e < 8; e++) kx[e] = qk_norm_apply(kx[e], ns, kn[8 * lc + e]);
}

// Scales and codes of one K row and one V row from their maxima (row_max): the reciprocal
// fast path of encode_fast, with the exact path for the whole wave when any lane needs it.
// Every lane of the wave must call it.
__device__ inline void row_codes(const float (&kx)[8], const float (&vx)[8], float km, float vm, float &ks,
                                 float &vs, uint32_t (&kc)[8], uint32_t (&vc)[8]) {
    ks = quant_scale(km);
    vs = quant_scale(vm);
    const float kr = __builtin_amdgcn_rcpf(ks), vr = __builtin_amdgcn_rcpf(vs);
    bool kneed = !(ks >= 1.17549435e-38f && ks <= 4.25352959e37f);
    bool vneed = !(vs >= 1.17549435e-38f && vs <= 4.25352959e37f);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        kc[e] = code_fast(kx[e] * kr, kneed);
        vc[e] = code_fast(vx[e] * vr, vneed);
    }
    if (__builtin_amdgcn_ballot_w64(kneed) != 0) {
#pragma unroll
        for (int e = 0; e < 8; e++) kc[e] = encode(kx[e], ks);
    }
    if (__builtin_amdgcn_ballot_w64(vneed) != 0) {
#pragma unroll
        for (int e = 0; e < 8; e++) vc[e] = encode(vx[e], vs);
    }
}

// hd = 64: quantizes and stores positions [lo, hi) of V block blk of one (sequence s, kv head
// h).  4 waves, 8 lanes per position (lane l = lane % 8 holds dims 8l..8l+7 of one position in
// kx / vx, raw, with its pairs' rotation in cs).  Wave w owns the 8 positions of V key group
// g = w: lane group r8 = lane / 8 holds position 4w + (r8 % 4) + 16 (r8 / 4), which is nibble
// r8 of the group's V words, so the words are OR-assembled across the wave's 8 lane groups
// (DPP row_ror:8, then two permlane swaps) and written by the wave.  Rows outside [lo, hi)
// may hold anything finite; they are never written.  Every lane of the workgroup must call it.
__device__ inline void store_block64(const KvLayerView &L, int s, int h, int blk, int lo, int hi,
                                     float (&kx)[8], const float (&vx)[8], const float2 (&cs)[4],
                                     int rot_pairs, int wave, int lane) {
    constexpr int HD = 64;
    const int r8 = lane >> 3, l = lane & 7;
    const int p0 = blk * kBlk;
    const int p = p0 + 4 * wave + (r8 & 3) + 16 * (r8 >> 2);
    const size_t row = (size_t)s * L.H + h;
    if (L.kn) row_qk_norm<8>(kx, L.kn, L.norm_eps, l, L.hdr);
#pragma unroll
    for (int m = 0; m < 4; m++)
        if (4 * l + m < rot_pairs) rope_rotate(kx[2 * m], kx[2 * m + 1], cs[m]);
    float km = 0.0f, vm = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        km = fmaxf(km, fabsf(kx[e]));
        vm = fmaxf(vm, fabsf(vx[e]));
    }
    km = row_max<8>(km);
    vm = row_max<8>(vm);
    float ks, vs;
    uint32_t kc[8], vc[8];
    row_codes(kx, vx, km, vm, ks, vs, kc, vc);
    if (p >= lo && p < hi) {
        uint32_t kw = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) kw |= kc[e] << (4 * e);
        reinterpret_cast<uint32_t *>(L.kp + row * L.P * (HD / 2))[k_word_idx<HD>(p, l)] = kw;
        if (l == 0) {
            L.ks[row * L.P + p] = ks;
            L.vs[row * L.P + p] = vs;
        }
    }
    // this lane group's nibble of the words of dims 8l + e, OR-ed over the 8 groups
    uint32_t vpart[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        uint32_t x = vc[e] << (4 * r8);
        x |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);  // row_ror:8
        auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        x = a[0] | a[1];
        auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        vpart[e] = b[0] | b[1];
    }
    uint32_t keep = 0;  // nibbles of positions outside [lo, hi)
#pragma unroll
    for (int n = 0; n < 8; n++) {
        const int pn = p0 + 4 * wave + (n & 3) + 16 * (n >> 2);
        if (pn < lo || pn >= hi) keep |= 0xFu << (4 * n);
    }
    // lane (r8, l) writes the word of dim 8l + r8
    const uint32_t w = r8 == 0 ? vpart[0] : r8 == 1 ? vpart[1] : r8 == 2 ? vpart[2] : r8 == 3 ? vpart[3]
                     : r8 == 4 ? vpart[4] : r8 == 5 ? vpart[5] : r8 == 6 ? vpart[6] : vpart[7];
    const int d = 8 * l + r8, td = d >> 4, dl = d & 15;
    uint32_t *dst = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / kBlk) + blk) * (HD * 16)) + v_word_idx(wave * 16 + dl, td);
    *dst = keep ? (*dst & keep) | (w & ~keep) : w;
}

// Quantizes and stores positions [lo, hi) of V block blk (positions p0 = 32 blk .. p0 + 31) of
// one (sequence s, kv head h), hd = 128, from registers laid out as the append kernel loads
// them: 4 waves, 16 lanes per position, lane l = lane % 16 holding dims 8l..8l+7 of positions
// p0 + 16 rd + 4 wave + lane / 16 (rd = 0, 1) in kx[rd] / vx[rd] (raw K and V), and the
// rotation of its 4 pairs at that position in cs[rd]; pairs at or past rot_pairs (0: no
// rotation) are left as they are.  Rows outside [lo, hi) may hold
// anything finite; they are never written.  Wave w assembles the V words with g = w from its
// 4 rows with permlane swaps and writes them itself (keeping the nibbles of positions outside
// [lo, hi)).  Reductions: 4 DPP steps within a 16-lane row.  Every lane of the workgroup
// must call it.
__device__ inline void store_block128(const KvLayerView &L, int s, int h, int blk, int lo, int hi,
                                      float (&kx)[2][8], float (&vx)[2][8], const float2 (&cs)[2][4],
                                      int rot_pairs, int wave, int lane) {
    constexpr int HD = 128;
    const int r = lane >> 4, l = lane & 15;
    const int p0 = blk * kBlk;
    const size_t row = (size_t)s * L.H + h;
    if (L.kn) {
        // QK norm of every K row before RoPE, its squares summed in the row's order across the
        // 16 lanes that hold it
#pragma unroll
        for (int rd = 0; rd < 2; rd++) {
            float sq[8];
#pragma unroll
            for (int e = 0; e < 8; e++) sq[e] = sq_rn(kx[rd][e]);
            const float ns = qk_norm_scale_from_sum(ordered_sum_row16(sq, l), L.hdr, L.norm_eps);
            const int lc = 8 * l < L.hdr ? l : 0;  // (a lane past the row keeps its zeros)
#pragma unroll
            for (int e = 0; e < 8; e++) kx[rd][e] = qk_norm_apply(kx[rd][e], ns, L.kn[8 * lc + e]);
        }
    }
    float km[2], vm[2];
#pragma unroll
    for (int rd = 0; rd < 2; rd++) {
        {
#pragma unroll
            for (int m = 0; m < 4; m++)
                if (4 * l + m < rot_pairs) rope_rotate(kx[rd][2 * m], kx[rd][2 * m + 1], cs[rd][m]);
        }
        km[rd] = 0.0f;
        vm[rd] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            km[rd] = fmaxf(km[rd], fabsf(kx[rd][e]));
            vm[rd] = fmaxf(vm[rd], fabsf(vx[rd][e]));
        }
    }
#pragma unroll
    for (int rd = 0; rd < 2; rd++) {
        km[rd] = fmaxf(km[rd], dpp_f<0xB1>(km[rd]));
        vm[rd] = fmaxf(vm[rd], dpp_f<0xB1>(vm[rd]));
    }
#pragma unroll
    for (int rd = 0; rd < 2; rd++) {
        km[rd] = fmaxf(km[rd], dpp_f<0x4E>(km[rd]));
        vm[rd] = fmaxf(vm[rd], dpp_f<0x4E>(vm[rd]));
    }
#pragma unroll
    for (int rd = 0; rd < 2; rd++) {
        km[rd] = fmaxf(km[rd], dpp_f<0x141>(km[rd]));
        vm[rd] = fmaxf(vm[rd], dpp_f<0x141>(vm[rd]));
    }
#pragma unroll
    for (int rd = 0; rd < 2; rd++) {
        km[rd] = fmaxf(km[rd], dpp_f<0x140>(km[rd]));
        vm[rd] = fmaxf(vm[rd], dpp_f<0x140>(vm[rd]));
    }

    uint32_t vpart[8];  // this row's nibbles of V words (dims 8l + e)
#pragma unroll
    for (int e = 0; e < 8; e++) vpart[e] = 0;
#pragma unroll
    for (int rd = 0; rd < 2; rd++) {
        const int p = p0 + 16 * rd + 4 * wave + r;
        const bool in = p >= lo && p < hi;
        const float ks = quant_scale(km[rd]), vs = quant_scale(vm[rd]);
        const float kr = __builtin_amdgcn_rcpf(ks), vr = __builtin_amdgcn_rcpf(vs);
        const bool k_ok = ks >= 1.17549435e-38f && ks <= 4.25352959e37f;
        const bool v_ok = vs >= 1.17549435e-38f && vs <= 4.25352959e37f;
        uint32_t kc[8], vc[8];
        bool kneed = !k_ok, vneed = !v_ok;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kc[e] = code_fast(kx[rd][e] * kr, kneed);
            vc[e] = code_fast(vx[rd][e] * vr, vneed);
        }
        if (__builtin_amdgcn_ballot_w64(kneed) != 0) {
#pragma unroll
            for (int e = 0; e < 8; e++) kc[e] = encode(kx[rd][e], ks);
        }
        if (__builtin_amdgcn_ballot_w64(vneed) != 0) {
#pragma unroll
            for (int e = 0; e < 8; e++) vc[e] = encode(vx[rd][e], vs);
        }
        uint32_t kw = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kw |= kc[e] << (4 * e);
            vpart[e] |= vc[e] << (4 * r + 16 * rd);
        }
        if (in) {
            reinterpret_cast<uint32_t *>(L.kp + row * L.P * (HD / 2))[k_word_idx<HD>(p, l)] = kw;
            if (l == 0) {
                L.ks[row * L.P + p] = ks;
                L.vs[row * L.P + p] = vs;
            }
        }
    }
    // OR the 4 rows' parts: lanes l, l+16, l+32, l+48 end up with the same 8 words
#pragma unroll
    for (int e = 0; e < 8; e++) {
        auto a = __builtin_amdgcn_permlane16_swap(vpart[e], vpart[e], false, false);
        vpart[e] = a[0] | a[1];
        auto b = __builtin_amdgcn_permlane32_swap(vpart[e], vpart[e], false, false);
        vpart[e] = b[0] | b[1];
    }
    // row r writes dims 8l + 2r and 8l + 2r + 1: word (g = wave, dl, td) of the block
    uint32_t keep = 0;  // nibbles of positions outside [lo, hi)
#pragma unroll
    for (int n = 0; n < 8; n++) {
        const int p = p0 + 4 * wave + (n & 3) + 16 * (n >> 2);
        if (p < lo || p >= hi) keep |= 0xFu << (4 * n);
    }
    uint32_t *vb = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / kBlk) + blk) * (HD * 16));
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int e = 2 * r + q;
        const uint32_t w = r == 0 ? (q ? vpart[1] : vpart[0])
                         : r == 1 ? (q ? vpart[3] : vpart[2])
                         : r == 2 ? (q ? vpart[5] : vpart[4])
                                  : (q ? vpart[7] : vpart[6]);
        const int d = 8 * l + e, td = d >> 4, dl = d & 15;
        uint32_t *dst = vb + v_word_idx(wave * 16 + dl, td);
        *dst = keep ? (*dst & keep) | (w & ~keep) : w;
    }
}


// Ordered sum of a row spread over 32 lanes (lane l holding the 8 squares of dims 8l..8l+7 in
// order), for hd 256: one lane at a time, in the row's order, the rows of the wave's two lane
// halves independently.  Every lane gets its half's total.
__device__ inline float ordered_sum_row32(const float (&sq)[8]) {
#pragma clang fp contract(off)
    const int base = __lane_id() & 32;
    float run = 0.0f;
    for (int i = 0; i < 32; i++) {
#pragma unroll
        for (int e = 0; e < 8; e++) run = run + __shfl(sq[e], base + i, 64);
    }
    return run;
}

// hd = 256: as store_block128 with 32 lanes per position (lane l = lane % 32 holding dims
// 8l..8l+7, K word l) and two rows per wave (r = lane / 32): wave w takes the 8 positions of
// V key group g = w, position p0 + 4w + 2 (rd % 2) + r + 16 (rd / 2) in kx[rd] / vx[rd]
// (rd = 0..3), which is nibble 2 (rd % 2) + r + 4 (rd / 2) of the group's V words.
__device__ inline void store_block256(const KvLayerView &L, int s, int h, int blk, int lo, int hi,
                                      float (&kx)[4][8], float (&vx)[4][8], const float2 (&cs)[4][4],
                                      int rot_pairs, int wave, int lane) {
    constexpr int HD = 256;
    const int r = lane >> 5, l = lane & 31;
    const int p0 = blk * kBlk;
    const size_t row = (size_t)s * L.H + h;
    if (L.kn) {
        const int lc = 8 * l < L.hdr ? l : 0;  // (a lane past the row keeps its zeros)
#pragma unroll
        for (int rd = 0; rd < 4; rd++) {
            float sq[8];
#pragma unroll
            for (int e = 0; e < 8; e++) sq[e] = sq_rn(kx[rd][e]);
            const float ns = qk_norm_scale_from_sum(ordered_sum_row32(sq), L.hdr, L.norm_eps);
#pragma unroll
            for (int e = 0; e < 8; e++) kx[rd][e] = qk_norm_apply(kx[rd][e], ns, L.kn[8 * lc + e]);
        }
    }
    uint32_t vpart[8];  // this lane's dims 8l + e: the nibbles of the wave's 8 positions
#pragma unroll
    for (int e = 0; e < 8; e++) vpart[e] = 0;
#pragma unroll
    for (int rd = 0; rd < 4; rd++) {
#pragma unroll
        for (int m = 0; m < 4; m++)
            if (4 * l + m < rot_pairs) rope_rotate(kx[rd][2 * m], kx[rd][2 * m + 1], cs[rd][m]);
        float km = 0.0f, vm = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            km = fmaxf(km, fabsf(kx[rd][e]));
            vm = fmaxf(vm, fabsf(vx[rd][e]));
        }
        // max over the 32 lanes of the row: 16-lane DPP steps, then across the two 16-lane rows
        km = row_max<16>(km);
        vm = row_max<16>(vm);
        {
            auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(km), __float_as_uint(km), false, false);
            km = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
            auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(vm), __float_as_uint(vm), false, false);
            vm = fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
        }
        float ks, vs;
        uint32_t kc[8], vc[8];
        row_codes(kx[rd], vx[rd], km, vm, ks, vs, kc, vc);
        const int n = 2 * (rd & 1) + r + 4 * (rd >> 1);  // nibble of this position in the words
        const int p = p0 + 4 * wave + 2 * (rd & 1) + r + 16 * (rd >> 1);
        if (p >= lo && p < hi) {
            uint32_t kw = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) kw |= kc[e] << (4 * e);
            reinterpret_cast<uint32_t *>(L.kp + row * L.P * (HD / 2))[k_word_idx<HD>(p, l)] = kw;
            if (l == 0) {
                L.ks[row * L.P + p] = ks;
                L.vs[row * L.P + p] = vs;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; e++) vpart[e] |= vc[e] << (4 * n);
    }
    // OR the two rows' parts: lanes l and l + 32 end up with the same 8 words
#pragma unroll
    for (int e = 0; e < 8; e++) {
        auto b = __builtin_amdgcn_permlane32_swap(vpart[e], vpart[e], false, false);
        vpart[e] = b[0] | b[1];
    }
    uint32_t keep = 0;  // nibbles of positions outside [lo, hi)
#pragma unroll
    for (int n = 0; n < 8; n++) {
        const int pn = p0 + 4 * wave + (n & 3) + 16 * (n >> 2);
        if (pn < lo || pn >= hi) keep |= 0xFu << (4 * n);
    }
    uint32_t *vb = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / kBlk) + blk) * (HD * 16));
    // row r writes the words of dims 8l + 4r .. 8l + 4r + 3
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int e = 4 * r + q;
        const uint32_t w = r == 0 ? (q == 0 ? vpart[0] : q == 1 ? vpart[1] : q == 2 ? vpart[2] : vpart[3])
                                  : (q == 0 ? vpart[4] : q == 1 ? vpart[5] : q == 2 ? vpart[6] : vpart[7]);
        const int d = 8 * l + e, td = d >> 4, dl = d & 15;
        uint32_t *dst = vb + v_word_idx(wave * 16 + dl, td);
        *dst = keep ? (*dst & keep) | (w & ~keep) : w;
    }
}
}  // namespace
}  // namespace ts
