// ts_kquant.h -- projection weights in the GGUF block formats Q4_K, Q5_K (below) and Q8_0,
// Q4_0 (further down) read at their own size inside the matrix-core loop of the split
// projections (decode shapes).
//
// The reference's main_qkv / main_attn_proj read every weight from the GGUF blob inside the dot
// product (src/backend/bindless/sh_layer_v1_int4.wgsl:502-520, sh_layer_v1.wgsl:777-790) with
// the values of src/core/dequant/q4_k.rs:75-123 and q5_k.rs:74-143:
//     w = (d * sc_j) * q - dmin * m_j      (sub-block j of 32 elements, q 4 or 5 bits).
// Here the sum over one 256-element super-block is taken apart as
//     sum_k x_k w_k = d * sum_j sc_j sum_{k in j} x_k q_k  -  dmin * sum_j m_j xsum_j
// and both inner sums run on v_mfma_f32_32x32x16_f16 with x split hi + lo:
//   * B operand of the first: q * sc_j, an integer below 2048, so exact in f16.  The k-steps
//     are arranged so that every lane's 8 elements of one instruction lie in one sub-block:
//     lane half hf of a 64-element chunk g takes bytes 16 hf .. 16 hf + 15 of the chunk's 32
//     qs bytes (one 16-byte load) -- k-steps 0, 1 their low nibbles (sub-block 2g), 2, 3
//     their high nibbles (sub-block 2g + 1).  The x operand reads the same elements.
//   * the second: xsum_j (the sub-block sums of x, f32 split hi + lo) against m_j, one
//     instruction per super-block with k = the 8 sub-blocks (the upper 8 k are zero).
// d and dmin are applied to the two f32 accumulators once per super-block (one FMA each per
// output).  A weight moves 144 / 256 = 0.5625 bytes (Q4_K) or 176 / 256 = 0.6875 (Q5_K)
// instead of 4 for the two-plane f16 form.
#pragma once
#include "ts_gemm.h"

namespace ts {
namespace {

constexpr int kGgmlQ4_0 = 2, kGgmlQ5_0 = 6, kGgmlQ8_0 = 8, kGgmlQ4K = 12, kGgmlQ5K = 13;

// Bytes of 256 elements of a row: one K-quant super-block, or 8 blocks of 32 (Q4_0: 18 bytes,
// Q5_0: 22, Q8_0: 34 each).
__host__ __device__ constexpr int kq_bytes(int t) {
    return t == kGgmlQ4K ? 144 : t == kGgmlQ5K ? 176 : t == kGgmlQ4_0 ? 144 : t == kGgmlQ5_0 ? 176 : 272;
}
template <int T>
struct KQ {
    static constexpr int BYTES = kq_bytes(T);
    static constexpr int QS = T == kGgmlQ4K ? 16 : 48;       // offset of the 128 qs bytes (K formats)
};
__host__ __device__ constexpr bool kq_type(int t) {
    return t == kGgmlQ4_0 || t == kGgmlQ5_0 || t == kGgmlQ8_0 || t == kGgmlQ4K || t == kGgmlQ5K;
}

// LDS of the K-quant slice loop: x of one super-block (4 chunks of 64) as hi/lo, and the f32
// sums of its 8 sub-blocks per row.
struct KqTiles {
    SplitTiles x;
    float xsum[32][8];
};

// One lane's share of one weight row's super-block: the 16-byte header (d, dmin, 12 packed
// scale bytes), its 16 qs bytes of each 64-element chunk, and for Q5_K its 16 qh bytes (the
// fifth bits of elements 16 hf .. 16 hf + 15 of every sub-block).
struct KqRegs {
    uint4 hdr, qs[4], qh;
};

template <int T>
__device__ __forceinline__ void kq_load(KqRegs &r, const uint8_t *blk, int hf) {
    r.hdr = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
    for (int g = 0; g < 4; g++) r.qs[g] = *reinterpret_cast<const uint4 *>(blk + KQ<T>::QS + 32 * g + 16 * hf);
    if constexpr (T == kGgmlQ5K)
        r.qh = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * hf);
    else
        r.qh = make_uint4(0u, 0u, 0u, 0u);
}

// The 6-bit scales and mins of the 8 sub-blocks (q4_k.rs:134-143, get_scale_min_k4), four
// per word, byte j % 4: sc of sub-blocks 0-3 and 4-7, m of 0-3 and 4-7.
struct KqScales {
    uint32_t sc03, sc47, m03, m47;
};
__device__ inline KqScales kq_scales(const uint4 &hdr) {
    const uint32_t y = hdr.y, z = hdr.z, w = hdr.w;  // scale bytes 0-3, 4-7, 8-11
    KqScales s;
    s.sc03 = y & 0x3F3F3F3Fu;
    s.m03 = z & 0x3F3F3F3Fu;
    s.sc47 = (w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u);
    s.m47 = ((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u);
    return s;
}
__device__ inline int kq_byte(uint32_t w, int b) { return (int)((w >> (8 * b)) & 0xFFu); }

// The B operands of chunk g for one weight row: k-step q in b[q], element i of the half8 the
// code of byte 8 (q & 1) + i of the lane's 16 (low nibble for q < 2, high for q >= 2), times
// its sub-block's scale.  Codes enter as f16 1024 + n (0x6400 | n) or, for a Q4_K high nibble
// left in place, 1024 + 16 n; one packed FMA per two codes gives n * sc exactly (every
// intermediate is an integer below 2^16 that f16 holds, or that integer over 16).
template <int T>
__device__ __forceinline__ void kq_operands(const KqRegs &r, const KqScales &s, int g, half8 (&b)[4],
                                            const DeqConst &dk) {
    const int scl = g < 2 ? kq_byte(s.sc03, 2 * g) : kq_byte(s.sc47, 2 * g - 4);
    const int sch = g < 2 ? kq_byte(s.sc03, 2 * g + 1) : kq_byte(s.sc47, 2 * g - 3);
    const _Float16 fl = (_Float16)scl, fh = (_Float16)sch;
    const half2_t ml = {fl, fl}, al = {(_Float16)(-1024.0f) * fl, (_Float16)(-1024.0f) * fl};
    // Q4_K high nibbles stay at bits 4-7 (1024 + 16 n): multiply by sc / 16, subtract 64 sc;
    // Q5_K high codes are moved down first (1024 + n): multiply by sc, subtract 1024 sc
    const _Float16 fhm = T == kGgmlQ4K ? fh * (_Float16)0.0625f : fh;
    const _Float16 fha = T == kGgmlQ4K ? (_Float16)(-64.0f) * fh : (_Float16)(-1024.0f) * fh;
    const half2_t mh = {fhm, fhm}, ah = {fha, fha};
    const uint32_t w[4] = {r.qs[g].x, r.qs[g].y, r.qs[g].z, r.qs[g].w};
    const uint32_t h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // byte pairs (0, 1) and (2, 3) of word i into the two 16-bit halves
        half2_t lo2[2], hi2[2];
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const uint32_t sel = p ? 0x0C030C02u : 0x0C010C00u;
            if constexpr (T == kGgmlQ4K) {
                const uint32_t sp = __builtin_amdgcn_perm(w[i], w[i], sel);
                lo2[p] = __builtin_bit_cast(half2_t, (sp & dk.lo) | dk.magic);  // 1024 + n
                hi2[p] = __builtin_bit_cast(half2_t, (sp & dk.hi) | dk.magic);  // 1024 + 16 n
            } else {
                // five-bit codes: the qh bit of sub-block 2g (low) / 2g + 1 (high) at bit 4
                const uint32_t cl = (w[i] & 0x0F0F0F0Fu) | (((h[i] >> (2 * g)) & 0x01010101u) << 4);
                const uint32_t ch = ((w[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (2 * g + 1)) & 0x01010101u) << 4);
                lo2[p] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(cl, cl, sel) | dk.magic);
                hi2[p] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(ch, ch, sel) | dk.magic);
            }
            // fused (one rounding of an exact integer): the product alone may exceed 2048,
            // where f16 drops odd integers
            lo2[p] = __builtin_elementwise_fma(lo2[p], ml, al);
            hi2[p] = __builtin_elementwise_fma(hi2[p], mh, ah);
        }
        // word i holds bytes 4i .. 4i + 3: k-step (i >> 1) (low) or 2 + (i >> 1) (high),
        // elements 4 (i & 1) .. + 3
        const int ql = i >> 1, e = 4 * (i & 1);
        b[ql][e + 0] = lo2[0][0]; b[ql][e + 1] = lo2[0][1];
        b[ql][e + 2] = lo2[1][0]; b[ql][e + 3] = lo2[1][1];
        b[2 + ql][e + 0] = hi2[0][0]; b[2 + ql][e + 1] = hi2[0][1];
        b[2 + ql][e + 2] = hi2[1][0]; b[2 + ql][e + 3] = hi2[1][1];
    }
}

// The B operand of the min product: m_0 .. m_7 of the row's super-block in lane half 0, zeros
// in lane half 1 (the upper 8 k of the instruction).
__device__ inline half8 kq_min_operand(const KqScales &s, int hf) {
    half8 m;
#pragma unroll
    for (int j = 0; j < 8; j++) m[j] = hf ? (_Float16)0.0f : (_Float16)(j < 4 ? kq_byte(s.m03, j) : kq_byte(s.m47, j - 4));
    return m;
}

// One slice of the reduction for a 32 x 256 tile over nbat super-blocks (the K-quant form of
// gemm_split_core, same thread roles and D layout): x of a super-block into LDS as hi/lo and
// its sub-block sums, the weight blocks straight into registers, one memory round trip per
// super-block.  wb[cb]: the lane's weight row of column block cb at the slice's first
// super-block; xs: the staging thread's 8 floats of its row at the slice's first chunk (null:
// a zero row).
template <int T>
__device__ __forceinline__ void gemm_split_kq(KqTiles (&sm)[2], const float *xs, const uint8_t *const (&wb)[2],
                                              int nbat, int tid, floatx16 (&acc)[2]) {
    constexpr int NB = 4;
    const int lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int si = tid >> 3, sc = tid & 7;
    const DeqConstV dk;
    zero(acc[0]);
    zero(acc[1]);
    // Super-block b + 1's x and weight blocks are loaded while b is multiplied; x goes through
    // LDS (double-buffered, one barrier per super-block), the weights stay in registers.
    float4 xu[NB], xv[NB];
    KqRegs r[2][2];  // [buffer][column block]
    auto load = [&](int b, KqRegs (&rr)[2]) {
        const bool on = b < nbat;
#pragma unroll
        for (int c = 0; c < NB; c++) {
            xu[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            xv[c] = xu[c];
            if (xs && on) {
                xu[c] = *reinterpret_cast<const float4 *>(xs + (b * NB + c) * kKC);
                xv[c] = *reinterpret_cast<const float4 *>(xs + (b * NB + c) * kKC + 4);
            }
        }
        if (on) {
#pragma unroll
            for (int cb = 0; cb < 2; cb++) kq_load<T>(rr[cb], wb[cb] + (size_t)b * KQ<T>::BYTES, hf);
        }
    };
    auto stage = [&](KqTiles &t) {
#pragma unroll
        for (int c = 0; c < NB; c++) {
            half8 h, l;
            split8(xu[c], xv[c], h, l);
            *reinterpret_cast<half8 *>(&t.x.hi[c][si][8 * sc]) = h;
            *reinterpret_cast<half8 *>(&t.x.lo[c][si][8 * sc]) = l;
            // sub-block sums: 4 staging threads (consecutive lanes) per 32 elements
            float v = ((xu[c].x + xu[c].y) + (xu[c].z + xu[c].w)) + ((xv[c].x + xv[c].y) + (xv[c].z + xv[c].w));
            v += __shfl_xor(v, 1, 64);
            v += __shfl_xor(v, 2, 64);
            if ((sc & 3) == 0) t.xsum[si][2 * c + (sc >> 2)] = v;
        }
    };
    auto compute = [&](const KqTiles &t, const KqRegs (&rr)[2]) {
        const KqScales s0 = kq_scales(rr[0].hdr), s1 = kq_scales(rr[1].hdr);
        floatx16 t0, t1;
        zero(t0);
        zero(t1);
#pragma unroll
        for (int g = 0; g < NB; g++) {
            half8 b0[4], b1[4];
            kq_operands<T>(rr[0], s0, g, b0, dk);
            kq_operands<T>(rr[1], s1, g, b1, dk);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int ko = 32 * (q >> 1) + 16 * hf + 8 * (q & 1);
                const half8 ah = *reinterpret_cast<const half8 *>(&t.x.hi[g][j][ko]);
                const half8 al = *reinterpret_cast<const half8 *>(&t.x.lo[g][j][ko]);
                t0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b0[q], t0, 0, 0, 0);
                t1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b1[q], t1, 0, 0, 0);
                t0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b0[q], t0, 0, 0, 0);
                t1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b1[q], t1, 0, 0, 0);
            }
        }
        // the min product: x sums of row j (split hi + lo) against m of the column's sub-blocks
        half8 sh, sl;
        {
            const float4 u = *reinterpret_cast<const float4 *>(&t.xsum[j][0]);
            const float4 v = *reinterpret_cast<const float4 *>(&t.xsum[j][4]);
            split8(u, v, sh, sl);
        }
        const half8 mb0 = kq_min_operand(s0, hf), mb1 = kq_min_operand(s1, hf);
        floatx16 u0, u1;
        zero(u0);
        zero(u1);
        u0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh, mb0, u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh, mb1, u1, 0, 0, 0);
        u0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(sl, mb0, u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(sl, mb1, u1, 0, 0, 0);
        // d and dmin of the lane's column (f16 at bytes 0 and 2 of the block)
        const float d0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(rr[0].hdr.x & 0xFFFFu));
        const float n0 = -(float)__builtin_bit_cast(_Float16, (uint16_t)(rr[0].hdr.x >> 16));
        const float d1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(rr[1].hdr.x & 0xFFFFu));
        const float n1 = -(float)__builtin_bit_cast(_Float16, (uint16_t)(rr[1].hdr.x >> 16));
#pragma unroll
        for (int e = 0; e < 16; e++) {
            acc[0][e] = __builtin_fmaf(n0, u0[e], __builtin_fmaf(d0, t0[e], acc[0][e]));
            acc[1][e] = __builtin_fmaf(n1, u1[e], __builtin_fmaf(d1, t1[e], acc[1][e]));
        }
    };
    load(0, r[0]);
    stage(sm[0]);
    // two super-blocks per trip so that the register buffers are indexed with constants
    for (int b = 0; b < nbat; b += 2) {
        load(b + 1, r[1]);
        __syncthreads();  // sm[0] staged (and sm[1] no longer read)
        compute(sm[0], r[0]);
        if (b + 1 >= nbat) break;  // uniform
        stage(sm[1]);
        load(b + 2, r[0]);
        __syncthreads();
        compute(sm[1], r[1]);
        if (b + 2 < nbat) stage(sm[0]);
    }
}


// ---- Q4_0 / Q5_0 / Q8_0: 32-element blocks with one f16 scale each ------------------------
//
// The reference's values (src/core/dequant/q4_0.rs, q5_0.rs, q8_0.rs): w = d * (n - 8) for the
// nibbles of Q4_0 (element e of a block: low nibble of byte e, element 16 + e: its high
// nibble), w = d * (n + 16 h - 16) for Q5_0 (the same nibbles, h = bit e of its 32-bit word of
// fifth bits) and w = d * q for the int8 codes of Q8_0.  The codes are exact in f16, the scale d is not
// foldable into them exactly, so each block's 32 elements run on the matrix cores into an
// accumulator of their own (two k-steps of v_mfma_f32_32x32x16_f16, x split hi + lo), which is
// then added to the row's sum times d (16 FMAs per lane).  With the k-step order of the
// K-quant loop, lane half hf takes elements 16 hf .. 16 hf + 15 of every block: Q8_0 bytes
// 16 hf .. 16 hf + 15 of its codes, Q4_0 nibble half hf of all 16 bytes.
//
// The blocks (18 / 34 bytes) are not 4-byte aligned in every position, but 256 elements are
// 144 / 272 bytes, a multiple of 16, so the alignment of block i within its 256 is fixed:
// codes start 2 mod 4 in the even blocks (read from the dword that holds d, 5 dwords, one
// byte-align per code word) and 0 mod 4 in the odd ones.  The scale of an odd block sits in
// the top half of the dword before its codes: for Q4_0 the last dword of the even block's
// read; for Q8_0 the last dword that lane half 1 reads of the even block (lane half 0 holds
// the even block's d), and one lane-half swap per block pair gives every lane both.
struct QbRegs {
    uint4 c[8];     // block i: the 4 dwords from the lane's first read position
    uint32_t t[4];  // even block 2k: its fifth dword
    uint32_t x[4];  // Q5_0: odd block 2k + 1: its fifth dword
    uint32_t y[4];  // Q5_0: even block 2k: its sixth dword
};

template <int T>
__device__ __forceinline__ void qb_load(QbRegs &r, const uint8_t *sb, int hf) {
    typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
    constexpr int BB = T == kGgmlQ8_0 ? 34 : T == kGgmlQ5_0 ? 22 : 18;
    const int off = T == kGgmlQ8_0 ? 16 * hf : 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int at = BB * i + off + ((i & 1) ? 2 : 0);  // a multiple of 4
        const u32x4a v = *reinterpret_cast<const u32x4a *>(sb + at);
        r.c[i] = make_uint4(v[0], v[1], v[2], v[3]);
        if (!(i & 1)) r.t[i >> 1] = *reinterpret_cast<const uint32_t *>(sb + at + 16);
        if constexpr (T == kGgmlQ5_0) {
            if (i & 1)
                r.x[i >> 1] = *reinterpret_cast<const uint32_t *>(sb + at + 16);
            else
                r.y[i >> 1] = *reinterpret_cast<const uint32_t *>(sb + at + 20);
        }
    }
}

// The lane's 16 code bytes of block i (4 words, byte 4w + b: code byte 4w + b of its share);
// Q5_0: the 16 qs bytes, and its qh word in *qh.
template <int T>
__device__ __forceinline__ void qb_words(const QbRegs &r, int i, uint32_t (&w)[4], uint32_t *qh = nullptr) {
    const uint4 c = r.c[i];
    if constexpr (T == kGgmlQ5_0) {
        // even block: dwords c.x .. c.w, t, x from the block's start (d, qh, qs, next d);
        // odd block: qh, then the 16 qs bytes in c.y .. c.w and x
        if (i & 1) {
            *qh = c.x;
            w[0] = c.y; w[1] = c.z; w[2] = c.w; w[3] = r.x[i >> 1];
        } else {
            const uint32_t t = r.t[i >> 1], u = r.y[i >> 1];
            *qh = __builtin_amdgcn_alignbyte(c.y, c.x, 2);
            w[0] = __builtin_amdgcn_alignbyte(c.z, c.y, 2);
            w[1] = __builtin_amdgcn_alignbyte(c.w, c.z, 2);
            w[2] = __builtin_amdgcn_alignbyte(t, c.w, 2);
            w[3] = __builtin_amdgcn_alignbyte(u, t, 2);
        }
        return;
    }
    if (i & 1) {
        w[0] = c.x; w[1] = c.y; w[2] = c.z; w[3] = c.w;
    } else {
        const uint32_t t = r.t[i >> 1];
        w[0] = __builtin_amdgcn_alignbyte(c.y, c.x, 2);
        w[1] = __builtin_amdgcn_alignbyte(c.z, c.y, 2);
        w[2] = __builtin_amdgcn_alignbyte(c.w, c.z, 2);
        w[3] = __builtin_amdgcn_alignbyte(t, c.w, 2);
    }
}

// The scales of blocks 2k and 2k + 1.
template <int T>
__device__ __forceinline__ void qb_scales(const QbRegs &r, int k, int hf, float &d0, float &d1) {
    const uint32_t lo = r.c[2 * k].x & 0xFFFFu;  // d of the even block (Q8_0: lane half 0's read)
    // d of the odd block (Q8_0: lane half 1's read; Q5_0: the even block's sixth dword)
    const uint32_t hi = (T == kGgmlQ5_0 ? r.y[k] : r.t[k]) >> 16;
    uint32_t e = lo, o = hi;
    if constexpr (T == kGgmlQ8_0) {
        const uint32_t mine = hf ? hi : lo;
        // element 0: lane half 0's value, element 1: lane half 1's, in every lane
        const auto sw = __builtin_amdgcn_permlane32_swap(mine, mine, false, false);
        e = sw[0];
        o = sw[1];
    }
    d0 = (float)__builtin_bit_cast(_Float16, (uint16_t)e);
    d1 = (float)__builtin_bit_cast(_Float16, (uint16_t)o);
}

// The B operands of block i's two k-steps: b[u] element e = code of byte 8u + e of the share
// (Q4_0: its nibble half hf), exact integers in f16.
template <int T>
__device__ __forceinline__ void qb_operands(const QbRegs &r, int i, int hf, half8 (&b)[2], const DeqConst &dk) {
    uint32_t w[4], qh = 0;
    qb_words<T>(r, i, w, &qh);
    const uint32_t hq = qh >> (16 * hf);  // Q5_0: the fifth bits of the lane's 16 elements
    const half2_t off = T == kGgmlQ8_0 ? half2_t{(_Float16)1152.0f, (_Float16)1152.0f}
                      : T == kGgmlQ5_0 ? half2_t{(_Float16)1040.0f, (_Float16)1040.0f}
                                       : half2_t{(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const uint32_t sel = p ? 0x0C030C02u : 0x0C010C00u;
            const uint32_t sp = __builtin_amdgcn_perm(w[q], w[q], sel);  // bytes 2p, 2p+1 -> halves
            uint32_t u;
            if constexpr (T == kGgmlQ8_0) {
                u = (sp ^ 0x00800080u) | dk.magic;  // 1024 + (q + 128)
            } else {
                u = ((hf ? (sp >> 4) : sp) & dk.lo) | dk.magic;  // 1024 + n
                if constexpr (T == kGgmlQ5_0) {
                    // bits 4q + 2p and 4q + 2p + 1 of hq to bit 4 of either half
                    const uint32_t b2 = hq >> (4 * q + 2 * p);
                    u |= ((b2 & 1u) << 4) | ((b2 & 2u) << 19);  // 1024 + n + 16 h
                }
            }
            const half2_t v = __builtin_bit_cast(half2_t, u) - off;
            b[q >> 1][4 * (q & 1) + 2 * p] = v[0];
            b[q >> 1][4 * (q & 1) + 2 * p + 1] = v[1];
        }
    }
}

// gemm_split_kq for Q4_0 / Q5_0 / Q8_0 rows (same thread roles, LDS x tiles and D layout).
template <int T>
__device__ __forceinline__ void gemm_split_qb(KqTiles (&sm)[2], const float *xs, const uint8_t *const (&wb)[2],
                                              int nbat, int tid, floatx16 (&acc)[2]) {
    constexpr int NB = 4;
    const int lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int si = tid >> 3, sc = tid & 7;
    const DeqConstV dk;
    zero(acc[0]);
    zero(acc[1]);
    float4 xu[NB], xv[NB];
    QbRegs r[2][2];  // [buffer][column block]
    auto load = [&](int b, QbRegs (&rr)[2]) {
        const bool on = b < nbat;
#pragma unroll
        for (int c = 0; c < NB; c++) {
            xu[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            xv[c] = xu[c];
            if (xs && on) {
                xu[c] = *reinterpret_cast<const float4 *>(xs + (b * NB + c) * kKC);
                xv[c] = *reinterpret_cast<const float4 *>(xs + (b * NB + c) * kKC + 4);
            }
        }
        if (on) {
#pragma unroll
            for (int cb = 0; cb < 2; cb++) qb_load<T>(rr[cb], wb[cb] + (size_t)b * KQ<T>::BYTES, hf);
        }
    };
    auto stage = [&](KqTiles &t) {
#pragma unroll
        for (int c = 0; c < NB; c++) {
            half8 h, l;
            split8(xu[c], xv[c], h, l);
            *reinterpret_cast<half8 *>(&t.x.hi[c][si][8 * sc]) = h;
            *reinterpret_cast<half8 *>(&t.x.lo[c][si][8 * sc]) = l;
        }
    };
    auto compute = [&](const KqTiles &t, const QbRegs (&rr)[2]) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float d[2][2];
            qb_scales<T>(rr[0], k, hf, d[0][0], d[0][1]);
            qb_scales<T>(rr[1], k, hf, d[1][0], d[1][1]);
#pragma unroll
            for (int ii = 0; ii < 2; ii++) {
                const int i = 2 * k + ii, g = i >> 1;  // block i: chunk g, k-steps 2 (i & 1) + u
                half8 b0[2], b1[2];
                qb_operands<T>(rr[0], i, hf, b0, dk);
                qb_operands<T>(rr[1], i, hf, b1, dk);
                floatx16 t0, t1;
                zero(t0);
                zero(t1);
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int q = 2 * (i & 1) + u;
                    const int ko = 32 * (q >> 1) + 16 * hf + 8 * (q & 1);
                    const half8 ah = *reinterpret_cast<const half8 *>(&t.x.hi[g][j][ko]);
                    const half8 al = *reinterpret_cast<const half8 *>(&t.x.lo[g][j][ko]);
                    t0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b0[u], t0, 0, 0, 0);
                    t1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b1[u], t1, 0, 0, 0);
                    t0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b0[u], t0, 0, 0, 0);
                    t1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b1[u], t1, 0, 0, 0);
                }
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    acc[0][e] = __builtin_fmaf(d[0][ii], t0[e], acc[0][e]);
                    acc[1][e] = __builtin_fmaf(d[1][ii], t1[e], acc[1][e]);
                }
            }
        }
    };
    load(0, r[0]);
    stage(sm[0]);
    for (int b = 0; b < nbat; b += 2) {
        load(b + 1, r[1]);
        __syncthreads();
        compute(sm[0], r[0]);
        if (b + 1 >= nbat) break;  // uniform
        stage(sm[1]);
        load(b + 2, r[0]);
        __syncthreads();
        compute(sm[1], r[1]);
        if (b + 2 < nbat) stage(sm[0]);
    }
}

// The slice loop of any block type read in the loop.
template <int T>
__device__ __forceinline__ void gemm_split_blocks(KqTiles (&sm)[2], const float *xs, const uint8_t *const (&wb)[2],
                                                  int nbat, int tid, floatx16 (&acc)[2]) {
    if constexpr (T == kGgmlQ4K || T == kGgmlQ5K)
        gemm_split_kq<T>(sm, xs, wb, nbat, tid, acc);
    else
        gemm_split_qb<T>(sm, xs, wb, nbat, tid, acc);
}

}  // namespace
}  // namespace ts
