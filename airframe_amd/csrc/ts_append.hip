// ts_append.hip -- RoPE-fused INT4 quantize-on-append for gfx950, plus the cache export and
// length-update kernels.
//
// Quantiser (bit-exact with cpu_quantize, src/backend/bindless/test_int4_parity.rs:56-75, and
// sh_quantize_kv.wgsl:56-89 apart from its half-to-even round): per head vector,
// scale = max|x| / 7 (1 when max|x| == 0), code = clamp(round_half_away(x/scale) + 8, 1, 15).
// K is first rotated at its absolute position (src/ops/reference/rope.rs:186-196) with the
// host-built table.  All arithmetic here is IEEE f32 with explicit round-to-nearest intrinsics
// (no contraction, correctly rounded division), which is what makes codes and scales
// identical to the CPU quantizer.
//
// One workgroup (4 waves) owns one 32-position V block of one (sequence, kv head): it
// quantizes every position of the block that falls in the append range from registers and
// writes the words itself (ts_store.h: each wave assembles the V words of one key group with
// lane swaps).  Owning the block means no two workgroups ever write the same V word, although
// a word interleaves 8 positions.
#include <algorithm>

#include "ts_store.h"

namespace ts {
namespace {

// hd = 64: 8 lanes per position, lane l holding dims 8l..8l+7 -- exactly K word l.  Wave w
// takes the 8 positions of V key group g = w (lane group r8 = lane / 8 holds position
// 4w + r8 % 4 + 16 (r8 / 4)), so store_block64 assembles the V words inside the wave.  No LDS.
// Source row of position p: src[((s*ld_tok) + (p - start)) * H + h][hd]; start is d_start[s]
// if d_start, else fixed_start.  Positions outside the append range load a valid neighbour's
// row and are never written.
__global__ __launch_bounds__(256) void quantize_rows64_kernel(KvLayerView L, const float *__restrict__ k,
                                                               const float *__restrict__ v,
                                                               const int32_t *__restrict__ d_start,
                                                               int32_t fixed_start, int32_t count,
                                                               int32_t ld_tok,
                                                               const float *__restrict__ rope,
                                                               int32_t rope_pairs) {
    constexpr int HD = 64;
    const int s = blockIdx.z, h = blockIdx.y;
    const int start = d_start ? d_start[s] : fixed_start;
    const int end = min(start + count, L.P);  // (a graph replayed past capacity writes nothing past it)
    const int blk = start / kBlk + blockIdx.x;
    const int p0 = blk * kBlk;
    if (p0 >= end) return;
    const int lo = max(p0, start), hi = min(p0 + kBlk, end);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r8 = lane >> 3, l = lane & 7;
    const int pc = min(max(p0 + 4 * wave + (r8 & 3) + 16 * (r8 >> 2), lo), hi - 1);
    float2 cs[4];
    rope_cs4(L, s, pc, rope, rope_pairs, l, cs);
    // rows of hdr floats; the stored dims past hdr quantize zeros (code 8)
    // (lanes past the row load its first dims, unconditionally, and drop them)
    const bool in = 8 * l < L.hdr;
    const size_t src = (((size_t)s * ld_tok + (pc - start)) * L.H + h) * L.hdr + 8 * (in ? l : 0);
    const float4 a0 = keep4(in, *reinterpret_cast<const float4 *>(k + src));
    const float4 a1 = keep4(in, *reinterpret_cast<const float4 *>(k + src + 4));
    const float4 b0 = keep4(in, *reinterpret_cast<const float4 *>(v + src));
    const float4 b1 = keep4(in, *reinterpret_cast<const float4 *>(v + src + 4));
    float kx[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float vx[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    store_block64(L, s, h, blk, lo, hi, kx, vx, cs, rope ? rope_pairs : 0, wave, lane);
}

// hd = 128: 16 lanes per position, lane l holding dims 8l..8l+7 -- exactly K word l.  Wave w
// takes positions 4w + r and 16 + 4w + r (r = lane / 16): the two halves of V words with
// g = w, so the V words are assembled across the wave's 4 rows with permlane swaps and
// written by the wave itself.  No LDS.  Max reductions: 4 DPP steps within a 16-lane row.
__global__ __launch_bounds__(256) void quantize_rows128_kernel(KvLayerView L, const float *__restrict__ k,
                                                                const float *__restrict__ v,
                                                                const int32_t *__restrict__ d_start,
                                                                int32_t fixed_start, int32_t count,
                                                                int32_t ld_tok,
                                                                const float *__restrict__ rope,
                                                                int32_t rope_pairs) {
    constexpr int HD = 128;
    const int s = blockIdx.z, h = blockIdx.y;
    const int start = d_start ? d_start[s] : fixed_start;
    const int end = min(start + count, L.P);  // (a graph replayed past capacity writes nothing past it)
    const int blk = start / kBlk + blockIdx.x;
    const int p0 = blk * kBlk;
    if (p0 >= end) return;
    const int lo = max(p0, start), hi = min(p0 + kBlk, end);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane >> 4, l = lane & 15;
    const size_t row = (size_t)s * L.H + h;

    float kx[2][8], vx[2][8];
    float2 cs[2][4];  // rotation of each pair (identity without a table or past rope_dim)
#pragma unroll
    for (int rd = 0; rd < 2; rd++) {
        const int pc = min(max(p0 + 16 * rd + 4 * wave + r, lo), hi - 1);
        const int pr = rot_of(L, s, pc);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int pair = 4 * l + m;
            cs[rd][m] = (rope && pair < rope_pairs)
                            ? *reinterpret_cast<const float2 *>(rope + ((size_t)pr * rope_pairs + pair) * 2)
                            : make_float2(1.0f, 0.0f);
        }
        // rows of hdr floats; the stored dims past hdr quantize zeros (code 8)
        // (lanes past the row load its first dims, unconditionally, and drop them)
        const bool in = 8 * l < L.hdr;
        const size_t src = (((size_t)s * ld_tok + (pc - start)) * L.H + h) * L.hdr + 8 * (in ? l : 0);
        const float4 *ks4 = reinterpret_cast<const float4 *>(k + src);
        const float4 *vs4 = reinterpret_cast<const float4 *>(v + src);
        const float4 a = keep4(in, ks4[0]), b = keep4(in, ks4[1]), c = keep4(in, vs4[0]), d = keep4(in, vs4[1]);
        kx[rd][0] = a.x; kx[rd][1] = a.y; kx[rd][2] = a.z; kx[rd][3] = a.w;
        kx[rd][4] = b.x; kx[rd][5] = b.y; kx[rd][6] = b.z; kx[rd][7] = b.w;
        vx[rd][0] = c.x; vx[rd][1] = c.y; vx[rd][2] = c.z; vx[rd][3] = c.w;
        vx[rd][4] = d.x; vx[rd][5] = d.y; vx[rd][6] = d.z; vx[rd][7] = d.w;
    }
    store_block128(L, s, h, blk, lo, hi, kx, vx, cs, rope ? rope_pairs : 0, wave, lane);
}

// hd = 256: 32 lanes per position, lane l holding dims 8l..8l+7 -- K word l; two rows per wave
// and four rounds (store_block256).  No LDS.
__global__ __launch_bounds__(256) void quantize_rows256_kernel(KvLayerView L, const float *__restrict__ k,
                                                                const float *__restrict__ v,
                                                                const int32_t *__restrict__ d_start,
                                                                int32_t fixed_start, int32_t count,
                                                                int32_t ld_tok,
                                                                const float *__restrict__ rope,
                                                                int32_t rope_pairs) {
    const int s = blockIdx.z, h = blockIdx.y;
    const int start = d_start ? d_start[s] : fixed_start;
    const int end = min(start + count, L.P);  // (a graph replayed past capacity writes nothing past it)
    const int blk = start / kBlk + blockIdx.x;
    const int p0 = blk * kBlk;
    if (p0 >= end) return;
    const int lo = max(p0, start), hi = min(p0 + kBlk, end);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane >> 5, l = lane & 31;

    float kx[4][8], vx[4][8];
    float2 cs[4][4];
#pragma unroll
    for (int rd = 0; rd < 4; rd++) {
        const int pc = min(max(p0 + 4 * wave + 2 * (rd & 1) + r + 16 * (rd >> 1), lo), hi - 1);
        const int pr = rot_of(L, s, pc);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int pair = 4 * l + m;
            cs[rd][m] = (rope && pair < rope_pairs)
                            ? *reinterpret_cast<const float2 *>(rope + ((size_t)pr * rope_pairs + pair) * 2)
                            : make_float2(1.0f, 0.0f);
        }
        // rows of hdr floats; the stored dims past hdr quantize zeros (code 8)
        const bool in = 8 * l < L.hdr;
        const size_t src = (((size_t)s * ld_tok + (pc - start)) * L.H + h) * L.hdr + 8 * (in ? l : 0);
        const float4 *ks4 = reinterpret_cast<const float4 *>(k + src);
        const float4 *vs4 = reinterpret_cast<const float4 *>(v + src);
        const float4 a = keep4(in, ks4[0]), b = keep4(in, ks4[1]), c = keep4(in, vs4[0]), d = keep4(in, vs4[1]);
        kx[rd][0] = a.x; kx[rd][1] = a.y; kx[rd][2] = a.z; kx[rd][3] = a.w;
        kx[rd][4] = b.x; kx[rd][5] = b.y; kx[rd][6] = b.z; kx[rd][7] = b.w;
        vx[rd][0] = c.x; vx[rd][1] = c.y; vx[rd][2] = c.z; vx[rd][3] = c.w;
        vx[rd][4] = d.x; vx[rd][5] = d.y; vx[rd][6] = d.z; vx[rd][7] = d.w;
    }
    store_block256(L, s, h, blk, lo, hi, kx, vx, cs, rope ? rope_pairs : 0, wave, lane);
}

// One thread per (position, kv head, word): reference layout [pos][H][HD/8].
template <int HD>
__global__ void export_kernel(KvLayerView L, int seq, int pos0, int n_pos, uint32_t *kp,
                              uint32_t *vp, float *ks, float *vs) {
    const int WPR = L.hdr / 8;  // the reference row: hdr dims
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)n_pos * L.H * WPR;
    if (idx >= total) return;
    const int u = idx % WPR;
    const int h = (idx / WPR) % L.H;
    const int pi = idx / (WPR * L.H);
    const int p = pos0 + pi;
    const size_t row = (size_t)seq * L.H + h;
    kp[idx] = reinterpret_cast<const uint32_t *>(L.kp + row * L.P * (HD / 2))[k_word_idx<HD>(p, u)];
    const uint32_t *vb = reinterpret_cast<const uint32_t *>(L.vp + (row * (L.P / 32) + p / 32) * (HD * 16));
    const int q = p % 32, tile = q / 16, g = (q % 16) / 4, r = q % 4, n = r + 4 * tile;
    uint32_t word = 0;
    for (int e = 0; e < 8; e++) {
        const int d = 8 * u + e, td = d / 16, dl = d % 16;
        const uint32_t src = vb[v_word_idx(g * 16 + dl, td)];
        word |= ((src >> (4 * n)) & 0xFu) << (4 * e);
    }
    vp[idx] = word;
    if (u == 0) {
        ks[(long)pi * L.H + h] = L.ks[row * L.P + p];
        vs[(long)pi * L.H + h] = L.vs[row * L.P + p];
    }
}

// Inverse of export_kernel: positions pos0..pos0+n_pos-1 of one sequence and layer from the
// reference layout.  K words and scales: one thread per (position, kv head, word).
template <int HD>
__global__ void import_k_kernel(KvLayerView L, int seq, int pos0, int n_pos, const uint32_t *kp,
                                const float *ks, const float *vs) {
    const int WPR = L.hdr / 8;  // the reference row: hdr dims (stored words past it keep code 8)
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)n_pos * L.H * WPR;
    if (idx >= total) return;
    const int u = idx % WPR;
    const int h = (idx / WPR) % L.H;
    const int p = pos0 + (int)(idx / (WPR * L.H));
    const size_t row = (size_t)seq * L.H + h;
    reinterpret_cast<uint32_t *>(L.kp + row * L.P * (HD / 2))[k_word_idx<HD>(p, u)] = kp[idx];
    if (u == 0) {
        L.ks[row * L.P + p] = ks[idx / WPR];
        L.vs[row * L.P + p] = vs[idx / WPR];
    }
}

// V words of the 32-position blocks the range touches: one thread per (kv head, block, word);
// each nibble comes from the reference-layout source if its position is in the range and is
// kept otherwise.  Word (g, dl, td) of a block holds dim 16 td + dl at positions 4g + n
// (n < 4) and 16 + 4g + n - 4 (n >= 4).
template <int HD>
__global__ void import_v_kernel(KvLayerView L, int seq, int pos0, int n_pos, const uint32_t *vp) {
    constexpr int WPB = HD * 4;  // words per block
    const int b0 = pos0 / 32, nb = (pos0 + n_pos - 1) / 32 - b0 + 1;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)L.H * nb * WPB) return;
    const int w = idx % WPB;
    const int b = b0 + (int)((idx / WPB) % nb);
    const int h = (int)(idx / ((long)WPB * nb));
    // w = v_word_idx(16 g + dl, td)
    const int c = w >> 2, ln = c & 63, td = ((c >> 6) << 2) | (w & 3);
    const int g = ln >> 4, dl = ln & 15;
    const int d = 16 * td + dl;
    if (d >= L.hdr) return;  // a stored dim past the reference row: keeps code 8
    const size_t row = (size_t)seq * L.H + h;
    uint32_t *dst = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / 32) + b) * (HD * 16)) + w;
    uint32_t word = *dst;
#pragma unroll
    for (int n = 0; n < 8; n++) {
        const int p = 32 * b + (n < 4 ? 4 * g + n : 16 + 4 * g + n - 4);
        if (p >= pos0 && p < pos0 + n_pos) {
            const uint32_t src = vp[((size_t)(p - pos0) * L.H + h) * (L.hdr / 8) + d / 8];
            word = (word & ~(0xFu << (4 * n))) | (((src >> (4 * (d % 8))) & 0xFu) << (4 * n));
        }
    }
    *dst = word;
}

// One round of an in-place compaction move: positions [a, b) of one sequence take the K words,
// scales and V nibbles of positions [a + S, b + S), with b - a <= S, so no position is both read
// and written in the round (a V word can hold both: its writer keeps the nibbles outside
// [a, b) as they are, so a concurrent reader of those sees the same values either way).
// Work items per kv head (grid.y): the K words of [a, b) (every stored word, the padding's
// too), then the V words of the blocks [a, b) touches (one thread per word: nibble
// read-modify-write), then the positions' two scales.
template <int HD>
__global__ void shift_move_kernel(KvLayerView L, int seq, int a, int b, int S) {
    // K: whole 16-byte chunks (4 words of one row) from hd 128 on, single words at hd 64
    // (where a chunk holds two rows)
    constexpr int CW = HD >= 128 ? 4 : 1;       // words per K item
    constexpr int WPR = HD / 8 / CW, WPB = HD * 4;  // K items per row, V words per block
    const int nk = (b - a) * WPR;
    const int b0 = a / 32, nb = (b - 1) / 32 - b0 + 1;
    const int nv = nb * WPB;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)nk + nv + (b - a)) return;
    const int h = blockIdx.y;
    const size_t row = (size_t)seq * L.H + h;
    if (idx < nk) {
        const int p = a + (int)(idx / WPR), c = (int)(idx % WPR);
        uint32_t *kw = reinterpret_cast<uint32_t *>(L.kp + row * L.P * (HD / 2));
        if constexpr (CW == 4) {
            // chunk c = (g, m / 2): words 8 m + 2 g + i (m even or odd pair, i = 0, 1) of the row
            const int u = 16 * (c >> 2) + 2 * (c & 3);
            *reinterpret_cast<uint4 *>(kw + k_word_idx<HD>(p, u)) =
                *reinterpret_cast<const uint4 *>(kw + k_word_idx<HD>(p + S, u));
        } else {
            kw[k_word_idx<HD>(p, c)] = kw[k_word_idx<HD>(p + S, c)];
        }
    } else if (idx < (long)nk + nv) {
        const int i = (int)(idx - nk);
        const int w = i % WPB, blk = b0 + i / WPB;
        // w = v_word_idx(16 g + dl, td)
        const int c = w >> 2, ln = c & 63, td = ((c >> 6) << 2) | (w & 3);
        const int g = ln >> 4, dl = ln & 15;
        const uint32_t *vb = reinterpret_cast<const uint32_t *>(L.vp + row * (L.P / 32) * (HD * 16));
        uint32_t *dst = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / 32) + blk) * (HD * 16)) + w;
        uint32_t word = *dst;
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const int p = 32 * blk + (n < 4 ? 4 * g + n : 16 + 4 * g + n - 4);
            if (p < a || p >= b) continue;
            const int q = p + S, qq = q & 31;
            const int gq = (qq & 15) >> 2, nq = (qq & 3) + 4 * (qq >> 4);
            const uint32_t src = vb[(size_t)(q >> 5) * (HD * 4) + v_word_idx(gq * 16 + dl, td)];
            word = (word & ~(0xFu << (4 * n))) | (((src >> (4 * nq)) & 0xFu) << (4 * n));
        }
        *dst = word;
    } else {
        const int p = a + (int)(idx - nk - nv);
        L.ks[row * L.P + p] = L.ks[row * L.P + p + S];
        L.vs[row * L.P + p] = L.vs[row * L.P + p + S];
    }
}

// mode 0: all lengths += value; mode 1: set (seq < 0: all sequences).
__global__ void len_update_kernel(int32_t *len, int n, int32_t seq, int32_t value, int mode) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (seq >= 0 && i != seq) return;
    len[i] = mode == 0 ? len[i] + value : value;
}

}  // namespace

hipError_t launch_quantize_rows(const KvLayerView &L, const float *k, const float *v,
                                const int32_t *d_start, int32_t fixed_start, int32_t count,
                                int32_t ld_tok, const float *rope, int32_t rope_pairs,
                                int32_t max_blocks, hipStream_t st) {
    dim3 grid(max_blocks, L.H, L.S);
    if (L.hd == 256)
        quantize_rows256_kernel<<<grid, 256, 0, st>>>(L, k, v, d_start, fixed_start, count, ld_tok, rope, rope_pairs);
    else if (L.hd == 128)
        quantize_rows128_kernel<<<grid, 256, 0, st>>>(L, k, v, d_start, fixed_start, count, ld_tok, rope, rope_pairs);
    else if (L.hd == 64)
        quantize_rows64_kernel<<<grid, 256, 0, st>>>(L, k, v, d_start, fixed_start, count, ld_tok, rope, rope_pairs);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_export(const KvLayerView &L, int seq, int pos0, int n_pos, uint32_t *kp,
                         uint32_t *vp, float *ks, float *vs, hipStream_t st) {
    const long total = (long)n_pos * L.H * (L.hdr / 8);
    const int blocks = (int)((total + 255) / 256);
    if (L.hd == 256)
        export_kernel<256><<<blocks, 256, 0, st>>>(L, seq, pos0, n_pos, kp, vp, ks, vs);
    else if (L.hd == 128)
        export_kernel<128><<<blocks, 256, 0, st>>>(L, seq, pos0, n_pos, kp, vp, ks, vs);
    else if (L.hd == 64)
        export_kernel<64><<<blocks, 256, 0, st>>>(L, seq, pos0, n_pos, kp, vp, ks, vs);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_import(const KvLayerView &L, int seq, int pos0, int n_pos, const uint32_t *kp,
                         const uint32_t *vp, const float *ks, const float *vs, hipStream_t st) {
    const long nk = (long)n_pos * L.H * (L.hdr / 8);
    const int nb = (pos0 + n_pos - 1) / 32 - pos0 / 32 + 1;
    const long nv = (long)L.H * nb * L.hd * 4;
    if (L.hd == 256) {
        import_k_kernel<256><<<(int)((nk + 255) / 256), 256, 0, st>>>(L, seq, pos0, n_pos, kp, ks, vs);
        import_v_kernel<256><<<(int)((nv + 255) / 256), 256, 0, st>>>(L, seq, pos0, n_pos, vp);
    } else if (L.hd == 128) {
        import_k_kernel<128><<<(int)((nk + 255) / 256), 256, 0, st>>>(L, seq, pos0, n_pos, kp, ks, vs);
        import_v_kernel<128><<<(int)((nv + 255) / 256), 256, 0, st>>>(L, seq, pos0, n_pos, vp);
    } else if (L.hd == 64) {
        import_k_kernel<64><<<(int)((nk + 255) / 256), 256, 0, st>>>(L, seq, pos0, n_pos, kp, ks, vs);
        import_v_kernel<64><<<(int)((nv + 255) / 256), 256, 0, st>>>(L, seq, pos0, n_pos, vp);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_shift_move(const KvLayerView &L, int seq, int keep, int shift, int n_move, hipStream_t st) {
    for (int a = keep; a < keep + n_move; a += shift) {
        const int b = std::min(a + shift, keep + n_move);
        const long items = (long)(b - a) * (L.hd >= 128 ? L.hd / 32 : L.hd / 8) +
                           (long)((b - 1) / 32 - a / 32 + 1) * L.hd * 4 + (b - a);
        const dim3 grid((unsigned)((items + 255) / 256), L.H);
        if (L.hd == 256)
            shift_move_kernel<256><<<grid, 256, 0, st>>>(L, seq, a, b, shift);
        else if (L.hd == 128)
            shift_move_kernel<128><<<grid, 256, 0, st>>>(L, seq, a, b, shift);
        else if (L.hd == 64)
            shift_move_kernel<64><<<grid, 256, 0, st>>>(L, seq, a, b, shift);
        else
            return hipErrorInvalidValue;
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_len_update(int32_t *d_len, int n, int32_t seq, int32_t value, int mode,
                             hipStream_t st) {
    len_update_kernel<<<(n + 255) / 256, 256, 0, st>>>(d_len, n, seq, value, mode);
    return hipGetLastError();
}

}  // namespace ts
