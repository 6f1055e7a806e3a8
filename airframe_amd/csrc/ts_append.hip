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
// quantizes every position of the block that falls in the append range, stages the codes in
// LDS, and writes whole words with 128-bit stores.  Owning the block means no two workgroups
// ever write the same V word, although a word interleaves 8 positions.
#include "ts_store128.h"

namespace ts {
namespace {

// Nibble n of the result = byte n of x (every byte < 16).
__device__ inline uint32_t pack8(uint64_t x) {
    x = (x | (x >> 4)) & 0x00FF00FF00FF00FFull;
    x = (x | (x >> 8)) & 0x0000FFFF0000FFFFull;
    x = (x | (x >> 16)) & 0x00000000FFFFFFFFull;
    return (uint32_t)x;
}

// start: first position written for this sequence (d_start[s] if d_start, else fixed_start).
// Source row of position p: src[((s*ld_tok) + (p - start)) * H + h][hd].
//
// Wave w quantizes positions w, w+4, ... of the block.  Every load of the wave is issued
// before any reduction (positions outside the append range load a valid neighbour's row and
// are never written), reductions use DPP and permlane swaps, and the quotient takes the
// reciprocal fast path of encode_fast.  Codes are staged in LDS as K [position][dim] and V
// [dim][position] bytes, so each output word is one 8-byte (K) or two 4-byte (V) LDS reads.
template <int HD>
__global__ __launch_bounds__(256) void quantize_rows_kernel(KvLayerView L, const float *__restrict__ k,
                                                             const float *__restrict__ v,
                                                             const int32_t *__restrict__ d_start,
                                                             int32_t fixed_start, int32_t count,
                                                             int32_t ld_tok,
                                                             const float *__restrict__ rope,
                                                             int32_t rope_pairs) {
    constexpr int PAIRS = HD / 2;
    constexpr int NTD = HD / 16;          // 16-dim tiles of the V block layout
    constexpr int PPW = kBlk / 4;         // positions per wave
    constexpr int NJ = (PAIRS + 63) / 64; // pairs per lane
    constexpr int VROW = kBlk + 4;        // V staging row (bytes): 36 keeps lane writes 2-way
    __shared__ __align__(16) uint8_t kc[kBlk][HD];
    __shared__ __align__(16) uint8_t vc[HD][VROW];
    __shared__ float ksc[kBlk], vsc[kBlk];
    const int s = blockIdx.z, h = blockIdx.y;
    const int start = d_start ? d_start[s] : fixed_start;
    const int end = start + count;
    const int blk = start / kBlk + blockIdx.x;
    const int p0 = blk * kBlk;
    if (p0 >= end) return;
    const int lo = max(p0, start), hi = min(p0 + kBlk, end);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    float kx[PPW][2 * NJ], vx[PPW][2 * NJ];
#pragma unroll
    for (int ii = 0; ii < PPW; ii++) {
        const int pc = min(max(p0 + wave + 4 * ii, lo), hi - 1);
        const size_t src = (((size_t)s * ld_tok + (pc - start)) * L.H + h) * HD;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int pi = min(lane + 64 * j, PAIRS - 1);  // lanes past the row repeat its end
            const float2 kk = *reinterpret_cast<const float2 *>(k + src + 2 * pi);
            const float2 vv = *reinterpret_cast<const float2 *>(v + src + 2 * pi);
            kx[ii][2 * j] = kk.x;
            kx[ii][2 * j + 1] = kk.y;
            vx[ii][2 * j] = vv.x;
            vx[ii][2 * j + 1] = vv.y;
        }
    }
    if (L.kn) {
        // QK norm of every K row before RoPE, the squares summed in order across the lanes
#pragma unroll
        for (int ii = 0; ii < PPW; ii++) {
            static_assert(NJ == 1, "the ordered sum reads one pair per lane");
            const float ns = qk_norm_scale_from_sum(
                ordered_sum_pairs(sq_rn(kx[ii][0]), sq_rn(kx[ii][1]), PAIRS), HD, L.norm_eps);
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int pi = min(lane + 64 * j, PAIRS - 1);
                kx[ii][2 * j] = qk_norm_apply(kx[ii][2 * j], ns, L.kn[2 * pi]);
                kx[ii][2 * j + 1] = qk_norm_apply(kx[ii][2 * j + 1], ns, L.kn[2 * pi + 1]);
            }
        }
    }
    float km[PPW], vm[PPW];
#pragma unroll
    for (int ii = 0; ii < PPW; ii++) {
        const int pc = min(max(p0 + wave + 4 * ii, lo), hi - 1);
        km[ii] = 0.0f;
        vm[ii] = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int pi = min(lane + 64 * j, PAIRS - 1);
            if (rope && pi < rope_pairs)
                rope_rotate(kx[ii][2 * j], kx[ii][2 * j + 1],
                            *reinterpret_cast<const float2 *>(
                                rope + ((size_t)rot_of(L, s, pc) * rope_pairs + pi) * 2));
            km[ii] = fmaxf(km[ii], fmaxf(fabsf(kx[ii][2 * j]), fabsf(kx[ii][2 * j + 1])));
            vm[ii] = fmaxf(vm[ii], fmaxf(fabsf(vx[ii][2 * j]), fabsf(vx[ii][2 * j + 1])));
        }
    }
#pragma unroll
    for (int ii = 0; ii < PPW; ii++) {
        km[ii] = wave_max_nonneg(km[ii]);
        vm[ii] = wave_max_nonneg(vm[ii]);
    }
#pragma unroll
    for (int ii = 0; ii < PPW; ii++) {
        const int i = wave + 4 * ii;
        const float ks = quant_scale(km[ii]);
        const float vs = quant_scale(vm[ii]);
        const float kr = __builtin_amdgcn_rcpf(ks), vr = __builtin_amdgcn_rcpf(vs);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int pi = lane + 64 * j;
            if (pi < PAIRS) {
                *reinterpret_cast<uint16_t *>(&kc[i][2 * pi]) =
                    (uint16_t)(encode_fast(kx[ii][2 * j], ks, kr) | (encode_fast(kx[ii][2 * j + 1], ks, kr) << 8));
                vc[2 * pi][i] = (uint8_t)encode_fast(vx[ii][2 * j], vs, vr);
                vc[2 * pi + 1][i] = (uint8_t)encode_fast(vx[ii][2 * j + 1], vs, vr);
            }
        }
        if (lane == 0) {
            ksc[i] = ks;
            vsc[i] = vs;
        }
    }
    __syncthreads();

    const size_t row = (size_t)s * L.H + h;
    // K rows: 16-byte quads, HD/32 per position.
    {
        constexpr int QPP = HD / 32;
        const int i = tid / QPP, quad = tid % QPP;
        if (tid < kBlk * QPP && p0 + i >= lo && p0 + i < hi) {
            const uint64_t *src = reinterpret_cast<const uint64_t *>(&kc[i][quad * 32]);
            const uint4 w = make_uint4(pack8(src[0]), pack8(src[1]), pack8(src[2]), pack8(src[3]));
            reinterpret_cast<uint4 *>(L.kp + (row * L.P + p0 + i) * (HD / 2))[quad] = w;
        }
    }
    if (tid < kBlk && p0 + tid >= lo && p0 + tid < hi) {
        L.ks[row * L.P + p0 + tid] = ksc[tid];
        L.vs[row * L.P + p0 + tid] = vsc[tid];
    }
    // V block: HD*4 words, 4 consecutive words per thread.  Word (g, dl, td) holds dim
    // 16 td + dl at positions 4g..4g+3 (nibbles 0-3) and 16+4g..16+4g+3 (nibbles 4-7).
    if (tid < HD) {
        const bool full = (lo == p0 && hi == p0 + kBlk);
        uint4 *dst = reinterpret_cast<uint4 *>(L.vp + (row * (L.P / kBlk) + blk) * (HD * 16)) + tid;
        uint4 old = make_uint4(0, 0, 0, 0);
        if (!full) old = *dst;
        uint32_t w[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int widx = tid * 4 + u;
            const int lanei = widx / NTD, td = widx % NTD;
            const int g = lanei >> 4, dl = lanei & 15;
            const int d = 16 * td + dl;
            const uint64_t x = (uint64_t)*reinterpret_cast<const uint32_t *>(&vc[d][4 * g]) |
                               ((uint64_t)*reinterpret_cast<const uint32_t *>(&vc[d][16 + 4 * g]) << 32);
            const uint32_t fresh = pack8(x);
            uint32_t keep = 0;  // nibbles of positions outside [lo, hi)
#pragma unroll
            for (int n = 0; n < 8; n++) {
                const int i = (n < 4) ? (4 * g + n) : (16 + 4 * g + (n - 4));
                if (p0 + i < lo || p0 + i >= hi) keep |= 0xFu << (4 * n);
            }
            w[u] = (w[u] & keep) | (fresh & ~keep);
        }
        *dst = make_uint4(w[0], w[1], w[2], w[3]);
    }
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
    const int end = start + count;
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
        const float4 *ks4 = reinterpret_cast<const float4 *>(k + (((size_t)s * ld_tok + (pc - start)) * L.H + h) * HD + 8 * l);
        const float4 *vs4 = reinterpret_cast<const float4 *>(v + (((size_t)s * ld_tok + (pc - start)) * L.H + h) * HD + 8 * l);
        const float4 a = ks4[0], b = ks4[1], c = vs4[0], d = vs4[1];
        kx[rd][0] = a.x; kx[rd][1] = a.y; kx[rd][2] = a.z; kx[rd][3] = a.w;
        kx[rd][4] = b.x; kx[rd][5] = b.y; kx[rd][6] = b.z; kx[rd][7] = b.w;
        vx[rd][0] = c.x; vx[rd][1] = c.y; vx[rd][2] = c.z; vx[rd][3] = c.w;
        vx[rd][4] = d.x; vx[rd][5] = d.y; vx[rd][6] = d.z; vx[rd][7] = d.w;
    }
    store_block128(L, s, h, blk, lo, hi, kx, vx, cs, rope ? rope_pairs : 0, wave, lane);
}

// One thread per (position, kv head, word): reference layout [pos][H][HD/8].
template <int HD>
__global__ void export_kernel(KvLayerView L, int seq, int pos0, int n_pos, uint32_t *kp,
                              uint32_t *vp, float *ks, float *vs) {
    constexpr int WPR = HD / 8, NTD = HD / 16;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)n_pos * L.H * WPR;
    if (idx >= total) return;
    const int u = idx % WPR;
    const int h = (idx / WPR) % L.H;
    const int pi = idx / (WPR * L.H);
    const int p = pos0 + pi;
    const size_t row = (size_t)seq * L.H + h;
    kp[idx] = reinterpret_cast<const uint32_t *>(L.kp + (row * L.P + p) * (HD / 2))[u];
    const uint32_t *vb = reinterpret_cast<const uint32_t *>(L.vp + (row * (L.P / 32) + p / 32) * (HD * 16));
    const int q = p % 32, tile = q / 16, g = (q % 16) / 4, r = q % 4, n = r + 4 * tile;
    uint32_t word = 0;
    for (int e = 0; e < 8; e++) {
        const int d = 8 * u + e, td = d / 16, dl = d % 16;
        const uint32_t src = vb[(g * 16 + dl) * NTD + td];
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
    constexpr int WPR = HD / 8;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)n_pos * L.H * WPR;
    if (idx >= total) return;
    const int u = idx % WPR;
    const int h = (idx / WPR) % L.H;
    const int p = pos0 + (int)(idx / (WPR * L.H));
    const size_t row = (size_t)seq * L.H + h;
    reinterpret_cast<uint32_t *>(L.kp + (row * L.P + p) * (HD / 2))[u] = kp[idx];
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
    constexpr int NTD = HD / 16, WPB = HD * 4;  // words per block
    const int b0 = pos0 / 32, nb = (pos0 + n_pos - 1) / 32 - b0 + 1;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)L.H * nb * WPB) return;
    const int w = idx % WPB;
    const int b = b0 + (int)((idx / WPB) % nb);
    const int h = (int)(idx / ((long)WPB * nb));
    const int g = w / (16 * NTD), dl = (w / NTD) % 16, td = w % NTD;
    const int d = 16 * td + dl;
    const size_t row = (size_t)seq * L.H + h;
    uint32_t *dst = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / 32) + b) * (HD * 16)) + w;
    uint32_t word = *dst;
#pragma unroll
    for (int n = 0; n < 8; n++) {
        const int p = 32 * b + (n < 4 ? 4 * g + n : 16 + 4 * g + n - 4);
        if (p >= pos0 && p < pos0 + n_pos) {
            const uint32_t src = vp[((size_t)(p - pos0) * L.H + h) * (HD / 8) + d / 8];
            word = (word & ~(0xFu << (4 * n))) | (((src >> (4 * (d % 8))) & 0xFu) << (4 * n));
        }
    }
    *dst = word;
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
    if (L.hd == 128)
        quantize_rows128_kernel<<<grid, 256, 0, st>>>(L, k, v, d_start, fixed_start, count, ld_tok, rope, rope_pairs);
    else if (L.hd == 64)
        quantize_rows_kernel<64><<<grid, 256, 0, st>>>(L, k, v, d_start, fixed_start, count, ld_tok, rope, rope_pairs);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_export(const KvLayerView &L, int seq, int pos0, int n_pos, uint32_t *kp,
                         uint32_t *vp, float *ks, float *vs, hipStream_t st) {
    const long total = (long)n_pos * L.H * (L.hd / 8);
    const int blocks = (int)((total + 255) / 256);
    if (L.hd == 128)
        export_kernel<128><<<blocks, 256, 0, st>>>(L, seq, pos0, n_pos, kp, vp, ks, vs);
    else if (L.hd == 64)
        export_kernel<64><<<blocks, 256, 0, st>>>(L, seq, pos0, n_pos, kp, vp, ks, vs);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_import(const KvLayerView &L, int seq, int pos0, int n_pos, const uint32_t *kp,
                         const uint32_t *vp, const float *ks, const float *vs, hipStream_t st) {
    const long nk = (long)n_pos * L.H * (L.hd / 8);
    const int nb = (pos0 + n_pos - 1) / 32 - pos0 / 32 + 1;
    const long nv = (long)L.H * nb * L.hd * 4;
    if (L.hd == 128) {
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

hipError_t launch_len_update(int32_t *d_len, int n, int32_t seq, int32_t value, int mode,
                             hipStream_t st) {
    len_update_kernel<<<(n + 255) / 256, 256, 0, st>>>(d_len, n, seq, value, mode);
    return hipGetLastError();
}

}  // namespace ts
