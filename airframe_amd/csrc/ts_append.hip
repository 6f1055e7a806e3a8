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
#include "ts_quant.h"

namespace ts {
namespace {

constexpr int kBlk = 32;

// start: first position written for this sequence (d_start[s] if d_start, else fixed_start).
// Source row of position p: src[((s*ld_tok) + (p - start)) * H + h][hd].
template <int HD>
__global__ __launch_bounds__(256) void quantize_rows_kernel(KvLayerView L, const float *__restrict__ k,
                                                             const float *__restrict__ v,
                                                             const int32_t *__restrict__ d_start,
                                                             int32_t fixed_start, int32_t count,
                                                             int32_t ld_tok,
                                                             const float *__restrict__ rope,
                                                             int32_t rope_pairs) {
    constexpr int PAIRS = HD / 2;
    constexpr int NTD = HD / 16;  // 16-dim tiles of the V block layout
    __shared__ uint8_t kc[kBlk][HD];
    __shared__ uint8_t vc[kBlk][HD];
    __shared__ float ksc[kBlk], vsc[kBlk];

    const int s = blockIdx.z, h = blockIdx.y;
    const int start = d_start ? d_start[s] : fixed_start;
    const int end = start + count;
    const int blk = start / kBlk + blockIdx.x;
    const int p0 = blk * kBlk;
    if (p0 >= end) return;
    const int lo = max(p0, start), hi = min(p0 + kBlk, end);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int i = wave; i < kBlk; i += 4) {
        const int p = p0 + i;
        if (p < lo || p >= hi) continue;
        const size_t src = (((size_t)s * ld_tok + (p - start)) * L.H + h) * HD;
        float kx[2 * ((PAIRS + 63) / 64)], vx[2 * ((PAIRS + 63) / 64)];
        float km = 0.0f, vm = 0.0f;
#pragma unroll
        for (int j = 0; j < (PAIRS + 63) / 64; j++) {
            const int pi = lane + 64 * j;
            float a = 0.f, b = 0.f, c = 0.f, d = 0.f;
            if (pi < PAIRS) {
                float2 kk = *reinterpret_cast<const float2 *>(k + src + 2 * pi);
                float2 vv = *reinterpret_cast<const float2 *>(v + src + 2 * pi);
                a = kk.x;
                b = kk.y;
                c = vv.x;
                d = vv.y;
                if (rope && pi < rope_pairs)
                    rope_rotate(a, b, *reinterpret_cast<const float2 *>(rope + ((size_t)p * rope_pairs + pi) * 2));
            }
            kx[2 * j] = a;
            kx[2 * j + 1] = b;
            vx[2 * j] = c;
            vx[2 * j + 1] = d;
            km = fmaxf(km, fmaxf(fabsf(a), fabsf(b)));
            vm = fmaxf(vm, fmaxf(fabsf(c), fabsf(d)));
        }
        km = wave_max(km);
        vm = wave_max(vm);
        const float ks = quant_scale(km);
        const float vs = quant_scale(vm);
#pragma unroll
        for (int j = 0; j < (PAIRS + 63) / 64; j++) {
            const int pi = lane + 64 * j;
            if (pi < PAIRS) {
                kc[i][2 * pi] = (uint8_t)encode(kx[2 * j], ks);
                kc[i][2 * pi + 1] = (uint8_t)encode(kx[2 * j + 1], ks);
                vc[i][2 * pi] = (uint8_t)encode(vx[2 * j], vs);
                vc[i][2 * pi + 1] = (uint8_t)encode(vx[2 * j + 1], vs);
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
            uint32_t w[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                uint32_t word = 0;
#pragma unroll
                for (int n = 0; n < 8; n++) word |= (uint32_t)kc[i][(quad * 4 + u) * 8 + n] << (4 * n);
                w[u] = word;
            }
            uint4 *dst = reinterpret_cast<uint4 *>(L.kp + (row * L.P + p0 + i) * (HD / 2)) + quad;
            *dst = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
    if (tid < kBlk && p0 + tid >= lo && p0 + tid < hi) {
        L.ks[row * L.P + p0 + tid] = ksc[tid];
        L.vs[row * L.P + p0 + tid] = vsc[tid];
    }
    // V block: HD*4 words, 4 consecutive words per thread.
    {
        const bool full = (lo == p0 && hi == p0 + kBlk);
        if (tid < HD) {
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
                uint32_t word = w[u];
#pragma unroll
                for (int n = 0; n < 8; n++) {
                    const int i = (n < 4) ? (4 * g + n) : (16 + 4 * g + (n - 4));
                    if (p0 + i >= lo && p0 + i < hi) {
                        word &= ~(0xFu << (4 * n));
                        word |= (uint32_t)vc[i][d] << (4 * n);
                    }
                }
                w[u] = word;
            }
            *dst = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
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
        quantize_rows_kernel<128><<<grid, 256, 0, st>>>(L, k, v, d_start, fixed_start, count, ld_tok, rope, rope_pairs);
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

hipError_t launch_len_update(int32_t *d_len, int n, int32_t seq, int32_t value, int mode,
                             hipStream_t st) {
    len_update_kernel<<<(n + 255) / 256, 256, 0, st>>>(d_len, n, seq, value, mode);
    return hipGetLastError();
}

}  // namespace ts
