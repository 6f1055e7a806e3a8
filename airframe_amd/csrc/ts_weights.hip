// ts_weights.hip -- projection weights in the GGUF formats of the reference's main_qkv and
// main_attn_proj (F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K), converted once, on the GPU,
// into the f16 row-major layout that ts_qkv_append and ts_attn_out_proj read.  The element
// values follow the reference's CPU dequantizers (src/core/dequant/), every product and
// difference rounded on its own (no contraction), and are then rounded to f16 (nearest even).
//
// One thread makes 8 consecutive elements of one block and writes them as one 16-byte store;
// it reads the block's header bytes itself (cached: the threads of a block share them).  The
// conversion is HBM-bound: a Q4_K weight reads 0.5625 bytes and writes 2 per element.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ts_internal.h"

namespace {

typedef _Float16 half8w __attribute__((ext_vector_type(8)));

enum : int { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14 };

// elements and bytes per block of a GGML type (ggml_types.rs), or 0
__host__ __device__ inline void block_shape(int type, int &epb, int &bpb) {
    switch (type) {
        case kF32: epb = 8; bpb = 32; break;  // (groups of 8 elements)
        case kF16: epb = 8; bpb = 16; break;
        case kQ4_0: epb = 32; bpb = 18; break;
        case kQ5_0: epb = 32; bpb = 22; break;
        case kQ8_0: epb = 32; bpb = 34; break;
        case kQ4_K: epb = 256; bpb = 144; break;
        case kQ5_K: epb = 256; bpb = 176; break;
        case kQ6_K: epb = 256; bpb = 210; break;
        default: epb = 0; bpb = 0;
    }
}

__device__ inline float f16_at(const uint8_t *p) {
    const uint16_t bits = (uint16_t)(p[0] | (p[1] << 8));
    return (float)__builtin_bit_cast(_Float16, bits);
}

// q4_k.rs:134-143: 6-bit scale and min of sub-block j from the 12 packed bytes
__device__ inline void scale_min_k4(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0F) | (((q[j - 4] >> 6) & 3) << 4);
        m = (q[j + 4] >> 4) | (((q[j] >> 6) & 3) << 4);
    }
}

// Elements e0 .. e0 + 7 of block b (e0 a multiple of 8) as f32 values.
template <int T>
__device__ inline void decode8(const uint8_t *b, int e0, float (&o)[8]) {
#pragma clang fp contract(off)
    if constexpr (T == kF32) {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = __builtin_bit_cast(float, (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) |
                                                                   ((uint32_t)b[4 * i + 2] << 16) | ((uint32_t)b[4 * i + 3] << 24));
    } else if constexpr (T == kF16) {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = f16_at(b + 2 * i);
    } else if constexpr (T == kQ4_0) {  // q4_0.rs:29-54: bytes' low nibbles are elements 0..15
        const float d = f16_at(b);
        const int hi = e0 >> 4, j0 = e0 & 15;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int byte = b[2 + j0 + i];
            o[i] = (float)(((hi ? byte >> 4 : byte) & 0x0F) - 8) * d;
        }
    } else if constexpr (T == kQ5_0) {  // q5_0.rs:46-86: the fifth bit of element e is qh bit e
        const float d = f16_at(b);
        const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        const int hi = e0 >> 4, j0 = e0 & 15;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int byte = b[6 + j0 + i];
            const int v = (((hi ? byte >> 4 : byte) & 0x0F) | (int)(((qh >> (e0 + i)) & 1) << 4)) - 16;
            o[i] = (float)v * d;
        }
    } else if constexpr (T == kQ8_0) {  // q8_0.rs:37-53
        const float d = f16_at(b);
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (float)(int8_t)b[2 + e0 + i] * d;
    } else if constexpr (T == kQ4_K || T == kQ5_K) {
        // q4_k.rs:75-123, q5_k.rs:74-143: 64-element chunk c, sub-block 2c (low nibbles of its
        // 32 bytes) then 2c + 1 (high nibbles); each value (d * sc) * q - dmin * m
        const float d = f16_at(b), dmin = f16_at(b + 2);
        const int c = e0 >> 6, sub = (e0 >> 5) & 1, l0 = e0 & 31;
        int sc, m;
        scale_min_k4(2 * c + sub, b + 4, sc, m);
        const float ds = d * (float)sc, dm = dmin * (float)m;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float q;
            if constexpr (T == kQ4_K) {
                const int byte = b[16 + 32 * c + l0 + i];
                q = (float)(sub ? byte >> 4 : byte & 0x0F);
            } else {
                const int byte = b[48 + 32 * c + l0 + i];
                const float hb = (float)((b[16 + l0 + i] >> (2 * c + sub)) & 1);
                q = (float)(sub ? byte >> 4 : byte & 0x0F) + hb * 16.0f;
            }
            const float a = ds * q;
            o[i] = a - dm;
        }
    } else {  // kQ6_K, q6_k.rs:72-131: half h of 128, part p of 32: (d * sc) * (q6 - 32)
        const int h = e0 >> 7, p = (e0 >> 5) & 3, l0 = e0 & 31;
        const float d = f16_at(b + 208);
        const int8_t *scl = reinterpret_cast<const int8_t *>(b + 192);
        const float ds = d * (float)scl[8 * h + (l0 >> 4) + 2 * p];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int l = l0 + i;
            const int lo = b[64 * h + l + (p & 1) * 32];
            const int q = (((p >> 1) ? lo >> 4 : lo & 0x0F) | (((b[128 + 32 * h + l] >> (2 * p)) & 3) << 4)) - 32;
            o[i] = ds * (float)q;
        }
    }
}

// PLANES 1: dst rows of n_cols f16.  PLANES 2: rows of 2 n_cols, the value rounded to f16 (hi)
// then the rest, v - hi (exact in f32), rounded to f16 (lo).
template <int T, int PLANES>
__global__ __launch_bounds__(256) void weights_to_f16_kernel(const uint8_t *__restrict__ src, uint64_t n8,
                                                             uint32_t cols8, half8w *__restrict__ dst) {
    int epb, bpb;
    block_shape(T, epb, bpb);
    const int gpb = epb / 8;  // groups of 8 per block
    for (uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x; g < n8; g += (uint64_t)gridDim.x * 256) {
        const uint64_t blk = g / gpb;
        const int e0 = (int)(g - blk * gpb) * 8;
        float o[8];
        decode8<T>(src + blk * bpb, e0, o);
        half8w h, l;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // The f32 value and the f32 rest are rounded first, each then converted to f16 on
            // its own: without the register barriers the compiler folds the last product or
            // the subtraction into the conversion (v_fma_mixlo_f16, one rounding instead of
            // two), and the f16 results differed from the reference's values rounded to f16.
            float v = o[i];
            asm volatile("" : "+v"(v));
            h[i] = (_Float16)v;
            float r = v - (float)h[i];
            asm volatile("" : "+v"(r));
            l[i] = (_Float16)r;
        }
        if (PLANES == 1) {
            dst[g] = h;
        } else {
            const uint64_t row = g / cols8, c8 = g - row * cols8;
            dst[row * 2 * cols8 + c8] = h;
            dst[row * 2 * cols8 + cols8 + c8] = l;
        }
    }
}

}  // namespace

extern "C" int ts_weights_src_bytes(int32_t ggml_type, int64_t n_rows, int64_t n_cols, uint64_t *bytes) {
    int epb, bpb;
    block_shape(ggml_type, epb, bpb);
    if (!bytes || n_rows <= 0 || n_cols <= 0) return TS_ERR_INVALID;
    if (!epb) return TS_ERR_UNSUPPORTED;
    if (n_cols % epb) return TS_ERR_INVALID;
    *bytes = (uint64_t)n_rows * (uint64_t)(n_cols / epb) * (uint64_t)bpb;
    return TS_OK;
}

static int weights_convert(int32_t ggml_type, const void *d_src, int64_t n_rows, int64_t n_cols, uint16_t *d_dst,
                           void *stream, int planes) {
    uint64_t bytes;
    const int rc = ts_weights_src_bytes(ggml_type, n_rows, n_cols, &bytes);
    if (rc) return rc;
    if (!d_src || !d_dst || ((uintptr_t)d_dst & 15)) return TS_ERR_INVALID;
    const uint64_t n8 = (uint64_t)n_rows * (uint64_t)n_cols / 8;
    const uint32_t cols8 = (uint32_t)(n_cols / 8);
    const int grid = (int)std::min<uint64_t>((n8 + 255) / 256, 8192);
    const hipStream_t st = (hipStream_t)stream;
    const uint8_t *s = (const uint8_t *)d_src;
    half8w *d = reinterpret_cast<half8w *>(d_dst);
#define TS_CONVERT(T)                                                                        \
    (planes == 1 ? (weights_to_f16_kernel<T, 1><<<grid, 256, 0, st>>>(s, n8, cols8, d), 0) \
                 : (weights_to_f16_kernel<T, 2><<<grid, 256, 0, st>>>(s, n8, cols8, d), 0))
    switch (ggml_type) {
        case kF32: TS_CONVERT(kF32); break;
        case kF16: TS_CONVERT(kF16); break;
        case kQ4_0: TS_CONVERT(kQ4_0); break;
        case kQ5_0: TS_CONVERT(kQ5_0); break;
        case kQ8_0: TS_CONVERT(kQ8_0); break;
        case kQ4_K: TS_CONVERT(kQ4_K); break;
        case kQ5_K: TS_CONVERT(kQ5_K); break;
        case kQ6_K: TS_CONVERT(kQ6_K); break;
        default: return TS_ERR_UNSUPPORTED;
    }
#undef TS_CONVERT
    return hipGetLastError() == hipSuccess ? TS_OK : TS_ERR_HIP;
}

extern "C" int ts_weights_to_f16(int32_t ggml_type, const void *d_src, int64_t n_rows, int64_t n_cols,
                                 uint16_t *d_dst, void *stream) {
    return weights_convert(ggml_type, d_src, n_rows, n_cols, d_dst, stream, 1);
}

extern "C" int ts_weights_to_f16x2(int32_t ggml_type, const void *d_src, int64_t n_rows, int64_t n_cols,
                                   uint16_t *d_dst, void *stream) {
    return weights_convert(ggml_type, d_src, n_rows, n_cols, d_dst, stream, 2);
}
