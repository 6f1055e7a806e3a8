// ts_gemm.h -- the matrix-core loops shared by the projection kernels (the QKV projection
// with the append as epilogue, and the attention output projection): C = X W^T with X f32
// [M][K] split hi + lo into f16 and W f16 [N][K] row-major, on v_mfma_f32_32x32x16_f16.
//
// Operand layout of the 32x32x16 instruction used throughout: lane (j = lane % 32,
// hf = lane / 32) supplies row j of A and column j of B with 8 consecutive k; within a chunk of
// 64, k-step q of lane half hf covers k = 32 hf + 8 q .. + 7, so a lane's B operands of one
// chunk are 64 contiguous bytes of its weight row.  D register 4q + r of a 32 x 32 block is
// row 8q + 4hf + r, column j.
#pragma once
#include "ts_mfma.h"

namespace ts {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kKC = 64;     // k per chunk
constexpr int kAStr = 72;   // LDS row stride of the x tiles (f16): 144 B spreads the rows' banks

// The 8 x values of one staging thread as hi and lo f16 halves.
__device__ inline void split8(const float4 &u, const float4 &v, half8 &hi, half8 &lo) {
    const float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const _Float16 h = (_Float16)x[e];
        hi[e] = h;
        lo[e] = (_Float16)(x[e] - (float)h);
    }
}

__device__ inline void zero(floatx16 &a) {
#pragma unroll
    for (int e = 0; e < 16; e++) a[e] = 0.0f;
}

// x tiles of MT rows, double-buffered, for the tile loop.
template <int MT>
struct XTiles {
    _Float16 hi[2][MT][kAStr];
    _Float16 lo[2][MT][kAStr];
};

// MT = 64 WR rows x 256 columns over nch chunks, 256 WR threads: wave (wr, wc) accumulates rows
// 64 wr + 32 rb + .., columns 64 wc + 32 cb + .. in acc[rb][cb].  Staging thread (si = tid / 4,
// sc = tid % 4) owns 16 floats of x row si per chunk: xs points at them for chunk 0 (null: a
// zero row).  wp[cb]: the lane's weight row of column block cb at its chunk-0 offset 32 hf.
// xwrap: x has xwrap chunks and weight chunk c multiplies x chunk c mod xwrap (nch = 2 xwrap:
// rows of two weight planes, hi then lo, against the same x; nch = xwrap: one plane).
// Both operands run D chunks ahead: x and the weights of chunk c + D are loaded into a ring of
// D register sets while chunk c is multiplied, and x of chunk c + 1 goes to LDS (hi/lo,
// double-buffered) after chunk c's matrix work, so each load has D - 1 iterations to arrive.
// D = 3 keeps two waves per SIMD; measured 10% faster than x one chunk and the weights two
// chunks ahead, while D = 4 drops to one wave per SIMD and is slower.
template <int WR, int D = 3>
__device__ __forceinline__ void gemm_tile_core(XTiles<64 * WR> &sm, const float *xs,
                                                    const _Float16 *const (&wp)[2], int nch, int xwrap,
                                                    int tid, floatx16 (&acc)[2][2]) {
    const int wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5, wr = wave >> 2;
    const int si = tid >> 2, sc = tid & 3;
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < 2; cb++) zero(acc[rb][cb]);

    float4 xq[D][4];
    half8 wq[D][2][4];
    auto load = [&](float4 (&x)[4], half8 (&w)[2][4], int c) {
        const bool on = c < nch;
        const int cx = c >= xwrap ? c - xwrap : c;
#pragma unroll
        for (int u = 0; u < 4; u++)
            x[u] = (xs && on) ? *reinterpret_cast<const float4 *>(xs + cx * kKC + 4 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                w[cb][q] = on ? *reinterpret_cast<const half8 *>(wp[cb] + c * kKC + 8 * q) : (half8)(_Float16)0.0f;
    };
    auto store_x = [&](int buf, const float4 (&x)[4]) {
        half8 h, l;
        split8(x[0], x[1], h, l);
        *reinterpret_cast<half8 *>(&sm.hi[buf][si][16 * sc]) = h;
        *reinterpret_cast<half8 *>(&sm.lo[buf][si][16 * sc]) = l;
        split8(x[2], x[3], h, l);
        *reinterpret_cast<half8 *>(&sm.hi[buf][si][16 * sc + 8]) = h;
        *reinterpret_cast<half8 *>(&sm.lo[buf][si][16 * sc + 8]) = l;
    };
#pragma unroll
    for (int u = 0; u < D; u++) load(xq[u], wq[u], u);
    store_x(0, xq[0]);
    __syncthreads();

    for (int c0 = 0; c0 < nch; c0 += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int c = c0 + u;
            if (c < nch) {  // uniform
                const int buf = c & 1;
#pragma unroll
                for (int q = 0; q < 4; q++) {
#pragma unroll
                    for (int rb = 0; rb < 2; rb++) {
                        const int row = 64 * wr + 32 * rb + j;
                        const half8 ah = *reinterpret_cast<const half8 *>(&sm.hi[buf][row][32 * hf + 8 * q]);
                        const half8 al = *reinterpret_cast<const half8 *>(&sm.lo[buf][row][32 * hf + 8 * q]);
#pragma unroll
                        for (int cb = 0; cb < 2; cb++) {
                            acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, wq[u][cb][q], acc[rb][cb], 0, 0, 0);
                            acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, wq[u][cb][q], acc[rb][cb], 0, 0, 0);
                        }
                    }
                }
                if (c + 1 < nch) store_x(buf ^ 1, xq[(u + 1) % D]);
                load(xq[u], wq[u], c + D);
                __syncthreads();
            }
        }
    }
}

// LDS of gemm_split_core: x of one batch (4 chunks) as hi/lo.
struct SplitTiles {
    _Float16 hi[4][32][kAStr];
    _Float16 lo[4][32][kAStr];
};

// One slice of the reduction for a 32 x 256 tile, 256 threads, in batches of 4 chunks (256 k)
// loaded in one go -- x into LDS as hi/lo (shared by the 4 waves), the weights straight into B
// operands -- so a batch costs one memory round trip, then 64 MFMAs per wave.  Wave w
// accumulates columns 64 w + 32 cb + .. in acc[cb].  Staging thread (si = tid / 8, sc = tid % 8)
// owns 8 floats of x row si per chunk (xs at chunk 0 of the row, null: a zero row); the slice
// starts at weight chunk c0, and weight chunk c multiplies x chunk c mod xwrap (as in
// gemm_tile_core); wp[cb]: the lane's weight row of column block cb at chunk c0, offset 32 hf.
__device__ __forceinline__ void gemm_split_core(SplitTiles &sm, const float *xs, int c0, int xwrap,
                                                const _Float16 *const (&wp)[2], int nbat, int tid,
                                                floatx16 (&acc)[2]) {
    constexpr int NB = 4;
    const int lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int si = tid >> 3, sc = tid & 7;
    zero(acc[0]);
    zero(acc[1]);
    for (int b = 0; b < nbat; b++) {
        const int ko = b * NB * kKC;
        float4 xu[NB], xv[NB];
        half8 wb[NB][2][4];
#pragma unroll
        for (int c = 0; c < NB; c++) {
            xu[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            xv[c] = xu[c];
            if (xs) {
                int cx = c0 + b * NB + c;
                cx = cx >= xwrap ? cx - xwrap : cx;
                xu[c] = *reinterpret_cast<const float4 *>(xs + cx * kKC);
                xv[c] = *reinterpret_cast<const float4 *>(xs + cx * kKC + 4);
            }
#pragma unroll
            for (int cb = 0; cb < 2; cb++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    wb[c][cb][q] = *reinterpret_cast<const half8 *>(wp[cb] + ko + c * kKC + 8 * q);
        }
        if (b > 0) __syncthreads();  // the previous batch's x tiles are no longer read
#pragma unroll
        for (int c = 0; c < NB; c++) {
            half8 h, l;
            split8(xu[c], xv[c], h, l);
            *reinterpret_cast<half8 *>(&sm.hi[c][si][8 * sc]) = h;
            *reinterpret_cast<half8 *>(&sm.lo[c][si][8 * sc]) = l;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NB; c++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const half8 ah = *reinterpret_cast<const half8 *>(&sm.hi[c][j][32 * hf + 8 * q]);
                const half8 al = *reinterpret_cast<const half8 *>(&sm.lo[c][j][32 * hf + 8 * q]);
#pragma unroll
                for (int cb = 0; cb < 2; cb++) {
                    acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, wb[c][cb][q], acc[cb], 0, 0, 0);
                    acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, wb[c][cb][q], acc[cb], 0, 0, 0);
                }
            }
    }
}

// Deterministic sum of n_split partial tiles (split stride `stride` float4s) of NR rows x 256
// columns starting at src, into tile[NR][tstr] of LDS: every thread issues the loads of all
// splits of two float4 before adding them, in split order.  256 threads.
template <int NR, int MAXS>
__device__ __forceinline__ void sum_partials(const float4 *src, size_t stride, int n_split, float *tile, int tstr,
                                             int tid) {
    constexpr int PER = NR / 4;            // float4 of the rows per thread
    constexpr int U = PER < 2 ? PER : 2;   // float4 per pass
#pragma unroll
    for (int pass = 0; pass < PER / U; pass++) {
        float4 v[U][MAXS];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int sp = 0; sp < MAXS; sp++)
                if (sp < n_split) v[u][sp] = src[sp * stride + (U * pass + u) * 256 + tid];
#pragma unroll
        for (int u = 0; u < U; u++) {
            float4 acc = v[u][0];
#pragma unroll
            for (int sp = 1; sp < MAXS; sp++)
                if (sp < n_split) {
                    acc.x = acc.x + v[u][sp].x;
                    acc.y = acc.y + v[u][sp].y;
                    acc.z = acc.z + v[u][sp].z;
                    acc.w = acc.w + v[u][sp].w;
                }
            const int e4 = (U * pass + u) * 256 + tid;
            *reinterpret_cast<float4 *>(tile + (e4 / 64) * tstr + 4 * (e4 % 64)) = acc;
        }
    }
}

}  // namespace
}  // namespace ts
