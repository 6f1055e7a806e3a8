// ts_qkv.hip -- the QKV projection with the INT4 append as its epilogue, for gfx950 (head_dim
// 128 or 64, f16 weights).
//
// Replaces main_qkv (src/backend/bindless/sh_layer_v1_int4.wgsl:454-575) followed by
// quantize_kv (dispatched at src/backend/bindless/pipeline/layer.rs:1092-1099): for every
// token, q = Wq x, k = Wk x, v = Wv x (one f32 dot per output over `dim` inputs, F16 weights,
// the formula slot 1 branch at :494-498), q to the caller, and k, v quantized straight into the
// cache at the token's position with the arithmetic of the append (optional QK norm of K,
// rotation of K, per-row scale, codes) -- the f32 K and V never leave the chip unless the
// caller asks for them.
//
// The GEMM runs on v_mfma_f32_32x32x16_f16.  x is split hi + lo into f16 (two MFMAs into
// one f32 accumulator; x must stay below 65504 in magnitude), the weights are f16 already.
// The matrix cores flush f16 subnormals, so a lo part below 2^-14 is dropped: an element
// |x| < ~2^-3 then carries f16 precision (2^-12 relative) rather than ~2^-22.  Both effects
// are bounded by 2^-12 * sum|x w|, the same order as the f32 reference's own sequential
// rounding over dim = 4096 terms (4096 * 2^-24).
//
// Column tiles are 256 wide: 256 / hd q heads, or 128 / hd pairs (K head h, V head h) side by
// side, so the epilogue holds whole head rows.  The epilogue works on 32-row units: for n_tok == 1 (decode)
// 32 sequences, one new token each at position len[s]; for n_tok > 1 the 32 positions of one V
// block of one sequence (the block owns its V words, as in the append kernel).
//   * Enough tiles (prefill, large batches): one workgroup per 64-row tile over all of dim
//     (gemm_tile_core), the epilogue on the finished tile.
//   * Few tiles (decode): 32-row tiles with the reduction over dim split across workgroups
//     (gemm_split_core, one memory round trip per slice), f32 partials, and a second kernel
//     that sums them in split order (deterministic) and runs the epilogue.
#include <type_traits>

#include "ts_gemm.h"
#include "ts_kquant.h"
#include "ts_store.h"

namespace ts {
namespace {

constexpr int kMT = 32;     // rows per tile
constexpr int kNT = 256;    // columns per tile
constexpr int kTStr = 260;  // LDS row stride of the output tile (f32)
constexpr int kMaxSplit = 16;  // most splits of the reduction over dim
// V blocks per row tile of the prefill kernel: 64 rows.  (128 rows, two row waves per column
// of waves, measured 270 vs 190 us on the config-5 shape: the row waves each load the same
// weights, so the larger tile only adds registers.)
constexpr int kBigBlocks = 2;


struct QkvArgs {
    KvLayerView L;
    const int32_t *len;    // start position of every sequence
    const float *x;        // [S][n_tok][dim]
    const _Float16 *wq, *wk, *wv;  // [n_head*hd][dim], [H*hd][dim], [H*hd][dim]
    const uint8_t *bq, *bk, *bv;   // the same rows as GGUF K-quant blocks (the K-quant kernels)
    size_t brow;                   // bytes of one block row: dim / 256 super-blocks
    float *q_out;          // [S][n_tok][n_head][hd]
    float *k_out, *v_out;  // optional raw projections [S][n_tok][H][hd]
    const float *rope;
    int rope_pairs;
    float *part;           // split partials [n_split][RT][CT][32][256], or null
    int dim, n_tok, n_head;
    int wld;               // weight row length: dim (f16 rows) or 2 dim (hi then lo planes)
    int hd, hpt;           // head dim; kv heads per column tile (128 / hd)
    int n_qt;              // q column tiles (ceil(n_head * hd / 256))
    int RT, CT;            // row and column tiles
    int kps, n_split;      // k per split (multiple of kKC), splits
    int n_wg;              // workgroups of the GEMM launch (before rounding up to 8)
};

// Rows of row tile rt.  n_tok == 1: sequences 32 rt .. 32 rt + 31.  Otherwise V block `blk` of
// sequence s (positions 32 blk ..), live rows [lo, hi).
struct RowTile {
    int s, blk, start, lo, hi;
    bool live;
};

__device__ inline RowTile row_tile(const QkvArgs &a, int rt) {
    RowTile t;
    if (a.n_tok == 1) {
        t.s = kMT * rt;
        t.blk = t.start = t.lo = t.hi = 0;
        t.live = true;
        return t;
    }
    const int nb = a.n_tok / kBlk + 2;
    t.s = rt / nb;
    t.start = a.len[t.s];
    const int end = min(t.start + a.n_tok, a.L.P);
    t.blk = t.start / kBlk + rt % nb;
    const int p0 = t.blk * kBlk;
    t.live = p0 < end;
    t.lo = max(p0, t.start);
    t.hi = min(p0 + kBlk, end);
    return t;
}

// x row of tile row i, or -1 when the row is empty.
__device__ inline int x_row(const QkvArgs &a, const RowTile &t, int i) {
    if (a.n_tok == 1) return t.s + i < a.L.S ? t.s + i : -1;
    const int p = t.blk * kBlk + i;
    return (p >= t.lo && p < t.hi) ? t.s * a.n_tok + (p - t.start) : -1;
}

// Weight row of column n (0..255) of column tile ct (clamped to a valid row past the last
// head).  A kv tile holds (K head, V head) pairs: columns 2 hd j .. + hd - 1 are K of head
// hpt (ct - n_qt) + j, the next hd columns V of the same head.
__device__ inline const _Float16 *w_row(const QkvArgs &a, int ct, int n) {
    if (ct < a.n_qt) {
        const int r = min(ct * kNT + n, a.n_head * a.hd - 1);
        return a.wq + (size_t)r * a.wld;
    }
    const int j = n / (2 * a.hd), c = n % (2 * a.hd);
    const int h = min((ct - a.n_qt) * a.hpt + j, a.L.H - 1);
    return c < a.hd ? a.wk + ((size_t)h * a.hd + c) * a.wld : a.wv + ((size_t)h * a.hd + c - a.hd) * a.wld;
}

// Block row of column n of column tile ct (K-quant weights; the same rows as w_row).
__device__ inline const uint8_t *kq_row(const QkvArgs &a, int ct, int n) {
    if (ct < a.n_qt) {
        const int r = min(ct * kNT + n, a.n_head * a.hd - 1);
        return a.bq + (size_t)r * a.brow;
    }
    const int j = n / (2 * a.hd), c = n % (2 * a.hd);
    const int h = min((ct - a.n_qt) * a.hpt + j, a.L.H - 1);
    return c < a.hd ? a.bk + ((size_t)h * a.hd + c) * a.brow : a.bv + ((size_t)h * a.hd + c - a.hd) * a.brow;
}

// Workgroup id -> (row tile, column tile, split), ordered so that each XCD (workgroups are
// dealt round-robin over 8) gets a contiguous run of column tiles: a weight tile is then read
// into one or two L2s, not all eight.
__device__ inline void tile_of(const QkvArgs &a, int id, int &rt, int &ct, int &sp) {
    const int per = (a.n_wg + 7) / 8;
    const int lin = (id % 8) * per + id / 8;
    rt = lin % a.RT;
    ct = (lin / a.RT) % a.CT;
    sp = lin / (a.RT * a.CT);
}

// Quantize-and-store of one new token per row (n_tok == 1): row i = sequence t.s + i at its
// position len[s], for tile rows r0 .. r0 + nr - 1 (nr a multiple of 4) held in tile[i - r0],
// K of kv head h in columns col0 .. col0 + HD - 1 and V in the next HD.  HD / 8 lanes per row
// (lane l = dims 8l..8l+7), 256 / (HD / 8) rows per pass of the 4 waves.  Each row owns its
// sequence's K row, scales and the nibbles of its position in the V block.
template <int HD>
__device__ void store_rows_single(const QkvArgs &a, const RowTile &t, const float (*tile)[kTStr],
                                  int r0, int nr, int h, int col0, int wave, int lane) {
    constexpr int LPR = HD / 8, RPW = 64 / LPR;  // rows per wave per pass
    const KvLayerView &L = a.L;
    const int r = lane / LPR, l = lane % LPR;
    for (int base = 0; base < nr; base += 4 * RPW) {
        if (base + RPW * wave >= nr) break;  // wave-uniform
        const int i = r0 + base + RPW * wave + r;
        const bool in_tile = i < r0 + nr;
        const float *trow = tile[min(i, r0 + nr - 1) - r0] + col0;
        const int s = min(t.s + i, L.S - 1);
        const int p = a.len[s];
        // (a graph replayed past the cache's capacity writes nothing past it)
        const bool live = in_tile && t.s + i < L.S && p < L.P;
        float kx[8], vx[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kx[e] = trow[8 * l + e];
            vx[e] = trow[HD + 8 * l + e];
        }
        if (L.kn) row_qk_norm<LPR>(kx, L.kn, L.norm_eps, l, L.hdr);
        if (a.rope) {
            float2 cs[4];
            rope_cs4(L, s, p, a.rope, a.rope_pairs, l, cs);
#pragma unroll
            for (int m = 0; m < 4; m++)
                if (4 * l + m < a.rope_pairs) rope_rotate(kx[2 * m], kx[2 * m + 1], cs[m]);
        }
        float km = 0.0f, vm = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            km = fmaxf(km, fabsf(kx[e]));
            vm = fmaxf(vm, fabsf(vx[e]));
        }
        km = row_max<LPR>(km);
        vm = row_max<LPR>(vm);
        float ks, vs;
        uint32_t kc[8], vc[8];
        row_codes(kx, vx, km, vm, ks, vs, kc, vc);
        if (!live) continue;
        const size_t row = (size_t)s * L.H + h;
        uint32_t kw = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) kw |= kc[e] << (4 * e);
        reinterpret_cast<uint32_t *>(L.kp + row * L.P * (HD / 2))[k_word_idx<HD>(p, l)] = kw;
        if (l == 0) {
            L.ks[row * L.P + p] = ks;
            L.vs[row * L.P + p] = vs;
        }
        // V: dims 8l + e live in words v_word_idx(g*16 + dl, td) with d = 16 td + dl; position
        // q = p % 32 is nibble (q % 4) + 4 (q / 16) of group g = (q % 16) / 4.
        const int q = p & 31, g = (q & 15) >> 2, n = (q & 3) + 4 * (q >> 4);
        uint32_t *vb = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / kBlk) + p / kBlk) * (HD * 16));
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int d = 8 * l + e, td = d >> 4, dl = d & 15;
            uint32_t *dst = vb + v_word_idx(g * 16 + dl, td);
            *dst = (*dst & ~(0xFu << (4 * n))) | (vc[e] << (4 * n));
        }
    }
}

// K/V stores of the (K, V) head pairs of kv column tile ct, for the tile rows in tile[].
template <int HD>
__device__ void store_kv_tile(const QkvArgs &a, const RowTile &t, int ct, const float (*tile)[kTStr], int r0,
                              int nr, int tid) {
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int j = 0; j < 128 / HD; j++) {
        const int h = (ct - a.n_qt) * (128 / HD) + j;
        if (h >= a.L.H) break;  // uniform
        const int col0 = 2 * HD * j;
        if (a.n_tok == 1) {
            store_rows_single<HD>(a, t, tile, r0, nr, h, col0, wave, lane);
            continue;
        }
        if constexpr (HD == 128) {
            const int r = lane >> 4, l = lane & 15;
            float kx[2][8], vx[2][8];
            float2 cs[2][4];
#pragma unroll
            for (int rd = 0; rd < 2; rd++) {
                const int i = 16 * rd + 4 * wave + r;
                const int pc = min(max(t.blk * kBlk + i, t.lo), t.hi - 1);
                rope_cs4(a.L, t.s, pc, a.rope, a.rope_pairs, l, cs[rd]);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    kx[rd][e] = tile[i][col0 + 8 * l + e];
                    vx[rd][e] = tile[i][col0 + HD + 8 * l + e];
                }
            }
            store_block128(a.L, t.s, h, t.blk, t.lo, t.hi, kx, vx, cs, a.rope ? a.rope_pairs : 0, wave, lane);
        } else {
            const int r8 = lane >> 3, l = lane & 7;
            const int i = 4 * wave + (r8 & 3) + 16 * (r8 >> 2);
            const int pc = min(max(t.blk * kBlk + i, t.lo), t.hi - 1);
            float2 cs[4];
            rope_cs4(a.L, t.s, pc, a.rope, a.rope_pairs, l, cs);
            float kx[8], vx[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kx[e] = tile[i][col0 + 8 * l + e];
                vx[e] = tile[i][col0 + HD + 8 * l + e];
            }
            store_block64(a.L, t.s, h, t.blk, t.lo, t.hi, kx, vx, cs, a.rope ? a.rope_pairs : 0, wave, lane);
        }
    }
}

// The epilogue of tile rows r0 .. r0 + nr - 1 of a finished 32 x 256 tile, held in LDS as
// tile[i - r0].  Block rows (n_tok > 1) need the whole tile (r0 = 0, nr = 32).  256 threads.
__device__ void qkv_epilogue(const QkvArgs &a, const RowTile &t, int ct, const float (*tile)[kTStr],
                             int r0, int nr, int tid) {
    if (ct < a.n_qt) {
        // q: 256 / hd heads side by side, contiguous in q_out
        const int c4 = tid & 63, i0 = tid >> 6;
        const int col = ct * kNT + 4 * c4;
        if (col >= a.n_head * a.hd) return;
        for (int i = r0 + i0; i < r0 + nr; i += 4) {
            const int xr = x_row(a, t, i);
            if (xr < 0) continue;
            const float4 v = *reinterpret_cast<const float4 *>(&tile[i - r0][4 * c4]);
            *reinterpret_cast<float4 *>(a.q_out + (size_t)xr * a.n_head * a.hd + col) = v;
        }
        return;
    }
    if (a.k_out) {
        const int c4 = tid & 63, i0 = tid >> 6;
        const int c = 4 * c4, j = c / (2 * a.hd), cc = c % (2 * a.hd);
        const int h = (ct - a.n_qt) * a.hpt + j;
        float *dst = cc < a.hd ? a.k_out : a.v_out;
        if (h < a.L.H)
            for (int i = r0 + i0; i < r0 + nr; i += 4) {
                const int xr = x_row(a, t, i);
                if (xr < 0) continue;
                *reinterpret_cast<float4 *>(dst + ((size_t)xr * a.L.H + h) * a.hd + cc % a.hd) =
                    *reinterpret_cast<const float4 *>(&tile[i - r0][c]);
            }
    }
    if (a.hd == 128)
        store_kv_tile<128>(a, t, ct, tile, r0, nr, tid);
    else
        store_kv_tile<64>(a, t, ct, tile, r0, nr, tid);
}

// One workgroup per tile over all of dim (grids with enough tiles): MT = 64 WR rows -- for
// block rows 2 WR consecutive V blocks of one sequence, for decode rows MT sequences -- through
// gemm_tile_core (each wave 64 x 64, 2 x 2 MFMA blocks: every weight operand feeds two row
// blocks and every x operand two column blocks).  The epilogue runs 32 rows at a time on a
// 32 x 256 LDS tile that reuses the x buffers.
template <int WR>
__global__ __launch_bounds__(256 * WR) void qkv_tile_kernel(QkvArgs a) {
    constexpr int MT = 64 * WR, NBLK = MT / kBlk;
    union Smem {
        XTiles<MT> x;
        float tile[kMT][kTStr];
    };
    __shared__ __align__(16) Smem sm;

    int rt, ct, sp;
    tile_of(a, blockIdx.x, rt, ct, sp);
    if (sp >= a.n_split) return;
    const bool single = a.n_tok == 1;  // decode rows: MT sequences, one token each
    const int nb4 = (a.n_tok / kBlk + 2 + NBLK - 1) / NBLK;
    const int s = single ? MT * rt : rt / nb4;
    const int start = single ? 0 : a.len[s], end = single ? a.n_tok : min(start + a.n_tok, a.L.P);
    const int blk0 = start / kBlk + NBLK * (rt % nb4);
    if (!single && blk0 * kBlk >= end) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wr = wave >> 2, wc = wave & 3;

    // staging role: row si (0..MT-1), 16 floats at k offset 16 sc of each chunk
    const int si = tid >> 2, sc = tid & 3;
    const int ps = blk0 * kBlk + si;
    const int xr = single ? (s + si < a.L.S ? s + si : -1)
                          : (ps >= start && ps < end) ? s * a.n_tok + (ps - start) : -1;
    const float *xs = xr >= 0 ? a.x + (size_t)xr * a.dim + 16 * sc : nullptr;
    const _Float16 *const wp[2] = {w_row(a, ct, 64 * wc + j) + 32 * hf, w_row(a, ct, 64 * wc + 32 + j) + 32 * hf};
    floatx16 acc[2][2];
    gemm_tile_core<WR>(sm.x, xs, wp, a.wld / kKC, a.dim / kKC, tid, acc);

    // Epilogue, one 32-row block at a time: the waves holding it (wr = b / 2, row block b % 2)
    // write it to the LDS tile, then the first 4 waves run the block's epilogue.  The block
    // index is a template constant so that acc is indexed with constants and stays in
    // registers.
    auto block = [&](auto bc) {
        constexpr int b = decltype(bc)::value;
        if constexpr (b < NBLK) {
            const int p0 = (blk0 + b) * kBlk;
            if (single ? s + kBlk * b >= a.L.S : p0 >= end) return;  // uniform
            if (wr == (b >> 1)) {
#pragma unroll
                for (int cb = 0; cb < 2; cb++)
#pragma unroll
                    for (int e = 0; e < 16; e++)
                        sm.tile[8 * (e >> 2) + 4 * hf + (e & 3)][64 * wc + 32 * cb + j] = acc[b & 1][cb][e];
            }
            __syncthreads();
            if (tid < 256) {
                RowTile t;
                t.s = single ? s + kBlk * b : s;
                t.start = start;
                t.blk = blk0 + b;
                t.lo = max(p0, start);
                t.hi = min(p0 + kBlk, end);
                t.live = true;
                qkv_epilogue(a, t, ct, sm.tile, 0, kMT, tid);
            }
            __syncthreads();
        }
    };
    block(std::integral_constant<int, 0>{});
    block(std::integral_constant<int, 1>{});
    block(std::integral_constant<int, 2>{});
    block(std::integral_constant<int, 3>{});
}

// One split of the reduction for small grids (decode) through gemm_split_core; the f32
// partial tile goes to the scratch buffer.
__global__ __launch_bounds__(256) void qkv_split_kernel(QkvArgs a) {
    __shared__ __align__(16) SplitTiles sm;

    int rt, ct, sp;
    tile_of(a, blockIdx.x, rt, ct, sp);
    if (sp >= a.n_split) return;
    const RowTile t = row_tile(a, rt);
    if (!t.live) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int xr = x_row(a, t, tid >> 3);
    const int kb = sp * a.kps;
    const int nbat = (min(kb + a.kps, a.wld) - kb) / (4 * kKC);
    const float *xs = xr >= 0 ? a.x + (size_t)xr * a.dim + 8 * (tid & 7) : nullptr;
    const _Float16 *const wp[2] = {w_row(a, ct, 64 * wave + j) + kb + 32 * hf,
                                   w_row(a, ct, 64 * wave + 32 + j) + kb + 32 * hf};
    floatx16 acc[2];
    gemm_split_core(sm, xs, kb / kKC, a.dim / kKC, wp, nbat, tid, acc);
    // D layout: register 4q + r of column block cb is row 8q + 4hf + r, column 64 wave + 32 cb + j
    float *dst = a.part + (((size_t)sp * a.RT + rt) * a.CT + ct) * (kMT * kNT);
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++)
            dst[(8 * (e >> 2) + 4 * hf + (e & 3)) * kNT + 64 * wave + 32 * cb + j] = acc[cb][e];
}

// The same with the weights as GGUF K-quant blocks read in the loop (gemm_split_kq); a slice
// is a whole number of 256-element super-blocks.  Also used with one slice (no split) for
// shapes with many tiles, the reduce kernel then only running the epilogue.
template <int T>
__global__ __launch_bounds__(256) void qkv_split_kq_kernel(QkvArgs a) {
    __shared__ __align__(16) KqTiles sm[2];

    int rt, ct, sp;
    tile_of(a, blockIdx.x, rt, ct, sp);
    if (sp >= a.n_split) return;
    const RowTile t = row_tile(a, rt);
    if (!t.live) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int xr = x_row(a, t, tid >> 3);
    const int kb = sp * a.kps;
    const int nbat = (min(kb + a.kps, a.dim) - kb) / 256;
    const float *xs = xr >= 0 ? a.x + (size_t)xr * a.dim + kb + 8 * (tid & 7) : nullptr;
    const size_t boff = (size_t)(kb / 256) * KQ<T>::BYTES;
    const uint8_t *const wb[2] = {kq_row(a, ct, 64 * wave + j) + boff, kq_row(a, ct, 64 * wave + 32 + j) + boff};
    floatx16 acc[2];
    gemm_split_blocks<T>(sm, xs, wb, nbat, tid, acc);
    float *dst = a.part + (((size_t)sp * a.RT + rt) * a.CT + ct) * (kMT * kNT);
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++)
            dst[(8 * (e >> 2) + 4 * hf + (e & 3)) * kNT + 64 * wave + 32 * cb + j] = acc[cb][e];
}

// Sum of the split partials of rows r0 .. r0 + NR - 1 of one tile, in split order, then their
// epilogue.  Decode rows are independent, so a tile is spread over 32 / NR workgroups (NR = 4: 4 vs 8
// rows per workgroup measured 23.4 vs 24.0 us on config 3 and 16.9 vs 17.5 us on config 2);
// block rows share V words and take the whole tile (NR = 32).  Each thread issues the loads
// of every split of two float4 before adding them.
template <int NR>
__global__ __launch_bounds__(256) void qkv_reduce_kernel(QkvArgs a) {
    __shared__ __align__(16) float tile[NR][kTStr];
    constexpr int G = kMT / NR;
    const int tix = blockIdx.x / G, r0 = (blockIdx.x % G) * NR;
    const int rt = tix % a.RT, ct = tix / a.RT;
    const RowTile t = row_tile(a, rt);
    if (!t.live) return;
    const int tid = threadIdx.x;
    const size_t stride = (size_t)a.RT * a.CT * (kMT * kNT) / 4;
    const float4 *src = reinterpret_cast<const float4 *>(a.part) + ((size_t)rt * a.CT + ct) * (kMT * kNT / 4) +
                        r0 * (kNT / 4);
    sum_partials<NR, kMaxSplit>(src, stride, a.n_split, &tile[0][0], kTStr, tid);
    __syncthreads();
    qkv_epilogue(a, t, ct, tile, r0, NR, tid);
}

}  // namespace

QkvPlan qkv_plan(int n_seq, int n_kv, int n_head, int hd, int dim, int n_tok) {
    QkvPlan p;
    const int hpt = 128 / hd;
    p.CT = (n_head * hd + kNT - 1) / kNT + (n_kv + hpt - 1) / hpt;
    p.kps = dim;
    p.n_split = 1;
    p.part_bytes = 0;
    // Fewer 32-row tiles than CUs (decode, short chunks): dim split into slices of whole 256s
    // (at most kMaxSplit), as many as keep all workgroups in one round on the 256 CUs; going just
    // past 256 leaves a short second round that costs more than the longer slices.
    const int rt32 = n_tok == 1 ? (n_seq + kMT - 1) / kMT : n_seq * (n_tok / kBlk + 2);
    const int tiles = rt32 * p.CT;
    if (tiles < 256 && dim % 256 == 0 && dim >= 512) {
        p.big = false;
        p.RT = rt32;
        const int want = std::min(kMaxSplit, std::max(2, 256 / tiles));
        const int nbat = dim / 256;
        const int per = (nbat + want - 1) / want;  // 256s per split
        p.kps = per * 256;
        p.n_split = (nbat + per - 1) / per;
        p.part_bytes = (uint64_t)p.n_split * tiles * kMT * kNT * sizeof(float);
        return p;
    }
    // Otherwise one workgroup per tile of 32 kBigBlocks rows over all of dim.
    p.big = true;
    const int mt = kBlk * kBigBlocks;
    p.RT = n_tok == 1 ? (n_seq + mt - 1) / mt : n_seq * ((n_tok / kBlk + 2 + kBigBlocks - 1) / kBigBlocks);
    return p;
}

QkvPlan qkv_plan_kq(int n_seq, int n_kv, int n_head, int hd, int dim, int n_tok) {
    QkvPlan p;
    const int hpt = 128 / hd;
    p.CT = (n_head * hd + kNT - 1) / kNT + (n_kv + hpt - 1) / hpt;
    p.big = false;
    p.RT = n_tok == 1 ? (n_seq + kMT - 1) / kMT : n_seq * (n_tok / kBlk + 2);
    const int tiles = p.RT * p.CT;
    // few tiles: dim split over workgroups; many tiles: one slice over all of dim
    // splits for about one workgroup per CU (256): measured on config 3's decode shapes, 512
    // and 1024 were no faster (the split count is capped at kMaxSplit anyway)
    const int want = tiles < 256 ? std::min(kMaxSplit, std::max(1, (256 + tiles - 1) / tiles)) : 1;
    const int nbat = dim / 256;
    const int per = (nbat + want - 1) / want;
    p.kps = per * 256;
    p.n_split = (nbat + per - 1) / per;
    p.part_bytes = (uint64_t)p.n_split * tiles * kMT * kNT * sizeof(float);
    return p;
}

hipError_t launch_qkv_kq(const KvLayerView &L, const int32_t *d_len, const float *x, int dim, int n_tok,
                         int ggml_type, const void *wq, const void *wk, const void *wv, int n_head,
                         float *q_out, float *k_out, float *v_out, const float *rope, int rope_pairs,
                         const QkvPlan &plan, float *part, hipStream_t st) {
    if ((L.hd != 128 && L.hd != 64) || dim % 256 != 0 || !part || !kq_type(ggml_type)) return hipErrorInvalidValue;
    QkvArgs a;
    a.L = L;
    a.len = d_len;
    a.x = x;
    a.wq = a.wk = a.wv = nullptr;
    a.bq = static_cast<const uint8_t *>(wq);
    a.bk = static_cast<const uint8_t *>(wk);
    a.bv = static_cast<const uint8_t *>(wv);
    a.brow = (size_t)(dim / 256) * kq_bytes(ggml_type);
    a.q_out = q_out;
    a.k_out = k_out;
    a.v_out = v_out;
    a.rope = rope;
    a.rope_pairs = rope ? rope_pairs : 0;
    a.part = part;
    a.dim = dim;
    a.wld = dim;
    a.n_tok = n_tok;
    a.n_head = n_head;
    a.hd = L.hd;
    a.hpt = 128 / L.hd;
    a.n_qt = (n_head * L.hd + kNT - 1) / kNT;
    a.RT = plan.RT;
    a.CT = plan.CT;
    a.kps = plan.kps;
    a.n_split = plan.n_split;
    a.n_wg = plan.RT * plan.CT * plan.n_split;
    const int grid = (a.n_wg + 7) / 8 * 8;
    if (ggml_type == kGgmlQ4K)
        qkv_split_kq_kernel<kGgmlQ4K><<<grid, 256, 0, st>>>(a);
    else if (ggml_type == kGgmlQ5K)
        qkv_split_kq_kernel<kGgmlQ5K><<<grid, 256, 0, st>>>(a);
    else if (ggml_type == kGgmlQ8_0)
        qkv_split_kq_kernel<kGgmlQ8_0><<<grid, 256, 0, st>>>(a);
    else if (ggml_type == kGgmlQ5_0)
        qkv_split_kq_kernel<kGgmlQ5_0><<<grid, 256, 0, st>>>(a);
    else
        qkv_split_kq_kernel<kGgmlQ4_0><<<grid, 256, 0, st>>>(a);
    if (n_tok == 1)
        qkv_reduce_kernel<4><<<plan.RT * plan.CT * (kMT / 4), 256, 0, st>>>(a);
    else
        qkv_reduce_kernel<kMT><<<plan.RT * plan.CT, 256, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_qkv(const KvLayerView &L, const int32_t *d_len, const float *x, int dim, int n_tok,
                      const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int n_head,
                      float *q_out, float *k_out, float *v_out, const float *rope, int rope_pairs,
                      const QkvPlan &plan, float *part, int planes, hipStream_t st) {
    if ((L.hd != 128 && L.hd != 64) || dim % kKC != 0 || (planes != 1 && planes != 2)) return hipErrorInvalidValue;
    QkvArgs a;
    a.L = L;
    a.len = d_len;
    a.x = x;
    a.wq = reinterpret_cast<const _Float16 *>(wq);
    a.wk = reinterpret_cast<const _Float16 *>(wk);
    a.wv = reinterpret_cast<const _Float16 *>(wv);
    a.q_out = q_out;
    a.k_out = k_out;
    a.v_out = v_out;
    a.rope = rope;
    a.rope_pairs = rope ? rope_pairs : 0;
    a.bq = a.bk = a.bv = nullptr;
    a.brow = 0;
    a.part = plan.n_split > 1 ? part : nullptr;
    a.dim = dim;
    a.wld = planes * dim;
    a.n_tok = n_tok;
    a.n_head = n_head;
    a.hd = L.hd;
    a.hpt = 128 / L.hd;
    a.n_qt = (n_head * L.hd + kNT - 1) / kNT;
    a.RT = plan.RT;
    a.CT = plan.CT;
    a.kps = plan.kps;
    a.n_split = plan.n_split;
    a.n_wg = plan.RT * plan.CT * plan.n_split;
    const int grid = (a.n_wg + 7) / 8 * 8;
    if (plan.big) {
        qkv_tile_kernel<kBigBlocks / 2><<<grid, 128 * kBigBlocks, 0, st>>>(a);
    } else {
        qkv_split_kernel<<<grid, 256, 0, st>>>(a);
        if (n_tok == 1)
            qkv_reduce_kernel<4><<<plan.RT * plan.CT * (kMT / 4), 256, 0, st>>>(a);
        else
            qkv_reduce_kernel<kMT><<<plan.RT * plan.CT, 256, 0, st>>>(a);
    }
    return hipGetLastError();
}

}  // namespace ts
