// ts_qkv.hip -- the QKV projection with the INT4 append as its epilogue, for gfx950 (head_dim
// 128, f16 weights).
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
// Tiles: 32 rows (tokens) x 256 columns, one workgroup of 4 waves, each wave 32 x 64 (two
// MFMA column blocks).  A column tile is two q heads, or the K head h next to the V head h,
// so the epilogue holds whole head rows.  Rows are
//   * n_tok == 1 (decode): 32 sequences, one new token each, at position len[s];
//   * n_tok > 1: the 32 positions of one V block of one sequence (the block owns its V words,
//     as in the append kernel).
// Large grids (prefill) run one workgroup per tile over all of dim: the k-chunk loop
// double-buffers x (converted to hi/lo once per workgroup, in LDS) and streams the weights
// straight into the B operands one chunk ahead, and the epilogue runs on the finished tile.
// Small grids (decode) split the reduction over `dim` across workgroups: each loads its whole
// slice in one round trip and writes an f32 partial tile, and a second kernel sums the
// partials in split order (deterministic) and runs the epilogue.
#include "ts_mfma.h"
#include "ts_store128.h"

namespace ts {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kMT = 32;     // rows per tile
constexpr int kNT = 256;    // columns per tile
constexpr int kKC = 64;     // k per chunk
constexpr int kAStr = 72;   // LDS row stride of the x tiles (f16): 144 B spreads the rows' banks
constexpr int kTStr = 260;  // LDS row stride of the output tile (f32)
constexpr int kMaxSplit = 16;  // most splits of the reduction over dim
#ifndef TS_QKV_BIG_BLOCKS
#define TS_QKV_BIG_BLOCKS 2
#endif
constexpr int kBigBlocks = TS_QKV_BIG_BLOCKS;  // V blocks per row tile of the prefill kernel


struct QkvArgs {
    KvLayerView L;
    const int32_t *len;    // start position of every sequence
    const float *x;        // [S][n_tok][dim]
    const _Float16 *wq, *wk, *wv;  // [n_head*128][dim], [H*128][dim], [H*128][dim]
    float *q_out;          // [S][n_tok][n_head][128]
    float *k_out, *v_out;  // optional raw projections [S][n_tok][H][128]
    const float *rope;
    int rope_pairs;
    float *part;           // split partials [n_split][RT][CT][32][256], or null
    int dim, n_tok, n_head;
    int n_qt;              // q column tiles (ceil(n_head / 2))
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
    const int end = t.start + a.n_tok;
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

// Weight row of column n (0..255) of column tile ct (clamped to a valid row past n_head).
__device__ inline const _Float16 *w_row(const QkvArgs &a, int ct, int n) {
    if (ct < a.n_qt) {
        const int r = min(ct * kNT + n, a.n_head * 128 - 1);
        return a.wq + (size_t)r * a.dim;
    }
    const int h = ct - a.n_qt;
    return n < 128 ? a.wk + ((size_t)h * 128 + n) * a.dim : a.wv + ((size_t)h * 128 + n - 128) * a.dim;
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

// Quantize-and-store of one new token per row (n_tok == 1): row i = sequence t.s + i at its
// position len[s], for tile rows r0 .. r0 + nr - 1 (nr a multiple of 4) held in tile[i - r0].
// 16 lanes per row (lane l = dims 8l..8l+7), rows r0 + 16 m + 4 wave + lane/16.
// Each row owns its sequence's K row, scales and the nibbles of its position in the V block.
__device__ void store_rows_single(const QkvArgs &a, const RowTile &t, const float (*tile)[kTStr],
                                  int r0, int nr, int h, int wave, int lane) {
    constexpr int HD = 128, NTD = HD / 16;
    const KvLayerView &L = a.L;
    const int r = lane >> 4, l = lane & 15;
    for (int base = 0; base < nr; base += 16) {
        if (base + 4 * wave >= nr) break;  // wave-uniform
        const int i = r0 + base + 4 * wave + r;
        const float *trow = tile[i - r0];
        const int s = min(t.s + i, L.S - 1);
        const bool live = t.s + i < L.S;
        const int p = a.len[s];
        float kx[8], vx[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kx[e] = trow[8 * l + e];
            vx[e] = trow[HD + 8 * l + e];
        }
        if (L.kn) {
            float sq[8];
#pragma unroll
            for (int e = 0; e < 8; e++) sq[e] = sq_rn(kx[e]);
            const float ns = qk_norm_scale_from_sum(ordered_sum_row16(sq, l), HD, L.norm_eps);
#pragma unroll
            for (int e = 0; e < 8; e++) kx[e] = qk_norm_apply(kx[e], ns, L.kn[8 * l + e]);
        }
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
        km = fmaxf(km, dpp_f<0xB1>(km));
        vm = fmaxf(vm, dpp_f<0xB1>(vm));
        km = fmaxf(km, dpp_f<0x4E>(km));
        vm = fmaxf(vm, dpp_f<0x4E>(vm));
        km = fmaxf(km, dpp_f<0x141>(km));
        vm = fmaxf(vm, dpp_f<0x141>(vm));
        km = fmaxf(km, dpp_f<0x140>(km));
        vm = fmaxf(vm, dpp_f<0x140>(vm));
        const float ks = quant_scale(km), vs = quant_scale(vm);
        const float kr = __builtin_amdgcn_rcpf(ks), vr = __builtin_amdgcn_rcpf(vs);
        bool kneed = !(ks >= 1.17549435e-38f && ks <= 4.25352959e37f);
        bool vneed = !(vs >= 1.17549435e-38f && vs <= 4.25352959e37f);
        uint32_t kc[8], vc[8];
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
        if (!live) continue;
        const size_t row = (size_t)s * L.H + h;
        uint32_t kw = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) kw |= kc[e] << (4 * e);
        reinterpret_cast<uint32_t *>(L.kp + (row * L.P + p) * (HD / 2))[l] = kw;
        if (l == 0) {
            L.ks[row * L.P + p] = ks;
            L.vs[row * L.P + p] = vs;
        }
        // V: dims 8l + e live in words (g*16 + dl)*NTD + td with d = 16 td + dl; position
        // q = p % 32 is nibble (q % 4) + 4 (q / 16) of group g = (q % 16) / 4.
        const int q = p & 31, g = (q & 15) >> 2, n = (q & 3) + 4 * (q >> 4);
        uint32_t *vb = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / kBlk) + p / kBlk) * (HD * 16));
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int d = 8 * l + e, td = d >> 4, dl = d & 15;
            uint32_t *dst = vb + (g * 16 + dl) * NTD + td;
            *dst = (*dst & ~(0xFu << (4 * n))) | (vc[e] << (4 * n));
        }
    }
}

// The epilogue of tile rows r0 .. r0 + nr - 1 of a finished 32 x 256 tile, held in LDS as
// tile[i - r0].  Block rows (n_tok > 1) need the whole tile (r0 = 0, nr = 32).  256 threads.
__device__ void qkv_epilogue(const QkvArgs &a, const RowTile &t, int ct, const float (*tile)[kTStr],
                             int r0, int nr, int tid) {
    const int wave = tid >> 6, lane = tid & 63;
    if (ct < a.n_qt) {
        // q: two heads side by side, contiguous in q_out
        const int c4 = tid & 63, i0 = tid >> 6;
        const int col = ct * kNT + 4 * c4;
        if (col >= a.n_head * 128) return;
        for (int i = r0 + i0; i < r0 + nr; i += 4) {
            const int xr = x_row(a, t, i);
            if (xr < 0) continue;
            const float4 v = *reinterpret_cast<const float4 *>(&tile[i - r0][4 * c4]);
            *reinterpret_cast<float4 *>(a.q_out + (size_t)xr * a.n_head * 128 + col) = v;
        }
        return;
    }
    const int h = ct - a.n_qt;
    if (a.k_out) {
        const int c4 = tid & 63, i0 = tid >> 6;
        float *dst = c4 < 32 ? a.k_out : a.v_out;
        const int c = 4 * (c4 & 31);
        for (int i = r0 + i0; i < r0 + nr; i += 4) {
            const int xr = x_row(a, t, i);
            if (xr < 0) continue;
            *reinterpret_cast<float4 *>(dst + ((size_t)xr * a.L.H + h) * 128 + c) =
                *reinterpret_cast<const float4 *>(&tile[i - r0][4 * c4]);
        }
    }
    if (a.n_tok == 1) {
        store_rows_single(a, t, tile, r0, nr, h, wave, lane);
        return;
    }
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
            kx[rd][e] = tile[i][8 * l + e];
            vx[rd][e] = tile[i][128 + 8 * l + e];
        }
    }
    store_block128(a.L, t.s, h, t.blk, t.lo, t.hi, kx, vx, cs, a.rope ? a.rope_pairs : 0, wave, lane);
}

__global__ __launch_bounds__(256) void qkv_gemm_kernel(QkvArgs a) {
    __shared__ __align__(16) _Float16 ahi[2][kMT][kAStr];
    __shared__ __align__(16) _Float16 alo[2][kMT][kAStr];
    __shared__ __align__(16) float tile[kMT][kTStr];

    int rt, ct, sp;
    tile_of(a, blockIdx.x, rt, ct, sp);
    if (sp >= a.n_split) return;
    const RowTile t = row_tile(a, rt);
    if (!t.live) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;

    // staging role: row si, 8 floats at k offset 8 sc of each chunk
    const int si = tid >> 3, sc = tid & 7;
    const int xr = x_row(a, t, si);
    const int kb = sp * a.kps;
    const int nch = (min(kb + a.kps, a.dim) - kb) / kKC;
    const float *xs = a.x + (size_t)max(xr, 0) * a.dim + kb + 8 * sc;

    // B role: columns 64 wave + 32 cb + j, 32 consecutive k (16 B per k-step) from 32 hf
    const _Float16 *wp[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++) wp[cb] = w_row(a, ct, 64 * wave + 32 * cb + j) + kb + 32 * hf;

    floatx16 acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[cb][e] = 0.0f;

    float4 xu = make_float4(0.f, 0.f, 0.f, 0.f), xv = xu;
    if (xr >= 0) {
        xu = *reinterpret_cast<const float4 *>(xs);
        xv = *reinterpret_cast<const float4 *>(xs + 4);
    }
    half8 wb[2][4];
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int q = 0; q < 4; q++) wb[cb][q] = *reinterpret_cast<const half8 *>(wp[cb] + 8 * q);
    {
        half8 h, l;
        split8(xu, xv, h, l);
        *reinterpret_cast<half8 *>(&ahi[0][si][8 * sc]) = h;
        *reinterpret_cast<half8 *>(&alo[0][si][8 * sc]) = l;
    }
    __syncthreads();

    for (int c = 0; c < nch; c++) {
        const int buf = c & 1;
        const bool more = c + 1 < nch;
        half8 wn[2][4];
        if (more) {
            if (xr >= 0) {
                xu = *reinterpret_cast<const float4 *>(xs + (c + 1) * kKC);
                xv = *reinterpret_cast<const float4 *>(xs + (c + 1) * kKC + 4);
            }
#pragma unroll
            for (int cb = 0; cb < 2; cb++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    wn[cb][q] = *reinterpret_cast<const half8 *>(wp[cb] + (c + 1) * kKC + 8 * q);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const half8 ah = *reinterpret_cast<const half8 *>(&ahi[buf][j][32 * hf + 8 * q]);
            const half8 al = *reinterpret_cast<const half8 *>(&alo[buf][j][32 * hf + 8 * q]);
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, wb[cb][q], acc[cb], 0, 0, 0);
                acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, wb[cb][q], acc[cb], 0, 0, 0);
            }
        }
        if (more) {
            half8 h, l;
            split8(xu, xv, h, l);
            *reinterpret_cast<half8 *>(&ahi[buf ^ 1][si][8 * sc]) = h;
            *reinterpret_cast<half8 *>(&alo[buf ^ 1][si][8 * sc]) = l;
#pragma unroll
            for (int cb = 0; cb < 2; cb++)
#pragma unroll
                for (int q = 0; q < 4; q++) wb[cb][q] = wn[cb][q];
        }
        __syncthreads();
    }

    // D layout: register 4q + r of column block cb is row 8q + 4hf + r, column 64 wave + 32 cb + j
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++) tile[8 * (e >> 2) + 4 * hf + (e & 3)][64 * wave + 32 * cb + j] = acc[cb][e];
    __syncthreads();
    qkv_epilogue(a, t, ct, tile, 0, kMT, tid);
}

// Block rows in tiles of 128 (prefill chunks): four consecutive V blocks blk0 .. blk0 + 3 of
// one sequence.  8 waves: wave (wr, wc) computes rows 64 wr .. + 63, columns 64 wc .. + 63
// (2 x 2 MFMA blocks), so each weight operand feeds two row blocks and each x operand two
// column blocks: half the operand traffic per MFMA of the 32-row tiles.  x is staged per
// chunk as hi/lo in LDS (double-buffered), the weights stream into registers one chunk ahead.
// The epilogue runs block by block on a 32 x 256 LDS tile that reuses the x buffers.
template <int WR>
__global__ __launch_bounds__(256 * WR) void qkv_gemm128_kernel(QkvArgs a) {
    constexpr int MT = 64 * WR, NBLK = MT / kBlk;
    union Smem {
        struct {
            _Float16 hi[2][MT][kAStr];
            _Float16 lo[2][MT][kAStr];
        } x;
        float tile[kMT][kTStr];
    };
    __shared__ __align__(16) Smem sm;

    int rt, ct, sp;
    tile_of(a, blockIdx.x, rt, ct, sp);
    if (sp >= a.n_split) return;
    const int nb4 = (a.n_tok / kBlk + 2 + NBLK - 1) / NBLK;
    const int s = rt / nb4;
    const int start = a.len[s], end = start + a.n_tok;
    const int blk0 = start / kBlk + NBLK * (rt % nb4);
    if (blk0 * kBlk >= end) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wr = wave >> 2, wc = wave & 3;

    // staging role: row si (0..MT-1), 16 floats at k offset 16 sc of each chunk
    const int si = tid >> 2, sc = tid & 3;
    const int ps = blk0 * kBlk + si;
    const int xr = (ps >= start && ps < end) ? s * a.n_tok + (ps - start) : -1;
    const float *xs = a.x + (size_t)max(xr, 0) * a.dim + 16 * sc;
    const int nch = a.dim / kKC;

    const _Float16 *wp[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++) wp[cb] = w_row(a, ct, 64 * wc + 32 * cb + j) + 32 * hf;

    floatx16 acc[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[rb][cb][e] = 0.0f;

    float4 xq[4];
    auto load_x = [&](int c) {
#pragma unroll
        for (int u = 0; u < 4; u++)
            xq[u] = xr >= 0 ? *reinterpret_cast<const float4 *>(xs + c * kKC + 4 * u)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto store_x = [&](int buf) {
        half8 h, l;
        split8(xq[0], xq[1], h, l);
        *reinterpret_cast<half8 *>(&sm.x.hi[buf][si][16 * sc]) = h;
        *reinterpret_cast<half8 *>(&sm.x.lo[buf][si][16 * sc]) = l;
        split8(xq[2], xq[3], h, l);
        *reinterpret_cast<half8 *>(&sm.x.hi[buf][si][16 * sc + 8]) = h;
        *reinterpret_cast<half8 *>(&sm.x.lo[buf][si][16 * sc + 8]) = l;
    };
    // weights two chunks ahead (wb: chunk c, wn: c + 1), x one chunk ahead (LDS double buffer)
    half8 wb[2][4], wn[2][4];
    auto load_w = [&](half8 (&w)[2][4], int c) {
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                w[cb][q] = c < nch ? *reinterpret_cast<const half8 *>(wp[cb] + c * kKC + 8 * q)
                                   : (half8)(_Float16)0.0f;
    };
    load_x(0);
    load_w(wb, 0);
    load_w(wn, 1);
    store_x(0);
    __syncthreads();

    for (int c = 0; c < nch; c++) {
        const int buf = c & 1;
        const bool more = c + 1 < nch;
        half8 wf[2][4];
        load_w(wf, c + 2);
        if (more) load_x(c + 1);
#pragma unroll
        for (int q = 0; q < 4; q++) {
#pragma unroll
            for (int rb = 0; rb < 2; rb++) {
                const int row = 64 * wr + 32 * rb + j;
                const half8 ah = *reinterpret_cast<const half8 *>(&sm.x.hi[buf][row][32 * hf + 8 * q]);
                const half8 al = *reinterpret_cast<const half8 *>(&sm.x.lo[buf][row][32 * hf + 8 * q]);
#pragma unroll
                for (int cb = 0; cb < 2; cb++) {
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, wb[cb][q], acc[rb][cb], 0, 0, 0);
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, wb[cb][q], acc[rb][cb], 0, 0, 0);
                }
            }
        }
        if (more) store_x(buf ^ 1);
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                wb[cb][q] = wn[cb][q];
                wn[cb][q] = wf[cb][q];
            }
        __syncthreads();
    }

    // Epilogue, one 32-row block at a time: the waves holding it (wr = b / 2, row block b % 2)
    // write it to the LDS tile, then the first 4 waves run the block's epilogue.
    // (unrolled, so that acc is indexed with constants and stays in registers)
#pragma unroll
    for (int b = 0; b < NBLK; b++) {
        const int p0 = (blk0 + b) * kBlk;
        if (p0 >= end) continue;  // uniform
        if (wr == (b >> 1)) {
            const int rb = b & 1;
#pragma unroll
            for (int cb = 0; cb < 2; cb++)
#pragma unroll
                for (int e = 0; e < 16; e++)
                    sm.tile[8 * (e >> 2) + 4 * hf + (e & 3)][64 * wc + 32 * cb + j] = acc[rb][cb][e];
        }
        __syncthreads();
        if (tid < 256) {
            RowTile t;
            t.s = s;
            t.start = start;
            t.blk = blk0 + b;
            t.lo = max(p0, start);
            t.hi = min(p0 + kBlk, end);
            t.live = true;
            qkv_epilogue(a, t, ct, sm.tile, 0, kMT, tid);
        }
        __syncthreads();
    }
}

// One split of the reduction for small grids (decode): the slice of dim, in batches of 4
// chunks (256), is loaded in one go -- x for all 4 chunks into LDS as hi/lo (shared by the 4
// waves), the weights straight into B operands (128 VGPRs) -- so a batch costs one memory
// round trip, then 64 MFMAs per wave; the f32 partial tile goes to the scratch buffer.
__global__ __launch_bounds__(256) void qkv_split_kernel(QkvArgs a) {
    constexpr int NB = 4;  // chunks per batch
    __shared__ __align__(16) _Float16 ahi[NB][kMT][kAStr];
    __shared__ __align__(16) _Float16 alo[NB][kMT][kAStr];

    int rt, ct, sp;
    tile_of(a, blockIdx.x, rt, ct, sp);
    if (sp >= a.n_split) return;
    const RowTile t = row_tile(a, rt);
    if (!t.live) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int si = tid >> 3, sc = tid & 7;
    const int xr = x_row(a, t, si);
    const int kb = sp * a.kps;
    const int nbat = (min(kb + a.kps, a.dim) - kb) / (NB * kKC);
    const float *xs = a.x + (size_t)max(xr, 0) * a.dim + kb + 8 * sc;
    const _Float16 *wp[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++) wp[cb] = w_row(a, ct, 64 * wave + 32 * cb + j) + kb + 32 * hf;

    floatx16 acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[cb][e] = 0.0f;

    for (int b = 0; b < nbat; b++) {
        const int ko = b * NB * kKC;
        float4 xu[NB], xv[NB];
        half8 wb[NB][2][4];
#pragma unroll
        for (int c = 0; c < NB; c++) {
            xu[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            xv[c] = xu[c];
            if (xr >= 0) {
                xu[c] = *reinterpret_cast<const float4 *>(xs + ko + c * kKC);
                xv[c] = *reinterpret_cast<const float4 *>(xs + ko + c * kKC + 4);
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
            *reinterpret_cast<half8 *>(&ahi[c][si][8 * sc]) = h;
            *reinterpret_cast<half8 *>(&alo[c][si][8 * sc]) = l;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NB; c++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const half8 ah = *reinterpret_cast<const half8 *>(&ahi[c][j][32 * hf + 8 * q]);
                const half8 al = *reinterpret_cast<const half8 *>(&alo[c][j][32 * hf + 8 * q]);
#pragma unroll
                for (int cb = 0; cb < 2; cb++) {
                    acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, wb[c][cb][q], acc[cb], 0, 0, 0);
                    acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, wb[c][cb][q], acc[cb], 0, 0, 0);
                }
            }
    }
    // D layout: register 4q + r of column block cb is row 8q + 4hf + r, column 64 wave + 32 cb + j
    float *dst = a.part + (((size_t)sp * a.RT + rt) * a.CT + ct) * (kMT * kNT);
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++)
            dst[(8 * (e >> 2) + 4 * hf + (e & 3)) * kNT + 64 * wave + 32 * cb + j] = acc[cb][e];
}

// Sum of the split partials of rows r0 .. r0 + NR - 1 of one tile, in split order, then their
// epilogue.  Decode rows are independent, so a tile is spread over 32 / NR workgroups (NR = 8);
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
    constexpr int PER = NR / 4;            // float4 of the rows per thread
    constexpr int U = PER < 2 ? PER : 2;   // float4 per pass
#pragma unroll
    for (int pass = 0; pass < PER / U; pass++) {
        float4 v[U][kMaxSplit];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int sp = 0; sp < kMaxSplit; sp++)
                if (sp < a.n_split) v[u][sp] = src[sp * stride + (U * pass + u) * 256 + tid];
#pragma unroll
        for (int u = 0; u < U; u++) {
            float4 acc = v[u][0];
#pragma unroll
            for (int sp = 1; sp < kMaxSplit; sp++)
                if (sp < a.n_split) {
                    acc.x = acc.x + v[u][sp].x;
                    acc.y = acc.y + v[u][sp].y;
                    acc.z = acc.z + v[u][sp].z;
                    acc.w = acc.w + v[u][sp].w;
                }
            const int e4 = (U * pass + u) * 256 + tid;
            *reinterpret_cast<float4 *>(&tile[e4 / (kNT / 4)][4 * (e4 % (kNT / 4))]) = acc;
        }
    }
    __syncthreads();
    qkv_epilogue(a, t, ct, tile, r0, NR, tid);
}

}  // namespace

QkvPlan qkv_plan(int n_seq, int n_kv, int n_head, int dim, int n_tok) {
    QkvPlan p;
    p.RT = n_tok == 1 ? (n_seq + kMT - 1) / kMT : n_seq * (n_tok / kBlk + 2);
    p.CT = (n_head + 1) / 2 + n_kv;
    const int tiles = p.RT * p.CT;
    p.kps = dim;
    p.n_split = 1;
    p.big = false;
    // Prefill chunks with enough work: 128-row tiles (four V blocks) over all of dim.
    const int rt_big = n_seq * ((n_tok / kBlk + 2 + kBigBlocks - 1) / kBigBlocks);
    if (n_tok > 1 && rt_big * p.CT >= 256) {
        p.big = true;
        p.RT = rt_big;
        p.part_bytes = 0;
        return p;
    }
    // Fewer tiles than CUs (decode): dim split into slices of whole 256s (at most kMaxSplit)
    // so that about 512 workgroups stream the weights.
    if (tiles < 256 && dim % 256 == 0 && dim >= 512) {
        const int want = std::min(kMaxSplit, std::max(2, (512 + tiles - 1) / tiles));
        const int nbat = dim / 256;
        const int per = (nbat + want - 1) / want;  // 256s per split
        p.kps = per * 256;
        p.n_split = (nbat + per - 1) / per;
    }
    p.part_bytes = p.n_split > 1 ? (uint64_t)p.n_split * tiles * kMT * kNT * sizeof(float) : 0;
    return p;
}

hipError_t launch_qkv(const KvLayerView &L, const int32_t *d_len, const float *x, int dim, int n_tok,
                      const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int n_head,
                      float *q_out, float *k_out, float *v_out, const float *rope, int rope_pairs,
                      const QkvPlan &plan, float *part, hipStream_t st) {
    if (L.hd != 128 || dim % kKC != 0) return hipErrorInvalidValue;
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
    a.part = plan.n_split > 1 ? part : nullptr;
    a.dim = dim;
    a.n_tok = n_tok;
    a.n_head = n_head;
    a.n_qt = (n_head + 1) / 2;
    a.RT = plan.RT;
    a.CT = plan.CT;
    a.kps = plan.kps;
    a.n_split = plan.n_split;
    a.n_wg = plan.RT * plan.CT * plan.n_split;
    const int grid = (a.n_wg + 7) / 8 * 8;
    if (plan.big) {
        qkv_gemm128_kernel<kBigBlocks / 2><<<grid, 128 * kBigBlocks, 0, st>>>(a);
    } else if (plan.n_split == 1) {
        qkv_gemm_kernel<<<grid, 256, 0, st>>>(a);
    } else {
        qkv_split_kernel<<<grid, 256, 0, st>>>(a);
        if (n_tok == 1)
            qkv_reduce_kernel<8><<<plan.RT * plan.CT * (kMT / 8), 256, 0, st>>>(a);
        else
            qkv_reduce_kernel<kMT><<<plan.RT * plan.CT, 256, 0, st>>>(a);
    }
    return hipGetLastError();
}

}  // namespace ts
