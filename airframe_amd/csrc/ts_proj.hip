// ts_proj.hip -- the attention output projection with the residual add, for gfx950 (f16
// weights).
//
// Replaces main_attn_proj (src/backend/bindless/sh_layer_v1.wgsl:763-821, F16 branch
// :777-781): for every token, dot = Wo a over attn_dim = n_head * head_dim inputs (the
// attention output after the split-K combine), stashed raw when asked (the reference keeps it
// for Gemma-2's post-attention norm, :812-815), and added to the residual stream:
// act = act + dot (:818-820).  Same matrix-core loops as the QKV projection (ts_gemm.h):
//   * enough 64-row tiles: one workgroup per 64 x 256 tile over all of attn_dim, the result
//     added to act straight from the accumulators;
//   * few tiles (decode): 32 x 256 tiles with attn_dim split across workgroups (f32
//     partials), then a kernel that sums the partials in split order and adds them to act.
// Taking the combine's output rather than the decode partials is deliberate: every column
// tile reads all of a token's attention output, so folding the combine into this kernel would
// redo it (n_split-fold reads of the partials) once per column tile.
#include "ts_gemm.h"
#include "ts_internal.h"
#include "ts_kquant.h"

namespace ts {
namespace {

constexpr int kPT = 256;        // columns per tile
constexpr int kMaxPSplit = 16;  // most splits of the reduction

struct ProjArgs {
    const float *a;      // [M][K] attention output
    const _Float16 *w;   // [N][K]
    const uint8_t *bw;   // the same rows as GGUF K-quant blocks (the K-quant kernel)
    size_t brow;         // bytes of one block row
    float *act;          // [M][N], += dot
    float *stash;        // [M][N] raw dot, or null
    float *part;         // [n_split][RT][CT][32][256] partials, or null
    int M, N, K;
    int KW;              // weight row length: K (f16 rows) or 2 K (hi then lo planes)
    int RT, CT, kps, n_split, n_wg;
};

__device__ inline void proj_tile_of(const ProjArgs &p, int id, int &rt, int &ct, int &sp) {
    const int per = (p.n_wg + 7) / 8;
    const int lin = (id % 8) * per + id / 8;  // a contiguous run of column tiles per XCD
    rt = lin % p.RT;
    ct = (lin / p.RT) % p.CT;
    sp = lin / (p.RT * p.CT);
}

__device__ inline void proj_out(const ProjArgs &p, int row, int col, float v) {
    if (row >= p.M || col >= p.N) return;
    const size_t i = (size_t)row * p.N + col;
    if (p.stash) p.stash[i] = v;
    p.act[i] = p.act[i] + v;
}

// 64-row tiles over all of K; the epilogue from the accumulators.
__global__ __launch_bounds__(256) void proj_tile_kernel(ProjArgs p) {
    __shared__ __align__(16) XTiles<64> sm;
    int rt, ct, sp;
    proj_tile_of(p, blockIdx.x, rt, ct, sp);
    if (sp >= 1) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int row0 = 64 * rt, col0 = kPT * ct + 64 * wave;
    const int si = tid >> 2, sc = tid & 3;
    const float *xs = row0 + si < p.M ? p.a + (size_t)(row0 + si) * p.K + 16 * sc : nullptr;
    const _Float16 *const wp[2] = {p.w + (size_t)min(col0 + j, p.N - 1) * p.KW + 32 * hf,
                                   p.w + (size_t)min(col0 + 32 + j, p.N - 1) * p.KW + 32 * hf};
    floatx16 acc[2][2];
    gemm_tile_core<1>(sm, xs, wp, p.KW / kKC, p.K / kKC, tid, acc);
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int e = 0; e < 16; e++)
                proj_out(p, row0 + 32 * rb + 8 * (e >> 2) + 4 * hf + (e & 3), col0 + 32 * cb + j, acc[rb][cb][e]);
}

// One split of the reduction on a 32-row tile; the partial to the scratch buffer.
__global__ __launch_bounds__(256) void proj_split_kernel(ProjArgs p) {
    __shared__ __align__(16) SplitTiles sm;
    int rt, ct, sp;
    proj_tile_of(p, blockIdx.x, rt, ct, sp);
    if (sp >= p.n_split) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int row0 = 32 * rt, col0 = kPT * ct + 64 * wave;
    const int kb = sp * p.kps;
    const int nbat = (min(kb + p.kps, p.KW) - kb) / (4 * kKC);
    const int si = tid >> 3, sc = tid & 7;
    const float *xs = row0 + si < p.M ? p.a + (size_t)(row0 + si) * p.K + 8 * sc : nullptr;
    const _Float16 *const wp[2] = {p.w + (size_t)min(col0 + j, p.N - 1) * p.KW + kb + 32 * hf,
                                   p.w + (size_t)min(col0 + 32 + j, p.N - 1) * p.KW + kb + 32 * hf};
    floatx16 acc[2];
    gemm_split_core(sm, xs, kb / kKC, p.K / kKC, wp, nbat, tid, acc);
    float *dst = p.part + (((size_t)sp * p.RT + rt) * p.CT + ct) * (32 * kPT);
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++)
            dst[(8 * (e >> 2) + 4 * hf + (e & 3)) * kPT + 64 * wave + 32 * cb + j] = acc[cb][e];
}

// The same with the weights as GGUF K-quant blocks read in the loop (gemm_split_kq); slices of
// whole super-blocks, one slice when the tiles alone fill the chip.
template <int T>
__global__ __launch_bounds__(256) void proj_split_kq_kernel(ProjArgs p) {
    __shared__ __align__(16) KqTiles sm[2];
    int rt, ct, sp;
    proj_tile_of(p, blockIdx.x, rt, ct, sp);
    if (sp >= p.n_split) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int row0 = 32 * rt, col0 = kPT * ct + 64 * wave;
    const int kb = sp * p.kps;
    const int nbat = (min(kb + p.kps, p.K) - kb) / 256;
    const int si = tid >> 3, sc = tid & 7;
    const float *xs = row0 + si < p.M ? p.a + (size_t)(row0 + si) * p.K + kb + 8 * sc : nullptr;
    const size_t boff = (size_t)(kb / 256) * KQ<T>::BYTES;
    const uint8_t *const wb[2] = {p.bw + (size_t)min(col0 + j, p.N - 1) * p.brow + boff,
                                  p.bw + (size_t)min(col0 + 32 + j, p.N - 1) * p.brow + boff};
    floatx16 acc[2];
    gemm_split_blocks<T>(sm, xs, wb, nbat, tid, acc);
    float *dst = p.part + (((size_t)sp * p.RT + rt) * p.CT + ct) * (32 * kPT);
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 16; e++)
            dst[(8 * (e >> 2) + 4 * hf + (e & 3)) * kPT + 64 * wave + 32 * cb + j] = acc[cb][e];
}

// Sum of the partials of NR rows of one tile in split order, added to act.
constexpr int kPRows = 4;  // rows per workgroup of the sum (4 vs 8: config 3 14.1 vs 15.0 us, config 2 11.5 vs 12.2)
__global__ __launch_bounds__(256) void proj_reduce_kernel(ProjArgs p) {
    constexpr int NR = kPRows;
    __shared__ __align__(16) float tile[NR][kPT + 4];
    const int tix = blockIdx.x / (32 / NR), r0 = (blockIdx.x % (32 / NR)) * NR;
    const int rt = tix % p.RT, ct = tix / p.RT;
    if (32 * rt + r0 >= p.M) return;
    const int tid = threadIdx.x;
    const size_t stride = (size_t)p.RT * p.CT * (32 * kPT) / 4;
    const float4 *src = reinterpret_cast<const float4 *>(p.part) + ((size_t)rt * p.CT + ct) * (32 * kPT / 4) +
                        r0 * (kPT / 4);
    // the residual this thread updates (row r0 + i, column tid of the tile), read while the
    // partials stream in
    const int col = kPT * ct + tid;
    float res[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const int row = 32 * rt + r0 + i;
        res[i] = (row < p.M && col < p.N) ? p.act[(size_t)row * p.N + col] : 0.0f;
    }
    sum_partials<NR, kMaxPSplit>(src, stride, p.n_split, &tile[0][0], kPT + 4, tid);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const int row = 32 * rt + r0 + i;
        if (row >= p.M || col >= p.N) continue;
        const float v = tile[i][tid];
        const size_t idx = (size_t)row * p.N + col;
        if (p.stash) p.stash[idx] = v;
        p.act[idx] = res[i] + v;
    }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float4 *p, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256)
        p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

}  // namespace

// Zeroes n floats (n a multiple of 4, p 16-byte aligned) with a kernel, so that a caller may
// capture it in a graph.
hipError_t launch_fill_zero(float *p, size_t n, hipStream_t st) {
    if (n % 4 || ((uintptr_t)p & 15)) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    const size_t n4 = n / 4;
    fill_zero_kernel<<<(int)std::min<size_t>((n4 + 255) / 256, 4096), 256, 0, st>>>(reinterpret_cast<float4 *>(p), n4);
    return hipGetLastError();
}

ProjPlan proj_plan(int M, int K, int N) {
    ProjPlan p;
    p.CT = (N + kPT - 1) / kPT;
    p.kps = K;
    p.n_split = 1;
    p.part_bytes = 0;
    const int rt32 = (M + 31) / 32;
    const int tiles = rt32 * p.CT;
    if (tiles < 256 && K % 256 == 0 && K >= 512) {
        p.RT = rt32;
        const int want = std::min(kMaxPSplit, std::max(2, (512 + tiles - 1) / tiles));
        const int nbat = K / 256;
        const int per = (nbat + want - 1) / want;
        p.kps = per * 256;
        p.n_split = (nbat + per - 1) / per;
        p.part_bytes = (uint64_t)p.n_split * tiles * 32 * kPT * sizeof(float);
        return p;
    }
    p.RT = (M + 63) / 64;
    return p;
}

ProjPlan proj_plan_kq(int M, int K, int N) {
    ProjPlan p;
    p.CT = (N + kPT - 1) / kPT;
    p.RT = (M + 31) / 32;
    const int tiles = p.RT * p.CT;
    // splits for about one workgroup per CU (256): measured on config 3's decode shapes, 512
    // and 1024 were no faster (the split count is capped at kMaxPSplit anyway)
    const int want = tiles < 256 ? std::min(kMaxPSplit, std::max(1, (256 + tiles - 1) / tiles)) : 1;
    const int nbat = K / 256;
    const int per = (nbat + want - 1) / want;
    p.kps = per * 256;
    p.n_split = (nbat + per - 1) / per;
    p.part_bytes = (uint64_t)p.n_split * tiles * 32 * kPT * sizeof(float);
    return p;
}

hipError_t launch_proj_kq(const float *a, int M, int K, int ggml_type, const void *w, int N, float *act,
                          float *stash, const ProjPlan &plan, float *part, hipStream_t st) {
    if (K % 256 != 0 || M <= 0 || N <= 0 || !part || !kq_type(ggml_type)) return hipErrorInvalidValue;
    ProjArgs p;
    p.a = a;
    p.w = nullptr;
    p.bw = static_cast<const uint8_t *>(w);
    p.brow = (size_t)(K / 256) * kq_bytes(ggml_type);
    p.act = act;
    p.stash = stash;
    p.part = part;
    p.M = M;
    p.N = N;
    p.K = K;
    p.KW = K;
    p.RT = plan.RT;
    p.CT = plan.CT;
    p.kps = plan.kps;
    p.n_split = plan.n_split;
    p.n_wg = plan.RT * plan.CT * plan.n_split;
    const int grid = (p.n_wg + 7) / 8 * 8;
    if (ggml_type == kGgmlQ4K)
        proj_split_kq_kernel<kGgmlQ4K><<<grid, 256, 0, st>>>(p);
    else if (ggml_type == kGgmlQ5K)
        proj_split_kq_kernel<kGgmlQ5K><<<grid, 256, 0, st>>>(p);
    else if (ggml_type == kGgmlQ8_0)
        proj_split_kq_kernel<kGgmlQ8_0><<<grid, 256, 0, st>>>(p);
    else if (ggml_type == kGgmlQ5_0)
        proj_split_kq_kernel<kGgmlQ5_0><<<grid, 256, 0, st>>>(p);
    else
        proj_split_kq_kernel<kGgmlQ4_0><<<grid, 256, 0, st>>>(p);
    proj_reduce_kernel<<<plan.RT * plan.CT * (32 / kPRows), 256, 0, st>>>(p);
    return hipGetLastError();
}

hipError_t launch_proj(const float *a, int M, int K, const uint16_t *w, int N, float *act, float *stash,
                       const ProjPlan &plan, float *part, int planes, hipStream_t st) {
    if (K % kKC != 0 || M <= 0 || N <= 0 || (planes != 1 && planes != 2)) return hipErrorInvalidValue;
    ProjArgs p;
    p.a = a;
    p.w = reinterpret_cast<const _Float16 *>(w);
    p.bw = nullptr;
    p.brow = 0;
    p.act = act;
    p.stash = stash;
    p.part = part;
    p.M = M;
    p.N = N;
    p.K = K;
    p.KW = planes * K;
    p.RT = plan.RT;
    p.CT = plan.CT;
    p.kps = plan.kps;
    p.n_split = plan.n_split;
    p.n_wg = plan.RT * plan.CT * plan.n_split;
    const int grid = (p.n_wg + 7) / 8 * 8;
    if (plan.n_split == 1) {
        proj_tile_kernel<<<grid, 256, 0, st>>>(p);
    } else {
        proj_split_kernel<<<grid, 256, 0, st>>>(p);
        proj_reduce_kernel<<<plan.RT * plan.CT * (32 / kPRows), 256, 0, st>>>(p);
    }
    return hipGetLastError();
}

}  // namespace ts
