// ts_decode.hip -- split-K GQA decode attention over the INT4 cache for gfx950.
//
// Semantics: the CPU reference attention (src/ops/reference/attention.rs:236-313): per query
// head, scores = q.k over all cached positions, times 1/sqrt(hd), softmax, times V, with q
// rotated at its absolute position and k/v the dequantized INT4 cache
// ((code - 8) * scale, test_int4_parity.rs:78-87).  The reference GPU kernel
// (sh_layer_v1_int4.wgsl:1042-1143) runs one thread per output element, each re-reading the
// whole K stream; here the work is organised around HBM instead:
//
// * grid = (split, kv head, sequence); a split is `chunk` positions (multiple of 64) of one
//   (sequence, kv head) stream, so every workgroup reads contiguous runs of K rows, V blocks
//   and scales exactly once for all G = n_head/n_kv query heads that share them.
// * each of the 4 waves takes 64-position windows round robin: K rows are 16-byte loads per
//   lane, V blocks 32-byte loads per lane, scales 16-byte loads.
// * QK^T and PV run on the matrix cores (v_mfma_f32_16x16x32_f16).  INT4 codes convert to
//   exact f16 integers with two bit tricks (0x6400|nibble is 1024+nibble; the second nibble of
//   a byte is taken as 1024+16*nibble and fixed with one packed f16 FMA), so K and V enter the
//   MFMA exactly.  The per-position scales are applied in f32 outside the MFMA: s_k on the
//   scores, s_v folded into the probabilities.
// * q and p are split hi + lo in f16 (x = hi + lo to ~22 bits), so the f32-accumulated MFMA
//   results carry f32-level accuracy: QK issues two MFMAs (hi, lo) into one accumulator; for
//   PV the lo part rides in the spare accumulator columns G..2G-1.
// * online softmax in the exp2 domain with one cross-lane max per 64 positions; the 4 waves
//   merge through LDS; splits merge in a second kernel (log-sum-exp combine) unless a
//   sequence fits one split.
#include "ts_mfma.h"

namespace ts {
namespace {

struct DecodeArgs {
    KvLayerView L;
    const int32_t *len;
    const float *q;
    const float *rope;
    int rope_pairs;
    int n_head;
    int G;
    int chunk;
    int n_split;
    float inv_sqrt_hd;
    float softcap;
    float *out;
    float *ws;  // partial o [S][n_head][n_split][hd], then m [..][n_split], l [..][n_split]
};

template <int HD>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
    constexpr int WPG = HD / 32;   // K words per lane group = MFMA k-steps per 16-row tile
    constexpr int NTD = HD / 16;   // 16-dim output tiles
    constexpr int ROWB = HD / 2;   // bytes per K row
    const KvLayerView &L = a.L;
    const int split = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
    const int qpos = a.len[s];
    const int n_ctx = qpos + 1;
    const int start = split * a.chunk;
    if (start >= n_ctx) return;
    const int end = min(start + a.chunk, n_ctx);
    const int n_split_s = (n_ctx + a.chunk - 1) / a.chunk;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, g = lane >> 4;
    const int G = a.G;

    // q operands (B of the QK MFMA): column n holds head n % G for n < 2G.
    half8 qh[WPG], ql[WPG];
    {
        const bool live = n < 2 * G;
        const int head = h * G + (live ? n % G : 0);
        const float *qrow = a.q + ((size_t)s * a.n_head + head) * HD;
#pragma unroll
        for (int t = 0; t < WPG; t++) {
            load_q8(a.rope, a.rope_pairs, qrow, WPG * g + t, qpos, qh[t], ql[t]);
            if (!live) {
                qh[t] = (half8)(_Float16)0.0f;
                ql[t] = (half8)(_Float16)0.0f;
            }
        }
    }
    const bool col_hi = n < G, col_lo = (n >= G) && (n < 2 * G);

    const size_t row = (size_t)s * L.H + h;
    const uint8_t *kbase = L.kp + row * L.P * ROWB;
    const uint8_t *vbase = L.vp + row * (L.P / 32) * (HD * 16);
    const float *ksb = L.ks + row * L.P;
    const float *vsb = L.vs + row * L.P;

    floatx4 o[NTD];
#pragma unroll
    for (int td = 0; td < NTD; td++) o[td] = (floatx4)0.0f;
    float m_run = kMinit, l_run = 0.0f;
    const float qk_scale = a.inv_sqrt_hd;

    for (int base = start + wave * 64; base < end; base += 256) {
        // ---- loads -----------------------------------------------------------------------
        uint32_t kw[4][WPG];
        floatx4 skv[4], svv[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            const uint8_t *kr = kbase + (size_t)(base + 16 * kt + n) * ROWB + g * (WPG * 4);
            if constexpr (WPG == 4) {
                const uint4 t4 = *reinterpret_cast<const uint4 *>(kr);
                kw[kt][0] = t4.x; kw[kt][1] = t4.y; kw[kt][2] = t4.z; kw[kt][3] = t4.w;
            } else {
                const uint2 t2 = *reinterpret_cast<const uint2 *>(kr);
                kw[kt][0] = t2.x; kw[kt][1] = t2.y;
            }
            skv[kt] = *reinterpret_cast<const floatx4 *>(ksb + base + 16 * kt + 4 * g);
            svv[kt] = *reinterpret_cast<const floatx4 *>(vsb + base + 16 * kt + 4 * g);
        }
        uint32_t vw[2][NTD];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const uint32_t *vr = reinterpret_cast<const uint32_t *>(vbase + (size_t)(base / 32 + b) * (HD * 16)) + lane * NTD;
#pragma unroll
            for (int q4 = 0; q4 < NTD / 4; q4++) {
                const uint4 t4 = reinterpret_cast<const uint4 *>(vr)[q4];
                vw[b][4 * q4 + 0] = t4.x; vw[b][4 * q4 + 1] = t4.y;
                vw[b][4 * q4 + 2] = t4.z; vw[b][4 * q4 + 3] = t4.w;
            }
        }
        // ---- S^T = K Q^T (rows: positions, columns: heads) --------------------------------------
        floatx4 sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            floatx4 acc = (floatx4)0.0f;
#pragma unroll
            for (int t = 0; t < WPG; t++) {
                const half8 ka = dequant8(kw[kt][t]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[t], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[t], acc, 0, 0, 0);
            }
            sc[kt] = acc;
        }
        // ---- online softmax (exp2 domain) ------------------------------------------------------
        float mloc = kMinit;
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int pos = base + 16 * kt + 4 * g + r;
                float x = sc[kt][r] * (skv[kt][r] * qk_scale);
                if (a.softcap > 0.0f) x = tanhf(x / a.softcap) * a.softcap;
                x = (pos < end) ? x * kLog2e : -INFINITY;
                sc[kt][r] = x;
                mloc = fmaxf(mloc, x);
            }
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        float psum = 0.0f;
        half2_t pp[4][2];  // [r][block]: (tile 2b, tile 2b+1) pair for slot r
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int pos = base + 16 * kt + 4 * g + r;
                const float p = exp2f(sc[kt][r] - m_new);
                psum += p;
                const float pv = (pos < end) ? p * svv[kt][r] : 0.0f;
                const _Float16 ph = (_Float16)pv;
                const _Float16 pl = (_Float16)(pv - (float)ph);
                const _Float16 sel = col_hi ? ph : (col_lo ? pl : (_Float16)0.0f);
                pp[r][kt >> 1][kt & 1] = sel;
            }
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int td = 0; td < NTD; td++) o[td] *= alpha;
        // ---- O^T += V^T P^T ------------------------------------------------------------------
#pragma unroll
        for (int b = 0; b < 2; b++) {
            half8 pb;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                pb[2 * r] = pp[r][b][0];
                pb[2 * r + 1] = pp[r][b][1];
            }
#pragma unroll
            for (int td = 0; td < NTD; td++) {
                const half8 va = dequant8(vw[b][td]);
                o[td] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[td], 0, 0, 0);
            }
        }
    }

    // ---- merge the 4 waves through LDS ---------------------------------------------------------
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    constexpr int OST = HD + 1;
    __shared__ float s_o[4][16 * OST];
    __shared__ float s_m[4][16], s_l[4][16];
    if (g == 0) {
        s_m[wave][n] = m_run;
        s_l[wave][n] = l_run;
    }
#pragma unroll
    for (int td = 0; td < NTD; td++)
#pragma unroll
        for (int r = 0; r < 4; r++) s_o[wave][n * OST + 16 * td + 4 * g + r] = o[td][r];
    __syncthreads();

    for (int idx = tid; idx < G * HD; idx += 256) {
        const int hh = idx / HD, d = idx % HD;
        float M = kMinit;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, s_m[w][hh]);
        float acc = 0.0f, lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float e = exp2f(s_m[w][hh] - M);
            acc += e * (s_o[w][hh * OST + d] + s_o[w][(hh + G) * OST + d]);
            lsum += e * s_l[w][hh];
        }
        const size_t head = (size_t)s * a.n_head + h * G + hh;
        if (n_split_s == 1) {
            a.out[head * HD + d] = lsum > 0.0f ? acc / lsum : 0.0f;
        } else {
            a.ws[(head * a.n_split + split) * HD + d] = acc;
            if (d == 0) {
                float *ml = a.ws + (size_t)L.S * a.n_head * a.n_split * HD;
                ml[head * a.n_split + split] = M;
                ml[(size_t)L.S * a.n_head * a.n_split + head * a.n_split + split] = lsum;
            }
        }
    }
}

// Log-sum-exp merge of the splits of one (sequence, head); one thread per dim.
template <int HD>
__global__ __launch_bounds__(HD) void decode_combine_kernel(DecodeArgs a) {
    const int head = blockIdx.x, s = blockIdx.y, d = threadIdx.x;
    const int n_ctx = a.len[s] + 1;
    const int ns = (n_ctx + a.chunk - 1) / a.chunk;
    if (ns <= 1) return;
    const size_t hidx = (size_t)s * a.n_head + head;
    const float *ml = a.ws + (size_t)a.L.S * a.n_head * a.n_split * HD;
    const float *mm = ml + hidx * a.n_split;
    const float *ll = ml + (size_t)a.L.S * a.n_head * a.n_split + hidx * a.n_split;
    float M = kMinit;
    for (int i = 0; i < ns; i++) M = fmaxf(M, mm[i]);
    float acc = 0.0f, lsum = 0.0f;
    for (int i = 0; i < ns; i++) {
        const float e = exp2f(mm[i] - M);
        acc += e * a.ws[(hidx * a.n_split + i) * HD + d];
        lsum += e * ll[i];
    }
    a.out[hidx * HD + d] = lsum > 0.0f ? acc / lsum : 0.0f;
}

}  // namespace

// Split plan: aim for ~kTargetWG workgroups in total so all 256 CUs get several, with each
// split a multiple of 64 positions.  n_split is non-decreasing in max_ctx.
DecodePlan decode_plan(int n_seq, int n_kv, int max_ctx) {
    constexpr int kTargetWG = 2048;
    const int units = n_seq * n_kv;
    int want = (kTargetWG + units - 1) / units;
    if (want < 1) want = 1;
    const int max_split_64 = (max_ctx + 63) / 64;
    if (want > max_split_64) want = max_split_64;
    int chunk = (max_ctx + want - 1) / want;
    chunk = (chunk + 63) / 64 * 64;
    DecodePlan p;
    p.chunk = chunk;
    p.n_split = (max_ctx + chunk - 1) / chunk;  // <= want
    p.cap = want;
    return p;
}

hipError_t launch_decode(const KvLayerView &L, const int32_t *d_len, const float *q, int n_head,
                         const float *rope, int rope_pairs, float softcap, float *out,
                         float *ws, const DecodePlan &plan, hipStream_t st) {
    DecodeArgs a;
    a.L = L;
    a.len = d_len;
    a.q = q;
    a.rope = rope;
    a.rope_pairs = rope_pairs;
    a.n_head = n_head;
    a.G = n_head / L.H;
    a.chunk = plan.chunk;
    a.n_split = plan.n_split;
    a.inv_sqrt_hd = 1.0f / sqrtf((float)L.hd);
    a.softcap = softcap;
    a.out = out;
    a.ws = ws;
    dim3 grid(plan.n_split, L.H, L.S);
    if (L.hd == 128) {
        decode_split_kernel<128><<<grid, 256, 0, st>>>(a);
        if (plan.n_split > 1) decode_combine_kernel<128><<<dim3(n_head, L.S), 128, 0, st>>>(a);
    } else if (L.hd == 64) {
        decode_split_kernel<64><<<grid, 256, 0, st>>>(a);
        if (plan.n_split > 1) decode_combine_kernel<64><<<dim3(n_head, L.S), 64, 0, st>>>(a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ts
