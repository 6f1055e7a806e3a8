// ts_prefill.hip -- chunked-prefill causal attention over the INT4 cache for gfx950.
//
// Semantics: the CPU reference attention with a KV cache (src/ops/reference/attention.rs:
// 236-313, causal mask softmax.rs:104-109): query t of the chunk sits at absolute position
// len+t and attends to positions 0..len+t of the dequantized INT4 cache.  It replaces the f32
// main_attn_out used by batched prefill (sh_layer_v1.wgsl:662-762), which recomputes every
// score per output element, with matrix-core tiles:
//
// * The (query token, head) pairs that share one kv head form the columns of the MFMA
//   N dimension: column c of a (sequence, kv head) is token c / G, head c % G.
// * grid = (column block of 128, kv head, sequence); each of the 4 waves owns 32 columns
//   (two 16-column tiles).  The workgroup walks the keys in 64-key windows: every thread
//   loads one 16-byte piece of the next window's K rows / V blocks / scales while the current
//   window is computed, then converts it to exact f16 integer codes in a double-buffered LDS
//   tile, so each code is converted once per workgroup and read by all 4 waves.
// * S^T = K Q^T with q split hi + lo (two f16 MFMAs into one f32 accumulator) and
//   1/sqrt(hd)*log2(e) folded into q; the score is scaled by s_k in f32, masked only in
//   windows that cross the causal diagonal, and enters an online softmax in the exp2 domain
//   whose running max is raised lazily; p*s_v goes to O^T += V^T P^T split hi + lo in f16
//   (two MFMAs) under an exponent bound that keeps it below 2^15.
// * Each wave owns whole output rows, so the result is written straight from registers.
#include "ts_mfma.h"

namespace ts {
namespace {

struct PrefillArgs {
    KvLayerView L;
    const int32_t *len;
    const float *q;
    const float *rope;
    int rope_pairs;
    int n_head;
    int G;
    int n_tok;
    float inv_sqrt_hd;
    float softcap;
    float *out;
};

#ifndef TS_PREFILL_NW
#define TS_PREFILL_NW 4
#endif

constexpr int kColsPerWave = 32;
constexpr int kWin = 64;  // keys per window

// Double-buffered window tiles.  K: [key][word] f16 codes; V^T: [dim][8-key group] f16 codes
// in the PV operand's key order.  Rows are unpadded; the 16-byte slots inside a row are
// rotated per row (k_slot, v_slot) so that the MFMA operand reads of a wave hit distinct LDS
// banks (measured on gfx950: 2x the read rate of padded rows).
template <int HD>
struct PrefillLds {
    half8 k[2][kWin][HD / 8];
    half8 v[2][HD][kWin / 8];
    float sk[2][kWin], sv[2][kWin];
    float svlog[2];  // log2 of the window's largest s_v
};

// The next window as one thread holds it in flight: its 16-byte pieces of the K window and of
// the V window (NK each; HD=64 with 4 waves has half a piece per thread, so half the threads
// take a K piece and half a V piece) and one scale.
template <int HD, int NW>
struct Pending {
    static constexpr int KCH = kWin * HD / 32;    // 16-byte pieces of the K window (= V window)
    static constexpr int NT = 64 * NW;            // threads
    static constexpr int NK = KCH >= NT ? KCH / NT : 1;
    static constexpr bool SPLIT = KCH < NT;       // threads [0, KCH) take K, [KCH, 2 KCH) take V
    static_assert(KCH % NT == 0 || 2 * KCH == NT, "window pieces must spread evenly");
    uint4 k[NK], v[SPLIT ? 1 : NK];
    float scale;
};

// Slot of word w in the K row of `key`, and of 8-key group cg in the V^T row `row`.
template <int HD>
__device__ inline int k_slot(int key, int w) {
    const int k = key & 15;
    if constexpr (HD == 128)
        return (w + k + 4 * (k >> 2)) & 15;
    else
        return ((w >> 1) + 4 * (w & 1) + k) & 7;
}
__device__ inline int v_slot(int row, int cg) { return (cg + row) & 7; }

// Which 16-byte piece of the window a staging thread owns.  The maps are chosen so that 16
// consecutive lanes write 16 different LDS bank groups:
//  K piece c: key (c & 15) + 16 * (c / (16 * PPR)), part (c >> 4) % PPR of the key's row;
//  V piece c: block c / HD, and within it lane group L = c % 64 of the packed layout, its
//  (HD/64)-th piece (c % HD) / 64.
template <int HD>
__device__ inline void k_piece(int c, int &key, int &part) {
    constexpr int PPR = HD / 32;  // 16-byte pieces per K row
    key = (c & 15) + 16 * (c / (16 * PPR));
    part = (c >> 4) % PPR;
}
template <int HD>
__device__ inline void v_piece(int cv, int &b, int &piece) {
    constexpr int PPL = HD / 64;  // 16-byte pieces per packed lane group
    b = cv / HD;
    piece = PPL * (cv % 64) + (cv % HD) / 64;
}

template <int HD, int NW>
__device__ inline void fetch_window(Pending<HD, NW> &pd, const uint8_t *kbase, const uint8_t *vbase,
                                    const float *ksb, const float *vsb, int base, int tid, int wave) {
    using P = Pending<HD, NW>;
    constexpr int ROWB = HD / 2;
    auto load_k = [&](int c) {
        int key, part;
        k_piece<HD>(c, key, part);
        return *reinterpret_cast<const uint4 *>(kbase + (size_t)(base + key) * ROWB + part * 16);
    };
    auto load_v = [&](int c) {
        int b, piece;
        v_piece<HD>(c, b, piece);
        return *reinterpret_cast<const uint4 *>(vbase + (size_t)(base / 32 + b) * (HD * 16) + piece * 16);
    };
    if constexpr (P::SPLIT) {
        // wave-uniform: the first KCH/64 waves take K pieces, the rest V pieces
        if (wave < P::KCH / 64)
            pd.k[0] = load_k(tid);
        else
            pd.k[0] = load_v(tid - P::KCH);
    } else {
#pragma unroll
        for (int i = 0; i < P::NK; i++) pd.k[i] = load_k(tid + P::NT * i);
#pragma unroll
        for (int i = 0; i < P::NK; i++) pd.v[i] = load_v(tid + P::NT * i);
    }
    if (tid < kWin)
        pd.scale = ksb[base + tid];
    else if (tid < 2 * kWin)
        pd.scale = vsb[base + tid - kWin];
}

template <int HD, int NW>
__device__ inline void stage_window(PrefillLds<HD> &sm, int buf, const Pending<HD, NW> &pd, int tid,
                                    int wave, float inv_s, const DeqConst &dc) {
    using P = Pending<HD, NW>;
    constexpr int NTD = HD / 16;
    auto put_k = [&](int c, const uint4 &x) {
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
        int key, part;
        k_piece<HD>(c, key, part);
#pragma unroll
        for (int j = 0; j < 4; j++) sm.k[buf][key][k_slot<HD>(key, 4 * part + j)] = dequant8(w[j], dc);
    };
    auto put_v = [&](int c, const uint4 &x) {
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
        int b, piece;
        v_piece<HD>(c, b, piece);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // word (gg*16 + dl)*NTD + td of the block holds dim 16td+dl, key group gg
            const int widx = 4 * piece + j;
            const int ln = widx / NTD, td = widx % NTD;
            const int row = 16 * td + (ln & 15);
            sm.v[buf][row][v_slot(row, 4 * b + (ln >> 4))] = dequant8(w[j], dc);
        }
    };
    if constexpr (P::SPLIT) {
        if (wave < P::KCH / 64)
            put_k(tid, pd.k[0]);
        else
            put_v(tid - P::KCH, pd.k[0]);
    } else {
#pragma unroll
        for (int i = 0; i < P::NK; i++) put_k(tid + P::NT * i, pd.k[i]);
#pragma unroll
        for (int i = 0; i < P::NK; i++) put_v(tid + P::NT * i, pd.v[i]);
    }
    if (tid < kWin) {
        sm.sk[buf][tid] = pd.scale * inv_s;  // undo the q operand scale (a power of two: exact)
    } else if (tid < 2 * kWin) {
        sm.sv[buf][tid - kWin] = pd.scale;
        float m = pd.scale;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (tid == kWin) sm.svlog[buf] = __log2f(m);
    }
}

// Scores of one 64-key window for one 16-column tile -> f16 probabilities (times s_v) in PV
// operand order, with the online-softmax state update.  MASK: the window crosses the causal
// diagonal of some column.
template <int NTD, bool SOFTCAP>
__device__ inline void window_softmax(floatx4 (&sc)[4], const float *sk, const float *sv, float svl,
                                      float softcap, bool mask, int base, int g, int qpos,
                                      float &m_run, float &l_run, floatx4 (&o)[NTD],
                                      half8 (&pb)[2], half8 (&pl)[2]) {
    // sk, sv: the window's scales in LDS; this lane's keys are 16kt + 4g + r.
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        const floatx4 sk4 = *reinterpret_cast<const floatx4 *>(sk + 16 * kt + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float x = sc[kt][r] * sk4[r];
            if (SOFTCAP) x = tanhf(x / softcap) * softcap * kLog2e;
            sc[kt][r] = x;
        }
    }
    if (mask) {
        // a real branch: only windows on the causal diagonal pay for the compares
        asm volatile("");
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (base + 16 * kt + 4 * g + r > qpos) sc[kt][r] = -INFINITY;
    }
    float mloc = kMinit;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) mloc = fmaxf(mloc, sc[kt][r]);
    mloc = group_max(mloc);
    // Keep p <= 2^8 and p*s_v <= 2^15 (f16 range); raise the running max only when the window
    // breaks either bound.
    const float need = fmaxf(mloc - 8.0f, mloc + svl - 15.0f);
    if (__builtin_amdgcn_ballot_w64(need > m_run) != 0) {
        const float m_new = need > m_run ? mloc + fmaxf(0.0f, svl - 15.0f) : m_run;
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int td = 0; td < NTD; td++) o[td] *= alpha;
    }
    float psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        const floatx4 sv4 = *reinterpret_cast<const floatx4 *>(sv + 16 * kt + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = __builtin_amdgcn_exp2f(sc[kt][r] - m_run);
            psum += p;
            // p * s_v = hi + lo in f16 (~22 bits): one f16 would carry a relative error of 2^-11
            // into the output whenever a few keys dominate the row
            const float pv = opaque(p * sv4[r]);
            const _Float16 hi = (_Float16)pv;
            pb[kt >> 1][2 * r + (kt & 1)] = hi;
            pl[kt >> 1][2 * r + (kt & 1)] = (_Float16)(pv - (float)hi);
        }
    }
    l_run += psum;
}

template <int HD, bool SOFTCAP>
__global__ __launch_bounds__(64 * TS_PREFILL_NW, 2) void prefill_kernel(PrefillArgs a) {
    constexpr int NW = TS_PREFILL_NW;
    constexpr int WPG = HD / 32;
    constexpr int NTD = HD / 16;
    constexpr int ROWB = HD / 2;
    constexpr int COLS = NW * kColsPerWave;  // columns per block
    const KvLayerView &L = a.L;
    // Workgroups are dispatched round robin over the 8 XCDs by linear id.  Give XCD x the
    // contiguous range [x*N/8, (x+1)*N/8) of (column block, kv head, sequence) in row order, so
    // the 16-odd blocks that read one (sequence, kv head) stream share an L2 and every XCD gets
    // the same mix of long and short blocks.
    int xb = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
    {
        const int n_wg = gridDim.x * gridDim.y * gridDim.z;
        if (n_wg % 8 == 0) {
            const int id = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
            const int logical = (id % 8) * (n_wg / 8) + id / 8;
            xb = logical % gridDim.x;
            h = (logical / gridDim.x) % gridDim.y;
            s = logical / (gridDim.x * gridDim.y);
        }
    }
    const int G = a.G;
    const int n_cols = a.n_tok * G;
    const int n_blk = (n_cols + COLS - 1) / COLS;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int len0 = a.len[s];
    const DeqConst dc;
    __shared__ PrefillLds<HD> sm;
    __shared__ float sm_qb[NW];

    const size_t row = (size_t)s * L.H + h;
    const uint8_t *kbase = L.kp + row * L.P * ROWB;
    const uint8_t *vbase = L.vp + row * (L.P / 32) * (HD * 16);
    const float *ksb = L.ks + row * L.P;
    const float *vsb = L.vs + row * L.P;
    const float qmul = SOFTCAP ? a.inv_sqrt_hd : a.inv_sqrt_hd * kLog2e;

    // Heavier column blocks (later tokens) first.
    {
        const int cblk = n_blk - 1 - xb;
        const int c_blk = cblk * COLS;
        const int c_wave = c_blk + wave * kColsPerWave;

        // Per column tile: this lane's column, its query position and q operands (rotated,
        // times 1/sqrt(hd) and, without softcap, log2(e); split hi/lo).
        // One power-of-two q scale per workgroup, from a bound over all its columns.
        float q_s, inv_s;
        {
            float qb = 0.0f;
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                const int c = min(c_wave + 16 * nt + n, n_cols - 1);
                const float *qrow = a.q + (((size_t)s * a.n_tok + c / G) * a.n_head + h * G + c % G) * HD;
#pragma unroll
                for (int t = 0; t < WPG; t++) qb = fmaxf(qb, q_bound8(qrow, WPG * g + t));
            }
            qb = wave_max(qb);
            if (lane == 0) sm_qb[wave] = qb;
            __syncthreads();
#pragma unroll
            for (int w = 0; w < NW; w++) qb = fmaxf(qb, sm_qb[w]);
            q_scale(qb * qmul, q_s, inv_s);
        }
        half8 qh[2][WPG], ql[2][WPG];
        int qpos[2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int c = c_wave + 16 * nt + n;
            const bool live = c < n_cols;
            const int cc = live ? c : 0;
            const int tok = cc / G, head = h * G + cc % G;
            qpos[nt] = live ? len0 + tok : -1;
            const float *qrow = a.q + (((size_t)s * a.n_tok + tok) * a.n_head + head) * HD;
#pragma unroll
            for (int t = 0; t < WPG; t++) {
                load_q8(a.rope, a.rope_pairs, qrow, WPG * g + t, len0 + tok, qmul * q_s, qh[nt][t], ql[nt][t]);
                if (!live) {
                    qh[nt][t] = (half8)(_Float16)0.0f;
                    ql[nt][t] = (half8)(_Float16)0.0f;
                }
            }
        }
        // Query positions this wave covers (inclusive); qmax < 0 for a wave with no columns.
        const int qmin_w = len0 + c_wave / G;
        const int qmax_w = c_wave < n_cols ? len0 + (min(c_wave + kColsPerWave, n_cols) - 1) / G : -1;
        const int key_end = len0 + (min(c_blk + COLS, n_cols) - 1) / G + 1;
        const int n_win = (key_end + kWin - 1) / kWin;

        floatx4 o[2][NTD];
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int td = 0; td < NTD; td++) o[nt][td] = (floatx4)0.0f;
        float m_run[2] = {kMinit, kMinit}, l_run[2] = {0.0f, 0.0f};

        Pending<HD, NW> pd;
        fetch_window<HD, NW>(pd, kbase, vbase, ksb, vsb, 0, tid, wave);
        stage_window<HD, NW>(sm, 0, pd, tid, wave, inv_s, dc);
        __syncthreads();

        for (int w = 0; w < n_win; w++) {
            const int buf = w & 1, base = w * kWin;
            const bool more = w + 1 < n_win;
            if (more) fetch_window<HD, NW>(pd, kbase, vbase, ksb, vsb, base + kWin, tid, wave);
            // keep the prefetch ahead of the compute below
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);

            if (base <= qmax_w) {
                floatx4 sc[2][4];
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
#pragma unroll
                    for (int kt = 0; kt < 4; kt++) sc[nt][kt] = (floatx4)0.0f;
#pragma unroll
                for (int kt = 0; kt < 4; kt++) {
#pragma unroll
                    for (int t = 0; t < WPG; t++) {
                        const half8 ka = sm.k[buf][16 * kt + n][k_slot<HD>(n, WPG * g + t)];
#pragma unroll
                        for (int nt = 0; nt < 2; nt++) {
                            sc[nt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[nt][t], sc[nt][kt], 0, 0, 0);
                            sc[nt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[nt][t], sc[nt][kt], 0, 0, 0);
                        }
                    }
                }
                const float svl = sm.svlog[buf];
                half8 pb[2][2], pl[2][2];  // [nt][32-key half]: p*s_v high and low f16 parts
                const bool mask = base + kWin - 1 > qmin_w;  // some key of the window is masked
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
                    window_softmax<NTD, SOFTCAP>(sc[nt], sm.sk[buf], sm.sv[buf], svl, a.softcap, mask, base,
                                                 g, qpos[nt], m_run[nt], l_run[nt], o[nt], pb[nt], pl[nt]);
#pragma unroll
                for (int b = 0; b < 2; b++) {
#pragma unroll
                    for (int td = 0; td < NTD; td++) {
                        const half8 va = sm.v[buf][16 * td + n][v_slot(n, 4 * b + g)];
#pragma unroll
                        for (int nt = 0; nt < 2; nt++) {
                            o[nt][td] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[nt][b], o[nt][td], 0, 0, 0);
                            o[nt][td] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[nt][b], o[nt][td], 0, 0, 0);
                        }
                    }
                }
            }
            if (more) stage_window<HD, NW>(sm, buf ^ 1, pd, tid, wave, inv_s, dc);
            __syncthreads();
        }

#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const float l = group_sum(l_run[nt]);
            if (qpos[nt] < 0) continue;
            const int c = c_wave + 16 * nt + n;
            const int tok = c / G, head = h * G + c % G;
            float *orow = a.out + (((size_t)s * a.n_tok + tok) * a.n_head + head) * HD;
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
            for (int td = 0; td < NTD; td++) {
                float4 v4 = make_float4(o[nt][td][0] * inv, o[nt][td][1] * inv, o[nt][td][2] * inv,
                                        o[nt][td][3] * inv);
                *reinterpret_cast<float4 *>(orow + 16 * td + 4 * g) = v4;
            }
        }
    }
}

}  // namespace

hipError_t launch_prefill(const KvLayerView &L, const int32_t *d_len, const float *q,
                          int n_head, int n_tok, const float *rope, int rope_pairs,
                          float softcap, float *out, hipStream_t st) {
    PrefillArgs a;
    a.L = L;
    a.len = d_len;
    a.q = q;
    a.rope = rope;
    a.rope_pairs = rope_pairs;
    a.n_head = n_head;
    a.G = n_head / L.H;
    a.n_tok = n_tok;
    a.inv_sqrt_hd = 1.0f / sqrtf((float)L.hd);
    a.softcap = softcap;
    a.out = out;
    const int n_cols = n_tok * a.G;
    const int cols = TS_PREFILL_NW * kColsPerWave;
    const int n_blk = (n_cols + cols - 1) / cols;
    dim3 grid(n_blk, L.H, L.S);
    const bool cap = softcap > 0.0f;
    if (L.hd == 128 && cap)
        prefill_kernel<128, true><<<grid, 64 * TS_PREFILL_NW, 0, st>>>(a);
    else if (L.hd == 128)
        prefill_kernel<128, false><<<grid, 64 * TS_PREFILL_NW, 0, st>>>(a);
    else if (L.hd == 64 && cap)
        prefill_kernel<64, true><<<grid, 64 * TS_PREFILL_NW, 0, st>>>(a);
    else if (L.hd == 64)
        prefill_kernel<64, false><<<grid, 64 * TS_PREFILL_NW, 0, st>>>(a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace ts
