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
//   (two 16-column tiles) and walks the keys 0..its last query position in 32-key windows.
//   Every window's K and V are dequantized once per wave (exact f16 integer codes) and feed
//   both column tiles.
// * S^T = K Q^T with q split hi + lo (two f16 MFMAs into one f32 accumulator), scale s_k and
//   1/sqrt(hd) applied in f32, causal mask per column, online softmax in the exp2 domain,
//   then O^T += V^T P^T with p*s_v in f16.
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

constexpr int kColsPerWave = 32;
constexpr int kColsPerBlock = 4 * kColsPerWave;

template <int HD>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
    constexpr int WPG = HD / 32;
    constexpr int NTD = HD / 16;
    constexpr int ROWB = HD / 2;
    const KvLayerView &L = a.L;
    // Heavier column blocks (later tokens) first.
    const int cblk = gridDim.x - 1 - blockIdx.x;
    const int h = blockIdx.y, s = blockIdx.z;
    const int G = a.G;
    const int n_cols = a.n_tok * G;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, g = lane >> 4;
    const int c_wave = cblk * kColsPerBlock + wave * kColsPerWave;
    if (c_wave >= n_cols) return;
    const int len0 = a.len[s];
    const DeqConst dc;

    // Per column tile: this lane's column, its token, query position and q operands.
    half8 qh[2][WPG], ql[2][WPG];
    int qpos[2];
    bool live[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int c = c_wave + 16 * nt + n;
        live[nt] = c < n_cols;
        const int cc = live[nt] ? c : 0;
        const int tok = cc / G, head = h * G + cc % G;
        qpos[nt] = live[nt] ? len0 + tok : -1;
        const float *qrow = a.q + (((size_t)s * a.n_tok + tok) * a.n_head + head) * HD;
#pragma unroll
        for (int t = 0; t < WPG; t++) {
            load_q8(a.rope, a.rope_pairs, qrow, WPG * g + t, len0 + tok, 1.0f, qh[nt][t], ql[nt][t]);
            if (!live[nt]) {
                qh[nt][t] = (half8)(_Float16)0.0f;
                ql[nt][t] = (half8)(_Float16)0.0f;
            }
        }
    }
    // Last key any column of this wave needs (inclusive).
    const int c_last = min(c_wave + kColsPerWave, n_cols) - 1;
    const int key_end = len0 + c_last / G + 1;

    const size_t row = (size_t)s * L.H + h;
    const uint8_t *kbase = L.kp + row * L.P * ROWB;
    const uint8_t *vbase = L.vp + row * (L.P / 32) * (HD * 16);
    const float *ksb = L.ks + row * L.P;
    const float *vsb = L.vs + row * L.P;

    floatx4 o[2][NTD];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int td = 0; td < NTD; td++) o[nt][td] = (floatx4)0.0f;
    float m_run[2] = {kMinit, kMinit}, l_run[2] = {0.0f, 0.0f};

    for (int base = 0; base < key_end; base += 32) {
        uint32_t kw[2][WPG];
        floatx4 skv[2], svv[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
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
        uint32_t vw[NTD];
        {
            const uint32_t *vr = reinterpret_cast<const uint32_t *>(vbase + (size_t)(base / 32) * (HD * 16)) + lane * NTD;
#pragma unroll
            for (int q4 = 0; q4 < NTD / 4; q4++) {
                const uint4 t4 = reinterpret_cast<const uint4 *>(vr)[q4];
                vw[4 * q4 + 0] = t4.x; vw[4 * q4 + 1] = t4.y;
                vw[4 * q4 + 2] = t4.z; vw[4 * q4 + 3] = t4.w;
            }
        }
        floatx4 sc[2][2];  // [nt][kt]
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int kt = 0; kt < 2; kt++) sc[nt][kt] = (floatx4)0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
#pragma unroll
            for (int t = 0; t < WPG; t++) {
                const half8 ka = dequant8(kw[kt][t], dc);
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    sc[nt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[nt][t], sc[nt][kt], 0, 0, 0);
                    sc[nt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[nt][t], sc[nt][kt], 0, 0, 0);
                }
            }
        }
        half8 pb[2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            float mloc = kMinit;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int pos = base + 16 * kt + 4 * g + r;
                    float x = sc[nt][kt][r] * (skv[kt][r] * a.inv_sqrt_hd);
                    if (a.softcap > 0.0f) x = tanhf(x / a.softcap) * a.softcap;
                    x = (pos <= qpos[nt]) ? x * kLog2e : -INFINITY;
                    sc[nt][kt][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            const float m_new = fmaxf(m_run[nt], mloc);
            const float alpha = exp2f(m_run[nt] - m_new);
            m_run[nt] = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int pos = base + 16 * kt + 4 * g + r;
                    const float p = exp2f(sc[nt][kt][r] - m_new);
                    psum += p;
                    const float pv = (pos <= qpos[nt]) ? p * svv[kt][r] : 0.0f;
                    pb[nt][2 * r + kt] = (_Float16)pv;
                }
            }
            l_run[nt] = l_run[nt] * alpha + psum;
#pragma unroll
            for (int td = 0; td < NTD; td++) o[nt][td] *= alpha;
        }
#pragma unroll
        for (int td = 0; td < NTD; td++) {
            const half8 va = dequant8(vw[td], dc);
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
                o[nt][td] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[nt], o[nt][td], 0, 0, 0);
        }
    }

#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        float l = l_run[nt];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        if (!live[nt]) continue;
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
    dim3 grid((n_cols + kColsPerBlock - 1) / kColsPerBlock, L.H, L.S);
    if (L.hd == 128)
        prefill_kernel<128><<<grid, 256, 0, st>>>(a);
    else if (L.hd == 64)
        prefill_kernel<64><<<grid, 256, 0, st>>>(a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace ts
