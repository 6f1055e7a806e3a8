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
//   and scales exactly once for all G = n_head/n_kv query heads that share them.  The chunk
//   is planned from the total context of the batch, so ragged batches get more splits for
//   their long sequences and the count of busy workgroups stays at the planned one.
// * each wave takes 64-position windows round robin; in the integer kernel every 16-byte load
//   instruction reads one contiguous kilobyte (the cache's chunk order puts each lane's K row
//   segment and V words there), non-temporally, and each workgroup starts its windows at its
//   own offset, so the concurrent streams spread over the HBM channels.
// * QK^T and PV run on the matrix cores (v_mfma_f32_16x16x32_f16).  INT4 codes convert to
//   exact f16 integers with two bit tricks (0x6400|nibble is 1024+nibble; the second nibble of
//   a byte is taken as 1024+16*nibble and fixed with one packed f16 FMA), so K and V enter the
//   MFMA exactly.  The per-position scales are applied in f32 outside the MFMA: s_k on the
//   scores, s_v folded into the probabilities.
// * q is split hi + lo in f16 (q = hi + lo to ~22 bits).  With G = n_head/n_kv <= 8 query
//   heads per kv head, 2G of the 16 MFMA columns carry the hi parts of the G heads and their
//   lo parts, so one MFMA gives both halves of every score (summed across lanes afterwards)
//   and scores carry f32-level accuracy; the probabilities enter PV split the same way.
// * online softmax in the exp2 domain with one cross-lane max per 64 positions and lazy
//   rescaling; s_v is folded into the probabilities under a per-window exponent bound so they
//   never leave f16 range.  A workgroup's waves merge through LDS; splits merge in a second
//   kernel (log-sum-exp combine) unless a sequence fits one split.
#include <stdlib.h>

#include "ts_mfma.h"
#include "ts_quant.h"

namespace ts {
namespace {

struct DecodeArgs {
    KvLayerView L;
    const int32_t *len;
    // hlen >= 0 (one sequence): its length, given by the host with the launch (as the
    // reference passes its uniforms) instead of read from len[] first: an eager call whose
    // host length is known to match the device's.  -1: read len[].
    int hlen;
    const float *q;
    const float *rope;
    int rope_pairs;
    int n_head;
    int G;   // query heads per workgroup: n_head / n_kv (integer kernel, up to 16), at most 8 per
             // group (16x16 kernel)
    int Gt;  // query heads per kv head (n_head / n_kv)
    int NG;  // head groups per kv head: grid.y = n_kv * NG (integer kernel: 1)
    int chunk;
    int n_split;  // grid.x: the last split of a sequence runs to its end
    float inv_sqrt_hd;
    float softcap;
    float *out;
    float *ws;  // partial o [S][n_head][n_split][hd], then m [..][n_split], l [..][n_split]

    // Fused append (ts_attn_decode_append): the new token's raw K and V, [S][H][hd], or null.
    const float *k_new, *v_new;

    // ts_attn_decode_append_advance: the lengths to advance by one (the array len points to)
    // and the arrival counter of the kernel that does it, or null.
    int32_t *adv_len;
    int32_t *adv_ctr;
};

// Every workgroup of the launch's last kernel calls this once, after its last read of the
// lengths: the workgroup that arrives last (all others have read them by then) advances every
// length by one and clears the counter for the next launch.  Call from all threads of the
// workgroup (the barrier orders this workgroup's length reads before its arrival).
__device__ inline void arrive_and_advance(const DecodeArgs &a) {
    if (!a.adv_ctr) return;
    if (a.hlen >= 0) {
        // the length came with the launch and no workgroup reads len[]: one plain store of the
        // advanced value, no arrival count (a returning atomic's round trip saved)
        if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) a.adv_len[0] = a.hlen + 1;
        return;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int n_wg = gridDim.x * gridDim.y * gridDim.z;
        if (atomicAdd(a.adv_ctr, 1) == n_wg - 1) {
            for (int s = 0; s < a.L.S; s++) a.adv_len[s] += 1;
            *a.adv_ctr = 0;
        }
    }
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One 64-position window of one (sequence, kv head) stream, as held by one lane in registers
// while it is in flight: K rows (tile kt, row n, the words of lane group g), V blocks (block b,
// words lane*NTD..), and one K and one V scale (position base + lane).
template <int HD>
struct Window {
    static constexpr int WPG = HD / 32, NTD = HD / 16;
    uint32_t kw[4][WPG];
    uint32_t vw[2][NTD];
    float sk, sv;
};

// Buffer resources of one (sequence, kv head) stream, bounded to the positions of one split:
// loads past the bound return zeros without touching memory, so prefetches can be issued
// unconditionally (which keeps the compiler's load counters static, so the wait before each
// window only covers that window's own loads).
struct Streams {
    __amdgpu_buffer_rsrc_t k, v;
    const float *ksb, *vsb;
    int last;  // last position of the split
};

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// K word that lane group g feeds to the 16x16 QK instruction at k-step t (of the WPG words of
// its row): the words the cache keeps together in one chunk for that row and group (the
// chunk order of k_word_idx), so one load per row brings them all.
template <int HD>
__device__ inline int k16_word(int g, int t) {
    if constexpr (HD >= 128) return 8 * (t >> 1) + 2 * g + (t & 1);
    else return 2 * g + t;
}

template <int HD>
__device__ __forceinline__ void load_window(Window<HD> &w, const Streams &st, int base, int n,
                                            int g, int lane) {
    constexpr int WPG = HD / 32, NTD = HD / 16, ROWB = HD / 2;
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        // row r = 16 kt + n of the window: words k16_word(g, 0..WPG-1) sit in chunk
        // ((r % 4) / (128 / HD)) * 64 + 16 g + r / 4, at word (r % 2) * 2 for hd 64
        const int r = 16 * kt + n;
        if constexpr (WPG == 8) {
            // hd 256: the 8 words sit in chunks (2 (r % 4) + c) * 64 + 16 g + r / 4, c = 0, 1
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int koff = ((2 * (r & 3) + c) * 64 + 16 * g + (r >> 2)) * 16;
                const u32x4 t4 = __builtin_amdgcn_raw_buffer_load_b128(st.k, koff, base * ROWB, 0);
                w.kw[kt][4 * c] = t4[0]; w.kw[kt][4 * c + 1] = t4[1]; w.kw[kt][4 * c + 2] = t4[2]; w.kw[kt][4 * c + 3] = t4[3];
            }
        } else if constexpr (WPG == 4) {
            const int koff = ((r & 3) * 64 + 16 * g + (r >> 2)) * 16;
            const u32x4 t4 = __builtin_amdgcn_raw_buffer_load_b128(st.k, koff, base * ROWB, 0);
            w.kw[kt][0] = t4[0]; w.kw[kt][1] = t4[1]; w.kw[kt][2] = t4[2]; w.kw[kt][3] = t4[3];
        } else {
            const int koff = (((r & 3) >> 1) * 64 + 16 * g + (r >> 2)) * 16 + 8 * (r & 1);
            const u32x2 t2 = __builtin_amdgcn_raw_buffer_load_b64(st.k, koff, base * ROWB, 0);
            w.kw[kt][0] = t2[0]; w.kw[kt][1] = t2[1];
        }
    }
#pragma unroll
    for (int b = 0; b < 2; b++) {
#pragma unroll
        for (int q4 = 0; q4 < NTD / 4; q4++) {
            // words 4 q4 .. 4 q4 + 3 of lane group `lane`: chunk q4 * 64 + lane
            const u32x4 t4 = __builtin_amdgcn_raw_buffer_load_b128(st.v, (q4 * 64 + lane) * 16 + b * (HD * 16), (base / 32) * (HD * 16), 0);
            w.vw[b][4 * q4 + 0] = t4[0]; w.vw[b][4 * q4 + 1] = t4[1];
            w.vw[b][4 * q4 + 2] = t4[2]; w.vw[b][4 * q4 + 3] = t4[3];
        }
    }
    // Scales: plain loads with the index clamped into the split; windows past the end re-read
    // valid, unused scales.
    const int sp = min(base + lane, st.last);
    w.sk = st.ksb[sp];
    w.sv = st.vsb[sp];
}

// Running state of one wave: O^T accumulators (column n = head, rows = dims 16td+4g+r), the
// reference exponent m (exp2 domain) and the softmax sum l.
template <int HD>
struct WaveState {
    floatx4 o[HD / 16];
    float m, l;
};

// q operands in LDS, [k-step t][lane], shared by the waves of a workgroup.  Column n of the
// MFMA (lane group n = lane & 15) carries the f16 high part of head n for n < G and the low
// part (q - hi) of head n - G for G <= n < 2G, so one MFMA computes both halves of every
// score; G <= 8 keeps 2G within the 16 columns.
template <int HD>
struct QLds {
    half8 p[HD / 32][64];
};

// live: this lane's column carries a head (n < 2G); lo_col: it carries the low parts (G <= n);
// partner4: byte address (for ds_bpermute) of the lane holding the other part of its scores.
template <int HD, bool SOFTCAP>
__device__ __forceinline__ void process_window(const Window<HD> &w, WaveState<HD> &st,
                                               const QLds<HD> &qs, float *stage, int base, int end,
                                               int lane, int g, bool live, bool lo_col, int partner4,
                                               float inv_s, float softcap, const DeqConst &dc) {
    constexpr int WPG = HD / 32, NTD = HD / 16;
    // Scales: one per lane in registers -> this wave's LDS stage -> the 4 positions each lane
    // holds per tile (16kt + 4g + r).  Same-wave LDS traffic is ordered: no barrier needed.
    stage[lane] = w.sk * inv_s;  // undo the q operand scale (a power of two: exact)
    stage[64 + lane] = w.sv;
    // ---- S^T = K Q^T (rows: positions, columns: heads), hi + lo q in one accumulator --------
    floatx4 sc[4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) sc[kt] = (floatx4)0.0f;
#pragma unroll
    for (int t = 0; t < WPG; t++) {
        const half8 qp = qs.p[t][lane];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            const half8 ka = dequant8(w.kw[kt][t], dc);
            sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qp, sc[kt], 0, 0, 0);
        }
    }
    // hi column + lo column: lanes n and n +- G swap partial scores and both hold the same sum
    // (a + b == b + a exactly), so the two columns run identical softmax arithmetic below.
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            sc[kt][r] += __int_as_float(__builtin_amdgcn_ds_bpermute(partner4, __float_as_int(sc[kt][r])));
    // ---- softmax ----------------------------------------------------------------------------
    // x = score * log2(e).  s_v is folded into the probabilities: P = 2^(x - m) * s_v, with the
    // window reference m >= max(x) + log2(max s_v), so P <= 1 always fits f16.
    float x[16], sv[16];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        const floatx4 sk4 = *reinterpret_cast<const floatx4 *>(stage + 16 * kt + 4 * g);
        const floatx4 sv4 = *reinterpret_cast<const floatx4 *>(stage + 64 + 16 * kt + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = sc[kt][r] * sk4[r];
            if constexpr (SOFTCAP) v = tanhf(v * (1.0f / kLog2e) / softcap) * softcap * kLog2e;
            x[4 * kt + r] = v;
            sv[4 * kt + r] = sv4[r];
        }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {  // positions past the split's end
        const int pos = base + 16 * (i >> 2) + 4 * g + (i & 3);
        if (pos >= end) {
            x[i] = -INFINITY;
            sv[i] = 0.0f;
        }
    }
    float xm = x[0], sm = sv[0];
#pragma unroll
    for (int i = 1; i < 16; i++) {
        xm = fmaxf(xm, x[i]);
        sm = fmaxf(sm, sv[i]);
    }
    xm = group_max(xm);
    sm = group_max(sm);
    float mw = xm + __builtin_amdgcn_logf(sm);
    mw = fminf(fmaxf(mw, xm - 64.0f), xm + 64.0f);
    // Rescale only when the reference would grow by more than 2^8; in between P stays below
    // 2^8 (fine for f16) and no accumulator is touched.
    if (__any(live && mw > st.m + 8.0f)) {
        asm volatile("" ::: "memory");  // keep this a branch: the multiply is the rare case
        const float m_new = fmaxf(st.m, mw);
        const float alpha = fast_exp2(st.m - m_new);
        st.l *= alpha;
#pragma unroll
        for (int td = 0; td < NTD; td++) st.o[td] *= alpha;
        st.m = m_new;
    }
    float psum = 0.0f, pv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float p = fast_exp2(x[i] - st.m);
        psum += p;
        pv[i] = p * sv[i];
    }
    st.l += psum;
    // ---- O^T += V^T P^T ---------------------------------------------------------------------
    // P = hi + lo in f16 (~22 bits, like q): the hi columns feed f16(P), the lo columns
    // P - f16(P); a single f16 P would carry a relative error of 2^-11 straight into the output
    // whenever one position dominates the softmax.  Columns past 2G hold finite garbage that
    // only feeds output columns never read.
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float hi = split_hi(pv[i]);
        pv[i] = lo_col ? pv[i] - hi : hi;
    }
#pragma unroll
    for (int b = 0; b < 2; b++) {
        half8 pb;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            // slots (2r, 2r+1) = positions 4g+r of tiles 2b and 2b+1
            const half2_t pr = {(_Float16)pv[4 * (2 * b) + r], (_Float16)pv[4 * (2 * b + 1) + r]};
            pb[2 * r] = pr[0];
            pb[2 * r + 1] = pr[1];
        }
#pragma unroll
        for (int td = 0; td < NTD; td++) {
            const half8 va = dequant8(w.vw[b][td], dc);
            st.o[td] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, st.o[td], 0, 0, 0);
        }
    }
}

// Fused append, run by one wave of the workgroup whose split holds position p = len[s]: the
// quantize-on-append of ts_append.hip for one (sequence, kv head) and one position, with the
// same arithmetic (ts_quant.h), so codes and scales are bit-identical.  Lane i owns the
// rotation pairs i + 64 j (j < PPL: one pair per lane up to head dim 128, two at 256), i.e.
// dims 2(i + 64j) and +1.  Writes the K row, both scales and the position's nibble of every V
// word (read-modify-write: only this workgroup touches the block), and leaves the dequantized
// row ((code - 8) * scale, the values the cache now holds) in kd / vd.
//
// Two phases, so a caller can issue every load of the append together (one memory round trip)
// before anything else: append_load, then append_store.
template <int HD>
struct AppendIn {
    static constexpr int PPL = HD > 128 ? 2 : 1;
    float k[PPL][2], v[PPL][2];  // raw new K / V of the lane's pairs
    float2 cs[PPL];              // rotation of each pair at the position's rotation position
    float kn[PPL][2];            // K norm weights of the pairs' dims (QK norm)
    uint32_t vold[PPL][2];       // the V words holding the pairs' dims at this position
};

template <int HD, bool NORM>
__device__ __forceinline__ void append_load(const DecodeArgs &a, int s, int h, int p, int lane, AppendIn<HD> &in,
                                            int hdr) {
    constexpr int PPL = AppendIn<HD>::PPL;
    const KvLayerView &L = a.L;
    const size_t row = (size_t)s * L.H + h;
    const int pr = rot_of(L, s, p);
    const int q = p & 31, gq = (q & 15) >> 2;
    const uint32_t *vb = reinterpret_cast<const uint32_t *>(L.vp + (row * (L.P / 32) + (p >> 5)) * (HD * 16));
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int i = lane + 64 * j;
        const bool on = i < HD / 2;
        // rows of hdr floats; the stored dims past them are 0 (their lanes load the row's
        // first pair, unconditionally, and drop it)
        const bool dim_in = on && 2 * i < hdr;
        const size_t src = row * hdr + 2 * (dim_in ? i : 0);
        const float2 kk = *reinterpret_cast<const float2 *>(a.k_new + src);
        const float2 vv = *reinterpret_cast<const float2 *>(a.v_new + src);
        in.k[j][0] = dim_in ? kk.x : 0.f; in.k[j][1] = dim_in ? kk.y : 0.f;
        in.v[j][0] = dim_in ? vv.x : 0.f; in.v[j][1] = dim_in ? vv.y : 0.f;
        const int ir = i < a.rope_pairs ? i : 0;
        in.cs[j] = *reinterpret_cast<const float2 *>(a.rope + ((size_t)pr * a.rope_pairs + ir) * 2);
        in.kn[j][0] = NORM && L.kn && dim_in ? L.kn[2 * i] : 1.0f;
        in.kn[j][1] = NORM && L.kn && dim_in ? L.kn[2 * i + 1] : 1.0f;
        const int ic = on ? i : 0;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int d = 2 * ic + e;
            in.vold[j][e] = vb[v_word_idx(gq * 16 + (d & 15), d >> 4)];
        }
    }
}

// write = false: only the dequantized rows (a head group other than the first, whose
// workgroup quantizes the same row for its own heads' scores).
template <int HD, bool NORM>
__device__ void append_store(const DecodeArgs &a, int s, int h, int p, int lane, const AppendIn<HD> &in,
                             float *kd, float *vd, int hdr, bool write = true) {
    constexpr int ROWB = HD / 2, PPL = AppendIn<HD>::PPL;
    const KvLayerView &L = a.L;
    const bool KN = NORM && L.kn != nullptr;  // QK norm of K
    const size_t row = (size_t)s * L.H + h;
    float k[PPL][2], v[PPL][2];
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        k[j][0] = in.k[j][0]; k[j][1] = in.k[j][1];
        v[j][0] = in.v[j][0]; v[j][1] = in.v[j][1];
    }
    // QK norm scale of the new K row: its squares summed in dimension order across the lanes
    // (pairs 0..63, then 64..127)
    float ns = 0.0f;
    if (KN) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < PPL; j++)
            sum = ordered_sum_pairs(sq_rn(k[j][0]), sq_rn(k[j][1]), HD / 2 < 64 ? HD / 2 : 64, sum);
        ns = qk_norm_scale_from_sum(sum, hdr, L.norm_eps);
    }
    float km = 0.0f, vm = 0.0f;
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int i = lane + 64 * j;
        if (i < HD / 2) {
            if (KN) {
                k[j][0] = qk_norm_apply(k[j][0], ns, in.kn[j][0]);
                k[j][1] = qk_norm_apply(k[j][1], ns, in.kn[j][1]);
            }
            if (i < a.rope_pairs) rope_rotate(k[j][0], k[j][1], in.cs[j]);
        }
        km = fmaxf(km, fmaxf(fabsf(k[j][0]), fabsf(k[j][1])));
        vm = fmaxf(vm, fmaxf(fabsf(v[j][0]), fabsf(v[j][1])));
    }
    const float ks = quant_scale(wave_max(km));
    const float vs = quant_scale(wave_max(vm));
    if (write && lane == 0) {
        L.ks[row * L.P + p] = ks;
        L.vs[row * L.P + p] = vs;
    }
    // V block p/32: dim d of key group gq sits in word v_word_idx(gq*16 + d%16, d/16), position
    // 4gq + r of tile t at nibble r + 4t.
    const int q = p & 31, t = q >> 4, gq = (q & 15) >> 2, nib = (q & 3) + 4 * t;
    uint32_t *vb = reinterpret_cast<uint32_t *>(L.vp + (row * (L.P / 32) + (p >> 5)) * (HD * 16));
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int i = lane + 64 * j;
        const bool on = i < HD / 2;
        const uint32_t c0 = encode(k[j][0], ks), c1 = encode(k[j][1], ks);
        const uint32_t e0 = encode(v[j][0], vs), e1 = encode(v[j][1], vs);
        // K row: word u holds dims 8u..8u+7 at bits 4*(d - 8u); pairs 4u..4u+3 share word u.
        uint32_t kw = on ? (c0 | (c1 << 4)) << (8 * (i & 3)) : 0u;
        kw |= __shfl_xor(kw, 1, 64);
        kw |= __shfl_xor(kw, 2, 64);
        if (write && on && (i & 3) == 0)
            reinterpret_cast<uint32_t *>(L.kp + row * L.P * ROWB)[k_word_idx<HD>(p, i >> 2)] = kw;
        if (on) {
            if (write) {
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int d = 2 * i + e;
                    vb[v_word_idx(gq * 16 + (d & 15), d >> 4)] =
                        (in.vold[j][e] & ~(0xFu << (4 * nib))) | ((e ? e1 : e0) << (4 * nib));
                }
            }
            kd[2 * i] = (float)((int)c0 - 8) * ks;
            kd[2 * i + 1] = (float)((int)c1 - 8) * ks;
            vd[2 * i] = (float)((int)e0 - 8) * vs;
            vd[2 * i + 1] = (float)((int)e1 - 8) * vs;
        }
    }
}

// Scores of the new position (dequantized row kd, in this wave's LDS) for the G query heads
// hb .. hb + G - 1 of sequence s, in the exp2 domain, from the rotated f32 q (as load_q8
// rotates it); one wave.  qp[hh][j]: dims 2(i + 64j), +1 of head hh's raw q, cs[j]: the
// rotation of that pair at the query's rotation position.
template <int HD, bool SOFTCAP, bool NORM, int GMAX>
__device__ void new_token_scores(const DecodeArgs &a, int s, int hb, int G, int lane,
                                 const float2 (&qp)[GMAX][AppendIn<HD>::PPL], const float2 (&cs)[AppendIn<HD>::PPL],
                                 const float *kd, float *xnew, int hdr) {
    constexpr int PPL = AppendIn<HD>::PPL;
    const float *const QN = NORM ? a.L.qn : nullptr;
    const float *qg = a.q + ((size_t)s * a.n_head + hb) * hdr;
    float nhs[GMAX];
    if (QN) q_norm_scales_wave<HD, GMAX>(qg, G, a.L.norm_eps, hdr, nhs);
    // (a guard, not a break: the loop unrolls fully, so qp stays in registers)
#pragma unroll
    for (int hh = 0; hh < GMAX; hh++) {
        if (hh >= G) continue;
        const float nh = QN ? nhs[hh] : 1.0f;
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < PPL; j++) {
            const int i = lane + 64 * j;
            float q0 = qp[hh][j].x, q1 = qp[hh][j].y;
            if (QN && 2 * i < hdr) {
                q0 = qk_norm_apply(q0, nh, QN[2 * i]);
                q1 = qk_norm_apply(q1, nh, QN[2 * i + 1]);
            }
            if (i < a.rope_pairs) rope_rotate(q0, q1, cs[j]);
            dot += i < HD / 2 ? q0 * kd[2 * i] + q1 * kd[2 * i + 1] : 0.0f;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o, 64);
        float x = dot * a.inv_sqrt_hd;
        if constexpr (SOFTCAP) x = tanhf(x / a.softcap) * a.softcap;
        if (lane == 0) xnew[hh] = x * kLog2e;
    }
}

// The raw q pairs new_token_scores takes: dims 2(i + 64j), +1 of query heads hb .. hb + G - 1.
template <int HD, int GMAX>
__device__ __forceinline__ void load_q_pairs(const DecodeArgs &a, int s, int hb, int G, int lane,
                                             float2 (&qp)[GMAX][AppendIn<HD>::PPL], int hdr) {
    const float *qg = a.q + ((size_t)s * a.n_head + hb) * hdr;
#pragma unroll
    for (int hh = 0; hh < GMAX; hh++)
#pragma unroll
        for (int j = 0; j < AppendIn<HD>::PPL; j++) {
            const int i = lane + 64 * j;
            const bool use = hh < G && i < HD / 2 && 2 * i < hdr;
            const float2 t = *reinterpret_cast<const float2 *>(qg + (size_t)(hh < G ? hh : 0) * hdr + 2 * (use ? i : 0));
            qp[hh][j] = make_float2(use ? t.x : 0.f, use ? t.y : 0.f);
        }
}

// Split partial of one head: unnormalized o (dim d), and with d == 0 the reference exponent m
// and the sum l, for decode_combine_kernel.
__device__ inline void store_partial(const DecodeArgs &a, size_t head, int split, int HD, int d, float acc,
                                     float M, float lsum) {
    const size_t rows = (size_t)a.L.S * a.n_head * a.n_split, r = head * a.n_split + split;
    a.ws[r * HD + d] = acc;
    if (d == 0) {
        a.ws[rows * HD + r] = M;
        a.ws[rows * (HD + 1) + r] = lsum;
    }
}

// PAD: the caller's head dim hdr is below the stored HD (rows of q, new K/V and the output are
// hdr floats; the stored dims past them hold zeros).
// NW waves per workgroup: 4 (two workgroups per CU up to 128 dims), or 8 / 16 for a plan that
// gives every (sequence, kv head) stream one workgroup (a CU) of its own and no split: the
// small-batch case, where the combine launch would be most of the step.
template <int HD, bool SOFTCAP, bool NORM, bool PAD, int NW>
__global__ __launch_bounds__(64 * NW, NW > 4 ? 1 : (HD > 128 ? 1 : 2)) void decode_split_kernel(DecodeArgs a) {
    constexpr int SPAN = 64 * NW;     // positions one round of windows covers
    constexpr int WPG = HD / 32;   // K words per lane group = MFMA k-steps per 16-row tile
    constexpr int NTD = HD / 16;   // 16-dim output tiles
    constexpr int ROWB = HD / 2;   // bytes per K row
    constexpr int OST = HD + 4;  // 16-byte rows of the merge area
    const KvLayerView &L = a.L;
    const int hdr = PAD ? L.hdr : HD;
    const float *const QN = NORM ? L.qn : nullptr;  // QK norm of q (compiled out when off)
    const int split = blockIdx.x, s = blockIdx.z;
    // kv head h, and head group gi of its a.Gt query heads (groups of 8)
    const int h = blockIdx.y / a.NG, gi = blockIdx.y - h * a.NG;
    const int start = split * a.chunk;
    const int tid = threadIdx.x, lane = tid & 63;
    // wave index in an SGPR: window bases are then provably wave-uniform and feed the scalar
    // offset of the buffer loads directly
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int G = min(a.G, a.Gt - 8 * gi);  // query heads of this workgroup
    const int hb = h * a.Gt + 8 * gi;       // the first of them within the sequence
    const size_t row = (size_t)s * L.H + h;
    const uint8_t *kbase = L.kp + row * L.P * ROWB;
    const uint8_t *vbase = L.vp + row * (L.P / 32) * (HD * 16);
    const float *ksb = L.ks + row * L.P;
    const float *vsb = L.vs + row * L.P;

    // The first window and the raw q go out before the sequence's length is known (a memory
    // round trip of its own): the first window is bounded by the stream's capacity, and the
    // positions of it past the split's end are masked like any tail.
    Streams str;
    str.k = make_rsrc(kbase, (uint32_t)L.P * ROWB);
    str.v = make_rsrc(vbase, (uint32_t)(L.P / 32) * (HD * 16));
    str.ksb = ksb;
    str.vsb = vsb;
    str.last = L.P - 1;
    Window<HD> w0, w1;
    int base = start + wave * 64;
    load_window<HD>(w0, str, base, n, g, lane);
    // accumulator column n: high parts of head h*G + n (n < G), low parts of head
    // h*G + n - G (G <= n < 2G), unused beyond
    const bool live = n < 2 * G, lo_col = n >= G;
    const int qhead = n < G ? n : (live ? n - G : 0);
    const float *qrow = a.q + ((size_t)s * a.n_head + hb + qhead) * hdr;
    float qraw[WPG][8];
#pragma unroll
    for (int t = 0; t < WPG; t++) q_read8(qrow, k16_word<HD>(g, t), nullptr, 1.0f, qraw[t], hdr);
    asm volatile("" ::: "memory");

    const int qpos = a.hlen >= 0 ? a.hlen : a.len[s];
    // a captured launch replayed past the cache's capacity (the host checks lengths only when a
    // call is made): no work, nothing written (the lengths still advance, as the combine
    // kernel's do)
    if (qpos >= L.P) {
        if (a.n_split == 1) arrive_and_advance(a);
        return;
    }
    const int qrot = rot_of(a.L, s, qpos);  // rotation position of the query
    const int n_ctx = qpos + 1;
    if (start >= n_ctx) return;  // (only with a split: its combine kernel advances the lengths)
    const int n_split_s = min((n_ctx + a.chunk - 1) / a.chunk, a.n_split);
    // With the fused append, this split's workgroup writes position qpos itself and adds its
    // score from registers; the window loop then stops short of it.
    const bool fused = a.k_new != nullptr && split == n_split_s - 1;
    // the last split runs to the end, also past chunk * n_split (a launch captured for shorter
    // contexts stays correct, only less balanced)
    const int end = fused ? qpos : (split == n_split_s - 1 ? n_ctx : start + a.chunk);
    const int partner4 = 4 * (n < G ? lane + G : (live ? lane - G : lane));
    const DeqConst dc;

    // LDS: q operands, per-wave scale stages; and the merge area, apart from them so that a
    // wave writes its share of the merge as soon as its windows are done.
    struct Smem {
        struct {
            QLds<HD> q;
            float stage[NW][128];
        } run;
        struct {
            __align__(16) float o[NW][16 * OST];
            float m[NW][8], l[NW][8];
        } merge;
    };
    __shared__ __align__(16) Smem sm;
    // fused append: the new position's dequantized K and V rows and its score per head
    __shared__ __align__(16) float kd[HD], vd[HD];
    __shared__ float xnew[8];

    // Later windows: bounded to the split (K rows are cut into segments spread over their
    // 64-position window: bound at the window)
    str.k = make_rsrc(kbase, (uint32_t)((end + 63) & ~63) * ROWB);
    str.v = make_rsrc(vbase, (uint32_t)((end + 31) / 32) * (HD * 16));
    str.last = max(end - 1, 0);

    // q operands: wave w builds k-step t = w (rotated, scaled by log2(e)/sqrt(hd), split hi/lo)
    // for all 64 lanes; zero in the columns past G.
    // One power-of-two scale for the G heads: every wave reads the bound of all of them.
    // QK norm scale of this lane's query head (each wave computes it for itself)
    const float ns = QN ? q_norm_scale_wave<HD>(a.q + ((size_t)s * a.n_head + hb) * hdr, G, qhead, L.norm_eps, hdr)
                        : 1.0f;
    if (QN) {
#pragma unroll
        for (int t = 0; t < WPG; t++)
            if (8 * k16_word<HD>(g, t) < hdr) {
#pragma unroll
                for (int e = 0; e < 8; e++) qraw[t][e] = qk_norm_apply(qraw[t][e], ns, QN[8 * k16_word<HD>(g, t) + e]);
            }
    }
    float q_s, inv_s;
    {
        float qb = 0.0f;
#pragma unroll
        for (int t = 0; t < WPG; t++)
#pragma unroll
            for (int e = 0; e < 8; e += 2) qb = fmaxf(qb, fabsf(qraw[t][e]) + fabsf(qraw[t][e + 1]));
        q_scale(wave_max(qb) * (a.inv_sqrt_hd * kLog2e), q_s, inv_s);
    }
#pragma unroll
    for (int t = 0; t < WPG; t++) {
        if (t % NW != wave) continue;
        half8 qh, ql;
        float2 cs[4];
        load_rot8(a.rope, a.rope_pairs, k16_word<HD>(g, t), qrot, cs);
        split_q8(qraw[t], cs, k16_word<HD>(g, t), a.rope_pairs, a.inv_sqrt_hd * kLog2e * q_s, qh, ql);
        sm.run.q.p[t][lane] = !live ? (half8)(_Float16)0.0f : (lo_col ? ql : qh);
    }
    __syncthreads();  // q operands
    // The appending wave (the last: it has the fewest windows) quantizes the new token and
    // scores it against every head before its windows; the others start at once.  kd, vd and
    // xnew are read after the barrier that opens the merge.
    if (fused && wave == NW - 1) {
        AppendIn<HD> ain;
        float2 qp[8][AppendIn<HD>::PPL];
        append_load<HD, NORM>(a, s, h, qpos, lane, ain, hdr);
        load_q_pairs<HD, 8>(a, s, hb, G, lane, qp, hdr);
        append_store<HD, NORM>(a, s, h, qpos, lane, ain, kd, vd, hdr, gi == 0);
        new_token_scores<HD, SOFTCAP, NORM, 8>(a, s, hb, G, lane, qp, ain.cs, kd, xnew, hdr);
    }

    WaveState<HD> st;
#pragma unroll
    for (int td = 0; td < NTD; td++) st.o[td] = (floatx4)0.0f;
    st.m = kMinit;
    st.l = 0.0f;
    float *stage = sm.run.stage[wave];

    // Register double buffering: window i+1 is in flight while window i is computed.  One form
    // for every window, the tail mask included (a masked and an unmasked copy cost 70 VGPRs
    // in moves at their join).
#define TS_STEP(CUR, NXT)                                                                       \
    {                                                                                          \
        load_window<HD>(NXT, str, base + SPAN, n, g, lane);                                     \
        /* keep the prefetch here: the scheduler would otherwise sink it below CUR's use */     \
        asm volatile("" ::: "memory");                                                         \
        __builtin_amdgcn_sched_barrier(0);                                                     \
        process_window<HD, SOFTCAP>(CUR, st, sm.run.q, stage, base, end, lane, g, live, lo_col, partner4, inv_s, a.softcap, dc); \
        base += SPAN;                                                                           \
        if (base >= end) break;                                                                \
    }
    while (base < end) {
        TS_STEP(w0, w1)
        TS_STEP(w1, w0)
    }
#undef TS_STEP

    // ---- merge the waves through LDS -----------------------------------------------------------
    // Each wave writes its O^T columns (16-byte stores), m and l; one barrier; then one float4
    // of dims per thread.  (Merge area shared with the q operands, a barrier before the writes,
    // scalar stores and one dim per thread: 0.1-0.3 us more per layer on configs 1 and 2.)
    const float l_run = group_sum(st.l);
    if (live) {
        if (g == 0 && !lo_col) {
            sm.merge.m[wave][n] = st.m;
            sm.merge.l[wave][n] = l_run;
        }
#pragma unroll
        for (int td = 0; td < NTD; td++)
            *reinterpret_cast<floatx4 *>(&sm.merge.o[wave][n * OST + 16 * td + 4 * g]) = st.o[td];
    }
    __syncthreads();

    constexpr int V4 = HD / 4;
    for (int idx = tid; idx < G * V4; idx += SPAN) {
        const int hh = idx / V4, d = 4 * (idx % V4);
        float M = kMinit;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sm.merge.m[w][hh]);
        if (fused) M = fmaxf(M, xnew[hh]);
        floatx4 acc = (floatx4)0.0f;
        float lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float e = exp2f(sm.merge.m[w][hh] - M);
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(&sm.merge.o[w][hh * OST + d]);
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(&sm.merge.o[w][(hh + G) * OST + d]);
            acc += e * (hi + lo);
            lsum += e * sm.merge.l[w][hh];
        }
        if (fused) {
            // the new position as one more partial: m = its score, l = 1, o = its V row
            const float e = exp2f(xnew[hh] - M);
            acc += e * *reinterpret_cast<const floatx4 *>(&vd[d]);
            lsum += e;
        }
        const size_t head = (size_t)s * a.n_head + hb + hh;
        if (n_split_s == 1) {
            // hdr is a multiple of 8: a float4 of dims lies wholly inside or outside the row
            if (d < hdr) {
                const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
                const floatx4 r = lsum > 0.0f ? acc * inv : (floatx4)0.0f;
                *reinterpret_cast<float4 *>(a.out + head * hdr + d) = make_float4(r[0], r[1], r[2], r[3]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) store_partial(a, head, split, HD, d + k, acc[k], M, lsum);
        }
    }
    // without a split this is the launch's last kernel: it advances the lengths itself
    if (a.n_split == 1) arrive_and_advance(a);
}

// The merge of one (sequence, head) over its ns > 1 splits (body of decode_combine_kernel).
template <int HD>
__device__ __forceinline__ void combine_rows(const DecodeArgs &a, int head, int s, int ns, int tid) {
    constexpr int V4 = HD / 4, NG = 256 / V4;
    __shared__ float4 part[NG][V4];
    __shared__ float lpart[NG];
    __shared__ float wmax[4];
    const size_t hidx = (size_t)s * a.n_head + head;
    const float *ml = a.ws + (size_t)a.L.S * a.n_head * a.n_split * HD;
    const float *mm = ml + hidx * a.n_split;
    const float *ll = ml + (size_t)a.L.S * a.n_head * a.n_split + hidx * a.n_split;

    const int g = tid / V4, j = tid % V4;
    const float4 *o4 = reinterpret_cast<const float4 *>(a.ws + hidx * a.n_split * HD);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float lsum = 0.0f;
    if (ns <= 4 * NG) {
        // Up to 4 splits per row group: every load is issued at once (each thread reads all ns
        // maxima itself besides its own rows), so the merge is one memory round trip, with no
        // reduction round for the maximum.  (Batch 1 has more than NG splits per head.)
        constexpr int R = 4;
        float mv[R * NG];
#pragma unroll
        for (int i = 0; i < R * NG; i++) mv[i] = i < ns ? mm[i] : kMinit;
        float4 x[R];
        float lg[R], mg[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = g + r * NG;
            const bool mine = i < ns;
            x[r] = mine ? o4[(size_t)i * V4 + j] : make_float4(0.f, 0.f, 0.f, 0.f);
            lg[r] = mine ? ll[i] : 0.0f;
            mg[r] = mine ? mm[i] : kMinit;
        }
        float M = kMinit;
#pragma unroll
        for (int i = 0; i < R * NG; i++) M = fmaxf(M, mv[i]);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float e = g + r * NG < ns ? exp2f(mg[r] - M) : 0.0f;
            acc.x += e * x[r].x;
            acc.y += e * x[r].y;
            acc.z += e * x[r].z;
            acc.w += e * x[r].w;
            lsum += e * lg[r];
        }
    } else {
        float M = kMinit;
        for (int i = tid; i < ns; i += 256) M = fmaxf(M, mm[i]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        if ((tid & 63) == 0) wmax[tid >> 6] = M;
        __syncthreads();
        M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
#pragma unroll 4
        for (int i = g; i < ns; i += NG) {
            const float e = exp2f(mm[i] - M);
            const float4 x = o4[(size_t)i * V4 + j];
            acc.x += e * x.x;
            acc.y += e * x.y;
            acc.z += e * x.z;
            acc.w += e * x.w;
            lsum += e * ll[i];
        }
    }
    part[g][j] = acc;
    if (j == 0) lpart[g] = lsum;
    __syncthreads();
    if (tid < V4 && 4 * tid < a.L.hdr) {
        float4 r = part[0][tid];
        float l = lpart[0];
#pragma unroll
        for (int k = 1; k < NG; k++) {
            const float4 x = part[k][tid];
            r.x += x.x;
            r.y += x.y;
            r.z += x.z;
            r.w += x.w;
            l += lpart[k];
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *o = a.out + hidx * a.L.hdr + 4 * tid;  // d_out rows of hdr floats
        o[0] = r.x * inv;
        o[1] = r.y * inv;
        o[2] = r.z * inv;
        o[3] = r.w * inv;
    }
}

// Log-sum-exp merge of the splits of one (sequence, head).  256 threads: HD/4 threads (one
// float4 of dims each) per split row, 1024/HD row groups striding over the splits, then an
// LDS reduction over the groups, so the dependent-load chain is ns/groups long, not ns.
template <int HD>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
    const int head = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    const int n_ctx = (a.hlen >= 0 ? a.hlen : a.len[s]) + 1;
    const int ns = min((n_ctx + a.chunk - 1) / a.chunk, a.n_split);
    if (ns > 1) combine_rows<HD>(a, head, s, ns, tid);
    arrive_and_advance(a);
}



// ---- G <= 16: QK^T on v_mfma_i32_16x16x64_i8 --------------------------------------------------
//
// QK^T runs in exact integer arithmetic, for up to 16 query heads per kv head in one, two or
// four halves of 4 heads (the description below is of one half; every other half has its own q
// operand and accumulators against the same K operand).  The B operand is K^T: column n of tile t is position
// 4n + t of the window, and lane 16 g + n supplies 16 dims of it as unsigned bytes -- the
// nibbles of two K words, even dims from (w & 0x0F0F0F0F), odd dims from (w >> 4) & 0x0F0F0F0F,
// 3 VALU ops per word.  The A operand holds q: row 4 h + c is base-128 digit c (c = 0 most
// significant) of head h's q, rotated and scaled to an integer of at most 2^27, so the 16 rows
// carry all 4 digits of all 4 heads.  The accumulators start at -8 * (sum of the row's digits),
// which takes the nibble bias out exactly, and the products are summed exactly in i32.  Output
// lane 16 h + n then holds the 4 digit sums of head h at position 4n + t; one f32 Horner step
// per digit gives the score (one rounding).  Each lane runs the softmax of its head at its 4
// positions; p * s_v goes through a per-wave LDS tile into the PV operand layout of the
// 16x16x32 f16 instruction (as above).

template <int HD>
struct Window8 {
    static constexpr int NKW = HD / 8, NTD = HD / 16;
    uint32_t kw[NKW];     // lane order q of k_word_idx: tile t, half m, word i at 2 (t HD/64 + m) + i
    uint32_t vw[2][NTD];  // V words, as Window
    floatx4 sk, sv;       // scales of positions base + 4n .. base + 4n + 3 (n = lane % 16)
};

// Buffer resources of one split for the integer kernel: K, V and both scale arrays (loads past
// the bound return zeros and touch no memory).
struct Streams4 {
    __amdgpu_buffer_rsrc_t k, v, sk, sv;
};

// Cache policy of the window loads: non-temporal.  Every byte is read exactly once per launch,
// and each instruction covers whole cache lines.
constexpr int kNT = 2;

// One window (64 positions from `base`, a multiple of 64): each K and V instruction reads one
// contiguous kilobyte (the cache's chunk order puts exactly this lane's operand words there);
// the scale instructions read the window's 256 bytes, every 16 bytes by the 4 lanes of a
// column.
template <int HD, int POL = kNT>
__device__ __forceinline__ void load_window8(Window8<HD> &w, const Streams4 &st, int base, int lane) {
    constexpr int NKW = HD / 8, NTD = HD / 16, ROWB = HD / 2;
#pragma unroll
    for (int j = 0; j < NKW / 4; j++) {
        const u32x4 t4 = __builtin_amdgcn_raw_buffer_load_b128(st.k, lane * 16 + j * 1024, base * ROWB, POL);
        w.kw[4 * j + 0] = t4[0]; w.kw[4 * j + 1] = t4[1]; w.kw[4 * j + 2] = t4[2]; w.kw[4 * j + 3] = t4[3];
    }
#pragma unroll
    for (int b = 0; b < 2; b++) {
#pragma unroll
        for (int q4 = 0; q4 < NTD / 4; q4++) {
            const u32x4 t4 = __builtin_amdgcn_raw_buffer_load_b128(st.v, lane * 16 + q4 * 1024 + b * (HD * 16), (base / 32) * (HD * 16), POL);
            w.vw[b][4 * q4 + 0] = t4[0]; w.vw[b][4 * q4 + 1] = t4[1];
            w.vw[b][4 * q4 + 2] = t4[2]; w.vw[b][4 * q4 + 3] = t4[3];
        }
    }
    const int so = (lane & 15) * 16;
    w.sk = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(st.sk, so, base * 4, POL));
    w.sv = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(st.sv, so, base * 4, POL));
}

template <int CTRL>
__device__ inline float dpp_any(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Max / sum over the 16 lanes of a DPP row (every lane gets the result).
__device__ inline float row_max16(float v) {
    v = fmaxf(v, dpp_any<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_any<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_any<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_any<0x140>(v));  // row_mirror
    return v;
}
__device__ inline float row_sum16(float v) {
    v += dpp_any<0xB1>(v);
    v += dpp_any<0x4E>(v);
    v += dpp_any<0x141>(v);
    v += dpp_any<0x140>(v);
    return v;
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Running state of one wave.  GH = 1 (G <= 4): O^T column n < 4 is head n from the high parts
// of p*s_v, 4 <= n < 8 head n - 4 from the low parts; GH = 2 (G <= 8): column n < 8 is head n
// from the high parts, 8 <= n < 16 head n - 8 from the low parts; GH = 4 (G <= 16): two sets
// of 16 columns, column n of set 0 head n from the high parts, of set 1 from the low parts.
// Lane 16 hg + n runs the softmax of heads hg + 4 hf (half hf): the exponent reference of each
// (uniform over the lane's row) and this lane's share of its softmax sum.
template <int GH>
constexpr int kPvSets = GH == 4 ? 2 : 1;
template <int HD, int GH>
struct WaveState8 {
    floatx4 o[kPvSets<GH>][HD / 16];
    float m[GH], l[GH];
};

// LDS slot of position `key` (0..63) of a window in the PV operand order: lane (n, g) of the
// 16x16x32 B operand reads slots 32b + 8g .. +7 = positions 32b + 16t + 4g + r at 2r + t.
__device__ inline int p_slot(int key) {
    return 32 * (key >> 5) + 8 * ((key >> 2) & 3) + 2 * (key & 3) + ((key >> 4) & 1);
}

// One window.  Half hf of the heads (4 hf .. 4 hf + 3) has its own q operand qa[hf] and bias:
// one i8 instruction per half and k-group, both on the same unpacked K operand.  pt: the wave's
// P tile, 8 GH columns.
template <int HD, bool SOFTCAP, int GH>
__device__ __forceinline__ void process_window8(const Window8<HD> &w, WaveState8<HD, GH> &st,
                                                const i32x4 (&qa)[GH][HD / 64], const i32x4 (&bias)[GH],
                                                const float (&qinv)[GH], _Float16 (*pt)[64], int base, int end,
                                                int lane, const bool (&live)[GH], float softcap, const DeqConst &dc) {
    constexpr int NTD = HD / 16, NM = HD / 64;
    const int n = lane & 15, hg = lane >> 4;
    // ---- S = Q K^T, exact -----------------------------------------------------------------
    i32x4 acc[GH][4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
        for (int hf = 0; hf < GH; hf++) acc[hf][t] = bias[hf];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const uint32_t w0 = w.kw[2 * (t * NM + m)], w1 = w.kw[2 * (t * NM + m) + 1];
            const i32x4 kb = {(int)(w0 & 0x0F0F0F0Fu), (int)((w0 >> 4) & 0x0F0F0F0Fu),
                              (int)(w1 & 0x0F0F0F0Fu), (int)((w1 >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
            for (int hf = 0; hf < GH; hf++)
                acc[hf][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[hf][m], kb, acc[hf][t], 0, 0, 0);
        }
    }
    // ---- softmax of heads hg (+ 4 hf) at positions base + 4n + t --------------------------
    float x[GH][4], sv[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        sv[t] = base + 4 * n + t >= end ? 0.0f : w.sv[t];  // positions past the split's end
#pragma unroll
        for (int hf = 0; hf < GH; hf++) {
            // digits 0..3 carry weights 2^21, 2^14, 2^7, 1; each digit sum is an exact integer
            // below 2^18, so the two pairs combine exactly in i32 (below 2^26) and the score
            // takes two conversions and one FMA.
            const int dhi = acc[hf][t][0] * 128 + acc[hf][t][1], dlo = acc[hf][t][2] * 128 + acc[hf][t][3];
            float v = fmaf((float)dhi, 16384.0f, (float)dlo);
            v *= qinv[hf] * w.sk[t];
            if constexpr (SOFTCAP) v = tanhf(v * (1.0f / kLog2e) / softcap) * softcap * kLog2e;
            x[hf][t] = base + 4 * n + t >= end ? -INFINITY : v;
        }
    }
    // P = 2^(x - m) * s_v must stay <= 2^8 (f16 range for its two parts, with room).  The
    // reference m of a head moves only when some position of the window breaks that: a ballot
    // in the common case, row reductions only then (to m = max(x) + log2(max s_v), P <= 1).
    float p[GH][4], pv[GH][4];
    bool need = false;
#pragma unroll
    for (int hf = 0; hf < GH; hf++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            p[hf][t] = live[hf] ? fast_exp2(x[hf][t] - st.m[hf]) : 0.0f;
            pv[hf][t] = p[hf][t] * sv[t];
            need |= !(pv[hf][t] <= 256.0f);
        }
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
        asm volatile("" ::: "memory");  // keep this a branch: the rescale is the rare case
        const float svl = __builtin_amdgcn_logf(row_max16(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]))));
        float al[GH];
#pragma unroll
        for (int hf = 0; hf < GH; hf++) {
            const float xm = row_max16(fmaxf(fmaxf(x[hf][0], x[hf][1]), fmaxf(x[hf][2], x[hf][3])));
            const float mw = fminf(fmaxf(xm + svl, xm - 64.0f), xm + 64.0f);
            const float m_new = fmaxf(st.m[hf], mw);
            al[hf] = fast_exp2(st.m[hf] - m_new);
            st.l[hf] *= al[hf];
            st.m[hf] = m_new;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                p[hf][t] = live[hf] ? fast_exp2(x[hf][t] - st.m[hf]) : 0.0f;
                pv[hf][t] = p[hf][t] * sv[t];
            }
        }
        // the O^T columns of head c take the factor of its row: head c of half hf is row c % 4
        // of al[hf] (lane 16 (c % 4))
        const int c = GH == 1 ? (lane & 3) : GH == 2 ? (lane & 7) : (lane & 15);
        float f = 1.0f;
#pragma unroll
        for (int hf = 0; hf < GH; hf++) {
            const float f0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al[hf]), 0));
            const float f1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al[hf]), 16));
            const float f2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al[hf]), 32));
            const float f3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al[hf]), 48));
            const int cc = c & 3;
            if ((c >> 2) == hf) f = cc == 0 ? f0 : cc == 1 ? f1 : cc == 2 ? f2 : f3;
        }
#pragma unroll
        for (int ps = 0; ps < kPvSets<GH>; ps++)
#pragma unroll
            for (int td = 0; td < NTD; td++) st.o[ps][td] *= f;
    }
#pragma unroll
    for (int hf = 0; hf < GH; hf++) st.l[hf] += (p[hf][0] + p[hf][1]) + (p[hf][2] + p[hf][3]);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int slot = p_slot(4 * n + t);
#pragma unroll
        for (int hf = 0; hf < GH; hf++) {
            const float hi = split_hi(pv[hf][t]);
            pt[4 * hf + hg][slot] = (_Float16)hi;
            pt[4 * GH + 4 * hf + hg][slot] = (_Float16)(pv[hf][t] - hi);
        }
    }
    // ---- O^T += V^T P^T (the wave's own LDS writes are ordered before its reads) -------------
    const int g = lane >> 4;
#pragma unroll
    for (int b = 0; b < 2; b++) {
        // GH = 1: columns 8..15 read real p values; their outputs are never used
        half8 pb[kPvSets<GH>];
#pragma unroll
        for (int ps = 0; ps < kPvSets<GH>; ps++)
            pb[ps] = *reinterpret_cast<const half8 *>(&pt[GH == 1 ? (n & 7) : 16 * ps + n][32 * b + 8 * g]);
        // every word of the block dequantized into its own registers first, so the conversions
        // of later words overlap the matrix instructions of earlier ones
        half8 va[NTD];
#pragma unroll
        for (int td = 0; td < NTD; td++) va[td] = dequant8(w.vw[b][td], dc);
#pragma unroll
        for (int ps = 0; ps < kPvSets<GH>; ps++)
#pragma unroll
            for (int td = 0; td < NTD; td++)
                st.o[ps][td] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[td], pb[ps], st.o[ps][td], 0, 0, 0);
    }
}

// NW waves per workgroup, D windows in registers per wave (D - 1 in flight while one is
// computed).  The plan places one workgroup per CU (NW = 4: one wave per SIMD; NW = 8 for
// 64-dim rows: two).
// PAD: the caller's head dim hdr is below the stored HD (rows of q, new K/V and the output are
// hdr floats; the stored dims past them hold code 8 = 0, so the integer QK^T and PV run
// unchanged over the whole stored row).
// GH: halves of 4 query heads per wave (1: G <= 4, 2: G <= 8, 4: G <= 16).  HG: head groups of
// the workgroup: with HG = 2, waves 0 .. NW/2 - 1 take query heads 0..7 and the others heads
// 8..15, both groups over the same windows in the same order (the second read of a window
// comes from L2, so cached loads), each with NW/2 waves.
template <int HD, bool SOFTCAP, bool NORM, bool PAD, int NW, int D, int GH, int HG = 1>
__global__ __launch_bounds__(64 * NW, NW / 4) void decode_split4_kernel(DecodeArgs a) {
    constexpr int NTD = HD / 16;
    constexpr int NM = HD / 64;  // i8 instructions per 16-position tile
    constexpr int OST = HD + 4;  // 16-byte rows of the merge area
    const KvLayerView &L = a.L;
    const int hdr = PAD ? L.hdr : HD;
    const float *const QN = NORM ? L.qn : nullptr;  // QK norm of q (compiled out when off)
    // grid (kv head, sequence, split): every sequence's split 0 is dispatched before any
    // split 1, so the splits that wait for a free CU are the last ones of the longest
    // sequences (config 4: 1.42 vs 1.45 ms per step against the split-fastest order)
    const int split = blockIdx.z, h = blockIdx.x, s = blockIdx.y;
    const int qpos = a.hlen >= 0 ? a.hlen : a.len[s];
    // a captured launch replayed past the cache's capacity (the host checks lengths only when a
    // call is made): no work, nothing written
    if (qpos >= L.P) return;
    const int qrot = rot_of(a.L, s, qpos);  // rotation position of the query
    const int n_ctx = qpos + 1;
    const int start = split * a.chunk;
    if (start >= n_ctx) return;
    const int n_split_s = min((n_ctx + a.chunk - 1) / a.chunk, a.n_split);
    const bool fused = a.k_new != nullptr && split == n_split_s - 1;
    // the last split runs to the end, also past chunk * n_split (a launch captured for shorter
    // contexts stays correct, only less balanced)
    const int end = fused ? qpos : (split == n_split_s - 1 ? n_ctx : start + a.chunk);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.G;
    const DeqConst dc;

    // per-wave p*s_v tiles, [column][slot]; and the merge area, apart from them so that a wave
    // writes its share of the merge as soon as its windows are done
    __shared__ _Float16 pts[NW][8 * GH][64];
    __shared__ __align__(16) float mo[NW][8 * GH * OST];  // O^T columns, OST floats apart
    __shared__ float mm_[NW][4 * GH], ml_[NW][4 * GH];
    __shared__ __align__(16) float kd[HD], vd[HD];
    __shared__ float xnew[4 * GH * HG < 8 ? 8 : 4 * GH * HG];
    __shared__ int32_t qsum[NW][GH][16];  // per wave and half: digit sums of the 16 q rows
    __shared__ float qinv_s[NW][GH][4];   // per wave and half: 2^-e of each head's q scale

    const size_t row = (size_t)s * L.H + h;
    constexpr int ROWB = HD / 2;
    Streams4 str;
    // K and the scales are bounded at the window: a window's K chunks mix its rows, and a
    // scale load covers 4 positions
    const uint32_t wend = (uint32_t)((end + 63) & ~63);
    str.k = make_rsrc(L.kp + row * L.P * ROWB, wend * ROWB);
    str.v = make_rsrc(L.vp + row * (L.P / 32) * (HD * 16), (uint32_t)((end + 31) / 32) * (HD * 16));
    str.sk = make_rsrc(L.ks + row * L.P, wend * 4);
    str.sv = make_rsrc(L.vs + row * L.P, wend * 4);

    // This wave's windows: claims j = wave, wave + NW, ... below nwin, taken in rotated order
    // starting at a per-workgroup offset, so that the workgroups streaming at the same time
    // read different regions of their streams (spread over the HBM channels).  Claim j reads
    // window (j + R) mod nwin.  The appending wave starts ~3 us late, so it keeps all but its
    // last kApp claims, which go round robin to the other waves after their own: the
    // assignment stays fixed (outputs are bit-reproducible) and the waves end together.
    // (Without the hand-over the appending wave ended ~2 us after the others: config 3
    // 1.880 vs 1.855 ms per step, measured with claims through an LDS counter.)  Window
    // indices past the wave's count load from past the bound (zeros, no memory traffic).
    // (per head group: NWG waves, wave wl of group hgp; only the appending wave's group hands
    // windows over)
    constexpr int NWG = NW / HG;
    const int hgp = __builtin_amdgcn_readfirstlane(wave / NWG), wl = wave - NWG * hgp;
    const int nwin = (end - start + 63) >> 6;
    const int own = wl < nwin ? (nwin - wl + NWG - 1) / NWG : 0;
    const int lastc = NWG - 1 < nwin ? (nwin - (NWG - 1) + NWG - 1) / NWG : 0;  // the last wave's claims
    const int kApp = fused && hgp == HG - 1 ? min(3, lastc / 3) : 0;
    const int keep = lastc - kApp;  // claims the last wave keeps
    const int extra = wl < NWG - 1 ? (kApp - wl + NWG - 2) / (NWG - 1) : 0;
    const int cnt = wl < NWG - 1 ? own + extra : keep;
    // (s 13 + h 5 + split 7: the workgroups on one XCD -- the same kv head for one split --
    // start at distinct windows; measured against (row 37 + split 11), whose offsets repeat
    // every 4 sequences of a head: config 3 1.798 vs 1.834 ms per step)
    const int R = nwin ? (int)((unsigned)(NWG * (s * 13 + h * 5 + split * 7)) % (unsigned)nwin) : 0;
    const int oob = start + 64 * nwin;
    auto win_base = [&](int i) {
        if (i >= cnt) return oob;
        const int j = i < own ? NWG * i + wl : NWG * (keep + (NWG - 1) * (i - own) + wl) + NWG - 1;
        int r = j + R;
        r = r >= nwin ? r - nwin : r;
        return start + 64 * r;
    };
    Window8<HD> w[D];
    // this wave's query heads: Gg of them from head hgb of the sequence (HG = 2: up to 8 a group)
    const int Gg = HG == 1 ? G : max(0, min(8, G - 8 * hgp));
    const int hgb = h * G + (HG == 1 ? 0 : 8 * hgp);

    // q operand: lane 16 g + n holds row n = 4 hh + c (digit c of head hh) for k-group g, i.e.
    // dims 64 m + 16 g .. + 15 of instruction m, bytes [even dims of word 8m + 2g, its odd
    // dims, even dims of word 8m + 2g + 1, its odd dims] like the K operand.  The raw q loads
    // go out before the windows' prefetch: loads complete in order, so consuming q then does
    // not wait for the windows.
    i32x4 qa[GH][NM], bias[GH];
    float qinv[GH];
    const bool appender = fused && wave == NW - 1;
    AppendIn<HD> ain;
    float2 qp[4 * GH * HG][AppendIn<HD>::PPL];
    {
        // half hf: lane 16 g + n holds digit dg of head hh + 4 hf
        const int n = lane & 15, g = lane >> 4, hh = n >> 2, dg = n & 3;
        bool hl[GH];
        float qx[GH][NM][16], nwv[NM][16];
        float2 qcs[NM][8];
#pragma unroll
        for (int hf = 0; hf < GH; hf++) {
            hl[hf] = hh + 4 * hf < Gg;
            const float *qrow = a.q + ((size_t)s * a.n_head + hgb + (hl[hf] ? hh + 4 * hf : 0)) * hdr;
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int d0 = 64 * m + 16 * g;
#pragma unroll
                for (int e4 = 0; e4 < 4; e4++) {
                    const bool in = d0 + 4 * e4 < hdr;  // stored dims past the row are 0
                    const float4 v4 = keep4(in, *reinterpret_cast<const float4 *>(qrow + (in ? d0 + 4 * e4 : 0)));
                    qx[hf][m][4 * e4] = v4.x; qx[hf][m][4 * e4 + 1] = v4.y;
                    qx[hf][m][4 * e4 + 2] = v4.z; qx[hf][m][4 * e4 + 3] = v4.w;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const int d0 = 64 * m + 16 * g;
#pragma unroll
            for (int e4 = 0; e4 < 4; e4++) {
                const bool in = d0 + 4 * e4 < hdr;
                if (QN) {
                    const float4 n4 = *reinterpret_cast<const float4 *>(QN + (in ? d0 + 4 * e4 : 0));  // (only
                    // multiplies dims that are zero past the row)
                    nwv[m][4 * e4] = n4.x; nwv[m][4 * e4 + 1] = n4.y; nwv[m][4 * e4 + 2] = n4.z; nwv[m][4 * e4 + 3] = n4.w;
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int pair = d0 / 2 + i;
                qcs[m][i] = pair < a.rope_pairs
                                ? *reinterpret_cast<const float2 *>(a.rope + ((size_t)qrot * a.rope_pairs + pair) * 2)
                                : make_float2(1.0f, 0.0f);
            }
        }
        // QK norm scale of this lane's head in each half (all heads' scales, then a select)
        float ns[GH];
#pragma unroll
        for (int hf = 0; hf < GH; hf++) ns[hf] = 1.0f;
        if (QN) {
            float nall[4 * GH];
            q_norm_scales_wave<HD, 4 * GH>(a.q + ((size_t)s * a.n_head + hgb) * hdr, Gg, L.norm_eps, hdr, nall);
#pragma unroll
            for (int hf = 0; hf < GH; hf++)
#pragma unroll
                for (int c = 0; c < 4; c++) ns[hf] = hh == c ? nall[4 * hf + c] : ns[hf];
        }
        // The appending wave (the last: it has the fewest windows) quantizes the new token and
        // scores it against every head before its windows; the others start at once.  Its
        // loads go out with q's.  kd, vd and xnew are read after the barrier that opens the
        // merge.
        if (appender) {
            append_load<HD, NORM>(a, s, h, qpos, lane, ain, hdr);
            load_q_pairs<HD, 4 * GH * HG>(a, s, h * G, G, lane, qp, hdr);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < D - 1; d++) load_window8<HD, HG == 1 ? kNT : 0>(w[d], str, win_base(d), lane);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hf = 0; hf < GH; hf++) {
        // rotated q times log2(e)/sqrt(hd) (rope.rs:186-196 after the optional QK norm)
        float qm = 0.0f;
#pragma unroll
        for (int m = 0; m < NM; m++) {
#pragma clang fp contract(off)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float x0 = qx[hf][m][2 * i], x1 = qx[hf][m][2 * i + 1];
                if (QN) {
                    x0 = qk_norm_apply(x0, ns[hf], nwv[m][2 * i]);
                    x1 = qk_norm_apply(x1, ns[hf], nwv[m][2 * i + 1]);
                }
                if ((64 * m + 16 * g) / 2 + i < a.rope_pairs) rope_rotate(x0, x1, qcs[m][i]);
                qx[hf][m][2 * i] = x0 * (a.inv_sqrt_hd * kLog2e);
                qx[hf][m][2 * i + 1] = x1 * (a.inv_sqrt_hd * kLog2e);
                qm = fmaxf(qm, fmaxf(fabsf(qx[hf][m][2 * i]), fabsf(qx[hf][m][2 * i + 1])));
            }
        }
        // head hh's integer scale 2^e: max |q| 2^e in [2^26, 2^27), so every digit fits int8
        qm = group_max(qm);
        int e = 0;
        if (qm > 0.0f && qm < 3.0e38f) e = 26 - min(max(ilogbf(qm), -100), 100);
        const float sc = ldexpf(1.0f, e);
        // digits: Q = d0 2^21 + d1 2^14 + d2 2^7 + d3, d1..d3 in [-64, 63], |d0| <= 64.  With
        // Q' = Q + 64 (2^21 + 2^14 + 2^7 + 1) > 0, D_c = d_c + 64 are the base-128 digits of Q'
        // (D_0 = Q' >> 21 <= 128), so this lane's digit is one shift and mask away.
        const int sh = 7 * (3 - dg);
        const uint32_t msk = dg == 0 ? 0xFFu : 0x7Fu;
        uint32_t dsum_raw = 0;
#pragma unroll
        for (int m = 0; m < NM; m++) {
            uint32_t reg[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int el = 0; el < 16; el++) {
                const int Q = hl[hf] ? (int)rintf(qx[hf][m][el] * sc) : 0;
                const uint32_t dig = ((uint32_t)(Q + 135274560) >> sh) & msk;
                dsum_raw += dig;
                // element el = dim 64 m + 16 g + el: word 8m + 2g + el / 8, parity el % 2 selects
                // the even (reg 0 / 2) or odd (reg 1 / 3) register, byte (el % 8) / 2
                const int rr = 2 * (el >> 3) + (el & 1), by = (el & 7) >> 1;
                reg[rr] |= ((dig + 192u) & 0xFFu) << (8 * by);  // the byte of D_c - 64
            }
            qa[hf][m] = (i32x4){(int)reg[0], (int)reg[1], (int)reg[2], (int)reg[3]};
        }
        int dsum = (int)dsum_raw - 64 * 16 * NM;
        // bias of accumulator (head hg, digit r): -8 * (digit sum of row 4 hg + r)
        dsum += __shfl_xor(dsum, 16, 64);
        dsum += __shfl_xor(dsum, 32, 64);
        if (g == 0) qsum[wave][hf][n] = dsum;
        if (g == 0 && dg == 0) qinv_s[wave][hf][hh] = ldexpf(1.0f, -e);
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        const int hg = lane >> 4;
#pragma unroll
        for (int hf = 0; hf < GH; hf++) {
            bias[hf] = (i32x4){-8 * qsum[wave][hf][4 * hg], -8 * qsum[wave][hf][4 * hg + 1],
                               -8 * qsum[wave][hf][4 * hg + 2], -8 * qsum[wave][hf][4 * hg + 3]};
            qinv[hf] = qinv_s[wave][hf][hg];
        }
    }
    if (appender) {
        append_store<HD, NORM>(a, s, h, qpos, lane, ain, kd, vd, hdr);
        new_token_scores<HD, SOFTCAP, NORM, 4 * GH * HG>(a, s, h * G, G, lane, qp, ain.cs, kd, xnew, hdr);
    }

    WaveState8<HD, GH> st;
#pragma unroll
    for (int ps = 0; ps < kPvSets<GH>; ps++)
#pragma unroll
        for (int td = 0; td < NTD; td++) st.o[ps][td] = (floatx4)0.0f;
    bool live[GH];
#pragma unroll
    for (int hf = 0; hf < GH; hf++) {
        st.m[hf] = kMinit;
        st.l[hf] = 0.0f;
        live[hf] = (lane >> 4) + 4 * hf < Gg;
    }
    _Float16 (*pt)[64] = pts[wave];

    int it = 0;
    if (cnt > 0) {
        while (true) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                load_window8<HD, HG == 1 ? kNT : 0>(w[(d + D - 1) % D], str, win_base(it + D - 1), lane);
                // keep the prefetch here: the scheduler would otherwise sink it below the use.
                // (Refilling a slot right after its window is processed instead measured
                // slower: config 3 1.871 vs 1.848 ms per step, config 4 1.63 vs 1.46.)
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                // (one form for every window, the tail mask included: a branch between a masked
                // and an unmasked copy made the compiler shuffle the accumulators at the join,
                // ~30 moves per window; config 4 1.396 vs 1.408 ms per step)
                process_window8<HD, SOFTCAP, GH>(w[d], st, qa, bias, qinv, pt, win_base(it), end, lane, live, a.softcap, dc);
                if (++it >= cnt) goto windows_done;
            }
        }
    }
windows_done:

    // ---- merge the waves through LDS ------------------------------------------------------------
    // Each wave writes its O^T columns (16-byte stores: lane (n, g) holds dims 16 td + 4 g ..
    // + 3 of column n), its m and l; one barrier; then one float4 of dims per thread.
    // (Merge area shared with the P tiles, a barrier before the writes, scalar stores and one
    // dim per thread: ~1.4 us from the last wave's loop end to the output.)
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int hf = 0; hf < GH; hf++) {
        const float l_run = row_sum16(st.l[hf]);
        if (n == 0) {
            mm_[wave][4 * hf + g] = st.m[hf];
            ml_[wave][4 * hf + g] = l_run;
        }
    }
#pragma unroll
    for (int ps = 0; ps < kPvSets<GH>; ps++)
        if (16 * ps + n < 8 * GH) {
#pragma unroll
            for (int td = 0; td < NTD; td++)
                *reinterpret_cast<floatx4 *>(&mo[wave][(16 * ps + n) * OST + 16 * td + 4 * g]) = st.o[ps][td];
        }
    __syncthreads();

    constexpr int V4 = HD / 4;
    for (int idx = tid; idx < G * V4; idx += 64 * NW) {
        const int hh = idx / V4, d = 4 * (idx % V4);
        // head hh is head lh of group grp, held by that group's NWG waves from wave wb
        const int grp = HG == 1 ? 0 : hh >> 3, lh = hh - 8 * grp, wb = NWG * grp;
        float M = kMinit;
#pragma unroll
        for (int w = 0; w < NWG; w++) M = fmaxf(M, mm_[wb + w][lh]);
        if (fused) M = fmaxf(M, xnew[hh]);
        floatx4 acc = (floatx4)0.0f;
        float lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < NWG; w++) {
            const float e = exp2f(mm_[wb + w][lh] - M);
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(&mo[wb + w][lh * OST + d]);
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(&mo[wb + w][(lh + 4 * GH) * OST + d]);
            acc += e * (hi + lo);
            lsum += e * ml_[wb + w][lh];
        }
        if (fused) {
            const float e = exp2f(xnew[hh] - M);
            acc += e * *reinterpret_cast<const floatx4 *>(&vd[d]);
            lsum += e;
        }
        const size_t head = (size_t)s * a.n_head + h * G + hh;
        if (n_split_s == 1) {
            // hdr is a multiple of 8: a float4 of dims lies wholly inside or outside the row
            const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
            if (d < hdr) {
                const floatx4 r = lsum > 0.0f ? acc * inv : (floatx4)0.0f;
                *reinterpret_cast<float4 *>(a.out + head * hdr + d) = make_float4(r[0], r[1], r[2], r[3]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) store_partial(a, head, split, HD, d + k, acc[k], M, lsum);
        }
    }
}

}  // namespace

// Split plan.  The integer kernel (G <= 8) runs one workgroup per CU (4 waves, 8 for 64-dim
// rows), the 16x16 kernel two per CU.  The chunk (positions per split, a multiple of 64) is the smallest one for which
// the busy workgroups of the whole batch, n_kv * sum_s ceil(n_ctx[s] / chunk), fit in that
// target: the batch's total context spread evenly, so ragged batches give their long
// sequences more splits and no CU gets a second workgroup.  (Measured on the config-3 shape
// with a loads-only probe of the same access pattern: one workgroup per stream and CU 43.2 us,
// two 44.7 us, three 45.6 us.)  Splits shorter than kMinChunk leave waves without a window.
namespace {
constexpr int kMinChunk = 256;
constexpr int kG4MinChunk = 1024;  // the integer kernel needs >= 4 windows per wave to pay off

int plan_chunk(const int32_t *n_ctx, int n_seq, int n_kv, int target) {
    int64_t total = 0;
    int max_ctx = 1;
    for (int s = 0; s < n_seq; s++) {
        total += n_ctx[s];
        max_ctx = std::max(max_ctx, (int)n_ctx[s]);
    }
    auto busy = [&](int chunk) {
        int64_t n = 0;
        for (int s = 0; s < n_seq; s++) n += (n_ctx[s] + chunk - 1) / chunk;
        return n * n_kv;
    };
    const int hi_c = std::max(kMinChunk, (max_ctx + 63) / 64 * 64);
    int lo_c = (int)std::min<int64_t>(hi_c, std::max<int64_t>(kMinChunk, (total * n_kv + target - 1) / target));
    lo_c = (lo_c + 63) / 64 * 64;
    // smallest multiple of 64 in [lo_c, hi_c] with busy <= target (busy is non-increasing)
    int lo = lo_c / 64, hi = hi_c / 64;
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (busy(64 * mid) <= target) hi = mid; else lo = mid + 1;
    }
    // More streams than the target (many sequences): no chunk meets it.  The balanced chunk
    // (the batch's work over the target) still splits the sequences much longer than the rest,
    // which would otherwise stream alone after the others finished; for a uniform batch it is
    // the whole sequence anyway.
    if (busy(64 * lo) > target) return lo_c;
    return 64 * lo;
}
}  // namespace

DecodePlan decode_plan(const int32_t *n_ctx, int n_seq, int n_kv, int G, int n_cu, int stored_hd, bool fused) {
    const int int_gmax = decode_int_gmax(stored_hd);
    DecodePlan p;
    p.nw = 4;
    int max_ctx = 1;
    for (int s = 0; s < n_seq; s++) max_ctx = std::max(max_ctx, (int)n_ctx[s]);
    p.g4 = false;
    if (G <= int_gmax) {  // the integer kernel: one, two or four halves of 4 query heads
        // Target 7/8 of the CUs, not all of them: a plan that fills every CU of a ragged
        // batch had ~24 busy workgroups wait 9-20 us for a CU (behind busy ones) while idle
        // splits freed others -- the dispatcher does not place a workgroup on just any free
        // CU of its XCD.  Over ten length draws of config 4: 0.441-0.679 of HBM peak (mean
        // 0.60) with every CU, 0.648-0.682 (mean 0.66) with 7/8.  Uniform batches (one split
        // per stream, config 3) are not affected.
        p.chunk = plan_chunk(n_ctx, n_seq, n_kv, n_cu - n_cu / 8);
        p.g4 = p.chunk >= kG4MinChunk;
    }
    // the 16x16 kernel takes up to 8 query heads per workgroup: more as several head groups
    if (!p.g4) p.chunk = plan_chunk(n_ctx, n_seq, n_kv * ((G + 7) / 8), 2 * n_cu);
    p.n_split = (max_ctx + p.chunk - 1) / p.chunk;
    // Few streams, short context: one wide workgroup per stream instead of a split, when its
    // waves cover the longest sequence's windows (the positions before the new token with the
    // fused append, which scores that one from registers) in one round.  No combine launch
    // (the split kernel then also advances the lengths), the merge stays in LDS.  The fewest
    // waves that cover it: 8 waves measured 9.1 us per step on config 1's shape (512 positions
    // + the new token), 16 waves 10.1, four-wave splits and a combine 10.5.  More than one
    // window per wave does not pay: 8.5 windows per wave took 26.6 us per layer on config 2's
    // shape against 10.0 with splits and a combine.
    const int n_win = (max_ctx - (fused ? 1 : 0) + 63) / 64;
    if (!p.g4 && n_win > 4 && (int64_t)n_seq * n_kv * ((G + 7) / 8) <= n_cu) {
        const int wmax = stored_hd <= 64 ? 16 : stored_hd <= 128 ? 8 : 4;
        for (int nw = 8; nw <= wmax; nw *= 2)
            if (n_win <= nw) {
                p.nw = nw;
                p.chunk = (max_ctx + 63) / 64 * 64;
                p.n_split = 1;
                break;
            }
    }
    return p;
}

int decode_cap(int n_kv, int max_seq, int n_cu) {
    // One sequence alone can take at most target / n_kv splits (plus one for rounding); the
    // 16x16 kernel's target, 2 n_cu, is the larger.
    return std::min((max_seq + 63) / 64, 2 * n_cu / n_kv + 2);
}

namespace {
// The integer kernel's static LDS (the arrays it declares), for the dynamic reservation below.
template <int HD, int NW, int GH, int HG>
constexpr size_t split4_static_lds() {
    return (size_t)NW * 8 * GH * 64 * 2          // pts
           + (size_t)NW * 8 * GH * (HD + 4) * 4  // mo
           + (size_t)2 * NW * 4 * GH * 4         // mm_, ml_
           + (size_t)2 * HD * 4 + (4 * GH * HG < 8 ? 8 : 4 * GH * HG) * 4  // kd, vd, xnew
           + (size_t)NW * GH * 16 * 4 + (size_t)NW * GH * 4 * 4;  // qsum, qinv_s
}

// One integer-kernel launch.  The kernel fits two workgroups per CU by registers, but the plan
// wants one per CU: an unused dynamic LDS reservation that takes the workgroup to 84 KB (more
// than half of a CU's 160 KB, and at most all of it) makes the dispatcher place busy workgroups
// on distinct CUs, also when the grid holds idle ones (splits past a short sequence's end)
// that exit at once.
template <int HD, bool SC, bool NM, bool PAD, int NW, int GH, int HG = 1>
void launch_split4(const DecodeArgs &a, int n_split, hipStream_t st) {
    constexpr size_t kOne = 84 * 1024, own = split4_static_lds<HD, NW, GH, HG>();
    static_assert(own <= 160 * 1024, "integer kernel LDS");
    constexpr size_t lds = own >= kOne ? 0 : kOne - own;
    decode_split4_kernel<HD, SC, NM, PAD, NW, 2, GH, HG><<<dim3(a.L.H, a.L.S, n_split), 64 * NW, lds, st>>>(a);
}

// 64-dim rows carry half the bytes per position for the same per-position softmax work: they
// run 8 waves (two per SIMD), so that one wave's softmax overlaps the other's loads.  Config-3
// shape with 64-dim rows: 1.170 vs 1.378 ms per step at 8 query heads per kv head, 1.017 vs
// 1.030 at 4; ragged config 4: 0.837 vs 0.886.  (With 128-dim rows and two halves of heads 8
// waves measured slower: 1.970 vs 1.888.)
template <int HD, bool SC, bool NM, bool PAD>
void launch_16x16_pad(const DecodeArgs &a, dim3 grid, int nw, hipStream_t st) {
    if (HD <= 128 && nw == 8)
        decode_split_kernel<HD, SC, NM, PAD, HD <= 128 ? 8 : 4><<<grid, 64 * 8, 0, st>>>(a);
    else if (HD <= 64 && nw == 16)
        decode_split_kernel<HD, SC, NM, PAD, HD <= 64 ? 16 : 4><<<grid, 64 * 16, 0, st>>>(a);
    else
        decode_split_kernel<HD, SC, NM, PAD, 4><<<grid, 64 * 4, 0, st>>>(a);
}

template <int HD, bool SC, bool NM>
void launch_16x16(const DecodeArgs &a, dim3 grid, int nw, bool pad, hipStream_t st) {
    if (pad) launch_16x16_pad<HD, SC, NM, true>(a, grid, nw, st);
    else launch_16x16_pad<HD, SC, NM, false>(a, grid, nw, st);
}

template <int HD, bool SC, bool NM>
void launch_integer(const DecodeArgs &a, int n_split, bool pad, int Gt, hipStream_t st) {
    constexpr int NW = HD == 64 ? 8 : 4;
    if constexpr (HD <= 128) {
        // More than 8 query heads per kv head (the plan allows them up to 128-dim rows).  On
        // 64-dim rows: two head groups of 4 waves, two halves each (config-3 shape with 128 q
        // heads 1.955 vs 2.199 ms per step); on 128-dim rows: four halves in one wave per SIMD
        // (2.86 vs 3.39 ms with head groups, whose second read of each window does not all come
        // from L2).
        if (Gt > 8) {
            if constexpr (HD == 64) {
                if (pad) launch_split4<HD, SC, NM, true, 8, 2, 2>(a, n_split, st);
                else launch_split4<HD, SC, NM, false, 8, 2, 2>(a, n_split, st);
            } else {
                if (pad) launch_split4<HD, SC, NM, true, 4, 4>(a, n_split, st);
                else launch_split4<HD, SC, NM, false, 4, 4>(a, n_split, st);
            }
            return;
        }
    }
    if (Gt > 4) {
        if (pad) launch_split4<HD, SC, NM, true, NW, 2>(a, n_split, st);
        else launch_split4<HD, SC, NM, false, NW, 2>(a, n_split, st);
    } else {
        if (pad) launch_split4<HD, SC, NM, true, NW, 1>(a, n_split, st);
        else launch_split4<HD, SC, NM, false, NW, 1>(a, n_split, st);
    }
}
}  // namespace

hipError_t launch_decode(const KvLayerView &L, int32_t *d_len, const int32_t *h_len, const float *q, int n_head,
                         const float *rope, int rope_pairs, float softcap, float *out,
                         float *ws, const DecodePlan &plan, const float *k_new,
                         const float *v_new, int32_t *adv, hipStream_t st) {
    DecodeArgs a;
    a.L = L;
    a.len = d_len;
    a.hlen = h_len && L.S == 1 ? h_len[0] : -1;
    a.q = q;
    a.rope = rope;
    a.rope_pairs = rope_pairs;
    a.n_head = n_head;
    a.Gt = n_head / L.H;
    a.NG = plan.g4 ? 1 : (a.Gt + 7) / 8;
    a.G = plan.g4 ? a.Gt : std::min(a.Gt, 8);
    a.chunk = plan.chunk;
    a.n_split = plan.n_split;
    a.inv_sqrt_hd = 1.0f / sqrtf((float)L.hdr);
    a.softcap = softcap;
    a.out = out;
    a.ws = ws;
    a.k_new = k_new;
    a.v_new = v_new;
    // with a split the combine kernel advances the lengths (the last of its workgroups to
    // arrive); without one a length update follows the decode launch
    // (the 16x16 kernel does it itself when there is no split)
    const bool adv_in_kernel = plan.n_split > 1 || !plan.g4;
    a.adv_len = adv && adv_in_kernel ? d_len : nullptr;
    a.adv_ctr = adv && adv_in_kernel ? adv : nullptr;
    dim3 grid(plan.n_split, L.H * a.NG, L.S);
    // The integer kernel does less VALU work per window than the 16x16 one but has the longer
    // per-window dependency chain; it runs when every wave streams at least 4 windows of its
    // split (plan.g4).
    const bool cap = softcap > 0.0f, norm = L.qn != nullptr || L.kn != nullptr;
    const bool pad = L.hdr != L.hd;
#define TS_SPLIT(HDV, SC, NM)                                                                  \
    (plan.g4 ? (launch_integer<HDV, SC, NM>(a, plan.n_split, pad, a.Gt, st), 0) \
             : (launch_16x16<HDV, SC, NM>(a, grid, plan.nw, pad, st), 0))
#define TS_SPLIT_HD(HDV)                                                                      \
    (cap ? (norm ? TS_SPLIT(HDV, true, true) : TS_SPLIT(HDV, true, false))                    \
         : (norm ? TS_SPLIT(HDV, false, true) : TS_SPLIT(HDV, false, false)))
    if (L.hd == 256) {
        TS_SPLIT_HD(256);
        if (plan.n_split > 1) decode_combine_kernel<256><<<dim3(n_head, L.S), 256, 0, st>>>(a);
    } else if (L.hd == 128) {
        TS_SPLIT_HD(128);
        if (plan.n_split > 1) decode_combine_kernel<128><<<dim3(n_head, L.S), 256, 0, st>>>(a);
    } else if (L.hd == 64) {
        TS_SPLIT_HD(64);
        if (plan.n_split > 1) decode_combine_kernel<64><<<dim3(n_head, L.S), 256, 0, st>>>(a);
    } else {
        return hipErrorInvalidValue;
    }
#undef TS_SPLIT_HD
#undef TS_SPLIT
    if (adv && !adv_in_kernel) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_len_update(d_len, L.S, -1, 1, 0, st);
    }
    return hipGetLastError();
}

}  // namespace ts
