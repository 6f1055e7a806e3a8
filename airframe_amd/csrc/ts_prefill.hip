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
// * grid = (column block of 128, kv head, sequence); each of the 4 waves owns 32 columns,
//   one N tile of v_mfma_f32_32x32x16_f16 (half the instructions of 16x16x32 for the same
//   work).  The workgroup walks the keys in 64-key windows:
//   every thread loads one 16-byte piece of the next window's K rows / V blocks / scales
//   while the current window is computed, then converts it to exact f16 integer codes in a
//   double-buffered LDS tile, so each code is converted once per workgroup and read by all
//   4 waves.
// * S^T = K Q^T with q split into an f16 high half (f16 MFMAs) and a low half as two fp6 terms
//   (one scaled fp6 MFMA per term and 64 dims, the K codes converted to fp6 from the same f16
//   operand registers), all into one f32 accumulator, with 1/sqrt(hd)*log2(e) and a
//   power-of-two range scale folded into q.  K rows enter the MFMA in
//   the order that leaves every lane holding, per 16-key step, exactly the 8 keys it supplies
//   to the PV operand, so P never moves between lanes.  The score is scaled by s_k in f32,
//   masked only in windows that cross the causal diagonal, and enters an online softmax in
//   the exp2 domain whose running max is raised lazily; p*s_v goes to O^T += V^T P^T split
//   hi + lo in f16 (two MFMAs) under an exponent bound that keeps it below 2^15.
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
    int q_delay;  // sleeps of ~1 us before the q read of the lightest column block (0: none)
};

constexpr int kPrefillNW = 4;  // waves per workgroup

constexpr int kColsPerWave = 32;
constexpr int kWin = 64;  // keys per window

// Double-buffered window tiles.  K: [key][word] f16 codes; V^T: [dim][8-key group] f16
// codes, each group in the PV operand's key order.  Rows are unpadded; the 16-byte slots
// inside a row are rotated per row (k_slot, v_slot) so that the MFMA operand reads of a wave
// hit distinct LDS banks (chosen by measurement on gfx950: 2x the rate of unrotated rows).
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

// Slot of word w in the K row of `key`, and of 8-key group sl in the V^T row `row`.
template <int HD>
__device__ inline int k_slot(int key, int w) { return (w + key) & (HD / 8 - 1); }
__device__ inline int v_slot(int row, int sl) { return (sl + (row >> 1)) & 7; }

// Key (within a 32-key tile) that accumulator row R of the QK MFMA stands for.  Lane half h
// holds rows 8q + 4h + r (q, r = 0..3); mapping them to keys 16(q/2) + 8h + 4(q%2) + r gives
// each lane half the 8 consecutive keys 16s + 8h .. +7 of 16-key step s, which is what the PV
// MFMA's B operand wants from it.
__device__ inline int qk_row_key(int R) {
    const int q = R >> 3, h = (R >> 2) & 1, r = R & 3;
    return 16 * (q >> 1) + 8 * h + 4 * (q & 1) + r;
}

// Which 16-byte piece of the window a staging thread owns.  The maps are chosen so that 16
// consecutive lanes write 16 different LDS bank groups:
//  K piece c: chunk k_chunk(c) of the window (the cache's K chunk order, k_word_idx), whose
//  word j is word u of key `key` (k_piece_word); 16 consecutive pieces hold 16 consecutive
//  keys;
//  V piece c: block c / HD, and within it lane group L = c % 64 of the packed layout, its
//  (HD/64)-th piece (c % HD) / 64.
template <int HD>
__device__ inline int k_chunk(int c) {
    if constexpr (HD == 256) {
        const int t = c & 3, n = ((c >> 2) & 3) + 4 * ((c >> 4) & 3), g = (c >> 6) & 3, mh = (c >> 8) & 1;
        return (2 * t + mh) * 64 + 16 * g + n;
    } else if constexpr (HD == 128) {
        const int t = c & 3, n = ((c >> 2) & 3) + 4 * ((c >> 4) & 3), g = (c >> 6) & 3;
        return t * 64 + 16 * g + n;
    } else {
        const int qc = c & 1, n = (c >> 1) & 15, g = (c >> 5) & 3;
        return qc * 64 + 16 * g + n;
    }
}
template <int HD>
__device__ inline void k_piece_word(int c, int j, int &key, int &u) {
    if constexpr (HD == 256) {
        const int t = c & 3, n = ((c >> 2) & 3) + 4 * ((c >> 4) & 3), g = (c >> 6) & 3, mh = (c >> 8) & 1;
        key = 4 * n + t;
        u = 16 * mh + 8 * (j >> 1) + 2 * g + (j & 1);
    } else if constexpr (HD == 128) {
        const int t = c & 3, n = ((c >> 2) & 3) + 4 * ((c >> 4) & 3), g = (c >> 6) & 3;
        key = 4 * n + t;
        u = 8 * (j >> 1) + 2 * g + (j & 1);
    } else {
        const int qc = c & 1, n = (c >> 1) & 15, g = (c >> 5) & 3;
        key = 4 * n + 2 * qc + (j >> 1);
        u = 2 * g + (j & 1);
    }
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
        return *reinterpret_cast<const uint4 *>(kbase + (size_t)base * ROWB + k_chunk<HD>(c) * 16);
    };
    auto load_v = [&](int c) {
        int b, piece;
        v_piece<HD>(c, b, piece);
        // piece = (HD/64) * ln + t: the t-th 16-byte chunk of lane group ln (v_word_idx)
        constexpr int PPL = HD / 64;
        const int chunk = (piece % PPL) * 64 + piece / PPL;
        return *reinterpret_cast<const uint4 *>(vbase + (size_t)(base / 32 + b) * (HD * 16) + chunk * 16);
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

// Staging of one window's codes, as 8 * NK parts of one 32-bit word each per thread (parts
// [0, 4 NK): K words, [4 NK, 8 NK): V words), so the caller can spread them over other work.
// Only for the layout where every thread holds NK K pieces and NK V pieces (!SPLIT).
template <int HD, int NW, class SM>
__device__ inline void stage_part(SM &sm, int buf, const Pending<HD, NW> &pd, int tid,
                                  int part, const DeqConst &dk) {
    using P = Pending<HD, NW>;
    static_assert(!P::SPLIT, "per-part staging needs whole K and V pieces per thread");
    const int i = (part % (4 * P::NK)) / 4, j = part % 4;
    const int c = tid + P::NT * i;
    if (part < 4 * P::NK) {
        const uint4 &x = pd.k[i];
        const uint32_t wj = j == 0 ? x.x : j == 1 ? x.y : j == 2 ? x.z : x.w;
        int key, u;
        k_piece_word<HD>(c, j, key, u);
        sm.k[buf][key][k_slot<HD>(key, u)] = dequant8_c(wj, dk);
    } else {
        // V: lane L holds 4 words of packed lane group ln = L (key group g = ln/16, dim row dl
        // = ln%16); lane L^16 holds the same words of key group g^1.  Words of groups 2p and
        // 2p+1 hold keys 8p..8p+7 in their low halves (nibbles 0-3) and 16+8p..16+8p+7 in
        // their high halves, so the even lane builds the dword of low halves, the odd lane the
        // one of high halves: one 8-key group of the V^T row each.
        const uint4 &x = pd.v[i];
        const uint32_t wj = j == 0 ? x.x : j == 1 ? x.y : j == 2 ? x.z : x.w;
        int b, piece;
        v_piece<HD>(c, b, piece);
        const int ln = c % 64, dl = ln & 15, odd = (ln >> 4) & 1, pair = ln >> 5;
        const int td0 = (c % HD) / 64 * 4;
        const int sl = 4 * b + 2 * odd + pair;
        // byte selects of v_perm_b32(pw, w): even lanes low(w) | low(pw) << 16, odd lanes
        // high(pw) | high(w) << 16 (one instruction, no lane-divergent branch)
        const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
        const uint32_t pw = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (threadIdx.x ^ 16), (int)wj);
        const uint32_t d = __builtin_amdgcn_perm(pw, wj, sel);
        const int row = 16 * (td0 + j) + dl;
        sm.v[buf][row][v_slot(row, sl)] = dequant8_c(d, dk);
    }
}

// All of one window's codes into LDS.
template <int HD, int NW, class SM>
__device__ inline void stage_codes(SM &sm, int buf, const Pending<HD, NW> &pd, int tid,
                                   int wave, const DeqConst &dk) {
    using P = Pending<HD, NW>;
    if constexpr (P::SPLIT) {
        // V staging as in stage_part, for a thread that holds one V piece
        auto put_k = [&](int c, const uint4 &x) {
            const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                int key, u;
                k_piece_word<HD>(c, j, key, u);
                sm.k[buf][key][k_slot<HD>(key, u)] = dequant8_c(w[j], dk);
            }
        };
        auto put_v = [&](int c, const uint4 &x) {
            const uint32_t w[4] = {x.x, x.y, x.z, x.w};
            int b, piece;
            v_piece<HD>(c, b, piece);
            const int ln = c % 64, dl = ln & 15, odd = (ln >> 4) & 1, pair = ln >> 5;
            const int td0 = (c % HD) / 64 * 4;
            const int sl = 4 * b + 2 * odd + pair;
            const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t pw = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (threadIdx.x ^ 16), (int)w[j]);
                const uint32_t d = __builtin_amdgcn_perm(pw, w[j], sel);
                const int row = 16 * (td0 + j) + dl;
                sm.v[buf][row][v_slot(row, sl)] = dequant8_c(d, dk);
            }
        };
        if (wave < P::KCH / 64)
            put_k(tid, pd.k[0]);
        else
            put_v(tid - P::KCH, pd.k[0]);
    } else {
#pragma unroll
        for (int part = 0; part < 8 * P::NK; part++) stage_part<HD, NW, SM>(sm, buf, pd, tid, part, dk);
    }
}

// The window's scales into LDS (kept apart from the code staging, which is branch-free so it
// can be scheduled in between the QK matrix-core instructions).
template <int HD, int NW, class SM>
__device__ inline void stage_scales(SM &sm, int buf, const Pending<HD, NW> &pd, int tid,
                                    float inv_s) {
    if (tid < kWin) {
        sm.sk[buf][tid] = pd.scale * inv_s;  // undo the q operand scale (a power of two: exact)
    } else if (tid < 2 * kWin) {
        sm.sv[buf][tid - kWin] = pd.scale;
        // (one whole wave: threads kWin .. 2 kWin - 1; the scales are >= 0)
        const float m = wave_max_nonneg(pd.scale);
        if (tid == kWin) sm.svlog[buf] = __log2f(m);
    }
}

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int int6v __attribute__((ext_vector_type(6)));
typedef int int8v __attribute__((ext_vector_type(8)));
typedef _Float16 half32 __attribute__((ext_vector_type(32)));
typedef float float32v __attribute__((ext_vector_type(32)));

// q's low half on the fp6 matrix-core path.  The low half q - f16(q) needs only a few bits of
// its own: it enters v_mfma_scale_f32_32x32x64_f8f6f4 as fp6 e2m3 (3 mantissa bits, largest
// 7.5) with a power-of-two scale, while the K codes on the other side (integers -7..7) are
// exact in e2m3.  That MFMA does 64 k-steps of 32x32 in about the time of one 32x32x16 f16
// MFMA (a quarter of the four f16 MFMAs it replaces); two terms (the second one the rounding
// rest of the first) keep q to about f16 hi + lo accuracy.
__device__ inline float exp2i(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }

// 4 k-steps of an f16 operand (32 values per lane, in operand order) as fp6 divided by s.
__device__ inline int6v fp6_of(const half8 (&x)[4], float s) {
    half32 v;
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int j = 0; j < 8; j++) v[8 * u + j] = x[u][j];
    return __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(v, s);
}

// o += a b^T over 64 k-steps, a: fp6 codes (scale 1), b: fp6 with scale 2^(e8 - 127).
__device__ inline floatx16 mfma_lo6(int6v a, int6v b, floatx16 c, int e8) {
    const int8v a8 = {a[0], a[1], a[2], a[3], a[4], a[5], 0, 0};
    const int8v b8 = {b[0], b[1], b[2], b[3], b[4], b[5], 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 2, 2, 0, 127, 0, e8);
}

// q's low half over one group of 4 k-steps (32 values lo[], f32) as two fp6 terms with fixed
// scales: q is scaled so that |q| < 2^14 (q_scale), so its f16 high half leaves |lo| <= 4
// (half an f16 ulp at 2^13); t1 = fp6(lo) rounds that to within 0.125, and t2 = fp6((lo - t1)
// / 2^-5) keeps the rest to 2^-8: q to ~2^-22 of its bound, as a second f16 half would.
constexpr int kQlo1E8 = 127, kQlo2E8 = 127 - 5;
__device__ inline void q_lo_terms(const float (&lo)[32], int6v &t1, int6v &t2) {
    floatx16 a, b;
#pragma unroll
    for (int i = 0; i < 16; i++) {  // the conversion interleaves its two sources
        a[i] = lo[2 * i];
        b[i] = lo[2 * i + 1];
    }
    t1 = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(a, b, 1.0f);
    const float32v back = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(t1, 1.0f);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        a[i] = lo[2 * i] - back[2 * i];
        b[i] = lo[2 * i + 1] - back[2 * i + 1];
    }
    t2 = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(a, b, exp2i(-5));
}

// split_q8 with the low half kept in f32 (the fp6 terms are taken from it).
__device__ inline void split_q8_f32(float (&x)[8], const float2 (&cs)[4], int u, int rope_pairs, float mul,
                                    half8 &hi, float *lo) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (4 * u + i < rope_pairs) rope_rotate(x[2 * i], x[2 * i + 1], cs[i]);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float v = opaque(x[kPerm[j]] * mul);
        const _Float16 h = (_Float16)v;
        hi[j] = h;
        lo[j] = v - (float)h;
    }
}

// Max / sum over the two lane halves (lanes l and l^32) that hold one column.
__device__ inline float half_max(float v) {
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float half_sum(float v) {
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Scores of one 64-key window for this lane's column, in place (sc[kb][4q + r] is key
// 32kb + qk_row_key(8q + 4h + r)), left relative to the running reference m_run:
// sc = x s_k - m_run (one FMA per score; softcap in between when on), causal mask, then the
// online-softmax state update.  The reference is raised only when the window breaks
// p <= 2^8 or p*s_v <= 2^15 (f16 range), and the scores move down with it; the first window
// (first, uniform; m_run = 0 and nothing accumulated yet) sets it from its own max.
template <int NDB, bool SOFTCAP>
__device__ inline void window_scores(floatx16 (&sc)[2], const float *sk, float svl, float softcap,
                                     bool mask, bool first, int base, int h, int qpos, float &m_run,
                                     float &l_run, floatx16 (&o)[NDB]) {
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const floatx4 sk4 = *reinterpret_cast<const floatx4 *>(sk + 32 * kb + 16 * (q >> 1) + 8 * h + 4 * (q & 1));
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float x;
                if constexpr (SOFTCAP) {
                    x = sc[kb][4 * q + r] * sk4[r];
                    x = tanhf(x / softcap) * softcap * kLog2e - m_run;
                } else {
                    x = __builtin_fmaf(sc[kb][4 * q + r], sk4[r], -m_run);
                }
                sc[kb][4 * q + r] = x;
            }
        }
    }
    if (mask) {
        // a real branch: only windows on the causal diagonal pay for the compares
        asm volatile("");
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (base + 32 * kb + 16 * (q >> 1) + 8 * h + 4 * (q & 1) + r > qpos) sc[kb][4 * q + r] = -INFINITY;
    }
    float mloc = kMinit;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int i = 0; i < 16; i++) mloc = fmaxf(mloc, sc[kb][i]);
    mloc = half_max(mloc);
    const float need = fmaxf(mloc - 8.0f, mloc + svl - 15.0f);  // relative to m_run
    if (__builtin_amdgcn_ballot_w64(first || need > 0.0f) != 0) {
        const float delta = (first || need > 0.0f) ? mloc + fmaxf(0.0f, svl - 15.0f) : 0.0f;
        if (!first) {
            const float alpha = exp2f(-delta);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; db++) o[db] *= alpha;
        }
        m_run += delta;
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int i = 0; i < 16; i++) sc[kb][i] = sc[kb][i] - delta;
    }
}

// Probabilities of 16-key step st (keys 16st + 8h + 0..7 of the window) times s_v, split
// hi + lo in f16 in the PV operand's slot order; adds the p to l_run.  p*s_v = hi + lo keeps
// ~22 bits: one f16 would carry a relative error of 2^-11 into the output whenever a few
// keys dominate the row.
__device__ inline void step_probs(const floatx16 (&sc)[2], const float *sv, int st, int h,
                                  float &l_run, half8 &pb, half8 &pl) {
    const int kb = st >> 1;
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
        const int q = 2 * (st & 1) + qq;
        const floatx4 sv4 = *reinterpret_cast<const floatx4 *>(sv + 32 * kb + 16 * (q >> 1) + 8 * h + 4 * (q & 1));
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = __builtin_amdgcn_exp2f(sc[kb][4 * q + r]);  // sc is relative
            l_run += p;
            // hi: the exact product p s_v rounded once to f16; lo: the exact remainder
            // p s_v - hi rounded once (both one fused multiply-add with an f16 result)
            const _Float16 hi = (_Float16)__builtin_fmaf(p, sv4[r], 0.0f);
            // key 16st + 8h + 4(q&1) + r: slot 2r + (q&1)
            pb[2 * r + (q & 1)] = hi;
            pl[2 * r + (q & 1)] = (_Float16)__builtin_fmaf(p, sv4[r], -(float)hi);
        }
    }
}

// PAD: the caller's head dim L.hdr is below the stored HD (q and output rows of hdr floats).
template <int HD, bool SOFTCAP, bool NORM, bool PAD>
__global__ __launch_bounds__(64 * kPrefillNW, HD > 128 ? 1 : 2) void prefill_kernel(PrefillArgs a) {
    constexpr int NW = kPrefillNW;
    constexpr int NKS = HD / 16;   // MFMA k-steps over the head dim
    constexpr int NDB = HD / 32;   // 32-dim output tiles
    constexpr int NG = NKS / 4;    // groups of 4 k-steps (one fp6 MFMA each)
    constexpr int ROWB = HD / 2;
    constexpr int COLS = NW * kColsPerWave;  // columns per block
    const KvLayerView &L = a.L;
    const float *const QN = NORM ? L.qn : nullptr;  // QK norm of q (compiled out when off)
    // Workgroups are dispatched round robin over the 8 XCDs by linear id.  Give XCD x the
    // contiguous range [x*N/8, (x+1)*N/8) of (column block, kv head, sequence) in row order, so
    // the 16-odd blocks that read one (sequence, kv head) stream share an L2 and every XCD gets
    // the same mix of long and short blocks.
    int xb = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
    {
        const int n_wg = gridDim.x * gridDim.y * gridDim.z;
        if (n_wg % 8 == 0) {
            const int id = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
            // Two workgroups share a CU.  The dispatch order within an XCD is reversed in
            // every second round of 32 (its CU count), so that a CU's two workgroups tend to
            // be one heavy (late-token) and one light block (4% faster on a 4 x 512-token
            // prefill).  The reversal is a permutation of the XCD's range.
            const int per = n_wg / 8;
            int k = id / 8;
            if ((k >> 5) & 1) {
                const int r0 = k & ~31, rl = min(32, per - r0);
                k = r0 + rl - 1 - (k - r0);
            }
            const int logical = (id % 8) * per + k;
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
    const int j = lane & 31, hf = lane >> 5;  // MFMA column / lane half
    const int len0 = a.len[s];
    // (dynamic: the hd-256 tiles take 128 KB)
    extern __shared__ __align__(16) unsigned char pf_smem[];
    PrefillLds<HD> &sm = *reinterpret_cast<PrefillLds<HD> *>(pf_smem);
    __shared__ float sm_qb[NW];

    const size_t row = (size_t)s * L.H + h;
    const uint8_t *kbase = L.kp + row * L.P * ROWB;
    const uint8_t *vbase = L.vp + row * (L.P / 32) * (HD * 16);
    const float *ksb = L.ks + row * L.P;
    const float *vsb = L.vs + row * L.P;
    const float qmul = SOFTCAP ? a.inv_sqrt_hd : a.inv_sqrt_hd * kLog2e;
    const int krow = qk_row_key(j);  // K row this lane feeds to the QK MFMA (within 32 keys)

    // Heavier column blocks (later tokens) first.
    const int cblk = n_blk - 1 - xb;
    const int c_blk = cblk * COLS;
    const int c_wave = c_blk + wave * kColsPerWave;
    const int c = c_wave + j;
    const bool live = c < n_cols;
    const int cc = live ? c : n_cols - 1;
    const int tok = cc / G;
    const int hdr = PAD ? L.hdr : HD;  // row length of q and the output (stored dims past it are 0)
    const float *qrow = a.q + (((size_t)s * a.n_tok + tok) * a.n_head + h * G + cc % G) * hdr;
    const int qpos = live ? len0 + tok : -1;

    // The first window's K and V loads go out before q is read.
    Pending<HD, NW> pd;
    const DeqConstV dk;
    fetch_window<HD, NW>(pd, kbase, vbase, ksb, vsb, 0, tid, wave);
    // Every workgroup reads its q rows at the start, all at once (33.5 MB for a 4 x 512-token
    // chunk of 32 heads), so the read is HBM-bound for several us.  When the whole grid runs in
    // one round, the blocks of the lighter half hold their reads back, the lightest longest
    // (a lighter block attends to fewer keys, so it still ends before the heavy ones), and the
    // heavy blocks, which set the launch's length, get their q sooner.
    if (a.q_delay > 0 && n_blk >= 2 && 2 * cblk < n_blk) {
        const int steps = (n_blk / 2 - cblk) * a.q_delay / (n_blk / 2);
        for (int i = 0; i < steps; i++) __builtin_amdgcn_s_sleep(32);  // 2048 clocks each
    }

    // q of this lane's column, read once: the QK norm scale (its q row walked in order), then
    // one power-of-two q scale per workgroup from a bound over all its columns, then the
    // rotation and the hi/lo split from the registers.
    const float ns = QN ? qk_norm_scale(qrow, hdr, L.norm_eps) : 1.0f;
    float q_s, inv_s;
    float xq[NKS][8];
    float2 cs[NKS][4];  // the rotation of each q pair, loaded beside q
    {
        const int qrot = rot_of(L, s, len0 + tok);
        float qb = 0.0f;
#pragma unroll
        for (int t = 0; t < NKS; t++) {
            q_read8(qrow, 2 * t + hf, QN, ns, xq[t], hdr);
            load_rot8(a.rope, a.rope_pairs, 2 * t + hf, qrot, cs[t]);
            // |a cos - b sin| <= |a| + |b|
            qb = fmaxf(qb, fmaxf(fmaxf(fabsf(xq[t][0]) + fabsf(xq[t][1]), fabsf(xq[t][2]) + fabsf(xq[t][3])),
                                 fmaxf(fabsf(xq[t][4]) + fabsf(xq[t][5]), fabsf(xq[t][6]) + fabsf(xq[t][7]))));
        }
        qb = wave_max(qb);
        if (lane == 0) sm_qb[wave] = qb;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; w++) qb = fmaxf(qb, sm_qb[w]);
        q_scale(qb * qmul, q_s, inv_s);
    }
    // q operands of this lane's column: k-step t holds dims 8(2t + hf) .. +7 in f16 (hi); the
    // rest as two fp6 terms per group of 4 k-steps.
    half8 qh[NKS];
    int6v ql1[NG], ql2[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) {
        float lo[32];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = 4 * g + u;
            split_q8_f32(xq[t], cs[t], 2 * t + hf, a.rope_pairs, qmul * q_s, qh[t], lo + 8 * u);
            if (!live) {
                qh[t] = (half8)(_Float16)0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) lo[8 * u + j] = 0.0f;
            }
        }
        q_lo_terms(lo, ql1[g], ql2[g]);
    }
    // Query positions this wave covers (inclusive); qmax < 0 for a wave with no columns.
    const int qmin_w = len0 + c_wave / G;
    const int qmax_w = c_wave < n_cols ? len0 + (min(c_wave + kColsPerWave, n_cols) - 1) / G : -1;
    // (clamped to the capacity: a graph replayed past it reads nothing past it)
    const int key_end = min(len0 + (min(c_blk + COLS, n_cols) - 1) / G + 1, L.P);
    const int n_win = (key_end + kWin - 1) / kWin;

    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++) o[db] = (floatx16)0.0f;
    float m_run = 0.0f, l_run = 0.0f;  // m_run: exp2 reference, set by the first window
    bool first = true;

    // Window w+1 is staged into LDS while window w's QK^T runs on the matrix cores (the
    // staging is VALU and LDS-write work); its global loads were issued one iteration earlier.
    stage_codes<HD, NW>(sm, 0, pd, tid, wave, dk);
    stage_scales<HD, NW>(sm, 0, pd, tid, inv_s);
    if (n_win > 1) fetch_window<HD, NW>(pd, kbase, vbase, ksb, vsb, kWin, tid, wave);
    __syncthreads();

    for (int w = 0; w < n_win; w++) {
        const int buf = w & 1, base = w * kWin;
        const bool more = w + 1 < n_win;
        // QK^T for both 32-key tiles, the two tiles' MFMAs alternating so that no MFMA waits
        // on the one just before it, with the next window's staging in between.  (A wave whose
        // columns all lie before the window computes scores it then drops: on the diagonal
        // only, and it keeps the staging in the MFMAs' basic block.)
        floatx16 sc[2] = {(floatx16)0.0f, (floatx16)0.0f};
        __builtin_amdgcn_s_setprio(3);
        using PD = Pending<HD, NW>;
        constexpr int NPART = PD::SPLIT ? 0 : 8 * PD::NK;  // staging parts, spread over k-steps
#pragma unroll
        for (int g = 0; g < NG; g++) {
            half8 ka0[4], ka1[4];
            ka0[0] = sm.k[buf][krow][k_slot<HD>(krow, 2 * (4 * g) + hf)];
            ka1[0] = sm.k[buf][32 + krow][k_slot<HD>(32 + krow, 2 * (4 * g) + hf)];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int t = 4 * g + u;
                if (u + 1 < 4) {
                    ka0[u + 1] = sm.k[buf][krow][k_slot<HD>(krow, 2 * (t + 1) + hf)];
                    ka1[u + 1] = sm.k[buf][32 + krow][k_slot<HD>(32 + krow, 2 * (t + 1) + hf)];
                }
                __builtin_amdgcn_sched_barrier(0);
                sc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka0[u], qh[t], sc[0], 0, 0, 0);
                sc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka1[u], qh[t], sc[1], 0, 0, 0);
                // (after the last window this writes the unused buffer)
                if constexpr (NPART > 0) {
#pragma unroll
                    for (int part = t * NPART / NKS; part < (t + 1) * NPART / NKS; part++)
                        stage_part<HD, NW>(sm, buf ^ 1, pd, tid, part, dk);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            // the low half of q over these 64 dims: the same codes as fp6
            const int6v k0 = fp6_of(ka0, 1.0f), k1 = fp6_of(ka1, 1.0f);
            sc[0] = mfma_lo6(k0, ql1[g], sc[0], kQlo1E8);
            sc[1] = mfma_lo6(k1, ql1[g], sc[1], kQlo1E8);
            sc[0] = mfma_lo6(k0, ql2[g], sc[0], kQlo2E8);
            sc[1] = mfma_lo6(k1, ql2[g], sc[1], kQlo2E8);
        }
        if constexpr (NPART == 0) stage_codes<HD, NW>(sm, buf ^ 1, pd, tid, wave, dk);
        __builtin_amdgcn_s_setprio(0);
        if (more) stage_scales<HD, NW>(sm, buf ^ 1, pd, tid, inv_s);
        if (w + 2 < n_win) fetch_window<HD, NW>(pd, kbase, vbase, ksb, vsb, base + 2 * kWin, tid, wave);
        if (base <= qmax_w) {
            const bool mask = base + kWin - 1 > qmin_w;  // some key of the window is masked
            window_scores<NDB, SOFTCAP>(sc, sm.sk[buf], sm.svlog[buf], a.softcap, mask, first,
                                        base, hf, qpos, m_run, l_run, o);
            first = false;
            // O^T += V^T P^T one 16-key step at a time: the exps of step st+1 overlap the
            // MFMAs of step st.
#pragma unroll
            for (int st = 0; st < 4; st++) {
                half8 pb, pl;  // p*s_v high and low f16 parts
                step_probs(sc, sm.sv[buf], st, hf, l_run, pb, pl);
                __builtin_amdgcn_s_setprio(2);
                half8 va[NDB];
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const int vr = 32 * db + j;
                    va[db] = sm.v[buf][vr][v_slot(vr, 2 * st + hf)];
                }
#pragma unroll
                for (int db = 0; db < NDB; db++) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[db], pb, o[db], 0, 0, 0);
#pragma unroll
                for (int db = 0; db < NDB; db++) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[db], pl, o[db], 0, 0, 0);
            }
            __builtin_amdgcn_s_setprio(0);
        }
        __syncthreads();
    }

    const float l = half_sum(l_run);
    if (live) {
        float *orow = a.out + (((size_t)s * a.n_tok + tok) * a.n_head + h * G + c % G) * hdr;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float4 v4 = make_float4(o[db][4 * q] * inv, o[db][4 * q + 1] * inv,
                                        o[db][4 * q + 2] * inv, o[db][4 * q + 3] * inv);
                if (32 * db + 8 * q + 4 * hf < hdr) *reinterpret_cast<float4 *>(orow + 32 * db + 8 * q + 4 * hf) = v4;
            }
    }
}

}  // namespace

hipError_t launch_prefill(const KvLayerView &L, const int32_t *d_len, const float *q,
                          int n_head, int n_tok, const float *rope, int rope_pairs,
                          float softcap, float *out, int n_cu, hipStream_t st) {
    PrefillArgs a;
    a.L = L;
    a.len = d_len;
    a.q = q;
    a.rope = rope;
    a.rope_pairs = rope_pairs;
    a.n_head = n_head;
    a.G = n_head / L.H;
    a.n_tok = n_tok;
    a.inv_sqrt_hd = 1.0f / sqrtf((float)L.hdr);
    a.softcap = softcap;
    a.out = out;
    const int n_cols = n_tok * a.G;
    const int cols = kPrefillNW * kColsPerWave;
    const int n_blk = (n_cols + cols - 1) / cols;
    dim3 grid(n_blk, L.H, L.S);
    // (the kernel fits two workgroups per CU below 256 dims, one at 256; measured on config
    // 5's shape: 8 sleep steps for the lightest block, +3.5%)
    const int64_t n_wg = (int64_t)n_blk * L.H * L.S;
    a.q_delay = n_wg <= (int64_t)n_cu * (L.hd > 128 ? 1 : 2) ? 8 : 0;
    const bool cap = softcap > 0.0f, norm = L.qn != nullptr;
#define TS_PF3(HDV, SC, NM, PD)                                                                          \
    {                                                                                                     \
        constexpr size_t lds = sizeof(PrefillLds<HDV>);                                                   \
        if (lds > 64 * 1024)                                                                              \
            (void)hipFuncSetAttribute((const void *)prefill_kernel<HDV, SC, NM, PD>,                      \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);              \
        prefill_kernel<HDV, SC, NM, PD><<<grid, 64 * kPrefillNW, lds, st>>>(a);                           \
    }
#define TS_PF2(HDV, PD)                                                                                    \
    {                                                                                                     \
        if (cap) { if (norm) TS_PF3(HDV, true, true, PD) else TS_PF3(HDV, true, false, PD) }              \
        else { if (norm) TS_PF3(HDV, false, true, PD) else TS_PF3(HDV, false, false, PD) }                \
    }
#define TS_PF(HDV) { if (L.hdr != L.hd) TS_PF2(HDV, true) else TS_PF2(HDV, false) }
    if (L.hd == 256)
        TS_PF(256)
    else if (L.hd == 128)
        TS_PF(128)
    else if (L.hd == 64)
        TS_PF(64)
    else
        return hipErrorInvalidValue;
#undef TS_PF
#undef TS_PF2
#undef TS_PF3
    return hipGetLastError();
}

}  // namespace ts
