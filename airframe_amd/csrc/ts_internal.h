// ts_internal.h -- shared definitions of the gfx950 INT4 KV-cache library (not part of the ABI).
//
// HBM layout of one layer (S sequences, H kv heads, P = max_seq rounded up to 64, hd dims):
//
//   K packed  [S][H][P/64][hd*32 bytes]        64-position windows.  Position p's row is the
//                                              reference's per-(pos, head) row (word u holds
//                                              dims 8u..8u+7, dim 8u+n in bits 4n..4n+3).  In
//                                              a window, row r = 4n + t (n < 16, t < 4) gives
//                                              lane L = 16 g + n the words 8m + 2g + i
//                                              (m < hd/64, i < 2) in lane order
//                                              q = (t*(hd/64) + m)*2 + i, and lane L's word q
//                                              sits at word 4 (64 (q/4) + L) + q%4 of the
//                                              window (k_word_idx)
//   V packed  [S][H][P/32][hd*16 bytes]        32-position blocks, "position-packed": word
//                                              (g, dl, td) of a block holds dim 16*td+dl at 8
//                                              positions (nibble n<4 -> position 4g+n, nibble
//                                              n>=4 -> position 16+4g+(n-4)); lane group
//                                              ln = g*16+dl owns words td = 0..hd/16-1, held in
//                                              16-byte chunks (td/4)*64 + ln (v_word_idx)
//   K scale   [S][H][P] f32
//   V scale   [S][H][P] f32
//
// Each (sequence, kv head) is one contiguous stream per buffer.  The chunk orders make every
// 16-byte load instruction of a decode wave read one contiguous kilobyte while each lane still
// receives exactly the data it feeds to the matrix cores: in K, the 16-dim slices (two words)
// that lane 16 g + n supplies to v_mfma_i32_16x16x64_i8 as column n (positions 4n + t) and
// k-group g; in V, the words of its own lane group.  Every V word is the 8 positions one lane
// feeds to one v_mfma_f32_16x16x32_f16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "../../include/turboshimmy.h"

namespace ts {

constexpr int kPosAlign = 64;  // P is a multiple of this (one decode window)

// Word index of K word u of position p, counted from the start of its (sequence, kv head)
// stream (the layout above).
template <int HD>
__host__ __device__ inline size_t k_word_idx(int p, int u) {
    const int r = p & 63, n = r >> 2, t = r & 3;
    const int g = (u & 7) >> 1, m = u >> 3, i = u & 1;
    const int q = ((t * (HD / 64) + m) << 1) + i;
    return (size_t)(p >> 6) * (HD * 8) + (size_t)((((q >> 2) << 6) + 16 * g + n) << 2) + (q & 3);
}

// Word index of V word (lane group ln = 16 g + dl, tile td) inside its 32-position block.
__host__ __device__ inline int v_word_idx(int ln, int td) { return ((((td >> 2) << 6) + ln) << 2) + (td & 3); }

struct KvLayerView {
    uint8_t *kp;  // K packed
    uint8_t *vp;  // V packed
    float *ks;    // K scales
    float *vs;    // V scales
    // Per sequence: window base (the shift total of all compactions) and sink count, or null
    // while no sequence has been compacted.  The K of slot p is stored rotated at rot_pos(p):
    // p for the sinks, p + window base otherwise.
    const int32_t *rot;
    const int32_t *sink;
    // QK norm of this layer (Qwen3): per-dim weights for q and K, or null (no norm), and eps
    const float *qn, *kn;
    float norm_eps;
    // hd: the stored head dim (64, 128 or 256: the kernels' template); hdr: the caller's head
    // dim (a multiple of 8, at most hd), the row length of q, K, V and outputs.  Stored dims
    // from hdr on hold code 8 (value 0).
    int S, H, P, hd, hdr;
};

__device__ __host__ inline int rot_pos(int p, int rot, int sink) { return p < sink ? p : p + rot; }

// Rotation position of slot p of sequence s (rot/sink are null while no sequence of the cache
// has been compacted, which saves the kernels two loads).
__device__ inline int rot_of(const KvLayerView &L, int s, int p) {
    return L.rot ? rot_pos(p, L.rot[s], L.sink[s]) : p;
}

}  // namespace ts

struct ts_kv {
    ts_kv_desc d;
    int P;                    // padded positions per (seq, head)
    uint64_t layer_bytes;
    uint8_t *base;            // one allocation for all layers
    int32_t *d_len;           // device mirror of lengths [n_seq], then window bases [n_seq]
                              // and sink counts [n_seq] (d_rot, d_sink), then d_adv
    int32_t *d_rot, *d_sink;
    int32_t *d_adv;           // arrival counter of a decode launch that advances the lengths
                              // (zero between launches)
    std::vector<int32_t> h_len, h_rot, h_sink;
    std::vector<const float *> q_norm, k_norm;  // per layer, device pointers or null
    std::vector<float> norm_eps;
    std::vector<int32_t> h_ctx;  // scratch for the decode plan: len + 1 per sequence
    // Set once a call that changes the device lengths was captured into a graph: replays of it
    // advance the device lengths without the host knowing, so decode launches read the device
    // lengths from then on instead of taking the host's as arguments.
    bool len_captured = false;
    int device;
    int n_cu;                    // compute units of the device (the decode plan's target)
    int hdp;                     // stored head dim (KvLayerView::hd)

    ts::KvLayerView layer(int l) const {
        ts::KvLayerView v;
        uint64_t nrow = (uint64_t)d.n_seq * d.n_head_kv * P;
        uint8_t *b = base + (uint64_t)l * layer_bytes;
        v.kp = b;
        v.vp = b + nrow * (hdp / 2);
        v.ks = (float *)(b + nrow * hdp);
        v.vs = v.ks + nrow;
        const bool compacted = std::any_of(h_rot.begin(), h_rot.end(), [](int32_t r) { return r != 0; });
        v.rot = compacted ? d_rot : nullptr;
        v.sink = compacted ? d_sink : nullptr;
        v.qn = q_norm[l];
        v.kn = k_norm[l];
        v.norm_eps = norm_eps[l];
        v.S = d.n_seq;
        v.H = d.n_head_kv;
        v.P = P;
        v.hd = hdp;
        v.hdr = d.head_dim;
        return v;
    }
};

struct ts_rope {
    float *d_table;  // [n_pos][rope_dim/2][2]
    int32_t n_pos;
    int32_t rope_dim;
};

namespace ts {

// Kernel launchers (defined in the .hip files).  All return hipError_t of the launch.
hipError_t launch_quantize_rows(const KvLayerView &L, const float *k, const float *v,
                                const int32_t *d_start, int32_t fixed_start, int32_t count,
                                int32_t ld_tok, const float *rope, int32_t rope_pairs,
                                int32_t max_blocks, hipStream_t st);
hipError_t launch_export(const KvLayerView &L, int seq, int pos0, int n_pos, uint32_t *kp,
                         uint32_t *vp, float *ks, float *vs, hipStream_t st);
hipError_t launch_import(const KvLayerView &L, int seq, int pos0, int n_pos, const uint32_t *kp,
                         const uint32_t *vp, const float *ks, const float *vs, hipStream_t st);
hipError_t launch_len_update(int32_t *d_len, int n, int32_t seq, int32_t value, int mode,
                             hipStream_t st);
// In-place compaction move of one sequence: slots [keep, keep + n_move) take slots
// [keep + shift, keep + shift + n_move), in ceil(n_move / shift) launches (rounds of shift slots,
// each reading only slots that later rounds no longer need).
hipError_t launch_shift_move(const KvLayerView &L, int seq, int keep, int shift, int n_move, hipStream_t st);

struct DecodePlan {
    int chunk;    // positions per split (multiple of 64)
    int n_split;  // splits of the longest sequence (grid.x)
    bool g4;      // the integer kernel, G <= 16 (QK^T on v_mfma_i32_16x16x64_i8)
    int nw;       // waves per workgroup of the 16x16 kernel (4, or 8 / 16 without a split)
};
// n_ctx: keys per sequence (len + 1), on the host; n_cu: compute units of the device;
// stored_hd: the stored head dim (64, 128 or 256); fused: the launch appends the new token
// (its position is scored from registers, not streamed).
DecodePlan decode_plan(const int32_t *n_ctx, int n_seq, int n_kv, int G, int n_cu, int stored_hd, bool fused);
// The integer kernel takes up to 16 query heads per kv head on stored rows up to 128 dims, 8 on
// 256-dim rows.
inline int decode_int_gmax(int stored_hd) { return stored_hd <= 128 ? 16 : 8; }
// Upper bound of plan.n_split for any lengths up to max_seq (sizes the workspace).
int decode_cap(int n_kv, int max_seq, int n_cu);
// adv: null, or the cache's arrival counter: the launch then also advances every length by
// one once all of its workgroups have read them (plans with a split: in the combine kernel;
// without: a length-update launch after the decode).  h_len: null, or the lengths of the n_seq
// sequences as the host knows them when they are known to match the device's (an eager
// call): with one sequence the kernels then take its length as an argument instead of reading
// d_len first.
hipError_t launch_decode(const KvLayerView &L, int32_t *d_len, const int32_t *h_len, const float *q, int n_head,
                         const float *rope, int rope_pairs, float softcap, float *out,
                         float *ws, const DecodePlan &plan, const float *k_new,
                         const float *v_new, int32_t *adv, hipStream_t st);
// n_cu: compute units of the device (the launch staggers its q reads when the grid fits them).
hipError_t launch_prefill(const KvLayerView &L, const int32_t *d_len, const float *q,
                          int n_head, int n_tok, const float *rope, int rope_pairs,
                          float softcap, float *out, int n_cu, hipStream_t st);

// Fused QKV projection + append (ts_qkv.hip): tiles and split of the reduction over dim.
struct QkvPlan {
    int RT, CT;           // row tiles, column tiles
    int kps, n_split;     // reduction length per split, splits
    bool big;             // one workgroup per 64-row tile over all of dim (else split)
    uint64_t part_bytes;  // scratch for the split partials (0 without a split)
};
QkvPlan qkv_plan(int n_seq, int n_kv, int n_head, int hd, int dim, int n_tok);
// GGUF block weights (Q4_K, Q5_K, Q8_0, Q4_0) read in the loop: always the split form (dim a multiple of
// 256), partials always in `part` (part_bytes > 0).
QkvPlan qkv_plan_kq(int n_seq, int n_kv, int n_head, int hd, int dim, int n_tok);
hipError_t launch_qkv_kq(const KvLayerView &L, const int32_t *d_len, const float *x, int dim, int n_tok,
                         int ggml_type, const void *wq, const void *wk, const void *wv, int n_head,
                         float *q_out, float *k_out, float *v_out, const float *rope, int rope_pairs,
                         const QkvPlan &plan, float *part, hipStream_t st);
hipError_t launch_qkv(const KvLayerView &L, const int32_t *d_len, const float *x, int dim, int n_tok,
                      const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int n_head,
                      float *q_out, float *k_out, float *v_out, const float *rope, int rope_pairs,
                      const QkvPlan &plan, float *part, int planes, hipStream_t st);

// Attention output projection (ts_proj.hip).
struct ProjPlan {
    int RT, CT, kps, n_split;
    uint64_t part_bytes;
};
ProjPlan proj_plan(int M, int K, int N);
ProjPlan proj_plan_kq(int M, int K, int N);  // block weights: split form, K a multiple of 256
hipError_t launch_proj_kq(const float *a, int M, int K, int ggml_type, const void *w, int N, float *act,
                          float *stash, const ProjPlan &plan, float *part, hipStream_t st);
hipError_t launch_proj(const float *a, int M, int K, const uint16_t *w, int N, float *act, float *stash,
                       const ProjPlan &plan, float *part, int planes, hipStream_t st);
hipError_t launch_fill_zero(float *p, size_t n, hipStream_t st);

}  // namespace ts
