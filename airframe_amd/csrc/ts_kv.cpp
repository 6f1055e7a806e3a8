// ts_kv.cpp -- host side of the C ABI: cache allocation and bookkeeping, RoPE table, argument
// checking and kernel dispatch.  Reference call surface: src/backend/bindless/kv_cache.rs
// (KVCache), pipeline/layer.rs:805-1246 (run_layer_with_cache_int4 / requantize_all_kv_int4),
// preflight.rs:28-142 (RoPE table).
#include <math.h>
#include <cmath>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <new>

#include "ts_internal.h"

namespace {

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// True when work enqueued on the stream now goes into a graph being captured.
static bool capturing(void *stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(as_stream(stream), &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}
// A call that changes the device lengths: note when it is being captured.
static void note_len_change(ts_kv *kv, void *stream) {
    if (capturing(stream)) kv->len_captured = true;
}

int hip_status(hipError_t e) { return e == hipSuccess ? TS_OK : TS_ERR_HIP; }

bool desc_valid(const ts_kv_desc *d) {
    return d && d->n_layers > 0 && d->n_seq > 0 && d->n_head_kv > 0 && d->head_dim > 0 &&
           d->max_seq > 0 && d->head_dim % 8 == 0;
}

// head_dim values the kernels take: any multiple of 8 up to 256, stored padded to 64, 128 or
// 256 dims (the reference accepts any multiple of 8: kv_cache.rs:150-156).
bool head_dim_built(int hd) { return hd % 8 == 0 && hd >= 8 && hd <= 256; }
int stored_head_dim(int hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : 256; }

int padded_positions(int max_seq) { return (max_seq + ts::kPosAlign - 1) / ts::kPosAlign * ts::kPosAlign; }

uint64_t layer_bytes_of(const ts_kv_desc *d) {
    return (uint64_t)d->n_seq * d->n_head_kv * padded_positions(d->max_seq) * (stored_head_dim(d->head_dim) + 8);
}

}  // namespace

extern "C" {

const char *ts_status_string(int status) {
    switch (status) {
        case TS_OK: return "ok";
        case TS_ERR_INVALID: return "invalid argument";
        case TS_ERR_OVERFLOW: return "KV cache overflow (context window exceeded)";
        case TS_ERR_UNSUPPORTED: return "unsupported configuration";
        case TS_ERR_HIP: return "HIP runtime error";
        case TS_ERR_NOMEM: return "device allocation failed";
        case TS_ERR_WORKSPACE: return "workspace too small";
        default: return "unknown status";
    }
}

// ---- RoPE ----------------------------------------------------------------------------------

// preflight.rs:71-111 (compute_rope_table), n_pos standing for the spec's n_ctx.  Per pair,
// in f32 with one rounding per operation (volatile keeps the compiler from fusing them):
// theta_i = 1 / base^(2i/rope_dim); with YaRN (scale < 1, 0 < alpha < beta; :82-84) the factor
// is (1 - ramp_i) scale + ramp_i, ramp_i = clamp((l_train / (2 pi / theta_i) - alpha) /
// (beta - alpha), 0, 1) with l_train = round(n_pos scale) (:77-81, :91-97); otherwise it is
// scale (:88-90).  Entry (pos, i) = (cos, sin)(pos * theta_i * factor_i).
int ts_rope_table_host_yarn(float *table, int32_t n_pos, int32_t rope_dim, float base, float scale,
                            float yarn_alpha, float yarn_beta) {
    if (!table || n_pos <= 0 || rope_dim <= 0 || (rope_dim & 1) || !(base > 0.0f) ||
        !(scale > 0.0f) || !std::isfinite(scale))
        return TS_ERR_INVALID;
    const int pairs = rope_dim / 2;
    const bool yarn = scale < 1.0f && yarn_alpha > 0.0f && yarn_beta > yarn_alpha;
    const float l_train = yarn ? (float)std::lround((float)n_pos * scale) : 0.0f;
    std::vector<float> theta(pairs);
    for (int i = 0; i < pairs; i++) {
        volatile float expo = (2.0f * (float)i) / (float)rope_dim;
        volatile float inv = 1.0f / powf(base, expo);
        float factor = scale;
        if (yarn) {
            volatile float wavelength = 6.2831855f / inv;  // 2 pi in f32
            volatile float x = l_train / wavelength;
            volatile float ramp = (x - yarn_alpha) / (yarn_beta - yarn_alpha);
            const float r = std::min(1.0f, std::max(0.0f, (float)ramp));
            volatile float unramped = (1.0f - r) * scale;
            factor = unramped + r;
        }
        theta[i] = inv * factor;
    }
    for (int p = 0; p < n_pos; p++) {
        float *row = table + (size_t)p * pairs * 2;
        for (int i = 0; i < pairs; i++) {
            volatile float angle = (float)p * theta[i];
            row[2 * i] = cosf(angle);
            row[2 * i + 1] = sinf(angle);
        }
    }
    return TS_OK;
}

int ts_rope_table_host(float *table, int32_t n_pos, int32_t rope_dim, float base, float scale) {
    return ts_rope_table_host_yarn(table, n_pos, rope_dim, base, scale, 0.0f, 0.0f);
}

int ts_rope_create(int32_t n_pos, int32_t rope_dim, float base, float scale, ts_rope **out) {
    return ts_rope_create_yarn(n_pos, rope_dim, base, scale, 0.0f, 0.0f, out);
}

int ts_rope_create_yarn(int32_t n_pos, int32_t rope_dim, float base, float scale, float yarn_alpha,
                        float yarn_beta, ts_rope **out) {
    if (!out) return TS_ERR_INVALID;
    *out = nullptr;
    std::vector<float> host;
    try {
        host.resize((size_t)std::max(n_pos, 1) * std::max(rope_dim, 2));
    } catch (...) {
        return TS_ERR_NOMEM;
    }
    int rc = ts_rope_table_host_yarn(host.data(), n_pos, rope_dim, base, scale, yarn_alpha, yarn_beta);
    if (rc) return rc;
    ts_rope *r = new (std::nothrow) ts_rope();
    if (!r) return TS_ERR_NOMEM;
    size_t bytes = (size_t)n_pos * rope_dim * sizeof(float);
    if (hipMalloc(&r->d_table, bytes) != hipSuccess) {
        delete r;
        return TS_ERR_NOMEM;
    }
    if (hipMemcpy(r->d_table, host.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) {
        hipFree(r->d_table);
        delete r;
        return TS_ERR_HIP;
    }
    r->n_pos = n_pos;
    r->rope_dim = rope_dim;
    *out = r;
    return TS_OK;
}

int ts_rope_destroy(ts_rope *rope) {
    if (!rope) return TS_ERR_INVALID;
    hipError_t e = hipFree(rope->d_table);
    delete rope;
    return hip_status(e);
}

int ts_rope_info(const ts_rope *rope, const float **d_table, int32_t *n_pos, int32_t *rope_dim) {
    if (!rope) return TS_ERR_INVALID;
    if (d_table) *d_table = rope->d_table;
    if (n_pos) *n_pos = rope->n_pos;
    if (rope_dim) *rope_dim = rope->rope_dim;
    return TS_OK;
}

// ---- cache -----------------------------------------------------------------------------------

// The kernels move f32 rows in 16-byte pieces.
static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Largest rotation position (exclusive) the next n_tok tokens of any sequence use: slots past
// the sinks are rotated at slot + window base.
static int64_t rot_end(const ts_kv *kv, int32_t n_tok) {
    int64_t m = 0;
    for (int s = 0; s < kv->d.n_seq; s++) m = std::max<int64_t>(m, (int64_t)kv->h_len[s] + kv->h_rot[s] + n_tok);
    return m;
}

int ts_kv_bytes(const ts_kv_desc *desc, uint64_t *bytes) {
    if (!desc_valid(desc) || !bytes) return TS_ERR_INVALID;
    if (!head_dim_built(desc->head_dim)) return TS_ERR_UNSUPPORTED;
    *bytes = layer_bytes_of(desc) * (uint64_t)desc->n_layers;
    return TS_OK;
}

int ts_kv_create(const ts_kv_desc *desc, ts_kv **out) {
    if (!out) return TS_ERR_INVALID;
    *out = nullptr;
    if (!desc_valid(desc)) return TS_ERR_INVALID;
    if (!head_dim_built(desc->head_dim)) return TS_ERR_UNSUPPORTED;
    ts_kv *kv = new (std::nothrow) ts_kv();
    if (!kv) return TS_ERR_NOMEM;
    kv->d = *desc;
    kv->P = padded_positions(desc->max_seq);
    kv->layer_bytes = layer_bytes_of(desc);
    kv->hdp = stored_head_dim(desc->head_dim);
    kv->h_len.assign(desc->n_seq, 0);
    kv->h_rot.assign(desc->n_seq, 0);
    kv->h_sink.assign(desc->n_seq, 0);
    kv->q_norm.assign(desc->n_layers, nullptr);
    kv->k_norm.assign(desc->n_layers, nullptr);
    kv->norm_eps.assign(desc->n_layers, 1e-6f);
    if (hipGetDevice(&kv->device) != hipSuccess ||
        hipDeviceGetAttribute(&kv->n_cu, hipDeviceAttributeMultiprocessorCount, kv->device) != hipSuccess ||
        kv->n_cu <= 0) {
        delete kv;
        return TS_ERR_HIP;
    }
    kv->h_ctx.assign(desc->n_seq, 0);
    uint64_t total = kv->layer_bytes * (uint64_t)desc->n_layers;
    if (hipMalloc(&kv->base, total) != hipSuccess) {
        delete kv;
        return TS_ERR_NOMEM;
    }
    const size_t len_ints = 3 * (size_t)desc->n_seq + 4;  // lengths, bases, sinks, arrival counter
    if (hipMalloc(&kv->d_len, sizeof(int32_t) * len_ints) != hipSuccess) {
        hipFree(kv->base);
        delete kv;
        return TS_ERR_NOMEM;
    }
    // Zero fill once at creation: unwritten positions then dequantize to finite values.
    if (hipMemset(kv->base, 0, total) != hipSuccess ||
        hipMemset(kv->d_len, 0, sizeof(int32_t) * len_ints) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        hipFree(kv->base);
        hipFree(kv->d_len);
        delete kv;
        return TS_ERR_HIP;
    }
    kv->d_rot = kv->d_len + desc->n_seq;
    kv->d_sink = kv->d_len + 2 * desc->n_seq;
    kv->d_adv = kv->d_len + 3 * desc->n_seq;
    *out = kv;
    return TS_OK;
}

int ts_kv_destroy(ts_kv *kv) {
    if (!kv) return TS_ERR_INVALID;
    hipError_t e1 = hipFree(kv->base);
    hipError_t e2 = hipFree(kv->d_len);
    delete kv;
    return (e1 == hipSuccess && e2 == hipSuccess) ? TS_OK : TS_ERR_HIP;
}

int ts_kv_desc_get(const ts_kv *kv, ts_kv_desc *desc) {
    if (!kv || !desc) return TS_ERR_INVALID;
    *desc = kv->d;
    return TS_OK;
}

int ts_kv_seq_len(const ts_kv *kv, int32_t seq, int32_t *len) {
    if (!kv || !len || seq < 0 || seq >= kv->d.n_seq) return TS_ERR_INVALID;
    *len = kv->h_len[seq];
    return TS_OK;
}

int ts_kv_max_len(const ts_kv *kv, int32_t *max_len) {
    if (!kv || !max_len) return TS_ERR_INVALID;
    *max_len = kv->d.max_seq;
    return TS_OK;
}

int ts_kv_increment(ts_kv *kv, int32_t n_tok, void *stream) {
    if (!kv || n_tok < 0) return TS_ERR_INVALID;
    for (int32_t l : kv->h_len)
        if ((int64_t)l + n_tok > kv->d.max_seq) return TS_ERR_OVERFLOW;
    if (n_tok == 0) return TS_OK;
    note_len_change(kv, stream);
    hipError_t e = ts::launch_len_update(kv->d_len, kv->d.n_seq, -1, n_tok, 0, as_stream(stream));
    if (e != hipSuccess) return TS_ERR_HIP;
    for (auto &l : kv->h_len) l += n_tok;
    return TS_OK;
}

int ts_kv_set_seq_len(ts_kv *kv, int32_t seq, int32_t len, void *stream) {
    if (!kv || seq < 0 || seq >= kv->d.n_seq || len < 0) return TS_ERR_INVALID;
    if (len > kv->d.max_seq) return TS_ERR_OVERFLOW;
    note_len_change(kv, stream);
    hipError_t e = ts::launch_len_update(kv->d_len, kv->d.n_seq, seq, len, 1, as_stream(stream));
    if (e != hipSuccess) return TS_ERR_HIP;
    kv->h_len[seq] = len;
    return TS_OK;
}

int ts_kv_reset(ts_kv *kv, void *stream) {
    if (!kv) return TS_ERR_INVALID;
    // lengths, window bases and sink counts: 3 n_seq consecutive ints
    note_len_change(kv, stream);
    hipError_t e = ts::launch_len_update(kv->d_len, 3 * kv->d.n_seq, -1, 0, 1, as_stream(stream));
    if (e != hipSuccess) return TS_ERR_HIP;
    std::fill(kv->h_len.begin(), kv->h_len.end(), 0);
    std::fill(kv->h_rot.begin(), kv->h_rot.end(), 0);
    std::fill(kv->h_sink.begin(), kv->h_sink.end(), 0);
    return TS_OK;
}

int ts_kv_reset_seq(ts_kv *kv, int32_t seq, void *stream) {
    if (!kv || seq < 0 || seq >= kv->d.n_seq) return TS_ERR_INVALID;
    hipStream_t st = as_stream(stream);
    note_len_change(kv, stream);
    hipError_t e = ts::launch_len_update(kv->d_len, kv->d.n_seq, seq, 0, 1, st);
    if (e == hipSuccess) e = ts::launch_len_update(kv->d_rot, kv->d.n_seq, seq, 0, 1, st);
    if (e == hipSuccess) e = ts::launch_len_update(kv->d_sink, kv->d.n_seq, seq, 0, 1, st);
    if (e != hipSuccess) return TS_ERR_HIP;
    kv->h_len[seq] = 0;
    kv->h_rot[seq] = 0;
    kv->h_sink[seq] = 0;
    return TS_OK;
}

int ts_kv_set_qk_norm(ts_kv *kv, int32_t layer, const float *d_q_norm, const float *d_k_norm,
                      float eps) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers || !(eps >= 0.0f) || !(eps < 1e30f) ||
        !aligned16(d_q_norm) || !aligned16(d_k_norm))
        return TS_ERR_INVALID;
    kv->q_norm[layer] = d_q_norm;
    kv->k_norm[layer] = d_k_norm;
    kv->norm_eps[layer] = eps;
    return TS_OK;
}

int ts_kv_window_base(const ts_kv *kv, int32_t seq, int32_t *base) {
    if (!kv || !base || seq < 0 || seq >= kv->d.n_seq) return TS_ERR_INVALID;
    *base = kv->h_rot[seq];
    return TS_OK;
}

int ts_kv_advance_window_base(ts_kv *kv, int32_t seq, int32_t shift_amt, void *stream) {
    if (!kv || seq < 0 || seq >= kv->d.n_seq || shift_amt < 0) return TS_ERR_INVALID;
    if ((int64_t)kv->h_rot[seq] + shift_amt > INT32_MAX / 2) return TS_ERR_OVERFLOW;
    if (shift_amt == 0) return TS_OK;
    note_len_change(kv, stream);
    hipError_t e = ts::launch_len_update(kv->d_rot, kv->d.n_seq, seq, shift_amt, 0, as_stream(stream));
    if (e != hipSuccess) return TS_ERR_HIP;
    kv->h_rot[seq] += shift_amt;
    return TS_OK;
}

int ts_kv_shift_workspace(const ts_kv *kv, uint64_t *bytes) {
    if (!kv || !bytes) return TS_ERR_INVALID;
    // positions x heads x (K and V words, two scales), reference layout
    *bytes = (uint64_t)kv->d.max_seq * kv->d.n_head_kv * (kv->d.head_dim + 8);
    return TS_OK;
}

int ts_kv_shift(ts_kv *kv, int32_t layer, int32_t seq, int32_t keep_sink, int32_t shift_amt,
                void *d_workspace, uint64_t workspace_bytes, void *stream) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers || seq < 0 || seq >= kv->d.n_seq ||
        keep_sink < 0 || shift_amt < 0 || keep_sink > kv->d.max_seq)
        return TS_ERR_INVALID;
    // one sink count per sequence: the slots below it are never moved, so their K keeps the
    // rotation of its own position
    if ((kv->h_sink[seq] != 0 || kv->h_rot[seq] != 0) && kv->h_sink[seq] != keep_sink)
        return TS_ERR_INVALID;
    // Every argument check runs before the sink count is recorded, so a refused call leaves
    // the cache as it was.  The move runs in place, in rounds of shift_amt slots (each one
    // launch), when there are few of them; a short shift of a long window goes through the
    // workspace instead (export the moved slots in the reference layout, import them at their
    // new place), and only that path needs the workspace.
    constexpr int64_t kMaxRounds = 8;
    const int64_t n_move = (int64_t)kv->h_len[seq] - keep_sink - shift_amt;
    const bool moves = n_move > 0 && shift_amt > 0;  // elements_to_shift == 0: nothing moves
    const bool in_place = moves && (n_move + shift_amt - 1) / shift_amt <= kMaxRounds;
    const uint64_t wpp = (uint64_t)kv->d.n_head_kv * (kv->d.head_dim / 8);  // words per position
    if (moves && !in_place) {
        const uint64_t need = (uint64_t)n_move * kv->d.n_head_kv * (kv->d.head_dim + 8);
        if (!d_workspace || workspace_bytes < need) return TS_ERR_WORKSPACE;
        if (!aligned16(d_workspace)) return TS_ERR_INVALID;
    }
    hipStream_t st = as_stream(stream);
    // The first call records the sink count, also when nothing moves, so that a caller who
    // advances the window base after every shift (as the reference's caller does) keeps the
    // sinks at their own rotation.
    if (kv->h_sink[seq] != keep_sink) {
        hipError_t e = ts::launch_len_update(kv->d_sink, kv->d.n_seq, seq, keep_sink, 1, st);
        if (e != hipSuccess) return TS_ERR_HIP;
        kv->h_sink[seq] = keep_sink;
    }
    if (!moves) return TS_OK;
    const ts::KvLayerView L = kv->layer(layer);
    if (in_place) return hip_status(ts::launch_shift_move(L, seq, keep_sink, shift_amt, (int)n_move, st));
    uint32_t *kp = (uint32_t *)d_workspace, *vp = kp + n_move * wpp;
    float *ks = (float *)(vp + n_move * wpp), *vs = ks + n_move * kv->d.n_head_kv;
    hipError_t e = ts::launch_export(L, seq, keep_sink + shift_amt, (int)n_move, kp, vp, ks, vs, st);
    if (e == hipSuccess) e = ts::launch_import(L, seq, keep_sink, (int)n_move, kp, vp, ks, vs, st);
    return hip_status(e);
}

int ts_kv_export(const ts_kv *kv, int32_t layer, int32_t seq, int32_t pos0, int32_t n_pos,
                 uint32_t *d_k_packed, uint32_t *d_v_packed, float *d_k_scale, float *d_v_scale,
                 void *stream) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers || seq < 0 || seq >= kv->d.n_seq ||
        pos0 < 0 || n_pos < 0 || (int64_t)pos0 + n_pos > kv->d.max_seq || !d_k_packed ||
        !d_v_packed || !d_k_scale || !d_v_scale)
        return TS_ERR_INVALID;
    if (n_pos == 0) return TS_OK;
    return hip_status(ts::launch_export(kv->layer(layer), seq, pos0, n_pos, d_k_packed,
                                        d_v_packed, d_k_scale, d_v_scale, as_stream(stream)));
}

// ---- hot path --------------------------------------------------------------------------------

static int check_rope(const ts_rope *rope, int hd, int64_t max_pos_exclusive) {
    if (!rope) return TS_ERR_INVALID;
    if (rope->rope_dim > hd) return TS_ERR_INVALID;
    if (max_pos_exclusive > rope->n_pos) return TS_ERR_INVALID;
    return TS_OK;
}


int ts_append_quant(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v, int32_t n_tok,
                    const ts_rope *rope, void *stream) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers || !aligned16(d_k) || !aligned16(d_v) || !d_k ||
        !d_v || n_tok < 0)
        return TS_ERR_INVALID;
    int32_t max_len = *std::max_element(kv->h_len.begin(), kv->h_len.end());
    if ((int64_t)max_len + n_tok > kv->d.max_seq) return TS_ERR_OVERFLOW;
    int rc = check_rope(rope, kv->d.head_dim, rot_end(kv, n_tok));
    if (rc) return rc;
    if (n_tok == 0) return TS_OK;
    // Blocks of 32 positions touched by [len, len+n_tok): at most n_tok/32 + 2.
    int32_t max_blocks = n_tok / 32 + 2;
    return hip_status(ts::launch_quantize_rows(kv->layer(layer), d_k, d_v, kv->d_len, 0, n_tok,
                                               n_tok, rope->d_table, rope->rope_dim / 2,
                                               max_blocks, as_stream(stream)));
}

int ts_requant_all(ts_kv *kv, int32_t layer, const float *d_k_cache, const float *d_v_cache,
                   int32_t seq_len, int32_t ld_pos, const ts_rope *rope, void *stream) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers || !d_k_cache || !d_v_cache || seq_len < 0 ||
        ld_pos < seq_len || !aligned16(d_k_cache) || !aligned16(d_v_cache))
        return TS_ERR_INVALID;
    if (seq_len > kv->d.max_seq) return TS_ERR_OVERFLOW;
    if (rope) {
        int32_t max_rot = *std::max_element(kv->h_rot.begin(), kv->h_rot.end());
        int rc = check_rope(rope, kv->d.head_dim, (int64_t)seq_len + max_rot);
        if (rc) return rc;
    }
    if (seq_len == 0) return TS_OK;
    int32_t blocks = (seq_len + 31) / 32;
    // K is taken as given: the reference normalizes its f32 cache before requantizing, so the
    // layer's QK norm is not applied again
    ts::KvLayerView L = kv->layer(layer);
    L.qn = L.kn = nullptr;
    return hip_status(ts::launch_quantize_rows(L, d_k_cache, d_v_cache, nullptr, 0,
                                               seq_len, ld_pos, rope ? rope->d_table : nullptr,
                                               rope ? rope->rope_dim / 2 : 0, blocks,
                                               as_stream(stream)));
}

// Any GQA group size: the decode takes more than 8 query heads per kv head as several head
// groups (each reads the kv head's stream).
static bool heads_ok(const ts_kv *kv, int32_t n_head) {
    return n_head > 0 && n_head % kv->d.n_head_kv == 0;
}

int ts_attn_decode_workspace(const ts_kv *kv, int32_t n_head, uint64_t *bytes) {
    if (!kv || !bytes || !heads_ok(kv, n_head)) return TS_ERR_INVALID;
    const int cap = ts::decode_cap(kv->d.n_head_kv, kv->d.max_seq, kv->n_cu);
    *bytes = (uint64_t)kv->d.n_seq * n_head * cap * (kv->hdp + 2) * sizeof(float);
    return TS_OK;
}

// Shared by ts_attn_decode, ts_attn_decode_append and ts_attn_decode_append_noalloc
// (k_new/v_new null for the first).  d_workspace: the caller's workspace of workspace_bytes,
// checked against the worst case the workspace query promises; or, with noalloc, the
// library's scratch array, checked against what this call's plan needs.
static int attn_decode(const ts_kv *kv, int32_t layer, const float *d_q, int32_t n_head,
                       const ts_rope *rope, float softcap, float *d_out, void *d_workspace,
                       uint64_t workspace_bytes, const float *k_new, const float *v_new,
                       void *stream, bool noalloc = false, bool advance = false) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers || !d_q || !d_out || !heads_ok(kv, n_head) ||
        !(softcap >= 0.0f) || !aligned16(d_q) || !aligned16(d_out))
        return TS_ERR_INVALID;
    int32_t max_len = *std::max_element(kv->h_len.begin(), kv->h_len.end());
    if (max_len + 1 > kv->d.max_seq) return TS_ERR_OVERFLOW;
    int rc = check_rope(rope, kv->d.head_dim, rot_end(kv, 1));
    if (rc) return rc;
    std::vector<int32_t> &ctx = const_cast<ts_kv *>(kv)->h_ctx;
    for (int s = 0; s < kv->d.n_seq; s++) ctx[s] = kv->h_len[s] + 1;
    ts::DecodePlan plan = ts::decode_plan(ctx.data(), kv->d.n_seq, kv->d.n_head_kv, n_head / kv->d.n_head_kv,
                                          kv->n_cu, kv->hdp, k_new != nullptr);
    if (plan.n_split > 1) {
        uint64_t need = 0;
        if (noalloc)  // partials [S][n_head][n_split][hd], then m and l [S][n_head][n_split]
            need = (uint64_t)kv->d.n_seq * n_head * plan.n_split * (kv->hdp + 2) * sizeof(float);
        else  // plan.n_split <= decode_cap(max_seq), the count the workspace was sized for
            ts_attn_decode_workspace(kv, n_head, &need);
        if (!d_workspace || workspace_bytes < need) return TS_ERR_WORKSPACE;
        if (!aligned16(d_workspace)) return TS_ERR_INVALID;
    }
    // An eager call takes the host's lengths as launch arguments (the device's agree with them
    // unless a captured call changed them); one being captured reads the device lengths, so
    // that replays see the lengths of their time.
    ts_kv *mkv = const_cast<ts_kv *>(kv);
    const bool cap = capturing(stream);
    if (cap && advance) mkv->len_captured = true;
    const int32_t *h_len = cap || kv->len_captured ? nullptr : kv->h_len.data();
    const int rc2 = hip_status(ts::launch_decode(kv->layer(layer), kv->d_len, h_len, d_q, n_head, rope->d_table,
                                                 rope->rope_dim / 2, softcap, d_out, (float *)d_workspace,
                                                 plan, k_new, v_new, advance ? kv->d_adv : nullptr,
                                                 as_stream(stream)));
    if (rc2 == TS_OK && advance)
        for (auto &l : const_cast<ts_kv *>(kv)->h_len) l += 1;
    return rc2;
}

int ts_attn_decode(const ts_kv *kv, int32_t layer, const float *d_q, int32_t n_head,
                   const ts_rope *rope, float softcap, float *d_out, void *d_workspace,
                   uint64_t workspace_bytes, void *stream) {
    return attn_decode(kv, layer, d_q, n_head, rope, softcap, d_out, d_workspace, workspace_bytes,
                       nullptr, nullptr, stream);
}

int ts_attn_decode_append(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v,
                          const float *d_q, int32_t n_head, const ts_rope *rope, float softcap,
                          float *d_out, void *d_workspace, uint64_t workspace_bytes, void *stream) {
    if (!d_k || !d_v || !aligned16(d_k) || !aligned16(d_v)) return TS_ERR_INVALID;
    return attn_decode(kv, layer, d_q, n_head, rope, softcap, d_out, d_workspace, workspace_bytes,
                       d_k, d_v, stream);
}

int ts_attn_decode_append_advance(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v,
                                  const float *d_q, int32_t n_head, const ts_rope *rope, float softcap,
                                  float *d_out, void *d_workspace, uint64_t workspace_bytes, void *stream) {
    if (!d_k || !d_v || !aligned16(d_k) || !aligned16(d_v)) return TS_ERR_INVALID;
    return attn_decode(kv, layer, d_q, n_head, rope, softcap, d_out, d_workspace, workspace_bytes,
                       d_k, d_v, stream, false, true);
}

// ---- allocation-free decode ----------------------------------------------------------------
//
// The split partials of ts_attn_decode_append_noalloc live in `scratch`, a file-scope device
// array: every GPU the library runs on holds one copy until the process ends, and every call
// on that GPU shares it (calls that overlap on one GPU race).  Nothing in it has to start at
// zero: each call writes every partial it reads.  Host code never uses the array's name as an
// address; the address comes from hipGetSymbolAddress, once per device.

namespace {
constexpr uint64_t kScratchBytes = 8ull << 20;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// This device's copy of `scratch` (the current device's; looked up on its first use).
int scratch_ptr(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TS_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TS_ERR_HIP;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TS_OK;
}
}  // namespace

int ts_attn_decode_append_noalloc(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v,
                                  const float *d_q, int32_t n_head, const ts_rope *rope, float softcap,
                                  float *d_out, void *stream) {
    if (!d_k || !d_v || !aligned16(d_k) || !aligned16(d_v)) return TS_ERR_INVALID;
    void *ws = nullptr;
    int rc = scratch_ptr(&ws);
    if (rc) return rc;
    return attn_decode(kv, layer, d_q, n_head, rope, softcap, d_out, ws, kScratchBytes, d_k, d_v, stream,
                       true);
}

int ts_attn_prefill(const ts_kv *kv, int32_t layer, const float *d_q, int32_t n_head,
                    int32_t n_tok, const ts_rope *rope, float softcap, float *d_out,
                    void *stream) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers || !d_q || !d_out || !heads_ok(kv, n_head) ||
        n_tok < 0 || !(softcap >= 0.0f) || !aligned16(d_q) || !aligned16(d_out))
        return TS_ERR_INVALID;
    int32_t max_len = *std::max_element(kv->h_len.begin(), kv->h_len.end());
    if ((int64_t)max_len + n_tok > kv->d.max_seq) return TS_ERR_OVERFLOW;
    int rc = check_rope(rope, kv->d.head_dim, rot_end(kv, n_tok));
    if (rc) return rc;
    if (n_tok == 0) return TS_OK;
    return hip_status(ts::launch_prefill(kv->layer(layer), kv->d_len, d_q, n_head, n_tok,
                                         rope->d_table, rope->rope_dim / 2, softcap, d_out,
                                         kv->n_cu, as_stream(stream)));
}

static bool qkv_shape_ok(const ts_kv *kv, int32_t dim, int32_t n_tok, int32_t n_head) {
    return dim > 0 && dim % 64 == 0 && n_tok >= 0 && heads_ok(kv, n_head);
}

// head_dim 64 and 128 run the fused kernel (ts_qkv.hip, the append as its epilogue); any other
// head_dim runs the projection kernel three times (q, K, V, each onto zeroed outputs: 0 + dot
// is the dot) and then the append kernel on the projected K and V.
static bool qkv_fused(const ts_kv *kv) { return kv->d.head_dim == 128 || kv->d.head_dim == 64; }

struct QkvGeneric {
    ts::ProjPlan pq, pk;
    uint64_t part_bytes;  // split partials, shared by the three projections (256-aligned)
    uint64_t kv_elems;    // floats of one of K / V: n_seq * n_tok * n_head_kv * head_dim
};

static QkvGeneric qkv_generic_plan(const ts_kv *kv, int32_t dim, int32_t n_tok, int32_t n_head, int planes) {
    QkvGeneric g;
    const int M = kv->d.n_seq * n_tok, hd = kv->d.head_dim;
    g.pq = ts::proj_plan(M, planes * dim, n_head * hd);
    g.pk = ts::proj_plan(M, planes * dim, kv->d.n_head_kv * hd);
    g.part_bytes = (std::max(g.pq.part_bytes, g.pk.part_bytes) + 255) / 256 * 256;
    g.kv_elems = (uint64_t)M * kv->d.n_head_kv * hd;
    return g;
}

int ts_qkv_workspace(const ts_kv *kv, int32_t dim, int32_t n_tok, int32_t n_head, uint64_t *bytes) {
    if (!kv || !bytes) return TS_ERR_INVALID;
    if (!qkv_shape_ok(kv, dim, n_tok, n_head)) return TS_ERR_INVALID;
    // enough for f16 rows and for two-plane rows (ts_qkv_append_x2); on the unfused path also
    // room for the projected K and V when the caller does not take them
    *bytes = 0;
    for (int planes = 1; n_tok > 0 && planes <= 2; planes++) {
        if (qkv_fused(kv)) {
            *bytes = std::max(*bytes, ts::qkv_plan(kv->d.n_seq, kv->d.n_head_kv, n_head, kv->d.head_dim,
                                                   planes * dim, n_tok).part_bytes);
        } else {
            const QkvGeneric g = qkv_generic_plan(kv, dim, n_tok, n_head, planes);
            *bytes = std::max(*bytes, g.part_bytes + 2 * g.kv_elems * sizeof(float));
        }
    }
    return TS_OK;
}

static int qkv_append_planes(ts_kv *kv, int32_t layer, const float *d_x, int32_t dim, int32_t n_tok,
                             const uint16_t *d_wq, const uint16_t *d_wk, const uint16_t *d_wv, int32_t n_head,
                             const ts_rope *rope, float *d_q, float *d_k, float *d_v, void *d_workspace,
                             uint64_t workspace_bytes, void *stream, int planes) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers) return TS_ERR_INVALID;
    if (!qkv_shape_ok(kv, dim, n_tok, n_head) || !d_x || !d_wq || !d_wk || !d_wv || !d_q ||
        !aligned16(d_x) || !aligned16(d_wq) || !aligned16(d_wk) || !aligned16(d_wv) ||
        !aligned16(d_q) || (!d_k) != (!d_v) || (d_k && (!aligned16(d_k) || !aligned16(d_v))))
        return TS_ERR_INVALID;
    int32_t max_len = *std::max_element(kv->h_len.begin(), kv->h_len.end());
    if ((int64_t)max_len + n_tok > kv->d.max_seq) return TS_ERR_OVERFLOW;
    int rc = check_rope(rope, kv->d.head_dim, rot_end(kv, n_tok));
    if (rc) return rc;
    if (n_tok == 0) return TS_OK;
    if (!qkv_fused(kv)) {
        const QkvGeneric g = qkv_generic_plan(kv, dim, n_tok, n_head, planes);
        const uint64_t need = g.part_bytes + (d_k ? 0 : 2 * g.kv_elems * sizeof(float));
        if (need > 0 && (!d_workspace || workspace_bytes < need || !aligned16(d_workspace))) return TS_ERR_WORKSPACE;
        float *part = static_cast<float *>(d_workspace);
        float *kb = d_k ? d_k : reinterpret_cast<float *>(static_cast<uint8_t *>(d_workspace) + g.part_bytes);
        float *vb = d_k ? d_v : kb + g.kv_elems;
        const hipStream_t st = as_stream(stream);
        const int M = kv->d.n_seq * n_tok, hd = kv->d.head_dim, H = kv->d.n_head_kv;
        hipError_t e = ts::launch_fill_zero(d_q, (size_t)M * n_head * hd, st);
        if (e == hipSuccess) e = ts::launch_fill_zero(kb, g.kv_elems, st);
        if (e == hipSuccess) e = ts::launch_fill_zero(vb, g.kv_elems, st);
        if (e == hipSuccess) e = ts::launch_proj(d_x, M, dim, d_wq, n_head * hd, d_q, nullptr, g.pq, part, planes, st);
        if (e == hipSuccess) e = ts::launch_proj(d_x, M, dim, d_wk, H * hd, kb, nullptr, g.pk, part, planes, st);
        if (e == hipSuccess) e = ts::launch_proj(d_x, M, dim, d_wv, H * hd, vb, nullptr, g.pk, part, planes, st);
        if (e == hipSuccess)
            e = ts::launch_quantize_rows(kv->layer(layer), kb, vb, kv->d_len, 0, n_tok, n_tok, rope->d_table,
                                         rope->rope_dim / 2, n_tok / 32 + 2, st);
        return hip_status(e);
    }
    const ts::QkvPlan plan = ts::qkv_plan(kv->d.n_seq, kv->d.n_head_kv, n_head, kv->d.head_dim, planes * dim, n_tok);
    if (plan.part_bytes > 0 && (!d_workspace || workspace_bytes < plan.part_bytes || !aligned16(d_workspace)))
        return TS_ERR_WORKSPACE;
    return hip_status(ts::launch_qkv(kv->layer(layer), kv->d_len, d_x, dim, n_tok, d_wq, d_wk, d_wv,
                                     n_head, d_q, d_k, d_v, rope->d_table, rope->rope_dim / 2, plan,
                                     static_cast<float *>(d_workspace), planes, as_stream(stream)));
}

int ts_qkv_append(ts_kv *kv, int32_t layer, const float *d_x, int32_t dim, int32_t n_tok,
                  const uint16_t *d_wq, const uint16_t *d_wk, const uint16_t *d_wv, int32_t n_head,
                  const ts_rope *rope, float *d_q, float *d_k, float *d_v, void *d_workspace,
                  uint64_t workspace_bytes, void *stream) {
    return qkv_append_planes(kv, layer, d_x, dim, n_tok, d_wq, d_wk, d_wv, n_head, rope, d_q, d_k, d_v,
                             d_workspace, workspace_bytes, stream, 1);
}

int ts_qkv_append_x2(ts_kv *kv, int32_t layer, const float *d_x, int32_t dim, int32_t n_tok,
                     const uint16_t *d_wq, const uint16_t *d_wk, const uint16_t *d_wv, int32_t n_head,
                     const ts_rope *rope, float *d_q, float *d_k, float *d_v, void *d_workspace,
                     uint64_t workspace_bytes, void *stream) {
    return qkv_append_planes(kv, layer, d_x, dim, n_tok, d_wq, d_wk, d_wv, n_head, rope, d_q, d_k, d_v,
                             d_workspace, workspace_bytes, stream, 2);
}

// ---- projections with GGUF K-quant weights read in the loop ----------------------------------

static bool kq_type_ok(int32_t t) {
    return t == TS_GGML_Q4_K || t == TS_GGML_Q5_K || t == TS_GGML_Q4_0 || t == TS_GGML_Q5_0 || t == TS_GGML_Q8_0;
}

struct QkvGenericKq {
    ts::ProjPlan pq, pk;
    uint64_t part_bytes, kv_elems;
};
static QkvGenericKq qkv_generic_plan_kq(const ts_kv *kv, int32_t dim, int32_t n_tok, int32_t n_head) {
    QkvGenericKq g;
    const int M = kv->d.n_seq * n_tok, hd = kv->d.head_dim;
    g.pq = ts::proj_plan_kq(M, dim, n_head * hd);
    g.pk = ts::proj_plan_kq(M, dim, kv->d.n_head_kv * hd);
    g.part_bytes = (std::max(g.pq.part_bytes, g.pk.part_bytes) + 255) / 256 * 256;
    g.kv_elems = (uint64_t)M * kv->d.n_head_kv * hd;
    return g;
}

int ts_qkv_gguf_workspace(const ts_kv *kv, int32_t ggml_type, int32_t dim, int32_t n_tok, int32_t n_head,
                          uint64_t *bytes) {
    if (!kv || !bytes || !qkv_shape_ok(kv, dim, n_tok, n_head) || dim % 256 != 0) return TS_ERR_INVALID;
    if (!kq_type_ok(ggml_type)) return TS_ERR_UNSUPPORTED;
    *bytes = 0;
    if (n_tok == 0) return TS_OK;
    if (qkv_fused(kv)) {
        *bytes = ts::qkv_plan_kq(kv->d.n_seq, kv->d.n_head_kv, n_head, kv->d.head_dim, dim, n_tok).part_bytes;
    } else {
        const QkvGenericKq g = qkv_generic_plan_kq(kv, dim, n_tok, n_head);
        *bytes = g.part_bytes + 2 * g.kv_elems * sizeof(float);
    }
    return TS_OK;
}

int ts_qkv_append_gguf(ts_kv *kv, int32_t layer, const float *d_x, int32_t dim, int32_t n_tok, int32_t ggml_type,
                       const void *d_wq, const void *d_wk, const void *d_wv, int32_t n_head, const ts_rope *rope,
                       float *d_q, float *d_k, float *d_v, void *d_workspace, uint64_t workspace_bytes,
                       void *stream) {
    if (!kv || layer < 0 || layer >= kv->d.n_layers) return TS_ERR_INVALID;
    if (!qkv_shape_ok(kv, dim, n_tok, n_head) || dim % 256 != 0 || !d_x || !d_wq || !d_wk || !d_wv || !d_q ||
        !aligned16(d_x) || !aligned16(d_wq) || !aligned16(d_wk) || !aligned16(d_wv) || !aligned16(d_q) ||
        (!d_k) != (!d_v) || (d_k && (!aligned16(d_k) || !aligned16(d_v))))
        return TS_ERR_INVALID;
    if (!kq_type_ok(ggml_type)) return TS_ERR_UNSUPPORTED;
    int32_t max_len = *std::max_element(kv->h_len.begin(), kv->h_len.end());
    if ((int64_t)max_len + n_tok > kv->d.max_seq) return TS_ERR_OVERFLOW;
    int rc = check_rope(rope, kv->d.head_dim, rot_end(kv, n_tok));
    if (rc) return rc;
    if (n_tok == 0) return TS_OK;
    const hipStream_t st = as_stream(stream);
    if (!qkv_fused(kv)) {
        const QkvGenericKq g = qkv_generic_plan_kq(kv, dim, n_tok, n_head);
        const uint64_t need = g.part_bytes + (d_k ? 0 : 2 * g.kv_elems * sizeof(float));
        if (!d_workspace || workspace_bytes < need || !aligned16(d_workspace)) return TS_ERR_WORKSPACE;
        float *part = static_cast<float *>(d_workspace);
        float *kb = d_k ? d_k : reinterpret_cast<float *>(static_cast<uint8_t *>(d_workspace) + g.part_bytes);
        float *vb = d_k ? d_v : kb + g.kv_elems;
        const int M = kv->d.n_seq * n_tok, hd = kv->d.head_dim, H = kv->d.n_head_kv;
        hipError_t e = ts::launch_fill_zero(d_q, (size_t)M * n_head * hd, st);
        if (e == hipSuccess) e = ts::launch_fill_zero(kb, g.kv_elems, st);
        if (e == hipSuccess) e = ts::launch_fill_zero(vb, g.kv_elems, st);
        if (e == hipSuccess) e = ts::launch_proj_kq(d_x, M, dim, ggml_type, d_wq, n_head * hd, d_q, nullptr, g.pq, part, st);
        if (e == hipSuccess) e = ts::launch_proj_kq(d_x, M, dim, ggml_type, d_wk, H * hd, kb, nullptr, g.pk, part, st);
        if (e == hipSuccess) e = ts::launch_proj_kq(d_x, M, dim, ggml_type, d_wv, H * hd, vb, nullptr, g.pk, part, st);
        if (e == hipSuccess)
            e = ts::launch_quantize_rows(kv->layer(layer), kb, vb, kv->d_len, 0, n_tok, n_tok, rope->d_table,
                                         rope->rope_dim / 2, n_tok / 32 + 2, st);
        return hip_status(e);
    }
    const ts::QkvPlan plan = ts::qkv_plan_kq(kv->d.n_seq, kv->d.n_head_kv, n_head, kv->d.head_dim, dim, n_tok);
    if (!d_workspace || workspace_bytes < plan.part_bytes || !aligned16(d_workspace)) return TS_ERR_WORKSPACE;
    return hip_status(ts::launch_qkv_kq(kv->layer(layer), kv->d_len, d_x, dim, n_tok, ggml_type, d_wq, d_wk, d_wv,
                                        n_head, d_q, d_k, d_v, rope->d_table, rope->rope_dim / 2, plan,
                                        static_cast<float *>(d_workspace), st));
}

int ts_attn_out_proj_gguf_workspace(int32_t ggml_type, int32_t n_tok, int32_t attn_dim, int32_t dim, uint64_t *bytes) {
    if (!bytes || n_tok < 0 || attn_dim <= 0 || attn_dim % 256 != 0 || dim <= 0) return TS_ERR_INVALID;
    if (!kq_type_ok(ggml_type)) return TS_ERR_UNSUPPORTED;
    *bytes = n_tok > 0 ? ts::proj_plan_kq(n_tok, attn_dim, dim).part_bytes : 0;
    return TS_OK;
}

int ts_attn_out_proj_gguf(const float *d_attn, int32_t n_tok, int32_t attn_dim, int32_t ggml_type, const void *d_wo,
                          int32_t dim, float *d_act, float *d_stash, void *d_workspace, uint64_t workspace_bytes,
                          void *stream) {
    if (!d_attn || !d_wo || !d_act || n_tok < 0 || attn_dim <= 0 || attn_dim % 256 != 0 || dim <= 0 ||
        !aligned16(d_attn) || !aligned16(d_wo) || !aligned16(d_act) || !aligned16(d_stash))
        return TS_ERR_INVALID;
    if (!kq_type_ok(ggml_type)) return TS_ERR_UNSUPPORTED;
    if (n_tok == 0) return TS_OK;
    const ts::ProjPlan plan = ts::proj_plan_kq(n_tok, attn_dim, dim);
    if (!d_workspace || workspace_bytes < plan.part_bytes || !aligned16(d_workspace)) return TS_ERR_WORKSPACE;
    return hip_status(ts::launch_proj_kq(d_attn, n_tok, attn_dim, ggml_type, d_wo, dim, d_act, d_stash, plan,
                                         static_cast<float *>(d_workspace), as_stream(stream)));
}

int ts_attn_out_proj_workspace(int32_t n_tok, int32_t attn_dim, int32_t dim, uint64_t *bytes) {
    if (!bytes || n_tok < 0 || attn_dim <= 0 || attn_dim % 64 != 0 || dim <= 0) return TS_ERR_INVALID;
    *bytes = 0;  // enough for f16 rows and for two-plane rows (ts_attn_out_proj_x2)
    for (int planes = 1; n_tok > 0 && planes <= 2; planes++)
        *bytes = std::max(*bytes, ts::proj_plan(n_tok, planes * attn_dim, dim).part_bytes);
    return TS_OK;
}

static int out_proj_planes(const float *d_attn, int32_t n_tok, int32_t attn_dim, const uint16_t *d_wo,
                           int32_t dim, float *d_act, float *d_stash, void *d_workspace,
                           uint64_t workspace_bytes, void *stream, int planes) {
    if (!d_attn || !d_wo || !d_act || n_tok < 0 || attn_dim <= 0 || attn_dim % 64 != 0 || dim <= 0 ||
        !aligned16(d_attn) || !aligned16(d_wo) || !aligned16(d_act) || !aligned16(d_stash))
        return TS_ERR_INVALID;
    if (n_tok == 0) return TS_OK;
    const ts::ProjPlan plan = ts::proj_plan(n_tok, planes * attn_dim, dim);
    if (plan.part_bytes > 0 && (!d_workspace || workspace_bytes < plan.part_bytes || !aligned16(d_workspace)))
        return TS_ERR_WORKSPACE;
    return hip_status(ts::launch_proj(d_attn, n_tok, attn_dim, d_wo, dim, d_act, d_stash, plan,
                                      static_cast<float *>(d_workspace), planes, as_stream(stream)));
}

int ts_attn_out_proj(const float *d_attn, int32_t n_tok, int32_t attn_dim, const uint16_t *d_wo,
                     int32_t dim, float *d_act, float *d_stash, void *d_workspace,
                     uint64_t workspace_bytes, void *stream) {
    return out_proj_planes(d_attn, n_tok, attn_dim, d_wo, dim, d_act, d_stash, d_workspace, workspace_bytes,
                           stream, 1);
}

int ts_attn_out_proj_x2(const float *d_attn, int32_t n_tok, int32_t attn_dim, const uint16_t *d_wo,
                        int32_t dim, float *d_act, float *d_stash, void *d_workspace,
                        uint64_t workspace_bytes, void *stream) {
    return out_proj_planes(d_attn, n_tok, attn_dim, d_wo, dim, d_act, d_stash, d_workspace, workspace_bytes,
                           stream, 2);
}

}  // extern "C"
