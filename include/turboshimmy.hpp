/*
 * turboshimmy.hpp -- C++ host side of airframe_amd's INT4 KV-cache path, over the C ABI of
 * turboshimmy.h.  It mirrors the reference's Rust surface for this path with the same names,
 * argument meanings and error behaviour, for C++ hosts and for tests that read like the
 * reference's own (src/backend/bindless/test_int4_parity.rs):
 *
 *   KVCache                     src/backend/bindless/kv_cache.rs:18-370
 *     new_int4                  :88-96 (plus the batch dimension n_seq of this path)
 *     get_seq_len / max_len     :236-240, :352-355
 *     get_window_base           :241-243
 *     reset                     :256-262
 *     set_seq_len               :265-274 (panics on overflow -> throws)
 *     advance_window_base       :277-279
 *     increment                 :284-293 (Result<(), String> -> Status)
 *     get_{k,v}_{packed,scale}_buffer  :312-345 (copies in the reference layout, export_layer)
 *     is_int4 / calculate_offset       :348-350, :366-369
 *   the INT4 steps of run_layer_with_cache_int4 (pipeline/layer.rs:805-1159): append_quant
 *   (quantize_kv), attn_decode (main_attn_out_int4), attn_decode_append (both, one launch),
 *   attn_prefill (batched main_attn_out), requant_all (requantize_all_kv_int4, :1161-1246),
 *   shift_int4 (RopeShiftPipeline::execute_int4, pipeline_shift.rs:360-566).
 *   RopeTable                   preflight.rs:71-142 (compute_rope_table + upload)
 *
 * Errors: the reference panics on programming errors (bad head_dim, getter misuse, a length
 * override past the window); here those throw turboshimmy::Error carrying the C status code.
 * The one recoverable error of the reference, increment()'s context overflow, is returned as a
 * Status, as the reference returns Err.  Unlike the reference, a failed increment leaves the
 * lengths unchanged (ts_kv_increment changes nothing on overflow).
 *
 * Device pointers (d_*) are HIP device allocations owned by the caller; `stream` is a
 * hipStream_t passed as void* (nullptr: the default stream).  Header only; link against
 * libturboshimmy.so.
 */
#ifndef TURBOSHIMMY_HPP
#define TURBOSHIMMY_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "turboshimmy.h"

namespace turboshimmy {

// A C status other than TS_OK, as an exception.
class Error : public std::runtime_error {
public:
    Error(int code, const std::string &what)
        : std::runtime_error(what + ": " + ts_status_string(code)), code_(code) {}
    int code() const noexcept { return code_; }

private:
    int code_;
};

inline void check(int rc, const char *what) {
    if (rc != TS_OK) throw Error(rc, what);
}

// Result<(), String>: is_ok() or the error code and message.
struct Status {
    int code = TS_OK;
    std::string message;
    bool is_ok() const noexcept { return code == TS_OK; }
    bool is_err() const noexcept { return code != TS_OK; }
};

// compute_rope_table + upload_rope_table (preflight.rs:71-142): cos/sin of pos * theta_i for
// n_pos positions, uploaded once.  Move-only.
class RopeTable {
public:
    RopeTable(int32_t n_pos, int32_t rope_dim, float base, float scale = 1.0f, float yarn_alpha = 0.0f,
              float yarn_beta = 0.0f) {
        check(ts_rope_create_yarn(n_pos, rope_dim, base, scale, yarn_alpha, yarn_beta, &h_), "ts_rope_create_yarn");
    }
    RopeTable(const RopeTable &) = delete;
    RopeTable &operator=(const RopeTable &) = delete;
    RopeTable(RopeTable &&o) noexcept : h_(std::exchange(o.h_, nullptr)) {}
    RopeTable &operator=(RopeTable &&o) noexcept {
        if (this != &o) {
            if (h_) ts_rope_destroy(h_);
            h_ = std::exchange(o.h_, nullptr);
        }
        return *this;
    }
    ~RopeTable() {
        if (h_) ts_rope_destroy(h_);
    }

    // The host table [n_pos][rope_dim / 2][2] (cos, sin), bit-identical to the uploaded one.
    static std::vector<float> host_table(int32_t n_pos, int32_t rope_dim, float base, float scale = 1.0f,
                                         float yarn_alpha = 0.0f, float yarn_beta = 0.0f) {
        std::vector<float> t((size_t)n_pos * (size_t)rope_dim);
        check(ts_rope_table_host_yarn(t.data(), n_pos, rope_dim, base, scale, yarn_alpha, yarn_beta),
              "ts_rope_table_host_yarn");
        return t;
    }

    const ts_rope *get() const noexcept { return h_; }
    int32_t n_pos() const { return info().second.first; }
    int32_t rope_dim() const { return info().second.second; }
    const float *device_table() const { return info().first; }

private:
    std::pair<const float *, std::pair<int32_t, int32_t>> info() const {
        const float *d = nullptr;
        int32_t n = 0, r = 0;
        check(ts_rope_info(h_, &d, &n, &r), "ts_rope_info");
        return {d, {n, r}};
    }
    ts_rope *h_ = nullptr;
};

// KVCache (kv_cache.rs) in its INT4 form, for n_seq independent sequences (the reference has
// one; every sequence here behaves like its own reference cache).  Move-only.
class KVCache {
public:
    // KVCache::new_int4 (kv_cache.rs:88-96).  head_dim must be a multiple of 8 (the reference
    // asserts it, kv_cache.rs:150-156); up to 256 is built here.
    static KVCache new_int4(int32_t n_layers, int32_t n_head_kv, int32_t head_dim, int32_t max_seq_len,
                            int32_t n_seq = 1) {
        const ts_kv_desc d{n_layers, n_seq, n_head_kv, head_dim, max_seq_len};
        ts_kv *h = nullptr;
        check(ts_kv_create(&d, &h), "KVCache::new_int4");
        return KVCache(h, d);
    }
    // Device bytes new_int4 would allocate (no GPU needed).
    static uint64_t bytes_for(int32_t n_layers, int32_t n_head_kv, int32_t head_dim, int32_t max_seq_len,
                              int32_t n_seq = 1) {
        const ts_kv_desc d{n_layers, n_seq, n_head_kv, head_dim, max_seq_len};
        uint64_t b = 0;
        check(ts_kv_bytes(&d, &b), "ts_kv_bytes");
        return b;
    }

    KVCache(const KVCache &) = delete;
    KVCache &operator=(const KVCache &) = delete;
    KVCache(KVCache &&o) noexcept : h_(std::exchange(o.h_, nullptr)), d_(o.d_) {}
    KVCache &operator=(KVCache &&o) noexcept {
        if (this != &o) {
            if (h_) ts_kv_destroy(h_);
            h_ = std::exchange(o.h_, nullptr);
            d_ = o.d_;
        }
        return *this;
    }
    ~KVCache() {
        if (h_) ts_kv_destroy(h_);
    }

    ts_kv *get() noexcept { return h_; }
    const ts_kv *get() const noexcept { return h_; }
    int32_t n_layers() const noexcept { return d_.n_layers; }
    int32_t n_seq() const noexcept { return d_.n_seq; }
    int32_t n_head_kv() const noexcept { return d_.n_head_kv; }
    int32_t head_dim() const noexcept { return d_.head_dim; }

    // ---- bookkeeping (kv_cache.rs:236-293, :348-369) -----------------------------------
    bool is_int4() const noexcept { return true; }
    uint32_t get_seq_len(int32_t seq = 0) const {
        int32_t v = 0;
        check(ts_kv_seq_len(h_, seq, &v), "KVCache::get_seq_len");
        return (uint32_t)v;
    }
    uint32_t max_len() const { return (uint32_t)d_.max_seq; }
    uint32_t get_window_base(int32_t seq = 0) const {
        int32_t v = 0;
        check(ts_kv_window_base(h_, seq, &v), "KVCache::get_window_base");
        return (uint32_t)v;
    }
    // reset(): every sequence's length, window base and sink count to 0; reset(seq): one.
    void reset(void *stream = nullptr) { check(ts_kv_reset(h_, stream), "KVCache::reset"); }
    void reset(int32_t seq, void *stream) { check(ts_kv_reset_seq(h_, seq, stream), "KVCache::reset"); }
    // The reference panics past the window; this throws Error(TS_ERR_OVERFLOW).
    void set_seq_len(uint32_t new_len, int32_t seq = 0, void *stream = nullptr) {
        check(ts_kv_set_seq_len(h_, seq, (int32_t)new_len, stream), "KVCache::set_seq_len");
    }
    void advance_window_base(uint32_t shift_amt, int32_t seq = 0, void *stream = nullptr) {
        check(ts_kv_advance_window_base(h_, seq, (int32_t)shift_amt, stream), "KVCache::advance_window_base");
    }
    // KVCache::increment: every sequence by n_tok positions (1 per decode token after all
    // layers); Err on context overflow, with the lengths unchanged.
    Status increment(int32_t n_tok = 1, void *stream = nullptr) {
        const int rc = ts_kv_increment(h_, n_tok, stream);
        if (rc == TS_OK) return {};
        if (rc == TS_ERR_OVERFLOW)
            return {rc, "KV cache overflow: " + std::to_string(max_seq_len_now() + (uint32_t)n_tok) + " > " +
                            std::to_string(max_len()) + " (context window exceeded)"};
        throw Error(rc, "KVCache::increment");
    }
    // Byte offset of (pos, head, dim) in the reference's f32 staging layout
    // [pos][n_head_kv][head_dim] (kv_cache.rs:366-369).
    size_t calculate_offset(uint32_t pos, uint32_t head, uint32_t dim) const noexcept {
        return (((size_t)pos * (size_t)d_.n_head_kv + head) * (size_t)d_.head_dim + dim) * 4;
    }

    // get_{k,v}_{packed,scale}_buffer (kv_cache.rs:312-345): positions [pos0, pos0 + n_pos)
    // of one sequence and layer copied into caller device buffers in the reference layout
    // (packed [n_pos][n_head_kv][head_dim / 8] u32, scales [n_pos][n_head_kv] f32).
    void export_layer(int32_t layer, int32_t seq, int32_t pos0, int32_t n_pos, uint32_t *d_k_packed,
                      uint32_t *d_v_packed, float *d_k_scale, float *d_v_scale, void *stream = nullptr) const {
        check(ts_kv_export(h_, layer, seq, pos0, n_pos, d_k_packed, d_v_packed, d_k_scale, d_v_scale, stream),
              "KVCache::export_layer");
    }

    // ---- the INT4 steps of run_layer_with_cache_int4 ------------------------------------
    // quantize_kv with K rotated at its absolute position: [n_seq][n_tok][n_head_kv][head_dim]
    // raw f32 at each sequence's length.  Lengths do not change.
    void append_quant(int32_t layer, const float *d_k, const float *d_v, int32_t n_tok, const RopeTable &rope,
                      void *stream = nullptr) {
        check(ts_append_quant(h_, layer, d_k, d_v, n_tok, rope.get(), stream), "KVCache::append_quant");
    }
    // requantize_all_kv_int4 for one layer from f32 caches [n_seq][ld_pos][n_head_kv][head_dim];
    // rope == nullptr: K already rotated.
    void requant_all(int32_t layer, const float *d_k_cache, const float *d_v_cache, int32_t seq_len, int32_t ld_pos,
                     const RopeTable *rope, void *stream = nullptr) {
        check(ts_requant_all(h_, layer, d_k_cache, d_v_cache, seq_len, ld_pos, rope ? rope->get() : nullptr, stream),
              "KVCache::requant_all");
    }
    uint64_t decode_workspace_bytes(int32_t n_head) const {
        uint64_t b = 0;
        check(ts_attn_decode_workspace(h_, n_head, &b), "ts_attn_decode_workspace");
        return b;
    }
    // main_attn_out_int4 for the token just appended: q [n_seq][n_head][head_dim] -> out.
    void attn_decode(int32_t layer, const float *d_q, int32_t n_head, const RopeTable &rope, float *d_out,
                     void *d_workspace, uint64_t workspace_bytes, float softcap = 0.0f, void *stream = nullptr) const {
        check(ts_attn_decode(h_, layer, d_q, n_head, rope.get(), softcap, d_out, d_workspace, workspace_bytes, stream),
              "KVCache::attn_decode");
    }
    // quantize_kv + main_attn_out_int4 of one decode token in one launch; advance = true for
    // the step's last layer also does increment(1) inside the launch.
    void attn_decode_append(int32_t layer, const float *d_k, const float *d_v, const float *d_q, int32_t n_head,
                            const RopeTable &rope, float *d_out, void *d_workspace, uint64_t workspace_bytes,
                            bool advance = false, float softcap = 0.0f, void *stream = nullptr) {
        const int rc = advance ? ts_attn_decode_append_advance(h_, layer, d_k, d_v, d_q, n_head, rope.get(), softcap,
                                                               d_out, d_workspace, workspace_bytes, stream)
                               : ts_attn_decode_append(h_, layer, d_k, d_v, d_q, n_head, rope.get(), softcap,
                                                       d_out, d_workspace, workspace_bytes, stream);
        check(rc, "KVCache::attn_decode_append");
    }
    // Batched-prefill main_attn_out over the INT4 cache for the n_tok tokens just appended
    // (causal).  q and out: [n_seq][n_tok][n_head][head_dim].
    void attn_prefill(int32_t layer, const float *d_q, int32_t n_head, int32_t n_tok, const RopeTable &rope,
                      float *d_out, float softcap = 0.0f, void *stream = nullptr) const {
        check(ts_attn_prefill(h_, layer, d_q, n_head, n_tok, rope.get(), softcap, d_out, stream),
              "KVCache::attn_prefill");
    }
    // RopeShiftPipeline::execute_int4 for one layer of one sequence.
    uint64_t shift_workspace_bytes() const {
        uint64_t b = 0;
        check(ts_kv_shift_workspace(h_, &b), "ts_kv_shift_workspace");
        return b;
    }
    void shift_int4(int32_t layer, int32_t keep_sink, int32_t shift_amt, int32_t seq, void *d_workspace,
                    uint64_t workspace_bytes, void *stream = nullptr) {
        check(ts_kv_shift(h_, layer, seq, keep_sink, shift_amt, d_workspace, workspace_bytes, stream),
              "KVCache::shift_int4");
    }
    // apply_qk_norm weights ([head_dim] f32 device arrays, or nullptr) for one layer.
    void set_qk_norm(int32_t layer, const float *d_q_norm, const float *d_k_norm, float eps = 1e-6f) {
        check(ts_kv_set_qk_norm(h_, layer, d_q_norm, d_k_norm, eps), "KVCache::set_qk_norm");
    }

private:
    KVCache(ts_kv *h, const ts_kv_desc &d) : h_(h), d_(d) {}
    uint32_t max_seq_len_now() const {
        uint32_t m = 0;
        for (int32_t s = 0; s < d_.n_seq; s++) {
            const uint32_t l = get_seq_len(s);
            m = l > m ? l : m;
        }
        return m;
    }
    ts_kv *h_ = nullptr;
    ts_kv_desc d_{};
};

}  // namespace turboshimmy

#endif /* TURBOSHIMMY_HPP */
