/*
 * turboshimmy.h -- C ABI of airframe_amd's MI355X (gfx950) INT4 KV-cache path.
 *
 * Drop-in boundary for airframe's TurboShimmy path (reference repository paths):
 *   KVCache                  src/backend/bindless/kv_cache.rs
 *   run_layer_with_cache_int4 (its quantize + INT4-attention part)
 *                            src/backend/bindless/pipeline/layer.rs:805-1159
 *   requantize_all_kv_int4   src/backend/bindless/pipeline/layer.rs:1161-1246
 *   RoPE table               src/backend/bindless/preflight.rs:28-142
 *
 * Conventions
 *   - Every function returns an int status: TS_OK (0) or a negative TS_ERR_* code.  Nothing
 *     aborts; the reference's panics (bad head_dim, getter misuse, overflow) become codes.
 *   - Pointers named d_* are device pointers owned by the caller; the cache's own buffers are
 *     allocated by ts_kv_create and freed by ts_kv_destroy.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Work is
 *     enqueued on it asynchronously; nothing synchronises the host unless stated.
 *   - A cache handle is not thread-safe: callers serialise use of one handle, as the
 *     reference does with its Arc<Mutex<KVCache>> (src/bin/shimmy_server_gpu.rs:839).
 *   - B = n_seq independent sequences.  The reference path has batch 1
 *     (pipeline/layer.rs:845-855); every sequence here behaves like its own reference cache.
 *
 * Quantisation (bit-exact with the reference CPU quantizer, test_int4_parity.rs:56-75):
 *   per (position, kv head) head vector x[hd]: scale = max|x|/7 (1 if 0);
 *   code = clamp(round_half_away(x/scale) + 8, 1, 15); dequant = (code - 8) * scale.
 *   K is rotated (RoPE at its absolute position, rope.rs:180-197) before quantisation,
 *   V is not (attention.rs:195-209 stores post-RoPE K).
 */
#ifndef TURBOSHIMMY_H
#define TURBOSHIMMY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TS_OK = 0,
    TS_ERR_INVALID = -1,     /* bad argument or shape (reference: panic / Err) */
    TS_ERR_OVERFLOW = -2,    /* context window exceeded (reference: KVCache::increment Err) */
    TS_ERR_UNSUPPORTED = -3, /* valid for the reference but not built here (e.g. head_dim) */
    TS_ERR_HIP = -4,         /* a HIP runtime call failed */
    TS_ERR_NOMEM = -5,       /* device allocation failed */
    TS_ERR_WORKSPACE = -6    /* caller workspace smaller than ts_attn_decode_workspace */
};

/* Human-readable text for a status code (static storage). */
const char *ts_status_string(int status);

/* ---- RoPE table ----------------------------------------------------------------------- */

typedef struct ts_rope ts_rope;

/* Fill a host table[n_pos][rope_dim/2][2] = (cos, sin)(pos * theta_i), n_pos in the place of
 * the spec's n_ctx.  Replaces PreflightResources::compute_rope_table (preflight.rs:71-111):
 * theta_i = 1 / base^(2i/rope_dim) times scale, or, with YaRN (scale < 1 and
 * 0 < yarn_alpha < yarn_beta), times (1 - ramp_i) scale + ramp_i with
 * ramp_i = clamp((l_train theta_i / (2 pi) - yarn_alpha) / (yarn_beta - yarn_alpha), 0, 1),
 * l_train = round(n_pos scale).  scale must be positive and finite.  Host only; needs no GPU. */
int ts_rope_table_host_yarn(float *table, int32_t n_pos, int32_t rope_dim, float base, float scale,
                            float yarn_alpha, float yarn_beta);
/* The same without YaRN parameters (a spec whose yarn_alpha = yarn_beta = 0): theta_i * scale. */
int ts_rope_table_host(float *table, int32_t n_pos, int32_t rope_dim, float base, float scale);

/* Build the table on the host and upload it (preflight.rs:114-142, upload_rope_table). */
int ts_rope_create_yarn(int32_t n_pos, int32_t rope_dim, float base, float scale, float yarn_alpha,
                        float yarn_beta, ts_rope **out);
int ts_rope_create(int32_t n_pos, int32_t rope_dim, float base, float scale, ts_rope **out);
int ts_rope_destroy(ts_rope *rope);
/* Device pointer of the uploaded table and its size (n_pos, rope_dim). */
int ts_rope_info(const ts_rope *rope, const float **d_table, int32_t *n_pos, int32_t *rope_dim);

/* ---- INT4 KV cache ---------------------------------------------------------------------- */

typedef struct ts_kv_desc {
    int32_t n_layers;
    int32_t n_seq;     /* independent sequences (batch) */
    int32_t n_head_kv;
    int32_t head_dim;  /* any multiple of 8 up to 256, as the reference (kv_cache.rs:150-156);
                        * stored padded to 64, 128 or 256 dims (the padding holds code 8,
                        * value 0); larger: TS_ERR_UNSUPPORTED */
    int32_t max_seq;   /* per-sequence capacity, positions */
} ts_kv_desc;

typedef struct ts_kv ts_kv;

/* Device bytes ts_kv_create would allocate for this descriptor (host only; no GPU needed).
 * Replaces the per-layer sizing of KVCache::new_inner (kv_cache.rs:98-233) minus the f32
 * staging buffers, which this path never allocates. */
int ts_kv_bytes(const ts_kv_desc *desc, uint64_t *bytes);

/* KVCache::new_int4 (kv_cache.rs:88-96).  Allocates packed K/V and scales for all layers and
 * sequences on the current HIP device, zero-filled; all lengths start at 0. */
int ts_kv_create(const ts_kv_desc *desc, ts_kv **out);
int ts_kv_destroy(ts_kv *kv);
int ts_kv_desc_get(const ts_kv *kv, ts_kv_desc *desc);

/* KVCache::get_seq_len / max_len (kv_cache.rs:236-240, :352-355): host-side lengths. */
int ts_kv_seq_len(const ts_kv *kv, int32_t seq, int32_t *len);
int ts_kv_max_len(const ts_kv *kv, int32_t *max_len);

/* KVCache::increment (kv_cache.rs:284-293) for every sequence, by n_tok positions (the
 * reference calls it once per token after all layers).  Returns TS_ERR_OVERFLOW, and changes
 * nothing, if any sequence would exceed max_seq. */
int ts_kv_increment(ts_kv *kv, int32_t n_tok, void *stream);

/* KVCache::set_seq_len (kv_cache.rs:265-274) for one sequence (TS_ERR_OVERFLOW instead of
 * the reference's panic).  Used for ragged batches. */
int ts_kv_set_seq_len(ts_kv *kv, int32_t seq, int32_t len, void *stream);

/* KVCache::reset (kv_cache.rs:256-259): all lengths, window bases and sink counts to 0;
 * buffers stay allocated. */
int ts_kv_reset(ts_kv *kv, void *stream);

/* KVCache::reset (kv_cache.rs:256-259) for one sequence: its length, window base and sink
 * count to 0, so a reused slot starts like a fresh reference cache; the others keep theirs. */
int ts_kv_reset_seq(ts_kv *kv, int32_t seq, void *stream);

/* Copy positions [pos0, pos0+n_pos) of one sequence and layer out of the cache into the
 * reference's layout (kv_cache.rs:26-37): packed [n_pos][n_head_kv][head_dim/8] u32, scales
 * [n_pos][n_head_kv] f32.  All four outputs are device pointers.  Stands in for the
 * get_{k,v}_{packed,scale}_buffer getters (kv_cache.rs:312-345). */
int ts_kv_export(const ts_kv *kv, int32_t layer, int32_t seq, int32_t pos0, int32_t n_pos,
                 uint32_t *d_k_packed, uint32_t *d_v_packed, float *d_k_scale, float *d_v_scale,
                 void *stream);

/* ---- QK norm (Qwen3) ------------------------------------------------------------------------ */

/* Per-head RMSNorm of q and K before RoPE for one layer: apply_qk_norm
 * (src/ops/reference/attention.rs:92-108, applied at :186-189; the GPU path's main_qk_norm,
 * sh_layer_v1_int4.wgsl:577-640, runs at the same point).  From then on ts_append_quant and
 * ts_attn_decode_append normalize each K head vector (x * 1/sqrt(mean(x^2) + eps) * w, the
 * squares summed in order in f32) before rotating and quantizing it, and the attention entry
 * points normalize q the same way before rotating it.  d_q_norm, d_k_norm: [head_dim] f32
 * device arrays (16-byte aligned) that must stay valid while set, or NULL to leave that side
 * unnormalized; eps as the reference (1e-6).  ts_requant_all takes K as given (the reference
 * normalizes its f32 cache before requantizing). */
int ts_kv_set_qk_norm(ts_kv *kv, int32_t layer, const float *d_q_norm, const float *d_k_norm,
                      float eps);

/* ---- sliding-window compaction ------------------------------------------------------------- */

/* KVCache::get_window_base / advance_window_base (kv_cache.rs:241-243, :277-279) for one
 * sequence: the total shift of all compactions so far.  The K of every slot at or past the
 * sequence's sink count is stored rotated at (slot + window base), so appends after a
 * compaction rotate K there and queries are rotated at (position + window base): window keys
 * then see the compacted distance and the sinks the logical one, as in
 * sh_layer_v1_int4.wgsl:1062-1080.  Call advance after ts_kv_shift of every layer, then
 * ts_kv_set_seq_len(len - shift_amt), as the reference's caller does. */
int ts_kv_window_base(const ts_kv *kv, int32_t seq, int32_t *base);
int ts_kv_advance_window_base(ts_kv *kv, int32_t seq, int32_t shift_amt, void *stream);

/* Device bytes of scratch ts_kv_shift needs at most (a snapshot of the moved slots).  A
 * shift whose moved slots take at most 8 rounds of shift_amt slots (ceil(n_move / shift_amt)
 * <= 8, n_move = len - keep_sink - shift_amt) runs in place and needs no workspace (d_workspace
 * may be NULL); a longer one needs n_move * n_head_kv * (head_dim + 8) bytes, 16-byte aligned,
 * and is otherwise refused with TS_ERR_WORKSPACE before anything changes. */
int ts_kv_shift_workspace(const ts_kv *kv, uint64_t *bytes);

/* RopeShiftPipeline::execute_int4 (pipeline_shift.rs:360-566, sh_rope_shift_int4.wgsl:44-84)
 * for one layer of one sequence: slots keep_sink + shift_amt .. len-1 move down by shift_amt
 * (packed K and V and both scales, copied unchanged through a snapshot in d_workspace); the
 * keep_sink sinks stay.  Nothing moves when len <= keep_sink + shift_amt.  The first call on a
 * sequence records keep_sink as its sink count, also when nothing moves; a different keep_sink
 * later is TS_ERR_INVALID (slots below the sink count keep the rotation of their own position)
 * until ts_kv_reset / ts_kv_reset_seq.  Lengths and the window base do not change. */
int ts_kv_shift(ts_kv *kv, int32_t layer, int32_t seq, int32_t keep_sink, int32_t shift_amt,
                void *d_workspace, uint64_t workspace_bytes, void *stream);

/* ---- hot path ------------------------------------------------------------------------------ */

/* Every device array these entry points read or write (k, v, q, out, workspace) must be
 * 16-byte aligned, as hipMalloc and torch allocations are; otherwise the call returns
 * TS_ERR_INVALID and launches nothing. */

/* RoPE-fused quantize-on-append.  Replaces quantize_kv (sh_quantize_kv.wgsl:39-90, dispatched
 * at layer.rs:1092-1099) plus the RoPE step of attention.rs:196-199.
 * d_k, d_v: [n_seq][n_tok][n_head_kv][head_dim] raw f32.  Token t of sequence s is written
 * at position len[s] + t; K is rotated there with `rope`.  Lengths do not change (call
 * ts_kv_increment after all layers, as the reference does). */
int ts_append_quant(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v, int32_t n_tok,
                    const ts_rope *rope, void *stream);

/* requantize_all_kv_int4 (layer.rs:1161-1246) for one layer: quantize positions
 * [0, seq_len) of every sequence from f32 caches d_k_cache, d_v_cache laid out
 * [n_seq][ld_pos][n_head_kv][head_dim] (ld_pos >= seq_len).  With rope != NULL, K is rotated
 * at each position first; with NULL it is taken as already rotated (the CPU KvCache stores
 * post-RoPE K).  Lengths do not change. */
int ts_requant_all(ts_kv *kv, int32_t layer, const float *d_k_cache, const float *d_v_cache,
                   int32_t seq_len, int32_t ld_pos, const ts_rope *rope, void *stream);

/* Bytes of scratch ts_attn_decode needs for n_head query heads (worst case over lengths up
 * to max_seq).  Host only. */
int ts_attn_decode_workspace(const ts_kv *kv, int32_t n_head, uint64_t *bytes);

/* INT4 GQA decode attention.  Replaces main_attn_out_int4 (sh_layer_v1_int4.wgsl:1042-1143,
 * dispatched at layer.rs:1100-1107) with the CPU path's semantics (attention.rs:236-313).
 * d_q: [n_seq][n_head][head_dim] raw f32 for the token just appended; it is rotated at
 * position len[s] and attends to positions 0..len[s] (len[s]+1 keys, the state between
 * ts_append_quant and ts_kv_increment, like CacheParams{current_pos, seq_len+1}).
 * d_out: [n_seq][n_head][head_dim] f32.  n_head must be a multiple of n_head_kv (any group
 * size; more than 8 query heads per kv head run as groups of 8).  softcap > 0 applies tanh(s/softcap)*softcap to the scaled scores
 * (sh_layer_v1_int4.wgsl:1116-1118).  d_workspace: ts_attn_decode_workspace bytes. */
int ts_attn_decode(const ts_kv *kv, int32_t layer, const float *d_q, int32_t n_head,
                   const ts_rope *rope, float softcap, float *d_out, void *d_workspace,
                   uint64_t workspace_bytes, void *stream);

/* ts_append_quant(kv, layer, d_k, d_v, 1, rope) followed by ts_attn_decode(...), in one launch:
 * the quantize_kv + main_attn_out_int4 pair that run_layer_with_cache_int4 dispatches back to
 * back for every decode token (layer.rs:1092-1107).  Writes the same codes and scales as
 * ts_append_quant; the new position's score is taken from its dequantized row directly.
 * d_k, d_v: [n_seq][n_head_kv][head_dim] raw f32; other arguments as ts_attn_decode.
 * Lengths do not change. */
int ts_attn_decode_append(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v,
                          const float *d_q, int32_t n_head, const ts_rope *rope, float softcap,
                          float *d_out, void *d_workspace, uint64_t workspace_bytes, void *stream);

/* ts_attn_decode_append without a workspace argument and without allocating anything: the
 * split partials go to a scratch array the library keeps on every GPU it runs on (8 MiB each,
 * until the process ends).  No counterpart in the reference: for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Returns TS_ERR_WORKSPACE when this call's partials, n_seq * n_head * splits * (hds + 2)
 * floats, would exceed 8 MiB, where hds is the stored head dim: head_dim rounded up to 64,
 * 128 or 256 (a call that needs no split needs none).  All calls on one GPU
 * share the array: calls that overlap on one GPU (other streams, other threads) race. */
int ts_attn_decode_append_noalloc(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v,
                                  const float *d_q, int32_t n_head, const ts_rope *rope, float softcap,
                                  float *d_out, void *stream);

/* ts_attn_decode_append for the last layer of a decode step, followed by ts_kv_increment(kv, 1)
 * (cache.increment(), server_inference.rs:1355-1358) in the same launch: with a split the
 * launch's last kernel (the combine kernel with a split, the 16x16 decode kernel without one)
 * advances the lengths once all of its workgroups have read them (an arrival counter kept in
 * the cache; with one sequence in an eager call, whose length is a launch argument, a plain
 * store), so the step needs no separate length-update launch; the integer decode kernel's
 * plans without a split are followed by a length update.  Same arguments and errors as
 * ts_attn_decode_append.  Lengths must not be read or changed by other work on the cache while
 * the call runs. */
int ts_attn_decode_append_advance(ts_kv *kv, int32_t layer, const float *d_k, const float *d_v,
                                  const float *d_q, int32_t n_head, const ts_rope *rope, float softcap,
                                  float *d_out, void *d_workspace, uint64_t workspace_bytes, void *stream);

/* Chunked-prefill attention over the INT4 cache.  Stands in for the f32 main_attn_out of
 * batched prefill (sh_layer_v1.wgsl:662-762, inference.rs:1160-1166) with the INT4 cache as
 * its source.  d_q: [n_seq][n_tok][n_head][head_dim] raw f32 for the n_tok tokens just
 * appended at len[s]..len[s]+n_tok-1; query t is rotated at len[s]+t and sees keys
 * 0..len[s]+t (causal).  d_out has the shape of d_q. */
int ts_attn_prefill(const ts_kv *kv, int32_t layer, const float *d_q, int32_t n_head,
                    int32_t n_tok, const ts_rope *rope, float softcap, float *d_out, void *stream);

/* ---- Projection weights in GGUF formats ------------------------------------------------- */

/* GGML type ids (ggml_types.rs) of the weight formats main_qkv and main_attn_proj read
 * (sh_layer_v1_int4.wgsl:497-520, sh_layer_v1.wgsl:777-790). */
enum {
    TS_GGML_F32 = 0,
    TS_GGML_F16 = 1,
    TS_GGML_Q4_0 = 2,
    TS_GGML_Q5_0 = 6,
    TS_GGML_Q8_0 = 8,
    TS_GGML_Q4_K = 12,
    TS_GGML_Q5_K = 13,
    TS_GGML_Q6_K = 14
};

/* Bytes of an [n_rows][n_cols] weight matrix of that type (n_cols a multiple of the block:
 * 32 for Q4_0/Q5_0/Q8_0, 256 for the K formats, 8 for F32/F16).  Host only. */
int ts_weights_src_bytes(int32_t ggml_type, int64_t n_rows, int64_t n_cols, uint64_t *bytes);

/* Convert a weight matrix of that type on the device into the f16 row-major [n_rows][n_cols]
 * that ts_qkv_append and ts_attn_out_proj take (d_dst 16-byte aligned), once at load.  Each
 * element is the reference's CPU dequantized value (src/core/dequant/, the F32 and block
 * branches of main_qkv) rounded to f16, nearest even: the projections then differ from the
 * reference's f32-weight dot by that rounding (relative 2^-11 per weight) on top of their own. */
int ts_weights_to_f16(int32_t ggml_type, const void *d_src, int64_t n_rows, int64_t n_cols,
                      uint16_t *d_dst, void *stream);

/* The same into two f16 planes per row, d_dst [n_rows][2 n_cols]: the first n_cols the value
 * rounded to f16 (hi), the next n_cols the rest (value - hi, exact in f32) rounded to f16 (lo).
 * ts_qkv_append_x2 and ts_attn_out_proj_x2 take such rows and multiply each x by hi + lo, so
 * the projections keep the f32 weights to about 22 bits.  Both forms hold values of f16
 * range only: a dequantized weight of magnitude 65520 or more (or a non-finite one, such as a
 * block scale that is inf or NaN) converts to an infinite or NaN hi, and the projections then
 * return non-finite values; the conversion does not check for it.  Dequantized GGUF weights
 * of real models stay orders of magnitude below that bound. */
int ts_weights_to_f16x2(int32_t ggml_type, const void *d_src, int64_t n_rows, int64_t n_cols,
                        uint16_t *d_dst, void *stream);

/* ---- QKV projection with the append as its epilogue ------------------------------------ */

/* Bytes of scratch ts_qkv_append and ts_qkv_append_x2 need for this shape (0 when the
 * projection is not split over dim).  Host only. */
int ts_qkv_workspace(const ts_kv *kv, int32_t dim, int32_t n_tok, int32_t n_head, uint64_t *bytes);

/* main_qkv (sh_layer_v1_int4.wgsl:454-575, F16 weights: the formula slot 1 branch at :494-498)
 * followed by quantize_kv (layer.rs:1092-1099), in one pass: for each token,
 * q = Wq x, k = Wk x, v = Wv x, with k and v quantized straight into the cache as
 * ts_append_quant would quantize them (QK norm of K when set, rotation of K, codes and
 * scales), so the f32 K and V are never written unless asked for.
 * d_x: [n_seq][n_tok][dim] f32 (the attention-normalized activations, |x| < 65504);
 * d_wq: [n_head*head_dim][dim], d_wk, d_wv: [n_head_kv*head_dim][dim], f16 row-major (GGUF
 * order: output row, then input column), 16-byte aligned.  Token t of sequence s goes to
 * position len[s] + t.  d_q: [n_seq][n_tok][n_head][head_dim] raw q (the attention entry
 * points apply the QK norm and rotation).  d_k, d_v: NULL, or [n_seq][n_tok][n_head_kv]
 * [head_dim] to receive the raw projections as well (the reference's f32 staging cache).
 * dim a multiple of 64.  head_dim 128 and 64 run one fused kernel; any other head_dim of the
 * cache runs the projection kernel for q, K and V, then the append kernel (the same codes as
 * ts_append_quant of those K and V; K and V staged in the workspace unless d_k, d_v are given).
 * Lengths do not change. */
int ts_qkv_append(ts_kv *kv, int32_t layer, const float *d_x, int32_t dim, int32_t n_tok,
                  const uint16_t *d_wq, const uint16_t *d_wk, const uint16_t *d_wv, int32_t n_head,
                  const ts_rope *rope, float *d_q, float *d_k, float *d_v, void *d_workspace,
                  uint64_t workspace_bytes, void *stream);

/* ts_qkv_append with weights of two f16 planes per row ([rows][2 dim], ts_weights_to_f16x2):
 * the reference's F32 and block-format weights (main_qkv, sh_layer_v1_int4.wgsl:502-520) at
 * about f32 accuracy.  Twice the weight bytes and matrix work of the f16 form. */
int ts_qkv_append_x2(ts_kv *kv, int32_t layer, const float *d_x, int32_t dim, int32_t n_tok,
                     const uint16_t *d_wq, const uint16_t *d_wk, const uint16_t *d_wv, int32_t n_head,
                     const ts_rope *rope, float *d_q, float *d_k, float *d_v, void *d_workspace,
                     uint64_t workspace_bytes, void *stream);

/* ---- attention output projection ---------------------------------------------------- */

/* Bytes of scratch ts_attn_out_proj and ts_attn_out_proj_x2 need for this shape (0 when the
 * reduction is not split).  Host only. */
int ts_attn_out_proj_workspace(int32_t n_tok, int32_t attn_dim, int32_t dim, uint64_t *bytes);

/* main_attn_proj (sh_layer_v1.wgsl:763-821, F16 weights: the formula slot 1 branch at
 * :777-781) for n_tok tokens: dot = Wo a over attn_dim = n_head * head_dim inputs, then
 * act = act + dot (:818-820), and dot itself into d_stash when given (the reference's stash
 * for Gemma-2's post-attention norm, :812-815).  d_attn: [n_tok][attn_dim] f32, the attention
 * output (ts_attn_decode / ts_attn_prefill); d_wo: [dim][attn_dim] f16 row-major; d_act:
 * [n_tok][dim] f32, updated in place; d_stash: NULL or [n_tok][dim] f32.  attn_dim a multiple
 * of 64; pointers 16-byte aligned.  Needs no cache. */
int ts_attn_out_proj(const float *d_attn, int32_t n_tok, int32_t attn_dim, const uint16_t *d_wo,
                     int32_t dim, float *d_act, float *d_stash, void *d_workspace,
                     uint64_t workspace_bytes, void *stream);
/* ts_attn_out_proj with d_wo of two f16 planes per row ([dim][2 attn_dim], ts_weights_to_f16x2):
 * main_attn_proj's F32 and block branches (sh_layer_v1.wgsl:782-790). */
int ts_attn_out_proj_x2(const float *d_attn, int32_t n_tok, int32_t attn_dim, const uint16_t *d_wo,
                        int32_t dim, float *d_act, float *d_stash, void *d_workspace,
                        uint64_t workspace_bytes, void *stream);

/* ---- projections with GGUF block weights read at their own size --------------------------- */

/* Bytes of scratch ts_qkv_append_gguf needs for this shape (ggml_type TS_GGML_Q4_K,
 * TS_GGML_Q5_K, TS_GGML_Q8_0, TS_GGML_Q4_0 or TS_GGML_Q5_0; dim a multiple of 256).  Host
 * only. */
int ts_qkv_gguf_workspace(const ts_kv *kv, int32_t ggml_type, int32_t dim, int32_t n_tok, int32_t n_head,
                          uint64_t *bytes);

/* ts_qkv_append with the weights as the GGUF blob's own Q4_K, Q5_K, Q8_0, Q4_0 or Q5_0 blocks,
 * read inside the projection loop as main_qkv reads them (sh_layer_v1_int4.wgsl:502-520; the
 * values of q4_k.rs:75-123, q5_k.rs:74-143, q8_0.rs, q4_0.rs, q5_0.rs), so a weight moves
 * 0.5625 (Q4_K, Q4_0), 0.6875 (Q5_K, Q5_0) or 1.0625 (Q8_0) bytes instead of the 4 of
 * ts_qkv_append_x2's planes.  d_wq:
 * [n_head*head_dim] rows of dim elements, d_wk, d_wv: [n_head_kv*head_dim] rows, all 16-byte
 * aligned (the blocks of one type for all three); dim a multiple of 256.  Results agree with the
 * f32-weight dot to f32 rounding (x is split hi + lo in f16, |x| < 65504, as in ts_qkv_append).
 * Any other type is TS_ERR_UNSUPPORTED: convert it once with ts_weights_to_f16x2.  The
 * workspace is always needed (ts_qkv_gguf_workspace). */
int ts_qkv_append_gguf(ts_kv *kv, int32_t layer, const float *d_x, int32_t dim, int32_t n_tok, int32_t ggml_type,
                       const void *d_wq, const void *d_wk, const void *d_wv, int32_t n_head, const ts_rope *rope,
                       float *d_q, float *d_k, float *d_v, void *d_workspace, uint64_t workspace_bytes,
                       void *stream);

/* Bytes of scratch ts_attn_out_proj_gguf needs (attn_dim a multiple of 256).  Host only. */
int ts_attn_out_proj_gguf_workspace(int32_t ggml_type, int32_t n_tok, int32_t attn_dim, int32_t dim,
                                    uint64_t *bytes);

/* ts_attn_out_proj with d_wo as the GGUF blob's Q4_K, Q5_K, Q8_0, Q4_0 or Q5_0 blocks ([dim] rows of
 * attn_dim elements, 16-byte aligned; attn_dim a multiple of 256), read in the loop as
 * main_attn_proj reads them (sh_layer_v1.wgsl:782-790). */
int ts_attn_out_proj_gguf(const float *d_attn, int32_t n_tok, int32_t attn_dim, int32_t ggml_type, const void *d_wo,
                          int32_t dim, float *d_act, float *d_stash, void *d_workspace, uint64_t workspace_bytes,
                          void *stream);

#ifdef __cplusplus
}
#endif
#endif /* TURBOSHIMMY_H */
