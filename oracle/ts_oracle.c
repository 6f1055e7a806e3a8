/*
 * ts_oracle.c -- CPU restatement of airframe's TurboShimmy INT4 KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels of
 * airframe_amd are compared against, and the CPU baseline timed beside them.
 * Nothing in the product library links, loads or calls it.
 *
 * Every function restates one piece of the reference (paths relative to the
 * reference repository root):
 *
 *   or_qk_norm_row      src/ops/reference/attention.rs:92-108 (apply_qk_norm), applied to q and
 *                       K before RoPE as at :186-199 (Qwen3)
 *   or_rope_table(_yarn) src/backend/bindless/preflight.rs:71-111  (compute_rope_table,
 *                       plain, linear and YaRN; theta as in src/ops/reference/rope.rs:150-152)
 *   or_rope_rotate      src/ops/reference/rope.rs:180-197          (adjacent-pair rotation)
 *   or_quantize_row     src/backend/bindless/test_int4_parity.rs:56-75 (cpu_quantize),
 *                       same arithmetic as sh_quantize_kv.wgsl:56-89
 *   or_dequantize_row   src/backend/bindless/test_int4_parity.rs:78-87 (cpu_dequantize)
 *   or_append           src/ops/reference/attention.rs:195-209 (RoPE on K at the absolute
 *                       position, V raw, store at current_len) + src/runtime/kvcache.rs:111-177,
 *                       with the store replaced by the INT4 quantizer (layout
 *                       src/backend/bindless/kv_cache.rs:26-37: packed [pos][n_kv][hd/8] u32,
 *                       scales [pos][n_kv] f32)
 *   or_shift            src/backend/bindless/sh_rope_shift_int4.wgsl:44-84 with
 *                       pipeline_shift.rs:360-566 (execute_int4): slide the INT4 rows down
 *   rot_pos             kv_cache.rs:41-46,277-279 (window_base) with the post-RoPE storage
 *                       of the CPU path: where each cache slot's K was rotated
 *   or_f16_to_f32       sh_layer_v1_int4.wgsl:7-34 (f16_to_f32 behind dequant_f16_at,
 *                       sh_dequant_any.wgsl:261-265)
 *   or_project          sh_layer_v1_int4.wgsl:454-575 (main_qkv, F16 branch :494-498): one
 *                       f32 dot per output, `dot += x[col] * w[row][col]` in column order
 *   or_project_f32      the same dot over f32 weights (F32 and block branches, :502-520)
 *   or_dequant          src/core/dequant/{q4_0,q5_0,q8_0,q4_k,q5_k,q6_k}.rs (GGUF weight
 *                       blocks to f32 element values)
 *   or_attn_proj        sh_layer_v1.wgsl:763-821 (main_attn_proj, F16 branch :777-781): the same
 *                       dot over attn_dim, stashed, then act = act + dot
 *   or_attend_head      src/ops/reference/attention.rs:236-313 (per-head QK^T, scale,
 *                       causal softmax, PV), src/ops/reference/matmul.rs:91-104 (f32 products
 *                       accumulated in f64), src/ops/reference/softmax.rs:91-129 (mask to -inf,
 *                       max, f32 exp, f64 sum, f64 reciprocal cast to f32 then multiply), reading
 *                       K and V through cpu_dequantize.  The optional tanh softcap follows
 *                       sh_layer_v1_int4.wgsl:1115-1118 (0 disables it; the CPU path has none).
 *
 * Build: gcc -O2 -fno-fast-math -ffp-contract=off (no FMA contraction anywhere), with
 * OpenMP only for the multi-threaded baseline entry point.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- RoPE ------------------------------------------------------------------------- */

/* table[pos][pair][0]=cos(pos*theta_pair), [1]=sin(...), compute_rope_table
 * (preflight.rs:71-111) with the table length n_pos standing for n_ctx:
 *   theta_i = 1/base^(2i/rope_dim)                                         (:87)
 *   YaRN when scale < 1 and 0 < alpha < beta (:82-84):
 *     l_train = round(n_pos * scale)                                        (:77-81)
 *     lambda_i = 2 pi / theta_i, ramp_i = clamp((l_train/lambda_i - alpha)/(beta - alpha), 0, 1)
 *     theta_i *= (1 - ramp_i) * scale + ramp_i                              (:91-97)
 *   otherwise theta_i *= scale (plain, linear)                              (:88-90)
 * All in f32, one rounding per operation, as the reference's Rust. */
int or_rope_table_yarn(float *table, int n_pos, int rope_dim, float base, float scale, float alpha,
                       float beta) {
    if (rope_dim <= 0 || (rope_dim & 1) || n_pos <= 0 || !(scale > 0.0f)) return -1;
    int n_pairs = rope_dim / 2;
    float *theta = (float *)malloc(sizeof(float) * n_pairs);
    if (!theta) return -1;
    int yarn = scale < 1.0f && alpha > 0.0f && beta > alpha;
    float l_train = yarn ? (float)(long)roundf((float)n_pos * scale) : 0.0f;
    for (int i = 0; i < n_pairs; i++) {
        float e = (2.0f * (float)i) / (float)rope_dim;
        float t = 1.0f / powf(base, e);
        if (!yarn) {
            theta[i] = t * scale;
            continue;
        }
        float lambda = 6.2831855f / t;
        float r = (l_train / lambda - alpha) / (beta - alpha);
        r = r < 0.0f ? 0.0f : (r > 1.0f ? 1.0f : r);
        float f = (1.0f - r) * scale;
        f = f + r;
        theta[i] = t * f;
    }
    for (int p = 0; p < n_pos; p++) {
        for (int i = 0; i < n_pairs; i++) {
            float angle = (float)p * theta[i];
            table[((size_t)p * n_pairs + i) * 2 + 0] = cosf(angle);
            table[((size_t)p * n_pairs + i) * 2 + 1] = sinf(angle);
        }
    }
    free(theta);
    return 0;
}

/* compute_rope_table of a spec without YaRN parameters (alpha = beta = 0): theta_i * scale. */
int or_rope_table(float *table, int n_pos, int rope_dim, float base, float scale) {
    return or_rope_table_yarn(table, n_pos, rope_dim, base, scale, 0.0f, 0.0f);
}

/* In-place rotation of one head vector at one position (rope.rs:186-196). */
void or_rope_rotate(float *x, int rope_dim, const float *table_row) {
    for (int i = 0; i < rope_dim / 2; i++) {
        float c = table_row[2 * i], s = table_row[2 * i + 1];
        float a = x[2 * i], b = x[2 * i + 1];
        float xc = a * c, ys = b * s, xs = a * s, yc = b * c;
        x[2 * i] = xc - ys;
        x[2 * i + 1] = xs + yc;
    }
}

/* ---- INT4 quantizer ------------------------------------------------------------------ */

/* Rust `f32 as i32`: saturating, NaN -> 0. */
static int32_t rust_f32_to_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

/* cpu_quantize: max_abs = fold(0, f32::max) over |x|; scale = max_abs/7 (1 if 0);
 * q = clamp(round(x/scale) + 8, 1, 15), round = half away from zero; word u holds elements
 * 8u..8u+7, element n in bits 4n..4n+3. */
void or_quantize_row(const float *x, int hd, float *scale_out, uint32_t *words) {
    float max_abs = 0.0f;
    for (int d = 0; d < hd; d++) max_abs = fmaxf(max_abs, fabsf(x[d]));
    float scale = (max_abs == 0.0f) ? 1.0f : max_abs / 7.0f;
    *scale_out = scale;
    for (int u = 0; u < hd / 8; u++) {
        uint32_t w = 0;
        for (int n = 0; n < 8; n++) {
            float r = roundf(x[u * 8 + n] / scale);
            int32_t q = rust_f32_to_i32(r);
            /* i32 + 8 cannot overflow here: |r| <= 8 whenever r is finite (|x| <= max_abs). */
            q = q + 8;
            if (q < 1) q = 1;
            if (q > 15) q = 15;
            w |= (uint32_t)q << (4 * n);
        }
        words[u] = w;
    }
}

void or_dequantize_row(const uint32_t *words, int hd, float scale, float *out) {
    for (int u = 0; u < hd / 8; u++)
        for (int n = 0; n < 8; n++) {
            uint32_t nib = (words[u] >> (4 * n)) & 0xFu;
            out[u * 8 + n] = ((float)nib - 8.0f) * scale;
        }
}

/* ---- cache append ---------------------------------------------------------------------- */

/* One sequence's INT4 cache in the reference layout. */
typedef struct {
    uint32_t *k_packed; /* [max_seq][n_kv][hd/8] */
    uint32_t *v_packed;
    float *k_scale; /* [max_seq][n_kv] */
    float *v_scale;
} or_cache;

/* ---- QKV projection ------------------------------------------------------------------ */

/* IEEE half bits -> f32 as the reference shaders decode weights: zero, subnormal
 * mant * 2^-24, normal (1 + mant/1024) * 2^(exp-15); inf and NaN decode to 0. */
float or_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u, e = (bits >> 10) & 0x1fu, mant = bits & 0x3ffu;
    float sign_f = sign ? -1.0f : 1.0f;
    if (e == 0) return mant == 0 ? sign_f * 0.0f : sign_f * ((float)mant / 16777216.0f);
    if (e == 0x1f) return 0.0f;
    float fraction = 1.0f + (float)mant / 1024.0f;
    return sign_f * ldexpf(fraction, (int)e - 15);
}

/* out[r][o] = sum over col of x[r][col] * w[o][col] for r < n_rows, o < n_out: one f32
 * accumulator per output, each product rounded to f32 and added in column order (the
 * reference's per-thread loop).  w: [n_out][dim] f16 bits.  OpenMP over outputs. */
/* main_qkv's F32 and block-format branches (sh_layer_v1_int4.wgsl:502-520): the same dot over
 * f32 weights (a block format's weights dequantized first, or_dequant). */
void or_project_f32(const float *x, int n_rows, int dim, const float *wf, int n_out, float *out) {
#pragma omp parallel for schedule(static)
    for (long ro = 0; ro < (long)n_rows * n_out; ro++) {
        const long r = ro / n_out, o = ro % n_out;
        const float *xr = x + (size_t)r * dim, *wr = wf + (size_t)o * dim;
        float dot = 0.0f;
        for (int c = 0; c < dim; c++) {
            float prod = xr[c] * wr[c];
            dot = dot + prod;
        }
        out[(size_t)r * n_out + o] = dot;
    }
}

/* ---- GGUF weight blocks ---------------------------------------------------------------
 * Element values of the reference's CPU dequantizers (src/core/dequant/), over n elements
 * (a whole number of blocks) of GGML type `type` (ggml_types.rs: F32 0, F16 1, Q4_0 2, Q5_0 6,
 * Q8_0 8, Q4_K 12, Q5_K 13, Q6_K 14).  Every product and difference is rounded on its own, as
 * in the Rust.  Returns 0, or -1 for an unknown type or a partial block. */
static float or_h(const uint8_t *p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* q4_k.rs:134-143 (q5_k.rs:146-155 is the same): 6-bit scale and min of sub-block j. */
static void or_scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | (((q[j - 4] >> 6) & 3) << 4);
        *m = ((q[j + 4] >> 4) & 0x0F) | (((q[j] >> 6) & 3) << 4);
    }
}

int or_dequant(int type, const uint8_t *src, long n, float *dst) {
    int epb, bpb;
    switch (type) {
        case 0: epb = 1; bpb = 4; break;
        case 1: epb = 1; bpb = 2; break;
        case 2: epb = 32; bpb = 18; break;
        case 6: epb = 32; bpb = 22; break;
        case 8: epb = 32; bpb = 34; break;
        case 12: epb = 256; bpb = 144; break;
        case 13: epb = 256; bpb = 176; break;
        case 14: epb = 256; bpb = 210; break;
        default: return -1;
    }
    if (n % epb) return -1;
    for (long blk = 0; blk < n / epb; blk++) {
        const uint8_t *b = src + blk * bpb;
        float *o = dst + blk * epb;
        if (type == 0) {
            memcpy(o, b, 4);
        } else if (type == 1) {
            o[0] = or_h(b);
        } else if (type == 2) { /* q4_0.rs:29-54: low nibbles 0..15, high 16..31, minus 8 */
            float d = or_h(b);
            for (int i = 0; i < 16; i++) {
                o[i] = (float)((b[2 + i] & 0x0F) - 8) * d;
                o[i + 16] = (float)(((b[2 + i] >> 4) & 0x0F) - 8) * d;
            }
        } else if (type == 6) { /* q5_0.rs:46-86: fifth bit of element e is bit e of qh */
            float d = or_h(b);
            uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
            for (int j = 0; j < 16; j++) {
                int v0 = (int)((b[6 + j] & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
                int v1 = (int)(((b[6 + j] >> 4) & 0x0F) | (((qh >> (j + 16)) & 1) << 4)) - 16;
                o[j] = (float)v0 * d;
                o[j + 16] = (float)v1 * d;
            }
        } else if (type == 8) { /* q8_0.rs:37-53 */
            float d = or_h(b);
            for (int i = 0; i < 32; i++) o[i] = (float)(int8_t)b[2 + i] * d;
        } else if (type == 12) { /* q4_k.rs:75-123 */
            float d = or_h(b), dmin = or_h(b + 2);
            const uint8_t *sc = b + 4, *q = b + 16;
            for (int c = 0; c < 4; c++) {
                int s0, m0, s1, m1;
                or_scale_min_k4(2 * c, sc, &s0, &m0);
                or_scale_min_k4(2 * c + 1, sc, &s1, &m1);
                float d1 = d * (float)s0, mm1 = dmin * (float)m0;
                float d2 = d * (float)s1, mm2 = dmin * (float)m1;
                for (int l = 0; l < 32; l++) {
                    float a = d1 * (float)(q[32 * c + l] & 0x0F);
                    o[64 * c + l] = a - mm1;
                    float e = d2 * (float)(q[32 * c + l] >> 4);
                    o[64 * c + 32 + l] = e - mm2;
                }
            }
        } else if (type == 13) { /* q5_k.rs:74-143 */
            float d = or_h(b), dmin = or_h(b + 2);
            const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
            for (int g = 0; g < 4; g++) {
                int s0, m0, s1, m1;
                or_scale_min_k4(2 * g, sc, &s0, &m0);
                or_scale_min_k4(2 * g + 1, sc, &s1, &m1);
                float d1 = d * (float)s0, mm1 = dmin * (float)m0;
                float d2 = d * (float)s1, mm2 = dmin * (float)m1;
                for (int l = 0; l < 32; l++) {
                    float q0 = (float)(qs[32 * g + l] & 0x0F) + (float)((qh[l] >> (2 * g)) & 1) * 16.0f;
                    float q1 = (float)(qs[32 * g + l] >> 4) + (float)((qh[l] >> (2 * g + 1)) & 1) * 16.0f;
                    float a = d1 * q0;
                    o[64 * g + l] = a - mm1;
                    float e = d2 * q1;
                    o[64 * g + 32 + l] = e - mm2;
                }
            }
        } else { /* q6_k.rs:72-131: two halves of 128, four 32-element parts each */
            const uint8_t *ql = b, *qh = b + 128;
            const int8_t *scl = (const int8_t *)(b + 192);
            float d = or_h(b + 208);
            for (int h = 0; h < 2; h++)
                for (int l = 0; l < 32; l++) {
                    int is = l / 16, li = 64 * h + l, hi = 32 * h + l;
                    int q1 = ((ql[li] & 0x0F) | ((qh[hi] & 3) << 4)) - 32;
                    int q2 = ((ql[li + 32] & 0x0F) | (((qh[hi] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[li] >> 4) | (((qh[hi] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[li + 32] >> 4) | (((qh[hi] >> 6) & 3) << 4)) - 32;
                    float f;
                    f = d * (float)scl[8 * h + is];     o[128 * h + l] = f * (float)q1;
                    f = d * (float)scl[8 * h + is + 2]; o[128 * h + l + 32] = f * (float)q2;
                    f = d * (float)scl[8 * h + is + 4]; o[128 * h + l + 64] = f * (float)q3;
                    f = d * (float)scl[8 * h + is + 6]; o[128 * h + l + 96] = f * (float)q4;
                }
        }
    }
    return 0;
}

void or_project(const float *x, int n_rows, int dim, const uint16_t *w, int n_out, float *out) {
    float *wf = (float *)malloc(sizeof(float) * (size_t)n_out * dim);
    if (!wf) return;
    for (size_t i = 0; i < (size_t)n_out * dim; i++) wf[i] = or_f16_to_f32(w[i]);
#pragma omp parallel for schedule(static)
    for (long ro = 0; ro < (long)n_rows * n_out; ro++) {
        const long r = ro / n_out, o = ro % n_out;
        const float *xr = x + (size_t)r * dim, *wr = wf + (size_t)o * dim;
        float dot = 0.0f;
        for (int c = 0; c < dim; c++) {
            float prod = xr[c] * wr[c];
            dot = dot + prod;
        }
        out[(size_t)r * n_out + o] = dot;
    }
    free(wf);
}

/* main_attn_proj for n_tok tokens: dot[t][o] = or_project(attn[t], wo[o]); stash[t][o] = dot
 * (stash may be NULL); act[t][o] = act[t][o] + dot (one f32 add, residual first). */
void or_attn_proj(const float *attn, int n_tok, int attn_dim, const uint16_t *wo, int dim, float *act,
                  float *stash) {
    float *dot = (float *)malloc(sizeof(float) * (size_t)n_tok * dim);
    if (!dot) return;
    or_project(attn, n_tok, attn_dim, wo, dim, dot);
    for (size_t i = 0; i < (size_t)n_tok * dim; i++) {
        if (stash) stash[i] = dot[i];
        act[i] = act[i] + dot[i];
    }
    free(dot);
}

/* ---- QK norm ------------------------------------------------------------------------- */

/* apply_qk_norm (src/ops/reference/attention.rs:92-108) for one head vector, in place:
 * rms_sq = (sum of x*x, summed in order from 0 in f32) / hd, scale = 1 / sqrt(rms_sq + eps),
 * x = x * scale * w (left to right).  w: [hd] (NULL: no norm). */
void or_qk_norm_row(float *x, int hd, const float *w, float eps) {
    if (!w) return;
    float sum = 0.0f;
    for (int d = 0; d < hd; d++) {
        float sq = x[d] * x[d];
        sum = sum + sq;
    }
    float rms_sq = sum / (float)hd;
    float scale = 1.0f / sqrtf(rms_sq + eps);
    for (int d = 0; d < hd; d++) {
        float t = x[d] * scale;
        x[d] = t * w[d];
    }
}

/* Rotation position of cache slot `pos` after sliding-window compaction: slots below n_sink
 * (the sinks, never moved) keep their own position; every other slot is rotated at
 * pos + rot, rot being the sequence's window base (kv_cache.rs:41-46, advanced by the shift
 * amount of every compaction, :277-279).  Without compaction rot = 0. */
static int rot_pos(int pos, int rot, int n_sink) { return pos < n_sink ? pos : pos + rot; }

/* Append n_tok tokens at positions pos0..pos0+n_tok-1.  k, v: [n_tok][n_kv][hd] raw f32.
 * K is rotated at its absolute position with the table (rope_dim <= hd), V is not. */
void or_append(or_cache c, int n_kv, int hd, int rope_dim, const float *table,
               const float *k, const float *v, int pos0, int n_tok, int rot, int n_sink,
               const float *k_norm, float eps) {
    float *tmp = (float *)malloc(sizeof(float) * hd);
    int n_pairs = rope_dim / 2;
    for (int t = 0; t < n_tok; t++) {
        int pos = pos0 + t;
        for (int h = 0; h < n_kv; h++) {
            size_t src = ((size_t)t * n_kv + h) * hd;
            size_t row = (size_t)pos * n_kv + h;
            memcpy(tmp, k + src, sizeof(float) * hd);
            or_qk_norm_row(tmp, hd, k_norm, eps);  /* attention.rs:186-189: norm before RoPE */
            or_rope_rotate(tmp, rope_dim, table + (size_t)rot_pos(pos, rot, n_sink) * n_pairs * 2);
            or_quantize_row(tmp, hd, &c.k_scale[row], c.k_packed + row * (hd / 8));
            or_quantize_row(v + src, hd, &c.v_scale[row], c.v_packed + row * (hd / 8));
        }
    }
    free(tmp);
}

/* ---- attention ---------------------------------------------------------------------------- */

/* One (sequence, query head) over n_q_tok query tokens at absolute positions
 * q_pos0..q_pos0+n_q_tok-1; keys 0..q_pos0+n_q_tok-1 (causal).  q: [n_q_tok][n_head][hd] raw
 * (rotated here at the query position plus the window base `rot`), out: [n_q_tok][n_head][hd]. */
void or_attend_head(or_cache c, int n_head, int n_kv, int hd, int rope_dim, const float *table,
                    const float *q, int q_pos0, int n_q_tok, int head, float softcap, float *out,
                    int rot, const float *q_norm, float eps) {
    int group = n_head / n_kv;
    int kvh = head / group;
    int key_len = q_pos0 + n_q_tok;
    int n_pairs = rope_dim / 2;
    float *qr = (float *)malloc(sizeof(float) * hd);
    float *kd = (float *)malloc(sizeof(float) * (size_t)key_len * hd);
    float *vd = (float *)malloc(sizeof(float) * (size_t)key_len * hd);
    float *row = (float *)malloc(sizeof(float) * key_len);
    for (int j = 0; j < key_len; j++) {
        size_t r = (size_t)j * n_kv + kvh;
        or_dequantize_row(c.k_packed + r * (hd / 8), hd, c.k_scale[r], kd + (size_t)j * hd);
        or_dequantize_row(c.v_packed + r * (hd / 8), hd, c.v_scale[r], vd + (size_t)j * hd);
    }
    float base_scale = 1.0f / sqrtf((float)hd);
    float scl = base_scale * 1.0f; /* per-head attention.scale is 1.0 (attention.rs:267-271) */
    for (int t = 0; t < n_q_tok; t++) {
        int qpos = q_pos0 + t;
        memcpy(qr, q + ((size_t)t * n_head + head) * hd, sizeof(float) * hd);
        or_qk_norm_row(qr, hd, q_norm, eps);
        or_rope_rotate(qr, rope_dim, table + (size_t)(qpos + rot) * n_pairs * 2);
        for (int j = 0; j < key_len; j++) {
            double acc = 0.0;
            for (int d = 0; d < hd; d++) acc += (double)(qr[d] * kd[(size_t)j * hd + d]);
            float s = (float)acc * scl;
            if (softcap > 0.0f) s = tanhf(s / softcap) * softcap;
            row[j] = s;
        }
        /* softmax.rs:104-127: query at absolute position qpos sees keys 0..=qpos */
        for (int j = qpos + 1; j < key_len; j++) row[j] = -INFINITY;
        float mx = -INFINITY;
        for (int j = 0; j < key_len; j++) mx = fmaxf(mx, row[j]);
        double sum = 0.0;
        for (int j = 0; j < key_len; j++) {
            row[j] = expf(row[j] - mx);
            sum += (double)row[j];
        }
        if (sum > 0.0) {
            float inv = (float)(1.0 / sum);
            for (int j = 0; j < key_len; j++) row[j] *= inv;
        }
        float *o = out + ((size_t)t * n_head + head) * hd;
        for (int d = 0; d < hd; d++) {
            double acc = 0.0;
            for (int j = 0; j < key_len; j++) acc += (double)(row[j] * vd[(size_t)j * hd + d]);
            o[d] = (float)acc;
        }
    }
    free(qr);
    free(kd);
    free(vd);
    free(row);
}

/* ---- batched entry points (one independent cache per sequence) ---------------------------- */

/* Caches for n_seq sequences laid out back to back: sequence s's k_packed starts at
 * k_packed + s*max_seq*n_kv*hd/8, its scales at k_scale + s*max_seq*n_kv. */
static or_cache seq_cache(uint32_t *kp, uint32_t *vp, float *ks, float *vs, int s, int max_seq,
                          int n_kv, int hd) {
    or_cache c;
    size_t wp = (size_t)s * max_seq * n_kv * (hd / 8), sp = (size_t)s * max_seq * n_kv;
    c.k_packed = kp + wp;
    c.v_packed = vp + wp;
    c.k_scale = ks + sp;
    c.v_scale = vs + sp;
    return c;
}

/* Append n_tok tokens to every sequence at its own length lens[s].  k, v: [n_seq][n_tok][n_kv][hd].
 * rot, n_sink: per-sequence window base and sink count (NULL: no compaction). */
void or_append_batch(uint32_t *kp, uint32_t *vp, float *ks, float *vs, int n_seq, int max_seq,
                     int n_kv, int hd, int rope_dim, const float *table, const float *k,
                     const float *v, const int32_t *lens, int n_tok, const int32_t *rot,
                     const int32_t *n_sink, const float *k_norm, float eps) {
    for (int s = 0; s < n_seq; s++) {
        size_t off = (size_t)s * n_tok * n_kv * hd;
        or_append(seq_cache(kp, vp, ks, vs, s, max_seq, n_kv, hd), n_kv, hd, rope_dim, table,
                  k + off, v + off, lens[s], n_tok, rot ? rot[s] : 0, n_sink ? n_sink[s] : 0,
                  k_norm, eps);
    }
}

/* Attention for n_tok query tokens of every sequence, queries at lens[s]..lens[s]+n_tok-1
 * (the tokens just appended).  q, out: [n_seq][n_tok][n_head][hd].  n_threads <= 1 runs the
 * faithful single-threaded loop; otherwise OpenMP over (sequence, head). */
void or_attend_batch(uint32_t *kp, uint32_t *vp, float *ks, float *vs, int n_seq, int max_seq,
                     int n_head, int n_kv, int hd, int rope_dim, const float *table, const float *q,
                     const int32_t *lens, int n_tok, float softcap, float *out, int n_threads,
                     const int32_t *rot, const float *q_norm, float eps) {
    long total = (long)n_seq * n_head;
    if (n_threads <= 1) {
        for (long i = 0; i < total; i++) {
            int s = (int)(i / n_head), h = (int)(i % n_head);
            size_t off = (size_t)s * n_tok * n_head * hd;
            or_attend_head(seq_cache(kp, vp, ks, vs, s, max_seq, n_kv, hd), n_head, n_kv, hd,
                           rope_dim, table, q + off, lens[s], n_tok, h, softcap, out + off,
                           rot ? rot[s] : 0, q_norm, eps);
        }
        return;
    }
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads)
#endif
    for (long i = 0; i < total; i++) {
        int s = (int)(i / n_head), h = (int)(i % n_head);
        size_t off = (size_t)s * n_tok * n_head * hd;
        or_attend_head(seq_cache(kp, vp, ks, vs, s, max_seq, n_kv, hd), n_head, n_kv, hd, rope_dim,
                       table, q + off, lens[s], n_tok, h, softcap, out + off, rot ? rot[s] : 0,
                       q_norm, eps);
    }
}

/* One (sequence, head) of a batch laid out as in or_attend_batch: used to check a sample of
 * heads at sizes where running every head would take minutes. */
void or_attend_one(uint32_t *kp, uint32_t *vp, float *ks, float *vs, int max_seq, int n_head,
                   int n_kv, int hd, int rope_dim, const float *table, const float *q_seq,
                   int q_pos0, int n_tok, int seq, int head, float softcap, float *out_seq,
                   int rot, const float *q_norm, float eps) {
    or_attend_head(seq_cache(kp, vp, ks, vs, seq, max_seq, n_kv, hd), n_head, n_kv, hd, rope_dim,
                   table, q_seq, q_pos0, n_tok, head, softcap, out_seq, rot, q_norm, eps);
}

/* ---- sliding-window compaction ---------------------------------------------------------- */

/* RopeShiftPipeline::execute_int4 / sh_rope_shift_int4.wgsl:44-84 for one sequence: slots
 * keep_sink + shift_amt .. old_len-1 move down by shift_amt (packed K/V words and both
 * scales, copied from a snapshot of the sources, as the reference copies from frozen
 * scratch buffers); the sinks 0..keep_sink-1 stay.  Nothing is moved when
 * old_len <= keep_sink + shift_amt (elements_to_shift saturates at 0, pipeline_shift.rs:381). */
void or_shift(or_cache c, int n_kv, int hd, int keep_sink, int shift_amt, int old_len) {
    int src0 = keep_sink + shift_amt;
    if (old_len <= src0) return;
    size_t n_move = (size_t)(old_len - src0) * n_kv, wpr = hd / 8;
    uint32_t *kw = (uint32_t *)malloc(n_move * wpr * 4), *vw = (uint32_t *)malloc(n_move * wpr * 4);
    float *ksn = (float *)malloc(n_move * 4), *vsn = (float *)malloc(n_move * 4);
    memcpy(kw, c.k_packed + (size_t)src0 * n_kv * wpr, n_move * wpr * 4);
    memcpy(vw, c.v_packed + (size_t)src0 * n_kv * wpr, n_move * wpr * 4);
    memcpy(ksn, c.k_scale + (size_t)src0 * n_kv, n_move * 4);
    memcpy(vsn, c.v_scale + (size_t)src0 * n_kv, n_move * 4);
    memcpy(c.k_packed + (size_t)keep_sink * n_kv * wpr, kw, n_move * wpr * 4);
    memcpy(c.v_packed + (size_t)keep_sink * n_kv * wpr, vw, n_move * wpr * 4);
    memcpy(c.k_scale + (size_t)keep_sink * n_kv, ksn, n_move * 4);
    memcpy(c.v_scale + (size_t)keep_sink * n_kv, vsn, n_move * 4);
    free(kw);
    free(vw);
    free(ksn);
    free(vsn);
}

void or_shift_seq(uint32_t *kp, uint32_t *vp, float *ks, float *vs, int max_seq, int n_kv, int hd,
                  int seq, int keep_sink, int shift_amt, int old_len) {
    or_shift(seq_cache(kp, vp, ks, vs, seq, max_seq, n_kv, hd), n_kv, hd, keep_sink, shift_amt, old_len);
}
