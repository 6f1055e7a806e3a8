// test_int4_parity.cpp -- the reference's INT4 parity tests
// (src/backend/bindless/test_int4_parity.rs:306-585) run on the MI355X through the C++ host
// side (include/turboshimmy.hpp), plus decode and prefill attention against the CPU oracle.
//
// The quantizer checks use the reference's own inputs.  Where the reference only bounds the
// round trip (its WGSL kernel rounds half to even, its CPU quantizer half away from zero),
// this path follows the CPU quantizer exactly, so codes and scales are compared bit for bit
// with the oracle's restatement of cpu_quantize (oracle/ts_oracle.c, or_quantize_row).  The
// oracle is test infrastructure: it is linked here only as the checker.
//
// Built by tests/cpp/Makefile (g++, HIP runtime, libturboshimmy.so, the oracle's C source);
// run by tests/test_gpu_cpp.py on a GPU.  Prints one line per test; exit status 0 when all
// pass.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "turboshimmy.hpp"

extern "C" {
// oracle/ts_oracle.c
void or_quantize_row(const float *x, int hd, float *scale_out, uint32_t *words);
void or_dequantize_row(const uint32_t *words, int hd, float scale, float *out);
int or_rope_table(float *table, int n_pos, int rope_dim, float base, float scale);
void or_append_batch(uint32_t *kp, uint32_t *vp, float *ks, float *vs, int n_seq, int max_seq, int n_kv, int hd,
                     int rope_dim, const float *table, const float *k, const float *v, const int32_t *lens, int n_tok,
                     const int32_t *rot, const int32_t *n_sink, const float *k_norm, float eps);
void or_attend_batch(uint32_t *kp, uint32_t *vp, float *ks, float *vs, int n_seq, int max_seq, int n_head, int n_kv,
                     int hd, int rope_dim, const float *table, const float *q, const int32_t *lens, int n_tok,
                     float softcap, float *out, int n_threads, const int32_t *rot, const float *q_norm, float eps);
}

namespace ts = turboshimmy;

namespace {

struct Failure {
    std::string msg;
};
void require(bool ok, const std::string &msg) {
    if (!ok) throw Failure{msg};
}
void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Failure{std::string(what) + ": " + hipGetErrorString(e)};
}

// A device array of T, filled from / read back to host vectors.
template <typename T>
struct Dev {
    T *p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { hip_ok(hipMalloc(&p, sizeof(T) * (n ? n : 1)), "hipMalloc"); }
    explicit Dev(const std::vector<T> &h) : Dev(h.size()) {
        hip_ok(hipMemcpy(p, h.data(), sizeof(T) * n, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    Dev(const Dev &) = delete;
    Dev &operator=(const Dev &) = delete;
    ~Dev() { (void)hipFree(p); }
    std::vector<T> host() const {
        std::vector<T> h(n);
        hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
        hip_ok(hipMemcpy(h.data(), p, sizeof(T) * n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
        return h;
    }
};

// One sequence's first n_pos positions of one layer, read back in the reference layout.
struct Exported {
    std::vector<uint32_t> kp, vp;
    std::vector<float> ks, vs;
};
Exported export_layer(const ts::KVCache &kv, int layer, int seq, int n_pos) {
    const int H = kv.n_head_kv(), w = kv.head_dim() / 8;
    Dev<uint32_t> kp((size_t)n_pos * H * w), vp((size_t)n_pos * H * w);
    Dev<float> ks((size_t)n_pos * H), vs((size_t)n_pos * H);
    kv.export_layer(layer, seq, 0, n_pos, kp.p, vp.p, ks.p, vs.p);
    return {kp.host(), vp.host(), ks.host(), vs.host()};
}

// Append one token (position 0 of sequence 0; RoPE at position 0 is the identity) and read
// back the codes and scales of its n_head_kv rows.
Exported quantize_at_pos0(const std::vector<float> &k, const std::vector<float> &v, int n_head_kv, int head_dim) {
    ts::KVCache kv = ts::KVCache::new_int4(1, n_head_kv, head_dim, 8);
    ts::RopeTable rope(8, head_dim, 10000.0f);
    Dev<float> dk(k), dv(v);
    kv.append_quant(0, dk.p, dv.p, 1, rope);
    return export_layer(kv, 0, 0, 1);
}

float max_err_after_round_trip(const std::vector<float> &x, const uint32_t *words, float scale) {
    std::vector<float> d(x.size());
    or_dequantize_row(words, (int)x.size(), scale, d.data());
    float e = 0.0f;
    for (size_t i = 0; i < x.size(); i++) e = std::fmax(e, std::fabs(x[i] - d[i]));
    return e;
}

// Codes and scale of one row bit-identical with the CPU quantizer, and the round trip bounded
// by half a step.
void expect_row_matches_cpu(const std::vector<float> &x, const uint32_t *words, float scale, const std::string &what) {
    const int hd = (int)x.size();
    std::vector<uint32_t> cw(hd / 8);
    float cs = 0.0f;
    or_quantize_row(x.data(), hd, &cs, cw.data());
    require(std::memcmp(&scale, &cs, sizeof(float)) == 0,
            what + " scale " + std::to_string(scale) + " vs CPU " + std::to_string(cs));
    for (int i = 0; i < hd / 8; i++) {
        char buf[96];
        std::snprintf(buf, sizeof buf, " word %d: GPU %08x CPU %08x", i, words[i], cw[i]);
        require(words[i] == cw[i], what + buf);
    }
    const float err = max_err_after_round_trip(x, words, scale);
    require(err <= cs / 2.0f + 1e-5f, what + " round-trip error " + std::to_string(err));
}

// ---- the reference's tests -------------------------------------------------------------------

// test_int4_parity.rs:306-392: one head of 64 dims, K a ramp, V a sinusoid.
void test_quantize_kv_single_head_parity() {
    const int hd = 64;
    std::vector<float> k(hd), v(hd);
    for (int d = 0; d < hd; d++) {
        k[d] = (float)d * 0.1f - 3.15f;
        v[d] = std::sin((float)d * 0.3f - 9.5f) * 2.5f;
    }
    const Exported o = quantize_at_pos0(k, v, 1, hd);
    expect_row_matches_cpu(k, o.kp.data(), o.ks[0], "K");
    expect_row_matches_cpu(v, o.vp.data(), o.vs[0], "V");
}

// test_int4_parity.rs:397-485: four heads with amplitudes 1, 2, 0.5, 7 get independent scales.
void test_quantize_kv_multi_head_independent_scales() {
    const int H = 4, hd = 64;
    const float amp[H] = {1.0f, 2.0f, 0.5f, 7.0f};
    std::vector<float> k((size_t)H * hd), v((size_t)H * hd);
    for (int h = 0; h < H; h++)
        for (int d = 0; d < hd; d++) {
            k[(size_t)h * hd + d] = amp[h] * (((float)d / (float)hd) * 2.0f - 1.0f);
            v[(size_t)h * hd + d] = amp[h] * ((float)d * 0.1f - 3.15f) / 3.15f;
        }
    const Exported o = quantize_at_pos0(k, v, H, hd);
    for (int h = 0; h < H; h++) {
        const std::vector<float> kh(k.begin() + (size_t)h * hd, k.begin() + (size_t)(h + 1) * hd);
        const std::vector<float> vh(v.begin() + (size_t)h * hd, v.begin() + (size_t)(h + 1) * hd);
        expect_row_matches_cpu(kh, o.kp.data() + (size_t)h * hd / 8, o.ks[h], "head " + std::to_string(h) + " K");
        expect_row_matches_cpu(vh, o.vp.data() + (size_t)h * hd / 8, o.vs[h], "head " + std::to_string(h) + " V");
    }
    require(o.ks[0] != o.ks[1] && o.ks[1] != o.ks[2] && o.ks[2] != o.ks[3], "per-head K scales differ");
}

// test_int4_parity.rs:490-520: a zero vector has scale exactly 1 and every nibble 8.
void test_quantize_kv_zero_vector_no_nan() {
    const std::vector<float> z(8, 0.0f);
    const Exported o = quantize_at_pos0(z, z, 1, 8);
    require(o.ks[0] == 1.0f && o.vs[0] == 1.0f, "zero vector: scale 1.0");
    require(o.kp[0] == 0x88888888u && o.vp[0] == 0x88888888u, "zero vector: words 0x88888888");
}

// test_int4_parity.rs:525-585: all +1000 saturates every nibble at 15; alternating +-1000
// stays within half a step.
void test_quantize_kv_extreme_values_clamped() {
    std::vector<float> big(8, 1000.0f), alt(8);
    for (int d = 0; d < 8; d++) alt[d] = d % 2 == 0 ? 1000.0f : -1000.0f;
    const Exported o = quantize_at_pos0(big, alt, 1, 8);
    require(o.kp[0] == 0xFFFFFFFFu, "all +1000: word 0xFFFFFFFF");
    require(o.ks[0] == 1000.0f / 7.0f, "all +1000: scale 1000/7");
    expect_row_matches_cpu(big, o.kp.data(), o.ks[0], "K");
    expect_row_matches_cpu(alt, o.vp.data(), o.vs[0], "V");
}

// ---- attention through the C++ KVCache against the oracle ---------------------------------

std::vector<float> normal(std::mt19937 &g, size_t n) {
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::vector<float> x(n);
    for (auto &e : x) e = nd(g);
    return x;
}

void expect_close(const std::vector<float> &got, const std::vector<float> &ref, const std::string &what) {
    double worst = 0.0;
    for (size_t i = 0; i < got.size(); i++) {
        const double err = std::fabs((double)got[i] - (double)ref[i]);
        require(std::isfinite(got[i]) && err <= 2e-3 + 1e-3 * std::fabs((double)ref[i]),
                what + ": element " + std::to_string(i) + " " + std::to_string(got[i]) + " vs " + std::to_string(ref[i]));
        worst = err > worst ? err : worst;
    }
    std::printf("    %s: max abs error %.3g\n", what.c_str(), worst);
}

// A prefill of C tokens per sequence (append, prefill attention, increment), then decode
// steps (the fused append + attention, the last layer advancing the lengths), layer 1 of a
// 2-layer cache; every output against the oracle's cache of the same tokens, and the cache
// itself bit-exact.
void test_prefill_then_decode_against_oracle() {
    const int S = 2, H = 2, G = 4, NH = H * G, hd = 128, C = 70, steps = 3, P = C + steps + 4;
    const float base = 500000.0f;
    std::mt19937 g(1234);
    ts::KVCache kv = ts::KVCache::new_int4(2, H, hd, P, S);
    ts::RopeTable rope(P, hd, base);
    std::vector<float> table((size_t)P * hd);
    require(or_rope_table(table.data(), P, hd, base, 1.0f) == 0, "oracle rope table");
    const std::vector<float> host_table = ts::RopeTable::host_table(P, hd, base);
    require(std::memcmp(host_table.data(), table.data(), table.size() * sizeof(float)) == 0,
            "RopeTable::host_table bit-identical with the oracle's");

    const size_t wrow = (size_t)P * H * (hd / 8), srow = (size_t)P * H;
    std::vector<uint32_t> okp(S * wrow), ovp(S * wrow);
    std::vector<float> oks(S * srow), ovs(S * srow);
    std::vector<int32_t> lens(S, 0);

    // prefill
    const std::vector<float> k = normal(g, (size_t)S * C * H * hd), v = normal(g, (size_t)S * C * H * hd);
    const std::vector<float> q = normal(g, (size_t)S * C * NH * hd);
    Dev<float> dk(k), dv(v), dq(q), dout((size_t)S * C * NH * hd);
    kv.append_quant(1, dk.p, dv.p, C, rope);
    kv.attn_prefill(1, dq.p, NH, C, rope, dout.p);
    or_append_batch(okp.data(), ovp.data(), oks.data(), ovs.data(), S, P, H, hd, hd, table.data(), k.data(), v.data(),
                    lens.data(), C, nullptr, nullptr, nullptr, 1e-6f);
    std::vector<float> ref((size_t)S * C * NH * hd);
    or_attend_batch(okp.data(), ovp.data(), oks.data(), ovs.data(), S, P, NH, H, hd, hd, table.data(), q.data(),
                    lens.data(), C, 0.0f, ref.data(), 4, nullptr, nullptr, 1e-6f);
    expect_close(dout.host(), ref, "prefill of 70 tokens");
    const ts::Status st = kv.increment(C);
    require(st.is_ok(), "increment after the prefill");
    for (auto &l : lens) l += C;
    require(kv.get_seq_len(0) == (uint32_t)C && kv.get_seq_len(1) == (uint32_t)C, "lengths after the prefill");

    // decode steps
    const uint64_t wsb = kv.decode_workspace_bytes(NH);
    Dev<uint8_t> ws(wsb);
    for (int t = 0; t < steps; t++) {
        const std::vector<float> k1 = normal(g, (size_t)S * H * hd), v1 = normal(g, (size_t)S * H * hd);
        const std::vector<float> q1 = normal(g, (size_t)S * NH * hd);
        Dev<float> dk1(k1), dv1(v1), dq1(q1), do1((size_t)S * NH * hd);
        kv.attn_decode_append(1, dk1.p, dv1.p, dq1.p, NH, rope, do1.p, ws.p, wsb, /*advance=*/true);
        or_append_batch(okp.data(), ovp.data(), oks.data(), ovs.data(), S, P, H, hd, hd, table.data(), k1.data(),
                        v1.data(), lens.data(), 1, nullptr, nullptr, nullptr, 1e-6f);
        std::vector<float> r1((size_t)S * NH * hd);
        or_attend_batch(okp.data(), ovp.data(), oks.data(), ovs.data(), S, P, NH, H, hd, hd, table.data(), q1.data(),
                        lens.data(), 1, 0.0f, r1.data(), 4, nullptr, nullptr, 1e-6f);
        expect_close(do1.host(), r1, "decode step " + std::to_string(t));
        for (auto &l : lens) l += 1;
        require(kv.get_seq_len(0) == (uint32_t)lens[0], "the fused launch advanced the lengths");
    }
    // the cache, bit-exact
    for (int s = 0; s < S; s++) {
        const Exported e = export_layer(kv, 1, s, lens[s]);
        const size_t nw = (size_t)lens[s] * H * (hd / 8), ns = (size_t)lens[s] * H;
        require(std::memcmp(e.kp.data(), okp.data() + s * wrow, nw * 4) == 0, "K words bit-exact");
        require(std::memcmp(e.vp.data(), ovp.data() + s * wrow, nw * 4) == 0, "V words bit-exact");
        require(std::memcmp(e.ks.data(), oks.data() + s * srow, ns * 4) == 0, "K scales bit-exact");
        require(std::memcmp(e.vs.data(), ovs.data() + s * srow, ns * 4) == 0, "V scales bit-exact");
    }
}

// KVCache's bookkeeping and error behaviour (kv_cache.rs:236-293, :366-369).
void test_kv_cache_bookkeeping() {
    ts::KVCache kv = ts::KVCache::new_int4(3, 8, 64, 16, 2);
    require(kv.is_int4() && kv.max_len() == 16 && kv.get_seq_len() == 0, "a new cache is empty");
    require(kv.calculate_offset(2, 3, 5) == ((2u * 8 + 3) * 64 + 5) * 4, "calculate_offset");
    require(kv.increment(16).is_ok() && kv.get_seq_len(1) == 16, "increment to the window");
    const ts::Status over = kv.increment();
    require(over.is_err() && over.code == TS_ERR_OVERFLOW && !over.message.empty(), "increment past the window is Err");
    require(kv.get_seq_len(0) == 16, "a refused increment changes nothing");
    bool threw = false;
    try {
        kv.set_seq_len(17, 0);
    } catch (const ts::Error &e) {
        threw = e.code() == TS_ERR_OVERFLOW;
    }
    require(threw, "set_seq_len past the window throws (the reference panics)");
    kv.set_seq_len(5, 1);
    kv.advance_window_base(3, 1);
    require(kv.get_seq_len(1) == 5 && kv.get_window_base(1) == 3 && kv.get_window_base(0) == 0, "per-sequence state");
    kv.reset(1, nullptr);
    require(kv.get_seq_len(1) == 0 && kv.get_window_base(1) == 0 && kv.get_seq_len(0) == 16, "reset of one sequence");
    kv.reset();
    require(kv.get_seq_len(0) == 0, "reset");
    threw = false;
    try {
        (void)ts::KVCache::new_int4(1, 8, 60, 16);
    } catch (const ts::Error &e) {
        threw = e.code() == TS_ERR_INVALID;
    }
    require(threw, "head_dim not a multiple of 8 throws (the reference asserts)");
}

}  // namespace

int main() {
    const std::pair<const char *, std::function<void()>> tests[] = {
        {"test_quantize_kv_single_head_parity", test_quantize_kv_single_head_parity},
        {"test_quantize_kv_multi_head_independent_scales", test_quantize_kv_multi_head_independent_scales},
        {"test_quantize_kv_zero_vector_no_nan", test_quantize_kv_zero_vector_no_nan},
        {"test_quantize_kv_extreme_values_clamped", test_quantize_kv_extreme_values_clamped},
        {"test_prefill_then_decode_against_oracle", test_prefill_then_decode_against_oracle},
        {"test_kv_cache_bookkeeping", test_kv_cache_bookkeeping},
    };
    int failed = 0;
    for (const auto &t : tests) {
        std::printf("%s ...\n", t.first);
        std::fflush(stdout);
        try {
            t.second();
            std::printf("PASS %s\n", t.first);
        } catch (const Failure &f) {
            std::printf("FAIL %s: %s\n", t.first, f.msg.c_str());
            failed++;
        } catch (const std::exception &e) {
            std::printf("FAIL %s: exception %s\n", t.first, e.what());
            failed++;
        }
        std::fflush(stdout);
    }
    std::printf("%d of %zu passed\n", (int)(sizeof tests / sizeof tests[0]) - failed, sizeof tests / sizeof tests[0]);
    return failed ? 1 : 0;
}
