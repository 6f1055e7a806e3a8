// ts_probe.hip -- HBM streaming ceilings for the decode's access pattern (a measurement tool,
// not part of the C ABI in include/turboshimmy.h; bench.py --stream-ceiling loads it).
//
// probe_decode_loads_kernel reads exactly what one ts_attn_decode launch of the G <= 4 kernel
// reads, in the same way: one workgroup of 4 waves per (sequence, kv head) stream, 64-position
// windows round robin over the waves starting at a per-workgroup offset, every K/V instruction
// one contiguous kilobyte, non-temporal, scales 16 bytes per 4 lanes, one window in flight
// while the previous one is consumed.  Consuming is an XOR into a register, so the launch time
// is the memory system's time for this pattern.  probe_flat_read_kernel reads one flat buffer
// grid-strided (every workgroup a different 4 KB piece at a time), the pattern HBM likes best.
// probe_mfma_rate_kernel issues independent matrix-core instructions back to back, 4 chains
// per wave, so the launch time is the matrix cores' issue rate for that instruction.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int kNT = 2;  // non-temporal

struct ProbeArgs {
    const uint8_t *kp, *vp;  // [rows][P/64][64 * HD / 2] and [rows][P/32][HD * 16] bytes
    const float *ks, *vs;    // [rows][P]
    int P, n_ctx;
    uint32_t *sink;
    // null, or per workgroup (row): start and end of its loads on the 100 MHz constant clock
    // (s_memrealtime) and the XCD it ran on (hardware register XCC_ID)
    uint64_t *stamps;
};

// XCC_ID (hardware register 20 on gfx94x/gfx950), bits 0..3: the XCD of this wave.
__device__ inline uint32_t xcd_id() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 0xFu; }

template <int HD>
__global__ __launch_bounds__(256, 1) void probe_decode_loads_kernel(ProbeArgs a) {
    constexpr int NW = 4, ROWB = HD / 2, NKW = HD / 8, NTD = HD / 16;
    const int row = blockIdx.y * gridDim.x + blockIdx.x;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int end = a.n_ctx;
    const uint32_t wend = (uint32_t)((end + 63) & ~63);
    const auto rk = rsrc(a.kp + (size_t)row * a.P * ROWB, wend * ROWB);
    const auto rv = rsrc(a.vp + (size_t)row * (a.P / 32) * (HD * 16), (uint32_t)((end + 31) / 32) * (HD * 16));
    const auto rs = rsrc(a.ks + (size_t)row * a.P, wend * 4);
    const auto rt = rsrc(a.vs + (size_t)row * a.P, wend * 4);
    const int nwin = (end + 63) >> 6;
    const int cnt = wave < nwin ? (nwin - wave + NW - 1) / NW : 0;
    const int rot = cnt ? (int)((unsigned)(blockIdx.y * 13 + blockIdx.x * 5) % (unsigned)cnt) : 0;
    auto win_base = [&](int i) {
        if (i >= cnt) return 64 * nwin;
        int r = i + rot;
        r = r >= cnt ? r - cnt : r;
        return 64 * (wave + NW * r);
    };
    u32x4 buf[2][NKW / 4 + NTD / 2 + 2];
    auto load = [&](u32x4 *w, int base) {
#pragma unroll
        for (int j = 0; j < NKW / 4; j++) w[j] = __builtin_amdgcn_raw_buffer_load_b128(rk, lane * 16 + j * 1024, base * ROWB, kNT);
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int q = 0; q < NTD / 4; q++)
                w[NKW / 4 + b * (NTD / 4) + q] =
                    __builtin_amdgcn_raw_buffer_load_b128(rv, lane * 16 + q * 1024 + b * (HD * 16), (base / 32) * (HD * 16), kNT);
        w[NKW / 4 + NTD / 2] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane & 15) * 16, base * 4, kNT);
        w[NKW / 4 + NTD / 2 + 1] = __builtin_amdgcn_raw_buffer_load_b128(rt, (lane & 15) * 16, base * 4, kNT);
    };
    uint32_t acc = 0;
    uint64_t t0 = 0;
    if (a.stamps) t0 = __builtin_amdgcn_s_memrealtime();
    load(buf[0], win_base(0));
    for (int it = 0; it < cnt; it += 2) {
#pragma unroll
        for (int d = 0; d < 2; d++) {
            load(buf[d ^ 1], win_base(it + d + 1));
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            if (it + d < cnt) {
#pragma unroll
                for (int j = 0; j < NKW / 4 + NTD / 2 + 2; j++) acc ^= buf[d][j].x ^ buf[d][j].y ^ buf[d][j].z ^ buf[d][j].w;
            }
        }
    }
    if (acc == 0x9E3779B9u) a.sink[0] = acc;  // keeps the loads; practically never taken
    if (a.stamps) {
        __syncthreads();  // every wave's last window consumed
        if (threadIdx.x == 0) {
            a.stamps[3 * row] = t0;
            a.stamps[3 * row + 1] = __builtin_amdgcn_s_memrealtime();
            a.stamps[3 * row + 2] = xcd_id();
        }
    }
}

// The same reads handed out dynamically: units of UW windows of one stream (unit u: chunk u /
// rows of stream u % rows) claimed one at a time from a device counter by a persistent grid,
// the next claim issued while the current unit streams.  Measures what a launch-wide work
// queue costs against the static placement above (no per-workgroup start offset is possible:
// all workgroups start at unit 0, 1, 2, ...).
template <int HD>
__global__ __launch_bounds__(256, 1) void probe_claim_loads_kernel(ProbeArgs a, int rows, int uw, int *ctr) {
    constexpr int NW = 4, ROWB = HD / 2, NKW = HD / 8, NTD = HD / 16, NL = NKW / 4 + NTD / 2 + 2;
    __shared__ int cl[2];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwin = a.n_ctx / 64, nunits = (nwin / uw) * rows;
    if (threadIdx.x == 0) cl[0] = atomicAdd(ctr, 1);
    __syncthreads();
    int u = cl[0], par = 1;
    uint32_t acc = 0;
    while (u < nunits) {  // every workgroup leaves once a claim passes the last unit
        if (threadIdx.x == 0) cl[par] = atomicAdd(ctr, 1);
        const int c = u / rows, row = u % rows;
        const uint32_t wend = (uint32_t)a.n_ctx;
        const auto rk = rsrc(a.kp + (size_t)row * a.P * ROWB, wend * ROWB);
        const auto rv = rsrc(a.vp + (size_t)row * (a.P / 32) * (HD * 16), wend / 32 * (HD * 16));
        const auto rs = rsrc(a.ks + (size_t)row * a.P, wend * 4);
        const auto rt = rsrc(a.vs + (size_t)row * a.P, wend * 4);
        const int cnt = uw / NW;
        u32x4 buf[2][NL];
        auto load = [&](u32x4 *w, int base) {
#pragma unroll
            for (int j = 0; j < NKW / 4; j++) w[j] = __builtin_amdgcn_raw_buffer_load_b128(rk, lane * 16 + j * 1024, base * ROWB, kNT);
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int q = 0; q < NTD / 4; q++)
                    w[NKW / 4 + b * (NTD / 4) + q] =
                        __builtin_amdgcn_raw_buffer_load_b128(rv, lane * 16 + q * 1024 + b * (HD * 16), (base / 32) * (HD * 16), kNT);
            w[NKW / 4 + NTD / 2] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane & 15) * 16, base * 4, kNT);
            w[NKW / 4 + NTD / 2 + 1] = __builtin_amdgcn_raw_buffer_load_b128(rt, (lane & 15) * 16, base * 4, kNT);
        };
        load(buf[0], 64 * (c * uw + wave));
        for (int it = 0; it < cnt; it += 2) {
#pragma unroll
            for (int d = 0; d < 2; d++) {
                load(buf[d ^ 1], it + d + 1 < cnt ? 64 * (c * uw + wave + NW * (it + d + 1)) : a.n_ctx);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                if (it + d < cnt) {
#pragma unroll
                    for (int j = 0; j < NL; j++) acc ^= buf[d][j].x ^ buf[d][j].y ^ buf[d][j].z ^ buf[d][j].w;
                }
            }
        }
        __syncthreads();
        u = cl[par];
        par ^= 1;
        __syncthreads();
    }
    if (acc == 0x9E3779B9u) a.sink[0] = acc;
}

__global__ __launch_bounds__(256) void probe_empty_kernel(uint32_t *sink) {
    if (threadIdx.x == 1000) sink[0] = 1;  // never: the launch itself is what is timed
}

template <int UN>
__global__ __launch_bounds__(256) void probe_flat_read_kernel(const u32x4 *__restrict__ p, size_t n, uint32_t *sink) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * 256 * UN;
    for (size_t i = (size_t)blockIdx.x * 256 * UN + threadIdx.x; i < n; i += stride) {
        u32x4 t[UN];
#pragma unroll
        for (int u = 0; u < UN; u++) t[u] = i + u * 256 < n ? __builtin_nontemporal_load(p + i + u * 256) : (u32x4)0u;
#pragma unroll
        for (int u = 0; u < UN; u++) acc ^= t[u].x ^ t[u].y ^ t[u].z ^ t[u].w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

typedef _Float16 half8p __attribute__((ext_vector_type(8)));
typedef int int8p __attribute__((ext_vector_type(8)));
typedef float float16p __attribute__((ext_vector_type(16)));

// KIND 0: v_mfma_f32_32x32x16_f16; 1: v_mfma_scale_f32_32x32x64_f8f6f4 with fp6 e2m3 operands;
// 2: the same with fp8 e4m3 operands; 3: fp6 A, fp8 B.
template <int KIND>
__global__ __launch_bounds__(256) void probe_mfma_rate_kernel(int iters, float *sink) {
    float16p c0 = (float16p)0.0f, c1 = (float16p)0.0f, c2 = (float16p)0.0f, c3 = (float16p)0.0f;
    const int l = threadIdx.x;
    const int8p a = {l, l + 1, l + 2, l + 3, l + 4, l + 5, 0, 0};
    const int8p b = {l, l + 1, l + 2, l + 3, l + 4, l + 5, l + 6, l + 7};
    const half8p h = (half8p)(_Float16)(l * 0.001f);
    for (int i = 0; i < iters; i++) {
        if constexpr (KIND == 0) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, h, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, h, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, h, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, h, c3, 0, 0, 0);
        } else {
            constexpr int FA = KIND == 2 ? 0 : 2, FB = KIND == 1 ? 2 : 0;
            const int8p aa = KIND == 2 ? b : a, bb = KIND == 1 ? a : b;
            c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aa, bb, c0, FA, FB, 0, 127, 0, 127);
            c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aa, bb, c1, FA, FB, 0, 127, 0, 127);
            c2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aa, bb, c2, FA, FB, 0, 127, 0, 127);
            c3 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aa, bb, c3, FA, FB, 0, 127, 0, 127);
        }
    }
    const float16p c = c0 + c1 + c2 + c3;
    float t = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; v++) t += c[v];
    if (t == 1234.5f) sink[0] = t;  // keeps the chains live
}

}  // namespace

// One launch of `grid` 256-thread workgroups, each wave issuing 4 * iters matrix-core
// instructions of kind `kind` (see probe_mfma_rate_kernel); returns a hipError_t.  Flops per
// instruction: 32768 for kind 0, 131072 for the others.
extern "C" int ts_probe_mfma_rate(int kind, int grid, int iters, void *sink, void *stream) {
    if (grid <= 0 || iters <= 0) return (int)hipErrorInvalidValue;
    const hipStream_t st = (hipStream_t)stream;
    float *sk = (float *)sink;
    switch (kind) {
        case 0: probe_mfma_rate_kernel<0><<<grid, 256, 0, st>>>(iters, sk); break;
        case 1: probe_mfma_rate_kernel<1><<<grid, 256, 0, st>>>(iters, sk); break;
        case 2: probe_mfma_rate_kernel<2><<<grid, 256, 0, st>>>(iters, sk); break;
        case 3: probe_mfma_rate_kernel<3><<<grid, 256, 0, st>>>(iters, sk); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// One loads-only pass of the decode pattern over rows = n_seq * n_kv streams of n_ctx
// positions (P = padded positions per stream, a multiple of 64).  Returns a hipError_t.
// stamps: null, or 3 x n_seq x n_kv u64 (per workgroup: start, end, XCD).
extern "C" int ts_probe_decode_loads(const void *kp, const void *vp, const void *ks, const void *vs,
                                     int n_seq, int n_kv, int hd, int P, int n_ctx, void *sink,
                                     void *stamps, void *stream) {
    if (P % 64 || n_ctx > P || n_ctx <= 0 || n_seq <= 0 || n_kv <= 0) return (int)hipErrorInvalidValue;
    ProbeArgs a{(const uint8_t *)kp, (const uint8_t *)vp, (const float *)ks, (const float *)vs, P, n_ctx,
                (uint32_t *)sink, (uint64_t *)stamps};
    const dim3 grid(n_kv, n_seq);
    // one workgroup per CU, as the decode's plan places them: an unused LDS reservation of
    // more than half the CU's 160 KB keeps a second one off
    const size_t lds = 96 * 1024;
    if (hd == 128) {
        hipFuncSetAttribute((const void *)probe_decode_loads_kernel<128>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        probe_decode_loads_kernel<128><<<grid, 256, lds, (hipStream_t)stream>>>(a);
    } else if (hd == 64) {
        hipFuncSetAttribute((const void *)probe_decode_loads_kernel<64>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        probe_decode_loads_kernel<64><<<grid, 256, lds, (hipStream_t)stream>>>(a);
    } else {
        return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// One grid-strided read of n16 16-byte elements.
extern "C" int ts_probe_flat_read(const void *p, size_t n16, int grid, void *sink, void *stream) {
    probe_flat_read_kernel<4><<<grid, 256, 0, (hipStream_t)stream>>>((const u32x4 *)p, n16, (uint32_t *)sink);
    return (int)hipGetLastError();
}

// The decode reads as units of uw windows (uw a multiple of 8 dividing n_ctx / 64) claimed from
// *counter (zeroed by the caller before each launch) by n_wg persistent workgroups.
extern "C" int ts_probe_claim_loads(const void *kp, const void *vp, const void *ks, const void *vs,
                                    int n_seq, int n_kv, int hd, int P, int n_ctx, int uw, int n_wg,
                                    int *counter, void *sink, void *stream) {
    if (hd != 128 || P % 64 || n_ctx > P || n_ctx % 64 || uw <= 0 || uw % 8 || (n_ctx / 64) % uw || n_wg <= 0 || !counter)
        return (int)hipErrorInvalidValue;
    ProbeArgs a{(const uint8_t *)kp, (const uint8_t *)vp, (const float *)ks, (const float *)vs, P, n_ctx,
                (uint32_t *)sink};
    const size_t lds = 96 * 1024;
    hipFuncSetAttribute((const void *)probe_claim_loads_kernel<128>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    probe_claim_loads_kernel<128><<<n_wg, 256, lds, (hipStream_t)stream>>>(a, n_seq * n_kv, uw, counter);
    return (int)hipGetLastError();
}

// An empty launch of `grid` workgroups (the per-launch cost of a kernel in a graph).
extern "C" int ts_probe_empty(int grid, void *sink, void *stream) {
    probe_empty_kernel<<<grid, 256, 0, (hipStream_t)stream>>>((uint32_t *)sink);
    return (int)hipGetLastError();
}

// Launch n instantiated graphs in order on one stream from a compiled loop: the timed steps of
// bench.py --host-loop c, so that the host's cost per step is that of hipGraphLaunch alone (as
// for a compiled host such as the reference's Rust one) and not the Python interpreter's.
extern "C" int ts_probe_graph_launch(void *const *execs, int n, void *stream) {
    if (n < 0 || (n > 0 && !execs)) return (int)hipErrorInvalidValue;
    for (int i = 0; i < n; i++) {
        const hipError_t e = hipGraphLaunch((hipGraphExec_t)execs[i], (hipStream_t)stream);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

// n_steps decode steps of n_layers layers from a compiled loop, each layer one call of the
// library's ts_attn_decode_append (fn_mid) or, for the step's last layer,
// ts_attn_decode_append_advance (fn_last), with the function pointers the caller looked up in
// libturboshimmy.so: what a compiled host (the reference's Rust one) would issue per step.
// k, v, q: n_sets x n_layers device pointers, step i taking set i % n_sets.
typedef int (*ts_probe_decode_fn)(void *kv, int32_t layer, const float *k, const float *v, const float *q,
                                  int32_t n_head, const void *rope, float softcap, float *out, void *ws,
                                  uint64_t ws_bytes, void *stream);
extern "C" int ts_probe_decode_steps(void *fn_mid, void *fn_last, void *kv, int n_layers, int n_steps, int n_sets,
                                     const float *const *k, const float *const *v, const float *const *q,
                                     int n_head, const void *rope, float *out, void *ws, uint64_t ws_bytes,
                                     void *stream) {
    if (!fn_mid || !fn_last || n_layers <= 0 || n_steps < 0 || n_sets <= 0) return (int)hipErrorInvalidValue;
    const ts_probe_decode_fn mid = (ts_probe_decode_fn)fn_mid, last = (ts_probe_decode_fn)fn_last;
    for (int i = 0; i < n_steps; i++) {
        const int set = i % n_sets;
        for (int l = 0; l < n_layers; l++) {
            const size_t at = (size_t)set * n_layers + l;
            const int rc = (l == n_layers - 1 ? last : mid)(kv, l, k[at], v[at], q[at], n_head, rope, 0.0f, out,
                                                             ws, ws_bytes, stream);
            if (rc != 0) return rc;
        }
    }
    return 0;
}
