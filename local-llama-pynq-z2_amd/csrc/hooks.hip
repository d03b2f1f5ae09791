// Test hooks of include/llm_hip.h: single device stages on caller data, for the parity tests.
#include <string.h>

#include <vector>

#include "../../include/llm_hip.h"
#include "host_common.h"
#include "prefill.h"
#include "ref_expf.h"
#include "seqsum.h"

namespace {
int hook_device(const char *who) {
    const int dev = hip_device_from_env(who);
    if (dev < 0) return -1;
    HIP_OR_FAIL(who, hipSetDevice(dev));
    return 0;
}
} // namespace

extern "C" int mvh_quantize(const float *x, int n, int flavor, int gs, int8_t *q, float *s) {
    if (!x || !q || !s || n <= 0 || (gs != 32 && gs != 64) || n % gs || (flavor != QF_QWEN && flavor != QF_RUNQ) ||
        (flavor == QF_QWEN && gs != 32) || n > 8192) {
        fprintf(stderr, "mvh_quantize: bad arguments (n=%d gs=%d flavor=%d)\n", n, gs, flavor);
        return -1;
    }
    if (hook_device("mvh_quantize")) return -1;
    float *dx = nullptr, *ds = nullptr;
    int8_t *dq = nullptr;
    int rc = -1;
    if (hipMalloc(&dx, (size_t)n * 4) == hipSuccess && hipMalloc(&dq, (size_t)n) == hipSuccess &&
        hipMalloc(&ds, (size_t)n / gs * 4) == hipSuccess &&
        hipMemcpy(dx, x, (size_t)n * 4, hipMemcpyHostToDevice) == hipSuccess &&
        launch_quantize_test(dx, n, flavor, gs, dq, ds, 0) == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(q, dq, (size_t)n, hipMemcpyDeviceToHost) == hipSuccess &&
        hipMemcpy(s, ds, (size_t)n / gs * 4, hipMemcpyDeviceToHost) == hipSuccess)
        rc = 0;
    else
        fprintf(stderr, "mvh_quantize: HIP error %s\n", hipGetErrorString(hipGetLastError()));
    hipFree(dx);
    hipFree(dq);
    hipFree(ds);
    return rc;
}

extern "C" int mvh_group_dots(const uint8_t *w, const int8_t *xq, int n, int d, int bits, int gs, int32_t *ival) {
    const int wbits = bits == 0 ? 8 : bits;
    if (!w || !xq || !ival || n <= 0 || d <= 0 || (bits != 0 && bits != 4 && bits != 8) || (gs != 32 && gs != 64) ||
        (bits != 0 && gs != 32) || n % gs) {
        fprintf(stderr, "mvh_group_dots: bad arguments (n=%d d=%d bits=%d gs=%d)\n", n, d, bits, gs);
        return -1;
    }
    if (hook_device("mvh_group_dots")) return -1;
    const int ng = n / gs;
    TiledMat T = tiled_describe(d, n, gs, wbits, 0, 16);
    const size_t wbytes = (size_t)d * n * wbits / 8, sbytes = (size_t)d * ng * 2;
    uint8_t *dw = nullptr, *dsc = nullptr, *dt = nullptr;
    int8_t *dx = nullptr;
    int32_t *di = nullptr;
    int *dmap = nullptr;
    std::vector<int> map(d);
    for (int i = 0; i < d; i++) map[i] = i;
    int rc = -1;
    if (hipMalloc(&dw, wbytes) == hipSuccess && hipMalloc(&dsc, sbytes) == hipSuccess &&
        hipMalloc(&dt, T.bytes) == hipSuccess && hipMalloc(&dx, (size_t)n) == hipSuccess &&
        hipMalloc(&di, (size_t)d * ng * 4) == hipSuccess && hipMalloc(&dmap, (size_t)d * 4) == hipSuccess &&
        hipMemcpy(dw, w, wbytes, hipMemcpyHostToDevice) == hipSuccess && hipMemset(dsc, 0, sbytes) == hipSuccess &&
        hipMemcpy(dx, xq, (size_t)n, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(dmap, map.data(), (size_t)d * 4, hipMemcpyHostToDevice) == hipSuccess) {
        T.data = dt;
        RepackArgs ra;
        memset(&ra, 0, sizeof ra);
        ra.T = T;
        ra.w[0] = dw;
        ra.s[0] = dsc;
        ra.rowmap = dmap;
        if (launch_repack(ra, 0) == hipSuccess && launch_group_dots_test(T, dx, di, 0) == hipSuccess &&
            hipDeviceSynchronize() == hipSuccess &&
            hipMemcpy(ival, di, (size_t)d * ng * 4, hipMemcpyDeviceToHost) == hipSuccess)
            rc = 0;
    }
    if (rc) fprintf(stderr, "mvh_group_dots: HIP error %s\n", hipGetErrorString(hipGetLastError()));
    hipFree(dw);
    hipFree(dsc);
    hipFree(dt);
    hipFree(dx);
    hipFree(di);
    hipFree(dmap);
    return rc;
}

extern "C" int mvh_prefill_gemm(const uint8_t *w, const void *ws, const int8_t *xq, const float *xs, int M, int n,
                                int d, int bits, int gs, int rb, int shape, float *y) {
    const int wbits = bits == 0 ? 8 : bits, sf32 = bits == 0;
    if (!w || !ws || !xq || !xs || !y || M < 1 || n <= 0 || d <= 0 || d % 4 || n % 16 ||
        (bits != 0 && bits != 4 && bits != 8) || (gs != 32 && gs != 64) || (bits != 0 && gs != 32) || n % gs ||
        (rb != 8 && rb != 16 && rb != 64) ||
        (shape != 0 && shape != 11 && shape != 12 && shape != 14 && shape != 21 && shape != 22 && shape != 24 &&
         shape != 41 && shape != 42)) {
        fprintf(stderr, "mvh_prefill_gemm: bad arguments (M=%d n=%d d=%d bits=%d gs=%d rb=%d shape=%d)\n", M, n, d,
                bits, gs, rb, shape);
        return -1;
    }
    if (hook_device("mvh_prefill_gemm")) return -1;
    const int ng = n / gs;
    TiledMat T = tiled_describe(d, n, gs, wbits, sf32, rb);
    const size_t wbytes = (size_t)d * n * wbits / 8, sbytes = (size_t)d * ng * (sf32 ? 4 : 2);
    uint8_t *dw = nullptr, *dsc = nullptr, *dt = nullptr;
    int8_t *dx = nullptr;
    float *dxs = nullptr, *dy = nullptr;
    int *dmap = nullptr;
    std::vector<int> map(d);
    for (int i = 0; i < d; i++) map[i] = i;
    // the caller's row-major activations in the GEMM's token-block tiles (padding tokens zero)
    const int MB = pf_blocks(M);
    const size_t abytes = pf_act_bytes(n, M), sfl = pf_scale_floats(ng, M);
    std::vector<int8_t> xt(abytes, 0);
    std::vector<float> st(sfl, 0.0f);
    for (int m = 0; m < M; m++) {
        for (int k = 0; k < n; k++) xt[pf_act_off(m, k, MB)] = xq[(size_t)m * n + k];
        for (int g = 0; g < ng; g++) st[pf_scale_off(m, g, MB)] = xs[(size_t)m * ng + g];
    }
    int rc = -1;
    if (hipMalloc(&dw, wbytes) == hipSuccess && hipMalloc(&dsc, sbytes) == hipSuccess &&
        hipMalloc(&dt, T.bytes) == hipSuccess && hipMalloc(&dx, abytes) == hipSuccess &&
        hipMalloc(&dxs, sfl * 4) == hipSuccess && hipMalloc(&dy, (size_t)M * d * 4) == hipSuccess &&
        hipMalloc(&dmap, (size_t)d * 4) == hipSuccess &&
        hipMemcpy(dw, w, wbytes, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(dsc, ws, sbytes, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(dx, xt.data(), abytes, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(dxs, st.data(), sfl * 4, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(dmap, map.data(), (size_t)d * 4, hipMemcpyHostToDevice) == hipSuccess) {
        T.data = dt;
        RepackArgs ra;
        memset(&ra, 0, sizeof ra);
        ra.T = T;
        ra.w[0] = dw;
        ra.s[0] = dsc;
        ra.rowmap = dmap;
        PgemmArgs g;
        memset(&g, 0, sizeof g);
        g.W = T;
        g.xq = dx;
        g.xs = dxs;
        g.y = dy;
        g.M = M;
        g.shape = shape;
        int dev = 0;
        hipGetDevice(&dev);
        g.simds = 4 * hip_cu_count(dev);
        if (launch_repack(ra, 0) == hipSuccess && launch_pgemm(wbits, gs, sf32, g, 0) == hipSuccess &&
            hipDeviceSynchronize() == hipSuccess &&
            hipMemcpy(y, dy, (size_t)M * d * 4, hipMemcpyDeviceToHost) == hipSuccess)
            rc = 0;
    }
    if (rc) fprintf(stderr, "mvh_prefill_gemm: HIP error %s\n", hipGetErrorString(hipGetLastError()));
    hipFree(dw);
    hipFree(dsc);
    hipFree(dt);
    hipFree(dx);
    hipFree(dxs);
    hipFree(dy);
    hipFree(dmap);
    return rc;
}

static int sample_hook(const char *who, int strict, const float *logits, int n, int count, float temperature,
                       float topp, unsigned long long *rng, int *rows, int skew = 0) {
    if (!logits || !rng || !rows || n < 2 || count < 1 || !(temperature > 0.0f)) {
        fprintf(stderr, "%s: bad arguments (n=%d count=%d temperature=%g)\n", who, n, count, temperature);
        return -1;
    }
    if (hook_device(who)) return -1;
    float *dl = nullptr, *dp = nullptr;
    int *dr = nullptr;
    SamplerState *dss = nullptr;
    void *dsc = nullptr; // the many-workgroup draw's buffers (taken for large n), or the strict draw's
    SamplerState st;
    st.temperature = temperature;
    st.topp = topp;
    st.rng = *rng;
    int rc = -1;
    const size_t ld = ((size_t)n + 3) & ~(size_t)3; // 16-byte aligned rows
    if (hipMalloc(&dl, (size_t)count * ld * 4) == hipSuccess && hipMalloc(&dp, (size_t)n * 4) == hipSuccess &&
        hipMalloc(&dr, (size_t)count * 4) == hipSuccess && hipMalloc(&dss, sizeof st) == hipSuccess &&
        hipMalloc(&dsc, strict ? sample_strict_scratch_bytes() : sample_scratch_bytes()) == hipSuccess &&
        hipMemcpy2D(dl, ld * 4, logits, (size_t)n * 4, (size_t)n * 4, count, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(dss, &st, sizeof st, hipMemcpyHostToDevice) == hipSuccess &&
        (!strict || sample_strict_set_skew(dsc, skew) == hipSuccess)) {
        rc = 0;
        for (int c = 0; c < count && !rc; c++) {
            SampleArgs a;
            memset(&a, 0, sizeof a);
            a.logits = dl + (size_t)c * ld;
            a.n = n;
            a.probs = dp;
            a.ss = dss;
            a.out_row = dr + c;
            a.scratch = strict ? nullptr : dsc;
            a.strict = strict;
            a.strict_scratch = strict ? dsc : nullptr;
            a.path = topp > 0.0f && topp < 1.0f ? 1 : 0;
            if (launch_sample(a, 0) != hipSuccess) rc = -1;
        }
        if (!rc && (hipDeviceSynchronize() != hipSuccess ||
                    hipMemcpy(rows, dr, (size_t)count * 4, hipMemcpyDeviceToHost) != hipSuccess ||
                    hipMemcpy(&st, dss, sizeof st, hipMemcpyDeviceToHost) != hipSuccess))
            rc = -1;
    }
    if (rc) fprintf(stderr, "%s: HIP error %s\n", who, hipGetErrorString(hipGetLastError()));
    else *rng = st.rng;
    hipFree(dl);
    hipFree(dp);
    hipFree(dr);
    hipFree(dss);
    hipFree(dsc);
    return rc;
}

extern "C" int mvh_sample(const float *logits, int n, int count, float temperature, float topp,
                          unsigned long long *rng, int *rows) {
    return sample_hook("mvh_sample", 0, logits, n, count, temperature, topp, rng, rows);
}

extern "C" int mvh_sample_strict(const float *logits, int n, int count, float temperature, float topp,
                                 unsigned long long *rng, int *rows) {
    return sample_hook("mvh_sample_strict", 1, logits, n, count, temperature, topp, rng, rows);
}

extern "C" int mvh_sample_strict_skew(const float *logits, int n, int count, float temperature, float topp,
                                      unsigned long long *rng, int *rows, int skew) {
    return sample_hook("mvh_sample_strict_skew", 1, logits, n, count, temperature, topp, rng, rows, skew);
}

// ref_expf (the reference libm's expf, used by the strict mode) over caller data, on the device and, with the
// same source compiled for the host, on the CPU; the tests hold both to the C library's own expf
__global__ void k_ref_expf(const float *x, int n, float *y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = ref_expf(x[i]);
}

extern "C" int mvh_ref_expf(const float *x, int n, float *y) {
    if (!x || !y || n <= 0 || n > (1 << 26)) {
        fprintf(stderr, "mvh_ref_expf: bad arguments (n=%d)\n", n);
        return -1;
    }
    if (hook_device("mvh_ref_expf")) return -1;
    float *dx = nullptr, *dy = nullptr;
    int rc = -1;
    if (hipMalloc(&dx, (size_t)n * 4) == hipSuccess && hipMalloc(&dy, (size_t)n * 4) == hipSuccess &&
        hipMemcpy(dx, x, (size_t)n * 4, hipMemcpyHostToDevice) == hipSuccess) {
        hipLaunchKernelGGL(k_ref_expf, dim3((n + 255) / 256), dim3(256), 0, 0, dx, n, dy);
        if (hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
            hipMemcpy(y, dy, (size_t)n * 4, hipMemcpyDeviceToHost) == hipSuccess)
            rc = 0;
    }
    if (rc) fprintf(stderr, "mvh_ref_expf: HIP error %s\n", hipGetErrorString(hipGetLastError()));
    hipFree(dx);
    hipFree(dy);
    return rc;
}

// The strict mode's sequential sums on their own: block_seq_sum (the RMSNorm sum of squares, the long softmax
// sums), wave_seq_sum (the short softmax sums) and seq_sum (a GEMV row's group products, one thread).
template <int WHICH>
__global__ void __launch_bounds__(1024) k_seq_sum(const float *x, int n, float *out) {
    extern __shared__ __align__(16) float s_terms[];
    for (int i = threadIdx.x; i < n; i += blockDim.x) s_terms[i] = x[i];
    __syncthreads();
    float s = 0.0f;
    if constexpr (WHICH == 0) {
        s = block_seq_sum(s_terms, n, (uint8_t *)(s_terms + ((n + 3) & ~3)));
    } else if constexpr (WHICH == 1) {
        if (threadIdx.x < WAVE) s = wave_seq_sum(s_terms, n);
    } else {
        if (threadIdx.x == 0) s = seq_sum(s_terms, n);
    }
    if (threadIdx.x == 0) out[0] = s;
}

extern "C" int mvh_seq_sum(const float *x, int n, int which, int threads, float *out) {
    if (!x || !out || n < 1 || n > 8192 || which < 0 || which > 2 ||
        (which == 0 && (threads < WAVE || threads > SEQ_MAX_WAVES * WAVE || threads % WAVE))) {
        fprintf(stderr, "mvh_seq_sum: bad arguments (n=%d which=%d threads=%d)\n", n, which, threads);
        return -1;
    }
    if (hook_device("mvh_seq_sum")) return -1;
    const int nt = which == 0 ? threads : WAVE;
    const size_t lds = (size_t)((n + 3) & ~3) * 4 + seq_sum_scratch_bytes(nt);
    float *dx = nullptr, *dout = nullptr;
    int rc = -1;
    if (hipMalloc(&dx, (size_t)n * 4) == hipSuccess && hipMalloc(&dout, 4) == hipSuccess &&
        hipMemcpy(dx, x, (size_t)n * 4, hipMemcpyHostToDevice) == hipSuccess) {
        if (which == 0) hipLaunchKernelGGL(k_seq_sum<0>, dim3(1), dim3(nt), lds, 0, dx, n, dout);
        else if (which == 1) hipLaunchKernelGGL(k_seq_sum<1>, dim3(1), dim3(nt), lds, 0, dx, n, dout);
        else hipLaunchKernelGGL(k_seq_sum<2>, dim3(1), dim3(nt), lds, 0, dx, n, dout);
        if (hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
            hipMemcpy(out, dout, 4, hipMemcpyDeviceToHost) == hipSuccess)
            rc = 0;
    }
    if (rc) fprintf(stderr, "mvh_seq_sum: HIP error %s\n", hipGetErrorString(hipGetLastError()));
    hipFree(dx);
    hipFree(dout);
    return rc;
}

extern "C" int mvh_ref_expf_host(const float *x, int n, float *y) {
    if (!x || !y || n < 0) return -1;
    for (int i = 0; i < n; i++) y[i] = ref_expf_with(x[i], ref_expf_tab_host);
    return 0;
}

extern "C" int mvh_gemv_shape(int rows, int n, int gs, int wbits, int sf32, int rb, int role, int ordered, int cus,
                              int *out) {
    static const int pro[6] = {PRO_NORM, PRO_ATTN, PRO_NORM, PRO_XQ, PRO_NORM, PRO_XQ};
    static const int epi[6] = {EPI_QKV, EPI_RESID, EPI_SWIGLU, EPI_RESID, EPI_ARGMAX, EPI_STORE};
    if (!out || rows < 1 || n < 1 || (gs != 32 && gs != 64) || n % gs || (wbits != 4 && wbits != 8) ||
        (rb != 8 && rb != 16 && rb != 32 && rb != 64) || role < 0 || role > 5 || cus < 1) {
        fprintf(stderr, "mvh_gemv_shape: bad arguments\n");
        return -1;
    }
    const TiledMat T = tiled_describe(rows, n, gs, wbits, sf32 != 0, rb);
    const GemvShape s = gemv_pick_shape(T, pro[role], epi[role], ordered, cus);
    out[0] = s.kw;
    out[1] = s.nb;
    out[2] = s.grid;
    out[3] = s.ord;
    return s.grid < 1 ? 1 : 0;
}

// A plain streaming read: block b reads its contiguous share of the buffer in 16-byte vectors, 8 in flight per
// thread, with the weight loads' cache policy (0, or 2 = non-temporal), and keeps one word per block so that
// no load is dead.  The floor of any kernel that must read those bytes once.
template <int POLICY>
__global__ void __launch_bounds__(256) k_read_floor(const uint8_t *p, uint32_t bytes, uint32_t *out) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)p, 0, (int)bytes, 0x00020000);
    const uint32_t vecs = bytes / 16, per = (vecs + gridDim.x - 1) / gridDim.x;
    const uint32_t v0 = blockIdx.x * per, v1 = min(v0 + per, vecs);
    uint32_t acc = 0;
    for (uint32_t v = v0 + threadIdx.x; v < v1; v += 8 * 256) {
        uint4 x[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t i = v + u * 256;
            const auto r = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(i < v1 ? i * 16 : 0x80000000u), 0, POLICY);
            x[u] = *(const uint4 *)&r;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) acc ^= x[u].x ^ x[u].y ^ x[u].z ^ x[u].w;
    }
    for (int o = 1; o < 64; o <<= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) atomicXor(&out[blockIdx.x], acc);
}

extern "C" int mvh_read_floor(size_t bytes, int copies, int blocks, int nt, int reps, float *us) {
    if (!us || bytes < 16 || bytes > 0x7fff0000u || copies < 1 || copies > 64 || blocks < 1 || blocks > 65536 ||
        reps < 1 || (size_t)copies * ((bytes + 255) & ~(size_t)255) > ((size_t)8 << 30)) {
        fprintf(stderr, "mvh_read_floor: bad arguments\n");
        return -1;
    }
    if (hook_device("mvh_read_floor")) return -1;
    const size_t stride = (bytes + 255) & ~(size_t)255;
    uint8_t *buf = nullptr;
    uint32_t *out = nullptr;
    hipStream_t st = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = -1;
    if (hipMalloc(&buf, (size_t)copies * stride) == hipSuccess && hipMalloc(&out, (size_t)blocks * 4) == hipSuccess &&
        hipMemset(buf, 0x5a, (size_t)copies * stride) == hipSuccess && hipMemset(out, 0, (size_t)blocks * 4) == hipSuccess &&
        hipStreamCreate(&st) == hipSuccess && hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess &&
        hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) == hipSuccess) {
        for (int c = 0; c < copies; c++) {
            if (nt) hipLaunchKernelGGL(k_read_floor<2>, dim3(blocks), dim3(256), 0, st, buf + c * stride, (uint32_t)bytes, out);
            else hipLaunchKernelGGL(k_read_floor<0>, dim3(blocks), dim3(256), 0, st, buf + c * stride, (uint32_t)bytes, out);
        }
        if (hipStreamEndCapture(st, &g) == hipSuccess && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess &&
            hipGraphLaunch(ge, st) == hipSuccess && hipGraphLaunch(ge, st) == hipSuccess &&
            hipEventRecord(e0, st) == hipSuccess) {
            bool ok = true;
            for (int r = 0; r < reps && ok; r++) ok = hipGraphLaunch(ge, st) == hipSuccess;
            float ms = 0.0f;
            if (ok && hipEventRecord(e1, st) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
                hipEventElapsedTime(&ms, e0, e1) == hipSuccess) {
                *us = ms * 1000.0f / (float)(reps * copies);
                rc = 0;
            }
        }
    }
    if (rc) fprintf(stderr, "mvh_read_floor: HIP error %s\n", hipGetErrorString(hipGetLastError()));
    if (ge) hipGraphExecDestroy(ge);
    if (g) hipGraphDestroy(g);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (st) hipStreamDestroy(st);
    hipFree(buf);
    hipFree(out);
    return rc;
}
