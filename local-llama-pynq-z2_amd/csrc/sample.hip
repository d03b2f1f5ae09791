// On-device sampler of the token loop: temperature, softmax, top-p and the xorshift64* coin of the llama2.c
// sampler that both reference hosts use (qwen.c:578-654, runq.c:830-967), as one 1024-thread workgroup.
//
// The reference (per generated token, on the host):
//   logits /= temperature; softmax (max, expf(x - max), sum, divide); coin = random_f32(&rng);
//   topp outside (0, 1): the first i with coin < cdf_i over the probabilities in index order (sample_mult);
//   else: candidates p_i >= (1 - topp) / (n - 1), sorted by descending probability (qsort), the prefix up to
//   the first cumulative sum > topp, r = coin * that sum, and the first candidate with r < its cdf.
//
// Here the cumulative sums are exact: every probability enters as a 64-bit fixed-point integer (p * 2^56,
// exact for the fp32 values that matter), so sums do not depend on their order.  The plain walk finds its
// crossing through chunk sums of 256 rows and one wave scan.  The top-p walk needs no sort: "the first
// position in descending-probability order (ties by ascending row) where the cumulative mass exceeds T" is
// found by a radix select over the probability bits, 8 bits per level, each level a histogram of masses,
// then the crossing inside a run of equal probabilities by its count in row order.  The reference's
// sequential fp32 sums differ from these exact ones by their rounding only; the coin, the RNG stream and
// every comparison (strict >, first index, the r = coin * cumulative product in fp32) are the reference's.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "device.h"
#include "kernels.h"

#define SMP_T 1024
#define SMP_W (SMP_T / WAVE)
#define SMP_CHUNK 256                                  // rows per chunk of the index-order walks (a float4 per lane)
#define SMP_MAX_CHUNKS 1024                            // n <= 262144
#define SMP_PER_THREAD (SMP_MAX_CHUNKS / SMP_T)        // chunk entries per thread in the chunk scans
#define SMP_UNROLL 8                                   // 16-byte loads in flight per thread in the row passes

typedef unsigned long long u64;

namespace {

struct SmpShared {
    u64 hist0[256];             // radix level 0 (top 8 key bits) over every candidate: mass per bucket
    u64 hist[256];              // deeper radix levels: mass per bucket
    u64 chunk[SMP_MAX_CHUNKS];  // per chunk: mass or count, then exclusive prefixes
    u64 wsum[SMP_W + 1];
    float wf[SMP_W];
    int wi[SMP_W];
    u64 bc_u[2];
    int bc_i[2];
    float bc_f;
};

// fixed-point mass of a probability: p * 2^56, exact for p >= 2^-32 (lower bits of smaller p truncate)
__device__ __forceinline__ u64 fixed_mass(float p) { return (u64)ldexp((double)p, 56); }

// f(row, value) over rows [0, n) of a 16-byte aligned array: each thread takes SMP_UNROLL float4 vectors at
// a time (all loads issued before any use), then the last n % 4 rows one by one
template <typename F>
__device__ __forceinline__ void for_rows(const float *x, int n, F f) {
    const int n4 = n >> 2;
    const float4 *x4 = (const float4 *)x;
    for (int base = threadIdx.x; base < n4; base += SMP_UNROLL * SMP_T) {
        float4 v[SMP_UNROLL];
#pragma unroll
        for (int u = 0; u < SMP_UNROLL; u++) v[u] = x4[min(base + u * SMP_T, n4 - 1)];
#pragma unroll
        for (int u = 0; u < SMP_UNROLL; u++) {
            const int k = base + u * SMP_T;
            if (k < n4) {
                f(4 * k, v[u].x);
                f(4 * k + 1, v[u].y);
                f(4 * k + 2, v[u].z);
                f(4 * k + 3, v[u].w);
            }
        }
    }
    for (int i = 4 * n4 + (int)threadIdx.x; i < n; i += SMP_T) f(i, x[i]);
}

// the four rows of a lane in a chunk (zero past n)
__device__ __forceinline__ float4 chunk_rows(const float *x, int n, int c, int lane) {
    const int i = c * SMP_CHUNK + 4 * lane;
    if (i + 3 < n) return *(const float4 *)(x + i);
    return make_float4(i < n ? x[i] : 0.0f, i + 1 < n ? x[i + 1] : 0.0f, i + 2 < n ? x[i + 2] : 0.0f, 0.0f);
}

__device__ __forceinline__ u64 wave_incl_scan_u64(u64 v) {
    const int lane = threadIdx.x & (WAVE - 1);
    for (int o = 1; o < WAVE; o <<= 1) {
        const u64 u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    return v;
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
    for (int o = 1; o < WAVE; o <<= 1) v += __shfl_xor(v, o);
    return v;
}

// exclusive scan of one u64 per thread in thread order; every thread gets the total
__device__ u64 block_excl_scan_u64(u64 v, SmpShared &sh, u64 *total) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const u64 inc = wave_incl_scan_u64(v);
    if (lane == WAVE - 1) sh.wsum[w] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        u64 run = 0;
        for (int k = 0; k < SMP_W; k++) {
            const u64 t = sh.wsum[k];
            sh.wsum[k] = run;
            run += t;
        }
        sh.wsum[SMP_W] = run;
    }
    __syncthreads();
    const u64 r = sh.wsum[w] + inc - v;
    *total = sh.wsum[SMP_W];
    __syncthreads();
    return r;
}

// Turns sh.chunk[0, nc) into exclusive prefixes; returns the first chunk whose running value passes `t`
// (prefix + entry > t), or -1 (with *total the sum of all entries).
__device__ int chunk_crossing(SmpShared &sh, int nc, u64 t, u64 *total) {
    const int c0 = threadIdx.x * SMP_PER_THREAD;
    u64 s = 0;
    for (int k = 0; k < SMP_PER_THREAD; k++)
        if (c0 + k < nc) s += sh.chunk[c0 + k];
    u64 run = block_excl_scan_u64(s, sh, total);
    int found = 0x7fffffff;
    for (int k = 0; k < SMP_PER_THREAD; k++)
        if (c0 + k < nc) {
            const u64 e = sh.chunk[c0 + k];
            sh.chunk[c0 + k] = run;
            if (found == 0x7fffffff && run + e > t) found = c0 + k;
            run += e;
        }
    // smallest crossing chunk over the block
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    for (int o = 1; o < WAVE; o <<= 1) found = min(found, __shfl_xor(found, o));
    if (lane == 0) sh.wi[w] = found;
    __syncthreads();
    int c = sh.wi[0];
    for (int k = 1; k < SMP_W; k++) c = min(c, sh.wi[k]);
    __syncthreads();
    return c == 0x7fffffff ? -1 : c;
}

// First row in index order where the exact cumulative mass of the rows exceeds t; -1 if none.
__device__ int select_index(const float *p, int n, u64 t, SmpShared &sh) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE, nc = (n + SMP_CHUNK - 1) / SMP_CHUNK;
    for (int c0 = w; c0 < nc; c0 += SMP_UNROLL * SMP_W) { // chunk masses, SMP_UNROLL chunks per wave at a time
        float4 v[SMP_UNROLL];
#pragma unroll
        for (int u = 0; u < SMP_UNROLL; u++) v[u] = chunk_rows(p, n, min(c0 + u * SMP_W, nc - 1), lane);
#pragma unroll
        for (int u = 0; u < SMP_UNROLL; u++) {
            const u64 s = wave_sum_u64(fixed_mass(v[u].x) + fixed_mass(v[u].y) + fixed_mass(v[u].z) +
                                       fixed_mass(v[u].w));
            if (lane == 0 && c0 + u * SMP_W < nc) sh.chunk[c0 + u * SMP_W] = s;
        }
    }
    __syncthreads();
    u64 total;
    const int c = chunk_crossing(sh, nc, t, &total);
    if (c < 0) return -1;
    if (w == 0) {
        const float4 v = chunk_rows(p, n, c, lane);
        const u64 q0 = fixed_mass(v.x), q1 = fixed_mass(v.y), q2 = fixed_mass(v.z), q3 = fixed_mass(v.w);
        const u64 e = sh.chunk[c] + wave_incl_scan_u64(q0 + q1 + q2 + q3) - (q0 + q1 + q2 + q3);
        const int j = e + q0 > t ? 0 : e + q0 + q1 > t ? 1 : e + q0 + q1 + q2 > t ? 2 : e + q0 + q1 + q2 + q3 > t ? 3 : 4;
        const u64 hit = __ballot(j < 4 && c * SMP_CHUNK + 4 * lane + j < n);
        const int l = __builtin_ctzll(hit);
        const int jl = __shfl(j, l);
        if (lane == 0) sh.bc_i[0] = c * SMP_CHUNK + 4 * l + jl;
    }
    __syncthreads();
    const int r = sh.bc_i[0];
    __syncthreads();
    return r;
}

// First position in (descending probability, ascending row) order among the candidates p >= cutoff where
// the exact cumulative mass exceeds t (t < the candidates' total mass); returns the row and, in *through,
// the cumulative mass through it.
__device__ int select_sorted(const float *p, int n, float cutoff, u64 t, SmpShared &sh, u64 *through) {
    unsigned prefix = 0;
    u64 before = 0;
    for (int lvl = 0; lvl < 4; lvl++) {
        const int sh_b = 24 - 8 * lvl;
        const u64 *hist = lvl == 0 ? sh.hist0 : sh.hist; // level 0 is shared by every select of the draw
        if (lvl > 0) {
            for (int b = threadIdx.x; b < 256; b += SMP_T) sh.hist[b] = 0;
            __syncthreads();
            int run_b = -1;
            u64 run_q = 0;
            for_rows(p, n, [&](int, float v) {
                if (!(v >= cutoff)) return;
                const unsigned key = ~__float_as_uint(v); // ascending key = descending probability
                if (lvl > 0 && (key >> (sh_b + 8)) != prefix) return;
                const int b = (key >> sh_b) & 255;
                if (b != run_b) { // runs of one bucket (most rows at the top levels) cost one LDS add
                    if (run_b >= 0) atomicAdd(&sh.hist[run_b], run_q);
                    run_b = b;
                    run_q = 0;
                }
                run_q += fixed_mass(v);
            });
            if (run_b >= 0) atomicAdd(&sh.hist[run_b], run_q);
            __syncthreads();
        }
        if (threadIdx.x == 0) {
            u64 acc = before;
            int chosen = 255;
            for (int b = 0; b < 256; b++) {
                if (acc + hist[b] > t) { chosen = b; break; }
                acc += hist[b];
            }
            sh.bc_u[0] = acc;
            sh.bc_i[0] = chosen;
        }
        __syncthreads();
        before = sh.bc_u[0];
        prefix = (prefix << 8) | (unsigned)sh.bc_i[0];
        __syncthreads();
    }
    // every candidate with key `prefix` has the same mass q: the crossing is the m-th of them in row order
    const float pv = __uint_as_float(~prefix);
    const u64 q = fixed_mass(pv);
    const u64 m = q ? (t - before) / q : 0;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE, nc = (n + SMP_CHUNK - 1) / SMP_CHUNK;
    auto ties = [&](float4 v) { return (int)(v.x == pv) + (int)(v.y == pv) + (int)(v.z == pv) + (int)(v.w == pv); };
    for (int c0 = w; c0 < nc; c0 += SMP_UNROLL * SMP_W) { // rows with probability pv per chunk
        float4 v[SMP_UNROLL];
#pragma unroll
        for (int u = 0; u < SMP_UNROLL; u++) v[u] = chunk_rows(p, n, min(c0 + u * SMP_W, nc - 1), lane);
#pragma unroll
        for (int u = 0; u < SMP_UNROLL; u++) {
            const u64 cnt = wave_sum_u64((u64)ties(v[u]));
            if (lane == 0 && c0 + u * SMP_W < nc) sh.chunk[c0 + u * SMP_W] = cnt;
        }
    }
    __syncthreads();
    u64 count;
    const int c = chunk_crossing(sh, nc, m, &count);
    if (w == 0 && c >= 0) {
        const float4 v = chunk_rows(p, n, c, lane); // rows past n read 0, which is never pv (pv >= cutoff > 0)
        const int tl = ties(v);
        const u64 before_l = sh.chunk[c] + wave_incl_scan_u64((u64)tl) - (u64)tl;
        const u64 hit = __ballot(tl > 0 && before_l <= m && m < before_l + (u64)tl);
        const int l = __builtin_ctzll(hit);
        if (lane == l) {
            int k = (int)(m - before_l), j = 0;
            const float r4[4] = {v.x, v.y, v.z, v.w};
            for (; j < 4; j++)
                if (r4[j] == pv && k-- == 0) break;
            sh.bc_i[1] = c * SMP_CHUNK + 4 * lane + j;
        }
    }
    __syncthreads();
    const int row = c >= 0 ? sh.bc_i[1] : -1;
    *through = before + (m + 1) * q;
    __syncthreads();
    return row;
}

} // namespace

__global__ void __launch_bounds__(SMP_T) k_sample(SampleArgs a) {
    __shared__ SmpShared sh;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wv = tid / WAVE;
    if (a.ctrl && a.ctrl->pos + 1 < a.ctrl->n_prompt) return; // the next token is forced: no draw
    const int n = a.n;
    const float temp = a.ss->temperature, topp = a.ss->topp;
    float *p = a.probs;

    // (1) logits / temperature (qwen.c:648): maximum (first row on ties) and the sum of exp(v - max), kept per
    // thread against a running maximum, then combined over the block (qwen.c:346-350)
    float mx = -INFINITY, s = 0.0f;
    int mi = 0x7fffffff;
    for_rows(a.logits, n, [&](int i, float x) {
        const float v = x / temp;
        if (v > mx) {
            s = s * expf(mx - v) + 1.0f;
            mx = v;
            mi = i;
        } else if (v > -INFINITY) { // a row at -inf (a masked logit) adds nothing
            s += expf(v - mx);
            if (v == mx && i < mi) mi = i;
        }
    });
    float tm = mx;
    int ti = mi;
    for (int o = 1; o < WAVE; o <<= 1) {
        const float ov = __shfl_xor(tm, o);
        const int oi = __shfl_xor(ti, o);
        if (ov > tm || (ov == tm && oi < ti)) { tm = ov; ti = oi; }
    }
    if (lane == 0) { sh.wf[wv] = tm; sh.wi[wv] = ti; }
    __syncthreads();
    float gm = sh.wf[0];
    mi = sh.wi[0];
    for (int k = 1; k < SMP_W; k++)
        if (sh.wf[k] > gm || (sh.wf[k] == gm && sh.wi[k] < mi)) { gm = sh.wf[k]; mi = sh.wi[k]; }
    if (mi == 0x7fffffff) mi = 0;
    __syncthreads();
    const float sum = block_sum(mx == -INFINITY ? 0.0f : s * expf(mx - gm), sh.wf);
    __syncthreads();

    // (2) the probabilities (qwen.c:351) and, over the top-p candidates, the radix level-0 masses
    const float cutoff = (1.0f - topp) / (n - 1);
    const bool use_topp = topp > 0.0f && topp < 1.0f;
    for (int b = tid; b < 256; b += SMP_T) sh.hist0[b] = 0;
    __syncthreads();
    {
        int run_b = -1;
        u64 run_q = 0;
        for_rows(a.logits, n, [&](int i, float x) {
            const float v = expf(x / temp - gm) / sum;
            p[i] = v;
            if (!use_topp || !(v >= cutoff)) return;
            const int b = (~__float_as_uint(v)) >> 24;
            if (b != run_b) {
                if (run_b >= 0) atomicAdd(&sh.hist0[run_b], run_q);
                run_b = b;
                run_q = 0;
            }
            run_q += fixed_mass(v);
        });
        if (run_b >= 0) atomicAdd(&sh.hist0[run_b], run_q);
    }
    __syncthreads();

    // (3) the coin (qwen.c:638-645, 651): xorshift64* on the device-resident state
    if (tid == 0) {
        u64 st = a.ss->rng;
        st ^= st >> 12;
        st ^= st << 25;
        st ^= st >> 27;
        a.ss->rng = st;
        const unsigned u = (unsigned)((st * 0x2545F4914F6CDD1Dull) >> 32);
        sh.bc_f = (float)(u >> 8) / 16777216.0f;
    }
    __syncthreads();
    const float coin = sh.bc_f;
    __syncthreads();
    int row;

    if (topp <= 0.0f || topp >= 1.0f) {
        // (4a) sample_mult (qwen.c:600-607): the first i with coin < cdf_i, else n - 1
        row = select_index(p, n, fixed_mass(coin), sh);
        if (row < 0) row = n - 1;
    } else {
        // (4b) sample_topp (qwen.c:616-636)
        u64 total = 0;
        for (int b = 0; b < 256; b++) total += sh.hist0[b];
        if (total == 0) {
            row = mi; // nothing reaches the cutoff (the reference reads before its buffer): the largest logit
        } else {
            const u64 tp = fixed_mass(topp);
            u64 cum;
            // the prefix through the first cumulative sum > topp, or every candidate
            const int last = select_sorted(p, n, cutoff, tp < total ? tp : total - 1, sh, &cum);
            const float r = coin * (float)ldexp((double)cum, -56);
            const u64 rt = fixed_mass(r);
            u64 unused;
            row = rt < cum ? select_sorted(p, n, cutoff, rt, sh, &unused) : last;
            if (row < 0) row = last;
        }
    }

    // the choice, as the only finite entry of the argmax partials that the next step start reads
    for (int k = tid; k < a.np; k += SMP_T) {
        a.pv[k] = k == 0 ? 0.0f : -INFINITY;
        a.pi[k] = k == 0 ? row : 0x7fffffff;
    }
    if (tid == 0 && a.out_row) *a.out_row = row;
}

hipError_t launch_sample(const SampleArgs &a, hipStream_t st) {
    if (a.n < 2 || a.n > SMP_MAX_CHUNKS * SMP_CHUNK || !a.logits || !a.probs || !a.ss ||
        ((uintptr_t)a.logits & 15) || ((uintptr_t)a.probs & 15) || (a.np > 0 && (!a.pv || !a.pi)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(SMP_T), 0, st, a);
    return hipGetLastError();
}
