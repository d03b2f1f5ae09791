// On-device sampler of the token loop: temperature, softmax, top-p and the xorshift64* coin of the llama2.c
// sampler that both reference hosts use (qwen.c:578-654, runq.c:830-967), as one 1024-thread workgroup.
//
// The reference (per generated token, on the host):
//   logits /= temperature; softmax (max, expf(x - max), sum, divide); coin = random_f32(&rng);
//   topp outside (0, 1): the first i with coin < cdf_i over the probabilities in index order (sample_mult);
//   else: candidates p_i >= (1 - topp) / (n - 1), sorted by descending probability (qsort), the prefix up to
//   the first cumulative sum > topp, r = coin * that sum, and the first candidate with r < its cdf.
// Here every thread owns a contiguous segment of the array, so each cumulative sum is a prefix over the
// segments (in thread order) plus a sequential walk inside one segment; a decision that the reference takes
// on its sequential sums is taken on these, which differ from them only in fp32 rounding (as the softmax sum,
// a deterministic tree here).  The candidate sort is a stable radix sort on the probability bits (equal
// probabilities keep ascending index order).  The coin and the RNG stream are bit-exact.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "device.h"
#include "kernels.h"

#define SMP_T 1024
#define SMP_W (SMP_T / WAVE)

namespace {

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
    const int lane = threadIdx.x & (WAVE - 1);
    for (int o = 1; o < WAVE; o <<= 1) {
        const T u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    return v;
}

// Exclusive scan over the block in thread order; every thread gets the total.  scratch: SMP_W + 1 elements.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T v, T *scratch, T *total) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const T inc = wave_incl_scan(v);
    T ex = __shfl_up(inc, 1);
    if (lane == 0) ex = T(0);
    if (lane == WAVE - 1) scratch[w] = inc;
    __syncthreads();
    if (w == 0) {
        const T s = lane < SMP_W ? scratch[lane] : T(0);
        const T si = wave_incl_scan(s);
        T se = __shfl_up(si, 1);
        if (lane == 0) se = T(0);
        if (lane < SMP_W) scratch[lane] = se; // the wave read its inputs above, in program order
        if (lane == SMP_W - 1) scratch[SMP_W] = si;
    }
    __syncthreads();
    const T r = scratch[w] + ex;
    *total = scratch[SMP_W];
    __syncthreads();
    return r;
}

// smallest value over the block (every thread gets it)
__device__ __forceinline__ int block_min_int(int v, int *scratch) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    for (int o = 1; o < WAVE; o <<= 1) v = min(v, __shfl_xor(v, o));
    if (lane == 0) scratch[w] = v;
    __syncthreads();
    int r = scratch[0];
    for (int k = 1; k < SMP_W; k++) r = min(r, scratch[k]);
    __syncthreads();
    return r;
}

} // namespace

__global__ void __launch_bounds__(SMP_T) k_sample(SampleArgs a) {
    __shared__ unsigned cnt[16 * SMP_T]; // radix digit counts, then offsets, laid out [digit][thread]
    __shared__ float fs[SMP_W + 1];
    __shared__ unsigned us[SMP_W + 1];
    __shared__ int is[SMP_W + 1];
    __shared__ float sv[SMP_W];
    __shared__ int si[SMP_W];
    __shared__ float bc_f;
    __shared__ int bc_i, bc_skip;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wv = tid / WAVE;
    if (a.ctrl && a.ctrl->pos + 1 < a.ctrl->n_prompt) return; // the next token is forced: no draw
    const int n = a.n;
    const float temp = a.ss->temperature, topp = a.ss->topp;
    const int seg = (n + SMP_T - 1) / SMP_T, b0 = min(tid * seg, n), b1 = min(b0 + seg, n);
    float *p = a.probs;

    // (1) logits / temperature (qwen.c:648) and their maximum, first index on ties
    float mx = -INFINITY;
    int mi = 0x7fffffff;
    for (int i = b0; i < b1; i++) {
        const float v = a.logits[i] / temp;
        p[i] = v;
        if (v > mx) { mx = v; mi = i; }
    }
    for (int o = 1; o < WAVE; o <<= 1) {
        const float ov = __shfl_xor(mx, o);
        const int oi = __shfl_xor(mi, o);
        if (ov > mx || (ov == mx && oi < mi)) { mx = ov; mi = oi; }
    }
    if (lane == 0) { sv[wv] = mx; si[wv] = mi; }
    __syncthreads();
    mx = sv[0];
    mi = si[0];
    for (int k = 1; k < SMP_W; k++)
        if (sv[k] > mx || (sv[k] == mx && si[k] < mi)) { mx = sv[k]; mi = si[k]; }
    if (mi == 0x7fffffff) mi = 0;

    // (2) softmax (qwen.c:346-352): exponentials, their sum, the division
    float s = 0.0f;
    for (int i = b0; i < b1; i++) {
        const float e = expf(p[i] - mx);
        p[i] = e;
        s += e;
    }
    float sum;
    block_excl_scan(s, fs, &sum);
    for (int i = b0; i < b1; i++) p[i] = p[i] / sum;

    // (3) the coin (qwen.c:638-645, 651): xorshift64* on the device-resident state
    if (tid == 0) {
        unsigned long long st = a.ss->rng;
        st ^= st >> 12;
        st ^= st << 25;
        st ^= st >> 27;
        a.ss->rng = st;
        const unsigned u = (unsigned)((st * 0x2545F4914F6CDD1Dull) >> 32);
        bc_f = (float)(u >> 8) / 16777216.0f;
    }
    __syncthreads();
    const float coin = bc_f;
    int row;

    if (topp <= 0.0f || topp >= 1.0f) {
        // (4a) sample_mult (qwen.c:600-607)
        float ps = 0.0f;
        for (int i = b0; i < b1; i++) ps += p[i];
        float tot;
        const float pre = block_excl_scan(ps, fs, &tot);
        float e = pre;
        for (int i = b0; i < b1; i++) e += p[i];
        const int t = block_min_int(b0 < b1 && coin < e ? tid : 0x7fffffff, is);
        if (tid == t) {
            float cdf = pre;
            int r = b1 - 1;
            for (int i = b0; i < b1; i++) {
                cdf += p[i];
                if (coin < cdf) { r = i; break; }
            }
            bc_i = r;
        }
        __syncthreads();
        row = t == 0x7fffffff ? n - 1 : bc_i;
    } else {
        // (4b) sample_topp (qwen.c:616-636): candidates in index order
        const float cutoff = (1.0f - topp) / (n - 1);
        unsigned c = 0;
        for (int i = b0; i < b1; i++) c += p[i] >= cutoff;
        unsigned n0;
        unsigned o = block_excl_scan(c, us, &n0);
        for (int i = b0; i < b1; i++)
            if (p[i] >= cutoff) {
                a.key[0][o] = ~__float_as_uint(p[i]); // ascending key = descending probability
                a.idx[0][o] = i;
                o++;
            }
        __syncthreads();
        if (n0 == 0) {
            row = mi; // nothing reaches the cutoff (the reference reads before its buffer): the largest logit
        } else {
            // stable LSD radix sort, 4 bits per pass; a pass whose digit is the same for all keys is skipped
            const int s2 = ((int)n0 + SMP_T - 1) / SMP_T, c0 = min(tid * s2, (int)n0), c1 = min(c0 + s2, (int)n0);
            int cur = 0;
            for (int pass = 0; pass < 8; pass++) {
                const int sh = 4 * pass;
                const unsigned *ks = a.key[cur];
                const int *ix = a.idx[cur];
                for (int d = 0; d < 16; d++) cnt[d * SMP_T + tid] = 0;
                for (int j = c0; j < c1; j++) cnt[((ks[j] >> sh) & 15) * SMP_T + tid]++;
                __syncthreads();
                unsigned run = 0;
                for (int k = 0; k < 16; k++) {
                    const unsigned v = cnt[16 * tid + k];
                    cnt[16 * tid + k] = run;
                    run += v;
                }
                unsigned tot;
                const unsigned base = block_excl_scan(run, us, &tot);
                for (int k = 0; k < 16; k++) cnt[16 * tid + k] += base;
                __syncthreads();
                if (tid == 0) {
                    int skip = 0;
                    for (int d = 0; d < 16; d++) {
                        const unsigned st0 = cnt[d * SMP_T], st1 = d < 15 ? cnt[(d + 1) * SMP_T] : n0;
                        if (st1 - st0 == n0) skip = 1;
                    }
                    bc_skip = skip;
                }
                __syncthreads();
                if (!bc_skip) {
                    unsigned *kd = a.key[1 - cur];
                    int *id = a.idx[1 - cur];
                    for (int j = c0; j < c1; j++) {
                        const unsigned k = ks[j];
                        const unsigned q = cnt[((k >> sh) & 15) * SMP_T + tid]++;
                        kd[q] = k;
                        id[q] = ix[j];
                    }
                    cur = 1 - cur;
                }
                __syncthreads();
            }
            const unsigned *sk = a.key[cur];
            const int *sx = a.idx[cur];
            // the prefix up to the first cumulative sum > topp (qwen.c:621-626)
            float ps = 0.0f;
            for (int j = c0; j < c1; j++) ps += __uint_as_float(~sk[j]);
            float tot;
            const float pre = block_excl_scan(ps, fs, &tot);
            float e = pre;
            for (int j = c0; j < c1; j++) e += __uint_as_float(~sk[j]);
            const int t1 = block_min_int(c0 < c1 && e > topp ? tid : 0x7fffffff, is);
            if (t1 == 0x7fffffff) {
                if (c0 < c1 && c1 == (int)n0) { bc_i = (int)n0 - 1; bc_f = e; } // every candidate
            } else if (tid == t1) {
                float cdf = pre;
                for (int j = c0; j < c1; j++) {
                    cdf += __uint_as_float(~sk[j]);
                    if (cdf > topp) { bc_i = j; bc_f = cdf; break; }
                }
            }
            __syncthreads();
            const int last = bc_i;
            const float r = coin * bc_f;
            __syncthreads();
            // the first candidate up to `last` with r < its cdf (qwen.c:627-634)
            const int t2 = block_min_int(c0 < c1 && c0 <= last && r < (c1 - 1 <= last ? e : INFINITY) ? tid : 0x7fffffff,
                                         is);
            if (tid == t2) {
                float cdf = pre;
                int q = last;
                for (int j = c0; j < c1 && j <= last; j++) {
                    cdf += __uint_as_float(~sk[j]);
                    if (r < cdf) { q = j; break; }
                }
                bc_i = q;
            }
            __syncthreads();
            row = sx[t2 == 0x7fffffff ? last : bc_i];
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
    if (a.n < 2 || !a.logits || !a.probs || !a.key[0] || !a.key[1] || !a.idx[0] || !a.idx[1] || !a.ss ||
        (a.np > 0 && (!a.pv || !a.pi)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(SMP_T), 0, st, a);
    return hipGetLastError();
}
