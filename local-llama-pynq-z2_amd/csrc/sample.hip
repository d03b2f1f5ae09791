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

// ------------------------------------------------------------------------------------------------------
// The same draw over many workgroups (large vocabularies).  One workgroup reads every row ten times or so
// (softmax, probabilities, four radix levels per top-p select, the ties), all on one CU; here each pass is a
// launch of SMB_NB workgroups over contiguous ranges of 256-row chunks, and the workgroups meet only through
// kernel boundaries:
//   ks_partial: per workgroup, the maximum (first row on ties) and the exp sum against it;
//   ks_probs:   the global maximum and sum from the partials (in workgroup order: the same in every
//               workgroup), the probabilities, the radix level-0 masses of the top-p candidates and the chunk
//               masses of the plain walk (exact 64-bit integers, added with atomics: order-free), the coin;
//   plain walk: ks_final takes the first chunk whose running mass passes the coin, then the row inside it;
//   top-p:      per select (A: the prefix through the first cumulative sum > topp, B: the coin inside it),
//               ks_level for levels 1..3 (the chosen prefix is recomputed from the histograms in every
//               workgroup), ks_ties (rows equal to the chosen probability, per chunk), ks_final.
// Every decision is the one-workgroup kernel's, on the same exact masses; only the softmax sum's fp32 rounding
// follows another partition of its terms.

#define SMB_T 256
#define SMB_NB 64
#define SMP_MULTI_MIN 8192

namespace {

struct SmpScratch {
    float pm[SMB_NB], ps[SMB_NB];
    int pi[SMB_NB];
    u64 H[7][256];             // level 0; select A levels 1-3; select B levels 1-3
    u64 cm[SMP_MAX_CHUNKS];    // chunk masses (plain walk)
    u64 tc[SMP_MAX_CHUNKS];    // rows equal to the chosen probability, per chunk
    u64 rt, cum_a;
    float coin;
    int mi, last_a, need_b;
};

struct SmbShared {
    u64 hist[256];
    u64 wsum[SMB_T / WAVE + 1];
    float wf[SMB_T / WAVE];
    int wi[SMB_T / WAVE];
    u64 bu[2];
    int bi[2];
    float bf[2];
};

__device__ __forceinline__ bool smb_forced(const SampleArgs &a) { return a.ctrl && a.ctrl->pos + 1 < a.ctrl->n_prompt; }

// the workgroup's chunks [c0, c1)
__device__ __forceinline__ void smb_range(int n, int *c0, int *c1) {
    const int nc = (n + SMP_CHUNK - 1) / SMP_CHUNK, per = (nc + gridDim.x - 1) / gridDim.x;
    *c0 = min((int)blockIdx.x * per, nc);
    *c1 = min(*c0 + per, nc);
}

// the lane's four probabilities of chunk c (rows past n read 0)
__device__ __forceinline__ float4 smb_rows(const float *x, int n, int c, int lane) { return chunk_rows(x, n, c, lane); }

__device__ __forceinline__ bool smb_use_topp(const SampleArgs &a) { return a.ss->topp > 0.0f && a.ss->topp < 1.0f; }

// exclusive scan of one u64 per thread over a SMB_T workgroup; every thread gets the total
__device__ u64 smb_excl_scan(u64 v, SmbShared &sh, u64 *total);

// State of top-p select `sel` (0: A, 1: B) after `levels` radix levels, by the whole workgroup (one bucket
// per thread, SMB_T = 256): the candidates' total mass, the select's threshold t, the chosen key prefix and
// the mass before it, as select_sorted chooses them (the first bucket whose running mass passes t, else the
// last).  False when the select has nothing to do (no candidate, or B not needed).
__device__ bool smb_select_state(const SampleArgs &a, const SmpScratch *S, int sel, int levels, SmbShared &sh,
                                 u64 *t_out, u64 *total_out, unsigned *prefix, u64 *before) {
    static_assert(SMB_T == 256, "one radix bucket per thread");
    const int b = threadIdx.x;
    // every level's bucket of this thread and the select's settings, loaded together
    const u64 h0 = S->H[0][b];
    u64 hv[4];
#pragma unroll
    for (int lvl = 1; lvl < 4; lvl++) hv[lvl] = lvl < levels ? S->H[3 * sel + lvl][b] : 0;
    const int need_b = S->need_b;
    const u64 rt = S->rt;
    const float topp = a.ss->topp;
    u64 total;
    const u64 pre0 = smb_excl_scan(h0, sh, &total);
    *total_out = total;
    if (total == 0) return false;
    u64 t;
    if (sel == 0) {
        const u64 tp = fixed_mass(topp);
        t = tp < total ? tp : total - 1;
    } else {
        if (!need_b) return false;
        t = rt;
    }
    *t_out = t;
    unsigned pr = 0;
    u64 bf = 0;
    for (int lvl = 0; lvl < levels; lvl++) {
        const u64 h = lvl == 0 ? h0 : hv[lvl];
        u64 lt;
        const u64 pre = lvl == 0 ? pre0 : smb_excl_scan(h, sh, &lt);
        if (lvl == 0) lt = total;
        // the first bucket whose running mass passes t
        const bool pass = bf + pre + h > t;
        const u64 ball = __ballot(pass);
        const int lane = b & (WAVE - 1), w = b / WAVE;
        if (lane == 0) sh.wi[w] = ball ? w * WAVE + __builtin_ctzll(ball) : 0x7fffffff;
        __syncthreads();
        int chosen = sh.wi[0];
        for (int k = 1; k < SMB_T / WAVE; k++) chosen = min(chosen, sh.wi[k]);
        if (chosen != 0x7fffffff && b == chosen) sh.bu[1] = pre;
        __syncthreads();
        if (chosen == 0x7fffffff) {
            chosen = 255;
            bf = bf + lt;
        } else {
            bf = bf + sh.bu[1];
        }
        __syncthreads();
        pr = (pr << 8) | (unsigned)chosen;
    }
    *prefix = pr;
    *before = bf;
    return true;
}

// the histogram in LDS added to the global one (buckets with mass only)
__device__ __forceinline__ void smb_flush(SmbShared &sh, u64 *global) {
    __syncthreads();
    for (int b = threadIdx.x; b < 256; b += SMB_T)
        if (sh.hist[b]) atomicAdd((unsigned long long *)&global[b], (unsigned long long)sh.hist[b]);
}

__device__ __forceinline__ void smb_hist_add(SmbShared &sh, int b, u64 q) { atomicAdd((unsigned long long *)&sh.hist[b], (unsigned long long)q); }

// The workgroup's rows of probabilities as float4 per lane: the first SMB_PF chunks of each wave, loaded before
// the radix state is worked out (they do not depend on it); later chunks (large vocabularies) are loaded as used.
#define SMB_PF 4
struct SmbRows {
    float4 v[SMB_PF];
    int c0, c1;
    __device__ __forceinline__ void load(const SampleArgs &a) {
        smb_range(a.n, &c0, &c1);
        const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
        for (int k = 0; k < SMB_PF; k++) {
            const int c = c0 + w + k * (SMB_T / WAVE);
            v[k] = smb_rows(a.probs, a.n, min(c, c1 - 1), lane);
        }
    }
    // f(chunk, float4 of the lane) over the workgroup's chunks
    template <typename F>
    __device__ __forceinline__ void each(const SampleArgs &a, F f) const {
        const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
        for (int k = 0; k < SMB_PF; k++) {
            const int c = c0 + w + k * (SMB_T / WAVE);
            if (c < c1) f(c, v[k]);
        }
        for (int c = c0 + w + SMB_PF * (SMB_T / WAVE); c < c1; c += SMB_T / WAVE) f(c, smb_rows(a.probs, a.n, c, lane));
    }
};

// a thread's run of masses in one bucket, added to the LDS histogram once per run (rows of near-equal
// probability share a bucket: one LDS atomic per row would serialize on it)
struct SmbRun {
    int b = -1;
    u64 q = 0;
    __device__ __forceinline__ void add(SmbShared &sh, int bucket, u64 mass) {
        if (bucket != b) {
            if (b >= 0) smb_hist_add(sh, b, q);
            b = bucket;
            q = 0;
        }
        q += mass;
    }
    __device__ __forceinline__ void end(SmbShared &sh) {
        if (b >= 0) smb_hist_add(sh, b, q);
    }
};

// the sampled row as the only finite entry of the argmax partials (as k_sample)
__device__ __forceinline__ void smb_emit(const SampleArgs &a, int row) {
    for (int k = threadIdx.x; k < a.np; k += SMB_T) {
        a.pv[k] = k == 0 ? 0.0f : -INFINITY;
        a.pi[k] = k == 0 ? row : 0x7fffffff;
    }
    if (threadIdx.x == 0 && a.out_row) *a.out_row = row;
}

// exclusive scan of one u64 per thread over a SMB_T workgroup; every thread gets the total
__device__ u64 smb_excl_scan(u64 v, SmbShared &sh, u64 *total) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const u64 inc = wave_incl_scan_u64(v);
    if (lane == WAVE - 1) sh.wsum[w] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        u64 run = 0;
        for (int k = 0; k < SMB_T / WAVE; k++) {
            const u64 x = sh.wsum[k];
            sh.wsum[k] = run;
            run += x;
        }
        sh.wsum[SMB_T / WAVE] = run;
    }
    __syncthreads();
    const u64 r = sh.wsum[w] + inc - v;
    *total = sh.wsum[SMB_T / WAVE];
    __syncthreads();
    return r;
}

// the first chunk whose running value passes t (prefix + entry > t) over e[0, nc), and the prefix before it;
// -1 if none
__device__ int smb_crossing(const u64 *e, int nc, u64 t, SmbShared &sh, u64 *prefix) {
    const int per = (nc + SMB_T - 1) / SMB_T, c0 = threadIdx.x * per;
    u64 s = 0;
    for (int k = 0; k < per; k++)
        if (c0 + k < nc) s += e[c0 + k];
    u64 total;
    u64 run = smb_excl_scan(s, sh, &total);
    int found = 0x7fffffff;
    u64 found_pre = 0;
    for (int k = 0; k < per; k++)
        if (c0 + k < nc) {
            const u64 x = e[c0 + k];
            if (found == 0x7fffffff && run + x > t) { found = c0 + k; found_pre = run; }
            run += x;
        }
    // the smallest crossing chunk (each thread's chunks are consecutive: the first thread that finds one)
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    int f = found;
    for (int o = 1; o < WAVE; o <<= 1) f = min(f, __shfl_xor(f, o));
    if (lane == 0) sh.wi[w] = f;
    __syncthreads();
    int c = sh.wi[0];
    for (int k = 1; k < SMB_T / WAVE; k++) c = min(c, sh.wi[k]);
    if (c != 0x7fffffff && found == c) sh.bu[0] = found_pre;
    __syncthreads();
    *prefix = sh.bu[0];
    __syncthreads();
    return c == 0x7fffffff ? -1 : c;
}

} // namespace

__global__ void __launch_bounds__(SMB_T) ks_partial(SampleArgs a) {
    __shared__ SmbShared sh;
    if (smb_forced(a)) return;
    SmpScratch *S = (SmpScratch *)a.scratch;
    for (int i = blockIdx.x * SMB_T + threadIdx.x; i < 7 * 256; i += gridDim.x * SMB_T) (&S->H[0][0])[i] = 0;
    int c0, c1;
    smb_range(a.n, &c0, &c1);
    const int n = a.n, lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const float temp = a.ss->temperature;
    float mx = -INFINITY, s = 0.0f;
    int mi = 0x7fffffff;
    auto take = [&](int i, float x) { // as k_sample's first pass
        const float v = x / temp;
        if (v > mx) {
            s = s * expf(mx - v) + 1.0f;
            mx = v;
            mi = i;
        } else if (v > -INFINITY) {
            s += expf(v - mx);
            if (v == mx && i < mi) mi = i;
        }
    };
    for (int c = c0 + w; c < c1; c += SMB_T / WAVE) {
        const int i = c * SMP_CHUNK + 4 * lane;
        const float4 v = smb_rows(a.logits, n, c, lane);
        if (i < n) take(i, v.x);
        if (i + 1 < n) take(i + 1, v.y);
        if (i + 2 < n) take(i + 2, v.z);
        if (i + 3 < n) take(i + 3, v.w);
    }
    float tm = mx;
    int ti = mi;
    for (int o = 1; o < WAVE; o <<= 1) {
        const float ov = __shfl_xor(tm, o);
        const int oi = __shfl_xor(ti, o);
        if (ov > tm || (ov == tm && oi < ti)) { tm = ov; ti = oi; }
    }
    if (lane == 0) { sh.wf[w] = tm; sh.wi[w] = ti; }
    __syncthreads();
    float bm = sh.wf[0];
    int bi = sh.wi[0];
    for (int k = 1; k < SMB_T / WAVE; k++)
        if (sh.wf[k] > bm || (sh.wf[k] == bm && sh.wi[k] < bi)) { bm = sh.wf[k]; bi = sh.wi[k]; }
    __syncthreads();
    const float bs = block_sum(mx == -INFINITY ? 0.0f : s * expf(mx - bm), sh.wf);
    if (threadIdx.x == 0) {
        S->pm[blockIdx.x] = bm;
        S->pi[blockIdx.x] = bi;
        S->ps[blockIdx.x] = bm == -INFINITY ? 0.0f : bs;
    }
}

__global__ void __launch_bounds__(SMB_T) ks_probs(SampleArgs a) {
    __shared__ SmbShared sh;
    if (smb_forced(a)) return;
    SmpScratch *S = (SmpScratch *)a.scratch;
    const int n = a.n, lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const float temp = a.ss->temperature, topp = a.ss->topp;
    // the maximum (first row on ties) and the sum over the workgroups' partials, one per lane of wave 0 (the
    // sum in a fixed butterfly order: every workgroup gets the same value)
    static_assert(SMB_NB <= WAVE, "one partial per lane");
    if (threadIdx.x < WAVE) {
        const int b = threadIdx.x;
        const bool ok = b < (int)gridDim.x;
        const float pm = ok ? S->pm[b] : -INFINITY, ps = ok ? S->ps[b] : 0.0f;
        const int pi = ok ? S->pi[b] : 0x7fffffff;
        float gm = pm;
        int mi = pi;
        for (int o = 1; o < WAVE; o <<= 1) {
            const float ov = __shfl_xor(gm, o);
            const int oi = __shfl_xor(mi, o);
            if (ov > gm || (ov == gm && oi < mi)) { gm = ov; mi = oi; }
        }
        float term = pm > -INFINITY ? ps * expf(pm - gm) : 0.0f;
        for (int o = 1; o < WAVE; o <<= 1) term += __shfl_xor(term, o);
        if (b == 0) {
            sh.bf[0] = gm;
            sh.bf[1] = term;
            sh.bi[0] = mi == 0x7fffffff ? 0 : mi;
        }
    }
    for (int b = threadIdx.x; b < 256; b += SMB_T) sh.hist[b] = 0;
    __syncthreads();
    const float gm = sh.bf[0], sum = sh.bf[1];
    const float cutoff = (1.0f - topp) / (n - 1);
    const bool use_topp = topp > 0.0f && topp < 1.0f;
    int c0, c1;
    smb_range(n, &c0, &c1);
    SmbRun run;
    for (int c = c0 + w; c < c1; c += SMB_T / WAVE) {
        const int i = c * SMP_CHUNK + 4 * lane;
        const float4 x = smb_rows(a.logits, n, c, lane);
        const float xs[4] = {x.x, x.y, x.z, x.w};
        float pv[4];
        u64 m = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            pv[j] = i + j < n ? expf(xs[j] / temp - gm) / sum : 0.0f; // qwen.c:351
            const u64 q = fixed_mass(pv[j]);
            m += q;
            if (use_topp && i + j < n && pv[j] >= cutoff) run.add(sh, (~__float_as_uint(pv[j])) >> 24, q);
        }
        if (i + 3 < n) *(float4 *)(a.probs + i) = make_float4(pv[0], pv[1], pv[2], pv[3]);
        else
            for (int j = 0; j < 4; j++)
                if (i + j < n) a.probs[i + j] = pv[j];
        const u64 cmass = wave_sum_u64(m);
        if (lane == 0) S->cm[c] = cmass;
    }
    run.end(sh);
    if (use_topp) smb_flush(sh, S->H[0]);
    // the coin (qwen.c:638-645, 651), once per draw
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        u64 st = a.ss->rng;
        st ^= st >> 12;
        st ^= st << 25;
        st ^= st >> 27;
        a.ss->rng = st;
        const unsigned u = (unsigned)((st * 0x2545F4914F6CDD1Dull) >> 32);
        S->coin = (float)(u >> 8) / 16777216.0f;
        S->mi = sh.bi[0];
    }
}

// radix level `lvl` (1..3) of select `sel`: masses of the candidates under the prefix chosen so far
__global__ void __launch_bounds__(SMB_T) ks_level(SampleArgs a, int sel, int lvl) {
    __shared__ SmbShared sh;
    if (smb_forced(a)) return;
    if (!smb_use_topp(a)) return;
    SmpScratch *S = (SmpScratch *)a.scratch;
    SmbRows rows;
    rows.load(a);
    u64 t, total, before;
    unsigned prefix;
    if (!smb_select_state(a, S, sel, lvl, sh, &t, &total, &prefix, &before)) return;
    for (int b = threadIdx.x; b < 256; b += SMB_T) sh.hist[b] = 0;
    __syncthreads();
    const int n = a.n, sh_b = 24 - 8 * lvl;
    const float cutoff = (1.0f - a.ss->topp) / (n - 1);
    SmbRun run;
    rows.each(a, [&](int, float4 v) { // rows past n read 0: never a candidate
        const float r4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (!(r4[j] >= cutoff)) continue;
            const unsigned key = ~__float_as_uint(r4[j]);
            if ((key >> (sh_b + 8)) != prefix) continue;
            run.add(sh, (key >> sh_b) & 255, fixed_mass(r4[j]));
        }
    });
    run.end(sh);
    smb_flush(sh, S->H[3 * sel + lvl]);
}

// rows equal to the chosen probability of select `sel`, per chunk
__global__ void __launch_bounds__(SMB_T) ks_ties(SampleArgs a, int sel) {
    __shared__ SmbShared sh;
    if (smb_forced(a) || !smb_use_topp(a)) return;
    SmpScratch *S = (SmpScratch *)a.scratch;
    SmbRows rows;
    rows.load(a);
    u64 t, total, before;
    unsigned prefix;
    if (!smb_select_state(a, S, sel, 4, sh, &t, &total, &prefix, &before)) return;
    const float pv = __uint_as_float(~prefix);
    const int lane = threadIdx.x & (WAVE - 1);
    rows.each(a, [&](int c, float4 v) { // rows past n read 0, which is never pv (pv >= cutoff > 0)
        const u64 cnt = wave_sum_u64((u64)((int)(v.x == pv) + (int)(v.y == pv) + (int)(v.z == pv) + (int)(v.w == pv)));
        if (lane == 0) S->tc[c] = cnt;
    });
}

// the end of a draw (one workgroup): plain walk (sel < 0) or the end of top-p select `sel`
__global__ void __launch_bounds__(SMB_T) ks_final(SampleArgs a, int sel) {
    __shared__ SmbShared sh;
    if (smb_forced(a)) return;
    SmpScratch *S = (SmpScratch *)a.scratch;
    const int n = a.n, lane = threadIdx.x & (WAVE - 1), nc = (n + SMP_CHUNK - 1) / SMP_CHUNK;
    if (sel < 0) { // sample_mult (qwen.c:600-607): the first i with coin < cdf_i, else n - 1
        if (smb_use_topp(a)) return;
        const u64 t = fixed_mass(S->coin);
        u64 pre;
        const int c = smb_crossing(S->cm, nc, t, sh, &pre);
        int row = n - 1;
        if (c >= 0) {
            if (threadIdx.x < WAVE) {
                const float4 v = smb_rows(a.probs, n, c, lane);
                const u64 q0 = fixed_mass(v.x), q1 = fixed_mass(v.y), q2 = fixed_mass(v.z), q3 = fixed_mass(v.w);
                const u64 e = pre + wave_incl_scan_u64(q0 + q1 + q2 + q3) - (q0 + q1 + q2 + q3);
                const int j = e + q0 > t ? 0 : e + q0 + q1 > t ? 1 : e + q0 + q1 + q2 > t ? 2 : e + q0 + q1 + q2 + q3 > t ? 3 : 4;
                const u64 hit = __ballot(j < 4 && c * SMP_CHUNK + 4 * lane + j < n);
                const int l = __builtin_ctzll(hit);
                const int jl = __shfl(j, l);
                if (lane == 0) sh.bi[0] = hit ? c * SMP_CHUNK + 4 * l + jl : n - 1;
            }
            __syncthreads();
            row = sh.bi[0];
        }
        smb_emit(a, row);
        return;
    }
    if (!smb_use_topp(a)) return;
    u64 t = 0, total = 0, before = 0;
    unsigned prefix = 0;
    const bool active = smb_select_state(a, S, sel, 4, sh, &t, &total, &prefix, &before);
    if (total == 0) { // nothing reaches the cutoff: the largest logit (as k_sample)
        if (sel == 1) smb_emit(a, S->mi);
        return;
    }
    int row = -1;
    u64 cum = 0;
    if (active) {
        const float pv = __uint_as_float(~prefix);
        const u64 q = fixed_mass(pv);
        const u64 m = q ? (t - before) / q : 0;
        u64 pre;
        const int c = smb_crossing(S->tc, nc, m, sh, &pre);
        if (c >= 0) {
            if (threadIdx.x < WAVE) {
                const float4 v = smb_rows(a.probs, n, c, lane);
                const int tl = (int)(v.x == pv) + (int)(v.y == pv) + (int)(v.z == pv) + (int)(v.w == pv);
                const u64 before_l = pre + wave_incl_scan_u64((u64)tl) - (u64)tl;
                const u64 hit = __ballot(tl > 0 && before_l <= m && m < before_l + (u64)tl);
                const int l = __builtin_ctzll(hit);
                if (lane == l) {
                    int k = (int)(m - before_l), j = 0;
                    const float r4[4] = {v.x, v.y, v.z, v.w};
                    for (; j < 4; j++)
                        if (r4[j] == pv && k-- == 0) break;
                    sh.bi[1] = c * SMP_CHUNK + 4 * lane + j;
                }
            }
            __syncthreads();
            row = sh.bi[1];
        }
        cum = before + (m + 1) * q;
    }
    if (sel == 0) { // the prefix's last candidate and mass; the coin's target inside it (qwen.c:631-636)
        if (threadIdx.x == 0) {
            S->last_a = row;
            S->cum_a = cum;
            const float r = S->coin * (float)ldexp((double)cum, -56);
            const u64 rt = fixed_mass(r);
            S->rt = rt;
            S->need_b = rt < cum;
        }
        return;
    }
    // select B: its row, or the prefix's last one (no crossing inside, or the coin past the prefix)
    if (!S->need_b || row < 0) row = S->last_a;
    smb_emit(a, row);
}

size_t sample_scratch_bytes() { return sizeof(SmpScratch); }

hipError_t launch_sample(const SampleArgs &a, hipStream_t st) {
    if (a.strict) return launch_sample_strict(a, st);
    if (a.n < 2 || a.n > SMP_MAX_CHUNKS * SMP_CHUNK || !a.logits || !a.probs || !a.ss ||
        ((uintptr_t)a.logits & 15) || ((uintptr_t)a.probs & 15) || (a.np > 0 && (!a.pv || !a.pi)))
        return hipErrorInvalidValue;
    if (!a.scratch || a.n < SMP_MULTI_MIN) {
        hipLaunchKernelGGL(k_sample, dim3(1), dim3(SMP_T), 0, st, a);
        return hipGetLastError();
    }
    if ((uintptr_t)a.scratch & 15) return hipErrorInvalidValue;
    // The plain or top-p path is read from the device-resident settings by every kernel; a.path leaves out the
    // other path's launches where the caller knows the settings (the kernels of a path that is not selected
    // return at once).
    const int nc = (a.n + SMP_CHUNK - 1) / SMP_CHUNK, nb = nc < SMB_NB ? nc : SMB_NB;
    hipLaunchKernelGGL(ks_partial, dim3(nb), dim3(SMB_T), 0, st, a);
    hipLaunchKernelGGL(ks_probs, dim3(nb), dim3(SMB_T), 0, st, a);
    if (a.path != 1) hipLaunchKernelGGL(ks_final, dim3(1), dim3(SMB_T), 0, st, a, -1);
    if (a.path != 0)
        for (int sel = 0; sel < 2; sel++) {
            for (int lvl = 1; lvl < 4; lvl++) hipLaunchKernelGGL(ks_level, dim3(nb), dim3(SMB_T), 0, st, a, sel, lvl);
            hipLaunchKernelGGL(ks_ties, dim3(nb), dim3(SMB_T), 0, st, a, sel);
            hipLaunchKernelGGL(ks_final, dim3(1), dim3(SMB_T), 0, st, a, sel);
        }
    return hipGetLastError();
}
