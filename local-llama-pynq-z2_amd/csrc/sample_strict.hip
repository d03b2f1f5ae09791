// Reference-order draw of the on-device sampler (the strict mode).  Every float operation of the reference's
// sample() (qwen.c:647-654 with softmax qwen.c:346-352 and the walks qwen.c:600-636; runq.c:944-967) in its
// order: v = logits / temperature; the maximum; e = expf(v - max) with the reference libm's expf (ref_expf);
// the softmax denominator as one sequential fp32 sum over the rows in index order; p = e / sum; the coin; then
//   plain walk (topp outside (0, 1)): the first row whose sequential cdf exceeds the coin, else the last row;
//   top-p: the rows with p >= (1 - topp) / (n - 1), by descending p (equal p in ascending row order: glibc's
//   qsort is a stable merge sort), the first prefix whose sequential sum exceeds topp (else all of them),
//   r = coin * that sum, and the first row of the prefix whose sequential sum exceeds r (else its last row).
//
// Sequential sums (one "scan" per sum; kernels kss_tot / kss_ra / kss_chain / kss_walk).  The m terms are cut
// into segments of L terms, one wave each.  The start of a segment is predicted with the rounding that the
// running sum applies there: the terms of every earlier segment rounded to the unit in the last place of the
// fp64 prefix at which that segment starts, summed in fp64 (exact: multiples of one unit).  Lane l of the
// segment's wave starts a chain l - 32 ulps from the predicted start (as bit patterns) and adds the segment's
// terms in order, one fp32 add per term as the reference does.  The walker (one workgroup) follows the true
// running sum: the start of a segment is the end of the one before, and it selects the lane that started from
// exactly that value.  Its waves compose their 32 segments' lane maps in parallel (ds_bpermute, each path's
// lanes kept in LDS), one thread chains the waves, and each wave reads off its segments' entries.  A start outside the 64 candidates sends
// the walk, from that wave on, to a wave-by-wave walk that adds such a segment again term by term.  Every value
// on the path is the reference's own running sum, so the result is exact for any terms.  A threshold query
// ("the first term after which the sum exceeds t") takes the first segment whose end exceeds t (the sum never
// decreases: every term is >= 0) and adds that segment again from its start.
//
// Sort (top-p): a stable LSD radix sort of the keys ~bits(p) (descending p; equal p keep their row order) over
// all rows, the rows under the cutoff keyed last, 8 bits per pass: a per-tile digit histogram (kss_hist), then
// a scatter whose tiles rank their items stably with ballots (kss_scatter).
#include <hip/hip_runtime.h>
#include <float.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include "device.h"
#include "kernels.h"
#include "ref_expf.h"

#define SS_T 256                 // threads of the segment and radix kernels (4 waves)
#define SS_WALK_T 1024           // the walker: 16 waves of SS_SEGW segments
#define SS_SEGW 32               // segments per walker wave
#define SS_SEG_MAX (SS_WALK_T / WAVE * SS_SEGW) // segments of one scan (512)
#define SS_LMAX 512              // terms per segment at most
#define SS_N_MAX 262144          // rows
#define SS_TILE 2048             // radix tile: 4 waves x 8 rows of 64 items
#define SS_TILES_MAX (SS_N_MAX / SS_TILE)
#define SS_MAXB 64               // workgroups of the maximum pass
#ifndef SS_MARK
#define SS_MARK(k) // phase marks of the walker (a timing probe defines it)
#endif

typedef unsigned long long u64;

namespace {

struct StrictScratch {
    float bmax[SS_MAXB];          // per workgroup: the maximum of logits / temperature
    int bidx[SS_MAXB];            //                and its first row
    double tot[SS_SEG_MAX];       // the current scan: each segment's terms summed in fp64
    double ra[SS_SEG_MAX];        //                   ... rounded to the ulp of the segment's predicted start
    uint32_t pb[SS_SEG_MAX];      //                   predicted start (bits)
    float ends[SS_SEG_MAX * 64];  //                   candidate chain ends [segment][lane]
    int ncand[SS_SEG_MAX];        // top-p candidates per segment of the probability pass
    float sum, coin;
    int skew; // tests: every predicted start but the first moved by this many ulps (0 in use)
    uint32_t hist[SS_TILES_MAX * 256];    // a radix pass's digit counts of each tile
    uint32_t key[2][SS_N_MAX], idx[2][SS_N_MAX];
};

// segments of a scan over m terms: L a multiple of 4 (16-byte rows in LDS), at most SS_SEG_MAX of them
struct Geo {
    int m, L, nseg;
};
__host__ __device__ inline Geo ss_geo(int m) {
    Geo g;
    g.m = m;
    int l = (m + SS_SEG_MAX - 1) / SS_SEG_MAX;
    l = (l + 3) & ~3;
    g.L = l < 16 ? 16 : l;
    g.nseg = (m + g.L - 1) / g.L;
    return g;
}

__device__ __forceinline__ bool ss_forced(const SampleArgs &a) { return a.ctrl && a.ctrl->pos + 1 < a.ctrl->n_prompt; }
__device__ __forceinline__ bool ss_topp(const SampleArgs &a) { return a.ss->topp > 0.0f && a.ss->topp < 1.0f; }
__device__ __forceinline__ StrictScratch *ss_of(const SampleArgs &a) { return (StrictScratch *)a.strict_scratch; }

// stages: the softmax denominator, the plain walk's cdf, the top-p walk over the sorted candidates
enum { ST_SOFTMAX = 0, ST_PLAIN = 1, ST_TOPP = 2 };

// whether a stage's kernels run in this draw (the other walk's return at once)
__device__ __forceinline__ bool ss_stage_on(const SampleArgs &a, int stage) {
    if (ss_forced(a)) return false;
    if (stage == ST_PLAIN) return !ss_topp(a);
    if (stage == ST_TOPP) return ss_topp(a);
    return true;
}

// term i of a stage's scan: e or p in row order, or the i-th largest candidate p (sorted keys)
__device__ __forceinline__ float ss_term(const SampleArgs &a, const StrictScratch *S, int stage, int i) {
    return stage == ST_TOPP ? __uint_as_float(~S->key[0][i]) : a.probs[i];
}

// terms in the scan: every row, or the top-p candidates
__device__ __forceinline__ int ss_len(const SampleArgs &a, const StrictScratch *S, int stage) {
    if (stage != ST_TOPP) return a.n;
    const Geo gp = ss_geo(a.n);
    const int lane = threadIdx.x & (WAVE - 1);
    int c = 0;
#pragma unroll
    for (int q = 0; q < SS_SEG_MAX / WAVE; q++) { // all loads in flight at once
        const int k = q * WAVE + lane;
        c += k < gp.nseg ? S->ncand[k] : 0;
    }
    for (int o = 1; o < WAVE; o <<= 1) c += __shfl_xor(c, o);
    return c;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int o = 1; o < WAVE; o <<= 1) v += __shfl_xor(v, o);
    return v;
}

// sum of x[j] for j < k (x in global memory, k <= SS_SEG_MAX), the same value in every lane
__device__ __forceinline__ double prefix_f64(const double *x, int k) {
    const int lane = threadIdx.x & (WAVE - 1);
    double v[SS_SEG_MAX / WAVE];
#pragma unroll
    for (int q = 0; q < SS_SEG_MAX / WAVE; q++) v[q] = q * WAVE + lane < k ? x[q * WAVE + lane] : 0.0; // in flight together
    double s = 0.0;
#pragma unroll
    for (int q = 0; q < SS_SEG_MAX / WAVE; q++) s += v[q];
    return wave_sum_f64(s);
}

// the unit in the last place of a float A >= 0 (2^-149 below the normals)
__device__ __forceinline__ double ulp_of(float A) {
    const int e = (int)(__float_as_uint(A) >> 23);
    return e == 0 ? 0x1p-149 : ldexp(1.0, e - 150);
}

// f(i, term i) over the terms of segment k (rows k L .. min(k L + L, m)) by the lanes of one wave, every lane's
// loads (at most SS_LMAX / WAVE = 8) in flight together
template <class Get, class F>
__device__ __forceinline__ void ss_seg_for(const Geo &g, int k, Get get, F f) {
    const int lane = threadIdx.x & (WAVE - 1), i0 = k * g.L, i1 = min(i0 + g.L, g.m);
    float x[SS_LMAX / WAVE];
#pragma unroll
    for (int q = 0; q < SS_LMAX / WAVE; q++) {
        const int i = i0 + q * WAVE + lane;
        x[q] = i < i1 ? get(i) : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < SS_LMAX / WAVE; q++) {
        const int i = i0 + q * WAVE + lane;
        if (i < i1) f(i, x[q]);
    }
}

__device__ void ss_emit(const SampleArgs &a, int row) {
    for (int k = threadIdx.x; k < a.np; k += blockDim.x) {
        a.pv[k] = k == 0 ? 0.0f : -INFINITY;
        a.pi[k] = k == 0 ? row : 0x7fffffff;
    }
    if (threadIdx.x == 0 && a.out_row) *a.out_row = row;
}

// The sequential sum of segment k from s over its terms (buf: the wave's LDS copy, zero-padded to L; adding
// +0 leaves a sum >= 0 unchanged), by every lane of the calling wave alike; *pos / *val get the first term
// index after which the sum exceeds t and the sum there (pos -1 if none).
__device__ __forceinline__ float ss_rechain(const SampleArgs &a, const StrictScratch *S, int stage, const Geo &g, int k,
                                         float s, float t, float *buf, int *pos, float *val) {
    const int lane = threadIdx.x & (WAVE - 1), i0 = k * g.L;
    for (int i = lane; i < g.L; i += WAVE) buf[i] = 0.0f;
    __builtin_amdgcn_wave_barrier();
    ss_seg_for(g, k, [&](int i) { return ss_term(a, S, stage, i); }, [&](int i, float x) { buf[i - i0] = x; });
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int p = -1;
    float v = 0.0f;
    auto add = [&](float x, int i) {
        s = s + x;
        if (p < 0 && s > t) {
            p = i;
            v = s;
        }
    };
    // the terms as broadcast reads, the next 16 in flight while the current 16 are added (L >= 16, L % 4 == 0)
    const float4 *b4 = (const float4 *)buf;
    float4 cur[4], nxt[4];
#pragma unroll
    for (int q = 0; q < 4; q++) cur[q] = b4[q];
    int i = 0;
    for (; i + 16 <= g.L; i += 16) {
        const int in = min(i + 16, g.L - 16) / 4;
#pragma unroll
        for (int q = 0; q < 4; q++) nxt[q] = b4[in + q];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            add(cur[q].x, i + 4 * q);
            add(cur[q].y, i + 4 * q + 1);
            add(cur[q].z, i + 4 * q + 2);
            add(cur[q].w, i + 4 * q + 3);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) cur[q] = nxt[q];
    }
    for (; i < g.L; i += 4) {
        const float4 x = b4[i / 4];
        add(x.x, i);
        add(x.y, i + 1);
        add(x.z, i + 2);
        add(x.w, i + 3);
    }
    __builtin_amdgcn_wave_barrier();
    *pos = p;
    *val = v;
    return s;
}

} // namespace

// (1) per workgroup: the maximum of logits / temperature (first row on ties); workgroup 0 draws the coin
// (qwen.c:638-645, 651: xorshift64* on the device-resident state)
__global__ void __launch_bounds__(SS_T) kss_max(SampleArgs a) {
    __shared__ float wf[SS_T / WAVE];
    __shared__ int wi[SS_T / WAVE];
    if (ss_forced(a)) return;
    StrictScratch *S = ss_of(a);
    const int n = a.n, per = (n + gridDim.x - 1) / gridDim.x, r0 = blockIdx.x * per, r1 = min(r0 + per, n);
    const float temp = a.ss->temperature;
    float mx = -INFINITY;
    int mi = 0x7fffffff;
    for (int i0 = r0 + threadIdx.x; i0 < r1; i0 += 8 * SS_T) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; u++) x[u] = i0 + u * SS_T < r1 ? a.logits[i0 + u * SS_T] : -INFINITY; // in flight together
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * SS_T;
            const float v = x[u] / temp;
            if (i < r1 && (v > mx || (v == mx && i < mi))) {
                mx = v;
                mi = i;
            }
        }
    }
    for (int o = 1; o < WAVE; o <<= 1) {
        const float ov = __shfl_xor(mx, o);
        const int oi = __shfl_xor(mi, o);
        if (ov > mx || (ov == mx && oi < mi)) {
            mx = ov;
            mi = oi;
        }
    }
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    if (lane == 0) {
        wf[w] = mx;
        wi[w] = mi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < SS_T / WAVE; k++)
            if (wf[k] > wf[0] || (wf[k] == wf[0] && wi[k] < wi[0])) {
                wf[0] = wf[k];
                wi[0] = wi[k];
            }
        S->bmax[blockIdx.x] = wf[0];
        S->bidx[blockIdx.x] = wi[0];
        if (blockIdx.x == 0) {
            u64 st = a.ss->rng;
            st ^= st >> 12;
            st ^= st << 25;
            st ^= st >> 27;
            a.ss->rng = st;
            const unsigned u = (unsigned)((st * 0x2545F4914F6CDD1Dull) >> 32);
            S->coin = (float)(u >> 8) / 16777216.0f;
        }
    }
}

// the maximum over the workgroups' partials (the same in every wave), its row in *row
__device__ float ss_global_max(const StrictScratch *S, int nb, int *row) {
    const int lane = threadIdx.x & (WAVE - 1);
    float mx = lane < nb ? S->bmax[lane] : -INFINITY;
    int mi = lane < nb ? S->bidx[lane] : 0x7fffffff;
    for (int o = 1; o < WAVE; o <<= 1) {
        const float ov = __shfl_xor(mx, o);
        const int oi = __shfl_xor(mi, o);
        if (ov > mx || (ov == mx && oi < mi)) {
            mx = ov;
            mi = oi;
        }
    }
    *row = mi == 0x7fffffff ? 0 : mi;
    return mx;
}

// (2) e = expf(logits / temperature - max) into probs, one wave per segment of the softmax scan, with its
// fp64 total (qwen.c:346-350)
__global__ void __launch_bounds__(SS_T) kss_exp(SampleArgs a, int nb) {
    if (ss_forced(a)) return;
    StrictScratch *S = ss_of(a);
    const Geo g = ss_geo(a.n);
    const int k = blockIdx.x * (SS_T / WAVE) + threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    int unused;
    const float gm = ss_global_max(S, nb, &unused);
    if (k >= g.nseg) return;
    const float temp = a.ss->temperature;
    double t = 0.0;
    ss_seg_for(g, k, [&](int i) { return a.logits[i]; }, [&](int i, float x) {
        const float e = ref_expf(x / temp - gm);
        a.probs[i] = e;
        t += (double)e;
    });
    t = wave_sum_f64(t);
    if (lane == 0) S->tot[k] = t;
}

// (3) p = e / sum in place (qwen.c:351), with the plain walk's segment totals; the top-p keys ~bits(p) for
// the candidates p >= (1 - topp) / (n - 1) (qwen.c:619-621), 0xffffffff (last) for the others, and the
// candidates per segment
__global__ void __launch_bounds__(SS_T) kss_probs(SampleArgs a) {
    if (ss_forced(a)) return;
    StrictScratch *S = ss_of(a);
    const Geo g = ss_geo(a.n);
    const int k = blockIdx.x * (SS_T / WAVE) + threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    if (k >= g.nseg) return;
    const float sum = S->sum, topp = a.ss->topp;
    const float cutoff = (1.0f - topp) / (a.n - 1);
    const bool topp_on = ss_topp(a);
    double t = 0.0;
    int c = 0;
    ss_seg_for(g, k, [&](int i) { return a.probs[i]; }, [&](int i, float e) {
        const float p = e / sum;
        a.probs[i] = p;
        t += (double)p;
        if (topp_on) {
            const bool cand = p >= cutoff;
            S->key[0][i] = cand ? ~__float_as_uint(p) : 0xffffffffu;
            S->idx[0][i] = (uint32_t)i;
            c += cand;
        }
    });
    t = wave_sum_f64(t);
    for (int o = 1; o < WAVE; o <<= 1) c += __shfl_xor(c, o);
    if (lane == 0) {
        S->tot[k] = t;
        S->ncand[k] = c;
    }
}

// segment totals of the top-p scan (the sorted candidates)
__global__ void __launch_bounds__(SS_T) kss_tot(SampleArgs a) {
    if (!ss_stage_on(a, ST_TOPP)) return;
    StrictScratch *S = ss_of(a);
    const Geo g = ss_geo(ss_len(a, S, ST_TOPP));
    const int k = blockIdx.x * (SS_T / WAVE) + threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    if (k >= g.nseg) return;
    double t = 0.0;
    ss_seg_for(g, k, [&](int i) { return ss_term(a, S, ST_TOPP, i); }, [&](int, float x) { t += (double)x; });
    t = wave_sum_f64(t);
    if (lane == 0) S->tot[k] = t;
}

// (4) each segment's advance as the running sum rounds it: its terms rounded to the ulp of the fp64 prefix
// at its start (the first segment, and any that starts from 0, its plain total)
__global__ void __launch_bounds__(SS_T) kss_ra(SampleArgs a, int stage) {
    if (!ss_stage_on(a, stage)) return;
    StrictScratch *S = ss_of(a);
    const Geo g = ss_geo(ss_len(a, S, stage));
    const int k = blockIdx.x * (SS_T / WAVE) + threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    if (k >= g.nseg) return;
    const float A = (float)prefix_f64(S->tot, k);
    if (A == 0.0f) {
        if (lane == 0) S->ra[k] = S->tot[k];
        return;
    }
    const double u = ulp_of(A);
    double r = 0.0;
    ss_seg_for(g, k, [&](int i) { return ss_term(a, S, stage, i); }, [&](int, float x) { r += rint((double)x / u) * u; });
    r = wave_sum_f64(r);
    if (lane == 0) S->ra[k] = r;
}

// (5) the candidate chains: lane l of segment k starts l - 32 ulps from the predicted start and adds the
// segment's terms in order (fp32, one rounding per add)
__global__ void __launch_bounds__(SS_T) kss_chain(SampleArgs a, int stage) {
    __shared__ float4 buf4[SS_T / WAVE][SS_LMAX / 4];
    if (!ss_stage_on(a, stage)) return;
    StrictScratch *S = ss_of(a);
    const Geo g = ss_geo(ss_len(a, S, stage));
    const int w = threadIdx.x / WAVE, k = blockIdx.x * (SS_T / WAVE) + w, lane = threadIdx.x & (WAVE - 1);
    if (k >= g.nseg) return;
    const uint32_t pbk = k == 0 ? 0u : __float_as_uint((float)prefix_f64(S->ra, k)) + (uint32_t)S->skew;
    float *buf = (float *)buf4[w];
    for (int i = lane; i < g.L; i += WAVE) buf[i] = 0.0f;
    __builtin_amdgcn_wave_barrier();
    ss_seg_for(g, k, [&](int i) { return ss_term(a, S, stage, i); }, [&](int i, float x) { buf[i - k * g.L] = x; });
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float s = __uint_as_float(pbk + (uint32_t)lane - 32u);
    const float4 *b = buf4[w];
    int i = 0;
    if (g.L >= 16) {
        // the next 16 terms in flight while the current 16 are added
        float4 cur[4], nxt[4];
#pragma unroll
        for (int q = 0; q < 4; q++) cur[q] = b[q];
        for (; i + 16 <= g.L; i += 16) {
            const int in = min(i + 16, g.L - 16) / 4;
#pragma unroll
            for (int q = 0; q < 4; q++) nxt[q] = b[in + q];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                s = s + cur[q].x;
                s = s + cur[q].y;
                s = s + cur[q].z;
                s = s + cur[q].w;
            }
#pragma unroll
            for (int q = 0; q < 4; q++) cur[q] = nxt[q];
        }
    }
    for (; i < g.L; i += 4) {
        const float4 x = b[i / 4];
        s = s + x.x;
        s = s + x.y;
        s = s + x.z;
        s = s + x.w;
    }
    S->ends[k * 64 + lane] = s;
    if (lane == 0) S->pb[k] = pbk;
}

// The slow walk of one wave (segments k0 .. k0 + SS_SEGW - 1): from the exact end of the segment before, each segment's
// entry and end; a start among the segment's candidates takes that candidate's end, any other start adds the
// segment again term by term.
__device__ __noinline__ void ss_slow_wave(const SampleArgs &a, const StrictScratch *S, int stage, const Geo &g,
                                          int k0, float *entry, float *endv, float *ebuf, float *xbuf) {
    const int lane = threadIdx.x & (WAVE - 1);
    for (int j = 0; j < SS_SEGW && k0 + j < g.nseg; j++) ebuf[j * 64 + lane] = S->ends[(k0 + j) * 64 + lane];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float s = k0 == 0 ? 0.0f : endv[k0 - 1];
    for (int j = 0; j < SS_SEGW && k0 + j < g.nseg; j++) {
        const int k = k0 + j;
        const uint32_t idx = __float_as_uint(s) - S->pb[k] + 32u;
        if (lane == 0) entry[k] = s;
        if (idx < 64u) {
            s = ebuf[j * 64 + idx];
        } else {
            int p;
            float pv;
            s = ss_rechain(a, S, stage, g, k, s, INFINITY, xbuf, &p, &pv);
        }
        if (lane == 0) endv[k] = s;
    }
}

// (6) the walk through the segments (one workgroup of 16 waves, wave w owning segments 32 w .. 32 w + 31), then
// the stage's result: the softmax denominator, the plain walk's row, or the top-p row
__global__ void __launch_bounds__(SS_WALK_T) kss_walk(SampleArgs a, int stage, int nb) {
    __shared__ float entry[SS_SEG_MAX], endv[SS_SEG_MAX];
    __shared__ float ebuf[SS_SEGW * 64];         // the candidate ends of the wave walking the slow way
    __shared__ __align__(16) float xbuf[SS_LMAX];   // terms of a segment added again
    __shared__ uint8_t fmap[SS_WALK_T / WAVE][64];
    __shared__ uint8_t trail[SS_WALK_T / WAVE][SS_SEGW][64]; // entry lane of each segment on each start lane's path
    __shared__ int wstart[SS_WALK_T / WAVE], wslow, kfirst[SS_WALK_T / WAVE];
    __shared__ int res_i[2];
    __shared__ float res_f[2];
    if (!ss_stage_on(a, stage)) return;
    StrictScratch *S = ss_of(a);
    const int m = ss_len(a, S, stage);
    if (stage == ST_TOPP && m == 0) { // no candidate (the reference reads before its buffer): the largest logit
        int row;
        ss_global_max(S, nb, &row);
        ss_emit(a, row);
        return;
    }
    const Geo g = ss_geo(m);
    const int w = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1), k0 = w * SS_SEGW;
    SS_MARK(0);
    const int nw = (g.nseg + SS_SEGW - 1) / SS_SEGW;

    // (A) every wave: the path of each start lane of its first segment through its segments (the candidate
    // ends in blocks of 16 segments, the second block's loads in flight while the first is composed)
    const uint32_t pbl = k0 + lane < g.nseg && lane < SS_SEGW ? S->pb[k0 + lane] : 0u;
    const uint32_t pbx = k0 + SS_SEGW < g.nseg ? S->pb[k0 + SS_SEGW] : 0u;
    auto load16 = [&](float(&eb)[16], int jb) {
#pragma unroll
        for (int q = 0; q < 16; q++) eb[q] = k0 + jb + q < g.nseg ? S->ends[(k0 + jb + q) * 64 + lane] : 0.0f;
    };
    // predicted start (bits) of segment k0 + j + 1
    auto next_pb = [&](int j) {
        return j < SS_SEGW - 1 ? (uint32_t)__builtin_amdgcn_readlane((int)pbl, j + 1) : pbx;
    };
    uint32_t cur = (uint32_t)lane, miss = 0;
    auto compose16 = [&](const float(&eb)[16], int jb) {
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int j = jb + q, k = k0 + j;
            if (k < g.nseg) trail[w][j][lane] = miss ? 0xffu : (uint8_t)cur;
            if (k + 1 < g.nseg) {
                const float v = __int_as_float(__builtin_amdgcn_ds_bpermute((int)(cur << 2), __float_as_int(eb[q])));
                const uint32_t nx = __float_as_uint(v) - next_pb(j) + 32u;
                miss |= nx >= 64u;
                cur = nx & 63u;
            }
        }
    };
    static_assert(SS_SEGW == 32, "two blocks of 16 segments");
    float e0[16], e1[16];
    load16(e0, 0);
    load16(e1, 16);
    compose16(e0, 0);
    SS_MARK(7);
    compose16(e1, 16);
    if (w < nw) fmap[w][lane] = miss ? 0xffu : (uint8_t)cur;
    __syncthreads();
    SS_MARK(1);

    // (B) the waves' start lanes (segment 0 starts at 0: lane 32 of a zero prediction); the first wave whose
    // path leaves the candidates walks the slow way, with every wave after it
    if (threadIdx.x == 0) {
        uint32_t s = 32;
        int slow = nw;
        for (int v = 0; v < nw; v++) {
            wstart[v] = (int)s;
            const uint32_t nx = fmap[v][s];
            if (nx == 0xffu) {
                slow = v;
                break;
            }
            s = nx;
        }
        wslow = slow;
    }
    __syncthreads();
    const int slow = wslow;
    SS_MARK(2);

    // (C) the waves before it: lane j reads segment k0 + j's entry lane on the wave's path, so its exact start,
    // and the end of that candidate
    if (w < nw && w < slow && lane < SS_SEGW && k0 + lane < g.nseg) {
        const uint32_t el = trail[w][lane][wstart[w]];
        const int k = k0 + lane;
        entry[k] = __uint_as_float(pbl + el - 32u);
        endv[k] = S->ends[k * 64 + el];
    }
    SS_MARK(3);
    // (D) from the slow wave on, one wave at a time: the exact running sum through its segments, a segment
    // whose start is not among its candidates added again term by term
    for (int v = slow; v < nw; v++) {
        __syncthreads();
        if (w == v) ss_slow_wave(a, S, stage, g, k0, entry, endv, ebuf, xbuf);
    }
    __syncthreads();

    SS_MARK(4);
    // (E) the stage's result
    const float total = endv[g.nseg - 1];
    // first segment whose end exceeds t among segments [0, kmax], every thread gets it (0x7fffffff: none)
    auto first_over = [&](float t, int kmax) {
        int hit = 0x7fffffff;
        if ((int)threadIdx.x < g.nseg && (int)threadIdx.x <= kmax && endv[threadIdx.x] > t) hit = threadIdx.x;
        for (int o = 1; o < WAVE; o <<= 1) hit = min(hit, __shfl_xor(hit, o));
        if (lane == 0) kfirst[w] = hit;
        __syncthreads();
        int r = kfirst[0];
        for (int q = 1; q < SS_WALK_T / WAVE; q++) r = min(r, kfirst[q]);
        __syncthreads();
        return r;
    };
    // the first term index after which the running sum exceeds t, inside segment k, and the sum there
    auto crossing = [&](int k, float t, float *val) {
        if (w == 0) {
            int p;
            float pv;
            ss_rechain(a, S, stage, g, k, entry[k], t, xbuf, &p, &pv);
            if (lane == 0) {
                res_i[0] = p;
                res_f[0] = pv;
            }
        }
        __syncthreads();
        const int p = res_i[0];
        *val = res_f[0];
        __syncthreads();
        return p;
    };
    if (stage == ST_SOFTMAX) {
        if (threadIdx.x == 0) S->sum = total;
        return;
    }
    const float coin = S->coin;
    if (stage == ST_PLAIN) { // qwen.c:600-607: the first i with coin < cdf_i, else n - 1
        const int kc = first_over(coin, g.nseg - 1);
        int row = a.n - 1;
        if (kc != 0x7fffffff) {
            float v;
            const int p = crossing(kc, coin, &v);
            if (p >= 0) row = kc * g.L + p;
        }
        ss_emit(a, row);
        return;
    }
    // top-p (qwen.c:623-635)
    const float topp = a.ss->topp;
    int last = g.m - 1;
    float cum = total;
    const int kc = first_over(topp, g.nseg - 1);
    if (kc != 0x7fffffff) {
        float v;
        const int p = crossing(kc, topp, &v);
        if (p >= 0) {
            last = kc * g.L + p;
            cum = v;
        }
    }
    SS_MARK(5);
    const float r = coin * cum;
    int j = last;
    const int k2 = first_over(r, last / g.L);
    if (k2 != 0x7fffffff) {
        float v;
        const int p = crossing(k2, r, &v);
        if (p >= 0 && k2 * g.L + p <= last) j = k2 * g.L + p;
    }
    SS_MARK(6);
    ss_emit(a, (int)S->idx[0][j]);
}

// (7) radix pass `pass` (bits 8 pass .. 8 pass + 7 of the keys): digit counts per tile
__global__ void __launch_bounds__(SS_T) kss_hist(SampleArgs a, int pass) {
    __shared__ uint32_t cnt[256];
    if (!ss_stage_on(a, ST_TOPP)) return;
    StrictScratch *S = ss_of(a);
    const uint32_t *key = S->key[pass & 1];
    cnt[threadIdx.x] = 0;
    __syncthreads();
    const int i0 = blockIdx.x * SS_TILE;
    uint32_t kq[SS_TILE / SS_T];
#pragma unroll
    for (int q = 0; q < SS_TILE / SS_T; q++) { // in flight together
        const int i = i0 + q * SS_T + threadIdx.x;
        kq[q] = i < a.n ? key[i] : 0u;
    }
#pragma unroll
    for (int q = 0; q < SS_TILE / SS_T; q++)
        if (i0 + q * SS_T + (int)threadIdx.x < a.n) atomicAdd(&cnt[(kq[q] >> (8 * pass)) & 255u], 1u);
    __syncthreads();
    S->hist[blockIdx.x * 256 + threadIdx.x] = cnt[threadIdx.x];
}

// ... and the stable scatter: an item's place is its digit's start over all tiles, plus the items of that digit
// in earlier tiles, earlier waves of its tile, earlier rows of its wave and earlier lanes of its row
__global__ void __launch_bounds__(SS_T) kss_scatter(SampleArgs a, int pass) {
    __shared__ uint32_t base[256], wcnt[SS_T / WAVE][256], wtot[SS_T / WAVE];
    if (!ss_stage_on(a, ST_TOPP)) return;
    StrictScratch *S = ss_of(a);
    const int n = a.n, ntiles = (n + SS_TILE - 1) / SS_TILE, b = blockIdx.x;
    const int d = threadIdx.x, lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE, sh = 8 * pass;
    const uint32_t *skey = S->key[pass & 1], *sidx = S->idx[pass & 1];
    uint32_t *dkey = S->key[(pass + 1) & 1], *didx = S->idx[(pass + 1) & 1];
    // digit d: items in earlier tiles, items in all tiles; then the exclusive scan over the digits
    uint32_t pre = 0, tot = 0;
    for (int t0 = 0; t0 < ntiles; t0 += 16) {
        uint32_t h[16];
#pragma unroll
        for (int q = 0; q < 16; q++) h[q] = t0 + q < ntiles ? S->hist[(t0 + q) * 256 + d] : 0u; // in flight together
#pragma unroll
        for (int q = 0; q < 16; q++) {
            tot += h[q];
            pre += t0 + q < b ? h[q] : 0u;
        }
    }
    uint32_t inc = tot;
    for (int o = 1; o < WAVE; o <<= 1) {
        const uint32_t u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
    }
    if (lane == WAVE - 1) wtot[w] = inc;
    for (int q = 0; q < SS_T / WAVE; q++) wcnt[q][d] = 0;
    __syncthreads();
    uint32_t before = 0;
    for (int q = 0; q < w; q++) before += wtot[q];
    base[d] = before + inc - tot + pre;
    __syncthreads();
    // the tile's items in order: wave w takes rows of 64 at i0 + 512 w + 64 r
    const int i0 = b * SS_TILE + w * (SS_TILE / (SS_T / WAVE));
    uint32_t kk[8], ii[8], rk[8];
    const u64 below = (1ull << lane) - 1ull;
#pragma unroll
    for (int r = 0; r < 8; r++) { // every row's loads in flight together
        const int i = i0 + r * WAVE + lane;
        kk[r] = i < n ? skey[i] : 0u;
        ii[r] = i < n ? sidx[i] : 0u;
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int i = i0 + r * WAVE + lane;
        const bool ok = i < n;
        const uint32_t dg = (kk[r] >> sh) & 255u;
        u64 same = __ballot(ok);
#pragma unroll
        for (int bit = 0; bit < 8; bit++) {
            const u64 m1 = __ballot((dg >> bit) & 1u);
            same &= (dg >> bit) & 1u ? m1 : ~m1;
        }
        const uint32_t lower = (uint32_t)__popcll(same & below);
        const uint32_t c0 = wcnt[w][dg];
        rk[r] = c0 + lower;
        // the group's lowest lane moves its digit's count on; the wave's LDS operations complete in order, so
        // the next row reads it
        if (ok && lower == 0) wcnt[w][dg] = c0 + (uint32_t)__popcll(same);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int i = i0 + r * WAVE + lane;
        if (i < n) {
            const uint32_t dg = (kk[r] >> sh) & 255u;
            uint32_t pos = base[dg] + rk[r];
            for (int q = 0; q < w; q++) pos += wcnt[q][dg];
            if (pos < (uint32_t)n) { // always (a permutation of the n items); kept as a bound on the store
                dkey[pos] = kk[r];
                didx[pos] = ii[r];
            }
        }
    }
}

size_t sample_strict_scratch_bytes() { return sizeof(StrictScratch); }

hipError_t sample_strict_set_skew(void *scratch, int skew) {
    return hipMemcpy((uint8_t *)scratch + offsetof(StrictScratch, skew), &skew, sizeof skew, hipMemcpyHostToDevice);
}

hipError_t launch_sample_strict(const SampleArgs &a, hipStream_t st) {
    if (a.n < 2 || a.n > SS_N_MAX || !a.logits || !a.probs || !a.ss || !a.strict_scratch ||
        ((uintptr_t)a.strict_scratch & 15) || (a.np > 0 && (!a.pv || !a.pi)))
        return hipErrorInvalidValue;
    const Geo g = ss_geo(a.n);
    const int nb = min(SS_MAXB, (a.n + SS_TILE - 1) / SS_TILE);
    // segment kernels: 4 segments per workgroup; the top-p scan's segments (over the candidates only, whose
    // count the device knows) may outnumber the rows' (shorter segments), so its kernels take the most
    const int segb = (g.nseg + SS_T / WAVE - 1) / (SS_T / WAVE), segmax = SS_SEG_MAX / (SS_T / WAVE);
    const int tiles = (a.n + SS_TILE - 1) / SS_TILE;
    hipLaunchKernelGGL(kss_max, dim3(nb), dim3(SS_T), 0, st, a);
    hipLaunchKernelGGL(kss_exp, dim3(segb), dim3(SS_T), 0, st, a, nb);
    hipLaunchKernelGGL(kss_ra, dim3(segb), dim3(SS_T), 0, st, a, (int)ST_SOFTMAX);
    hipLaunchKernelGGL(kss_chain, dim3(segb), dim3(SS_T), 0, st, a, (int)ST_SOFTMAX);
    hipLaunchKernelGGL(kss_walk, dim3(1), dim3(SS_WALK_T), 0, st, a, (int)ST_SOFTMAX, nb);
    hipLaunchKernelGGL(kss_probs, dim3(segb), dim3(SS_T), 0, st, a);
    if (a.path != 1) { // the plain walk over p in row order
        hipLaunchKernelGGL(kss_ra, dim3(segb), dim3(SS_T), 0, st, a, (int)ST_PLAIN);
        hipLaunchKernelGGL(kss_chain, dim3(segb), dim3(SS_T), 0, st, a, (int)ST_PLAIN);
        hipLaunchKernelGGL(kss_walk, dim3(1), dim3(SS_WALK_T), 0, st, a, (int)ST_PLAIN, nb);
    }
    if (a.path != 0) { // top-p: sort, then the walk over the sorted candidates
        for (int pass = 0; pass < 4; pass++) {
            hipLaunchKernelGGL(kss_hist, dim3(tiles), dim3(SS_T), 0, st, a, pass);
            hipLaunchKernelGGL(kss_scatter, dim3(tiles), dim3(SS_T), 0, st, a, pass);
        }
        hipLaunchKernelGGL(kss_tot, dim3(segmax), dim3(SS_T), 0, st, a);
        hipLaunchKernelGGL(kss_ra, dim3(segmax), dim3(SS_T), 0, st, a, (int)ST_TOPP);
        hipLaunchKernelGGL(kss_chain, dim3(segmax), dim3(SS_T), 0, st, a, (int)ST_TOPP);
        hipLaunchKernelGGL(kss_walk, dim3(1), dim3(SS_WALK_T), 0, st, a, (int)ST_TOPP, nb);
    }
    return hipGetLastError();
}
