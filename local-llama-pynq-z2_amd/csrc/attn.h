// Attention of one kv head's query heads over a range of positions (device code shared by the decode and
// prefill kernels of libmatvec_hip.so; internal header).
//
// qwen.c:526-546 / runq.c:530-568: score_t = (q . k_t) / sqrtf(hs) as a sequential dot in the reference's
// order, softmax, weighted sum of V.  Here the softmax is online over sub-chunks of ATT_SUB positions (running
// max and sum, rescaled partial sums), K and V staged in LDS.
#pragma once
#include "device.h"
#include "kernels.h"
#include "ref_expf.h"
#include "seqsum.h"

#ifndef KERNEL_MARK
#define KERNEL_MARK(k)
#endif

typedef float f32x4 __attribute__((ext_vector_type(4)));
// 16-byte vectors per thread for one sub-chunk of K (and as many of V): ATT_SUB * hs / 4 <= ATT_VEC * 256
#define ATT_VEC 4

// LDS floats of attn_range for kv_mul query heads of size hs.  K rows are padded to hs + 4 floats: the score
// loop's lanes read different rows at the same column, which a power-of-two stride would put in one bank.
__host__ __device__ inline size_t attn_lds_floats(int kv_mul, int hs) {
    return (size_t)kv_mul * hs + (size_t)ATT_SUB * (2 * hs + 4) + (size_t)kv_mul * ATT_SUB + 3 * (size_t)kv_mul;
}

// Block of 256 threads.  q: the kv_mul * hs query values of kv head kvh (16-byte aligned); kc, vc: the layer's
// caches [ctx][kv_dim].  On return acc[k] holds the exp-weighted value sum of output (j, e) = tid + 256 k
// (head j of the group, element e) and ml_max / ml_sum point at the kv_mul running maxima / sums in LDS.
// Every thread of the block must call it (barriers inside); t_begin < t_end.
__device__ __forceinline__ void attn_range(const float *q, const float *kc, const float *vc, int kv_dim, int kvh,
                                           int hs, int kv_mul, int t_begin, int t_end, float *sm, float (&acc)[4],
                                           const float **ml_max, const float **ml_sum) {
    const int hs4 = hs / 4, tid = threadIdx.x, nt = blockDim.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid & (WAVE - 1), nw = nt / WAVE;
    const int ks = hs + 4;
    float *sq = sm;                          // kv_mul * hs
    float *sk = sq + kv_mul * hs;            // ATT_SUB * ks
    float *sv = sk + ATT_SUB * ks;           // ATT_SUB * hs
    float *sc = sv + ATT_SUB * hs;           // kv_mul * ATT_SUB scores, then exponentials
    float *sm_ = sc + kv_mul * ATT_SUB;      // kv_mul running max
    float *sl = sm_ + kv_mul;                // kv_mul running sum
    float *sf = sl + kv_mul;                 // kv_mul rescale factor of this step
    const float rs = sqrtf((float)hs);

    // Every global load of a sub-chunk is issued before the first is waited for: q of the kv_mul heads with
    // the first sub-chunk, each later sub-chunk while the previous one is computed.  Vector indices past
    // the end are clamped; their stores write the last vector's own value again.
    const int nq4 = kv_mul * hs4; // <= nt
    const f32x4 rq = ((const f32x4 *)q)[min(tid, nq4 - 1)];
    f32x4 rk[ATT_VEC], rv[ATT_VEC];
    // vector k of this thread in a sub-chunk: row t, column vector c (clamped to the sub-chunk's last)
    auto kv_index = [&](int t0, int k, int *t, int *c) {
        const int cnt = min(ATT_SUB, t_end - t0) * hs4, i = min(tid + k * nt, cnt - 1);
        *t = i / hs4;
        *c = i - *t * hs4;
    };
    auto load_kv = [&](int t0) {
#pragma unroll
        for (int k = 0; k < ATT_VEC; k++) {
            int t, c;
            kv_index(t0, k, &t, &c);
            const size_t gi = (size_t)(t0 + t) * kv_dim + (size_t)kvh * hs + 4 * c;
            rk[k] = *(const f32x4 *)(kc + gi);
            rv[k] = *(const f32x4 *)(vc + gi);
        }
    };
    load_kv(t_begin);
    asm volatile("" ::: "memory"); // every load above is issued before the first store waits for one
    ((f32x4 *)sq)[min(tid, nq4 - 1)] = rq;
    if (tid < kv_mul) { sm_[tid] = -INFINITY; sl[tid] = 0.0f; }
    KERNEL_MARK(1);
    // each thread owns outputs (j, e) = o, o + nt, ... of the kv_mul * hs accumulators
    for (int k = 0; k < 4; k++) acc[k] = 0.0f;
    const int n_out = kv_mul * hs;
    for (int t0 = t_begin; t0 < t_end; t0 += ATT_SUB) {
        const int T = min(ATT_SUB, t_end - t0);
#pragma unroll
        for (int k = 0; k < ATT_VEC; k++) {
            int t, c;
            kv_index(t0, k, &t, &c);
            *(f32x4 *)(sk + t * ks + 4 * c) = rk[k];
            *(f32x4 *)(sv + t * hs + 4 * c) = rv[k];
        }
        __syncthreads();
        KERNEL_MARK(2);
        if (t0 + ATT_SUB < t_end) load_kv(t0 + ATT_SUB);
        for (int i = tid; i < kv_mul * T; i += nt) { // score = (q . k) / sqrtf(hs), e in order
            const int j = i / T, t = i - j * T;
            const f32x4 *qq = (const f32x4 *)(sq + j * hs), *kk = (const f32x4 *)(sk + t * ks);
            float d = 0.0f;
#pragma unroll 4
            for (int e4 = 0; e4 < hs4; e4++) {
                const f32x4 a4 = qq[e4], b4 = kk[e4];
                d += a4.x * b4.x;
                d += a4.y * b4.y;
                d += a4.z * b4.z;
                d += a4.w * b4.w;
            }
            sc[j * ATT_SUB + t] = d / rs;
        }
        __syncthreads();
        KERNEL_MARK(3);
        for (int j = wave; j < kv_mul; j += nw) { // online softmax statistics, one wave per head
            float v = lane < T ? sc[j * ATT_SUB + lane] : -INFINITY;
            float mx = wave_max(v);
            const float m_old = sm_[j], m_new = fmaxf(m_old, mx);
            const float e = lane < T ? expf(v - m_new) : 0.0f;
            if (lane < T) sc[j * ATT_SUB + lane] = e;
            const float sum = wave_sum(e);
            if (lane == 0) {
                const float f = m_old == -INFINITY ? 0.0f : expf(m_old - m_new);
                sf[j] = f;
                sl[j] = sl[j] * f + sum;
                sm_[j] = m_new;
            }
        }
        __syncthreads();
        KERNEL_MARK(4);
        for (int k = 0; k < 4; k++) {
            const int o = tid + k * nt;
            if (o < n_out) {
                const int j = o / hs, e = o - j * hs;
                float v = acc[k] * sf[j];
                const float *sj = sc + j * ATT_SUB, *se = sv + e;
#pragma unroll 8
                for (int t = 0; t < T; t++) v += sj[t] * se[t * hs];
                acc[k] = v;
            }
        }
        __syncthreads(); // the next sub-chunk's stores overwrite sk, sv and sc
        KERNEL_MARK(5);
    }
    *ml_max = sm_;
    *ml_sum = sl;
}

// ------------------------------------------------------------------------------------------------------
// Reference-order attention (the strict mode): one query head over positions 0 .. P-1 with every float
// operation of qwen.c:526-546 / runq.c:530-568 in the reference's order, so the result is bitwise the
// reference's:
//   score_t = (sum over i in order of q[i] * k_t[i]) / sqrtf(hs);  max over t (exact in any order);
//   e_t = expf(score_t - max) (ref_expf: the reference libm's expf);  sum = e_0 + e_1 + ... in position order;
//   a_t = e_t / sum;  out[e] = ((0 + a_0 v_0[e]) + a_1 v_1[e]) + ... in position order.
// The scores (a position per thread) and the products run in parallel, V staged in LDS tiles whose loads run
// ahead; the running sums are the reference's chains (the softmax sum by the block's speculative segments when
// long).  Block of 256 threads, hs <= 256.
// Block-wide (barriers inside); every thread of the block calls it.  sm: attn_strict_lds_floats floats.

// Positions of V one tile stages in LDS (8192 floats at most: 8 16-byte loads per thread of 256).
__host__ __device__ inline int attn_strict_tile(int hs) { return 8192 / hs < 256 ? 8192 / hs : 256; }
__host__ __device__ inline size_t attn_strict_lds_floats(int hs, int P, int threads) {
    return (size_t)hs + (((size_t)P + 3) & ~(size_t)3) + (((size_t)threads / WAVE + 4 + 3) & ~(size_t)3) +
           seq_sum_scratch_bytes(threads) / 4 + 4 + (size_t)attn_strict_tile(hs) * hs;
}

// HS: the head size as a compile-time constant (64, 128: a full tile's chain is straight-line code, so the
// next tile's loads stay in flight under it), or 0 for any other hs.
template <int HS>
__device__ __forceinline__ void attn_strict_head(const float *q, const float *kc, const float *vc, int kv_dim,
                                                 int koff, int hs_arg, int P, float *sm, float *out) {
    const int hs = HS ? HS : hs_arg;
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & (WAVE - 1), wave = tid / WAVE, nw = nt / WAVE;
    float *sq = sm, *sc = sm + hs, *sred = sc + ((P + 3) & ~3);
    uint8_t *sscr = (uint8_t *)(sred + ((nw + 4 + 3) & ~3)); // the sequential sum's scratch (16-byte aligned)
    float *svt = (float *)(sscr + seq_sum_scratch_bytes(nt) + 16); // a tile of V rows [CH][hs]
    const int CH = attn_strict_tile(hs), hs4 = hs / 4, ntile = (P + CH - 1) / CH;
    // V tiles: 8 16-byte loads per thread (vector j * 256 + tid of the tile: position / hs4, column % hs4), rows
    // past P read nothing; the first tile's loads leave now, behind the scores
    const auto rv = __builtin_amdgcn_make_buffer_rsrc((void *)(vc + koff), 0, (int)(((size_t)(P - 1) * kv_dim + hs) * 4),
                                                      0x00020000);
    auto vtile_load = [&](int k, f32x4 (&r)[8]) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int idx = j * 256 + tid, t = k * CH + idx / hs4, c = idx - (idx / hs4) * hs4;
            const bool ok = idx < CH * hs4 && t < P;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rv, ok ? (uint32_t)(t * kv_dim + 4 * c) * 4u : 0x80000000u, 0, 0);
            r[j] = *(const f32x4 *)&v;
        }
    };
    auto vtile_store = [&](const f32x4 (&r)[8]) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int idx = j * 256 + tid;
            if (idx < CH * hs4) ((f32x4 *)svt)[idx] = r[j];
        }
    };
    f32x4 vr[8];
    vtile_load(0, vr);
    KERNEL_MARK(0);
    for (int i = tid; i < hs; i += nt) sq[i] = q[i];
    __syncthreads();
    KERNEL_MARK(1);
    const float rs = sqrtf((float)hs);
    const f32x4 *q4 = (const f32x4 *)sq;
    // scores: a position per thread, its K row through a buffer resource (the row's offset per lane, the
    // column's as a scalar), 4 vectors a batch, two batches in flight (ping-pong: each waits for its own loads)
    const auto rk = __builtin_amdgcn_make_buffer_rsrc((void *)(kc + koff), 0, (int)(((size_t)(P - 1) * kv_dim + hs) * 4),
                                                      0x00020000);
    auto kbatch = [&](uint32_t vo, int c, f32x4 (&b)[4]) { // vectors c .. c+3 of the row (past hs4: zeros)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rk, c + j < hs4 ? vo : 0x80000000u, (c + j) * 16, 0);
            b[j] = *(const f32x4 *)&v;
        }
    };
    auto kuse = [&](float d, int c, const f32x4 (&b)[4]) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f32x4 kk = b[j], qq = q4[c + j];
            d += qq.x * kk.x;
            d += qq.y * kk.y;
            d += qq.z * kk.z;
            d += qq.w * kk.w;
        }
        return d;
    };
    float mx = -INFINITY;
    for (int t0 = 0; t0 < P; t0 += nt) {
        const int t = t0 + tid;
        const uint32_t vo = (uint32_t)min(t, P - 1) * (uint32_t)kv_dim * 4u;
        float d = 0.0f;
        if constexpr (HS != 0) { // the whole row in flight at once
            f32x4 kr[HS / 4];
#pragma unroll
            for (int j = 0; j < HS / 4; j++) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(rk, vo, j * 16, 0);
                kr[j] = *(const f32x4 *)&v;
            }
#pragma unroll
            for (int j = 0; j < HS / 4; j++) {
                const f32x4 kk = kr[j], qq = q4[j];
                d += qq.x * kk.x;
                d += qq.y * kk.y;
                d += qq.z * kk.z;
                d += qq.w * kk.w;
            }
        } else if ((hs4 & 7) == 0) { // whole batches: no guards inside the chain
            f32x4 bA[4], bB[4];
            kbatch(vo, 0, bA);
            for (int c = 0; c < hs4; c += 8) {
                kbatch(vo, c + 4, bB);
                d = kuse(d, c, bA);
                kbatch(vo, c + 8, bA);
                d = kuse(d, c + 4, bB);
            }
        } else {
            const f32x4 *k4 = (const f32x4 *)(kc + (size_t)min(t, P - 1) * kv_dim + koff);
            for (int c = 0; c < hs4; c++) {
                const f32x4 kk = k4[c], qq = q4[c];
                d += qq.x * kk.x;
                d += qq.y * kk.y;
                d += qq.z * kk.z;
                d += qq.w * kk.w;
            }
        }
        if (t < P) {
            const float sct = d / rs;
            sc[t] = sct;
            mx = fmaxf(mx, sct);
        }
    }
    KERNEL_MARK(2);
    mx = wave_max(mx);
    if (lane == 0) sred[wave] = mx;
    __syncthreads();
    for (int w = 0; w < nw; w++) mx = fmaxf(mx, sred[w]);
    for (int t = tid; t < P; t += nt) sc[t] = ref_expf(sc[t] - mx);
    __syncthreads();
    KERNEL_MARK(3);
    float sum;
    if (P <= 256) { // a short sum: one chain (wave 0, broadcast reads), cheaper than the block's segments
        if (wave == 0) {
            const float v = wave_seq_sum(sc, P);
            if (lane == 0) sred[nw] = v;
        }
        __syncthreads();
        sum = sred[nw];
    } else {
        sum = block_seq_sum(sc, P, sscr);
        __syncthreads(); // every wave's walk may still read the exponentials that the division below overwrites
    }
    KERNEL_MARK(4);
    for (int t = tid; t < P; t += nt) sc[t] = sc[t] / sum;
    __syncthreads();
    KERNEL_MARK(5);
    // values: an element per thread in the reference's position order, from the V tile in LDS; the next tile's
    // loads are in flight while this one is summed
    float acc = 0.0f;
    const int e = tid < hs ? tid : 0;
    for (int k = 0; k < ntile; k++) {
        vtile_store(vr);
        __syncthreads();
        if (k + 1 < ntile) vtile_load(k + 1, vr);
        const int t0 = k * CH, T = min(CH, P - t0);
        if (tid < hs) {
            const float *vt = svt + e;
            const f32x4 *w4 = (const f32x4 *)(sc + t0);
            if (HS && T == CH) { // a full tile: straight-line code
                constexpr int CHC = HS ? (8192 / HS < 256 ? 8192 / HS : 256) : 4;
#pragma unroll
                for (int t = 0; t < CHC; t += 4) {
                    const f32x4 w = w4[t / 4];
                    acc += w.x * vt[t * HS];
                    acc += w.y * vt[(t + 1) * HS];
                    acc += w.z * vt[(t + 2) * HS];
                    acc += w.w * vt[(t + 3) * HS];
                }
            } else {
                int t = 0;
                for (; t + 4 <= T; t += 4) {
                    const f32x4 w = w4[t / 4];
                    acc += w.x * vt[t * hs];
                    acc += w.y * vt[(t + 1) * hs];
                    acc += w.z * vt[(t + 2) * hs];
                    acc += w.w * vt[(t + 3) * hs];
                }
                for (; t < T; t++) acc += sc[t0 + t] * vt[t * hs];
            }
        }
        __syncthreads(); // the next tile's stores overwrite this one
    }
    if (tid < hs) out[tid] = acc;
    KERNEL_MARK(6);
}
