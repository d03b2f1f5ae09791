// Sequential fp32 sums, bit for bit, by a whole block (gfx950, wave64).
//
// The reference adds the terms of a sum one after another in fp32 (rmsnorm's sum of squares, qwen.c:339 /
// runq.c:396; the softmax denominator, qwen.c:349): s_k = fl(s_{k-1} + a_k).  One lane spends a dependent add
// per term, 8.4 cycles on gfx950: 3.1 us for 896 terms, 12.6 us for 3584.
//
// Speculative segments.  The terms are cut into one segment per wave.  Before a segment the running sum is some
// fp32 value s; the exact sum of the terms before the segment, rounded to fp32 (predicted as the fp64 sum of the
// segments' fp32 totals), lies within a few ulps of s, because the reference's roundings drift from the exact
// sum by a random walk (about sqrt(k/36) ulps after k terms of one sign).  Lane l of the segment's wave starts
// from the fp32 value l - 32 ulps away from that prediction (its bit pattern +- l - 32) and adds the segment's
// terms in order, the reference's own operation: all 64 candidate chains advance together, one add per term.
// Wave 0 then walks the segments: s after segment 0 is its exact chain (the lane that started from 0); s after
// segment k is the end of the lane of segment k whose start equals s bit for bit, or, when s lies outside the
// 64 candidates, segment k added again one term at a time from s.  Either way every step is the reference's
// fp32 add from the reference's running value, so the result is the sequential sum exactly, for any terms
// (signs, inf, NaN).  The walk is one wave's (the block's other waves would only compete for its VALU slots)
// and its result reaches the rest of the block through LDS.
//
// The last < 16 terms of a chain are loaded together and entered through a jump into a run of adds
// (seq_add_tail), not one dependent load and add after another.

#pragma once
#include <type_traits>

#include "device.h"

#define SEQ_MAX_WAVES 16 // segments (waves) a block may use


// s + a[i] + ... + a[i1 - 1] in order (a: LDS, the same addresses in every lane): blocks of 32 terms read at
// once, then batches of 16 as broadcast reads, then the remaining < 16 terms through seq_add_tail (a sum of fewer
// than 16 terms: one read and add after another).  a is 16-byte aligned and i a multiple of 4.  (The blocks of
// 32: a 448-term chain 6.0k -> 4.6k cycles, 112 terms 1.7k -> 1.5k, measured alone on 512 threads.)
__device__ __forceinline__ float seq_chain(float s, const float *a, int i, int i1) {
    const float4 *a4 = (const float4 *)a;
    // whole blocks of 32 terms: the block's eight 16-byte reads issued together, then its 32 adds
    while (i + 32 <= i1) {
        float4 t4[8];
#pragma unroll
        for (int r = 0; r < 8; r++) t4[r] = a4[i / 4 + r];
#pragma unroll
        for (int r = 0; r < 8; r++) {
            s = s + t4[r].x;
            s = s + t4[r].y;
            s = s + t4[r].z;
            s = s + t4[r].w;
        }
        i += 32;
    }
    if (i + 16 <= i1) {
        float4 cur[4], nxt[4];
#pragma unroll
        for (int r = 0; r < 4; r++) cur[r] = a4[i / 4 + r];
        for (; i + 16 <= i1; i += 16) {
            const int in = min(i + 16, i1 - 16) & ~3;
#pragma unroll
            for (int r = 0; r < 4; r++) nxt[r] = a4[in / 4 + r];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                s = s + cur[r].x;
                s = s + cur[r].y;
                s = s + cur[r].z;
                s = s + cur[r].w;
            }
#pragma unroll
            for (int r = 0; r < 4; r++) cur[r] = nxt[r];
        }
    }
    if (i < i1 && i1 >= 16) {
        const float *b = a + (i1 - 16); // one base address, immediate offsets
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; u++) t[u] = b[u];
        s = seq_add_tail(s, t, i1 - i);
    } else {
        for (; i < i1; i++) s = s + a[i];
    }
    return s;
}

// LDS the block function needs: every segment's 64 candidate ends, the segments' fp64 totals and predicted
// start bits.
__host__ __device__ inline size_t seq_sum_scratch_bytes(int threads) {
    const int nw = threads / 64;
    return (size_t)nw * 64 * 4 + (size_t)nw * 8 + (size_t)nw * 4 + 16;
}

// s_0 = 0, s_k = fl(s_{k-1} + a[k-1]) as one chain by the whole wave (every lane the same values; a: LDS, 16-byte
// aligned): the terms as broadcast reads, the next 16 in flight while the current 16 are added.
__device__ __forceinline__ float wave_seq_sum(const float *a, int n) { return seq_chain(0.0f, a, 0, n); }

// Inclusive prefix sum of a double over each row of 16 lanes (DPP row shifts on both halves).
__device__ __forceinline__ double row_incl_scan_f64(double v) {
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) {
        const int lo = __double2loint(v), hi = __double2hiint(v);
        int l2, h2;
        switch (sh) { // DPP controls are immediates
        case 1: l2 = __builtin_amdgcn_update_dpp(0, lo, 0x111, 0xf, 0xf, true); h2 = __builtin_amdgcn_update_dpp(0, hi, 0x111, 0xf, 0xf, true); break;
        case 2: l2 = __builtin_amdgcn_update_dpp(0, lo, 0x112, 0xf, 0xf, true); h2 = __builtin_amdgcn_update_dpp(0, hi, 0x112, 0xf, 0xf, true); break;
        case 4: l2 = __builtin_amdgcn_update_dpp(0, lo, 0x114, 0xf, 0xf, true); h2 = __builtin_amdgcn_update_dpp(0, hi, 0x114, 0xf, 0xf, true); break;
        default: l2 = __builtin_amdgcn_update_dpp(0, lo, 0x118, 0xf, 0xf, true); h2 = __builtin_amdgcn_update_dpp(0, hi, 0x118, 0xf, 0xf, true); break;
        }
        v += __hiloint2double(h2, l2);
    }
    return v;
}

// s_0 = 0, s_k = fl(s_{k-1} + a[k-1]): the reference's sequential sum of a[0 .. n).  a: LDS, 16-byte aligned, read
// by every wave; scratch: seq_sum_scratch_bytes(blockDim.x) bytes of LDS, 16-byte aligned; at most SEQ_MAX_WAVES
// waves.  Every thread of the block calls it with the same n (barriers inside); every thread gets the result.
__device__ __forceinline__ float block_seq_sum(const float *a, int n, uint8_t *scratch) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), nw = blockDim.x / WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    float *ends = (float *)scratch;                       // [nw][64]
    double *tot = (double *)(ends + (size_t)nw * WAVE);   // [nw]
    uint32_t *pbits = (uint32_t *)(tot + nw);             // [nw], then the result
    // segments of L terms (a multiple of 4: every segment starts 16-byte aligned)
    const int L = ((n + nw - 1) / nw + 3) & ~3;
    const int q0 = min(wave * L, n), q1 = min(q0 + L, n);
    // (1) each segment's total (fp32 by DPP: within a few ulps of the exact total), for the predictions; a
    // lane's loads of the segment issued together
    float t = 0.0f;
    for (int i0 = q0; i0 < q1; i0 += 4 * WAVE) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = a[min(i0 + k * WAVE + lane, n - 1)];
#pragma unroll
        for (int k = 0; k < 4; k++) t += i0 + k * WAVE + lane < q1 ? v[k] : 0.0f;
    }
    t = wave_sum(t);
    if (lane == 0) tot[wave] = (double)t;
    __syncthreads();
    // (2) the candidate chains: lane l starts l - 32 ulps from the predicted start (segment 0: lane 32 from 0);
    // the prediction is the fp64 sum of the totals before the segment (a row scan of the <= 16 totals)
    const double pref = row_incl_scan_f64(lane < nw ? tot[min(lane, SEQ_MAX_WAVES - 1)] : 0.0);
    const double pd = wave == 0 ? 0.0 : __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(pref), wave - 1),
                                                          __builtin_amdgcn_readlane(__double2loint(pref), wave - 1));
    const uint32_t pb = __float_as_uint((float)pd);
    if (lane == 0) pbits[wave] = pb;
    const float s = seq_chain(__uint_as_float(pb + (uint32_t)lane - (uint32_t)(WAVE / 2)), a, q0, q1);
    ends[(size_t)wave * WAVE + lane] = s;
    __syncthreads();
    // (3) the walk, by wave 0 (the others wait at the barrier after it): each step takes the end of the lane
    // whose start is the running sum; a step outside the candidates sends the walk to the term-by-term path
    uint32_t *res = pbits + nw;
    if (wave == 0) {
        auto walk = [&](auto nwc) {
            constexpr int NW = decltype(nwc)::value;
            float e[NW];
#pragma unroll
            for (int k = 0; k < NW; k++) e[k] = ends[(size_t)min(k, nw - 1) * WAVE + lane];
            const uint32_t pl = pbits[min(lane, nw - 1)];
            uint32_t sb = __builtin_amdgcn_readlane(__float_as_uint(e[0]), WAVE / 2), miss = 0;
#pragma unroll
            for (int k = 1; k < NW; k++) { // every step, the ones past the last segment without effect
                const uint32_t idx = sb - __builtin_amdgcn_readlane(pl, k) + (uint32_t)(WAVE / 2);
                const uint32_t nsb = __builtin_amdgcn_readlane(__float_as_uint(e[k]), idx & (WAVE - 1));
                const bool live = k < nw;
                miss |= live && idx >= (uint32_t)WAVE;
                sb = live ? nsb : sb;
            }
            if (miss) { // again, with the term-by-term path for the segments whose start is not a candidate
                sb = __builtin_amdgcn_readlane(__float_as_uint(e[0]), WAVE / 2);
                for (int k = 1; k < nw; k++) {
                    const uint32_t idx = sb - __builtin_amdgcn_readlane(pl, k) + (uint32_t)(WAVE / 2);
                    if (idx < (uint32_t)WAVE) {
                        sb = __builtin_amdgcn_readlane(__float_as_uint(ends[(size_t)k * WAVE + lane]), idx);
                    } else {
                        const int k0 = min(k * L, n), k1 = min(k0 + L, n);
                        sb = __builtin_amdgcn_readfirstlane(__float_as_uint(seq_chain(__uint_as_float(sb), a, k0, k1)));
                    }
                }
            }
            return sb;
        };
        const uint32_t sb = nw <= 8 ? walk(std::integral_constant<int, 8>{})
                                    : walk(std::integral_constant<int, SEQ_MAX_WAVES>{});
        if (lane == 0) res[0] = sb;
    }
    __syncthreads();
    return __uint_as_float(res[0]);
}
