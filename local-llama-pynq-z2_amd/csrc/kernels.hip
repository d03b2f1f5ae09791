// Kernels of libmatvec_hip.so for gfx950: tiled int4/int8 GEMV with fused prologues and epilogues,
// decode attention, embedding lookup, argmax reduction and the weight repack.
//
// Reference roles: the GEMV is hls4/matvec4.cpp / hls/matvec.cpp (math in hls4/matvec4.h:1-4 and
// hls/matvec.h:1-4, CPU form qwen.c:407-457 and runq.c:429-458); the prologues and epilogues are the
// element-wise steps of forward() around each matmul (qwen.c:515-565, runq.c:497-605); attention is
// qwen.c:526-546 / runq.c:530-568; argmax is qwen.c:591-598 with the head_ids map of qwen.c:683.
#include "device.h"
#include "kernels.h"

// Phase hooks for timing studies: a harness that includes this file may define KERNEL_MARK(k) to record
// a timestamp of phase k; the library's own build compiles them away.
#ifndef KERNEL_MARK
#define KERNEL_MARK(k)
#endif

#include <math.h>

#include <algorithm>

#include "attn.h"

// ------------------------------------------------------------------------------------------------------
// exact int32 group sums

// int4 segment (16 B, repacked so dword j carries elements 4j..4j+3 low and 16+4j..16+4j+3 high) against
// 32 int8 activations.  Each nibble is moved to the top of its byte, which reads it as 16 * (signed value)
// with no sign extension; the sum is then exactly 16 * ival and one arithmetic shift recovers ival.
__device__ __forceinline__ int dot_q4(const uint4 w, const uint32_t *x) {
    int acc = 0;
    acc = __builtin_amdgcn_sdot4((int)((w.x << 4) & 0xF0F0F0F0u), (int)x[0], acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.x & 0xF0F0F0F0u), (int)x[4], acc, false);
    acc = __builtin_amdgcn_sdot4((int)((w.y << 4) & 0xF0F0F0F0u), (int)x[1], acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.y & 0xF0F0F0F0u), (int)x[5], acc, false);
    acc = __builtin_amdgcn_sdot4((int)((w.z << 4) & 0xF0F0F0F0u), (int)x[2], acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.z & 0xF0F0F0F0u), (int)x[6], acc, false);
    acc = __builtin_amdgcn_sdot4((int)((w.w << 4) & 0xF0F0F0F0u), (int)x[3], acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.w & 0xF0F0F0F0u), (int)x[7], acc, false);
    return acc >> 4;
}

// int8 segment of 16 bytes (piece) against 16 int8 activations
__device__ __forceinline__ int dot_q8_piece(const uint4 w, const uint32_t *x, int acc) {
    acc = __builtin_amdgcn_sdot4((int)w.x, (int)x[0], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.y, (int)x[1], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.z, (int)x[2], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w, (int)x[3], acc, false);
    return acc;
}

template <int WB, int GSZ>
__device__ __forceinline__ int seg_dot(const uint4 *wv, const uint32_t *x) {
    if constexpr (WB == 4) {
        return dot_q4(wv[0], x);
    } else {
        int acc = 0;
#pragma unroll
        for (int p = 0; p < GSZ / 16; p++) acc = dot_q8_piece(wv[p], x + 4 * p, acc);
        return acc;
    }
}

// ------------------------------------------------------------------------------------------------------
// GEMV

// Per-format constants.  A batch (the loads one wave keeps in flight per buffer) is 4 KiB of weights:
// 4 chunks of int4 x 32, 2 of int8 x 32, 1 of int8 x 64, so registers stay bounded in every format.
template <int WB, int GSZ, int SF32>
struct Fmt {
    static constexpr int SB = GSZ * WB / 8; // bytes per (row, group) segment
    static constexpr int PIECES = SB / 16;
    static constexpr int SCB = SF32 ? 4 : 2;
    static constexpr int UNROLL = 4 / PIECES;
    // a scale as loaded: fp32 bits, or the fp16 scales of the lane pair (lane & ~1, lane | 1) as one dword,
    // split at use (a 16-bit load would be widened right after it, making the compiler wait for it there)
    using ST = uint32_t;
};

__device__ __forceinline__ float rope_pair_out(float self, float partner, bool first, float c, float s) {
    // qwen.c:483-485 / runq.c:516-519: first = a*c - b*s, second = b*c + a*s (a first, b second element)
    if (first) {
        float t1 = self * c, t2 = partner * s;
        return t1 - t2;
    }
    float t1 = self * c, t2 = partner * s;
    return t1 + t2;
}

// Weights are read through a buffer resource: the record's byte offset is a scalar, the lane's position in the
// record a per-lane constant, so a chunk costs one scalar multiply-add of address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const TiledMat &W) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)W.data, 0, (int)(W.bytes < 0x7fffffffu ? W.bytes : 0x7fffffffu),
                                            0x00020000);
}

// Cache policy of the weight loads (the buffer load's cache-policy operand): 0, or 2 = non-temporal (`nt`).
// GemvArgs::nt selects non-temporal loads when a decode step streams more weights than the MALL keeps.
//
// A buffer load whose lane offset is at or past the resource's size returns zeros without touching memory.
// Loads with nothing to read (a chunk past the row-block's end, a batch past the wave's stream) take this
// offset, so every call issues the same instructions: the compiler then knows exactly how many loads are in
// flight when a batch is used, and waits for that batch alone instead of draining the ones behind it.
#define OOB_OFFSET 0x80000000u
template <int WB, int GSZ, int SF32, int POLICY>
__device__ __forceinline__ void load_batch(__amdgpu_buffer_rsrc_t rs, uint32_t rb_off, uint32_t rec_bytes, int nchunks,
                                           int c0, int kw, int lane, bool live,
                                           uint4 (&wv)[Fmt<WB, GSZ, SF32>::UNROLL][Fmt<WB, GSZ, SF32>::PIECES],
                                           typename Fmt<WB, GSZ, SF32>::ST (&sr)[Fmt<WB, GSZ, SF32>::UNROLL]) {
    using F = Fmt<WB, GSZ, SF32>;
#pragma unroll
    for (int u = 0; u < F::UNROLL; u++) {
        const bool ok = live && c0 + u * kw < nchunks;
        const uint32_t soff = rb_off + (uint32_t)min(c0 + u * kw, nchunks - 1) * rec_bytes;
#pragma unroll
        for (int p = 0; p < F::PIECES; p++) {
            const uint32_t voff = ok ? (uint32_t)(lane * 16 + p * 1024) : OOB_OFFSET;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voff, soff, POLICY);
            wv[u][p] = *(const uint4 *)&v;
        }
        const uint32_t voff_s = ok ? (uint32_t)(64 * F::SB + (SF32 ? lane * 4 : (lane & ~1) * 2)) : OOB_OFFSET;
        sr[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)voff_s, soff, POLICY);
    }
}

// The lane's scale from what load_batch read: fp32 bits, or its half of the lane pair's two fp16 scales.
template <int SF32>
__device__ __forceinline__ float scale_of(uint32_t v) {
    if constexpr (SF32) return __uint_as_float(v);
    return f16_bits_to_f32((uint16_t)((__lane_id() & 1) ? v >> 16 : v));
}

// groups of one batch, added to the lane's running sum in chunk order: p_g = ((float)ival * ws) * xs
template <int WB, int GSZ, int SF32>
__device__ __forceinline__ float use_batch(float acc, int nchunks, int c0, int kw, int gpc, int g_lane, const int8_t *sxq,
                                           const float *sxs,
                                           const uint4 (&wv)[Fmt<WB, GSZ, SF32>::UNROLL][Fmt<WB, GSZ, SF32>::PIECES],
                                           const typename Fmt<WB, GSZ, SF32>::ST (&sr)[Fmt<WB, GSZ, SF32>::UNROLL]) {
    using F = Fmt<WB, GSZ, SF32>;
#pragma unroll
    for (int u = 0; u < F::UNROLL; u++) {
        const int c = c0 + u * kw;
        if (c < nchunks) {
            const int g = c * gpc + g_lane;
            const int iv = seg_dot<WB, GSZ>(wv[u], (const uint32_t *)(sxq + g * GSZ));
            const float sc = scale_of<SF32>(sr[u]);
            float p = (float)iv * sc; // qwen.c:452, runq.c:452
            p = p * sxs[g];
            acc = acc + p;
        }
    }
    return acc;
}

// Logical row R of the fused QKV matrix with NeoX pairing: element, partner element, frequency index.
__device__ __forceinline__ void qkv_neox_row(int R, int hs, int *e, int *ep, int *i, bool *first) {
    const int half = hs / 2, blk = R / 16, r = R & 15, per = half / 8;
    const int hh = blk / per;
    *i = (blk - hh * per) * 8 + (r & 7);
    *first = r < 8;
    *e = hh * hs + (r < 8 ? *i : half + *i);
    *ep = hh * hs + (r < 8 ? half + *i : *i);
}

// Smallest power of two >= s (s in 1..64): the lanes that one head's attention slices take in the merge.
__device__ __forceinline__ int pow2_at_least(int s) {
    int w = 1;
    while (w < s) w <<= 1;
    return w;
}

// Merge weights of the attention slices of head h (SW lanes per head, lane k holds slice k's (max, sum)):
// exp(m_k - m) / sum_j l_j exp(m_j - m), m the largest slice maximum (the softmax of qwen.c:346-352 taken
// over the slices).
__device__ __forceinline__ void merge_weights(float2 st, int h, int k, int S, int SW, int nh, float *wgt) {
    const bool ok = h < nh && k < S;
    const float mk = ok ? st.x : -INFINITY;
    const float m = group_max(mk, SW);
    const float f = ok ? expf(mk - m) : 0.0f;
    float l = ok ? st.y * f : 0.0f;
    for (int off = 1; off < SW; off <<= 1) l += __shfl_xor(l, off);
    if (ok) wgt[h * S + k] = f * (1.0f / l);
}

// Ordered mode: the batch's group products p_g = ((float)ival * ws) * xs, each stored at (row, group) in LDS,
// so that one lane per row can add them in group order afterwards (runq.c:452-456 adds them sequentially).
template <int WB, int GSZ, int SF32>
__device__ __forceinline__ void store_batch(float *sprod, int ng, int row_l, int nchunks, int c0, int kw, int gpc,
                                            int g_lane, const int8_t *sxq, const float *sxs,
                                            const uint4 (&wv)[Fmt<WB, GSZ, SF32>::UNROLL][Fmt<WB, GSZ, SF32>::PIECES],
                                            const typename Fmt<WB, GSZ, SF32>::ST (&sr)[Fmt<WB, GSZ, SF32>::UNROLL]) {
    using F = Fmt<WB, GSZ, SF32>;
#pragma unroll
    for (int u = 0; u < F::UNROLL; u++) {
        const int c = c0 + u * kw, g = c * gpc + g_lane;
        if (c < nchunks && g < ng) { // groups past n (padding of the last chunk) have no slot
            const int iv = seg_dot<WB, GSZ>(wv[u], (const uint32_t *)(sxq + g * GSZ));
            const float sc = scale_of<SF32>(sr[u]);
            float p = (float)iv * sc; // qwen.c:452, runq.c:452
            p = p * sxs[g];
            sprod[row_l * (ng + 1) + g] = p;
        }
    }
}

// 16 bytes as a native vector: copied as a register value (a struct copy would go through memory)
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Vectors of 16 bytes per thread that a prologue loads in its first pass, before the weights.
#define PRO_VEC 4
// Slices of attention partials one merge pass loads per thread.
#define MERGE_KB 8

// The decode GEMV.  WB/GSZ/SF32: weight format; PRO/EPI: prologue and epilogue; D: weight batches in flight per
// wave; NT: non-temporal weight loads (GemvArgs::nt).
template <int WB, int GSZ, int SF32, int PRO, int EPI, int D, int NT>
__global__ void __launch_bounds__(D == 4 ? 512 : 1024) k_gemv(GemvArgs a) {
    using F = Fmt<WB, GSZ, SF32>;
    // the activation quantization flavour follows the weight format: fp16 scales are the Qwen .qwb path
    // (qwen.c quantize), fp32 scales the llama2.c .bin path (runq.c quantize); the launcher checks it
    constexpr int QF = SF32 ? QF_RUNQ : QF_QWEN;
    extern __shared__ __align__(16) uint8_t lds[];
    const TiledMat &W = a.W;
    const int rb = W.rb, gpc = WAVE / rb, ngp = W.nchunks * gpc, ngp4 = (ngp + 3) & ~3;
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & (WAVE - 1), nw = nt / WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE); // uniform: wave-level branches stay scalar
    const int n = W.n;
    int8_t *sxq = (int8_t *)lds;                          // ngp * GSZ
    float *sxs = (float *)(lds + (size_t)ngp * GSZ);      // ngp4
    float *sred = sxs + ngp4;                             // nw * 64
    float *srow = sred + nw * WAVE;                       // nb * rb
    // ordered mode: the group products of the iteration's rows, rows_it x (ng + 1) (padded against bank
    // conflicts), summed per row in group order by finish()
    const int ngs = W.ng + 1;
    float *sprod = srow + a.nb * rb;
    float *sv = sprod + (a.ord ? a.nb * rb * ngs : 0);    // prologue / epilogue floats
    // wave = my_kw * nb + my_nb (nb a power of two); the launcher precomputes every quotient the shape needs
    const int my_nb = wave & (a.nb - 1), my_kw = wave >> a.nb_log2;
    const int rows_it = a.nb * rb;
    const int g_lane = lane >> a.rb_log2;
    const int it0 = blockIdx.x;
    KERNEL_MARK(0);
    const bool need_pos = PRO == PRO_ATTN || EPI == EPI_QKV || EPI == EPI_ARGMAX;
    const int pos = need_pos ? a.ctrl->pos : 0;

    // The weight stream: the batches of all the block's iterations (it0, it0 + grid, ...) form one stream per
    // wave, bpi batches per iteration, D register buffers in a ring; the next iteration's first batches are in
    // flight while the current one is reduced and finished.  issue() always issues a whole batch (past the
    // stream's end, out-of-range loads that read nothing), so the number of loads behind every batch is the
    // same on every path.
    const int cnt_w = a.kw_base + (my_kw < a.kw_rem);           // chunks of a row-block for this wave (>= 1)
    const int bpi = (cnt_w + F::UNROLL - 1) / F::UNROLL;         // batches per iteration
    const int n_my = a.it_base + (it0 < a.it_rem);               // iterations it0, it0 + grid, ... < n_it
    const int total = n_my * bpi;
    float pre_x = 0.0f; // EPI_RESID: out[R] of the first iteration's row
    int iss_it = it0, iss_bi = 0, iss_n = 0; // the next batch to issue, batches issued
    const __amdgpu_buffer_rsrc_t wrs = weight_rsrc(W);
    const uint32_t rec = (uint32_t)W.rec, rb_bytes = (uint32_t)W.nchunks * rec;
    auto issue = [&](uint4 (&w)[F::UNROLL][F::PIECES], typename F::ST (&sr)[F::UNROLL]) {
        const int b = min(iss_it * a.nb + my_nb, W.nblocks - 1);
        load_batch<WB, GSZ, SF32, NT ? 2 : 0>(wrs, (uint32_t)b * rb_bytes, rec, W.nchunks, my_kw + iss_bi * F::UNROLL * a.kw, a.kw,
                                  lane, iss_n < total, w, sr);
        iss_n++;
        if (++iss_bi == bpi) {
            iss_bi = 0;
            iss_it += gridDim.x;
        }
    };
    uint4 wr[D][F::UNROLL][F::PIECES];
    typename F::ST sr[D][F::UNROLL];
    // The attention merge needs the position before it can read its operands: one weight batch goes out
    // first and is in flight meanwhile.
    constexpr int D_PRE = PRO == PRO_ATTN ? 1 : 0;
#pragma unroll
    for (int d = 0; d < D_PRE; d++) issue(wr[d], sr[d]);

    // (1) the prologue's operands for its first pass, issued before the rest of the weights: loads complete
    // in issue order, so waiting for these does not also wait for the weights issued after them.  Indices
    // past the end are clamped (the values are loaded and never used).  Vectors beyond the first pass (longer
    // inputs than the block covers) are loaded and parked in LDS here too, so that no load issued after the
    // weights has to be waited for before the weights are used.
    u32x4 px[PRO_VEC];      // PRO_XQ: 16 int8 activations each
    float pxs[2];           // PRO_XQ: group scales
    float4 pn[PRO_VEC], pg[PRO_VEC]; // PRO_NORM: x and gains
    float2 pst = make_float2(0.0f, 0.0f); // PRO_ATTN: (max, sum) of one (head, slice)
    float4 pab[MERGE_KB];   // PRO_ATTN: value sums of the first slot's first slices
    int S = 1, SW = 1;      // PRO_ATTN: slices of this step, lanes per head in the statistics
    if constexpr (PRO == PRO_XQ) {
        const u32x4 *src = (const u32x4 *)a.xq;
        const int nq = n / 16;
#pragma unroll
        for (int k = 0; k < PRO_VEC; k++) px[k] = src[min(tid + k * nt, nq - 1)];
#pragma unroll
        for (int k = 0; k < 2; k++) pxs[k] = a.xs[min(tid + k * nt, W.ng - 1)];
        for (int i = PRO_VEC * nt + tid; i < nq; i += nt) ((u32x4 *)sxq)[i] = src[i];
        for (int i = 2 * nt + tid; i < W.ng; i += nt) sxs[i] = a.xs[i];
    } else if constexpr (PRO == PRO_NORM) {
        const float4 *x4 = (const float4 *)a.x, *w4 = (const float4 *)a.norm_w;
        const int nv = n / 4;
#pragma unroll
        for (int k = 0; k < PRO_VEC; k++) {
            const int i = min(tid + k * nt, nv - 1);
            pn[k] = x4[i];
            pg[k] = w4[i];
        }
        float4 *sv4 = (float4 *)sv; // x in sv, gains in the n floats after it
        for (int i = PRO_VEC * nt + tid; i < nv; i += nt) {
            sv4[i] = x4[i];
            sv4[nv + i] = w4[i];
        }
    } else if constexpr (PRO == PRO_ATTN) {
        const int hs = a.head_size, SP = a.att_splits, nh = a.n_heads;
        int chunk;
        att_slices(pos, SP, &S, &chunk);
        SW = pow2_at_least(S);
        const int h = wave * (WAVE / SW) + lane / SW, k = lane & (SW - 1);
        pst = ((const float2 *)a.att_ml)[(size_t)min(h, nh - 1) * SP + min(k, S - 1)];
        const int v = min(tid, n / 4 - 1), hh = 4 * v / hs, e = 4 * v - hh * hs;
#pragma unroll
        for (int kk = 0; kk < MERGE_KB; kk++)
            pab[kk] = *(const float4 *)(a.att_acc + ((size_t)hh * SP + min(kk, S - 1)) * hs + e);
    }

    asm volatile("" ::: "memory"); // keep the issue order: prologue operands, then weights

    // (2) the wave's first D weight batches
#pragma unroll
    for (int d = D_PRE; d < D; d++) issue(wr[d], sr[d]);

    // (3) the epilogue operands of this thread's first row (clamped row index, used only for valid rows)
    float pre_b = 0.0f, pre_bp = 0.0f, pre_c = 0.0f, pre_s = 0.0f;
    {
        const int R = min(it0 * rows_it + tid, W.rows - 1);
        if constexpr (EPI == EPI_RESID) pre_x = a.out[R];
        if constexpr (EPI == EPI_QKV) {
            // the same loads on both pairings (the interleaved pairing has no bias: out-of-range reads)
            const int half = a.head_size / 2, rot = a.dim + a.kv_dim, Rr = min(R, rot - 1);
            const bool neox = a.rope_kind == ROPE_NEOX;
            int i, ib = 0, ibp = 0;
            if (neox) {
                int e, ep;
                bool first;
                qkv_neox_row(Rr, a.head_size, &e, &ep, &i, &first);
                ib = R < rot ? e : R;
                ibp = R < rot ? ep : R;
            } else {
                const int e = Rr < a.dim ? Rr : Rr - a.dim;
                i = (e % a.head_size) / 2;
            }
            const __amdgpu_buffer_rsrc_t brs =
                __builtin_amdgcn_make_buffer_rsrc((void *)a.bias, 0, a.bias ? W.rows * 4 : 0, 0x00020000);
            pre_b = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(brs, neox ? ib * 4 : (int)OOB_OFFSET, 0, 0));
            pre_bp = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(brs, neox ? ibp * 4 : (int)OOB_OFFSET, 0, 0));
            pre_c = a.rope_cos[(size_t)pos * half + i];
            pre_s = a.rope_sin[(size_t)pos * half + i];
        }
    }
    asm volatile("" ::: "memory"); // every load above is issued before the prologue's work begins

    KERNEL_MARK(1);
    // (4) prologue: int8 activations and their scales into LDS
    bool in_regs = false; // PRO_NORM: normalized and quantized straight from the registers
    if constexpr (PRO == PRO_XQ) {
        const int nq = n / 16;
        u32x4 *dst = (u32x4 *)sxq;
        // stores at the clamped index too: a thread past the end writes the last vector's own value again
        // (an unconditional use keeps the compiler from moving the loads down to here)
#pragma unroll
        for (int k = 0; k < PRO_VEC; k++) dst[min(tid + k * nt, nq - 1)] = px[k];
#pragma unroll
        for (int k = 0; k < 2; k++) sxs[min(tid + k * nt, W.ng - 1)] = pxs[k];
    } else {
        float4 *sv4 = (float4 *)sv;
        if constexpr (PRO == PRO_NORM) {
            // rmsnorm (qwen.c:337-344, runq.c:394-407): ss = sum x^2; ss /= n; ss += eps; ss = 1/sqrtf(ss)
            const int nv = n / 4;
            float part = 0.0f;
#pragma unroll
            for (int k = 0; k < PRO_VEC; k++)
                if (tid + k * nt < nv) {
                    const float4 v = pn[k];
                    part += v.x * v.x;
                    part += v.y * v.y;
                    part += v.z * v.z;
                    part += v.w * v.w;
                }
            // vectors beyond the first pass were parked in LDS by this same thread (x in sv, gains after it)
            for (int i = PRO_VEC * nt + tid; i < nv; i += nt) {
                const float4 v = sv4[i];
                part += v.x * v.x;
                part += v.y * v.y;
                part += v.z * v.z;
                part += v.w * v.w;
            }
            KERNEL_MARK(2);
            float ss;
            if (a.strict) { // one running sum of the rounded squares in element order, as the reference's loop
                // the squares x[i] * x[i] (each rounded, as the reference's), and after them the sum's scratch: in
                // x's own area when x stays in registers, else after x and the gains parked in LDS
                const bool regs = nv <= PRO_VEC * nt;
                float4 *q4 = (float4 *)(regs ? sv : sv + 2 * n);
#pragma unroll
                for (int k = 0; k < PRO_VEC; k++)
                    if (tid + k * nt < nv) {
                        const float4 v = pn[k];
                        q4[tid + k * nt] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
                    }
                for (int i = PRO_VEC * nt + tid; i < nv; i += nt) {
                    const float4 v = sv4[i];
                    q4[i] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
                }
                __syncthreads();
                ss = block_seq_sum((const float *)q4, n, (uint8_t *)((float *)q4 + n));
            } else {
                ss = block_sum(part, sred);
            }
            ss /= (float)n;
            ss += a.eps;
            ss = 1.0f / sqrtf(ss);
            in_regs = nv <= PRO_VEC * nt;
            if (in_regs) { // the whole vector is in registers: normalize and quantize in one pass
#pragma unroll
                for (int k = 0; k < PRO_VEC; k++)
                    if (k * nt < nv) { // uniform; a slot past nv belongs to a group that is wholly past it
                        const int i = tid + k * nt;
                        const float4 v = pn[k], g = pg[k];
                        const float4 o = make_float4(g.x * (ss * v.x), g.y * (ss * v.y), g.z * (ss * v.z), g.w * (ss * v.w));
                        quantize_slot(o, i, i < nv, GSZ, QF, sxq, sxs);
                    }
            } else {
#pragma unroll
                for (int k = 0; k < PRO_VEC; k++)
                    if (tid + k * nt < nv) {
                        const float4 v = pn[k], g = pg[k];
                        sv4[tid + k * nt] = make_float4(g.x * (ss * v.x), g.y * (ss * v.y), g.z * (ss * v.z), g.w * (ss * v.w));
                    }
                for (int i = PRO_VEC * nt + tid; i < nv; i += nt) {
                    const float4 v = sv4[i], g = sv4[nv + i];
                    sv4[i] = make_float4(g.x * (ss * v.x), g.y * (ss * v.y), g.z * (ss * v.z), g.w * (ss * v.w));
                }
            }
        } else { // PRO_ATTN: merge the attention slices of every head, then xb = acc / l
            // statistics: SW lanes per head, lane k holds slice k
            const int hs = a.head_size, SP = a.att_splits, nh = a.n_heads, hpp = nw * (WAVE / SW);
            float *wgt = sv + n; // nh * S
            const int k = lane & (SW - 1), h_lane = wave * (WAVE / SW) + lane / SW;
            merge_weights(pst, h_lane, k, S, SW, nh, wgt);
            for (int h0 = hpp; h0 < nh; h0 += hpp) {
                const int h = h0 + h_lane;
                merge_weights(((const float2 *)a.att_ml)[(size_t)min(h, nh - 1) * SP + min(k, S - 1)], h, k, S, SW,
                              nh, wgt);
            }
            __syncthreads();
            KERNEL_MARK(2);
            // value slots of 4 elements: sum over slices in slice order
            const int nv = n / 4;
            for (int v0 = 0; v0 < nv; v0 += nt) {
                const int v = min(v0 + tid, nv - 1), hh = 4 * v / hs, e = 4 * v - hh * hs;
                float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                for (int k0 = 0; k0 < S; k0 += MERGE_KB) {
                    if (v0 != 0 || k0 != 0) {
#pragma unroll
                        for (int kk = 0; kk < MERGE_KB; kk++)
                            pab[kk] = *(const float4 *)(a.att_acc + ((size_t)hh * SP + min(k0 + kk, S - 1)) * hs + e);
                    }
#pragma unroll
                    for (int kk = 0; kk < MERGE_KB; kk++)
                        if (k0 + kk < S) {
                            const float w = wgt[hh * S + k0 + kk];
                            acc.x += pab[kk].x * w;
                            acc.y += pab[kk].y * w;
                            acc.z += pab[kk].z * w;
                            acc.w += pab[kk].w * w;
                        }
                }
                if (v0 + tid < nv) sv4[v0 + tid] = acc;
            }
        }
        if (!in_regs) {
            __syncthreads();
            KERNEL_MARK(3);
            block_quantize(sv, n, GSZ, QF, sxq, sxs);
        }
        for (int i = n + tid; i < ngp * GSZ; i += nt) sxq[i] = 0;
    }
    for (int i = W.ng + tid; i < ngp; i += nt) sxs[i] = 0.0f;
    if constexpr (PRO == PRO_XQ)
        for (int i = n + tid; i < ngp * GSZ; i += nt) sxq[i] = 0;
    __syncthreads();
    KERNEL_MARK(4);

    // (5) reduction and epilogue of iteration `it` (every wave calls it once per iteration: barriers inside)
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    auto finish = [&](int it, float acc) {
        KERNEL_MARK(5);
        if (a.ord) { // every group product is in LDS: one thread per row adds them in group order
            __syncthreads();
            if (tid < rows_it) srow[tid] = seq_sum(sprod + tid * ngs, W.ng);
        } else {
            acc = wave_sum_from(acc, rb); // lanes holding the same row
            if (lane < rb) sred[wave * rb + lane] = acc;
            __syncthreads();
            if (tid < rows_it) {
                const int nbi = tid >> a.rb_log2, r = tid & (rb - 1);
                float v = 0.0f;
                for (int k = 0; k < a.kw; k++) v += sred[(k * a.nb + nbi) * rb + r];
                srow[tid] = v;
            }
        }
        __syncthreads();
        KERNEL_MARK(6);

        const int R = it * rows_it + tid; // logical row of this thread
        const bool first_it = it == it0;
        if constexpr (EPI == EPI_STORE) {
            if (tid < rows_it && R < W.rows) a.out[R] = srow[tid];
        } else if constexpr (EPI == EPI_RESID) {
            // the first iteration's operand was read at the start; later ones (blocks of several
            // iterations) read theirs here
            if (tid < rows_it && R < W.rows) a.out[R] = (first_it ? pre_x : a.out[R]) + srow[tid]; // qwen.c:551, 565
        } else if constexpr (EPI == EPI_ARGMAX) {
            if (tid < rows_it && R < W.rows) {
                const float v = srow[tid];
                a.out[R] = v;
                if (a.logits_hist) a.logits_hist[(size_t)pos * W.rows + R] = v;
                if (v > best_v) { best_v = v; best_i = R; } // rows grow with it: strict > keeps the first
            }
        } else if constexpr (EPI == EPI_QKV) {
            if (tid < rows_it && R < W.rows) {
                const int dim = a.dim, kvd = a.kv_dim, hs = a.head_size, half = hs / 2;
                const float v = srow[tid];
                if (a.rope_kind == ROPE_NEOX) {
                    // rows [0, dim + kv) hold q then k in blocks of 16: 8 first-half rows, then their 8 partners
                    if (R < dim + kvd) {
                        int e, ep, i;
                        bool first;
                        qkv_neox_row(R, hs, &e, &ep, &i, &first);
                        float bs = pre_b, bp = pre_bp, c = pre_c, sn = pre_s;
                        if (!first_it) {
                            bs = a.bias[e];
                            bp = a.bias[ep];
                            c = a.rope_cos[(size_t)pos * half + i];
                            sn = a.rope_sin[(size_t)pos * half + i];
                        }
                        const float o = rope_pair_out(v + bs, srow[tid ^ 8] + bp, first, c, sn);
                        if (e < dim) a.q[e] = o;
                        else a.kc[(size_t)pos * kvd + (e - dim)] = o;
                    } else {
                        const float bs = first_it ? pre_b : a.bias[R];
                        a.vc[(size_t)pos * kvd + (R - dim - kvd)] = v + bs;
                    }
                } else {
                    // natural order q, k, v; pairs (2i, 2i+1) rotate (runq.c:506-521)
                    if (R < dim + kvd) {
                        const int e = R < dim ? R : R - dim;
                        const int i = (e % hs) / 2;
                        float c = pre_c, sn = pre_s;
                        if (!first_it) {
                            c = a.rope_cos[(size_t)pos * half + i];
                            sn = a.rope_sin[(size_t)pos * half + i];
                        }
                        const float partner = srow[tid ^ 1];
                        // first: v0*fcr - v1*fci; second: v0*fci + v1*fcr (v0 first, v1 second)
                        float o;
                        if ((e & 1) == 0) { float t1 = v * c, t2 = partner * sn; o = t1 - t2; }
                        else { float t1 = partner * sn, t2 = v * c; o = t1 + t2; }
                        if (R < dim) a.q[e] = o;
                        else a.kc[(size_t)pos * kvd + e] = o;
                    } else {
                        a.vc[(size_t)pos * kvd + (R - dim - kvd)] = v;
                    }
                }
            }
        } else if constexpr (EPI == EPI_SWIGLU) {
            // each row-block holds rb/2 gate rows then the rb/2 matching up rows (qwen.c:556-562)
            const int hb = rb / 2, per_it = a.nb * hb;
            if (tid < rows_it) {
                const int nbi = tid >> a.rb_log2, r = tid & (rb - 1);
                if (r < hb) {
                    float g = srow[tid], u = srow[tid + hb];
                    float sig = 1.0f / (1.0f + (a.strict ? ref_expf(-g) : expf(-g)));
                    g = g * sig;
                    sv[nbi * hb + r] = g * u;
                }
            }
            __syncthreads();
            const int j0 = it * per_it;
            if (j0 < a.dim) { // a.dim holds the hidden size here
                const int cnt = min(per_it, a.dim - j0);
                if (a.hf)
                    for (int i = tid; i < cnt; i += nt) a.hf[j0 + i] = sv[i];
                block_quantize(sv, cnt, GSZ, QF, a.hq + j0, a.hs + j0 / GSZ);
            }
        }
        __syncthreads();
    };

    // (6) the stream: consume a batch, refill its buffer with the batch D ahead
    int use_it = it0, use_bi = 0;
    float acc = 0.0f;
    auto use = [&](const uint4 (&w)[F::UNROLL][F::PIECES], const typename F::ST (&sr)[F::UNROLL]) {
        if (use_it * a.nb + my_nb < W.nblocks) {
            if (a.ord)
                store_batch<WB, GSZ, SF32>(sprod, W.ng, my_nb * rb + (lane & (rb - 1)), W.nchunks,
                                           my_kw + use_bi * F::UNROLL * a.kw, a.kw, gpc, g_lane, sxq, sxs, w, sr);
            else
                acc = use_batch<WB, GSZ, SF32>(acc, W.nchunks, my_kw + use_bi * F::UNROLL * a.kw, a.kw, gpc, g_lane,
                                              sxq, sxs, w, sr);
        }
        use_bi++;
    };
    if (EPI == EPI_ARGMAX || a.ord) {
        // several iterations per block (a persistent grid over the long head, or ordered sums, whose per-row
        // running sums at the end of an iteration are long): reduce and finish each iteration as its last
        // batch is used, while the next iteration's batches are in flight
        for (int q = 0; q < total; q += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                if (q + d < total) {
                    use(wr[d], sr[d]);
                    if (use_bi == bpi) {
                        finish(use_it, acc);
                        acc = 0.0f;
                        use_bi = 0;
                        use_it += gridDim.x;
                    }
                }
                issue(wr[d], sr[d]); // past the stream's end: loads that read nothing
            }
        }
    } else {
        // one iteration per block (the launcher runs one block per iteration).  Whole rounds of D uses, each
        // refilling its buffer, while a later round remains; then the last round uses what is in flight.
        // Batches past this wave's count (at most D - 1, when D does not divide it) read nothing.
        const int nbat_r = (total + D - 1) / D * D;
        int j = 0;
        for (; j < nbat_r - D; j += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                use(wr[d], sr[d]);
                issue(wr[d], sr[d]);
            }
        }
#pragma unroll
        for (int d = 0; d < D; d++)
            if (j + d < total) use(wr[d], sr[d]);
        finish(it0, acc);
    }
    if constexpr (EPI == EPI_ARGMAX) {
        // block argmax: larger value wins, equal values keep the lower row (first strict maximum)
        float v = best_v;
        int i = best_i;
        for (int off = 1; off < WAVE; off <<= 1) {
            float ov = __shfl_xor(v, off);
            int oi = __shfl_xor(i, off);
            if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
        }
        int *si = (int *)(sred + nw);
        if (lane == 0) { sred[wave] = v; si[wave] = i; }
        __syncthreads();
        if (tid == 0) {
            for (int k = 1; k < nw; k++)
                if (sred[k] > v || (sred[k] == v && si[k] < i)) { v = sred[k]; i = si[k]; }
            a.part_val[blockIdx.x] = v;
            a.part_idx[blockIdx.x] = i;
        }
    }
    KERNEL_MARK(7);
}

size_t gemv_lds_bytes(const GemvArgs &a, int pro, int epi, int threads) {
    const TiledMat &W = a.W;
    const int ngp = W.nchunks * (WAVE / W.rb), ngp4 = (ngp + 3) & ~3;
    size_t b = (size_t)ngp * W.gs + (size_t)ngp4 * 4 + (size_t)(threads / WAVE) * WAVE * 4 + (size_t)a.nb * W.rb * 4;
    if (a.ord) b += (size_t)a.nb * W.rb * (W.ng + 1) * 4; // group products of the ordered mode
    size_t extra = 0;
    if (pro == PRO_NORM) {
        extra = (size_t)W.n * 8;
        // the strict sum's squares and scratch: in x's area when x stays in registers, else after x and the gains
        if (a.strict) {
            const size_t scr = seq_sum_scratch_bytes(threads);
            extra = W.n / 4 <= PRO_VEC * threads ? std::max(extra, (size_t)W.n * 4 + scr) : (size_t)W.n * 12 + scr;
        }
    }
    if (pro == PRO_ATTN) extra = (size_t)W.n * 4 + (size_t)a.n_heads * a.att_splits * 4;
    if (epi == EPI_SWIGLU) extra = extra > (size_t)a.nb * W.rb * 2 ? extra : (size_t)a.nb * W.rb * 2;
    return b + extra + 16;
}

template <int WB, int GSZ, int SF32, int PRO, int EPI>
static hipError_t launch_one(const GemvArgs &a, int grid, hipStream_t st) {
    const int threads = a.kw * a.nb * WAVE;
    const size_t lds = gemv_lds_bytes(a, PRO, EPI, threads);
    // the QKV epilogue keeps one weight batch in flight per wave: with two, its 1024-thread kernels would not fit
    // their registers
    if (a.depth == 1 || EPI == EPI_QKV) {
        if (a.nt) hipLaunchKernelGGL((k_gemv<WB, GSZ, SF32, PRO, EPI, 1, 1>), dim3(grid), dim3(threads), lds, st, a);
        else hipLaunchKernelGGL((k_gemv<WB, GSZ, SF32, PRO, EPI, 1, 0>), dim3(grid), dim3(threads), lds, st, a);
    } else if constexpr (EPI != EPI_QKV) {
        if (a.nt) hipLaunchKernelGGL((k_gemv<WB, GSZ, SF32, PRO, EPI, 2, 1>), dim3(grid), dim3(threads), lds, st, a);
        else hipLaunchKernelGGL((k_gemv<WB, GSZ, SF32, PRO, EPI, 2, 0>), dim3(grid), dim3(threads), lds, st, a);
    }
    return hipGetLastError();
}

static int log2_exact(int v) { // log2 of a power of two, -1 otherwise
    int k = 0;
    while ((1 << k) < v) k++;
    return (1 << k) == v ? k : -1;
}

template <int WB, int GSZ, int SF32>
static hipError_t launch_fmt(int pro, int epi, const GemvArgs &a, int grid, hipStream_t st) {
#define CASE(P, E) if (pro == P && epi == E) return launch_one<WB, GSZ, SF32, P, E>(a, grid, st)
    CASE(PRO_XQ, EPI_STORE);
    CASE(PRO_XQ, EPI_RESID);
    CASE(PRO_NORM, EPI_QKV);
    CASE(PRO_ATTN, EPI_RESID);
    CASE(PRO_NORM, EPI_SWIGLU);
    CASE(PRO_NORM, EPI_ARGMAX);
#undef CASE
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(int wbits, int gs, int sf32, int pro, int epi, const GemvArgs &args, int grid, hipStream_t st) {
    // quotients of the launch shape, so the kernel divides nothing: nb and rb are powers of two
    GemvArgs a = args;
    const int nb_log2 = log2_exact(a.nb), rb_log2 = log2_exact(a.W.rb);
    if (nb_log2 < 0 || rb_log2 < 0 || a.kw < 1 || a.kw > a.W.nchunks || a.kw * a.nb > 16 || grid < 1) return hipErrorInvalidValue;
    a.nb_log2 = nb_log2;
    a.rb_log2 = rb_log2;
    a.n_it = (a.W.nblocks + a.nb - 1) / a.nb;
    a.kw_base = a.W.nchunks / a.kw;
    a.kw_rem = a.W.nchunks % a.kw;
    a.it_base = a.n_it / grid;
    a.it_rem = a.n_it % grid;
    // the kernels quantize activations in the flavour of their weight format (QF in k_gemv)
    if (pro != PRO_XQ || epi == EPI_SWIGLU)
        if (a.qflavor != (sf32 ? QF_RUNQ : QF_QWEN) || a.W.gs != gs) return hipErrorInvalidValue;
    // one block per iteration, except the head's argmax epilogue and ordered sums (persistent grids)
    if (epi != EPI_ARGMAX && !a.ord && grid != a.n_it) return hipErrorInvalidValue;
    // stream depth: 2 batches in flight per wave when some wave has a second batch to read, else 1
    const int pieces = gs * wbits / 8 / 16, unroll = pieces > 0 && pieces <= 4 ? 4 / pieces : 1; // Fmt::UNROLL
    const int max_total = (a.kw_base + (a.kw_rem > 0) + unroll - 1) / unroll * (a.it_base + (a.it_rem > 0));
    a.depth = a.depth != 1 && max_total >= 2 ? 2 : 1;
    // the prologues read their inputs as 16-byte vectors (8 bytes for the attention statistics)
    auto al = [](const void *p, uintptr_t m) { return ((uintptr_t)p & (m - 1)) == 0; };
    if (a.W.n % 32 || a.W.bytes >= 0x7fffffffu || (pro == PRO_XQ && !al(a.xq, 16)) || (pro == PRO_NORM && (!al(a.x, 16) || !al(a.norm_w, 16))) ||
        (pro == PRO_ATTN && (!al(a.att_acc, 16) || !al(a.att_ml, 8) || a.head_size % 4 || a.att_splits < 1 ||
                             a.att_splits > 64)))
        return hipErrorInvalidValue;
    if (wbits == 4 && gs == 32 && !sf32) return launch_fmt<4, 32, 0>(pro, epi, a, grid, st);
    if (wbits == 8 && gs == 32 && !sf32) return launch_fmt<8, 32, 0>(pro, epi, a, grid, st);
    if (wbits == 8 && gs == 32 && sf32) return launch_fmt<8, 32, 1>(pro, epi, a, grid, st);
    if (wbits == 8 && gs == 64 && sf32) return launch_fmt<8, 64, 1>(pro, epi, a, grid, st);
    return hipErrorInvalidValue;
}

// ------------------------------------------------------------------------------------------------------
// decode attention (qwen.c:526-546, runq.c:530-568), split over positions.  The P = pos+1 positions are
// cut into S = min(splits, ceil(P/32)) equal slices; block (kv head, slice) holds the slice's K and V rows
// in LDS 32 positions at a time and serves the kv_mul query heads that share the kv head.  It leaves the
// slice's running max, sum of exponentials and exp-weighted value sum (online softmax), which the
// o-projection's prologue merges.  Scores are sequential dot products in the reference's order.

__global__ void __launch_bounds__(256) k_attention(AttnArgs a) {
    extern __shared__ __align__(16) float sm[];
    const int pos = a.ctrl->pos;
    const int kvh = blockIdx.x / a.splits, s = blockIdx.x - kvh * a.splits;
    int S, chunk;
    att_slices(pos, a.splits, &S, &chunk);
    if (s >= S) return;
    KERNEL_MARK(0);
    const int t_begin = s * chunk, t_end = min(t_begin + chunk, pos + 1);
    const int hs = a.hs, kv_mul = a.n_heads / a.n_kv, tid = threadIdx.x, nt = blockDim.x;
    float acc[4];
    const float *ml_max, *ml_sum;
    attn_range(a.q + (size_t)kvh * kv_mul * hs, a.kc, a.vc, a.kv_dim, kvh, hs, kv_mul, t_begin, t_end, sm, acc,
               &ml_max, &ml_sum);
    const int n_out = kv_mul * hs;
    for (int k = 0; k < 4; k++) {
        const int o = tid + k * nt;
        if (o < n_out) {
            const int j = o / hs, e = o - j * hs;
            a.acc[((size_t)(kvh * kv_mul + j) * a.splits + s) * hs + e] = acc[k];
        }
    }
    if (tid < kv_mul) {
        float *ml = a.ml + ((size_t)(kvh * kv_mul + tid) * a.splits + s) * 2;
        ml[0] = ml_max[tid];
        ml[1] = ml_sum[tid];
    }
    KERNEL_MARK(7);
}

// Decode attention when every slice has at most 64 positions (ATT_SHORT_MAX).  One block per (kv head,
// slice): its threads stage the group's queries, the slice's K rows (padded to hs + 4 floats) and V rows in
// LDS with one round of coalesced buffer loads (rows past the slice fall outside the buffer range and read
// nothing), then wave j takes query head kvh * kv_mul + j with no further barrier.  Scores: lane t holds
// position t0 + t and forms q . k in the reference's element order; the slice's max and sum of exponentials by
// DPP.  Values: lane l holds elements EPL * l ..: the sum over t of exp(s_t - max) * v[t][e] in position order,
// the weight taken from lane t.  Leaves the same per-slice partials as k_attention.
#define ATT_SHORT_MAX 64
#define ATT_SHORT_LOADS 8   // K (and V) loads per thread: ceil(ATT_SHORT_MAX / rows per pass) <= 8
static inline size_t attn_short_lds_floats(int kv_mul, int hs) {
    return (size_t)kv_mul * hs + (size_t)ATT_SHORT_MAX * (hs + 4) + (size_t)ATT_SHORT_MAX * hs;
}

template <int EPL>
__global__ void __launch_bounds__(512) k_attention_short(AttnArgs a) {
    extern __shared__ __align__(16) float sm[];
    const int pos = a.ctrl->pos;
    const int kvh = blockIdx.x / a.splits, s = blockIdx.x - kvh * a.splits;
    int S, chunk;
    att_slices(pos, a.splits, &S, &chunk);
    if (s >= S) return;
    KERNEL_MARK(0);
    const int kv_mul = a.n_heads / a.n_kv, hs = a.hs, hs4 = hs / 4, ks = hs + 4, nt = blockDim.x;
    const int tid = threadIdx.x, t0 = s * chunk, T = min(chunk, pos + 1 - t0); // 1 <= T <= 64
    float *sq = sm, *sk = sq + kv_mul * hs, *sv = sk + ATT_SHORT_MAX * ks;
    {
        const auto rq = __builtin_amdgcn_make_buffer_rsrc((void *)(a.q + (size_t)kvh * kv_mul * hs), 0,
                                                          kv_mul * hs * 4, 0x00020000);
        const size_t kv_off = (size_t)t0 * a.kv_dim + (size_t)kvh * hs;
        const int span = ((T - 1) * a.kv_dim + hs) * 4;
        const auto rk = __builtin_amdgcn_make_buffer_rsrc((void *)(a.kc + kv_off), 0, span, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc((void *)(a.vc + kv_off), 0, span, 0x00020000);
        const int rs = nt / hs4, r0 = tid / hs4, c = tid - r0 * hs4; // rows per pass, this thread's row, column
        const unsigned OUT = 0x40000000u;                             // past every range: reads nothing
        const auto qv = __builtin_amdgcn_raw_buffer_load_b128(rq, tid < kv_mul * hs4 ? tid * 16 : OUT, 0, 0);
        u32x4 kr[ATT_SHORT_LOADS], vr[ATT_SHORT_LOADS];
#pragma unroll
        for (int k = 0; k < ATT_SHORT_LOADS; k++) {
            const int t = r0 + k * rs;
            const unsigned o = (r0 < rs && t < T) ? (unsigned)(t * a.kv_dim + 4 * c) * 4 : OUT;
            kr[k] = __builtin_amdgcn_raw_buffer_load_b128(rk, o, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < ATT_SHORT_LOADS; k++) {
            const int t = r0 + k * rs;
            const unsigned o = (r0 < rs && t < T) ? (unsigned)(t * a.kv_dim + 4 * c) * 4 : OUT;
            vr[k] = __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, 0);
        }
        if (tid < kv_mul * hs4) *(u32x4 *)(sq + 4 * tid) = qv;
#pragma unroll
        for (int k = 0; k < ATT_SHORT_LOADS; k++) {
            const int t = r0 + k * rs;
            if (r0 < rs && t < T) *(u32x4 *)(sk + t * ks + 4 * c) = kr[k];
        }
#pragma unroll
        for (int k = 0; k < ATT_SHORT_LOADS; k++) {
            const int t = r0 + k * rs;
            if (r0 < rs && t < T) *(u32x4 *)(sv + t * hs + 4 * c) = vr[k];
        }
    }
    __syncthreads();
    KERNEL_MARK(1);
    const int j = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid & (WAVE - 1);
    if (j >= kv_mul) return;
    const int h = kvh * kv_mul + j;
    const f32x4 *k4 = (const f32x4 *)(sk + min(lane, T - 1) * ks), *q4 = (const f32x4 *)(sq + j * hs);
    float d = 0.0f;
#pragma unroll 4
    for (int c4 = 0; c4 < hs4; c4++) {
        const f32x4 kk = k4[c4], qq = q4[c4];
        d += qq.x * kk.x;
        d += qq.y * kk.y;
        d += qq.z * kk.z;
        d += qq.w * kk.w;
    }
    const bool valid = lane < T;
    const float score = d / sqrtf((float)hs);
    const float mx = wave_max(valid ? score : -INFINITY);
    const float w = valid ? expf(score - mx) : 0.0f;
    const float l = wave_sum(w);
    KERNEL_MARK(2);
    const int e = min(lane * EPL, hs - EPL);
    const float *vp = sv + e;
    float acc[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[i] = 0.0f;
    int t = 0;
    for (; t + 8 <= T; t += 8) {
        float v[8][EPL];
#pragma unroll
        for (int u = 0; u < 8; u++)
#pragma unroll
            for (int i = 0; i < EPL; i++) v[u][i] = vp[(t + u) * hs + i];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float p = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), t + u));
#pragma unroll
            for (int i = 0; i < EPL; i++) acc[i] += p * v[u][i];
        }
    }
    for (; t < T; t++) {
        const float p = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), t));
#pragma unroll
        for (int i = 0; i < EPL; i++) acc[i] += p * vp[t * hs + i];
    }
    if (lane * EPL < hs) {
        float *o = a.acc + ((size_t)h * a.splits + s) * hs + lane * EPL;
#pragma unroll
        for (int i = 0; i < EPL; i++) o[i] = acc[i];
    }
    if (lane == 0) {
        float *ml = a.ml + ((size_t)h * a.splits + s) * 2;
        ml[0] = mx;
        ml[1] = l;
    }
    KERNEL_MARK(7);
}

// Reference-order decode attention: block h is query head h over positions 0 .. pos (attn_strict_head); the
// output goes to acc[h][0..hs) with (max, sum) = (0, 1), one slice whose merge is the identity.
template <int HS>
__global__ void __launch_bounds__(256) k_attention_strict(AttnArgs a) {
    extern __shared__ __align__(16) float sm[];
    const int pos = a.ctrl->pos, h = blockIdx.x, kv_mul = a.n_heads / a.n_kv, hs = a.hs;
    attn_strict_head<HS>(a.q + (size_t)h * hs, a.kc, a.vc, a.kv_dim, (h / kv_mul) * hs, hs, pos + 1, sm,
                         a.acc + (size_t)h * hs);
    if (threadIdx.x == 0) {
        a.ml[2 * h] = 0.0f;
        a.ml[2 * h + 1] = 1.0f;
    }
}

hipError_t launch_attention_strict(const AttnArgs &a, hipStream_t st) {
    const size_t lds = attn_strict_lds_floats(a.hs, a.max_pos, 256) * 4;
    // the K and V reads go through buffer resources: a layer's cache must stay below 2 GiB
    if (a.hs % 4 || a.hs > 256 || ((uintptr_t)a.kc & 15) || (a.kv_dim % 4) || a.max_pos < 1 || lds > 65536 ||
        a.n_heads % a.n_kv ||
        (size_t)(a.max_pos + 64) * a.kv_dim * 4 >= 0x7fffffffu)
        return hipErrorInvalidValue;
    if (a.hs == 64) hipLaunchKernelGGL(k_attention_strict<64>, dim3(a.n_heads), dim3(256), lds, st, a);
    else if (a.hs == 128) hipLaunchKernelGGL(k_attention_strict<128>, dim3(a.n_heads), dim3(256), lds, st, a);
    else hipLaunchKernelGGL(k_attention_strict<0>, dim3(a.n_heads), dim3(256), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
    const int kv_mul = a.n_heads / a.n_kv;
    // at most 64 slices: the partial buffers and the o projection's merge (PRO_ATTN) hold that many per head
    if (a.hs % 4 || a.hs > 128 || ((uintptr_t)a.q & 15) || ((uintptr_t)a.kc & 15) || ((uintptr_t)a.vc & 15) ||
        (a.kv_dim % 4) || a.splits < 1 || a.splits > 64 || a.max_pos < 1)
        return hipErrorInvalidValue;
    // longest slice over every position the cache holds: ceil(P / S) with S = min(splits, ceil(P / ATT_SUB))
    const int longest = std::max(ATT_SUB, (a.max_pos + a.splits - 1) / a.splits);
    const int nt = WAVE * std::max(kv_mul, 4);
    if (longest <= ATT_SHORT_MAX && kv_mul <= 8 && (a.hs % 4) == 0 && a.hs <= 2 * WAVE &&
        (ATT_SHORT_MAX + nt / (a.hs / 4) - 1) / (nt / (a.hs / 4)) <= ATT_SHORT_LOADS) {
        const size_t lds = attn_short_lds_floats(kv_mul, a.hs) * 4;
        if (a.hs <= WAVE) hipLaunchKernelGGL(k_attention_short<1>, dim3(a.n_kv * a.splits), dim3(nt), lds, st, a);
        else hipLaunchKernelGGL(k_attention_short<2>, dim3(a.n_kv * a.splits), dim3(nt), lds, st, a);
        return hipGetLastError();
    }
    const int threads = 256;
    if (kv_mul * a.hs > 4 * threads) return hipErrorInvalidValue;
    const size_t lds = attn_lds_floats(kv_mul, a.hs) * 4;
    hipLaunchKernelGGL(k_attention, dim3(a.n_kv * a.splits), dim3(threads), lds, st, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------------
// embedding row (qwen.c:498-501, runq.c:490-492) and the step's position/token bookkeeping

// The head kernel's per-block argmax partials, read by a whole block: the first STEP_PV per thread as one
// round of loads (clamped indices), issued before anything they do not depend on is waited for.
#define STEP_THREADS 1024
#define STEP_PV 4
struct Partials {
    float v[STEP_PV];
    int i[STEP_PV];
};
__device__ __forceinline__ Partials load_partials(const float *pv, const int *pi, int np) {
    Partials p;
#pragma unroll
    for (int k = 0; k < STEP_PV; k++) {
        const int j = min((int)threadIdx.x + k * (int)blockDim.x, np - 1);
        p.v[k] = pv[j];
        p.i[k] = pi[j];
    }
    return p;
}

// argmax over the partials: larger value wins, equal values keep the lower row
__device__ __forceinline__ void block_argmax(const Partials &p, const float *pv, const int *pi, int np, float *sv,
                                             int *si, float *v_out, int *i_out) {
    float v = -INFINITY;
    int i = 0x7fffffff;
    auto take = [&](float x, int xi) {
        if (x > v || (x == v && xi < i)) { v = x; i = xi; }
    };
#pragma unroll
    for (int k = 0; k < STEP_PV; k++)
        if ((int)threadIdx.x + k * (int)blockDim.x < np) take(p.v[k], p.i[k]);
    for (int k = threadIdx.x + STEP_PV * blockDim.x; k < np; k += blockDim.x) take(pv[k], pi[k]);
    for (int off = 1; off < WAVE; off <<= 1) {
        float ov = __shfl_xor(v, off);
        int oi = __shfl_xor(i, off);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    if (lane == 0) { sv[wave] = v; si[wave] = i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x / WAVE); k++)
            if (sv[k] > v || (sv[k] == v && si[k] < i)) { v = sv[k]; i = si[k]; }
        if (i == 0x7fffffff) i = 0; // every logit NaN: the reference keeps row 0
        *v_out = v;
        *i_out = i;
    }
}

// Start of a step.  Generate mode: finish the previous step's argmax (qwen.c:591-598, head_ids map
// qwen.c:683), advance the position and take the prompt token or the argmax (prompt forcing,
// qwen.c:677-683).  Then the embedding row of the token (qwen.c:498-501, runq.c:490-492).  The dependent
// reads form a short chain: control block (with the partials already in flight), head_ids and the prompt
// token together, then the embedding row in one round.
__global__ void __launch_bounds__(STEP_THREADS) k_step_start(EmbedArgs a) {
    __shared__ float sv[STEP_THREADS / WAVE];
    __shared__ int si[STEP_THREADS / WAVE];
    __shared__ int tok_s;
    __shared__ float bv;
    __shared__ int bi, s_mode, s_prev, s_tok, s_np;
    StepCtrl *c = a.ctrl;
    const Partials part = load_partials(a.pv, a.pi, a.np);
    // one read of the control block for the whole block, before thread 0 advances it below
    if (threadIdx.x == 0) {
        s_mode = c->mode;
        s_prev = c->pos;
        s_tok = c->token;
        s_np = c->n_prompt;
    }
    __syncthreads();
    const int mode = s_mode, prev = s_prev;
    if (mode == 1 && prev >= 0) block_argmax(part, a.pv, a.pi, a.np, sv, si, &bv, &bi);
    if (threadIdx.x == 0) {
        int pos = prev, token = s_tok;
        if (mode == 1) {
            pos = prev + 1;
            const int forced = pos < s_np ? a.prompt[pos] : 0;
            if (prev >= 0) {
                const int next = a.head_ids ? a.head_ids[bi] : bi;
                c->next_token = next;
                if (a.gen) a.gen[prev] = next;
                token = pos < s_np ? forced : next;
            } else {
                token = pos < s_np ? forced : c->next_token;
            }
            c->pos = pos;
            c->token = token;
        }
        if (a.tokens) a.tokens[pos] = token;
        tok_s = token;
    }
    __syncthreads();
    const int token = tok_s, ngr = a.dim / a.gs, nt = blockDim.x;
    const int8_t *__restrict__ er = a.emb_q + (size_t)token * a.dim;
    float *__restrict__ x = a.x;
    auto scale = [&](int g) {
        return a.sf32 ? ((const float *)a.emb_s)[(size_t)token * ngr + g]
                      : f16_bits_to_f32(((const uint16_t *)a.emb_s)[(size_t)token * ngr + g]);
    };
    int8_t q[STEP_PV];
    float sc[STEP_PV];
#pragma unroll
    for (int k = 0; k < STEP_PV; k++) {
        const int e = min((int)threadIdx.x + k * nt, a.dim - 1);
        q[k] = er[e];
        sc[k] = scale(e / a.gs);
    }
#pragma unroll
    for (int k = 0; k < STEP_PV; k++) {
        const int e = threadIdx.x + k * nt;
        if (e < a.dim) x[e] = (float)q[k] * sc[k];
    }
    for (int e = threadIdx.x + STEP_PV * nt; e < a.dim; e += nt) x[e] = (float)er[e] * scale(e / a.gs);
}

hipError_t launch_embed(const EmbedArgs &a, hipStream_t st) {
    if (a.np < 1 || a.dim < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_step_start, dim3(1), dim3(STEP_THREADS), 0, st, a);
    return hipGetLastError();
}

// final argmax of a step over the head kernel's partials (qwen.c:591-598) and the head_ids map (qwen.c:683)
__global__ void __launch_bounds__(STEP_THREADS) k_argmax(ArgmaxArgs a) {
    __shared__ float sv[STEP_THREADS / WAVE];
    __shared__ int si[STEP_THREADS / WAVE];
    __shared__ float bv;
    __shared__ int bi;
    const Partials part = load_partials(a.pv, a.pi, a.np);
    block_argmax(part, a.pv, a.pi, a.np, sv, si, &bv, &bi);
    if (threadIdx.x == 0) {
        const int next = a.head_ids ? a.head_ids[bi] : bi;
        a.ctrl->next_token = next;
        if (a.gen) a.gen[a.ctrl->pos] = next;
    }
}

hipError_t launch_argmax(const ArgmaxArgs &a, hipStream_t st) {
    if (a.np < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(STEP_THREADS), 0, st, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------------
// repack: reference row-major planes -> chunk records (layout in tiled.h).  One thread per (record, lane).

__global__ void k_repack(RepackArgs a) {
    const TiledMat &T = a.T;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nrec = (size_t)T.nblocks * T.nchunks;
    if (gid >= nrec * WAVE) return;
    const int lane = (int)(gid % WAVE);
    const size_t recno = gid / WAVE;
    const int b = (int)(recno / T.nchunks), c = (int)(recno - (size_t)b * T.nchunks);
    const int rb = T.rb, row = b * rb + lane % rb, g = c * (WAVE / rb) + lane / rb;
    const int sb = T.gs * T.wbits / 8, scb = T.sf32 ? 4 : 2;
    uint8_t *rec = (uint8_t *)T.data + recno * T.rec;
    uint8_t seg[64];
    uint32_t sc = 0;
    for (int i = 0; i < sb; i++) seg[i] = 0;
    if (row < T.rows && g < T.ng) {
        const int m = a.rowmap[row];
        const int src = m >> 28, sr = m & 0x0fffffff;
        const size_t rowbytes = (size_t)T.n * T.wbits / 8;
        const uint8_t *w = a.w[src] + (size_t)sr * rowbytes + (size_t)g * sb;
        if (T.wbits == 4) {
            // element e of the group sits in byte e/2, low nibble for even e (qwen.c:45, 447)
            for (int j = 0; j < 4; j++)
                for (int k = 0; k < 4; k++) {
                    const int e0 = 4 * j + k, e1 = 16 + 4 * j + k;
                    const int n0 = (w[e0 >> 1] >> ((e0 & 1) * 4)) & 15, n1 = (w[e1 >> 1] >> ((e1 & 1) * 4)) & 15;
                    seg[4 * j + k] = (uint8_t)(n0 | (n1 << 4));
                }
        } else {
            for (int i = 0; i < sb; i++) seg[i] = w[i];
        }
        const uint8_t *s = a.s[src] + ((size_t)sr * T.ng + g) * scb;
        sc = scb == 4 ? (uint32_t)s[0] | ((uint32_t)s[1] << 8) | ((uint32_t)s[2] << 16) | ((uint32_t)s[3] << 24)
                      : (uint32_t)s[0] | ((uint32_t)s[1] << 8);
    }
    for (int p = 0; p < sb / 16; p++) {
        uint4 v;
        v.x = seg[16 * p + 0] | (seg[16 * p + 1] << 8) | (seg[16 * p + 2] << 16) | ((uint32_t)seg[16 * p + 3] << 24);
        v.y = seg[16 * p + 4] | (seg[16 * p + 5] << 8) | (seg[16 * p + 6] << 16) | ((uint32_t)seg[16 * p + 7] << 24);
        v.z = seg[16 * p + 8] | (seg[16 * p + 9] << 8) | (seg[16 * p + 10] << 16) | ((uint32_t)seg[16 * p + 11] << 24);
        v.w = seg[16 * p + 12] | (seg[16 * p + 13] << 8) | (seg[16 * p + 14] << 16) | ((uint32_t)seg[16 * p + 15] << 24);
        *(uint4 *)(rec + (size_t)p * 1024 + lane * 16) = v;
    }
    if (scb == 4) *(uint32_t *)(rec + (size_t)WAVE * sb + lane * 4) = sc;
    else *(uint16_t *)(rec + (size_t)WAVE * sb + lane * 2) = (uint16_t)sc;
}

hipError_t launch_repack(const RepackArgs &a, hipStream_t st) {
    const size_t threads = (size_t)a.T.nblocks * a.T.nchunks * WAVE;
    hipLaunchKernelGGL(k_repack, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------------
// test hooks

__global__ void __launch_bounds__(256) k_quantize_test(const float *x, int n, int flavor, int gs, int8_t *q, float *s) {
    extern __shared__ float xv[];
    for (int i = threadIdx.x; i < n; i += blockDim.x) xv[i] = x[i];
    __syncthreads();
    block_quantize(xv, n, gs, flavor, q, s);
}

hipError_t launch_quantize_test(const float *x, int n, int flavor, int gs, int8_t *q, float *s, hipStream_t st) {
    hipLaunchKernelGGL(k_quantize_test, dim3(1), dim3(256), (size_t)n * 4, st, x, n, flavor, gs, q, s);
    return hipGetLastError();
}

// per-(row, group) int32 sums through the GEMV's own seg_dot on tiled records
template <int WB, int GSZ>
__global__ void k_group_dots(TiledMat T, const int8_t *xq, int32_t *ival) {
    using F = Fmt<WB, GSZ, 0>;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nrec = (size_t)T.nblocks * T.nchunks;
    if (gid >= nrec * WAVE) return;
    const int lane = (int)(gid % WAVE);
    const size_t recno = gid / WAVE;
    const int b = (int)(recno / T.nchunks), c = (int)(recno - (size_t)b * T.nchunks);
    const int row = b * T.rb + lane % T.rb, g = c * (WAVE / T.rb) + lane / T.rb;
    if (row >= T.rows || g >= T.ng) return;
    const uint8_t *rec = T.data + recno * T.rec;
    uint4 wv[F::PIECES];
    for (int p = 0; p < F::PIECES; p++) wv[p] = *(const uint4 *)(rec + p * 1024 + lane * 16);
    uint32_t xw[GSZ / 4];
    for (int k = 0; k < GSZ / 4; k++) xw[k] = ((const uint32_t *)(xq + (size_t)g * GSZ))[k];
    ival[(size_t)row * T.ng + g] = seg_dot<WB, GSZ>(wv, xw);
}

hipError_t launch_group_dots_test(const TiledMat &T, const int8_t *xq, int32_t *ival, hipStream_t st) {
    const size_t threads = (size_t)T.nblocks * T.nchunks * WAVE;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (T.wbits == 4 && T.gs == 32) hipLaunchKernelGGL((k_group_dots<4, 32>), grid, dim3(256), 0, st, T, xq, ival);
    else if (T.wbits == 8 && T.gs == 32) hipLaunchKernelGGL((k_group_dots<8, 32>), grid, dim3(256), 0, st, T, xq, ival);
    else if (T.wbits == 8 && T.gs == 64) hipLaunchKernelGGL((k_group_dots<8, 64>), grid, dim3(256), 0, st, T, xq, ival);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
