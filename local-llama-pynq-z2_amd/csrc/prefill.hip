// Prefill kernels of libmatvec_hip.so for gfx950: the prompt's positions through a layer together.
//
// The reference processes a prompt one position at a time with the same forward() (qwen.c:674-681); no
// batched prefill exists there (README.md:386-387).  Here the M positions of a chunk share each weight
// read: the layer matrices become int8 MFMA GEMMs (v_mfma_i32_32x32x32_i8) over the tiled records the decode
// GEMV reads, with the per-group int32 sums exact and the group terms p = ((float)ival * ws) * xs added in
// group order, which is the reference's matmul (qwen.c:436-456, runq.c:429-458) for every (row, token).
// The element-wise steps of forward() run per token, and attention is causal over the KV cache.
#include "attn.h"
#include "prefill.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// groups of the prefill GEMM's K loop whose loads are in flight at once
#define PF_STAGES 4

// ------------------------------------------------------------------------------------------------------
// GEMM: y[m][r] = sum_g ((float)ival(r, m, g) * ws[r][g]) * xs[m][g], groups in order.
//
// One wave per PF_RT x 32 rows x 32 tokens (PF_RT MFMAs per group share the token operand).  Lane layout
// of one MFMA: A (rows x K): lane l holds row l%32, K = 16 (l/32) .. +16; B (K x tokens): token l%32, same K
// half; D: token l%32, rows 8i + 4 (l/32) + j in d[4i + j].  int4 weights enter as 16 * q (the nibble at the
// top of its byte, as in the GEMV), so D holds 16 * ival; their fp16 scales are taken as ws / 16, an exact
// power-of-two step, and (16 ival) * (ws / 16) rounds to the same float as ival * ws.
//
// Blocks are laid out so that all token tiles of one row tile run on the same XCD (block b goes to XCD b % 8):
// each weight tile is read from HBM once and served from that XCD's L2 to its other token tiles.
#define PF_RT 1 // 32-row tiles per wave (2 measured slower: the extra registers halve the waves per SIMD)

template <int WB, int GSZ, int SF32>
__global__ void __launch_bounds__(64) k_pgemm(PgemmArgs a) {
    constexpr int SB = GSZ * WB / 8, SCB = SF32 ? 4 : 2, KC = GSZ / 32, RT = PF_RT;
    const TiledMat &W = a.W;
    const int xt = (W.rows + 32 * RT - 1) / (32 * RT), yt = (a.M + 31) / 32;
    // block -> (row tile, token tile): XCD j = b % 8 takes row tiles j, j + 8, ...
    const int b = blockIdx.x, xcd = b & 7, idx = b >> 3;
    const int tx = xcd + 8 * (idx / yt), ty = idx - (idx / yt) * yt;
    if (tx >= xt) return;
    const int l = threadIdx.x, h = l >> 5, rl = l & 31;
    const int r0 = tx * 32 * RT, m0 = ty * 32;
    const int rb = W.rb, gpc = WAVE / rb, n = W.n, ng = W.ng;
    const int tok = min(m0 + rl, a.M - 1);
    int bA[RT], laneA[RT]; // the lane's A row of each row tile: record block and lane (+ gi * rb per group)
#pragma unroll
    for (int t = 0; t < RT; t++) {
        const int rowA = min(r0 + 32 * t + rl, W.rows - 1);
        bA[t] = rowA / rb;
        laneA[t] = rowA - bA[t] * rb;
    }
    // Each lane loads and converts the scale of its A rows and shares them through LDS; a lane's outputs
    // need rows r0 + 32t + 8i + 4h .. +3 (t < RT, i = 0..3).
    __shared__ __align__(16) float s_sc[32 * RT];
    const int8_t *xrow = a.xq + (size_t)tok * n + 16 * h;
    const float *xsrow = a.xs + (size_t)tok * ng;

    // A ring of PF_STAGES groups in flight.  A stage holds raw loaded words only: the int4 unpacking and the
    // scale conversion happen when the group is used, so issuing a stage never waits for its loads.
    constexpr int NS = PF_STAGES;
    uint4 wr[NS][RT][KC];                             // int4: the lane's 16-byte segment; int8: the K-half piece
    v4i bv[NS][KC];
    uint32_t sr[NS][RT];                              // raw scales of the lane's A rows
    float xs[NS];
    auto load = [&](int g, int st) {
        const int c = g / gpc, gi = g - c * gpc;
#pragma unroll
        for (int t = 0; t < RT; t++) {
            const uint8_t *recA = W.data + ((size_t)bA[t] * W.nchunks + c) * W.rec;
#pragma unroll
            for (int kc = 0; kc < KC; kc++) {
                if constexpr (WB == 4) wr[st][t][kc] = *(const uint4 *)(recA + (size_t)(gi * rb + laneA[t]) * 16);
                else wr[st][t][kc] = *(const uint4 *)(recA + (size_t)(2 * kc + h) * 1024 + (size_t)(gi * rb + laneA[t]) * 16);
            }
            const uint8_t *sp = recA + 64 * SB + (size_t)(gi * rb + laneA[t]) * SCB;
            if constexpr (SF32) sr[st][t] = *(const uint32_t *)sp;
            else sr[st][t] = *(const uint16_t *)sp;
        }
#pragma unroll
        for (int kc = 0; kc < KC; kc++) bv[st][kc] = *(const v4i *)(xrow + (size_t)g * GSZ + 32 * kc);
        xs[st] = xsrow[g];
    };
    float acc[RT][16];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int k = 0; k < 16; k++) acc[t][k] = 0.0f;
    auto compute = [&](int st) {
        v16i d[RT];
#pragma unroll
        for (int t = 0; t < RT; t++) {
            d[t] = v16i{};
#pragma unroll
            for (int kc = 0; kc < KC; kc++) {
                v4i av;
                if constexpr (WB == 4) {
                    const uint4 w = wr[st][t][kc];
                    const uint32_t m = 0xF0F0F0F0u;
                    if (h == 0) av = v4i{(int)((w.x << 4) & m), (int)((w.y << 4) & m), (int)((w.z << 4) & m), (int)((w.w << 4) & m)};
                    else av = v4i{(int)(w.x & m), (int)(w.y & m), (int)(w.z & m), (int)(w.w & m)};
                } else {
                    av = v4i{(int)wr[st][t][kc].x, (int)wr[st][t][kc].y, (int)wr[st][t][kc].z, (int)wr[st][t][kc].w};
                }
                d[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[st][kc], d[t], 0, 0, 0);
            }
        }
        // the group's row scales: one conversion per lane and row tile, shared through LDS (the block is this
        // one wave, so the barriers cost next to nothing)
        if (h == 0)
#pragma unroll
            for (int t = 0; t < RT; t++)
                s_sc[32 * t + rl] = SF32 ? __uint_as_float(sr[st][t])
                                         : f16_bits_to_f32((uint16_t)sr[st][t]) * (WB == 4 ? 0.0625f : 1.0f);
        __syncthreads();
        float4 ws4[RT][4];
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) ws4[t][i] = *(const float4 *)(s_sc + 32 * t + 8 * i + 4 * h);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float ws = j == 0 ? ws4[t][i].x : j == 1 ? ws4[t][i].y : j == 2 ? ws4[t][i].z : ws4[t][i].w;
                    float p = (float)d[t][4 * i + j] * ws; // qwen.c:452, runq.c:452
                    p = p * xs[st];
                    acc[t][4 * i + j] = acc[t][4 * i + j] + p;
                }
    };
#pragma unroll
    for (int st = 0; st < NS - 1; st++)
        if (st < ng) load(st, st);
    for (int g0 = 0; g0 < ng; g0 += NS) {
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const int g = g0 + st;
            if (g >= ng) break;
            if (g + NS - 1 < ng) load(g + NS - 1, (st + NS - 1) % NS);
            compute(st);
        }
    }
    const int m = m0 + rl;
    if (m < a.M) {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int R = r0 + 32 * t + 8 * i + 4 * h;
                float *dst = a.y + (size_t)m * W.rows + R;
                if (R + 3 < W.rows) *(float4 *)dst = make_float4(acc[t][4 * i], acc[t][4 * i + 1], acc[t][4 * i + 2], acc[t][4 * i + 3]);
                else
                    for (int j = 0; j < 4; j++)
                        if (R + j < W.rows) dst[j] = acc[t][4 * i + j];
            }
    }
}

hipError_t launch_pgemm(int wbits, int gs, int sf32, const PgemmArgs &a, hipStream_t st) {
    const TiledMat &W = a.W;
    // rows in whole groups of 4 (scale loads), 16-byte aligned activation rows and output rows
    if (a.M < 1 || W.rows % 4 || W.n % gs || W.n % 16 || ((uintptr_t)a.xq & 15) || ((uintptr_t)a.y & 15) ||
        W.gs != gs || W.wbits != wbits || W.sf32 != sf32)
        return hipErrorInvalidValue;
    const int xt = (W.rows + 32 * PF_RT - 1) / (32 * PF_RT), yt = (a.M + 31) / 32;
    const unsigned blocks = (unsigned)(8 * ((xt + 7) / 8) * yt);
#define PG(WB_, GS_, SF_)                                                                                      \
    if (wbits == WB_ && gs == GS_ && sf32 == SF_) {                                                           \
        hipLaunchKernelGGL((k_pgemm<WB_, GS_, SF_>), dim3(blocks), dim3(64), 0, st, a);                       \
        return hipGetLastError();                                                                             \
    }
    PG(4, 32, 0)
    PG(8, 32, 0)
    PG(8, 32, 1)
    PG(8, 64, 1)
#undef PG
    return hipErrorInvalidValue;
}

// ------------------------------------------------------------------------------------------------------
// per-token element-wise steps (one block of 256 threads per token)

// embedding rows (qwen.c:498-501, runq.c:490-492)
__global__ void __launch_bounds__(256) k_p_embed(ProwArgs a) {
    const int m = blockIdx.x, token = a.ids[m], ngr = a.dim / a.gs;
    const int8_t *er = a.emb_q + (size_t)token * a.dim;
    for (int i = threadIdx.x; i < a.dim; i += blockDim.x) {
        const int g = i / a.gs;
        const float sc = a.emb_sf32 ? ((const float *)a.emb_s)[(size_t)token * ngr + g]
                                    : f16_bits_to_f32(((const uint16_t *)a.emb_s)[(size_t)token * ngr + g]);
        a.x[(size_t)m * a.dim + i] = (float)er[i] * sc;
    }
}

// rmsnorm (qwen.c:337-344, runq.c:394-407) of x[m], then int8 quantization (qwen.c:354-364 / runq.c:244-270)
__global__ void __launch_bounds__(256) k_p_norm_quant(ProwArgs a) {
    extern __shared__ __align__(16) float sv[]; // dim floats + 4 per wave
    const int m = blockIdx.x, n = a.dim;
    const float *x = a.x + (size_t)m * n;
    float part = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i];
        sv[i] = v;
        part += v * v;
    }
    float ss = block_sum(part, sv + n);
    ss /= (float)n;
    ss += a.eps;
    ss = 1.0f / sqrtf(ss);
    for (int i = threadIdx.x; i < n; i += blockDim.x) sv[i] = a.norm_w[i] * (ss * sv[i]);
    __syncthreads();
    block_quantize(sv, n, a.gs, a.qflavor, a.oq + (size_t)m * n, a.os + (size_t)m * (n / a.gs));
}

// int8 quantization of z[m] (the attention output, qwen.c:549 / runq.c:571)
__global__ void __launch_bounds__(256) k_p_quant(ProwArgs a) {
    extern __shared__ __align__(16) float sv[];
    const int m = blockIdx.x, n = a.width;
    for (int i = threadIdx.x; i < n; i += blockDim.x) sv[i] = a.z[(size_t)m * n + i];
    __syncthreads();
    block_quantize(sv, n, a.gs, a.qflavor, a.oq + (size_t)m * n, a.os + (size_t)m * (n / a.gs));
}

// QKV rows of token m: bias (qwen.c:521-522), RoPE at position p0 + m (qwen.c:478-488 NeoX pairs; runq.c:506-521
// interleaved pairs), q to q[m], k and v into the caches.  Logical rows follow the fused matrix's order.
__global__ void __launch_bounds__(256) k_p_qkv(ProwArgs a) {
    const int m = blockIdx.x, pos = a.p0 + m, dim = a.dim, kvd = a.kv_dim, hs = a.head_size, half = hs / 2;
    const int rows = dim + 2 * kvd;
    const float *y = a.y + (size_t)m * rows;
    for (int R = threadIdx.x; R < rows; R += blockDim.x) {
        const float v = y[R];
        if (a.rope_kind == ROPE_NEOX) {
            if (R < dim + kvd) {
                const int blk = R / 16, r = R & 15, per = half / 8, hh = blk / per, i = (blk - hh * per) * 8 + (r & 7);
                const bool first = r < 8;
                const int e = hh * hs + (first ? i : half + i), ep = hh * hs + (first ? half + i : i);
                const float c = a.rope_cos[(size_t)pos * half + i], sn = a.rope_sin[(size_t)pos * half + i];
                const float self = v + a.bias[e], partner = y[R ^ 8] + a.bias[ep];
                float o;
                if (first) { float t1 = self * c, t2 = partner * sn; o = t1 - t2; }
                else { float t1 = self * c, t2 = partner * sn; o = t1 + t2; }
                if (e < dim) a.q[(size_t)m * dim + e] = o;
                else a.kc[(size_t)pos * kvd + (e - dim)] = o;
            } else {
                a.vc[(size_t)pos * kvd + (R - dim - kvd)] = v + a.bias[R];
            }
        } else {
            if (R < dim + kvd) {
                const int e = R < dim ? R : R - dim, i = (e % hs) / 2;
                const float c = a.rope_cos[(size_t)pos * half + i], sn = a.rope_sin[(size_t)pos * half + i];
                const float partner = y[R ^ 1];
                float o;
                if ((e & 1) == 0) { float t1 = v * c, t2 = partner * sn; o = t1 - t2; }
                else { float t1 = partner * sn, t2 = v * c; o = t1 + t2; }
                if (R < dim) a.q[(size_t)m * dim + e] = o;
                else a.kc[(size_t)pos * kvd + e] = o;
            } else {
                a.vc[(size_t)pos * kvd + (R - dim - kvd)] = v;
            }
        }
    }
}

// x += y (qwen.c:551, 565; runq.c:575-577, 603-605)
__global__ void __launch_bounds__(256) k_p_resid(ProwArgs a) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, total = (size_t)a.M * a.dim;
    if (i < total) a.x[i] = a.x[i] + a.y[i];
}

// SwiGLU of token m (qwen.c:556-562, runq.c:589-596), then int8 quantization of h.  The gate/up matrix's rows
// come in row-blocks of gu_rb: gu_rb/2 gate rows, then the matching up rows.
__global__ void __launch_bounds__(256) k_p_swiglu_quant(ProwArgs a) {
    extern __shared__ __align__(16) float sv[];
    const int m = blockIdx.x, hid = a.hidden, hb = a.gu_rb / 2;
    const float *y = a.y + (size_t)m * 2 * hid;
    for (int j = threadIdx.x; j < hid; j += blockDim.x) {
        const int b = j / hb, r = j - b * hb;
        float g = y[b * a.gu_rb + r];
        const float u = y[b * a.gu_rb + hb + r];
        const float sig = 1.0f / (1.0f + expf(-g));
        g = g * sig;
        sv[j] = g * u;
    }
    __syncthreads();
    block_quantize(sv, hid, a.gs, a.qflavor, a.oq + (size_t)m * hid, a.os + (size_t)m * (hid / a.gs));
}

// causal attention of token m over positions 0 .. p0 + m, cut into slices of att_sl positions: block =
// (kv head, token, slice) leaves the slice's running max, sum of exponentials and exp-weighted value sums
__global__ void __launch_bounds__(256) k_p_attention(ProwArgs a) {
    extern __shared__ __align__(16) float sm[];
    const int kvh = blockIdx.x, m = blockIdx.y, s = blockIdx.z, hs = a.head_size, kv_mul = a.n_heads / a.n_kv;
    const int t_begin = s * a.att_sl, t_end = min(t_begin + a.att_sl, a.p0 + m + 1);
    if (t_begin >= t_end) return;
    float acc[4];
    const float *ml_max, *ml_sum;
    attn_range(a.q + (size_t)m * a.dim + (size_t)kvh * kv_mul * hs, a.kc, a.vc, a.kv_dim, kvh, hs, kv_mul, t_begin,
               t_end, sm, acc, &ml_max, &ml_sum);
    const int n_out = kv_mul * hs;
    for (int k = 0; k < 4; k++) {
        const int o = threadIdx.x + k * blockDim.x;
        if (o < n_out) {
            const int j = o / hs, e = o - j * hs, h = kvh * kv_mul + j;
            a.att_acc[(((size_t)m * a.n_heads + h) * a.att_smax + s) * hs + e] = acc[k];
        }
    }
    if (threadIdx.x < kv_mul) {
        const int h = kvh * kv_mul + threadIdx.x;
        float *ml = a.att_ml + (((size_t)m * a.n_heads + h) * a.att_smax + s) * 2;
        ml[0] = ml_max[threadIdx.x];
        ml[1] = ml_sum[threadIdx.x];
    }
}

// merge of token m's slices: out[m][h*hs + e] = sum_s acc_s[e] * exp(max_s - max) / sum_s l_s * exp(max_s - max)
__global__ void __launch_bounds__(256) k_p_attn_merge(ProwArgs a, float *out) {
    const int m = blockIdx.x, hs = a.head_size, S = (a.p0 + m + a.att_sl) / a.att_sl;
    for (int o = threadIdx.x; o < a.dim; o += blockDim.x) {
        const int h = o / hs, e = o - h * hs;
        const float *ml = a.att_ml + ((size_t)m * a.n_heads + h) * a.att_smax * 2;
        const float *acc = a.att_acc + ((size_t)m * a.n_heads + h) * a.att_smax * hs + e;
        float mx = ml[0];
        for (int k = 1; k < S; k++) mx = fmaxf(mx, ml[2 * k]);
        float l = 0.0f, v = 0.0f;
        for (int k = 0; k < S; k++) {
            const float f = expf(ml[2 * k] - mx);
            l += ml[2 * k + 1] * f;
            v += acc[(size_t)k * hs] * f;
        }
        out[(size_t)m * a.dim + o] = v / l;
    }
}

hipError_t launch_p_embed(const ProwArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(k_p_embed, dim3(a.M), dim3(256), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_p_norm_quant(const ProwArgs &a, hipStream_t st) {
    if (a.dim % 4 || ((uintptr_t)a.oq & 3)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_p_norm_quant, dim3(a.M), dim3(256), (size_t)(a.dim + 8) * 4, st, a);
    return hipGetLastError();
}
hipError_t launch_p_quant(const ProwArgs &a, hipStream_t st) {
    if (a.width % 4 || ((uintptr_t)a.oq & 3)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_p_quant, dim3(a.M), dim3(256), (size_t)a.width * 4, st, a);
    return hipGetLastError();
}
hipError_t launch_p_qkv(const ProwArgs &a, hipStream_t st) {
    if (a.rope_kind == ROPE_NEOX && !a.bias) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_p_qkv, dim3(a.M), dim3(256), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_p_resid(const ProwArgs &a, hipStream_t st) {
    const size_t total = (size_t)a.M * a.dim;
    hipLaunchKernelGGL(k_p_resid, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_p_swiglu_quant(const ProwArgs &a, hipStream_t st) {
    if (a.hidden % 4 || ((uintptr_t)a.oq & 3)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_p_swiglu_quant, dim3(a.M), dim3(256), (size_t)a.hidden * 4, st, a);
    return hipGetLastError();
}
hipError_t launch_p_attention(const ProwArgs &a, float *out, hipStream_t st) {
    const int kv_mul = a.n_heads / a.n_kv;
    if (kv_mul * a.head_size > 1024 || a.head_size % 4 || a.head_size > 128 || ((uintptr_t)a.q & 15) ||
        ((uintptr_t)a.kc & 15) || ((uintptr_t)a.vc & 15) || a.kv_dim % 4 || a.dim % 4 || a.att_sl < ATT_SUB ||
        a.att_smax < 1 || a.att_smax > PREFILL_ATT_SMAX || (a.p0 + a.M + a.att_sl - 1) / a.att_sl > a.att_smax)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_p_attention, dim3(a.n_kv, a.M, a.att_smax), dim3(256),
                       attn_lds_floats(kv_mul, a.head_size) * 4, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_p_attn_merge, dim3(a.M), dim3(256), 0, st, a, out);
    return hipGetLastError();
}
