// Prefill kernels of libmatvec_hip.so for gfx950: the prompt's positions through a layer together.
//
// The reference processes a prompt one position at a time with the same forward() (qwen.c:674-681); no
// batched prefill exists there (README.md:386-387).  Here the M positions of a chunk share each weight
// read: the layer matrices become int8 MFMA GEMMs (v_mfma_i32_32x32x32_i8) over the tiled records the decode
// GEMV reads, with the per-group int32 sums exact and the group terms p = ((float)ival * ws) * xs added in
// group order, which is the reference's matmul (qwen.c:436-456, runq.c:429-458) for every (row, token).
// The element-wise steps of forward() run per token, and attention is causal over the KV cache.
#include <type_traits>

#include "attn.h"
#include "prefill.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// K groups of each wave of the prefill GEMM whose loads are in flight at once (one per chunk).  Residency
// matters more than depth here: 2 stages and 1 product buffer (below) measured 14% faster on the 512-token
// gate/up GEMM than 4 stages and 2 buffers, which hold twice the registers and LDS per block.
#ifndef PF_STAGES
#define PF_STAGES 2
#endif
// product buffers of the prefill GEMM: 2 lets a chunk's sum overlap the next chunk's products (one barrier
// per chunk); 1 halves the LDS of a block (a second barrier per chunk) so more blocks stay resident
#ifndef PF_PBUF
#define PF_PBUF 1
#endif

// ------------------------------------------------------------------------------------------------------
// GEMM: y[m][r] = sum_g ((float)ival(r, m, g) * ws[r][g]) * xs[m][g], groups in order.
//
// One block of PF_KW = 4 waves per 32 rows x 32 tokens.  The K groups are dealt round-robin over the waves:
// in chunk c wave w takes group 4c + w, runs its MFMA and forms the group's 16 products per lane; the
// products go through LDS and each thread adds, for its 4 outputs, the chunk's 4 products in group order.
// The sum is therefore the sequential one, while the MFMA, unpacking and product work is spread over the
// four SIMDs of a CU (a single wave per tile leaves the down projection's 152 groups on one SIMD).
//
// Lane layout of one MFMA: A (rows x K): lane l holds row l%32, K = 16 (l/32) .. +16; B (K x tokens): token
// l%32, same K half; D: token l%32, rows 8i + 4 (l/32) + j in d[4i + j].  int4 weights enter as 16 * q (the
// nibble at the top of its byte, as in the GEMV), so D holds 16 * ival; their fp16 scales are taken as
// ws / 16, an exact power-of-two step, and (16 ival) * (ws / 16) rounds to the same float as ival * ws.
// Thread (w, l) owns the outputs of slot i = w: token l%32, rows 8w + 4 (l/32) .. +3.
//
// Blocks are laid out so that all token tiles of one row tile run on the same XCD (block b goes to XCD b % 8):
// each weight tile is read from HBM once and served from that XCD's L2 to its other token tiles.
#define PF_KW 4

template <int WB, int GSZ, int SF32>
__global__ void __launch_bounds__(64 * PF_KW) k_pgemm(PgemmArgs a) {
    constexpr int SB = GSZ * WB / 8, SCB = SF32 ? 4 : 2, KC = GSZ / 32, KW = PF_KW;
    const TiledMat &W = a.W;
    const int xt = (W.rows + 31) / 32, yt = (a.M + 31) / 32;
    // block -> (row tile, token tile): XCD j = b % 8 takes row tiles j, j + 8, ...
    const int b = blockIdx.x, xcd = b & 7, idx = b >> 3;
    const int tx = xcd + 8 * (idx / yt), ty = idx - (idx / yt) * yt;
    if (tx >= xt) return; // the whole block
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, h = l >> 5, rl = l & 31;
    const int r0 = tx * 32, m0 = ty * 32;
    const int rb = W.rb, gpc = WAVE / rb, n = W.n, ng = W.ng;
    const int tok = min(m0 + rl, a.M - 1);
    const int rowA = min(r0 + rl, W.rows - 1), bA = rowA / rb, laneA = rowA - bA * rb;
    // per wave: the converted scales of the tile's 32 rows for its current group (lanes rl convert row rl,
    // every lane reads rows 8i + 4h .. +3); per chunk (two buffers): every wave's products, [wave][i][lane]
    __shared__ __align__(16) float s_sc[KW][32];
    __shared__ __align__(16) float4 s_p[PF_PBUF][KW][4][WAVE];
    const int8_t *xrow = a.xq + (size_t)tok * n + 16 * h;
    const float *xsrow = a.xs + (size_t)tok * ng;
    const int nib_shift = h ? 0 : 4; // int4: lanes of the low K half take the low nibbles, moved to the top

    // A ring of PF_STAGES of this wave's groups in flight.  A stage holds raw loaded words only: the int4
    // unpacking and the scale conversion happen when the group is used, so issuing a stage never waits.
    constexpr int NS = PF_STAGES;
    uint4 wr[NS][KC]; // int4: the lane's 16-byte segment; int8: the K-half piece
    v4i bv[NS][KC];
    using ScaleBits = typename std::conditional<SF32 != 0, uint32_t, uint16_t>::type;
    ScaleBits sr[NS]; // raw scale of the lane's A row
    float xs[NS];
    auto load = [&](int g, int st) {
        const int c = g / gpc, gi = g - c * gpc;
        const uint8_t *recA = W.data + ((size_t)bA * W.nchunks + c) * W.rec;
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            if constexpr (WB == 4) wr[st][kc] = *(const uint4 *)(recA + (size_t)(gi * rb + laneA) * 16);
            else wr[st][kc] = *(const uint4 *)(recA + (size_t)(2 * kc + h) * 1024 + (size_t)(gi * rb + laneA) * 16);
        }
        const uint8_t *sp = recA + 64 * SB + (size_t)(gi * rb + laneA) * SCB;
        sr[st] = *(const ScaleBits *)sp;
#pragma unroll
        for (int kc = 0; kc < KC; kc++) bv[st][kc] = *(const v4i *)(xrow + (size_t)g * GSZ + 32 * kc);
        xs[st] = xsrow[g];
    };
    // the products of stage st into s_p[buf][w]
    auto products = [&](int st, int buf) {
        v16i d = v16i{};
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            v4i av;
            if constexpr (WB == 4) {
                const uint4 q = wr[st][kc];
                const uint32_t m = 0xF0F0F0F0u;
                av = v4i{(int)((q.x << nib_shift) & m), (int)((q.y << nib_shift) & m), (int)((q.z << nib_shift) & m),
                         (int)((q.w << nib_shift) & m)};
            } else {
                av = v4i{(int)wr[st][kc].x, (int)wr[st][kc].y, (int)wr[st][kc].z, (int)wr[st][kc].w};
            }
            d = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[st][kc], d, 0, 0, 0);
        }
        // one scale conversion per lane, exchanged within the wave through its own LDS slots
        if (h == 0)
            s_sc[w][rl] = SF32 ? __uint_as_float(sr[st]) : f16_bits_to_f32(sr[st]) * (WB == 4 ? 0.0625f : 1.0f);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 ws4 = *(const float4 *)(&s_sc[w][8 * i + 4 * h]);
            float4 p;
            p.x = (float)d[4 * i] * ws4.x; // qwen.c:452, runq.c:452
            p.y = (float)d[4 * i + 1] * ws4.y;
            p.z = (float)d[4 * i + 2] * ws4.z;
            p.w = (float)d[4 * i + 3] * ws4.w;
            p.x = p.x * xs[st];
            p.y = p.y * xs[st];
            p.z = p.z * xs[st];
            p.w = p.w * xs[st];
            s_p[buf][w][i][l] = p;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier(); // this wave's scale reads come before its next group's scale writes
    };
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int nc = (ng + KW - 1) / KW; // chunks; wave w's group in chunk c is KW c + w when below ng
    // Every stage is loaded and used, past the last group too (clamped to it; its products are not added):
    // with no branch around the loads the compiler's count of loads in flight stays exact, so waiting for
    // one stage does not wait for the stages issued after it.
#pragma unroll
    for (int st = 0; st < NS - 1; st++) load(min(KW * st + w, ng - 1), st);
    for (int c0 = 0; c0 < nc; c0 += NS) {
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const int c = c0 + st;
            if (c >= nc) break;
            load(min(KW * (c + NS - 1) + w, ng - 1), (st + NS - 1) % NS);
            const int buf = PF_PBUF == 2 ? (c & 1) : 0;
            products(st, buf); // past the last group: a clamped copy that the sum below skips
            __syncthreads();
            const int cnt = ng - KW * c;
#pragma unroll
            for (int v = 0; v < KW; v++) { // the chunk's groups in order
                if (v < cnt) {
                    const float4 p = s_p[buf][v][w][l];
                    acc.x = acc.x + p.x;
                    acc.y = acc.y + p.y;
                    acc.z = acc.z + p.z;
                    acc.w = acc.w + p.w;
                }
            }
            // with two buffers no second barrier: the next chunk writes the other buffer, and the one after
            // that writes this buffer only after the next chunk's barrier, which every thread reaches after
            // these reads
            if (PF_PBUF == 1) __syncthreads();
        }
    }
    const int m = m0 + rl, R = r0 + 8 * w + 4 * h;
    if (m < a.M) {
        float *dst = a.y + (size_t)m * W.rows + R;
        if (R + 3 < W.rows) *(float4 *)dst = acc;
        else {
            const float v[4] = {acc.x, acc.y, acc.z, acc.w};
            for (int j = 0; j < 4; j++)
                if (R + j < W.rows) dst[j] = v[j];
        }
    }
}

hipError_t launch_pgemm(int wbits, int gs, int sf32, const PgemmArgs &a, hipStream_t st) {
    const TiledMat &W = a.W;
    // rows in whole groups of 4 (scale loads), 16-byte aligned activation rows and output rows
    if (a.M < 1 || W.rows % 4 || W.n % gs || W.n % 16 || ((uintptr_t)a.xq & 15) || ((uintptr_t)a.y & 15) ||
        W.gs != gs || W.wbits != wbits || W.sf32 != sf32)
        return hipErrorInvalidValue;
    const int xt = (W.rows + 31) / 32, yt = (a.M + 31) / 32;
    const unsigned blocks = (unsigned)(8 * ((xt + 7) / 8) * yt);
#define PG(WB_, GS_, SF_)                                                                                      \
    if (wbits == WB_ && gs == GS_ && sf32 == SF_) {                                                           \
        hipLaunchKernelGGL((k_pgemm<WB_, GS_, SF_>), dim3(blocks), dim3(64 * PF_KW), 0, st, a);                \
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

// rmsnorm (qwen.c:337-344, runq.c:394-407) of x[m], then int8 quantization (qwen.c:354-364 / runq.c:244-270).
// With RESID the residual add of the previous GEMM comes first: x[m] += y[m] (qwen.c:551, 565; runq.c:575-577,
// 603-605), stored back, then normalized.
template <bool RESID>
__global__ void __launch_bounds__(256) k_p_norm_quant(ProwArgs a) {
    extern __shared__ __align__(16) float sv[]; // dim floats + 4 per wave
    const int m = blockIdx.x, n = a.dim;
    float *x = a.x + (size_t)m * n;
    float part = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = x[i];
        if constexpr (RESID) {
            v = v + a.y[(size_t)m * n + i];
            x[i] = v;
        }
        sv[i] = v;
        part += v * v;
    }
    float ss;
    if (a.strict) { // one running sum in element order (qwen.c:339, runq.c:396-398)
        __syncthreads();
        if (threadIdx.x == 0) sv[n] = seq_sum_squares(sv, n);
        __syncthreads();
        ss = sv[n];
    } else {
        ss = block_sum(part, sv + n);
    }
    ss /= (float)n;
    ss += a.eps;
    ss = 1.0f / sqrtf(ss);
    for (int i = threadIdx.x; i < n; i += blockDim.x) sv[i] = a.norm_w[i] * (ss * sv[i]);
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
    const int m = blockIdx.x, hid = a.hidden, hb = a.gu_rb / 2; // hb: a multiple of 4
    const float *y = a.y + (size_t)m * 2 * hid;
    // 16-byte loads of 4 gate and the 4 matching up values, V pairs per thread issued before any is used
    constexpr int V = 8;
    const int step = 4 * blockDim.x;
    for (int j0 = 4 * threadIdx.x; j0 < hid; j0 += V * step) {
        float4 g4[V], u4[V];
#pragma unroll
        for (int k = 0; k < V; k++) {
            const int j = min(j0 + k * step, hid - 4), b = j / hb, r = j - b * hb;
            g4[k] = *(const float4 *)(y + b * a.gu_rb + r);
            u4[k] = *(const float4 *)(y + b * a.gu_rb + hb + r);
        }
#pragma unroll
        for (int k = 0; k < V; k++) {
            const int j = j0 + k * step;
            if (j < hid) {
                const float g[4] = {g4[k].x, g4[k].y, g4[k].z, g4[k].w}, u[4] = {u4[k].x, u4[k].y, u4[k].z, u4[k].w};
                float h[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float sig = 1.0f / (1.0f + (a.strict ? ref_expf(-g[e]) : expf(-g[e])));
                    const float gs = g[e] * sig;
                    h[e] = gs * u[e];
                }
                *(float4 *)(sv + j) = make_float4(h[0], h[1], h[2], h[3]);
            }
        }
    }
    __syncthreads();
    block_quantize(sv, hid, a.gs, a.qflavor, a.oq + (size_t)m * hid, a.os + (size_t)m * (hid / a.gs));
}

// ------------------------------------------------------------------------------------------------------
// causal attention (qwen.c:526-546, runq.c:530-568) of the chunk's tokens over the KV cache
//
// The positions 0 .. p0 + m of token m are cut into slices of att_sl (a multiple of 16); each slice leaves
// its running max, sum of exponentials and exp-weighted value sums, and k_p_attn_merge combines a token's
// slices.  A token with a single slice gets its output straight from the slice kernel.

typedef float f32x4v __attribute__((ext_vector_type(4)));
// key positions staged in LDS per step: 4 tiles of 16 (2 for a head size of 128, within 64 KB of LDS)
__host__ __device__ constexpr int pa_kc(int hs) { return hs >= 128 ? 32 : 64; }

// Block = (kv head, tile of 16 consecutive tokens, slice); wave j is query head kv_mul * kvh + j, so the K/V
// rows staged for the slice serve all heads of the group.  fp32 MFMA (16x16x4) with lane l = 16 g + r:
//   scores S^T = K Q^T: A lane = K[key r][dim], B lane = Q[token r][dim]; in step u lane group g takes
//     dim g * HS/4 + u (a permutation of the dot's terms), so each lane reads its K row as 16-byte vectors;
//     D lane = S[token r][keys 4g + i], i = 0..3: every lane's scores belong to its own token r;
//   values O^T += V^T P^T: A lane = V[key 4g + u][16 dt + r], B lane = P[token r][key 4g + u], the lane's
//     own probability; D lane = O[token r][16 dt + 4g + i].
// The online softmax (running max and sum per token) therefore needs no data movement except the max over
// the four lanes of a token.
// With `direct`, a token whose positions all fall in slice 0 gets its output here, normalized and quantized
// to int8 for the o projection (a group of gs values lies inside one head: hs % gs == 0); every other token
// leaves its slice partials for k_p_attn_merge.
template <int HS>
__global__ void __launch_bounds__(512) k_p_flash(ProwArgs a, int direct) {
    constexpr int H4 = HS / 4, KS = HS + 4, DT = HS / 16, PA_KC = pa_kc(HS);
    extern __shared__ __align__(16) float sm[];
    float *sk = sm, *sv = sm + PA_KC * KS; // [PA_KC][KS] each
    const int kvh = blockIdx.x, m0 = 16 * blockIdx.y, s = blockIdx.z, kv_mul = a.n_heads / a.n_kv;
    const int t_begin = s * a.att_sl;
    const int t_stop = min(t_begin + a.att_sl, a.p0 + min(m0 + 16, a.M)); // keys of the slice any token sees
    if (t_begin >= t_stop) return; // the whole block
    const int tid = threadIdx.x, nt = blockDim.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, g = l >> 4, r = l & 15;
    const int h = kvh * kv_mul + w, m = min(m0 + r, a.M - 1), qlim = a.p0 + m;
    const float rinv = 1.0f / sqrtf((float)HS);

    float qv[H4];
    {
        const f32x4v *qp = (const f32x4v *)(a.q + (size_t)m * a.dim + (size_t)h * HS + g * H4);
#pragma unroll
        for (int i = 0; i < H4 / 4; i++) {
            const f32x4v v = qp[i];
            qv[4 * i] = v.x;
            qv[4 * i + 1] = v.y;
            qv[4 * i + 2] = v.z;
            qv[4 * i + 3] = v.w;
        }
    }
    f32x4v o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f; // l_run: this lane's share (its keys 4g + i) of the token's sum

    for (int tc = t_begin; tc < t_stop; tc += PA_KC) {
        const int nk = min(PA_KC, t_stop - tc);
        // stage K and V rows tc .. tc + PA_KC - 1 (rows past the slice's last are clamped to it: finite values
        // that the mask or a zero probability removes)
        for (int i = tid; i < PA_KC * H4; i += nt) {
            const int k = i / H4, c = i - k * H4;
            const size_t gi = (size_t)(tc + min(k, nk - 1)) * a.kv_dim + (size_t)kvh * HS + 4 * c;
            const f32x4v kk = *(const f32x4v *)(a.kc + gi), vv = *(const f32x4v *)(a.vc + gi);
            *(f32x4v *)(sk + k * KS + 4 * c) = kk;
            *(f32x4v *)(sv + k * KS + 4 * c) = vv;
        }
        __syncthreads();
        const int ntile = (nk + 15) / 16;
        f32x4v sc[PA_KC / 16];
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < PA_KC / 16; kt++) {
            sc[kt] = f32x4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            if (kt < ntile) {
                f32x4v d = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
                const float *kr = sk + (16 * kt + r) * KS + g * H4;
#pragma unroll
                for (int i = 0; i < H4 / 4; i++) {
                    const f32x4v kk = *(const f32x4v *)(kr + 4 * i);
                    d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.x, qv[4 * i], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.y, qv[4 * i + 1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.z, qv[4 * i + 2], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.w, qv[4 * i + 3], d, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = tc + 16 * kt + 4 * g + i;
                    const float x = t <= qlim ? d[i] * rinv : -INFINITY;
                    sc[kt][i] = x;
                    mx = fmaxf(mx, x);
                }
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        if (m_new > -INFINITY) { // else no key of this token so far: nothing to add
            const float f = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
            m_run = m_new;
            l_run *= f;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[dt] *= f;
#pragma unroll
            for (int kt = 0; kt < PA_KC / 16; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float e = sc[kt][i] == -INFINITY ? 0.0f : expf(sc[kt][i] - m_new);
                    sc[kt][i] = e;
                    l_run += e;
                }
        } else {
#pragma unroll
            for (int kt = 0; kt < PA_KC / 16; kt++) sc[kt] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int kt = 0; kt < PA_KC / 16; kt++) {
            if (kt < ntile) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float *vr = sv + (16 * kt + 4 * g + u) * KS + r;
#pragma unroll
                    for (int dt = 0; dt < DT; dt++)
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[16 * dt], sc[kt][u], o[dt], 0, 0, 0);
                }
            }
        }
        __syncthreads(); // the next step's staging overwrites sk and sv
    }
    float l_tot = l_run + __shfl_xor(l_run, 16);
    l_tot = l_tot + __shfl_xor(l_tot, 32);
    const int S_m = (a.p0 + m) / a.att_sl + 1;
    const bool tok_ok = m0 + r < a.M;
    if (direct && s == 0) {
        // the 4 lanes of token r hold its dims 16 dt + 4 g + i; a group of gs dims is gs / 16 tiles dt of
        // those lanes: its max over the lane's values, then over the 4 lanes (every lane takes part)
        const bool mine = tok_ok && S_m == 1;
        const int tiles = a.gs / 16; // 2 or 4, uniform
        f32x4v val[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++) val[dt] = o[dt] / l_tot;
        int8_t *oq = a.oq + (size_t)m * a.dim + (size_t)h * HS + 4 * g;
        float *os = a.os + ((size_t)m * a.dim + (size_t)h * HS) / a.gs;
#pragma unroll
        for (int g0 = 0; g0 < DT; g0++) {
            if (g0 % tiles) continue; // not the first tile of a group
            float mx = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (k < tiles && g0 + k < DT)
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(val[g0 + k].x), fabsf(val[g0 + k].y)),
                                         fmaxf(fabsf(val[g0 + k].z), fabsf(val[g0 + k].w))));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float scale = quant_scale(mx, a.qflavor), inv = quant_inv(scale);
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (mine && k < tiles && g0 + k < DT) {
                    const f32x4v v = val[g0 + k];
                    const uint32_t b0 = (uint8_t)quant_one(v.x, scale, inv, a.qflavor);
                    const uint32_t b1 = (uint8_t)quant_one(v.y, scale, inv, a.qflavor);
                    const uint32_t b2 = (uint8_t)quant_one(v.z, scale, inv, a.qflavor);
                    const uint32_t b3 = (uint8_t)quant_one(v.w, scale, inv, a.qflavor);
                    *(uint32_t *)(oq + 16 * (g0 + k)) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
                }
            if (mine && g == 0) os[16 * g0 / a.gs] = scale;
        }
        if (S_m == 1) return;
    }
    if (!tok_ok || s >= S_m) return; // no token here, or none of its positions in this slice
    const size_t e0 = ((size_t)m * a.n_heads + h) * a.att_smax + s;
    float *acc = a.att_acc + e0 * HS + 4 * g;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) *(f32x4v *)(acc + 16 * dt) = o[dt];
    if (g == 0) {
        a.att_ml[2 * e0] = m_run;
        a.att_ml[2 * e0 + 1] = l_tot;
    }
}

// causal attention of token m over positions 0 .. p0 + m, cut into slices of att_sl positions: block =
// (kv head, token, slice) leaves the slice's running max, sum of exponentials and exp-weighted value sums
// (the generic path, for head sizes and group sizes k_p_flash does not take)
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

// merge of token m's S slices: with mx the largest slice max, w_s = exp(max_s - mx) / sum_k l_k exp(max_k - mx)
// and out[h*hs + e] = sum_s acc_s[e] * w_s, then the row quantized to int8 for the o projection (qwen.c:549,
// runq.c:571).  Tokens with one slice were done by k_p_flash, unless `all` (then every token is merged here).
__global__ void __launch_bounds__(256) k_p_attn_merge(ProwArgs a, int all) {
    extern __shared__ __align__(16) float sm[]; // dim floats of the row, then [n_heads][att_smax] weights
    float *row = sm, *wgt = sm + a.dim;
    const int m = blockIdx.x, hs = a.head_size, S = (a.p0 + m) / a.att_sl + 1;
    if (S == 1 && !all) return;
    // fixed-trip loops with the slice count as a predicate: every load of a row is issued before the first
    // is waited for
    for (int h = threadIdx.x; h < a.n_heads; h += blockDim.x) {
        const float *ml = a.att_ml + ((size_t)m * a.n_heads + h) * a.att_smax * 2;
        float mv[PREFILL_ATT_SMAX], lv[PREFILL_ATT_SMAX];
#pragma unroll
        for (int k = 0; k < PREFILL_ATT_SMAX; k++)
            if (k < S) { mv[k] = ml[2 * k]; lv[k] = ml[2 * k + 1]; }
        float mx = mv[0];
#pragma unroll
        for (int k = 1; k < PREFILL_ATT_SMAX; k++)
            if (k < S) mx = fmaxf(mx, mv[k]);
        float l = 0.0f;
#pragma unroll
        for (int k = 0; k < PREFILL_ATT_SMAX; k++)
            if (k < S) {
                mv[k] = expf(mv[k] - mx);
                l += lv[k] * mv[k];
            }
        const float il = 1.0f / l;
#pragma unroll
        for (int k = 0; k < PREFILL_ATT_SMAX; k++)
            if (k < S) wgt[h * a.att_smax + k] = mv[k] * il;
    }
    __syncthreads();
    for (int o = threadIdx.x; o < a.dim; o += blockDim.x) {
        const int h = o / hs, e = o - h * hs;
        const float *acc = a.att_acc + ((size_t)m * a.n_heads + h) * a.att_smax * hs + e;
        const float *wh = wgt + h * a.att_smax;
        float x[PREFILL_ATT_SMAX];
#pragma unroll
        for (int k = 0; k < PREFILL_ATT_SMAX; k++)
            if (k < S) x[k] = acc[(size_t)k * hs];
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < PREFILL_ATT_SMAX; k++)
            if (k < S) v += x[k] * wh[k];
        row[o] = v;
    }
    __syncthreads();
    block_quantize(row, a.dim, a.gs, a.qflavor, a.oq + (size_t)m * a.dim, a.os + (size_t)m * (a.dim / a.gs));
}

// Reference-order causal attention: block (h, m) is query head h of token m over positions 0 .. p0 + m
// (attn_strict_head); the fp32 output row goes to xb[m], quantized afterwards by k_p_quant_rows.
__global__ void __launch_bounds__(256) k_p_attn_strict(ProwArgs a) {
    extern __shared__ __align__(16) float sm[];
    const int h = blockIdx.x, m = blockIdx.y, hs = a.head_size, kv_mul = a.n_heads / a.n_kv;
    attn_strict_head(a.q + (size_t)m * a.dim + (size_t)h * hs, a.kc, a.vc, a.kv_dim, (h / kv_mul) * hs, hs,
                     a.p0 + m + 1, sm, a.xb + (size_t)m * a.dim + (size_t)h * hs);
}

// int8 quantization of the rows xb[m] (qwen.c:549, runq.c:571) into the o projection's input
__global__ void __launch_bounds__(256) k_p_quant_rows(ProwArgs a) {
    extern __shared__ __align__(16) float sv[];
    const int m = blockIdx.x, n = a.dim;
    for (int i = threadIdx.x; i < n; i += blockDim.x) sv[i] = a.xb[(size_t)m * n + i];
    __syncthreads();
    block_quantize(sv, n, a.gs, a.qflavor, a.oq + (size_t)m * n, a.os + (size_t)m * (n / a.gs));
}

hipError_t launch_p_embed(const ProwArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(k_p_embed, dim3(a.M), dim3(256), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_p_norm_quant(const ProwArgs &a, bool resid, hipStream_t st) {
    if (a.dim % 4 || ((uintptr_t)a.oq & 3)) return hipErrorInvalidValue;
    if (resid) hipLaunchKernelGGL(k_p_norm_quant<true>, dim3(a.M), dim3(256), (size_t)(a.dim + 8) * 4, st, a);
    else hipLaunchKernelGGL(k_p_norm_quant<false>, dim3(a.M), dim3(256), (size_t)(a.dim + 8) * 4, st, a);
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
    if (a.hidden % 4 || a.gu_rb % 8 || ((uintptr_t)a.oq & 3) || ((uintptr_t)a.y & 15)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_p_swiglu_quant, dim3(a.M), dim3(256), (size_t)a.hidden * 4, st, a);
    return hipGetLastError();
}
hipError_t launch_p_attention(const ProwArgs &a, hipStream_t st) {
    const int kv_mul = a.n_heads / a.n_kv, hs = a.head_size;
    if (a.strict) {
        const size_t lds = attn_strict_lds_floats(hs, a.p0 + a.M, 256) * 4;
        if (hs % 4 || ((uintptr_t)a.kc & 15) || a.kv_dim % 4 || a.dim % 4 || a.dim % a.gs || !a.xb ||
            ((uintptr_t)a.oq & 3) || lds > 65536 || a.n_heads % a.n_kv)
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_p_attn_strict, dim3(a.n_heads, a.M), dim3(256), lds, st, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_p_quant_rows, dim3(a.M), dim3(256), (size_t)a.dim * 4, st, a);
        return hipGetLastError();
    }
    if (kv_mul * hs > 1024 || hs % 4 || hs > 128 || ((uintptr_t)a.q & 15) || ((uintptr_t)a.kc & 15) ||
        ((uintptr_t)a.vc & 15) || ((uintptr_t)a.oq & 3) || ((uintptr_t)a.att_acc & 15) || a.kv_dim % 4 ||
        a.dim % 4 || a.dim % a.gs || a.att_sl < ATT_SUB || a.att_sl % 16 || a.att_smax < 1 ||
        a.att_smax > PREFILL_ATT_SMAX || (a.p0 + a.M + a.att_sl - 1) / a.att_sl > a.att_smax || a.n_heads % a.n_kv)
        return hipErrorInvalidValue;
    const size_t merge_lds = ((size_t)a.dim + (size_t)a.n_heads * a.att_smax) * 4;
    const bool flash = kv_mul <= 8 && (hs == 16 || hs == 32 || hs == 48 || hs == 64 || hs == 128);
    // single-slice tokens quantized by the slice kernel when a quantization group stays inside one head
    const int direct = flash && hs % a.gs == 0 && (a.gs == 32 || a.gs == 64);
    if (flash) {
        const dim3 grid(a.n_kv, (a.M + 15) / 16, a.att_smax);
        const size_t lds = (size_t)2 * pa_kc(hs) * (hs + 4) * 4;
#define PF_FLASH(HS_)                                                                                         \
    if (hs == HS_) hipLaunchKernelGGL(k_p_flash<HS_>, grid, dim3(64 * kv_mul), lds, st, a, direct);
        PF_FLASH(16) PF_FLASH(32) PF_FLASH(48) PF_FLASH(64) PF_FLASH(128)
#undef PF_FLASH
    } else {
        hipLaunchKernelGGL(k_p_attention, dim3(a.n_kv, a.M, a.att_smax), dim3(256),
                           attn_lds_floats(kv_mul, hs) * 4, st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if ((a.p0 + a.M - 1) / a.att_sl == 0 && direct) return hipSuccess; // every token has one slice
    hipLaunchKernelGGL(k_p_attn_merge, dim3(a.M), dim3(256), merge_lds, st, a, direct ? 0 : 1);
    return hipGetLastError();
}
