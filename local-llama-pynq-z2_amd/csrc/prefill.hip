// Prefill kernels of libmatvec_hip.so for gfx950: the prompt's positions through a layer together.
//
// The reference processes a prompt one position at a time with the same forward() (qwen.c:674-681); no
// batched prefill exists there (README.md:386-387).  Here the M positions of a chunk share each weight
// read: the layer matrices become int8 MFMA GEMMs (v_mfma_i32_16x16x32_i8) over the tiled records the decode
// GEMV reads, with the per-group int32 sums exact and the group terms p = ((float)ival * ws) * xs added in
// group order, which is the reference's matmul (qwen.c:436-456, runq.c:429-458) for every (row, token).
// The element-wise steps of forward() run per token, and attention is causal over the KV cache.
#include <type_traits>

#include "attn.h"
#include "prefill.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// block_quantize into the token-block tiles of the next GEMM's input (token m of MB blocks)
__device__ __forceinline__ void block_quantize_tiles(const float *v, int n, int gs, int flavor, int8_t *q, float *s,
                                                     int m, int MB) {
    const int nq = n / 4;
    for (int i0 = 0; i0 < nq; i0 += blockDim.x) {
        const int i = i0 + threadIdx.x;
        const bool ok = i < nq; // whole groups are in or out: nq is a multiple of gs / 4
        float scale;
        const uint32_t packed = quantize_pack(((const float4 *)v)[ok ? i : 0], gs, flavor, &scale);
        if (ok) {
            *(uint32_t *)(q + pf_act_off(m, 4 * i, MB)) = packed;
            if ((i & (gs / 4 - 1)) == 0) s[pf_scale_off(m, i / (gs / 4), MB)] = scale;
        }
    }
}

// ------------------------------------------------------------------------------------------------------
// GEMM: y[m][r] = sum_g ((float)ival(r, m, g) * ws[r][g]) * xs[m][g], groups in order.
//
// One wave per tile of 16 TA rows x 16 TB tokens: the wave runs all K groups of its tile in order and keeps its
// 4 TA TB sums in registers, so no product crosses waves and no barrier is needed.
//
// Per group and 32-element chunk, TA x TB v_mfma_i32_16x16x32_i8.  Lane l = 16 j + t holds row t of A and
// token t of B, 8 elements of the chunk each: 4 j .. 4 j + 3 and 16 + 4 j .. 16 + 4 j + 3 (the int32 sum
// does not depend on how K is split over the lanes, only that A and B split it alike); D: token t, rows
// 4 j .. 4 j + 3.  In the tiled weight records those elements are dword j of a row's int4 segment (low and
// high nibbles) or of its two int8 pieces, so:
//
//  - A: one 16-byte load per lane fetches whole segments, lane row r (16 lanes) taking the segment of (row
//    block r % TA, group r / TA of the load) for its 16 rows; a 4 x 4 transpose of those dwords across the
//    lane rows (v_permlane32_swap, v_permlane16_swap) leaves on lane row j dword j of all four segments.  int4
//    nibbles enter as 16 q (moved to the top of their bytes), with the scale divided by 16: 16 s * (ws / 16)
//    rounds like s * ws.
//  - B: one 16-byte load per lane and token block brings two chunks (the input layout of pf_act_off).
//  - activation scales: one float4 per lane and token block for 4 groups (pf_scale_off).
//  - weight scales: each lane loads and converts TA of the 64 TA (row, group) scales of 4 groups, and they
//    reach the lanes that apply them through the wave's LDS slots.
//
// With fp16 scales every group's MFMA starts from PG_MAGIC_I instead of 0, so the bits of a result are the
// float PG_MAGIC + s exactly (s = the group's int32 sum, |s| <= 2^19 < 2^22).  With ws the row's scale and
// nc = -PG_MAGIC * ws, which is exact (1.5 * 2^23 times an fp16 value needs 13 significant bits),
// fmaf(PG_MAGIC + s, ws, nc) = RN(s * ws): the reference's ((float)ival) * ws (qwen.c:452) in one
// instruction, bitwise, for finite scales.  Then p * xs and the add in group order: 3 VALU instructions per
// output and group.  fp32 scales (3 ws is not always a float) take a conversion instead.
//
// The loads of the next 4 groups are in flight while the current 4 run; group g's MFMAs are issued before
// group g - 1's products, whose sums they do not touch.  Block = 4 waves = 4 consecutive token tiles of one
// row tile (they read the same weights); a row tile's token tiles run on one XCD (block b goes to XCD b % 8),
// where its weights stay in L2.
#define PG_MAGIC_I 0x4B400000
#define PG_MAGIC 12582912.0f
#define PG_RSRC3 0x00020000 // buffer resource word 3 for gfx9: 32-bit data format, raw (no swizzle, no stride)

// 4 x 4 transpose of dwords across the 4 lane rows: on entry lane row r holds x[0..3] of its own segment; on
// return lane row j holds in x[i] dword j of lane row i's segment.
__device__ __forceinline__ void lane_row_transpose(uint32_t (&x)[4]) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false); // x0 rows 2,3 <-> x2 rows 0,1
    const auto s13 = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
    const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false); // odd rows <-> even rows
    const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    x[0] = s01[0];
    x[1] = s01[1];
    x[2] = s23[0];
    x[3] = s23[1];
}

// EK: the epilogue: 0 stores y, 1 SwiGLU + quantization of h (PgemmArgs::swiglu), 2 bias + RoPE + the q / K / V
// writes (PgemmArgs::qkv)
template <int WB, int GSZ, int SF32, int TA, int TB, int EK>
__global__ void __launch_bounds__(256) k_pgemm(PgemmArgs a) {
    constexpr bool SWG = EK == 1;
    constexpr int KC = GSZ / 32;             // 32-element chunks per group
    constexpr int AP = WB == 4 ? 1 : 2 * KC; // 16-byte pieces per (row, group) weight segment
    constexpr int GA = 4 / TA;               // groups per A load
    constexpr int NAL = TA;                  // A loads per piece and 4 groups
    constexpr int NBL = 2 * KC;              // B loads per token block and 4 groups (chunk pairs)
    constexpr int NB = 2;                    // steps of loads in flight
    constexpr int SB = GSZ * WB / 8, SCB = SF32 ? 4 : 2;
    static_assert(TA == 1 || TA == 2 || TA == 4, "row blocks per tile");
    const TiledMat &W = a.W;
    const int xt = (W.rows + 16 * TA - 1) / (16 * TA), yt = (a.M + 16 * TB - 1) / (16 * TB), y4 = (yt + 3) / 4;
    const int b = blockIdx.x, xcd = b & 7, idx = b >> 3;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // SwiGLU epilogue: a quantization group of 32 hidden values is RT row tiles (8 TA hidden values each), so a
    // block is RT row tiles x NTY token tiles, and its waves exchange per-token maxima once at the end
    constexpr int RT = SWG ? 4 / TA : 1, NTY = 4 / RT;
    int tx, ty;
    if constexpr (SWG) {
        const int yb = (yt + NTY - 1) / NTY, gx = xcd + 8 * (idx / yb), tyb = idx - (idx / yb) * yb;
        tx = gx * RT + w % RT;
        ty = tyb * NTY + w / RT;
    } else {
        tx = xcd + 8 * (idx / y4);
        ty = 4 * (idx - (idx / y4) * y4) + w;
    }
    const bool valid = tx < xt && ty < yt;
    if constexpr (!SWG) {
        if (!valid) return; // the whole wave (the waves of a block share nothing but the block)
    } else { // past the matrix or the tokens: a valid tile computed again, nothing stored, for the barrier
        tx = min(tx, xt - 1);
        ty = min(ty, yt - 1);
    }
    const int l = threadIdx.x & 63, q = l >> 4, c16 = l & 15;
    const int r0 = tx * 16 * TA, m0 = ty * 16 * TB, MB = (a.M + 15) >> 4;
    const int rb = W.rb, ng = W.ng, gpc = WAVE / rb, lg = 31 - __builtin_clz(gpc);
    const int nq = (ng + 3) >> 2, nfull = ng >> 2; // 4-group steps, the full ones
    const uint32_t rstride = (uint32_t)W.nchunks * (uint32_t)W.rec;

    // Per-lane parts of the load offsets.  A record offset is (row block, chunk c, slot gi) -> b * rstride
    // + c * rec + ...; for the 4 groups g0 .. g0 + 3 of a step (g0 a multiple of 4) the chunk and slot of
    // group g0 + e split into a part common to the wave (c0 = g0 >> lg, gi0 = g0 & (gpc - 1)) and a per-lane
    // part (e >> lg, e & (gpc - 1)), since gpc is 1, 2, 4 or 8.  Rows past the matrix clamp to its last row.
    uint32_t offA[NAL], offS[TA];
#pragma unroll
    for (int s = 0; s < NAL; s++) {
        const int e = s * GA + q / TA; // group of this lane row within the step
        const int row = min(r0 + 16 * (q % TA) + c16, W.rows - 1), bA = row / rb, la = row - bA * rb;
        offA[s] = bA * rstride + (e >> lg) * (uint32_t)W.rec + ((e & (gpc - 1)) * rb + la) * 16;
    }
#pragma unroll
    for (int t = 0; t < TA; t++) {
        const int ent = 64 * t + l, e = ent / (16 * TA), rho = ent - e * 16 * TA;
        const int row = min(r0 + rho, W.rows - 1), bS = row / rb, la = row - bS * rb;
        offS[t] = bS * rstride + (e >> lg) * (uint32_t)W.rec + 64 * SB + ((e & (gpc - 1)) * rb + la) * SCB;
    }
    uint32_t offB[TB], offX[TB];
#pragma unroll
    for (int j = 0; j < TB; j++) {
        const int tb = min(ty * TB + j, MB - 1); // past the last token block: clamped, outputs not stored
        offB[j] = (uint32_t)tb * 1024 + 16 * l;
        offX[j] = (uint32_t)(16 * tb + c16) * 16;
    }

    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)W.data, 0, (int)W.bytes, PG_RSRC3);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.xq, 0, (int)pf_act_bytes(W.n, a.M), PG_RSRC3);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.xs, 0, (int)(pf_scale_floats(ng, a.M) * 4), PG_RSRC3);

    // the loads of two steps: the current one and the next
    uint4 ar[NB][NAL][AP]; // raw A segments
    uint32_t sr[NB][TA];   // raw weight scales
    uint4 br[NB][TB][NBL]; // B chunk pairs
    float4 xr[NB][TB];     // activation scales of the 4 groups
    // Loads of step qs (groups 4 qs ..) into buffer k: a full step (clamp false) with offsets common to the
    // wave, or the last step of ng % 4 groups, whose lanes clamp their groups to ng - 1 (per-lane offsets).
    // The two kinds are separate call sites: one load sequence must not hold both (buffer loads cannot fault,
    // so the compiler would issue both and wait between them).
    auto load = [&](int qs, int k, bool clamp) {
        const int g0 = 4 * qs;
        if (!clamp) {
            const int c0 = g0 >> lg, gi0 = g0 & (gpc - 1);
            const int wo = c0 * (int)W.rec + gi0 * rb * 16, so = c0 * (int)W.rec + gi0 * rb * SCB;
#pragma unroll
            for (int s = 0; s < NAL; s++)
#pragma unroll
                for (int p = 0; p < AP; p++) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rw, offA[s] + p * 1024, wo, 0);
                    ar[k][s][p] = make_uint4(v[0], v[1], v[2], v[3]);
                }
#pragma unroll
            for (int t = 0; t < TA; t++) {
                if constexpr (SF32) sr[k][t] = __builtin_amdgcn_raw_buffer_load_b32(rw, offS[t], so, 0);
                else sr[k][t] = __builtin_amdgcn_raw_buffer_load_b16(rw, offS[t], so, 0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < NAL; s++) {
                const int g = min(g0 + s * GA + q / TA, ng - 1), c = g >> lg, gi = g & (gpc - 1);
                const int row = min(r0 + 16 * (q % TA) + c16, W.rows - 1), bA = row / rb, la = row - bA * rb;
                const uint32_t o = bA * rstride + c * (uint32_t)W.rec + (gi * rb + la) * 16;
#pragma unroll
                for (int p = 0; p < AP; p++) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rw, o + p * 1024, 0, 0);
                    ar[k][s][p] = make_uint4(v[0], v[1], v[2], v[3]);
                }
            }
#pragma unroll
            for (int t = 0; t < TA; t++) {
                const int ent = 64 * t + l, e = ent / (16 * TA), rho = ent - e * 16 * TA;
                const int g = min(g0 + e, ng - 1), c = g >> lg, gi = g & (gpc - 1);
                const int row = min(r0 + rho, W.rows - 1), bS = row / rb, la = row - bS * rb;
                const uint32_t o = bS * rstride + c * (uint32_t)W.rec + 64 * SB + (gi * rb + la) * SCB;
                if constexpr (SF32) sr[k][t] = __builtin_amdgcn_raw_buffer_load_b32(rw, o, 0, 0);
                else sr[k][t] = __builtin_amdgcn_raw_buffer_load_b16(rw, o, 0, 0);
            }
        }
        // chunk pairs of the step (4 KC chunks from chunk 4 KC qs), within the input's last pair
        const int np = (ng * KC + 1) >> 1;
#pragma unroll
        for (int j = 0; j < TB; j++) {
#pragma unroll
            for (int t = 0; t < NBL; t++) {
                const int pr = min(2 * KC * (g0 >> 2) + t, np - 1);
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(rx, offB[j], pr * MB * 1024, 0);
                br[k][j][t] = make_uint4(v[0], v[1], v[2], v[3]);
            }
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, offX[j], (g0 >> 2) * MB * 256, 0);
            xr[k][j] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                   __uint_as_float(v[3]));
        }
    };

    // the step's weights after the transpose: wa[k][s][p][i] = dword q of lane row i's segment of A load s
    uint32_t wa[NAL][AP][4];
    __shared__ __align__(16) float s_ws[4][NB][4][16 * TA], s_nc[4][NB][4][16 * TA];
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // begin a step from buffer k: transpose the A segments, convert this lane's weight scales into LDS
    // buffer k (then wave_sync before any read of it)
    auto begin = [&](int k) {
#pragma unroll
        for (int s = 0; s < NAL; s++)
#pragma unroll
            for (int p = 0; p < AP; p++) {
                uint32_t x[4] = {ar[k][s][p].x, ar[k][s][p].y, ar[k][s][p].z, ar[k][s][p].w};
                lane_row_transpose(x);
#pragma unroll
                for (int i = 0; i < 4; i++) wa[s][p][i] = x[i];
            }
#pragma unroll
        for (int t = 0; t < TA; t++) {
            const int ent = 64 * t + l, e = ent / (16 * TA), rho = ent - e * 16 * TA;
            const float ws = SF32 ? __uint_as_float(sr[k][t])
                                  : f16_bits_to_f32((uint16_t)sr[k][t]) * (WB == 4 ? 0.0625f : 1.0f);
            s_ws[w][k][e][rho] = ws;
            s_nc[w][k][e][rho] = -(PG_MAGIC * ws);
        }
    };
    const v4i c0 = SF32 ? v4i{0, 0, 0, 0} : v4i{PG_MAGIC_I, PG_MAGIC_I, PG_MAGIC_I, PG_MAGIC_I};
    // MFMAs of group e of the step in buffer k
    auto mfma = [&](int k, int e, v4i (&dn)[TA][TB]) {
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            const int ch = e * KC + kc; // chunk within the step: pair ch / 2, half ch % 2
#pragma unroll
            for (int i = 0; i < TA; i++) {
                const int s = e / GA, li = (e % GA) * TA + i; // A load and lane row of (group e, block i)
                uint32_t lo, hi;
                if constexpr (WB == 4) {
                    const uint32_t x = wa[s][0][li];
                    lo = (x << 4) & 0xF0F0F0F0u;
                    hi = x & 0xF0F0F0F0u;
                } else {
                    lo = wa[s][2 * kc][li];
                    hi = wa[s][2 * kc + 1][li];
                }
                const long av = (long)(((uint64_t)hi << 32) | lo);
#pragma unroll
                for (int j = 0; j < TB; j++) {
                    const uint4 &v = br[k][j][ch >> 1];
                    const long bw = (ch & 1) ? (long)(((uint64_t)v.w << 32) | v.z) : (long)(((uint64_t)v.y << 32) | v.x);
                    dn[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bw, kc == 0 ? c0 : dn[i][j], 0, 0, 0);
                }
            }
        }
    };
    float acc[TA][TB][4];
#pragma unroll
    for (int i = 0; i < TA; i++)
#pragma unroll
        for (int j = 0; j < TB; j++)
#pragma unroll
            for (int k = 0; k < 4; k++) acc[i][j][k] = 0.0f;
    // the weight scales of this lane's output rows for group e of the step in buffer k, read from LDS one
    // group ahead of their use (by group parity)
    float4 scw[2][TA], scn[2][TA];
    auto read_scales = [&](int k, int e) {
#pragma unroll
        for (int i = 0; i < TA; i++) {
            scw[e & 1][i] = *(const float4 *)(&s_ws[w][k][e][16 * i + 4 * q]);
            scn[e & 1][i] = *(const float4 *)(&s_nc[w][k][e][16 * i + 4 * q]);
        }
    };
    // products of group e of the step in buffer k (MFMA results d, scales read by read_scales) added to the
    // sums; x: the group's activation scales when they are not in xr[k] any more
    auto products = [&](const v4i (&d)[TA][TB], int k, int e, const float *x) {
#pragma unroll
        for (int i = 0; i < TA; i++) {
            const float4 ws4 = scw[e & 1][i], nc4 = scn[e & 1][i];
            const float wsv[4] = {ws4.x, ws4.y, ws4.z, ws4.w}, ncv[4] = {nc4.x, nc4.y, nc4.z, nc4.w};
#pragma unroll
            for (int j = 0; j < TB; j++) {
                const float xv[4] = {xr[k][j].x, xr[k][j].y, xr[k][j].z, xr[k][j].w};
                const float xe = x ? x[j] : xv[e];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float p = SF32 ? (float)d[i][j][r] * wsv[r] : fmaf(__int_as_float(d[i][j][r]), wsv[r], ncv[r]);
                    p = p * xe; // qwen.c:452, runq.c:452
                    acc[i][j][r] = acc[i][j][r] + p;
                }
            }
        }
    };
    v4i d[2][TA][TB]; // MFMA results by group parity
    // Step qs from buffer k (k = qs & 1).  The next step's loads go first, into buffer k ^ 1 (next = 0 none,
    // 1 a full step, 2 the last, partial step); of that buffer only the previous step's group 3 activation
    // scales are still needed, and are kept aside.  Group e's scale reads and MFMAs precede group e - 1's
    // products (group 0's predecessor: the previous step's group 3), so the LDS and MFMA latencies pass during
    // VALU work.  The scheduling barrier after each group keeps that order (the compiler would otherwise
    // hoist later groups' scale reads, holding their registers).  In the partial step groups past ng are
    // skipped.
    auto step = [&](int qs, int k, int next, bool last) {
        float x3[TB];
#pragma unroll
        for (int j = 0; j < TB; j++) x3[j] = xr[k ^ 1][j].w;
        if (next == 1) load(qs + 1, k ^ 1, false);
        if (next == 2) load(qs + 1, k ^ 1, true);
        begin(k);
        wave_sync();
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int g = 4 * qs + e;
            if (last && g >= ng) break;
            read_scales(k, e);
            mfma(k, e, d[e & 1]);
            if (e == 0) {
                if (qs > 0) products(d[1], k ^ 1, 3, x3);
            } else {
                products(d[(e - 1) & 1], k, e - 1, nullptr);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // QKV epilogue operands of every (row, token) of the tile: the bias of the row and of its RoPE partner
    // (NeoX), and cos / sin at the token's position, loaded together in the epilogue.  (Loading them ahead of
    // the weights costs the 16 x 16 tile a wave of occupancy, 106 -> 130 VGPRs, and measured slower: the
    // 512-token Qwen2-0.5B-shape QKV GEMM 9.8 -> 10.6 us.)
    [[maybe_unused]] float pb[TA][TB][4], pbp[TA][TB][4], pc[TA][TB][4], ps[TA][TB][4];
    auto qkv_operands = [&]() __attribute__((always_inline)) {
        const int dim = a.dim, hs = a.head_size, half = hs / 2, rot = dim + a.kv_dim;
        const bool neox = a.rope_kind == ROPE_NEOX;
#pragma unroll
        for (int i = 0; i < TA; i++)
#pragma unroll
            for (int j = 0; j < TB; j++) {
                const int m = min(m0 + 16 * j + c16, a.M - 1), pos = a.p0 + m;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int R = min(r0 + 16 * i + 4 * q + k, W.rows - 1), Rr = min(R, rot - 1);
                    int ii, ib = R, ibp = R;
                    if (neox) {
                        const int blk = Rr / 16, r = Rr & 15, per = half / 8, hh = blk / per;
                        ii = (blk - hh * per) * 8 + (r & 7);
                        if (R < rot) {
                            ib = hh * hs + (r < 8 ? ii : half + ii);
                            ibp = hh * hs + (r < 8 ? half + ii : ii);
                        }
                        pb[i][j][k] = a.bias[ib];
                        pbp[i][j][k] = a.bias[ibp];
                    } else {
                        const int e = Rr < dim ? Rr : Rr - dim;
                        ii = (e % hs) / 2;
                    }
                    pc[i][j][k] = a.rope_cos[(size_t)pos * half + ii];
                    ps[i][j][k] = a.rope_sin[(size_t)pos * half + ii];
                }
            }
    };
    const bool partial = nq > nfull;
    int qs = 0;
    if (nfull > 0) {
        load(0, 0, false);
        // full steps followed by full steps, two at a time (buffers 0, 1), then the last one or two full steps
        for (; qs + 2 < nfull; qs += 2) {
            step(qs, 0, 1, false);
            step(qs + 1, 1, 1, false);
        }
        if (qs + 2 == nfull) {
            step(qs, 0, 1, false);
            step(qs + 1, 1, partial ? 2 : 0, false);
        } else {
            step(qs, 0, partial ? 2 : 0, false);
        }
        qs = nfull;
    } else {
        load(0, 0, true);
    }
    if (partial) { // a last step of ng % 4 groups
        if (qs & 1) step(qs, 1, 0, true);
        else step(qs, 0, 0, true);
    }
    // the products of the last group, ng - 1: group (ng - 1) % 4 of step nq - 1, buffer (nq - 1) & 1
    {
        const int e = (ng - 1) & 3, k = (nq - 1) & 1;
#pragma unroll
        for (int kk = 0; kk < 2; kk++)
#pragma unroll
            for (int ee = 0; ee < 4; ee++)
                if (kk == k && ee == e) products(d[ee & 1], kk, ee, nullptr);
    }
    if constexpr (EK == 2) {
        // k_p_qkv's operations on the tile (qwen.c:515-524 / runq.c:500-521): lane row k of row tile i holds row
        // R = r0 + 16 i + 4 q + k of token m; its NeoX partner R ^ 8 (same block of 16) is lane row k of the lane
        // l ^ 32, its interleaved partner R ^ 1 lane row k ^ 1 of this lane.  The bias and RoPE operands of
        // every (row, token) are loaded before (qkv_operands), then the outputs computed in k_p_qkv's order.
        const int dim = a.dim, kvd = a.kv_dim, hs = a.head_size, half = hs / 2, rot = dim + kvd;
        const bool neox = a.rope_kind == ROPE_NEOX;
        qkv_operands();
        float part[TA][TB][4];
#pragma unroll
        for (int i = 0; i < TA; i++)
#pragma unroll
            for (int j = 0; j < TB; j++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    // the NeoX partner, from the lane across the halves (every lane takes part in the swap)
                    const uint32_t vb = __float_as_uint(acc[i][j][k]);
                    const auto sw = __builtin_amdgcn_permlane32_swap(vb, vb, false, false);
                    part[i][j][k] = __uint_as_float((q >> 1) ? sw[0] : sw[1]);
                }
#pragma unroll
        for (int i = 0; i < TA; i++)
#pragma unroll
            for (int j = 0; j < TB; j++) {
                const int m = m0 + 16 * j + c16, pos = a.p0 + m;
                if (m >= a.M) continue;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int R = r0 + 16 * i + 4 * q + k;
                    if (R >= W.rows) continue;
                    const float v = acc[i][j][k];
                    if (neox) {
                        if (R < rot) {
                            const int blk = R / 16, r = R & 15, per = half / 8, hh = blk / per;
                            const int ii = (blk - hh * per) * 8 + (r & 7);
                            const bool first = r < 8;
                            const int e = hh * hs + (first ? ii : half + ii);
                            const float c = pc[i][j][k], sn = ps[i][j][k];
                            const float self = v + pb[i][j][k], partner = part[i][j][k] + pbp[i][j][k];
                            float o;
                            if (first) { float t1 = self * c, t2 = partner * sn; o = t1 - t2; }
                            else { float t1 = self * c, t2 = partner * sn; o = t1 + t2; }
                            if (e < dim) a.q[(size_t)m * dim + e] = o;
                            else a.kc[(size_t)pos * kvd + (e - dim)] = o;
                        } else {
                            a.vc[(size_t)pos * kvd + (R - rot)] = v + pb[i][j][k];
                        }
                    } else {
                        if (R < rot) {
                            const int e = R < dim ? R : R - dim;
                            const float c = pc[i][j][k], sn = ps[i][j][k], partner = acc[i][j][k ^ 1];
                            float o;
                            if ((e & 1) == 0) { float t1 = v * c, t2 = partner * sn; o = t1 - t2; }
                            else { float t1 = partner * sn, t2 = v * c; o = t1 + t2; }
                            if (R < dim) a.q[(size_t)m * dim + e] = o;
                            else a.kc[(size_t)pos * kvd + e] = o;
                        } else {
                            a.vc[(size_t)pos * kvd + (R - rot)] = v;
                        }
                    }
                }
            }
    } else if constexpr (!SWG) {
#pragma unroll
        for (int j = 0; j < TB; j++) {
            const int m = m0 + 16 * j + c16;
            if (m >= a.M) continue;
#pragma unroll
            for (int i = 0; i < TA; i++) {
                const int R = r0 + 16 * i + 4 * q; // rows % 4 == 0: R < rows means all four rows are
                if (R < W.rows)
                    *(float4 *)(a.y + (size_t)m * W.rows + R) =
                        make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
            }
        }
    } else {
        // SwiGLU (qwen.c:556-562, runq.c:589-596) and int8 quantization of h, as k_p_swiglu_quant does it.  Row
        // block tx TA + i holds 8 gate rows, then their 8 up rows: in the MFMA layout lane rows 0, 1 hold gate
        // rows 4 q + r and lane rows 2, 3 the matching up rows of the same token; permlane32_swap gives every
        // lane the other half, so each lane has (gate, up) pairs.  Lane rows 0, 1 take r = 0, 1 and lane rows
        // 2, 3 take r = 2, 3 of gate rows 4 (q & 1) + r: h of hidden value 8 (tx TA + i) + 4 (q & 1) + r of
        // token m0 + 16 j + c16.
        __shared__ float s_gmax[4][16 * TB];
        const int half = q >> 1, qq = q & 1;
        float hv[TA][TB][2], pm[TB];
#pragma unroll
        for (int j = 0; j < TB; j++) pm[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < TA; i++)
#pragma unroll
            for (int j = 0; j < TB; j++)
#pragma unroll
                for (int rr = 0; rr < 2; rr++) {
                    // this lane's r = 2 half + rr: its own value, and its partner's for the same r, which the
                    // partner sends (each lane sends the r its partner takes: rr for lane rows 0, 1, 2 + rr for 2, 3)
                    const float own = half ? acc[i][j][2 + rr] : acc[i][j][rr];
                    const uint32_t sb = __float_as_uint(half ? acc[i][j][rr] : acc[i][j][2 + rr]);
                    const auto sw = __builtin_amdgcn_permlane32_swap(sb, sb, false, false);
                    const float other = __uint_as_float(half ? sw[0] : sw[1]);
                    const float g = half ? other : own, u = half ? own : other;
                    const float sig = 1.0f / (1.0f + (a.strict ? ref_expf(-g) : expf(-g)));
                    const float gs = g * sig;
                    hv[i][j][rr] = gs * u;
                    pm[j] = fmaxf(pm[j], fabsf(hv[i][j][rr]));
                }
        // the token's max over this wave's 8 TA hidden values (all four lane rows), then over the group's RT waves
#pragma unroll
        for (int j = 0; j < TB; j++) {
            pm[j] = fmaxf(pm[j], __shfl_xor(pm[j], 16));
            pm[j] = fmaxf(pm[j], __shfl_xor(pm[j], 32));
            if (q == 0) s_gmax[w][16 * j + c16] = valid ? pm[j] : 0.0f;
        }
        __syncthreads();
        const int MB = (a.M + 15) >> 4, w0 = (w / RT) * RT;
#pragma unroll
        for (int j = 0; j < TB; j++) {
            float gm = s_gmax[w0][16 * j + c16];
#pragma unroll
            for (int k = 1; k < RT; k++) gm = fmaxf(gm, s_gmax[w0 + k][16 * j + c16]);
            const float scale = quant_scale(gm, a.qflavor), inv = quant_inv(scale);
            const int m = m0 + 16 * j + c16;
            if (!valid || m >= a.M) continue;
#pragma unroll
            for (int i = 0; i < TA; i++) {
                const uint32_t b0 = (uint8_t)quant_one(hv[i][j][0], scale, inv, a.qflavor);
                const uint32_t b1 = (uint8_t)quant_one(hv[i][j][1], scale, inv, a.qflavor);
                const int k0 = 8 * (tx * TA + i) + 4 * qq + 2 * half;
                *(uint16_t *)(a.hq + pf_act_off(m, k0, MB)) = (uint16_t)(b0 | (b1 << 8));
            }
            if (w == w0 && q == 0) a.hsc[pf_scale_off(m, (8 * tx * TA) / 32, MB)] = scale;
        }
    }
}

hipError_t launch_pgemm(int wbits, int gs, int sf32, const PgemmArgs &a, hipStream_t st) {
    const TiledMat &W = a.W;
    // rows in whole groups of 4 (float4 outputs), aligned input and output, int4 only with groups of 32
    if (a.M < 1 || W.rows % 4 || W.n % gs || ((uintptr_t)a.xq & 15) || ((uintptr_t)a.xs & 15) ||
        ((uintptr_t)a.y & 15) || W.gs != gs || W.wbits != wbits || W.sf32 != sf32 || (wbits == 4 && gs != 32))
        return hipErrorInvalidValue;
    // buffer loads address the matrix and the input with 31-bit sizes
    if (W.bytes >= ((size_t)1 << 31) || pf_act_bytes(W.n, a.M) >= ((size_t)1 << 31) ||
        pf_scale_floats(W.ng, a.M) * 4 >= ((size_t)1 << 31))
        return hipErrorInvalidValue;
    const int shape = a.shape ? a.shape : pgemm_pick_shape(W.rows, a.M, a.simds);
    const int TA = shape / 10, TB = shape % 10;
    if (a.qkv) {
        // q, k and v rows (NeoX: with the bias, q and k in blocks of 16), shapes 11 and 22
        const int rot = a.dim + a.kv_dim, half = a.head_size / 2;
        if (W.rows != a.dim + 2 * a.kv_dim || a.head_size % 2 || !a.q || !a.kc || !a.vc || !a.rope_cos ||
            !a.rope_sin || a.p0 < 0 || (TA != TB) || (TA != 1 && TA != 2) || a.swiglu ||
            (a.rope_kind == ROPE_NEOX && (!a.bias || rot % 16 || half % 8)) ||
            (a.rope_kind != ROPE_NEOX && a.rope_kind != ROPE_INTERLEAVED))
            return hipErrorInvalidValue;
        const int xt = (W.rows + 16 * TA - 1) / (16 * TA), yt = (a.M + 16 * TB - 1) / (16 * TB);
        const unsigned blocks = (unsigned)(8 * ((xt + 7) / 8) * ((yt + 3) / 4));
#define PGQ(WB_, GS_, SF_, T_)                                                                                 \
        if (wbits == WB_ && gs == GS_ && sf32 == SF_ && TA == T_) {                                           \
            hipLaunchKernelGGL((k_pgemm<WB_, GS_, SF_, T_, T_, 2>), dim3(blocks), dim3(256), 0, st, a);       \
            return hipGetLastError();                                                                         \
        }
        PGQ(4, 32, 0, 1) PGQ(4, 32, 0, 2) PGQ(8, 32, 0, 1) PGQ(8, 32, 0, 2) PGQ(8, 32, 1, 1) PGQ(8, 32, 1, 2)
        PGQ(8, 64, 1, 1) PGQ(8, 64, 1, 2)
#undef PGQ
        return hipErrorInvalidValue;
    }
    if (a.swiglu) {
        // gate/up in row-blocks of 8 + 8, whole quantization groups of 32 hidden values, int4 weights
        if (wbits != 4 || W.rb != 16 || W.rows % 64 || ((uintptr_t)a.hq & 3) || ((uintptr_t)a.hsc & 3) ||
            !a.hq || !a.hsc || (TA != 1 && TA != 2) || (TB != 1 && TB != 2))
            return hipErrorInvalidValue;
        const int RT = 4 / TA, NTY = 4 / RT;
        const int xt = W.rows / (16 * TA), yt = (a.M + 16 * TB - 1) / (16 * TB);
        const unsigned blocks = (unsigned)(8 * ((xt / RT + 7) / 8) * ((yt + NTY - 1) / NTY));
#define PGS(TA_, TB_)                                                                                          \
        if (TA == TA_ && TB == TB_) {                                                                         \
            hipLaunchKernelGGL((k_pgemm<4, 32, 0, TA_, TB_, 1>), dim3(blocks), dim3(256), 0, st, a);         \
            return hipGetLastError();                                                                         \
        }
        PGS(1, 1) PGS(1, 2) PGS(2, 1) PGS(2, 2)
#undef PGS
        return hipErrorInvalidValue;
    }
#define PGW(WB_, GS_, SF_, TA_, TB_)                                                                           \
    if (TA == TA_ && TB == TB_) {                                                                             \
        const int xt = (W.rows + 16 * TA_ - 1) / (16 * TA_), yt = (a.M + 16 * TB_ - 1) / (16 * TB_);          \
        const unsigned blocks = (unsigned)(8 * ((xt + 7) / 8) * ((yt + 3) / 4));                              \
        hipLaunchKernelGGL((k_pgemm<WB_, GS_, SF_, TA_, TB_, 0>), dim3(blocks), dim3(256), 0, st, a);        \
        return hipGetLastError();                                                                             \
    }
#define PG(WB_, GS_, SF_)                                                                                      \
    if (wbits == WB_ && gs == GS_ && sf32 == SF_) {                                                           \
        PGW(WB_, GS_, SF_, 1, 1)                                                                              \
        PGW(WB_, GS_, SF_, 1, 2)                                                                              \
        PGW(WB_, GS_, SF_, 1, 4)                                                                              \
        PGW(WB_, GS_, SF_, 2, 1)                                                                              \
        PGW(WB_, GS_, SF_, 2, 2)                                                                              \
        PGW(WB_, GS_, SF_, 2, 4)                                                                              \
        PGW(WB_, GS_, SF_, 4, 1)                                                                              \
        PGW(WB_, GS_, SF_, 4, 2)                                                                              \
        return hipErrorInvalidValue;                                                                          \
    }
    PG(4, 32, 0)
    PG(8, 32, 0)
    PG(8, 32, 1)
    PG(8, 64, 1)
#undef PG
#undef PGW
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
    extern __shared__ __align__(16) float sv[]; // dim floats + 8, then the strict mode's squares and sum scratch
    const int m = blockIdx.x, n = a.dim, nt = blockDim.x;
    float *x = a.x + (size_t)m * n;
    const float *y = a.y + (size_t)m * n;
    // the first NQ passes' loads (x, y and the gains) are issued before the first store: a store to x could
    // alias y, so a load after it would wait for it; each thread keeps its elements and their order
    constexpr int NQ = 4;
    float xv[NQ], yv[NQ], gv[NQ];
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int i = min(threadIdx.x + k * nt, n - 1);
        xv[k] = x[i];
        if constexpr (RESID) yv[k] = y[i];
        gv[k] = a.norm_w[i];
    }
    float part = 0.0f;
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int i = threadIdx.x + k * nt;
        if (i < n) {
            float v = xv[k];
            if constexpr (RESID) {
                v = v + yv[k];
                x[i] = v;
            }
            sv[i] = v;
            part += v * v;
        }
    }
    for (int i = threadIdx.x + NQ * nt; i < n; i += nt) {
        float v = x[i];
        if constexpr (RESID) {
            v = v + y[i];
            x[i] = v;
        }
        sv[i] = v;
        part += v * v;
    }
    float ss;
    if (a.strict) { // one running sum of the rounded squares in element order (qwen.c:339, runq.c:396-398)
        float *sq = sv + n + 8; // the squares (each rounded, as the reference's), then the sum's scratch
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += nt) sq[i] = sv[i] * sv[i];
        __syncthreads();
        ss = block_seq_sum(sq, n, (uint8_t *)(sq + n));
    } else {
        ss = block_sum(part, sv + n);
    }
    ss /= (float)n;
    ss += a.eps;
    ss = 1.0f / sqrtf(ss);
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int i = threadIdx.x + k * nt;
        if (i < n) sv[i] = gv[k] * (ss * sv[i]);
    }
    for (int i = threadIdx.x + NQ * nt; i < n; i += nt) sv[i] = a.norm_w[i] * (ss * sv[i]);
    __syncthreads();
    block_quantize_tiles(sv, n, a.gs, a.qflavor, a.oq, a.os, m, pf_blocks(a.M));
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
    block_quantize_tiles(sv, hid, a.gs, a.qflavor, a.oq, a.os, m, pf_blocks(a.M));
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
//
// BF (head sizes that are multiples of 32): the same products on `v_mfma_f32_16x16x32_bf16`.  Every fp32 operand
// is split into three bf16 pieces, x = hi + mid + lo exactly (each piece the round-to-nearest of what is left:
// 8 significant bits, |mid| <= 2^-9 |x|, |lo| <= 2^-18 |x|, every remainder exact in fp32), and a product takes
// six piece products (mm, hl, lh, hm, mh, hh: smallest first); the three left out (ml, lm, ll) are below
// 2^-25 of the product, under fp32 rounding.  bf16 products are exact in fp32.  A and B lanes pair the same
// 8 terms (lane group g, slot j), so the layouts are:
//   scores: K rows staged as three bf16 planes [key][HS + 8]; slot j of chunk c is dim g * HS/4 + 8c + j;
//   values: V staged transposed, three planes [dim][PA_KC + 8], keys of a 32-key chunk stored in the order
//     of the probability lanes (slot j < 4: key 4g + j of the chunk's first 16, j >= 4: of its second 16).
typedef __bf16 pa_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pa_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 pa_bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t pa_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t pa_bf2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((pa_f32x2){x, y}, pa_bf16x2));
}
// (x, y) = p[0] + p[1] + p[2], each word a pair of bf16 (x in the low half)
__device__ __forceinline__ void pa_split3(float x, float y, uint32_t *p) {
    p[0] = pa_bf2(x, y);
    const float x1 = x - __uint_as_float(p[0] << 16), y1 = y - __uint_as_float(p[0] & 0xffff0000u);
    p[1] = pa_bf2(x1, y1);
    p[2] = pa_bf2(x1 - __uint_as_float(p[1] << 16), y1 - __uint_as_float(p[1] & 0xffff0000u));
}
__device__ __forceinline__ pa_bf16x8 pa_bf8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(pa_bf16x8, (pa_u32x4){a, b, c, d});
}
// d += A . B over the split operands (pieces h, m, l), smallest products first
__device__ __forceinline__ f32x4v pa_mfma6(const pa_bf16x8 (&A)[3], const pa_bf16x8 (&B)[3], f32x4v d) {
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[1], B[1], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0], B[2], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2], B[0], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0], B[1], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[1], B[0], d, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0], B[0], d, 0, 0, 0);
}
__host__ __device__ constexpr size_t pa_lds_bytes(int hs, int bf) {
    return bf ? (size_t)2 * 3 * ((size_t)pa_kc(hs) * (hs + 8) + (size_t)hs * (pa_kc(hs) + 8))
              : (size_t)2 * pa_kc(hs) * (hs + 4) * 4;
}

template <int HS, int BF>
__global__ void __launch_bounds__(512) k_p_flash(ProwArgs a, int direct) {
    constexpr int H4 = HS / 4, KS = HS + 4, DT = HS / 16, PA_KC = pa_kc(HS);
    constexpr int KSB = HS + 8, VSB = PA_KC + 8, NCH = HS / 32; // BF: plane strides (bf16), dim chunks
    static_assert(!BF || (HS % 32 == 0 && PA_KC % 32 == 0), "split-bf16 products take 32-element chunks");
    extern __shared__ __align__(16) float sm[];
    float *sk = sm, *sv = sm + PA_KC * KS; // [PA_KC][KS] each
    uint16_t *skb = (uint16_t *)sm, *svb = skb + 3 * PA_KC * KSB; // BF: [3][PA_KC][KSB], [3][HS][VSB]
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
    pa_bf16x8 qb[BF ? NCH : 1][3]; // BF: the query's pieces, chunk c slot j = qv[8c + j]
    if constexpr (BF) {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            uint32_t w[4][3];
#pragma unroll
            for (int j = 0; j < 4; j++) pa_split3(qv[8 * c + 2 * j], qv[8 * c + 2 * j + 1], w[j]);
#pragma unroll
            for (int p = 0; p < 3; p++) qb[c][p] = pa_bf8(w[0][p], w[1][p], w[2][p], w[3][p]);
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
            if constexpr (BF) {
                uint32_t k0[3], k1[3], v0[3], v1[3];
                pa_split3(kk.x, kk.y, k0);
                pa_split3(kk.z, kk.w, k1);
                pa_split3(vv.x, vv.y, v0);
                pa_split3(vv.z, vv.w, v1);
                // the key's slot in its 32-key chunk: lane group g = (k % 16) / 4 holds slots 8g .. 8g + 7
                const int kk32 = k & 31, kp = (k & ~31) + ((kk32 & 15) >> 2) * 8 + (kk32 >> 4) * 4 + (kk32 & 3);
#pragma unroll
                for (int p = 0; p < 3; p++) {
                    *(uint2 *)(skb + (p * PA_KC + k) * KSB + 4 * c) = make_uint2(k0[p], k1[p]);
                    uint16_t *vt = svb + (p * HS + 4 * c) * VSB + kp;
                    vt[0] = (uint16_t)v0[p];
                    vt[VSB] = (uint16_t)(v0[p] >> 16);
                    vt[2 * VSB] = (uint16_t)v1[p];
                    vt[3 * VSB] = (uint16_t)(v1[p] >> 16);
                }
            } else {
                *(f32x4v *)(sk + k * KS + 4 * c) = kk;
                *(f32x4v *)(sv + k * KS + 4 * c) = vv;
            }
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
                if constexpr (BF) {
#pragma unroll
                    for (int c = 0; c < NCH; c++) {
                        pa_bf16x8 kb[3];
#pragma unroll
                        for (int p = 0; p < 3; p++)
                            kb[p] = __builtin_bit_cast(
                                pa_bf16x8, *(const pa_u32x4 *)(skb + (p * PA_KC + 16 * kt + r) * KSB + g * H4 + 8 * c));
                        d = pa_mfma6(kb, qb[c], d);
                    }
                } else {
                    const float *kr = sk + (16 * kt + r) * KS + g * H4;
#pragma unroll
                    for (int i = 0; i < H4 / 4; i++) {
                        const f32x4v kk = *(const f32x4v *)(kr + 4 * i);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.x, qv[4 * i], d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.y, qv[4 * i + 1], d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.z, qv[4 * i + 2], d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.w, qv[4 * i + 3], d, 0, 0, 0);
                    }
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
        if constexpr (BF) {
            // chunk ch = tiles 2ch, 2ch + 1 (a tile past ntile has probabilities 0 and finite staged rows)
#pragma unroll
            for (int ch = 0; ch < PA_KC / 32; ch++) {
                if (2 * ch < ntile) {
                    uint32_t w[4][3];
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        pa_split3(sc[2 * ch][2 * j], sc[2 * ch][2 * j + 1], w[j]);
                        pa_split3(sc[2 * ch + 1][2 * j], sc[2 * ch + 1][2 * j + 1], w[2 + j]);
                    }
                    pa_bf16x8 pb[3];
#pragma unroll
                    for (int p = 0; p < 3; p++) pb[p] = pa_bf8(w[0][p], w[1][p], w[2][p], w[3][p]);
#pragma unroll
                    for (int dt = 0; dt < DT; dt++) {
                        pa_bf16x8 vb[3];
#pragma unroll
                        for (int p = 0; p < 3; p++)
                            vb[p] = __builtin_bit_cast(
                                pa_bf16x8, *(const pa_u32x4 *)(svb + (p * HS + 16 * dt + r) * VSB + 32 * ch + 8 * g));
                        o[dt] = pa_mfma6(vb, pb, o[dt]);
                    }
                }
            }
        } else {
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
        const int MB = pf_blocks(a.M), k0 = h * HS + 4 * g; // this lane's elements k0 + 16 dt .. +3
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
                    *(uint32_t *)(a.oq + pf_act_off(m, k0 + 16 * (g0 + k), MB)) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
                }
            if (mine && g == 0) a.os[pf_scale_off(m, (h * HS + 16 * g0) / a.gs, MB)] = scale;
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
    // is waited for.  The value partials of this thread's first MP outputs do not depend on the weights:
    // they are loaded first, together with the statistics (one round trip for a row of up to MP * 256 values).
    constexpr int MP = 4;
    float xp[MP][PREFILL_ATT_SMAX];
#pragma unroll
    for (int p = 0; p < MP; p++) {
        const int o = threadIdx.x + p * blockDim.x;
        if (o < a.dim) {
            const int h = o / hs, e = o - h * hs;
            const float *acc = a.att_acc + ((size_t)m * a.n_heads + h) * a.att_smax * hs + e;
#pragma unroll
            for (int k = 0; k < PREFILL_ATT_SMAX; k++)
                if (k < S) xp[p][k] = acc[(size_t)k * hs];
        }
    }
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
#pragma unroll
    for (int p = 0; p < MP; p++) {
        const int o = threadIdx.x + p * blockDim.x;
        if (o < a.dim) {
            const float *wh = wgt + (o / hs) * a.att_smax;
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < PREFILL_ATT_SMAX; k++)
                if (k < S) v += xp[p][k] * wh[k];
            row[o] = v;
        }
    }
    for (int o = threadIdx.x + MP * blockDim.x; o < a.dim; o += blockDim.x) {
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
    block_quantize_tiles(row, a.dim, a.gs, a.qflavor, a.oq, a.os, m, pf_blocks(a.M));
}

// Reference-order causal attention: block (h, m) is query head h of token m over positions 0 .. p0 + m
// (attn_strict_head); the fp32 output row goes to xb[m], quantized afterwards by k_p_quant_rows.
template <int HS>
__global__ void __launch_bounds__(256) k_p_attn_strict(ProwArgs a) {
    extern __shared__ __align__(16) float sm[];
    const int h = blockIdx.x, m = blockIdx.y, hs = a.head_size, kv_mul = a.n_heads / a.n_kv;
    attn_strict_head<HS>(a.q + (size_t)m * a.dim + (size_t)h * hs, a.kc, a.vc, a.kv_dim, (h / kv_mul) * hs, hs,
                     a.p0 + m + 1, sm, a.xb + (size_t)m * a.dim + (size_t)h * hs);
}

// Strict prefill attention over tiles of tokens (qwen.c:526-546 for each token and head, in the reference's
// order): block = (kv head, G consecutive tokens); its rows are the tokens x the kv head's query heads, so one
// staging of a K or V tile (SPA_T positions, shared by every row) serves G x kv_mul heads.  Each (row,
// position) score is the sequential dot q . k over the head's elements, then / sqrtf(hs), kept in LDS (rows of
// SP floats, the launcher's bound on the positions); the row's maximum; expf(s - max) (ref_expf); the sum in
// position order (one lane per row, all rows of the block in one wave: one wave64 add per position); the
// division; then out[e] accumulated in position order over the V tiles, a (row, element) pair per thread.
#define SPA_T 64 // positions per K/V tile
#define SPA_NS 4 // score chains per thread and tile (rows x SPA_T <= 4 x 256)
__host__ __device__ inline size_t spa_lds_floats(int rows, int hs, int sp) {
    return (size_t)rows * hs + (size_t)rows * sp + (size_t)SPA_T * (hs + 4) + 2 * (size_t)rows;
}
// One tile of G tokens (from m0) of kv head kvh; NV: value chains per thread (rows x hs <= NV x 256).
template <int HS, int NV>
__device__ __forceinline__ void spa_tile(const ProwArgs &a, int G, int SP, int kvh, int m0, float *sm) {
    const int hs = HS ? HS : a.head_size, kv_mul = a.n_heads / a.n_kv;
    const int gn = min(G, a.M - m0), R = gn * kv_mul, Rmax = G * kv_mul;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE, HP = hs + 4, hs4 = hs / 4;
    const int Pmax = a.p0 + m0 + gn; // positions of the tile's last token
    float *qs = sm, *sc = qs + (size_t)Rmax * hs, *kv = sc + (size_t)Rmax * SP, *rmax = kv + SPA_T * HP,
          *rsum = rmax + Rmax;
    const int koff = kvh * hs;
    auto row_pos = [&](int r) { return a.p0 + m0 + r / kv_mul + 1; };          // P of row r
    auto row_head = [&](int r) { return kvh * kv_mul + r % kv_mul; };          // query head of row r
    auto row_tok = [&](int r) { return m0 + r / kv_mul; };                     // token of row r
    __syncthreads(); // a previous tile's rows are consumed
    for (int r = wave; r < R; r += 4)
        for (int c = lane; c < hs4; c += WAVE)
            ((float4 *)(qs + r * hs))[c] = *(const float4 *)(a.q + (size_t)row_tok(r) * a.dim + (size_t)row_head(r) * hs + 4 * c);
    // a K or V tile: positions t0 .. t0 + SPA_T - 1 (below Pmax) of the kv head, rows of hs + 4 floats in LDS;
    // fetch() puts all of a thread's loads (SPA_T x hs / 1024 vectors) in flight at once, put() stores them
    constexpr int FV = (HS ? HS : 256) * SPA_T / 1024; // vectors per thread (hs <= 256)
    // (buffer loads: a position past the range reads zeros through an out-of-range offset, so every load is issued
    // unconditionally and each staging waits for its own tile's loads only)
    const int nrec = (int)(((size_t)(Pmax - 1) * a.kv_dim + hs) * 4);
    const auto rs_k = __builtin_amdgcn_make_buffer_rsrc((void *)(a.kc + koff), 0, nrec, 0x00020000);
    const auto rs_v = __builtin_amdgcn_make_buffer_rsrc((void *)(a.vc + koff), 0, nrec, 0x00020000);
    auto fetch = [&](__amdgpu_buffer_rsrc_t rs, int t0, float4 (&f)[FV]) {
#pragma unroll
        for (int j = 0; j < FV; j++) {
            const int idx = tid + 256 * j, tt = idx / hs4, c = idx - tt * hs4;
            const bool ok = tt < SPA_T && t0 + tt < Pmax;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(
                rs, ok ? (uint32_t)((t0 + tt) * a.kv_dim + 4 * c) * 4u : 0x80000000u, 0, 0);
            f[j] = *(const float4 *)&v;
        }
    };
    auto put = [&](const float4 (&f)[FV]) {
#pragma unroll
        for (int j = 0; j < FV; j++) {
            const int idx = tid + 256 * j, tt = idx / hs4, c = idx - tt * hs4;
            if (HS || tt < SPA_T) *(float4 *)(kv + tt * HP + 4 * c) = f[j]; // (a fixed head size fills FV exactly)
        }
    };
    // DK tiles in flight: a tile's compute is shorter than a round trip to the cache, so the loads of the tiles
    // DK ahead leave as each tile is staged (register sets used in turn, the tile loop unrolled by DK)
    constexpr int DK = (HS && HS <= 64) ? 4 : 2;
    float4 fr[DK][FV];
    const int nkt = (Pmax + SPA_T - 1) / SPA_T;
    KERNEL_MARK(0);
    const float rs = sqrtf((float)hs);
    // (1) scores: thread tid takes position tt = tid % 64 of the tile for rows tid / 64 + 4 j (j < SPA_NS), its
    // K row read once per 4 elements for all of them; each score the sequential dot over the head's elements
    const int s_tt = tid % SPA_T, s_r0 = tid / SPA_T;
#pragma unroll
    for (int dd = 0; dd < DK; dd++) fetch(rs_k, dd * SPA_T, fr[dd]); // (tiles past the range: zeros, no traffic)
    for (int k0 = 0; k0 < nkt; k0 += DK)
#pragma unroll
    for (int dd = 0; dd < DK; dd++) {
        const int kt = k0 + dd, t0 = kt * SPA_T;
        if (kt >= nkt) break;
        __syncthreads(); // the previous tile is consumed
        put(fr[dd]);
        __syncthreads();
        fetch(rs_k, (kt + DK) * SPA_T, fr[dd]);
        float d[SPA_NS];
#pragma unroll
        for (int j = 0; j < SPA_NS; j++) d[j] = 0.0f;
        const float4 *kr = (const float4 *)(kv + s_tt * HP);
        const float4 *qr[SPA_NS];
#pragma unroll
        for (int j = 0; j < SPA_NS; j++) qr[j] = (const float4 *)(qs + min(s_r0 + 4 * j, Rmax - 1) * hs);
#pragma unroll 4
        for (int c = 0; c < hs4; c++) {
            const float4 k4 = kr[c];
#pragma unroll
            for (int j = 0; j < SPA_NS; j++) {
                const float4 q4 = qr[j][c];
                d[j] += q4.x * k4.x;
                d[j] += q4.y * k4.y;
                d[j] += q4.z * k4.z;
                d[j] += q4.w * k4.w;
            }
        }
        const int t = t0 + s_tt;
#pragma unroll
        for (int j = 0; j < SPA_NS; j++) {
            const int r = s_r0 + 4 * j;
            if (r < R && t < row_pos(r)) sc[(size_t)r * SP + t] = d[j] / rs;
        }
    }
    __syncthreads();
    KERNEL_MARK(1);
    // (2) a wave per row: its maximum, then its exponentials (positions past the row, up to the tile's last
    // token's, set to 0: the sums below then add +0 there, which leaves a positive sum unchanged)
    for (int r = wave; r < R; r += 4) {
        float *row = sc + (size_t)r * SP;
        const int P = row_pos(r);
        float mx = -INFINITY;
        for (int t = lane; t < P; t += WAVE) mx = fmaxf(mx, row[t]);
        mx = wave_max(mx);
        for (int t = lane; t < Pmax; t += WAVE) row[t] = t < P ? ref_expf(row[t] - mx) : 0.0f;
    }
    __syncthreads();
    KERNEL_MARK(2);
    // (3) the sums in position order: lane r of wave 0 adds row r, 8 positions in flight
    if (wave == 0 && lane < R) {
        const float *row = sc + (size_t)lane * SP;
        const float4 *row4 = (const float4 *)row;
        float s = 0.0f;
        int t = 0;
        for (; t + 8 <= Pmax; t += 8) {
            const float4 v0 = row4[t / 4], v1 = row4[t / 4 + 1];
            s = s + v0.x;
            s = s + v0.y;
            s = s + v0.z;
            s = s + v0.w;
            s = s + v1.x;
            s = s + v1.y;
            s = s + v1.z;
            s = s + v1.w;
        }
        for (; t < Pmax; t++) s = s + row[t];
        rsum[lane] = s;
    }
    __syncthreads();
    KERNEL_MARK(3);
    // the probabilities (0 stays 0 past the row: the value sums add +0 there)
    for (int r = wave; r < R; r += 4) {
        float *row = sc + (size_t)r * SP;
        const float sum = rsum[r];
        for (int t = lane; t < Pmax; t += WAVE) row[t] = row[t] / sum;
    }
    KERNEL_MARK(4);
    // (4) values: thread tid takes element e = tid % hs of rows tid / hs + (256 / hs) j, the V element read once
    // per position for all of them; positions in order over the tiles
    const int v_e = tid % hs, v_r0 = tid / hs, v_rs = 256 / hs;
    float acc[NV];
    const float *pr[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        acc[j] = 0.0f;
        pr[j] = sc + (size_t)min(v_r0 + v_rs * j, Rmax - 1) * SP;
    }
#pragma unroll
    for (int dd = 0; dd < DK; dd++) fetch(rs_v, dd * SPA_T, fr[dd]);
    for (int k0 = 0; k0 < nkt; k0 += DK)
#pragma unroll
    for (int dd = 0; dd < DK; dd++) {
        const int kt = k0 + dd, t0 = kt * SPA_T;
        if (kt >= nkt) break;
        __syncthreads(); // the probabilities are written, the previous tile consumed
        put(fr[dd]);
        __syncthreads();
        fetch(rs_v, (kt + DK) * SPA_T, fr[dd]);
        const int T = min(SPA_T, Pmax - t0);
        const float *vt = kv + v_e;
        int tt = 0;
        // 4 positions a step: each row's 4 weights in one load (rows and t0 are 16-byte aligned), then the
        // products and adds position by position; a full tile as straight-line code (the loads of later steps
        // scheduled ahead of earlier steps' arithmetic)
        auto step4 = [&](int s) {
            const float v0 = vt[s * HP], v1 = vt[(s + 1) * HP], v2 = vt[(s + 2) * HP], v3 = vt[(s + 3) * HP];
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const float4 w = *(const float4 *)(pr[j] + t0 + s);
                acc[j] += w.x * v0;
                acc[j] += w.y * v1;
                acc[j] += w.z * v2;
                acc[j] += w.w * v3;
            }
        };
        if (T == SPA_T) {
#pragma unroll
            for (int s = 0; s < SPA_T; s += 4) step4(s);
            tt = SPA_T;
        }
        for (; tt + 4 <= T; tt += 4) {
            const float v0 = vt[tt * HP], v1 = vt[(tt + 1) * HP], v2 = vt[(tt + 2) * HP], v3 = vt[(tt + 3) * HP];
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const float4 w = *(const float4 *)(pr[j] + t0 + tt);
                acc[j] += w.x * v0;
                acc[j] += w.y * v1;
                acc[j] += w.z * v2;
                acc[j] += w.w * v3;
            }
        }
        for (; tt < T; tt++) {
            const float v = vt[tt * HP];
#pragma unroll
            for (int j = 0; j < NV; j++) acc[j] += pr[j][t0 + tt] * v;
        }
    }
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int r = v_r0 + v_rs * j;
        if (r < R) a.xb[(size_t)row_tok(r) * a.dim + (size_t)row_head(r) * hs + v_e] = acc[j];
    }
    KERNEL_MARK(5);
}

// Strict prefill attention over tiles of tokens (qwen.c:526-546 for each token and head, in the reference's
// order): a tile = G consecutive tokens of one kv head; its rows are the tokens x the kv head's query heads, so
// one staging of a K or V tile (SPA_T positions, shared by every row) serves G x kv_mul heads.  Each (row,
// position) score is the sequential dot q . k over the head's elements, then / sqrtf(hs), kept in LDS (rows of
// SP floats, the launcher's bound on the positions); the row's maximum; expf(s - max) (ref_expf); the sum in
// position order (one lane per row, every row of the tile in one wave: one wave64 add per position); the
// division; then out[e] accumulated in position order over the V tiles, (row, element) chains per thread.
// One tile per block, the longest causal ranges first (two blocks per CU at 512 tokens; pairing a short and a
// long range in one block, every block the same work, measured 6% slower: fewer waves in flight per CU).
template <int HS, int NV>
__global__ void __launch_bounds__(256) k_p_attn_strict_rows(ProwArgs a, int G, int SP) {
    extern __shared__ __align__(16) float sm[];
    const int ntiles = (a.M + G - 1) / G, y = ntiles - 1 - (int)blockIdx.y;
    spa_tile<HS, NV>(a, G, SP, blockIdx.x, y * G, sm);
}

// int8 quantization of the rows xb[m] (qwen.c:549, runq.c:571) into the o projection's input
__global__ void __launch_bounds__(256) k_p_quant_rows(ProwArgs a) {
    extern __shared__ __align__(16) float sv[];
    const int m = blockIdx.x, n = a.dim;
    for (int i = threadIdx.x; i < n; i += blockDim.x) sv[i] = a.xb[(size_t)m * n + i];
    __syncthreads();
    block_quantize_tiles(sv, n, a.gs, a.qflavor, a.oq, a.os, m, pf_blocks(a.M));
}

hipError_t launch_p_embed(const ProwArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(k_p_embed, dim3(a.M), dim3(256), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_p_norm_quant(const ProwArgs &a, bool resid, hipStream_t st) {
    if (a.dim % 4 || ((uintptr_t)a.oq & 3)) return hipErrorInvalidValue;
    // dim floats, 8 for the block sum, then the strict mode's squares and sequential sum's scratch
    const size_t lds = (size_t)(a.dim + 8) * 4 + (a.strict ? (size_t)a.dim * 4 + seq_sum_scratch_bytes(256) : 0);
    if (resid) hipLaunchKernelGGL(k_p_norm_quant<true>, dim3(a.M), dim3(256), lds, st, a);
    else hipLaunchKernelGGL(k_p_norm_quant<false>, dim3(a.M), dim3(256), lds, st, a);
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
        // (the K and V reads go through buffer resources: a layer's cache stays below 2 GiB)
        if (hs % 4 || hs > 256 || ((uintptr_t)a.kc & 15) || a.kv_dim % 4 || a.dim % 4 || a.dim % a.gs || !a.xb ||
            ((uintptr_t)a.oq & 3) || lds > 65536 || a.n_heads % a.n_kv ||
            (size_t)(a.p0 + a.M + 64) * a.kv_dim * 4 >= 0x7fffffffu)
            return hipErrorInvalidValue;
        // tiles of G tokens when their rows' scores fit LDS (G x kv_mul rows, positions up to p0 + M), else a
        // block per (head, token) that streams the positions
        // score rows of SP = 4 x odd floats: 16-byte aligned (the value chains read 4 weights a load) and the sums'
        // lanes, one per row, on distinct banks
        const int kvm = a.n_heads / a.n_kv, SP = 4 * (((a.p0 + a.M + 3) / 4) | 1);
        int G = 0;
        for (int g = 4; g >= 1 && !G; g /= 2)
            if (g * kvm <= 4 * SPA_NS && g * kvm * hs <= 8 * 256 && hs <= 256 && 256 % hs == 0 &&
                spa_lds_floats(g * kvm, hs, SP) * 4 <= 65536)
                G = g;
        if (G) {
            const int ntiles = (a.M + G - 1) / G;
            const dim3 grid(a.n_kv, ntiles);
            const size_t sl = spa_lds_floats(G * kvm, hs, SP) * 4;
            const bool nv4 = G * kvm * hs <= 4 * 256;
#define SPA_LAUNCH(H)                                                                                          \
            if (nv4) hipLaunchKernelGGL((k_p_attn_strict_rows<H, 4>), grid, dim3(256), sl, st, a, G, SP);      \
            else hipLaunchKernelGGL((k_p_attn_strict_rows<H, 8>), grid, dim3(256), sl, st, a, G, SP);
            if (hs == 64) {
                SPA_LAUNCH(64)
            } else if (hs == 128) {
                SPA_LAUNCH(128)
            } else {
                SPA_LAUNCH(0)
            }
#undef SPA_LAUNCH
        } else if (hs == 64) hipLaunchKernelGGL(k_p_attn_strict<64>, dim3(a.n_heads, a.M), dim3(256), lds, st, a);
        else if (hs == 128) hipLaunchKernelGGL(k_p_attn_strict<128>, dim3(a.n_heads, a.M), dim3(256), lds, st, a);
        else hipLaunchKernelGGL(k_p_attn_strict<0>, dim3(a.n_heads, a.M), dim3(256), lds, st, a);
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
        const int bf = a.flash_bf && hs % 32 == 0;
        void (*kern)(ProwArgs, int) = nullptr;
        if (bf) kern = hs == 32 ? k_p_flash<32, 1> : hs == 64 ? k_p_flash<64, 1> : k_p_flash<128, 1>;
        else kern = hs == 16 ? k_p_flash<16, 0> : hs == 32 ? k_p_flash<32, 0> : hs == 48 ? k_p_flash<48, 0>
                  : hs == 64 ? k_p_flash<64, 0> : k_p_flash<128, 0>;
        hipLaunchKernelGGL(kern, grid, dim3(64 * kv_mul), pa_lds_bytes(hs, bf), st, a, direct);
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
