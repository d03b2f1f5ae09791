// Batched prompt processing (prefill) kernels of libmatvec_hip.so (internal header).
//
// The prompt's M positions go through each layer together: per-token RMSNorm + int8 quantization, an int8
// MFMA GEMM over the same tiled weights the decode GEMV reads, per-token epilogues and causal attention over
// the KV cache.  fp32 activation matrices are row-major, [M][width]; the GEMM's int8 input is in token-block
// tiles (pf_act_off below).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tiled.h"

// The int8 GEMM input of M tokens x n elements in token-block tiles, laid out so that every load of the GEMM
// moves 16 bytes per lane.  Elements come in chunks of 32 (k / 32) and tokens in blocks of 16 (MB = ceil(M /
// 16) blocks; the tokens past M in the last block are never written and only reach outputs that are not
// stored).  One 1 KiB block holds a pair of chunks for a token block: lane l = 16 j + t (token t of the
// block) has 16 bytes, 8 per chunk of the pair: elements 4 j .. 4 j + 3 and 16 + 4 j .. 16 + 4 j + 3 of the
// chunk, the K slice that lane row j of a v_mfma_i32_16x16x32_i8 B operand takes here (the GEMM gives its A
// operand the same slice).  Blocks are ordered [chunk pair][token block].  The fp32 group scales come as a
// float4 per token and 4 groups: [group / 4][16 MB tokens][group % 4].
__host__ __device__ inline size_t pf_act_off(int m, int k, int MB) {
    const int c = k >> 5, e = k & 31;
    return ((size_t)(c >> 1) * MB + (m >> 4)) * 1024 + 16 * (16 * ((e & 15) >> 2) + (m & 15)) + 8 * (c & 1) +
           4 * (e >> 4) + (e & 3);
}
__host__ __device__ inline size_t pf_scale_off(int m, int g, int MB) {
    return ((size_t)(g >> 2) * MB * 16 + m) * 4 + (g & 3);
}
__host__ __device__ inline int pf_blocks(int M) { return (M + 15) / 16; }
// bytes of the int8 input of n elements (whole chunk pairs) and floats of its scales (whole group quads)
__host__ __device__ inline size_t pf_act_bytes(int n, int M) { return (size_t)((n / 32 + 1) / 2) * pf_blocks(M) * 1024; }
__host__ __device__ inline size_t pf_scale_floats(int ng, int M) { return (size_t)((ng + 3) / 4) * pf_blocks(M) * 64; }

struct PgemmArgs {
    TiledMat W;             // d = W.rows output columns, n = W.n inputs
    const int8_t *xq;       // token-block tiles (pf_act_off), pf_act_bytes(n, M)
    const float *xs;        // their scales (pf_scale_off), pf_scale_floats(n / gs, M)
    float *y;               // [M][d]
    int M;
    int shape;              // 0: pgemm_pick_shape; 10 TA + TB: one wave per 16 TA rows x 16 TB tokens
                            // (TA 1, 2, 4; TB 1, 2, 4; not 44)
    int simds;              // SIMDs of the device (0: 1024)
    // swiglu = 1: W is the gate/up matrix (row-blocks of 16: 8 gate rows, then the 8 matching up rows) and the
    // epilogue writes h = silu(gate) * up quantized (groups of 32, flavour qflavor; strict: the reference
    // libm's expf) into the token-block tiles hq / hsc instead of y (int4 weights, shapes 11, 12, 21, 22)
    int swiglu, qflavor, strict;
    int8_t *hq;             // pf_act_bytes(rows / 2, M); must not alias xq
    float *hsc;             // pf_scale_floats(rows / 64, M)
    // qkv = 1: W is the fused QKV matrix (rows of q, then k, then v; NeoX: q and k in blocks of 16, 8 rows and
    // their 8 RoPE partners) and the epilogue does k_p_qkv's work with the rows instead of storing y: bias,
    // RoPE at position p0 + m, q rows to q [M][dim], K and V rows to the layer's caches (shapes 11 and 22)
    int qkv;
    const float *bias;      // [dim + 2 kv_dim] (NeoX) or NULL (interleaved pairs)
    const float *rope_cos, *rope_sin; // [ctx][head_size / 2]
    float *q, *kc, *vc;
    int p0, dim, kv_dim, head_size, rope_kind;
};

// Tile shape of the prefill GEMM for d output rows and M tokens on a device of `simds` SIMDs.  The smallest
// tile (16 x 16) needs the most instructions per output but gives the most waves; 32 x 32 tiles pay off once
// they still give every SIMD 4 waves (measured on the 512-token Qwen2-0.5B-shape GEMMs: 32 x 32 for the
// 9728-row gate/up, 16 x 16 for QKV, o and down).
static inline int pgemm_pick_shape(int d, int M, int simds) {
    if (simds <= 0) simds = 1024;
    const long waves22 = (long)((d + 31) / 32) * ((M + 31) / 32);
    return waves22 >= 4L * simds ? 22 : 11;
}

struct ProwArgs {           // per-token elementwise kernels
    int M, p0;              // tokens, position of the first one
    int dim, kv_dim, head_size, hidden, gs, qflavor, rope_kind, gu_rb;
    float eps;
    const int *ids;         // [M] token ids (embedding)
    const int8_t *emb_q;    // embedding table
    const void *emb_s;
    int emb_sf32;
    float *x;               // [M][dim] residual stream
    const float *norm_w;    // [dim]
    const float *y;         // [M][rows] GEMM output
    const float *bias;      // [dim + 2 kv] or NULL
    const float *rope_cos, *rope_sin; // [ctx][hs/2]
    float *q;               // [M][dim]
    float *kc, *vc;         // this layer's caches [ctx][kv_dim]
    int8_t *oq;             // quantized output (the next GEMM's input), token-block tiles (pf_act_off)
    float *os;              // its scales (pf_scale_off)
    int n_heads, n_kv;
    int strict;             // 1: reference order (sequential RMSNorm sum, reference-order attention, libm expf)
    float *xb;              // strict attention: [M][dim] output rows before quantization
    // attention slices: positions of token m in slices of att_sl, at most att_smax per token; partials
    // ml [M][n_heads][att_smax][2] (max, sum of exp) and acc [M][n_heads][att_smax][hs]
    int att_sl, att_smax;
    float *att_ml, *att_acc;
    int flash_bf;           // 1: the slice kernel's products on bf16 MFMA over split operands (head sizes % 32 == 0)
};

// Slices of at least 64 positions, at most 16 per token for a chunk ending at position `end`.
static inline void prefill_att_slices(int end, int *sl, int *smax) {
    int s = (end + 15) / 16;
    if (s < 64) s = 64;
    s = (s + 31) / 32 * 32;
    *sl = s;
    *smax = (end + s - 1) / s;
}
#define PREFILL_ATT_SMAX 16

hipError_t launch_pgemm(int wbits, int gs, int sf32, const PgemmArgs &a, hipStream_t st);
hipError_t launch_p_embed(const ProwArgs &a, hipStream_t st);
hipError_t launch_p_norm_quant(const ProwArgs &a, bool resid, hipStream_t st); // resid: x += y first
hipError_t launch_p_qkv(const ProwArgs &a, hipStream_t st);
hipError_t launch_p_resid(const ProwArgs &a, hipStream_t st);
hipError_t launch_p_swiglu_quant(const ProwArgs &a, hipStream_t st);
hipError_t launch_p_attention(const ProwArgs &a, hipStream_t st); // slices, merge; int8 output in oq/os
