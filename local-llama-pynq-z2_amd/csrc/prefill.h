// Batched prompt processing (prefill) kernels of libmatvec_hip.so (internal header).
//
// The prompt's M positions go through each layer together: per-token RMSNorm + int8 quantization, an int8
// MFMA GEMM over the same tiled weights the decode GEMV reads, per-token epilogues and causal attention over
// the KV cache.  Row-major activation matrices: [M][width].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tiled.h"

struct PgemmArgs {
    TiledMat W;             // d = W.rows output columns, n = W.n inputs
    const int8_t *xq;       // [M][n]
    const float *xs;        // [M][n / gs]
    float *y;               // [M][d]
    int M;
};

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
    int8_t *oq;             // [M][width] quantized output (the next GEMM's input)
    float *os;              // [M][width / gs]
    int n_heads, n_kv;
    int strict;             // 1: reference order (sequential RMSNorm sum, reference-order attention, libm expf)
    float *xb;              // strict attention: [M][dim] output rows before quantization
    // attention slices: positions of token m in slices of att_sl, at most att_smax per token; partials
    // ml [M][n_heads][att_smax][2] (max, sum of exp) and acc [M][n_heads][att_smax][hs]
    int att_sl, att_smax;
    float *att_ml, *att_acc;
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
