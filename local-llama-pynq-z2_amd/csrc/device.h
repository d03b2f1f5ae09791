// Device helpers shared by every kernel of libmatvec_hip.so (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "tiled.h"

#define WAVE 64


// fp16 bits -> fp32 with the hardware conversion (v_cvt_f32_f16); exact for zero, subnormals and normals,
// which is what qwen.c:84-94 computes for every scale a valid file can hold.
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// What the reference's (int8_t)roundf(v) gives on x86-64: cvttss2si to int32 (NaN and |v| >= 2^31 become
// 0x80000000), then the low byte.  Spelled out because the GPU's own conversion saturates instead.
__device__ __forceinline__ int8_t x86_round_to_i8(float r) {
    if (!(fabsf(r) < 2147483648.0f)) return 0;
    return (int8_t)(uint8_t)((uint32_t)(int32_t)r & 0xffu);
}

// Scale of one group from its max |x|, and the quantized value of one element, in each flavour:
//   qwen (qwen.c:359-362): scale = wmax * (1/127), inv = scale > 0 ? 1/scale : 0, q = roundf(x * inv)
//   runq (runq.c:260-266): scale = wmax / 127,     q = round(x / scale)
// Division is IEEE (the library is built without fast-math) and nothing is contracted into an FMA.
__device__ __forceinline__ float quant_scale(float wmax, int flavor) {
    return flavor == QF_QWEN ? wmax * (1.0f / 127.0f) : wmax / 127.0f;
}
__device__ __forceinline__ float quant_inv(float scale) { return scale > 0.0f ? 1.0f / scale : 0.0f; }
__device__ __forceinline__ int8_t quant_one(float x, float scale, float inv, int flavor) {
    if (flavor == QF_QWEN) return x86_round_to_i8(roundf(x * inv));
    return x86_round_to_i8(roundf(x / scale));
}

// Butterfly sum / max over the lanes of a wave that differ only in the bits of [lo, 64).
__device__ __forceinline__ float wave_sum_from(float v, int lo) {
    for (int off = lo; off < WAVE; off <<= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float group_max(float v, int width) { // max over aligned groups of `width` lanes
    for (int off = width >> 1; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Value of another lane of the same row of 16 lanes through a DPP operand (no LDS round trip).  CTRL is
// the gfx9 DPP control: 0xB1 = lane ^ 1, 0x4E = lane ^ 2 (quad permutes), 0x141 = 7 - lane within each 8
// (half-row mirror), 0x140 = 15 - lane within the row (row mirror).  Call with the whole wave active.
template <int CTRL>
__device__ __forceinline__ float dpp_get(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Max over aligned groups of 8 (or 16) lanes.  Max is exact, so the mirrors pair lanes as well as a
// butterfly would: after the quad steps every lane holds its quad's max, and lane i with lane 7 - i (15 - i)
// joins two quads (two eights).
__device__ __forceinline__ float max8(float m) {
    m = fmaxf(m, dpp_get<0xB1>(m));
    m = fmaxf(m, dpp_get<0x4E>(m));
    return fmaxf(m, dpp_get<0x141>(m));
}
__device__ __forceinline__ float max16(float m) {
    m = max8(m);
    return fmaxf(m, dpp_get<0x140>(m));
}
// Max over the whole wave (every lane gets it).
__device__ __forceinline__ float wave_max(float m) {
    m = max16(m);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Sum of a whole wave in a fixed order: pairs, quads, eights and rows of 16 by DPP, then the four row sums
// as (row0 + row1) + (row2 + row3).  Every lane gets the result.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_get<0xB1>(v);
    v += dpp_get<0x4E>(v);
    v += dpp_get<0x141>(v);
    v += dpp_get<0x140>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Deterministic block-wide sum (fixed order: wave_sum, then waves in index order).  `scratch` needs one
// float per wave and must not be read by anyone else at the time of the call.  Every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float *scratch) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
    v = wave_sum(v);
    if (lane == 0) scratch[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += scratch[i];
    return t;
}

// s + t[16 - r] + ... + t[15] in that order, r in [0, 16): one jump into a run of adds (the last terms of a sum
// arrive loaded together as the final 16 of the range, instead of one load and add after another).
__device__ __forceinline__ float seq_add_tail(float s, const float (&t)[16], int r) {
    switch (r) {
    case 15: s = s + t[1]; [[fallthrough]];
    case 14: s = s + t[2]; [[fallthrough]];
    case 13: s = s + t[3]; [[fallthrough]];
    case 12: s = s + t[4]; [[fallthrough]];
    case 11: s = s + t[5]; [[fallthrough]];
    case 10: s = s + t[6]; [[fallthrough]];
    case 9: s = s + t[7]; [[fallthrough]];
    case 8: s = s + t[8]; [[fallthrough]];
    case 7: s = s + t[9]; [[fallthrough]];
    case 6: s = s + t[10]; [[fallthrough]];
    case 5: s = s + t[11]; [[fallthrough]];
    case 4: s = s + t[12]; [[fallthrough]];
    case 3: s = s + t[13]; [[fallthrough]];
    case 2: s = s + t[14]; [[fallthrough]];
    case 1: s = s + t[15]; [[fallthrough]];
    default: break;
    }
    return s;
}

// Sum of n floats in index order (one thread; p in LDS, any alignment): the reads of the next 16 values are
// issued before the current 16 are added, and the last n % 16 are read together and entered by seq_add_tail;
// 17 to 31 values are read in one round, both batches at once (sums of fewer than 16 values: one read and add
// after another).
__device__ __forceinline__ float seq_sum(const float *p, int n) {
    float v = 0.0f;
    int g = 0;
    if (n > 16 && n < 32) { // both batches read at once: the first 16 values and the last 16
        const float *b = p + (n - 16);
        float t0[16], t[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            t0[u] = p[u];
            t[u] = b[u];
        }
#pragma unroll
        for (int u = 0; u < 16; u++) v += t0[u];
        return seq_add_tail(v, t, n - 16);
    }
    if (n >= 16) {
        float cur[16], nxt[16];
#pragma unroll
        for (int u = 0; u < 16; u++) cur[u] = p[u];
        for (; g + 16 <= n; g += 16) {
            const int gn = min(g + 16, n - 16);
#pragma unroll
            for (int u = 0; u < 16; u++) nxt[u] = p[gn + u];
#pragma unroll
            for (int u = 0; u < 16; u++) v += cur[u];
#pragma unroll
            for (int u = 0; u < 16; u++) cur[u] = nxt[u];
        }
    }
    if (g < n && n >= 16) {
        // the final 16 values from one base address (immediate offsets: no per-value address registers kept
        // live across a caller's loop)
        const float *b = p + (n - 16);
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; u++) t[u] = b[u];
        v = seq_add_tail(v, t, n - g);
    } else {
        for (; g < n; g++) v += p[g];
    }
    return v;
}

// The int8 codes of 4 consecutive values x of a group of gs values (32 or 64) spread over gs/4 lanes of one
// DPP row, packed little-endian, and the group's scale.  Every lane of the wave calls it (the group max is
// max8 / max16 across lanes).
__device__ __forceinline__ uint32_t quantize_pack(float4 x, int gs, int flavor, float *scale_out) {
    float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
    m = gs == 64 ? max16(m) : max8(m);
    const float scale = quant_scale(m, flavor), inv = quant_inv(scale);
    const uint32_t b0 = (uint8_t)quant_one(x.x, scale, inv, flavor);
    const uint32_t b1 = (uint8_t)quant_one(x.y, scale, inv, flavor);
    const uint32_t b2 = (uint8_t)quant_one(x.z, scale, inv, flavor);
    const uint32_t b3 = (uint8_t)quant_one(x.w, scale, inv, flavor);
    *scale_out = scale;
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// Quantize the 4 consecutive values x of vector slot i (group of gs values = gs/4 lanes of one DPP row; every
// lane of the wave calls it, `ok` marks the lanes whose slot exists, whole groups are in or out).
__device__ __forceinline__ void quantize_slot(float4 x, int i, bool ok, int gs, int flavor, int8_t *q, float *s) {
    float scale;
    const uint32_t packed = quantize_pack(x, gs, flavor, &scale);
    if (ok) {
        ((uint32_t *)q)[i] = packed;
        if ((i & (gs / 4 - 1)) == 0) s[i / (gs / 4)] = scale;
    }
}

// Quantize n floats held in LDS (`v`, 16-byte aligned) into int8 `q` (4-byte aligned) and fp32 scales `s`
// (LDS or global), groups of gs (32 or 64; n a multiple of gs), by the whole block.  Each lane takes 4
// consecutive values, so a group is gs/4 = 8 or 16 lanes of one DPP row and its max is max8 / max16.

__device__ __forceinline__ void block_quantize(const float *v, int n, int gs, int flavor, int8_t *q, float *s) {
    const int nq = n / 4;
    for (int i0 = 0; i0 < nq; i0 += blockDim.x) {
        const int i = i0 + threadIdx.x;
        const bool ok = i < nq; // whole groups are in or out: nq is a multiple of gs / 4
        quantize_slot(((const float4 *)v)[ok ? i : 0], i, ok, gs, flavor, q, s);
    }
}
