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

// Deterministic block-wide sum (fixed order: lanes in a butterfly, then waves in index order).
// `scratch` needs one float per wave.  Every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float *scratch) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
    v = wave_sum_from(v, 1);
    __syncthreads();
    if (lane == 0) scratch[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += scratch[i];
    return t;
}

// Quantize n floats held in LDS (`v`) into int8 `q` and fp32 scales `s` (LDS or global), groups of gs
// (32 or 64), by the whole block: a group of gs lanes per group, max by butterfly (exact in any order).
__device__ __forceinline__ void block_quantize(const float *v, int n, int gs, int flavor, int8_t *q, float *s) {
    const int gpp = blockDim.x / gs; // groups per pass
    const int ng = n / gs;
    const int my = threadIdx.x / gs, e = threadIdx.x % gs;
    for (int g0 = 0; g0 < ng; g0 += gpp) {
        const int g = g0 + my;
        float x = (my < gpp && g < ng) ? v[g * gs + e] : 0.0f;
        float m = group_max(fabsf(x), gs);
        if (my < gpp && g < ng) {
            float scale = quant_scale(m, flavor), inv = quant_inv(scale);
            q[g * gs + e] = quant_one(x, scale, inv, flavor);
            if (e == 0) s[g] = scale;
        }
    }
}
