// Tiled weight layout of the GEMV kernels (host and device).
//
// The reference keeps a matrix as a row-major weight plane plus a scale plane (qwen.c:44-47, runq.c:38-44).
// At upload the library repacks each matrix (or a stack of matrices fused into one launch) into chunk
// records that one wavefront reads with fully coalesced 16-byte loads:
//
//   row-block b = RB consecutive logical rows; chunk c = the next 64/RB groups of those rows;
//   record(b, c) = [piece p][lane l][16 B] weights (SB/16 pieces), then [lane l] scales (2 or 4 B);
//   lane l holds row b*RB + l%RB, group c*(64/RB) + l/RB.
//
// SB = bytes of one (row, group) segment: 16 for int4 x 32, 32 for int8 x 32, 64 for int8 x 64.  One wave
// load instruction therefore reads 1 KiB of contiguous weights, and its scale load 128 or 256 contiguous
// bytes.  Rows past the matrix and groups past the row are zero (weights and scales), so they add 0.
// int4 segments are also reordered inside: dword j holds elements 4j..4j+3 in its low nibbles and
// 16+4j..16+4j+3 in its high nibbles, so both halves line up with the natural int8 activation dwords.
#pragma once
#include <stddef.h>
#include <stdint.h>

// Activation quantization flavours: the two reference quantize() functions (qwen.c:354-364, runq.c:244-270).
enum { QF_QWEN = 0, QF_RUNQ = 1 };

struct TiledMat {
    const uint8_t *data; // device
    int rows;            // logical rows (all fused matrices)
    int n;               // input length
    int ng;              // groups per row (n / gs)
    int gs;              // 32 or 64
    int wbits;           // 4 or 8
    int sf32;            // scales: 0 fp16, 1 fp32
    int rb;              // rows per row-block: 8, 16, 32 or 64
    int nchunks;         // chunks per row-block
    int nblocks;         // row-blocks
    size_t rec;          // bytes per chunk record
    size_t bytes;        // total
};

static inline int tiled_seg_bytes(int wbits, int gs) { return gs * wbits / 8; }

static inline TiledMat tiled_describe(int rows, int n, int gs, int wbits, int sf32, int rb) {
    TiledMat t;
    t.data = 0;
    t.rows = rows;
    t.n = n;
    t.gs = gs;
    t.ng = n / gs;
    t.wbits = wbits;
    t.sf32 = sf32;
    t.rb = rb;
    const int gpc = 64 / rb;
    t.nchunks = (t.ng + gpc - 1) / gpc;
    t.nblocks = (rows + rb - 1) / rb;
    t.rec = (size_t)64 * tiled_seg_bytes(wbits, gs) + (size_t)64 * (sf32 ? 4 : 2);
    t.bytes = t.rec * (size_t)t.nchunks * (size_t)t.nblocks;
    return t;
}

// Algorithmic bytes of one GEMV over d rows x n inputs: weights, scales, int8 activations with their fp32
// scales, fp32 outputs (the per-call figure B of the bandwidth roofline).
static inline double gemv_algo_bytes(double d, double n, int wbits, int gs, int sf32) {
    return d * n * wbits / 8.0 + d * (n / gs) * (sf32 ? 4.0 : 2.0) + n + (n / gs) * 4.0 + d * 4.0;
}
