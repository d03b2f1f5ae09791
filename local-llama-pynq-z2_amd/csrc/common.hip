// Launch-shape choice for the GEMV kernels and the bounded stream wait (internal).
#include <time.h>

#include <algorithm>

#include "host_common.h"

// Shapes follow from the tiled matrix: a row-block has `nchunks` chunk records of 1 KiB+ each; its chunks are
// split over kw waves, and an iteration is nb row-blocks.  Epilogues that need whole groups of rows fix nb:
// SwiGLU quantizes gs hidden values per group, each row-block yields rb/2 of them.
//   Latency shape (when every iteration's block fits on the chip at once, 16 waves per CU): about 4 chunks
//   per wave, so all loads are in flight together and a block's latency chain is one round trip plus its
//   prologue.
//   Streaming shape (larger matrices): about 16 chunks per wave (a whole row-block per wave for SwiGLU).
//   Every GEMV runs one block per iteration, except the head's argmax and ordered sums: a persistent grid of
//   as many blocks as fit at once, each paying its prologue once and streaming its iterations back to back.
static void gemv_split(GemvShape &s, int C, int per_wave, const TiledMat &T, int epi) {
    s.kw = (C + per_wave - 1) / per_wave;
    if (s.kw > 16) s.kw = 16;
    if (s.kw < 1) s.kw = 1;
    s.nb = 4 / s.kw > 1 ? 4 / s.kw : 1;
    if (epi == EPI_SWIGLU) {
        s.nb = T.gs / (T.rb / 2);
        if (s.nb * s.kw > 16) s.kw = 16 / s.nb;
        if (s.kw < 1) s.kw = 1;
    }
}

GemvShape gemv_pick_shape(const TiledMat &T, int pro, int epi, int ordered, int cus) {
    GemvShape s;
    const int C = T.nchunks;
    // bit 1: the RMSNorm prologue sums sequentially (strict mode): its block-wide sum runs one segment per wave
    // (the head over a short input keeps its 4-wave blocks, which fill the chip twice over: Qwen2-0.5B shape
    // 22.2 -> 13.7 us; over the 3584 inputs of the 7B shape the 8 segments win, 100 -> 93 us)
    const int seq_norm = (ordered & 2) && pro == PRO_NORM && (epi != EPI_ARGMAX || T.n > 1024);
    ordered &= 1;
    if (cus < 1) cus = 1;
    s.ord = 0;
    if (ordered) {
        // Ordered sums (runq): the unordered split when the group products of one iteration's rows fit in
        // 64 KiB of LDS (they are then added per row in group order), else one wave per 64-row block whose
        // lanes each own a row and add its groups in order.  That second form needs 64-row blocks, a wave of
        // its own per row-block (kw 1: no RMSNorm segments, no attention merge) and free row-blocks per
        // iteration (no SwiGLU quantization group): any other matrix whose products overflow has no ordered
        // shape, and grid 0 says so.
        gemv_split(s, C, 4, T, epi);
        if ((size_t)s.nb * T.rb * (T.ng + 1) * 4 <= 65536) {
            s.ord = 1;
            ordered = 0; // shaped like the unordered GEMV from here on
        } else if (T.rb == 64 && epi != EPI_SWIGLU && pro != PRO_ATTN && !seq_norm) {
            s.kw = 1;
            s.nb = 4;
        } else {
            s.kw = s.nb = 1;
            s.grid = 0;
            s.depth = 2;
            return s;
        }
    } else {
        gemv_split(s, C, 4, T, epi);
        // the attention merge reads every slice's partials before the block's first product: one row-block per
        // block (more waves per row-block below) spreads the weights over twice the CUs (Qwen2-0.5B o GEMV:
        // 4.45 -> 4.26 µs in the step graph)
        if (pro == PRO_ATTN) s.nb = 1;
        // the QKV GEMV: when its row-blocks fit one per CU, one row-block per block with two chunks per wave
        // (Qwen2-0.5B shape: 36 -> 72 blocks of 4 waves, 4.15 -> 4.03 µs in the step graph)
        if (epi == EPI_QKV && T.nblocks <= cus && (C + 1) / 2 <= 16) {
            s.kw = (C + 1) / 2;
            s.nb = 1;
        }
    }
    int iters = (T.nblocks + s.nb - 1) / s.nb;
    int waves = s.kw * s.nb;
    int resident = cus * (waves < 16 ? 16 / waves : 1);
    if (iters > resident) {
        if (!ordered) {
            // streaming split: about 16 chunks per wave; the SwiGLU epilogue's blocks (4 row-blocks, 32 hidden
            // values) measured fastest with one wave per row-block reading all of its chunks (unordered sums)
            gemv_split(s, C, epi == EPI_SWIGLU && !s.ord ? C : 16, T, epi);
            if (s.ord && (size_t)s.nb * T.rb * (T.ng + 1) * 4 > 65536) s.nb = 1; // keep the products in LDS
            iters = (T.nblocks + s.nb - 1) / s.nb;
            waves = s.kw * s.nb;
            resident = cus * (waves < 16 ? 16 / waves : 1);
        }
        // the head's argmax and ordered sums run a persistent grid; every other GEMV one block per iteration
        s.grid = (epi == EPI_ARGMAX || s.ord) && iters > resident ? resident : iters;
    } else {
        // latency shape: when the iterations outnumber the CUs, some CUs hold two blocks and finish last;
        // more row-blocks per iteration (more waves per block) keep it at one block per CU (a wider rule that
        // also regrouped the streaming shapes' blocks measured slower)
        while (iters > cus && epi != EPI_SWIGLU && (s.kw * s.nb * 2) <= 16 &&
               !(s.ord && (size_t)s.nb * 2 * T.rb * (T.ng + 1) * 4 > 65536)) {
            s.nb *= 2;
            iters = (T.nblocks + s.nb - 1) / s.nb;
        }
        s.grid = iters;
        // Ordered sums: one row-block per block, so that a small matrix is spread over as many CUs as it has
        // row-blocks (a CU pulls its block's bytes at a few tens of GB/s; the llama2.c 768/12L shapes: 12 ->
        // 96 blocks for o and down, 2834 -> 3169 tok/s with 8-row blocks).  Not where that would put more
        // blocks than CUs: the Qwen2-7B shape's strict QKV GEMV keeps 144 blocks of two row-blocks instead of
        // 288 of one (13.6 -> 11.6 us; the CUs holding two blocks ran two sequential RMSNorm sums).  The
        // SwiGLU epilogue's row-blocks per block are fixed by the quantization group.
        if (s.ord && epi != EPI_SWIGLU && T.nblocks <= cus) {
            s.nb = 1;
            s.grid = T.nblocks;
        }
    }
    // The attention merge gives each thread one 4-value slot of the input: a block covers the whole input
    // in one pass (a second pass would read its operands after the weights are issued).
    if (pro == PRO_ATTN)
        while (s.kw * s.nb * 64 < T.n / 4 && s.kw * s.nb < 16 && s.kw < C) s.kw++;
    // the strict RMSNorm's sequential sum takes one segment per wave: at least 8 waves where the chunks allow,
    // a persistent grid shrinking to what then fits at once
    if (seq_norm) {
        const int iters_now = (T.nblocks + s.nb - 1) / s.nb;
        const bool persistent = s.grid < iters_now;
        while (s.kw * s.nb < 8 && s.kw < C) s.kw++;
        const int w = s.kw * s.nb;
        if (persistent) s.grid = std::min(iters_now, cus * (w < 16 ? 16 / w : 1));
    }
    if (s.grid < 1) s.grid = 1;
    s.depth = 2;
    return s;
}

// Long rows with few of them (a down projection) take 8-row blocks, so that the grid still covers the chip.
int gemv_row_block(int d, int n) { return n >= 4096 && d <= 8192 ? 8 : 16; }

int stream_wait(hipStream_t st, long timeout_ms, const char *who) {
    struct timespec t0, t;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (unsigned i = 0;; i++) {
        hipError_t e = hipStreamQuery(st);
        if (e == hipSuccess) return 0;
        if (e != hipErrorNotReady) {
            fprintf(stderr, "%s: %s\n", who, hipGetErrorString(e));
            return -1;
        }
        clock_gettime(CLOCK_MONOTONIC, &t);
        const long ms = (t.tv_sec - t0.tv_sec) * 1000L + (t.tv_nsec - t0.tv_nsec) / 1000000L;
        if (ms >= timeout_ms) return 1;
        if (i > 64) {
            struct timespec sl = {0, 20000};
            nanosleep(&sl, nullptr);
        }
    }
}
