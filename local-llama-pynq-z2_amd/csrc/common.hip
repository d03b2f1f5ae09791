// Launch-shape choice for the GEMV kernels and the bounded stream wait (internal).
#include <time.h>

#include "host_common.h"

// Shapes follow from the tiled matrix: a row-block has `nchunks` chunk records of 1 KiB+ each.  The chunks of
// a row-block are split over kw waves so that each wave holds at most a few batches, and one block takes
// one iteration (row-blocks of one block: nb), so that the whole grid's loads are in flight at once and a
// block's latency chain is one load round trip plus its prologue.  Epilogues that need whole groups of rows
// fix nb: SwiGLU quantizes gs hidden values per group, each row-block yields rb/2 of them.
GemvShape gemv_pick_shape(const TiledMat &T, int pro, int epi, int ordered) {
    (void)pro;
    GemvShape s;
    const int C = T.nchunks;
    if (ordered) {
        s.kw = 1;
        s.nb = 4;
    } else {
        s.kw = (C + 3) / 4;
        if (s.kw > 16) s.kw = 16;
        if (s.kw < 1) s.kw = 1;
        s.nb = 4 / s.kw > 1 ? 4 / s.kw : 1;
    }
    if (epi == EPI_SWIGLU) {
        s.nb = T.gs / (T.rb / 2);
        if (s.nb * s.kw > 16) s.kw = 16 / s.nb;
        if (s.kw < 1) s.kw = 1;
    }
    const int iters = (T.nblocks + s.nb - 1) / s.nb;
    s.grid = iters < 65535 ? iters : 65535;
    if (s.grid < 1) s.grid = 1;
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
