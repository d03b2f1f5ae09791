// Launch-shape choice for the GEMV kernels and the bounded stream wait (internal).
#include <time.h>

#include "host_common.h"

// Shapes follow from the tiled matrix: a row-block has `nchunks` chunk records of 1 KiB+ each.  Long rows
// (many chunks) split their chunks over several waves of a block (kw), short rows put several row-blocks
// into one block (nb), so a block always has 4..16 waves.  Epilogues that need whole groups of rows in one
// iteration fix nb: SwiGLU quantizes gs hidden values per group, each row-block yields rb/2 of them.
GemvShape gemv_pick_shape(const TiledMat &T, int pro, int epi, int ordered) {
    GemvShape s;
    const int C = T.nchunks;
    if (ordered) {
        s.kw = 1;
        s.nb = 4;
    } else {
        s.kw = C >= 48 ? 8 : C >= 16 ? 4 : C >= 6 ? 2 : 1;
        s.nb = 8 / s.kw > 0 ? 8 / s.kw : 1;
        if (s.nb < 1) s.nb = 1;
    }
    if (epi == EPI_SWIGLU) {
        s.nb = T.gs / (T.rb / 2);
        if (s.nb * s.kw > 16) s.kw = 16 / s.nb;
        if (s.kw < 1) s.kw = 1;
    }
    const int iters = (T.nblocks + s.nb - 1) / s.nb;
    // blocks that normalize x first keep that prologue rare: at most ~2 blocks per CU
    const int cap = pro == PRO_NORM || pro == PRO_ATTN ? 512 : 4096;
    s.grid = iters < cap ? iters : cap;
    if (s.grid < 1) s.grid = 1;
    return s;
}

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
