// Host-side helpers shared by the drop-in API, the model API and the test hooks (internal header).
#pragma once
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#include "kernels.h"

// Print "<who>: <what>: <hip error>" to stderr and return -1 from the calling function.
#define HIP_OR_FAIL(who, call)                                                                        \
    do {                                                                                             \
        hipError_t e_ = (call);                                                                      \
        if (e_ != hipSuccess) {                                                                      \
            fprintf(stderr, "%s: %s failed: %s\n", who, #call, hipGetErrorString(e_));              \
            return -1;                                                                               \
        }                                                                                            \
    } while (0)

// Device ordinal from FPGA_MEMIDX (the reference's memory-bank selector, matvec_fpga.cpp:83-91), default 0.
// Returns -1 with a message on a malformed value.
static inline int hip_device_from_env(const char *who) {
    const char *e = getenv("FPGA_MEMIDX");
    if (!e) return 0;
    char *end;
    long v = strtol(e, &end, 0);
    if (!*e || *end || v < 0) {
        fprintf(stderr, "%s: bad FPGA_MEMIDX '%s'\n", who, e);
        return -1;
    }
    return (int)v;
}

// GEMV launch shape for a tiled matrix: waves per row-block (K split inside the block), row-blocks per
// block iteration, and the grid.  `ordered` keeps each row's groups in one lane, summed in order.  `cus` is
// the device's compute-unit count (hip_cu_count).
struct GemvShape {
    int kw, nb, grid, depth;
    int ord; // ordered sums through LDS group products (GemvArgs::ord)
};
// ordered: bit 0 the group products summed in group order, bit 1 the strict mode's sequential RMSNorm sum.
// grid 0: no shape adds this matrix's groups in order (products beyond 64 KiB of LDS outside the 64-row form).
GemvShape gemv_pick_shape(const TiledMat &T, int pro, int epi, int ordered, int cus);

// Compute units of device `dev` (0 with a message on failure).
static inline int hip_cu_count(int dev) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        fprintf(stderr, "hip: cannot read the compute-unit count of device %d\n", dev);
        return 0;
    }
    return n;
}
// Row-block size for a plain matrix of d rows x n inputs (fused QKV and gate/up keep 16 for their pairing).
int gemv_row_block(int d, int n);

// Wait for the stream with a time limit (the reference's 5 s ap_done poll, matvec_fpga.cpp:34, 156-170).
// Returns 0, 1 on time-out, -1 on a HIP error (message printed).
int stream_wait(hipStream_t st, long timeout_ms, const char *who);
