/* Drop-in replacement for the reference's board driver API (driver/matvec_fpga.h:8-37), implemented by
 * libmatvec_hip.so on one MI355X.  The signatures, argument meanings, ownership rules and error convention
 * are the reference's; the reference's hosts (qwen/qwen.c and runq/runq.c built with -DFPGA) link against
 * this library unchanged.
 *
 * Memory model.  fpga_alloc() returns pinned host memory and keeps an HBM twin of the same size; *phys is
 * the twin's device address, which the matvec calls take.  The reference's buffers are coherent and
 * uncached, so its callers never sync; this library gives the same guarantees per call:
 *   - the weight and scale ranges (w/wq, ws) are copied to HBM the first time they are used as weights and
 *     then kept resident (repacked once into the GEMV kernels' tiled layout); the reference's callers write
 *     weights once at load (qwen.c:162-163, runq.c:167-168) and never again,
 *   - the activation ranges (xq, xs) are copied host->device on every call,
 *   - the output range is copied device->host before the call returns.
 * Calls are synchronous, like the reference's (run_kernel polls ap_done, matvec_fpga.cpp:156-170).  State is
 * process-global and not thread-safe, like the reference's (its file-scope state, matvec_fpga.cpp:50-56).
 *
 * Differences from the reference contract, all of them relaxations:
 *   - n may be up to MATVEC_HIP_MAX_N (the reference stops at MAX_N 8192, matvec_fpga.cpp:33, 178, 212), so
 *     the Qwen2-7B down projection (n = 18944) runs;
 *   - one library exports both fpga_matvec (runq flavour) and fpga_matvec4 (qwen flavour); the reference
 *     builds one or the other (#ifndef MATVEC4, matvec_fpga.cpp:172-233);
 *   - fpga_matvec, like the reference's, takes any address; ranges that the kernel cannot read or write as
 *     aligned vectors are staged through aligned device buffers inside the call.
 * Env: FPGA_MEMIDX = HIP device ordinal (the reference's bank index, matvec_fpga.cpp:83-91);
 *      FPGA_TIMEOUT_MS = completion wait limit, default 5000 (the reference's TIMEOUT_S, matvec_fpga.cpp:34);
 *      LLM_STRICT = 1: fpga_matvec4 adds each row's groups in order, as qwen.c's matmul_cpu does
 *      (qwen.c:452-455), so a -DFPGA qwen.c reproduces the CPU build's logits bit for bit. */
#pragma once
#include <stddef.h>
#include <stdint.h>

#define MATVEC_HIP_MAX_N 32768

#ifdef __cplusplus
extern "C" {
#endif

/* matvec_fpga.h:12-15.  Select the HIP device and create the library's stream.  Idempotent.
 * Returns 0, or -1 with a message on stderr. */
int fpga_open(void);

/* matvec_fpga.h:17-19.  Pinned host buffer plus an HBM twin, both kept until fpga_close().  Returns the CPU
 * pointer and stores the device address in *phys; NULL with a message on stderr on failure. */
void *fpga_alloc(size_t bytes, uint64_t *phys);

/* matvec_fpga.h:21-22.  Same, silent on failure; the reason is printed by the next fpga_alloc(). */
void *fpga_alloc_try(size_t bytes, uint64_t *phys);

/* matvec_fpga.h:24-26 (math: hls/matvec.h:1-19, runq.c:429-458).  int8 weights with fp32 scales per group of
 * gs (32 or 64), int8 activations with fp32 scales:
 *   out[i] = sum_g ((float)(sum_k wq[i*n + g*gs + k] * xq[g*gs + k]) * ws[(i*n)/gs + g]) * xs[g]
 * Group sums are exact int32; the groups of a row are added in order, so the result is bit-identical to
 * runq.c's matmul(), which is the reference kernel's own test bar (hls/matvec_tb.cpp:82-83).
 * Arguments are device addresses from fpga_alloc().  Returns 0, or -1 with a message on stderr. */
int fpga_matvec(uint64_t wq, uint64_t ws, uint64_t xq, uint64_t xs, uint64_t out, int n, int d, int gs);

/* matvec_fpga.h:28-30 (math: hls4/matvec4.h:1-21, qwen.c:407-457).  int4 (wbits 4) or int8 (wbits 8) weights
 * with fp16 scales per group of 32, int8 activations with fp32 scales:
 *   out[i] = sum_g ((float)(group int sum) * f16(ws[i*n/32 + g])) * xs[g]
 * Group sums are exact int32; the fp32 sum over groups is taken in a tree, within the reference testbench's
 * bound |out - exact| <= 1e-5 * sum_g |term_g| (hls4/matvec4_tb.cpp:1-7, 19, 67-79), or in group order with
 * LLM_STRICT=1.  Every address must be 64-byte aligned and n % 32 == 0, as the reference requires
 * (matvec_fpga.cpp:212-216).  Returns 0, or -1 with a message on stderr. */
int fpga_matvec4(uint64_t w, uint64_t ws, uint64_t xq, uint64_t xs, uint64_t out, int n, int d, int wbits);

/* matvec_fpga.h:32-33.  Free every buffer and the device state.  Safe to call more than once. */
void fpga_close(void);

#ifdef __cplusplus
}
#endif
