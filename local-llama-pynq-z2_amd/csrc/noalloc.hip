// mvh_sample_noalloc (include/llm_hip.h): the on-device sampler over caller logits, as mvh_sample, with every
// device buffer it needs in one file-scope device array instead of memory allocated per call.  It is for
// callers that cannot allocate device memory (tight serving loops, harnesses that forbid hipMalloc): the call
// makes no hipMalloc, hipFree or other allocating call.
//
// The array is `scratch` below: staged logits (count rows of n rounded up to 4 floats, at most
// NA_LOGITS floats), the probabilities of one row (n <= NA_PROBS), the sampled rows (count <= NA_ROWS), the
// sampler state and the buffers of the many-workgroup draw that mvh_sample takes for large n (so both entry
// points draw alike).  Each GPU holds its own copy until the process ends.  Host code never uses the name
// `scratch` as an address: its device address on each GPU is looked up once, with that GPU current, by
// hipGetSymbolAddress, and only that address reaches copies and kernels.  Every call on one GPU shares the
// array; calls that overlap on one GPU (other host threads) race.  Nothing in it has to start at zero: the
// staged logits and the state are copied in before the kernels run, and the kernels write every probability,
// row and draw buffer before they read it back (the radix histograms are cleared by the draw's first kernel).
#include <string.h>

#include "../../include/llm_hip.h"
#include "host_common.h"

namespace {
constexpr size_t NA_LOGITS = (size_t)1 << 21; // staged logits, floats (8 MiB): 8 rows of a 152064-row head
constexpr size_t NA_PROBS = (size_t)1 << 18;  // probabilities of one row, floats: the sampler's largest n
constexpr size_t NA_ROWS = 4096;              // sampled rows
constexpr size_t OFF_PROBS = NA_LOGITS * 4;
constexpr size_t OFF_ROWS = OFF_PROBS + NA_PROBS * 4;
constexpr size_t OFF_STATE = OFF_ROWS + NA_ROWS * 4;
constexpr size_t OFF_DRAW = OFF_STATE + 256;
constexpr size_t NA_DRAW = (size_t)64 << 10; // the many-workgroup draw's buffers (sample_scratch_bytes())
constexpr size_t NA_BYTES = OFF_DRAW + NA_DRAW;
} // namespace

static __device__ __align__(256) uint8_t scratch[NA_BYTES];

namespace {
constexpr int NA_MAX_DEVICES = 64;
uint8_t *scratch_dev[NA_MAX_DEVICES]; // device address of `scratch` on each device, once looked up

// The device address of this device's `scratch`, looked up on the first call with device `dev` current.
uint8_t *scratch_on(int dev, const char *who) {
    if (dev < 0 || dev >= NA_MAX_DEVICES) {
        fprintf(stderr, "%s: device %d is beyond the %d devices this library tracks\n", who, dev, NA_MAX_DEVICES);
        return nullptr;
    }
    if (!scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "%s: no address for the scratch array on device %d: %s\n", who, dev, hipGetErrorString(e));
            return nullptr;
        }
        scratch_dev[dev] = (uint8_t *)p;
    }
    return scratch_dev[dev];
}
} // namespace

extern "C" int mvh_sample_noalloc(const float *logits, int n, int count, float temperature, float topp,
                                  unsigned long long *rng, int *rows) {
    const char *who = "mvh_sample_noalloc";
    if (!logits || !rng || !rows || n < 2 || count < 1 || !(temperature > 0.0f)) {
        fprintf(stderr, "%s: bad arguments (n=%d count=%d temperature=%g)\n", who, n, count, temperature);
        return -1;
    }
    const size_t ld = ((size_t)n + 3) & ~(size_t)3; // 16-byte aligned rows
    if ((size_t)n > NA_PROBS || (size_t)count > NA_ROWS || (size_t)count * ld > NA_LOGITS) {
        fprintf(stderr, "%s: %d rows of %d logits exceed the scratch array (at most %zu logits per row, %zu rows, "
                "%zu logits in all)\n", who, count, n, NA_PROBS, NA_ROWS, NA_LOGITS);
        return -1;
    }
    if (sample_scratch_bytes() > NA_DRAW) {
        fprintf(stderr, "%s: internal error: the draw's buffers need %zu bytes, %zu reserved\n", who,
                sample_scratch_bytes(), NA_DRAW);
        return -1;
    }
    const int dev = hip_device_from_env(who);
    if (dev < 0) return -1;
    HIP_OR_FAIL(who, hipSetDevice(dev));
    uint8_t *s = scratch_on(dev, who);
    if (!s) return -1;
    float *dl = (float *)s, *dp = (float *)(s + OFF_PROBS);
    int *dr = (int *)(s + OFF_ROWS);
    SamplerState *dss = (SamplerState *)(s + OFF_STATE);
    SamplerState st;
    st.temperature = temperature;
    st.topp = topp;
    st.rng = *rng;
    HIP_OR_FAIL(who, hipMemcpy2D(dl, ld * 4, logits, (size_t)n * 4, (size_t)n * 4, count, hipMemcpyHostToDevice));
    HIP_OR_FAIL(who, hipMemcpy(dss, &st, sizeof st, hipMemcpyHostToDevice));
    for (int c = 0; c < count; c++) {
        SampleArgs a;
        memset(&a, 0, sizeof a);
        a.logits = dl + (size_t)c * ld;
        a.n = n;
        a.probs = dp;
        a.ss = dss;
        a.out_row = dr + c;
        a.scratch = s + OFF_DRAW;
        a.path = topp > 0.0f && topp < 1.0f ? 1 : 0;
        HIP_OR_FAIL(who, launch_sample(a, 0));
    }
    HIP_OR_FAIL(who, hipStreamSynchronize(0));
    HIP_OR_FAIL(who, hipMemcpy(rows, dr, (size_t)count * 4, hipMemcpyDeviceToHost));
    HIP_OR_FAIL(who, hipMemcpy(&st, dss, sizeof st, hipMemcpyDeviceToHost));
    *rng = st.rng;
    return 0;
}
