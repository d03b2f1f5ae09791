// The reference's board driver API (driver/matvec_fpga.h) on one MI355X.  See include/matvec_fpga.h for
// the contract; this file keeps the reference driver's behaviour where it is observable: idempotent open
// (matvec_fpga.cpp:117-124), the alloc / alloc_try pair with the failure reason kept for the next alloc
// (126-154), argument validation with one stderr line and -1 (178-182, 212-216), a completion time limit
// (156-170, 192-196, 226-230) and a close that frees everything (235-243).
#include <algorithm>
#include <map>
#include <string.h>
#include <time.h>
#include <tuple>
#include <vector>

#include "../../include/matvec_fpga.h"
#include "host_common.h"

namespace {

struct Buf {
    uint8_t *host, *dev;
    size_t size;
};

struct Weight { // one matrix, uploaded and repacked at its first use
    uint8_t *tiled;
    TiledMat T;
    GemvShape shape;
};
// a matrix is identified by its planes' device addresses, its shape and its format code
// (wbits | gs << 8 | sf32 << 16 | ordered << 24)
typedef std::tuple<uint64_t, uint64_t, int, int, int> WeightKey;

struct State {
    bool open = false;
    int device = 0;
    hipStream_t st = nullptr;
    long timeout_ms = 5000;
    std::vector<Buf> bufs;       // sorted by dev
    std::map<WeightKey, Weight> weights; // node-based: a Weight's address stays valid as others are added
    size_t total = 0;
    char last_err[256] = "";
    uint8_t *stage = nullptr;    // int rowmap for repacks
    int8_t *xstage = nullptr;    // activations whose device address is not 16-byte aligned (the kernel reads
                                 // them as 16-byte vectors)
    float *sstage = nullptr;     // activation scales whose device address is not 4-byte aligned
    float *ostage = nullptr;     // outputs whose device address is not 4-byte aligned
    size_t ostage_n = 0;
    int strict = 0;              // LLM_STRICT=1: fpga_matvec4 adds a row's groups in order (qwen.c:452-455)
    int *rowmap = nullptr;
    size_t rowmap_n = 0;
};

State S;

// buffer holding [addr, addr + len) of device addresses, or NULL
const Buf *find(uint64_t addr, size_t len) {
    auto it = std::upper_bound(S.bufs.begin(), S.bufs.end(), addr,
                               [](uint64_t a, const Buf &b) { return a < (uint64_t)b.dev; });
    if (it == S.bufs.begin()) return nullptr;
    --it;
    const uint64_t base = (uint64_t)it->dev;
    if (addr < base || addr - base + len > it->size) return nullptr;
    return &*it;
}

uint8_t *host_of(const Buf *b, uint64_t addr) { return b->host + (addr - (uint64_t)b->dev); }

int ensure_rowmap(size_t rows) {
    if (rows <= S.rowmap_n) return 0;
    if (S.rowmap) hipFree(S.rowmap);
    S.rowmap = nullptr;
    std::vector<int> m(rows);
    for (size_t i = 0; i < rows; i++) m[i] = (int)i; // source 0, row i
    HIP_OR_FAIL("fpga", hipMalloc(&S.rowmap, rows * sizeof(int)));
    HIP_OR_FAIL("fpga", hipMemcpy(S.rowmap, m.data(), rows * sizeof(int), hipMemcpyHostToDevice));
    S.rowmap_n = rows;
    return 0;
}

// the resident tiled copy of a weight matrix; uploads and repacks it the first time
const Weight *weight(const char *who, uint64_t w, uint64_t ws, int n, int d, int wbits, int gs, int sf32, int ordered) {
    const WeightKey key(w, ws, n, d, wbits | gs << 8 | sf32 << 16 | ordered << 24);
    const auto found = S.weights.find(key);
    if (found != S.weights.end()) return &found->second;
    const size_t wbytes = (size_t)d * n * wbits / 8, sbytes = (size_t)d * (n / gs) * (sf32 ? 4 : 2);
    const Buf *bw = find(w, wbytes), *bs = find(ws, sbytes);
    if (!bw || !bs) {
        fprintf(stderr, "%s: weight or scale range is not inside a buffer from fpga_alloc()\n", who);
        return nullptr;
    }
    // raw planes host -> their HBM twins, then into the tiled layout
    if (hipMemcpyAsync((void *)w, host_of(bw, w), wbytes, hipMemcpyHostToDevice, S.st) != hipSuccess ||
        hipMemcpyAsync((void *)ws, host_of(bs, ws), sbytes, hipMemcpyHostToDevice, S.st) != hipSuccess) {
        fprintf(stderr, "%s: weight upload failed\n", who);
        return nullptr;
    }
    if (ensure_rowmap((size_t)d)) return nullptr;
    Weight x;
    x.T = tiled_describe(d, n, gs, wbits, sf32, ordered ? 64 : 16);
    if (hipMalloc(&x.tiled, x.T.bytes) != hipSuccess) {
        fprintf(stderr, "%s: cannot allocate %zu bytes of HBM for a weight matrix\n", who, x.T.bytes);
        return nullptr;
    }
    x.T.data = x.tiled;
    RepackArgs ra;
    memset(&ra, 0, sizeof ra);
    ra.T = x.T;
    ra.w[0] = (const uint8_t *)w;
    ra.s[0] = (const uint8_t *)ws;
    ra.rowmap = S.rowmap;
    if (launch_repack(ra, S.st) != hipSuccess || hipStreamSynchronize(S.st) != hipSuccess) {
        fprintf(stderr, "%s: weight repack failed\n", who);
        hipFree(x.tiled);
        return nullptr;
    }
    x.shape = gemv_pick_shape(x.T, PRO_XQ, EPI_STORE, ordered, hip_cu_count(S.device));
    if (x.shape.grid < 1) {
        fprintf(stderr, "%s: no GEMV shape for a %d x %d matrix\n", who, d, n);
        hipFree(x.tiled);
        return nullptr;
    }
    return &S.weights.emplace(key, x).first->second;
}

int run(const char *who, const Weight *W, uint64_t xq, uint64_t xs, uint64_t out, int n, int d, int gs) {
    const Buf *bx = find(xq, (size_t)n), *bxs = find(xs, (size_t)(n / gs) * 4), *bo = find(out, (size_t)d * 4);
    if (!bx || !bxs || !bo) {
        fprintf(stderr, "%s: xq, xs or out range is not inside a buffer from fpga_alloc()\n", who);
        return -1;
    }
    int8_t *xdev = (int8_t *)xq;
    if (xq & 15) {
        if (!S.xstage) HIP_OR_FAIL(who, hipMalloc(&S.xstage, MATVEC_HIP_MAX_N));
        xdev = S.xstage;
    }
    // the kernel reads the scales and writes the outputs as floats: ranges at addresses that are not 4-byte
    // aligned go through aligned staging buffers (the reference's driver takes any address for fpga_matvec)
    float *sdev = (float *)xs, *odev = (float *)out;
    if (xs & 3) {
        if (!S.sstage) HIP_OR_FAIL(who, hipMalloc(&S.sstage, MATVEC_HIP_MAX_N / 32 * 4));
        sdev = S.sstage;
    }
    if (out & 3) {
        if ((size_t)d > S.ostage_n) {
            if (S.ostage) hipFree(S.ostage);
            S.ostage = nullptr;
            S.ostage_n = 0;
            HIP_OR_FAIL(who, hipMalloc(&S.ostage, (size_t)d * 4));
            S.ostage_n = (size_t)d;
        }
        odev = S.ostage;
    }
    HIP_OR_FAIL(who, hipMemcpyAsync(xdev, host_of(bx, xq), (size_t)n, hipMemcpyHostToDevice, S.st));
    HIP_OR_FAIL(who, hipMemcpyAsync(sdev, host_of(bxs, xs), (size_t)(n / gs) * 4, hipMemcpyHostToDevice, S.st));
    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.W = W->T;
    a.kw = W->shape.kw;
    a.nb = W->shape.nb;
    a.depth = W->shape.depth;
    a.ord = W->shape.ord;
    a.xq = xdev;
    a.xs = sdev;
    a.out = odev;
    HIP_OR_FAIL(who, launch_gemv(W->T.wbits, W->T.gs, W->T.sf32, PRO_XQ, EPI_STORE, a, W->shape.grid, S.st));
    if (odev != (float *)out) // keep the twin equal to the host copy
        HIP_OR_FAIL(who, hipMemcpyAsync((void *)out, odev, (size_t)d * 4, hipMemcpyDeviceToDevice, S.st));
    HIP_OR_FAIL(who, hipMemcpyAsync(host_of(bo, out), odev, (size_t)d * 4, hipMemcpyDeviceToHost, S.st));
    int r = stream_wait(S.st, S.timeout_ms, who);
    if (r == 1) {
        fprintf(stderr, "%s: kernel did not finish in %ld ms (n=%d d=%d)\n", who, S.timeout_ms, n, d);
        return -1;
    }
    return r;
}

int open_impl() {
    int dev = hip_device_from_env("fpga");
    if (dev < 0) return -1;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        fprintf(stderr, "fpga: no HIP device found\n");
        return -1;
    }
    if (dev >= count) {
        fprintf(stderr, "fpga: FPGA_MEMIDX %d but only %d HIP device(s)\n", dev, count);
        return -1;
    }
    HIP_OR_FAIL("fpga", hipSetDevice(dev));
    HIP_OR_FAIL("fpga", hipStreamCreateWithFlags(&S.st, hipStreamNonBlocking));
    S.device = dev;
    if (const char *e = getenv("FPGA_TIMEOUT_MS")) {
        char *end;
        long v = strtol(e, &end, 0);
        if (!*e || *end || v < 0) {
            fprintf(stderr, "fpga: bad FPGA_TIMEOUT_MS '%s'\n", e);
            return -1;
        }
        S.timeout_ms = v;
    }
    if (const char *e = getenv("LLM_STRICT")) S.strict = atoi(e) != 0;
    S.open = true;
    return 0;
}

} // namespace

extern "C" int fpga_open(void) {
    if (S.open) return 0;
    if (open_impl()) {
        fpga_close();
        return -1;
    }
    return 0;
}

extern "C" void *fpga_alloc_try(size_t bytes, uint64_t *phys) {
    if (!S.open || !bytes) {
        snprintf(S.last_err, sizeof S.last_err, "%s", S.open ? "zero size" : "fpga_open() not called");
        return nullptr;
    }
    hipSetDevice(S.device);
    void *h = nullptr, *d = nullptr;
    hipError_t e = hipHostMalloc(&h, bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(&d, bytes);
    if (e != hipSuccess) {
        snprintf(S.last_err, sizeof S.last_err, "%zu bytes failed after %.1f MiB already allocated: %s", bytes,
                 S.total / 1048576.0, hipGetErrorString(e));
        if (h) hipHostFree(h);
        return nullptr;
    }
    memset(h, 0, bytes);
    if (hipMemset(d, 0, bytes) != hipSuccess) {
        snprintf(S.last_err, sizeof S.last_err, "clearing %zu bytes failed", bytes);
        hipHostFree(h);
        hipFree(d);
        return nullptr;
    }
    Buf b = {(uint8_t *)h, (uint8_t *)d, bytes};
    S.bufs.insert(std::upper_bound(S.bufs.begin(), S.bufs.end(), b,
                                   [](const Buf &x, const Buf &y) { return x.dev < y.dev; }),
                  b);
    S.total += bytes;
    *phys = (uint64_t)d;
    return h;
}

extern "C" void *fpga_alloc(size_t bytes, uint64_t *phys) {
    void *p = fpga_alloc_try(bytes, phys);
    if (!p) fprintf(stderr, "fpga_alloc: %s\n", S.last_err);
    return p;
}

extern "C" int fpga_matvec(uint64_t wq, uint64_t ws, uint64_t xq, uint64_t xs, uint64_t out, int n, int d, int gs) {
    if (!S.open) {
        fprintf(stderr, "fpga_matvec: fpga_open() not called\n");
        return -1;
    }
    if ((gs != 32 && gs != 64) || n <= 0 || n > MATVEC_HIP_MAX_N || n % gs || d <= 0) {
        fprintf(stderr, "fpga_matvec: unsupported n=%d d=%d gs=%d (need gs 32 or 64, n %% gs == 0, n <= %d)\n",
                n, d, gs, MATVEC_HIP_MAX_N);
        return -1;
    }
    hipSetDevice(S.device);
    const Weight *W = weight("fpga_matvec", wq, ws, n, d, 8, gs, 1, 1);
    if (!W) return -1;
    return run("fpga_matvec", W, xq, xs, out, n, d, gs);
}

extern "C" int fpga_matvec4(uint64_t w, uint64_t ws, uint64_t xq, uint64_t xs, uint64_t out, int n, int d, int wbits) {
    if (!S.open) {
        fprintf(stderr, "fpga_matvec4: fpga_open() not called\n");
        return -1;
    }
    if ((wbits != 4 && wbits != 8) || n <= 0 || n > MATVEC_HIP_MAX_N || n % 32 || d <= 0 || ((w | ws | xq | xs | out) & 63)) {
        fprintf(stderr, "fpga_matvec4: unsupported n=%d d=%d wbits=%d or a buffer not 64-byte aligned "
                "(need wbits 4 or 8, n %% 32 == 0, n <= %d)\n", n, d, wbits, MATVEC_HIP_MAX_N);
        return -1;
    }
    hipSetDevice(S.device);
    const Weight *W = weight("fpga_matvec4", w, ws, n, d, wbits, 32, 0, S.strict);
    if (!W) return -1;
    return run("fpga_matvec4", W, xq, xs, out, n, d, 32);
}

extern "C" void fpga_close(void) {
    if (S.open) {
        hipSetDevice(S.device);
        if (S.st) hipStreamSynchronize(S.st);
    }
    for (auto &x : S.weights) hipFree(x.second.tiled);
    S.weights.clear();
    for (Buf &b : S.bufs) {
        hipHostFree(b.host);
        hipFree(b.dev);
    }
    S.bufs.clear();
    if (S.rowmap) hipFree(S.rowmap);
    S.rowmap = nullptr;
    S.rowmap_n = 0;
    for (void *p : {(void *)S.xstage, (void *)S.sstage, (void *)S.ostage})
        if (p) hipFree(p);
    S.xstage = nullptr;
    S.sstage = nullptr;
    S.ostage = nullptr;
    S.ostage_n = 0;
    if (S.st) hipStreamDestroy(S.st);
    S.st = nullptr;
    S.total = 0;
    S.open = false;
}
