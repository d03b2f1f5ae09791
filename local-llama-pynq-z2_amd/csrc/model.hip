// Device-resident decode loop (include/llm_hip.h): model upload, one decode step as a fixed kernel
// sequence, hipGraph replay, greedy generation, per-kernel profiling.
//
// One step (forward(), qwen.c:490-573 / runq.c:477-615) is 5 * n_layers + 3 kernels:
//   embed                      token row of the embedding table -> x (qwen.c:498-501)
//   per layer:
//     qkv    GEMV  prologue rmsnorm(x)+quantize, epilogue bias + RoPE + KV-cache write (qwen.c:516-524)
//     attention    split-K over positions, GQA heads of one kv head per block (qwen.c:526-546)
//     o      GEMV  prologue merges the attention splits + quantize, epilogue x += (qwen.c:548-551)
//     gateup GEMV  prologue rmsnorm(x)+quantize, epilogue SwiGLU + quantize (qwen.c:553-563)
//     down   GEMV  int8 input, epilogue x += (qwen.c:564-565)
//   head   GEMV  prologue final rmsnorm+quantize, epilogue logits + per-block argmax (qwen.c:568-572)
//   argmax       block partials -> row -> head_ids[row] (qwen.c:591-598, 683)
// Every kernel reads the position from the StepCtrl block in device memory, so the captured graph is the
// same for every position.
#include <fcntl.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/llm_hip.h"
#include "host_common.h"
#include "prefill.h"

namespace {


struct Layer {
    TiledMat qkv, o, gu, down;
    GemvShape s_qkv, s_o, s_gu, s_down;
};

enum { K_EMBED, K_QKV, K_ATTN, K_O, K_GU, K_DOWN, K_HEAD, K_ARGMAX, K_COUNT };
const char *k_names[K_COUNT] = {"step_start", "qkv_gemv", "attention", "o_gemv", "gateup_gemv", "down_gemv",
                                "head_gemv", "argmax"};

struct Prof { // events around every launch of a step
    std::vector<hipEvent_t> ev;
    std::vector<int> kind;
    std::vector<double> bytes;
    size_t used = 0;
};

} // namespace

struct llm_model {
    llm_info info;
    int kind = 0, hs = 0, kv_dim = 0, gs = 32, qflavor = 0, emb_sf32 = 0, ctx = 0, att_splits = 1;
    // Decode GEMVs load their weights as non-temporal when one step streams more than 3/4 of the MALL
    // (256 MB on MI355X): each weight byte is read once per step and could not stay cached until the next.
    // Measured on the step graph: Qwen2-0.5B shapes (265 MB per step) 0.642 -> 0.608 ms, Qwen2-7B shapes
    // 1.634 -> 1.547 ms; the llama2.c 288/6L and 768/12L shapes (17 and 124 MB, MALL-resident) 3-6% slower
    // with it, so they keep the default policy.
    int weights_nt = 0;
    int head_nt = 0; // the same choice for the head GEMV alone (LLM_HEAD_NT overrides)
    // Reference-order mode (llm_set_strict, LLM_STRICT=1): every float operation in the reference's order, so
    // logits are bitwise those of qwen.c / runq.c built with strict IEEE flags.  GEMV group products summed per
    // row in group order, RMSNorm's sum of squares as one running sum, attention by attn_strict_head, and the
    // reference libm's expf (ref_expf) in SiLU and softmax.
    int strict = 0;
    int device = 0;
    hipStream_t st = nullptr;
    std::vector<void *> allocs;
    std::vector<Layer> L;
    uint8_t *wts = nullptr;
    float *norms = nullptr, *biases = nullptr, *rope_cos = nullptr, *rope_sin = nullptr;
    int8_t *emb_q = nullptr;
    void *emb_s = nullptr;
    TiledMat head;
    GemvShape s_head;
    int32_t *head_ids_d = nullptr;
    std::vector<int32_t> head_ids_h;
    float *kc = nullptr, *vc = nullptr, *x = nullptr, *q = nullptr, *att_ml = nullptr, *att_acc = nullptr;
    float *logits = nullptr, *hist = nullptr, *part_v = nullptr, *hsc = nullptr;
    int8_t *hq = nullptr;
    int *part_i = nullptr;
    int part_cap = 0; // argmax partials allocated (the larger head grid of the two modes)
    StepCtrl *ctrl = nullptr;
    int *prompt = nullptr, *tokens = nullptr, *gen = nullptr;
    hipGraphExec_t g_plain = nullptr, g_hist = nullptr;
    // on-device sampler (temperature > 0): settings and RNG on the device, scratch, the sampling step graphs
    bool sampling = false;
    SamplerState *ss = nullptr;
    float *smp_p = nullptr;
    void *smp_scratch = nullptr; // the many-workgroup draw's buffers (large vocabularies)
    void *smp_strict = nullptr;  // the reference-order draw's buffers (strict mode)
    int smp_path = -1;           // top-p (1) or the plain walk (0): the sampled step graphs launch that path only
    hipGraphExec_t g_plain_s = nullptr, g_hist_s = nullptr;
    // prefill: activation matrices of up to pf_cap tokens (allocated on first use)
    int pf_cap = 0, prefill_on = 1;
    float *pf_x = nullptr, *pf_y = nullptr, *pf_q = nullptr, *pf_s = nullptr;
    float *pf_ml = nullptr, *pf_acc = nullptr; // attention slice partials
    int8_t *pf_a = nullptr;
    int *pf_ids = nullptr;
    // h of the SwiGLU in the gate/up GEMM's epilogue (the down GEMM's input; pf_a is the gate/up input then),
    // on by default where the shapes allow it (LLM_PF_SWIGLU=0 at llm_open: the separate SwiGLU kernel)
    int8_t *pf_h = nullptr;
    float *pf_hs = nullptr;
    int pf_swiglu = 1;
    // bias, RoPE and the q / K / V writes in the QKV GEMM's epilogue instead of k_p_qkv (LLM_PF_QKV=0 at
    // llm_open: the separate kernel)
    int pf_qkv = 1;
    // the prefill attention's products on bf16 MFMA over three-piece splits of the fp32 operands
    // (LLM_PF_FLASH_BF=0 at llm_open: fp32 MFMA)
    int pf_flash_bf = 1;
    // file mapping during load
    const uint8_t *file = nullptr;
    size_t file_size = 0;
};

namespace {

template <typename T>
int dalloc(llm_model *m, T **p, size_t bytes) {
    void *v = nullptr;
    if (hipMalloc(&v, bytes ? bytes : 16) != hipSuccess) {
        fprintf(stderr, "llm_open: cannot allocate %zu bytes of HBM\n", bytes);
        return -1;
    }
    if (hipMemset(v, 0, bytes ? bytes : 16) != hipSuccess) return -1;
    m->allocs.push_back(v);
    *p = (T *)v;
    return 0;
}

// ---- GEMV argument blocks of one step

GemvArgs base_args(const llm_model *m, const TiledMat &T, const GemvShape &s) {
    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.W = T;
    a.kw = s.kw;
    a.nb = s.nb;
    a.depth = s.depth;
    a.ord = s.ord;
    a.qflavor = m->qflavor;
    a.nt = m->weights_nt;
    a.ctrl = m->ctrl;
    a.eps = m->info.rms_eps;
    a.strict = m->strict;
    return a;
}

const float *attn_norm(const llm_model *m, int l) { return m->norms + (size_t)l * m->info.dim; }
const float *ffn_norm(const llm_model *m, int l) { return m->norms + (size_t)(m->info.n_layers + l) * m->info.dim; }
const float *out_norm(const llm_model *m) { return m->norms + (size_t)2 * m->info.n_layers * m->info.dim; }

double attn_bytes(const llm_model *m, int pos) { // K and V rows read, q read, partials written
    return 2.0 * (pos + 1) * m->kv_dim * 4.0 + m->info.dim * 4.0 + m->info.n_heads * 4.0 * (m->hs + 2);
}

hipError_t launch_finalize(llm_model *m) {
    ArgmaxArgs g;
    g.pv = m->part_v;
    g.pi = m->part_i;
    g.np = m->s_head.grid;
    g.head_ids = m->head_ids_d;
    g.ctrl = m->ctrl;
    g.gen = m->gen;
    return launch_argmax(g, m->st);
}

// algorithmic bytes of one launch of a kernel kind (attention at position pos)
double kind_bytes(const llm_model *m, int kind, int pos) {
    const llm_info &I = m->info;
    const int dim = I.dim, wb = m->kind == 0 ? 4 : 8, sf = m->kind == 0 ? 0 : 1;
    switch (kind) {
    case K_EMBED: return dim + dim / m->gs * (m->emb_sf32 ? 4.0 : 2.0) + dim * 4.0;
    case K_QKV: return gemv_algo_bytes(m->L[0].qkv.rows, dim, wb, m->gs, sf);
    case K_ATTN: return attn_bytes(m, pos);
    case K_O: return gemv_algo_bytes(dim, dim, wb, m->gs, sf);
    case K_GU: return gemv_algo_bytes(m->L[0].gu.rows, dim, wb, m->gs, sf);
    case K_DOWN: return gemv_algo_bytes(dim, I.hidden_dim, wb, m->gs, sf);
    case K_HEAD: return gemv_algo_bytes(m->head.rows, dim, 8, m->gs, m->head.sf32);
    case K_ARGMAX: return m->s_head.grid * 8.0;
    }
    return 0;
}

// final rmsnorm + head GEMV of m->x (qwen.c:568-572): logits and per-block argmax partials
hipError_t launch_head(llm_model *m, bool hist) {
    GemvArgs a = base_args(m, m->head, m->s_head);
    a.x = m->x;
    a.norm_w = out_norm(m);
    a.out = m->logits;
    a.logits_hist = hist ? m->hist : nullptr;
    a.part_val = m->part_v;
    a.part_idx = m->part_i;
    a.nt = m->head_nt;
    return launch_gemv(8, m->gs, m->head.sf32, PRO_NORM, EPI_ARGMAX, a, m->s_head.grid, m->st);
}

// the on-device sampler over the head logits; it leaves its choice in the argmax partials
hipError_t launch_sampler(llm_model *m) {
    SampleArgs a;
    memset(&a, 0, sizeof a);
    a.logits = m->logits;
    a.n = m->info.n_logits;
    a.probs = m->smp_p;
    a.ss = m->ss;
    a.ctrl = m->ctrl;
    a.pv = m->part_v;
    a.pi = m->part_i;
    a.np = m->s_head.grid;
    a.scratch = m->smp_scratch;
    a.path = m->smp_path;
    a.strict = m->strict;
    a.strict_scratch = m->smp_strict;
    return launch_sample(a, m->st);
}

// Enqueue one decode step on m->st.  prof != NULL records events around every launch.  Kernel kinds whose
// bit is set in `skip` are left out (the in-graph timing of llm_profile_graph compares such steps).  With
// `sampled`, the sampler follows the head.
int enqueue_step(llm_model *m, bool hist, Prof *prof, int pos_hint, bool finalize, unsigned skip = 0,
                 bool sampled = false) {
    const llm_info &I = m->info;
    const int dim = I.dim, kv = m->kv_dim;
    auto mark = [&](int kind, double bytes) {
        if (!prof) return;
        if (prof->used + 2 > prof->ev.size()) {
            for (int i = 0; i < 64; i++) {
                hipEvent_t e;
                hipEventCreate(&e);
                prof->ev.push_back(e);
            }
        }
        hipEventRecord(prof->ev[prof->used++], m->st);
        prof->kind.push_back(kind);
        prof->bytes.push_back(bytes);
    };
    auto done = [&]() {
        if (prof) hipEventRecord(prof->ev[prof->used++], m->st);
    };
    const int wb = m->kind == 0 ? 4 : 8, sf = m->kind == 0 ? 0 : 1;

    EmbedArgs e;
    e.emb_q = m->emb_q;
    e.emb_s = m->emb_s;
    e.sf32 = m->emb_sf32;
    e.dim = dim;
    e.gs = m->gs;
    e.x = m->x;
    e.ctrl = m->ctrl;
    e.prompt = m->prompt;
    e.tokens = m->tokens;
    e.pv = m->part_v;
    e.pi = m->part_i;
    e.np = m->s_head.grid;
    e.head_ids = m->head_ids_d;
    e.gen = m->gen;
    auto on = [&](int kind) { return !(skip & (1u << kind)); };
    if (on(K_EMBED)) {
        mark(K_EMBED, kind_bytes(m, K_EMBED, pos_hint));
        HIP_OR_FAIL("llm", launch_embed(e, m->st));
        done();
    }

    for (int l = 0; l < I.n_layers; l++) {
        const Layer &Ly = m->L[l];
        float *kc = m->kc + (size_t)l * m->ctx * kv, *vc = m->vc + (size_t)l * m->ctx * kv;

        GemvArgs a = base_args(m, Ly.qkv, Ly.s_qkv);
        a.x = m->x;
        a.norm_w = attn_norm(m, l);
        a.bias = m->biases ? m->biases + (size_t)l * (dim + 2 * kv) : nullptr;
        a.q = m->q;
        a.kc = kc;
        a.vc = vc;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.dim = dim;
        a.kv_dim = kv;
        a.head_size = m->hs;
        a.rope_kind = m->kind == 0 ? ROPE_NEOX : ROPE_INTERLEAVED;
        if (a.rope_kind == ROPE_NEOX && !a.bias) {
            fprintf(stderr, "llm: internal error: Qwen layer %d has no bias table\n", l);
            return -1;
        }
        if (on(K_QKV)) {
            mark(K_QKV, kind_bytes(m, K_QKV, pos_hint));
            HIP_OR_FAIL("llm", launch_gemv(wb, m->gs, sf, PRO_NORM, EPI_QKV, a, Ly.s_qkv.grid, m->st));
            done();
        }

        AttnArgs t;
        t.q = m->q;
        t.kc = kc;
        t.vc = vc;
        t.ml = m->att_ml;
        t.acc = m->att_acc;
        t.n_heads = I.n_heads;
        t.n_kv = I.n_kv_heads;
        t.hs = m->hs;
        t.kv_dim = kv;
        t.splits = m->att_splits;
        t.max_pos = m->ctx;
        t.ctrl = m->ctrl;
        if (on(K_ATTN)) {
            mark(K_ATTN, kind_bytes(m, K_ATTN, pos_hint));
            if (m->strict) {
                t.splits = 1;
                HIP_OR_FAIL("llm", launch_attention_strict(t, m->st));
            } else {
                HIP_OR_FAIL("llm", launch_attention(t, m->st));
            }
            done();
        }

        a = base_args(m, Ly.o, Ly.s_o);
        a.att_ml = m->att_ml;
        a.att_acc = m->att_acc;
        a.n_heads = I.n_heads;
        a.head_size = m->hs;
        a.att_splits = m->strict ? 1 : m->att_splits; // strict: one slice, merged as the identity
        a.out = m->x;
        if (on(K_O)) {
            mark(K_O, kind_bytes(m, K_O, pos_hint));
            HIP_OR_FAIL("llm", launch_gemv(wb, m->gs, sf, PRO_ATTN, EPI_RESID, a, Ly.s_o.grid, m->st));
            done();
        }

        a = base_args(m, Ly.gu, Ly.s_gu);
        a.x = m->x;
        a.norm_w = ffn_norm(m, l);
        a.hq = m->hq;
        a.hs = m->hsc;
        a.dim = I.hidden_dim; // SwiGLU epilogue: number of hidden values
        if (on(K_GU)) {
            mark(K_GU, kind_bytes(m, K_GU, pos_hint));
            HIP_OR_FAIL("llm", launch_gemv(wb, m->gs, sf, PRO_NORM, EPI_SWIGLU, a, Ly.s_gu.grid, m->st));
            done();
        }

        a = base_args(m, Ly.down, Ly.s_down);
        a.xq = m->hq;
        a.xs = m->hsc;
        a.out = m->x;
        if (on(K_DOWN)) {
            mark(K_DOWN, kind_bytes(m, K_DOWN, pos_hint));
            HIP_OR_FAIL("llm", launch_gemv(wb, m->gs, sf, PRO_XQ, EPI_RESID, a, Ly.s_down.grid, m->st));
            done();
        }
    }

    if (on(K_HEAD)) {
        mark(K_HEAD, kind_bytes(m, K_HEAD, pos_hint));
        HIP_OR_FAIL("llm", launch_head(m, hist));
        done();
    }
    if (sampled) HIP_OR_FAIL("llm", launch_sampler(m));

    if (finalize) { // the step's own argmax; in a captured sequence the next step's start kernel does it
        mark(K_ARGMAX, kind_bytes(m, K_ARGMAX, pos_hint));
        HIP_OR_FAIL("llm", launch_finalize(m));
        done();
    }
    return 0;
}

int capture(llm_model *m, bool hist, hipGraphExec_t *out, unsigned skip = 0, bool sampled = false) {
    hipGraph_t g;
    HIP_OR_FAIL("llm", hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(m, hist, nullptr, 0, false, skip, sampled);
    hipError_t e = hipStreamEndCapture(m->st, &g);
    if (rc || e != hipSuccess) {
        fprintf(stderr, "llm: graph capture failed: %s\n", hipGetErrorString(e));
        return -1;
    }
    e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
        fprintf(stderr, "llm: graph instantiation failed: %s\n", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

int set_ctrl(llm_model *m, int pos, int token, int n_prompt, int mode) {
    StepCtrl c;
    memset(&c, 0, sizeof c);
    c.pos = pos;
    c.token = token;
    c.n_prompt = n_prompt;
    c.mode = mode;
    HIP_OR_FAIL("llm", hipMemcpyAsync(m->ctrl, &c, sizeof c, hipMemcpyHostToDevice, m->st));
    HIP_OR_FAIL("llm", hipStreamSynchronize(m->st));
    return 0;
}

// ---- upload helpers

// Repack `nsrc` raw reference matrices (rows of n values) into one tiled matrix with the given logical row
// order.  Raw planes are copied from the file mapping to a staging area in HBM first.
int upload_tiled(llm_model *m, TiledMat *T, uint8_t *dst, const uint8_t *const *w, const uint8_t *const *s,
                 const int *rows_per_src, int nsrc, const std::vector<int> &rowmap, uint8_t *stage, int *rowmap_d) {
    RepackArgs ra;
    memset(&ra, 0, sizeof ra);
    size_t off = 0;
    const size_t rowbytes = (size_t)T->n * T->wbits / 8, srow = (size_t)T->ng * (T->sf32 ? 4 : 2);
    for (int i = 0; i < nsrc; i++) {
        const size_t wb = rowbytes * rows_per_src[i], sb = srow * rows_per_src[i];
        HIP_OR_FAIL("llm_open", hipMemcpy(stage + off, w[i], wb, hipMemcpyHostToDevice));
        ra.w[i] = stage + off;
        off += (wb + 255) & ~(size_t)255;
        HIP_OR_FAIL("llm_open", hipMemcpy(stage + off, s[i], sb, hipMemcpyHostToDevice));
        ra.s[i] = stage + off;
        off += (sb + 255) & ~(size_t)255;
    }
    HIP_OR_FAIL("llm_open", hipMemcpy(rowmap_d, rowmap.data(), rowmap.size() * sizeof(int), hipMemcpyHostToDevice));
    T->data = dst;
    ra.T = *T;
    ra.rowmap = rowmap_d;
    HIP_OR_FAIL("llm_open", launch_repack(ra, 0));
    HIP_OR_FAIL("llm_open", hipDeviceSynchronize());
    return 0;
}

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// logical row orders of the fused matrices
std::vector<int> rowmap_natural(int rows) {
    std::vector<int> r(rows);
    for (int i = 0; i < rows; i++) r[i] = i;
    return r;
}
std::vector<int> rowmap_qkv_neox(int dim, int kv, int hs) { // blocks of 16: 8 first-half rows, 8 partners
    std::vector<int> r(dim + 2 * kv);
    const int half = hs / 2, per = half / 8;
    for (int R = 0; R < dim + kv; R++) {
        const int blk = R / 16, rr = R & 15, hh = blk / per, i = (blk - hh * per) * 8 + (rr & 7);
        const int e = hh * hs + (rr < 8 ? i : half + i);
        r[R] = e < dim ? e : (1 << 28) | (e - dim);
    }
    for (int R = dim + kv; R < dim + 2 * kv; R++) r[R] = (2 << 28) | (R - dim - kv);
    return r;
}
std::vector<int> rowmap_qkv_natural(int dim, int kv) {
    std::vector<int> r(dim + 2 * kv);
    for (int R = 0; R < dim + 2 * kv; R++)
        r[R] = R < dim ? R : R < dim + kv ? (1 << 28) | (R - dim) : (2 << 28) | (R - dim - kv);
    return r;
}
std::vector<int> rowmap_gateup(int hidden, int rb) { // row-block: rb/2 gate rows, then the same up rows
    std::vector<int> r(2 * hidden);
    const int h = rb / 2;
    for (int R = 0; R < 2 * hidden; R++) {
        const int b = R / rb, rr = R % rb, j = b * h + (rr % h);
        r[R] = rr < h ? j : (1 << 28) | j;
    }
    return r;
}

struct Src { const uint8_t *w, *s; };

// GEMV launch shapes of every matrix: group products summed in group order for runq (whose reference sums
// them sequentially, runq.c:452-456, as its FPGA kernel's test bar demands) and in the strict mode.
int pick_shapes(llm_model *m) {
    const int cus = hip_cu_count(m->device);
    if (!cus) return -1;
    // bit 0: ordered group sums; bit 1: the strict mode's sequential RMSNorm sum (it shapes the norm GEMVs)
    const int ord = (m->kind == 1 || m->strict) | (m->strict ? 2 : 0);
    for (Layer &ly : m->L) {
        ly.s_qkv = gemv_pick_shape(ly.qkv, PRO_NORM, EPI_QKV, ord, cus);
        ly.s_o = gemv_pick_shape(ly.o, PRO_ATTN, EPI_RESID, ord, cus);
        ly.s_gu = gemv_pick_shape(ly.gu, PRO_NORM, EPI_SWIGLU, ord, cus);
        ly.s_down = gemv_pick_shape(ly.down, PRO_XQ, EPI_RESID, ord, cus);
    }
    const GemvShape h = gemv_pick_shape(m->head, PRO_NORM, EPI_ARGMAX, ord, cus);
    for (const Layer &ly : m->L)
        for (const auto &[sh, T] : {std::pair<const GemvShape &, const TiledMat &>{ly.s_qkv, ly.qkv}, {ly.s_o, ly.o},
                                    {ly.s_gu, ly.gu}, {ly.s_down, ly.down}, {h, m->head}})
            if (sh.grid < 1) {
                fprintf(stderr, "llm: the group products of a %d x %d matrix in %d-row blocks exceed 64 KiB of LDS: "
                        "no GEMV shape adds them in group order (%s)\n", T.rows, T.n, T.rb,
                        m->kind == 1 ? "runq models" : "the strict mode");
                return -1;
            }
    if (m->part_cap && h.grid > m->part_cap) { // the argmax partials are sized at load for both modes
        fprintf(stderr, "llm: internal error: head grid %d over %d partials\n", h.grid, m->part_cap);
        return -1;
    }
    m->s_head = h;
    return 0;
}

int finish_setup(llm_model *m) {
    const llm_info &I = m->info;
    if (const char *e = getenv("LLM_STRICT")) m->strict = atoi(e) != 0;
    // the argmax partials are sized for the larger of the two head grids (fast and ordered)
    // (a .qwb too wide for ordered sums loads in the fast mode only: llm_set_strict(1) then fails)
    int head_grid = 0;
    for (int st = 0; st < 2; st++) {
        const int keep = m->strict;
        m->strict = st;
        const int r = pick_shapes(m);
        m->strict = keep;
        if (r && (st == 0 || m->kind == 1 || keep)) return -1;
        if (!r) head_grid = std::max(head_grid, m->s_head.grid);
    }
    if (pick_shapes(m)) return -1;
    // attention slices: up to 64 per kv head, each at least ATT_SUB positions
    m->att_splits = (m->ctx + ATT_SUB - 1) / ATT_SUB;
    if (m->att_splits > 64) m->att_splits = 64;
    const size_t kvn = (size_t)I.n_layers * m->ctx * m->kv_dim;
    if (dalloc(m, &m->kc, kvn * 4) || dalloc(m, &m->vc, kvn * 4) || dalloc(m, &m->x, (size_t)I.dim * 4) ||
        dalloc(m, &m->q, (size_t)I.dim * 4) ||
        dalloc(m, &m->att_ml, (size_t)I.n_heads * m->att_splits * 2 * 4) ||
        dalloc(m, &m->att_acc, (size_t)I.n_heads * m->att_splits * m->hs * 4) ||
        dalloc(m, &m->logits, (size_t)I.n_logits * 4) || dalloc(m, &m->part_v, (size_t)head_grid * 4) ||
        dalloc(m, &m->part_i, (size_t)head_grid * 4) || dalloc(m, &m->hq, (size_t)I.hidden_dim) ||
        dalloc(m, &m->hsc, (size_t)I.hidden_dim / m->gs * 4) || dalloc(m, &m->ctrl, sizeof(StepCtrl)) ||
        dalloc(m, &m->prompt, (size_t)m->ctx * 4) || dalloc(m, &m->tokens, (size_t)m->ctx * 4) ||
        dalloc(m, &m->gen, (size_t)m->ctx * 4))
        return -1;
    m->part_cap = head_grid;
    // RoPE tables with the reference's own formulas (host libm, so the values are the reference's)
    const int half = m->hs / 2;
    std::vector<float> c((size_t)m->ctx * half), s((size_t)m->ctx * half);
    for (int p = 0; p < m->ctx; p++)
        for (int i = 0; i < half; i++) {
            if (m->kind == 0) { // qwen.c:504-507
                double a = p * pow((double)I.rope_theta, -2.0 * i / m->hs);
                c[(size_t)p * half + i] = (float)cos(a);
                s[(size_t)p * half + i] = (float)sin(a);
            } else { // runq.c:508-512
                float freq = 1.0f / powf(10000.0f, (2 * i) / (float)m->hs);
                float val = p * freq;
                c[(size_t)p * half + i] = cosf(val);
                s[(size_t)p * half + i] = sinf(val);
            }
        }
    if (dalloc(m, &m->rope_cos, c.size() * 4) || dalloc(m, &m->rope_sin, s.size() * 4)) return -1;
    HIP_OR_FAIL("llm_open", hipMemcpy(m->rope_cos, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    HIP_OR_FAIL("llm_open", hipMemcpy(m->rope_sin, s.data(), s.size() * 4, hipMemcpyHostToDevice));
    // algorithmic GEMV bytes of one step
    const int wb = m->kind == 0 ? 4 : 8, sf = m->kind == 0 ? 0 : 1;
    double b = 0;
    for (const Layer &ly : m->L)
        b += gemv_algo_bytes(ly.qkv.rows, I.dim, wb, m->gs, sf) + gemv_algo_bytes(I.dim, I.dim, wb, m->gs, sf) +
             gemv_algo_bytes(ly.gu.rows, I.dim, wb, m->gs, sf) + gemv_algo_bytes(I.dim, I.hidden_dim, wb, m->gs, sf);
    const double head_b = gemv_algo_bytes(m->head.rows, I.dim, 8, m->gs, m->head.sf32);
    m->info.gemv_bytes_per_token = b + head_b;
    m->weights_nt = b + head_b > 0.75 * 256e6;
    m->head_nt = m->weights_nt;
    if (const char *e = getenv("LLM_WEIGHTS_NT")) m->weights_nt = m->head_nt = atoi(e) != 0; // 0 / 1: override
    if (const char *e = getenv("LLM_HEAD_NT")) m->head_nt = atoi(e) != 0;
    if (const char *e = getenv("LLM_PF_SWIGLU")) m->pf_swiglu = atoi(e) != 0;
    if (const char *e = getenv("LLM_PF_QKV")) m->pf_qkv = atoi(e) != 0;
    if (const char *e = getenv("LLM_PF_FLASH_BF")) m->pf_flash_bf = atoi(e) != 0;
    return 0;
}

int load_qwb(llm_model *m, const char *path, int ctx) {
    const uint8_t *f = m->file;
    int32_t h[10];
    memcpy(h, f + 8, 40);
    llm_info &I = m->info;
    m->kind = I.kind = 0;
    I.dim = h[0]; I.hidden_dim = h[1]; I.n_layers = h[2]; I.n_heads = h[3]; I.n_kv_heads = h[4];
    I.vocab_size = h[5]; I.n_logits = h[6];
    const int max_seq = h[7], gsz = h[8], emb_bits = h[9];
    memcpy(&I.rope_theta, f + 48, 4);
    memcpy(&I.rms_eps, f + 52, 4);
    uint32_t ver;
    memcpy(&ver, f + 4, 4);
    if (memcmp(f, "QWB1", 4) || ver != 1) {
        fprintf(stderr, "%s: not a .qwb version 1 file\n", path);
        return -1;
    }
    if (I.n_heads <= 0 || I.n_kv_heads <= 0 || I.dim <= 0) {
        fprintf(stderr, "%s: bad header\n", path);
        return -1;
    }
    const int hs = I.dim / I.n_heads, kv = hs * I.n_kv_heads;
    // qwen.c:223-228, plus whole 16-row RoPE blocks for the fused QKV tiles (hs % 16)
    if (gsz != 32 || emb_bits != 8 || I.dim % I.n_heads || I.n_heads % I.n_kv_heads || hs % 2 || I.dim % 128 ||
        kv % 16 || I.hidden_dim % 128 || hs % 16 || hs > 256 || I.n_heads / I.n_kv_heads > 16) {
        fprintf(stderr, "%s: unsupported config (group %d, embedding %d-bit, dim %d, heads %d/%d)\n", path, gsz,
                emb_bits, I.dim, I.n_heads, I.n_kv_heads);
        return -1;
    }
    m->hs = hs;
    m->kv_dim = kv;
    m->gs = 32;
    m->qflavor = QF_QWEN;
    m->emb_sf32 = 0;
    m->ctx = ctx < max_seq ? ctx : max_seq;
    if (m->ctx < 1) {
        fprintf(stderr, "%s: context %d\n", path, m->ctx);
        return -1;
    }
    I.ctx = m->ctx;
    I.group_size = 32;
    // walk (qwen.c:237-262)
    size_t off = 256;
    auto take = [&](size_t bytes) { const uint8_t *p = f + off; off += (bytes + 63) & ~(size_t)63; return p; };
    const int Lc = I.n_layers, dim = I.dim, hid = I.hidden_dim;
    const float *an = (const float *)take((size_t)Lc * dim * 4), *fn = (const float *)take((size_t)Lc * dim * 4);
    const float *bq = (const float *)take((size_t)Lc * dim * 4), *bk = (const float *)take((size_t)Lc * kv * 4);
    const float *bv = (const float *)take((size_t)Lc * kv * 4), *on = (const float *)take((size_t)dim * 4);
    const int32_t *hid_ids = (const int32_t *)take((size_t)I.n_logits * 4);
    const int shp[7][2] = {{dim, dim}, {kv, dim}, {kv, dim}, {dim, dim}, {hid, dim}, {dim, hid}, {hid, dim}};
    std::vector<Src> mats[7];
    for (int a = 0; a < 7; a++)
        for (int l = 0; l < Lc; l++) {
            Src sr;
            sr.w = take((size_t)shp[a][0] * shp[a][1] / 2);
            sr.s = take((size_t)shp[a][0] * shp[a][1] / 32 * 2);
            mats[a].push_back(sr);
        }
    Src head;
    head.w = take((size_t)I.n_logits * dim);
    head.s = take((size_t)I.n_logits * dim / 32 * 2);
    Src emb;
    emb.w = take((size_t)I.vocab_size * dim);
    emb.s = take((size_t)I.vocab_size * dim / 32 * 2);
    if (off != m->file_size) {
        fprintf(stderr, "%s: size %zu, but the header describes %zu bytes\n", path, m->file_size, off);
        return -1;
    }
    for (int i = 0; i < I.n_logits; i++)
        if (hid_ids[i] < 0 || hid_ids[i] >= I.vocab_size) {
            fprintf(stderr, "%s: head id %d out of range\n", path, hid_ids[i]);
            return -1;
        }
    // tiled matrices, one allocation
    m->L.resize(Lc);
    size_t total = 0;
    for (Layer &ly : m->L) {
        ly.qkv = tiled_describe(dim + 2 * kv, dim, 32, 4, 0, 16);
        ly.o = tiled_describe(dim, dim, 32, 4, 0, gemv_row_block(dim, dim));
        ly.gu = tiled_describe(2 * hid, dim, 32, 4, 0, 16);
        ly.down = tiled_describe(dim, hid, 32, 4, 0, gemv_row_block(dim, hid));
        total += round256(ly.qkv.bytes) + round256(ly.o.bytes) + round256(ly.gu.bytes) + round256(ly.down.bytes);
    }
    m->head = tiled_describe(I.n_logits, dim, 32, 8, 0, 16);
    total += round256(m->head.bytes);
    I.weight_bytes = (double)total;
    if (dalloc(m, &m->wts, total)) return -1;
    // staging for the largest raw group (the head, or a layer's fused matrices): each plane rounded to 256 B
    auto q4_raw = [](size_t rows, size_t n) { return round256(rows * n / 2) + round256(rows * n / 16); };
    size_t stage_b = round256((size_t)I.n_logits * dim) + round256((size_t)I.n_logits * dim / 16);
    stage_b = std::max(stage_b, q4_raw(dim, dim) + 2 * q4_raw(kv, dim)); // qkv
    stage_b = std::max(stage_b, 2 * q4_raw(hid, dim));                   // gate, up
    stage_b = std::max(stage_b, q4_raw(dim, hid));                       // down (o: dim x dim, within qkv)
    stage_b += 4096;
    uint8_t *stage;
    int *rowmap_d;
    const int max_rows = I.n_logits > 2 * hid ? I.n_logits : 2 * hid;
    if (dalloc(m, &stage, stage_b) || dalloc(m, &rowmap_d, (size_t)(max_rows + dim + 2 * kv) * 4)) return -1;
    uint8_t *p = m->wts;
    const std::vector<int> map_qkv = rowmap_qkv_neox(dim, kv, hs), map_gu = rowmap_gateup(hid, 16);
    for (int l = 0; l < Lc; l++) {
        Layer &ly = m->L[l];
        {
            const uint8_t *w[3] = {mats[0][l].w, mats[1][l].w, mats[2][l].w}, *s[3] = {mats[0][l].s, mats[1][l].s, mats[2][l].s};
            const int rows[3] = {dim, kv, kv};
            if (upload_tiled(m, &ly.qkv, p, w, s, rows, 3, map_qkv, stage, rowmap_d)) return -1;
            p += round256(ly.qkv.bytes);
        }
        {
            const uint8_t *w[1] = {mats[3][l].w}, *s[1] = {mats[3][l].s};
            const int rows[1] = {dim};
            if (upload_tiled(m, &ly.o, p, w, s, rows, 1, rowmap_natural(dim), stage, rowmap_d)) return -1;
            p += round256(ly.o.bytes);
        }
        {
            const uint8_t *w[2] = {mats[4][l].w, mats[6][l].w}, *s[2] = {mats[4][l].s, mats[6][l].s}; // gate w1, up w3
            const int rows[2] = {hid, hid};
            if (upload_tiled(m, &ly.gu, p, w, s, rows, 2, map_gu, stage, rowmap_d)) return -1;
            p += round256(ly.gu.bytes);
        }
        {
            const uint8_t *w[1] = {mats[5][l].w}, *s[1] = {mats[5][l].s};
            const int rows[1] = {dim};
            if (upload_tiled(m, &ly.down, p, w, s, rows, 1, rowmap_natural(dim), stage, rowmap_d)) return -1;
            p += round256(ly.down.bytes);
        }
    }
    {
        const uint8_t *w[1] = {head.w}, *s[1] = {head.s};
        const int rows[1] = {I.n_logits};
        if (upload_tiled(m, &m->head, p, w, s, rows, 1, rowmap_natural(I.n_logits), stage, rowmap_d)) return -1;
    }
    // embedding table stays in the reference layout (one row read per token)
    if (dalloc(m, &m->emb_q, (size_t)I.vocab_size * dim) || dalloc(m, (uint8_t **)&m->emb_s, (size_t)I.vocab_size * dim / 16))
        return -1;
    HIP_OR_FAIL("llm_open", hipMemcpy(m->emb_q, emb.w, (size_t)I.vocab_size * dim, hipMemcpyHostToDevice));
    HIP_OR_FAIL("llm_open", hipMemcpy(m->emb_s, emb.s, (size_t)I.vocab_size * dim / 16, hipMemcpyHostToDevice));
    // norms [attn L][ffn L][out], biases per layer [bq | bk | bv]
    std::vector<float> nv((size_t)(2 * Lc + 1) * dim), bb((size_t)Lc * (dim + 2 * kv));
    memcpy(nv.data(), an, (size_t)Lc * dim * 4);
    memcpy(nv.data() + (size_t)Lc * dim, fn, (size_t)Lc * dim * 4);
    memcpy(nv.data() + (size_t)2 * Lc * dim, on, (size_t)dim * 4);
    for (int l = 0; l < Lc; l++) {
        float *d = bb.data() + (size_t)l * (dim + 2 * kv);
        memcpy(d, bq + (size_t)l * dim, (size_t)dim * 4);
        memcpy(d + dim, bk + (size_t)l * kv, (size_t)kv * 4);
        memcpy(d + dim + kv, bv + (size_t)l * kv, (size_t)kv * 4);
    }
    if (dalloc(m, &m->norms, nv.size() * 4) || dalloc(m, &m->biases, bb.size() * 4) ||
        dalloc(m, &m->head_ids_d, (size_t)I.n_logits * 4))
        return -1;
    HIP_OR_FAIL("llm_open", hipMemcpy(m->norms, nv.data(), nv.size() * 4, hipMemcpyHostToDevice));
    HIP_OR_FAIL("llm_open", hipMemcpy(m->biases, bb.data(), bb.size() * 4, hipMemcpyHostToDevice));
    HIP_OR_FAIL("llm_open", hipMemcpy(m->head_ids_d, hid_ids, (size_t)I.n_logits * 4, hipMemcpyHostToDevice));
    m->head_ids_h.assign(hid_ids, hid_ids + I.n_logits);
    return 0;
}

int load_bin(llm_model *m, const char *path) {
    const uint8_t *f = m->file;
    uint32_t magic;
    int32_t ver, h[7], gs;
    memcpy(&magic, f, 4);
    memcpy(&ver, f + 4, 4);
    memcpy(h, f + 8, 28);
    const uint8_t shared = f[36];
    memcpy(&gs, f + 37, 4);
    llm_info &I = m->info;
    if (magic != 0x616b3432) { fprintf(stderr, "Bad magic number\n"); return -1; }
    if (ver != 2) { fprintf(stderr, "Bad version %d, need version 2\n", ver); return -1; }
    m->kind = I.kind = 1;
    I.dim = h[0]; I.hidden_dim = h[1]; I.n_layers = h[2]; I.n_heads = h[3]; I.n_kv_heads = h[4];
    I.vocab_size = h[5]; I.n_logits = h[5];
    I.rope_theta = 10000.0f;
    I.rms_eps = 1e-5f;
    if (gs != 32 && gs != 64) { // runq.c:340
        fprintf(stderr, "%s: group size %d (the kernels take 32 or 64)\n", path, gs);
        return -1;
    }
    if (I.n_heads <= 0 || I.n_kv_heads <= 0 || I.dim % I.n_heads || I.n_heads % I.n_kv_heads || I.dim % gs ||
        I.hidden_dim % 64 || (I.dim / I.n_heads) % 4 || I.dim / I.n_heads > 256 || I.n_heads / I.n_kv_heads > 16) {
        fprintf(stderr, "%s: unsupported config (dim %d, hidden %d, heads %d/%d, gs %d)\n", path, I.dim,
                I.hidden_dim, I.n_heads, I.n_kv_heads, gs);
        return -1;
    }
    const int dim = I.dim, hid = I.hidden_dim, Lc = I.n_layers;
    m->hs = dim / I.n_heads;
    m->kv_dim = dim * I.n_kv_heads / I.n_heads;
    const int kv = m->kv_dim;
    if ((kv * 2 + dim) % 2 || kv % gs) {
        fprintf(stderr, "%s: kv_dim %d not a multiple of the group size\n", path, kv);
        return -1;
    }
    m->gs = gs;
    m->qflavor = QF_RUNQ;
    m->emb_sf32 = 1;
    m->ctx = h[6];
    I.ctx = m->ctx;
    I.group_size = gs;
    const uint8_t *p = f + 256;
    const float *ra = (const float *)p;
    p += (size_t)Lc * dim * 4;
    const float *rf = (const float *)p;
    p += (size_t)Lc * dim * 4;
    const float *rfin = (const float *)p;
    p += (size_t)dim * 4;
    auto tensor = [&](size_t nel) { Src s; s.w = p; p += nel; s.s = p; p += nel / gs * 4; return s; };
    Src tok = tensor((size_t)I.vocab_size * dim);
    const size_t nel[7] = {(size_t)dim * dim, (size_t)dim * kv, (size_t)dim * kv, (size_t)dim * dim,
                           (size_t)dim * hid, (size_t)dim * hid, (size_t)dim * hid};
    std::vector<Src> mats[7];
    for (int a = 0; a < 7; a++)
        for (int l = 0; l < Lc; l++) mats[a].push_back(tensor(nel[a]));
    Src cls = shared ? tok : tensor((size_t)I.vocab_size * dim);
    if ((size_t)(p - f) > m->file_size) {
        fprintf(stderr, "%s: file is shorter than its header describes\n", path);
        return -1;
    }
    // tiled layer matrices in row-blocks of RQ_RB: the ordered GEMVs (each row's group products added in
    // order, runq.c:440-457) run one row-block per block, so the small runq matrices cover the chip (288/6L:
    // 6958 -> 7217 tok/s against 64-row blocks, 768/12L: 2834 -> 3169); the head keeps 64-row blocks
    constexpr int RQ_RB = 8;
    m->L.resize(Lc);
    size_t total = 0;
    for (Layer &ly : m->L) {
        ly.qkv = tiled_describe(dim + 2 * kv, dim, gs, 8, 1, RQ_RB);
        ly.o = tiled_describe(dim, dim, gs, 8, 1, RQ_RB);
        ly.gu = tiled_describe(2 * hid, dim, gs, 8, 1, RQ_RB);
        ly.down = tiled_describe(dim, hid, gs, 8, 1, RQ_RB);
        total += round256(ly.qkv.bytes) + round256(ly.o.bytes) + round256(ly.gu.bytes) + round256(ly.down.bytes);
    }
    m->head = tiled_describe(I.vocab_size, dim, gs, 8, 1, 64);
    total += round256(m->head.bytes);
    I.weight_bytes = (double)total;
    if (dalloc(m, &m->wts, total)) return -1;
    size_t stage_b = round256((size_t)I.vocab_size * dim) + round256((size_t)I.vocab_size * dim / gs * 4) + 4096;
    const size_t qkv_raw = 3 * (round256((size_t)dim * dim) + round256((size_t)dim * dim / gs * 4)) + 4096;
    const size_t gu_raw = 2 * (round256((size_t)hid * dim) + round256((size_t)hid * dim / gs * 4)) + 4096;
    if (qkv_raw > stage_b) stage_b = qkv_raw;
    if (gu_raw > stage_b) stage_b = gu_raw;
    uint8_t *stage;
    int *rowmap_d;
    const int max_rows = I.vocab_size > 2 * hid ? I.vocab_size : 2 * hid;
    if (dalloc(m, &stage, stage_b) || dalloc(m, &rowmap_d, (size_t)(max_rows + 3 * dim) * 4)) return -1;
    uint8_t *q = m->wts;
    const std::vector<int> map_qkv = rowmap_qkv_natural(dim, kv), map_gu = rowmap_gateup(hid, RQ_RB);
    for (int l = 0; l < Lc; l++) {
        Layer &ly = m->L[l];
        {
            const uint8_t *w[3] = {mats[0][l].w, mats[1][l].w, mats[2][l].w}, *s[3] = {mats[0][l].s, mats[1][l].s, mats[2][l].s};
            const int rows[3] = {dim, kv, kv};
            if (upload_tiled(m, &ly.qkv, q, w, s, rows, 3, map_qkv, stage, rowmap_d)) return -1;
            q += round256(ly.qkv.bytes);
        }
        {
            const uint8_t *w[1] = {mats[3][l].w}, *s[1] = {mats[3][l].s};
            const int rows[1] = {dim};
            if (upload_tiled(m, &ly.o, q, w, s, rows, 1, rowmap_natural(dim), stage, rowmap_d)) return -1;
            q += round256(ly.o.bytes);
        }
        {
            const uint8_t *w[2] = {mats[4][l].w, mats[6][l].w}, *s[2] = {mats[4][l].s, mats[6][l].s};
            const int rows[2] = {hid, hid};
            if (upload_tiled(m, &ly.gu, q, w, s, rows, 2, map_gu, stage, rowmap_d)) return -1;
            q += round256(ly.gu.bytes);
        }
        {
            const uint8_t *w[1] = {mats[5][l].w}, *s[1] = {mats[5][l].s};
            const int rows[1] = {dim};
            if (upload_tiled(m, &ly.down, q, w, s, rows, 1, rowmap_natural(dim), stage, rowmap_d)) return -1;
            q += round256(ly.down.bytes);
        }
    }
    {
        const uint8_t *w[1] = {cls.w}, *s[1] = {cls.s};
        const int rows[1] = {I.vocab_size};
        if (upload_tiled(m, &m->head, q, w, s, rows, 1, rowmap_natural(I.vocab_size), stage, rowmap_d)) return -1;
    }
    if (dalloc(m, &m->emb_q, (size_t)I.vocab_size * dim) ||
        dalloc(m, (uint8_t **)&m->emb_s, (size_t)I.vocab_size * dim / gs * 4))
        return -1;
    HIP_OR_FAIL("llm_open", hipMemcpy(m->emb_q, tok.w, (size_t)I.vocab_size * dim, hipMemcpyHostToDevice));
    HIP_OR_FAIL("llm_open", hipMemcpy(m->emb_s, tok.s, (size_t)I.vocab_size * dim / gs * 4, hipMemcpyHostToDevice));
    std::vector<float> nv((size_t)(2 * Lc + 1) * dim);
    memcpy(nv.data(), ra, (size_t)Lc * dim * 4);
    memcpy(nv.data() + (size_t)Lc * dim, rf, (size_t)Lc * dim * 4);
    memcpy(nv.data() + (size_t)2 * Lc * dim, rfin, (size_t)dim * 4);
    if (dalloc(m, &m->norms, nv.size() * 4)) return -1;
    HIP_OR_FAIL("llm_open", hipMemcpy(m->norms, nv.data(), nv.size() * 4, hipMemcpyHostToDevice));
    return 0;
}

// ---- prefill (batched prompt processing)

const int PREFILL_CHUNK = 512; // tokens per pass through the layers

int prefill_alloc(llm_model *m, int M) {
    if (M <= m->pf_cap) return 0;
    const llm_info &I = m->info;
    const int dim = I.dim, hid = I.hidden_dim, rows = std::max(dim + 2 * m->kv_dim, 2 * hid), wmax = std::max(dim, hid);
    for (void *p : {(void *)m->pf_x, (void *)m->pf_y, (void *)m->pf_q, (void *)m->pf_s,
                    (void *)m->pf_a, (void *)m->pf_ids, (void *)m->pf_ml, (void *)m->pf_acc, (void *)m->pf_h,
                    (void *)m->pf_hs})
        if (p) hipFree(p);
    m->pf_cap = 0;
    // the GEMM input in token-block tiles (rounded up to 16 tokens, whole chunk pairs and scale quads)
    if (hipMalloc(&m->pf_x, (size_t)M * dim * 4) != hipSuccess || hipMalloc(&m->pf_y, (size_t)M * rows * 4) != hipSuccess ||
        hipMalloc(&m->pf_q, (size_t)M * dim * 4) != hipSuccess ||
        hipMalloc(&m->pf_s, pf_scale_floats(wmax / m->gs, M) * 4) != hipSuccess ||
        hipMalloc(&m->pf_a, pf_act_bytes(wmax, M)) != hipSuccess || hipMalloc(&m->pf_ids, (size_t)M * 4) != hipSuccess ||
        hipMalloc(&m->pf_ml, (size_t)M * I.n_heads * PREFILL_ATT_SMAX * 2 * 4) != hipSuccess ||
        hipMalloc(&m->pf_acc, (size_t)M * I.n_heads * PREFILL_ATT_SMAX * m->hs * 4) != hipSuccess ||
        hipMalloc(&m->pf_h, pf_act_bytes(hid, M)) != hipSuccess ||
        hipMalloc(&m->pf_hs, pf_scale_floats(hid / m->gs, M) * 4) != hipSuccess) {
        fprintf(stderr, "llm_prefill: cannot allocate the activations of %d tokens\n", M);
        return -1;
    }
    m->pf_cap = M;
    return 0;
}

// positions p0 .. p0 + M - 1 (token ids in host memory) through every layer; the residual stream of the chunk
// is left in pf_x and its K/V rows in the caches
int prefill_chunk(llm_model *m, const int *ids, int p0, int M) {
    const llm_info &I = m->info;
    const int dim = I.dim, kv = m->kv_dim, wb = m->kind == 0 ? 4 : 8, sf = m->kind == 0 ? 0 : 1;
    HIP_OR_FAIL("llm_prefill", hipMemcpyAsync(m->pf_ids, ids, (size_t)M * 4, hipMemcpyHostToDevice, m->st));
    ProwArgs pa;
    memset(&pa, 0, sizeof pa);
    pa.M = M;
    pa.p0 = p0;
    pa.dim = dim;
    pa.kv_dim = kv;
    pa.head_size = m->hs;
    pa.hidden = I.hidden_dim;
    pa.gs = m->gs;
    pa.qflavor = m->qflavor;
    pa.rope_kind = m->kind == 0 ? ROPE_NEOX : ROPE_INTERLEAVED;
    pa.eps = I.rms_eps;
    pa.ids = m->pf_ids;
    pa.emb_q = m->emb_q;
    pa.emb_s = m->emb_s;
    pa.emb_sf32 = m->emb_sf32;
    pa.x = m->pf_x;
    pa.y = m->pf_y;
    pa.rope_cos = m->rope_cos;
    pa.rope_sin = m->rope_sin;
    pa.q = m->pf_q;
    pa.oq = m->pf_a;
    pa.os = m->pf_s;
    pa.n_heads = I.n_heads;
    pa.n_kv = I.n_kv_heads;
    prefill_att_slices(p0 + M, &pa.att_sl, &pa.att_smax);
    pa.att_ml = m->pf_ml;
    pa.att_acc = m->pf_acc;
    pa.strict = m->strict;
    pa.flash_bf = m->pf_flash_bf;
    pa.xb = m->pf_y; // strict attention rows: the QKV GEMM output is consumed by then
    HIP_OR_FAIL("llm_prefill", launch_p_embed(pa, m->st));
    PgemmArgs g;
    memset(&g, 0, sizeof g);
    g.xq = m->pf_a;
    g.xs = m->pf_s;
    g.y = m->pf_y;
    g.M = M;
    g.simds = 4 * hip_cu_count(m->device);
    g.qflavor = m->qflavor;
    g.strict = m->strict;
    g.hq = m->pf_h;
    g.hsc = m->pf_hs;
    // the SwiGLU epilogue takes int4 gate/up rows in blocks of 8 + 8, groups of 32 and the 16 x 16 .. 32 x 32
    // tiles (the shape the gate/up GEMM gets for M tokens)
    const int gu_shape = pgemm_pick_shape(m->L[0].gu.rows, M, g.simds);
    const bool fuse_swiglu = m->pf_swiglu && wb == 4 && m->gs == 32 && m->L[0].gu.rb == 16 &&
                             m->L[0].gu.rows % 64 == 0 && (gu_shape == 11 || gu_shape == 22);
    // the QKV epilogue takes the 16 x 16 and 32 x 32 tiles
    const int qkv_shape = pgemm_pick_shape(m->L[0].qkv.rows, M, g.simds);
    const bool fuse_qkv = m->pf_qkv && (qkv_shape == 11 || qkv_shape == 22);
    PgemmArgs gq = g;
    gq.qkv = 1;
    gq.rope_cos = m->rope_cos;
    gq.rope_sin = m->rope_sin;
    gq.q = m->pf_q;
    gq.p0 = p0;
    gq.dim = dim;
    gq.kv_dim = kv;
    gq.head_size = m->hs;
    gq.rope_kind = pa.rope_kind;
    for (int l = 0; l < I.n_layers; l++) {
        const Layer &Ly = m->L[l];
        pa.kc = m->kc + (size_t)l * m->ctx * kv;
        pa.vc = m->vc + (size_t)l * m->ctx * kv;
        pa.bias = m->biases ? m->biases + (size_t)l * (dim + 2 * kv) : nullptr;
        pa.norm_w = attn_norm(m, l);
        // after the first layer, the previous down projection's output (in y) joins x before the norm
        HIP_OR_FAIL("llm_prefill", launch_p_norm_quant(pa, l > 0, m->st));
        if (fuse_qkv) {
            gq.W = Ly.qkv;
            gq.bias = pa.bias;
            gq.kc = pa.kc;
            gq.vc = pa.vc;
            HIP_OR_FAIL("llm_prefill", launch_pgemm(wb, m->gs, sf, gq, m->st));
        } else {
            g.W = Ly.qkv;
            HIP_OR_FAIL("llm_prefill", launch_pgemm(wb, m->gs, sf, g, m->st));
            HIP_OR_FAIL("llm_prefill", launch_p_qkv(pa, m->st));
        }
        HIP_OR_FAIL("llm_prefill", launch_p_attention(pa, m->st)); // the o projection's int8 input
        g.W = Ly.o;
        HIP_OR_FAIL("llm_prefill", launch_pgemm(wb, m->gs, sf, g, m->st));
        pa.norm_w = ffn_norm(m, l);
        HIP_OR_FAIL("llm_prefill", launch_p_norm_quant(pa, true, m->st)); // x += o output, then the FFN norm
        g.W = Ly.gu;
        if (fuse_swiglu) { // h straight from the gate/up GEMM into pf_h, the down GEMM's input
            g.swiglu = 1;
            HIP_OR_FAIL("llm_prefill", launch_pgemm(wb, m->gs, sf, g, m->st));
            g.swiglu = 0;
            g.xq = m->pf_h;
            g.xs = m->pf_hs;
        } else {
            HIP_OR_FAIL("llm_prefill", launch_pgemm(wb, m->gs, sf, g, m->st));
            pa.gu_rb = Ly.gu.rb;
            HIP_OR_FAIL("llm_prefill", launch_p_swiglu_quant(pa, m->st));
        }
        g.W = Ly.down;
        HIP_OR_FAIL("llm_prefill", launch_pgemm(wb, m->gs, sf, g, m->st));
        g.xq = m->pf_a;
        g.xs = m->pf_s;
        if (l == I.n_layers - 1) HIP_OR_FAIL("llm_prefill", launch_p_resid(pa, m->st));
    }
    return 0;
}

// Positions pos0 .. pos0 + n - 1 (the cache below pos0 kept), then the head of the last one: logits, argmax
// partials, and (finalize) its argmax into gen[pos0 + n - 1].  Afterwards the step state is position
// pos0 + n - 1, as after those forward() calls.
int prefill_all(llm_model *m, const int *ids, int n, bool sampled = false, int pos0 = 0) {
    if (prefill_alloc(m, std::min(n, PREFILL_CHUNK))) return -1;
    for (int i = 0; i < n; i += PREFILL_CHUNK) {
        const int M = std::min(PREFILL_CHUNK, n - i);
        if (prefill_chunk(m, ids + i, pos0 + i, M)) return -1;
        if (i + M == n)
            HIP_OR_FAIL("llm_prefill", hipMemcpyAsync(m->x, m->pf_x + (size_t)(M - 1) * m->info.dim,
                                                      (size_t)m->info.dim * 4, hipMemcpyDeviceToDevice, m->st));
    }
    HIP_OR_FAIL("llm_prefill", hipMemcpyAsync(m->tokens + pos0, ids, (size_t)n * 4, hipMemcpyHostToDevice, m->st));
    if (set_ctrl(m, pos0 + n - 1, ids[n - 1], 0, 0)) return -1;
    HIP_OR_FAIL("llm_prefill", launch_head(m, false));
    if (sampled) HIP_OR_FAIL("llm_prefill", launch_sampler(m));
    HIP_OR_FAIL("llm_prefill", launch_finalize(m));
    return 0;
}

void free_model(llm_model *m) {
    if (m->st) hipStreamSynchronize(m->st);
    for (hipGraphExec_t g : {m->g_plain, m->g_hist, m->g_plain_s, m->g_hist_s})
        if (g) hipGraphExecDestroy(g);
    for (void *p : m->allocs) hipFree(p);
    if (m->hist) hipFree(m->hist);
    for (void *p : {(void *)m->pf_x, (void *)m->pf_y, (void *)m->pf_q, (void *)m->pf_s,
                    (void *)m->pf_a, (void *)m->pf_ids, (void *)m->pf_ml, (void *)m->pf_acc, (void *)m->pf_h,
                    (void *)m->pf_hs})
        if (p) hipFree(p);
    if (m->st) hipStreamDestroy(m->st);
    if (m->file) munmap((void *)m->file, m->file_size);
    delete m;
}

} // namespace

extern "C" llm_model *llm_open(const char *path, int ctx) {
    const int dev = hip_device_from_env("llm_open");
    if (dev < 0) return nullptr;
    if (hipSetDevice(dev) != hipSuccess) {
        fprintf(stderr, "llm_open: cannot select HIP device %d\n", dev);
        return nullptr;
    }
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        fprintf(stderr, "Couldn't open file %s\n", path);
        return nullptr;
    }
    struct stat stt;
    fstat(fd, &stt);
    llm_model *m = new llm_model();
    memset(&m->info, 0, sizeof m->info);
    m->device = dev;
    m->file_size = (size_t)stt.st_size;
    void *mp = m->file_size >= 256 ? mmap(nullptr, m->file_size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    close(fd);
    if (mp == MAP_FAILED) {
        fprintf(stderr, "%s: cannot map the file (or shorter than a header)\n", path);
        delete m;
        return nullptr;
    }
    m->file = (const uint8_t *)mp;
    if (hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking) != hipSuccess) {
        fprintf(stderr, "llm_open: cannot create a stream\n");
        free_model(m);
        return nullptr;
    }
    int rc;
    uint32_t magic;
    memcpy(&magic, m->file, 4);
    if (!memcmp(m->file, "QWB1", 4)) rc = load_qwb(m, path, ctx);
    else if (magic == 0x616b3432) rc = load_bin(m, path);
    else {
        fprintf(stderr, "%s: neither a .qwb nor a llama2.c .bin file\n", path);
        rc = -1;
    }
    if (rc == 0) rc = finish_setup(m);
    munmap((void *)m->file, m->file_size);
    m->file = nullptr;
    if (rc) {
        free_model(m);
        return nullptr;
    }
    return m;
}

extern "C" int llm_get_info(const llm_model *m, llm_info *info) {
    if (!m || !info) return -1;
    *info = m->info;
    return 0;
}

extern "C" const int32_t *llm_head_ids(const llm_model *m) {
    return m && m->kind == 0 && !m->head_ids_h.empty() ? m->head_ids_h.data() : nullptr;
}

extern "C" int llm_forward(llm_model *m, int token, int pos, float *logits) {
    if (!m) return -1;
    if (pos < 0 || pos >= m->ctx || token < 0 || token >= m->info.vocab_size) {
        fprintf(stderr, "llm_forward: token %d / position %d out of range (vocab %d, context %d)\n", token, pos,
                m->info.vocab_size, m->ctx);
        return -1;
    }
    hipSetDevice(m->device);
    if (set_ctrl(m, pos, token, 0, 0)) return -1;
    if (enqueue_step(m, false, nullptr, pos, true)) return -1;
    if (logits)
        HIP_OR_FAIL("llm_forward", hipMemcpyAsync(logits, m->logits, (size_t)m->info.n_logits * 4,
                                                  hipMemcpyDeviceToHost, m->st));
    HIP_OR_FAIL("llm_forward", hipStreamSynchronize(m->st));
    return 0;
}

static double now_ms() {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e3 + t.tv_nsec / 1e6;
}

// The token loop from position pos0: the n_prompt tokens forced at pos0 .. pos0 + n_prompt - 1 (the KV cache
// below pos0 is what earlier calls left), then up to max_new generated tokens.  stop_id >= 0 replaces the
// format's stop ids.  Positions are absolute: prompt, tokens and gen are indexed by position.
static int generate_from(llm_model *m, int pos0, const int *prompt, int n_prompt, int max_new, int stop_id, int *out,
                         float *logits, llm_timing *timing) {
    if (!m || !prompt || n_prompt < 1 || max_new < 1 || pos0 < 0 || (logits && pos0 > 0)) {
        fprintf(stderr, "llm_generate: bad arguments\n");
        return -1;
    }
    if (pos0 + n_prompt > m->ctx) { // a prompt ending at the last position still yields one token from it
        fprintf(stderr, "prompt (%d tokens from position %d) does not fit -c %d\n", n_prompt, pos0, m->ctx);
        return -1;
    }
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= m->info.vocab_size) {
            fprintf(stderr, "token id %d out of range\n", prompt[i]);
            return -1;
        }
    hipSetDevice(m->device);
    const bool hist = logits != nullptr, smp = m->sampling;
    hipGraphExec_t *g = smp ? (hist ? &m->g_hist_s : &m->g_plain_s) : (hist ? &m->g_hist : &m->g_plain);
    if (hist && !m->hist) {
        if (hipMalloc(&m->hist, (size_t)m->ctx * m->info.n_logits * 4) != hipSuccess) {
            fprintf(stderr, "llm_generate: no room for the logits history\n");
            return -1;
        }
    }
    if (!*g && capture(m, hist, g, 0, smp)) return -1;
    HIP_OR_FAIL("llm_generate", hipMemcpy(m->prompt + pos0, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice));
    const int end_prompt = pos0 + n_prompt; // positions below take their token from the prompt
    if (set_ctrl(m, pos0 - 1, 0, end_prompt, 1)) return -1;
    // positions: the prompt, then one per generated token, within the context
    const int last_pos = std::min(end_prompt - 1 + max_new - 1, m->ctx - 1);
    const double t0 = now_ms();
    if (m->prefill_on && !hist && n_prompt > 1) {
        // the prompt in one batched pass; the first decode step then finishes its last position's argmax
        if (prefill_all(m, prompt, n_prompt, smp, pos0)) return -1;
        if (set_ctrl(m, end_prompt - 1, prompt[n_prompt - 1], end_prompt, 1)) return -1;
    } else {
        for (int p = 0; p < n_prompt; p++) HIP_OR_FAIL("llm_generate", hipGraphLaunch(*g, m->st));
    }
    HIP_OR_FAIL("llm_generate", hipStreamSynchronize(m->st));
    const double t1 = now_ms();
    std::vector<int> gen(m->ctx);
    // gen[p] is the argmax of position p; generated token k is gen[n_prompt - 1 + k].  Steps run in batches,
    // then the batch's tokens are read back and checked for stop ids (qwen.c:684, runq.c:1016).
    const int batch = 16;
    int ran = end_prompt - 1, checked = end_prompt - 1, n_out = 0, used = end_prompt - 1;
    bool done = false;
    while (!done) {
        const int upto = ran + batch < last_pos ? ran + batch : last_pos;
        for (int p = ran + 1; p <= upto; p++) HIP_OR_FAIL("llm_generate", hipGraphLaunch(*g, m->st));
        ran = upto > ran ? upto : ran;
        HIP_OR_FAIL("llm_generate", launch_finalize(m)); // argmax of the batch's last step
        HIP_OR_FAIL("llm_generate", hipMemcpyAsync(gen.data() + checked, m->gen + checked,
                                                   (size_t)(ran - checked + 1) * 4, hipMemcpyDeviceToHost, m->st));
        HIP_OR_FAIL("llm_generate", hipStreamSynchronize(m->st));
        for (int p = checked; p <= ran; p++) {
            const int next = gen[p];
            used = p;
            const bool stop = stop_id >= 0 ? next == stop_id
                                           : m->kind == 0 ? (next == 151645 || next == 151643) : next == 1;
            if (stop) { done = true; break; }
            out[n_out++] = next;
            if (n_out >= max_new || p >= m->ctx - 1) { done = true; break; }
        }
        checked = ran + 1;
        if (ran >= last_pos) done = true;
    }
    const int pos = used;
    const double t2 = now_ms();
    if (timing) {
        timing->n_prompt = n_prompt;
        timing->n_generated = n_out;
        timing->n_forward = pos + 1 - pos0;
        timing->prompt_ms = t1 - t0;
        timing->decode_ms = t2 - t1;
    }
    if (hist)
        HIP_OR_FAIL("llm_generate", hipMemcpy(logits, m->hist, (size_t)(pos + 1) * m->info.n_logits * 4,
                                              hipMemcpyDeviceToHost));
    return n_out;
}

extern "C" int llm_generate(llm_model *m, const int *prompt, int n_prompt, int max_new, int *out, float *logits,
                            llm_timing *timing) {
    return generate_from(m, 0, prompt, n_prompt, max_new, -1, out, logits, timing);
}

extern "C" int llm_continue(llm_model *m, int pos0, const int *tokens, int n, int max_new, int stop_id, int *out,
                            llm_timing *timing) {
    return generate_from(m, pos0, tokens, n, max_new, stop_id, out, nullptr, timing);
}

extern "C" int llm_decode_replay(llm_model *m, int steps, double *ms) {
    if (!m || steps < 1) return -1;
    hipSetDevice(m->device);
    StepCtrl c;
    HIP_OR_FAIL("llm_decode_replay", hipMemcpy(&c, m->ctrl, sizeof c, hipMemcpyDeviceToHost));
    if (c.pos + steps >= m->ctx) {
        fprintf(stderr, "llm_decode_replay: %d steps from position %d do not fit the context %d\n", steps, c.pos, m->ctx);
        return -1;
    }
    c.mode = 1;
    c.n_prompt = 0;
    HIP_OR_FAIL("llm_decode_replay", hipMemcpy(m->ctrl, &c, sizeof c, hipMemcpyHostToDevice));
    hipGraphExec_t *g = m->sampling ? &m->g_plain_s : &m->g_plain;
    if (!*g && capture(m, false, g, 0, m->sampling)) return -1;
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    hipEventRecord(e0, m->st);
    for (int i = 0; i < steps; i++) HIP_OR_FAIL("llm_decode_replay", hipGraphLaunch(*g, m->st));
    hipEventRecord(e1, m->st);
    HIP_OR_FAIL("llm_decode_replay", hipEventSynchronize(e1));
    float t = 0;
    hipEventElapsedTime(&t, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (ms) *ms = t;
    return 0;
}

extern "C" int llm_profile(llm_model *m, int steps, llm_kernel_stat *stats, int max_stats) {
    if (!m || steps < 1 || !stats) return -1;
    hipSetDevice(m->device);
    StepCtrl c;
    HIP_OR_FAIL("llm_profile", hipMemcpy(&c, m->ctrl, sizeof c, hipMemcpyDeviceToHost));
    if (c.pos + steps >= m->ctx) {
        fprintf(stderr, "llm_profile: %d steps from position %d do not fit the context %d\n", steps, c.pos, m->ctx);
        return -1;
    }
    c.mode = 1;
    c.n_prompt = 0;
    HIP_OR_FAIL("llm_profile", hipMemcpy(m->ctrl, &c, sizeof c, hipMemcpyHostToDevice));
    Prof pr;
    double tot[K_COUNT] = {0}, bytes[K_COUNT] = {0};
    int cnt[K_COUNT] = {0};
    for (int s = 0; s < steps; s++) {
        pr.used = 0;
        pr.kind.clear();
        pr.bytes.clear();
        if (enqueue_step(m, false, &pr, c.pos + 1 + s, false)) return -1;
        HIP_OR_FAIL("llm_profile", hipStreamSynchronize(m->st));
        for (size_t i = 0; i < pr.kind.size(); i++) {
            float t = 0;
            hipEventElapsedTime(&t, pr.ev[2 * i], pr.ev[2 * i + 1]);
            tot[pr.kind[i]] += t;
            bytes[pr.kind[i]] += pr.bytes[i];
            cnt[pr.kind[i]]++;
        }
    }
    for (hipEvent_t e : pr.ev) hipEventDestroy(e);
    int n = 0;
    for (int k = 0; k < K_COUNT && n < max_stats; k++) {
        if (!cnt[k]) continue;
        memset(&stats[n], 0, sizeof stats[n]);
        snprintf(stats[n].name, sizeof stats[n].name, "%s", k_names[k]);
        stats[n].launches = cnt[k];
        stats[n].total_ms = tot[k];
        stats[n].bytes_per_launch = bytes[k] / cnt[k];
        n++;
    }
    return n;
}

// In-graph kernel times: the step graph is replayed `steps` times from the current position, then once per
// kernel kind with that kind's launches left out; the difference is that kind's time inside the replayed
// graph (its duration plus its share of the gaps between graph nodes), so launch and event overheads of
// eager timing do not enter it.  Each variant runs `rounds` times, alternating with the full step, and the
// medians are used.  The step control (position, token) is restored at the end.
extern "C" int llm_profile_graph(llm_model *m, int steps, int rounds, llm_kernel_stat *stats, int max_stats,
                                 double *step_ms) {
    if (!m || steps < 1 || rounds < 1 || !stats) return -1;
    hipSetDevice(m->device);
    StepCtrl saved, c;
    HIP_OR_FAIL("llm_profile_graph", hipMemcpy(&saved, m->ctrl, sizeof saved, hipMemcpyDeviceToHost));
    if (saved.pos + steps >= m->ctx) {
        fprintf(stderr, "llm_profile_graph: %d steps from position %d do not fit the context %d\n", steps, saved.pos,
                m->ctx);
        return -1;
    }
    c = saved;
    c.mode = 1;
    c.n_prompt = 0;
    const int kinds[] = {K_EMBED, K_QKV, K_ATTN, K_O, K_GU, K_DOWN, K_HEAD};
    const int nk = sizeof kinds / sizeof kinds[0];
    const int per_step[] = {1, m->info.n_layers, m->info.n_layers, m->info.n_layers, m->info.n_layers,
                            m->info.n_layers, 1};
    std::vector<hipGraphExec_t> g(nk + 1, nullptr);
    int rc = capture(m, false, &g[nk]);
    for (int k = 0; k < nk && !rc; k++) rc = capture(m, false, &g[k], 1u << kinds[k]);
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    auto run = [&](hipGraphExec_t ge, double *ms) -> int {
        HIP_OR_FAIL("llm_profile_graph", hipMemcpyAsync(m->ctrl, &c, sizeof c, hipMemcpyHostToDevice, m->st));
        hipEventRecord(e0, m->st);
        for (int i = 0; i < steps; i++) HIP_OR_FAIL("llm_profile_graph", hipGraphLaunch(ge, m->st));
        hipEventRecord(e1, m->st);
        HIP_OR_FAIL("llm_profile_graph", hipEventSynchronize(e1));
        float t = 0;
        hipEventElapsedTime(&t, e0, e1);
        *ms = t;
        return 0;
    };
    std::vector<std::vector<double>> full(nk), part(nk);
    if (!rc && run(g[nk], step_ms)) rc = -1; // warm-up
    for (int r = 0; r < rounds && !rc; r++)
        for (int k = 0; k < nk && !rc; k++) {
            double a = 0, b = 0;
            if (run(g[nk], &a) || run(g[k], &b)) rc = -1;
            full[k].push_back(a);
            part[k].push_back(b);
        }
    for (hipGraphExec_t ge : g)
        if (ge) hipGraphExecDestroy(ge);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (hipMemcpy(m->ctrl, &saved, sizeof saved, hipMemcpyHostToDevice) != hipSuccess) rc = -1;
    if (rc) return -1;
    auto median = [](std::vector<double> v) {
        std::sort(v.begin(), v.end());
        return v[v.size() / 2];
    };
    std::vector<double> all;
    int n = 0;
    for (int k = 0; k < nk && n < max_stats; k++) {
        const double tf = median(full[k]), tp = median(part[k]);
        all.insert(all.end(), full[k].begin(), full[k].end());
        memset(&stats[n], 0, sizeof stats[n]);
        snprintf(stats[n].name, sizeof stats[n].name, "%s", k_names[kinds[k]]);
        stats[n].launches = per_step[k] * steps;
        stats[n].total_ms = tf - tp;
        stats[n].bytes_per_launch = kind_bytes(m, kinds[k], saved.pos + 1 + steps / 2);
        n++;
    }
    if (step_ms) *step_ms = median(all) / steps;
    return n;
}

extern "C" int llm_read_state(llm_model *m, int which, int layer, float *dst, size_t count) {
    if (!m || !dst) return -1;
    hipSetDevice(m->device);
    const float *src;
    size_t avail;
    if (which == 0) { src = m->x; avail = (size_t)m->info.dim; }
    else if ((which == 1 || which == 2) && layer >= 0 && layer < m->info.n_layers) {
        src = (which == 1 ? m->kc : m->vc) + (size_t)layer * m->ctx * m->kv_dim;
        avail = (size_t)m->ctx * m->kv_dim;
    } else return -1;
    if (count > avail) count = avail;
    HIP_OR_FAIL("llm_read_state", hipMemcpy(dst, src, count * 4, hipMemcpyDeviceToHost));
    return 0;
}

extern "C" int llm_prefill(llm_model *m, const int *ids, int n, float *logits) {
    if (!m || !ids || n < 1 || n > m->ctx) {
        fprintf(stderr, "llm_prefill: bad arguments\n");
        return -1;
    }
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= m->info.vocab_size) {
            fprintf(stderr, "llm_prefill: token id %d out of range\n", ids[i]);
            return -1;
        }
    hipSetDevice(m->device);
    if (prefill_all(m, ids, n)) return -1;
    if (logits)
        HIP_OR_FAIL("llm_prefill", hipMemcpyAsync(logits, m->logits, (size_t)m->info.n_logits * 4,
                                                  hipMemcpyDeviceToHost, m->st));
    HIP_OR_FAIL("llm_prefill", hipStreamSynchronize(m->st));
    return 0;
}

extern "C" int llm_set_sampler(llm_model *m, float temperature, float topp, unsigned long long seed) {
    if (!m) return -1;
    hipSetDevice(m->device);
    HIP_OR_FAIL("llm_set_sampler", hipStreamSynchronize(m->st));
    const size_t n = (size_t)m->info.n_logits;
    if (!m->ss && (dalloc(m, &m->ss, sizeof(SamplerState)) || dalloc(m, &m->smp_p, n * 4) ||
                   dalloc(m, (uint8_t **)&m->smp_scratch, sample_scratch_bytes()) ||
                   dalloc(m, (uint8_t **)&m->smp_strict, sample_strict_scratch_bytes())))
        return -1;
    SamplerState st;
    st.temperature = temperature;
    st.topp = topp;
    st.rng = seed;
    HIP_OR_FAIL("llm_set_sampler", hipMemcpy(m->ss, &st, sizeof st, hipMemcpyHostToDevice));
    m->sampling = temperature > 0.0f; // the reference samples unless the temperature is 0 (qwen.c:647)
    // the sampled step graphs hold one path's launches: captured again when the other one is set
    const int path = topp > 0.0f && topp < 1.0f ? 1 : 0;
    if (path != m->smp_path) {
        for (hipGraphExec_t *g : {&m->g_plain_s, &m->g_hist_s})
            if (*g) {
                hipGraphExecDestroy(*g);
                *g = nullptr;
            }
        m->smp_path = path;
    }
    return 0;
}

extern "C" int llm_sampler_state(llm_model *m, unsigned long long *rng) {
    if (!m || !rng) return -1;
    if (!m->ss) { *rng = 0; return 0; }
    hipSetDevice(m->device);
    SamplerState st;
    HIP_OR_FAIL("llm_sampler_state", hipMemcpy(&st, m->ss, sizeof st, hipMemcpyDeviceToHost));
    *rng = st.rng;
    return 0;
}

extern "C" int llm_set_strict(llm_model *m, int on) {
    if (!m) return -1;
    hipSetDevice(m->device);
    HIP_OR_FAIL("llm_set_strict", hipStreamSynchronize(m->st));
    if ((on != 0) == (m->strict != 0)) return 0;
    m->strict = on != 0;
    if (pick_shapes(m)) {
        m->strict = !m->strict;
        pick_shapes(m);
        return -1;
    }
    // the captured step graphs hold the other mode's kernels and shapes
    for (hipGraphExec_t *g : {&m->g_plain, &m->g_hist, &m->g_plain_s, &m->g_hist_s})
        if (*g) {
            hipGraphExecDestroy(*g);
            *g = nullptr;
        }
    return 0;
}

extern "C" int llm_get_strict(const llm_model *m) { return m ? m->strict : -1; }

extern "C" int llm_set_prefill(llm_model *m, int on) {
    if (!m) return -1;
    m->prefill_on = on != 0;
    return 0;
}

extern "C" void llm_close(llm_model *m) {
    if (!m) return;
    hipSetDevice(m->device);
    free_model(m);
}
