/* CPU oracle for the decode token loop: a plain-C restatement of the reference's arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Compiled with strict IEEE flags (no -ffast-math, no FMA
 * contraction) so that every float operation happens in the order written, which is the order of the
 * reference's plain-C path; the pinning tests then demand bit-exact agreement with the reference's own
 * functions built the same way.
 *
 * Parity status per function (how each is pinned, all in tests/test_oracle.py):
 *   or_f16               closed form (every one of the 65536 bit patterns against ldexp), reference f16()
 *   or_quantize_qwen     reference quantize() bit-exact; crafted groups (ties, zero, tiny, +-127)
 *   or_quantize_runq     reference runq quantize() bit-exact; crafted groups
 *   or_matvec4(_groups)  reference matmul_cpu() bit-exact; brute-force group sums; unit scales give ival
 *   or_matvec_runq       reference runq matmul() bit-exact (the reference testbench's own bar)
 *   or_rmsnorm/softmax   reference functions bit-exact
 *   or_rope_*            reference rope() bit-exact; closed form at pos 0 (identity)
 *   or_argmax            reference sample_argmax(); ties resolve to the lowest index
 *   or_sample            xorshift stream against the published xorshift64* constants; reference sampler
 *                        reached through the reference binaries' -t/-p/-s runs
 *   or_open/or_forward   whole-model logits bit-exact against the reference binaries and libraries,
 *                        and against the committed golden fixtures
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------------------- */
/* scalar helpers */

/* fp16 bits -> float (qwen.c:84-94): exact for zero, subnormals and normals.  The reference rebiases
 * exponent 31 like a normal number because scales never hold inf/nan; this restatement gives IEEE inf/nan
 * there instead, which is what the GPU's hardware conversion does.  Valid files never contain it. */
float or_f16(uint16_t h) {
    int e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(1024 + m), e - 25);
    return (h >> 15) ? -v : v;
}

uint16_t or_f32_to_f16(float f) {
    union { float f; uint32_t u; } in = { .f = f };
    uint32_t u = in.u, sign = (u >> 16) & 0x8000;
    int32_t e = (int32_t)((u >> 23) & 0xff) - 127 + 15;
    uint32_t m = u & 0x7fffff;
    if (((u >> 23) & 0xff) == 0xff) return (uint16_t)(sign | 0x7c00 | (m ? 0x200 : 0));
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) { /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000;
        int shift = 14 - e;
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (m >> 13), rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

/* What x86-64 produces for the reference's (int8_t)roundf(v): cvttss2si to int32 (out-of-range and NaN
 * give 0x80000000), then the low byte.  Spelled out so the result does not rest on undefined behaviour. */
static int8_t x86_to_i8(double r) {
    if (!(fabs(r) < 2147483648.0)) return 0;
    return (int8_t)(uint8_t)((uint32_t)(int32_t)r & 0xff);
}

/* ---------------------------------------------------------------------------------------------------- */
/* quantization */

/* qwen.c:354-364: scale = max|x| * (1/127), q = roundf(x * (1/scale)), halves away from zero */
void or_quantize_qwen(int8_t *q, float *s, const float *x, int n) {
    for (int g = 0; g < n / 32; g++) {
        float wmax = 0.0f;
        for (int i = 0; i < 32; i++) wmax = fmaxf(wmax, fabsf(x[g * 32 + i]));
        float scale = wmax * (1.0f / 127.0f);
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        s[g] = scale;
        for (int i = 0; i < 32; i++) q[g * 32 + i] = x86_to_i8(roundf(x[g * 32 + i] * inv));
    }
}

/* runq.c:244-270: scale = max|x| / 127, q = round(x / scale); scale 0 gives q 0 (x86) */
void or_quantize_runq(int8_t *q, float *s, const float *x, int n, int gs) {
    for (int g = 0; g < n / gs; g++) {
        float wmax = 0.0f;
        for (int i = 0; i < gs; i++) {
            float v = fabsf(x[g * gs + i]);
            if (v > wmax) wmax = v;
        }
        float scale = wmax / 127.0f;
        s[g] = scale;
        for (int i = 0; i < gs; i++) {
            float v = x[g * gs + i] / scale;
            q[g * gs + i] = x86_to_i8(round((double)v));
        }
    }
}

/* ---------------------------------------------------------------------------------------------------- */
/* GEMV */

/* signed element k of a 4-bit row (two's complement; element 2i in the low nibble of byte i: qwen.c:45, 447) */
static inline int nib(const uint8_t *row, int k) {
    int b = row[k >> 1];
    int v = (k & 1) ? (b >> 4) : (b & 15);
    return v >= 8 ? v - 16 : v;
}

void or_matvec4_groups(int32_t *ival, const uint8_t *w, const int8_t *xq, int n, int d, int bits) {
    const int ng = n / 32;
    const size_t row = (size_t)n * bits / 8;
    for (int i = 0; i < d; i++) {
        const uint8_t *r = w + (size_t)i * row;
        for (int g = 0; g < ng; g++) {
            int32_t acc = 0;
            for (int k = 0; k < 32; k++) {
                int wv = bits == 4 ? nib(r, g * 32 + k) : (int8_t)r[g * 32 + k];
                acc += wv * xq[g * 32 + k];
            }
            ival[(size_t)i * ng + g] = acc;
        }
    }
}

/* Order of the fp32 sum over a row's groups: 1 (default) is the reference's sequential loop; k > 1 keeps
 * k interleaved partial sums added as a tree at the end.  Only the tolerance-rationale test changes it, to
 * show how far the reference's own arithmetic moves under a mere reordering of that sum. */
static int sum_ways = 1;
void or_set_sum_ways(int k) { sum_ways = k >= 1 && k <= 8 ? k : 1; }

/* qwen.c:436-456 (plain C path): per row, groups summed in order, p_g = ((float)ival * ws) * xs */
void or_matvec4(float *out, const uint8_t *w, const uint16_t *ws, const int8_t *xq, const float *xs, int n, int d,
                int bits) {
    const int ng = n / 32;
    const size_t row = (size_t)n * bits / 8;
    for (int i = 0; i < d; i++) {
        const uint8_t *r = w + (size_t)i * row;
        const uint16_t *s = ws + (size_t)i * ng;
        float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int g = 0; g < ng; g++) {
            int32_t acc = 0;
            for (int k = 0; k < 32; k++) {
                int wv = bits == 4 ? nib(r, g * 32 + k) : (int8_t)r[g * 32 + k];
                acc += wv * xq[g * 32 + k];
            }
            float p = (float)acc * or_f16(s[g]);
            p = p * xs[g];
            part[g % sum_ways] = part[g % sum_ways] + p;
        }
        float val = part[0];
        for (int k = 1; k < sum_ways; k++) val = val + part[k];
        out[i] = val;
    }
}

void or_matvec_runq_groups(int32_t *ival, const int8_t *wq, const int8_t *xq, int n, int d, int gs) {
    const int ng = n / gs;
    for (int i = 0; i < d; i++)
        for (int g = 0; g < ng; g++) {
            int32_t acc = 0;
            for (int k = 0; k < gs; k++) acc += (int32_t)xq[g * gs + k] * (int32_t)wq[(size_t)i * n + g * gs + k];
            ival[(size_t)i * ng + g] = acc;
        }
}

/* runq.c:429-458: val += ((float)ival * ws) * xs, groups in order */
void or_matvec_runq(float *out, const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int n, int d,
                    int gs) {
    const int ng = n / gs;
    for (int i = 0; i < d; i++) {
        float val = 0.0f;
        for (int g = 0; g < ng; g++) {
            int32_t acc = 0;
            for (int k = 0; k < gs; k++) acc += (int32_t)xq[g * gs + k] * (int32_t)wq[(size_t)i * n + g * gs + k];
            float p = (float)acc * ws[(size_t)i * ng + g];
            p = p * xs[g];
            val = val + p;
        }
        out[i] = val;
    }
}

/* ---------------------------------------------------------------------------------------------------- */
/* element-wise blocks */

/* qwen.c:337-344 (runq.c:394-407 is the same with eps 1e-5f) */
static int norm_ways = 1;
void or_set_norm_ways(int k) { norm_ways = k >= 1 && k <= 8 ? k : 1; }

void or_rmsnorm(float *o, const float *x, const float *w, int n, float eps) {
    float ss = 0.0f;
    if (norm_ways == 1) {
        for (int j = 0; j < n; j++) ss += x[j] * x[j];
    } else { /* tolerance experiments only: k interleaved partial sums, added in order */
        float part[8] = {0};
        for (int j = 0; j < n; j++) part[j % norm_ways] += x[j] * x[j];
        for (int k = 0; k < norm_ways; k++) ss += part[k];
    }
    ss /= (float)n;
    ss += eps;
    ss = 1.0f / sqrtf(ss);
    for (int j = 0; j < n; j++) o[j] = w[j] * (ss * x[j]);
}

/* expf of the C library the reference links (glibc on the hosts here), element by element: the function the
 * reference's softmax (qwen.c:350, runq.c:420) and SiLU (qwen.c:560, runq.c:592) call */
void or_expf(const float *x, int n, float *y) {
    for (int i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* qwen.c:346-352 */
void or_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

/* qwen.c:503-508: angle pos * theta^(-2i/hs) in double, then cast */
void or_rope_angles(float *c, float *s, int hs, int pos, float theta) {
    for (int i = 0; i < hs / 2; i++) {
        double a = pos * pow((double)theta, -2.0 * i / hs);
        c[i] = (float)cos(a);
        s[i] = (float)sin(a);
    }
}

/* qwen.c:478-488: rotate-half pairs (i, i + hs/2) of every head */
void or_rope_neox(float *v, int n_heads, int hs, const float *c, const float *s) {
    for (int h = 0; h < n_heads; h++) {
        float *p = v + (size_t)h * hs;
        for (int i = 0; i < hs / 2; i++) {
            float a = p[i], b = p[i + hs / 2];
            float a1 = a * c[i], b1 = b * s[i];
            float b2 = b * c[i], a2 = a * s[i];
            p[i] = a1 - b1;
            p[i + hs / 2] = b2 + a2;
        }
    }
}

/* runq.c:506-521: interleaved pairs (i, i+1), float powf/cosf/sinf, theta 10000 */
void or_rope_runq(float *q, float *k, int dim, int kv_dim, int hs, int pos) {
    for (int i = 0; i < dim; i += 2) {
        int hd = i % hs;
        float freq = 1.0f / powf(10000.0f, hd / (float)hs);
        float val = pos * freq;
        float fcr = cosf(val), fci = sinf(val);
        for (int v = 0; v < (i < kv_dim ? 2 : 1); v++) {
            float *vec = v == 0 ? q : k;
            float v0 = vec[i], v1 = vec[i + 1];
            float a = v0 * fcr, b = v1 * fci, c2 = v0 * fci, d2 = v1 * fcr;
            vec[i] = a - b;
            vec[i + 1] = c2 + d2;
        }
    }
}

/* qwen.c:591-598: first index of the strict maximum */
int or_argmax(const float *p, int n) {
    int mi = 0;
    float mp = p[0];
    for (int i = 1; i < n; i++)
        if (p[i] > mp) { mi = i; mp = p[i]; }
    return mi;
}

/* ---------------------------------------------------------------------------------------------------- */
/* sampler: xorshift64* (qwen.c:638-645) and the llama2.c sampling rules (qwen.c:600-654) */

unsigned int or_random_u32(unsigned long long *state) {
    unsigned long long x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return (unsigned int)((x * 0x2545F4914F6CDD1Dull) >> 32);
}

float or_random_f32(unsigned long long *state) { return (or_random_u32(state) >> 8) / 16777216.0f; }

typedef struct { float p; int i; } or_pi;
/* qwen.c:609-614 orders by probability only; C leaves the order of equal keys to qsort, and glibc's qsort
 * (a merge sort while the array fits in memory) keeps them in their input order, i.e. ascending index.  The
 * index tie-break states that order explicitly. */
static int by_prob_desc(const void *a, const void *b) {
    float x = ((const or_pi *)a)->p, y = ((const or_pi *)b)->p;
    if (x != y) return x > y ? -1 : 1;
    int i = ((const or_pi *)a)->i, j = ((const or_pi *)b)->i;
    return i < j ? -1 : i > j ? 1 : 0;
}

int or_sample(float *logits, int n, float temperature, float topp, unsigned long long *rng) {
    if (temperature == 0.0f) return or_argmax(logits, n);
    for (int i = 0; i < n; i++) logits[i] /= temperature;
    or_softmax(logits, n);
    float coin = or_random_f32(rng);
    if (topp <= 0 || topp >= 1) { /* qwen.c:600-607 */
        float cdf = 0.0f;
        for (int i = 0; i < n; i++) {
            cdf += logits[i];
            if (coin < cdf) return i;
        }
        return n - 1;
    }
    /* qwen.c:616-636: keep p >= (1-topp)/(n-1), sort descending, cut where the sum passes topp */
    or_pi *c = malloc((size_t)n * sizeof *c);
    int n0 = 0;
    const float cutoff = (1.0f - topp) / (n - 1);
    for (int i = 0; i < n; i++)
        if (logits[i] >= cutoff) { c[n0].i = i; c[n0].p = logits[i]; n0++; }
    qsort(c, n0, sizeof *c, by_prob_desc);
    float cum = 0.0f;
    int last = n0 - 1;
    for (int i = 0; i < n0; i++) {
        cum += c[i].p;
        if (cum > topp) { last = i; break; }
    }
    float r = coin * cum, cdf = 0.0f;
    int res = c[last].i;
    for (int i = 0; i <= last; i++) {
        cdf += c[i].p;
        if (r < cdf) { res = c[i].i; break; }
    }
    free(c);
    return res;
}

/* ---------------------------------------------------------------------------------------------------- */
/* whole models */

typedef struct { const uint8_t *w; const uint16_t *s; int n, d, bits; } q4mat;   /* .qwb matrix */
typedef struct { const int8_t *q; const float *s; } q8t;                         /* runq tensor */

struct or_model {
    int kind; /* 0 qwen (.qwb), 1 runq (.bin) */
    uint8_t *file;
    size_t size;
    /* config */
    int dim, hidden, L, heads, kv_heads, vocab, head_k, max_seq, gs, hs, kv_dim, ctx;
    float theta, eps;
    /* qwen weights */
    const float *attn_norm, *ffn_norm, *bq, *bk, *bv, *out_norm;
    const int32_t *head_ids;
    q4mat *wq, *wk, *wv, *wo, *w1, *w2, *w3, head, emb;
    /* runq weights */
    const float *rms_att, *rms_ffn, *rms_final;
    q8t tok, *rwq, *rwk, *rwv, *rwo, *rw1, *rw2, *rw3, cls;
    /* state */
    float *x, *xb, *xb2, *hb, *hb2, *q, *att, *logits, *kc, *vc, *rc, *rs;
    int8_t *xq;
    float *xs;
};

static size_t pad64(size_t b) { return (b + 63) & ~(size_t)63; }

/* .qwb walk (qwen.c:211-271; layout gguf2qwb.py:5-14) */
static int open_qwb(or_model *m, const char *path) {
    const uint8_t *b = m->file;
    int32_t h[10];
    memcpy(h, b + 8, 40);
    m->dim = h[0]; m->hidden = h[1]; m->L = h[2]; m->heads = h[3]; m->kv_heads = h[4]; m->vocab = h[5];
    m->head_k = h[6]; m->max_seq = h[7]; m->gs = h[8];
    int emb_bits = h[9];
    memcpy(&m->theta, b + 48, 4);
    memcpy(&m->eps, b + 52, 4);
    if (memcmp(b + 4, "\1\0\0\0", 4)) { fprintf(stderr, "%s: not a .qwb version 1 file\n", path); return -1; }
    if (m->heads <= 0 || m->kv_heads <= 0) { fprintf(stderr, "%s: bad header\n", path); return -1; }
    m->hs = m->dim / m->heads;
    m->kv_dim = m->hs * m->kv_heads;
    if (m->gs != 32 || emb_bits != 8 || m->dim % m->heads || m->heads % m->kv_heads || m->hs % 2 || m->dim % 128 ||
        m->kv_dim % 16 || m->hidden % 128) { /* qwen.c:223-228 */
        fprintf(stderr, "%s: unsupported config\n", path);
        return -1;
    }
    size_t off = 256;
#define TAKE(bytes) (off += pad64(bytes), b + off - pad64(bytes))
    int L = m->L, dim = m->dim, kv = m->kv_dim;
    m->attn_norm = (const float *)TAKE((size_t)L * dim * 4);
    m->ffn_norm = (const float *)TAKE((size_t)L * dim * 4);
    m->bq = (const float *)TAKE((size_t)L * dim * 4);
    m->bk = (const float *)TAKE((size_t)L * kv * 4);
    m->bv = (const float *)TAKE((size_t)L * kv * 4);
    m->out_norm = (const float *)TAKE((size_t)dim * 4);
    m->head_ids = (const int32_t *)TAKE((size_t)m->head_k * 4);
    q4mat **lists[7] = { &m->wq, &m->wk, &m->wv, &m->wo, &m->w1, &m->w2, &m->w3 };
    int shapes[7][2] = { { dim, dim }, { kv, dim }, { kv, dim }, { dim, dim }, { m->hidden, dim }, { dim, m->hidden },
                         { m->hidden, dim } };
    for (int a = 0; a < 7; a++) {
        *lists[a] = calloc(L, sizeof(q4mat));
        for (int l = 0; l < L; l++) {
            q4mat *q = &(*lists[a])[l];
            q->d = shapes[a][0]; q->n = shapes[a][1]; q->bits = 4;
            q->w = TAKE((size_t)q->d * q->n / 2);
            q->s = (const uint16_t *)TAKE((size_t)q->d * q->n / 32 * 2);
        }
    }
    m->head = (q4mat){ .n = dim, .d = m->head_k, .bits = 8 };
    m->head.w = TAKE((size_t)m->head_k * dim);
    m->head.s = (const uint16_t *)TAKE((size_t)m->head_k * dim / 32 * 2);
    m->emb = (q4mat){ .n = dim, .d = m->vocab, .bits = 8 };
    m->emb.w = TAKE((size_t)m->vocab * dim);
    m->emb.s = (const uint16_t *)TAKE((size_t)m->vocab * dim / 32 * 2);
#undef TAKE
    if (off != m->size) { fprintf(stderr, "%s: size %zu, header describes %zu\n", path, m->size, off); return -1; }
    return 0;
}

/* llama2.c v2 .bin (runq.c:291-357) */
static int open_bin(or_model *m, const char *path) {
    const uint8_t *b = m->file;
    int32_t h[7];
    memcpy(h, b + 8, 28);
    m->dim = h[0]; m->hidden = h[1]; m->L = h[2]; m->heads = h[3]; m->kv_heads = h[4]; m->vocab = h[5];
    m->max_seq = h[6];
    uint8_t shared = b[36];
    memcpy(&m->gs, b + 37, 4);
    int version;
    memcpy(&version, b + 4, 4);
    if (version != 2) { fprintf(stderr, "%s: bad version %d\n", path, version); return -1; }
    if (m->gs <= 0 || m->heads <= 0 || m->kv_heads <= 0 || m->dim % m->gs || m->hidden % m->gs) {
        fprintf(stderr, "%s: unsupported config\n", path);
        return -1;
    }
    m->hs = m->dim / m->heads;
    m->kv_dim = m->dim * m->kv_heads / m->heads;
    m->eps = 1e-5f;
    m->theta = 10000.0f;
    m->head_k = m->vocab;
    const uint8_t *p = b + 256;
    int L = m->L, dim = m->dim;
    m->rms_att = (const float *)p; p += (size_t)L * dim * 4;
    m->rms_ffn = (const float *)p; p += (size_t)L * dim * 4;
    m->rms_final = (const float *)p; p += (size_t)dim * 4;
#define TENSOR(t, nel) do { (t).q = (const int8_t *)p; p += (size_t)(nel); (t).s = (const float *)p; p += (size_t)(nel) / m->gs * 4; } while (0)
    TENSOR(m->tok, (size_t)m->vocab * dim);
    q8t **lists[7] = { &m->rwq, &m->rwk, &m->rwv, &m->rwo, &m->rw1, &m->rw2, &m->rw3 };
    size_t nel[7] = { (size_t)dim * dim, (size_t)dim * m->kv_dim, (size_t)dim * m->kv_dim, (size_t)dim * dim,
                      (size_t)dim * m->hidden, (size_t)dim * m->hidden, (size_t)dim * m->hidden };
    for (int a = 0; a < 7; a++) {
        *lists[a] = calloc(L, sizeof(q8t));
        for (int l = 0; l < L; l++) TENSOR((*lists[a])[l], nel[a]);
    }
    if (shared) m->cls = m->tok;
    else TENSOR(m->cls, (size_t)m->vocab * dim);
#undef TENSOR
    if ((size_t)(p - b) > m->size) { fprintf(stderr, "%s: file too short\n", path); return -1; }
    return 0;
}

or_model *or_open(const char *path, int ctx) {
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "cannot open %s\n", path); return NULL; }
    or_model *m = calloc(1, sizeof *m);
    fseek(f, 0, SEEK_END);
    m->size = (size_t)ftell(f);
    fseek(f, 0, SEEK_SET);
    m->file = malloc(m->size);
    if (m->size < 256 || fread(m->file, 1, m->size, f) != m->size) {
        fprintf(stderr, "%s: short file\n", path);
        fclose(f);
        or_close(m);
        return NULL;
    }
    fclose(f);
    uint32_t magic;
    memcpy(&magic, m->file, 4);
    int rc;
    if (!memcmp(m->file, "QWB1", 4)) { m->kind = 0; rc = open_qwb(m, path); }
    else if (magic == 0x616b3432) { m->kind = 1; rc = open_bin(m, path); }
    else { fprintf(stderr, "%s: unknown format\n", path); rc = -1; }
    if (rc) { or_close(m); return NULL; }
    /* qwen: ctx = min(-c, max_seq_len) (qwen.c:325); runq: the cache is seq_len long (runq.c:203) */
    m->ctx = m->kind == 0 ? (ctx < m->max_seq ? ctx : m->max_seq) : m->max_seq;
    int maxn = m->hidden > m->dim ? m->hidden : m->dim;
    m->x = calloc(m->dim, 4); m->xb = calloc(m->dim, 4); m->xb2 = calloc(m->dim, 4);
    m->hb = calloc(m->hidden, 4); m->hb2 = calloc(m->hidden, 4); m->q = calloc(m->dim, 4);
    m->att = calloc((size_t)m->heads * m->ctx, 4);
    m->logits = calloc(m->head_k, 4);
    m->kc = calloc((size_t)m->L * m->ctx * m->kv_dim, 4);
    m->vc = calloc((size_t)m->L * m->ctx * m->kv_dim, 4);
    m->rc = calloc(m->hs / 2, 4); m->rs = calloc(m->hs / 2, 4);
    m->xq = calloc(maxn, 1); m->xs = calloc(maxn, 4);
    return m;
}

int or_n_logits(const or_model *m) { return m->head_k; }
const int32_t *or_head_ids(const or_model *m) { return m->kind == 0 ? m->head_ids : NULL; }
int or_ctx(const or_model *m) { return m->ctx; }
int or_kind(const or_model *m) { return m->kind; }

void or_close(or_model *m) {
    if (!m) return;
    q4mat *a[7] = { m->wq, m->wk, m->wv, m->wo, m->w1, m->w2, m->w3 };
    q8t *r[7] = { m->rwq, m->rwk, m->rwv, m->rwo, m->rw1, m->rw2, m->rw3 };
    for (int i = 0; i < 7; i++) { free(a[i]); free(r[i]); }
    free(m->x); free(m->xb); free(m->xb2); free(m->hb); free(m->hb2); free(m->q); free(m->att); free(m->logits);
    free(m->kc); free(m->vc); free(m->rc); free(m->rs); free(m->xq); free(m->xs); free(m->file); free(m);
}

/* attention of one layer over positions 0..pos (qwen.c:526-546, runq.c:530-568), result into xb */
static void attention(or_model *m, int l, int pos) {
    int hs = m->hs, kv_mul = m->heads / m->kv_heads;
    size_t loff = (size_t)l * m->ctx * m->kv_dim;
    for (int h = 0; h < m->heads; h++) {
        const float *q = m->q + (size_t)h * hs;
        float *att = m->att + (size_t)h * m->ctx;
        for (int t = 0; t <= pos; t++) {
            const float *k = m->kc + loff + (size_t)t * m->kv_dim + (size_t)(h / kv_mul) * hs;
            float score = 0.0f;
            for (int i = 0; i < hs; i++) score += q[i] * k[i];
            att[t] = score / sqrtf((float)hs);
        }
        or_softmax(att, pos + 1);
        float *xb = m->xb + (size_t)h * hs;
        memset(xb, 0, (size_t)hs * 4);
        for (int t = 0; t <= pos; t++) {
            const float *v = m->vc + loff + (size_t)t * m->kv_dim + (size_t)(h / kv_mul) * hs;
            float a = att[t];
            for (int i = 0; i < hs; i++) xb[i] += a * v[i];
        }
    }
}

static void swiglu(float *hb, const float *hb2, int n) { /* qwen.c:558-562, runq.c:589-596 */
    for (int i = 0; i < n; i++) {
        float v = hb[i];
        v *= (1.0f / (1.0f + expf(-v)));
        hb[i] = v * hb2[i];
    }
}

static void mv4(or_model *m, float *out, const q4mat *w) { or_matvec4(out, w->w, w->s, m->xq, m->xs, w->n, w->d, w->bits); }
static void mvr(or_model *m, float *out, const q8t *w, int n, int d) { or_matvec_runq(out, w->q, w->s, m->xq, m->xs, n, d, m->gs); }

/* qwen.c:490-573 */
static const float *forward_qwen(or_model *m, int token, int pos) {
    int dim = m->dim, kv = m->kv_dim, hs = m->hs;
    const int8_t *er = (const int8_t *)m->emb.w + (size_t)token * dim;
    const uint16_t *es = m->emb.s + (size_t)token * dim / 32;
    for (int i = 0; i < dim; i++) m->x[i] = er[i] * or_f16(es[i / 32]);
    or_rope_angles(m->rc, m->rs, hs, pos, m->theta);
    for (int l = 0; l < m->L; l++) {
        size_t loff = (size_t)l * m->ctx * kv;
        float *k = m->kc + loff + (size_t)pos * kv, *v = m->vc + loff + (size_t)pos * kv;
        or_rmsnorm(m->xb, m->x, m->attn_norm + (size_t)l * dim, dim, m->eps);
        or_quantize_qwen(m->xq, m->xs, m->xb, dim);
        mv4(m, m->q, &m->wq[l]);
        mv4(m, k, &m->wk[l]);
        mv4(m, v, &m->wv[l]);
        for (int i = 0; i < dim; i++) m->q[i] += m->bq[(size_t)l * dim + i];
        for (int i = 0; i < kv; i++) { k[i] += m->bk[(size_t)l * kv + i]; v[i] += m->bv[(size_t)l * kv + i]; }
        or_rope_neox(m->q, m->heads, hs, m->rc, m->rs);
        or_rope_neox(k, m->kv_heads, hs, m->rc, m->rs);
        attention(m, l, pos);
        or_quantize_qwen(m->xq, m->xs, m->xb, dim);
        mv4(m, m->xb2, &m->wo[l]);
        for (int i = 0; i < dim; i++) m->x[i] += m->xb2[i];
        or_rmsnorm(m->xb, m->x, m->ffn_norm + (size_t)l * dim, dim, m->eps);
        or_quantize_qwen(m->xq, m->xs, m->xb, dim);
        mv4(m, m->hb, &m->w1[l]);
        mv4(m, m->hb2, &m->w3[l]);
        swiglu(m->hb, m->hb2, m->hidden);
        or_quantize_qwen(m->xq, m->xs, m->hb, m->hidden);
        mv4(m, m->xb, &m->w2[l]);
        for (int i = 0; i < dim; i++) m->x[i] += m->xb[i];
    }
    or_rmsnorm(m->x, m->x, m->out_norm, dim, m->eps);
    or_quantize_qwen(m->xq, m->xs, m->x, dim);
    mv4(m, m->logits, &m->head); /* the reference splits this into 2048-row calls; rows are independent */
    return m->logits;
}

/* runq.c:477-615 */
static const float *forward_runq(or_model *m, int token, int pos) {
    int dim = m->dim, kv = m->kv_dim, hs = m->hs, gs = m->gs;
    for (int i = 0; i < dim; i++) m->x[i] = m->tok.q[(size_t)token * dim + i] * m->tok.s[((size_t)token * dim + i) / gs];
    for (int l = 0; l < m->L; l++) {
        size_t loff = (size_t)l * m->ctx * kv;
        float *k = m->kc + loff + (size_t)pos * kv, *v = m->vc + loff + (size_t)pos * kv;
        or_rmsnorm(m->xb, m->x, m->rms_att + (size_t)l * dim, dim, 1e-5f);
        or_quantize_runq(m->xq, m->xs, m->xb, dim, gs);
        mvr(m, m->q, &m->rwq[l], dim, dim);
        mvr(m, k, &m->rwk[l], dim, kv);
        mvr(m, v, &m->rwv[l], dim, kv);
        or_rope_runq(m->q, k, dim, kv, hs, pos);
        attention(m, l, pos);
        or_quantize_runq(m->xq, m->xs, m->xb, dim, gs);
        mvr(m, m->xb2, &m->rwo[l], dim, dim);
        for (int i = 0; i < dim; i++) m->x[i] += m->xb2[i];
        or_rmsnorm(m->xb, m->x, m->rms_ffn + (size_t)l * dim, dim, 1e-5f);
        or_quantize_runq(m->xq, m->xs, m->xb, dim, gs);
        mvr(m, m->hb, &m->rw1[l], dim, m->hidden);
        mvr(m, m->hb2, &m->rw3[l], dim, m->hidden);
        swiglu(m->hb, m->hb2, m->hidden);
        or_quantize_runq(m->xq, m->xs, m->hb, m->hidden, gs);
        mvr(m, m->xb, &m->rw2[l], m->hidden, dim);
        for (int i = 0; i < dim; i++) m->x[i] += m->xb[i];
    }
    or_rmsnorm(m->x, m->x, m->rms_final, dim, 1e-5f);
    or_quantize_runq(m->xq, m->xs, m->x, dim, gs);
    mvr(m, m->logits, &m->cls, dim, m->vocab);
    return m->logits;
}

const float *or_forward(or_model *m, int token, int pos) {
    return m->kind == 0 ? forward_qwen(m, token, pos) : forward_runq(m, token, pos);
}

/* greedy generate with the reference's stop rules: qwen.c:669-712 (stop ids 151645/151643, at most
 * `steps` new tokens, ctx positions) or runq.c:982-1036 (stop on BOS 1, `steps` positions in total) */
int or_generate_greedy(or_model *m, const int *prompt, int n_prompt, int steps, int *out, int max_out) {
    int n = 0, token = prompt[0];
    if (m->kind == 0) {
        for (int pos = 0; pos < m->ctx; pos++) {
            const float *lg = or_forward(m, token, pos);
            if (pos < n_prompt - 1) { token = prompt[pos + 1]; continue; }
            int next = m->head_ids[or_argmax(lg, m->head_k)];
            if (next == 151645 || next == 151643) break;
            if (n < max_out) out[n] = next;
            n++;
            if (n >= steps) break;
            token = next;
        }
    } else {
        if (steps <= 0 || steps > m->max_seq) steps = m->max_seq;
        for (int pos = 0; pos < steps;) {
            const float *lg = or_forward(m, token, pos);
            int next = pos < n_prompt - 1 ? prompt[pos + 1] : or_argmax(lg, m->vocab);
            pos++;
            if (next == 1) break;
            if (pos >= n_prompt) {
                if (n < max_out) out[n] = next;
                n++;
            }
            token = next;
        }
    }
    return n;
}
