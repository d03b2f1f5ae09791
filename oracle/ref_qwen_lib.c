/* Test harness (oracle infrastructure only): exposes the reference's own qwen.c functions as a shared
 * library so that the CPU restatement in oracle.c can be checked against them function by function.
 * The recipe in oracle/Makefile compiles this file with -I pointing at the reference's qwen/ directory;
 * the reference source is included where it lies, never copied.  Its static functions are visible inside
 * this translation unit, so each wrapper below just forwards to one of them.  Build output: oracle/_ref/. */
#define main qwen_reference_main
#include "qwen.c"
#undef main

float refq_f16(uint16_t h) { return f16(h); }                                       /* qwen.c:84-94 */
void refq_quantize(int8_t *q, float *s, const float *x, int n) { quantize(q, s, x, n); } /* qwen.c:355-364 */
void refq_rmsnorm(float *o, const float *x, const float *w, int n, float eps) { rmsnorm(o, x, w, n, eps); } /* 337-344 */
void refq_softmax(float *x, int n) { softmax(x, n); }                                  /* qwen.c:346-352 */
void refq_rope(float *v, int n_heads, int hs, const float *c, const float *s) { rope(v, n_heads, hs, c, s); } /* 478-488 */
int refq_argmax(const float *p, int n) { return sample_argmax(p, n); }                /* qwen.c:591-598 */
/* sample (qwen.c:647-654) with a Sampler of caller settings; *rng in and out */
int refq_sample(float *logits, int n, float temperature, float topp, unsigned long long *rng) {
    Sampler s = { .vocab_size = n, .temperature = temperature, .topp = topp, .rng_state = *rng,
                  .probindex = malloc((size_t)n * sizeof(ProbIndex)) };
    int r = sample(&s, logits);
    *rng = s.rng_state;
    free(s.probindex);
    return r;
}

/* matmul_cpu (qwen.c:407-457) on caller-owned planes */
void refq_matmul(float *out, const uint8_t *w, const uint16_t *s, int n, int d, int bits, const int8_t *xq,
                 const float *xs) {
    Matrix m;
    memset(&m, 0, sizeof m);
    m.w = w; m.s = s; m.n = n; m.d = d; m.bits = bits;
    matmul_cpu(out, &m, xq, xs);
}

/* whole model: build_transformer (qwen.c:320-330) and forward (qwen.c:490-573) */
void *refq_open(const char *path, int ctx) {
    Transformer *t = calloc(1, sizeof *t);
    build_transformer(t, path, ctx);
    return t;
}
const float *refq_forward(void *t, int token, int pos) { return forward((Transformer *)t, token, pos); }
int refq_head_k(void *t) { return ((Transformer *)t)->c.head_k; }
const int32_t *refq_head_ids(void *t) { return ((Transformer *)t)->w.head_ids; }
/* the residual stream after forward(): x holds the final rmsnorm output (qwen.c:569) */
const float *refq_x(void *t) { return ((Transformer *)t)->s.x; }
const float *refq_kv(void *t, int which) { Transformer *m = t; return which ? m->s.value_cache : m->s.key_cache; }
