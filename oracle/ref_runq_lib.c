/* Test harness (oracle infrastructure only): the reference's runq.c compiled as a library, in the
 * llama2.c test pattern (TESTING hides its main, runq.c:1142).  All of runq.c's functions are external,
 * so the library exports quantize, matmul, rmsnorm, forward, ... directly; the few helpers below only
 * fill runq.c's structs from plain pointers.  The reference source is included where it lies (the recipe
 * passes -I to the reference's runq/ directory).  Build output: oracle/_ref/. */
#define TESTING
#include "runq.c"

/* runq.c:244-270 with the global GS set first */
void refr_quantize(int8_t *q, float *s, float *x, int n, int gs) {
    GS = gs;
    QuantizedTensor t = { .q = q, .s = s };
    quantize(&t, x, n);
}
/* runq.c:429-458 (matmul, or matmul_cpu in an FPGA build) */
void refr_matmul(float *out, int8_t *xq, float *xs, int8_t *wq, float *ws, int n, int d, int gs) {
    GS = gs;
    QuantizedTensor x = { .q = xq, .s = xs }, w = { .q = wq, .s = ws };
#ifdef FPGA
    matmul_cpu(out, &x, &w, n, d);
#else
    matmul(out, &x, &w, n, d);
#endif
}
void refr_rmsnorm(float *o, float *x, float *w, int n) { rmsnorm(o, x, w, n); }
void *refr_open(const char *path) {
    Transformer *t = calloc(1, sizeof *t);
    build_transformer(t, (char *)path);
    return t;
}
float *refr_forward(void *t, int token, int pos) { return forward((Transformer *)t, token, pos); }
int refr_vocab(void *t) { return ((Transformer *)t)->config.vocab_size; }
int refr_seq_len(void *t) { return ((Transformer *)t)->config.seq_len; }
int refr_argmax(float *p, int n) { return sample_argmax(p, n); }
/* key (which 0) or value (1) cache of the reference's RunState: [n_layers][seq_len][kv_dim] */
float *refr_kv(void *t, int which) {
    Transformer *x = (Transformer *)t;
    return which ? x->state.value_cache : x->state.key_cache;
}
