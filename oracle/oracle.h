/* CPU oracle for the decode token loop: a plain-C restatement of the reference's arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may load
 * it, and only as the checker.  The HIP library never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Each one is pinned by tests/test_oracle.py
 * against the reference's own functions (oracle/_ref/, built from the reference sources by oracle/Makefile),
 * against committed golden vectors (tests/golden/) and against closed forms. */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float or_f16(uint16_t h);                                              /* qwen.c:84-94 */
uint16_t or_f32_to_f16(float f);                                       /* round to nearest even (generator) */

/* activation quantization, int8 per group */
void or_quantize_qwen(int8_t *q, float *s, const float *x, int n);     /* qwen.c:354-364, group 32 */
void or_quantize_runq(int8_t *q, float *s, const float *x, int n, int gs); /* runq.c:244-270 */

/* GEMV: qwen flavour (int4/int8 weights, fp16 scales, group 32) and runq flavour (int8, fp32 scales) */
void or_matvec4(float *out, const uint8_t *w, const uint16_t *ws, const int8_t *xq, const float *xs, int n, int d,
                int bits);                                             /* qwen.c:436-456 */
void or_set_sum_ways(int k); /* 1 = reference order (default); k partial sums otherwise (tolerance test only) */
void or_matvec4_groups(int32_t *ival, const uint8_t *w, const int8_t *xq, int n, int d, int bits); /* qwen.c:443-451 */
void or_matvec_runq(float *out, const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int n, int d,
                    int gs);                                           /* runq.c:429-458 */
void or_matvec_runq_groups(int32_t *ival, const int8_t *wq, const int8_t *xq, int n, int d, int gs); /* runq.c:448-451 */

void or_rmsnorm(float *o, const float *x, const float *w, int n, float eps); /* qwen.c:337-344, runq.c:394-407 */
void or_set_norm_ways(int k); /* 1 = reference order (default); k partial sums of x^2 (tolerance test only) */
void or_softmax(float *x, int n);                                      /* qwen.c:346-352, runq.c:409-427 */
void or_expf(const float *x, int n, float *y); /* the C library's expf, as qwen.c:350 / 560 and runq.c:420 / 592 call it */
void or_rope_angles(float *c, float *s, int hs, int pos, float theta); /* qwen.c:503-508 */
void or_rope_neox(float *v, int n_heads, int hs, const float *c, const float *s); /* qwen.c:478-488 */
void or_rope_runq(float *q, float *k, int dim, int kv_dim, int hs, int pos); /* runq.c:506-521 */
int or_argmax(const float *p, int n);                                  /* qwen.c:591-598, runq.c:843-854 */

/* xorshift sampler (qwen.c:638-654, runq.c:933-967) */
unsigned int or_random_u32(unsigned long long *state);
float or_random_f32(unsigned long long *state);
int or_sample(float *logits, int n, float temperature, float topp, unsigned long long *rng);

/* whole models: .qwb Qwen2 (qwen.c:195-573) and llama2.c v2 .bin (runq.c:273-615) */
typedef struct or_model or_model;
or_model *or_open(const char *path, int ctx_or_steps); /* detects the format from the magic; NULL + stderr */
const float *or_forward(or_model *m, int token, int pos);
int or_n_logits(const or_model *m);        /* head_k (qwen) or vocab (runq) */
const int32_t *or_head_ids(const or_model *m); /* NULL for runq (identity) */
int or_ctx(const or_model *m);
int or_kind(const or_model *m);             /* 0 qwen, 1 runq */
/* greedy generation with the reference's stop rules: writes up to max_out ids, returns how many */
int or_generate_greedy(or_model *m, const int *prompt, int n_prompt, int steps, int *out, int max_out);
void or_close(or_model *m);

#ifdef __cplusplus
}
#endif
