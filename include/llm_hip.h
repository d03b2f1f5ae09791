/* Extension ABI of libmatvec_hip.so: the whole decode token loop resident on one MI355X.
 *
 * The drop-in API (matvec_fpga.h) moves only the GEMVs to the GPU, one synchronous call each.  This API
 * is what the reference's hosts would call to move the rest of forward() too (qwen.c:490-573,
 * runq.c:477-615): the model file is uploaded once (weights repacked into the GEMV tiles, KV cache in HBM),
 * and one decode step is a fixed sequence of kernels that reads its position and token from device memory,
 * captured once as a hipGraph and replayed per token.  Both of the reference's formats are accepted:
 * .qwb (Qwen2, qwen.c:195-271) and llama2.c v2 .bin (runq, runq.c:318-357).
 *
 * Numerics follow the reference: int8 group quantization of activations (qwen.c:354-364 or runq.c:244-270,
 * bit-exact for the same input), exact int32 group sums, the per-group product ((float)ival * ws) * xs,
 * RoPE tables computed on the host with the reference's own libm calls.  Two modes (llm_set_strict):
 *   fast (default for .qwb): sums over groups, RMSNorm and softmax reductions run in parallel trees, so each
 *     layer output matches the reference within fp32 rounding (an int8 re-quantization that lands on the
 *     other side of a rounding boundary then moves deeper layers by more; see llm_set_strict);
 *   strict (LLM_STRICT=1 at llm_open, or llm_set_strict): every float operation of forward() in the
 *     reference's order and the reference libm's expf, so logits and token streams, greedy or sampled (the
 *     sampler's softmax and cumulative sums sequential as the reference's), are bitwise those of qwen.c /
 *     runq.c built with strict IEEE flags.  llama2.c .bin GEMVs always sum their groups in order.
 * Errors: -1 (or NULL) with a message on stderr, the reference's convention (matvec_fpga.h:15). */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct llm_model llm_model;

typedef struct {
    int kind;                  /* 0: .qwb Qwen2 (qwen.c), 1: llama2.c v2 .bin (runq.c) */
    int dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size;
    int n_logits;              /* head_k (qwen.c:39) or vocab_size (runq) */
    int ctx;                   /* KV cache positions: min(ctx, max_seq_len) (qwen.c:325) or seq_len (runq) */
    int group_size;
    float rope_theta, rms_eps;
    double gemv_bytes_per_token; /* algorithmic GEMV bytes of one decode step: weights, scales, activations, outputs */
    double weight_bytes;       /* resident tiled weight bytes in HBM */
} llm_info;

typedef struct {
    int n_prompt, n_generated, n_forward;
    double prompt_ms, decode_ms; /* decode: forwards after the prompt's last one, qwen.c:682, 709-711 */
} llm_timing;

/* build_transformer (qwen.c:320-330, runq.c:359-367): open, validate and upload a model.  ctx caps the
 * KV cache for .qwb files (qwen's -c); .bin files always get seq_len positions.  NULL on failure. */
llm_model *llm_open(const char *path, int ctx);
int llm_get_info(const llm_model *m, llm_info *info);
/* head_ids of a .qwb (qwen.c:57); NULL for .bin, whose logits are indexed by token id */
const int32_t *llm_head_ids(const llm_model *m);

/* forward (qwen.c:490-573, runq.c:477-615): one position; the logits of the head rows go to `logits`
 * (n_logits floats, host memory) when it is not NULL.  Eager launches, synchronous. */
int llm_forward(llm_model *m, int token, int pos, float *logits);

/* generate with greedy sampling (qwen.c:669-712 at -t 0; runq.c:982-1036 at -t 0), the whole loop on the
 * device: prompt forcing, argmax over the head rows, head_ids mapping, one hipGraph replay per position.
 * Stop rules follow the model kind: .qwb stops at <|im_end|> 151645 / <|endoftext|> 151643, after
 * max_new tokens or at a full context; .bin stops at BOS (1) or when max_new + n_prompt - 1 positions...
 * (runq's steps clamp, runq.c:1200) are done.  Generated ids go to out (room for max_new).  When `logits`
 * is not NULL, every position's head logits are appended to it (the --logits dump, qwen.c:676), so it needs
 * room for (n_prompt + max_new) * n_logits floats.  Returns the number of generated ids, or -1. */
int llm_generate(llm_model *m, const int *prompt, int n_prompt, int max_new, int *out, float *logits,
                 llm_timing *timing);

/* The token loop continued from an earlier llm_generate / llm_continue, for multi-turn dialogs (runq's chat
 * loop, runq.c:1055-1140): the n tokens are forced at positions pos0 .. pos0 + n - 1 over the KV cache that
 * earlier calls left below pos0, then up to max_new tokens are generated (argmax, or the sampler of
 * llm_set_sampler) until stop_id is generated (not stored; -1: the format's stop ids, as llm_generate) or
 * the context is full.  Returns the number of generated ids written to out, or -1.  Steps run in batches,
 * so after a stop the device's sampler state may have advanced past the stop's draw: a caller that
 * continues a sampled stream sets the state it wants with llm_set_sampler first. */
int llm_continue(llm_model *m, int pos0, const int *tokens, int n, int max_new, int stop_id, int *out,
                 llm_timing *timing);

/* Decode throughput: replays the captured step graph `steps` times from the current position (after a
 * prompt was forced by llm_generate or llm_forward) with no host round trips, and returns the elapsed time
 * of exactly those replays in *ms (HIP events on the library's stream).  With the sampler on
 * (llm_set_sampler, temperature > 0) the replayed steps draw their tokens with it. */
int llm_decode_replay(llm_model *m, int steps, double *ms);

/* Per-kernel timing of decode steps: runs `steps` steps with HIP events around every launch (on the
 * library's stream), and fills one record per kernel kind with its launch count, total device time and
 * algorithmic bytes per launch.  Returns the number of records written (at most max_stats), or -1. */
typedef struct {
    char name[40];
    int launches;
    double total_ms;
    double bytes_per_launch; /* algorithmic HBM bytes of one launch (weights + scales + activations + outputs) */
} llm_kernel_stat;
int llm_profile(llm_model *m, int steps, llm_kernel_stat *stats, int max_stats);

/* Per-kernel time inside the replayed step graph: the graph is replayed `steps` times from the current
 * position, and again with each kernel kind's launches left out (`rounds` alternating repetitions, medians);
 * a kind's total_ms is the difference, i.e. its device time in the graph including its share of the gaps
 * between nodes, with no launch or event overhead.  *step_ms receives the median full-step time.  The step
 * control (position, next token) is restored afterwards; the KV rows the replays wrote lie past it and are
 * rewritten by the next steps.  Returns the number of records, or -1. */
int llm_profile_graph(llm_model *m, int steps, int rounds, llm_kernel_stat *stats, int max_stats, double *step_ms);

/* Batched prompt processing (prefill; the reference runs the prompt one forward() per position,
 * qwen.c:674-681): positions 0..n-1 pass through each layer together, in chunks of up to 512 tokens.  The
 * layer matrices become int8 MFMA GEMMs with exact int32 group sums and the reference's per-group product
 * and group order; attention is causal over the KV cache.  Fills the KV cache like n forward() calls and
 * leaves the logits of position n-1 in `logits` (n_logits floats, may be NULL); the step state is then
 * position n-1.  Returns 0 or -1. */
int llm_prefill(llm_model *m, const int *ids, int n, float *logits);
/* Whether llm_generate runs the prompt through llm_prefill (on by default) or one decode step per prompt
 * position.  The --logits history (llm_generate with `logits`) always uses the per-position steps. */
int llm_set_prefill(llm_model *m, int on);

/* Reference-order ("strict") mode on or off; no counterpart in the reference, whose CPU loops are this order
 * (qwen.c:337-352 rmsnorm and softmax, 407-457 matmul_cpu, 526-546 attention, 558-562 SiLU; runq.c:394-428,
 * 429-458, 530-568, 589-596).  On: GEMV group products added per row in group order, RMSNorm's sum of squares
 * as one running sum, attention per head as scores -> max -> expf -> running sum -> divide -> position-ordered
 * weighted sum of V, and expf evaluated as the reference's glibc computes it.  Applies to decode steps and
 * to the batched prefill (whose GEMM keeps the group order in both modes).  Slower than the fast mode (the
 * running sums are single dependency chains).  The step graphs are re-captured on the next call.
 * llm_get_strict returns 1, 0, or -1 for a NULL model.  Returns 0 or -1. */
int llm_set_strict(llm_model *m, int on);
int llm_get_strict(const llm_model *m);

/* Sampling in llm_generate (the reference's sampler, qwen.c:578-654 / runq.c:830-967, which its hosts run on
 * the CPU per token): with temperature > 0 every generated token is drawn on the device inside the step
 * graph (logits / temperature, softmax, top-p when 0 < topp < 1 else the plain cdf walk, xorshift64* coin
 * from `seed`); temperature 0 restores greedy argmax.  The RNG state lives on the device and advances once
 * per drawn token, as the reference's does; forced prompt positions draw nothing.  Returns 0 or -1. */
int llm_set_sampler(llm_model *m, float temperature, float topp, unsigned long long seed);
/* the sampler's current RNG state (0 before llm_set_sampler) */
int llm_sampler_state(llm_model *m, unsigned long long *rng);

void llm_close(llm_model *m);

/* ---- test hooks: no counterpart in the reference; they expose single device stages so the tests can
 * hold each one against the oracle (like the reference's FPGA_CHECK side-by-side check, qwen.c:464-472) --- */

/* activation quantization on the device: flavor 0 = qwen.c:354-364 (group 32), 1 = runq.c:244-270 (gs) */
int mvh_quantize(const float *x, int n, int flavor, int gs, int8_t *q, float *s);
/* exact int32 group sums of a matrix in the reference layout (qwen planes: bits 4 or 8, group 32; or runq
 * int8 with group gs when bits == 0), computed by the GEMV kernels' own dot-product code: ival[d][n/gs] */
int mvh_group_dots(const uint8_t *w, const int8_t *xq, int n, int d, int bits, int gs, int32_t *ival);
/* the on-device sampler on caller logits: `count` vectors of n logits drawn one after another with one RNG
 * state (*rng in, the advanced state out), temperature > 0; rows[count] receives the sampled rows */
int mvh_sample(const float *logits, int n, int count, float temperature, float topp, unsigned long long *rng,
               int *rows);
/* the same with the strict mode's draw: every float operation of the reference's sample() in its order
 * (sequential softmax sum and cumulative sums, candidates in qsort's order), so rows and RNG state are those of
 * the reference's sampler for any logits; n <= 262144 */
int mvh_sample_strict(const float *logits, int n, int count, float temperature, float topp,
                      unsigned long long *rng, int *rows);
/* mvh_sample_strict with every predicted segment start of its sequential sums moved by `skew` ulps: from 32 on,
 * no start is among its segment's candidates and every sum takes the term-by-term path (its tests) */
int mvh_sample_strict_skew(const float *logits, int n, int count, float temperature, float topp,
                           unsigned long long *rng, int *rows, int skew);
/* the prefill GEMM on caller data: y[m][r] for M tokens, weights in the reference layout (qwen planes: bits 4
 * or 8 with fp16 scales, group 32; runq: bits 0 = int8 with fp32 scales, group gs), tiled with row-blocks of
 * rb (8, 16 or 64) rows; xq [M][n] int8, xs [M][n/gs], y [M][d].  shape: 0 the library's choice, 10 TA + TB
 * one wave per 16 TA rows x 16 TB tokens: 11, 12, 14, 21, 22, 24, 41 or 42 */
int mvh_prefill_gemm(const uint8_t *w, const void *ws, const int8_t *xq, const float *xs, int M, int n, int d,
                     int bits, int gs, int rb, int shape, float *y);
/* the floor of a kernel that reads `bytes` once: `copies` launches of a plain streaming read (`blocks`
 * workgroups, 8 loads of 16 bytes in flight per thread, non-temporal loads when nt != 0) over distinct buffers,
 * captured as one graph and replayed `reps` times; *us gets the mean time per launch */
int mvh_read_floor(size_t bytes, int copies, int blocks, int nt, int reps, float *us);
/* the GEMV launch shape the library picks for a matrix, on the host (no device needed): rows x n weights in
 * groups of gs, wbits 4 or 8, scales fp32 (sf32 1) or fp16, row-blocks of rb rows, role 0 QKV, 1 attention output, 2 gate/up, 3 down,
 * 4 the output head's argmax, 5 a drop-in GEMV; ordered: bit 0 groups added in order, bit 1 the strict
 * RMSNorm; cus the device's compute units.  out[4] = waves per row-block, row-blocks per iteration, grid,
 * ordered-in-LDS flag.  0, 1 when no shape adds this matrix's groups in order, -1 on bad arguments. */
int mvh_gemv_shape(int rows, int n, int gs, int wbits, int sf32, int rb, int role, int ordered, int cus, int *out);
/* mvh_sample with no device allocation: no counterpart in the reference; for callers that cannot allocate
 * device memory (tight serving loops, harnesses that forbid hipMalloc).  Same arguments, draws and RNG state as
 * mvh_sample, but every device buffer lives in a fixed array inside the library (about 9 MiB per GPU, held
 * until the process ends): n <= 262144, count <= 4096 and count * (n rounded up to 4) <= 2^21, otherwise -1
 * with a message.  Calls that overlap on one GPU (several host threads) share that array and race. */
int mvh_sample_noalloc(const float *logits, int n, int count, float temperature, float topp,
                       unsigned long long *rng, int *rows);
/* expf as the reference's C library evaluates it (the strict mode's softmax and SiLU), over n floats: on the
 * device (n <= 2^26), and the same restatement compiled for the host CPU (no GPU involved) */
int mvh_ref_expf(const float *x, int n, float *y);
int mvh_ref_expf_host(const float *x, int n, float *y);
/* the strict mode's sequential fp32 sum s = ((0 + x[0]) + x[1]) + ... (rmsnorm's sum of squares and the
 * softmax sum, qwen.c:339 and qwen.c:349; a row's group products, qwen.c:441-452) by one of its device forms,
 * n <= 8192: which 0 = the block's speculative segments with `threads` threads (64..1024, a multiple of 64),
 * 1 = one wave's chain, 2 = one thread's chain (`threads` ignored).  0 on success, -1 on bad arguments. */
int mvh_seq_sum(const float *x, int n, int which, int threads, float *out);
/* device state after the last llm_forward/llm_generate step: 0 = residual stream x (dim floats, after the
 * final rmsnorm like qwen.c:569), 1 = key cache of layer `layer` (ctx * kv_dim), 2 = value cache */
int llm_read_state(llm_model *m, int which, int layer, float *dst, size_t count);

#ifdef __cplusplus
}
#endif
