// Kernel argument blocks and host-side launchers of libmatvec_hip.so (internal header).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tiled.h"

// Per-step control block in device memory.  The step's kernels read the position and token from here,
// so one captured graph serves every position.
struct StepCtrl {
    int pos;        // position of the current step
    int token;      // input token of the current step
    int next_token; // argmax of the current step, mapped through head_ids
    int n_prompt;   // generate mode: positions < n_prompt take their token from the prompt
    int mode;       // 0: pos/token set by the host; 1: the embed kernel advances pos and picks the token
    int pad[3];
};

// Attention positions are processed in sub-chunks of this many rows (LDS staging of K and V).
#define ATT_SUB 32

// Position slices of one attention step: P = pos + 1 positions in S = min(splits, ceil(P / ATT_SUB)) slices
// of `chunk` positions (the attention kernel and the o-projection's merge use the same split).
__device__ __forceinline__ void att_slices(int pos, int splits, int *S, int *chunk) {
    const int P = pos + 1;
    int s = (P + ATT_SUB - 1) / ATT_SUB;
    if (s > splits) s = splits;
    *S = s;
    *chunk = (P + s - 1) / s;
}


// Prologues: how the int8 activation vector reaches LDS.
enum { PRO_XQ = 0, PRO_NORM = 1, PRO_ATTN = 2 };
// Epilogues: what happens to the finished rows.
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_SWIGLU = 3, EPI_ARGMAX = 4 };
// RoPE pairing of the fused QKV matrix.
enum { ROPE_NEOX = 0, ROPE_INTERLEAVED = 1 };

struct GemvArgs {
    TiledMat W;
    int kw, nb;             // waves per row-block, row-blocks per block iteration (a power of two)
    int depth;              // weight batches in flight per wave: 2 or 4
    int ord;                // 1: each row's group products are added in group order (bit-exact sequential sum)
    // derived by launch_gemv: log2(nb), log2(W.rb), iterations, chunks per wave (kw_base + (my_kw < kw_rem)),
    // iterations per block (it_base + (block < it_rem))
    int nb_log2, rb_log2, n_it, kw_base, kw_rem, it_base, it_rem;
    int qflavor;            // activation quantization flavour (QF_QWEN / QF_RUNQ)
    int nt;                 // 1: non-temporal weight loads (the step's weights stream past the caches)
    int strict;             // 1: reference order (sequential RMSNorm sum, the reference libm's expf in SiLU)
    const StepCtrl *ctrl;
    // PRO_XQ
    const int8_t *xq;
    const float *xs;
    // PRO_NORM: x (n floats) -> rmsnorm(norm_w, eps) -> quantize
    const float *x;
    const float *norm_w;
    float eps;
    // PRO_ATTN: combine split attention partials -> quantize
    const float *att_ml;    // [n_heads][splits][2] (max score, sum of exp)
    const float *att_acc;   // [n_heads][splits][hs]
    int n_heads, head_size, att_splits;
    // EPI_STORE / EPI_RESID / EPI_ARGMAX: out[row] (= or +=)
    float *out;
    // EPI_ARGMAX
    float *logits_hist;     // optional [ctx][rows]
    float *part_val;
    int *part_idx;
    // EPI_QKV
    const float *bias;      // [dim + 2*kv_dim] or NULL
    float *q, *kc, *vc;     // q [dim]; layer bases of the caches [ctx][kv_dim]
    const float *rope_cos, *rope_sin; // [ctx][head_size/2]
    int dim, kv_dim, rope_kind;
    // EPI_SWIGLU
    int8_t *hq;
    float *hs;
    float *hf;              // optional fp32 h
};

struct AttnArgs {
    const float *q;         // [n_heads * hs]
    const float *kc, *vc;   // layer bases [ctx][kv_dim]
    float *ml, *acc;        // partials, see GemvArgs
    int n_heads, n_kv, hs, kv_dim, splits; // splits: maximum number of position slices (grid)
    int max_pos;            // positions the cache holds (the launcher picks the kernel for the longest slice)
    const StepCtrl *ctrl;
};

struct EmbedArgs {
    const int8_t *emb_q;    // [vocab][dim]
    const void *emb_s;      // [vocab][dim/gs] fp16 or fp32
    int sf32, dim, gs;
    float *x;
    StepCtrl *ctrl;
    const int *prompt;      // generate mode
    int *tokens;            // [ctx] input token of every position
    // generate mode: the previous step's argmax partials, finished here
    const float *pv;
    const int *pi;
    int np;
    const int *head_ids;    // NULL: identity
    int *gen;               // [ctx] argmax result of every position
};

struct ArgmaxArgs {
    const float *pv;
    const int *pi;
    int np;
    const int *head_ids;    // NULL: identity
    StepCtrl *ctrl;
    int *gen;               // [ctx] argmax result of every position
};

// Device-resident sampler settings and RNG state (the reference's Sampler, qwen.c:583-589).
struct SamplerState {
    float temperature, topp;
    unsigned long long rng;
};

struct SampleArgs {
    const float *logits;    // [n] head logits
    int n;
    float *probs;           // [n] scratch: probabilities
    SamplerState *ss;
    const StepCtrl *ctrl;   // generate mode: no draw while the next token is a prompt token; NULL: always draw
    float *pv;              // [np] argmax partials of the step: the choice becomes the only finite entry
    int *pi;
    int np;
    int *out_row;           // optional: the sampled row
    // the many-workgroup path's buffers (sample_scratch_bytes()), taken for n >= SMP_MULTI_MIN; NULL: the whole
    // draw in one workgroup
    void *scratch;
    int path;               // many-workgroup path: the kernels launched, 0 the plain walk, 1 top-p, else both
                            // (each returns at once unless the device-resident settings select it)
    // strict mode: the reference-order draw (sample_strict.hip) with its buffers (sample_strict_scratch_bytes())
    int strict;
    void *strict_scratch;
};
hipError_t launch_sample(const SampleArgs &a, hipStream_t st);
size_t sample_scratch_bytes();
hipError_t launch_sample_strict(const SampleArgs &a, hipStream_t st);
size_t sample_strict_scratch_bytes();
// tests: move every predicted segment start of the strict draw's sums by `skew` ulps (0 after allocation)
hipError_t sample_strict_set_skew(void *scratch, int skew);

struct RepackArgs {
    TiledMat T;             // output (T.data writable)
    const uint8_t *w[4];    // raw weight planes, row-major (reference layout)
    const uint8_t *s[4];    // raw scale planes
    const int *rowmap;      // logical row -> (source << 28) | source row
};

// host launchers (kernels.hip); each returns the launch error
hipError_t launch_gemv(int wbits, int gs, int sf32, int pro, int epi, const GemvArgs &a, int grid, hipStream_t st);
size_t gemv_lds_bytes(const GemvArgs &a, int pro, int epi, int threads);
hipError_t launch_attention(const AttnArgs &a, hipStream_t st);
// reference-order attention (one block per query head); leaves acc [n_heads][hs] and ml = (0, 1) per head,
// i.e. the partials of a single slice that the o projection's merge passes through unchanged
hipError_t launch_attention_strict(const AttnArgs &a, hipStream_t st);
hipError_t launch_embed(const EmbedArgs &a, hipStream_t st);
hipError_t launch_argmax(const ArgmaxArgs &a, hipStream_t st);
hipError_t launch_repack(const RepackArgs &a, hipStream_t st);
hipError_t launch_quantize_test(const float *x, int n, int flavor, int gs, int8_t *q, float *s, hipStream_t st);
hipError_t launch_group_dots_test(const TiledMat &T, const int8_t *xq, int32_t *ival, hipStream_t st);
