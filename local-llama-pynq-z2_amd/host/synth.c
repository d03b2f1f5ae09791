/* Synthetic model writer: seeded random-init weights in the reference's two on-disk formats.
 *
 *   synth qwb  <out.qwb> <preset> [seed]    Qwen2 .qwb v1: Q4_0 layer planes, Q8_0 head + embedding, fp16 scales
 *   synth bin  <out.bin> <preset> [seed]    llama2.c v2 .bin (runq): Q8_0 tensors with fp32 scales
 *   presets:  qwb: tiny, c3 (Qwen2 0.5B shape), c5 (Qwen2 7B shape)    bin: tiny, c1 (288/6L), c2 (768/12L)
 *   A preset can be overridden key by key: synth qwb out.qwb c3 7 dim=1024 layers=2 ...
 *   head_ids=<file> (qwb): the trimmed head's token ids from a file of little-endian int32, ascending (e.g. a
 *   set the reference ships, qwen/head_tokens_65536.npy's array); head_k becomes its length.
 *
 * Formats (kept exactly as the reference reads them):
 *   .qwb: header "<4sI10i2f" in 256 bytes (qwen.c:37-42, 216-221), every array padded to 64 bytes (qwen.c:195-199),
 *         order attn_norm, ffn_norm, bq, bk, bv, output_norm, head_ids, wq, wk, wv, wo, w1, w2, w3, head, embedding
 *         (qwen.c:237-258; tools/gguf2qwb.py:5-14).  int4 element 2i in the low nibble of byte i (qwen.c:45).
 *   .bin: header "<Ii7iBi" in 256 bytes, fp32 norms, then int8 tensors each followed by its fp32 scales
 *         (runq.c:291-357; tools/bin2q80.py:48-59).
 *
 * Weights are N(0, 0.02) from a counter-based generator (splitmix64 of (seed, tensor, element) into a
 * Box-Muller draw), so any row can be produced independently and in parallel; norm gains are 1.0.
 * Quantizers: Q4_0 as llama.cpp defines it (d = max/-8 with max the signed value of largest |x|, stored fp16,
 * nibble = min(15, (int8)(x/d + 8.5)), value = nibble - 8); Q8_0 with d = max|x|/127 and q = roundf(x/d).
 * The trimmed Qwen head takes seeded ascending head_ids that leave out the stop ids 151643 and 151645. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int dim, hidden, layers, heads, kv_heads, vocab, head_k, max_seq, gs;
    float theta, eps;
} Cfg;

static uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static uint64_t g_seed;

/* N(0, 0.02) for element e of tensor t */
static float gauss(uint32_t t, uint64_t e) {
    uint64_t h = splitmix(splitmix(g_seed * 0x2545F4914F6CDD1Dull + t) ^ e);
    float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    float u2 = ((float)((h >> 16) & 0xFFFFFF) + 0.5f) * (1.0f / 16777216.0f);
    return 0.02f * sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958648f * u2);
}

static uint16_t f32_to_f16(float f) { /* round to nearest even */
    union { float f; uint32_t u; } in = { .f = f };
    uint32_t u = in.u, sign = (u >> 16) & 0x8000;
    int32_t e = (int32_t)((u >> 23) & 0xff) - 112;
    uint32_t m = u & 0x7fffff;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000;
        int sh = 14 - e;
        uint32_t r = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (m >> 13), rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

static FILE *out;
static size_t written;

static void put(const void *p, size_t n) {
    if (n && fwrite(p, 1, n, out) != n) { perror("write"); exit(1); }
    written += n;
}
static void pad64(void) {
    static const char z[64];
    put(z, (64 - written % 64) % 64);
}

/* one Q4_0 row of n values into n/2 packed bytes and n/32 fp16 scales */
static void q4_row(const float *x, int n, uint8_t *w, uint16_t *s) {
    for (int b = 0; b < n / 32; b++) {
        const float *v = x + b * 32;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; j++)
            if (amax < fabsf(v[j])) { amax = fabsf(v[j]); mx = v[j]; }
        float d = mx / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        s[b] = f32_to_f16(d);
        for (int j = 0; j < 32; j += 2) {
            int a = (int8_t)(v[j] * id + 8.5f), c = (int8_t)(v[j + 1] * id + 8.5f);
            a = a < 15 ? a : 15;
            c = c < 15 ? c : 15;
            w[(b * 32 + j) / 2] = (uint8_t)(((a - 8) & 15) | (((c - 8) & 15) << 4));
        }
    }
}

/* one Q8_0 row: scale max|x|/127 (fp32), q = roundf(x / d) */
static void q8_row(const float *x, int n, int gs, int8_t *q, float *s) {
    for (int b = 0; b < n / gs; b++) {
        float amax = 0.0f;
        for (int j = 0; j < gs; j++) amax = fmaxf(amax, fabsf(x[b * gs + j]));
        float d = amax / 127.0f;
        s[b] = d;
        for (int j = 0; j < gs; j++) q[b * gs + j] = d != 0.0f ? (int8_t)roundf(x[b * gs + j] / d) : 0;
    }
}

#define ROWS 256 /* rows generated per batch */

/* matrix of d rows x n, tensor id t, rows taken from `rows` (NULL: 0..d-1) */
static void write_matrix(uint32_t t, int d, int n, int bits, const int32_t *rows, int fmt_bin, int gs) {
    size_t wrow = fmt_bin ? (size_t)n : (size_t)n * bits / 8, ng = (size_t)n / gs;
    float *x = malloc((size_t)ROWS * n * sizeof(float));
    uint8_t *w = malloc((size_t)ROWS * wrow);
    void *s = malloc((size_t)ROWS * ng * (fmt_bin ? 4 : 2));
    float *fscr = malloc((size_t)ROWS * ng * sizeof(float));
    uint8_t *sall = NULL;
    size_t sbytes = (size_t)d * ng * (fmt_bin ? 4 : 2);
    /* .qwb: weight plane, then scale plane (each 64-padded); .bin: q then s (unpadded) */
    sall = malloc(sbytes);
    for (int r0 = 0; r0 < d; r0 += ROWS) {
        int nr = d - r0 < ROWS ? d - r0 : ROWS;
#pragma omp parallel for schedule(static)
        for (int r = 0; r < nr; r++) {
            uint64_t row = rows ? (uint64_t)rows[r0 + r] : (uint64_t)(r0 + r);
            float *xr = x + (size_t)r * n;
            for (int k = 0; k < n; k++) xr[k] = gauss(t, row * (uint64_t)n + k);
            if (fmt_bin) q8_row(xr, n, gs, (int8_t *)(w + (size_t)r * wrow), (float *)s + (size_t)r * ng);
            else if (bits == 4) q4_row(xr, n, w + (size_t)r * wrow, (uint16_t *)s + (size_t)r * ng);
            else {
                float *fs = fscr + (size_t)r * ng;
                q8_row(xr, n, 32, (int8_t *)(w + (size_t)r * wrow), fs);
                for (size_t b = 0; b < ng; b++) ((uint16_t *)s)[(size_t)r * ng + b] = f32_to_f16(fs[b]);
            }
        }
        put(w, (size_t)nr * wrow);
        memcpy(sall + (size_t)r0 * ng * (fmt_bin ? 4 : 2), s, (size_t)nr * ng * (fmt_bin ? 4 : 2));
    }
    if (!fmt_bin) pad64();
    put(sall, sbytes);
    if (!fmt_bin) pad64();
    free(x); free(w); free(s); free(sall); free(fscr);
}

static void write_f32(const float *v, size_t n, int padded) {
    put(v, n * 4);
    if (padded) pad64();
}

static int set_key(Cfg *c, const char *kv) {
    char key[32];
    double v;
    if (sscanf(kv, "%31[^=]=%lf", key, &v) != 2) return -1;
    if (!strcmp(key, "dim")) c->dim = (int)v;
    else if (!strcmp(key, "hidden")) c->hidden = (int)v;
    else if (!strcmp(key, "layers")) c->layers = (int)v;
    else if (!strcmp(key, "heads")) c->heads = (int)v;
    else if (!strcmp(key, "kv_heads")) c->kv_heads = (int)v;
    else if (!strcmp(key, "vocab")) c->vocab = (int)v;
    else if (!strcmp(key, "head_k")) c->head_k = (int)v;
    else if (!strcmp(key, "max_seq")) c->max_seq = (int)v;
    else if (!strcmp(key, "gs")) c->gs = (int)v;
    else if (!strcmp(key, "theta")) c->theta = (float)v;
    else if (!strcmp(key, "eps")) c->eps = (float)v;
    else return -1;
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 4) {
        fprintf(stderr, "usage: synth qwb|bin <out> <preset> [seed] [key=value ...]\n");
        return 1;
    }
    int is_bin = !strcmp(argv[1], "bin");
    if (!is_bin && strcmp(argv[1], "qwb")) { fprintf(stderr, "format must be qwb or bin\n"); return 1; }
    const char *p = argv[3];
    Cfg c;
    if (!is_bin && !strcmp(p, "tiny")) c = (Cfg){ 128, 256, 2, 4, 2, 512, 256, 64, 32, 1e6f, 1e-6f };
    else if (!is_bin && !strcmp(p, "c3")) c = (Cfg){ 896, 4864, 24, 14, 2, 151936, 65536, 1024, 32, 1e6f, 1e-6f };
    else if (!is_bin && !strcmp(p, "c5")) c = (Cfg){ 3584, 18944, 28, 28, 4, 152064, 152064, 4096, 32, 1e6f, 1e-6f };
    else if (is_bin && !strcmp(p, "tiny")) c = (Cfg){ 64, 128, 2, 4, 4, 256, 256, 32, 32, 1e4f, 1e-5f };
    else if (is_bin && !strcmp(p, "c1")) c = (Cfg){ 288, 768, 6, 6, 6, 32000, 32000, 256, 32, 1e4f, 1e-5f };
    else if (is_bin && !strcmp(p, "c2")) c = (Cfg){ 768, 2048, 12, 12, 12, 32000, 32000, 1024, 32, 1e4f, 1e-5f };
    else { fprintf(stderr, "unknown preset %s\n", p); return 1; }
    g_seed = argc > 4 ? strtoull(argv[4], NULL, 10) : 1;
    int32_t *given_ids = NULL;
    int n_given = 0;
    for (int i = 5; i < argc; i++) {
        if (!strncmp(argv[i], "head_ids=", 9)) {
            FILE *f = fopen(argv[i] + 9, "rb");
            long bytes = -1;
            if (f && !fseek(f, 0, SEEK_END)) bytes = ftell(f);
            if (!f || bytes <= 0 || bytes % 4) { fprintf(stderr, "cannot read head ids from %s\n", argv[i] + 9); return 1; }
            rewind(f);
            given_ids = malloc((size_t)bytes);
            if (fread(given_ids, 1, (size_t)bytes, f) != (size_t)bytes) { fprintf(stderr, "short read of %s\n", argv[i] + 9); return 1; }
            fclose(f);
            n_given = (int)(bytes / 4);
            c.head_k = n_given;
            continue;
        }
        if (set_key(&c, argv[i])) { fprintf(stderr, "bad override %s\n", argv[i]); return 1; }
    }
    if (given_ids && c.head_k != n_given) { // a head_k override next to the file: the file's count rules
        fprintf(stderr, "head_k=%d does not match the %d ids of the head_ids file\n", c.head_k, n_given);
        return 1;
    }
    if (given_ids)
        for (int i = 0; i < c.head_k; i++)
            if (given_ids[i] < 0 || given_ids[i] >= c.vocab || (i && given_ids[i] <= given_ids[i - 1])) {
                fprintf(stderr, "head id %d at %d is out of range or not ascending\n", given_ids[i], i);
                return 1;
            }
    if (is_bin) c.head_k = c.vocab;
    int hs = c.dim / c.heads, kv = hs * c.kv_heads, L = c.layers;
    out = fopen(argv[2], "wb");
    if (!out) { perror(argv[2]); return 1; }
    char header[256] = { 0 };
    float *ones = malloc((size_t)(c.dim > c.hidden ? c.dim : c.hidden) * 4);
    for (int i = 0; i < (c.dim > c.hidden ? c.dim : c.hidden); i++) ones[i] = 1.0f;
    uint32_t t = 1; /* tensor ids for the generator */
    if (!is_bin) {
        int32_t h[10] = { c.dim, c.hidden, L, c.heads, c.kv_heads, c.vocab, c.head_k, c.max_seq, 32, 8 };
        memcpy(header, "QWB1", 4);
        uint32_t ver = 1;
        memcpy(header + 4, &ver, 4);
        memcpy(header + 8, h, 40);
        memcpy(header + 48, &c.theta, 4);
        memcpy(header + 52, &c.eps, 4);
        put(header, 256);
        for (int l = 0; l < L; l++) write_f32(ones, c.dim, 1); /* attn_norm */
        for (int l = 0; l < L; l++) write_f32(ones, c.dim, 1); /* ffn_norm */
        int bn[3] = { c.dim, kv, kv };
        for (int b = 0; b < 3; b++) { /* bq, bk, bv ~ N(0, 0.02) */
            float *v = malloc((size_t)bn[b] * 4);
            for (int l = 0; l < L; l++) {
                for (int i = 0; i < bn[b]; i++) v[i] = gauss(t, (uint64_t)l * bn[b] + i);
                write_f32(v, bn[b], 1);
            }
            t++;
            free(v);
        }
        write_f32(ones, c.dim, 1); /* output_norm */
        /* head_ids: ascending; the full vocabulary when head_k == vocab, else a seeded subset without stop ids */
        int32_t *ids = malloc((size_t)c.head_k * 4);
        if (given_ids) {
            memcpy(ids, given_ids, (size_t)c.head_k * 4);
        } else if (c.head_k >= c.vocab) {
            c.head_k = c.vocab;
            for (int i = 0; i < c.vocab; i++) ids[i] = i;
        } else {
            int32_t *cand = malloc((size_t)c.vocab * 4);
            int nc = 0;
            for (int i = 0; i < c.vocab; i++)
                if (i != 151643 && i != 151645) cand[nc++] = i;
            uint64_t st = splitmix(g_seed ^ 0x1D5EED);
            for (int i = 0; i < c.head_k; i++) { /* partial Fisher-Yates */
                st = splitmix(st);
                int j = i + (int)(st % (uint64_t)(nc - i));
                int32_t tmp = cand[i]; cand[i] = cand[j]; cand[j] = tmp;
            }
            memcpy(ids, cand, (size_t)c.head_k * 4);
            free(cand);
            uint8_t *bm = calloc((size_t)c.vocab, 1); /* ascending order through a bitmap */
            for (int i = 0; i < c.head_k; i++) bm[ids[i]] = 1;
            int k = 0;
            for (int i = 0; i < c.vocab; i++)
                if (bm[i]) ids[k++] = i;
            free(bm);
        }
        put(ids, (size_t)c.head_k * 4);
        pad64();
        int shp[7][2] = { { c.dim, c.dim }, { kv, c.dim }, { kv, c.dim }, { c.dim, c.dim }, { c.hidden, c.dim },
                          { c.dim, c.hidden }, { c.hidden, c.dim } };
        for (int a = 0; a < 7; a++)
            for (int l = 0; l < L; l++) write_matrix(t++, shp[a][0], shp[a][1], 4, NULL, 0, 32);
        uint32_t emb_t = t++;
        write_matrix(emb_t, c.head_k, c.dim, 8, ids, 0, 32); /* head = embedding rows head_ids (tied) */
        write_matrix(emb_t, c.vocab, c.dim, 8, NULL, 0, 32);
        free(ids);
    } else {
        int32_t h[7] = { c.dim, c.hidden, L, c.heads, c.kv_heads, c.vocab, c.max_seq };
        uint32_t magic = 0x616b3432, ver = 2;
        memcpy(header, &magic, 4);
        memcpy(header + 4, &ver, 4);
        memcpy(header + 8, h, 28);
        header[36] = 1; /* shared classifier */
        memcpy(header + 37, &c.gs, 4);
        put(header, 256);
        for (int l = 0; l < L; l++) write_f32(ones, c.dim, 0);
        for (int l = 0; l < L; l++) write_f32(ones, c.dim, 0);
        write_f32(ones, c.dim, 0);
        write_matrix(t++, c.vocab, c.dim, 8, NULL, 1, c.gs); /* token embedding = classifier */
        int shp[7][2] = { { c.dim, c.dim }, { kv, c.dim }, { kv, c.dim }, { c.dim, c.dim }, { c.hidden, c.dim },
                          { c.dim, c.hidden }, { c.hidden, c.dim } };
        for (int a = 0; a < 7; a++)
            for (int l = 0; l < L; l++) write_matrix(t++, shp[a][0], shp[a][1], 8, NULL, 1, c.gs);
    }
    free(ones);
    if (fclose(out)) { perror("close"); return 1; }
    fprintf(stderr, "wrote %s: %.1f MiB (%s %s, seed %llu)\n", argv[2], written / 1048576.0, argv[1], p,
            (unsigned long long)g_seed);
    return 0;
}
