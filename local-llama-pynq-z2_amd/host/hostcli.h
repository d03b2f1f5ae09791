/* Shared pieces of the C host programs qwen_hip and runq_hip: prompt-id parsing and the llama2.c sampler
 * (temperature, softmax, top-p, xorshift64* coin; qwen.c:578-654, runq.c:830-967), used when -t > 0.
 * Greedy decoding (-t 0) never comes here: the argmax runs on the device inside the step graph. */
#pragma once
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static int *parse_ids(const char *arg, int *n) { /* qwen.c:771-777 */
    int *ids = calloc(strlen(arg) / 2 + 2, sizeof(int));
    *n = 0;
    for (const char *c = arg; *c;) {
        char *end;
        long v = strtol(c, &end, 10);
        if (end == c || (*end && *end != ',') || v < 0) { fprintf(stderr, "bad --ids\n"); exit(EXIT_FAILURE); }
        ids[(*n)++] = (int)v;
        c = *end ? end + 1 : end;
    }
    return ids;
}

static long now_ms(void) {
    struct timespec t;
    clock_gettime(CLOCK_REALTIME, &t);
    return t.tv_sec * 1000 + t.tv_nsec / 1000000;
}

typedef struct { float p; int i; } HostProb;
typedef struct { int n; float temperature, topp; unsigned long long rng; HostProb *buf; } HostSampler;

static unsigned int hs_u32(unsigned long long *s) { /* xorshift64*, qwen.c:638-643 */
    *s ^= *s >> 12;
    *s ^= *s << 25;
    *s ^= *s >> 27;
    return (unsigned int)((*s * 0x2545F4914F6CDD1Dull) >> 32);
}
static float hs_f32(unsigned long long *s) { return (hs_u32(s) >> 8) / 16777216.0f; }

static int hs_argmax(const float *p, int n) {
    int mi = 0;
    for (int i = 1; i < n; i++)
        if (p[i] > p[mi]) mi = i;
    return mi;
}

static int hs_cmp(const void *a, const void *b) {
    float x = ((const HostProb *)a)->p, y = ((const HostProb *)b)->p;
    return x > y ? -1 : x < y ? 1 : 0;
}

/* qwen.c:647-654: returns a row of the logits */
static int hs_sample(HostSampler *s, float *logits) {
    int n = s->n;
    if (s->temperature == 0.0f) return hs_argmax(logits, n);
    for (int i = 0; i < n; i++) logits[i] /= s->temperature;
    float mx = logits[0], sum = 0.0f;
    for (int i = 1; i < n; i++) if (logits[i] > mx) mx = logits[i];
    for (int i = 0; i < n; i++) { logits[i] = expf(logits[i] - mx); sum += logits[i]; }
    for (int i = 0; i < n; i++) logits[i] /= sum;
    float coin = hs_f32(&s->rng);
    if (s->topp <= 0 || s->topp >= 1) {
        float cdf = 0.0f;
        for (int i = 0; i < n; i++) { cdf += logits[i]; if (coin < cdf) return i; }
        return n - 1;
    }
    int n0 = 0;
    const float cutoff = (1.0f - s->topp) / (n - 1);
    for (int i = 0; i < n; i++)
        if (logits[i] >= cutoff) { s->buf[n0].i = i; s->buf[n0].p = logits[i]; n0++; }
    qsort(s->buf, n0, sizeof(HostProb), hs_cmp);
    float cum = 0.0f;
    int last = n0 - 1;
    for (int i = 0; i < n0; i++) { cum += s->buf[i].p; if (cum > s->topp) { last = i; break; } }
    float r = coin * cum, cdf = 0.0f;
    for (int i = 0; i <= last; i++) { cdf += s->buf[i].p; if (r < cdf) return s->buf[i].i; }
    return s->buf[last].i;
}
