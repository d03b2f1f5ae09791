/* runq_hip: the llama2.c int8 token loop of runq/runq.c (generate, runq.c:982-1036) on one MI355X through
 * libmatvec_hip.so's device-resident API, for token-id prompts:
 *   runq_hip model.bin --ids a,b,c [-n steps] [-t temp] [-p topp] [-s seed] [--logits file]
 * -n counts positions including the prompt and is clamped to seq_len (runq.c:1200); generation stops at
 * BOS (1) (runq.c:1016).  The whole loop runs on the device: the argmax at -t 0, the reference's sampler
 * (runq.c:830-967) at -t > 0.  stdout: generated ids; stderr: decode rate (tokens after the prompt / time). */
#include <stdint.h>

#include "hostcli.h"
#include "llm_hip.h"

int main(int argc, char **argv) {
    if (argc < 2) { fprintf(stderr, "usage: runq_hip model.bin --ids a,b,c [-n N] [-t T] [-p P] [-s S] [--logits f]\n"); return 1; }
    char *ids_arg = NULL, *logits_path = NULL;
    float temperature = 0.0f, topp = 0.9f;
    int steps = 256;
    unsigned long long seed = 1;
    for (int i = 2; i + 1 < argc; i += 2) {
        if (!strcmp(argv[i], "--ids")) ids_arg = argv[i + 1];
        else if (!strcmp(argv[i], "--logits")) logits_path = argv[i + 1];
        else if (!strcmp(argv[i], "-n")) steps = atoi(argv[i + 1]);
        else if (!strcmp(argv[i], "-t")) temperature = atof(argv[i + 1]);
        else if (!strcmp(argv[i], "-p")) topp = atof(argv[i + 1]);
        else if (!strcmp(argv[i], "-s")) seed = strtoull(argv[i + 1], NULL, 10);
        else { fprintf(stderr, "bad option %s\n", argv[i]); return 1; }
    }
    if (!ids_arg) { fprintf(stderr, "--ids is required\n"); return 1; }
    int n_ids;
    int *ids = parse_ids(ids_arg, &n_ids);
    llm_model *m = llm_open(argv[1], 0);
    if (!m) return 1;
    llm_info info;
    llm_get_info(m, &info);
    if (info.kind != 1) { fprintf(stderr, "%s: not a llama2.c .bin model\n", argv[1]); return 1; }
    if (steps <= 0 || steps > info.ctx) steps = info.ctx;
    for (int i = 0; i < n_ids; i++)
        if (ids[i] >= info.vocab_size) { fprintf(stderr, "token id %d out of range\n", ids[i]); return 1; }
    if (n_ids > steps) { fprintf(stderr, "prompt longer than the positions to run\n"); return 1; }
    FILE *dump = NULL;
    if (logits_path && !(dump = fopen(logits_path, "wb"))) { fprintf(stderr, "cannot write %s\n", logits_path); return 1; }
    const int max_new = steps - n_ids + 1; /* positions n_ids-1 .. steps-1 each yield one token */
    if (llm_set_sampler(m, temperature, topp, seed)) return 1;
    int *out = calloc(max_new, sizeof(int));
    float *lg = dump ? malloc((size_t)(n_ids + max_new) * info.n_logits * sizeof(float)) : NULL;
    llm_timing t;
    const int n_gen = llm_generate(m, ids, n_ids, max_new, out, lg, &t);
    if (n_gen < 0) return 1;
    for (int i = 0; i < n_gen; i++) printf(i ? ",%d" : "%d", out[i]);
    if (dump) fwrite(lg, sizeof(float), (size_t)t.n_forward * info.n_logits, dump);
    const int n_fwd_gen = t.n_forward - n_ids;
    const double gen_s = t.decode_ms / 1000.0;
    free(out);
    free(lg);
    printf("\n");
    fprintf(stderr, "prompt: %d tokens; generated: %d tokens, %.2f tok/s\n", n_ids, n_gen,
            n_fwd_gen ? n_fwd_gen / (gen_s + 1e-12) : 0.0);
    if (dump) fclose(dump);
    llm_close(m);
    free(ids);
    return 0;
}
