/* Test harness (oracle infrastructure only): a token-id driver for the reference's runq.c, built the way
 * llama2.c tests it (TESTING hides runq.c's own main, runq.c:1142), so no tokenizer.bin is needed.
 *   runq_ids model.bin --ids a,b,c [-n steps] [-t temp] [-p topp] [-s seed] [--logits file]
 * Follows runq.c's generate() (runq.c:982-1036): prompt forcing, sampling through runq.c's sample(),
 * stop on BOS (1), steps clamped to seq_len (runq.c:1200).  Prints the generated ids comma separated on
 * stdout, and on stderr the decode rate in qwen.c's definition (tokens generated after the prompt /
 * time after the prompt) next to runq's own figure (runq.c:1029-1033). */
#define TESTING
#include "runq.c"

int main(int argc, char **argv) {
    if (argc < 2) { fprintf(stderr, "usage: runq_ids model.bin --ids a,b,c [-n N] [-t T] [-p P] [-s S] [--logits f]\n"); return 1; }
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
    int *ids = calloc(strlen(ids_arg) + 1, sizeof(int)), n_ids = 0;
    for (char *c = ids_arg, *end; *c; c = *end ? end + 1 : end) {
        long v = strtol(c, &end, 10);
        if (end == c || (*end && *end != ',') || v < 0) { fprintf(stderr, "bad --ids\n"); return 1; }
        ids[n_ids++] = (int)v;
    }
    Transformer t;
    build_transformer(&t, argv[1]);
    if (steps <= 0 || steps > t.config.seq_len) steps = t.config.seq_len;
    for (int i = 0; i < n_ids; i++)
        if (ids[i] >= t.config.vocab_size) { fprintf(stderr, "token id %d out of range\n", ids[i]); return 1; }
    Sampler sampler;
    build_sampler(&sampler, t.config.vocab_size, temperature, topp, seed);
    FILE *dump = NULL;
    if (logits_path && !(dump = fopen(logits_path, "wb"))) { fprintf(stderr, "cannot write %s\n", logits_path); return 1; }
    long start = time_in_ms(), prompt_done = start, gen_start = 0;
    int token = ids[0], pos = 0, n_gen = 0, next;
    while (pos < steps) {
        float *logits = forward(&t, token, pos);
        if (dump) fwrite(logits, sizeof(float), t.config.vocab_size, dump);
        if (pos < n_ids - 1) next = ids[pos + 1];
        else {
            if (pos == n_ids - 1) prompt_done = time_in_ms();
            next = sample(&sampler, logits);
        }
        pos++;
        if (next == 1) break;
        if (pos >= n_ids) { printf(n_gen ? ",%d" : "%d", next); n_gen++; }
        token = next;
        if (gen_start == 0) gen_start = time_in_ms();
    }
    long end = time_in_ms();
    printf("\n");
    int n_fwd_gen = n_gen > 0 ? n_gen - 1 : 0; /* forwards run after the prompt, as qwen.c counts them */
    fprintf(stderr, "prompt: %d tokens; generated: %d tokens, %.2f tok/s (runq's own figure: %.2f tok/s)\n", n_ids,
            n_gen, n_fwd_gen ? n_fwd_gen * 1000.0 / (end - prompt_done + 1e-9) : 0.0,
            pos > 1 ? (pos - 1) / (double)(end - gen_start + 1e-9) * 1000 : 0.0);
    if (dump) fclose(dump);
    free_sampler(&sampler);
    free_transformer(&t);
    free(ids);
    return 0;
}
