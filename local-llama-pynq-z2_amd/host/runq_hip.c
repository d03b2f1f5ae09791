/* runq_hip: the llama2.c int8 token loop of runq/runq.c (generate, runq.c:982-1036) on one MI355X through
 * libmatvec_hip.so's device-resident API:
 *   runq_hip model.bin [-i text] [-z tokenizer.bin] [-m generate|chat] [-y system] [--ids a,b,c] [-n steps]
 *            [-t temp] [-p topp] [-s seed] [--logits file]
 * Options and defaults of runq.c's CLI (runq.c:1145-1200: -t 1.0, -p 0.9, -s time, -n 256, -z tokenizer.bin).
 * A text prompt is encoded by the llama2.c tokenizer (BOS, dummy prefix; llama_tokenizer.c) and, as runq.c
 * does, every token after the first is printed as its piece: the rest of the prompt, then the generated text
 * (runq.c:1018-1020).  With --ids the prompt is token ids and stdout the generated ids, comma separated.
 * -n counts positions including the prompt and is clamped to seq_len (runq.c:1200); generation stops at
 * BOS (1) (runq.c:1016).  The whole loop runs on the device: the argmax at -t 0, the reference's sampler
 * (runq.c:830-967) at -t > 0.  stderr: decode rate (tokens after the prompt / time).
 * -m chat [-y system] is runq.c's chat loop (runq.c:1055-1140): turns read from stdin, Llama 2 chat schema,
 * each turn continuing the same KV cache (llm_continue), the assistant's turn ending at EOS (2). */
#include <stdint.h>
#include <time.h>

#include "hostcli.h"
#include "llama_tokenizer.h"
#include "llm_hip.h"

/* xorshift64* state after `draws` coins (the reference's random_u32, runq.c:933-939; the returned value is
 * not needed to advance the state) */
static unsigned long long rng_advance(unsigned long long s, long draws) {
    for (long i = 0; i < draws; i++) {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
    }
    return s;
}

static void read_stdin(const char *guide, char *buf, size_t size) { /* runq.c:1038-1047 */
    printf("%s", guide);
    if (fgets(buf, (int)size, stdin) != NULL) {
        const size_t len = strlen(buf);
        if (len > 0 && buf[len - 1] == '\n') buf[len - 1] = '\0';
    }
}

/* runq.c's chat loop.  The reference draws a coin at every position when sampling (the draws at prompt
 * positions are discarded), feeds EOS at the position after it is drawn and prints the piece drawn there;
 * the host keeps the exact coin state and hands it to the device before each call. */
static int chat(llm_model *m, LlamaTokenizer *tok, const char *cli_user, const char *cli_system, int steps,
                float temperature, float topp, unsigned long long seed) {
    char system_prompt[512] = "", user_prompt[512] = "", rendered[1152];
    int *ptok = malloc(1152 * sizeof(int)), *gen = malloc(((size_t)steps + 1) * sizeof(int)), n_ptok = 0;
    const int sampled = temperature > 0.0f;
    unsigned long long rng = seed;
    int pos = 0;
    if (!ptok || !gen) return 1;
    while (pos < steps) {
        if (pos == 0) {
            if (!cli_system) read_stdin("Enter system prompt (optional): ", system_prompt, sizeof system_prompt);
            else snprintf(system_prompt, sizeof system_prompt, "%s", cli_system);
        }
        if (pos == 0 && cli_user) snprintf(user_prompt, sizeof user_prompt, "%s", cli_user);
        else read_stdin("User: ", user_prompt, sizeof user_prompt);
        if (pos == 0 && system_prompt[0] != '\0')
            snprintf(rendered, sizeof rendered, "[INST] <<SYS>>\n%s\n<</SYS>>\n\n%s [/INST]", system_prompt, user_prompt);
        else
            snprintf(rendered, sizeof rendered, "[INST] %s [/INST]", user_prompt);
        if (llama_encode(tok, rendered, 1, 0, ptok, &n_ptok)) return 1;
        printf("Assistant: ");
        if (pos + n_ptok > steps) { /* the prompt runs into the step limit: forced positions, nothing printed */
            if (sampled && llm_set_sampler(m, temperature, topp, rng)) return 1;
            if (llm_continue(m, pos, ptok, steps - pos, 1, 2, gen, NULL) < 0) return 1;
            pos = steps;
            break;
        }
        /* the prompt (coins at all but its last position discarded), then the reply up to EOS */
        if (sampled) {
            rng = rng_advance(rng, n_ptok - 1);
            if (llm_set_sampler(m, temperature, topp, rng)) return 1;
        }
        const int max_new = steps - (pos + n_ptok) + 1;
        const int k = llm_continue(m, pos, ptok, n_ptok, max_new, 2, gen, NULL);
        if (k < 0) return 1;
        int prev = ptok[n_ptok - 1];
        for (int i = 0; i < k; i++) {
            llama_print_piece(llama_decode(tok, prev, gen[i]), stdout);
            prev = gen[i];
        }
        if (k == max_new) { pos = steps; break; } /* out of steps mid-reply */
        printf("\n");                            /* EOS drawn at position pos + n_ptok - 1 + k */
        if (sampled) rng = rng_advance(rng, k + 1);
        pos += n_ptok + k;
        if (pos >= steps) break;
        /* EOS fed at the next position; the piece drawn there is printed (runq.c:1114-1134) */
        if (sampled && llm_set_sampler(m, temperature, topp, rng)) return 1;
        const int eos = 2;
        const int r = llm_continue(m, pos, &eos, 1, 1, 2, gen, NULL);
        if (r < 0) return 1;
        if (r == 1) llama_print_piece(llama_decode(tok, 2, gen[0]), stdout);
        else printf("\n");
        if (sampled) rng = rng_advance(rng, 1);
        pos += 1;
    }
    printf("\n");
    free(ptok);
    free(gen);
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: runq_hip model.bin [-i text] [-z tokenizer.bin] [--ids a,b,c] [-n N] [-t T] [-p P] [-s S] [--logits f]\n");
        return 1;
    }
    char *ids_arg = NULL, *logits_path = NULL, *prompt = NULL, *tokenizer_path = "tokenizer.bin", *mode = "generate";
    char *system_prompt = NULL;
    float temperature = 1.0f, topp = 0.9f;
    int steps = 256;
    unsigned long long seed = 0;
    for (int i = 2; i + 1 < argc; i += 2) {
        if (!strcmp(argv[i], "--ids")) ids_arg = argv[i + 1];
        else if (!strcmp(argv[i], "--logits")) logits_path = argv[i + 1];
        else if (!strcmp(argv[i], "-n")) steps = atoi(argv[i + 1]);
        else if (!strcmp(argv[i], "-t")) temperature = atof(argv[i + 1]);
        else if (!strcmp(argv[i], "-p")) topp = atof(argv[i + 1]);
        else if (!strcmp(argv[i], "-s")) seed = strtoull(argv[i + 1], NULL, 10);
        else if (!strcmp(argv[i], "-i")) prompt = argv[i + 1];
        else if (!strcmp(argv[i], "-z")) tokenizer_path = argv[i + 1];
        else if (!strcmp(argv[i], "-m")) mode = argv[i + 1];
        else if (!strcmp(argv[i], "-y")) system_prompt = argv[i + 1];
        else { fprintf(stderr, "bad option %s\n", argv[i]); return 1; }
    }
    if (seed == 0) seed = (unsigned int)time(NULL);
    if (temperature < 0.0f) temperature = 0.0f;
    if (topp < 0.0f || 1.0f < topp) topp = 0.9f;
    llm_model *m = llm_open(argv[1], 0);
    if (!m) return 1;
    llm_info info;
    llm_get_info(m, &info);
    if (info.kind != 1) { fprintf(stderr, "%s: not a llama2.c .bin model\n", argv[1]); return 1; }
    if (strcmp(mode, "generate") && strcmp(mode, "chat")) { fprintf(stderr, "unknown mode: %s\n", mode); return 1; }
    if (!strcmp(mode, "chat")) {
        if (steps <= 0 || steps > info.ctx) steps = info.ctx;
        LlamaTokenizer *ct = llama_tok_load(tokenizer_path, info.vocab_size);
        if (!ct || llm_set_sampler(m, temperature, topp, seed)) return 1;
        const int rc = chat(m, ct, prompt, system_prompt, steps, temperature, topp, seed);
        llama_tok_free(ct);
        llm_close(m);
        return rc;
    }
    int n_ids;
    int *ids;
    LlamaTokenizer *tok = NULL;
    if (ids_arg) ids = parse_ids(ids_arg, &n_ids);
    else {
        if (!(tok = llama_tok_load(tokenizer_path, info.vocab_size))) return 1;
        const char *text = prompt ? prompt : "";
        if (!(ids = malloc((strlen(text) + 3) * sizeof(int))) || llama_encode(tok, text, 1, 0, ids, &n_ids)) return 1;
    }
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
    if (tok) { /* the pieces of every token after the first: prompt, then generated (runq.c:1018-1020) */
        int prev = ids[0];
        for (int i = 1; i < n_ids + n_gen; i++) {
            const int next = i < n_ids ? ids[i] : out[i - n_ids];
            llama_print_piece(llama_decode(tok, prev, next), stdout);
            prev = next;
        }
    } else
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
    llama_tok_free(tok);
    free(ids);
    return 0;
}
