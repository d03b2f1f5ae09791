/* runq_hip: the llama2.c int8 token loop of runq/runq.c (generate, runq.c:982-1036) on one MI355X through
 * libmatvec_hip.so's device-resident API:
 *   runq_hip model.bin [-i text] [-z tokenizer.bin] [--ids a,b,c] [-n steps] [-t temp] [-p topp] [-s seed]
 *            [--logits file]
 * Options and defaults of runq.c's CLI (runq.c:1145-1200: -t 1.0, -p 0.9, -s time, -n 256, -z tokenizer.bin).
 * A text prompt is encoded by the llama2.c tokenizer (BOS, dummy prefix; llama_tokenizer.c) and, as runq.c
 * does, every token after the first is printed as its piece: the rest of the prompt, then the generated text
 * (runq.c:1018-1020).  With --ids the prompt is token ids and stdout the generated ids, comma separated.
 * -n counts positions including the prompt and is clamped to seq_len (runq.c:1200); generation stops at
 * BOS (1) (runq.c:1016).  The whole loop runs on the device: the argmax at -t 0, the reference's sampler
 * (runq.c:830-967) at -t > 0.  stderr: decode rate (tokens after the prompt / time).  (runq.c's chat mode is
 * not carried.) */
#include <stdint.h>
#include <time.h>

#include "hostcli.h"
#include "llama_tokenizer.h"
#include "llm_hip.h"

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: runq_hip model.bin [-i text] [-z tokenizer.bin] [--ids a,b,c] [-n N] [-t T] [-p P] [-s S] [--logits f]\n");
        return 1;
    }
    char *ids_arg = NULL, *logits_path = NULL, *prompt = NULL, *tokenizer_path = "tokenizer.bin";
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
