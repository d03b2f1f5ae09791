/* qwen_hip: the Qwen2 .qwb token loop of qwen/qwen.c (generate + CLI, qwen.c:669-817) on one MI355X through
 * libmatvec_hip.so's device-resident API.  Same options and output as qwen.c:
 *   qwen_hip model.qwb [-i text] [-m chat|raw] [-z tokenizer] [--ids a,b,c] [-t temp] [-p topp] [-s seed]
 *            [-n new] [-c ctx] [--logits file]
 * A text prompt goes through the Qwen tokenizer (qwen_tokenizer.c; by default qwen_tokenizer.bin next to the
 * model), inside the Qwen chat template unless -m raw (qwen.c:778-797); the generated tokens are printed as
 * their bytes.  With --ids the prompt is token ids and the output the generated ids, comma separated
 * (qwen.c:696).  stderr: the prompt/generation rate line (qwen.c:709-711).  The whole loop runs on the
 * device (hipGraph per token): the argmax at -t 0, the reference's sampler (temperature, top-p, xorshift
 * coin; qwen.c:578-654) at -t > 0. */
#include <stdint.h>
#include <time.h>

#include "hostcli.h"
#include "llm_hip.h"
#include "qwen_tokenizer.h"

static void usage(void) {
    fprintf(stderr, "Usage: qwen_hip <model.qwb> [-i text] [-m chat|raw] [-z tokenizer] [--ids a,b,c] [-t temp] [-p topp]\n"
                    "                [-s seed] [-n new] [-c ctx] [--logits file]\n");
    exit(EXIT_FAILURE);
}

/* the prompt's ids from the tokenizer: the text, inside the chat template in chat mode; added tokens in the
 * text become their ids (qwen.c:778-797) */
static int *text_prompt(Tokenizer *tok, const char *prompt, const char *mode, int *n_ids) {
    const char *tmpl = "<|im_start|>system\nYou are Qwen, created by Alibaba Cloud. You are a helpful assistant."
                       "<|im_end|>\n<|im_start|>user\n%s<|im_end|>\n<|im_start|>assistant\n";
    const int chat = !strcmp(mode, "chat");
    const size_t len = strlen(tmpl) + strlen(prompt) + 1;
    char *text = calloc(len, 1);
    int *ids = calloc(len, sizeof(int)); /* never more ids than bytes */
    if (!text || !ids) { fprintf(stderr, "out of memory\n"); exit(EXIT_FAILURE); }
    if (chat) snprintf(text, len, tmpl, prompt);
    else snprintf(text, len, "%s", prompt);
    *n_ids = tok_encode(tok, text, 1, ids, (int)len);
    free(text);
    if (*n_ids < 1) { fprintf(stderr, "empty prompt\n"); exit(EXIT_FAILURE); }
    return ids;
}

int main(int argc, char **argv) {
    char *ids_arg = NULL, *logits_path = NULL, *prompt = "", *mode = "chat", *tokenizer_path = NULL;
    float temperature = 0.7f, topp = 0.8f;
    int steps = 256, ctx = 1024;
    unsigned long long seed = 0;
    if (argc < 2) usage();
    for (int i = 2; i < argc; i += 2) { /* qwen.c:743-760 */
        if (i + 1 >= argc || argv[i][0] != '-') usage();
        if (!strcmp(argv[i], "--ids")) { ids_arg = argv[i + 1]; continue; }
        if (!strcmp(argv[i], "--logits")) { logits_path = argv[i + 1]; continue; }
        if (strlen(argv[i]) != 2) usage();
        switch (argv[i][1]) {
        case 't': temperature = atof(argv[i + 1]); break;
        case 'p': topp = atof(argv[i + 1]); break;
        case 's': seed = strtoull(argv[i + 1], NULL, 10); break;
        case 'n': steps = atoi(argv[i + 1]); break;
        case 'c': ctx = atoi(argv[i + 1]); break;
        case 'i': prompt = argv[i + 1]; break;
        case 'm': mode = argv[i + 1]; break;
        case 'z': tokenizer_path = argv[i + 1]; break;
        default: usage();
        }
    }
    if (seed == 0) seed = (unsigned int)time(NULL);
    if (temperature < 0.0f) temperature = 0.0f;
    if (topp < 0.0f || 1.0f < topp) topp = 0.8f;
    if (steps < 1 || ctx < 2) usage();
    if (strcmp(mode, "chat") && strcmp(mode, "raw")) usage();
    int n_ids;
    int *ids;
    Tokenizer *tok = NULL;
    if (ids_arg) ids = parse_ids(ids_arg, &n_ids);
    else {
        char default_tok[4096];
        if (!tokenizer_path) { /* qwen_tokenizer.bin in the model's directory */
            const char *slash = strrchr(argv[1], '/');
            const int dir = slash ? (int)(slash - argv[1] + 1) : 0;
            snprintf(default_tok, sizeof default_tok, "%.*sqwen_tokenizer.bin", dir, argv[1]);
            tokenizer_path = default_tok;
        }
        if (!(tok = tok_load(tokenizer_path))) return 1;
        ids = text_prompt(tok, prompt, mode, &n_ids);
    }
    llm_model *m = llm_open(argv[1], ctx);
    if (!m) return 1;
    llm_info info;
    llm_get_info(m, &info);
    if (info.kind != 0) { fprintf(stderr, "%s: not a .qwb model\n", argv[1]); return 1; }
    for (int i = 0; i < n_ids; i++)
        if (ids[i] >= info.vocab_size) { fprintf(stderr, "token id %d out of range\n", ids[i]); return 1; }
    if (n_ids >= info.ctx) { fprintf(stderr, "prompt (%d tokens) does not fit -c %d\n", n_ids, info.ctx); return 1; }
    FILE *dump = NULL;
    if (logits_path && !(dump = fopen(logits_path, "wb"))) { fprintf(stderr, "cannot write %s\n", logits_path); return 1; }
    if (llm_set_sampler(m, temperature, topp, seed)) return 1;
    int *out = calloc(steps, sizeof(int));
    float *lg = NULL;
    if (dump) lg = malloc((size_t)(n_ids + steps) * info.n_logits * sizeof(float));
    llm_timing t;
    const int n_gen = llm_generate(m, ids, n_ids, steps, out, lg, &t);
    if (n_gen < 0) return 1;
    for (int i = 0; i < n_gen; i++) {
        if (tok) {
            int len;
            const char *piece = tok_decode(tok, out[i], &len);
            if (piece) fwrite(piece, 1, (size_t)len, stdout);
        } else
            printf(i ? ",%d" : "%d", out[i]);
    }
    if (dump) fwrite(lg, sizeof(float), (size_t)t.n_forward * info.n_logits, dump);
    const int n_fwd_gen = t.n_forward - n_ids;
    const double prompt_s = t.prompt_ms / 1000.0, gen_s = t.decode_ms / 1000.0;
    if (t.n_forward == info.ctx && n_gen < steps) fprintf(stderr, "\n(context of %d tokens full)", info.ctx);
    free(out);
    free(lg);
    printf("\n");
    fprintf(stderr, "prompt: %d tokens in %.2f s (%.2f tok/s); generated: %d tokens, %.2f tok/s\n", n_ids, prompt_s,
            n_ids / (prompt_s + 1e-12), n_gen, n_fwd_gen ? n_fwd_gen / (gen_s + 1e-12) : 0.0);
    if (dump) fclose(dump);
    llm_close(m);
    tok_free(tok);
    free(ids);
    return 0;
}
