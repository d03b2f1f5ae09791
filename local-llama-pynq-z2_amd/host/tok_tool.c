/* tok_tool: command-line access to the hosts' tokenizers, for tests and for preparing --ids prompts.
 *   tok_tool qwen <qwen_tokenizer.bin> enc [-s] [file]   encode NUL-separated cases (a file without NUL is one
 *                                                        case): one line of space-separated ids per case;
 *                                                        -s: added tokens in the text become their ids
 *   tok_tool qwen <qwen_tokenizer.bin> dec [file]        one line of ids per case in; the bytes, then NUL, out
 *   tok_tool llama <tokenizer.bin> <vocab> enc [file]    runq's encode (BOS, dummy prefix) per case
 *   tok_tool llama <tokenizer.bin> <vocab> dec [file]    runq's decode of each line (printable pieces only)
 * file "-" or none: stdin.  The qwen form has the input/output contract of the reference's qwen/tok_test.c. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "llama_tokenizer.h"
#include "qwen_tokenizer.h"

static char *slurp(const char *path, size_t *len) {
    FILE *f = (!path || !strcmp(path, "-")) ? stdin : fopen(path, "rb");
    if (!f) { perror(path); exit(1); }
    size_t cap = 1 << 16, n = 0, r;
    char *b = (char *)malloc(cap + 1);
    while (b && (r = fread(b + n, 1, cap - n, f)) > 0) {
        n += r;
        if (n == cap) b = (char *)realloc(b, (cap *= 2) + 1);
    }
    if (!b) exit(1);
    b[n] = 0;
    if (f != stdin) fclose(f);
    *len = n;
    return b;
}

static int usage(void) {
    fprintf(stderr, "usage: tok_tool qwen <qwen_tokenizer.bin> enc [-s] [file] | dec [file]\n"
                    "       tok_tool llama <tokenizer.bin> <vocab_size> enc [file] | dec [file]\n");
    return 2;
}

/* calls fn(case, ctx) for each case of the input: NUL-separated (enc) or one per line (dec) */
static void each_case(char *in, size_t len, int lines, void (*fn)(char *, void *), void *ctx) {
    for (char *p = in; p < in + len;) {
        char *e = (char *)memchr(p, lines ? '\n' : 0, (size_t)(in + len - p));
        if (!e) e = in + len;
        *e = 0;
        fn(p, ctx);
        p = e + 1;
    }
}

typedef struct {
    Tokenizer *q;
    LlamaTokenizer *l;
    int special, *ids;
    size_t cap;
    int rc;
} Ctx;

static void print_ids(const int *ids, int n) {
    for (int i = 0; i < n; i++) printf(i ? " %d" : "%d", ids[i]);
    putchar('\n');
}

static void qwen_enc(char *s, void *v) {
    Ctx *c = (Ctx *)v;
    int n;
    while ((n = tok_encode(c->q, s, c->special, c->ids, (int)c->cap)) < 0) {
        c->cap *= 2;
        if (!(c->ids = (int *)realloc(c->ids, c->cap * sizeof(int)))) exit(1);
    }
    print_ids(c->ids, n);
}

static void qwen_dec(char *s, void *v) {
    Ctx *c = (Ctx *)v;
    for (char *q = s;;) {
        char *end;
        const long id = strtol(q, &end, 10);
        if (end == q) break;
        int n;
        const char *b = tok_decode(c->q, (int)id, &n);
        if (!b) { fprintf(stderr, "bad id %ld\n", id); c->rc = 1; }
        else fwrite(b, 1, (size_t)n, stdout);
        q = end;
    }
    putchar(0);
}

static void llama_enc(char *s, void *v) {
    Ctx *c = (Ctx *)v;
    const size_t need = strlen(s) + 3;
    if (need > c->cap && !(c->ids = (int *)realloc(c->ids, (c->cap = need) * sizeof(int)))) exit(1);
    int n;
    if (llama_encode(c->l, s, 1, 0, c->ids, &n)) { c->rc = 1; return; }
    print_ids(c->ids, n);
}

static void llama_dec(char *s, void *v) {
    Ctx *c = (Ctx *)v;
    int prev = -1;
    for (char *q = s;;) {
        char *end;
        const long id = strtol(q, &end, 10);
        if (end == q) break;
        const char *piece = llama_decode(c->l, prev, (int)id);
        if (!piece) { fprintf(stderr, "bad id %ld\n", id); c->rc = 1; }
        else llama_print_piece(piece, stdout);
        prev = (int)id;
        q = end;
    }
    putchar(0);
}

int main(int argc, char **argv) {
    if (argc < 4) return usage();
    Ctx c = {0};
    c.cap = 1024;
    c.ids = (int *)malloc(c.cap * sizeof(int));
    int a = 3;
    if (!strcmp(argv[1], "qwen")) {
        if (!(c.q = tok_load(argv[2]))) return 1;
    } else if (!strcmp(argv[1], "llama")) {
        if (argc < 5) return usage();
        if (!(c.l = llama_tok_load(argv[2], atoi(argv[3])))) return 1;
        a = 4;
    } else
        return usage();
    const int dec = !strcmp(argv[a], "dec");
    if (!dec && strcmp(argv[a], "enc")) return usage();
    const char *file = NULL;
    for (int i = a + 1; i < argc; i++) {
        if (!strcmp(argv[i], "-s")) c.special = 1;
        else file = argv[i];
    }
    size_t len;
    char *in = slurp(file, &len);
    if (c.q) each_case(in, len, dec, dec ? qwen_dec : qwen_enc, &c);
    else each_case(in, len, dec, dec ? llama_dec : llama_enc, &c);
    fflush(stdout);
    free(in);
    free(c.ids);
    tok_free(c.q);
    llama_tok_free(c.l);
    return c.rc;
}
