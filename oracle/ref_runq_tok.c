/* Test harness (oracle infrastructure only): runq.c's own tokenizer (build_tokenizer, encode, decode,
 * safe_printf; runq.c:615-823) behind the command-line contract of the hosts' tok_tool "llama" mode:
 *   ref_runq_tok <tokenizer.bin> <vocab_size> enc [file]   NUL-separated cases, one line of ids each (BOS on)
 *   ref_runq_tok <tokenizer.bin> <vocab_size> dec [file]   one line of ids per case, printable pieces + NUL out
 * The reference source is included where it lies (the recipe passes -I to its runq/ directory); TESTING
 * hides runq.c's main (runq.c:1142).  Build output: oracle/_ref/. */
#define TESTING
#include "runq.c"

static char *slurp_all(const char *path, size_t *len) {
    FILE *f = (!path || !strcmp(path, "-")) ? stdin : fopen(path, "rb");
    if (!f) { perror(path); exit(1); }
    size_t cap = 1 << 16, n = 0, r;
    char *b = malloc(cap + 1);
    while ((r = fread(b + n, 1, cap - n, f)) > 0) {
        n += r;
        if (n == cap) b = realloc(b, (cap *= 2) + 1);
    }
    b[n] = 0;
    if (f != stdin) fclose(f);
    *len = n;
    return b;
}

int main(int argc, char **argv) {
    if (argc < 4) { fprintf(stderr, "usage: ref_runq_tok <tokenizer.bin> <vocab> enc|dec [file]\n"); return 2; }
    Tokenizer t;
    build_tokenizer(&t, argv[1], atoi(argv[2]));
    const int dec = !strcmp(argv[3], "dec");
    size_t len;
    char *in = slurp_all(argc > 4 ? argv[4] : NULL, &len);
    for (char *p = in; p < in + len;) {
        char *e = memchr(p, dec ? '\n' : 0, (size_t)(in + len - p));
        if (!e) e = in + len;
        *e = 0;
        if (dec) {
            int prev = -1;
            for (char *q = p;;) {
                char *end;
                long id = strtol(q, &end, 10);
                if (end == q) break;
                safe_printf(decode(&t, prev, (int)id));
                prev = (int)id;
                q = end;
            }
            putchar(0);
        } else {
            int *ids = malloc((strlen(p) + 3) * sizeof(int)), n;
            encode(&t, p, 1, 0, ids, &n);
            for (int i = 0; i < n; i++) printf(i ? " %d" : "%d", ids[i]);
            putchar('\n');
            free(ids);
        }
        p = e + 1;
    }
    free_tokenizer(&t);
    return 0;
}
