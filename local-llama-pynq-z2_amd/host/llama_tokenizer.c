/* llama2.c tokenizer of runq (interface and semantics: llama_tokenizer.h).
 *
 * The vocabulary is looked up through a hash table of its strings (the first id of a repeated string).
 * Merging keeps, for each adjacent pair, the id and score of its concatenation, and recomputes only the two
 * pairs next to a merge; each round takes the highest score, the leftmost on ties, as the reference's full
 * rescan does. */
#include "llama_tokenizer.h"

#include <ctype.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

struct LlamaTokenizer {
    int n;
    char **piece;
    float *score;
    int *slot_id; /* hash table of the pieces: id + 1 per slot, 0 = empty */
    uint32_t mask;
    size_t maxlen;
    char bytes[512]; /* "b\0" for every byte b */
    /* scratch of the merge loop */
    char *cat;
    int *pair_id;
    float *pair_score;
    size_t cap;
};

static uint32_t hash_str(const char *s) {
    uint32_t h = 2166136261u; /* FNV-1a */
    for (; *s; s++) h = (h ^ (uint8_t)*s) * 16777619u;
    return h;
}

static int lookup(const LlamaTokenizer *t, const char *s) {
    for (uint32_t h = hash_str(s) & t->mask;; h = (h + 1) & t->mask) {
        const int v = t->slot_id[h];
        if (!v) return -1;
        if (!strcmp(t->piece[v - 1], s)) return v - 1;
    }
}

void llama_tok_free(LlamaTokenizer *t) {
    if (!t) return;
    if (t->piece)
        for (int i = 0; i < t->n; i++) free(t->piece[i]);
    free(t->piece);
    free(t->score);
    free(t->slot_id);
    free(t->cat);
    free(t->pair_id);
    free(t->pair_score);
    free(t);
}

LlamaTokenizer *llama_tok_load(const char *path, int vocab_size) {
    LlamaTokenizer *t = (LlamaTokenizer *)calloc(1, sizeof *t);
    FILE *f = fopen(path, "rb");
    int max_len;
    if (!t || !f || vocab_size < 3) {
        fprintf(stderr, "couldn't load %s\n", path);
        goto fail;
    }
    t->n = vocab_size;
    t->piece = (char **)calloc((size_t)vocab_size, sizeof(char *));
    t->score = (float *)malloc((size_t)vocab_size * sizeof(float));
    uint32_t slots = 64;
    while (slots < 2u * (uint32_t)vocab_size) slots *= 2;
    t->mask = slots - 1;
    t->slot_id = (int *)calloc(slots, sizeof(int));
    if (!t->piece || !t->score || !t->slot_id || fread(&max_len, sizeof(int), 1, f) != 1) goto bad_read;
    for (int i = 0; i < vocab_size; i++) {
        int len;
        if (fread(t->score + i, sizeof(float), 1, f) != 1 || fread(&len, sizeof(int), 1, f) != 1 || len < 0) goto bad_read;
        if (!(t->piece[i] = (char *)malloc((size_t)len + 1))) goto bad_read;
        if (len && fread(t->piece[i], (size_t)len, 1, f) != 1) goto bad_read;
        t->piece[i][len] = 0;
        const size_t sl = strlen(t->piece[i]);
        if (sl > t->maxlen) t->maxlen = sl;
        uint32_t h = hash_str(t->piece[i]) & t->mask;
        while (t->slot_id[h] && strcmp(t->piece[t->slot_id[h] - 1], t->piece[i])) h = (h + 1) & t->mask;
        if (!t->slot_id[h]) t->slot_id[h] = i + 1;
    }
    fclose(f);
    for (int b = 0; b < 256; b++) { t->bytes[2 * b] = (char)b; t->bytes[2 * b + 1] = 0; }
    if (!(t->cat = (char *)malloc(2 * t->maxlen + 8))) goto fail;
    return t;
bad_read:
    fprintf(stderr, "failed read\n");
fail:
    if (f) fclose(f);
    llama_tok_free(t);
    return NULL;
}

/* id and score of the concatenation tokens[i] + tokens[i + 1] (id -1 when it is not in the vocabulary) */
static void pair_at(LlamaTokenizer *t, const int *tok, int i) {
    if (tok[i] < 0 || tok[i + 1] < 0) { /* the dummy prefix of a vocabulary without " " */
        t->pair_id[i] = -1;
        return;
    }
    const char *a = t->piece[tok[i]], *b = t->piece[tok[i + 1]];
    const size_t la = strlen(a);
    memcpy(t->cat, a, la);
    strcpy(t->cat + la, b);
    const int id = lookup(t, t->cat);
    t->pair_id[i] = id;
    t->pair_score[i] = id >= 0 ? t->score[id] : 0.0f;
}

int llama_encode(LlamaTokenizer *t, const char *text, int bos, int eos, int *tokens, int *n_tokens) {
    if (!text) { fprintf(stderr, "cannot encode NULL text\n"); return -1; }
    int n = 0;
    if (bos) tokens[n++] = 1;
    if (text[0]) tokens[n++] = lookup(t, " "); /* dummy prefix */
    /* one token per UTF-8 character (a lead byte and at most 3 continuation bytes), or its bytes */
    char ch[8];
    for (const char *c = text; *c;) {
        size_t len = 1;
        ch[0] = *c++;
        while (len < 4 && (*c & 0xC0) == 0x80) ch[len++] = *c++;
        ch[len] = 0;
        const int id = lookup(t, ch);
        if (id >= 0) tokens[n++] = id;
        else
            for (size_t k = 0; k < len; k++) tokens[n++] = (uint8_t)ch[k] + 3;
    }
    /* merges: the highest-scoring pair, leftmost on ties, until no adjacent pair forms a piece (BOS's piece
     * takes part like any other) */
    if ((size_t)n > t->cap) {
        free(t->pair_id);
        free(t->pair_score);
        t->cap = (size_t)n + 64;
        t->pair_id = (int *)malloc(t->cap * sizeof(int));
        t->pair_score = (float *)malloc(t->cap * sizeof(float));
        if (!t->pair_id || !t->pair_score) { t->cap = 0; return -1; }
    }
    for (int i = 0; i + 1 < n; i++) pair_at(t, tokens, i);
    for (;;) {
        float best = -1e10f;
        int at = -1;
        for (int i = 0; i + 1 < n; i++)
            if (t->pair_id[i] >= 0 && t->pair_score[i] > best) { best = t->pair_score[i]; at = i; }
        if (at < 0) break;
        tokens[at] = t->pair_id[at];
        memmove(tokens + at + 1, tokens + at + 2, (size_t)(n - at - 2) * sizeof(int));
        memmove(t->pair_id + at + 1, t->pair_id + at + 2, (size_t)(n > at + 2 ? n - at - 3 : 0) * sizeof(int));
        memmove(t->pair_score + at + 1, t->pair_score + at + 2, (size_t)(n > at + 2 ? n - at - 3 : 0) * sizeof(float));
        n--;
        if (at > 0) pair_at(t, tokens, at - 1);
        if (at + 1 < n) pair_at(t, tokens, at);
    }
    if (eos) tokens[n++] = 2;
    *n_tokens = n;
    return 0;
}

const char *llama_decode(LlamaTokenizer *t, int prev_token, int token) {
    if (token < 0 || token >= t->n) return NULL;
    const char *p = t->piece[token];
    if (prev_token == 1 && p[0] == ' ') p++;
    unsigned char b;
    if (sscanf(p, "<0x%02hhX>", &b) == 1) p = t->bytes + 2 * b;
    return p;
}

void llama_print_piece(const char *piece, FILE *f) {
    if (!piece || !piece[0]) return;
    if (!piece[1]) {
        const unsigned char b = (unsigned char)piece[0];
        if (!(isprint(b) || isspace(b))) return;
    }
    fputs(piece, f);
}
