/* Qwen2 / Qwen2.5 byte-level BPE tokenizer (interface: qwen_tokenizer.h).
 *
 * Data file "QWTOK001" (the reference's format, tools/qwen_tok_export.py:21-41; little-endian, every
 * section padded to 4 bytes):
 *   magic[8], u32 hdr[12] = n_vocab, n_added, n_merges, blob_len, n_uni, n_dec, dec_pool_len, n_comp, 0...
 *   u8 tok_len[n_vocab], u8 blob[blob_len], u32 merges[n_merges][3] (left, right, merged; index = rank),
 *   n_added x (u32 id, u32 len, text[len]), u32 uni[n_uni] (run-length: start | payload << 21, payload =
 *   class (0 other, 1 letter, 2 number, 3 white space) | NFC-may-change << 2 | combining class << 3),
 *   u32 dec_cp[n_dec], dec_off[n_dec + 1], dec_pool[dec_pool_len] (full canonical decompositions),
 *   u32 comp[n_comp][3] (first, second, composite) sorted by (first, second).
 *
 * Encoding (what Hugging Face `tokenizers` does for Qwen2.5, qwen/tokenizer.c:1-12 states the same pipeline):
 *   1. split the text at added tokens (when allowed): the leftmost position where one starts, the longest
 *      one there;
 *   2. NFC each piece between them.  Only maximal runs of non-ASCII characters that hold a character the
 *      table marks as possibly changed by NFC are rewritten, together with the ASCII character before the
 *      run (an ASCII letter can take a combining mark); everything else is left as it is;
 *   3. the pre-tokenizer regex of Qwen2
 *        (?i:'s|'t|'re|'ve|'m|'ll|'d) | [^\r\n\p{L}\p{N}]?\p{L}+ | \p{N} | ?[^\s\p{L}\p{N}]+[\r\n]* |
 *        \s*[\r\n]+ | \s+(?!\S) | \s+
 *      evaluated by hand with the outcome of a backtracking engine (first alternative that matches, greedy);
 *   4. each pre-token's bytes become single-byte tokens, merged by BPE: the pair of lowest merge rank first,
 *      the leftmost of equal ranks, until no pair has a merge.
 * Bytes that are not valid UTF-8 are kept as they are: class "other", never normalized.
 * Not thread-safe (scratch buffers live in the Tokenizer). */
#include "qwen_tokenizer.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { CL_OTHER = 0, CL_LETTER = 1, CL_NUMBER = 2, CL_SPACE = 3 };
#define NOT_UTF8 0x110000u /* a byte b that does not decode stands for the code point NOT_UTF8 + b */

typedef struct {
    uint32_t id, len;
    const char *text;
} Special;

typedef struct {
    uint32_t rank, pos; /* queue order: rank, then position */
    int32_t left, right; /* the symbol ids the pair had when queued */
} Cand;

typedef struct {
    void *p;
    size_t n, cap;
} Grow;

struct Tokenizer {
    uint8_t *file;
    uint32_t n_vocab, n_added, n_merges, n_ids;
    const uint8_t *tlen, *blob;
    uint32_t *toff;                 /* n_vocab + 1 byte offsets into blob */
    const uint32_t *merges;         /* [rank][3] */
    uint64_t *mkey;                 /* merge table, open addressing: key = left << 32 | right, 0 = empty */
    uint32_t *mval;                 /* rank of the key at the same slot */
    uint32_t mmask;
    Special *spec;
    uint8_t spec_lead[256];
    uint32_t n_uni, n_dec, n_comp, pool_len;
    const uint32_t *uni, *dec_cp, *dec_off, *dec_pool, *comp;
    int32_t byte_tok[256];
    uint8_t ascii_cls[128];
    uint32_t hit_lo, hit_hi, hit_val; /* last run looked up: [hit_lo, hit_hi) -> payload */
    /* scratch */
    Grow cps, marks, out, sym, queue;
};

static int grow(Grow *g, size_t want, size_t elem) {
    if (want <= g->cap) return 0;
    size_t c = g->cap ? g->cap : 64;
    while (c < want) c *= 2;
    void *q = realloc(g->p, c * elem);
    if (!q) return -1;
    g->p = q;
    g->cap = c;
    return 0;
}

/* ------------------------------------------------------------------------------------------------------
 * UTF-8 and the Unicode table */

/* one character of s[0..n): its length, the code point in *cp (NOT_UTF8 + byte for a byte that does not
 * start a well-formed character: overlong forms, surrogates and values past U+10FFFF included) */
static int utf8_next(const uint8_t *s, size_t n, uint32_t *cp) {
    const uint32_t b = s[0];
    if (b < 0x80) {
        *cp = b;
        return 1;
    }
    int need;
    uint32_t v, min;
    if (b >= 0xC2 && b <= 0xDF) { need = 1; v = b & 0x1F; min = 0x80; }
    else if (b >= 0xE0 && b <= 0xEF) { need = 2; v = b & 0x0F; min = 0x800; }
    else if (b >= 0xF0 && b <= 0xF4) { need = 3; v = b & 0x07; min = 0x10000; }
    else { *cp = NOT_UTF8 + b; return 1; }
    if ((size_t)need >= n) { *cp = NOT_UTF8 + b; return 1; }
    for (int k = 1; k <= need; k++) {
        if ((s[k] & 0xC0) != 0x80) { *cp = NOT_UTF8 + b; return 1; }
        v = v << 6 | (s[k] & 0x3F);
    }
    if (v < min || v > 0x10FFFF || (v >= 0xD800 && v <= 0xDFFF)) { *cp = NOT_UTF8 + b; return 1; }
    *cp = v;
    return need + 1;
}

static int utf8_put(Grow *o, uint32_t cp) {
    if (grow(o, o->n + 4, 1)) return -1;
    uint8_t *d = (uint8_t *)o->p + o->n;
    if (cp >= NOT_UTF8) { d[0] = (uint8_t)(cp - NOT_UTF8); o->n += 1; }
    else if (cp < 0x80) { d[0] = (uint8_t)cp; o->n += 1; }
    else if (cp < 0x800) { d[0] = (uint8_t)(0xC0 | cp >> 6); d[1] = (uint8_t)(0x80 | (cp & 0x3F)); o->n += 2; }
    else if (cp < 0x10000) {
        d[0] = (uint8_t)(0xE0 | cp >> 12); d[1] = (uint8_t)(0x80 | (cp >> 6 & 0x3F)); d[2] = (uint8_t)(0x80 | (cp & 0x3F));
        o->n += 3;
    } else {
        d[0] = (uint8_t)(0xF0 | cp >> 18); d[1] = (uint8_t)(0x80 | (cp >> 12 & 0x3F));
        d[2] = (uint8_t)(0x80 | (cp >> 6 & 0x3F)); d[3] = (uint8_t)(0x80 | (cp & 0x3F));
        o->n += 4;
    }
    return 0;
}

static uint32_t payload(Tokenizer *t, uint32_t cp) {
    if (cp >= NOT_UTF8) return 0;
    if (cp >= t->hit_lo && cp < t->hit_hi) return t->hit_val;
    uint32_t lo = 0, hi = t->n_uni; /* the last run starting at or before cp (the first starts at 0) */
    while (hi - lo > 1) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if ((t->uni[mid] & 0x1FFFFF) <= cp) lo = mid;
        else hi = mid;
    }
    t->hit_lo = t->uni[lo] & 0x1FFFFF;
    t->hit_hi = lo + 1 < t->n_uni ? (t->uni[lo + 1] & 0x1FFFFF) : NOT_UTF8;
    t->hit_val = t->uni[lo] >> 21;
    return t->hit_val;
}

static unsigned char_class(Tokenizer *t, uint32_t cp) { return cp < 128 ? t->ascii_cls[cp] : payload(t, cp) & 3; }
static unsigned comb_class(Tokenizer *t, uint32_t cp) { return payload(t, cp) >> 3 & 0xFF; }

/* ------------------------------------------------------------------------------------------------------
 * NFC (Unicode Standard Annex 15): canonical decomposition, canonical ordering, canonical composition.
 * Hangul syllables are decomposed and composed arithmetically (Unicode 3.12); the rest uses the tables. */

enum { H_SBASE = 0xAC00, H_LBASE = 0x1100, H_VBASE = 0x1161, H_TBASE = 0x11A7, H_LCOUNT = 19, H_VCOUNT = 21,
       H_TCOUNT = 28, H_NCOUNT = H_VCOUNT * H_TCOUNT, H_SCOUNT = H_LCOUNT * H_NCOUNT };

static int push_cp(Grow *g, uint32_t cp) {
    if (grow(g, g->n + 1, sizeof(uint32_t))) return -1;
    ((uint32_t *)g->p)[g->n++] = cp;
    return 0;
}

static int decompose_into(Tokenizer *t, uint32_t cp, Grow *g) {
    if (cp >= H_SBASE && cp < H_SBASE + H_SCOUNT) {
        const uint32_t s = cp - H_SBASE;
        if (push_cp(g, H_LBASE + s / H_NCOUNT) || push_cp(g, H_VBASE + s % H_NCOUNT / H_TCOUNT)) return -1;
        return s % H_TCOUNT ? push_cp(g, H_TBASE + s % H_TCOUNT) : 0;
    }
    uint32_t lo = 0, hi = t->n_dec;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (t->dec_cp[mid] < cp) lo = mid + 1;
        else hi = mid;
    }
    if (lo < t->n_dec && t->dec_cp[lo] == cp) {
        for (uint32_t k = t->dec_off[lo]; k < t->dec_off[lo + 1]; k++)
            if (push_cp(g, t->dec_pool[k])) return -1;
        return 0;
    }
    return push_cp(g, cp);
}

static uint32_t compose(const Tokenizer *t, uint32_t a, uint32_t b) {
    if (a >= H_LBASE && a < H_LBASE + H_LCOUNT && b >= H_VBASE && b < H_VBASE + H_VCOUNT)
        return H_SBASE + ((a - H_LBASE) * H_VCOUNT + (b - H_VBASE)) * H_TCOUNT;
    if (a >= H_SBASE && a < H_SBASE + H_SCOUNT && (a - H_SBASE) % H_TCOUNT == 0 && b > H_TBASE &&
        b < H_TBASE + H_TCOUNT)
        return a + (b - H_TBASE);
    uint32_t lo = 0, hi = t->n_comp;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        const uint32_t *e = t->comp + 3 * (size_t)mid;
        if (e[0] < a || (e[0] == a && e[1] < b)) lo = mid + 1;
        else hi = mid;
    }
    const uint32_t *e = t->comp + 3 * (size_t)lo;
    return lo < t->n_comp && e[0] == a && e[1] == b ? e[2] : 0;
}

/* NFC of the code points src[0..n), appended to t->out as UTF-8 */
static int nfc_append(Tokenizer *t, const uint32_t *src, size_t n) {
    Grow *d = &t->marks; /* decomposed code points, then their combining classes after them */
    d->n = 0;
    for (size_t i = 0; i < n; i++)
        if (decompose_into(t, src[i], d)) return -1;
    const size_t m = d->n;
    if (grow(d, 2 * m, sizeof(uint32_t))) return -1;
    uint32_t *c = (uint32_t *)d->p, *cc = c + m;
    for (size_t i = 0; i < m; i++) cc[i] = comb_class(t, c[i]);
    /* canonical ordering: a stable sort of each run of non-starters by combining class */
    for (size_t i = 1; i < m; i++) {
        const uint32_t x = c[i], k = cc[i];
        if (!k) continue;
        size_t j = i;
        for (; j > 0 && cc[j - 1] > k; j--) { c[j] = c[j - 1]; cc[j] = cc[j - 1]; }
        c[j] = x;
        cc[j] = k;
    }
    /* canonical composition: a character joins the last starter unless something in between blocks it
     * (after the ordering, only the character just before it can) */
    size_t w = 0, starter = (size_t)-1;
    for (size_t i = 0; i < m; i++) {
        const uint32_t x = c[i], k = cc[i];
        if (starter != (size_t)-1 && (w - 1 == starter || (cc[w - 1] != 0 && cc[w - 1] < k))) {
            const uint32_t y = compose(t, c[starter], x);
            if (y) {
                c[starter] = y;
                continue;
            }
        }
        if (k == 0) starter = w;
        c[w] = x;
        cc[w] = k;
        w++;
    }
    for (size_t i = 0; i < w; i++)
        if (utf8_put(&t->out, c[i])) return -1;
    return 0;
}

/* NFC of s[0..n): s itself when nothing changes, else t->out's bytes; NULL when out of memory */
static const uint8_t *normalize(Tokenizer *t, const uint8_t *s, size_t n, size_t *outn) {
    size_t copied = 0; /* s[0..copied) is in t->out already (once t->out is in use) */
    int used = 0;
    for (size_t i = 0; i < n;) {
        if (s[i] < 0x80) { i++; continue; }
        size_t e = i;
        int dirty = 0;
        while (e < n && s[e] >= 0x80) {
            uint32_t cp;
            e += (size_t)utf8_next(s + e, n - e, &cp);
            if (payload(t, cp) & 4) dirty = 1;
        }
        if (dirty) {
            const size_t from = i > 0 ? i - 1 : i; /* the ASCII character before the run joins it */
            if (!used) { t->out.n = 0; used = 1; }
            if (grow(&t->out, t->out.n + (from - copied), 1)) return NULL;
            memcpy((uint8_t *)t->out.p + t->out.n, s + copied, from - copied);
            t->out.n += from - copied;
            t->cps.n = 0;
            for (size_t k = from; k < e;) {
                uint32_t cp;
                k += (size_t)utf8_next(s + k, e - k, &cp);
                if (push_cp(&t->cps, cp)) return NULL;
            }
            if (nfc_append(t, (const uint32_t *)t->cps.p, t->cps.n)) return NULL;
            copied = e;
        }
        i = e;
    }
    if (!used) { *outn = n; return s; }
    if (grow(&t->out, t->out.n + (n - copied), 1)) return NULL;
    memcpy((uint8_t *)t->out.p + t->out.n, s + copied, n - copied);
    t->out.n += n - copied;
    *outn = t->out.n;
    return (const uint8_t *)t->out.p;
}

/* ------------------------------------------------------------------------------------------------------
 * pre-tokenizer: the end of the pre-token starting at s[i] (i < n) */

/* length of the contraction after an apostrophe at s[0..n) (case-insensitive s t m d re ve ll; the long s
 * U+017F folds to s under the (?i) of the regex), 0 if none */
static size_t contraction_len(const uint8_t *s, size_t n) {
    if (n == 0) return 0;
    const int c = s[0] | 0x20;
    if (c == 's' || c == 't' || c == 'm' || c == 'd') return 1;
    if (n >= 2 && ((c == 'r' || c == 'v') && (s[1] | 0x20) == 'e')) return 2;
    if (n >= 2 && c == 'l' && (s[1] | 0x20) == 'l') return 2;
    if (n >= 2 && s[0] == 0xC5 && s[1] == 0xBF) return 2;
    return 0;
}

static size_t skip_class(Tokenizer *t, const uint8_t *s, size_t j, size_t n, unsigned cls) {
    while (j < n) {
        uint32_t cp;
        const int l = utf8_next(s + j, n - j, &cp);
        if (char_class(t, cp) != cls) break;
        j += (size_t)l;
    }
    return j;
}

static size_t pretoken_end(Tokenizer *t, const uint8_t *s, size_t i, size_t n) {
    uint32_t c, d;
    const size_t l = (size_t)utf8_next(s + i, n - i, &c);
    const unsigned k = char_class(t, c);
    size_t j;
    /* 1. 's 't 're 've 'm 'll 'd */
    if (c == '\'' && (j = contraction_len(s + i + 1, n - i - 1)) > 0) return i + 1 + j;
    /* 2. [^\r\n\p{L}\p{N}]?\p{L}+ : letters, possibly after one character that is none of those */
    if (k == CL_LETTER) return skip_class(t, s, i + l, n, CL_LETTER);
    if (c != '\r' && c != '\n' && k != CL_NUMBER && i + l < n) {
        const size_t l2 = (size_t)utf8_next(s + i + l, n - i - l, &d);
        if (char_class(t, d) == CL_LETTER) return skip_class(t, s, i + l + l2, n, CL_LETTER);
    }
    /* 3. \p{N} : one digit */
    if (k == CL_NUMBER) return i + l;
    /* 4.  ?[^\s\p{L}\p{N}]+[\r\n]* : an optional space, other characters, trailing line breaks */
    j = c == ' ' ? i + 1 : i;
    if (j < n) {
        const size_t l2 = (size_t)utf8_next(s + j, n - j, &d);
        if (char_class(t, d) == CL_OTHER) {
            j = skip_class(t, s, j + l2, n, CL_OTHER);
            while (j < n && (s[j] == '\r' || s[j] == '\n')) j++;
            return j;
        }
    }
    /* c is white space: W = the maximal white-space run starting at i */
    size_t end = i, last = i, after_nl = 0;
    while (end < n) {
        const size_t l2 = (size_t)utf8_next(s + end, n - end, &d);
        if (char_class(t, d) != CL_SPACE) break;
        last = end;
        if (d == '\r' || d == '\n') after_nl = end + l2;
        end += l2;
    }
    if (after_nl) return after_nl; /* 5. \s*[\r\n]+ : through W's last line break */
    if (end == n) return end;      /* 6. \s+(?!\S) : all of W at the end of the text, */
    if (last > i) return last;     /*    else W without its last character */
    return end;                    /* 7. \s+ */
}

/* ------------------------------------------------------------------------------------------------------
 * BPE over one pre-token */

static uint64_t pair_key(uint32_t a, uint32_t b) { return (uint64_t)a << 32 | b; }
static uint32_t slot_of(uint64_t key, uint32_t mask) {
    uint64_t h = (key + 1) * 0x9E3779B97F4A7C15ull;
    return (uint32_t)(h >> 40) & mask;
}

static int rank_of(const Tokenizer *t, int32_t a, int32_t b) {
    const uint64_t key = pair_key((uint32_t)a, (uint32_t)b) + 1; /* +1: key 0 marks an empty slot */
    for (uint32_t h = slot_of(key, t->mmask);; h = (h + 1) & t->mmask) {
        if (t->mkey[h] == 0) return -1;
        if (t->mkey[h] == key) return (int)t->mval[h];
    }
}

typedef struct {
    int32_t id, prev, next;
} Sym;

static int cand_less(const Cand *a, const Cand *b) { return a->rank < b->rank || (a->rank == b->rank && a->pos < b->pos); }

static int queue_pair(Tokenizer *t, const Sym *sy, int32_t p) {
    const int32_t q = sy[p].next;
    const int r = rank_of(t, sy[p].id, sy[q].id);
    if (r < 0) return 0;
    Grow *g = &t->queue;
    if (grow(g, g->n + 1, sizeof(Cand))) return -1;
    Cand *h = (Cand *)g->p, x = {(uint32_t)r, (uint32_t)p, sy[p].id, sy[q].id};
    size_t i = g->n++;
    while (i > 0 && cand_less(&x, &h[(i - 1) / 2])) { h[i] = h[(i - 1) / 2]; i = (i - 1) / 2; }
    h[i] = x;
    return 0;
}

static Cand queue_pop(Tokenizer *t) {
    Grow *g = &t->queue;
    Cand *h = (Cand *)g->p, top = h[0], x = h[--g->n];
    size_t i = 0;
    for (;;) {
        size_t c = 2 * i + 1;
        if (c >= g->n) break;
        if (c + 1 < g->n && cand_less(&h[c + 1], &h[c])) c++;
        if (!cand_less(&h[c], &x)) break;
        h[i] = h[c];
        i = c;
    }
    if (g->n) h[i] = x;
    return top;
}

/* appends the ids of the pre-token w[0..n) to ids; -1 when they do not fit or memory runs out */
static int bpe(Tokenizer *t, const uint8_t *w, size_t n, int *ids, int *cnt, int max_ids) {
    if (grow(&t->sym, n, sizeof(Sym))) return -1;
    Sym *sy = (Sym *)t->sym.p;
    const int32_t end = (int32_t)n;
    for (int32_t i = 0; i < end; i++) sy[i] = (Sym){t->byte_tok[w[i]], i - 1, i + 1};
    t->queue.n = 0;
    for (int32_t i = 0; i + 1 < end; i++)
        if (queue_pair(t, sy, i)) return -1;
    while (t->queue.n) {
        const Cand c = queue_pop(t);
        const int32_t p = (int32_t)c.pos, q = sy[p].next;
        if (sy[p].id != c.left || q >= end || sy[q].id != c.right) continue; /* merged away since queued */
        sy[p].id = (int32_t)t->merges[3 * (size_t)c.rank + 2];
        sy[q].id = -1;
        sy[p].next = sy[q].next;
        if (sy[q].next < end) sy[sy[q].next].prev = p;
        if (sy[p].prev >= 0 && queue_pair(t, sy, sy[p].prev)) return -1;
        if (sy[p].next < end && queue_pair(t, sy, p)) return -1;
    }
    for (int32_t i = 0; i < end; i = sy[i].next) {
        if (*cnt >= max_ids) return -1;
        ids[(*cnt)++] = sy[i].id;
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------------
 * encode / decode */

static int encode_plain(Tokenizer *t, const uint8_t *s, size_t n, int *ids, int *cnt, int max_ids) {
    s = normalize(t, s, n, &n);
    if (!s) return -1;
    for (size_t i = 0; i < n;) {
        const size_t j = pretoken_end(t, s, i, n);
        if (bpe(t, s + i, j - i, ids, cnt, max_ids)) return -1;
        i = j;
    }
    return 0;
}

int tok_encode(Tokenizer *t, const char *text, int allow_special, int *ids, int max_ids) {
    const uint8_t *s = (const uint8_t *)text;
    const size_t n = strlen(text);
    int cnt = 0;
    size_t from = 0;
    for (size_t k = 0; k <= n; k++) {
        const Special *best = NULL;
        if (k < n && allow_special && t->spec_lead[s[k]])
            for (uint32_t a = 0; a < t->n_added; a++) {
                const Special *x = &t->spec[a];
                if (x->len <= n - k && !memcmp(s + k, x->text, x->len) && (!best || x->len > best->len)) best = x;
            }
        if (!best && k < n) continue;
        if (encode_plain(t, s + from, k - from, ids, &cnt, max_ids)) return -1;
        if (!best) break;
        if (cnt >= max_ids) return -1;
        ids[cnt++] = (int)best->id;
        from = k + best->len;
        k = from - 1;
    }
    return cnt;
}

const char *tok_decode(Tokenizer *t, int id, int *len) {
    if (id >= 0 && (uint32_t)id < t->n_vocab) {
        *len = t->tlen[id];
        return (const char *)t->blob + t->toff[id];
    }
    for (uint32_t a = 0; a < t->n_added; a++)
        if (t->spec[a].id == (uint32_t)id) {
            *len = (int)t->spec[a].len;
            return t->spec[a].text;
        }
    *len = 0;
    return NULL;
}

int tok_id(Tokenizer *t, const char *added_token) {
    const size_t n = strlen(added_token);
    for (uint32_t a = 0; a < t->n_added; a++)
        if (t->spec[a].len == n && !memcmp(t->spec[a].text, added_token, n)) return (int)t->spec[a].id;
    return -1;
}

int tok_vocab_size(Tokenizer *t) { return (int)t->n_ids; }

/* ------------------------------------------------------------------------------------------------------
 * load */

void tok_free(Tokenizer *t) {
    if (!t) return;
    free(t->file);
    free(t->toff);
    free(t->mkey);
    free(t->mval);
    free(t->spec);
    free(t->cps.p);
    free(t->marks.p);
    free(t->out.p);
    free(t->sym.p);
    free(t->queue.p);
    free(t);
}

typedef struct {
    const uint8_t *p, *end;
} Cursor;

/* the next section of `bytes` bytes (then padding to 4), or NULL when the file is too short */
static const void *take(Cursor *c, size_t bytes) {
    const size_t padded = (bytes + 3) & ~(size_t)3;
    if (padded < bytes || padded > (size_t)(c->end - c->p)) return NULL;
    const void *r = c->p;
    c->p += padded;
    return r;
}

Tokenizer *tok_load(const char *path) {
    Tokenizer *t = (Tokenizer *)calloc(1, sizeof *t);
    const char *why = "out of memory";
    FILE *f = NULL;
    if (!t) goto fail;
    why = "cannot read the file";
    if (!(f = fopen(path, "rb")) || fseek(f, 0, SEEK_END)) goto fail;
    const long size = ftell(f);
    if (size < 56 || fseek(f, 0, SEEK_SET)) goto fail;
    if (!(t->file = (uint8_t *)malloc((size_t)size)) || fread(t->file, 1, (size_t)size, f) != (size_t)size) goto fail;
    fclose(f);
    f = NULL;
    why = "not a QWTOK001 tokenizer file, or a damaged one";
    if (memcmp(t->file, "QWTOK001", 8)) goto fail;
    uint32_t h[12];
    memcpy(h, t->file + 8, sizeof h);
    t->n_vocab = h[0]; t->n_added = h[1]; t->n_merges = h[2]; t->n_uni = h[4]; t->n_dec = h[5]; t->pool_len = h[6];
    t->n_comp = h[7];
    if (t->n_vocab < 256 || t->n_vocab > (1u << 24) || t->n_merges > (1u << 24) || t->n_uni == 0 ||
        t->n_added > (1u << 16))
        goto fail;
    Cursor c = {t->file + 56, t->file + size};
    if (!(t->tlen = (const uint8_t *)take(&c, t->n_vocab)) || !(t->blob = (const uint8_t *)take(&c, h[3])) ||
        !(t->merges = (const uint32_t *)take(&c, (size_t)t->n_merges * 12)))
        goto fail;
    if (!(t->spec = (Special *)calloc(t->n_added + 1, sizeof(Special)))) goto fail;
    t->n_ids = t->n_vocab;
    for (uint32_t a = 0; a < t->n_added; a++) {
        const uint32_t *e = (const uint32_t *)take(&c, 8);
        if (!e || e[1] == 0 || !(t->spec[a].text = (const char *)take(&c, e[1]))) goto fail;
        t->spec[a].id = e[0];
        t->spec[a].len = e[1];
        t->spec_lead[(uint8_t)t->spec[a].text[0]] = 1;
        if (e[0] >= t->n_ids) t->n_ids = e[0] + 1;
    }
    if (!(t->uni = (const uint32_t *)take(&c, (size_t)t->n_uni * 4)) ||
        !(t->dec_cp = (const uint32_t *)take(&c, (size_t)t->n_dec * 4)) ||
        !(t->dec_off = (const uint32_t *)take(&c, ((size_t)t->n_dec + 1) * 4)) ||
        !(t->dec_pool = (const uint32_t *)take(&c, (size_t)t->pool_len * 4)) ||
        !(t->comp = (const uint32_t *)take(&c, (size_t)t->n_comp * 12)))
        goto fail;
    for (uint32_t i = 0; i < t->n_dec; i++)
        if (t->dec_off[i] > t->dec_off[i + 1] || t->dec_off[i + 1] > t->pool_len) goto fail;
    /* token offsets; every byte needs a one-byte token */
    if (!(t->toff = (uint32_t *)malloc(((size_t)t->n_vocab + 1) * 4))) goto fail;
    uint64_t off = 0;
    for (uint32_t i = 0; i < t->n_vocab; i++) { t->toff[i] = (uint32_t)off; off += t->tlen[i]; }
    if (off != h[3]) goto fail;
    t->toff[t->n_vocab] = (uint32_t)off;
    for (int b = 0; b < 256; b++) t->byte_tok[b] = -1;
    for (uint32_t i = 0; i < t->n_vocab; i++)
        if (t->tlen[i] == 1 && t->byte_tok[t->blob[t->toff[i]]] < 0) t->byte_tok[t->blob[t->toff[i]]] = (int32_t)i;
    for (int b = 0; b < 256; b++)
        if (t->byte_tok[b] < 0) goto fail;
    /* merge table, load factor <= 1/2 */
    uint32_t slots = 1024;
    while (slots < 2 * t->n_merges) slots *= 2;
    t->mmask = slots - 1;
    if (!(t->mkey = (uint64_t *)calloc(slots, 8)) || !(t->mval = (uint32_t *)malloc((size_t)slots * 4))) goto fail;
    for (uint32_t r = 0; r < t->n_merges; r++) {
        const uint32_t *m = t->merges + 3 * (size_t)r;
        if (m[0] >= t->n_vocab || m[1] >= t->n_vocab || m[2] >= t->n_vocab) goto fail;
        const uint64_t key = pair_key(m[0], m[1]) + 1;
        uint32_t s = slot_of(key, t->mmask);
        while (t->mkey[s] && t->mkey[s] != key) s = (s + 1) & t->mmask;
        if (t->mkey[s]) continue; /* a repeated pair keeps its first (lowest) rank */
        t->mkey[s] = key;
        t->mval[s] = r;
    }
    t->hit_lo = t->hit_hi = 0;
    for (uint32_t cp = 0; cp < 128; cp++) t->ascii_cls[cp] = (uint8_t)(payload(t, cp) & 3);
    return t;
fail:
    fprintf(stderr, "tok_load(%s): %s\n", path, why);
    if (f) fclose(f);
    tok_free(t);
    return NULL;
}
