/* Qwen2 / Qwen2.5 byte-level BPE tokenizer of the C hosts (interface: qwen_tokenizer.h).
 *
 * Data: the "QWTOK001" file that the reference's tools/qwen_tok_export.py:21-41 writes (little-endian, every
 * section zero-padded to 4 bytes):
 *   magic[8], u32 hdr[12] = n_vocab, n_added, n_merges, blob_len, n_uni, n_dec, dec_pool_len, n_comp, 0...;
 *   u8 tok_len[n_vocab]; u8 blob[blob_len] (token bytes in id order); u32 merges[n_merges][3] (left, right,
 *   merged; the index is the merge rank); n_added x (u32 id, u32 len, u8 text[len]); u32 uni[n_uni] (runs of
 *   code points: start | payload << 21, payload = class (0 other, 1 letter, 2 number, 3 white space) |
 *   "NFC may change the text here" << 2 | canonical combining class << 3); u32 dec_cp[n_dec],
 *   dec_off[n_dec + 1], dec_pool[] (full canonical decompositions); u32 comp[n_comp][3] (first, second,
 *   composite).
 *
 * tok_encode gives the ids of Hugging Face `tokenizers` for the Qwen2 tokenizer.json:
 *   1. with allow_special, added tokens are cut out of the raw text: at the leftmost position where one
 *      starts, the longest one there;
 *   2. every span between them is put in NFC (UAX #15).  The span is cut before each "quiet" code point (a
 *      starter that NFC leaves alone and that never composes with what precedes it); only the pieces holding
 *      another code point are decomposed, reordered and recomposed;
 *   3. the normalized span is cut into pre-tokens by the Qwen2 Split regex
 *        (?i:'s|'t|'re|'ve|'m|'ll|'d) | [^\r\n\p{L}\p{N}]?\p{L}+ | \p{N} | ?[^\s\p{L}\p{N}]+[\r\n]* |
 *        \s*[\r\n]+ | \s+(?!\S) | \s+
 *      as a table of seven matchers over classified code points, tried in that order, each returning what a
 *      backtracking engine's greedy match of that alternative consumes;
 *   4. each pre-token's UTF-8 bytes start as the 256 single-byte tokens and are merged by BPE: the adjacent
 *      pair of lowest merge rank, the leftmost one among equal ranks, found with a min-tree over the pairs.
 * Bytes that are not UTF-8 become one-byte units of class "other" that normalization never touches.
 * One open-addressing hash map type serves the merges, the decompositions and the compositions.
 * Not thread-safe: a Tokenizer owns its scratch memory. */
#include "qwen_tokenizer.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { K_OTHER = 0, K_LETTER = 1, K_NUMBER = 2, K_SPACE = 3 };
#define PAY_DIRTY 4u
#define PSEUDO 0x110000u /* an undecodable byte b is the unit PSEUDO + b */
#define NO_PAIR UINT64_MAX

/* Hangul syllables (Unicode ch. 3.12) */
#define H_S 0xAC00u
#define H_L 0x1100u
#define H_V 0x1161u
#define H_T 0x11A7u
#define H_VN 21u
#define H_TN 28u
#define H_SN 11172u

/* ---- growable scratch ---------------------------------------------------------------------------------- */

typedef struct {
    void *p;
    size_t cap;
} Scratch;

static void *reserve(Scratch *s, size_t bytes) {
    if (bytes > s->cap) {
        size_t c = s->cap ? s->cap : 4096;
        while (c < bytes) c *= 2;
        void *q = realloc(s->p, c);
        if (!q) return NULL;
        s->p = q;
        s->cap = c;
    }
    return s->p;
}

/* ---- 64-bit key -> 32-bit value map (linear probing, keys never equal to EMPTY) -------------------------- */

#define EMPTY UINT64_MAX

typedef struct {
    uint64_t *key;
    uint32_t *val;
    size_t mask;
} Map;

static size_t slot_of(uint64_t k, size_t mask) {
    k ^= k >> 33;
    k *= 0xFF51AFD7ED558CCDull;
    k ^= k >> 29;
    return (size_t)k & mask;
}

static int map_init(Map *m, size_t entries) {
    size_t cap = 64;
    while (cap < entries * 2) cap *= 2;
    m->key = malloc(cap * sizeof *m->key);
    m->val = malloc(cap * sizeof *m->val);
    m->mask = cap - 1;
    if (!m->key || !m->val) return -1;
    memset(m->key, 0xFF, cap * sizeof *m->key);
    return 0;
}

/* keeps the first value given for a key */
static void map_put(Map *m, uint64_t k, uint32_t v) {
    size_t i = slot_of(k, m->mask);
    while (m->key[i] != EMPTY) {
        if (m->key[i] == k) return;
        i = (i + 1) & m->mask;
    }
    m->key[i] = k;
    m->val[i] = v;
}

static int64_t map_get(const Map *m, uint64_t k) {
    for (size_t i = slot_of(k, m->mask);; i = (i + 1) & m->mask) {
        if (m->key[i] == k) return m->val[i];
        if (m->key[i] == EMPTY) return -1;
    }
}

static void map_free(Map *m) {
    free(m->key);
    free(m->val);
}

/* ---- the tokenizer ---------------------------------------------------------------------------------------- */

typedef struct {
    uint32_t cp;  /* code point, or PSEUDO + byte */
    uint32_t off; /* byte offset in the span */
    uint16_t pay; /* Unicode payload */
    uint8_t len;  /* bytes */
} Unit;

typedef struct {
    uint32_t cp, ccc;
} Mark;

struct Tokenizer {
    uint8_t *data; /* the whole file: pieces, merges, added texts and Unicode tables point into it */
    uint32_t n_base, n_ids, n_added, n_runs;
    uint32_t *piece_at;  /* [n_ids] offset of the id's bytes in data */
    uint16_t *piece_len; /* [n_ids] their length, 0 where no id exists */
    const uint32_t *merges, *runs, *dec_off, *dec_pool;
    uint32_t *added_ids; /* added token ids, longest text first */
    uint8_t lead[32];    /* bitmap of the added tokens' first bytes */
    int32_t byte_tok[256];
    uint16_t low_pay[256]; /* payload of U+0000 .. U+00FF */
    Map pair_rank;         /* (left << 32 | right) -> merge rank */
    Map decomp;            /* code point -> index into dec_off */
    Map compose;           /* (first << 32 | second) -> composite */
    Scratch norm, units, marks, sym, tree, out;
};

/* the payload of the last run that starts at or before cp (runs[0] starts at 0) */
static uint32_t run_payload(const Tokenizer *t, uint32_t cp) {
    const uint32_t *r = t->runs;
    size_t n = t->n_runs;
    while (n > 1) {
        const size_t half = n / 2;
        if ((r[half] & 0x1FFFFF) <= cp) r += half;
        n -= half;
    }
    return *r >> 21;
}

static uint32_t payload(const Tokenizer *t, uint32_t cp) {
    if (cp < 256) return t->low_pay[cp];
    return cp >= PSEUDO ? 0 : run_payload(t, cp);
}

static inline unsigned unit_class(const Unit *u) { return u->pay & 3u; }
static inline int is_dirty(const Unit *u) { return (u->pay & PAY_DIRTY) != 0; }
static inline int is_crlf(uint32_t cp) { return cp == '\r' || cp == '\n'; }

/* One code point at s[0 .. n): its length in bytes.  Overlong forms, surrogates, values past U+10FFFF and cut
 * sequences come back one byte at a time as PSEUDO + byte. */
static int utf8_unit(const uint8_t *s, size_t n, uint32_t *cp) {
    static const uint8_t tail[16] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 2, 3};
    static const uint32_t least[4] = {0, 0x80, 0x800, 0x10000};
    const uint32_t b = s[0];
    const int k = tail[b >> 4];
    if (b < 0x80) {
        *cp = b;
        return 1;
    }
    if (k && (size_t)k < n && b < 0xF5) {
        uint32_t v = b & (0x3Fu >> k);
        int i = 1;
        for (; i <= k && (s[i] & 0xC0) == 0x80; i++) v = v << 6 | (s[i] & 0x3F);
        if (i > k && v >= least[k] && v < PSEUDO && (v & 0xFFFFF800u) != 0xD800u) {
            *cp = v;
            return k + 1;
        }
    }
    *cp = PSEUDO + b;
    return 1;
}

static size_t utf8_write(uint8_t *o, uint32_t cp) {
    if (cp >= PSEUDO) {
        o[0] = (uint8_t)(cp - PSEUDO);
        return 1;
    }
    if (cp < 0x80) {
        o[0] = (uint8_t)cp;
        return 1;
    }
    size_t n = cp < 0x800 ? 2 : cp < 0x10000 ? 3 : 4;
    for (size_t i = n - 1; i > 0; i--, cp >>= 6) o[i] = (uint8_t)(0x80 | (cp & 0x3F));
    o[0] = (uint8_t)((0xF00u >> n) | cp); /* 2: 0xC0, 3: 0xE0, 4: 0xF0 lead bits */
    return n;
}

/* the units of s[0 .. n) into t->units; NULL when out of memory */
static Unit *split_units(Tokenizer *t, const uint8_t *s, size_t n, size_t *count) {
    Unit *u = reserve(&t->units, (n + 1) * sizeof(Unit));
    if (!u) return NULL;
    size_t k = 0;
    for (size_t i = 0; i < n; k++) {
        const int l = utf8_unit(s + i, n - i, &u[k].cp);
        u[k].off = (uint32_t)i;
        u[k].len = (uint8_t)l;
        u[k].pay = (uint16_t)payload(t, u[k].cp);
        i += (size_t)l;
    }
    *count = k;
    return u;
}

/* ---- NFC ------------------------------------------------------------------------------------------------ */

static uint32_t ccc_of(const Tokenizer *t, uint32_t cp) { return payload(t, cp) >> 3 & 0xFF; }

static uint32_t composite(const Tokenizer *t, uint32_t a, uint32_t b) {
    if (a - H_L < 19 && b - H_V < H_VN) return H_S + ((a - H_L) * H_VN + (b - H_V)) * H_TN;
    if (a - H_S < H_SN && (a - H_S) % H_TN == 0 && b - H_T - 1 < H_TN - 1) return a + (b - H_T);
    const int64_t c = map_get(&t->compose, (uint64_t)a << 32 | b);
    return c < 0 ? 0 : (uint32_t)c;
}

/* appends the canonical decomposition of cp to m (room for 4 code points); returns the new count */
static size_t decompose(const Tokenizer *t, uint32_t cp, Mark *m, size_t k) {
    if (cp - H_S < H_SN) {
        const uint32_t s = cp - H_S;
        m[k++].cp = H_L + s / (H_VN * H_TN);
        m[k++].cp = H_V + s % (H_VN * H_TN) / H_TN;
        if (s % H_TN) m[k++].cp = H_T + s % H_TN;
        return k;
    }
    const int64_t e = cp < PSEUDO ? map_get(&t->decomp, cp) : -1;
    if (e < 0) {
        m[k++].cp = cp;
        return k;
    }
    for (uint32_t i = t->dec_off[e]; i < t->dec_off[e + 1]; i++) m[k++].cp = t->dec_pool[i];
    return k;
}

/* NFC of the units u[0 .. k) appended to o; returns the bytes written (at most 4 per code point) */
static size_t nfc_piece(Tokenizer *t, const Unit *u, size_t k, uint8_t *o, Mark *m) {
    size_t n = 0;
    for (size_t i = 0; i < k; i++) n = decompose(t, u[i].cp, m, n);
    for (size_t i = 0; i < n; i++) m[i].ccc = m[i].cp < PSEUDO ? ccc_of(t, m[i].cp) : 0;
    /* canonical order: every run of non-starters sorted by combining class, equal classes kept in order */
    for (size_t i = 0; i < n;) {
        if (!m[i].ccc) {
            i++;
            continue;
        }
        size_t e = i;
        while (e < n && m[e].ccc) e++;
        for (size_t a = i + 1; a < e; a++) {
            const Mark x = m[a];
            size_t b = a;
            for (; b > i && m[b - 1].ccc > x.ccc; b--) m[b] = m[b - 1];
            m[b] = x;
        }
        i = e;
    }
    /* canonical composition: a mark joins the last starter unless something between blocks it */
    size_t w = 0, bytes = 0;
    long st = -1;
    for (size_t i = 0; i < n; i++) {
        const Mark x = m[i];
        if (st >= 0) {
            const int adjacent = (size_t)st == w - 1;
            if (adjacent || m[w - 1].ccc < x.ccc) {
                const uint32_t c = composite(t, m[st].cp, x.cp);
                if (c) {
                    m[st].cp = c;
                    continue;
                }
            }
        }
        if (!x.ccc) st = (long)w;
        m[w++] = x;
    }
    for (size_t i = 0; i < w; i++) bytes += utf8_write(o + bytes, m[i].cp);
    return bytes;
}

/* NFC of s[0 .. n): s itself when nothing can change, else t->norm; NULL when out of memory */
static const uint8_t *nfc(Tokenizer *t, const uint8_t *s, size_t n, size_t *out_n) {
    size_t nu;
    Unit *u = split_units(t, s, n, &nu);
    if (!u) return NULL;
    size_t first = 0;
    while (first < nu && !is_dirty(&u[first])) first++;
    if (first == nu) {
        *out_n = n;
        return s;
    }
    /* a canonical decomposition is at most 4 code points, and composition only shortens */
    uint8_t *o = reserve(&t->norm, 16 * nu + 16);
    Mark *m = reserve(&t->marks, (4 * nu + 4) * sizeof(Mark));
    if (!o || !m) return NULL;
    size_t on = 0;
    for (size_t a = 0; a < nu;) {
        /* quiet units that no following unit depends on are copied as they are */
        size_t b = a;
        while (b < nu && !is_dirty(&u[b]) && !(b + 1 < nu && is_dirty(&u[b + 1]))) b++;
        const size_t from = u[a].off, to = b < nu ? u[b].off : n;
        memcpy(o + on, s + from, to - from);
        on += to - from;
        if (b == nu) break;
        /* a piece: its head (quiet, or the span's first unit) and the units up to the next quiet one */
        size_t e = b + 1;
        while (e < nu && is_dirty(&u[e])) e++;
        on += nfc_piece(t, u + b, e - b, o + on, m);
        a = e;
    }
    *out_n = on;
    return o;
}

/* ---- pre-tokenizer: the alternatives of the Split regex, each the length of its match in units (0 = none) */

typedef size_t (*Alternative)(const Unit *u, size_t i, size_t n);

static size_t run_of(const Unit *u, size_t i, size_t n, unsigned cls) {
    size_t j = i;
    while (j < n && unit_class(&u[j]) == cls) j++;
    return j - i;
}

/* (?i:'s|'t|'re|'ve|'m|'ll|'d): under Oniguruma's case folding the only other spelling is U+017F for s */
static size_t alt_contraction(const Unit *u, size_t i, size_t n) {
    static const char *const tails[] = {"s", "t", "re", "ve", "m", "ll", "d"};
    if (u[i].cp != '\'') return 0;
    for (size_t k = 0; k < sizeof tails / sizeof *tails; k++) {
        const size_t len = strlen(tails[k]);
        size_t j = 0;
        for (; j < len && i + 1 + j < n; j++) {
            const uint32_t c = u[i + 1 + j].cp, want = (uint32_t)tails[k][j];
            if (c != want && c != want - 32 && !(want == 's' && c == 0x17F)) break;
        }
        if (j == len) return 1 + len;
    }
    return 0;
}

/* [^\r\n\p{L}\p{N}]?\p{L}+ */
static size_t alt_letters(const Unit *u, size_t i, size_t n) {
    size_t lead = 0;
    if (unit_class(&u[i]) != K_LETTER) {
        if (unit_class(&u[i]) == K_NUMBER || is_crlf(u[i].cp)) return 0;
        lead = 1;
    }
    const size_t m = run_of(u, i + lead, n, K_LETTER);
    return m ? lead + m : 0;
}

/* \p{N} */
static size_t alt_number(const Unit *u, size_t i, size_t n) {
    (void)n;
    return unit_class(&u[i]) == K_NUMBER;
}

/*  ?[^\s\p{L}\p{N}]+[\r\n]* */
static size_t alt_symbols(const Unit *u, size_t i, size_t n) {
    size_t j = i + (u[i].cp == ' ');
    const size_t m = run_of(u, j, n, K_OTHER);
    if (!m) return 0; /* without the space the run would start on white space */
    for (j += m; j < n && is_crlf(u[j].cp); j++) {
    }
    return j - i;
}

/* \s*[\r\n]+ : through the last CR / LF of the white-space run */
static size_t alt_newlines(const Unit *u, size_t i, size_t n) {
    const size_t m = run_of(u, i, n, K_SPACE);
    size_t end = 0;
    for (size_t k = 0; k < m; k++)
        if (is_crlf(u[i + k].cp)) end = k + 1;
    return end;
}

/* \s+(?!\S) : the run when it ends the text, else the run but its last unit */
static size_t alt_trailing_space(const Unit *u, size_t i, size_t n) {
    const size_t m = run_of(u, i, n, K_SPACE);
    return i + m == n ? m : m ? m - 1 : 0;
}

/* \s+ */
static size_t alt_space(const Unit *u, size_t i, size_t n) { return run_of(u, i, n, K_SPACE); }

static const Alternative split_regex[] = {alt_contraction, alt_letters, alt_number, alt_symbols,
                                          alt_newlines, alt_trailing_space, alt_space};

static size_t pretoken(const Unit *u, size_t i, size_t n) {
    for (size_t a = 0; a < sizeof split_regex / sizeof *split_regex; a++) {
        const size_t m = split_regex[a](u, i, n);
        if (m) return m;
    }
    return 1; /* every class has an alternative above; kept for safety */
}

/* ---- BPE -------------------------------------------------------------------------------------------------- */

/* key of the pair that starts at slot i: rank << 32 | i (lowest rank, then leftmost), NO_PAIR without a merge */
static uint64_t pair_key(const Tokenizer *t, int32_t a, int32_t b, size_t i) {
    const int64_t r = map_get(&t->pair_rank, (uint64_t)(uint32_t)a << 32 | (uint32_t)b);
    return r < 0 ? NO_PAIR : (uint64_t)r << 32 | i;
}

/* min-tree with `leaves` leaves in tr[leaves .. 2 leaves) */
static void tree_set(uint64_t *tr, size_t leaves, size_t i, uint64_t key) {
    size_t k = leaves + i;
    tr[k] = key;
    for (k >>= 1; k; k >>= 1) {
        const uint64_t l = tr[2 * k], r = tr[2 * k + 1], v = l < r ? l : r;
        if (tr[k] == v) break;
        tr[k] = v;
    }
}

/* BPE of the bytes w[0 .. n) (n >= 1): the ids in order into t->out; returns their count, -1 on no memory */
static long bpe(Tokenizer *t, const uint8_t *w, size_t n) {
    int32_t *out = reserve(&t->out, n * sizeof(int32_t));
    if (!out) return -1;
    if (n == 1) {
        out[0] = t->byte_tok[w[0]];
        return 1;
    }
    size_t leaves = 1;
    while (leaves < n) leaves *= 2;
    int32_t *sym = reserve(&t->sym, 3 * n * sizeof(int32_t));
    uint64_t *tr = reserve(&t->tree, 2 * leaves * sizeof(uint64_t));
    if (!sym || !tr) return -1;
    int32_t *next = sym + n, *prev = sym + 2 * n; /* neighbours among the live slots (n / -1 at the ends) */
    for (size_t i = 0; i < n; i++) {
        sym[i] = t->byte_tok[w[i]];
        next[i] = (int32_t)i + 1;
        prev[i] = (int32_t)i - 1;
    }
    for (size_t i = 0; i < 2 * leaves; i++) tr[i] = NO_PAIR;
    for (size_t i = 0; i + 1 < n; i++) tr[leaves + i] = pair_key(t, sym[i], sym[i + 1], i);
    for (size_t k = leaves - 1; k; k--) tr[k] = tr[2 * k] < tr[2 * k + 1] ? tr[2 * k] : tr[2 * k + 1];
    while (tr[1] != NO_PAIR) {
        const size_t p = (uint32_t)tr[1], q = (size_t)next[p];
        sym[p] = (int32_t)t->merges[3 * (tr[1] >> 32) + 2];
        next[p] = next[q];
        if ((size_t)next[q] < n) prev[next[q]] = (int32_t)p;
        tree_set(tr, leaves, q, NO_PAIR);
        tree_set(tr, leaves, p, (size_t)next[p] < n ? pair_key(t, sym[p], sym[next[p]], p) : NO_PAIR);
        if (prev[p] >= 0) tree_set(tr, leaves, (size_t)prev[p], pair_key(t, sym[prev[p]], sym[p], (size_t)prev[p]));
    }
    long c = 0;
    for (size_t i = 0; i < n; i = (size_t)next[i]) out[c++] = sym[i];
    return c;
}

/* ---- encode / decode ------------------------------------------------------------------------------------- */

/* ids of one span without added tokens, appended at ids[*count] */
static int encode_span(Tokenizer *t, const uint8_t *s, size_t n, int *ids, int max_ids, int *count) {
    if (!n) return 0;
    size_t m, nu;
    const uint8_t *x = nfc(t, s, n, &m);
    if (!x) return -1;
    const Unit *u = split_units(t, x, m, &nu);
    if (!u) return -1;
    for (size_t i = 0; i < nu;) {
        const size_t k = pretoken(u, i, nu), from = u[i].off, to = i + k < nu ? u[i + k].off : m;
        const long c = bpe(t, x + from, to - from);
        if (c < 0 || c > (long)max_ids - *count) return -1;
        memcpy(ids + *count, t->out.p, (size_t)c * sizeof(int));
        *count += (int)c;
        i += k;
    }
    return 0;
}

int tok_encode(Tokenizer *t, const char *text, int allow_special, int *ids, int max_ids) {
    const uint8_t *s = (const uint8_t *)text;
    const size_t n = strlen(text);
    int count = 0;
    if (max_ids < 0) max_ids = 0;
    for (size_t pos = 0;;) {
        /* the next added token: leftmost start, longest text there */
        size_t at = n;
        int64_t hit = -1;
        for (size_t k = pos; allow_special && hit < 0 && k < n; k++) {
            if (!(t->lead[s[k] >> 3] >> (s[k] & 7) & 1)) continue;
            for (uint32_t a = 0; a < t->n_added; a++) {
                const uint32_t id = t->added_ids[a], len = t->piece_len[id];
                if (len <= n - k && !memcmp(s + k, t->data + t->piece_at[id], len)) {
                    hit = id;
                    at = k;
                    break;
                }
            }
        }
        if (encode_span(t, s + pos, at - pos, ids, max_ids, &count)) return -1;
        if (hit < 0) return count;
        if (count >= max_ids) return -1;
        ids[count++] = (int)hit;
        pos = at + t->piece_len[hit];
    }
}

const char *tok_decode(Tokenizer *t, int id, int *len) {
    const int known = id >= 0 && (uint32_t)id < t->n_ids && t->piece_len[id];
    *len = known ? t->piece_len[id] : 0;
    return known ? (const char *)t->data + t->piece_at[id] : NULL;
}

int tok_id(Tokenizer *t, const char *added_token) {
    const size_t n = strlen(added_token);
    for (uint32_t a = 0; a < t->n_added; a++) {
        const uint32_t id = t->added_ids[a];
        if (t->piece_len[id] == n && !memcmp(t->data + t->piece_at[id], added_token, n)) return (int)id;
    }
    return -1;
}

int tok_vocab_size(Tokenizer *t) { return (int)t->n_ids; }

/* ---- load ----------------------------------------------------------------------------------------------------- */

void tok_free(Tokenizer *t) {
    if (!t) return;
    map_free(&t->pair_rank);
    map_free(&t->decomp);
    map_free(&t->compose);
    Scratch *s[] = {&t->norm, &t->units, &t->marks, &t->sym, &t->tree, &t->out};
    for (size_t i = 0; i < sizeof s / sizeof *s; i++) free(s[i]->p);
    free(t->piece_at);
    free(t->piece_len);
    free(t->added_ids);
    free(t->data);
    free(t);
}

typedef struct {
    const uint8_t *at, *end;
} Cursor;

/* the next section of `bytes` bytes (padded to 4), NULL past the end of the file */
static const void *section(Cursor *c, uint64_t bytes) {
    const uint64_t padded = (bytes + 3) & ~(uint64_t)3;
    if (padded > (uint64_t)(c->end - c->at)) return NULL;
    const void *p = c->at;
    c->at += padded;
    return p;
}

static uint8_t *read_file(const char *path, size_t *size) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    uint8_t *buf = NULL;
    long n = -1;
    if (!fseek(f, 0, SEEK_END)) n = ftell(f);
    if (n > 0 && !fseek(f, 0, SEEK_SET) && (buf = malloc((size_t)n)) && fread(buf, 1, (size_t)n, f) == (size_t)n) {
        *size = (size_t)n;
    } else {
        free(buf);
        buf = NULL;
    }
    fclose(f);
    return buf;
}

/* parses the file held in t->data; returns NULL or what is wrong with it */
static const char *parse(Tokenizer *t, size_t size) {
    Cursor c = {t->data, t->data + size};
    const char *magic = section(&c, 8);
    const uint32_t *h = section(&c, 48);
    if (!magic || !h || memcmp(magic, "QWTOK001", 8)) return "not a QWTOK001 file";
    const uint32_t n_vocab = h[0], n_added = h[1], n_merges = h[2], blob_len = h[3], n_runs = h[4], n_dec = h[5],
                   pool_len = h[6], n_comp = h[7];
    if (n_vocab < 256 || n_vocab > (1u << 20) || n_added > 4096 || n_runs == 0) return "bad header";
    const uint8_t *len = section(&c, n_vocab), *blob = section(&c, blob_len);
    t->merges = section(&c, 12ull * n_merges);
    if (!len || !blob || !t->merges) return "file too short";
    t->n_base = n_vocab;
    t->n_added = n_added;
    /* ids: the base vocabulary, then the added tokens (their ids given in the file) */
    const uint32_t **added = calloc(n_added + 1, sizeof *added);
    if (!added) return "out of memory";
    uint32_t n_ids = n_vocab;
    const char *why = NULL;
    for (uint32_t a = 0; a < n_added && !why; a++) {
        const uint32_t *e = section(&c, 8);
        if (!e || !section(&c, e[1])) why = "file too short";
        else if (e[0] < n_vocab || e[0] >= (1u << 20) || e[1] == 0 || e[1] > 0xFFFF) why = "bad added token";
        else {
            added[a] = e;
            if (e[0] + 1 > n_ids) n_ids = e[0] + 1;
        }
    }
    t->runs = why ? NULL : section(&c, 4ull * n_runs);
    const uint32_t *dec_cp = section(&c, 4ull * n_dec);
    t->dec_off = section(&c, 4ull * n_dec + 4);
    t->dec_pool = section(&c, 4ull * pool_len);
    const uint32_t *comp = section(&c, 12ull * n_comp);
    if (!why && (!t->runs || !dec_cp || !t->dec_off || !t->dec_pool || !comp)) why = "file too short";
    if (!why && (t->runs[0] & 0x1FFFFF)) why = "bad Unicode table";
    for (uint32_t i = 0; !why && i < n_dec; i++)
        if (t->dec_off[i] > t->dec_off[i + 1] || t->dec_off[i + 1] > pool_len || t->dec_off[i + 1] - t->dec_off[i] > 4)
            why = "bad decomposition table";
    t->n_ids = n_ids;
    t->piece_at = calloc(n_ids, sizeof *t->piece_at);
    t->piece_len = calloc(n_ids, sizeof *t->piece_len);
    t->added_ids = calloc(n_added + 1, sizeof *t->added_ids);
    if (!why && (!t->piece_at || !t->piece_len || !t->added_ids)) why = "out of memory";
    if (why) {
        free(added);
        return why;
    }
    uint64_t off = (uint64_t)(blob - t->data);
    for (uint32_t i = 0; i < n_vocab; i++) {
        t->piece_at[i] = (uint32_t)off;
        t->piece_len[i] = len[i];
        off += len[i];
        if (!len[i]) why = "empty token";
    }
    if (off != (uint64_t)(blob - t->data) + blob_len) why = "token lengths do not add up to the blob";
    for (uint32_t a = 0; a < n_added; a++) {
        const uint32_t id = added[a][0];
        if (t->piece_len[id]) why = "an id twice";
        t->piece_at[id] = (uint32_t)((const uint8_t *)(added[a] + 2) - t->data);
        t->piece_len[id] = (uint16_t)added[a][1];
        t->added_ids[a] = id;
        const uint8_t b = ((const uint8_t *)(added[a] + 2))[0];
        t->lead[b >> 3] |= (uint8_t)(1u << (b & 7));
    }
    free(added);
    /* longest added token first (the match taken at a position), ties by id */
    for (uint32_t a = 1; a < n_added; a++) {
        const uint32_t id = t->added_ids[a];
        uint32_t b = a;
        for (; b > 0 && t->piece_len[t->added_ids[b - 1]] < t->piece_len[id]; b--) t->added_ids[b] = t->added_ids[b - 1];
        t->added_ids[b] = id;
    }
    for (int b = 0; b < 256; b++) t->byte_tok[b] = -1;
    for (uint32_t i = 0; i < n_vocab; i++)
        if (len[i] == 1) t->byte_tok[t->data[t->piece_at[i]]] = (int32_t)i;
    for (int b = 0; b < 256; b++)
        if (t->byte_tok[b] < 0) why = "a single-byte token is missing";
    if (why) return why;
    t->n_runs = n_runs;
    for (uint32_t cp = 0; cp < 256; cp++) t->low_pay[cp] = (uint16_t)run_payload(t, cp);
    if (map_init(&t->pair_rank, n_merges) || map_init(&t->decomp, n_dec) || map_init(&t->compose, n_comp))
        return "out of memory";
    for (uint32_t r = 0; r < n_merges; r++) {
        const uint32_t *m = t->merges + 3 * r;
        if (m[0] >= n_vocab || m[1] >= n_vocab || m[2] >= n_vocab) return "merge with an unknown id";
        map_put(&t->pair_rank, (uint64_t)m[0] << 32 | m[1], r);
    }
    for (uint32_t i = 0; i < n_dec; i++) map_put(&t->decomp, dec_cp[i], i);
    for (uint32_t i = 0; i < n_comp; i++) map_put(&t->compose, (uint64_t)comp[3 * i] << 32 | comp[3 * i + 1], comp[3 * i + 2]);
    return NULL;
}

Tokenizer *tok_load(const char *path) {
    Tokenizer *t = calloc(1, sizeof *t);
    size_t size = 0;
    const char *why = "out of memory";
    if (t) {
        t->data = read_file(path, &size);
        why = !t->data ? "cannot read the file" : size > 0xFFFFFFF0u ? "file too large" : parse(t, size);
    }
    if (!why) return t;
    fprintf(stderr, "qwen tokenizer %s: %s\n", path, why);
    tok_free(t);
    return NULL;
}
