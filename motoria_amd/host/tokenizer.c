/*
 * The tokenizer of a .mia file (its MTK1 blob) and the Qwen3 chat-turn text,
 * giving the ids the reference's tokenizer gives for the same text
 * (src/tokenizer/bpe.c of the reference; the rules are restated below).
 *
 * Structure:
 *   - the blob is read by a bounds-checked little-endian reader into one
 *     allocation of piece bytes and offsets;
 *   - merges go into an open-addressing hash table keyed by the id pair
 *     (a pair listed twice keeps its first, lowest rank);
 *   - special tokens are indexed by their first byte (listed order kept);
 *   - a plain segment (the text between two special tokens) is decoded once
 *     into an array of characters with their class, and a rule table over
 *     that array cuts it into pre-tokens;
 *   - each pre-token's byte pieces are merged with a binary heap of
 *     candidate pairs keyed by (rank, position), stale entries skipped by
 *     version numbers: every step merges the lowest-rank adjacent pair,
 *     leftmost among equal ranks.
 *
 * The encoding rules (the contract the ids depend on):
 *   1. At the cursor, the longest special token whose bytes start there is
 *      emitted whole (the first listed among equally long ones).
 *   2. Otherwise the plain text up to the next position where a special
 *      token starts is cut into pre-tokens. Character classes: ASCII letters
 *      (either case), digits, newline (\n \r), space (space \t \v \f), and
 *      every other ASCII byte punctuation; a multi-byte UTF-8 character is a
 *      letter, except those led by C2 and the E2 80 xx / E3 80 xx rows, which
 *      are punctuation; a lead byte promising more bytes than the segment
 *      holds takes what is left. At each position the first rule that
 *      applies gives the pre-token:
 *        a. an apostrophe and an English contraction suffix, any case:
 *           're 've 'll (three characters), else 's 't 'm 'd (two);
 *        b. a run of letters;
 *        c. one character that is neither newline nor digit, followed by a
 *           run of letters;
 *        d. one digit;
 *        e. a run of punctuation, optionally led by one space (byte 0x20),
 *           and the newlines right after it;
 *        f. whitespace (space and newline characters): up to and including
 *           the last newline of the run when it has one; else the whole run
 *           when it is one character long or reaches the end of the
 *           segment; else all of it but its last character (which then
 *           leads the next pre-token).
 *   3. A pre-token's bytes become their one-byte pieces (the lowest id of
 *      that byte; bytes without one are dropped), and adjacent pieces merge
 *      lowest rank first, leftmost first among equal ranks, until no listed
 *      pair remains.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mia/serve.h"

/* ---- the tokenizer ------------------------------------------------------------ */

typedef struct {
    uint64_t key; /* a << 32 | b, or EMPTY */
    uint32_t rank, result;
} merge_slot;

#define EMPTY UINT64_MAX

struct mia_bpe {
    int n_vocab;
    uint32_t *off;        /* [n_vocab + 1] piece offsets into bytes */
    unsigned char *bytes; /* every piece's bytes, in id order */
    int single[256];      /* the lowest id whose piece is that one byte, or -1 */
    merge_slot *table;    /* open addressing, `mask + 1` slots */
    uint64_t mask;
    int *sp_ids;          /* special ids grouped by first byte, listed order */
    int sp_from[257];     /* group of byte c: sp_ids[sp_from[c] .. sp_from[c + 1]) */
    int eos, im_start, im_end;
};

static uint64_t pair_key(uint32_t a, uint32_t b) { return (uint64_t)a << 32 | b; }

static uint64_t slot_of(uint64_t key, uint64_t mask) {
    uint64_t h = key * 0x9E3779B97F4A7C15ull; /* Fibonacci hashing */
    return (h ^ (h >> 29)) & mask;
}

static const merge_slot *merge_find(const mia_bpe *t, uint32_t a, uint32_t b) {
    if (!t->table) return NULL;
    const uint64_t key = pair_key(a, b);
    for (uint64_t i = slot_of(key, t->mask);; i = (i + 1) & t->mask) {
        if (t->table[i].key == key) return &t->table[i];
        if (t->table[i].key == EMPTY) return NULL;
    }
}

/* Inserts unless the pair is there already (its earlier rank stays). */
static void merge_add(mia_bpe *t, uint32_t a, uint32_t b, uint32_t rank, uint32_t result) {
    const uint64_t key = pair_key(a, b);
    for (uint64_t i = slot_of(key, t->mask);; i = (i + 1) & t->mask) {
        if (t->table[i].key == key) return;
        if (t->table[i].key == EMPTY) {
            t->table[i] = (merge_slot){key, rank, result};
            return;
        }
    }
}

/* Little-endian reads from [at, end); `ok` drops to 0 on the first read past
 * the end and stays there. */
typedef struct {
    const unsigned char *at, *end;
    int ok;
} reader;

static const unsigned char *take(reader *r, size_t n) {
    if (!r->ok || (size_t)(r->end - r->at) < n) {
        r->ok = 0;
        return NULL;
    }
    const unsigned char *p = r->at;
    r->at += n;
    return p;
}

static uint32_t take_le(reader *r, int nbytes) {
    const unsigned char *p = take(r, (size_t)nbytes);
    uint32_t v = 0;
    for (int i = nbytes - 1; p && i >= 0; i--) v = v << 8 | p[i];
    return v;
}

void mia_bpe_close(mia_bpe *t) {
    if (!t) return;
    free(t->off);
    free(t->bytes);
    free(t->table);
    free(t->sp_ids);
    free(t);
}

/* MTK1 layout: "MTK1", then u32 vocabulary size, merge count, special
 * count, end-of-text id, <|im_start|> id, <|im_end|> id; each piece as u16
 * length + bytes; each merge as u32 a, b, result (rank = its place in the
 * list); each special as a u32 id. Everything little-endian. */
int mia_bpe_open(mia_bpe **out, const unsigned char *blob, size_t n) {
    *out = NULL;
    if (!blob) return -1;
    reader r = {blob, blob + n, 1};
    const unsigned char *magic = take(&r, 4);
    if (!magic || memcmp(magic, "MTK1", 4) != 0) return -1;
    uint32_t head[6];
    for (int i = 0; i < 6; i++) head[i] = take_le(&r, 4);
    const uint32_t nv = head[0], nm = head[1], ns = head[2];
    if (!r.ok || nv == 0 || nv > (1u << 24) || nm > (1u << 24) || ns > nv) return -1;

    mia_bpe *t = calloc(1, sizeof *t);
    if (!t) return -1;
    t->n_vocab = (int)nv;
    t->eos = head[3] < nv ? (int)head[3] : -1;
    t->im_start = head[4] < nv ? (int)head[4] : -1;
    t->im_end = head[5] < nv ? (int)head[5] : -1;
    memset(t->single, 0xff, sizeof t->single);
    t->off = malloc(sizeof(uint32_t) * ((size_t)nv + 1));
    t->bytes = malloc(n); /* the pieces cannot outgrow the blob */
    if (!t->off || !t->bytes) goto fail;
    uint32_t used = 0;
    for (uint32_t id = 0; id < nv; id++) {
        const uint32_t len = take_le(&r, 2);
        const unsigned char *p = take(&r, len);
        if (!p) goto fail;
        t->off[id] = used;
        memcpy(t->bytes + used, p, len);
        used += len;
        if (len == 1 && t->single[p[0]] < 0) t->single[p[0]] = (int)id;
    }
    t->off[nv] = used;

    uint64_t cap = 16;
    while (cap < 2 * (uint64_t)nm) cap <<= 1;
    t->mask = cap - 1;
    t->table = malloc(sizeof(merge_slot) * cap);
    if (!t->table) goto fail;
    for (uint64_t i = 0; i < cap; i++) t->table[i].key = EMPTY;
    for (uint32_t rank = 0; rank < nm; rank++) {
        const uint32_t a = take_le(&r, 4), b = take_le(&r, 4), res = take_le(&r, 4);
        if (!r.ok || a >= nv || b >= nv || res >= nv) goto fail;
        merge_add(t, a, b, rank, res);
    }

    int *listed = malloc(sizeof(int) * (ns ? ns : 1));
    t->sp_ids = malloc(sizeof(int) * (ns ? ns : 1));
    if (!listed || !t->sp_ids) {
        free(listed);
        goto fail;
    }
    int count[257] = {0};
    int kept = 0;
    for (uint32_t i = 0; i < ns; i++) {
        const uint32_t id = take_le(&r, 4);
        if (!r.ok || id >= nv) {
            free(listed);
            goto fail;
        }
        if (t->off[id + 1] > t->off[id]) { /* an empty piece never matches */
            listed[kept++] = (int)id;
            count[t->bytes[t->off[id]] + 1]++;
        }
    }
    for (int c = 0; c < 256; c++) count[c + 1] += count[c];
    memcpy(t->sp_from, count, sizeof t->sp_from);
    for (int i = 0; i < kept; i++) t->sp_ids[count[t->bytes[t->off[listed[i]]]]++] = listed[i];
    free(listed);
    *out = t;
    return 0;
fail:
    mia_bpe_close(t);
    return -1;
}

int mia_bpe_vocab(const mia_bpe *t) { return t->n_vocab; }
int mia_bpe_im_start(const mia_bpe *t) { return t->im_start; }

const unsigned char *mia_bpe_piece(const mia_bpe *t, int id, int *len) {
    if (id < 0 || id >= t->n_vocab) {
        *len = 0;
        return (const unsigned char *)"";
    }
    *len = (int)(t->off[id + 1] - t->off[id]);
    return t->bytes + t->off[id];
}

int mia_bpe_is_stop(const mia_bpe *t, int id) {
    return id >= 0 && (id == t->eos || id == t->im_end);
}

/* The special token starting at s (n bytes left), by rule 1, or -1. */
static int special_at(const mia_bpe *t, const unsigned char *s, size_t n, size_t *len) {
    int best = -1;
    size_t best_len = 0;
    for (int i = t->sp_from[s[0]]; i < t->sp_from[s[0] + 1]; i++) {
        const int id = t->sp_ids[i];
        const size_t l = t->off[id + 1] - t->off[id];
        if (l > best_len && l <= n && memcmp(s, t->bytes + t->off[id], l) == 0) {
            best = id;
            best_len = l;
        }
    }
    *len = best_len;
    return best;
}

/* ---- pre-tokens (rule 2) ---------------------------------------------------------- */

enum { LET, DIG, SPC, NL, PUN };

/* Classes of the ASCII bytes. */
static unsigned char ascii_class(unsigned c) {
    if ((c | 0x20) >= 'a' && (c | 0x20) <= 'z') return LET;
    if (c >= '0' && c <= '9') return DIG;
    switch (c) {
    case '\n': case '\r': return NL;
    case ' ': case '\t': case '\v': case '\f': return SPC;
    default: return PUN;
    }
}

typedef struct {
    uint32_t at;       /* byte offset in the segment */
    unsigned char len; /* bytes */
    unsigned char cls;
} chr;

/* Decodes s[0..n) into characters; returns their count. */
static size_t decode(const unsigned char *s, size_t n, chr *out) {
    size_t k = 0;
    for (size_t i = 0; i < n; k++) {
        const unsigned c = s[i];
        size_t len = 1;
        unsigned char cls;
        if (c < 0x80) {
            cls = ascii_class(c);
        } else {
            len = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : c >= 0xC0 ? 2 : 1;
            if (len > n - i) len = n - i;
            const int punct_row = (c == 0xE2 || c == 0xE3) && n - i > 1 && s[i + 1] == 0x80;
            cls = (c == 0xC2 || punct_row) ? PUN : LET;
        }
        out[k] = (chr){(uint32_t)i, (unsigned char)len, cls};
        i += len;
    }
    return k;
}

/* First character at or after i whose class is not in `set` (a bit mask). */
static size_t skip(const chr *c, size_t m, size_t i, unsigned set) {
    while (i < m && (set >> c[i].cls & 1u)) i++;
    return i;
}

#define BIT(k) (1u << (k))

static int lower_is(const unsigned char *s, const chr *c, size_t m, size_t i, char want) {
    return i < m && c[i].len == 1 && (s[c[i].at] | 0x20) == (unsigned char)want;
}

/* Characters of the pre-token starting at character i (m in the segment). */
static size_t pretoken_chars(const unsigned char *s, const chr *c, size_t m, size_t i) {
    /* a. contractions */
    if (c[i].len == 1 && s[c[i].at] == '\'') {
        static const char three[3][2] = {{'r', 'e'}, {'v', 'e'}, {'l', 'l'}};
        for (int k = 0; k < 3; k++)
            if (lower_is(s, c, m, i + 1, three[k][0]) && lower_is(s, c, m, i + 2, three[k][1]))
                return 3;
        for (const char *two = "stmd"; *two; two++)
            if (lower_is(s, c, m, i + 1, *two)) return 2;
    }
    const unsigned cls = c[i].cls;
    /* b. letters */
    if (cls == LET) return skip(c, m, i, BIT(LET)) - i;
    /* c. one leading character, then letters */
    if (cls != NL && cls != DIG && i + 1 < m && c[i + 1].cls == LET)
        return skip(c, m, i + 1, BIT(LET)) - i;
    /* d. a digit */
    if (cls == DIG) return 1;
    /* e. punctuation, optionally led by a space byte, with its newlines */
    const size_t lead = (c[i].len == 1 && s[c[i].at] == ' ' && i + 1 < m && c[i + 1].cls == PUN);
    if (c[i + lead].cls == PUN) return skip(c, m, skip(c, m, i + lead, BIT(PUN)), BIT(NL)) - i;
    /* f. whitespace */
    const size_t end = skip(c, m, i, BIT(SPC) | BIT(NL));
    for (size_t j = end; j > i; j--)
        if (c[j - 1].cls == NL) return j - i;
    return (end == m || end - i == 1) ? end - i : end - i - 1;
}

/* ---- merges (rule 3) ---------------------------------------------------------- */

typedef struct {
    uint32_t rank;
    int left, right;     /* symbol indices */
    unsigned lver, rver; /* their versions when the entry was made */
} cand;

static int cand_before(const cand *x, const cand *y) {
    return x->rank != y->rank ? x->rank < y->rank : x->left < y->left;
}

typedef struct {
    cand *h;
    int n;
} heap;

static void heap_push(heap *q, cand v) {
    int i = q->n++;
    while (i > 0 && cand_before(&v, &q->h[(i - 1) / 2])) {
        q->h[i] = q->h[(i - 1) / 2];
        i = (i - 1) / 2;
    }
    q->h[i] = v;
}

static cand heap_pop(heap *q) {
    const cand top = q->h[0], last = q->h[--q->n];
    int i = 0;
    for (;;) {
        int kid = 2 * i + 1;
        if (kid >= q->n) break;
        if (kid + 1 < q->n && cand_before(&q->h[kid + 1], &q->h[kid])) kid++;
        if (!cand_before(&q->h[kid], &last)) break;
        q->h[i] = q->h[kid];
        i = kid;
    }
    if (q->n) q->h[i] = last;
    return top;
}

/* Work space of one encode call, sized for its longest pre-token. */
typedef struct {
    int *id, *next, *prev;
    unsigned *ver;
    cand *cands;
} symbols;

static void offer(const mia_bpe *t, const symbols *y, heap *q, int l, int r) {
    if (l < 0 || r < 0) return;
    const merge_slot *g = merge_find(t, (uint32_t)y->id[l], (uint32_t)y->id[r]);
    if (g) heap_push(q, (cand){g->rank, l, r, y->ver[l], y->ver[r]});
}

/* The ids of pre-token bytes s[0..n) appended to out; returns their count. */
static int merge_bytes(const mia_bpe *t, const unsigned char *s, size_t n, symbols *y, int *out) {
    int m = 0;
    for (size_t i = 0; i < n; i++) {
        const int id = t->single[s[i]];
        if (id < 0) continue;
        y->id[m] = id;
        y->prev[m] = m - 1;
        y->next[m] = m + 1;
        y->ver[m] = 0;
        m++;
    }
    if (m == 0) return 0;
    y->next[m - 1] = -1;
    heap q = {y->cands, 0};
    for (int i = 0; i + 1 < m; i++) offer(t, y, &q, i, i + 1);
    while (q.n) {
        const cand c = heap_pop(&q);
        const int l = c.left, r = c.right;
        if (y->ver[l] != c.lver || y->ver[r] != c.rver || y->next[l] != r) continue;
        /* r is merged into l (a merged-away symbol is never offered again:
         * its version moves on and no neighbour links to it) */
        y->id[l] = (int)merge_find(t, (uint32_t)y->id[l], (uint32_t)y->id[r])->result;
        y->ver[l]++;
        y->ver[r]++;
        y->next[l] = y->next[r];
        if (y->next[r] >= 0) y->prev[y->next[r]] = l;
        offer(t, y, &q, y->prev[l], l);
        offer(t, y, &q, l, y->next[l]);
    }
    int k = 0;
    for (int i = 0; i >= 0; i = y->next[i]) out[k++] = y->id[i];
    return k;
}

int mia_bpe_encode(const mia_bpe *t, const char *text, int *out, int max) {
    const unsigned char *s = (const unsigned char *)text;
    const size_t n = strlen(text);
    const size_t room = n ? n : 1;
    chr *chars = malloc(sizeof(chr) * room);
    int *ids = malloc(sizeof(int) * room);
    symbols y = {malloc(sizeof(int) * room), malloc(sizeof(int) * room),
                 malloc(sizeof(int) * room), malloc(sizeof(unsigned) * room),
                 /* every merge offers at most two pairs */
                 malloc(sizeof(cand) * (3 * room + 1))};
    long count = -1;
    if (chars && ids && y.id && y.next && y.prev && y.ver && y.cands) {
        count = 0;
        size_t pos = 0;
        while (pos < n && count >= 0) {
            size_t len;
            const int sp = special_at(t, s + pos, n - pos, &len);
            if (sp >= 0) {
                if (count < max) out[count++] = sp;
                else count = -1;
                pos += len;
                continue;
            }
            size_t end = pos + 1;
            while (end < n && special_at(t, s + end, n - end, &len) < 0) end++;
            const size_t m = decode(s + pos, end - pos, chars);
            for (size_t i = 0; i < m && count >= 0;) {
                const size_t k = pretoken_chars(s + pos, chars, m, i);
                const size_t b0 = chars[i].at, b1 = chars[i + k - 1].at + chars[i + k - 1].len;
                const int got = merge_bytes(t, s + pos + b0, b1 - b0, &y, ids);
                if (got > max - count) {
                    count = -1;
                } else {
                    memcpy(out + count, ids, sizeof(int) * (size_t)got);
                    count += got;
                }
                i += k;
            }
            pos = end;
        }
    }
    free(chars);
    free(ids);
    free(y.id);
    free(y.next);
    free(y.prev);
    free(y.ver);
    free(y.cands);
    return (int)count;
}

/* ---- the chat turn ------------------------------------------------------------- */

/* The Qwen3 template of one user turn (src/model/runtime.c:84-95 of the
 * reference: the model was trained on it). */
char *mia_chat_turn_text(const char *user, int think, int continuing) {
    const char *parts[] = {
        continuing ? "<|im_end|>\n" : "",
        "<|im_start|>user\n",
        user,
        "<|im_end|>\n<|im_start|>assistant\n",
        think ? "" : "<think>\n\n</think>\n\n",
    };
    size_t n = 1;
    for (size_t i = 0; i < sizeof parts / sizeof parts[0]; i++) n += strlen(parts[i]);
    char *s = malloc(n), *w = s;
    if (!s) return NULL;
    for (size_t i = 0; i < sizeof parts / sizeof parts[0]; i++) {
        const size_t l = strlen(parts[i]);
        memcpy(w, parts[i], l);
        w += l;
    }
    *w = '\0';
    return s;
}
