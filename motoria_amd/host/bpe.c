/*
 * The byte-level BPE tokenizer of a .mia file (MTK1 blob) and the Qwen3
 * chat-turn text: the ids of src/tokenizer/bpe.c of the reference for the
 * same text, and the text of src/model/runtime.c:84-95.
 *
 * Encoding: the longest special token at the cursor is emitted whole
 * (bpe.c:232-243, the first listed among equally long ones); the text up
 * to the next special is cut into pre-tokens by the reference's
 * approximation of the Qwen2 pattern (bpe.c:118-187); each pre-token's
 * bytes become their single-byte pieces (bytes without one are dropped) and
 * adjacent pairs merge lowest rank first, leftmost among equal ranks
 * (bpe.c:206-230). Merges are kept sorted by pair for binary search.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdlib.h>
#include <string.h>

#include "mia/serve.h"

typedef struct {
    uint64_t pair; /* a << 32 | b */
    uint32_t rank, result;
} bpe_merge;

struct mia_bpe {
    int n_vocab;
    uint32_t *start; /* [n_vocab + 1]: piece i is bytes[start[i] .. start[i+1]) */
    unsigned char *bytes;
    int byte_piece[256]; /* the first one-byte piece of each byte, or -1 */
    bpe_merge *merge;    /* one entry per pair (its lowest rank), sorted by pair */
    size_t n_merge;
    int *special;
    int n_special;
    int eos, im_start, im_end;
};

typedef struct {
    const unsigned char *p;
    size_t n, at;
    int short_read;
} cursor;

static uint32_t take_u32(cursor *c) {
    if (c->n - c->at < 4) {
        c->short_read = 1;
        return 0;
    }
    const unsigned char *q = c->p + c->at;
    c->at += 4;
    return (uint32_t)q[0] | (uint32_t)q[1] << 8 | (uint32_t)q[2] << 16 | (uint32_t)q[3] << 24;
}

static uint32_t take_u16(cursor *c) {
    if (c->n - c->at < 2) {
        c->short_read = 1;
        return 0;
    }
    const unsigned char *q = c->p + c->at;
    c->at += 2;
    return (uint32_t)q[0] | (uint32_t)q[1] << 8;
}

static int by_pair_then_rank(const void *x, const void *y) {
    const bpe_merge *a = x, *b = y;
    if (a->pair != b->pair) return a->pair < b->pair ? -1 : 1;
    return (a->rank > b->rank) - (a->rank < b->rank);
}

void mia_bpe_close(mia_bpe *t) {
    if (!t) return;
    free(t->start);
    free(t->bytes);
    free(t->merge);
    free(t->special);
    free(t);
}

int mia_bpe_open(mia_bpe **out, const unsigned char *blob, size_t n) {
    *out = NULL;
    if (!blob || n < 28 || memcmp(blob, "MTK1", 4) != 0) return -1;
    cursor c = {blob, n, 4, 0};
    const uint32_t nv = take_u32(&c), nm = take_u32(&c), ns = take_u32(&c);
    const uint32_t eos = take_u32(&c), ims = take_u32(&c), ime = take_u32(&c);
    if (nv == 0 || nv > (1u << 24) || nm > (1u << 24) || ns > nv) return -1;
    mia_bpe *t = calloc(1, sizeof(*t));
    if (!t) return -1;
    t->n_vocab = (int)nv;
    t->eos = eos < nv ? (int)eos : -1;
    t->im_start = ims < nv ? (int)ims : -1;
    t->im_end = ime < nv ? (int)ime : -1;
    t->start = malloc(sizeof(uint32_t) * ((size_t)nv + 1));
    t->bytes = malloc(n); /* the pieces are part of the blob */
    t->merge = malloc(sizeof(bpe_merge) * (nm ? nm : 1));
    t->special = malloc(sizeof(int) * (ns ? ns : 1));
    if (!t->start || !t->bytes || !t->merge || !t->special) goto bad;
    for (int b = 0; b < 256; b++) t->byte_piece[b] = -1;
    uint32_t used = 0;
    for (uint32_t i = 0; i < nv; i++) {
        const uint32_t len = take_u16(&c);
        if (c.short_read || n - c.at < len) goto bad;
        memcpy(t->bytes + used, blob + c.at, len);
        c.at += len;
        t->start[i] = used;
        if (len == 1 && t->byte_piece[t->bytes[used]] < 0) t->byte_piece[t->bytes[used]] = (int)i;
        used += len;
    }
    t->start[nv] = used;
    for (uint32_t r = 0; r < nm; r++) {
        const uint32_t a = take_u32(&c), b = take_u32(&c), res = take_u32(&c);
        if (c.short_read || a >= nv || b >= nv || res >= nv) goto bad;
        t->merge[r] = (bpe_merge){(uint64_t)a << 32 | b, r, res};
    }
    /* a pair listed twice keeps its first (lowest) rank */
    qsort(t->merge, nm, sizeof(bpe_merge), by_pair_then_rank);
    size_t k = 0;
    for (size_t i = 0; i < nm; i++)
        if (k == 0 || t->merge[k - 1].pair != t->merge[i].pair) t->merge[k++] = t->merge[i];
    t->n_merge = k;
    for (uint32_t i = 0; i < ns; i++) {
        const uint32_t id = take_u32(&c);
        if (c.short_read || id >= nv) goto bad;
        t->special[i] = (int)id;
    }
    t->n_special = (int)ns;
    *out = t;
    return 0;
bad:
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
    *len = (int)(t->start[id + 1] - t->start[id]);
    return t->bytes + t->start[id];
}

int mia_bpe_is_stop(const mia_bpe *t, int id) {
    return id >= 0 && (id == t->eos || id == t->im_end);
}

/* ---- pre-tokens ------------------------------------------------------------ */

enum { K_LETTER, K_DIGIT, K_SPACE, K_NEWLINE, K_PUNCT };

/* Class of the character at s (n > 0 bytes left) and its byte length. ASCII
 * by the obvious tests; a multi-byte UTF-8 character is a letter, except
 * U+0080..U+00BF (lead byte C2) and the U+2000 / U+3000 punctuation rows
 * (E2 80 .., E3 80 ..). A lead byte promising more bytes than remain is cut
 * to what remains. */
static int klass(const unsigned char *s, size_t n, size_t *len) {
    const unsigned c = s[0];
    if (c < 0x80) {
        *len = 1;
        const unsigned low = c | 0x20;
        if (low >= 'a' && low <= 'z') return K_LETTER;
        if (c >= '0' && c <= '9') return K_DIGIT;
        if (c == '\n' || c == '\r') return K_NEWLINE;
        if (c == ' ' || c == '\t' || c == '\v' || c == '\f') return K_SPACE;
        return K_PUNCT;
    }
    const size_t want = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : c >= 0xC0 ? 2 : 1;
    *len = want < n ? want : n;
    if (c == 0xC2) return K_PUNCT;
    if ((c == 0xE2 || c == 0xE3) && n > 1 && s[1] == 0x80) return K_PUNCT;
    return K_LETTER;
}

/* End of the run of characters of class k1 or k2 starting at byte i. */
static size_t run_end(const unsigned char *s, size_t n, size_t i, int k1, int k2) {
    while (i < n) {
        size_t l;
        const int k = klass(s + i, n - i, &l);
        if (k != k1 && k != k2) break;
        i += l;
    }
    return i;
}

/* Byte length of the pre-token at s (n > 0). In order: an English
 * contraction ('s 't 'm 'd 're 've 'll, any case); a run of letters,
 * optionally led by one character that is neither a newline nor a digit;
 * one digit; a run of punctuation, optionally led by one space, with the
 * newlines after it; otherwise whitespace: up to the last newline of the
 * run, else the whole run when it ends the text or is one character, else
 * all but its last space (which then leads the next word). */
static size_t pretoken(const unsigned char *s, size_t n) {
    if (s[0] == '\'' && n >= 2) {
        const unsigned a = s[1] | 0x20, b = n >= 3 ? (s[2] | 0x20) : 0;
        if (n >= 3 && ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')))
            return 3;
        if (a == 's' || a == 't' || a == 'm' || a == 'd') return 2;
    }
    size_t l0, l1;
    const int k0 = klass(s, n, &l0);
    if (k0 == K_LETTER) return run_end(s, n, 0, K_LETTER, K_LETTER);
    if (k0 != K_NEWLINE && k0 != K_DIGIT && l0 < n && klass(s + l0, n - l0, &l1) == K_LETTER)
        return run_end(s, n, l0, K_LETTER, K_LETTER);
    if (k0 == K_DIGIT) return l0;
    const size_t lead = (s[0] == ' ' && n > 1 && klass(s + 1, n - 1, &l1) == K_PUNCT) ? 1 : 0;
    if (klass(s + lead, n - lead, &l1) == K_PUNCT)
        return run_end(s, n, run_end(s, n, lead, K_PUNCT, K_PUNCT), K_NEWLINE, K_NEWLINE);
    const size_t end = run_end(s, n, 0, K_SPACE, K_NEWLINE);
    size_t after_nl = 0;
    for (size_t i = 0; i < end; i++)
        if (s[i] == '\n' || s[i] == '\r') after_nl = i + 1;
    if (after_nl) return after_nl;
    return (end == n || end == 1) ? end : end - 1;
}

/* ---- merges ------------------------------------------------------------------ */

static const bpe_merge *find_merge(const mia_bpe *t, int a, int b) {
    const uint64_t key = (uint64_t)(uint32_t)a << 32 | (uint32_t)b;
    size_t lo = 0, hi = t->n_merge;
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        if (t->merge[mid].pair < key)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo < t->n_merge && t->merge[lo].pair == key ? &t->merge[lo] : NULL;
}

/* The ids of one pre-token s[0..n) into ids (room for n); returns the count. */
static int merge_pretoken(const mia_bpe *t, const unsigned char *s, size_t n, int *ids) {
    int m = 0;
    for (size_t i = 0; i < n; i++)
        if (t->byte_piece[s[i]] >= 0) ids[m++] = t->byte_piece[s[i]];
    for (;;) {
        int at = -1;
        uint32_t best_rank = 0, best_result = 0;
        for (int i = 0; i + 1 < m; i++) {
            const bpe_merge *g = find_merge(t, ids[i], ids[i + 1]);
            if (g && (at < 0 || g->rank < best_rank)) {
                at = i;
                best_rank = g->rank;
                best_result = g->result;
            }
        }
        if (at < 0) return m;
        ids[at] = (int)best_result;
        for (int i = at + 1; i + 1 < m; i++) ids[i] = ids[i + 1];
        m--;
    }
}

/* The longest special token that s[0..n) starts with (the first listed
 * among equally long ones), or -1; its length in *len. */
static int special_here(const mia_bpe *t, const unsigned char *s, size_t n, size_t *len) {
    int id = -1;
    *len = 0;
    for (int i = 0; i < t->n_special; i++) {
        const int sp = t->special[i];
        const size_t l = t->start[sp + 1] - t->start[sp];
        if (l > *len && l <= n && memcmp(s, t->bytes + t->start[sp], l) == 0) {
            id = sp;
            *len = l;
        }
    }
    return id;
}

int mia_bpe_encode(const mia_bpe *t, const char *text, int *out, int max) {
    const unsigned char *s = (const unsigned char *)text;
    const size_t n = strlen(text);
    int *ids = malloc(sizeof(int) * (n ? n : 1));
    if (!ids) return -1;
    int count = 0, rc = 0;
    size_t pos = 0;
    while (pos < n && rc == 0) {
        size_t sl;
        const int sp = special_here(t, s + pos, n - pos, &sl);
        if (sp >= 0) {
            if (count >= max) {
                rc = -1;
                break;
            }
            out[count++] = sp;
            pos += sl;
            continue;
        }
        size_t end = pos + 1; /* the plain text runs to the next special */
        while (end < n && special_here(t, s + end, n - end, &sl) < 0) end++;
        while (pos < end) {
            const size_t pl = pretoken(s + pos, end - pos);
            const int m = merge_pretoken(t, s + pos, pl, ids);
            if (m > max - count) {
                rc = -1;
                break;
            }
            memcpy(out + count, ids, sizeof(int) * (size_t)m);
            count += m;
            pos += pl;
        }
    }
    free(ids);
    return rc ? -1 : count;
}

/* ---- chat turn -------------------------------------------------------------- */

char *mia_chat_turn_text(const char *user, int think, int continuing) {
    static const char close_prev[] = "<|im_end|>\n";
    static const char open_user[] = "<|im_start|>user\n";
    static const char open_reply[] = "<|im_end|>\n<|im_start|>assistant\n";
    static const char no_think[] = "<think>\n\n</think>\n\n";
    const size_t n = (continuing ? strlen(close_prev) : 0) + strlen(open_user) + strlen(user) +
                     strlen(open_reply) + (think ? 0 : strlen(no_think)) + 1;
    char *s = malloc(n);
    if (!s) return NULL;
    s[0] = '\0';
    if (continuing) strcat(s, close_prev);
    strcat(s, open_user);
    strcat(s, user);
    strcat(s, open_reply);
    if (!think) strcat(s, no_think);
    return s;
}
