/*
 * .mia model files (the reference's on-disk format) into the HBM expert
 * table of a mia_moe handle.
 *
 * mia_file_probe reads and checks the 112-byte header (the reference's
 * mia_header, include/mia/mia_file.h:10-21, with the checks of
 * src/storage/mia_file.c:49-61), walks the dense section in the order the
 * converter lays it out (NewLayout, tools/internal/mia/format.go:129-165;
 * the reader's walk, src/storage/mia_file.c:73-97) and checks that the walk
 * ends at dense_size, that the expert blob holds gate/up/down at the
 * reference's offsets (src/storage/mia_file.c:98-106) and that the file is
 * long enough for every blob. mia_moe_load_file then uploads each layer's
 * ffn_norm and router and every (layer, expert) blob, read at
 * experts_offset + (layer * n_experts + expert) * expert_blob_size
 * (src/storage/mia_file.c:121-126), through pinned staging in batches.
 */
#define _FILE_OFFSET_BITS 64
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include "moe_internal.h"

enum { HEADER_BYTES = 112, TENSOR_ALIGN = 64, BATCH = 8 };

static uint64_t align_up64(uint64_t n, uint64_t a) { return (n + a - 1) / a * a; }

static uint32_t le32(const unsigned char *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static uint64_t le64(const unsigned char *p) { return le32(p) | (uint64_t)le32(p + 4) << 32; }
static float lef32(const unsigned char *p) {
    const uint32_t u = le32(p);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static int perr(char *err, size_t errlen, const char *fmt, ...) {
    if (err && errlen) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, errlen, fmt, ap);
        va_end(ap);
    }
    return -1;
}

static int pread_all(int fd, void *dst, size_t n, uint64_t off) {
    unsigned char *p = dst;
    while (n > 0) {
        const size_t want = n < ((size_t)64 << 20) ? n : ((size_t)64 << 20);
        const ssize_t got = pread(fd, p, want, (off_t)off);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return -1;
        p += got;
        n -= (size_t)got;
        off += (uint64_t)got;
    }
    return 0;
}

/* Bytes of a rows x cols tensor in the dense section: matrices in the
 * file's weight type (36-byte Q8_0 blocks or fp32), vectors and routers
 * fp32 (tools/internal/mia/format.go:104-110,131-142). */
static uint64_t tensor_bytes(uint32_t wtype, uint64_t rows, uint64_t cols, int quantized) {
    if (quantized && wtype == MIA_Q8_0) return rows * (cols / MIA_QK) * 36;
    return rows * cols * 4;
}

uint64_t mia_dense_walk(const mia_file_info *h, int want_layer, mia_layer_offsets *lo,
                        uint64_t *token_embd, uint64_t *output_norm, uint64_t *output) {
    const uint64_t d = h->dim, hd = h->head_dim, V = h->vocab;
    const uint64_t qd = (uint64_t)h->n_heads * hd, kvd = (uint64_t)h->n_kv_heads * hd;
    uint64_t off = 0;
    /* records the cursor in *dst, then steps over one tensor (64-byte aligned) */
#define TAKE(dst, rows, cols, q)                                                              \
    do {                                                                                      \
        if (dst) *(dst) = off;                                                                \
        off = align_up64(off + tensor_bytes(h->wtype, rows, cols, q), TENSOR_ALIGN);          \
    } while (0)
    TAKE(token_embd, V, d, 1);
    for (uint32_t l = 0; l < h->n_layers; l++) {
        mia_layer_offsets *L = lo && (int)l == want_layer ? lo : NULL;
        TAKE(L ? &L->attn_norm : NULL, 1, d, 0);
        TAKE(L ? &L->wq : NULL, qd, d, 1);
        TAKE(L ? &L->wk : NULL, kvd, d, 1);
        TAKE(L ? &L->wv : NULL, kvd, d, 1);
        TAKE(L ? &L->wo : NULL, d, qd, 1);
        TAKE(L ? &L->q_norm : NULL, 1, hd, 0);
        TAKE(L ? &L->k_norm : NULL, 1, hd, 0);
        TAKE(L ? &L->ffn_norm : NULL, 1, d, 0);
        TAKE(L ? &L->router : NULL, h->n_experts, d, 0);
    }
    TAKE(output_norm, 1, d, 0);
    TAKE(output, V, d, 1);
#undef TAKE
    return off;
}

int mia_file_probe(const char *path, mia_file_info *h, char *err, size_t errlen) {
    memset(h, 0, sizeof(*h));
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return perr(err, errlen, "open %s: %s", path, strerror(errno));
    unsigned char b[HEADER_BYTES];
    struct stat st;
    int rc = 0;
    if (pread_all(fd, b, sizeof b, 0) != 0 || memcmp(b, "MIA1", 4) != 0 || le32(b + 4) != 1)
        rc = perr(err, errlen, "%s: not a MIA v1 file", path);
    else if (fstat(fd, &st) != 0)
        rc = perr(err, errlen, "stat %s: %s", path, strerror(errno));
    close(fd);
    if (rc) return rc;
    h->version = le32(b + 4);
    h->wtype = le32(b + 8);
    h->dim = le32(b + 12);
    h->n_layers = le32(b + 16);
    h->n_heads = le32(b + 20);
    h->n_kv_heads = le32(b + 24);
    h->head_dim = le32(b + 28);
    h->vocab = le32(b + 32);
    h->n_experts = le32(b + 36);
    h->n_active = le32(b + 40);
    h->expert_hidden = le32(b + 44);
    h->norm_topk = le32(b + 48);
    h->rope_theta = lef32(b + 52);
    h->norm_eps = lef32(b + 56);
    h->dense_offset = le64(b + 64);
    h->dense_size = le64(b + 72);
    h->experts_offset = le64(b + 80);
    h->expert_blob_size = le64(b + 88);
    h->tok_offset = le64(b + 96);
    h->tok_size = le64(b + 104);
    /* the reference reader's shape checks (src/storage/mia_file.c:53-61) */
    if (h->wtype > MIA_Q8_0 || h->n_kv_heads == 0 || h->n_heads % h->n_kv_heads != 0 ||
        h->n_active > h->n_experts || h->head_dim % 2 != 0 || h->dim % MIA_QK != 0 ||
        h->expert_hidden % MIA_QK != 0 || (h->n_heads * h->head_dim) % MIA_QK != 0)
        return perr(err, errlen, "%s: unsupported model shape", path);
    if (h->dim == 0 || h->n_layers == 0 || h->n_experts == 0 || h->n_active == 0 ||
        h->expert_hidden == 0)
        return perr(err, errlen, "%s: empty MoE shape", path);
    const uint64_t end = mia_dense_walk(h, -1, NULL, NULL, NULL, NULL);
    if (end != h->dense_size)
        return perr(err, errlen, "%s: dense layout mismatch (%llu vs %llu)", path,
                    (unsigned long long)end, (unsigned long long)h->dense_size);
    /* blob geometry (src/storage/mia_file.c:98-106) */
    const uint64_t mat = tensor_bytes(h->wtype, h->expert_hidden, h->dim, 1);
    h->off_up = align_up64(mat, TENSOR_ALIGN);
    h->off_down = h->off_up + align_up64(mat, TENSOR_ALIGN);
    if (h->off_down + tensor_bytes(h->wtype, h->dim, h->expert_hidden, 1) > h->expert_blob_size)
        return perr(err, errlen, "%s: expert blob too small", path);
    const uint64_t fsize = (uint64_t)st.st_size;
    const uint64_t experts_end =
        h->experts_offset + (uint64_t)h->n_layers * h->n_experts * h->expert_blob_size;
    if (h->dense_offset + h->dense_size > fsize || experts_end > fsize ||
        h->dense_offset + h->dense_size > h->experts_offset ||
        (h->tok_size && h->tok_offset + h->tok_size > fsize))
        return perr(err, errlen, "%s: truncated (%llu bytes, experts end at %llu)", path,
                    (unsigned long long)fsize, (unsigned long long)experts_end);
    return 0;
}

int mia_file_layer_offsets(const mia_file_info *h, int layer, uint64_t *ffn_norm,
                           uint64_t *router) {
    if (layer < 0 || (uint32_t)layer >= h->n_layers) return -1;
    mia_layer_offsets lo;
    mia_dense_walk(h, layer, &lo, NULL, NULL, NULL);
    *ffn_norm = h->dense_offset + lo.ffn_norm;
    *router = h->dense_offset + lo.router;
    return 0;
}

/* Reads the blobs of (l, e0 .. e0+n) into pinned host memory and queues
 * their upload and repack; `d_stage` is device staging for n blobs. */
/* The stream marks (include/mia_hip.h) mia_moe_load_file records after
 * each of its two staging buffers' batches. */
#define LOAD_MARK 14

static int stage_batch(mia_moe *m, int fd, const mia_file_info *h, int l, int e0, int n,
                       unsigned char *h_stage, void *d_stage) {
    mhip_ctx *g = mia_moe_gpu(m);
    const uint64_t blob = h->expert_blob_size;
    const uint64_t first = h->experts_offset + ((uint64_t)l * h->n_experts + e0) * blob;
    if (pread_all(fd, h_stage, (size_t)(blob * n), first) != 0) return -2;
    int experts[BATCH];
    for (int i = 0; i < n; i++) experts[i] = e0 + i;
    mhip_dims s = {(int)h->dim, (int)h->n_experts, (int)h->n_active, (int)h->expert_hidden,
                   (int)h->norm_topk, h->norm_eps};
    if (mhip_h2d_async(g, d_stage, h_stage, (size_t)(blob * n)) ||
        mhip_table_repack(g, &s, mia_moe_table(m), l, experts, n, d_stage, (size_t)blob,
                          (size_t)h->off_up, (size_t)h->off_down))
        return -1;
    return 0;
}

int mia_moe_load_file(mia_moe *m, const char *path) {
    char err[256];
    mia_file_info h;
    if (mia_file_probe(path, &h, err, sizeof err)) return mia_moe_fail(m, "%s", err);
    const mia_moe_config *c = mia_moe_cfg(m);
    if (h.wtype != MIA_Q8_0)
        return mia_moe_fail(m, "%s: weight type %u: the HBM table holds Q8_0 experts", path,
                            h.wtype);
    if ((int)h.dim != c->dim || (int)h.n_layers != c->n_layers ||
        (int)h.n_experts != c->n_experts || (int)h.n_active != c->n_active ||
        (int)h.expert_hidden != c->expert_hidden || (int)h.norm_topk != c->norm_topk ||
        h.norm_eps != c->norm_eps)
        return mia_moe_fail(m, "%s: shape %u/%u/%u/%u/%u (topk %u, eps %g) differs from the "
                               "handle's %d/%d/%d/%d/%d (topk %d, eps %g)",
                            path, h.dim, h.n_layers, h.n_experts, h.n_active, h.expert_hidden,
                            h.norm_topk, (double)h.norm_eps, c->dim, c->n_layers, c->n_experts,
                            c->n_active, c->expert_hidden, c->norm_topk, (double)c->norm_eps);
    if (h.expert_blob_size != mia_moe_blob_bytes(m) || h.off_up != mia_moe_off_up(m) ||
        h.off_down != mia_moe_off_down(m))
        return mia_moe_fail(m, "%s: expert blob geometry differs from the table's", path);
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return mia_moe_fail(m, "open %s: %s", path, strerror(errno));
    mhip_ctx *g = mia_moe_gpu(m);
    const size_t d = h.dim, E = h.n_experts, blob = (size_t)h.expert_blob_size;
    const int nb = (int)(E < BATCH ? E : BATCH);
    float *norm = malloc(d * 4), *router = malloc(d * E * 4);
    unsigned char *hs[2] = {mhip_host_malloc(g, blob * nb), mhip_host_malloc(g, blob * nb)};
    void *ds[2] = {mhip_malloc(g, blob * nb), mhip_malloc(g, blob * nb)};
    int rc = 0;
    if (!norm || !router || !hs[0] || !hs[1] || !ds[0] || !ds[1])
        rc = mia_moe_fail(m, "%s: staging buffers: %s", path, mhip_error(g));
    for (uint32_t l = 0; !rc && l < h.n_layers; l++) {
        uint64_t fn, rt;
        mia_file_layer_offsets(&h, (int)l, &fn, &rt);
        if (pread_all(fd, norm, d * 4, fn) || pread_all(fd, router, d * E * 4, rt))
            rc = mia_moe_fail(m, "%s: reading layer %u norm/router", path, l);
        else if (mia_moe_set_layer(m, (int)l, norm, router))
            rc = -1;
    }
    /* experts: two pinned batches, so batch k is read from the file while
     * batch k - 1 uploads and is repacked. Buffer k & 1 is reused only once
     * the stream has passed batch k - 2's repack (stream mark LOAD_MARK +
     * (k & 1), recorded after it), not the whole stream. */
    int k = 0;
    for (uint32_t l = 0; !rc && l < h.n_layers; l++)
        for (int e0 = 0; !rc && e0 < (int)E; e0 += nb, k++) {
            const int n = (int)E - e0 < nb ? (int)E - e0 : nb;
            if (k >= 2 && mhip_mark_wait(g, LOAD_MARK + (k & 1))) {
                rc = mia_moe_fail(m, "%s", mhip_error(g));
                break;
            }
            const int r = stage_batch(m, fd, &h, (int)l, e0, n, hs[k & 1], ds[k & 1]);
            if (r == -2)
                rc = mia_moe_fail(m, "%s: reading experts %d..%d of layer %u", path, e0,
                                  e0 + n - 1, l);
            else if (r || mhip_mark(g, LOAD_MARK + (k & 1)))
                rc = mia_moe_fail(m, "%s", mhip_error(g));
        }
    if (mhip_sync(g) && !rc) rc = mia_moe_fail(m, "%s", mhip_error(g));
    close(fd);
    free(norm);
    free(router);
    for (int i = 0; i < 2; i++) {
        if (hs[i]) mhip_host_free(g, hs[i]);
        if (ds[i]) mhip_free(g, ds[i]);
    }
    return rc;
}
