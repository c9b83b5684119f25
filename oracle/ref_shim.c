/*
 * Harness that reaches the reference's own MoE layer, in the manner of the
 * reference's mia-dump harness (src/app/dump.c:11-54).
 *
 * TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile (target `ref`) from the
 * reference sources where they lie; the output goes to oracle/_ref/ and is
 * never committed. It validates the C restatement (mia_oracle.c) and writes
 * the golden vectors under tests/golden/.
 *
 * moe() is static in src/model/forward.c:167, so this file includes that
 * translation unit and calls it on a mia_model built around in-memory
 * expert blobs, which the reference's own LRU cache (expert_cache.c) fetches
 * through the mia_expert_loader port (include/mia/expert_cache.h:8).
 */
#include "src/model/forward.c"

#include <string.h>

typedef struct {
    const unsigned char *const *blobs;
    size_t blob_size;
    int order[64];
    int n_loaded;
} table_loader;

/* Records the order in which moe() asks for experts (= its idx[j] order on a
 * fresh cache, since one token's K experts are distinct). */
static int table_load(void *ctx, int layer, int expert, void *dst) {
    table_loader *t = ctx;
    (void)layer;
    if (!t->blobs[expert]) return -1;
    memcpy(dst, t->blobs[expert], t->blob_size);
    if (t->n_loaded < 64) t->order[t->n_loaded] = expert;
    t->n_loaded++;
    return 0;
}

/*
 * Runs the reference moe() for T tokens (one mia_model per token, fresh
 * cache each time) in place on x[T][dim]. Also returns, per token, the expert
 * order moe() loaded (idx_loaded[T][K]) and the routing prologue recomputed
 * with the reference's own static helpers: xn, logits, idx, w. Returns 0 or
 * the failing rc.
 */
int ref_moe_layer(int dim, int n_experts, int n_active, int expert_hidden,
                  int norm_topk, float norm_eps, int T, float *x,
                  const float *ffn_norm, const float *router,
                  const unsigned char *const *blobs, size_t blob_size,
                  int *idx_loaded, int *idx, float *w, float *logits,
                  float *xn_out) {
    mia_file f;
    memset(&f, 0, sizeof(f));
    f.h.dim = (uint32_t)dim;
    f.h.n_layers = 1;
    f.h.n_heads = 1;
    f.h.n_kv_heads = 1;
    f.h.head_dim = 32;
    f.h.vocab = 1;
    f.h.n_experts = (uint32_t)n_experts;
    f.h.n_active = (uint32_t)n_active;
    f.h.expert_hidden = (uint32_t)expert_hidden;
    f.h.norm_topk = (uint32_t)norm_topk;
    f.h.norm_eps = norm_eps;
    f.h.expert_blob_size = blob_size;
    f.wt = MIA_Q8_0;
    mia_layer layer;
    memset(&layer, 0, sizeof(layer));
    layer.ffn_norm = ffn_norm;
    layer.router = router;
    f.layers = &layer;
    /* src/storage/mia_file.c:98-101 */
    size_t mat = (size_t)expert_hidden * mia_row_bytes(MIA_Q8_0, dim);
    f.off_up = (mat + 63) / 64 * 64;
    f.off_down = 2 * f.off_up;

    dims s = dims_of(&f.h);
    for (int t = 0; t < T; t++) {
        table_loader tl;
        memset(&tl, 0, sizeof(tl));
        tl.blobs = blobs;
        tl.blob_size = blob_size;
        mia_expert_cache cache;
        mia_model m;
        if (mia_cache_init(&cache, 1, n_experts, blob_size, n_experts, table_load, &tl))
            return -2;
        if (mia_model_init(&m, &f, &cache, 1)) {
            mia_cache_free(&cache);
            return -3;
        }
        float *xt = x + (size_t)t * dim;
        memcpy(m.x, xt, sizeof(float) * (size_t)dim);

        /* Routing prologue with the reference's helpers, in moe()'s order
         * (src/model/forward.c:174-181), to expose its intermediates. */
        rmsnorm(m.xn, m.x, layer.ffn_norm, s.d, f.h.norm_eps);
        if (xn_out) memcpy(xn_out + (size_t)t * dim, m.xn, sizeof(float) * (size_t)dim);
        mia_matvec(m.router, layer.router, MIA_F32, m.xn, NULL, s.E, s.d);
        if (logits) memcpy(logits + (size_t)t * s.E, m.router, sizeof(float) * (size_t)s.E);
        softmax(m.router, s.E);
        int id[64];
        top_k(m.router, s.E, s.K, id);
        float sum = 0, wj[64];
        for (int j = 0; j < s.K; j++) sum += wj[j] = m.router[id[j]];
        if (f.h.norm_topk)
            for (int j = 0; j < s.K; j++) wj[j] /= sum;
        if (idx) memcpy(idx + (size_t)t * s.K, id, sizeof(int) * (size_t)s.K);
        if (w) memcpy(w + (size_t)t * s.K, wj, sizeof(float) * (size_t)s.K);

        int rc = moe(&m, s, 0);
        if (idx_loaded)
            for (int j = 0; j < s.K; j++)
                idx_loaded[(size_t)t * s.K + j] = j < tl.n_loaded ? tl.order[j] : -1;
        memcpy(xt, m.x, sizeof(float) * (size_t)dim);
        mia_model_free(&m);
        mia_cache_free(&cache);
        if (rc) return rc;
    }
    return 0;
}

/*
 * The reference's whole-model step on a .mia file, in the manner of
 * src/app/dump.c: mia_file_open (src/storage/mia_file.c), an expert cache of
 * n_slots slots over mia_file_read_expert, mia_model_init and
 * mia_model_step (src/model/forward.c:199-217) for tokens[0..n) at positions
 * 0..n-1. logits[n][vocab]. Returns 0, or the failing step's position + 1
 * (or a negative code when opening failed; err receives the reason).
 */
int ref_model_logits(const char *path, int max_seq, int n_slots, int n, const int *tokens,
                     float *logits, char *err, size_t errlen) {
    mia_file f;
    if (mia_file_open(&f, path, err, errlen) != 0) return -1;
    mia_expert_cache cache;
    if (mia_cache_init(&cache, (int)f.h.n_layers, (int)f.h.n_experts, f.h.expert_blob_size,
                       n_slots, mia_file_read_expert, &f) != 0) {
        mia_file_close(&f);
        return -2;
    }
    mia_model m;
    if (mia_model_init(&m, &f, &cache, max_seq) != 0) {
        mia_cache_free(&cache);
        mia_file_close(&f);
        return -3;
    }
    int rc = 0;
    for (int p = 0; p < n; p++) {
        const float *lg = mia_model_step(&m, tokens[p], p);
        if (!lg) {
            rc = p + 1;
            break;
        }
        memcpy(logits + (size_t)p * f.h.vocab, lg, sizeof(float) * f.h.vocab);
    }
    mia_model_free(&m);
    mia_cache_free(&cache);
    mia_file_close(&f);
    return rc;
}

/*
 * The reference's own sampler (src/tokenizer/sampler.c): `draws` calls of
 * mia_sample on fresh copies of logits[n] (it overwrites them) with one
 * sampler state, the picked tokens into out[draws].
 */
#include "mia/sampler.h"

int ref_sample(const float *logits, int n, float temperature, float top_p, uint64_t seed,
               int draws, int *out) {
    mia_sampler s;
    if (mia_sampler_init(&s, temperature, top_p, n, seed) != 0) return -1;
    float *work = malloc(sizeof(float) * (size_t)n);
    if (!work) {
        mia_sampler_free(&s);
        return -1;
    }
    for (int d = 0; d < draws; d++) {
        memcpy(work, logits, sizeof(float) * (size_t)n);
        out[d] = mia_sample(&s, work);
    }
    free(work);
    mia_sampler_free(&s);
    return 0;
}

/*
 * The reference's own tokenizer (src/tokenizer/bpe.c) and chat template
 * (src/model/runtime.c:84-95): ids of `text` under the MTK1 blob, or -1
 * (load failure: -2).
 */
#include "mia/tokenizer.h"

int ref_tok_encode(const unsigned char *blob, size_t n, const char *text, int *out, int max) {
    mia_tokenizer t;
    if (mia_tok_load(&t, blob, n) != 0) return -2;
    const int r = mia_tok_encode(&t, text, out, max);
    mia_tok_free(&t);
    return r;
}

