/*
 * C99 host side of the MoE FFN path: the public entry points of
 * include/mia/moe.h over the thin HIP C ABI (include/mia_hip.h).
 */
#include "mia/moe.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "moe_internal.h"

struct mia_moe {
    mia_moe_config cfg; /* as opened */
    mhip_ctx *gpu;
    mhip_dims dims;
    mhip_layout lay;
    int n_layers, max_tokens, flags;
    size_t blob_bytes, off_up, off_down;
    void *d_table;      /* [L][E] experts, lay.expert_bytes apart */
    float *d_router_t;  /* [L][dim][E] */
    float *d_router_dl; /* [L][E][dim], decode layout (mhip_router_decode_layout) */
    void *d_dws;        /* persistent decode workspace */
    int *d_didx;        /* [L][K] routing of the last decode-stack call */
    float *h_stage;     /* pinned: x in [dim], x out [dim], idx [K], w [K] of one-token calls */
    float *d_dw;        /* [L][K] */
    float *d_norm;      /* [L][dim] */
    float *d_router;    /* [E][dim] upload staging */
    void *d_scratch;
    mhip_scratch sc;
    float *d_x;         /* [max_tokens][dim] staging of host-pointer calls */
    float *d_bias;      /* [E] */
    void *d_blob;       /* one .mia blob */
    unsigned char *h_blob;
    mhip_graph *graph; /* mia_moe_stack_graph's recording ... */
    int g_l0, g_l1, g_T, g_flags;
    float *g_x;         /* ... and the arguments it was recorded with */
    char err[512];
};

static int fail(mia_moe *m, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(m->err, sizeof(m->err), fmt, ap);
    va_end(ap);
    return -1;
}

static int gpu_fail(mia_moe *m) { return fail(m, "%s", mhip_error(m->gpu)); }

int mia_moe_fail(mia_moe *m, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(m->err, sizeof(m->err), fmt, ap);
    va_end(ap);
    return -1;
}
void *mia_moe_table(mia_moe *m) { return m->d_table; }
void mia_moe_get_tensors(const mia_moe *m, mia_moe_tensors *t) {
    t->table = m->d_table;
    t->router_dl = m->d_router_dl;
    t->router_t = m->d_router_t;
    t->norm = m->d_norm;
    t->lay = m->lay;
    t->dims = m->dims;
}
const mia_moe_config *mia_moe_cfg(const mia_moe *m) { return &m->cfg; }
static int check_status(mia_moe *m, int l0);

static size_t align_up(size_t n, size_t a) { return (n + a - 1) / a * a; }

const char *mia_moe_error(const mia_moe *m) { return m ? m->err : "null handle"; }
size_t mia_moe_blob_bytes(const mia_moe *m) { return m->blob_bytes; }
size_t mia_moe_off_up(const mia_moe *m) { return m->off_up; }
size_t mia_moe_off_down(const mia_moe *m) { return m->off_down; }
mhip_ctx *mia_moe_gpu(mia_moe *m) { return m->gpu; }
const mhip_scratch *mia_moe_scratch(const mia_moe *m) { return &m->sc; }
void mia_moe_set_flags(mia_moe *m, int flags) { m->flags = flags; }

void mia_moe_close(mia_moe *m) {
    if (!m) return;
    if (m->gpu) {
        mhip_sync(m->gpu);
        mhip_graph_destroy(m->graph);
        mhip_free(m->gpu, m->d_table);
        mhip_free(m->gpu, m->d_router_t);
        mhip_free(m->gpu, m->d_router_dl);
        mhip_free(m->gpu, m->d_dws);
        mhip_free(m->gpu, m->d_didx);
        mhip_host_free(m->gpu, m->h_stage);
        mhip_free(m->gpu, m->d_dw);
        mhip_free(m->gpu, m->d_norm);
        mhip_free(m->gpu, m->d_router);
        mhip_free(m->gpu, m->d_scratch);
        mhip_free(m->gpu, m->d_x);
        mhip_free(m->gpu, m->d_bias);
        mhip_free(m->gpu, m->d_blob);
        mhip_close(m->gpu);
    }
    free(m->h_blob);
    free(m);
}

int mia_moe_open(mia_moe **out, const mia_moe_config *cfg, char *err, size_t errlen) {
    *out = NULL;
    mia_moe *m = calloc(1, sizeof(*m));
    if (!m) {
        if (err && errlen) snprintf(err, errlen, "out of host memory");
        return -1;
    }
    m->cfg = *cfg;
    m->dims.dim = cfg->dim;
    m->dims.n_experts = cfg->n_experts;
    m->dims.n_active = cfg->n_active;
    m->dims.expert_hidden = cfg->expert_hidden;
    m->dims.norm_topk = cfg->norm_topk;
    m->dims.norm_eps = cfg->norm_eps;
    m->n_layers = cfg->n_layers;
    m->max_tokens = cfg->max_tokens;
    int rc = 0;
    if (mhip_layout_of(&m->dims, &m->lay) != 0)
        rc = fail(m, "unsupported MoE shape: dim=%d experts=%d active=%d hidden=%d", cfg->dim,
                  cfg->n_experts, cfg->n_active, cfg->expert_hidden);
    else if (cfg->n_layers < 1 || cfg->max_tokens < 1 ||
             (long)cfg->max_tokens * cfg->n_active > 65535)
        rc = fail(m, "n_layers=%d max_tokens=%d: need >= 1 and max_tokens*n_active <= 65535",
                  cfg->n_layers, cfg->max_tokens);
    char gerr[256] = "";
    if (!rc && mhip_open(&m->gpu, cfg->device, gerr, sizeof(gerr)) != 0)
        rc = fail(m, "GPU: %s", gerr);
    if (!rc) {
        const size_t d = (size_t)cfg->dim, E = (size_t)cfg->n_experts;
        /* .mia blob geometry: 36-byte blocks, 64-byte tensor alignment,
         * 16 KiB blob alignment. */
        const size_t mat = (size_t)cfg->expert_hidden * (d / 32) * 36;
        m->off_up = align_up(mat, 64);
        m->off_down = 2 * m->off_up;
        m->blob_bytes = align_up(m->off_down + d * ((size_t)cfg->expert_hidden / 32) * 36, 16384);
        const size_t table = (size_t)cfg->n_layers * E * m->lay.expert_bytes;
        const size_t scratch = mhip_scratch_bytes(&m->dims, cfg->max_tokens);
        m->d_table = mhip_malloc(m->gpu, table);
        m->d_router_t = mhip_malloc(m->gpu, (size_t)cfg->n_layers * d * E * 4);
        m->d_router_dl = mhip_malloc(m->gpu, (size_t)cfg->n_layers * d * E * 4);
        m->d_dws = mhip_malloc(m->gpu, mhip_decode_ws_bytes());
        m->d_didx = mhip_malloc(m->gpu, (size_t)cfg->n_layers * cfg->n_active * 4);
        m->d_dw = mhip_malloc(m->gpu, (size_t)cfg->n_layers * cfg->n_active * 4);
        m->d_norm = mhip_malloc(m->gpu, (size_t)cfg->n_layers * d * 4);
        m->d_router = mhip_malloc(m->gpu, d * E * 4);
        m->d_scratch = mhip_malloc(m->gpu, scratch);
        m->d_x = mhip_malloc(m->gpu, (size_t)cfg->max_tokens * d * 4);
        m->d_bias = mhip_malloc(m->gpu, E * 4);
        m->d_blob = mhip_malloc(m->gpu, m->blob_bytes);
        m->h_blob = malloc(m->blob_bytes);
        m->h_stage = (float *)mhip_host_malloc(m->gpu, (2 * d + 2 * (size_t)cfg->n_active) * 4);
        if (!m->d_table || !m->d_router_t || !m->d_router_dl || !m->d_dws || !m->d_didx ||
            !m->d_dw || !m->d_norm || !m->d_router || !m->d_scratch || !m->d_x || !m->d_bias ||
            !m->d_blob || !m->h_stage)
            rc = fail(m, "HBM allocation (%.2f GiB table): %s", table / 1073741824.0,
                      mhip_error(m->gpu));
        else if (!m->h_blob)
            rc = fail(m, "out of host memory");
        if (!rc) {
            mhip_scratch_carve(&m->dims, cfg->max_tokens, m->d_scratch, &m->sc);
            if (mhip_zero(m->gpu, m->sc.status, 16) ||
                mhip_zero(m->gpu, m->d_table, table) ||
                mhip_zero(m->gpu, m->d_router_t, (size_t)cfg->n_layers * d * E * 4) ||
                mhip_zero(m->gpu, m->d_router_dl, (size_t)cfg->n_layers * d * E * 4) ||
                mhip_fill_f32(m->gpu, m->d_norm, (size_t)cfg->n_layers * d, 1.0f) ||
                mhip_sync(m->gpu))
                rc = gpu_fail(m);
        }
    }
    if (rc) {
        if (err && errlen) snprintf(err, errlen, "%s", m->err);
        mia_moe_close(m);
        return -1;
    }
    *out = m;
    return 0;
}

static int check_slot(mia_moe *m, int layer, int expert) {
    if (layer < 0 || layer >= m->n_layers || expert < 0 || expert >= m->dims.n_experts)
        return fail(m, "expert (%d, %d) out of range (%d layers, %d experts)", layer, expert,
                    m->n_layers, m->dims.n_experts);
    return 0;
}

int mia_moe_load_expert(mia_moe *m, int layer, int expert, const void *blob) {
    if (check_slot(m, layer, expert)) return -1;
    if (mhip_h2d(m->gpu, m->d_blob, blob, m->blob_bytes) ||
        mhip_table_repack(m->gpu, &m->dims, m->d_table, layer, &expert, 1, m->d_blob,
                          m->blob_bytes, m->off_up, m->off_down) ||
        mhip_sync(m->gpu))
        return gpu_fail(m);
    return 0;
}

int mia_moe_load_experts(mia_moe *m, mia_expert_loader load, void *ctx) {
    for (int l = 0; l < m->n_layers; l++)
        for (int e = 0; e < m->dims.n_experts; e++) {
            if (load(ctx, l, e, m->h_blob) != 0)
                return fail(m, "expert loader failed for layer %d expert %d", l, e);
            if (mia_moe_load_expert(m, l, e, m->h_blob)) return -1;
        }
    return 0;
}

int mia_moe_read_expert(mia_moe *m, int layer, int expert, void *blob) {
    if (check_slot(m, layer, expert)) return -1;
    if (mhip_table_unpack(m->gpu, &m->dims, m->d_table, layer, expert, m->d_blob, m->blob_bytes,
                          m->off_up, m->off_down) ||
        mhip_d2h(m->gpu, blob, m->d_blob, m->blob_bytes))
        return gpu_fail(m);
    return 0;
}

int mia_moe_set_layer(mia_moe *m, int layer, const float *ffn_norm, const float *router) {
    if (layer < 0 || layer >= m->n_layers) return fail(m, "layer %d out of range", layer);
    const size_t d = (size_t)m->dims.dim, E = (size_t)m->dims.n_experts;
    if (mhip_h2d(m->gpu, m->d_norm + layer * d, ffn_norm, d * 4) ||
        mhip_h2d(m->gpu, m->d_router, router, d * E * 4) ||
        mhip_router_decode_layout(m->gpu, &m->dims, m->d_router_dl + layer * d * E, m->d_router) ||
        mhip_router_transpose(m->gpu, &m->dims, m->d_router_t + layer * d * E, m->d_router) ||
        mhip_sync(m->gpu))
        return gpu_fail(m);
    return 0;
}

int mia_moe_synth(mia_moe *m, uint64_t seed) {
    const size_t d = (size_t)m->dims.dim, E = (size_t)m->dims.n_experts;
    if (mhip_table_synth(m->gpu, &m->dims, m->d_table, seed, 0, m->n_layers)) return gpu_fail(m);
    for (int l = 0; l < m->n_layers; l++)
        if (mhip_router_synth(m->gpu, &m->dims, m->d_router_t + l * d * E,
                              m->d_router_dl + l * d * E, seed, l))
            return gpu_fail(m);
    if (mhip_fill_f32(m->gpu, m->d_norm, (size_t)m->n_layers * d, 1.0f) || mhip_sync(m->gpu))
        return gpu_fail(m);
    return 0;
}

static int run_layer(mia_moe *m, int layer, float *d_x, int T, const float *d_bias) {
    if (layer < 0 || layer >= m->n_layers) return fail(m, "layer %d out of range", layer);
    if (T < 0 || T > m->max_tokens)
        return fail(m, "T=%d outside [0, max_tokens=%d]", T, m->max_tokens);
    const size_t d = (size_t)m->dims.dim, E = (size_t)m->dims.n_experts;
    const unsigned char *tl =
        (const unsigned char *)m->d_table + (size_t)layer * E * m->lay.expert_bytes;
    if (mhip_moe_layer(m->gpu, &m->dims, &m->lay, tl, m->d_router_t + layer * d * E,
                       m->d_norm + layer * d, d_bias, d_x, T, &m->sc, m->flags))
        return gpu_fail(m);
    return 0;
}

/* The device status words describe the last public layer or stack call:
 * cleared (fill kernel) before its first launch. */
static int clear_status(mia_moe *m) {
    if (mhip_zero(m->gpu, m->sc.status, 16)) return gpu_fail(m);
    return 0;
}

int mia_moe_layer_dev(mia_moe *m, int layer, float *d_x, int T, const float *d_bias) {
    if (clear_status(m)) return -1;
    return run_layer(m, layer, d_x, T, d_bias);
}

int mia_moe_stack_dev(mia_moe *m, int l0, int l1, float *d_x, int T) {
    if (l0 < 0 || l1 > m->n_layers || l0 > l1)
        return fail(m, "layer range [%d, %d) outside [0, %d)", l0, l1, m->n_layers);
    if (clear_status(m)) return -1;
    for (int l = l0; l < l1; l++)
        if (run_layer(m, l, d_x, T, NULL)) return -1;
    return 0;
}

int mia_moe_stack_graph(mia_moe *m, int l0, int l1, float *d_x, int T) {
    if (l0 < 0 || l1 > m->n_layers || l0 > l1)
        return fail(m, "layer range [%d, %d) outside [0, %d)", l0, l1, m->n_layers);
    if (T < 0 || T > m->max_tokens)
        return fail(m, "T=%d outside [0, max_tokens=%d]", T, m->max_tokens);
    if (!m->graph || m->g_l0 != l0 || m->g_l1 != l1 || m->g_x != d_x || m->g_T != T ||
        m->g_flags != m->flags) {
        mhip_graph_destroy(m->graph);
        m->graph = NULL;
        if (mhip_graph_begin(m->gpu)) return gpu_fail(m);
        const int rc = mia_moe_stack_dev(m, l0, l1, d_x, T);
        char why[512];
        snprintf(why, sizeof why, "%s", m->err);
        if (mhip_graph_end(m->gpu, rc ? NULL : &m->graph)) return gpu_fail(m);
        if (rc) return fail(m, "recording the stack: %s", why);
        m->g_l0 = l0;
        m->g_l1 = l1;
        m->g_x = d_x;
        m->g_T = T;
        m->g_flags = m->flags;
    }
    if (mhip_graph_launch(m->gpu, m->graph)) return gpu_fail(m);
    return 0;
}

int mia_moe_decode_dev(mia_moe *m, int l0, int l1, float *d_x, const float *d_bias) {
    if (l0 < 0 || l1 > m->n_layers || l0 > l1)
        return fail(m, "layer range [%d, %d) outside [0, %d)", l0, l1, m->n_layers);
    const size_t d = (size_t)m->dims.dim, E = (size_t)m->dims.n_experts,
                 K = (size_t)m->dims.n_active;
    if (mhip_decode_stack(m->gpu, &m->dims, &m->lay,
                          (const unsigned char *)m->d_table + (size_t)l0 * E * m->lay.expert_bytes,
                          m->d_router_dl + l0 * d * E, m->d_router_t + l0 * d * E,
                          m->d_norm + l0 * d, d_bias, d_x, l1 - l0, m->d_dws, m->d_didx + l0 * K,
                          m->d_dw + l0 * K, m->flags))
        return gpu_fail(m);
    return 0;
}

int mia_moe_decode_status(mia_moe *m, int status[4]) {
    if (mhip_decode_status(m->gpu, m->d_dws, status)) return gpu_fail(m);
    return 0;
}

int mia_moe_decode_trace(mia_moe *m, unsigned long long *out) {
    if (mhip_decode_trace(m->gpu, m->d_dws, out)) return gpu_fail(m);
    return 0;
}

/* Layers [l0, l1) of one token per stage on m->d_x (the bit-exact path),
 * each layer's routing copied to the decode routing arrays. */
static int decode_per_stage(mia_moe *m, int l0, int l1, const float *d_bias) {
    const size_t K = (size_t)m->dims.n_active;
    if (clear_status(m)) return -1;
    for (int l = l0; l < l1; l++) {
        if (run_layer(m, l, m->d_x, 1, d_bias)) return -1;
        if (mhip_d2d(m->gpu, m->d_didx + l * K, m->sc.idx, K * 4) ||
            mhip_d2d(m->gpu, m->d_dw + l * K, m->sc.w, K * 4))
            return gpu_fail(m);
    }
    return check_status(m, l0);
}

int mia_moe_decode(mia_moe *m, int l0, int l1, float *x, const float *bias, int *idx, float *w) {
    const size_t d = (size_t)m->dims.dim, E = (size_t)m->dims.n_experts,
                 K = (size_t)m->dims.n_active;
    if (mhip_h2d(m->gpu, m->d_x, x, d * 4)) return gpu_fail(m);
    if (bias && mhip_h2d(m->gpu, m->d_bias, bias, E * 4)) return gpu_fail(m);
    if (mia_moe_decode_dev(m, l0, l1, m->d_x, bias ? m->d_bias : NULL)) return -1;
    int st[4];
    if (mhip_sync(m->gpu) || mhip_decode_status(m->gpu, m->d_dws, st)) return gpu_fail(m);
    if (st[0]) {
        /* The launch aborted (a wait timed out, workgroups not placed as it
         * needs, or a forced abort) and left d_x invalid; x (host) is
         * untouched: run the layers per stage instead. mia_moe_decode_status
         * still shows the aborted launch. */
        if (mhip_h2d(m->gpu, m->d_x, x, d * 4) ||
            decode_per_stage(m, l0, l1, bias ? m->d_bias : NULL))
            return -1;
    }
    if (mhip_d2h(m->gpu, x, m->d_x, d * 4) ||
        (idx && mhip_d2h(m->gpu, idx, m->d_didx + l0 * K, (size_t)(l1 - l0) * K * 4)) ||
        (w && mhip_d2h(m->gpu, w, m->d_dw + l0 * K, (size_t)(l1 - l0) * K * 4)))
        return gpu_fail(m);
    return 0;
}

int mia_moe_status(mia_moe *m, int status[4]) {
    if (mhip_d2h(m->gpu, status, m->sc.status, 16)) return gpu_fail(m);
    return 0;
}

/* Fails when the last call's layers met an expert index out of range,
 * naming the first such layer (l0 = the call's first layer). */
static int check_status(mia_moe *m, int l0) {
    int st[4];
    if (mia_moe_status(m, st)) return -1;
    if (st[0] & 1)
        return fail(m, "router produced an expert index out of range (layer %d)",
                    l0 + (st[2] > 0 ? st[2] - 1 : 0));
    return 0;
}

/* One token through one layer in a launch of the persistent decode kernel
 * with the exact router (bit-equal to the reference, like the per-stage
 * path, and several times faster at T = 1). x and the routing travel through
 * the pinned staging buffer with queued copies, so the call waits for the
 * device once (in the status read). Returns 1 (x untouched) when the launch
 * aborted: the caller then runs the layer per stage. */
static int decode_one_layer(mia_moe *m, int layer, float *x, const float *bias, int *idx,
                            float *w) {
    const size_t d = (size_t)m->dims.dim, E = (size_t)m->dims.n_experts,
                 K = (size_t)m->dims.n_active;
    float *hx = m->h_stage, *hy = m->h_stage + d, *hw = m->h_stage + 2 * d + K;
    int *hi = (int *)(m->h_stage + 2 * d);
    if (layer < 0 || layer >= m->n_layers) return fail(m, "layer %d out of range", layer);
    memcpy(hx, x, d * 4);
    if (mhip_h2d_async(m->gpu, m->d_x, hx, d * 4)) return gpu_fail(m);
    if (bias && mhip_h2d(m->gpu, m->d_bias, bias, E * 4)) return gpu_fail(m);
    if (mhip_decode_stack(m->gpu, &m->dims, &m->lay,
                          (const unsigned char *)m->d_table +
                              (size_t)layer * E * m->lay.expert_bytes,
                          m->d_router_dl + layer * d * E, m->d_router_t + layer * d * E,
                          m->d_norm + layer * d, bias ? m->d_bias : NULL, m->d_x, 1, m->d_dws,
                          m->d_didx + layer * K, m->d_dw + layer * K,
                          m->flags | MHIP_FORCE_EXACT_ROUTER))
        return gpu_fail(m);
    if (mhip_d2h_async(m->gpu, hy, m->d_x, d * 4) ||
        mhip_d2h_async(m->gpu, hi, m->d_didx + layer * K, K * 4) ||
        mhip_d2h_async(m->gpu, hw, m->d_dw + layer * K, K * 4))
        return gpu_fail(m);
    int st[4];
    /* the status read waits for the stream, copies above included */
    if (mhip_decode_status(m->gpu, m->d_dws, st)) return gpu_fail(m);
    if (st[0]) return 1;
    memcpy(x, hy, d * 4);
    if (idx) memcpy(idx, hi, K * 4);
    if (w) memcpy(w, hw, K * 4);
    return 0;
}

int mia_moe_layer_ex(mia_moe *m, int layer, float *x, int T, const float *bias, int *idx,
                     float *w, float *logits) {
    if (T < 0 || T > m->max_tokens)
        return fail(m, "T=%d outside [0, max_tokens=%d]", T, m->max_tokens);
    if (T == 0) return 0;
    if (T == 1 && !logits && !(m->flags & MHIP_EXACT_EXPERTS)) {
        const int ok = mhip_decode_supported(m->gpu, &m->dims);
        if (ok < 0) return gpu_fail(m);
        if (ok) {
            const int rc = decode_one_layer(m, layer, x, bias, idx, w);
            if (rc <= 0) return rc;
            /* the launch aborted (a wait timed out, or workgroups were not
             * placed as it needs): x is untouched, and the per-stage path
             * below gives the same bits (mia_moe_decode_status still
             * shows the aborted launch) */
        }
    }
    const size_t d = (size_t)m->dims.dim, E = (size_t)m->dims.n_experts,
                 K = (size_t)m->dims.n_active;
    if (clear_status(m)) return -1;
    if (mhip_h2d(m->gpu, m->d_x, x, (size_t)T * d * 4)) return gpu_fail(m);
    if (bias && mhip_h2d(m->gpu, m->d_bias, bias, E * 4)) return gpu_fail(m);
    if (run_layer(m, layer, m->d_x, T, bias ? m->d_bias : NULL)) return -1;
    if (mhip_d2h(m->gpu, x, m->d_x, (size_t)T * d * 4) ||
        (idx && mhip_d2h(m->gpu, idx, m->sc.idx, (size_t)T * K * 4)) ||
        (w && mhip_d2h(m->gpu, w, m->sc.w, (size_t)T * K * 4)) ||
        (logits && mhip_d2h(m->gpu, logits, m->sc.logits, (size_t)T * E * 4)))
        return gpu_fail(m);
    return check_status(m, layer);
}

int mia_moe_layer(mia_moe *m, int layer, float *x, int T) {
    return mia_moe_layer_ex(m, layer, x, T, NULL, NULL, NULL, NULL);
}

int mia_moe_stack(mia_moe *m, int l0, int l1, float *x, int T) {
    if (T < 0 || T > m->max_tokens)
        return fail(m, "T=%d outside [0, max_tokens=%d]", T, m->max_tokens);
    if (T == 0) return 0;
    const size_t d = (size_t)m->dims.dim;
    if (mhip_h2d(m->gpu, m->d_x, x, (size_t)T * d * 4)) return gpu_fail(m);
    if (mia_moe_stack_dev(m, l0, l1, m->d_x, T)) return -1;
    if (mhip_d2h(m->gpu, x, m->d_x, (size_t)T * d * 4)) return gpu_fail(m);
    return check_status(m, l0);
}
