/*
 * mia_model_step on one GPU (include/mia/model_gpu.h): the token's
 * embedding, n_layers x (attention, MoE), final rmsnorm and output head, all
 * on device memory (src/model/forward.c:199-217 of the reference).
 *
 * The .mia file's dense section is uploaded as it is laid out (36-byte
 * Q8_0 blocks, fp32 vectors), so each tensor's device address is the
 * dense walk's offset. Where the shape allows it, a layer is two launches:
 * the one-launch attention (mhip_attention_layer) and the one-layer launch
 * of the persistent decode kernel (the exact router in exact mode); else
 * the per-stage kernels, which are bit-exact. Both launches report aborts
 * into per-layer slots; should one abort, the step restores x from the copy
 * taken before that launch and reruns from there per stage (the KV rows of
 * the later layers are rewritten).
 */
#define _FILE_OFFSET_BITS 64
#define _POSIX_C_SOURCE 200809L
#include "mia/model_gpu.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "moe_internal.h"

struct mia_gpu_model {
    mia_file_info info;
    mia_moe *moe;
    mhip_ctx *gpu;
    mia_moe_tensors mt;
    mhip_attn_dims ad;
    int max_seq, flags, decode_ok, attn_ok, stack_ok, aborts;
    int logits_ok; /* d_logits holds the last step's logits */
    unsigned char *d_dense;
    mia_layer_offsets *lo;   /* [L] */
    uint64_t off_embd, off_onorm, off_out;
    float *d_kc, *d_vc;      /* [L][max_seq][kvd] */
    double *d_rope;          /* [max_seq][head_dim/2][2] */
    void *d_scratch;
    float *d_x;              /* [dim] residual */
    float *d_xsave;          /* [L][dim] x before each layer's MoE */
    float *d_xin;            /* [L][dim] x before each layer's attention (one-launch path) */
    void *d_aws;             /* workspace of the one-launch attention */
    mhip_attn_layer *d_al;   /* [L] each layer's attention tensors and cache (model stack) */
    void *d_mws;             /* workspace of the model stack */
    int *d_status;           /* [L][4] decode status per layer, then [L] attention aborts */
    float *d_logits;         /* [vocab] */
    void *d_sample;          /* mhip_sample scratch for vocab logits */
    int *d_token, *h_token;  /* the sampled token (device, pinned) */
    float *h_logits;         /* pinned [vocab] */
    int *h_status;           /* pinned [L][4] */
    float *d_xb;             /* [PREFILL_MAX][dim] the residuals of a prompt batch */
    void *d_bscratch;        /* mhip_attention_batch scratch for PREFILL_MAX tokens */
    unsigned char *d_apack;  /* [L] each layer's attention weights packed for batches */
    size_t apack_bytes;      /* per layer (0: not packed, the vector rows run) */
    char err[512];
};

/* Prompt tokens per batch of mia_gpu_model_prefill, at most (every MoE
 * path is bit-exact, so a batch of any size gives the feeds' bits; from
 * MHIP_GEMM_MIN_A assignments on its experts run on the matrix cores). */
enum { PREFILL_MAX = 1024 };

static int mfail(mia_gpu_model *m, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(m->err, sizeof(m->err), fmt, ap);
    va_end(ap);
    return -1;
}

const char *mia_gpu_model_error(const mia_gpu_model *m) { return m ? m->err : "null handle"; }
int mia_gpu_model_vocab(const mia_gpu_model *m) { return (int)m->info.vocab; }
void mia_gpu_model_set_flags(mia_gpu_model *m, int flags) { m->flags = flags; }
int mia_gpu_model_aborts(const mia_gpu_model *m) { return m->aborts; }

int mia_gpu_model_trace(mia_gpu_model *m, unsigned long long *out) {
    if (!m->stack_ok) return mfail(m, "no model stack at this shape");
    if (mhip_decode_trace(m->gpu, m->d_mws, out)) return mfail(m, "%s", mhip_error(m->gpu));
    return 0;
}

void mia_gpu_model_close(mia_gpu_model *m) {
    if (!m) return;
    if (m->gpu) {
        mhip_sync(m->gpu);
        mhip_free(m->gpu, m->d_dense);
        mhip_free(m->gpu, m->d_kc);
        mhip_free(m->gpu, m->d_vc);
        mhip_free(m->gpu, m->d_rope);
        mhip_free(m->gpu, m->d_scratch);
        mhip_free(m->gpu, m->d_x);
        mhip_free(m->gpu, m->d_xsave);
        mhip_free(m->gpu, m->d_xb);
        mhip_free(m->gpu, m->d_bscratch);
        mhip_free(m->gpu, m->d_apack);
        mhip_free(m->gpu, m->d_xin);
        mhip_free(m->gpu, m->d_aws);
        mhip_free(m->gpu, m->d_al);
        mhip_free(m->gpu, m->d_mws);
        mhip_free(m->gpu, m->d_status);
        mhip_free(m->gpu, m->d_logits);
        mhip_free(m->gpu, m->d_sample);
        mhip_free(m->gpu, m->d_token);
        mhip_host_free(m->gpu, m->h_token);
        mhip_host_free(m->gpu, m->h_logits);
        mhip_host_free(m->gpu, m->h_status);
    }
    mia_moe_close(m->moe);
    free(m->lo);
    free(m);
}

/* The dense section, read through pinned staging in 64 MiB pieces. */
static int upload_dense(mia_gpu_model *m, const char *path) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return mfail(m, "open %s: %s", path, strerror(errno));
    const size_t chunk = (size_t)64 << 20;
    unsigned char *h = mhip_host_malloc(m->gpu, chunk);
    int rc = h ? 0 : mfail(m, "pinned staging: %s", mhip_error(m->gpu));
    for (uint64_t done = 0; !rc && done < m->info.dense_size;) {
        const size_t n = m->info.dense_size - done < chunk ? (size_t)(m->info.dense_size - done)
                                                           : chunk;
        size_t got = 0;
        while (got < n) {
            const ssize_t r = pread(fd, h + got, n - got, (off_t)(m->info.dense_offset + done + got));
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) break;
            got += (size_t)r;
        }
        if (got != n)
            rc = mfail(m, "%s: reading the dense section", path);
        else if (mhip_h2d(m->gpu, m->d_dense + done, h, n))
            rc = mfail(m, "%s", mhip_error(m->gpu));
        done += n;
    }
    if (h) mhip_host_free(m->gpu, h);
    close(fd);
    return rc;
}

/* Opens the MoE handle and allocates and fills everything but the weights
 * for the shape in m->info. */
static int setup(mia_gpu_model *m, int max_seq, int device) {
    const mia_file_info *h = &m->info;
    char e2[256];
    if (h->wtype != MIA_Q8_0)
        return mfail(m, "weight type %u; the GPU model runs Q8_0 models", h->wtype);
    if (max_seq < 1) return mfail(m, "max_seq=%d", max_seq);
    mia_moe_config c = {(int)h->dim, (int)h->n_layers, (int)h->n_experts, (int)h->n_active,
                        (int)h->expert_hidden, (int)h->norm_topk, h->norm_eps, PREFILL_MAX,
                        device};
    if (mia_moe_open(&m->moe, &c, e2, sizeof e2)) return mfail(m, "%s", e2);
    m->gpu = mia_moe_gpu(m->moe);
    m->max_seq = max_seq;
    m->flags = MHIP_FORCE_EXACT_ROUTER;
    mia_moe_get_tensors(m->moe, &m->mt);
    m->ad = (mhip_attn_dims){(int)h->dim, (int)h->n_heads, (int)h->n_kv_heads, (int)h->head_dim,
                             h->norm_eps};
    const int ok = mhip_decode_supported(m->gpu, &m->mt.dims);
    if (ok < 0) return mfail(m, "%s", mhip_error(m->gpu));
    m->decode_ok = ok > 0;
    const int aok = mhip_attention_layer_supported(m->gpu, &m->ad, max_seq);
    if (aok < 0) return mfail(m, "%s", mhip_error(m->gpu));
    m->attn_ok = aok > 0 && m->decode_ok;
    const int sok = mhip_model_stack_supported(m->gpu, &m->mt.dims, &m->ad, max_seq);
    if (sok < 0) return mfail(m, "%s", mhip_error(m->gpu));
    m->stack_ok = sok > 0 && m->attn_ok;
    const size_t L = h->n_layers, kvd = (size_t)h->n_kv_heads * h->head_dim;
    const size_t half = h->head_dim / 2, ws = mhip_attention_scratch_bytes(&m->ad, max_seq);
    m->lo = calloc(L, sizeof(*m->lo));
    for (size_t l = 0; m->lo && l < L; l++)
        mia_dense_walk(h, (int)l, &m->lo[l], &m->off_embd, &m->off_onorm, &m->off_out);
    m->d_dense = mhip_malloc(m->gpu, (size_t)h->dense_size);
    m->d_kc = mhip_malloc(m->gpu, L * max_seq * kvd * 4);
    m->d_vc = mhip_malloc(m->gpu, L * max_seq * kvd * 4);
    m->d_rope = mhip_malloc(m->gpu, (size_t)max_seq * half * 2 * 8);
    m->d_scratch = mhip_malloc(m->gpu, ws);
    m->d_x = mhip_malloc(m->gpu, (size_t)h->dim * 4);
    m->d_xsave = mhip_malloc(m->gpu, L * h->dim * 4);
    m->d_status = mhip_malloc(m->gpu, L * 20);
    m->d_logits = mhip_malloc(m->gpu, (size_t)h->vocab * 4);
    m->h_logits = mhip_host_malloc(m->gpu, (size_t)h->vocab * 4);
    m->h_status = mhip_host_malloc(m->gpu, L * 20);
    if (m->attn_ok) {
        m->d_xin = mhip_malloc(m->gpu, L * h->dim * 4);
        m->d_aws = mhip_malloc(m->gpu, mhip_attention_layer_ws_bytes());
        if (!m->d_xin || !m->d_aws) return mfail(m, "device memory: %s", mhip_error(m->gpu));
    }
    if (m->stack_ok) {
        m->d_al = mhip_malloc(m->gpu, L * sizeof(mhip_attn_layer));
        m->d_mws = mhip_malloc(m->gpu, mhip_model_stack_ws_bytes());
        if (!m->d_al || !m->d_mws || !m->lo || !m->d_dense || !m->d_kc || !m->d_vc)
            return mfail(m, "device memory: %s", mhip_error(m->gpu));
        mhip_attn_layer *al = malloc(L * sizeof(*al));
        if (!al) return mfail(m, "out of host memory");
        for (size_t l = 0; l < L; l++) {
            const mia_layer_offsets *o = &m->lo[l];
            const unsigned char *b = m->d_dense;
            al[l].attn_norm = (const float *)(b + o->attn_norm);
            al[l].q_norm = (const float *)(b + o->q_norm);
            al[l].k_norm = (const float *)(b + o->k_norm);
            al[l].wq = b + o->wq;
            al[l].wk = b + o->wk;
            al[l].wv = b + o->wv;
            al[l].wo = b + o->wo;
            al[l].kc = m->d_kc + l * max_seq * kvd;
            al[l].vc = m->d_vc + l * max_seq * kvd;
        }
        const int e = mhip_h2d(m->gpu, m->d_al, al, L * sizeof(*al));
        free(al);
        if (e) return mfail(m, "%s", mhip_error(m->gpu));
    }
    const size_t sb = mhip_sample_scratch_bytes((int)h->vocab);
    if (!sb) return mfail(m, "vocabulary of %u tokens: no sampler for it", h->vocab);
    m->d_sample = mhip_malloc(m->gpu, sb);
    m->d_token = mhip_malloc(m->gpu, sizeof(int));
    m->h_token = mhip_host_malloc(m->gpu, sizeof(int));
    if (!m->lo || !m->d_dense || !m->d_kc || !m->d_vc || !m->d_rope || !m->d_scratch ||
        !m->d_x || !m->d_xsave || !m->d_status || !m->d_logits || !m->h_logits ||
        !m->h_status || !m->d_sample || !m->d_token || !m->h_token)
        return mfail(m, "device memory: %s", mhip_error(m->gpu));
    /* RoPE angles as the reference computes them (forward.c:86-89) */
    double *t = malloc((size_t)max_seq * half * 2 * 8);
    if (!t) return mfail(m, "out of host memory");
    for (size_t p = 0; p < (size_t)max_seq; p++)
        for (size_t i = 0; i < half; i++) {
            const double freq = pow((double)h->rope_theta, -2.0 * (double)i / h->head_dim);
            const double a = (double)p * freq;
            t[(p * half + i) * 2] = cos(a);
            t[(p * half + i) * 2 + 1] = sin(a);
        }
    const int rc = mhip_h2d(m->gpu, m->d_rope, t, (size_t)max_seq * half * 2 * 8) ||
                   mhip_zero(m->gpu, m->d_kc, L * max_seq * kvd * 4) ||
                   mhip_zero(m->gpu, m->d_vc, L * max_seq * kvd * 4) ||
                   mhip_zero(m->gpu, m->d_scratch, ws) || mhip_sync(m->gpu);
    free(t);
    return rc ? mfail(m, "%s", mhip_error(m->gpu)) : 0;
}

static int finish(mia_gpu_model *m, int rc, mia_gpu_model **out, char *err, size_t errlen) {
    if (rc) {
        if (err && errlen) snprintf(err, errlen, "%s", m->err);
        mia_gpu_model_close(m);
        return -1;
    }
    *out = m;
    return 0;
}

int mia_gpu_model_open(mia_gpu_model **out, const char *path, int max_seq, int device,
                       char *err, size_t errlen) {
    *out = NULL;
    mia_gpu_model *m = calloc(1, sizeof(*m));
    if (!m) {
        if (err && errlen) snprintf(err, errlen, "out of host memory");
        return -1;
    }
    char e2[256];
    int rc = mia_file_probe(path, &m->info, e2, sizeof e2) ? mfail(m, "%s", e2) : 0;
    if (!rc) rc = setup(m, max_seq, device);
    if (!rc && mia_moe_load_file(m->moe, path)) rc = mfail(m, "%s", mia_moe_error(m->moe));
    if (!rc) rc = upload_dense(m, path);
    return finish(m, rc, out, err, errlen);
}

/* Q8_0 matrix [rows][cols] at d_dense + off from N(0, 0.02) values. */
static int synth_q8(mia_gpu_model *m, float *tmp, uint64_t off, size_t rows, size_t cols,
                    uint64_t seed, uint64_t stream) {
    const size_t n = rows * cols;
    if (mhip_synth_f32(m->gpu, tmp, n, seed, stream, 0.02) ||
        mhip_quantize_q8(m->gpu, tmp, m->d_dense + off, (int)n))
        return mfail(m, "%s", mhip_error(m->gpu));
    return 0;
}

int mia_gpu_model_synth(mia_gpu_model **out, const mia_file_info *shape, int max_seq,
                        int device, uint64_t seed, char *err, size_t errlen) {
    *out = NULL;
    mia_gpu_model *m = calloc(1, sizeof(*m));
    if (!m) {
        if (err && errlen) snprintf(err, errlen, "out of host memory");
        return -1;
    }
    mia_file_info *h = &m->info;
    *h = *shape;
    h->dense_offset = 0;
    h->dense_size = mia_dense_walk(h, -1, NULL, NULL, NULL, NULL);
    int rc = 0;
    if (!h->dim || h->dim % MIA_QK || !h->n_layers || !h->n_heads || !h->n_kv_heads ||
        h->n_heads % h->n_kv_heads || !h->head_dim || h->head_dim % 2 || !h->vocab ||
        !h->n_experts || !h->n_active || h->n_active > h->n_experts || !h->expert_hidden ||
        h->expert_hidden % MIA_QK || ((uint64_t)h->n_heads * h->head_dim) % MIA_QK)
        rc = mfail(m, "unsupported model shape");
    if (!rc) rc = setup(m, max_seq, device);
    if (!rc && mia_moe_synth(m->moe, seed)) rc = mfail(m, "%s", mia_moe_error(m->moe));
    const uint64_t d = h->dim, qd = (uint64_t)h->n_heads * h->head_dim,
                   kvd = (uint64_t)h->n_kv_heads * h->head_dim;
    const uint64_t big = (uint64_t)h->vocab * d > qd * d ? (uint64_t)h->vocab * d : qd * d;
    float *tmp = rc ? NULL : mhip_malloc(m->gpu, big * 4);
    if (!rc && !tmp) rc = mfail(m, "device memory: %s", mhip_error(m->gpu));
    if (!rc) rc = synth_q8(m, tmp, m->off_embd, h->vocab, d, seed, 1);
    for (uint32_t l = 0; !rc && l < h->n_layers; l++) {
        const mia_layer_offsets *o = &m->lo[l];
        const uint64_t st = 16 + 8 * (uint64_t)l;
        rc = synth_q8(m, tmp, o->wq, qd, d, seed, st) ||
             synth_q8(m, tmp, o->wk, kvd, d, seed, st + 1) ||
             synth_q8(m, tmp, o->wv, kvd, d, seed, st + 2) ||
             synth_q8(m, tmp, o->wo, d, qd, seed, st + 3);
        if (!rc &&
            (mhip_fill_f32(m->gpu, (float *)(m->d_dense + o->attn_norm), d, 1.0f) ||
             mhip_fill_f32(m->gpu, (float *)(m->d_dense + o->q_norm), h->head_dim, 1.0f) ||
             mhip_fill_f32(m->gpu, (float *)(m->d_dense + o->k_norm), h->head_dim, 1.0f) ||
             mhip_fill_f32(m->gpu, (float *)(m->d_dense + o->ffn_norm), d, 1.0f) ||
             mhip_synth_f32(m->gpu, (float *)(m->d_dense + o->router), (size_t)h->n_experts * d,
                            seed, st + 4, 0.02)))
            rc = mfail(m, "%s", mhip_error(m->gpu));
    }
    if (!rc) rc = synth_q8(m, tmp, m->off_out, h->vocab, d, seed, 2);
    if (!rc && (mhip_fill_f32(m->gpu, (float *)(m->d_dense + m->off_onorm), d, 1.0f) ||
                mhip_sync(m->gpu)))
        rc = mfail(m, "%s", mhip_error(m->gpu));
    if (tmp) mhip_free(m->gpu, tmp);
    return finish(m, rc, out, err, errlen);
}

/* Queues the attention of layer l at pos (and, with save, the copy of the
 * new x that an aborted MoE launch of the layer restarts from). */
static int attention(mia_gpu_model *m, int l, int pos, int save) {
    const size_t kvd = (size_t)m->info.n_kv_heads * m->info.head_dim;
    const mia_layer_offsets *o = &m->lo[l];
    const unsigned char *b = m->d_dense;
    float *kc = m->d_kc + (size_t)l * m->max_seq * kvd, *vc = m->d_vc + (size_t)l * m->max_seq * kvd;
    if (mhip_attention(m->gpu, &m->ad, (const float *)(b + o->attn_norm), b + o->wq, b + o->wk,
                       b + o->wv, b + o->wo, (const float *)(b + o->q_norm),
                       (const float *)(b + o->k_norm), m->d_rope, kc, vc, pos, m->max_seq, m->d_x,
                       save ? m->d_xsave + (size_t)l * m->info.dim : NULL, m->d_scratch, 0))
        return mfail(m, "%s", mhip_error(m->gpu));
    return 0;
}

/* The same as one launch (the step's common path): x before and after are
 * kept for the reruns, aborts are reported into the layer's attention slot
 * (after the decode status words). */
static int attention_layer(mia_gpu_model *m, int l, int pos) {
    const size_t kvd = (size_t)m->info.n_kv_heads * m->info.head_dim, d = m->info.dim;
    const mia_layer_offsets *o = &m->lo[l];
    const unsigned char *b = m->d_dense;
    float *kc = m->d_kc + (size_t)l * m->max_seq * kvd, *vc = m->d_vc + (size_t)l * m->max_seq * kvd;
    if (mhip_attention_layer(m->gpu, &m->ad, (const float *)(b + o->attn_norm), b + o->wq,
                             b + o->wk, b + o->wv, b + o->wo, (const float *)(b + o->q_norm),
                             (const float *)(b + o->k_norm), m->d_rope, kc, vc, pos, m->max_seq,
                             m->d_x, m->d_xin + l * d, m->d_xsave + l * d, m->d_aws,
                             m->d_status + 4 * (size_t)m->info.n_layers + l,
                             m->flags & (MHIP_ATTN_FORCE_ABORT | MHIP_FORCE_SEQ_RMS)))
        return mfail(m, "%s", mhip_error(m->gpu));
    return 0;
}

/* Queues the MoE of layer l on d_x: one decode launch reporting into its
 * status slot, or (per_stage, or no decode launch for this shape) the
 * per-stage kernels. */
static int moe(mia_gpu_model *m, int l, int per_stage) {
    if (per_stage || !m->decode_ok || (m->flags & MHIP_EXACT_EXPERTS)) {
        if (mia_moe_layer_dev(m->moe, l, m->d_x, 1, NULL))
            return mfail(m, "%s", mia_moe_error(m->moe));
        return 0;
    }
    const mia_moe_tensors *t = &m->mt;
    const size_t d = (size_t)t->dims.dim, E = (size_t)t->dims.n_experts;
    if (mhip_decode_stack_noalloc(m->gpu, &t->dims, &t->lay,
                                  (const unsigned char *)t->table +
                                      (size_t)l * E * t->lay.expert_bytes,
                                  t->router_dl + (size_t)l * E * d, t->router_t + (size_t)l * E * d,
                                  t->norm + (size_t)l * d, NULL, m->d_x, 1, NULL, NULL,
                                  m->d_status + 4 * l,
                                  m->flags & (MHIP_FORCE_EXACT_ROUTER | MHIP_DECODE_CERTIFIED |
                                              MHIP_DECODE_FORCE_ABORT | MHIP_DECODE_CHAINS_FIRST |
                                              MHIP_FORCE_SEQ_RMS)))
        return mfail(m, "%s", mhip_error(m->gpu));
    return 0;
}

/* What follows the last layer: the final rmsnorm and the output head
 * (forward.c:214-215), then either the logits' copy to host or the sampler
 * on the device logits and the token's copy. */
typedef struct {
    mhip_sampler *s; /* NULL: copy the logits */
    uint64_t rng;    /* s->rng before the step (a rerun draws again from it) */
    int no_head;     /* a prompt position whose logits nobody reads */
} step_tail;

static int tail(mia_gpu_model *m, step_tail *t) {
    const mia_file_info *h = &m->info;
    if (t->no_head) return 0;
    if (mhip_output_head(m->gpu, &m->ad, (const float *)(m->d_dense + m->off_onorm),
                         m->d_dense + m->off_out, (int)h->vocab, m->d_x, m->d_logits,
                         m->d_scratch, 0))
        return mfail(m, "%s", mhip_error(m->gpu));
    if (!t->s) {
        if (mhip_d2h_async(m->gpu, m->h_logits, m->d_logits, (size_t)h->vocab * 4))
            return mfail(m, "%s", mhip_error(m->gpu));
        return 0;
    }
    t->s->rng = t->rng;
    if (mhip_sample(m->gpu, t->s, m->d_logits, m->d_sample, m->d_token) ||
        mhip_d2h_async(m->gpu, m->h_token, m->d_token, sizeof(int)))
        return mfail(m, "%s", mhip_error(m->gpu));
    return 0;
}

/* The step's layers as one launch of the model stack (x in d_x holds the
 * embedding row), then the tail; one wait. After an abort (rare) the token
 * reruns from the embedding row through the per-stage kernels. */
static int run_stack(mia_gpu_model *m, int pos, step_tail *t) {
    const int L = (int)m->info.n_layers, d = (int)m->info.dim;
    const mia_moe_tensors *mt = &m->mt;
    if (mhip_d2d(m->gpu, m->d_xin, m->d_x, (size_t)d * 4) ||
        mhip_model_stack(m->gpu, &mt->dims, &mt->lay, mt->table, mt->router_dl, mt->router_t,
                         mt->norm, NULL, &m->ad, m->d_al, m->d_rope, pos, m->max_seq, m->d_x, L,
                         m->d_mws, m->d_status,
                         m->flags & (MHIP_FORCE_EXACT_ROUTER | MHIP_DECODE_CERTIFIED |
                                     MHIP_DECODE_FORCE_ABORT | MHIP_ATTN_FORCE_ABORT |
                                     MHIP_DECODE_CHAINS_FIRST |
                                     MHIP_FORCE_SEQ_RMS | MHIP_DECODE_TRACE)))
        return mfail(m, "%s", mhip_error(m->gpu));
    if (tail(m, t)) return -1;
    if (mhip_d2h_async(m->gpu, m->h_status, m->d_status, 4 * sizeof(int)) || mhip_sync(m->gpu))
        return mfail(m, "%s", mhip_error(m->gpu));
    m->aborts = m->h_status[0] != 0;
    if (m->aborts) {
        if (mhip_d2d(m->gpu, m->d_x, m->d_xin, (size_t)d * 4)) return mfail(m, "%s", mhip_error(m->gpu));
        for (int l = 0; l < L; l++)
            if (attention(m, l, pos, 0) || moe(m, l, 1)) return -1;
        if (tail(m, t)) return -1;
        if (mhip_sync(m->gpu)) return mfail(m, "%s", mhip_error(m->gpu));
    }
    m->logits_ok = !t->no_head;
    return 0;
}

/* One step, then the tail; 0 or -1. */
static int run_step(mia_gpu_model *m, int token, int pos, step_tail *t) {
    const mia_file_info *h = &m->info;
    m->logits_ok = 0;
    const int L = (int)h->n_layers, d = (int)h->dim;
    if (pos < 0 || pos >= m->max_seq || token < 0 || token >= (int)h->vocab)
        return mfail(m, "token %d at position %d outside [0, %u) x [0, %d)", token, pos, h->vocab,
                     m->max_seq);
    if (t->s && t->s->n != (int)h->vocab)
        return mfail(m, "sampler over %d logits, the vocabulary has %u", t->s->n, h->vocab);
    const int decode = m->decode_ok && !(m->flags & MHIP_EXACT_EXPERTS);
    /* forward.c:205-208: the embedding row, dequantized */
    const size_t row = (size_t)(d / MIA_QK) * 36;
    if (mhip_dequantize_q8(m->gpu, m->d_dense + m->off_embd + (size_t)token * row, m->d_x, d))
        return mfail(m, "%s", mhip_error(m->gpu));
    if (decode && m->stack_ok && !(m->flags & MHIP_MODEL_PER_LAYER))
        return run_stack(m, pos, t);
    const int one = decode && m->attn_ok;
    if (one && mhip_zero(m->gpu, m->d_status + 4 * (size_t)L, (size_t)L * 4))
        return mfail(m, "%s", mhip_error(m->gpu));
    for (int l = 0; l < L; l++) {
        if ((one ? attention_layer(m, l, pos) : attention(m, l, pos, decode)) || moe(m, l, 0))
            return -1;
    }
    /* the tail is queued before the launches' status is known: one wait per
     * step; an abort (rare) reruns from the first aborted launch */
    if (tail(m, t)) return -1;
    if ((decode && mhip_d2h_async(m->gpu, m->h_status, m->d_status, (size_t)L * (one ? 20 : 16))) ||
        mhip_sync(m->gpu))
        return mfail(m, "%s", mhip_error(m->gpu));
    m->aborts = 0;
    int first = -1, first_attn = 0;
    for (int l = 0; decode && l < L; l++) {
        const int a = one && m->h_status[4 * L + l], b = m->h_status[4 * l] != 0;
        m->aborts += a + b;
        if (first < 0 && (a || b)) {
            first = l;
            first_attn = a;
        }
    }
    if (first < 0) {
        m->logits_ok = !t->no_head;
        return 0;
    }
    /* an aborted attention launch restarts from x before it, an aborted MoE
     * launch from x after its layer's attention */
    if (mhip_d2d(m->gpu, m->d_x, (first_attn ? m->d_xin : m->d_xsave) + (size_t)first * d,
                 (size_t)d * 4))
        return mfail(m, "%s", mhip_error(m->gpu));
    if ((first_attn && attention(m, first, pos, 0)) || moe(m, first, 1)) return -1;
    for (int l = first + 1; l < L; l++)
        if (attention(m, l, pos, 0) || moe(m, l, 1)) return -1;
    if (tail(m, t)) return -1;
    if (mhip_sync(m->gpu)) return mfail(m, "%s", mhip_error(m->gpu));
    m->logits_ok = !t->no_head;
    return 0;
}

const float *mia_gpu_model_step(mia_gpu_model *m, int token, int pos) {
    step_tail t = {NULL, 0, 0};
    return run_step(m, token, pos, &t) ? NULL : m->h_logits;
}

int mia_gpu_model_feed(mia_gpu_model *m, int token, int pos) {
    step_tail t = {NULL, 0, 1};
    return run_step(m, token, pos, &t);
}

/* n prompt tokens at positions pos .. pos + n - 1 in batches of equal size
 * (up to PREFILL_MAX): each layer's attention for the batch
 * (mhip_attention_batch) and its MoE for the batch (the per-stage kernels
 * for T tokens), the KV rows written as n feeds write them
 * (forward.c:205-213 per token, bit-equal). */
int mia_gpu_model_prefill(mia_gpu_model *m, const int *tokens, int n, int pos) {
    const mia_file_info *h = &m->info;
    m->logits_ok = 0;
    if (n < 0 || !tokens || pos < 0 || pos + n > m->max_seq)
        return mfail(m, "prefill of %d tokens at position %d outside [0, %d)", n, pos,
                     m->max_seq);
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= (int)h->vocab)
            return mfail(m, "token %d outside [0, %u)", tokens[i], h->vocab);
    const int L = (int)h->n_layers, d = (int)h->dim;
    const size_t kvd = (size_t)h->n_kv_heads * h->head_dim, row = (size_t)(d / MIA_QK) * 36;
    const int bmax = PREFILL_MAX;
    if (n == 0) return 0;
    if (!m->d_xb) {
        m->d_xb = mhip_malloc(m->gpu, (size_t)bmax * d * 4);
        m->d_bscratch =
            mhip_malloc(m->gpu, mhip_attention_batch_scratch_bytes(&m->ad, bmax, m->max_seq));
        if (!m->d_xb || !m->d_bscratch) return mfail(m, "device memory: %s", mhip_error(m->gpu));
        /* the attention weights packed once for the matrix-core rows; a
         * shape they do not fit keeps the vector rows */
        const size_t pb = mhip_attention_pack_bytes(&m->ad);
        m->d_apack = pb ? mhip_malloc(m->gpu, pb * (size_t)L) : NULL;
        if (m->d_apack) {
            for (int l = 0; l < L; l++) {
                const mia_layer_offsets *o = &m->lo[l];
                const unsigned char *b = m->d_dense;
                if (mhip_attention_pack(m->gpu, &m->ad, b + o->wq, b + o->wk, b + o->wv, b + o->wo,
                                        m->d_apack + (size_t)l * pb)) {
                    mhip_free(m->gpu, m->d_apack);
                    m->d_apack = NULL;
                    break;
                }
            }
        }
        m->apack_bytes = m->d_apack ? pb : 0;
    }
    const int nbat = (n + bmax - 1) / bmax, bsz = (n + nbat - 1) / nbat;
    for (int b0 = 0; b0 < n; b0 += bsz) {
        const int nb = n - b0 < bsz ? n - b0 : bsz;
        for (int i = 0; i < nb; i++)
            if (mhip_dequantize_q8(m->gpu, m->d_dense + m->off_embd + (size_t)tokens[b0 + i] * row,
                                   m->d_xb + (size_t)i * d, d))
                return mfail(m, "%s", mhip_error(m->gpu));
        for (int l = 0; l < L; l++) {
            const mia_layer_offsets *o = &m->lo[l];
            const unsigned char *b = m->d_dense;
            float *kc = m->d_kc + (size_t)l * m->max_seq * kvd;
            float *vc = m->d_vc + (size_t)l * m->max_seq * kvd;
            if (mhip_attention_batch(m->gpu, &m->ad, (const float *)(b + o->attn_norm), b + o->wq,
                                     b + o->wk, b + o->wv, b + o->wo,
                                     (const float *)(b + o->q_norm),
                                     (const float *)(b + o->k_norm), m->d_rope, kc, vc,
                                     pos + b0, nb, m->max_seq, m->d_xb,
                                     m->d_apack ? m->d_apack + (size_t)l * m->apack_bytes : NULL,
                                     m->d_bscratch, m->flags & MHIP_FORCE_SEQ_RMS))
                return mfail(m, "%s", mhip_error(m->gpu));
            if (mia_moe_layer_dev(m->moe, l, m->d_xb, nb, NULL))
                return mfail(m, "%s", mia_moe_error(m->moe));
        }
    }
    if (mhip_sync(m->gpu)) return mfail(m, "%s", mhip_error(m->gpu));
    return 0;
}

int mia_gpu_model_sample(mia_gpu_model *m, mhip_sampler *s) {
    if (!s) return mfail(m, "null sampler");
    if (!m->logits_ok) return mfail(m, "no logits: the last call was not a step");
    if (s->n != (int)m->info.vocab)
        return mfail(m, "sampler over %d logits, the vocabulary has %u", s->n, m->info.vocab);
    if (mhip_sample(m->gpu, s, m->d_logits, m->d_sample, m->d_token) ||
        mhip_d2h_async(m->gpu, m->h_token, m->d_token, sizeof(int)) || mhip_sync(m->gpu))
        return mfail(m, "%s", mhip_error(m->gpu));
    return *m->h_token;
}

const mia_file_info *mia_gpu_model_info(const mia_gpu_model *m) { return &m->info; }

int mia_gpu_model_step_sample(mia_gpu_model *m, int token, int pos, mhip_sampler *s) {
    if (!s) return mfail(m, "null sampler");
    step_tail t = {s, s->rng, 0};
    if (run_step(m, token, pos, &t)) {
        s->rng = t.rng;
        return -1;
    }
    return *m->h_token;
}
