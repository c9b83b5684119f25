/*
 * CPU restatement of motorIa's Q8_0 MoE FFN path (test infrastructure only;
 * see mia_oracle.h). Written from the reference's behaviour, not its text.
 */
#include "mia_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "mia/synth.h"

/* src/tensor/quant.c:6-9 */
size_t orc_row_bytes(int wtype, int cols) {
    if (wtype == ORC_Q8_0) return (size_t)(cols / ORC_QK) * sizeof(orc_block_q8);
    return (size_t)cols * sizeof(float);
}

/* src/tensor/quant.c:11-27: per 32-block absmax/127 scale, multiply by the
 * reciprocal, round half away from zero. */
void orc_quantize_row_q8(const float *x, orc_block_q8 *y, int n) {
    for (int b = 0; b < n / ORC_QK; b++) {
        const float *v = x + (size_t)b * ORC_QK;
        float amax = 0.0f;
        for (int i = 0; i < ORC_QK; i++) {
            float a = fabsf(v[i]);
            amax = a > amax ? a : amax;
        }
        float d = amax / 127.0f;
        float inv = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = d;
        for (int i = 0; i < ORC_QK; i++) y[b].q[i] = (int8_t)roundf(v[i] * inv);
    }
}

/* src/tensor/quant.c:29-38 */
void orc_dequantize_row(int wtype, const void *src, float *dst, int n) {
    if (wtype == ORC_F32) {
        memcpy(dst, src, sizeof(float) * (size_t)n);
        return;
    }
    const orc_block_q8 *q = (const orc_block_q8 *)src;
    for (int b = 0; b < n / ORC_QK; b++)
        for (int i = 0; i < ORC_QK; i++)
            dst[b * ORC_QK + i] = q[b].d * (float)q[b].q[i];
}

/* src/tensor/matmul.c:13-17: one rounded product, one rounded add, in order. */
static float dot_f32(const float *a, const float *b, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + a[i] * b[i];
    return s;
}

/* src/tensor/matmul.c:19-28: exact int32 block dot, then
 * s = s + ((float)acc * d_w) * d_x, blocks in order. */
static float dot_q8(const orc_block_q8 *a, const orc_block_q8 *b, int nb) {
    float s = 0.0f;
    for (int k = 0; k < nb; k++) {
        int32_t acc = 0;
        for (int i = 0; i < ORC_QK; i++) acc += (int32_t)a[k].q[i] * b[k].q[i];
        s = s + ((float)acc * a[k].d) * b[k].d;
    }
    return s;
}

/* Rows [r0, r1) of the scalar row loop (src/tensor/matmul.c:66-81). */
static void rows_kernel(float *out, const void *w, int wtype, const float *x,
                        const orc_block_q8 *xq, int r0, int r1, int cols) {
    if (wtype == ORC_F32) {
        const float *wf = (const float *)w;
        for (int r = r0; r < r1; r++) out[r] = dot_f32(wf + (size_t)r * cols, x, cols);
        return;
    }
    const int nb = cols / ORC_QK;
    const orc_block_q8 *wq = (const orc_block_q8 *)w;
    for (int r = r0; r < r1; r++) out[r] = dot_q8(wq + (size_t)r * nb, xq, nb);
}

/* src/tensor/matmul.c:89-106: quantize x once (Q8), then the row loop; with
 * nthreads > 1, chunks of 64 rows spread over threads when the matrix is
 * large enough (the reference's GCD split on Apple, CHUNK_ROWS = 64,
 * PARALLEL_MIN_WORK = 65536). Each row is one sequential dot either way, so
 * the split changes no bits. */
static void matvec_mt(float *out, const void *w, int wtype, const float *x,
                      orc_block_q8 *xq, int rows, int cols, int nthreads) {
    if (wtype == ORC_Q8_0) orc_quantize_row_q8(x, xq, cols);
    if (nthreads > 1 && (long)rows * cols >= 65536 && rows > 64) {
        const int chunks = (rows + 63) / 64;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
        for (int c = 0; c < chunks; c++) {
            const int r0 = c * 64, r1 = r0 + 64 < rows ? r0 + 64 : rows;
            rows_kernel(out, w, wtype, x, xq, r0, r1, cols);
        }
        return;
    }
    rows_kernel(out, w, wtype, x, xq, 0, rows, cols);
}

/* src/tensor/matmul.c:91-106 on x86 (one thread). */
void orc_matvec(float *out, const void *w, int wtype, const float *x,
                orc_block_q8 *xq, int rows, int cols) {
    matvec_mt(out, w, wtype, x, xq, rows, cols, 1);
}

/* src/model/forward.c:75-81: sum of squares in double, in order. */
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss = ss + (double)x[i] * (double)x[i];
    float inv = (float)(1.0 / sqrt(ss / n + (double)eps));
    for (int i = 0; i < n; i++) out[i] = (x[i] * inv) * w[i];
}

float orc_expf(float x) { return expf(x); }

/* src/model/forward.c:95-101 */
void orc_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++) mx = x[i] > mx ? x[i] : mx;
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum = sum + x[i];
    }
    for (int i = 0; i < n; i++) x[i] = x[i] / sum;
}

/* src/model/forward.c:104-114: k rounds of "largest untaken", strict '>',
 * so the lowest index wins a tie and the result is in descending order. */
void orc_top_k(const float *p, int n, int k, int *idx) {
    for (int j = 0; j < k; j++) {
        int best = -1;
        for (int i = 0; i < n; i++) {
            int used = 0;
            for (int t = 0; t < j; t++) used |= idx[t] == i;
            if (used) continue;
            if (best < 0 || p[i] > p[best]) best = i;
        }
        idx[j] = best;
    }
}

/* src/model/forward.c:176-181: softmax in place, top-K, then the gate
 * weights p[idx_j], divided by their sum (in j order) when norm_topk. */
void orc_route(float *logits, int E, int K, int norm_topk, int *idx, float *w) {
    orc_softmax(logits, E);
    orc_top_k(logits, E, K, idx);
    float sum = 0.0f;
    for (int j = 0; j < K; j++) {
        w[j] = logits[idx[j]];
        sum = sum + w[j];
    }
    if (norm_topk)
        for (int j = 0; j < K; j++) w[j] = w[j] / sum;
}

static size_t align_up(size_t n, size_t a) { return (n + a - 1) / a * a; }

/* src/storage/mia_file.c:98-101 (64-byte tensor alignment inside the blob) */
size_t orc_off_up(const orc_dims *s) {
    return align_up((size_t)s->expert_hidden * orc_row_bytes(ORC_Q8_0, s->dim), 64);
}
size_t orc_off_down(const orc_dims *s) { return 2 * orc_off_up(s); }
/* tools/internal/mia/format.go:160-163 (blob padded to 16 KiB) */
size_t orc_blob_bytes(const orc_dims *s) {
    return align_up(orc_off_down(s) + (size_t)s->dim * orc_row_bytes(ORC_Q8_0, s->expert_hidden),
                    16384);
}

/* src/model/forward.c:167-197 for one token (the experts come from the table
 * instead of the LRU cache; the cache never changes bits,
 * tools/e2e/e2e_test.go:114-122). */
static int moe_token(const orc_dims *s, float *x, const float *ffn_norm,
                     const float *router, const float *bias,
                     const unsigned char *const *blobs, int *idx_out,
                     float *w_out, float *logits_out, float *xn_out,
                     float *scratch, orc_block_q8 *xq, int row_threads) {
    const int d = s->dim, E = s->n_experts, K = s->n_active, eh = s->expert_hidden;
    int idx[64];
    float w[64];
    if (K > 64) return -1;
    float *xn = scratch, *prob = xn + d, *gate = prob + E, *up = gate + eh,
          *tmp = up + eh;

    orc_rmsnorm(xn, x, ffn_norm, d, s->norm_eps);
    matvec_mt(prob, router, ORC_F32, xn, NULL, E, d, row_threads);
    if (bias)
        for (int e = 0; e < E; e++) prob[e] = prob[e] + bias[e];
    if (logits_out) memcpy(logits_out, prob, sizeof(float) * (size_t)E);
    if (xn_out) memcpy(xn_out, xn, sizeof(float) * (size_t)d);
    orc_route(prob, E, K, s->norm_topk, idx, w);
    if (idx_out) memcpy(idx_out, idx, sizeof(int) * (size_t)K);
    if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)K);

    const size_t off_up = orc_off_up(s), off_down = orc_off_down(s);
    for (int j = 0; j < K; j++) {
        const unsigned char *blob = blobs[idx[j]];
        if (!blob) return -1;
        matvec_mt(gate, blob, ORC_Q8_0, xn, xq, eh, d, row_threads);
        matvec_mt(up, blob + off_up, ORC_Q8_0, xn, xq, eh, d, row_threads);
        for (int i = 0; i < eh; i++) {
            float g = gate[i];
            gate[i] = (g / (1.0f + expf(-g))) * up[i];
        }
        matvec_mt(tmp, blob + off_down, ORC_Q8_0, gate, xq, d, eh, row_threads);
        for (int i = 0; i < d; i++) x[i] = x[i] + w[j] * tmp[i];
    }
    return 0;
}

static int scratch_floats(const orc_dims *s) {
    return 2 * s->dim + s->n_experts + 2 * s->expert_hidden;
}

int orc_moe_layer(const orc_dims *s, int T, float *x, const float *ffn_norm,
                  const float *router, const float *bias,
                  const unsigned char *const *blobs, int *idx, float *w,
                  float *logits, float *xn, int nthreads) {
    const int d = s->dim, E = s->n_experts, K = s->n_active;
    const int maxd = d > s->expert_hidden ? d : s->expert_hidden;
    int rc = 0;
    if (nthreads < 1) nthreads = 1;
    if (T == 1 && nthreads > 1) {
        /* One token: threads over 64-row chunks of each matrix, each chunk
         * loop a top-level parallel region (the pool's threads are reused). */
        float *scratch = malloc(sizeof(float) * (size_t)scratch_floats(s));
        orc_block_q8 *xq = malloc(sizeof(orc_block_q8) * (size_t)(maxd / ORC_QK));
        if (!scratch || !xq ||
            moe_token(s, x, ffn_norm, router, bias, blobs, idx, w, logits, xn, scratch, xq,
                      nthreads))
            rc = 1;
        free(scratch);
        free(xq);
        return rc ? -1 : 0;
    }
    /* Tokens are independent (the reference steps them one at a time), so
     * threads over tokens change no bits. */
#pragma omp parallel num_threads(nthreads) reduction(| : rc)
    {
        float *scratch = malloc(sizeof(float) * (size_t)scratch_floats(s));
        orc_block_q8 *xq = malloc(sizeof(orc_block_q8) * (size_t)(maxd / ORC_QK));
        if (!scratch || !xq) rc |= 1;
#pragma omp for schedule(dynamic, 1)
        for (int t = 0; t < T; t++) {
            if (!scratch || !xq) continue;
            if (moe_token(s, x + (size_t)t * d, ffn_norm, router, bias, blobs,
                          idx ? idx + (size_t)t * K : NULL, w ? w + (size_t)t * K : NULL,
                          logits ? logits + (size_t)t * E : NULL,
                          xn ? xn + (size_t)t * d : NULL, scratch, xq, 1))
                rc |= 1;
        }
        free(scratch);
        free(xq);
    }
    return rc ? -1 : 0;
}

/* src/model/forward.c:210-213 without the attention call. */
int orc_moe_stack(const orc_dims *s, int L, int T, float *x,
                  const float *ffn_norm, const float *router,
                  const unsigned char *const *blobs, int nthreads) {
    for (int l = 0; l < L; l++) {
        int rc = orc_moe_layer(s, T, x, ffn_norm + (size_t)l * s->dim,
                               router + (size_t)l * s->n_experts * s->dim, NULL,
                               blobs + (size_t)l * s->n_experts, NULL, NULL, NULL, NULL,
                               nthreads);
        if (rc) return rc;
    }
    return 0;
}

/* ---- expert-bucketed restatement of the same layer (a checker for large T) ----
 *
 * orc_moe_layer_bucketed computes, for every (token, weight row), the same
 * sequential chain as dot_q8 and every other value in the same order as
 * moe_token; only the loop nest differs: tokens are grouped by expert (the
 * stable bucketing of orc_dispatch) and each weight row meets 16 tokens of
 * its bucket at once. The block dot is accumulated in float: every partial
 * sum of 32 products of two int8 codes is an integer below 2^24, so it is
 * exact in any order and equals (float) of the int32 dot. Pinned bit-equal to
 * orc_moe_layer by tests/test_oracle.py. */
typedef float orc_v16 __attribute__((vector_size(64)));

/* out[r * ostride + t] for the four consecutive Q8_0 weight rows w (nb
 * blocks each) against tokens t < n of a bucket held transposed:
 * xf[(32 k + i) * tp + t] = code i of block k of token t (as float; zero for
 * t >= n), xs[k * tp + t] its scale; tp is a multiple of 16. */
__attribute__((target_clones("avx512f", "avx2", "default")))
static void rows4_bucket(const orc_block_q8 *w, int nb, const float *xf, const float *xs,
                         int tp, int n, float *out, int ostride) {
    for (int t0 = 0; t0 < n; t0 += 16) {
        orc_v16 s0 = {0}, s1 = {0}, s2 = {0}, s3 = {0};
        for (int k = 0; k < nb; k++) {
            orc_v16 a0 = {0}, a1 = {0}, a2 = {0}, a3 = {0};
            const float *xk = xf + (size_t)k * ORC_QK * tp + t0;
            const orc_block_q8 *w0 = w + k, *w1 = w + nb + k, *w2 = w + 2 * nb + k,
                               *w3 = w + 3 * nb + k;
            for (int i = 0; i < ORC_QK; i++) {
                orc_v16 xv;
                memcpy(&xv, xk + (size_t)i * tp, sizeof xv);
                a0 = a0 + (float)w0->q[i] * xv;
                a1 = a1 + (float)w1->q[i] * xv;
                a2 = a2 + (float)w2->q[i] * xv;
                a3 = a3 + (float)w3->q[i] * xv;
            }
            orc_v16 sv;
            memcpy(&sv, xs + (size_t)k * tp + t0, sizeof sv);
            s0 = s0 + (a0 * w0->d) * sv;
            s1 = s1 + (a1 * w1->d) * sv;
            s2 = s2 + (a2 * w2->d) * sv;
            s3 = s3 + (a3 * w3->d) * sv;
        }
        for (int t = 0; t < 16 && t0 + t < n; t++) {
            out[t0 + t] = s0[t];
            out[(size_t)ostride + t0 + t] = s1[t];
            out[2 * (size_t)ostride + t0 + t] = s2[t];
            out[3 * (size_t)ostride + t0 + t] = s3[t];
        }
    }
}

/* Q8_0 (quant.c:11-27) of the 32-values blocks of column t of v[rows][tp]
 * (rows a multiple of 32), in place: v receives the codes as floats, sc[k *
 * tp + t] the block scales. */
static void quant_column(float *v, float *sc, int rows, int tp, int t) {
    float blk[ORC_QK];
    orc_block_q8 q;
    for (int k = 0; k < rows / ORC_QK; k++) {
        for (int i = 0; i < ORC_QK; i++) blk[i] = v[(size_t)(k * ORC_QK + i) * tp + t];
        orc_quantize_row_q8(blk, &q, ORC_QK);
        for (int i = 0; i < ORC_QK; i++) v[(size_t)(k * ORC_QK + i) * tp + t] = (float)q.q[i];
        sc[(size_t)k * tp + t] = q.d;
    }
}

/* rmsnorm, router chains (+bias), softmax/top-K/gate weights of T tokens
 * (forward.c:75-81,175-181); xn[T][d] receives the rmsnorm output. The E
 * chains of a token advance together over the transposed router, each in the
 * reference's order (a rounded product, then a rounded add). */
static int route_phase(const orc_dims *s, int T, const float *x, const float *ffn_norm,
                       const float *router, const float *bias, float *xn, int *idx, float *w,
                       float *logits_out, int nthreads) {
    const int d = s->dim, E = s->n_experts, K = s->n_active;
    int rc = 0;
    float *wt = malloc(sizeof(float) * (size_t)d * E);
    if (!wt) return -1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int i = 0; i < d; i++)
        for (int e = 0; e < E; e++) wt[(size_t)i * E + e] = router[(size_t)e * d + i];
#pragma omp parallel num_threads(nthreads) reduction(| : rc)
    {
        float *lg = malloc(sizeof(float) * (size_t)E);
        if (!lg) rc |= 1;
#pragma omp for schedule(static)
        for (int t = 0; t < T; t++) {
            if (!lg) continue;
            float *xt = xn + (size_t)t * d;
            orc_rmsnorm(xt, x + (size_t)t * d, ffn_norm, d, s->norm_eps);
            for (int e = 0; e < E; e++) lg[e] = 0.0f;
            for (int i = 0; i < d; i++) {
                const float xv = xt[i];
                const float *wr = wt + (size_t)i * E;
                for (int e = 0; e < E; e++) lg[e] = lg[e] + wr[e] * xv;
            }
            if (bias)
                for (int e = 0; e < E; e++) lg[e] = lg[e] + bias[e];
            if (logits_out) memcpy(logits_out + (size_t)t * E, lg, sizeof(float) * (size_t)E);
            orc_route(lg, E, K, s->norm_topk, idx + (size_t)t * K, w + (size_t)t * K);
        }
        free(lg);
    }
    free(wt);
    return rc ? -1 : 0;
}

int orc_route_tokens(const orc_dims *s, int T, const float *x, const float *ffn_norm,
                     const float *router, const float *bias, int *idx, float *w,
                     float *logits, int nthreads) {
    if (s->n_active > 64 || T < 0) return -1;
    if (T == 0) return 0;
    float *xn = malloc(sizeof(float) * (size_t)T * s->dim);
    if (!xn) return -1;
    const int rc = route_phase(s, T, x, ffn_norm, router, bias, xn, idx, w, logits,
                               nthreads < 1 ? 1 : nthreads);
    free(xn);
    return rc;
}

int orc_moe_layer_bucketed(const orc_dims *s, int T, float *x, const float *ffn_norm,
                           const float *router, const float *bias,
                           const unsigned char *const *blobs, int *idx_out, float *w_out,
                           float *logits_out, int nthreads) {
    const int d = s->dim, E = s->n_experts, K = s->n_active, eh = s->expert_hidden;
    const int nb = d / ORC_QK, A = T * K;
    if (K > 64 || d % ORC_QK || eh % ORC_QK || T < 0) return -1;
    if (T == 0) return 0;
    if (nthreads < 1) nthreads = 1;
    const size_t off_up = orc_off_up(s), off_down = orc_off_down(s);
    int rc = 0;
    float *xn = malloc(sizeof(float) * (size_t)T * d);
    int *idx = malloc(sizeof(int) * (size_t)A);
    float *w = malloc(sizeof(float) * (size_t)A);
    int *counts = malloc(sizeof(int) * (size_t)E), *offsets = malloc(sizeof(int) * (size_t)(E + 1));
    int *perm = malloc(sizeof(int) * (size_t)A), *pos = malloc(sizeof(int) * (size_t)A);
    size_t *boff = malloc(sizeof(size_t) * (size_t)(E + 1));
    int *tps = malloc(sizeof(int) * (size_t)E);
    float *xf = NULL, *xs = NULL, *gu = NULL, *hs = NULL, *tmp = NULL;
    if (!xn || !idx || !w || !counts || !offsets || !perm || !pos || !boff || !tps) {
        rc = -1;
        goto out;
    }
    rc = route_phase(s, T, x, ffn_norm, router, bias, xn, idx, w, logits_out, nthreads);
    if (rc || orc_dispatch(idx, T, K, E, counts, offsets, perm, pos)) {
        rc = -1;
        goto out;
    }
    if (idx_out) memcpy(idx_out, idx, sizeof(int) * (size_t)A);
    if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)A);
    boff[0] = 0;
    for (int e = 0; e < E; e++) {
        if (counts[e] && !blobs[e]) rc = -1; /* a cache miss whose load failed */
        tps[e] = (counts[e] + 15) / 16 * 16;
        boff[e + 1] = boff[e] + (size_t)tps[e];
    }
    if (rc) goto out;
    const size_t cols = boff[E];
    xf = calloc((size_t)d * cols, sizeof(float));
    xs = calloc((size_t)nb * cols, sizeof(float));
    gu = calloc((size_t)2 * eh * cols, sizeof(float));
    hs = calloc((size_t)(eh / ORC_QK) * cols, sizeof(float));
    tmp = calloc((size_t)d * cols, sizeof(float));
    if (!xf || !xs || !gu || !hs || !tmp) {
        rc = -1;
        goto out;
    }
    /* each bucket's Q8(xn) rows, transposed; bucket e's columns start at
     * boff[e] of a d x cols array, so a bucket's column stride is cols */
#pragma omp parallel num_threads(nthreads)
    {
        orc_block_q8 *q = malloc(sizeof(orc_block_q8) * (size_t)nb);
#pragma omp for schedule(dynamic, 1)
        for (int e = 0; e < E; e++) {
            if (!q) continue;
            for (int a = 0; a < counts[e]; a++) {
                const int t = perm[offsets[e] + a] / K;
                orc_quantize_row_q8(xn + (size_t)t * d, q, d);
                const size_t c = boff[e] + (size_t)a;
                for (int k = 0; k < nb; k++) {
                    xs[(size_t)k * cols + c] = q[k].d;
                    for (int i = 0; i < ORC_QK; i++)
                        xf[(size_t)(k * ORC_QK + i) * cols + c] = (float)q[k].q[i];
                }
            }
        }
        if (!q) rc = -1;
        free(q);
    }
    if (rc) goto out;
    /* gate/up rows (gate in gu[0..eh), up in gu[eh..2eh)), 32 rows per task */
    {
        const int chunks = 2 * eh / 32;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1) collapse(2)
        for (int e = 0; e < E; e++)
            for (int c = 0; c < chunks; c++) {
                if (!counts[e]) continue;
                const int r0 = c * 32, mat = r0 / eh, rr = r0 % eh;
                const orc_block_q8 *wm =
                    (const orc_block_q8 *)(blobs[e] + (mat ? off_up : 0)) + (size_t)rr * nb;
                for (int r = 0; r < 32; r += 4)
                    rows4_bucket(wm + (size_t)r * nb, nb, xf + boff[e], xs + boff[e], (int)cols,
                                 counts[e], gu + (size_t)(r0 + r) * cols + boff[e], (int)cols);
            }
    }
    /* SwiGLU (forward.c:189-191), then Q8(h) per assignment: the codes
     * replace h in gu[0..eh) */
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 16)
    for (int a = 0; a < A; a++) {
        const int e = idx[perm[a]];
        const int c = (int)boff[e] + (a - offsets[e]);
        for (int r = 0; r < eh; r++) {
            const float g = gu[(size_t)r * cols + c];
            gu[(size_t)r * cols + c] = (g / (1.0f + expf(-g))) * gu[(size_t)(eh + r) * cols + c];
        }
        quant_column(gu, hs, eh, (int)cols, c);
    }
    /* down rows, 32 per task */
    {
        const int chunks = d / 32, nbh = eh / ORC_QK;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1) collapse(2)
        for (int e = 0; e < E; e++)
            for (int c = 0; c < chunks; c++) {
                if (!counts[e]) continue;
                const orc_block_q8 *wm = (const orc_block_q8 *)(blobs[e] + off_down) +
                                         (size_t)c * 32 * nbh;
                for (int r = 0; r < 32; r += 4)
                    rows4_bucket(wm + (size_t)r * nbh, nbh, gu + boff[e], hs + boff[e],
                                 (int)cols, counts[e],
                                 tmp + (size_t)(c * 32 + r) * cols + boff[e], (int)cols);
            }
    }
    /* combine (forward.c:194): x_i = x_i + w_j * tmp_j,i, j in top-K order */
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int t = 0; t < T; t++)
        for (int j = 0; j < K; j++) {
            const int a = pos[t * K + j], e = idx[t * K + j];
            const size_t c = boff[e] + (size_t)(a - offsets[e]);
            const float wj = w[t * K + j];
            float *xt = x + (size_t)t * d;
            for (int i = 0; i < d; i++) xt[i] = xt[i] + wj * tmp[(size_t)i * cols + c];
        }
out:
    free(xn);
    free(idx);
    free(w);
    free(counts);
    free(offsets);
    free(perm);
    free(pos);
    free(boff);
    free(tps);
    free(xf);
    free(xs);
    free(gu);
    free(hs);
    free(tmp);
    return rc;
}

/* ---- one whole model step (src/model/forward.c:118-165,199-217) ---------- */

/* forward.c:84-93: NeoX rotary embedding (element i pairs with i + hd/2),
 * angles and rotation in double, each element rounded to float once. */
static void orc_rope(float *x, int hd, int pos, float theta) {
    const int half = hd / 2;
    for (int i = 0; i < half; i++) {
        const double freq = pow((double)theta, -2.0 * i / hd);
        const double a = pos * freq, c = cos(a), sn = sin(a);
        const float x0 = x[i], x1 = x[i + half];
        x[i] = (float)(x0 * c - x1 * sn);
        x[i + half] = (float)(x0 * sn + x1 * c);
    }
}

void orc_rope_row(float *x, int hd, int pos, float theta) { orc_rope(x, hd, pos, theta); }

/* forward.c:118-165: attention of the token at `pos` for layer l, in place
 * on x; the layer's K and V rows are written to kc/vc[pos]. */
static int orc_attention(const orc_model *m, int l, int pos, float *x, float *kc, float *vc) {
    const int d = m->moe.dim, hd = m->head_dim, nh = m->n_heads, nkv = m->n_kv_heads;
    const int qd = nh * hd, kvd = nkv * hd;
    const float eps = m->moe.norm_eps;
    const int maxd = d > qd ? d : qd;
    float *xn = malloc(sizeof(float) * (size_t)d), *q = malloc(sizeof(float) * (size_t)qd);
    float *k = malloc(sizeof(float) * (size_t)kvd), *v = malloc(sizeof(float) * (size_t)kvd);
    float *att = malloc(sizeof(float) * (size_t)qd), *tmp = malloc(sizeof(float) * (size_t)d);
    float *scores = malloc(sizeof(float) * (size_t)(pos + 1));
    orc_block_q8 *xq = malloc(sizeof(orc_block_q8) * (size_t)(maxd / ORC_QK));
    int rc = 0;
    if (!xn || !q || !k || !v || !att || !tmp || !scores || !xq) {
        rc = -1;
        goto out;
    }
    orc_rmsnorm(xn, x, m->attn_norm[l], d, eps);
    orc_matvec(q, m->wq[l], m->wtype, xn, xq, qd, d);
    orc_matvec(k, m->wk[l], m->wtype, xn, xq, kvd, d);
    orc_matvec(v, m->wv[l], m->wtype, xn, xq, kvd, d);
    for (int h = 0; h < nh; h++) {
        orc_rmsnorm(q + h * hd, q + h * hd, m->q_norm[l], hd, eps);
        orc_rope(q + h * hd, hd, pos, m->rope_theta);
    }
    for (int h = 0; h < nkv; h++) {
        orc_rmsnorm(k + h * hd, k + h * hd, m->k_norm[l], hd, eps);
        orc_rope(k + h * hd, hd, pos, m->rope_theta);
    }
    memcpy(kc + (size_t)pos * kvd, k, sizeof(float) * (size_t)kvd);
    memcpy(vc + (size_t)pos * kvd, v, sizeof(float) * (size_t)kvd);
    const int group = nh / nkv;
    const float scale = 1.0f / sqrtf((float)hd);
    for (int h = 0; h < nh; h++) {
        const float *qh = q + h * hd;
        const int kvh = h / group;
        for (int t = 0; t <= pos; t++) {
            const float *kt = kc + (size_t)t * kvd + kvh * hd;
            float dot = 0.0f;
            for (int i = 0; i < hd; i++) dot = dot + qh[i] * kt[i];
            scores[t] = dot * scale;
        }
        orc_softmax(scores, pos + 1);
        float *o = att + h * hd;
        for (int i = 0; i < hd; i++) o[i] = 0.0f;
        for (int t = 0; t <= pos; t++) {
            const float *vt = vc + (size_t)t * kvd + kvh * hd;
            for (int i = 0; i < hd; i++) o[i] = o[i] + scores[t] * vt[i];
        }
    }
    orc_matvec(tmp, m->wo[l], m->wtype, att, xq, d, qd);
    for (int i = 0; i < d; i++) x[i] = x[i] + tmp[i];
out:
    free(xn);
    free(q);
    free(k);
    free(v);
    free(att);
    free(tmp);
    free(scores);
    free(xq);
    return rc;
}

int orc_model_step(const orc_model *m, float *kc, float *vc, int max_seq, int token, int pos,
                   float *logits, float *x_out, int nthreads) {
    const int d = m->moe.dim, E = m->moe.n_experts, V = m->vocab;
    const int kvd = m->n_kv_heads * m->head_dim;
    if (pos < 0 || pos >= max_seq || token < 0 || token >= V || m->wtype != ORC_Q8_0) return -1;
    const int maxd = d > m->moe.expert_hidden ? d : m->moe.expert_hidden;
    float *x = malloc(sizeof(float) * (size_t)d), *xn = malloc(sizeof(float) * (size_t)d);
    float *scratch = malloc(sizeof(float) * (size_t)scratch_floats(&m->moe));
    orc_block_q8 *xq = malloc(sizeof(orc_block_q8) * (size_t)(maxd / ORC_QK));
    int rc = 0;
    if (!x || !xn || !scratch || !xq) {
        rc = -1;
        goto out;
    }
    /* forward.c:205-208: the token's embedding row, dequantized */
    orc_dequantize_row(m->wtype,
                       (const unsigned char *)m->token_embd +
                           (size_t)token * orc_row_bytes(m->wtype, d),
                       x, d);
    for (int l = 0; l < m->n_layers && !rc; l++) {
        const size_t off = (size_t)l * max_seq * kvd;
        rc = orc_attention(m, l, pos, x, kc + off, vc + off);
        if (!rc)
            rc = moe_token(&m->moe, x, m->ffn_norm[l], m->router[l], NULL,
                           m->blobs + (size_t)l * E, NULL, NULL, NULL, NULL, scratch, xq,
                           nthreads);
    }
    if (rc) goto out;
    if (x_out) memcpy(x_out, x, sizeof(float) * (size_t)d);
    /* forward.c:214-215: final norm and output head */
    orc_rmsnorm(xn, x, m->output_norm, d, m->moe.norm_eps);
    float *hq = malloc(sizeof(orc_block_q8) * (size_t)(d / ORC_QK));
    if (!hq) {
        rc = -1;
        goto out;
    }
    matvec_mt(logits, m->output, m->wtype, xn, (orc_block_q8 *)hq, V, d, nthreads);
    free(hq);
out:
    free(x);
    free(xn);
    free(scratch);
    free(xq);
    return rc;
}

int orc_dispatch(const int *idx, int T, int K, int E, int *counts,
                 int *offsets, int *perm, int *pos) {
    const int A = T * K;
    if (E <= 0 || T < 0 || K < 0) return -1;
    for (int e = 0; e < E; e++) counts[e] = 0;
    for (int a = 0; a < A; a++) {
        if (idx[a] < 0 || idx[a] >= E) return -1;
        counts[idx[a]]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < E; e++) offsets[e + 1] = offsets[e] + counts[e];
    int *fill = calloc((size_t)E, sizeof(int));
    if (!fill) return -1;
    for (int a = 0; a < A; a++) {
        int e = idx[a];
        int p = offsets[e] + fill[e]++;
        perm[p] = a;
        if (pos) pos[a] = p;
    }
    free(fill);
    return 0;
}

void orc_synth_x(uint64_t seed, int T, int dim, float *x) {
    uint64_t key = mia_synth_key(seed, MIA_STREAM_X);
    for (size_t i = 0; i < (size_t)T * dim; i++) x[i] = mia_synth_f32(key, i, 1.0);
}

void orc_synth_router(uint64_t seed, int layer, const orc_dims *s, float *w) {
    uint64_t key = mia_synth_key(seed, MIA_STREAM_ROUTER + (uint64_t)layer);
    for (size_t i = 0; i < (size_t)s->n_experts * s->dim; i++)
        w[i] = mia_synth_f32(key, i, 0.02);
}

/* One expert in the reference blob format: gate [eh x d] at 0, up at off_up,
 * down [d x eh] at off_down, every row quantized with orc_quantize_row_q8
 * (the converter's QuantizeRowQ8, tools/internal/mia/format.go:67-89). */
void orc_synth_expert_blob(uint64_t seed, int layer, int expert,
                           const orc_dims *s, unsigned char *blob) {
    const int d = s->dim, eh = s->expert_hidden;
    const size_t offs[3] = {0, orc_off_up(s), orc_off_down(s)};
    memset(blob, 0, orc_blob_bytes(s));
    if (d > 8192 || eh > 8192) return;
    for (int m = 0; m < 3; m++) {
        int rows = m < 2 ? eh : d, cols = m < 2 ? d : eh;
        uint64_t key = mia_synth_key(
            seed, MIA_STREAM_EXPERT + ((uint64_t)layer * s->n_experts + expert) * 3 + m);
        size_t rb = orc_row_bytes(ORC_Q8_0, cols);
#pragma omp parallel for schedule(static)
        for (int r = 0; r < rows; r++) {
            float row[8192];
            for (int c = 0; c < cols; c++)
                row[c] = mia_synth_f32(key, (uint64_t)r * cols + c, 0.02);
            orc_quantize_row_q8(row, (orc_block_q8 *)(blob + offs[m] + rb * r), cols);
        }
    }
}

/* ---- token sampler (src/tokenizer/sampler.c) ------------------------------------ */

void orc_sampler_init(orc_sampler *s, float temperature, float top_p, int n, uint64_t seed) {
    s->temperature = temperature;
    s->top_p = (top_p > 0.0f && top_p <= 1.0f) ? top_p : 1.0f;
    s->n = n;
    s->rng = seed ? seed : 0x2545F4914F6CDD1DULL;
}

/* xorshift64* (shifts 12, 25, 27; multiplier 2685821657736338717), the top
 * 24 bits of the product over 2^24 */
float orc_sampler_rand01(orc_sampler *s) {
    uint64_t x = s->rng;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    s->rng = x;
    return (float)((x * 0x2545F4914F6CDD1DULL) >> 40) / 16777216.0f;
}

typedef struct {
    float p;
    int i;
} orc_cand;

static int cand_order(const void *a, const void *b) {
    const orc_cand *x = a, *y = b;
    if (x->p != y->p) return x->p > y->p ? -1 : 1;
    return (x->i > y->i) - (x->i < y->i);
}

int orc_sample(orc_sampler *s, const float *logits) {
    const int n = s->n;
    int best = 0;
    for (int i = 1; i < n; i++)
        if (logits[i] > logits[best]) best = i;
    if (s->temperature <= 0.0f) return best;
    float *e = malloc(sizeof(float) * (size_t)n);
    orc_cand *c = malloc(sizeof(orc_cand) * (size_t)n);
    if (!e || !c) {
        free(e);
        free(c);
        return -1;
    }
    /* :42-44: e_i = expf((l_i - max) / T), summed in index order */
    const float mx = logits[best];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        e[i] = expf((logits[i] - mx) / s->temperature);
        sum = sum + e[i];
    }
    /* :46-51: candidates p >= (1 - top_p) / (n - 1) */
    const float cutoff = (1.0f - s->top_p) / (float)(n > 1 ? n - 1 : 1);
    int m = 0;
    for (int i = 0; i < n; i++) {
        const float p = e[i] / sum;
        if (p >= cutoff) {
            c[m].p = p;
            c[m].i = i;
            m++;
        }
    }
    /* :53-66: the shortest prefix whose running sum reaches top_p; r in
     * [0, cum); the first candidate whose running sum exceeds r. The draw
     * is taken even with no candidate (the state advances as the
     * reference's does). */
    if (m > 0) qsort(c, (size_t)m, sizeof(orc_cand), cand_order);
    float cum = 0.0f;
    int last = m - 1;
    for (int i = 0; i < m; i++) {
        cum = cum + c[i].p;
        if (cum >= s->top_p) {
            last = i;
            break;
        }
    }
    const float r = orc_sampler_rand01(s) * cum;
    int tok = m > 0 ? c[last].i : best;
    float acc = 0.0f;
    for (int i = 0; i <= last; i++) {
        acc = acc + c[i].p;
        if (r < acc) {
            tok = c[i].i;
            break;
        }
    }
    free(e);
    free(c);
    return tok;
}
