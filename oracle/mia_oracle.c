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

/* src/tensor/matmul.c:66-87,91-106 on x86: quantize x once (Q8), then the
 * scalar row loop. The Apple-only GCD row split does not change any bits. */
void orc_matvec(float *out, const void *w, int wtype, const float *x,
                orc_block_q8 *xq, int rows, int cols) {
    if (wtype == ORC_F32) {
        const float *wf = (const float *)w;
        for (int r = 0; r < rows; r++) out[r] = dot_f32(wf + (size_t)r * cols, x, cols);
        return;
    }
    orc_quantize_row_q8(x, xq, cols);
    const int nb = cols / ORC_QK;
    const orc_block_q8 *wq = (const orc_block_q8 *)w;
    for (int r = 0; r < rows; r++) out[r] = dot_q8(wq + (size_t)r * nb, xq, nb);
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
                     float *scratch, orc_block_q8 *xq) {
    const int d = s->dim, E = s->n_experts, K = s->n_active, eh = s->expert_hidden;
    int idx[64];
    float w[64];
    if (K > 64) return -1;
    float *xn = scratch, *prob = xn + d, *gate = prob + E, *up = gate + eh,
          *tmp = up + eh;

    orc_rmsnorm(xn, x, ffn_norm, d, s->norm_eps);
    orc_matvec(prob, router, ORC_F32, xn, NULL, E, d);
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
        orc_matvec(gate, blob, ORC_Q8_0, xn, xq, eh, d);
        orc_matvec(up, blob + off_up, ORC_Q8_0, xn, xq, eh, d);
        for (int i = 0; i < eh; i++) {
            float g = gate[i];
            gate[i] = (g / (1.0f + expf(-g))) * up[i];
        }
        orc_matvec(tmp, blob + off_down, ORC_Q8_0, gate, xq, d, eh);
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
    /* Tokens are independent (the reference steps them one at a time), so
     * threads over tokens change no bits. */
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) reduction(| : rc)
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
                          xn ? xn + (size_t)t * d : NULL, scratch, xq))
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
