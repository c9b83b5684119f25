/*
 * The reference's Q8_0 tensor ops (include/mia/quant.h, include/mia/matmul.h)
 * with their host-pointer interface, executed by the HIP kernels of
 * include/mia_hip.h on a lazily opened context of device 0 (or
 * $MIA_DEVICE). The functions return void in the reference interface, so a
 * GPU failure is recorded for mia_tensor_error (include/mia/tensor_error.h)
 * and the call's outputs are filled with NaN; with $MIA_ABORT_ON_GPU_ERROR
 * set the process aborts instead. Matrices registered with
 * mia_matvec_register (include/mia/matvec_cache.h) stay in HBM.
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mia/matmul.h"
#include "mia/matvec_cache.h"
#include "mia/quant.h"
#include "mia/tensor_error.h"
#include "mia_hip.h"

static mhip_ctx *g_ctx;
static void *g_buf[4];
static size_t g_cap[4];
static char g_err[512];       /* the first failure not yet read */
static unsigned g_nerr;       /* failures since the last mia_tensor_error */

/* Registered (device-resident) matrices, keyed by host pointer. */
typedef struct {
    const void *w;
    mia_wtype t;
    int rows, cols;
    void *d_w;
} resident;
static resident *g_res;
static int g_nres, g_capres;

/* Records a failure (the first one until it is read), or aborts when the
 * caller asked for that. */
static void record(const char *fmt, ...) {
    char msg[sizeof g_err];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    if (getenv("MIA_ABORT_ON_GPU_ERROR")) {
        fprintf(stderr, "motoria: %s\n", msg);
        abort();
    }
    if (g_nerr++ == 0) memcpy(g_err, msg, sizeof g_err);
}

static void fail(const char *what) {
    record("%s: %s", what, g_ctx ? mhip_error(g_ctx) : "no GPU context");
}

static void fill_nan(float *p, size_t n) {
    for (size_t i = 0; i < n; i++) p[i] = NAN;
}

/* The context, or NULL (recorded) when no GPU can be opened. */
static mhip_ctx *ctx(void) {
    if (!g_ctx) {
        char err[256];
        const char *dev = getenv("MIA_DEVICE");
        if (mhip_open(&g_ctx, dev ? atoi(dev) : 0, err, sizeof(err)) != 0) {
            g_ctx = NULL;
            record("cannot open a GPU for the tensor ops: %s", err);
        }
    }
    return g_ctx;
}

/* Grow-only device staging buffer number `i`, or NULL (recorded). */
static void *buf(int i, size_t bytes) {
    if (bytes > g_cap[i]) {
        if (g_buf[i]) mhip_free(g_ctx, g_buf[i]);
        g_cap[i] = 0;
        g_buf[i] = mhip_malloc(g_ctx, bytes);
        if (!g_buf[i]) {
            fail("device staging buffer");
            return NULL;
        }
        g_cap[i] = bytes;
    }
    return g_buf[i];
}

const char *mia_tensor_error(void) {
    static char out[sizeof g_err + 64];
    if (!g_nerr) return NULL;
    if (g_nerr > 1)
        snprintf(out, sizeof out, "%s (and %u more failures)", g_err, g_nerr - 1);
    else
        snprintf(out, sizeof out, "%s", g_err);
    g_nerr = 0;
    return out;
}

size_t mia_row_bytes(mia_wtype t, int cols) {
    if (t == MIA_Q8_0) return (size_t)(cols / MIA_QK) * sizeof(mia_block_q8);
    return (size_t)cols * sizeof(float);
}

void mia_quantize_row_q8(const float *x, mia_block_q8 *y, int n) {
    if (n < MIA_QK) return;
    const int nb = n / MIA_QK;
    const size_t xb = (size_t)nb * MIA_QK * sizeof(float), yb = (size_t)nb * sizeof(mia_block_q8);
    mhip_ctx *c = ctx();
    float *dx = c ? buf(0, xb) : NULL;
    void *dy = dx ? buf(1, yb) : NULL;
    if (!dy || mhip_h2d(c, dx, x, xb) || mhip_quantize_q8(c, dx, dy, nb * MIA_QK) ||
        mhip_d2h(c, y, dy, yb)) {
        if (c && dy) fail("quantize_row_q8");
        for (int b = 0; b < nb; b++) {
            y[b].d = NAN;
            memset(y[b].q, 0, sizeof y[b].q);
        }
    }
}

void mia_dequantize_row(mia_wtype t, const void *src, float *dst, int n) {
    if (n <= 0) return;
    if (t == MIA_F32) { /* a copy, as src/tensor/quant.c:30-33 */
        memcpy(dst, src, sizeof(float) * (size_t)n);
        return;
    }
    const int nb = n / MIA_QK;
    if (!nb) return;
    mhip_ctx *c = ctx();
    const size_t sb = (size_t)nb * sizeof(mia_block_q8), db = (size_t)nb * MIA_QK * sizeof(float);
    void *ds = c ? buf(1, sb) : NULL;
    float *dd = ds ? buf(0, db) : NULL;
    if (!dd || mhip_h2d(c, ds, src, sb) || mhip_dequantize_q8(c, ds, dd, nb * MIA_QK) ||
        mhip_d2h(c, dst, dd, db)) {
        if (c && dd) fail("dequantize_row");
        fill_nan(dst, (size_t)nb * MIA_QK);
    }
}

static int find_resident(const void *w) {
    for (int i = 0; i < g_nres; i++)
        if (g_res[i].w == w) return i;
    return -1;
}

int mia_matvec_register(const void *w, mia_wtype t, int rows, int cols) {
    if (!w || rows <= 0 || cols <= 0 || (t != MIA_F32 && t != MIA_Q8_0) ||
        (t == MIA_Q8_0 && cols % MIA_QK))
        return -1;
    mia_matvec_unregister(w);
    if (g_nres == g_capres) {
        const int cap = g_capres ? 2 * g_capres : 16;
        resident *r = realloc(g_res, sizeof(resident) * (size_t)cap);
        if (!r) return -1;
        g_res = r;
        g_capres = cap;
    }
    mhip_ctx *c = ctx();
    if (!c) return -1;
    const size_t wb = (size_t)rows * mia_row_bytes(t, cols);
    void *d = mhip_malloc(c, wb);
    if (!d) return -1;
    if (mhip_h2d(c, d, w, wb)) {
        mhip_free(c, d);
        return -1;
    }
    g_res[g_nres++] = (resident){w, t, rows, cols, d};
    return 0;
}

int mia_matvec_unregister(const void *w) {
    const int i = find_resident(w);
    if (i < 0) return -1;
    mhip_free(g_ctx, g_res[i].d_w);
    g_res[i] = g_res[--g_nres];
    return 0;
}

void mia_matvec(float *out, const void *w, mia_wtype t, const float *x, mia_block_q8 *xq,
                int rows, int cols) {
    if (rows <= 0) return;
    mhip_ctx *c = ctx();
    const size_t wb = (size_t)rows * mia_row_bytes(t, cols);
    const size_t xb = (size_t)cols * sizeof(float);
    const size_t qb = t == MIA_Q8_0 ? (size_t)(cols / MIA_QK) * sizeof(mia_block_q8) : 0;
    /* a registered matrix of this type and shape is read from HBM */
    const int r = find_resident(w);
    const int hit = r >= 0 && g_res[r].t == t && g_res[r].rows == rows && g_res[r].cols == cols;
    void *dw = !c ? NULL : hit ? g_res[r].d_w : buf(0, wb);
    float *dx = dw ? buf(1, xb ? xb : 4) : NULL;
    void *dq = dx ? buf(2, qb ? qb : 4) : NULL;
    float *dout = dq ? buf(3, (size_t)rows * sizeof(float)) : NULL;
    if (!dout || (!hit && mhip_h2d(c, dw, w, wb)) || mhip_h2d(c, dx, x, xb) ||
        mhip_matvec(c, dout, dw, (int)t, dx, dq, rows, cols) ||
        mhip_d2h(c, out, dout, (size_t)rows * sizeof(float)) ||
        (qb && xq && mhip_d2h(c, xq, dq, qb))) {
        if (dout) fail("matvec");
        fill_nan(out, (size_t)rows);
    }
}

void mia_matvec_scalar(float *out, const void *w, mia_wtype t, const float *x,
                       mia_block_q8 *xq, int rows, int cols) {
    mia_matvec(out, w, t, x, xq, rows, cols);
}
