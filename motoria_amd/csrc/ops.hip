// The reference's Q8_0 tensor ops (include/mia/quant.h:18-21,
// include/mia/matmul.h:11-16) on device pointers, in the reference's 36-byte
// block format. Results are bit-equal to its scalar x86 kernels
// (src/tensor/quant.c:11-38, src/tensor/matmul.c:13-28): the int8 block dot
// is exact, and every fp32 sum runs in the reference's order.
#include "mhip_internal.h"

namespace {

constexpr int QK = mhip::QK;

// One thread per block: src/tensor/quant.c:11-27.
__global__ __launch_bounds__(256) void k_quantize_ref(const float *x, uint8_t *y, int nblocks) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *v = x + (size_t)b * QK;
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) {
        float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    const float dsc = amax / 127.0f;
    const float inv = dsc != 0.0f ? 1.0f / dsc : 0.0f;
    uint32_t *dst = (uint32_t *)(y + (size_t)b * 36);
    dst[0] = __float_as_uint(dsc);
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
        for (int k = 0; k < 4; k++) {
            int8_t q = (int8_t)roundf(v[w * 4 + k] * inv);
            word |= (uint32_t)(uint8_t)q << (8 * k);
        }
        dst[1 + w] = word;
    }
}

// src/tensor/quant.c:29-38
__global__ __launch_bounds__(256) void k_dequantize_ref(const uint8_t *y, float *x, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint8_t *blk = y + (size_t)(i / QK) * 36;
    const float dsc = __uint_as_float(*(const uint32_t *)blk);
    x[i] = dsc * (float)(int8_t)blk[4 + i % QK];
}

// src/tensor/matmul.c:13-17: one thread per row, products and adds rounded
// one at a time, i ascending.
__global__ __launch_bounds__(256) void k_matvec_f32(float *out, const float *w, const float *x,
                                                    int rows, int cols) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float *wr = w + (size_t)r * cols;
    float s = 0.0f;
    for (int i = 0; i < cols; i++) s = s + wr[i] * x[i];
    out[r] = s;
}

__device__ __forceinline__ void load_block36(const uint8_t *p, float *d, int4 *c0, int4 *c1) {
    const uint32_t *s = (const uint32_t *)p;
    *d = __uint_as_float(s[0]);
    *c0 = make_int4((int)s[1], (int)s[2], (int)s[3], (int)s[4]);
    *c1 = make_int4((int)s[5], (int)s[6], (int)s[7], (int)s[8]);
}

// src/tensor/matmul.c:19-28,76-80: one thread per row, blocks in order.
__global__ __launch_bounds__(256) void k_matvec_q8_ref(float *out, const uint8_t *w,
                                                       const uint8_t *xq, int rows, int nb) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint8_t *wr = w + (size_t)r * nb * 36;
    float s = 0.0f;
    for (int b = 0; b < nb; b++) {
        float dw, dx;
        int4 w0, w1, x0, x1;
        load_block36(wr + (size_t)b * 36, &dw, &w0, &w1);
        load_block36(xq + (size_t)b * 36, &dx, &x0, &x1);
        s = s + mhip_dev::block_term(mhip_dev::dot32_i8(w0, w1, x0, x1), dw, dx);
    }
    out[r] = s;
}

}  // namespace

extern "C" {

int mhip_quantize_q8(mhip_ctx *c, const float *d_x, void *d_blocks, int n) {
    if (n < 0 || n % QK) return mhip::fail(c, "quantize: n=%d is not a multiple of 32", n);
    if (!n) return 0;
    if (mhip::use_device(c)) return -1;
    const int nb = n / QK;
    k_quantize_ref<<<mhip::blocks_for(nb, 256), 256, 0, c->stream>>>(d_x, (uint8_t *)d_blocks,
                                                                      nb);
    return mhip::check_launch(c, "quantize_q8");
}

int mhip_dequantize_q8(mhip_ctx *c, const void *d_blocks, float *d_x, int n) {
    if (n < 0 || n % QK) return mhip::fail(c, "dequantize: n=%d is not a multiple of 32", n);
    if (!n) return 0;
    if (mhip::use_device(c)) return -1;
    k_dequantize_ref<<<mhip::blocks_for(n, 256), 256, 0, c->stream>>>(
        (const uint8_t *)d_blocks, d_x, n);
    return mhip::check_launch(c, "dequantize_q8");
}

int mhip_matvec(mhip_ctx *c, float *d_out, const void *d_w, int wtype, const float *d_x,
                void *d_xq, int rows, int cols) {
    if (rows < 0 || cols < 0) return mhip::fail(c, "matvec: negative shape");
    if (!rows) return 0;
    if (mhip::use_device(c)) return -1;
    if (wtype == 0) {
        k_matvec_f32<<<mhip::blocks_for(rows, 256), 256, 0, c->stream>>>(
            d_out, (const float *)d_w, d_x, rows, cols);
        return mhip::check_launch(c, "matvec_f32");
    }
    if (wtype != 1) return mhip::fail(c, "matvec: unknown weight type %d", wtype);
    if (cols % QK) return mhip::fail(c, "matvec: cols=%d is not a multiple of 32", cols);
    if (mhip_quantize_q8(c, d_x, d_xq, cols)) return -1;
    k_matvec_q8_ref<<<mhip::blocks_for(rows, 256), 256, 0, c->stream>>>(
        d_out, (const uint8_t *)d_w, (const uint8_t *)d_xq, rows, cols / QK);
    return mhip::check_launch(c, "matvec_q8");
}

}  // extern "C"
