#ifndef MIA_MATMUL_H
#define MIA_MATMUL_H
/*
 * out[r] = sum_c W[r][c] * x[c]: the interface of the reference's
 * include/mia/matmul.h:11-16. W is row-major of type `t`; for Q8_0, `xq`
 * receives x quantized to cols/MIA_QK blocks (as in the reference); for F32
 * it may be NULL. Runs on the GPU with results bit-equal to the reference's
 * scalar x86 kernels (src/tensor/matmul.c:13-28). A GPU failure fills `out`
 * with NaN and is reported by mia_tensor_error (include/mia/tensor_error.h).
 */
#include "mia/quant.h"

/* Replaces src/tensor/matmul.c:91-106. */
void mia_matvec(float *out, const void *w, mia_wtype t, const float *x,
                mia_block_q8 *xq, int rows, int cols);

/* Replaces src/tensor/matmul.c:83-87 (same kernel: the GPU path has one
 * summation order, the reference's scalar one). */
void mia_matvec_scalar(float *out, const void *w, mia_wtype t, const float *x,
                       mia_block_q8 *xq, int rows, int cols);

#endif
