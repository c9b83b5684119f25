#ifndef MIA_QUANT_H
#define MIA_QUANT_H
/*
 * Q8_0 block format and tensor ops: the interface of the reference's
 * include/mia/quant.h:7-21, same names, types and argument meaning.
 *
 * The ops run on the GPU (HIP kernels through include/mia_hip.h) on the
 * default device context; host pointers are copied in and out. There is no
 * CPU implementation. These functions have no error return in the reference
 * interface: a missing or failing GPU fills the outputs with NaN and is
 * reported by mia_tensor_error (include/mia/tensor_error.h).
 */
#include <stddef.h>
#include <stdint.h>

#define MIA_QK 32 /* values per quantization block */

typedef enum { MIA_F32 = 0, MIA_Q8_0 = 1 } mia_wtype;

/* value = d * q, 36 bytes (include/mia/quant.h:11-15 of the reference). */
typedef struct {
    float d;
    int8_t q[MIA_QK];
} mia_block_q8;

/* Bytes of one row of `cols` values (cols % MIA_QK == 0 for Q8_0).
 * Replaces src/tensor/quant.c:6-9. */
size_t mia_row_bytes(mia_wtype t, int cols);

/* Per-block absmax/127 scale, round half away from zero.
 * Replaces src/tensor/quant.c:11-27. */
void mia_quantize_row_q8(const float *x, mia_block_q8 *y, int n);

/* Replaces src/tensor/quant.c:29-38. */
void mia_dequantize_row(mia_wtype t, const void *src, float *dst, int n);

#endif
