#ifndef MIA_MATVEC_CACHE_H
#define MIA_MATVEC_CACHE_H
/*
 * Device-resident weights for mia_matvec (include/mia/matmul.h). No
 * counterpart in the reference, whose matrices stay in host memory: here
 * mia_matvec runs on the GPU and otherwise uploads the whole matrix on every
 * call. A registered matrix is uploaded once; later mia_matvec calls with
 * the same pointer, type and shape read its HBM copy (only x goes over
 * PCIe). The caller promises not to change the registered host bytes until
 * it unregisters them (the engine's dense tensors never change after
 * mia_file_open). Not thread-safe, like the rest of the engine.
 */
#include "mia/quant.h"

#ifdef __cplusplus
extern "C" {
#endif

/* 0, or -1 (bad shape, or the device copy could not be made). Registering
 * the same pointer again replaces its entry. */
int mia_matvec_register(const void *w, mia_wtype t, int rows, int cols);
/* 0 if w was registered (its device copy is freed), -1 otherwise. */
int mia_matvec_unregister(const void *w);

#ifdef __cplusplus
}
#endif
#endif
