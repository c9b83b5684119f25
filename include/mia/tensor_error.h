#ifndef MIA_TENSOR_ERROR_H
#define MIA_TENSOR_ERROR_H
/*
 * Failures of the tensor ops of include/mia/quant.h and include/mia/matmul.h.
 * No counterpart in the reference, whose CPU ops cannot fail: here they run
 * on a GPU, and their reference signatures return void. A failing call
 * (no GPU, a failed copy, allocation or launch) fills its outputs with NaN
 * (a Q8_0 output with NaN scales) and records the failure for this query;
 * with the environment variable MIA_ABORT_ON_GPU_ERROR set, it prints the
 * message and aborts instead. Not thread-safe, like the rest of the engine.
 */
#ifdef __cplusplus
extern "C" {
#endif

/* The first failure since the last call (with the count of later ones), or
 * NULL when every op since then succeeded; reading it clears it. The string
 * stays valid until the next call. */
const char *mia_tensor_error(void);

#ifdef __cplusplus
}
#endif
#endif
