/* Accessors of the mia_moe handle shared by the host sources of the
 * library (not exported). */
#ifndef MIA_MOE_INTERNAL_H
#define MIA_MOE_INTERNAL_H
#include "mia/moe.h"

#define MIA_INTERNAL __attribute__((visibility("hidden")))

/* Sets the handle's error message; returns -1. */
MIA_INTERNAL int mia_moe_fail(mia_moe *m, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
/* The HBM table (layer 0, expert 0) and the shape the handle was opened with. */
MIA_INTERNAL void *mia_moe_table(mia_moe *m);
MIA_INTERNAL const mia_moe_config *mia_moe_cfg(const mia_moe *m);

/* Device tensors of the handle (decode-stack arguments for one layer). */
typedef struct {
    const void *table;       /* layer 0, expert 0 */
    const float *router_dl;  /* [L][E][dim], decode layout */
    const float *router_t;   /* [L][dim][E] */
    const float *norm;       /* [L][dim] */
    mhip_layout lay;
    mhip_dims dims;
} mia_moe_tensors;
MIA_INTERNAL void mia_moe_get_tensors(const mia_moe *m, mia_moe_tensors *t);

/* Offsets (from dense_offset) of one layer's dense tensors and of the
 * model-wide ones, in the converter's order (NewLayout). */
typedef struct {
    uint64_t attn_norm, wq, wk, wv, wo, q_norm, k_norm, ffn_norm, router;
} mia_layer_offsets;
/* Walks the dense section; fills lo for `layer` (when not NULL) and the
 * model-wide offsets (when not NULL); returns the section's end. */
MIA_INTERNAL uint64_t mia_dense_walk(const mia_file_info *h, int layer, mia_layer_offsets *lo,
                                     uint64_t *token_embd, uint64_t *output_norm,
                                     uint64_t *output);

#endif
