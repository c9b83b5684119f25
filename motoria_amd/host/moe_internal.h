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

#endif
