#ifndef MIA_EXPERT_CACHE_H
#define MIA_EXPERT_CACHE_H
/*
 * Storage port of the reference (include/mia/expert_cache.h:7-8): fills
 * `dst` (one expert blob in the .mia format) with expert (layer, expert) and
 * returns 0 on success. mia_file_read_expert (src/storage/mia_file.c:121-126)
 * has this signature.
 *
 * The reference's fixed-capacity LRU cache behind this port
 * (src/storage/expert_cache.c) has no counterpart here: every expert of
 * every layer stays resident in HBM (include/mia/moe.h), loaded once
 * through this port by mia_moe_load_experts.
 */
typedef int (*mia_expert_loader)(void *ctx, int layer, int expert, void *dst);

#endif
