#ifndef MIA_MOE_H
#define MIA_MOE_H
/*
 * Public Q8_0 MoE FFN entry points on one GPU.
 *
 * The reference's layer is `static int moe(mia_model*, dims, int l)`
 * (src/model/forward.c:167-197), called once per layer and token from
 * mia_model_step (src/model/forward.c:210-213), with experts fetched through
 * an LRU cache fed by the mia_expert_loader port. Here the layer is public,
 * takes T tokens at once, and reads every expert of every layer from one
 * HBM-resident table (48 x 128 Q8_0 experts of Qwen3-30B-A3B, 36.2 GB with the
 * block-major scale copies).
 *
 * Conventions follow the reference engine: C99, functions return 0 or -1
 * (with a message in mia_moe_error), rich error text at open time through
 * (char *err, size_t errlen), not thread-safe (one host thread per handle).
 */
#include <stddef.h>
#include <stdint.h>

#include "mia/expert_cache.h"
#include "mia/quant.h"
#include "mia_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mia_moe mia_moe;

/* Model shape: the MoE fields of the .mia header (include/mia/mia_file.h:
 * 10-21 of the reference) plus the sizes of this handle. */
typedef struct {
    int dim;           /* header dim (2048) */
    int n_layers;      /* header n_layers (48) */
    int n_experts;     /* header n_experts (128) */
    int n_active;      /* header n_active (8) */
    int expert_hidden; /* header expert_hidden (768) */
    int norm_topk;     /* header norm_topk (1 for Qwen3) */
    float norm_eps;    /* header norm_eps (1e-6) */
    int max_tokens;    /* largest T passed to one call */
    int device;        /* HIP device ordinal */
} mia_moe_config;

int mia_moe_open(mia_moe **out, const mia_moe_config *cfg, char *err, size_t errlen);
void mia_moe_close(mia_moe *m);
const char *mia_moe_error(const mia_moe *m);

/* Reference blob geometry for this shape (src/storage/mia_file.c:98-101,
 * tools/internal/mia/format.go:160-163). */
size_t mia_moe_blob_bytes(const mia_moe *m);
size_t mia_moe_off_up(const mia_moe *m);
size_t mia_moe_off_down(const mia_moe *m);

/* Fill the whole table through the reference's storage port: one call of
 * `load` per (layer, expert) into a host buffer, uploaded and regrouped in
 * HBM. A failing load returns -1 naming the expert; the table keeps what was
 * loaded before (the reference's cache likewise leaves no poisoned slot,
 * src/storage/expert_cache.c:76-79). */
int mia_moe_load_experts(mia_moe *m, mia_expert_loader load, void *ctx);
/* One expert from a host blob in the .mia format. */
int mia_moe_load_expert(mia_moe *m, int layer, int expert, const void *blob);
/* Read one expert back in the .mia blob format (padding zeroed). */
int mia_moe_read_expert(mia_moe *m, int layer, int expert, void *blob);
/* Dense per-layer MoE weights: ffn_norm[dim] and router[E][dim] (fp32, the
 * layout of mia_layer.ffn_norm/router, include/mia/mia_file.h:23-26). */
int mia_moe_set_layer(mia_moe *m, int layer, const float *ffn_norm, const float *router);
/* Seeded synthetic weights generated in HBM (include/mia/synth.h): experts
 * and routers ~ N(0, 0.02), ffn_norm = 1. */
int mia_moe_synth(mia_moe *m, uint64_t seed);

/* ---- .mia model files --------------------------------------------------
 * The header of a .mia file (the reference's mia_header,
 * include/mia/mia_file.h:10-21: 112 bytes, little-endian) and the expert
 * blob offsets derived from it (src/storage/mia_file.c:98-101). */
typedef struct {
    uint32_t version, wtype, dim, n_layers, n_heads, n_kv_heads, head_dim, vocab;
    uint32_t n_experts, n_active, expert_hidden, norm_topk;
    float rope_theta, norm_eps;
    uint64_t dense_offset, dense_size;
    uint64_t experts_offset, expert_blob_size;
    uint64_t tok_offset, tok_size;
    uint64_t off_up, off_down; /* up and down matrices inside a blob */
} mia_file_info;

/* Reads and checks a .mia file's header: magic "MIA1", version 1, the
 * reference reader's shape rules (src/storage/mia_file.c:53-61), the dense
 * section laid out as the converter's NewLayout (tools/internal/mia/
 * format.go:129-165; the walk must end at dense_size), gate/up/down fitting
 * the blob, and a file long enough for every expert blob. 0, or -1 with the
 * reason in err. Reads no tensor. */
int mia_file_probe(const char *path, mia_file_info *info, char *err, size_t errlen);
/* File offsets of layer `layer`'s ffn_norm[dim] and router[E][dim] (fp32)
 * in a probed file. 0, or -1 for a layer out of range. */
int mia_file_layer_offsets(const mia_file_info *info, int layer, uint64_t *ffn_norm,
                           uint64_t *router);
/* Fills the handle from a .mia file: every layer's ffn_norm and router
 * (mia_moe_set_layer) and every (layer, expert) blob into the HBM table,
 * bit-identical to filling it through the loader port with the reference's
 * mia_file_read_expert. The file's shape, norm settings and Q8_0 weight type
 * must be the handle's. Reading the file overlaps the uploads (two pinned
 * staging batches); the call records stream marks 14 and 15 of the handle's
 * context (mhip_mark). */
int mia_moe_load_file(mia_moe *m, const char *path);

/* One layer, moe() semantics, in place on host x[T][dim]. Bit-equal to the
 * reference at every T (with MHIP_FAST_DOWN set through mia_moe_set_flags,
 * within ~1e-6 relative from MHIP_GEMM_MIN_A assignments on). One
 * token (T = 1) runs as one launch of the persistent decode kernel with the
 * exact router where mhip_decode_supported allows it, else per stage; a
 * decode launch that aborts is rerun per stage (same bits). A failing call
 * names the first layer that met an expert index out of range. */
int mia_moe_layer(mia_moe *m, int layer, float *x, int T);
/* As mia_moe_layer with an optional logit bias[E] (added after the router,
 * before the softmax) and optional outputs idx[T][K], w[T][K] and
 * logits[T][E]. NULL skips any of them; asking for the logits keeps the
 * per-stage path. */
int mia_moe_layer_ex(mia_moe *m, int layer, float *x, int T, const float *bias, int *idx,
                     float *w, float *logits);
/* Layers [l0, l1) of RMSNorm -> MoE -> residual, in place on host x[T][dim]. */
int mia_moe_stack(mia_moe *m, int l0, int l1, float *x, int T);

/* Device-pointer forms: d_x[T][dim] (and d_bias[E]) live in HBM; the work is
 * queued on the handle's stream and returns before it completes. */
int mia_moe_layer_dev(mia_moe *m, int layer, float *d_x, int T, const float *d_bias);
int mia_moe_stack_dev(mia_moe *m, int l0, int l1, float *d_x, int T);
/* mia_moe_stack_dev as one HIP graph (no counterpart in the reference): the
 * first call records the stack's launches (kernel nodes only) and every call
 * replays them as one submission; a call with other arguments (or after
 * mia_moe_set_flags) records again. The recording holds d_x: replays read
 * and write that buffer. Results are bit-identical to mia_moe_stack_dev's. */
int mia_moe_stack_graph(mia_moe *m, int l0, int l1, float *d_x, int T);

/* Decode of one token through layers [l0, l1) in a single persistent launch
 * (the Qwen3-30B-A3B shape on a 256-CU MI355X; mhip_decode_stack). x[dim]
 * (host) is updated in place; idx/w ([l1-l0][K]) receive the routing when
 * not NULL; bias (E floats) applies to every layer when not NULL. Every
 * layer is bit-equal to the reference's moe() on its input, so x, idx and w
 * after any number of layers are bit-equal to the reference's chain of
 * layers from the same x (forward.c:210-213 without the attention). With
 * MHIP_DECODE_CERTIFIED set through mia_moe_set_flags the gate weights come
 * from the parallel router logits instead: indices bit-equal layer by
 * layer, each layer's output within ~1e-6 relative of the reference's on the
 * same input, but a many-layer output that drifts (about 1e-1 relative after
 * 48 layers, as those differences flip Q8 codes). Should the launch abort,
 * the layers are rerun per stage (bit-equal to the reference) and
 * mia_moe_decode_status shows the aborted launch. */
int mia_moe_decode(mia_moe *m, int l0, int l1, float *x, const float *bias, int *idx, float *w);
/* Same on device memory, queued on the handle's stream; check
 * mia_moe_decode_status after the stream completes. */
int mia_moe_decode_dev(mia_moe *m, int l0, int l1, float *d_x, const float *d_bias);
/* status[0] abort bits (nonzero: the output is invalid), [1] rmsnorm
 * fallbacks, [2] layers routed by the exact fallback. Waits for the stream. */
int mia_moe_decode_status(mia_moe *m, int status[4]);
/* Stage timestamps of the last decode call made with MHIP_DECODE_TRACE
 * (see mhip_decode_trace). */
int mia_moe_decode_trace(mia_moe *m, unsigned long long *out);

/* The handle's device context (memory, copies, stream marks of mia_hip.h)
 * and the scratch of the last call (routing, dispatch, intermediates). */
mhip_ctx *mia_moe_gpu(mia_moe *m);
const mhip_scratch *mia_moe_scratch(const mia_moe *m);
/* Flags forwarded to mhip_moe_layer (e.g. MHIP_FORCE_SEQ_RMS). */
void mia_moe_set_flags(mia_moe *m, int flags);
/* Device diagnostics: status[0] bit 0 = an expert index out of range;
 * status[1] = tokens whose rmsnorm sum took the sequential path. Waits for
 * the stream. */
int mia_moe_status(mia_moe *m, int status[4]);

#ifdef __cplusplus
}
#endif
#endif
