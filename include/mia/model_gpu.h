#ifndef MIA_MODEL_GPU_H
#define MIA_MODEL_GPU_H
/*
 * The reference engine's model step, mia_model_step (include/mia/model.h:21-23
 * and src/model/forward.c:199-217 of the reference), with every tensor in
 * HBM on one GPU: the token's embedding, then per layer the attention block
 * (forward.c:118-165, KV cache in HBM) and the MoE FFN (the HBM expert table
 * of include/mia/moe.h), then the final rmsnorm and the output head. Only
 * the logits cross PCIe. Q8_0 models.
 *
 * Conventions follow the reference engine: C99, 0/-1 (or NULL) returns with
 * the reason in mia_gpu_model_error, rich error text at open time, one host
 * thread per handle.
 */
#include <stddef.h>
#include <stdint.h>

#include "mia/moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mia_gpu_model mia_gpu_model;

/* Opens a .mia file (mia_file_probe's checks), uploads its dense section,
 * expert table, norms and routers to device `device`, and sizes the KV cache
 * for max_seq positions. */
int mia_gpu_model_open(mia_gpu_model **out, const char *path, int max_seq, int device,
                       char *err, size_t errlen);
/* No counterpart in the reference: a model of the given shape (the
 * mia_file_info header fields; wtype Q8_0) with seeded synthetic weights
 * generated in HBM (matrices ~ N(0, 0.02) quantized to Q8_0, norms 1, the
 * MoE handle's mia_moe_synth), for benchmarks at shapes whose files would
 * not fit a test's disk. */
int mia_gpu_model_synth(mia_gpu_model **out, const mia_file_info *shape, int max_seq,
                        int device, uint64_t seed, char *err, size_t errlen);
void mia_gpu_model_close(mia_gpu_model *m);
const char *mia_gpu_model_error(const mia_gpu_model *m);
int mia_gpu_model_vocab(const mia_gpu_model *m);

/* Feeds `token` at position `pos` (sequential from 0) and returns the
 * vocabulary logits (owned by the handle, valid until the next call), or
 * NULL when pos is outside [0, max_seq) or token outside [0, vocab), or on a
 * device error. */
const float *mia_gpu_model_step(mia_gpu_model *m, int token, int pos);

/* The step without the output head: the KV cache of every layer gains the
 * token's row, no logits are formed (a prompt position whose logits nobody
 * reads, src/app/serve.c:91-106). 0 or -1. */
int mia_gpu_model_feed(mia_gpu_model *m, int token, int pos);

/* n feeds in one call (no counterpart in the reference, whose serve loop
 * feeds a prompt one token at a time): tokens[0..n) at positions
 * pos .. pos + n - 1, in batches of equal size (at most 1024 tokens)
 * through each layer at once (the attention of the batch with
 * mhip_attention_batch, its MoE on the per-stage kernels for T tokens, the
 * matrix-core ones from MHIP_GEMM_MIN_A assignments on), so the weights are
 * read once per batch instead of once per token. The KV rows written are bit-equal to n calls of
 * mia_gpu_model_feed; no logits are formed. 0 or -1. */
int mia_gpu_model_prefill(mia_gpu_model *m, const int *tokens, int n, int pos);

/* The token sampler (mhip_sample) on the logits of the last
 * mia_gpu_model_step / _step_sample call, left on the device: the picked
 * id, or -1 (also when the last call was a feed or failed). */
int mia_gpu_model_sample(mia_gpu_model *m, mhip_sampler *s);

/* The model's header fields (mia_file_probe's view of the file, or the
 * shape mia_gpu_model_synth was given). */
const mia_file_info *mia_gpu_model_info(const mia_gpu_model *m);

/* The step followed by the token sampler on the device logits
 * (mhip_sample, src/tokenizer/sampler.c:33-66 of the reference; s->n must
 * be the vocabulary size): returns the picked token id, or -1. Only the id
 * crosses PCIe; s->rng advances as mia_sample's would. */
int mia_gpu_model_step_sample(mia_gpu_model *m, int token, int pos, mhip_sampler *s);

/* Flags of the MoE layers (include/mia_hip.h), as mia_moe_set_flags. At the
 * Qwen3-30B-A3B shape a step is one launch of the model stack (every
 * layer's attention and MoE, mhip_model_stack); MHIP_MODEL_PER_LAYER asks
 * for one attention and one MoE launch per layer instead (the same bits).
 * By default (0, or MHIP_FORCE_EXACT_ROUTER) the decode kernel's MoE uses the
 * reference's sequential router chains: logits bit-equal to the
 * reference's. MHIP_DECODE_CERTIFIED: the gate weights from the certified
 * parallel router logits instead (expert indices bit-equal, gate weights
 * within ~1e-6 relative; through the requantizations of later layers the
 * logits then move by whole Q8 steps, ~5e-4 of max|logit| each, up to ~1e-2
 * in all). MHIP_EXACT_EXPERTS: the
 * per-stage kernels (bit-equal, no decode launch). MHIP_DECODE_FORCE_ABORT:
 * every decode launch aborts and the step reruns per stage (a test of that
 * fallback). MHIP_DECODE_CHAINS_FIRST (under the exact router): the
 * exact chains before the expert stream in every layer (the path of a
 * layer whose ranking is not certified). MHIP_ATTN_FORCE_ABORT: every
 * one-launch attention (mhip_attention_layer, used where the shape allows
 * it) aborts and the step reruns from that layer per stage. Either forced
 * abort stops a model stack launch, and the token reruns per stage. */
void mia_gpu_model_set_flags(mia_gpu_model *m, int flags);
/* Launches of the last step (model stack, or decode and one-launch
 * attention) that aborted (their layers rerun per stage). */
int mia_gpu_model_aborts(const mia_gpu_model *m);
/* With MHIP_DECODE_TRACE in the flags, the model stack launch of the last
 * step records the stage timestamps of mhip_decode_trace; this copies them
 * out (out[MHIP_TRACE_NL][256][MHIP_TRACE_SLOTS]). 0 or -1 (no model stack
 * at this shape). Diagnostic. */
int mia_gpu_model_trace(mia_gpu_model *m, unsigned long long *out);

#ifdef __cplusplus
}
#endif
#endif
