#ifndef MIA_HIP_H
#define MIA_HIP_H
/*
 * Thin C ABI over the gfx950 HIP kernels of the Q8_0 MoE FFN path.
 *
 * Plain pointers and sizes only. Every pointer named d_* is device memory
 * (HBM) obtained from mhip_malloc; every launch is asynchronous on the
 * context's stream. Functions return 0 on success or -1 with a message in
 * mhip_error(). Not thread-safe: one host thread per context, as the
 * reference engine is (include/mia/model.h:7 of the reference).
 *
 * The C host library (include/mia/moe.h, quant.h, matmul.h) is built on this
 * layer; tests and benchmarks may also call it directly.
 */
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mhip_ctx mhip_ctx;

/* Shape of one MoE layer (Qwen3-30B-A3B: 2048, 128, 8, 768). */
typedef struct {
    int dim;           /* d, multiple of 32, <= 8192 */
    int n_experts;     /* E, <= 256 */
    int n_active;      /* K, <= 64 and <= E */
    int expert_hidden; /* eh, multiple of 32, <= 8192 */
    int norm_topk;     /* 1: renormalise the K gate weights to sum to 1 */
    float norm_eps;    /* rmsnorm epsilon */
} mhip_dims;

/*
 * HBM layout of one expert in the resident table (bytes; each section is
 * 256-byte aligned). Codes are row-major int8, scales row-major fp32 with one
 * scale per 32-value block; values and bytes-per-weight are those of the
 * reference's 36-byte Q8_0 blocks, only regrouped (codes apart from scales)
 * so that rows load as aligned 16-byte vectors. A second, block-major copy
 * of the scales serves the matrix-core kernels, which read one block of
 * many rows at a time.
 */
typedef struct {
    size_t gate_q, up_q, down_q;    /* [eh][d], [eh][d], [d][eh] int8 */
    size_t gate_s, up_s, down_s;    /* [eh][d/32], [eh][d/32], [d][eh/32] fp32 */
    size_t gate_st, up_st, down_st; /* [d/32][eh], [d/32][eh], [eh/32][d] fp32 (same values) */
    size_t expert_bytes;            /* stride between experts */
} mhip_layout;

int mhip_layout_of(const mhip_dims *s, mhip_layout *out);

/* ---- context, memory, stream ---------------------------------------- */
int mhip_device_count(void);
int mhip_open(mhip_ctx **out, int device, char *err, size_t errlen);
void mhip_close(mhip_ctx *c);
const char *mhip_error(const mhip_ctx *c);
void *mhip_malloc(mhip_ctx *c, size_t bytes);
int mhip_free(mhip_ctx *c, void *d_ptr);
int mhip_h2d(mhip_ctx *c, void *d_dst, const void *src, size_t bytes);
int mhip_d2h(mhip_ctx *c, void *dst, const void *d_src, size_t bytes);
int mhip_d2d(mhip_ctx *c, void *d_dst, const void *d_src, size_t bytes);
/* Pinned (page-locked) host memory, and copies queued on the context's
 * stream without waiting (the host buffer must be pinned and stay untouched
 * until the stream has passed the copy, e.g. until mhip_sync). */
void *mhip_host_malloc(mhip_ctx *c, size_t bytes);
int mhip_host_free(mhip_ctx *c, void *h_ptr);
int mhip_h2d_async(mhip_ctx *c, void *d_dst, const void *h_src, size_t bytes);
int mhip_d2h_async(mhip_ctx *c, void *h_dst, const void *d_src, size_t bytes);
int mhip_zero(mhip_ctx *c, void *d_ptr, size_t bytes); /* fill kernel, not memset */
int mhip_sync(mhip_ctx *c);
/* Milliseconds between two points of the context's stream (HIP events). */
int mhip_mark(mhip_ctx *c, int slot); /* slot 0..15 */
int mhip_elapsed(mhip_ctx *c, int slot0, int slot1, float *ms);
/* Waits on the host until the stream has passed the last mhip_mark of slot
 * (at once if the slot was never marked). */
int mhip_mark_wait(mhip_ctx *c, int slot);

/* Per-stage kernel timing. While a mask is set, every launch of a selected
 * stage of mhip_moe_layer is bracketed by two HIP events on the context's
 * stream (up to max_launches launches; later ones are not timed).
 * mhip_stage_time waits for them and returns the summed milliseconds and the
 * number of timed launches of one stage. mask 0 turns timing off. */
#define MHIP_STAGE_RMSNORM 0
#define MHIP_STAGE_ROUTER 1
#define MHIP_STAGE_DISPATCH 2
#define MHIP_STAGE_GATEUP 3
#define MHIP_STAGE_DOWN 4
#define MHIP_STAGE_COMBINE 5
#define MHIP_STAGE_DECODE 6 /* the persistent decode-stack kernel */
#define MHIP_N_STAGES 7
int mhip_stage_timing(mhip_ctx *c, unsigned mask, int max_launches);
int mhip_stage_time(mhip_ctx *c, int stage, double *ms, int *launches);

/* ---- expert table ----------------------------------------------------- */
/* Repack n reference-format blobs (d_blobs, blob_bytes apart; gate at 0, up
 * at off_up, down at off_down) into table slots (layer, experts[i]). */
int mhip_table_repack(mhip_ctx *c, const mhip_dims *s, void *d_table,
                      int layer, const int *experts, int n,
                      const void *d_blobs, size_t blob_bytes, size_t off_up,
                      size_t off_down);
/* Inverse: table slot -> reference-format blob (zero padded). */
int mhip_table_unpack(mhip_ctx *c, const mhip_dims *s, const void *d_table,
                      int layer, int expert, void *d_blob, size_t blob_bytes,
                      size_t off_up, size_t off_down);
/* Seeded synthetic experts for layers [l0, l1) generated in HBM, bit-equal
 * to include/mia/synth.h quantized on the host. */
int mhip_table_synth(mhip_ctx *c, const mhip_dims *s, void *d_table,
                     uint64_t seed, int l0, int l1);
/* Router of layer l, transposed (d_router_t[i*E + e] = W[e][i]) and, when
 * d_router_dl is not NULL, in the decode layout (below). */
int mhip_router_synth(mhip_ctx *c, const mhip_dims *s, float *d_router_t,
                      float *d_router_dl, uint64_t seed, int layer);
int mhip_router_transpose(mhip_ctx *c, const mhip_dims *s, float *d_router_t,
                          const float *d_router);
/* Decode layout of one layer's router from the row-major W[E][d]: within
 * each expert row, element i = 32 L + 4 k + c (L < d/32, k < 8, c < 4) is
 * stored at (k * d/32 + L) * 4 + c, so the decode kernel's lane L reads its
 * 32 consecutive elements as 8 fully contiguous 1 KB loads. */
int mhip_router_decode_layout(mhip_ctx *c, const mhip_dims *s, float *d_router_dl,
                              const float *d_router);
int mhip_synth_f32(mhip_ctx *c, float *d_out, size_t n, uint64_t seed,
                   uint64_t stream, double sigma);
int mhip_fill_f32(mhip_ctx *c, float *d_out, size_t n, float value);

/* ---- the MoE layer, one kernel per stage ------------------------------ */
/* Scratch for one layer call over up to max_tokens tokens. */
typedef struct {
    float *xn;        /* [T][d]   rmsnorm output */
    int8_t *xq;       /* [T][d]   Q8 codes of xn */
    float *xs;        /* [T][d/32] Q8 scales of xn */
    float *logits;    /* [T][E]   router logits (after bias) */
    int *idx;         /* [T][K]   selected experts, descending probability */
    float *w;         /* [T][K]   gate weights */
    int *counts;      /* [E] */
    int *offsets;     /* [E+1] */
    int *perm;        /* [T*K]   assignment t*K+j in expert-bucketed order */
    int *pos;         /* [T*K]   inverse of perm */
    int *groups;      /* [1 + 3*E]: n_groups, then (expert, begin, end) */
    float *h;         /* [T*K][eh] SwiGLU output, bucketed order */
    float *tmp;       /* [T*K][d]  down output, bucketed order */
    int *status;      /* [4] device-side error/diagnostic words */
    void *xdq;        /* [T][d]    fp16: the Q8 codes of xn (matrix-core path) */
    void *hdq;        /* [T*K][eh] fp16: the Q8 codes of h, bucketed (matrix-core path) */
    int *gtile;       /* [E+1]     tiles of MHIP_GEMM_TM rows before each group */
    float *xsb;       /* [d/32][T*K] Q8 scales of xn per assignment, bucketed (matrix-core path) */
    int8_t *hq;       /* [T*K][eh] Q8 codes of h, bucketed (vector path) */
    float *hs;        /* Q8 scales of h, bucketed: [T*K][eh/32] (vector path), or
                         [eh/32][T*K] block-major (matrix-core path) */
    int *glight;      /* [E+1]     light tiles (at most MHIP_GEMM_TM/2 rows) before each group */
} mhip_scratch;

/* Rows of one expert bucket per matrix-core tile. */
#define MHIP_GEMM_TM 128

size_t mhip_scratch_bytes(const mhip_dims *s, int max_tokens);
int mhip_scratch_carve(const mhip_dims *s, int max_tokens, void *d_base,
                       mhip_scratch *out);

/* Flags for mhip_moe_layer and mhip_decode_stack. */
#define MHIP_FORCE_SEQ_RMS 1      /* always take the sequential rmsnorm sum */
#define MHIP_FORCE_EXACT_ROUTER 2 /* decode stack: the reference's exact router chains
                                     (routing and gate weights bit-equal); the default,
                                     and it overrides MHIP_DECODE_CERTIFIED */
#define MHIP_DECODE_TRACE 4       /* decode stack: record stage timestamps */
#define MHIP_EXACT_EXPERTS 8      /* layer: bit-exact expert products at every T */
#define MHIP_DECODE_FORCE_ABORT 16 /* decode stack: report abort bit 4 and stop after the
                                      start barrier (tests the callers' abort handling) */
#define MHIP_DECODE_CHAINS_FIRST 32 /* decode stack, under the exact router: the exact
                                       chains before the expert stream in every layer, as for
                                       a layer whose ranking is not certified (without it they
                                       run beside the stream when it is) */
#define MHIP_DECODE_CERTIFIED 256 /* decode stack: gate weights from the certified
                                     parallel router logits (expert indices still bit-equal,
                                     weights within ~1e-6 relative, so over many layers the
                                     output drifts from the reference's; not the default) */
#define MHIP_FAST_DOWN 512        /* layer, matrix-core path: each down block term added
                                     with one fused multiply-add (expert outputs within a
                                     few fp32 ulps instead of bit-equal; not the default) */

/*
 * One MoE layer (rmsnorm -> router/top-K -> dispatch -> gate/up+SwiGLU ->
 * down -> combine) in place on d_x[T][d] (16-byte aligned, as every
 * mhip_malloc pointer is). d_table/d_router_t/d_norm point to
 * this layer's experts, transposed router and ffn_norm. d_bias (E floats) is
 * added to the logits when non-NULL.
 *
 * Routing (indices, order, gate weights) and the layer output are bit-equal
 * to the reference at every T. From MHIP_GEMM_MIN_A assignments on (and when
 * the shape allows: d a multiple of 256, expert_hidden of 128) the expert
 * products run on the matrix cores: the gate/up and down block dots stay
 * exact integers and each block term is added in the reference's rounding
 * order. MHIP_FAST_DOWN adds the down terms with one fused multiply-add
 * instead (outputs within ~1e-6 relative); MHIP_EXACT_EXPERTS keeps the
 * vector kernels at every T.
 */
#define MHIP_GEMM_MIN_A 2048
int mhip_moe_layer(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                   const void *d_table_layer, const float *d_router_t,
                   const float *d_norm, const float *d_bias, float *d_x, int T,
                   const mhip_scratch *sc, int flags);
/* Calls of mhip_moe_layer on this context whose expert products ran on the
 * matrix-core kernels (diagnostic: which path a call took). */
unsigned long long mhip_matrix_layers(const mhip_ctx *c);

/*
 * Decode (one token) through L consecutive layers in one persistent launch:
 * the Qwen3-30B-A3B shape only (dim 2048, 128 experts, n_active <= 8,
 * expert_hidden 768) on a 256-CU MI355X. d_table/d_router ([L][E][d], each
 * layer in the decode layout of mhip_router_decode_layout)/
 * d_router_t ([L][d][E])/d_norm ([L][d]) start at the first layer; d_bias
 * (E floats, every layer) may be NULL; d_x[d] is updated in place; L is at
 * most MHIP_DECODE_MAX_LAYERS (-1 beyond, before any device work). d_ws is a
 * workspace of mhip_decode_ws_bytes() bytes (not shared by concurrent
 * launches). d_idx/d_w ([L][n_active]) receive the routing when non-NULL.
 * Every layer is bit-equal to the reference's moe() (forward.c:167-197) on
 * its input, so the output of any number of layers is the reference's
 * chain's, bit for bit: the ranking is certified from parallel logits with
 * a rigorous bound (or, where it cannot be, taken from the reference's
 * sequential logit chains), and the gate weights come from those sequential
 * chains, which run beside the expert stream. With MHIP_DECODE_CERTIFIED
 * (and without MHIP_FORCE_EXACT_ROUTER) the gate weights come from the
 * parallel logits instead: indices still bit-equal, weights within ~1e-6
 * relative, a layer's output within a few ulps, and a many-layer output
 * that drifts from the reference's as those differences flip Q8 codes
 * (about 1e-1 relative after 48 layers). After the stream completes,
 * mhip_decode_status reports [0] abort bits (1: workgroups not on the
 * expected XCDs, 2: a wait timed out, 4: MHIP_DECODE_FORCE_ABORT, 8: a NaN
 * probability in a layer routed from a certified ranking; the output is
 * then invalid and the layer is rerun per stage), [1] rmsnorm fallbacks,
 * [2] layers whose gate weights came from the exact chains.
 */
#define MHIP_DECODE_MAX_LAYERS 256 /* layers of one decode-stack launch */
size_t mhip_decode_ws_bytes(void);
/* 1 when mhip_decode_stack can run this shape on this device (the
 * Qwen3-30B-A3B expert shape, 2048/128/<=8/768, and one 512-thread workgroup
 * on every one of 256 CUs), 0 when it cannot (no error is set), -1 when the
 * device query fails. */
int mhip_decode_supported(mhip_ctx *c, const mhip_dims *s);
int mhip_decode_stack(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                      const void *d_table, const float *d_router, const float *d_router_t,
                      const float *d_norm, const float *d_bias, float *d_x, int L,
                      void *d_ws, int *d_idx, float *d_w, int flags);
/*
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). mhip_decode_stack without the workspace argument: the
 * workspace is a device-resident array of the library, one per GPU, of
 * mhip_decode_ws_bytes() bytes (0.95 MiB, held until the process ends; its
 * address is taken once per device when a context is opened). The call
 * queues the launch and, when d_status (device int[4]) is not NULL, a copy
 * of this launch's status words ([0] abort bits, [1] rmsnorm fallbacks,
 * [2] exact-router layers, [3] 0) into it; it allocates nothing. L is at most
 * MHIP_DECODE_MAX_LAYERS (-1 beyond). Every call on one GPU shares that
 * GPU's workspace, so the calls of one GPU are serialized: the host side
 * under a lock (calls from several threads are safe), the launches in order
 * (a call on another stream than the previous call's waits for that launch
 * through an event, which is not an allocation). Under stream capture the
 * capturing caller must order the captured calls against any other call on
 * the same GPU itself: the launch is captured without that wait.
 */
int mhip_decode_stack_noalloc(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                              const void *d_table, const float *d_router,
                              const float *d_router_t, const float *d_norm, const float *d_bias,
                              float *d_x, int L, int *d_idx, float *d_w, int *d_status,
                              int flags);
int mhip_decode_status(mhip_ctx *c, const void *d_ws, int status[4]);
/* With MHIP_DECODE_TRACE set: the 100 MHz real-time counter read by thread 0
 * of each of the 256 workgroups at up to MHIP_TRACE_SLOTS stage boundaries
 * of layers MHIP_TRACE_L0 .. MHIP_TRACE_L0 + MHIP_TRACE_NL - 1
 * (out[MHIP_TRACE_NL][256][MHIP_TRACE_SLOTS]; slots not reached stay 0).
 * Diagnostic. */
#define MHIP_TRACE_L0 8
#define MHIP_TRACE_NL 8
#define MHIP_TRACE_SLOTS 48
int mhip_decode_trace(mhip_ctx *c, const void *d_ws, unsigned long long *out);

/* ---- attention and output head of one token (decode) ---------------------
 * src/model/forward.c:118-165 and :214-215 of the reference, bit-equal to its
 * x86 build. Dense weights are device copies of the .mia file's tensors:
 * wq [n_heads*head_dim][dim], wk/wv [n_kv_heads*head_dim][dim],
 * wo [dim][n_heads*head_dim], output [vocab][dim] in 36-byte Q8_0 blocks;
 * attn_norm/output_norm [dim], q_norm/k_norm [head_dim] fp32. */
typedef struct {
    int dim, n_heads, n_kv_heads, head_dim; /* head_dim even, <= 256; dim, heads*head_dim <= 8192 */
    float norm_eps;
} mhip_attn_dims;

size_t mhip_attention_scratch_bytes(const mhip_attn_dims *s, int max_seq);
/* Attention of the token at `pos` for one layer, in place on d_x[dim]
 * (x += Wo attention(rmsnorm(x))); d_x_copy, when not NULL, receives the
 * new x too. d_kc/d_vc: this layer's K and V cache,
 * [max_seq][n_kv_heads*head_dim] fp32; row pos is written, rows < pos read.
 * d_rope: [max_seq][head_dim/2][2] doubles, cos and sin of
 * pos * theta^(-2i/head_dim) as the host libm gives them (the reference's
 * angles, forward.c:84-93). d_scratch: mhip_attention_scratch_bytes(). */
int mhip_attention(mhip_ctx *c, const mhip_attn_dims *s, const float *d_attn_norm,
                   const void *d_wq, const void *d_wk, const void *d_wv, const void *d_wo,
                   const float *d_q_norm, const float *d_k_norm, const double *d_rope,
                   float *d_kc, float *d_vc, int pos, int max_seq, float *d_x,
                   float *d_x_copy, void *d_scratch, int flags);
/* No counterpart in the reference, which feeds a prompt one token at a time:
 * mhip_attention for the n consecutive tokens at positions pos .. pos + n - 1
 * in one go, in place on d_x[n][dim]. Every token's result and cache rows
 * are bit-equal to n calls of mhip_attention in position order (the rows of
 * all n tokens are appended before any score; token t reads rows
 * 0 .. pos + t). d_scratch: mhip_attention_batch_scratch_bytes(s, n,
 * max_seq) bytes (0 for invalid arguments). */
size_t mhip_attention_batch_scratch_bytes(const mhip_attn_dims *s, int n, int max_seq);
int mhip_attention_batch(mhip_ctx *c, const mhip_attn_dims *s, const float *d_attn_norm,
                         const void *d_wq, const void *d_wk, const void *d_wv, const void *d_wo,
                         const float *d_q_norm, const float *d_k_norm, const double *d_rope,
                         float *d_kc, float *d_vc, int pos, int n, int max_seq, float *d_x,
                         const void *d_pack, void *d_scratch, int flags);
/* The layer's Q, K, V and O weights repacked for mhip_attention_batch's
 * matrix-core rows (no counterpart in the reference): codes as fp16
 * integers, scales block-major; d_pack holds mhip_attention_pack_bytes(s)
 * bytes (0 for shapes whose rows are not multiples of 64, which keep the
 * vector kernels). With d_pack given, batches of 512
 * tokens or more form their Q/K/V and O rows on the matrix cores, with the
 * same bits (exact block dots, block terms in block order); NULL keeps the
 * vector kernels. */
size_t mhip_attention_pack_bytes(const mhip_attn_dims *s);
int mhip_attention_pack(mhip_ctx *c, const mhip_attn_dims *s, const void *d_wq, const void *d_wk,
                        const void *d_wv, const void *d_wo, void *d_pack);
/* logits[vocab] = output Q8(rmsnorm(x, output_norm)) (forward.c:214-215);
 * d_scratch as for mhip_attention. */
int mhip_output_head(mhip_ctx *c, const mhip_attn_dims *s, const float *d_output_norm,
                     const void *d_output, int vocab, const float *d_x, float *d_logits,
                     void *d_scratch, int flags);

/*
 * No counterpart in the reference: mhip_attention in one launch for callers
 * that step a whole model (the same forward.c:118-165 arithmetic, bit-equal;
 * the Qwen3-30B-A3B attention shape only: dim 2048, 32/4 heads of 128). Every
 * CU takes part: the rmsnorm, q/k/v rows, heads and Wo rows meet through
 * tagged words in d_ws (mhip_attention_layer_ws_bytes(), 256-byte aligned,
 * not shared by overlapping launches; the context clears it when it first
 * sees it). d_x is updated in place; d_x_in / d_x_out (may be NULL) receive
 * x before and after. *d_status (may be NULL) gets abort bits OR'ed in (2: a
 * wait for another workgroup ran out, 4: MHIP_ATTN_FORCE_ABORT); the caller
 * clears it. An aborted launch leaves d_x as it was (d_x_in is written in
 * any case) but its cache row and d_x_out are invalid: the caller reruns
 * the layer with mhip_attention. _supported: 1 when the shape, max_seq and the device
 * (256 CUs, one 512-thread workgroup each) fit, 0 when not, -1 on an error.
 */
#define MHIP_ATTN_FORCE_ABORT 64 /* the one-launch attention reports abort bit 4 and
                                    stops after its start barrier (a test of the
                                    callers' rerun) */
size_t mhip_attention_layer_ws_bytes(void);
/* With MHIP_DECODE_TRACE in flags, a launch records the 100 MHz real-time
 * counter of each of its 256 workgroups at MHIP_ATTN_TRACE_SLOTS phase
 * boundaries (start, started, norm, q/k/v out, head in, head out, heads in,
 * end); this copies them out (out[256][MHIP_ATTN_TRACE_SLOTS]). Diagnostic. */
#define MHIP_ATTN_TRACE_SLOTS 8
int mhip_attention_layer_trace(mhip_ctx *c, const void *d_ws, unsigned long long *out);
int mhip_attention_layer_supported(mhip_ctx *c, const mhip_attn_dims *s, int max_seq);
int mhip_attention_layer(mhip_ctx *c, const mhip_attn_dims *s, const float *d_attn_norm,
                         const void *d_wq, const void *d_wk, const void *d_wv, const void *d_wo,
                         const float *d_q_norm, const float *d_k_norm, const double *d_rope,
                         float *d_kc, float *d_vc, int pos, int max_seq, float *d_x,
                         float *d_x_in, float *d_x_out, void *d_ws, int *d_status, int flags);

/*
 * No counterpart in the reference, whose mia_model_step (forward.c:199-217)
 * calls the attention and moe() of each layer in turn: every layer of one
 * token -- the attention of mhip_attention_layer, then the MoE of
 * mhip_decode_stack -- in one launch, for callers that step a whole model at
 * the Qwen3-30B-A3B shape (the MoE shape of mhip_decode_stack and the
 * attention shape of mhip_attention_layer). Bit-equal to running those two
 * per layer. d_al[L] (device) holds each layer's attention tensors and its
 * K/V cache; d_x is the token's embedding row on entry and x after layer
 * L - 1 on exit; d_ws: mhip_model_stack_ws_bytes() (256-byte aligned; the
 * context clears it when it first sees it). *d_status (int[4], device)
 * receives the launch's status words as mhip_decode_status gives them
 * ([0] abort bits: 1, 2 as there, 4 when MHIP_DECODE_FORCE_ABORT or
 * MHIP_ATTN_FORCE_ABORT asked for one); after an abort d_x and the cache
 * rows at pos are invalid and the caller reruns the token per layer.
 * _supported: 1 when the shapes, max_seq and the device fit, 0 when not, -1
 * on an error.
 */
typedef struct {
    const float *attn_norm, *q_norm, *k_norm; /* [dim], [head_dim], [head_dim] */
    const void *wq, *wk, *wv, *wo;             /* Q8_0 rows */
    float *kc, *vc;                            /* [max_seq][n_kv_heads*head_dim] */
} mhip_attn_layer;
#define MHIP_MODEL_STACK_MAX_SEQ 8192 /* positions whose scores fit the kernel's LDS */
#define MHIP_MODEL_PER_LAYER 128      /* mia_gpu_model steps: one launch per layer's
                                         attention and per layer's MoE, not the stack */
size_t mhip_model_stack_ws_bytes(void);
int mhip_model_stack_supported(mhip_ctx *c, const mhip_dims *s, const mhip_attn_dims *as,
                               int max_seq);
int mhip_model_stack(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                     const void *d_table, const float *d_router_dl, const float *d_router_t,
                     const float *d_norm, const float *d_bias, const mhip_attn_dims *as,
                     const mhip_attn_layer *d_al, const double *d_rope, int pos, int max_seq,
                     float *d_x, int L, void *d_ws, int *d_status, int flags);

/* ---- HIP graphs -----------------------------------------------------------
 * No counterpart in the reference. The launches queued on a context between
 * mhip_graph_begin and mhip_graph_end are recorded (not run) into a graph,
 * which mhip_graph_launch replays on the context's stream as one
 * submission. Only kernel launches and device-to-device copies may be
 * queued meanwhile (the library's clears are fill kernels; stage-timing
 * events are skipped while capturing); a call that waits for the device
 * fails the capture. The graph replays the recorded arguments: the same
 * pointers, shapes and flags. mhip_graph_end(c, NULL) ends a capture and
 * drops it (also after an error inside it). */
typedef struct mhip_graph mhip_graph;
int mhip_graph_begin(mhip_ctx *c);
int mhip_graph_end(mhip_ctx *c, mhip_graph **out);
int mhip_graph_launch(mhip_ctx *c, mhip_graph *g);
void mhip_graph_destroy(mhip_graph *g);

/* ---- token sampler on device logits -------------------------------------
 * src/tokenizer/sampler.c of the reference: mhip_sampler is mia_sampler
 * (include/mia/sampler.h:11-16) without its host buffer; init as
 * mia_sampler_init (sampler.c:6-14: top_p outside (0, 1] becomes 1, seed 0
 * the default state). mhip_sample is mia_sample (sampler.c:33-66) on
 * d_logits[n] (left unchanged): the picked token id goes to *d_token
 * (device int) and s->rng advances as the reference's does (once per call
 * with temperature > 0). Same picks as the reference; candidates of equal
 * probability in ascending index (glibc's merge-sort qsort). Where the
 * reference reads outside its buffer (no candidate: NaN logits, or a
 * cutoff above every probability) the greedy token is picked. */
#define MHIP_SAMPLE_MAX_N (1 << 21)
typedef struct {
    float temperature, top_p;
    int n;
    uint64_t rng;
} mhip_sampler;
void mhip_sampler_init(mhip_sampler *s, float temperature, float top_p, int n, uint64_t seed);
/* Device scratch of mhip_sample for n logits (0 when n is outside
 * [1, MHIP_SAMPLE_MAX_N]). */
size_t mhip_sample_scratch_bytes(int n);
int mhip_sample(mhip_ctx *c, mhip_sampler *s, const float *d_logits, void *d_scratch,
                int *d_token);
/* The sampler's running sums on their own (no counterpart in the reference,
 * whose sampler.c:43,55,64 adds them in loops): s_0 = 0, s_{k+1} =
 * fl(s_k + d_v[k]) for k < n, every addition in fp32 in index order, the
 * result bit-equal to that loop, for d_v[n] (16-byte aligned, readable up
 * to n rounded up to a multiple of 4 values) of values >= 0 (other values
 * are added one at a time, as the loop would). mode
 * MHIP_CHAIN_SUM runs all n additions; MHIP_CHAIN_GE stops after the first
 * addition that makes s >= thr, MHIP_CHAIN_GT after the first that makes
 * thr < s. d_out (device, 2 ints): [0] the bits of s after the last
 * addition done, [1] the index of the stopping element (n if none). */
#define MHIP_CHAIN_SUM 0
#define MHIP_CHAIN_GE 1
#define MHIP_CHAIN_GT 2
int mhip_chain_f32(mhip_ctx *c, const float *d_v, int n, int mode, float thr, int *d_out);

/* ---- reference tensor ops on device pointers ---------------------------- */
/* Q8_0 blocks in the reference's 36-byte format. */
int mhip_quantize_q8(mhip_ctx *c, const float *d_x, void *d_blocks, int n);
int mhip_dequantize_q8(mhip_ctx *c, const void *d_blocks, float *d_x, int n);
/* out = W x (wtype 0: fp32 rows; 1: Q8_0 rows of 36-byte blocks, x is
 * quantized into d_xq first). Bit-equal to the reference's scalar kernels. */
int mhip_matvec(mhip_ctx *c, float *d_out, const void *d_w, int wtype,
                const float *d_x, void *d_xq, int rows, int cols);

#ifdef __cplusplus
}
#endif
#endif
