#ifndef MIA_ORACLE_H
#define MIA_ORACLE_H
/*
 * CPU restatement of motorIa's Q8_0 MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY: this is the parity checker and the CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may
 * load it. The product (motoria_amd/) never links, calls or falls back to it.
 *
 * Semantics follow the reference's Linux/x86 build (scalar dot products, no
 * threading), compiled -std=c99 -O3 -ffp-contract=off so no product is fused
 * into an add. Each function cites the reference lines it restates.
 *
 * Parity pinning (what checks each function besides retyping its formula):
 *   orc_quantize_row_q8  known answers of tests/test_quant.c:24-41 and
 *                        tools/internal/mia/format_test.go:35-55; bit-equal to
 *                        the reference build (oracle/_ref) on random rows.
 *   orc_matvec           closed form / tolerance of tests/test_matmul.c:6-60;
 *                        bit-equal to oracle/_ref.
 *   orc_rmsnorm          unit-RMS invariant (tools/internal/ref/ref_test.go:18-28);
 *                        bit-equal to oracle/_ref inside the layer.
 *   orc_softmax/top_k    known answers (ref_test.go:30-56), tie rule, brute force.
 *   orc_moe_layer        bit-equal to oracle/_ref (real moe()) on golden vectors.
 *   orc_moe_layer_bucketed  bit-equal to orc_moe_layer (loop nest only differs).
 *   orc_model_step       bit-equal to oracle/_ref's mia_model_step (golden
 *                        logits of tests/golden/model_*.npz); RoPE against
 *                        its closed form (a rotation preserves norms).
 *   orc_dispatch         brute-force stable sort; permutation invariants.
 */
#include <stddef.h>
#include <stdint.h>

#define ORC_QK 32
enum { ORC_F32 = 0, ORC_Q8_0 = 1 };

/* include/mia/quant.h:12-15: 36-byte block, value = d * q. */
typedef struct {
    float d;
    int8_t q[ORC_QK];
} orc_block_q8;

typedef struct {
    int dim;           /* d: hidden size (2048) */
    int n_experts;     /* E (128) */
    int n_active;      /* K (8) */
    int expert_hidden; /* eh (768) */
    int norm_topk;     /* renormalise the top-K gates (Qwen3: 1) */
    float norm_eps;    /* rmsnorm epsilon (1e-6) */
} orc_dims;

size_t orc_row_bytes(int wtype, int cols);
void orc_quantize_row_q8(const float *x, orc_block_q8 *y, int n);
void orc_dequantize_row(int wtype, const void *src, float *dst, int n);
void orc_matvec(float *out, const void *w, int wtype, const float *x,
                orc_block_q8 *xq, int rows, int cols);
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
void orc_softmax(float *x, int n);
void orc_top_k(const float *p, int n, int k, int *idx);
float orc_expf(float x);
/* Softmax in place over logits[E], top-K idx[K], gate weights w[K]. */
void orc_route(float *logits, int E, int K, int norm_topk, int *idx, float *w);

/* Offsets of up/down inside a reference-format expert blob
 * (src/storage/mia_file.c:98-101) and the blob size (format.go:160-163). */
size_t orc_off_up(const orc_dims *s);
size_t orc_off_down(const orc_dims *s);
size_t orc_blob_bytes(const orc_dims *s);

/*
 * One MoE layer over T independent tokens, in place on x[T][dim]
 * (src/model/forward.c:167-197 applied per token). blobs[e] points to expert
 * e of this layer in the reference blob format, or NULL if unavailable (the
 * call then fails like a cache miss whose load failed). bias may be NULL.
 * Optional outputs (NULL to skip): idx[T][K], w[T][K], logits[T][E] (after
 * the bias), xn[T][dim]. Returns 0, or -1 (K > 64 or a missing expert).
 * nthreads > 1 spreads tokens over OpenMP threads, or, for one token, the
 * 64-row chunks of every matrix (the reference's CHUNK_ROWS split; same
 * bits).
 */
int orc_moe_layer(const orc_dims *s, int T, float *x, const float *ffn_norm,
                  const float *router, const float *bias,
                  const unsigned char *const *blobs, int *idx, float *w,
                  float *logits, float *xn, int nthreads);

/* MoE-only stack: layers l = 0..L-1 of RMSNorm -> MoE -> residual.
 * blobs[l*E + e], ffn_norm[l*dim], router[l*E*dim]. */
int orc_moe_stack(const orc_dims *s, int L, int T, float *x,
                  const float *ffn_norm, const float *router,
                  const unsigned char *const *blobs, int nthreads);

/* The same layer as orc_moe_layer (same bits), computed expert by expert:
 * tokens bucketed by expert, 16 tokens per weight-row pass (for large T).
 * Optional outputs idx[T][K], w[T][K], logits[T][E]. Returns 0 or -1. */
int orc_moe_layer_bucketed(const orc_dims *s, int T, float *x, const float *ffn_norm,
                           const float *router, const float *bias,
                           const unsigned char *const *blobs, int *idx, float *w,
                           float *logits, int nthreads);

/* Routing only (rmsnorm, router chains + bias, softmax, top-K, gate weights)
 * of T tokens, the first half of orc_moe_layer (same bits). Outputs
 * idx[T][K], w[T][K], logits[T][E] (after the bias; may be NULL). */
int orc_route_tokens(const orc_dims *s, int T, const float *x, const float *ffn_norm,
                     const float *router, const float *bias, int *idx, float *w,
                     float *logits, int nthreads);

/* A whole model (the tensors a .mia file holds, src/model/forward.c). */
typedef struct {
    orc_dims moe;                        /* dim and the MoE shape, norm_eps */
    int n_layers, n_heads, n_kv_heads, head_dim, vocab, wtype;
    float rope_theta;
    const void *token_embd, *output;     /* [vocab][dim] in wtype */
    const float *output_norm;            /* [dim] */
    const float *const *attn_norm;       /* [L] -> [dim] */
    const float *const *q_norm;          /* [L] -> [head_dim] */
    const float *const *k_norm;          /* [L] -> [head_dim] */
    const float *const *ffn_norm;        /* [L] -> [dim] */
    const float *const *router;          /* [L] -> [E][dim] */
    const void *const *wq, *const *wk, *const *wv, *const *wo; /* [L], in wtype */
    const unsigned char *const *blobs;   /* [L * E] expert blobs (Q8_0) */
} orc_model;

/* mia_model_step (src/model/forward.c:199-217) for the token at `pos`:
 * embedding, n_layers x (attention, MoE), final rmsnorm and output head into
 * logits[vocab]. kc/vc: the caller's KV cache, [L][max_seq][n_kv_heads *
 * head_dim] floats, positions < pos already filled by earlier steps.
 * x_out (optional) receives the residual after the last layer. nthreads
 * spreads 64-row chunks of the large matrices over threads (same bits).
 * Q8_0 models only. Returns 0 or -1. */
int orc_model_step(const orc_model *m, float *kc, float *vc, int max_seq, int token, int pos,
                   float *logits, float *x_out, int nthreads);
/* forward.c:84-93 on one head row, in place (exposed for tests). */
void orc_rope_row(float *x, int hd, int pos, float theta);

/* The token sampler (src/tokenizer/sampler.c). init: top_p outside (0, 1]
 * becomes 1, seed 0 the default state (:6-14). */
typedef struct {
    float temperature, top_p;
    int n;
    uint64_t rng;
} orc_sampler;
void orc_sampler_init(orc_sampler *s, float temperature, float top_p, int n, uint64_t seed);
/* xorshift64* step and its 24-bit float in [0, 1) (:20-25). */
float orc_sampler_rand01(orc_sampler *s);
/* mia_sample (:33-66) on logits[n] (not modified): greedy when temperature
 * <= 0, else the nucleus draw; candidates in descending probability, equal
 * probabilities in ascending index (the order the reference's qsort gives
 * with glibc's merge sort). An empty candidate list (logits with NaN, or a
 * cutoff above every probability), where the reference reads outside its
 * buffer, returns the greedy token. */
int orc_sample(orc_sampler *s, const float *logits);

/* Stable counting sort of the T*K assignments (t, j) by expert idx[t][j],
 * t-major then j. counts[E], offsets[E+1], perm[T*K] = t*K + j in bucketed
 * order, pos[t*K + j] = its position in perm. Returns 0 or -1 (bad index). */
int orc_dispatch(const int *idx, int T, int K, int E, int *counts,
                 int *offsets, int *perm, int *pos);

/* Synthetic tensors (same generator as include/mia/synth.h). */
void orc_synth_x(uint64_t seed, int T, int dim, float *x);
void orc_synth_router(uint64_t seed, int layer, const orc_dims *s, float *w);
void orc_synth_expert_blob(uint64_t seed, int layer, int expert,
                           const orc_dims *s, unsigned char *blob);

#endif
