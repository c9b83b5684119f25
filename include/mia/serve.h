#ifndef MIA_SERVE_H
#define MIA_SERVE_H
/*
 * Text side of the serve protocol on the GPU engine: the byte-level BPE
 * tokenizer of a .mia file (the MTK1 blob, src/tokenizer/bpe.c of the
 * reference: same ids for the same text), the Qwen3 chat-turn text
 * (src/model/runtime.c:84-95), and the mia-serve line protocol
 * (src/app/serve.c:145-226, tools/internal/engine/protocol.go:1-13) over
 * mia_gpu_model.
 */
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mia_bpe mia_bpe;

/* Reads an MTK1 blob (the reference reader's checks: magic, counts, ids in
 * range, no truncation); 0 or -1. */
int mia_bpe_open(mia_bpe **out, const unsigned char *blob, size_t n);
void mia_bpe_close(mia_bpe *t);
/* UTF-8 text to ids: returns the count (<= max), or -1 when more than max
 * ids would be needed (mia_tok_encode, bpe.c:245-270). */
int mia_bpe_encode(const mia_bpe *t, const char *text, int *out, int max);
/* The bytes of id (length in *len; an empty piece for ids out of range). */
const unsigned char *mia_bpe_piece(const mia_bpe *t, int id, int *len);
/* 1 for the end-of-text and <|im_end|> ids (bpe.c:112-114). */
int mia_bpe_is_stop(const mia_bpe *t, int id);
int mia_bpe_vocab(const mia_bpe *t);
/* The <|im_start|> id, or -1 when the vocabulary has none. */
int mia_bpe_im_start(const mia_bpe *t);

/* The chat text of one user turn (malloc'd): when `continuing`, the
 * previous assistant reply is closed first; think = 0 adds the empty
 * thinking block (runtime.c:84-95). */
char *mia_chat_turn_text(const char *user, int think, int continuing);

/* The mia-serve loop: loads `model` onto `device` with a context of `ctx`
 * positions and the sampler seeded with `seed`, prints READY to `out`, then
 * answers CHAT / RESET / QUIT lines read from `in` until QUIT or end of
 * input (SIGUSR1 cancels a running CHAT). Returns 0, or 1 when the model
 * cannot be opened or chat with (the reason on stderr). */
int mia_serve(const char *model, int ctx, uint64_t seed, int device, FILE *in, FILE *out);

#ifdef __cplusplus
}
#endif
#endif
