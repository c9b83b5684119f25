/*
 * The mia-serve line protocol over the GPU engine (src/app/serve.c of the
 * reference; tools/internal/engine/protocol.go:1-13 documents it):
 *
 *   -> CHAT <nbytes> <max_tokens> <temperature> <top_p> <think>\n<nbytes bytes>
 *   -> RESET\n            -> QUIT\n
 *   <- READY k=v ...      once, after the model is loaded
 *   <- PROG <done> <total> per prompt token
 *   <- TOK <n> <hits> <misses>\n<n bytes>
 *   <- DONE k=v ...       end of a CHAT (reason stop | length | ctx | cancel)
 *   <- OK                 end of a RESET
 *   <- ERR <code> <msg>   the command failed; the engine stays usable
 *
 * One conversation's KV cache stays in HBM between turns, so a turn
 * prefills only its own tokens; SIGUSR1 cancels a running CHAT. Prompt
 * positions other than the last run without the output head
 * (mia_gpu_model_feed); the sampler runs on the device logits and, as in
 * the reference's loop (serve.c:108-136), only when a token is about to be
 * drawn, so its state advances identically. Every expert is resident: the
 * expert-cache counters of TOK and DONE count every expert use as a hit.
 */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <fcntl.h>
#include <signal.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include "mia/model_gpu.h"
#include "mia/serve.h"

#define MAX_MESSAGE (1 << 20)

static volatile sig_atomic_t g_cancel = 0;
static void on_usr1(int sig) {
    (void)sig;
    g_cancel = 1;
}

static double seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + ts.tv_nsec * 1e-9;
}

typedef struct {
    mia_gpu_model *m;
    mia_bpe *tok;
    mhip_sampler smp;
    FILE *out;
    int ctx, pos;
    int *ids;
    unsigned long long hits; /* expert uses: layers x active experts per step */
    int per_step;
} server;

static void say_err(server *s, const char *code, const char *msg) {
    fprintf(s->out, "ERR %s %s\n", code, msg);
    fflush(s->out);
}

static void say_done(server *s, const char *reason, int prompt, int gen, double prefill_s,
                     double gen_s) {
    fprintf(s->out,
            "DONE reason=%s prompt=%d gen=%d prefill_s=%.3f gen_s=%.3f ctx_used=%d ctx_max=%d "
            "hits=%llu misses=0\n",
            reason, prompt, gen, prefill_s, gen_s, s->pos, s->ctx, s->hits);
    fflush(s->out);
}

static void engine_failed(server *s) {
    char msg[600];
    snprintf(msg, sizeof msg, "forward pass failed on the GPU (%s); conversation was reset",
             mia_gpu_model_error(s->m));
    s->pos = 0;
    say_err(s, "engine", msg);
}

static void chat(server *s, const char *user, int max_tokens, float temp, float top_p,
                 int think) {
    g_cancel = 0;
    s->smp.temperature = temp;
    s->smp.top_p = top_p > 0.0f && top_p <= 1.0f ? top_p : 1.0f;
    char *text = mia_chat_turn_text(user, think, s->pos > 0);
    const int n = text ? mia_bpe_encode(s->tok, text, s->ids, s->ctx) : -1;
    free(text);
    const int left = s->ctx - s->pos - 1; /* room for at least one reply token */
    if (n < 0 || n > left) {
        char msg[200];
        if (n < 0)
            snprintf(msg, sizeof msg,
                     "this message is longer than the whole context (%d tokens); start a new "
                     "chat or shorten it",
                     s->ctx);
        else
            snprintf(msg, sizeof msg,
                     "this message needs %d tokens but only %d are left; start a new chat", n,
                     left);
        say_err(s, "context_full", msg);
        return;
    }
    const int start = s->pos;
    const double t0 = seconds();
    for (int i = 0; i < n; i++) {
        if (g_cancel) { /* roll back: later steps overwrite these positions */
            s->pos = start;
            say_done(s, "cancel", i, 0, seconds() - t0, 0);
            return;
        }
        const int rc = i + 1 < n ? mia_gpu_model_feed(s->m, s->ids[i], s->pos)
                                 : (mia_gpu_model_step(s->m, s->ids[i], s->pos) ? 0 : -1);
        if (rc) {
            engine_failed(s);
            return;
        }
        s->hits += (unsigned long long)s->per_step;
        s->pos++;
        fprintf(s->out, "PROG %d %d\n", i + 1, n);
        fflush(s->out);
    }
    const double t1 = seconds();
    const char *reason = "length";
    int gen = 0;
    while (gen < max_tokens) {
        if (s->pos >= s->ctx) {
            reason = "ctx";
            break;
        }
        const int next = mia_gpu_model_sample(s->m, &s->smp);
        if (next < 0) {
            engine_failed(s);
            return;
        }
        if (mia_bpe_is_stop(s->tok, next)) {
            reason = "stop";
            break;
        }
        int len;
        const unsigned char *piece = mia_bpe_piece(s->tok, next, &len);
        fprintf(s->out, "TOK %d %llu 0\n", len, s->hits);
        fwrite(piece, 1, (size_t)len, s->out);
        fflush(s->out);
        gen++;
        if (!mia_gpu_model_step(s->m, next, s->pos)) {
            engine_failed(s);
            return;
        }
        s->hits += (unsigned long long)s->per_step;
        s->pos++;
        if (g_cancel) {
            reason = "cancel";
            break;
        }
    }
    say_done(s, reason, n, gen, t1 - t0, seconds() - t1);
}

/* The MTK1 blob of the file (header tok_offset / tok_size). */
static int read_tokenizer(const char *path, mia_bpe **tok, char *err, size_t errlen) {
    mia_file_info h;
    if (mia_file_probe(path, &h, err, errlen)) return -1;
    if (!h.tok_size) {
        snprintf(err, errlen, "%s holds no tokenizer", path);
        return -1;
    }
    unsigned char *blob = malloc((size_t)h.tok_size);
    const int fd = open(path, O_RDONLY);
    size_t got = 0;
    while (blob && fd >= 0 && got < h.tok_size) {
        const ssize_t r = pread(fd, blob + got, (size_t)h.tok_size - got, (off_t)(h.tok_offset + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) break;
        got += (size_t)r;
    }
    if (fd >= 0) close(fd);
    int rc = 0;
    if (!blob || got != h.tok_size) {
        snprintf(err, errlen, "%s: reading the tokenizer failed", path);
        rc = -1;
    } else if (mia_bpe_open(tok, blob, (size_t)h.tok_size)) {
        snprintf(err, errlen, "%s: the tokenizer blob is not a valid MTK1 blob", path);
        rc = -1;
    }
    free(blob);
    return rc;
}

int mia_serve(const char *model, int ctx, uint64_t seed, int device, FILE *in, FILE *out) {
    struct sigaction sa;
    memset(&sa, 0, sizeof sa);
    sa.sa_handler = on_usr1;
    sa.sa_flags = SA_RESTART;
    sigaction(SIGUSR1, &sa, NULL);

    static server s;
    memset(&s, 0, sizeof s);
    s.out = out;
    s.ctx = ctx;
    char err[600];
    if (ctx < 2) {
        fprintf(stderr, "error: context of %d positions\n", ctx);
        return 1;
    }
    if (read_tokenizer(model, &s.tok, err, sizeof err)) {
        fprintf(stderr, "error: %s\n", err);
        return 1;
    }
    if (mia_bpe_im_start(s.tok) < 0) {
        fprintf(stderr, "error: tokenizer has no <|im_start|>; this model cannot chat\n");
        mia_bpe_close(s.tok);
        return 1;
    }
    if (mia_gpu_model_open(&s.m, model, ctx, device, err, sizeof err)) {
        fprintf(stderr, "error: %s\n", err);
        mia_bpe_close(s.tok);
        return 1;
    }
    const mia_file_info *h = mia_gpu_model_info(s.m);
    s.per_step = (int)(h->n_layers * h->n_active);
    s.ids = malloc(sizeof(int) * (size_t)ctx);
    char *msg = malloc(MAX_MESSAGE + 1);
    if (!s.ids || !msg) {
        fprintf(stderr, "error: out of memory\n");
        mia_gpu_model_close(s.m);
        mia_bpe_close(s.tok);
        free(s.ids);
        free(msg);
        return 1;
    }
    mhip_sampler_init(&s.smp, 0.7f, 0.8f, (int)h->vocab, seed);
    const int total = (int)(h->n_layers * h->n_experts);
    fprintf(stderr,
            "mia-serve: %u layers, %u experts (top-%u), q8_0 | HBM: dense %.2f GiB + %d "
            "resident experts (%.2f GiB), context %d\n",
            h->n_layers, h->n_experts, h->n_active, (double)h->dense_size / (1 << 30), total,
            (double)total * (double)h->expert_blob_size / (1 << 30), ctx);
    fprintf(out,
            "READY layers=%u experts=%u active=%u ctx=%d slots=%d total=%d wtype=q8_0 "
            "dense_gib=%.2f cache_gib=%.2f\n",
            h->n_layers, h->n_experts, h->n_active, ctx, total, total,
            (double)h->dense_size / (1 << 30),
            (double)total * (double)h->expert_blob_size / (1 << 30));
    fflush(out);

    char line[256];
    while (fgets(line, sizeof line, in)) {
        int nbytes, max_tokens, think;
        float temp, top_p;
        if (!strcmp(line, "RESET\n")) {
            s.pos = 0;
            fprintf(out, "OK\n");
            fflush(out);
        } else if (sscanf(line, "CHAT %d %d %f %f %d", &nbytes, &max_tokens, &temp, &top_p,
                          &think) == 5) {
            if (nbytes < 0 || nbytes > MAX_MESSAGE ||
                fread(msg, 1, (size_t)nbytes, in) != (size_t)nbytes) {
                say_err(&s, "bad_request", "message too large or truncated");
                continue;
            }
            msg[nbytes] = '\0';
            chat(&s, msg, max_tokens, temp, top_p, think);
        } else if (!strcmp(line, "QUIT\n")) {
            break;
        } else {
            say_err(&s, "bad_request", "unknown command");
        }
    }
    free(msg);
    free(s.ids);
    mia_gpu_model_close(s.m);
    mia_bpe_close(s.tok);
    return 0;
}
