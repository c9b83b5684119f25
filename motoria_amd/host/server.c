/*
 * mia-serve on the GPU engine: the line protocol the reference's Go engine
 * speaks to its server process (tools/internal/engine/protocol.go:1-13; the
 * reference's server is src/app/serve.c), over mia_gpu_model.
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
 * A session keeps one conversation: its KV cache stays in HBM between
 * turns, so a turn prefills only its own text. A CHAT runs in three
 * phases:
 *   admit    the turn's chat text is tokenized and must leave room for at
 *            least one reply token (else ERR context_full);
 *   prefill  the prompt tokens before the last run in batches of up to
 *            PREFILL_CHUNK at the next positions without the output head
 *            (mia_gpu_model_prefill: the KV rows n feeds would write), a
 *            PROG for each token once its batch is done; the last token is
 *            a step; a cancel here (checked between batches) takes the
 *            conversation back to where the turn started;
 *   generate the sampler draws from the device logits of the last step
 *            (mia_gpu_model_sample) while tokens and context remain; a stop
 *            token ends the turn without being sent; each sent token is
 *            run to give the logits of the next draw, so the sampler state
 *            (carried from turn to turn) advances once per draw.
 * SIGUSR1 cancels a running CHAT (checked before each prompt batch and
 * after each generated token). A failing GPU step answers ERR engine and
 * starts a new conversation. Every expert is resident in HBM: the
 * expert-cache counters of TOK and DONE count each expert use as a hit.
 */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <fcntl.h>
#include <signal.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include "mia/model_gpu.h"
#include "mia/serve.h"

enum { MESSAGE_MAX = 1 << 20, PREFILL_CHUNK = 1024 };

static volatile sig_atomic_t g_stop_turn;
static void on_cancel_signal(int sig) {
    (void)sig;
    g_stop_turn = 1;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

typedef struct {
    mia_gpu_model *model;
    mia_bpe *tok;
    mhip_sampler sampler;
    FILE *out;
    int ctx_max;             /* positions of the KV cache */
    int used;                /* positions of the conversation so far */
    int *prompt;             /* [ctx_max] ids of the turn being admitted */
    int uses_per_step;       /* layers x active experts */
    unsigned long long uses; /* expert uses so far (all hits) */
    char *message;           /* [MESSAGE_MAX + 1] */
} session;

/* One protocol line (printf format, the newline added) and a flush. */
static void reply(session *s, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfprintf(s->out, fmt, ap);
    va_end(ap);
    fputc('\n', s->out);
    fflush(s->out);
}

/* A turn's figures, reported in its DONE line. */
typedef struct {
    int prompt, gen;
    double t0, t_prefill, t_end;
} turn;

static void reply_done(session *s, const char *why, const turn *t) {
    reply(s,
          "DONE reason=%s prompt=%d gen=%d prefill_s=%.3f gen_s=%.3f ctx_used=%d ctx_max=%d "
          "hits=%llu misses=0",
          why, t->prompt, t->gen, t->t_prefill - t->t0, t->t_end - t->t_prefill, s->used,
          s->ctx_max, s->uses);
}

/* A failed GPU step: the conversation's cache is no longer trustworthy. */
static void engine_lost(session *s) {
    reply(s, "ERR engine GPU step failed (%s); the conversation starts over",
          mia_gpu_model_error(s->model));
    s->used = 0;
}

/* Runs `id` at the next position, ending in the logits the sampler draws
 * from. 0, or -1 (reported). */
static int advance(session *s, int id) {
    if (!mia_gpu_model_step(s->model, id, s->used)) {
        engine_lost(s);
        return -1;
    }
    s->used++;
    s->uses += (unsigned long long)s->uses_per_step;
    return 0;
}

static void run_chat(session *s, const char *text, int max_tokens, float temperature,
                     float top_p, int think) {
    g_stop_turn = 0;
    s->sampler.temperature = temperature;
    s->sampler.top_p = (top_p > 0.0f && top_p <= 1.0f) ? top_p : 1.0f;

    /* admit */
    char *chat_text = mia_chat_turn_text(text, think, s->used > 0);
    const int n = chat_text ? mia_bpe_encode(s->tok, chat_text, s->prompt, s->ctx_max) : -1;
    free(chat_text);
    const int room = s->ctx_max - s->used - 1;
    if (n < 0) {
        reply(s, "ERR context_full the message alone exceeds the %d-token context; shorten it",
              s->ctx_max);
        return;
    }
    if (n > room) {
        reply(s, "ERR context_full the message takes %d tokens and the context has %d free; "
                 "reset to start over", n, room);
        return;
    }

    /* prefill */
    turn t = {n, 0, now_s(), 0.0, 0.0};
    const int first = s->used;
    for (int i = 0; i < n;) {
        if (g_stop_turn) {
            s->used = first; /* the next turn overwrites these positions */
            t.prompt = i;
            t.t_prefill = t.t_end = now_s();
            reply_done(s, "cancel", &t);
            return;
        }
        if (i == n - 1) {
            if (advance(s, s->prompt[i])) return;
            reply(s, "PROG %d %d", n, n);
            break;
        }
        const int c = n - 1 - i < PREFILL_CHUNK ? n - 1 - i : PREFILL_CHUNK;
        if (mia_gpu_model_prefill(s->model, s->prompt + i, c, s->used)) {
            engine_lost(s);
            return;
        }
        s->used += c;
        s->uses += (unsigned long long)s->uses_per_step * (unsigned long long)c;
        for (int j = 1; j <= c; j++) reply(s, "PROG %d %d", i + j, n);
        i += c;
    }
    t.t_prefill = now_s();

    /* generate */
    const char *why = "length";
    while (t.gen < max_tokens) {
        if (s->used >= s->ctx_max) {
            why = "ctx";
            break;
        }
        const int id = mia_gpu_model_sample(s->model, &s->sampler);
        if (id < 0) {
            engine_lost(s);
            return;
        }
        if (mia_bpe_is_stop(s->tok, id)) {
            why = "stop";
            break;
        }
        int len;
        const unsigned char *bytes = mia_bpe_piece(s->tok, id, &len);
        fprintf(s->out, "TOK %d %llu 0\n", len, s->uses);
        fwrite(bytes, 1, (size_t)len, s->out);
        fflush(s->out);
        t.gen++;
        if (advance(s, id)) return;
        if (g_stop_turn) {
            why = "cancel";
            break;
        }
    }
    t.t_end = now_s();
    reply_done(s, why, &t);
}

/* ---- commands ------------------------------------------------------------------ */

/* Each handler gets the rest of its line (after the command word) and the
 * input stream (CHAT reads its message from it); 1 ends the loop. */
static int cmd_chat(session *s, const char *args, FILE *in) {
    int nbytes, max_tokens, think;
    float temperature, top_p;
    if (sscanf(args, "%d %d %f %f %d", &nbytes, &max_tokens, &temperature, &top_p, &think) != 5) {
        reply(s, "ERR bad_request CHAT wants <nbytes> <max_tokens> <temperature> <top_p> <think>");
        return 0;
    }
    if (nbytes < 0 || nbytes > MESSAGE_MAX) {
        reply(s, "ERR bad_request message size %d outside [0, %d]", nbytes, MESSAGE_MAX);
        return 0;
    }
    if (fread(s->message, 1, (size_t)nbytes, in) != (size_t)nbytes) {
        reply(s, "ERR bad_request the message ended after fewer than %d bytes", nbytes);
        return 0;
    }
    s->message[nbytes] = '\0';
    run_chat(s, s->message, max_tokens, temperature, top_p, think);
    return 0;
}

static int cmd_reset(session *s, const char *args, FILE *in) {
    (void)args;
    (void)in;
    s->used = 0;
    reply(s, "OK");
    return 0;
}

static int cmd_quit(session *s, const char *args, FILE *in) {
    (void)s;
    (void)args;
    (void)in;
    return 1;
}

static const struct {
    const char *word;
    int (*run)(session *, const char *, FILE *);
    int takes_args;
} COMMANDS[] = {
    {"CHAT", cmd_chat, 1},
    {"RESET", cmd_reset, 0},
    {"QUIT", cmd_quit, 0},
};

/* Dispatches one input line (its newline removed); 1 ends the loop. */
static int dispatch(session *s, char *line, FILE *in) {
    char *args = strchr(line, ' ');
    if (args) *args++ = '\0';
    for (size_t i = 0; i < sizeof COMMANDS / sizeof COMMANDS[0]; i++) {
        if (strcmp(line, COMMANDS[i].word) != 0) continue;
        if (!COMMANDS[i].takes_args && args) break; /* e.g. "RESET x" */
        return COMMANDS[i].run(s, args ? args : "", in);
    }
    reply(s, "ERR bad_request unknown command");
    return 0;
}

/* ---- set-up ---------------------------------------------------------------------- */

/* The file's MTK1 blob (header tok_offset / tok_size) into *tok. */
static int load_tokenizer(const char *path, mia_bpe **tok, char *err, size_t errlen) {
    mia_file_info h;
    if (mia_file_probe(path, &h, err, errlen)) return -1;
    if (h.tok_size == 0) {
        snprintf(err, errlen, "%s has no tokenizer", path);
        return -1;
    }
    unsigned char *blob = malloc((size_t)h.tok_size);
    const int fd = open(path, O_RDONLY);
    size_t got = 0;
    while (blob && fd >= 0 && got < h.tok_size) {
        const ssize_t r =
            pread(fd, blob + got, (size_t)h.tok_size - got, (off_t)(h.tok_offset + got));
        if (r > 0) got += (size_t)r;
        else if (!(r < 0 && errno == EINTR)) break;
    }
    if (fd >= 0) close(fd);
    int rc = -1;
    if (!blob || got != h.tok_size)
        snprintf(err, errlen, "%s: cannot read its tokenizer", path);
    else if (mia_bpe_open(tok, blob, (size_t)h.tok_size))
        snprintf(err, errlen, "%s: its tokenizer is not a valid MTK1 blob", path);
    else
        rc = 0;
    free(blob);
    return rc;
}

static void session_free(session *s) {
    if (s->model) mia_gpu_model_close(s->model);
    mia_bpe_close(s->tok);
    free(s->prompt);
    free(s->message);
}

int mia_serve(const char *model, int ctx, uint64_t seed, int device, FILE *in, FILE *out) {
    struct sigaction sa;
    memset(&sa, 0, sizeof sa);
    sa.sa_handler = on_cancel_signal;
    sa.sa_flags = SA_RESTART;
    sigaction(SIGUSR1, &sa, NULL);

    session s;
    memset(&s, 0, sizeof s);
    s.out = out;
    s.ctx_max = ctx;
    char err[600] = "";
    int ok = ctx >= 2;
    if (!ok) snprintf(err, sizeof err, "a context of %d positions cannot hold a turn", ctx);
    if (ok) ok = load_tokenizer(model, &s.tok, err, sizeof err) == 0;
    if (ok && mia_bpe_im_start(s.tok) < 0) {
        snprintf(err, sizeof err, "the tokenizer has no <|im_start|>: not a chat model");
        ok = 0;
    }
    if (ok) ok = mia_gpu_model_open(&s.model, model, ctx, device, err, sizeof err) == 0;
    if (ok) {
        s.prompt = malloc(sizeof(int) * (size_t)ctx);
        s.message = malloc(MESSAGE_MAX + 1);
        if (!s.prompt || !s.message) {
            snprintf(err, sizeof err, "out of host memory");
            ok = 0;
        }
    }
    if (!ok) {
        fprintf(stderr, "mia-serve: %s\n", err);
        session_free(&s);
        return 1;
    }

    const mia_file_info *h = mia_gpu_model_info(s.model);
    s.uses_per_step = (int)(h->n_layers * h->n_active);
    mhip_sampler_init(&s.sampler, 0.7f, 0.8f, (int)h->vocab, seed);
    const int resident = (int)(h->n_layers * h->n_experts);
    const double dense_gib = (double)h->dense_size / (1 << 30);
    const double experts_gib = (double)resident * (double)h->expert_blob_size / (1 << 30);
    fprintf(stderr, "mia-serve: %u layers x %u experts (top %u), Q8_0, all resident in HBM "
                    "(dense %.2f GiB, experts %.2f GiB); context %d\n",
            h->n_layers, h->n_experts, h->n_active, dense_gib, experts_gib, ctx);
    /* the expert-cache fields say every expert has a slot */
    reply(&s, "READY layers=%u experts=%u active=%u ctx=%d slots=%d total=%d wtype=q8_0 "
              "dense_gib=%.2f cache_gib=%.2f",
          h->n_layers, h->n_experts, h->n_active, ctx, resident, resident, dense_gib,
          experts_gib);

    char line[256];
    while (fgets(line, sizeof line, in)) {
        const size_t len = strlen(line);
        if (len && line[len - 1] == '\n') line[len - 1] = '\0';
        if (dispatch(&s, line, in)) break;
    }
    session_free(&s);
    return 0;
}
