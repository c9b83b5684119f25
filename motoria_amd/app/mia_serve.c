/*
 * mia-serve on the GPU engine (include/mia/serve.h). Its options are the
 * ones the reference's Go engine passes to the server it starts
 * (tools/internal/engine): -m, -c, --seed, and --ram, which is accepted and
 * ignored since every expert is resident in HBM; --device picks the GPU.
 *
 *   mia-serve -m model.mia [-c 4096] [--seed N] [--device D] [--ram SIZE]
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "mia/serve.h"

typedef struct {
    const char *model;
    int ctx, device;
    unsigned long long seed;
} options;

static void set_model(options *o, const char *v) { o->model = v; }
static void set_ctx(options *o, const char *v) { o->ctx = atoi(v); }
static void set_seed(options *o, const char *v) { o->seed = strtoull(v, NULL, 10); }
static void set_device(options *o, const char *v) { o->device = atoi(v); }
static void ignore(options *o, const char *v) {
    (void)o;
    (void)v;
}

static const struct {
    const char *name;
    void (*set)(options *, const char *);
} OPTIONS[] = {
    {"-m", set_model}, {"-c", set_ctx}, {"--seed", set_seed},
    {"--device", set_device}, {"--ram", ignore},
};

static int usage(const char *prog) {
    fprintf(stderr, "usage: %s -m model.mia [-c 4096] [--seed N] [--device D] [--ram SIZE]\n",
            prog);
    return 2;
}

int main(int argc, char **argv) {
    options o = {NULL, 4096, 0, (unsigned long long)time(NULL)};
    for (int i = 1; i < argc; i += 2) {
        size_t k = 0;
        while (k < sizeof OPTIONS / sizeof OPTIONS[0] && strcmp(argv[i], OPTIONS[k].name)) k++;
        if (k == sizeof OPTIONS / sizeof OPTIONS[0]) {
            fprintf(stderr, "%s: unknown option %s\n", argv[0], argv[i]);
            return usage(argv[0]);
        }
        if (i + 1 >= argc) {
            fprintf(stderr, "%s: option %s needs a value\n", argv[0], argv[i]);
            return usage(argv[0]);
        }
        OPTIONS[k].set(&o, argv[i + 1]);
    }
    if (!o.model) return usage(argv[0]);
    return mia_serve(o.model, o.ctx, (uint64_t)o.seed, o.device, stdin, stdout);
}
