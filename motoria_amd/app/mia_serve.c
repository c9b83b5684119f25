/*
 * mia-serve on the GPU engine: the reference's server command line
 * (src/app/serve.c:145-160) over mia_serve (include/mia/serve.h).
 *
 *   mia-serve -m model.mia [-c 4096] [--seed N] [--device D] [--ram SIZE]
 *
 * --ram is accepted for the reference's callers (tools/internal/engine
 * passes it) and ignored: every expert is resident in HBM.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "mia/serve.h"

int main(int argc, char **argv) {
    const char *model = NULL;
    int ctx = 4096, device = 0;
    unsigned long long seed = (unsigned long long)time(NULL);
    for (int i = 1; i + 1 < argc; i += 2) {
        if (!strcmp(argv[i], "-m")) model = argv[i + 1];
        else if (!strcmp(argv[i], "-c")) ctx = atoi(argv[i + 1]);
        else if (!strcmp(argv[i], "--seed")) seed = strtoull(argv[i + 1], NULL, 10);
        else if (!strcmp(argv[i], "--device")) device = atoi(argv[i + 1]);
        else if (strcmp(argv[i], "--ram") != 0) {
            fprintf(stderr, "unknown option %s\n", argv[i]);
            return 2;
        }
    }
    if (!model) {
        fprintf(stderr, "usage: %s -m model.mia [-c 4096] [--seed N] [--device D] [--ram SIZE]\n",
                argv[0]);
        return 2;
    }
    return mia_serve(model, ctx, (uint64_t)seed, device, stdin, stdout);
}
