// Device context, memory and timing for the thin C ABI (include/mia_hip.h).
#include <cstdlib>
#include <cstring>

#include "mhip_internal.h"

namespace mhip {

int fail(mhip_ctx *c, const char *fmt, ...) {
    if (c) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(c->err, sizeof(c->err), fmt, ap);
        va_end(ap);
    }
    return -1;
}

int check(mhip_ctx *c, hipError_t e, const char *what) {
    if (e == hipSuccess) return 0;
    return fail(c, "%s: %s", what, hipGetErrorString(e));
}

int check_launch(mhip_ctx *c, const char *what) {
    return check(c, hipGetLastError(), what);
}

int use_device(mhip_ctx *c) {
    return check(c, hipSetDevice(c->device), "hipSetDevice");
}

int check_dims(mhip_ctx *c, const mhip_dims *s) {
    if (!s) return fail(c, "null dims");
    if (s->dim <= 0 || s->dim % QK || s->dim > 8192)
        return fail(c, "dim %d: need a positive multiple of 32, <= 8192", s->dim);
    if (s->expert_hidden <= 0 || s->expert_hidden % QK || s->expert_hidden > 4096)
        return fail(c, "expert_hidden %d: need a positive multiple of 32, <= 4096",
                    s->expert_hidden);
    if (s->n_experts <= 0 || s->n_experts > 256)
        return fail(c, "n_experts %d: need 1..256", s->n_experts);
    if (s->n_active <= 0 || s->n_active > 64 || s->n_active > s->n_experts)
        return fail(c, "n_active %d: need 1..min(64, n_experts)", s->n_active);
    return 0;
}

int stage_begin(mhip_ctx *c, int stage) {
    if (c->capturing || !(c->st_mask & (1u << stage)) || c->st_n >= c->st_cap) return -1;
    const int slot = c->st_n++;
    c->st_stage[slot] = stage;
    (void)hipEventRecord(c->st_ev[2 * slot], c->stream);
    return slot;
}

void stage_end(mhip_ctx *c, int slot) {
    if (slot >= 0) (void)hipEventRecord(c->st_ev[2 * slot + 1], c->stream);
}

}  // namespace mhip

namespace {

void free_stage_events(mhip_ctx *c) {
    if (c->st_ev) {
        for (int i = 0; i < 2 * c->st_cap; i++)
            if (c->st_ev[i]) (void)hipEventDestroy(c->st_ev[i]);
    }
    free(c->st_ev);
    free(c->st_stage);
    c->st_ev = nullptr;
    c->st_stage = nullptr;
    c->st_cap = c->st_n = 0;
    c->st_mask = 0;
}

__global__ void k_fill_bytes(uint8_t *p, size_t n, uint8_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

__global__ void k_fill_u32(uint32_t *p, size_t n, uint32_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

}  // namespace

extern "C" {

int mhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int mhip_open(mhip_ctx **out, int device, char *err, size_t errlen) {
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        if (err && errlen) snprintf(err, errlen, "no HIP device: %s", hipGetErrorString(e));
        return -1;
    }
    if (device < 0 || device >= n) {
        if (err && errlen) snprintf(err, errlen, "device %d out of range (%d devices)", device, n);
        return -1;
    }
    mhip_ctx *c = (mhip_ctx *)calloc(1, sizeof(mhip_ctx));
    if (!c) {
        if (err && errlen) snprintf(err, errlen, "out of host memory");
        return -1;
    }
    c->device = device;
    int rc = mhip::use_device(c);
    if (!rc) rc = mhip::check(c, hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking),
                              "hipStreamCreate");
    for (int i = 0; i < 16 && !rc; i++)
        rc = mhip::check(c, hipEventCreate(&c->marks[i]), "hipEventCreate");
    if (!rc) rc = mhip::decode_noalloc_setup(c);
    if (rc) {
        if (err && errlen) snprintf(err, errlen, "%s", c->err);
        mhip_close(c);
        return -1;
    }
    *out = c;
    return 0;
}

void mhip_close(mhip_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (int i = 0; i < 16; i++)
        if (c->marks[i]) (void)hipEventDestroy(c->marks[i]);
    free_stage_events(c);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    free(c);
}

int mhip_stage_timing(mhip_ctx *c, unsigned mask, int max_launches) {
    if (mhip::use_device(c)) return -1;
    if (mhip::check(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return -1;
    free_stage_events(c);
    if (!mask || max_launches <= 0) return 0;
    c->st_ev = (hipEvent_t *)calloc((size_t)2 * max_launches, sizeof(hipEvent_t));
    c->st_stage = (int *)calloc((size_t)max_launches, sizeof(int));
    if (!c->st_ev || !c->st_stage) {
        free_stage_events(c);
        return mhip::fail(c, "out of host memory");
    }
    c->st_cap = max_launches;
    for (int i = 0; i < 2 * max_launches; i++)
        if (mhip::check(c, hipEventCreate(&c->st_ev[i]), "hipEventCreate")) {
            free_stage_events(c);
            return -1;
        }
    c->st_mask = mask;
    return 0;
}

int mhip_stage_time(mhip_ctx *c, int stage, double *ms, int *launches) {
    *ms = 0.0;
    *launches = 0;
    if (mhip::use_device(c)) return -1;
    if (mhip::check(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return -1;
    for (int i = 0; i < c->st_n; i++) {
        if (c->st_stage[i] != stage) continue;
        float t = 0.0f;
        if (mhip::check(c, hipEventElapsedTime(&t, c->st_ev[2 * i], c->st_ev[2 * i + 1]),
                        "hipEventElapsedTime"))
            return -1;
        *ms += t;
        (*launches)++;
    }
    return 0;
}

const char *mhip_error(const mhip_ctx *c) { return c ? c->err : "null context"; }

void *mhip_malloc(mhip_ctx *c, size_t bytes) {
    if (mhip::use_device(c)) return nullptr;
    void *p = nullptr;
    if (mhip::check(c, hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
    return p;
}

int mhip_free(mhip_ctx *c, void *d_ptr) {
    if (!d_ptr) return 0;
    if (mhip::use_device(c)) return -1;
    // Kernels queued on the stream may still read the buffer.
    if (mhip::check(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return -1;
    return mhip::check(c, hipFree(d_ptr), "hipFree");
}

int mhip_h2d(mhip_ctx *c, void *d_dst, const void *src, size_t bytes) {
    if (mhip::use_device(c)) return -1;
    if (mhip::check(c, hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, c->stream),
                    "hipMemcpyAsync h2d"))
        return -1;
    return mhip::check(c, hipStreamSynchronize(c->stream), "h2d sync");
}

int mhip_d2h(mhip_ctx *c, void *dst, const void *d_src, size_t bytes) {
    if (mhip::use_device(c)) return -1;
    if (mhip::check(c, hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, c->stream),
                    "hipMemcpyAsync d2h"))
        return -1;
    return mhip::check(c, hipStreamSynchronize(c->stream), "d2h sync");
}

void *mhip_host_malloc(mhip_ctx *c, size_t bytes) {
    if (mhip::use_device(c)) return nullptr;
    void *p = nullptr;
    if (mhip::check(c, hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault),
                    "hipHostMalloc"))
        return nullptr;
    return p;
}

int mhip_host_free(mhip_ctx *c, void *h_ptr) {
    if (!h_ptr) return 0;
    if (mhip::use_device(c)) return -1;
    // Copies queued on the stream may still use the buffer.
    if (mhip::check(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return -1;
    return mhip::check(c, hipHostFree(h_ptr), "hipHostFree");
}

int mhip_h2d_async(mhip_ctx *c, void *d_dst, const void *h_src, size_t bytes) {
    if (mhip::use_device(c)) return -1;
    return mhip::check(c, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, c->stream),
                       "hipMemcpyAsync h2d");
}

int mhip_d2h_async(mhip_ctx *c, void *h_dst, const void *d_src, size_t bytes) {
    if (mhip::use_device(c)) return -1;
    return mhip::check(c, hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, c->stream),
                       "hipMemcpyAsync d2h");
}

int mhip_d2d(mhip_ctx *c, void *d_dst, const void *d_src, size_t bytes) {
    if (mhip::use_device(c)) return -1;
    return mhip::check(c, hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, c->stream),
                       "hipMemcpyAsync d2d");
}

int mhip_zero(mhip_ctx *c, void *d_ptr, size_t bytes) {
    if (!bytes) return 0;
    if (mhip::use_device(c)) return -1;
    const unsigned grid = 1024;
    if ((uintptr_t)d_ptr % 4 == 0 && bytes % 4 == 0)
        k_fill_u32<<<grid, 256, 0, c->stream>>>((uint32_t *)d_ptr, bytes / 4, 0u);
    else
        k_fill_bytes<<<grid, 256, 0, c->stream>>>((uint8_t *)d_ptr, bytes, 0);
    return mhip::check_launch(c, "fill");
}

int mhip_fill_f32(mhip_ctx *c, float *d_out, size_t n, float value) {
    if (!n) return 0;
    if (mhip::use_device(c)) return -1;
    uint32_t bits;
    memcpy(&bits, &value, 4);
    k_fill_u32<<<1024, 256, 0, c->stream>>>((uint32_t *)d_out, n, bits);
    return mhip::check_launch(c, "fill_f32");
}

int mhip_sync(mhip_ctx *c) {
    if (mhip::use_device(c)) return -1;
    return mhip::check(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

int mhip_mark(mhip_ctx *c, int slot) {
    if (slot < 0 || slot >= 16) return mhip::fail(c, "mark slot %d out of range", slot);
    return mhip::check(c, hipEventRecord(c->marks[slot], c->stream), "hipEventRecord");
}

int mhip_mark_wait(mhip_ctx *c, int slot) {
    if (slot < 0 || slot >= 16) return mhip::fail(c, "mark slot %d out of range", slot);
    return mhip::check(c, hipEventSynchronize(c->marks[slot]), "hipEventSynchronize");
}

int mhip_elapsed(mhip_ctx *c, int slot0, int slot1, float *ms) {
    if (slot0 < 0 || slot0 >= 16 || slot1 < 0 || slot1 >= 16)
        return mhip::fail(c, "mark slot out of range");
    if (mhip::check(c, hipEventSynchronize(c->marks[slot1]), "hipEventSynchronize")) return -1;
    return mhip::check(c, hipEventElapsedTime(ms, c->marks[slot0], c->marks[slot1]),
                       "hipEventElapsedTime");
}

}  // extern "C"

// ---- HIP graphs ---------------------------------------------------------------

struct mhip_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

extern "C" {

int mhip_graph_begin(mhip_ctx *c) {
    if (c->capturing) return mhip::fail(c, "a capture is already open on this context");
    if (mhip::use_device(c)) return -1;
    if (mhip::check(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal),
                    "hipStreamBeginCapture"))
        return -1;
    c->capturing = 1;
    return 0;
}

int mhip_graph_end(mhip_ctx *c, mhip_graph **out) {
    if (out) *out = nullptr;
    if (!c->capturing) return mhip::fail(c, "no capture is open on this context");
    c->capturing = 0;
    hipGraph_t g = nullptr;
    if (mhip::check(c, hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture")) {
        if (g) (void)hipGraphDestroy(g);
        return -1;
    }
    if (!out) {  // the caller abandons the capture
        (void)hipGraphDestroy(g);
        return 0;
    }
    mhip_graph *r = (mhip_graph *)calloc(1, sizeof(mhip_graph));
    if (!r) {
        (void)hipGraphDestroy(g);
        return mhip::fail(c, "out of host memory");
    }
    r->graph = g;
    if (mhip::check(c, hipGraphInstantiate(&r->exec, g, nullptr, nullptr, 0),
                    "hipGraphInstantiate")) {
        (void)hipGraphDestroy(g);
        free(r);
        return -1;
    }
    *out = r;
    return 0;
}

int mhip_graph_launch(mhip_ctx *c, mhip_graph *g) {
    if (!g) return mhip::fail(c, "null graph");
    if (mhip::use_device(c)) return -1;
    return mhip::check(c, hipGraphLaunch(g->exec, c->stream), "hipGraphLaunch");
}

void mhip_graph_destroy(mhip_graph *g) {
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    free(g);
}

}  // extern "C"
