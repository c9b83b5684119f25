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

}  // namespace mhip

namespace {

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
    if (c->stream) (void)hipStreamDestroy(c->stream);
    free(c);
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

int mhip_elapsed(mhip_ctx *c, int slot0, int slot1, float *ms) {
    if (slot0 < 0 || slot0 >= 16 || slot1 < 0 || slot1 >= 16)
        return mhip::fail(c, "mark slot out of range");
    if (mhip::check(c, hipEventSynchronize(c->marks[slot1]), "hipEventSynchronize")) return -1;
    return mhip::check(c, hipEventElapsedTime(ms, c->marks[slot0], c->marks[slot1]),
                       "hipEventElapsedTime");
}

}  // extern "C"
