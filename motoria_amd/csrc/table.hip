// HBM-resident expert table: layout, upload/repack from the reference blob
// format, read-back, and the seeded synthetic generator.
//
// The reference streams one 5,308,416-byte blob per (layer, expert) from disk
// through an LRU cache (src/storage/expert_cache.c:59-85,
// src/storage/mia_file.c:121-126). Here every blob of every layer sits in one
// HBM allocation, regrouped once at upload: int8 codes of a matrix form a
// dense row-major array, the fp32 block scales a second array beside it, and
// a block-major copy of those scales a third (for the matrix-core kernels).
#include "mhip_internal.h"
#include "mia/synth.h"

namespace {

constexpr int QK = mhip::QK;

inline size_t align256(size_t n) { return (n + 255) / 256 * 256; }

struct ExpertGeom {
    int d, eh, E;
    size_t gate_q, up_q, down_q, gate_s, up_s, down_s, gate_st, up_st, down_st, expert_bytes;
};

ExpertGeom geom_of(const mhip_dims *s, const mhip_layout &l) {
    ExpertGeom g;
    g.d = s->dim;
    g.eh = s->expert_hidden;
    g.E = s->n_experts;
    g.gate_q = l.gate_q;
    g.up_q = l.up_q;
    g.down_q = l.down_q;
    g.gate_s = l.gate_s;
    g.up_s = l.up_s;
    g.down_s = l.down_s;
    g.gate_st = l.gate_st;
    g.up_st = l.up_st;
    g.down_st = l.down_st;
    g.expert_bytes = l.expert_bytes;
    return g;
}

// Which matrix / row / block a flat block number q of one expert names.
struct BlockRef {
    int m, row, blk, cols, nb;
};

__device__ __forceinline__ BlockRef block_ref(const ExpertGeom &g, size_t q) {
    const int nbd = g.d / QK, nbh = g.eh / QK;
    const size_t per_gu = (size_t)g.eh * nbd;
    BlockRef b;
    if (q < 2 * per_gu) {
        b.m = q < per_gu ? 0 : 1;
        size_t local = q - (size_t)b.m * per_gu;
        b.row = (int)(local / nbd);
        b.blk = (int)(local % nbd);
        b.cols = g.d;
        b.nb = nbd;
    } else {
        size_t local = q - 2 * per_gu;
        b.m = 2;
        b.row = (int)(local / nbh);
        b.blk = (int)(local % nbh);
        b.cols = g.eh;
        b.nb = nbh;
    }
    return b;
}

// Codes and scale of a block; *scale_t is the scale's block-major copy (may
// be null when not wanted).
__device__ __forceinline__ void block_addr(const ExpertGeom &g, uint8_t *expert,
                                           const BlockRef &b, int8_t **codes, float **scale,
                                           float **scale_t) {
    const size_t qoff = b.m == 0 ? g.gate_q : b.m == 1 ? g.up_q : g.down_q;
    const size_t soff = b.m == 0 ? g.gate_s : b.m == 1 ? g.up_s : g.down_s;
    const size_t toff = b.m == 0 ? g.gate_st : b.m == 1 ? g.up_st : g.down_st;
    const int rows = b.m == 2 ? g.d : g.eh;
    *codes = (int8_t *)(expert + qoff + (size_t)b.row * b.cols + (size_t)b.blk * QK);
    *scale = (float *)(expert + soff) + (size_t)b.row * b.nb + b.blk;
    if (scale_t) *scale_t = (float *)(expert + toff) + (size_t)b.blk * rows + b.row;
}

// One thread per 32-value block: draw 32 N(0, 0.02) values, quantize them
// exactly as src/tensor/quant.c:11-27 does, store codes and scale.
__global__ __launch_bounds__(256) void k_table_synth(ExpertGeom g, uint8_t *table, uint64_t seed,
                                                     int l0, size_t blocks_per_expert) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= blocks_per_expert) return;
    const int e = blockIdx.y % g.E;
    const int l = l0 + blockIdx.y / g.E;
    const BlockRef b = block_ref(g, q);
    const uint64_t key =
        mia_synth_key(seed, MIA_STREAM_EXPERT + ((uint64_t)l * g.E + e) * 3 + b.m);
    const uint64_t i0 = (uint64_t)b.row * b.cols + (uint64_t)b.blk * QK;
    float v[QK];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < QK; i++) {
        v[i] = mia_synth_f32(key, i0 + i, 0.02);
        float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    const float dsc = amax / 127.0f;
    const float inv = dsc != 0.0f ? 1.0f / dsc : 0.0f;
    union {
        int8_t c[QK];
        int4 v4[2];
    } out;
#pragma unroll
    for (int i = 0; i < QK; i++) out.c[i] = (int8_t)roundf(v[i] * inv);
    int8_t *codes;
    float *scale, *scale_t;
    block_addr(g, table + ((size_t)l * g.E + e) * g.expert_bytes, b, &codes, &scale, &scale_t);
    ((int4 *)codes)[0] = out.v4[0];
    ((int4 *)codes)[1] = out.v4[1];
    *scale = dsc;
    *scale_t = dsc;
}

// Reference blob (36-byte blocks) -> table slot.
__global__ __launch_bounds__(256) void k_repack(ExpertGeom g, uint8_t *expert,
                                                const uint8_t *blob, size_t off_up,
                                                size_t off_down, size_t blocks_per_expert) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= blocks_per_expert) return;
    const BlockRef b = block_ref(g, q);
    const size_t moff = b.m == 0 ? 0 : b.m == 1 ? off_up : off_down;
    const uint8_t *src = blob + moff + ((size_t)b.row * b.nb + b.blk) * 36;
    const uint32_t *s32 = (const uint32_t *)src;  // blocks are 4-byte aligned
    int8_t *codes;
    float *scale, *scale_t;
    block_addr(g, expert, b, &codes, &scale, &scale_t);
    *scale = __uint_as_float(s32[0]);
    *scale_t = __uint_as_float(s32[0]);
    int4 c0 = make_int4((int)s32[1], (int)s32[2], (int)s32[3], (int)s32[4]);
    int4 c1 = make_int4((int)s32[5], (int)s32[6], (int)s32[7], (int)s32[8]);
    ((int4 *)codes)[0] = c0;
    ((int4 *)codes)[1] = c1;
}

// Table slot -> reference blob (the caller zeroes the blob's padding).
__global__ __launch_bounds__(256) void k_unpack(ExpertGeom g, const uint8_t *expert,
                                                uint8_t *blob, size_t off_up,
                                                size_t off_down, size_t blocks_per_expert) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= blocks_per_expert) return;
    const BlockRef b = block_ref(g, q);
    const size_t moff = b.m == 0 ? 0 : b.m == 1 ? off_up : off_down;
    uint32_t *dst = (uint32_t *)(blob + moff + ((size_t)b.row * b.nb + b.blk) * 36);
    int8_t *codes;
    float *scale;
    block_addr(g, (uint8_t *)expert, b, &codes, &scale, nullptr);
    const int4 c0 = ((const int4 *)codes)[0];
    const int4 c1 = ((const int4 *)codes)[1];
    dst[0] = __float_as_uint(*scale);
    dst[1] = (uint32_t)c0.x;
    dst[2] = (uint32_t)c0.y;
    dst[3] = (uint32_t)c0.z;
    dst[4] = (uint32_t)c0.w;
    dst[5] = (uint32_t)c1.x;
    dst[6] = (uint32_t)c1.y;
    dst[7] = (uint32_t)c1.z;
    dst[8] = (uint32_t)c1.w;
}

// Position of element i of a router row in the decode layout: i = 32 L +
// 4 k + c goes to (k * d/32 + L) * 4 + c.
__device__ __forceinline__ int router_dl_pos(int i, int d) {
    return (((i & 31) >> 2) * (d / 32) + (i >> 5)) * 4 + (i & 3);
}

// Router of one layer, transposed (out_t[i*E + e] = W[e][i]) and, when
// out_dl is not null, in the decode layout.
__global__ __launch_bounds__(256) void k_router_synth(float *out_t, float *out_dl, int d, int E,
                                                      uint64_t key) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)d * E) return;
    const int e = (int)(q / d), i = (int)(q % d);
    const float v = mia_synth_f32(key, q, 0.02);
    out_t[(size_t)i * E + e] = v;
    if (out_dl) out_dl[(size_t)e * d + router_dl_pos(i, d)] = v;
}

__global__ __launch_bounds__(256) void k_router_dl(float *out, const float *in, int E, int d) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)d * E) return;
    const int e = (int)(q / d), i = (int)(q % d);
    out[(size_t)e * d + router_dl_pos(i, d)] = in[q];
}

__global__ __launch_bounds__(256) void k_transpose(float *out, const float *in, int E, int d) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)d * E) return;
    const int e = (int)(q / d), i = (int)(q % d);
    out[(size_t)i * E + e] = in[q];
}

__global__ __launch_bounds__(256) void k_synth_f32(float *out, size_t n, uint64_t key,
                                                   double sigma) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < n) out[q] = mia_synth_f32(key, q, sigma);
}

size_t blocks_per_expert(const mhip_dims *s) {
    return (size_t)2 * s->expert_hidden * (s->dim / QK) +
           (size_t)s->dim * (s->expert_hidden / QK);
}

}  // namespace

extern "C" {

int mhip_layout_of(const mhip_dims *s, mhip_layout *out) {
    if (mhip::check_dims(nullptr, s)) return -1;
    const size_t d = s->dim, eh = s->expert_hidden;
    size_t off = 0;
    out->gate_q = off;
    off = align256(off + eh * d);
    out->up_q = off;
    off = align256(off + eh * d);
    out->down_q = off;
    off = align256(off + d * eh);
    out->gate_s = off;
    off = align256(off + eh * (d / QK) * 4);
    out->up_s = off;
    off = align256(off + eh * (d / QK) * 4);
    out->down_s = off;
    off = align256(off + d * (eh / QK) * 4);
    out->gate_st = off;
    off = align256(off + eh * (d / QK) * 4);
    out->up_st = off;
    off = align256(off + eh * (d / QK) * 4);
    out->down_st = off;
    off = align256(off + d * (eh / QK) * 4);
    out->expert_bytes = off;
    return 0;
}

int mhip_table_synth(mhip_ctx *c, const mhip_dims *s, void *d_table, uint64_t seed, int l0,
                     int l1) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    if (l0 < 0 || l1 <= l0) return mhip::fail(c, "bad layer range [%d, %d)", l0, l1);
    mhip_layout lay;
    mhip_layout_of(s, &lay);
    const ExpertGeom g = geom_of(s, lay);
    const size_t bpe = blocks_per_expert(s);
    // Launch a few layers at a time so no grid dimension overflows.
    for (int l = l0; l < l1; l++) {
        dim3 grid(mhip::blocks_for(bpe, 256), (unsigned)s->n_experts);
        k_table_synth<<<grid, 256, 0, c->stream>>>(g, (uint8_t *)d_table, seed, l, bpe);
        if (mhip::check_launch(c, "table_synth")) return -1;
    }
    return 0;
}

int mhip_table_repack(mhip_ctx *c, const mhip_dims *s, void *d_table, int layer,
                      const int *experts, int n, const void *d_blobs, size_t blob_bytes,
                      size_t off_up, size_t off_down) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    mhip_layout lay;
    mhip_layout_of(s, &lay);
    const ExpertGeom g = geom_of(s, lay);
    const size_t bpe = blocks_per_expert(s);
    const size_t need_down = (size_t)s->dim * (s->expert_hidden / QK) * 36;
    if (off_up % 4 || off_down % 4 || blob_bytes % 4 || off_down + need_down > blob_bytes)
        return mhip::fail(c, "repack: blob geometry does not fit");
    for (int i = 0; i < n; i++) {
        if (experts[i] < 0 || experts[i] >= s->n_experts)
            return mhip::fail(c, "repack: expert %d out of range", experts[i]);
        uint8_t *dst = (uint8_t *)d_table +
                       ((size_t)layer * s->n_experts + experts[i]) * lay.expert_bytes;
        k_repack<<<mhip::blocks_for(bpe, 256), 256, 0, c->stream>>>(
            g, dst, (const uint8_t *)d_blobs + (size_t)i * blob_bytes, off_up, off_down, bpe);
        if (mhip::check_launch(c, "repack")) return -1;
    }
    return 0;
}

int mhip_table_unpack(mhip_ctx *c, const mhip_dims *s, const void *d_table, int layer,
                      int expert, void *d_blob, size_t blob_bytes, size_t off_up,
                      size_t off_down) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    if (expert < 0 || expert >= s->n_experts)
        return mhip::fail(c, "unpack: expert %d out of range", expert);
    mhip_layout lay;
    mhip_layout_of(s, &lay);
    const ExpertGeom g = geom_of(s, lay);
    const size_t bpe = blocks_per_expert(s);
    const size_t need_down = (size_t)s->dim * (s->expert_hidden / QK) * 36;
    if (off_up % 4 || off_down % 4 || off_down + need_down > blob_bytes)
        return mhip::fail(c, "unpack: blob geometry does not fit");
    if (mhip_zero(c, d_blob, blob_bytes)) return -1;
    const uint8_t *src =
        (const uint8_t *)d_table + ((size_t)layer * s->n_experts + expert) * lay.expert_bytes;
    k_unpack<<<mhip::blocks_for(bpe, 256), 256, 0, c->stream>>>(g, src, (uint8_t *)d_blob,
                                                                  off_up, off_down, bpe);
    return mhip::check_launch(c, "unpack");
}

int mhip_router_synth(mhip_ctx *c, const mhip_dims *s, float *d_router_t, float *d_router_dl,
                      uint64_t seed, int layer) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    const size_t n = (size_t)s->dim * s->n_experts;
    const uint64_t key = mia_synth_key(seed, MIA_STREAM_ROUTER + (uint64_t)layer);
    k_router_synth<<<mhip::blocks_for(n, 256), 256, 0, c->stream>>>(d_router_t, d_router_dl,
                                                                     s->dim, s->n_experts, key);
    return mhip::check_launch(c, "router_synth");
}

int mhip_router_decode_layout(mhip_ctx *c, const mhip_dims *s, float *d_router_dl,
                              const float *d_router) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    const size_t n = (size_t)s->dim * s->n_experts;
    k_router_dl<<<mhip::blocks_for(n, 256), 256, 0, c->stream>>>(d_router_dl, d_router,
                                                                  s->n_experts, s->dim);
    return mhip::check_launch(c, "router_decode_layout");
}

int mhip_router_transpose(mhip_ctx *c, const mhip_dims *s, float *d_router_t,
                          const float *d_router) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    const size_t n = (size_t)s->dim * s->n_experts;
    k_transpose<<<mhip::blocks_for(n, 256), 256, 0, c->stream>>>(d_router_t, d_router,
                                                                  s->n_experts, s->dim);
    return mhip::check_launch(c, "router_transpose");
}

int mhip_synth_f32(mhip_ctx *c, float *d_out, size_t n, uint64_t seed, uint64_t stream,
                   double sigma) {
    if (!n) return 0;
    if (mhip::use_device(c)) return -1;
    k_synth_f32<<<mhip::blocks_for(n, 256), 256, 0, c->stream>>>(
        d_out, n, mia_synth_key(seed, stream), sigma);
    return mhip::check_launch(c, "synth_f32");
}

}  // extern "C"
