// Internal declarations shared by the HIP translation units of libmotoria.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "mia_hip.h"

struct mhip_ctx {
    int device;
    hipStream_t stream;
    hipEvent_t marks[16];
    // stage timing (mhip_stage_timing)
    unsigned st_mask;
    int st_cap, st_n;
    hipEvent_t *st_ev;  // [2 * st_cap]
    int *st_stage;      // [st_cap]
    unsigned decode_epoch;  // launches of the decode kernel (tags its exchanged data)
    const void *decode_ws;  // workspace those tags were written to
    int decode_checked;           // 0 unknown, 1 the decode launch fits the device, 2 it does not
    int decode_cus, decode_occ;   // the CU count and occupancy that check found
    int capturing;                // between mhip_graph_begin and mhip_graph_end
    unsigned long long matrix_layers;  // mhip_moe_layer calls that took the matrix-core kernels
    unsigned attn_epoch;          // launches of the one-launch attention (its exchange tags)
    const void *attn_ws;          // the workspace those tags were written to
    char err[512];
};

namespace mhip {

constexpr int QK = 32;

int fail(mhip_ctx *c, const char *fmt, ...);
// Checks a HIP status (and the launch status when `launch` is set).
int check(mhip_ctx *c, hipError_t e, const char *what);
int check_launch(mhip_ctx *c, const char *what);
int use_device(mhip_ctx *c);

// Validates shapes every kernel of the path assumes; returns 0 or fail().
int check_dims(mhip_ctx *c, const mhip_dims *s);

// Brackets one launch of `stage` with events when stage timing selects it.
// stage_begin returns the record slot or -1; stage_end closes that slot.
int stage_begin(mhip_ctx *c, int stage);
void stage_end(mhip_ctx *c, int slot);

inline unsigned blocks_for(size_t n, unsigned per) {
    return (unsigned)((n + per - 1) / per);
}

// Once per device (at context set-up, that device current): the device
// address of the allocation-free decode workspace (decode.hip).
int decode_noalloc_setup(mhip_ctx *c);

// rmsnorm + Q8_0 of T rows of d values (the certified sum of moe_layer.hip;
// status[1] counts rows that took the sequential sum). Queues one launch.
void launch_rmsnorm_q8(hipStream_t st, const float *x, const float *w, float *xn, int8_t *xq,
                       float *xs, int T, int d, float eps, int force_seq, int *status);

// Matrix-core expert products (moe_gemm.hip).
bool gemm_path_fits(const mhip_dims *s);
int gemm_max_tiles(int A, int E);
int launch_gateup_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                       const void *d_table_layer, const mhip_scratch *sc, int A);
int launch_down_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                     const void *d_table_layer, const mhip_scratch *sc, int A, bool exact);

}  // namespace mhip

// ---- device helpers --------------------------------------------------------

#include "expf_glibc.h"

namespace mhip_dev {

__device__ __forceinline__ float expf_glibc(float x) { return mia_expf_glibc(x); }


// Exact int32 dot of two 32-value int8 blocks held as 2 x int4.
__device__ __forceinline__ int dot32_i8(const int4 a0, const int4 a1, const int4 b0,
                                        const int4 b1) {
    int acc = 0;
    acc = __builtin_amdgcn_sdot4(a0.x, b0.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a0.y, b0.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a0.z, b0.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a0.w, b0.w, acc, false);
    acc = __builtin_amdgcn_sdot4(a1.x, b1.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a1.y, b1.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a1.z, b1.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a1.w, b1.w, acc, false);
    return acc;
}

// The reference's per-block term ((float)acc * d_w) * d_x, two roundings.
__device__ __forceinline__ float block_term(int acc, float dw, float dx) {
    return ((float)acc * dw) * dx;
}

}  // namespace mhip_dev
