// One Qwen3-MoE FFN layer over T tokens on the resident expert table:
//
//   k_rmsnorm_q8          rmsnorm + Q8_0 quantization of xn      forward.c:174, quant.c:11-27
//   k_router_logits_wide  router chains for T > 1 (tokens across the lanes)
//   k_router              softmax, top-K, gate weights (and the chains at T = 1)
//                                                                 forward.c:175-181
//   k_disp_*              stable bucketing of the T*K assignments by expert
//   k_gateup              gate/up Q8 products + SwiGLU          forward.c:186-191
//   k_quant_h, k_down     Q8(h) + down Q8 product               forward.c:192-193
//   k_combine             x += w_j * tmp_j, j in top-K order    forward.c:194
//
// Every fp32 value is produced in the reference's operation order, so the
// results are bit-equal to the reference C path (src/model/forward.c:167-197
// on x86): block dots are exact int32, the per-row sums over 32-value blocks
// run in block order, and sums the reference takes in double are either
// reproduced exactly or certified (see k_rmsnorm_q8). For large batches the
// gate/up and down stages switch to the matrix-core kernels of moe_gemm.hip
// (exact block dots; h and Q8(h) bit-equal, the expert outputs within a few
// ulps); routing and dispatch stay bit-exact.
//
// Status words (sc->status, cleared by the host per call): [0] bit 0 = an
// expert index out of range; [1] rmsnorm sums that took the sequential path;
// [2] 1 + the ordinal (since the clear) of the first layer launch that met a
// bad index; [3] layer launches completed since the clear.
#include "mhip_internal.h"

namespace {

constexpr int QK = mhip::QK;
constexpr int NT = 256;  // threads per workgroup of the GEMV stages
constexpr int TB = 4;    // tokens per pass of the GEMV stages

__host__ __device__ inline size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// ---- rmsnorm + Q8 -------------------------------------------------------
//
// The reference sums x^2 in double, sequentially (forward.c:77-78), then
// inv = (float)(1/sqrt(ss/n + eps)). Each x^2 is exact in double; only the
// order of the additions is at stake. A tree sum S differs from the
// sequential one by at most (n + log2 n) * 2^-53 * S (all terms are >= 0),
// so with S -/+ m, m = (n + 64) * 2^-52 * S, the two inv candidates bracket
// the reference's inv (every IEEE step is monotone). When they agree they are
// the reference's value; otherwise (probability ~1e-5 per token) one thread
// redoes the sequential sum. status[1] counts those fallbacks.
__global__ __launch_bounds__(NT) void k_rmsnorm_q8(const float *__restrict__ x,
                                                   const float *__restrict__ w,
                                                   float *__restrict__ xn,
                                                   int8_t *__restrict__ xq,
                                                   float *__restrict__ xs,
                                                   _Float16 *__restrict__ xq16, int d, float eps,
                                                   int force_seq, int *status) {
    __shared__ double part[NT / 64];
    __shared__ float inv_sh;
    const int t = blockIdx.x;
    const float *xt = x + (size_t)t * d;
    double s = 0.0;
    for (int i = threadIdx.x; i < d; i += NT) {
        const double v = (double)xt[i];
        s = s + v * v;
    }
    for (int o = 32; o > 0; o >>= 1) s = s + __shfl_xor(s, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double S = part[0];
        for (int i = 1; i < NT / 64; i++) S = S + part[i];
        const double m = S * ((double)(d + 64) * 0x1p-52);
        const float lo = (float)(1.0 / sqrt((S + m) / d + (double)eps));
        const float hi = (float)(1.0 / sqrt((S - m) / d + (double)eps));
        float inv = lo;
        if (force_seq || lo != hi) {
            double ss = 0.0;
            for (int i = 0; i < d; i++) ss = ss + (double)xt[i] * (double)xt[i];
            inv = (float)(1.0 / sqrt(ss / d + (double)eps));
            atomicAdd(&status[1], 1);
        }
        inv_sh = inv;
    }
    __syncthreads();
    const float inv = inv_sh;
    const int nb = d / QK;
    // 32 consecutive threads own one block; d is a multiple of 32, so a
    // block is either wholly inside [0, d) or wholly outside.
    for (int i0 = 0; i0 < d; i0 += NT) {
        const int i = i0 + threadIdx.x;
        const bool in = i < d;
        const float v = in ? (xt[i] * inv) * w[i] : 0.0f;
        float a = fabsf(v);
        for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
        const float dsc = a / 127.0f;
        const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
        if (in) {
            const float q = roundf(v * qi);
            xn[(size_t)t * d + i] = v;
            xq[(size_t)t * d + i] = (int8_t)q;
            if (xq16) xq16[(size_t)t * d + i] = (_Float16)q;
            if ((i & 31) == 0) xs[(size_t)t * nb + i / QK] = dsc;
        }
    }
}

// The same for d == 2048 with one wavefront per token (four per workgroup):
// lane b owns the 32-block b of the row, so the Q8_0 block maximum is the
// lane's own, and only the sum of squares crosses lanes (a wavefront tree
// with the same certified bracket; lane 0 redoes the sequential sum when the
// bracket is ambiguous).
constexpr int RN_D = 2048;
__global__ __launch_bounds__(256) void k_rmsnorm_q8_w(const float *__restrict__ x,
                                                     const float *__restrict__ w,
                                                     float *__restrict__ xn,
                                                     int8_t *__restrict__ xq,
                                                     float *__restrict__ xs,
                                                     _Float16 *__restrict__ xq16, int T,
                                                     float eps, int force_seq, int *status) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), b = threadIdx.x & 63;
    if (t >= T) return;  // a whole wavefront: no workgroup barrier follows
    const float4 *xr = (const float4 *)(x + (size_t)t * RN_D + 32 * b);
    const float4 *wr = (const float4 *)(w + 32 * b);
    float v[32];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float4 q = xr[k];
        v[4 * k] = q.x;
        v[4 * k + 1] = q.y;
        v[4 * k + 2] = q.z;
        v[4 * k + 3] = q.w;
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 32; k++) ss = ss + (double)v[k] * (double)v[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss = ss + __shfl_xor(ss, o);
    ss = __shfl(ss, 0);  // one value for the whole wavefront (lanes summed in different orders)
    const double m = ss * ((double)(RN_D + 64) * 0x1p-52);
    const float lo = (float)(1.0 / sqrt((ss + m) / RN_D + (double)eps));
    const float hi = (float)(1.0 / sqrt((ss - m) / RN_D + (double)eps));
    float inv = lo;
    if (force_seq || lo != hi) {  // the same branch in every lane of the wavefront
        float r = 0.0f;
        if (b == 0) {
            const float *xt = x + (size_t)t * RN_D;
            double sq = 0.0;
            for (int i = 0; i < RN_D; i++) sq = sq + (double)xt[i] * (double)xt[i];
            r = (float)(1.0 / sqrt(sq / RN_D + (double)eps));
            atomicAdd(&status[1], 1);
        }
        inv = __shfl(r, 0);
    }
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float4 q = wr[k];
        v[4 * k] = (v[4 * k] * inv) * q.x;
        v[4 * k + 1] = (v[4 * k + 1] * inv) * q.y;
        v[4 * k + 2] = (v[4 * k + 2] * inv) * q.z;
        v[4 * k + 3] = (v[4 * k + 3] * inv) * q.w;
    }
#pragma unroll
    for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(v[k]));
    const float dsc = amax / 127.0f;
    const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
    float4 *xo = (float4 *)(xn + (size_t)t * RN_D + 32 * b);
#pragma unroll
    for (int k = 0; k < 8; k++)
        xo[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    union {
        int8_t c[32];
        int4 q[2];
    } qc;
#pragma unroll
    for (int k = 0; k < 32; k++) qc.c[k] = (int8_t)roundf(v[k] * qi);
    int4 *qo = (int4 *)(xq + (size_t)t * RN_D + 32 * b);
    qo[0] = qc.q[0];
    qo[1] = qc.q[1];
    if (xq16) {
        typedef _Float16 h8v __attribute__((ext_vector_type(8)));
        h8v *ho = (h8v *)(xq16 + (size_t)t * RN_D + 32 * b);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            h8v hv;
#pragma unroll
            for (int e = 0; e < 8; e++) hv[e] = (_Float16)qc.c[8 * k + e];
            ho[k] = hv;
        }
    }
    xs[(size_t)t * (RN_D / QK) + b] = dsc;
}

// The same for many tokens, with every access coalesced: load k (k < 8) of
// a wavefront is one contiguous 1 KB run, lane L taking elements
// 256 k + 4 L .. + 3, so a 32-block is the four values of eight consecutive
// lanes of one load and its maximum is taken over them by DPP (order-free).
// The sum of squares is the per-lane sequential sums and a wavefront tree,
// bracketed as above. Without xq (the matrix-core path reads only the fp16
// codes) the int8 codes are not written.
template <int CTRL>
__device__ __forceinline__ float dpp_max_f(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                                CTRL, 0xf, 0xf, false)));
}
__global__ __launch_bounds__(256) void k_rmsnorm_q8_c(const float *__restrict__ x,
                                                     const float *__restrict__ w,
                                                     float *__restrict__ xn,
                                                     int8_t *__restrict__ xq,
                                                     float *__restrict__ xs,
                                                     _Float16 *__restrict__ xq16, int T,
                                                     float eps, int force_seq, int *status) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), L = threadIdx.x & 63;
    if (t >= T) return;  // a whole wavefront: no workgroup barrier follows
    const float4 *xr = (const float4 *)(x + (size_t)t * RN_D) + L;
    float4 v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = xr[64 * k];
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        ss = ss + (double)v[k].x * (double)v[k].x;
        ss = ss + (double)v[k].y * (double)v[k].y;
        ss = ss + (double)v[k].z * (double)v[k].z;
        ss = ss + (double)v[k].w * (double)v[k].w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss = ss + __shfl_xor(ss, o);
    ss = __shfl(ss, 0);  // one value for the whole wavefront (lanes summed in different orders)
    const double m = ss * ((double)(RN_D + 64) * 0x1p-52);
    const float lo = (float)(1.0 / sqrt((ss + m) / RN_D + (double)eps));
    const float hi = (float)(1.0 / sqrt((ss - m) / RN_D + (double)eps));
    float inv = lo;
    if (force_seq || lo != hi) {  // the same branch in every lane of the wavefront
        float r = 0.0f;
        if (L == 0) {
            const float *xt = x + (size_t)t * RN_D;
            double sq = 0.0;
            for (int i = 0; i < RN_D; i++) sq = sq + (double)xt[i] * (double)xt[i];
            r = (float)(1.0 / sqrt(sq / RN_D + (double)eps));
            atomicAdd(&status[1], 1);
        }
        inv = __shfl(r, 0);
    }
    const float4 *wr = (const float4 *)w + L;
    float4 *xo = (float4 *)(xn + (size_t)t * RN_D) + L;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float4 q = wr[64 * k];
        v[k] = make_float4((v[k].x * inv) * q.x, (v[k].y * inv) * q.y, (v[k].z * inv) * q.z,
                           (v[k].w * inv) * q.w);
        xo[64 * k] = v[k];
    }
    typedef _Float16 h4v __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int k = 0; k < 8; k++) {
        // a NaN counts as 0 in the block maximum, as in the sequential max
        float am = fmaxf(fmaxf(fmaxf(0.0f, fabsf(v[k].x)), fabsf(v[k].y)),
                         fmaxf(fabsf(v[k].z), fabsf(v[k].w)));
        am = dpp_max_f<0xB1>(am);   // quad_perm [1,0,3,2]
        am = dpp_max_f<0x4E>(am);   // quad_perm [2,3,0,1]
        am = dpp_max_f<0x141>(am);  // row_half_mirror: the other quad of the 8 lanes
        const float dsc = am / 127.0f;
        const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
        const int c0 = (int)roundf(v[k].x * qi), c1 = (int)roundf(v[k].y * qi),
                  c2 = (int)roundf(v[k].z * qi), c3 = (int)roundf(v[k].w * qi);
        if (xq)
            ((int *)(xq + (size_t)t * RN_D))[L + 64 * k] =
                (c0 & 0xff) | (c1 & 0xff) << 8 | (c2 & 0xff) << 16 | (int)((unsigned)c3 << 24);
        if (xq16) {
            const h4v hv = {(_Float16)c0, (_Float16)c1, (_Float16)c2, (_Float16)c3};
            ((h4v *)(xq16 + (size_t)t * RN_D))[L + 64 * k] = hv;
        }
        if ((L & 7) == 0) xs[(size_t)t * (RN_D / QK) + 8 * k + L / 8] = dsc;
    }
}
// Tokens from which the coalesced kernel takes over (fewer tokens fill too
// few CUs for its shorter per-lane work to pay).
constexpr int RN_COALESCED_T = 256;

// Softmax, top-K and renormalisation of token t's logits (forward.c:95-114,
// 178-181): thread e < E holds logit l (threads >= E hold -inf); every
// thread of the workgroup calls it (E <= blockDim.x). p: E floats of LDS;
// keys (16-byte aligned), red, sum_sh, top: LDS scratch (E keys,
// blockDim.x / 64 floats, one float, K ints).
__device__ __forceinline__ void route_select(float l, int t, int E, int K, int norm_topk,
                                             float *p, unsigned long long *keys, float *red,
                                             float *sum_sh, int *top,
                                             int *__restrict__ idx_out,
                                             float *__restrict__ w_out) {
    const int tid = threadIdx.x;
    // max over E (order-free)
    float mx = l;
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) mx = fmaxf(mx, red[i]);
    if (tid < E) p[tid] = mhip_dev::expf_glibc(l - mx);
    __syncthreads();
    if (tid == 0) {
        // in index order, sixteen values read ahead of their additions
        float sum = 0.0f;
        int i = 0;
        for (; i + 16 <= E; i += 16) {
            float4 q[4];
#pragma unroll
            for (int k = 0; k < 4; k++) q[k] = *(const float4 *)&p[i + 4 * k];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                sum = sum + q[k].x;
                sum = sum + q[k].y;
                sum = sum + q[k].z;
                sum = sum + q[k].w;
            }
        }
        for (; i < E; i++) sum = sum + p[i];
        *sum_sh = sum;
    }
    __syncthreads();
    if (tid < E) p[tid] = p[tid] / *sum_sh;
    __syncthreads();

    // Top-K (forward.c:104-114: the largest untaken probability, the lowest
    // index among equal ones) as ranks: probabilities are >= +0, so their
    // bit patterns order like the values, and the low word ~index makes the
    // lowest index win a tie; an entry's rank is the number of larger keys,
    // and ranks 0..K-1 are the K picks in order.
    if (tid < E)
        keys[tid] = ((unsigned long long)__float_as_uint(p[tid]) << 32) |
                    (unsigned long long)(0xFFFFFFFFu - (unsigned)tid);
    __syncthreads();
    if (tid < E) {
        const unsigned long long ke = keys[tid];
        int rk = 0;
        int i = 0;
        for (; i + 2 <= E; i += 2) {
            const ulonglong2 kv = *(const ulonglong2 *)&keys[i];
            rk += (int)(kv.x > ke) + (int)(kv.y > ke);
        }
        for (; i < E; i++) rk += (int)(keys[i] > ke);
        if (rk < K) top[rk] = tid;
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int j = 0; j < K; j++) sum = sum + p[top[j]];
        for (int j = 0; j < K; j++) {
            const float wj = p[top[j]];
            idx_out[(size_t)t * K + j] = top[j];
            w_out[(size_t)t * K + j] = norm_topk ? wj / sum : wj;
        }
    }
}

// ---- router ---------------------------------------------------------------
//
// Thread e computes logit e as the reference's sequential fp32 chain
// (matmul.c:13-17) over xn staged in LDS, reading the transposed router so
// a wavefront's loads are contiguous. Softmax (forward.c:95-101) uses the
// restated glibc expf and a sequential sum; top-K (forward.c:104-114) takes
// the largest untaken probability, lowest index on ties; the gate weights
// are renormalised as forward.c:178-181.
//
// With have_logits set (every shape with d % 64 == 0 and E % 4 == 0), the
// logits (bias included) were already computed by k_router_logits_wide (or
// k_router_logits) and only the selection runs.
__global__ __launch_bounds__(256) void k_router(const float *__restrict__ xn,
                                                const float *__restrict__ wt,
                                                const float *__restrict__ bias,
                                                float *__restrict__ logits,
                                                int *__restrict__ idx_out,
                                                float *__restrict__ w_out, int d, int E, int K,
                                                int norm_topk, int have_logits) {
    extern __shared__ __align__(16) float sh[];
    float *p = sh;        // [E]
    float *xs = sh + E;   // [d] (chains computed here)
    __shared__ __align__(16) unsigned long long keys[256];
    __shared__ float red[4];
    __shared__ float sum_sh;
    __shared__ int top[64];
    const int t = blockIdx.x;
    const int tid = threadIdx.x;
    if (!have_logits) {
        for (int i = tid; i < d; i += blockDim.x) xs[i] = xn[(size_t)t * d + i];
        __syncthreads();
    }

    float l = -__builtin_inff();
    if (tid < E && have_logits) {
        l = logits[(size_t)t * E + tid];
    } else if (tid < E) {
        const float *col = wt + tid;
        float s = 0.0f;
        int i = 0;
        for (; i + 8 <= d; i += 8) {
            float wv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) wv[k] = col[(size_t)(i + k) * E];
#pragma unroll
            for (int k = 0; k < 8; k++) s = s + wv[k] * xs[i + k];
        }
        for (; i < d; i++) s = s + col[(size_t)i * E] * xs[i];
        if (bias) s = s + bias[tid];
        l = s;
        logits[(size_t)t * E + tid] = s;
    }
    route_select(l, t, E, K, norm_topk, p, keys, red, &sum_sh, top, idx_out, w_out);
}

// ---- router logits for many tokens ----------------------------------------------
//
// The same sequential fp32 chains (matmul.c:13-17, plus the bias), tiled:
// a workgroup takes 2C tokens, thread (e, g) runs the chains of expert e for
// tokens g*C .. g*C+C-1 (C independent chains, one weight read for all).
// The workgroup's xn rows sit in LDS (transposed) for the whole kernel; the
// transposed router streams through an RL_NS-stage LDS ring of RL_I rows,
// loaded straight from global memory (global_load_lds, issued from inline
// assembly that sets M0) RL_NS-1 chunks ahead, with explicit waits. Each
// wavefront issues four 1 KB loads per chunk. Needs E == 128.
constexpr int RL_I = 32;
constexpr int RL_NS = 4;
constexpr int RL_E = 128;

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void rl_dma16(unsigned lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g)
                 : "memory", "m0");
}
// 4 bytes per lane, lane i's at lds + 4 i.
__device__ __forceinline__ void rl_dma4(unsigned lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(g)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

template <int C>
__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ xn,
                                                       const float *__restrict__ wt,
                                                       const float *__restrict__ bias,
                                                       float *__restrict__ logits, int T, int d) {
    constexpr int TT = 2 * C;
    extern __shared__ __align__(16) float rl_sh[];
    float (*Wr)[RL_I][RL_E] = (float (*)[RL_I][RL_E])rl_sh;  // [stage][i][e]
    float *Xs = rl_sh + RL_NS * RL_I * RL_E;                  // [i][TT]
    const int tid = threadIdx.x, e = tid & (RL_E - 1), g = tid >> 7;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int t0 = blockIdx.x * TT;
    const int nch = d / RL_I;
    // chunk ch -> stage ch % RL_NS; wavefront w loads rows 8w..8w+7 of the
    // chunk, two 512-byte rows per instruction
    const unsigned ring = (unsigned)(uintptr_t)rl_sh;
    auto issue = [&](int ch) {
        const int k = min(ch, nch - 1);
        const unsigned st = ring + (unsigned)((ch % RL_NS) * RL_I * RL_E * 4);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int row = 8 * wave + 2 * q;
            rl_dma16(st + (unsigned)(row * RL_E * 4),
                     wt + (size_t)(k * RL_I + row + (lane >> 5)) * RL_E + 4 * (lane & 31));
        }
    };
#pragma unroll
    for (int c = 0; c < RL_NS - 1; c++) issue(c);
    // xn of the workgroup's tokens, transposed, while the first chunks load
    for (int f = tid; f < TT * (d / 4); f += 256) {
        const int t = f / (d / 4), i4 = f % (d / 4);
        const float4 v = t0 + t < T ? *(const float4 *)(xn + (size_t)(t0 + t) * d + 4 * i4)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        Xs[(4 * i4 + 0) * TT + t] = v.x;
        Xs[(4 * i4 + 1) * TT + t] = v.y;
        Xs[(4 * i4 + 2) * TT + t] = v.z;
        Xs[(4 * i4 + 3) * TT + t] = v.w;
    }
    float s[C];
#pragma unroll
    for (int c = 0; c < C; c++) s[c] = 0.0f;
    for (int ch = 0; ch < nch; ch++) {
        // this wavefront's loads of chunk ch are done (later ones may still
        // be in flight), then every wavefront's (and the xn staging)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((RL_NS - 2) * 4) : "memory");
        __syncthreads();
        issue(ch + RL_NS - 1);  // into the stage read in chunk ch - 1
        const float(*W)[RL_E] = Wr[ch % RL_NS];
        const float *X = Xs + (size_t)ch * RL_I * TT + g * C;
#pragma unroll 8
        for (int ii = 0; ii < RL_I; ii++) {
            const float w = W[ii][e];
#pragma unroll
            for (int c = 0; c < C; c++) s[c] = s[c] + w * X[ii * TT + c];
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the reloads past the end
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int t = t0 + g * C + c;
        if (t < T) logits[(size_t)t * RL_E + e] = bias ? s[c] + bias[e] : s[c];
    }
}

size_t router_logits_lds(int C, int d) {
    return ((size_t)RL_NS * RL_I * RL_E + (size_t)d * 2 * C) * sizeof(float);
}

// ---- router logits for batches of tokens --------------------------------------------
//
// The same chains with the tokens across the lanes: a workgroup takes RW_T = 64
// tokens (lane = token) and 4 CPL experts (wavefront w: experts CPL w ..
// CPL w + CPL - 1), so every lane runs CPL chains over one token and every
// router value is a wavefront-wide broadcast. xn (token-major, rows padded to
// RW_I + 4 floats so that eight lanes reading 16 bytes of their own rows hit
// distinct banks) and the router values (wavefront-major) go through LDS in
// chunks of RW_I values of i, double-buffered in LDS and 4 / CPL chunks ahead
// in registers; each lane reads four values of i of both with 16-byte reads.
// CPL trades chains per lane against workgroups (CPL = 1 for a few tokens).
// Needs d % RW_I == 0 and E % (4 CPL) == 0.
constexpr int RW_T = 64, RW_I = 64, RW_LD = RW_I + 4;

template <int CPL>
struct alignas(4 * CPL) RwVec {
    float v[CPL];
};

template <int CPL>
__global__ __launch_bounds__(256, 2) void k_router_logits_wide(const float *__restrict__ xn,
                                                               const float *__restrict__ wt,
                                                               const float *__restrict__ bias,
                                                               float *__restrict__ logits, int T,
                                                               int d, int E) {
    typedef RwVec<CPL> V;
    // chunks in flight in registers: a chunk's compute shrinks with CPL, so
    // fewer chains per lane prefetch further ahead
    constexpr int NP = 4 / CPL;
    constexpr int BI = 32;  // one chain per lane: values of i read from LDS per batch
    __shared__ __align__(16) float Xs[2][RW_T][RW_LD];
    __shared__ __align__(16) V Ws[2][4][RW_I];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * RW_T, e0 = blockIdx.y * 4 * CPL;
    // this thread's loads of a chunk: 16 values of xn row tt (from i0 + 16 q),
    // and the CPL router values of row i0 + tid / 4, experts e0 + CPL (tid % 4) ..
    const int tt = tid >> 2, q = tid & 3;
    const float *xsrc = xn + (size_t)min(t0 + tt, T - 1) * d + 16 * q;
    const float *wsrc = wt + (size_t)(tid >> 2) * E + e0 + CPL * (tid & 3);
    float4 xr[NP][4];
    V wr[NP];
    auto gload = [&](int ch, int sl) {
        const int i0 = ch * RW_I;
#pragma unroll
        for (int k = 0; k < 4; k++) xr[sl][k] = *(const float4 *)(xsrc + i0 + 4 * k);
        wr[sl] = *(const V *)(wsrc + (size_t)i0 * E);
    };
    auto lstore = [&](int sl, int b) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float *dst = &Xs[b][tt][16 * q + 4 * k];
            dst[0] = xr[sl][k].x;
            dst[1] = xr[sl][k].y;
            dst[2] = xr[sl][k].z;
            dst[3] = xr[sl][k].w;
        }
        Ws[b][tid & 3][tid >> 2] = wr[sl];
    };
    float s[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) s[c] = 0.0f;
    const int nch = d / RW_I;
    // chunk c travels in register slot c % NP, then LDS buffer c & 1
    gload(0, 0);
    lstore(0, 0);
#pragma unroll
    for (int p = 1; p <= NP; p++)
        if (p < nch) gload(p, p % NP);
    __syncthreads();
    for (int ch = 0; ch < nch; ch += NP) {
#pragma unroll
        for (int u = 0; u < NP; u++) {
            const int c = ch + u;
            if (c >= nch) break;
            const int b = c & 1;
            if constexpr (CPL == 1) {
                // one chain per lane: BI values of i at a time, all their LDS
                // reads first (one wait), then the additions back to back
#pragma unroll
                for (int ii = 0; ii < RW_I; ii += BI) {
                    float x[BI];
                    V w[BI];
#pragma unroll
                    for (int j = 0; j < BI; j += 4) {
                        const float4 x4 = *(const float4 *)&Xs[b][lane][ii + j];
                        x[j] = x4.x;
                        x[j + 1] = x4.y;
                        x[j + 2] = x4.z;
                        x[j + 3] = x4.w;
                    }
#pragma unroll
                    for (int j = 0; j < BI; j++) w[j] = Ws[b][wave][ii + j];
#pragma unroll
                    for (int j = 0; j < BI; j++) s[0] = s[0] + w[j].v[0] * x[j];
                }
            } else {
#pragma unroll 4
                for (int ii = 0; ii < RW_I; ii += 4) {
                    const float4 x4 = *(const float4 *)&Xs[b][lane][ii];
                    const float x[4] = {x4.x, x4.y, x4.z, x4.w};
                    V w[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) w[j] = Ws[b][wave][ii + j];
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int k = 0; k < CPL; k++) s[k] = s[k] + w[j].v[k] * x[j];
                }
            }
            // buffer b ^ 1 was last read in chunk c - 1, before the barrier
            // that ended it; slot (u + 1) % NP then takes chunk c + 1 + NP
            if (c + 1 < nch) lstore((u + 1) % NP, b ^ 1);
            if (c + 1 + NP < nch) gload(c + 1 + NP, (u + 1) % NP);
            __syncthreads();
        }
    }
    const int t = t0 + lane;
    if (t < T) {
        const int e = e0 + CPL * wave;
        V o;
#pragma unroll
        for (int c = 0; c < CPL; c++) o.v[c] = bias ? s[c] + bias[e + c] : s[c];
        *(V *)(logits + (size_t)t * E + e) = o;
    }
}

// ---- router logits, one chain per lane (small batches) ------------------------------
//
// The chains of matmul.c:13-17 (plus the bias) with one chain per lane, so a
// chain's own dependent issue (the product, then the addition) sets the
// pace: in workgroup (g, b), chain wavefront u < NC runs, lane l, the chain
// of expert 64g + l for token NC b + u; wavefront NC only loads. It streams
// the router rows of each chunk (RX_I values of i x 64 experts, 256 bytes
// per i in the transposed router) into an RX_NS-stage LDS ring with
// global_load_lds, RX_NS - 1 chunks ahead, one workgroup barrier per chunk;
// a wavefront that issues those loads is held at the issue for as long as
// the memory pipeline takes them, which is why no chain wavefront issues
// any. A chain reads its router values from LDS (one 4-byte read per lane
// per i) and xn through scalar loads (the same for every lane, so the
// product takes it as a scalar operand), chunk c + 1 while it adds chunk c.
// Measured at T = 64 (128 chains of 2048 terms per CU-sized workgroup):
// ~14.6 us against ~25 us for the tokens-across-lanes kernel below.
constexpr int RX_I = 32, RX_NS = 8, RX_E = 64;
constexpr int RX_DQ = RX_I / 4;  // 1 KB loads per chunk
static_assert((RX_NS - 1) * RX_DQ <= 63, "the loads in flight fit the wait counter");

constexpr size_t router_lanes_lds() { return (size_t)RX_NS * RX_I * RX_E * sizeof(float); }

__device__ __forceinline__ void rx_opaque_v(float &v) {
    float t = v;
    asm volatile("" : "+v"(t));
    v = t;
}
__device__ __forceinline__ void rx_opaque_s(float &v) {
    float t = v;
    asm volatile("" : "+s"(t));
    v = t;
}

// Needs E % 64 == 0 and d % (2 RX_I) == 0.
template <int NC>
__global__ __launch_bounds__(64 * (NC + 1)) void k_router_logits_lanes(
    const float *__restrict__ xn, const float *__restrict__ wt, const float *__restrict__ bias,
    float *__restrict__ logits, int T, int d, int E) {
    extern __shared__ __align__(16) float rx_sh[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nch = d / RX_I;
    if (wave == NC) {
        // chunk c -> stage c % RX_NS, four 256-byte rows per load (lane l:
        // row 4q + l / 16, experts 4 (l % 16) ..); chunks past the end
        // re-read the last one, so every chunk's wait is the same
        const unsigned ring = (unsigned)(uintptr_t)rx_sh;
        const float *wsrc = wt + (size_t)(lane >> 4) * E + blockIdx.x * RX_E + 4 * (lane & 15);
        auto issue = [&](int c) {
            const int k = min(c, nch - 1);
            const unsigned st = ring + (unsigned)((c % RX_NS) * RX_I * RX_E * 4);
#pragma unroll
            for (int q = 0; q < RX_DQ; q++)
                rl_dma16(st + (unsigned)(4 * q * RX_E * 4), wsrc + (size_t)(k * RX_I + 4 * q) * E);
        };
        for (int c = 0; c < RX_NS - 1; c++) issue(c);
        // chunk 0 is in; then, before each chunk c's barrier, chunk c + 1
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((RX_NS - 2) * RX_DQ) : "memory");
        __syncthreads();
        for (int c = 0; c < nch; c++) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((RX_NS - 3) * RX_DQ) : "memory");
            __syncthreads();
            issue(c + RX_NS - 1);  // into the stage of chunk c - 1, read before
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the reloads past the end
        return;
    }
    const int e = blockIdx.x * RX_E + lane, t = blockIdx.y * NC + wave;
    const float *xr = xn + (size_t)min(t, T - 1) * d;
    float wr[2][RX_I], xs[2][RX_I];
    auto lread = [&](int c, int b) {
        const float *W = rx_sh + (size_t)(c % RX_NS) * RX_I * RX_E + lane;
        const float *X = xr + min(c, nch - 1) * RX_I;
#pragma unroll
        for (int j = 0; j < RX_I; j++) wr[b][j] = W[j * RX_E];
#pragma unroll
        for (int j = 0; j < RX_I; j++) xs[b][j] = X[j];
    };
    // the reads of a chunk pass through an opaque copy after the additions
    // of the chunk before, so their wait lands there and not at their first
    // use (and their loads are not moved next to it)
    auto settle = [&](int b) {
#pragma unroll
        for (int j = 0; j < RX_I; j++) rx_opaque_v(wr[b][j]);
#pragma unroll
        for (int j = 0; j < RX_I; j++) rx_opaque_s(xs[b][j]);
    };
    float s = 0.0f;
    auto body = [&](int c, int cur) {
        __syncthreads();  // chunk c + 1 is in the ring
        lread(c + 1, cur ^ 1);
        // the scheduler keeps the reads, the additions and the settling in
        // this order
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < RX_I; j++) s = s + wr[cur][j] * xs[cur][j];
        __builtin_amdgcn_sched_barrier(0);
        settle(cur ^ 1);
    };
    __syncthreads();  // chunk 0 is in the ring
    lread(0, 0);
    settle(0);
    for (int c = 0; c < nch; c += 2) {
        body(c, 0);
        body(c + 1, 1);
    }
    if (t < T) logits[(size_t)t * E + e] = bias ? s + bias[e] : s;
}

// ---- rmsnorm, router and selection of one token, fused -----------------------------
//
// For a few tokens (each layer's chains are latency-bound there), one
// workgroup per token does the whole front of the layer, in place of the
// rmsnorm, router-logit and selection launches: wavefront 0 forms the
// rmsnorm and Q8(xn) as k_rmsnorm_q8_w does (lane b owns block b;
// forward.c:75-81, quant.c:11-27) and keeps xn in LDS; wavefronts 0 and 1
// then run the chains of experts 64 w + lane (matmul.c:13-17: the products
// and additions in i order, bit for bit) over the transposed router, which
// wavefronts 2 and 3 stream into an NR_NS-stage LDS ring with
// global_load_lds, NR_CI rows (16 KB) per chunk, NR_NS - 1 chunks ahead, one
// workgroup barrier per chunk (as k_router_logits_lanes, for all 128 experts
// of one token); a chain wave reads chunk c + 1's router values and xn while
// it adds chunk c. The logits (+ bias) then go through route_select. Needs
// d == 2048, E == 128.
constexpr int NR_CI = 32;                    // rows of i per chunk
constexpr int NR_NS = 8;                     // ring stages (NR_NS - 1 chunks, 112 KB, in flight)
constexpr int NR_E = 128;
constexpr int NR_W = 4;                      // wavefronts: 2 chains, 2 ring loaders
constexpr int NR_DQ = NR_CI * NR_E * 4 / 1024 / 2;  // 1 KB loads per chunk per loader wave (8)
static_assert((NR_NS - 1) * NR_DQ <= 63, "the loads in flight fit the wait counter");
constexpr int NR_MAX_T = 256;                // tokens per layer up to which the fused front runs

__global__ __launch_bounds__(64 * NR_W) void k_norm_route(const float *__restrict__ x,
                                                    const float *__restrict__ w,
                                                    const float *__restrict__ wt,
                                                    const float *__restrict__ bias,
                                                    float *__restrict__ xn,
                                                    int8_t *__restrict__ xq,
                                                    float *__restrict__ xs,
                                                    float *__restrict__ logits,
                                                    int *__restrict__ idx_out,
                                                    float *__restrict__ w_out, int K,
                                                    int norm_topk, float eps, int force_seq,
                                                    int *status) {
    __shared__ __align__(16) float ring[NR_NS][NR_CI][NR_E];
    __shared__ __align__(16) float xn_l[RN_D];
    __shared__ __align__(16) float p[NR_E];
    __shared__ __align__(16) unsigned long long keys[NR_E];
    __shared__ float red[NR_W];
    __shared__ float sum_sh;
    __shared__ int top[64];
    constexpr int NCH = RN_D / NR_CI;
    const int t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // loader wave 2 + q takes loads NR_DQ q .. of a chunk: load k gives lane
    // L row 2 k + L / 32 of the chunk, experts 4 (L % 32) .. + 3 (the chunk
    // is one contiguous 16 KB run of the transposed router)
    const unsigned ring0 = (unsigned)(uintptr_t)&ring[0][0][0];
    auto issue = [&](int c) {
        const int k0 = NR_DQ * (wave - 2);
        const int cc = c < NCH ? c : NCH - 1;  // past the end: reload the last chunk
        const unsigned st = ring0 + (unsigned)((c % NR_NS) * NR_CI * NR_E * 4);
        const float *src = wt + (size_t)cc * NR_CI * NR_E + 4 * lane;
#pragma unroll
        for (int q = 0; q < NR_DQ; q++)
            rl_dma16(st + (unsigned)((k0 + q) * 1024), src + (size_t)(k0 + q) * 256);
    };
    if (wave >= 2)
        for (int c = 0; c < NR_NS - 1; c++) issue(c);
    if (wave == 0) {
        const int b = lane;
        const float4 *xr = (const float4 *)(x + (size_t)t * RN_D + 32 * b);
        const float4 *wr = (const float4 *)(w + 32 * b);
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 q = xr[k];
            v[4 * k] = q.x;
            v[4 * k + 1] = q.y;
            v[4 * k + 2] = q.z;
            v[4 * k + 3] = q.w;
        }
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < 32; k++) ss = ss + (double)v[k] * (double)v[k];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss = ss + __shfl_xor(ss, o);
        ss = __shfl(ss, 0);
        const double m = ss * ((double)(RN_D + 64) * 0x1p-52);
        const float lo = (float)(1.0 / sqrt((ss + m) / RN_D + (double)eps));
        const float hi = (float)(1.0 / sqrt((ss - m) / RN_D + (double)eps));
        float inv = lo;
        if (force_seq || lo != hi) {
            float r = 0.0f;
            if (b == 0) {
                const float *xt = x + (size_t)t * RN_D;
                double sq = 0.0;
                for (int i = 0; i < RN_D; i++) sq = sq + (double)xt[i] * (double)xt[i];
                r = (float)(1.0 / sqrt(sq / RN_D + (double)eps));
                atomicAdd(&status[1], 1);
            }
            inv = __shfl(r, 0);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 q = wr[k];
            v[4 * k] = (v[4 * k] * inv) * q.x;
            v[4 * k + 1] = (v[4 * k + 1] * inv) * q.y;
            v[4 * k + 2] = (v[4 * k + 2] * inv) * q.z;
            v[4 * k + 3] = (v[4 * k + 3] * inv) * q.w;
        }
        float amax = 0.0f;
#pragma unroll
        for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(v[k]));
        const float dsc = amax / 127.0f;
        const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
        float4 *xo = (float4 *)(xn + (size_t)t * RN_D + 32 * b);
        float4 *xl = (float4 *)(xn_l + 32 * b);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 q = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
            xo[k] = q;
            xl[k] = q;
        }
        union {
            int8_t c[32];
            int4 q[2];
        } qc;
#pragma unroll
        for (int k = 0; k < 32; k++) qc.c[k] = (int8_t)roundf(v[k] * qi);
        int4 *qo = (int4 *)(xq + (size_t)t * RN_D + 32 * b);
        qo[0] = qc.q[0];
        qo[1] = qc.q[1];
        xs[(size_t)t * (RN_D / QK) + b] = dsc;
    }
    float s = 0.0f;
    if (wave >= 2) {
        // chunk 0 is in; then, before each chunk c's barrier, chunk c + 1
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NR_NS - 2) * NR_DQ) : "memory");
        __syncthreads();  // xn and chunk 0
        for (int c = 0; c < NCH; c++) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NR_NS - 3) * NR_DQ) : "memory");
            __syncthreads();
            issue(c + NR_NS - 1);  // into the stage of chunk c - 1, read before
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the reloads past the end
    } else {
        const int e = 64 * wave + lane;
        float wr[2][NR_CI], xv[2][NR_CI];
        auto lread = [&](int c, int b) {
            const float *W = &ring[c % NR_NS][0][e];
            const float *X = &xn_l[(c < NCH ? c : NCH - 1) * NR_CI];
#pragma unroll
            for (int j = 0; j < NR_CI; j++) wr[b][j] = W[j * NR_E];
#pragma unroll
            for (int j = 0; j < NR_CI; j += 4) {
                const float4 q = *(const float4 *)&X[j];
                xv[b][j] = q.x;
                xv[b][j + 1] = q.y;
                xv[b][j + 2] = q.z;
                xv[b][j + 3] = q.w;
            }
        };
        // the reads of a chunk pass through an opaque copy after the
        // additions of the chunk before, so their wait lands there
        auto settle = [&](int b) {
#pragma unroll
            for (int j = 0; j < NR_CI; j++) rx_opaque_v(wr[b][j]);
#pragma unroll
            for (int j = 0; j < NR_CI; j++) rx_opaque_v(xv[b][j]);
        };
        auto body = [&](int c, int cur) {
            __syncthreads();  // chunk c + 1 is in the ring
            lread(c + 1, cur ^ 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NR_CI; j++) s = s + wr[cur][j] * xv[cur][j];
            __builtin_amdgcn_sched_barrier(0);
            settle(cur ^ 1);
        };
        __syncthreads();  // xn and chunk 0
        lread(0, 0);
        settle(0);
        for (int c = 0; c < NCH; c += 2) {
            body(c, 0);
            body(c + 1, 1);
        }
        if (bias) s = s + bias[e];
        logits[(size_t)t * NR_E + e] = s;
    }
    const float l = tid < NR_E ? s : -__builtin_inff();
    route_select(l, t, NR_E, K, norm_topk, p, keys, red, &sum_sh, top, idx_out, w_out);
}

// ---- dispatch -------------------------------------------------------------
//
// Stable counting sort of the A = T*K assignments a = t*K + j by expert
// idx[a]: within an expert the order is by t (then j), the order in which
// the reference visits tokens. Three small kernels over chunks of DCH
// consecutive assignments, one wavefront per chunk:
//   k_disp_count    per-chunk expert counts           -> hist[e][chunk]
//   k_disp_scan     per expert, exclusive scan over the chunks; counts
//   k_disp_scatter  offsets, the list of non-empty experts as (expert,
//                   begin, end) groups, gtile[g], the number of tm-row
//                   tiles before group g (gtile[n_groups] = all tiles), and
//                   glight[g], the light tiles among them; then
//                   each chunk in order, 64 assignments per step: the rank
//                   of a lane among the step's lanes with the same expert
//                   comes from one ballot per bit of the expert index.
// Up to DSMALL chunks, one workgroup does all three (k_disp_small).
// status[0] |= 1 on a bad index (the assignment is then counted as expert 0),
// and status[2] names the first layer launch that met one.
constexpr int DCH = 256;               // assignments per chunk (4 steps of 64)
constexpr int DWG = 4;                 // chunks (wavefronts) per workgroup

// Keeps the compiler from moving LDS accesses across this point; a
// wavefront's own LDS operations execute in program order.
__device__ __forceinline__ void wave_order() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}


// Lanes of the wavefront whose key equals this lane's (keys < 2^bits; -1
// matches no lane).
__device__ __forceinline__ uint64_t same_key_lanes(int key, int bits) {
    uint64_t m = __ballot(key >= 0);
    for (int b = 0; b < bits; b++) {
        const uint64_t on = __ballot(key >= 0 && ((key >> b) & 1));
        m &= ((key >> b) & 1) ? on : ~on;
    }
    return key >= 0 ? m : 0ull;
}

constexpr int DSTEP = DCH / 64;  // assignments of a chunk per lane

// This lane's keys of chunk ch, one per step of 64 (-1 past the end; an
// expert id outside 0..E-1 counts as expert 0 and is reported in status):
// the loads are issued together, then validated.
__device__ __forceinline__ void disp_chunk_keys(const int *idx, int A, int E, int ch, int *status,
                                                int (&key)[DSTEP]) {
    const int lane = threadIdx.x & 63;
    int raw[DSTEP];
#pragma unroll
    for (int s = 0; s < DSTEP; s++) {
        const int a = ch * DCH + s * 64 + lane;
        raw[s] = a < A ? idx[a] : 0;
    }
#pragma unroll
    for (int s = 0; s < DSTEP; s++) {
        const int a = ch * DCH + s * 64 + lane;
        if (a >= A) {
            key[s] = -1;
        } else if (raw[s] < 0 || raw[s] >= E) {
            atomicOr(&status[0], 1);
            atomicCAS(&status[2], 0, status[3] + 1);
            key[s] = 0;
        } else {
            key[s] = raw[s];
        }
    }
}

// One wavefront counts its chunk's keys into cnt[E] (zeroed by the caller).
__device__ __forceinline__ void disp_count_chunk(const int (&key)[DSTEP], int *cnt) {
#pragma unroll
    for (int s = 0; s < DSTEP; s++)
        if (key[s] >= 0) atomicAdd(&cnt[key[s]], 1);
}

// One wavefront places chunk ch (its keys) in order; bs[E] holds each
// expert's next position and is advanced.
__device__ __forceinline__ void disp_scatter_chunk(const int (&key)[DSTEP], int ch, int bits,
                                                   int *bs, int *perm, int *pos) {
    const int lane = threadIdx.x & 63;
    const uint64_t below = (1ull << lane) - 1;
#pragma unroll
    for (int s = 0; s < DSTEP; s++) {
        const int a = ch * DCH + s * 64 + lane;
        const int k = key[s];
        const uint64_t m = same_key_lanes(k, bits);
        if (k >= 0) {
            const int p = bs[k] + __popcll(m & below);
            perm[p] = a;
            pos[a] = p;
        }
        wave_order();
        // the highest lane of each key advances that key's position
        if (k >= 0 && (m >> lane) == 1ull) bs[k] += __popcll(m);
        wave_order();
    }
}

__global__ __launch_bounds__(64 * DWG) void k_disp_count(const int *__restrict__ idx, int A, int E,
                                                         int nch, int *__restrict__ hist,
                                                         int *status) {
    extern __shared__ int cnt[];  // [DWG][E]
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ch = blockIdx.x * DWG + w;
    int *c = cnt + w * E;
    for (int e = lane; e < E; e += 64) c[e] = 0;
    __syncthreads();
    if (ch < nch) {
        int key[DSTEP];
        disp_chunk_keys(idx, A, E, ch, status, key);
        disp_count_chunk(key, c);
    }
    __syncthreads();
    if (ch < nch)
        for (int e = lane; e < E; e += 64) hist[(size_t)e * nch + ch] = c[e];
}

// The dispatch tables (counts, offsets[E+1], the list of non-empty experts as
// (expert, begin, end) groups, gtile[g], the number of tm-row tiles before
// group g, and glight[g], the number of light tiles before group g) from
// parallel scans: every thread of the workgroup calls (blockDim >= 256,
// E <= 256); thread x < E owns expert x. A group's tiles are tm rows each
// but its last, which holds the remaining rows and is light when those are at
// most tm / 2. Four exclusive scans over the experts (rows, non-empty
// experts, tiles, light tiles) give each expert's offset, its group number,
// its first tile and its light tiles before it. off[E] (LDS) receives the
// offsets; with write_tables the global tables are written too.
// sc: 16 ints of LDS.
__device__ void disp_tables(int E, const int *tot, int *off, int *sc, bool write_tables,
                            int *counts, int *offsets, int *groups, int *gtile, int *glight,
                            int tm) {
    const int x = threadIdx.x, lane = x & 63, w = x >> 6;
    const bool in = x < E;
    const int n = in ? tot[x] : 0;
    const int ne = n > 0 ? 1 : 0, nt = (n + tm - 1) / tm;
    const int nl = n % tm != 0 && n % tm <= tm / 2 ? 1 : 0;
    int a = n, b = ne, c = nt, l = nl;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int ua = __shfl_up(a, o), ub = __shfl_up(b, o), uc = __shfl_up(c, o),
                  ul = __shfl_up(l, o);
        if (lane >= o) {
            a += ua;
            b += ub;
            c += uc;
            l += ul;
        }
    }
    if (w < 4 && lane == 63) {
        sc[w] = a;
        sc[4 + w] = b;
        sc[8 + w] = c;
        sc[12 + w] = l;
    }
    __syncthreads();
    int pa = 0, pb = 0, pc = 0, pl = 0, ta = 0, tb = 0, tc = 0, tl = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if (k < w) {
            pa += sc[k];
            pb += sc[4 + k];
            pc += sc[8 + k];
            pl += sc[12 + k];
        }
        ta += sc[k];
        tb += sc[4 + k];
        tc += sc[8 + k];
        tl += sc[12 + k];
    }
    if (in) {
        const int ea = pa + a - n, eb = pb + b - ne, ec = pc + c - nt, el = pl + l - nl;
        off[x] = ea;
        if (write_tables) {
            counts[x] = n;
            offsets[x] = ea;
            if (ne) {
                groups[1 + 3 * eb] = x;
                groups[2 + 3 * eb] = ea;
                groups[3 + 3 * eb] = ea + n;
                gtile[eb] = ec;
                glight[eb] = el;
            }
        }
    }
    if (write_tables && x == 0) {
        offsets[E] = ta;
        groups[0] = tb;
        gtile[tb] = tc;
        glight[tb] = tl;
    }
    __syncthreads();
}

// Workgroup e: exclusive prefix of expert e's counts over the chunks, in
// place; the total goes to counts[e].
__global__ __launch_bounds__(256) void k_disp_scan(int nch, int *__restrict__ hist,
                                                   int *__restrict__ counts) {
    __shared__ int wsum[4];
    __shared__ int carry;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int *row = hist + (size_t)blockIdx.x * nch;
    if (threadIdx.x == 0) carry = 0;
    for (int c0 = 0; c0 < nch; c0 += 256) {
        const int c = c0 + threadIdx.x;
        const int v = c < nch ? row[c] : 0;
        int inc = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(inc, o);
            if (lane >= o) inc += u;
        }
        if (lane == 63) wsum[w] = inc;
        __syncthreads();
        int pre = carry;
        for (int k = 0; k < w; k++) pre += wsum[k];
        if (c < nch) row[c] = pre + inc - v;
        __syncthreads();
        if (threadIdx.x == 255) carry = pre + inc;
        __syncthreads();
    }
    if (threadIdx.x == 0) counts[blockIdx.x] = carry;
}

// Every workgroup derives the experts' first positions from counts[];
// workgroup 0 also writes offsets, groups, gtile and glight.
__global__ __launch_bounds__(64 * DWG) void k_disp_scatter(const int *__restrict__ idx, int A,
                                                           int E, int nch, int bits,
                                                           const int *__restrict__ hist,
                                                           int *__restrict__ counts,
                                                           int *__restrict__ offsets,
                                                           int *__restrict__ groups,
                                                           int *__restrict__ gtile,
                                                           int *__restrict__ glight, int tm,
                                                           int *__restrict__ perm,
                                                           int *__restrict__ pos,
                                                           int *status) {
    extern __shared__ int lds_s[];
    int *base = lds_s;                 // [DWG][E]: next position of each expert
    int *tot = lds_s + DWG * E;        // [E]
    int *off = tot + E;                // [E]
    int *sc = off + E;                 // [16]
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int e = threadIdx.x; e < E; e += blockDim.x) tot[e] = counts[e];
    __syncthreads();
    disp_tables(E, tot, off, sc, blockIdx.x == 0, counts, offsets, groups, gtile, glight, tm);
    const int ch = blockIdx.x * DWG + w;
    if (ch >= nch) return;  // a whole wavefront: no workgroup barrier follows
    int key[DSTEP];
    disp_chunk_keys(idx, A, E, ch, status, key);
    int *bs = base + w * E;
    for (int e = lane; e < E; e += 64) bs[e] = off[e] + hist[(size_t)e * nch + ch];
    wave_order();
    disp_scatter_chunk(key, ch, bits, bs, perm, pos);
}

// All three steps in one workgroup, one wavefront per chunk, for up to
// DSMALL chunks.
constexpr int DSMALL = 16;
__global__ __launch_bounds__(64 * DSMALL) void k_disp_small(const int *__restrict__ idx, int A,
                                                            int E, int nch, int bits,
                                                            int *__restrict__ counts,
                                                            int *__restrict__ offsets,
                                                            int *__restrict__ perm,
                                                            int *__restrict__ pos,
                                                            int *__restrict__ groups,
                                                            int *__restrict__ gtile,
                                                            int *__restrict__ glight, int tm,
                                                            int *status) {
    extern __shared__ int lds_i[];
    int *hist = lds_i;                 // [DSMALL][E]
    int *tot = lds_i + DSMALL * E;     // [E]
    int *off = tot + E;                // [E]
    int *sc = off + E;                 // [16]
    const int w = threadIdx.x >> 6;
    // the chunk's keys are requested before the histogram is cleared, and
    // kept for the scatter
    int key[DSTEP];
    if (w < nch) disp_chunk_keys(idx, A, E, w, status, key);
    for (int i = threadIdx.x; i < DSMALL * E; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    if (w < nch) disp_count_chunk(key, hist + w * E);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        int run = 0;
        for (int c = 0; c < nch; c++) {
            const int v = hist[c * E + e];
            hist[c * E + e] = run;
            run += v;
        }
        tot[e] = run;
    }
    __syncthreads();
    disp_tables(E, tot, off, sc, true, counts, offsets, groups, gtile, glight, tm);
    if (w < nch) {
        int *bs = hist + w * E;
        for (int e = threadIdx.x & 63; e < E; e += 64) bs[e] += off[e];
        wave_order();
        disp_scatter_chunk(key, w, bits, bs, perm, pos);
    }
}

// Sequential fp32 sum of the n floats at p (LDS), in order. Sixteen values
// are read before they are added, so the chain waits for the LDS once per
// sixteen values rather than once per value.
__device__ __forceinline__ float lds_seq_sum(const float *p, int n) {
    float s = 0.0f;
    int b = 0;
    for (; b + 16 <= n; b += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = p[b + j];
#pragma unroll
        for (int j = 0; j < 16; j++) s = s + v[j];
    }
    for (; b < n; b++) s = s + p[b];
    return s;
}

// ---- gate/up + SwiGLU --------------------------------------------------------

// Float offset of k_gateup's staged codes in its LDS (16-byte aligned) and
// the kernel's LDS bytes.
__host__ __device__ inline int gateup_xq_off(int d, int R) {
    const int nb = d / QK;
    const int f = TB * 2 * R * (nb + 1) + TB * 2 * R + TB * nb + TB;
    return (f + 3) / 4 * 4;
}
inline size_t gateup_lds(int d, int R) { return (size_t)gateup_xq_off(d, R) * 4 + (size_t)TB * d; }

//
// Workgroup = (group g of one expert, R consecutive rows of h). Its 2R weight
// rows (R of gate, R of up) are split into (row, 32-block) pairs, one pair
// per thread per step, codes held in registers across the expert's tokens.
// For TB tokens at a time the tokens' Q8(xn) rows and scales are staged in
// LDS (one round of independent loads), each pair's exact int32 dot is
// turned into the reference's term ((float)acc*d_w)*d_x and parked in LDS;
// then one thread per (token, row) adds its row's terms in block order, and
// SwiGLU g/(1+expf(-g))*u (forward.c:190) produces h, written in bucketed
// order.
template <int PK>
__global__ __launch_bounds__(NT, 6) void k_gateup(const uint8_t *__restrict__ table, mhip_layout lay,
                                               const int8_t *__restrict__ xq,
                                               const float *__restrict__ xs,
                                               const int *__restrict__ groups,
                                               const int *__restrict__ perm,
                                               float *__restrict__ h, int d, int eh, int K,
                                               int R) {
    // [TB][2R][nb+1] terms, gu[TB][2R], xs_l[TB][nb], tk[TB], then (16-byte
    // aligned) xq_l[TB][d] codes
    extern __shared__ float terms[];
    const int nb = d / QK;
    const int nrc = eh / R;
    const int g = blockIdx.x / nrc;
    const int rc = blockIdx.x % nrc;
    if (g >= groups[0]) return;
    const int e = groups[1 + 3 * g], b0 = groups[2 + 3 * g], b1 = groups[3 + 3 * g];
    const uint8_t *ex = table + (size_t)e * lay.expert_bytes;
    const int P = 2 * R * nb;
    const int ld = nb + 1;
    float *gu = terms + TB * 2 * R * ld;
    float *xs_l = gu + TB * 2 * R;
    int8_t *xq_l = (int8_t *)(terms + gateup_xq_off(d, R));

    // A pass's tokens (uniform loads); their Q8 rows and scales go straight
    // into LDS, 1 KB of codes or 64 scales per wavefront instruction. The
    // first pass's copies are issued before the weights, so they arrive
    // with them.
    auto stage = [&](int base, int ntok) {
        int tkn[TB];
#pragma unroll
        for (int j = 0; j < TB; j++) tkn[j] = j < ntok ? perm[base + j] / K : 0;
        const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int nck = (d + 1023) / 1024, ncs = (nb + 63) / 64;
        const unsigned xl = (unsigned)(uintptr_t)xq_l, sl = (unsigned)(uintptr_t)xs_l;
        for (int j = wave; j < ntok * nck; j += NT / 64) {
            const int tb = j / nck, q = j % nck, off = 1024 * q + 16 * lane;
            if (off < d)
                rl_dma16(__builtin_amdgcn_readfirstlane(xl + (unsigned)(tb * d + 1024 * q)),
                         xq + (size_t)tkn[tb] * d + off);
        }
        for (int j = wave; j < ntok * ncs; j += NT / 64) {
            const int tb = j / ncs, q = j % ncs, b = 64 * q + lane;
            if (b < nb)
                rl_dma4(__builtin_amdgcn_readfirstlane(sl + (unsigned)(4 * (tb * nb + 64 * q))),
                        xs + (size_t)tkn[tb] * nb + b);
        }
    };
    if (b0 < b1) stage(b0, b1 - b0 < TB ? b1 - b0 : TB);
    int4 wc0[PK], wc1[PK];
    float wd[PK];
    int prow[PK], pblk[PK];
#pragma unroll
    for (int k = 0; k < PK; k++) {
        const int p = threadIdx.x + NT * k;
        prow[k] = p < P ? p / nb : -1;
        pblk[k] = p < P ? p % nb : 0;
        if (p < P) {
            const int wr = prow[k];
            const bool is_gate = wr < R;
            const int row = rc * R + (is_gate ? wr : wr - R);
            const int4 *src = (const int4 *)(ex + (is_gate ? lay.gate_q : lay.up_q) +
                                             (size_t)row * d + (size_t)pblk[k] * QK);
            wc0[k] = src[0];
            wc1[k] = src[1];
            wd[k] = ((const float *)(ex + (is_gate ? lay.gate_s : lay.up_s)))[(size_t)row * nb +
                                                                             pblk[k]];
        }
    }
    for (int base = b0; base < b1; base += TB) {
        const int ntok = b1 - base < TB ? b1 - base : TB;
        if (base != b0) stage(base, ntok);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PK; k++) {
            if (prow[k] < 0) continue;
            for (int tb = 0; tb < ntok; tb++) {
                const int4 *xv = (const int4 *)(xq_l + (size_t)tb * d + (size_t)pblk[k] * QK);
                const int acc = mhip_dev::dot32_i8(wc0[k], wc1[k], xv[0], xv[1]);
                terms[(tb * 2 * R + prow[k]) * ld + pblk[k]] =
                    mhip_dev::block_term(acc, wd[k], xs_l[tb * nb + pblk[k]]);
            }
        }
        __syncthreads();
        for (int c = threadIdx.x; c < ntok * 2 * R; c += NT) {
            gu[c] = lds_seq_sum(terms + c * ld, nb);
        }
        __syncthreads();
        for (int c = threadIdx.x; c < ntok * R; c += NT) {
            const int tb = c / R, r = c % R;
            const float gv = gu[tb * 2 * R + r];
            const float uv = gu[tb * 2 * R + R + r];
            h[(size_t)(base + tb) * eh + rc * R + r] =
                (gv / (1.0f + mhip_dev::expf_glibc(-gv))) * uv;
        }
        __syncthreads();
    }
}

// ---- Q8(h) -----------------------------------------------------------------------
//
// One thread per 32-block of h (quant.c:11-27), once per assignment row:
// codes to hq, scales to hs, both in bucketed order.
__global__ __launch_bounds__(256) void k_quant_h(const float *__restrict__ h,
                                                 int8_t *__restrict__ hq,
                                                 float *__restrict__ hs, int nblocks) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float4 *v4 = (const float4 *)(h + (size_t)b * QK);
    float v[QK];
#pragma unroll
    for (int i = 0; i < QK / 4; i++) {
        const float4 f = v4[i];
        v[4 * i] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < QK; i++) {
        const float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    const float dsc = amax / 127.0f;
    const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
    union {
        int8_t c[QK];
        int4 q[2];
    } out;
#pragma unroll
    for (int i = 0; i < QK; i++) out.c[i] = (int8_t)roundf(v[i] * qi);
    int4 *dst = (int4 *)(hq + (size_t)b * QK);
    dst[0] = out.q[0];
    dst[1] = out.q[1];
    hs[b] = dsc;
}

// ---- down ----------------------------------------------------------------------
//
// Workgroup = (group g, R rows of down). For TB tokens at a time the rows'
// Q8(h) codes and scales (k_quant_h) are staged in LDS, the (row, block)
// pairs produce the reference's terms, and one thread per (token, row) sums
// them in block order into tmp (bucketed order).
template <int PK>
__global__ __launch_bounds__(NT) void k_down(const uint8_t *__restrict__ table, mhip_layout lay,
                                             const int8_t *__restrict__ hq_g,
                                             const float *__restrict__ hs_g,
                                             const int *__restrict__ groups,
                                             float *__restrict__ tmp, int d, int eh, int R) {
    extern __shared__ float terms[];  // [TB][R][nbh+1], hs[TB][nbh], hq[TB][eh] bytes
    const int nbh = eh / QK;
    const int nrc = d / R;
    const int g = blockIdx.x / nrc;
    const int rc = blockIdx.x % nrc;
    if (g >= groups[0]) return;
    const int e = groups[1 + 3 * g], b0 = groups[2 + 3 * g], b1 = groups[3 + 3 * g];
    const uint8_t *ex = table + (size_t)e * lay.expert_bytes;
    const int P = R * nbh;
    const int ld = nbh + 1;
    float *hs = terms + TB * R * ld;
    int8_t *hq = (int8_t *)(hs + TB * nbh);

    // A pass's rows base .. base + ntok - 1 of the bucket (contiguous):
    // codes and scales straight into LDS, 1 KB of codes or 64 scales per
    // wavefront instruction; the first pass's copies are issued before the
    // weights, so they arrive with them.
    auto stage = [&](int base, int ntok) {
        const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int nbytes = ntok * eh, nst = ntok * nbh;
        const unsigned ql = (unsigned)(uintptr_t)hq, sl = (unsigned)(uintptr_t)hs;
        for (int q = wave; 1024 * q < nbytes; q += NT / 64) {
            const int off = 1024 * q + 16 * lane;
            if (off < nbytes)
                rl_dma16(__builtin_amdgcn_readfirstlane(ql + (unsigned)(1024 * q)),
                         hq_g + (size_t)base * eh + off);
        }
        for (int q = wave; 64 * q < nst; q += NT / 64) {
            const int b = 64 * q + lane;
            if (b < nst)
                rl_dma4(__builtin_amdgcn_readfirstlane(sl + (unsigned)(256 * q)),
                        hs_g + (size_t)base * nbh + b);
        }
    };
    if (b0 < b1) stage(b0, b1 - b0 < TB ? b1 - b0 : TB);
    int4 wc0[PK], wc1[PK];
    float wd[PK];
    int prow[PK], pblk[PK];
#pragma unroll
    for (int k = 0; k < PK; k++) {
        const int p = threadIdx.x + NT * k;
        prow[k] = p < P ? p / nbh : -1;
        pblk[k] = p < P ? p % nbh : 0;
        if (p < P) {
            const int row = rc * R + prow[k];
            const int4 *src =
                (const int4 *)(ex + lay.down_q + (size_t)row * eh + (size_t)pblk[k] * QK);
            wc0[k] = src[0];
            wc1[k] = src[1];
            wd[k] = ((const float *)(ex + lay.down_s))[(size_t)row * nbh + pblk[k]];
        }
    }
    for (int base = b0; base < b1; base += TB) {
        const int ntok = b1 - base < TB ? b1 - base : TB;
        if (base != b0) stage(base, ntok);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PK; k++) {
            if (prow[k] < 0) continue;
            for (int tb = 0; tb < ntok; tb++) {
                const int4 *xv = (const int4 *)(hq + (size_t)tb * eh + (size_t)pblk[k] * QK);
                const int acc = mhip_dev::dot32_i8(wc0[k], wc1[k], xv[0], xv[1]);
                terms[(tb * R + prow[k]) * ld + pblk[k]] =
                    mhip_dev::block_term(acc, wd[k], hs[tb * nbh + pblk[k]]);
            }
        }
        __syncthreads();
        for (int c = threadIdx.x; c < ntok * R; c += NT) {
            const int tb = c / R, r = c % R;
            tmp[(size_t)(base + tb) * d + rc * R + r] = lds_seq_sum(terms + c * ld, nbh);
        }
        __syncthreads();
    }
}

// ---- combine -------------------------------------------------------------------
// x_i = x_i + w_j * tmp_j,i for j = 0..K-1 in top-K order (forward.c:194).
// Four consecutive elements per thread (d % 4 == 0); the K rows of a token
// are requested before the ordered sum consumes them. One thread counts the
// layer launch in status[3].
__global__ __launch_bounds__(256) void k_combine(float *__restrict__ x,
                                                 const float *__restrict__ w,
                                                 const int *__restrict__ pos,
                                                 const float *__restrict__ tmp, int d, int K,
                                                 int *__restrict__ status) {
    const int t = blockIdx.y;
    const int i = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (t == 0 && i == 0) status[3] += 1;
    if (i >= d) return;
    float4 *xp = (float4 *)(x + (size_t)t * d + i);
    float4 v = *xp;
    for (int j0 = 0; j0 < K; j0 += 8) {
        float4 tv[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j0 + j < K) {
                // read once: non-temporal (55 against 66 us at T = 4096)
                typedef float f4n __attribute__((ext_vector_type(4)));
                const f4n q = __builtin_nontemporal_load(
                    (const f4n *)(tmp + (size_t)pos[t * K + j0 + j] * d + i));
                tv[j] = make_float4(q.x, q.y, q.z, q.w);
            }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j0 + j < K) {
                const float wj = w[t * K + j0 + j];
                v.x = v.x + wj * tv[j].x;
                v.y = v.y + wj * tv[j].y;
                v.z = v.z + wj * tv[j].z;
                v.w = v.w + wj * tv[j].w;
            }
    }
    *xp = v;
}

// Rows per workgroup: the largest power of two <= 32 with 2R*nb <= PK*NT
// pairs (gate/up), R*nbh <= PKD*NT (down; three pairs per thread hold the
// 32 x 24 pairs of the 768-wide down rows exactly).
constexpr int PK = 4;
constexpr int PKD = 3;

int rows_gateup(int nb) {
    int r = 32;
    while (r > 1 && 2 * r * nb > PK * NT) r >>= 1;
    return r;
}

int rows_down(int nbh) {
    int r = 32;
    while (r > 1 && r * nbh > PKD * NT) r >>= 1;
    return r;
}

}  // namespace

namespace mhip {

void launch_rmsnorm_q8(hipStream_t st, const float *x, const float *w, float *xn, int8_t *xq,
                       float *xs, int T, int d, float eps, int force_seq, int *status) {
    if (d == RN_D)
        k_rmsnorm_q8_w<<<(T + 3) / 4, 256, 0, st>>>(x, w, xn, xq, xs, nullptr, T, eps, force_seq,
                                                    status);
    else
        k_rmsnorm_q8<<<T, NT, 0, st>>>(x, w, xn, xq, xs, nullptr, d, eps, force_seq, status);
}

}  // namespace mhip

extern "C" {

size_t mhip_scratch_bytes(const mhip_dims *s, int T) {
    const size_t d = s->dim, E = s->n_experts, K = s->n_active, eh = s->expert_hidden;
    const size_t A = (size_t)T * K;
    size_t n = 0;
    n += align256(T * d * 4);          // xn
    n += align256(T * d);              // xq
    n += align256(T * (d / QK) * 4);   // xs
    n += align256(T * E * 4);          // logits
    n += align256(A * 4);              // idx
    n += align256(A * 4);              // w
    n += align256(E * 4);              // counts
    n += align256((E + 1) * 4);        // offsets
    n += align256(A * 4);              // perm
    n += align256(A * 4);              // pos
    n += align256((1 + 3 * E) * 4);    // groups
    n += align256(A * eh * 4);         // h
    n += align256(A * d * 4);          // tmp
    n += align256(4 * 4);              // status
    n += align256(T * d * 2);          // xdq
    n += align256(A * eh * 2);         // hdq
    n += align256((E + 1) * 4);        // gtile
    n += align256(A * (d / QK) * 4);   // xsb
    n += align256(A * eh);             // hq
    n += align256(A * (eh / QK) * 4);  // hs
    n += align256((E + 1) * 4);        // glight
    return n;
}

int mhip_scratch_carve(const mhip_dims *s, int T, void *d_base, mhip_scratch *o) {
    const size_t d = s->dim, E = s->n_experts, K = s->n_active, eh = s->expert_hidden;
    const size_t A = (size_t)T * K;
    uint8_t *p = (uint8_t *)d_base;
    auto take = [&](size_t bytes) {
        void *r = p;
        p += align256(bytes);
        return r;
    };
    o->xn = (float *)take(T * d * 4);
    o->xq = (int8_t *)take(T * d);
    o->xs = (float *)take(T * (d / QK) * 4);
    o->logits = (float *)take(T * E * 4);
    o->idx = (int *)take(A * 4);
    o->w = (float *)take(A * 4);
    o->counts = (int *)take(E * 4);
    o->offsets = (int *)take((E + 1) * 4);
    o->perm = (int *)take(A * 4);
    o->pos = (int *)take(A * 4);
    o->groups = (int *)take((1 + 3 * E) * 4);
    o->h = (float *)take(A * eh * 4);
    o->tmp = (float *)take(A * d * 4);
    o->status = (int *)take(4 * 4);
    o->xdq = take(T * d * 2);
    o->hdq = take(A * eh * 2);
    o->gtile = (int *)take((E + 1) * 4);
    o->xsb = (float *)take(A * (d / QK) * 4);
    o->hq = (int8_t *)take(A * eh);
    o->hs = (float *)take(A * (eh / QK) * 4);
    o->glight = (int *)take((E + 1) * 4);
    return 0;
}

int mhip_moe_layer(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                   const void *d_table_layer, const float *d_router_t, const float *d_norm,
                   const float *d_bias, float *d_x, int T, const mhip_scratch *sc, int flags) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    if (T <= 0) return T == 0 ? 0 : mhip::fail(c, "T=%d", T);
    const int d = s->dim, E = s->n_experts, K = s->n_active, eh = s->expert_hidden;
    const int A = T * K;
    if (A > 65535) return mhip::fail(c, "T*K=%d exceeds 65535 assignments", A);
    if ((uintptr_t)d_x % 16) return mhip::fail(c, "d_x is not 16-byte aligned");
    const int nb = d / QK, nbh = eh / QK;
    hipStream_t st = c->stream;
    const bool mfma = !(flags & MHIP_EXACT_EXPERTS) && A >= MHIP_GEMM_MIN_A &&
                      mhip::gemm_path_fits(s);
    if (mfma) c->matrix_layers++;

    // a few tokens: rmsnorm, router and selection as one launch per layer
    // (recorded as the router stage)
    const bool fused = !mfma && d == RN_D && E == NR_E && K <= 64 && T <= NR_MAX_T;
    int slot = fused ? -1 : mhip::stage_begin(c, MHIP_STAGE_RMSNORM);
    if (fused)
        ;
    else if (d == RN_D && T >= RN_COALESCED_T)
        k_rmsnorm_q8_c<<<(T + 3) / 4, 256, 0, st>>>(d_x, d_norm, sc->xn, mfma ? nullptr : sc->xq,
                                                    sc->xs, mfma ? (_Float16 *)sc->xdq : nullptr,
                                                    T, s->norm_eps,
                                                    (flags & MHIP_FORCE_SEQ_RMS) ? 1 : 0,
                                                    sc->status);
    else if (d == RN_D)
        k_rmsnorm_q8_w<<<(T + 3) / 4, 256, 0, st>>>(d_x, d_norm, sc->xn, sc->xq, sc->xs,
                                                    mfma ? (_Float16 *)sc->xdq : nullptr, T,
                                                    s->norm_eps,
                                                    (flags & MHIP_FORCE_SEQ_RMS) ? 1 : 0,
                                                    sc->status);
    else
        k_rmsnorm_q8<<<T, NT, 0, st>>>(d_x, d_norm, sc->xn, sc->xq, sc->xs,
                                       mfma ? (_Float16 *)sc->xdq : nullptr, d, s->norm_eps,
                                       (flags & MHIP_FORCE_SEQ_RMS) ? 1 : 0, sc->status);
    if (!fused) {
        mhip::stage_end(c, slot);
        if (mhip::check_launch(c, "rmsnorm_q8")) return -1;
    }

    const int rthreads = E <= 64 ? 64 : E <= 128 ? 128 : 256;
    // The tiled chains for more than one token; one workgroup per token else.
    const bool tiled = T > 1 && E == RL_E && d % RL_I == 0 && d / RL_I >= RL_NS - 1;
    // chains per lane of the batched router: the most that still gives every
    // CU a workgroup
    const int ntg = (T + RW_T - 1) / RW_T;
    const int cpl = ntg * (E / 16) >= 256 && E % 16 == 0 ? 4
                    : ntg * (E / 8) >= 256 && E % 8 == 0 ? 2
                                                          : 1;
    const bool wide = d % RW_I == 0 && E % (4 * cpl) == 0;
    // one chain per lane while the chains fill at most 1024 wavefronts
    const bool lanes = T > 1 && ntg * E <= 1024 && E % RX_E == 0 && d % (2 * RX_I) == 0;
    const bool have_logits = lanes || wide || tiled;
    const size_t rsh = (size_t)(E + (have_logits ? 0 : d)) * sizeof(float);
    slot = mhip::stage_begin(c, MHIP_STAGE_ROUTER);
    if (fused) {
        k_norm_route<<<T, 64 * NR_W, 0, st>>>(d_x, d_norm, d_router_t, d_bias, sc->xn, sc->xq, sc->xs,
                                        sc->logits, sc->idx, sc->w, K, s->norm_topk, s->norm_eps,
                                        (flags & MHIP_FORCE_SEQ_RMS) ? 1 : 0, sc->status);
    } else if (lanes) {
        // one chain wavefront per workgroup while that fills at most one
        // workgroup per CU, two beyond
        const size_t lsh = router_lanes_lds();
        const bool one = (size_t)T * (E / RX_E) <= 256;
        const void *fn = one ? (const void *)k_router_logits_lanes<1>
                             : (const void *)k_router_logits_lanes<2>;
        if (mhip::check(c, hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lsh),
                        "router LDS attribute"))
            return -1;
        if (one)
            k_router_logits_lanes<1><<<dim3(E / RX_E, T), 128, lsh, st>>>(
                sc->xn, d_router_t, d_bias, sc->logits, T, d, E);
        else
            k_router_logits_lanes<2><<<dim3(E / RX_E, (T + 1) / 2), 192, lsh, st>>>(
                sc->xn, d_router_t, d_bias, sc->logits, T, d, E);
    } else if (wide) {
        const dim3 g(ntg, E / (4 * cpl));
        if (cpl == 4)
            k_router_logits_wide<4><<<g, 256, 0, st>>>(sc->xn, d_router_t, d_bias, sc->logits, T, d, E);
        else if (cpl == 2)
            k_router_logits_wide<2><<<g, 256, 0, st>>>(sc->xn, d_router_t, d_bias, sc->logits, T, d, E);
        else
            k_router_logits_wide<1><<<g, 256, 0, st>>>(sc->xn, d_router_t, d_bias, sc->logits, T, d, E);
    } else if (tiled) {
        const int C = T >= 4096 ? 4 : T >= 2048 ? 2 : 1;
        const size_t lsh = router_logits_lds(C, d);
        const void *fn = C == 4 ? (const void *)k_router_logits<4>
                         : C == 2 ? (const void *)k_router_logits<2>
                                  : (const void *)k_router_logits<1>;
        if (lsh > 65536 &&
            mhip::check(c, hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lsh),
                        "router LDS attribute"))
            return -1;
        if (C == 4)
            k_router_logits<4><<<(T + 7) / 8, 256, lsh, st>>>(sc->xn, d_router_t, d_bias, sc->logits, T, d);
        else if (C == 2)
            k_router_logits<2><<<(T + 3) / 4, 256, lsh, st>>>(sc->xn, d_router_t, d_bias, sc->logits, T, d);
        else
            k_router_logits<1><<<(T + 1) / 2, 256, lsh, st>>>(sc->xn, d_router_t, d_bias, sc->logits, T, d);
    }
    if (!fused)
        k_router<<<T, rthreads, rsh, st>>>(sc->xn, d_router_t, d_bias, sc->logits, sc->idx, sc->w,
                                           d, E, K, s->norm_topk, have_logits ? 1 : 0);
    mhip::stage_end(c, slot);
    if (mhip::check_launch(c, "router")) return -1;

    // dispatch; the per-chunk counts live in tmp, which the down stage
    // writes only later
    const int nch = (A + DCH - 1) / DCH;
    const int dgrid = (nch + DWG - 1) / DWG;
    int bits = 0;
    while ((1 << bits) < E) bits++;
    int *dhist = (int *)sc->tmp;
    slot = mhip::stage_begin(c, MHIP_STAGE_DISPATCH);
    if (nch <= DSMALL) {
        k_disp_small<<<1, 64 * DSMALL, (DSMALL * E + 2 * E + 16) * 4, st>>>(
            sc->idx, A, E, nch, bits, sc->counts, sc->offsets, sc->perm, sc->pos, sc->groups,
            sc->gtile, sc->glight, MHIP_GEMM_TM, sc->status);
    } else {
        k_disp_count<<<dgrid, 64 * DWG, DWG * E * 4, st>>>(sc->idx, A, E, nch, dhist, sc->status);
        k_disp_scan<<<E, 256, 0, st>>>(nch, dhist, sc->counts);
        k_disp_scatter<<<dgrid, 64 * DWG, ((DWG + 2) * E + 16) * 4, st>>>(
            sc->idx, A, E, nch, bits, dhist, sc->counts, sc->offsets, sc->groups, sc->gtile,
            sc->glight, MHIP_GEMM_TM, sc->perm, sc->pos, sc->status);
    }
    mhip::stage_end(c, slot);
    if (mhip::check_launch(c, "dispatch")) return -1;

    if (mfma) {
        slot = mhip::stage_begin(c, MHIP_STAGE_GATEUP);
        int e = mhip::launch_gateup_mfma(st, s, lay, d_table_layer, sc, A);
        mhip::stage_end(c, slot);
        if (mhip::check(c, (hipError_t)e, "gateup_mfma launch")) return -1;
        slot = mhip::stage_begin(c, MHIP_STAGE_DOWN);
        e = mhip::launch_down_mfma(st, s, lay, d_table_layer, sc, A, !(flags & MHIP_FAST_DOWN));
        mhip::stage_end(c, slot);
        if (mhip::check(c, (hipError_t)e, "down_mfma launch")) return -1;
        dim3 cg(mhip::blocks_for(d, 1024), T);
        slot = mhip::stage_begin(c, MHIP_STAGE_COMBINE);
        k_combine<<<cg, 256, 0, st>>>(d_x, sc->w, sc->pos, sc->tmp, d, K, sc->status);
        mhip::stage_end(c, slot);
        return mhip::check_launch(c, "combine");
    }

    const int G = A < E ? A : E;  // at most this many non-empty experts
    const int Rg = rows_gateup(nb);
    const size_t gsh = gateup_lds(d, Rg);
    slot = mhip::stage_begin(c, MHIP_STAGE_GATEUP);
    k_gateup<PK><<<(unsigned)G * (eh / Rg), NT, gsh, st>>>(
        (const uint8_t *)d_table_layer, *lay, sc->xq, sc->xs, sc->groups, sc->perm, sc->h, d, eh,
        K, Rg);
    mhip::stage_end(c, slot);
    if (mhip::check_launch(c, "gateup")) return -1;

    const int Rd = rows_down(nbh);
    const size_t dsh2 = ((size_t)TB * Rd * (nbh + 1) + (size_t)TB * nbh) * sizeof(float) +
                        (size_t)TB * eh;
    slot = mhip::stage_begin(c, MHIP_STAGE_DOWN);
    const int nbq = A * nbh;
    k_quant_h<<<(nbq + 255) / 256, 256, 0, st>>>(sc->h, sc->hq, sc->hs, nbq);
    k_down<PKD><<<(unsigned)G * (d / Rd), NT, dsh2, st>>>((const uint8_t *)d_table_layer, *lay,
                                                         sc->hq, sc->hs, sc->groups, sc->tmp, d,
                                                         eh, Rd);
    mhip::stage_end(c, slot);
    if (mhip::check_launch(c, "down")) return -1;

    dim3 cg(mhip::blocks_for(d, 1024), T);
    slot = mhip::stage_begin(c, MHIP_STAGE_COMBINE);
    k_combine<<<cg, 256, 0, st>>>(d_x, sc->w, sc->pos, sc->tmp, d, K, sc->status);
    mhip::stage_end(c, slot);
    return mhip::check_launch(c, "combine");
}

unsigned long long mhip_matrix_layers(const mhip_ctx *c) { return c ? c->matrix_layers : 0; }

}  // extern "C"
