// The one-token attention of a layer of the Qwen3-30B-A3B shape (dim 2048,
// 32 query and 4 key/value heads of 128): the pieces that k_attn_layer
// (attn_layer.hip, one launch per layer) and the model stack (decode.hip,
// every layer of a token in one launch) share. Every value follows
// src/model/forward.c:118-165 of the reference in its order.
#pragma once

#include "mhip_internal.h"

namespace mhip_attn {

constexpr int D = 2048, NH = 32, NKV = 4, HD = 128;
constexpr int QD = NH * HD, KVD = NKV * HD, NROWS = QD + 2 * KVD;  // 4096, 512, 5120
constexpr int NB = D / 32, NBO = QD / 32;                            // 64, 128 blocks
constexpr int GROUP = NH / NKV;
constexpr int NT = 512, NW = NT / 64;         // the workgroup of both kernels
constexpr int KLD = HD + 4;                   // K row stride in LDS (rows on distinct banks)
static_assert(NB == 64 && NBO == 128, "one (two) block(s) per lane");

// Pointers into global memory (address space 1). Loads and stores through
// them compile to global_* instructions also where the pointer was read from
// memory; a generic pointer of that kind gives flat_* ones, which the
// compiler has to wait for together with LDS traffic.
template <class T> using gptr = __attribute__((address_space(1))) T *;
template <class T> __device__ __forceinline__ gptr<T> glob(T *p) { return (gptr<T>)p; }
// 16 bytes through such a pointer (the load goes through the built-in vector
// type: float4's assignment operators take generic references only)
typedef float f4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4(gptr<const float4> p) {
    const f4v v = *(gptr<const f4v>)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ld4(const float4 *p) { return *p; }

// One 36-byte block (scale, 32 codes) of a weight row as 9 dwords.
struct Blk {
    float d;
    int4 c0, c1;
};
__device__ __forceinline__ Blk load_blk(gptr<const uint8_t> p) {
    const gptr<const unsigned> u = (gptr<const unsigned>)p;
    Blk b;
    b.d = __uint_as_float(u[0]);
    b.c0 = make_int4((int)u[1], (int)u[2], (int)u[3], (int)u[4]);
    b.c1 = make_int4((int)u[5], (int)u[6], (int)u[7], (int)u[8]);
    return b;
}

// s_waitcnt vmcnt(0) with the other counters left alone (expcnt 7,
// lgkmcnt 15), for __builtin_amdgcn_s_waitcnt
constexpr int WAIT_VM0 = 0x0F70;

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from global memory straight into LDS, lane i's at
// lds + 16 i (lds wave-uniform); completion is counted by vmcnt.
__device__ __forceinline__ void dma16(unsigned lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// A DPP move of x (lanes of rows outside ROWS keep their own value, resp. 0
// for the double).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, ROWS, 0xf, false));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_d0(double x) {
    const uint64_t u = (uint64_t)__double_as_longlong(x);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, ROWS, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, ROWS, 0xf, false);
    return __longlong_as_double((long long)(((uint64_t)(unsigned)hi << 32) | (unsigned)lo));
}

// The maximum of v over each half wavefront (lanes 0-31, 32-63), in every
// lane of that half, by DPP moves (quad exchanges, row mirrors, the row
// broadcast): exact for values that are not NaN, in any order.
__device__ __forceinline__ float max32(float v, int lane) {
    v = fmaxf(v, dpp_f<0xB1, 0xf>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E, 0xf>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141, 0xf>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f<0x140, 0xf>(v));  // row_mirror: every lane holds its row's maximum
    v = fmaxf(v, dpp_f<0x142, 0xa>(v));  // row_bcast:15 into rows 1 and 3
    const float h0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float h1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return lane < 32 ? h0 : h1;
}

// The sum of v over the wavefront, in lane 63 (other lanes hold partial
// sums), by DPP moves of the two halves of each double; the order of the
// additions is fixed but not the index order.
__device__ __forceinline__ double wave_sum63(double v) {
    v = v + dpp_d0<0xB1, 0xf>(v);
    v = v + dpp_d0<0x4E, 0xf>(v);
    v = v + dpp_d0<0x141, 0xf>(v);
    v = v + dpp_d0<0x140, 0xf>(v);
    v = v + dpp_d0<0x142, 0xa>(v);  // rows 1, 3: + the row below (rows 0, 2: + 0)
    v = v + dpp_d0<0x143, 0xc>(v);  // rows 2, 3: + lane 31 (rows 0, 1: + 0)
    return v;
}

// Lane L's double, in every lane.
__device__ __forceinline__ double readlane_d(double x, int L) {
    const uint64_t u = (uint64_t)__double_as_longlong(x);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, L);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), L);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// The maximum of v over the wavefront, in every lane (as max32, then lane
// 31's value into rows 2 and 3).
__device__ __forceinline__ float max64(float v) {
    v = fmaxf(v, dpp_f<0xB1, 0xf>(v));
    v = fmaxf(v, dpp_f<0x4E, 0xf>(v));
    v = fmaxf(v, dpp_f<0x141, 0xf>(v));
    v = fmaxf(v, dpp_f<0x140, 0xf>(v));
    v = fmaxf(v, dpp_f<0x142, 0xa>(v));
    v = fmaxf(v, dpp_f<0x143, 0xc>(v));  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// DPP moves of the whole wavefront by one lane (lane 0 receives 0, resp.
// lane 63's value).
__device__ __forceinline__ float shr1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x138, 0xf, 0xf, false));
}
__device__ __forceinline__ float ror1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x13C, 0xf, 0xf, false));
}

// forward.c:75-81 over one head's row in LDS by one lane: the index-order
// double sum of squares.
__device__ inline float head_inv_seq(const float *row, float eps) {
    double ss = 0.0;
    for (int i = 0; i < HD; i += 32) {
        float4 r4[8];
#pragma unroll
        for (int j = 0; j < 8; j++) r4[j] = *(const float4 *)(row + i + 4 * j);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            ss = ss + (double)r4[j].x * (double)r4[j].x;
            ss = ss + (double)r4[j].y * (double)r4[j].y;
            ss = ss + (double)r4[j].z * (double)r4[j].z;
            ss = ss + (double)r4[j].w * (double)r4[j].w;
        }
    }
    return (float)(1.0 / sqrt(ss / HD + (double)eps));
}

// The same by one wavefront: lane l squares elements 2l, 2l+1 in double
// (exact), a butterfly adds the 128 squares in some order, and the bracket
// S -/+ (n + 64) 2^-52 S, which holds the index-order sum as well, gives the
// scale when both ends round to the same float; otherwise lane 0 runs the
// index-order sum.
__device__ __forceinline__ float head_inv_wave(const float *row, float eps, int lane, bool force_seq) {
    const float2 v = *(const float2 *)(row + 2 * lane);
    double ss = (double)v.x * (double)v.x + (double)v.y * (double)v.y;
    ss = readlane_d(wave_sum63(ss), 63);
    const double m = ss * ((double)(HD + 64) * 0x1p-52);
    const float lo = (float)(1.0 / sqrt((ss + m) / HD + (double)eps));
    const float hi = (float)(1.0 / sqrt((ss - m) / HD + (double)eps));
    if (lo == hi && !force_seq) return lo;  // the same in every lane
    float r = 0.0f;
    if (lane == 0) r = head_inv_seq(row, eps);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
}

// The normalized row, NeoX-rotated (forward.c:127-139): element i with
// i + HD/2 by the angle (c, sn), w0 = w[i], w1 = w[i + HD/2] the norm weight.
__device__ __forceinline__ void head_rope(const float *row, float inv, float w0, float w1,
                                          double c, double sn, float *dst, int i) {
    const int half = HD / 2;
    const float x0 = (row[i] * inv) * w0;
    const float x1 = (row[i + half] * inv) * w1;
    dst[i] = (float)((double)x0 * c - (double)x1 * sn);
    dst[i + half] = (float)((double)x0 * sn + (double)x1 * c);
}

// LDS of one query head's work; NPRE cache positions are staged in LDS.
template <int NPRE>
struct HeadLds {
    alignas(16) float tq[HD], tk[HD], tv[HD], qs[HD], ks[HD];
    alignas(16) float Ks[NPRE][KLD];  // the head's first cache rows
    alignas(16) float Vs[NPRE][HD];
    float red[NW];
    alignas(16) int8_t hq[HD];        // Q8 codes of the head's output
    float dsc[HD / 32];               // and their block scales
    float inv_q, inv_k, sum;
};

// What a head's threads request before they wait for its q/k/v rows: the
// first NPRE rows of the group's key and value cache, and (threads < HD)
// the RoPE angle and norm weights of element tid % (HD / 2) (threads below
// HD / 2 rotate q, the next HD / 2 k). The cache rows go to registers
// (DMA false) or straight into the head's LDS (DMA true).
struct HeadRope {
    float rw0, rw1;
    double rc, rs;
};
template <int NPRE, bool DMA = false>
struct HeadPre : HeadRope {
    static constexpr int KPF = NPRE * HD / 4 / NT;  // float4 of the K (and V) rows per thread
    static_assert(KPF * 4 * NT == NPRE * HD, "whole staging rounds");
    float4 kp[KPF], vp[KPF];
};
template <int NPRE>
struct HeadPre<NPRE, true> : HeadRope {};

template <int NPRE, bool DMA>
__device__ __forceinline__ void head_prefetch(HeadPre<NPRE, DMA> &p, HeadLds<NPRE> &s, int h,
                                              int pos, gptr<const float> kc,
                                              gptr<const float> vc, gptr<const float> q_norm,
                                              gptr<const float> k_norm, gptr<const double> rope,
                                              int tid) {
    // (only threads below HD read these: the others' stay unset, so no
    // register write has to wait for an older load of the same register)
    const int g = h / GROUP, npre = min(pos, NPRE);
    if (tid < HD) {
        const int i = tid % (HD / 2);
        const gptr<const float> w = tid < HD / 2 ? q_norm : k_norm;
        p.rw0 = w[i];
        p.rw1 = w[i + HD / 2];
        const gptr<const double> rp = rope + (size_t)pos * (HD / 2) * 2;
        p.rc = rp[2 * i];
        p.rs = rp[2 * i + 1];
    }
    if constexpr (DMA) {
        // wavefront w moves rows 2q, 2q + 1 for q = w, w + NW, ...: the V rows
        // are contiguous in LDS (one instruction), the K rows KLD apart (one
        // instruction per half wavefront). Rows past npre that a pair holds
        // are read from row min(t, pos), in the cache, and never used.
        static_assert(NPRE % 2 == 0, "row pairs");
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int half = lane >> 5, c = lane & 31;
        const unsigned ks = (unsigned)(uintptr_t)&s.Ks[0][0], vs = (unsigned)(uintptr_t)&s.Vs[0][0];
        for (int q = wave; 2 * q < npre; q += NW) {
            const int t0 = 2 * q, t = min(t0 + half, pos);
            const size_t off = (size_t)t * KVD + (size_t)g * HD + 4 * c;
            dma16(__builtin_amdgcn_readfirstlane(vs + (unsigned)(t0 * HD * 4)), (const float *)(vc + off));
            const unsigned k0 = __builtin_amdgcn_readfirstlane(ks + (unsigned)(t0 * KLD * 4));
            const unsigned k1 = __builtin_amdgcn_readfirstlane(ks + (unsigned)((t0 + 1) * KLD * 4 - 32 * 16));
            if (half == 0) dma16(k0, (const float *)(kc + off));
            else dma16(k1, (const float *)(kc + off));
        }
    } else {
#pragma unroll
        for (int j = 0; j < HeadPre<NPRE>::KPF; j++) {
            const int f = tid + NT * j, t = f / (HD / 4), c = f % (HD / 4);
            if (t < npre) {
                p.kp[j] = ld4((gptr<const float4>)(kc + (size_t)t * KVD + (size_t)g * HD + 4 * c));
                p.vp[j] = ld4((gptr<const float4>)(vc + (size_t)t * KVD + (size_t)g * HD + 4 * c));
            }
        }
    }
}

// q.k_t for one position: the sequential fp32 dot over the HD elements, the
// key row (in LDS or global memory) read 32 values ahead.
template <class P4>
__device__ __forceinline__ float head_dot(const float *qs, P4 k4p) {
    float dot = 0.0f;
    for (int i = 0; i < HD / 4; i += 8) {
        float4 k4[8];
#pragma unroll
        for (int j = 0; j < 8; j++) k4[j] = ld4(k4p + i + j);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            dot = dot + qs[4 * (i + j)] * k4[j].x;
            dot = dot + qs[4 * (i + j) + 1] * k4[j].y;
            dot = dot + qs[4 * (i + j) + 2] * k4[j].z;
            dot = dot + qs[4 * (i + j) + 3] * k4[j].w;
        }
    }
    return dot;
}

// A phase mark that does nothing (head_run's default).
struct NoMark {
    __device__ void operator()(int) const {}
};

// Query head h (forward.c:127-163) by a whole workgroup, every thread
// calling, once s.tq, s.tk, s.tv hold its q row and its group's k and v
// rows (with DMA, after head_prefetch issued the cache rows' copies): the
// head norms, RoPE, the cache append (by the group's first head),
// scores q.k_t * scale (sequential fp32 dots, one position per thread, the
// key row read 32 values ahead), softmax (the maximum, the restated expf,
// the sequential sum, the division), the mix in position order, and Q8 of
// the head's output into s.hq / s.dsc. sc: pos + 1 floats of LDS.
// mark(i), i = 0..8, runs after each of its barriers (a caller's phase trace).
template <int NPRE, bool DMA, class Mark = NoMark>
__device__ inline void head_run(HeadLds<NPRE> &s, float *sc, const HeadPre<NPRE, DMA> &p, int h,
                                int pos, gptr<float> kcg, gptr<float> vcg, float eps, float scale,
                                bool force_seq, const uint64_t *etab, Mark mark = Mark()) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = h / GROUP, n = pos + 1, npre = min(pos, NPRE);
    if constexpr (DMA) {
        // this wavefront's cache rows are in (a wait the compiler sees: it
        // then also counts every earlier load of the wavefront as done)
        __builtin_amdgcn_s_waitcnt(WAIT_VM0);
    } else {
#pragma unroll
        for (int j = 0; j < HeadPre<NPRE>::KPF; j++) {
            const int f = tid + NT * j, t = f / (HD / 4), c = f % (HD / 4);
            if (t < npre) {
                *(float4 *)&s.Ks[t][4 * c] = p.kp[j];
                *(float4 *)&s.Vs[t][4 * c] = p.vp[j];
            }
        }
    }
    __syncthreads();
    mark(0);
    if (wave < 2) {
        const float inv = head_inv_wave(wave == 0 ? s.tq : s.tk, eps, lane, force_seq);
        if (lane == 0) (wave == 0 ? s.inv_q : s.inv_k) = inv;
    }
    __syncthreads();
    mark(1);
    if (tid < HD / 2) head_rope(s.tq, s.inv_q, p.rw0, p.rw1, p.rc, p.rs, s.qs, tid);
    else if (tid < HD) head_rope(s.tk, s.inv_k, p.rw0, p.rw1, p.rc, p.rs, s.ks, tid - HD / 2);
    __syncthreads();
    mark(2);
    if (h % GROUP == 0 && tid < HD) {
        kcg[(size_t)pos * KVD + (size_t)g * HD + tid] = s.ks[tid];
        vcg[(size_t)pos * KVD + (size_t)g * HD + tid] = s.tv[tid];
    }
    for (int t = tid; t < n; t += NT) {
        // a key row in LDS (the new one, or staged) or in the cache
        const float dot = t == pos || t < npre
                              ? head_dot(s.qs, (const float4 *)(t == pos ? s.ks : &s.Ks[t][0]))
                              : head_dot(s.qs, (gptr<const float4>)(kcg + (size_t)t * KVD +
                                                                    (size_t)g * HD));
        sc[t] = dot * scale;
    }
    __syncthreads();
    mark(3);
    float mx = -__builtin_inff();
    for (int t = tid; t < n; t += NT) mx = fmaxf(mx, sc[t]);
    mx = max64(mx);  // (fmaxf keeps the larger of a number and a NaN: any order gives this)
    if (lane == 0) s.red[wave] = mx;
    __syncthreads();
    mark(4);
#pragma unroll
    for (int w = 0; w < NW; w++) mx = fmaxf(mx, s.red[w]);
    for (int t = tid; t < n; t += NT) sc[t] = mia_expf_glibc_tab(sc[t] - mx, etab);
    __syncthreads();
    mark(5);
    if (tid == 0) {
        float sum = 0.0f;
        for (int t = 0; t < n; t++) sum = sum + sc[t];
        s.sum = sum;
    }
    __syncthreads();
    mark(6);
    const float sum = s.sum;
    for (int t = tid; t < n; t += NT) sc[t] = sc[t] / sum;
    __syncthreads();
    mark(7);
    if (tid < HD) {
        const gptr<const float> vt = vcg + (size_t)g * HD + tid;
        float o = 0.0f;
        int t = 0;
        for (; t < npre; t++) o = o + sc[t] * s.Vs[t][tid];
        for (; t + 16 <= pos; t += 16) {
            float vv[16];
#pragma unroll
            for (int j = 0; j < 16; j++) vv[j] = vt[(size_t)(t + j) * KVD];
#pragma unroll
            for (int j = 0; j < 16; j++) o = o + sc[t + j] * vv[j];
        }
        for (; t < pos; t++) o = o + sc[t] * vt[(size_t)t * KVD];
        o = o + sc[pos] * s.tv[tid];
        const float am = max32(fmaxf(0.0f, fabsf(o)), lane);  // a NaN counts as 0
        const float d = am / 127.0f;
        const float qi = d != 0.0f ? 1.0f / d : 0.0f;
        s.hq[tid] = (int8_t)roundf(o * qi);
        if ((lane & 31) == 0) s.dsc[tid / 32] = d;
    }
    __syncthreads();
    mark(8);
}

}  // namespace mhip_attn
