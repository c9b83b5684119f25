// Persistent single-launch decode of a stack of Qwen3-MoE FFN layers at batch
// 1 (one token through layers 0..L-1, src/model/forward.c:210-213 without the
// attention call), for the Qwen3-30B-A3B shape (dim 2048, 128 experts, top-K
// with K <= 8, expert_hidden 768).
//
// Layout on the chip. The grid is 256 workgroups of 512 threads, one per CU;
// workgroup b runs on XCD b % 8 (checked against HW_REG_XCC_ID at start).
// XCD k owns routed expert slot k: its 32 workgroups stream that expert's
// gate/up/down rows (5.3 MB) while the other XCDs stream theirs, so each
// expert's intermediate h stays inside one XCD. Every XCD recomputes the
// (tiny) router and top-K itself, so the only cross-XCD traffic per layer is
// the K expert outputs (K x 8 KB) gathered by the combine.
//
// Per layer, on every XCD:
//   A  x (8 KB) -> certified rmsnorm -> xn, Q8(xn) in LDS; 4 router logits per
//      workgroup by a parallel sum with a rigorous bound on the distance to
//      the reference's sequential fp32 chain                 [XCD sync]
//   B  all 128 logits -> top-K + certification -> gate weights (if the
//      ordering is not certified, the exact sequential logits are computed
//      and routing follows the reference bit for bit)
//   C  gate/up rows of expert idx[k] + SwiGLU -> h (768 floats) [XCD sync]
//      (the down rows and the next layer's router rows are loaded meanwhile)
//   D  Q8(h) -> down rows -> the expert's output rows, published device-wide
//   E  combine x_r += w_j * out_j,r in top-K order for 64 rows [XCD sync]
//
// Intra-XCD synchronisation is an L2 atomic counter; cross-XCD data is written
// with device-scope stores and read with device-scope loads after a
// point-to-point flag. No agent-scope cache maintenance is issued.
//
// Results: top-K indices bit-equal to the reference (certified, with an exact
// fallback); expert products, SwiGLU, Q8(h), down and combine follow the
// reference's rounding order; the gate weights come from the parallel logits
// (relative error ~1e-6 against the reference's), unless the exact fallback
// ran for that layer.
#include "mhip_internal.h"

namespace {

constexpr int NX = 8;            // XCDs
constexpr int WPX = 32;          // workgroups per XCD
constexpr int NWG = NX * WPX;    // 256
constexpr int NT = 512;          // threads per workgroup
constexpr int NWAVE = NT / 64;
constexpr int D = 2048, E = 128, EH = 768, KMAX = 8;
constexpr int NB = D / 32, NBH = EH / 32;
constexpr int HROWS = EH / WPX;             // 24 h rows per workgroup
constexpr int GU_RW = 2 * HROWS / NWAVE;    // 6 weight rows per wave (3 gate, 3 up)
constexpr int DROWS = D / WPX;              // 64 down rows per workgroup
constexpr int DPK = DROWS * NBH / NT;       // 3 (row, block) pairs per thread
constexpr int LPW = E / WPX;                // 4 logits per workgroup
constexpr long SPIN = 1L << 18;

typedef int v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld_stream(const void *p) {
    const v4i v = __builtin_nontemporal_load((const v4i *)p);
    return make_int4(v.x, v.y, v.z, v.w);
}

static_assert(NB == 64, "one 32-block per lane");
static_assert(GU_RW * NWAVE == 2 * HROWS && DPK * NT == DROWS * NBH, "tiling");

struct DecodeWs {
    unsigned gstart[64];          // start barrier (device scope)
    unsigned cnt[NX][64];         // intra-XCD counters, monotonic
    unsigned tflag[NWG][16];      // expert-output rows published (layer + 1)
    unsigned xflag[NX][16];       // exact logits published (layer + 1)
    int status[16];               // [0] abort bits, [1] rms fallbacks, [2] router fallbacks
    float x[NX][D];
    double lg[NX][E][2];          // parallel logit sum S and bound B
    float lx[NX][E];              // exact logits (fallback)
    float h[NX][EH];
    float out[2][KMAX][D];        // expert outputs, double-buffered by layer parity
    unsigned long long trace[2][64][12];  // stage timestamps of two workgroups (diagnostic)
};

struct DecodeArgs {
    const uint8_t *table;         // layer 0, experts expert_bytes apart, layers E*expert_bytes
    mhip_layout lay;
    const float *router;          // [L][E][D]
    const float *router_t;        // [L][D][E]
    const float *norm;            // [L][D]
    const float *bias;            // [E] or null
    float *x;                     // [D] in/out
    DecodeWs *ws;
    int *idx_out;                 // [L][K] or null
    float *w_out;                 // [L][K] or null
    int L, K, norm_topk, flags;
    float eps;
};

__device__ __forceinline__ unsigned xcc_id() {
    return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));
}
__device__ __forceinline__ unsigned ld_dev(const unsigned *p) {
    return __hip_atomic_load((unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_devf(const float *p) {
    return __uint_as_float(ld_dev((const unsigned *)p));
}
__device__ __forceinline__ double ld_devd(const double *p) {
    unsigned long long v = __hip_atomic_load((unsigned long long *)p, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
    return __longlong_as_double((long long)v);
}
__device__ __forceinline__ void st_dev(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_devf(float *p, float v) { st_dev((unsigned *)p, __float_as_uint(v)); }
__device__ __forceinline__ void st_devd(double *p, double v) {
    __hip_atomic_store((unsigned long long *)p, (unsigned long long)__double_as_longlong(v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Abort bits: 1 = workgroup not on the expected XCD, 2 = a wait timed out.
__device__ __forceinline__ bool aborted(DecodeWs *ws) {
    return ld_dev((const unsigned *)&ws->status[0]) != 0;
}

// All of this workgroup's stores complete, then one arrival on the XCD
// counter; wait until all WPX workgroups of the XCD arrived `phase` times.
__device__ void xcd_sync(DecodeWs *ws, int xcd, unsigned phase) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned *c = &ws->cnt[xcd][0];
        __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        long s = 0;
        while (ld_dev(c) < phase * WPX) {
            if (++s > SPIN || ((s & 255) == 0 && aborted(ws))) {
                atomicOr(&ws->status[0], 2);
                break;
            }
        }
    }
    __syncthreads();
}

__device__ void wait_flag(DecodeWs *ws, const unsigned *flag, unsigned value) {
    long s = 0;
    while (ld_dev(flag) < value) {
        if (++s > SPIN || ((s & 255) == 0 && aborted(ws))) {
            atomicOr(&ws->status[0], 2);
            break;
        }
    }
}

// Wavefront-wide inclusive prefix sum with DPP (row_shr 1/2/4/8 inside each
// row of 16 lanes, then row_bcast 15/31 across rows); lanes receive 0 where
// there is no source lane.
template <int CTRL, int ROW_MASK, bool ZERO_FILL>
__device__ __forceinline__ double dpp_d(double v) {
    int lo = __double2loint(v), hi = __double2hiint(v);
    lo = __builtin_amdgcn_update_dpp(0, lo, CTRL, ROW_MASK, 0xf, ZERO_FILL);
    hi = __builtin_amdgcn_update_dpp(0, hi, CTRL, ROW_MASK, 0xf, ZERO_FILL);
    return __hiloint2double(hi, lo);
}
__device__ __forceinline__ double wave_scan_d(double v) {
    v = v + dpp_d<0x111, 0xf, true>(v);
    v = v + dpp_d<0x112, 0xf, true>(v);
    v = v + dpp_d<0x114, 0xf, true>(v);
    v = v + dpp_d<0x118, 0xf, true>(v);
    v = v + dpp_d<0x142, 0xa, false>(v);
    v = v + dpp_d<0x143, 0xc, false>(v);
    return v;
}
__device__ __forceinline__ double lane63_d(double v) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), 63),
                            __builtin_amdgcn_readlane(__double2loint(v), 63));
}
// Wavefront-wide maximum (order-free): the same DPP pattern with max, lanes
// without a source keep their own value. Returned in every lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_keep_d(double v) {
    const int lo = __double2loint(v), hi = __double2hiint(v);
    return __hiloint2double(__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xf, false),
                            __builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ double wave_max_d(double v) {
    v = fmax(v, dpp_keep_d<0x111, 0xf>(v));
    v = fmax(v, dpp_keep_d<0x112, 0xf>(v));
    v = fmax(v, dpp_keep_d<0x114, 0xf>(v));
    v = fmax(v, dpp_keep_d<0x118, 0xf>(v));
    v = fmax(v, dpp_keep_d<0x142, 0xa>(v));
    v = fmax(v, dpp_keep_d<0x143, 0xc>(v));
    return lane63_d(v);
}
__device__ __forceinline__ float lanef(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double laned(double v, int lane) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                            __builtin_amdgcn_readlane(__double2loint(v), lane));
}

// One round of "largest untaken value, lowest index on ties" over the 128
// values held two per lane (v0 for index lane, v1 for index lane + 64), in
// one wavefront. Returns the winning index (uniform); -1 if none (all taken
// or NaN).
__device__ __forceinline__ int wave_argmax_d(double v0, double v1, bool t0, bool t1, int lane) {
    const double ninf = -__builtin_inf();
    const double a0 = t0 ? ninf : v0, a1 = t1 ? ninf : v1;
    const double m = wave_max_d(fmax(a0, a1));
    const unsigned long long lo = __ballot(!t0 && a0 == m);
    if (lo) return __builtin_ctzll(lo);
    const unsigned long long hi = __ballot(!t1 && a1 == m);
    if (hi) return 64 + __builtin_ctzll(hi);
    return -1;
}

__device__ __forceinline__ float wave_sum_f(float v) {
    // through double: exact for the wave-wide sum of 64 floats' partials
    return (float)lane63_d(wave_scan_d((double)v));
}

// LDS. `scr` is reused by stages that never overlap: the exact-router
// products (B, fallback), the gate/up terms (C) and the down terms and
// gathered expert outputs (D, E).
constexpr int GU_LD = NB + 4;     // 16-byte aligned rows
constexpr int DN_LD = NBH + 4;
constexpr int SCR = 8192;         // floats
static_assert(NWAVE * GU_RW * GU_LD <= SCR && DROWS * DN_LD <= SCR && LPW * D <= SCR, "scr");

struct Lds {
    alignas(16) float x[D];
    alignas(16) float xn[D];
    alignas(16) int8_t xq[D];
    alignas(16) float scr[SCR];
    alignas(16) float hs[EH];
    alignas(16) int8_t hq[EH];
    float xs[NB];
    float hsc[NBH];
    float gu[NWAVE][GU_RW];
    alignas(16) float p[E];       // probabilities (or exp values)
    float lf[E];                  // fp32 logits
    double c[E];                  // ranking centre of each logit
    double r[E];                  // its bound
    double part[NT];
    double wtot[LPW][64];
    double wabs[LPW][64];
    int order[KMAX + 1];
    float inv;
    float sum;
    int idx[KMAX];
    float w[KMAX];
    int fallback;
};

// Sequential fp32 sum of n (multiple of 4) LDS floats starting at p, in
// order, with 16-byte reads.
__device__ __forceinline__ float lds_seq_sum(const float *p, int n, float s) {
    const float4 *v = (const float4 *)p;
#pragma unroll 4
    for (int k = 0; k < n / 4; k++) {
        const float4 q = v[k];
        s = s + q.x;
        s = s + q.y;
        s = s + q.z;
        s = s + q.w;
    }
    return s;
}

// Diagnostic: workgroups 0 and 1 (XCDs 0 and 1) record the 100 MHz real-time
// counter at each stage boundary of the first 64 layers.
#define TRACE(slot)                                                                       \
    do {                                                                                  \
        if ((a.flags & MHIP_DECODE_TRACE) && blockIdx.x < 2 && tid == 0 && l < 64)       \
            ws->trace[blockIdx.x][l][slot] = __builtin_amdgcn_s_memrealtime();            \
    } while (0)

__global__ __launch_bounds__(NT) void k_decode_stack(DecodeArgs a) {
    __shared__ Lds sh;
    DecodeWs *ws = a.ws;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int xcd = blockIdx.x % NX, rank = blockIdx.x / NX;
    const int K = a.K;
    const size_t layer_bytes = (size_t)E * a.lay.expert_bytes;

    // Start: every workgroup checks its XCD, then a device-wide barrier.
    if (tid == 0) {
        if (xcc_id() != (unsigned)xcd) atomicOr(&ws->status[0], 1);
        __builtin_amdgcn_s_waitcnt(0);
        __hip_atomic_fetch_add(&ws->gstart[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_flag(ws, &ws->gstart[0], NWG);
    }
    __syncthreads();
    if (aborted(ws)) return;

    unsigned phase = 0;
    // Router rows of this workgroup's logits (waves 0..LPW-1), next layer first.
    float4 rrow[8];
#define LOAD_ROUTER(layer)                                                                 \
    do {                                                                                   \
        if (wave < LPW) {                                                                  \
            const float4 *src_ = (const float4 *)(a.router +                               \
                                                  ((size_t)(layer) * E + rank * LPW + wave) * D + \
                                                  lane * 32);                              \
            _Pragma("unroll") for (int k_ = 0; k_ < 8; k_++) rrow[k_] = src_[k_];          \
        }                                                                                  \
    } while (0)
    LOAD_ROUTER(0);
    for (int i = tid; i < D; i += NT) sh.x[i] = a.x[i];

    for (int l = 0; l < a.L; l++) {
        const float *wnorm = a.norm + (size_t)l * D;
        TRACE(0);
        // ---- A: rmsnorm (certified), xn, Q8(xn) -----------------------------------
        __syncthreads();
        {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < D / NT; k++) {
                const double v = (double)sh.x[tid + NT * k];
                ss = ss + v * v;
            }
            ss = lane63_d(wave_scan_d(ss));
            if (lane == 0) sh.part[wave] = ss;
        }
        __syncthreads();
        if (tid == 0) {
            // Any summation order is within (n + log2 n) 2^-53 S of the
            // reference's sequential sum (all terms >= 0); S -/+ m brackets it.
            double S = 0.0;
            for (int k = 0; k < NWAVE; k++) S = S + sh.part[k];
            const double m = S * ((double)(D + 64) * 0x1p-52);
            const float lo = (float)(1.0 / sqrt((S + m) / D + (double)a.eps));
            const float hi = (float)(1.0 / sqrt((S - m) / D + (double)a.eps));
            float inv = lo;
            if ((a.flags & MHIP_FORCE_SEQ_RMS) || lo != hi) {
                double sq = 0.0;
                for (int i = 0; i < D; i++) sq = sq + (double)sh.x[i] * (double)sh.x[i];
                inv = (float)(1.0 / sqrt(sq / D + (double)a.eps));
                if (blockIdx.x == 0) atomicAdd(&ws->status[1], 1);
            }
            sh.inv = inv;
        }
        __syncthreads();
        {
            const float inv = sh.inv;
#pragma unroll
            for (int k = 0; k < D / NT; k++) {
                const int i = tid + NT * k;
                sh.xn[i] = (sh.x[i] * inv) * wnorm[i];
            }
        }
        __syncthreads();
        if (tid < NB) {
            // Q8_0 of one 32-block (quant.c:11-27)
            const float4 *v4 = (const float4 *)&sh.xn[tid * 32];
            float v[32];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 q = v4[k];
                v[4 * k] = q.x;
                v[4 * k + 1] = q.y;
                v[4 * k + 2] = q.z;
                v[4 * k + 3] = q.w;
            }
            float am = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) am = fmaxf(am, fabsf(v[i]));
            const float dsc = am / 127.0f;
            const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
            union {
                int8_t c[32];
                int4 v4[2];
            } q;
#pragma unroll
            for (int i = 0; i < 32; i++) q.c[i] = (int8_t)roundf(v[i] * qi);
            ((int4 *)&sh.xq[tid * 32])[0] = q.v4[0];
            ((int4 *)&sh.xq[tid * 32])[1] = q.v4[1];
            sh.xs[tid] = dsc;
        }
        // Parallel logits with a bound. The reference's logit is the
        // sequential fp32 chain over p_i = fl(W_ei * xn_i); S = sum p_i in
        // double, and |chain - S| <= 2^-24 * sum_k |S_k| (S_k the prefix sums).
        // p_i = fl(W_ei * xn_i) for this lane's 32 elements (recomputed in the
        // second pass rather than held across the barrier)
        if (wave < LPW) {
            const float4 *xv4 = (const float4 *)&sh.xn[lane * 32];
            double tot = 0.0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 wv = rrow[k], xv = xv4[k];
                tot = tot + (double)(wv.x * xv.x);
                tot = tot + (double)(wv.y * xv.y);
                tot = tot + (double)(wv.z * xv.z);
                tot = tot + (double)(wv.w * xv.w);
            }
            const double incl = wave_scan_d(tot);
            double run = incl - tot;  // exclusive prefix of this lane
            double absum = 0.0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 wv = rrow[k], xv = xv4[k];
                run = run + (double)(wv.x * xv.x);
                absum = absum + fabs(run);
                run = run + (double)(wv.y * xv.y);
                absum = absum + fabs(run);
                run = run + (double)(wv.z * xv.z);
                absum = absum + fabs(run);
                run = run + (double)(wv.w * xv.w);
                absum = absum + fabs(run);
            }
            const double S = lane63_d(incl);
            const double A = lane63_d(wave_scan_d(absum));
            if (lane == 0) {
                const int e = rank * LPW + wave;
                st_devd(&ws->lg[xcd][e][0], S);
                st_devd(&ws->lg[xcd][e][1], A * 0x1p-24 * (1.0 + 0x1p-8) + 1e-30);
            }
        }
        TRACE(1);
        xcd_sync(ws, xcd, ++phase);
        TRACE(2);

        // ---- B: top-K, certification, gate weights (wavefront 0, registers) --------
        if (wave == 0) {
            // lane holds experts lane and lane + 64
            const double S0 = ld_devd(&ws->lg[xcd][lane][0]);
            const double S1 = ld_devd(&ws->lg[xcd][lane + 64][0]);
            const double B0 = ld_devd(&ws->lg[xcd][lane][1]);
            const double B1 = ld_devd(&ws->lg[xcd][lane + 64][1]);
            const float bias0 = a.bias ? a.bias[lane] : 0.0f;
            const float bias1 = a.bias ? a.bias[lane + 64] : 0.0f;
            const double c0 = S0 + (double)bias0, c1 = S1 + (double)bias1;
            const float lf0 = a.bias ? (float)S0 + bias0 : (float)S0;
            const float lf1 = a.bias ? (float)S1 + bias1 : (float)S1;
            TRACE(10);
            const double bmax = wave_max_d(fmax(B0, B1));
            bool t0 = false, t1 = false, ok = (a.flags & MHIP_FORCE_EXACT_ROUTER) == 0;
            const int need = K < E ? K + 1 : K;
            double top = 0.0, prev = 0.0;
            int sel[KMAX + 1];
            bool valid = true;
#pragma unroll
            for (int j = 0; j < KMAX + 1; j++) {
                sel[j] = 0;
                if (j < need && valid) {
                    const int win = wave_argmax_d(c0, c1, t0, t1, lane);
                    if (win < 0) {  // NaN logits: take the exact path
                        ok = false;
                        valid = false;
                    } else {
                        sel[j] = win;
                        if (win == lane) t0 = true;
                        if (win == lane + 64) t1 = true;
                        const double cw = laned(win < 64 ? c0 : c1, win & 63);
                        if (j == 0) top = cw;
                        if (j > 0) {
                            // Margin for the fp32 roundings between the logit and
                            // the probability (logit+bias, l-mx, expf, division).
                            const double tau = 0x1p-19 * (2.0 + fabs(top) + fabs(prev));
                            if (!(prev - cw > 2.0 * bmax + tau)) ok = false;
                        }
                        prev = cw;
                    }
                }
            }
            TRACE(11);
            if (ok) {
                // Softmax of the parallel logits (forward.c:95-101 in shape; the
                // gate weights only need the 1e-3 tolerance).
                const float mx = lanef(sel[0] < 64 ? lf0 : lf1, sel[0] & 63);
                const float e0 = mhip_dev::expf_glibc(lf0 - mx);
                const float e1 = mhip_dev::expf_glibc(lf1 - mx);
                const float sum = wave_sum_f(e0 + e1);
                float pj[KMAX], wsum = 0.0f;
#pragma unroll
                for (int j = 0; j < KMAX; j++) {
                    if (j < K) {
                        pj[j] = lanef(sel[j] < 64 ? e0 : e1, sel[j] & 63) / sum;
                        wsum = wsum + pj[j];
                    }
                }
                if (lane == 0) {
#pragma unroll
                    for (int j = 0; j < KMAX; j++) {
                        if (j < K) {
                            sh.idx[j] = sel[j];
                            sh.w[j] = a.norm_topk ? pj[j] / wsum : pj[j];
                        }
                    }
                }
            }
            if (lane == 0) sh.fallback = ok ? 0 : 1;
        }
        __syncthreads();
        if (sh.fallback) {
            // Exact logits, the reference's sequential chain: each workgroup
            // computes its 4 (one per wave: products to LDS, lane 0 sums them
            // in order), then the XCD exchanges them.
            if (wave < LPW) {
                const int e = rank * LPW + wave;
                const float4 *src = (const float4 *)(a.router + ((size_t)l * E + e) * D + lane * 32);
                float *pw = &sh.scr[wave * D];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 wv = src[k];
                    const float *xv = &sh.xn[lane * 32 + 4 * k];
                    pw[lane * 32 + 4 * k + 0] = wv.x * xv[0];
                    pw[lane * 32 + 4 * k + 1] = wv.y * xv[1];
                    pw[lane * 32 + 4 * k + 2] = wv.z * xv[2];
                    pw[lane * 32 + 4 * k + 3] = wv.w * xv[3];
                }
            }
            __syncthreads();
            if (wave < LPW && lane == 0) {
                const int e = rank * LPW + wave;
                float s = lds_seq_sum(&sh.scr[wave * D], D, 0.0f);
                if (a.bias) s = s + a.bias[e];
                st_devf(&ws->lx[xcd][e], s);
            }
            xcd_sync(ws, xcd, ++phase);
            if (tid < E) sh.lf[tid] = ld_devf(&ws->lx[xcd][tid]);
            __syncthreads();
            if (tid == 0) {
                // forward.c:95-101 exactly: first maximum, sequential sum.
                float mx = sh.lf[0];
                for (int i = 1; i < E; i++) mx = sh.lf[i] > mx ? sh.lf[i] : mx;
                sh.inv = mx;
            }
            __syncthreads();
            if (tid < E) sh.p[tid] = mhip_dev::expf_glibc(sh.lf[tid] - sh.inv);
            __syncthreads();
            if (tid == 0) sh.sum = lds_seq_sum(sh.p, E, 0.0f);
            __syncthreads();
            if (tid < E) sh.p[tid] = sh.p[tid] / sh.sum;
            __syncthreads();
            if (tid < E) {
                // forward.c:104-114: descending p, lowest index on ties
                const float pe = sh.p[tid];
                int rk = 0;
                for (int i = 0; i < E; i++) {
                    const float pi = sh.p[i];
                    rk += (int)(pi > pe) + ((int)(pi == pe) & (int)(i < tid));
                }
                if (rk < K) sh.idx[rk] = tid;
            }
            __syncthreads();
            if (tid == 0) {
                float wsum = 0.0f;
                for (int j = 0; j < K; j++) wsum = wsum + sh.p[sh.idx[j]];
                for (int j = 0; j < K; j++)
                    sh.w[j] = a.norm_topk ? sh.p[sh.idx[j]] / wsum : sh.p[sh.idx[j]];
                if (xcd == 0 && rank == 0) atomicAdd(&ws->status[2], 1);
            }
        }
        __syncthreads();
        TRACE(3);
        if (blockIdx.x == 0 && tid < K) {
            if (a.idx_out) a.idx_out[(size_t)l * K + tid] = sh.idx[tid];
            if (a.w_out) a.w_out[(size_t)l * K + tid] = sh.w[tid];
        }

        // ---- C: gate/up + SwiGLU for expert slot `xcd` -----------------------------
        const bool active = xcd < K;
        int4 dq0[DPK], dq1[DPK];
        float dsc[DPK];
        if (active) {
            const int ex = sh.idx[xcd];
            const uint8_t *eb = a.table + (size_t)l * layer_bytes + (size_t)ex * a.lay.expert_bytes;
            // this wave's rows: gate h0..h0+2, then up h0..h0+2
            const int h0 = rank * HROWS + wave * (GU_RW / 2);
            int4 gq0[GU_RW], gq1[GU_RW];
            float gs[GU_RW];
#pragma unroll
            for (int r = 0; r < GU_RW; r++) {
                const int row = h0 + (r % (GU_RW / 2));
                const size_t qoff = (r < GU_RW / 2 ? a.lay.gate_q : a.lay.up_q) + (size_t)row * D +
                                    (size_t)lane * 32;
                const size_t soff = (r < GU_RW / 2 ? a.lay.gate_s : a.lay.up_s);
                const int4 *src = (const int4 *)(eb + qoff);
                gq0[r] = ld_stream(src);
                gq1[r] = ld_stream(src + 1);
                gs[r] = ((const float *)(eb + soff))[(size_t)row * NB + lane];
            }
            // down rows of this workgroup (used after the next sync)
#pragma unroll
            for (int k = 0; k < DPK; k++) {
                const int pidx = tid + NT * k;
                const int row = rank * DROWS + pidx / NBH, blk = pidx % NBH;
                const int4 *src =
                    (const int4 *)(eb + a.lay.down_q + (size_t)row * EH + (size_t)blk * 32);
                dq0[k] = ld_stream(src);
                dq1[k] = ld_stream(src + 1);
                dsc[k] = ((const float *)(eb + a.lay.down_s))[(size_t)row * NBH + blk];
            }
            if (l + 1 < a.L) LOAD_ROUTER(l + 1);
            const int4 *xv = (const int4 *)&sh.xq[lane * 32];
            const int4 x0 = xv[0], x1 = xv[1];
            const float dx = sh.xs[lane];
            float *terms = &sh.scr[wave * GU_RW * GU_LD];
#pragma unroll
            for (int r = 0; r < GU_RW; r++)
                terms[r * GU_LD + lane] =
                    mhip_dev::block_term(mhip_dev::dot32_i8(gq0[r], gq1[r], x0, x1), gs[r], dx);
            __syncthreads();
            if (lane < GU_RW) sh.gu[wave][lane] = lds_seq_sum(&terms[lane * GU_LD], NB, 0.0f);
            __syncthreads();
            if (lane < GU_RW / 2) {
                const float g = sh.gu[wave][lane], u = sh.gu[wave][GU_RW / 2 + lane];
                st_devf(&ws->h[xcd][h0 + lane], (g / (1.0f + mhip_dev::expf_glibc(-g))) * u);
            }
        } else if (l + 1 < a.L) {
            LOAD_ROUTER(l + 1);
        }
        TRACE(4);
        xcd_sync(ws, xcd, ++phase);
        TRACE(5);

        // ---- D: Q8(h) and down ------------------------------------------------------
        const int par = l & 1;
        if (active) {
            {
                const float h0 = ld_devf(&ws->h[xcd][tid]);
                const float h1 = tid + NT < EH ? ld_devf(&ws->h[xcd][tid + NT]) : 0.0f;
                sh.hs[tid] = h0;
                if (tid + NT < EH) sh.hs[tid + NT] = h1;
            }
            __syncthreads();
            if (tid < NBH) {
                const float4 *v4 = (const float4 *)&sh.hs[tid * 32];
                float v[32];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 q = v4[k];
                    v[4 * k] = q.x;
                    v[4 * k + 1] = q.y;
                    v[4 * k + 2] = q.z;
                    v[4 * k + 3] = q.w;
                }
                float am = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; i++) am = fmaxf(am, fabsf(v[i]));
                const float d = am / 127.0f;
                const float qi = d != 0.0f ? 1.0f / d : 0.0f;
                union {
                    int8_t c[32];
                    int4 v4[2];
                } q;
#pragma unroll
                for (int i = 0; i < 32; i++) q.c[i] = (int8_t)roundf(v[i] * qi);
                ((int4 *)&sh.hq[tid * 32])[0] = q.v4[0];
                ((int4 *)&sh.hq[tid * 32])[1] = q.v4[1];
                sh.hsc[tid] = d;
            }
            __syncthreads();
            float *dterm = sh.scr;
#pragma unroll
            for (int k = 0; k < DPK; k++) {
                const int pidx = tid + NT * k;
                const int row = pidx / NBH, blk = pidx % NBH;
                const int4 *hv = (const int4 *)&sh.hq[blk * 32];
                dterm[row * DN_LD + blk] = mhip_dev::block_term(
                    mhip_dev::dot32_i8(dq0[k], dq1[k], hv[0], hv[1]), dsc[k], sh.hsc[blk]);
            }
            __syncthreads();
            if (tid < DROWS)
                st_devf(&ws->out[par][xcd][rank * DROWS + tid],
                        lds_seq_sum(&dterm[tid * DN_LD], NBH, 0.0f));
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0) st_dev(&ws->tflag[blockIdx.x][0], (unsigned)(l + 1));
        }
        TRACE(6);

        // ---- E: combine rows rank*64 .. +64 in top-K order ---------------------------
        if (tid < K) wait_flag(ws, &ws->tflag[rank * NX + tid][0], (unsigned)(l + 1));
        __syncthreads();
        TRACE(7);
        {
            // thread (j, r) fetches expert j's output row r; then one thread
            // per row adds them in top-K order
            const int j = tid / DROWS, r = tid % DROWS;
            if (j < K) sh.scr[r * KMAX + j] = ld_devf(&ws->out[par][j][rank * DROWS + r]);
        }
        __syncthreads();
        if (tid < DROWS) {
            const int r = rank * DROWS + tid;
            float v = sh.x[r];
            for (int j = 0; j < K; j++) v = v + sh.w[j] * sh.scr[tid * KMAX + j];
            st_devf(&ws->x[xcd][r], v);
            if (l == a.L - 1 && xcd == 0) a.x[r] = v;
        }
        TRACE(8);
        xcd_sync(ws, xcd, ++phase);
        TRACE(9);
        if (l + 1 < a.L) {
            float xv[D / NT];
#pragma unroll
            for (int k = 0; k < D / NT; k++) xv[k] = ld_devf(&ws->x[xcd][tid + NT * k]);
#pragma unroll
            for (int k = 0; k < D / NT; k++) sh.x[tid + NT * k] = xv[k];
        }
    }
}

}  // namespace

extern "C" {

size_t mhip_decode_ws_bytes(void) { return (sizeof(DecodeWs) + 255) / 256 * 256; }

int mhip_decode_stack(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                      const void *d_table, const float *d_router, const float *d_router_t,
                      const float *d_norm, const float *d_bias, float *d_x, int L, void *d_ws,
                      int *d_idx, float *d_w, int flags) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    if (s->dim != D || s->n_experts != E || s->expert_hidden != EH || s->n_active > KMAX)
        return mhip::fail(c, "decode stack: shape %d/%d/%d/%d is not the supported "
                             "2048/128/<=8/768", s->dim, s->n_experts, s->n_active,
                          s->expert_hidden);
    if (L <= 0) return L == 0 ? 0 : mhip::fail(c, "decode stack: L=%d", L);
    hipDeviceProp_t prop;
    if (mhip::check(c, hipGetDeviceProperties(&prop, c->device), "hipGetDeviceProperties"))
        return -1;
    int occ = 0;
    if (mhip::check(c, hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_decode_stack, NT, 0),
                    "occupancy"))
        return -1;
    if (prop.multiProcessorCount != NWG || occ < 1)
        return mhip::fail(c, "decode stack needs %d CUs with one %d-thread workgroup each "
                             "(device has %d CUs, occupancy %d)", NWG, NT,
                          prop.multiProcessorCount, occ);
    DecodeWs *ws = (DecodeWs *)d_ws;
    // Counters, flags and status start at zero (fill kernel, no memset).
    if (mhip_zero(c, ws, offsetof(DecodeWs, x))) return -1;
    DecodeArgs a;
    a.table = (const uint8_t *)d_table;
    a.lay = *lay;
    a.router = d_router;
    a.router_t = d_router_t;
    a.norm = d_norm;
    a.bias = d_bias;
    a.x = d_x;
    a.ws = ws;
    a.idx_out = d_idx;
    a.w_out = d_w;
    a.L = L;
    a.K = s->n_active;
    a.norm_topk = s->norm_topk;
    a.flags = flags;
    a.eps = s->norm_eps;
    void *args[] = {&a};
    int slot = mhip::stage_begin(c, MHIP_STAGE_DECODE);
    hipError_t e = hipLaunchCooperativeKernel((const void *)k_decode_stack, dim3(NWG), dim3(NT),
                                              args, 0, c->stream);
    mhip::stage_end(c, slot);
    return mhip::check(c, e, "decode stack launch");
}

int mhip_decode_status(mhip_ctx *c, const void *d_ws, int status[4]) {
    const DecodeWs *ws = (const DecodeWs *)d_ws;
    return mhip_d2h(c, status, ws->status, 4 * sizeof(int));
}

int mhip_decode_trace(mhip_ctx *c, const void *d_ws, unsigned long long *out) {
    const DecodeWs *ws = (const DecodeWs *)d_ws;
    return mhip_d2h(c, out, ws->trace, sizeof(ws->trace));
}

}  // extern "C"
