// Persistent single-launch decode of a stack of Qwen3-MoE FFN layers at batch
// 1 (one token through layers 0..L-1, src/model/forward.c:210-213 without the
// attention call), for the Qwen3-30B-A3B shape (dim 2048, 128 experts, top-K
// with K <= 8, expert_hidden 768).
//
// Layout on the chip. The grid is 256 workgroups of 512 threads, one per CU,
// 32 on each XCD; a workgroup reads its XCD from HW_REG_XCC_ID and takes a
// rank among that XCD's workgroups from a per-XCD ticket at start (an XCD
// that receives more than 32 aborts the launch). XCD k owns routed expert
// slot k: its 32 workgroups stream that expert's
// gate/up/down rows (5.3 MB) while the other XCDs stream theirs, so each
// expert's intermediate h stays inside one XCD. Every XCD recomputes the
// (tiny) router and top-K itself, so the only cross-XCD traffic per layer is
// the K expert outputs (K x 8 KB) gathered by the combine.
//
// Inside a workgroup the waves have two roles. Waves 0-3 stream the gate/up
// rows, finish their h values without a workgroup barrier, and stream the
// workgroup's down rows behind them: each wave requests a down row pair in
// the registers of a gate/up row it has just used, so the down rows follow
// the gate/up rows in the CU's queue (which takes vector memory instructions
// in order, and holds a wave that waits to issue one) and need no registers
// of their own. Waves 4-7 (the router waves) hold the router rows: they form
// the parallel logits, Q8(xn) and, under the exact router, the reference's
// sequential logit chains, which run beside the stream because these waves
// issue no load during it (the next layer's router rows are requested once
// h is in).
//
// Per layer, on every XCD:
//   A  x (8 KB) -> certified rmsnorm -> xn, Q8(xn) in LDS; 4 router logits per
//      workgroup (one per down wave) by a parallel sum with a rigorous bound
//      on the distance to the reference's sequential fp32 chain  [XCD sync]
//   B  all 128 logits -> ranks (LDS, 512 threads) -> top-K + certification
//      on a router wave, which hands its verdict to the others in LDS, while
//      the gate/up waves request their first rows of the rank-k expert
//      (if the ordering is not certified, the exact sequential logits are
//      computed, routing follows the reference bit for bit, and the rows are
//      requested again)
//   C  gate/up rows of expert idx[k] + SwiGLU -> h (768 floats) [XCD sync]
//      (the down rows are loaded behind them; the router waves run the
//      exact logit chains meanwhile)
//   D  Q8(h) -> down rows -> the expert's output rows, published device-wide
//      (the next layer's router rows are loaded meanwhile)
//   E  softmax of the exact logits -> gate weights; combine
//      x_r += w_j * out_j,r in top-K order for 64 rows [XCD sync]
//
// Exchanged data carries its own readiness: every value goes out as one
// 64-bit device-scope store of (fp32 value, tag), the tag naming the launch
// and the layer, and its readers poll those words until the tag matches. No
// separate flag, barrier or store acknowledgement sits between a producer
// and its readers, and no agent-scope cache maintenance is issued. (The rare
// exact-router fallback uses an L2 atomic counter per XCD.)
//
// Results: top-K indices bit-equal to the reference (certified, with an exact
// fallback); expert products, SwiGLU, Q8(h), down and combine follow the
// reference's rounding order; the gate weights come from the reference's
// sequential logit chains (the default: every layer bit-equal), or with
// MHIP_DECODE_CERTIFIED from the parallel logits (relative error ~1e-6
// against the reference's) unless the exact fallback ran for that layer.
//
// The same body (decode_body.inc) compiles twice: k_decode_stack, the MoE
// alone, and k_model_stack, which runs each layer's attention (attn_stage:
// rmsnorm, Q/K/V rows, the 32 heads with the KV cache, Wo and the residual,
// src/model/forward.c:118-165) before that layer's MoE, so a whole decode
// token is one launch (forward.c:210-213).
#include <mutex>

#include "attn_common.h"
#include "mhip_internal.h"

namespace {

namespace at = mhip_attn;

constexpr int NX = 8;            // XCDs
constexpr int WPX = 32;          // workgroups per XCD
constexpr int NWG = NX * WPX;    // 256
constexpr int NT = 512;          // threads per workgroup
constexpr int NWAVE = NT / 64;
constexpr int D = 2048, E = 128, EH = 768, KMAX = 8;
constexpr int NB = D / 32, NBH = EH / 32;
constexpr int HROWS = EH / WPX;                 // 24 h rows per workgroup
constexpr int DROWS = D / WPX;                  // 64 down rows per workgroup
constexpr int LPW = E / WPX;                    // 4 logits per workgroup
constexpr int NGU = 4;                          // waves 0..3: gate/up
constexpr int NDN = NWAVE - NGU;                // waves 4..7: router rows
constexpr int GU_H = HROWS / NGU;               // 6 h rows per gate/up wave
constexpr int GU_R = 2 * GU_H;                  // its 12 weight rows
constexpr int DPK = DROWS * NBH / (NGU * 64);   // 6 down (row, block) pairs per gate/up thread
// gate/up rows of a gate/up wave requested while the ranking is certified
// (all 12 held across the certification and its fallback spill registers)
constexpr int GU_SPEC = 8;
constexpr long SPIN = 1L << 18;

typedef int v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld_stream(const void *p) {
    const v4i v = __builtin_nontemporal_load((const v4i *)p);
    return make_int4(v.x, v.y, v.z, v.w);
}

static_assert(NB == 64, "one 32-block per lane");
static_assert(LPW == NDN, "one router row per down wave");
static_assert(GU_H * NGU == HROWS && DPK * NGU * 64 == DROWS * NBH && DPK <= GU_R, "tiling");
static_assert(NT == 4 * E, "ranks: four threads per expert");

// Tagged words: (tag << 32) | fp32 bits.
typedef unsigned long long tw;

struct alignas(64) Ticket {
    unsigned n;                   // workgroups of this XCD that arrived (one cache line each)
};

struct DecodeWs {
    unsigned gstart[64];          // start barrier: NWG arrivals per launch, never reset
    Ticket xtick[2][NX];          // per-XCD rank tickets, by launch parity
    tw status[32];                // (epoch << 32) | value: [0] abort bits,
                                  // [1] rms fallbacks, [2] router fallbacks
    // Every per-XCD array starts on a 256-byte boundary, so no cache line
    // holds data of two XCDs.
    alignas(256) tw x[NX][D];     // residual stream after each layer, per XCD
    alignas(256) tw lgs[NX][E];   // parallel logit sum S, rounded to fp32
    alignas(256) tw lgb[NX][E];   // its bound, widened for that rounding
    alignas(256) tw lx[NX][E];    // exact logits (fallback)
    alignas(256) tw h[NX][EH];    // SwiGLU output of the XCD's expert
    alignas(256) tw out[2][KMAX][D];  // expert outputs, double-buffered by layer parity
    // stage timestamps of every workgroup for layers MHIP_TRACE_L0 .. +MHIP_TRACE_NL (diagnostic)
    unsigned long long trace[MHIP_TRACE_NL][NWG][MHIP_TRACE_SLOTS];
};

static_assert(offsetof(DecodeWs, lgb) == offsetof(DecodeWs, lgs) + NX * E * sizeof(tw),
              "lgb follows lgs");

// Exchange words of the attention of the model stack (every layer's
// attention before its MoE, k_model_stack), tagged like the MoE's.
struct AttnXWs {
    alignas(256) tw qkv[at::NROWS];    // q, k, v of the token
    alignas(256) tw attq[at::QD / 4];  // the heads' Q8 codes, four per word
    alignas(256) tw atts[at::NBO];     // their block scales
    alignas(256) tw xa[D];             // x after the attention
    alignas(256) tw xl[NX][D];         // the same, republished in each XCD's L2
};

struct DecodeArgs {
    const uint8_t *table;         // layer 0, experts expert_bytes apart, layers E*expert_bytes
    mhip_layout lay;
    const float *router;          // [L][E][D], decode layout
    const float *router_t;        // [L][D][E]
    const float *norm;            // [L][D]
    const float *bias;            // [E] or null
    float *x;                     // [D] in/out
    DecodeWs *ws;
    int *idx_out;                 // [L][K] or null
    float *w_out;                 // [L][K] or null
    int L, K, norm_topk, flags;
    float eps;
    unsigned epoch;               // tag of this launch (bits 8..31 of every tag)
    // k_model_stack only: the attention of each layer before its MoE
    const mhip_attn_layer *al;    // [L], device
    AttnXWs *xw;
    const double *rope;           // [max_seq][HD / 2] (cos, sin)
    int pos;
    float scale;                  // 1 / sqrt(head_dim)
};

// The allocation-free entry point's workspace (the array `scratch` below):
// its size, and per device the address of that device's copy and the epoch
// of the last launch that used it (shared by every context of the device;
// calls that overlap on one GPU race, like two launches on one workspace).
constexpr size_t STATIC_WS_BYTES = (sizeof(DecodeWs) + 255) / 256 * 256;
constexpr int MAX_DEVICES = 64;
struct StaticWs {
    std::mutex mu;        // held while a call sets up, tags and queues its launch
    void *ptr;            // device address of this device's copy (0 until set up)
    unsigned epoch;       // launches since it was last cleared
    hipEvent_t done;      // recorded after each launch queued outside stream capture
    hipStream_t last;     // the stream of that launch (null before the first)
};
StaticWs g_static_ws[MAX_DEVICES];

__device__ __forceinline__ unsigned xcc_id() {
    return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));
}
__device__ __forceinline__ unsigned ld_dev(const unsigned *p) {
    return __hip_atomic_load((unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Status words carry the epoch of the launch that wrote them in their high
// half (a word of an earlier launch reads as 0), so they need no clearing
// between launches.
enum { ST_ABORT = 0, ST_RMS = 1, ST_ROUTER = 2 };
__device__ __forceinline__ unsigned status_get(DecodeWs *ws, int i, unsigned epoch) {
    const tw v = __hip_atomic_load(&ws->status[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (unsigned)(v >> 32) == epoch ? (unsigned)v : 0u;
}
// status[i] |= bits, or += 1 when `add` (device-scope compare-and-swap).
__device__ void status_update(DecodeWs *ws, int i, unsigned epoch, bool add, unsigned bits) {
    tw old = __hip_atomic_load(&ws->status[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
        const unsigned cur = (unsigned)(old >> 32) == epoch ? (unsigned)old : 0u;
        const tw w = ((tw)epoch << 32) | (add ? cur + 1 : (cur | bits));
        if (w == old) return;
        const tw prev = atomicCAS(&ws->status[i], old, w);
        if (prev == old) return;
        old = prev;
    }
}
// Abort bits: 1 = workgroup not on the expected XCD, 2 = a wait timed out,
// 4 = forced by the caller (MHIP_DECODE_FORCE_ABORT; every workgroup leaves
// after the start barrier).
__device__ __forceinline__ bool aborted(DecodeWs *ws, unsigned epoch) {
    return status_get(ws, ST_ABORT, epoch) != 0;
}

// Two kinds of exchange. Data read only inside the writer's XCD (x, logits,
// h) meets in that XCD's L2: workgroup-scope stores (the L1 writes through)
// and non-temporal loads, which the L1 does not keep, so every poll reads the
// L2 (a scope-0/1 load may hit a stale L1 line and never see the store).
// Measured hand-off between two CUs of one XCD: ~290 ns one way, against
// ~460 ns with device-scope accesses. Expert outputs, read by every XCD, use
// device-scope (sc1) stores and loads.
template <bool LOCAL>
__device__ __forceinline__ void put_tagged(tw *p, float v, unsigned tag) {
    const tw w = ((tw)tag << 32) | __float_as_uint(v);
    if (LOCAL)
        __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
        __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// N words p[0], p[stride], ... read from the L2 (one wait for all of them).
template <int N> struct L2Load;
template <> struct L2Load<1> {
    __device__ static void run(tw *v, const tw *p, int) {
        asm volatile("global_load_dwordx2 %0, %1, off nt\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(v[0]) : "v"(p) : "memory");
    }
};
template <> struct L2Load<2> {
    __device__ static void run(tw *v, const tw *p, int s) {
        asm volatile("global_load_dwordx2 %0, %2, off nt\n\t"
                     "global_load_dwordx2 %1, %3, off nt\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1]) : "v"(p), "v"(p + s) : "memory");
    }
};
template <> struct L2Load<3> {
    __device__ static void run(tw *v, const tw *p, int s) {
        asm volatile("global_load_dwordx2 %0, %3, off nt\n\t"
                     "global_load_dwordx2 %1, %4, off nt\n\t"
                     "global_load_dwordx2 %2, %5, off nt\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2])
                     : "v"(p), "v"(p + s), "v"(p + 2 * s) : "memory");
    }
};
template <> struct L2Load<4> {
    __device__ static void run(tw *v, const tw *p, int s) {
        asm volatile("global_load_dwordx2 %0, %4, off nt\n\t"
                     "global_load_dwordx2 %1, %5, off nt\n\t"
                     "global_load_dwordx2 %2, %6, off nt\n\t"
                     "global_load_dwordx2 %3, %7, off nt\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                     : "v"(p), "v"(p + s), "v"(p + 2 * s), "v"(p + 3 * s) : "memory");
    }
};
// Three words p[0], p[s], p[2s] and two words q[0], q[t], read from the L2
// with one wait.
struct L2Load32 {
    __device__ static void run(tw *v, const tw *p, int s, const tw *q, int t) {
        asm volatile("global_load_dwordx2 %0, %5, off nt\n\t"
                     "global_load_dwordx2 %1, %6, off nt\n\t"
                     "global_load_dwordx2 %2, %7, off nt\n\t"
                     "global_load_dwordx2 %3, %8, off nt\n\t"
                     "global_load_dwordx2 %4, %9, off nt\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4])
                     : "v"(p), "v"(p + s), "v"(p + 2 * s), "v"(q), "v"(q + t) : "memory");
    }
};
template <int N, bool LOCAL>
__device__ __forceinline__ void load_words(tw *v, const tw *p, int stride) {
    if (LOCAL) {
        L2Load<N>::run(v, p, stride);
    } else {
#pragma unroll
        for (int k = 0; k < N; k++)
            v[k] = __hip_atomic_load((tw *)(p + k * stride), __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    }
}
// The values of the N words p[0], p[stride], ... once each carries `tag`
// (polled together). After SPIN rounds, or once the launch has aborted, sets
// abort bit 2 and returns whatever is there.
template <int N, bool LOCAL>
__device__ __forceinline__ void get_tagged(DecodeWs *ws, const tw *p, int stride, unsigned tag,
                                           float *out) {
    tw v[N];
    load_words<N, LOCAL>(v, p, stride);
    long s = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < N; k++) ready = ready && (unsigned)(v[k] >> 32) == tag;
        if (ready) break;
        if (++s > SPIN || ((s & 255) == 0 && aborted(ws, tag >> 8))) {
            status_update(ws, ST_ABORT, tag >> 8, false, 2);
            break;
        }
        load_words<N, LOCAL>(v, p, stride);
    }
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = __uint_as_float((unsigned)v[k]);
}

// get_tagged over the XCD-local words p[0], p[s], p[2s] (out[0..2]) and
// q[0], q[t] (out[3..4]), polled together: words that are long published
// cost no wait of their own beside words still on their way.
__device__ __forceinline__ void get_tagged_3_2(DecodeWs *ws, const tw *p, int s, const tw *q,
                                               int t, unsigned tag, float *out) {
    tw v[5];
    L2Load32::run(v, p, s, q, t);
    long n = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < 5; k++) ready = ready && (unsigned)(v[k] >> 32) == tag;
        if (ready) break;
        if (++n > SPIN || ((n & 255) == 0 && aborted(ws, tag >> 8))) {
            status_update(ws, ST_ABORT, tag >> 8, false, 2);
            break;
        }
        L2Load32::run(v, p, s, q, t);
    }
#pragma unroll
    for (int k = 0; k < 5; k++) out[k] = __uint_as_float((unsigned)v[k]);
}

__device__ void wait_flag(DecodeWs *ws, const unsigned *flag, unsigned value, unsigned epoch) {
    long s = 0;
    while (ld_dev(flag) < value) {
        if (++s > SPIN || ((s & 255) == 0 && aborted(ws, epoch))) {
            status_update(ws, ST_ABORT, epoch, false, 2);
            break;
        }
    }
}

// Orders LDS traffic between the lanes of one wavefront (LDS operations of a
// wavefront execute in program order; this keeps the compiler from moving
// them across the point).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

// v from the lane DPP control CTRL names (every lane has a source).
template <int CTRL>
__device__ __forceinline__ float dpp_keep_f(float v) {
    const int b = __float_as_int(v);
    return __int_as_float(__builtin_amdgcn_update_dpp(b, b, CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum_f(float v) {
    // through double: exact for the wave-wide sum of 64 floats' partials
    return (float)lane63_d(wave_scan_d((double)v));
}

// Exact int32 dot of 16 int8 codes (four v_dot4).
__device__ __forceinline__ int dot16_i8(const int4 a, const int4 b) {
    int acc = 0;
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

__device__ __forceinline__ float4 i4_as_f4(const int4 v) {
    return make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z),
                       __int_as_float(v.w));
}

// LDS. `scr` is reused by stages that never overlap: the exact-router
// products (B, fallback), the gate/up terms (C) and the down terms (D).
// A lane reading its own 32-block of xn with 16-byte reads: blocks 36
// floats apart put eight consecutive lanes on distinct banks (a 128-byte
// stride would put every lane on the same four banks).
constexpr int XN_LD = 36;
constexpr int GU_LD = NB + 4;     // 16-byte aligned rows
constexpr int DN_LD = NBH + 4;
constexpr int SCR = 8192;         // floats
static_assert(NGU * GU_R * GU_LD <= SCR && DROWS * DN_LD <= SCR && LPW * D <= SCR, "scr");

struct Lds {
    alignas(16) float x[D];
    alignas(16) float xn[NB * XN_LD];  // 32-blocks XN_LD floats apart
    alignas(16) float xt[NB * XN_LD];  // fl(x * w), w the norm weight, laid out as xn
    alignas(16) int8_t xq[D];
    alignas(16) float scr[SCR];
    // expert outputs gathered for the combine; apart from scr, because rows
    // of other XCDs can arrive while wave 0 still sums this XCD's down terms
    alignas(16) float og[KMAX * DROWS];
    alignas(16) int8_t hq[EH];
    float xs[NB];
    float hsc[NBH];
    float gu[NGU][GU_R];
    alignas(16) uint64_t key[E];  // ranking key: S + bias made monotone, expert index in the low bits
    double c[E];                  // S + bias
    double bpart[E / 64];         // largest bound among each 64 experts
    float mxpart[E / 64];         // exact router: largest logit among each 64 experts
    float lf[E];                  // fp32 logits (+ bias)
    alignas(16) float p[E];       // probabilities (fallback)
    float bias[E];
    uint64_t etab[32];            // expf table
    int rk[4][E];                 // partial ranks
    double part[NGU];             // the gate/up waves' partial sums of squares
    unsigned ptag[NGU];           // the layer tag once part[w] is set
    unsigned invtag;              // the layer tag once inv is set
    unsigned ctag;                // the layer tag once the ranking's verdict is set
    int order[E];                 // expert of each rank (ranks 0..K used)
    float inv;
    float sum;
    int idx[KMAX];
    float w[KMAX];
    int fallback;
    int shadow_on;                // exact router, certified ranking: the chains run in stage C
    int nanflag;
    int role[2];                  // this workgroup's XCD and rank within it
};

// Sequential fp32 sum of N (a compile-time multiple of 4) LDS floats at p,
// in order: every value is read before the first addition, so the chain
// waits for the LDS once.
template <int N>
__device__ __forceinline__ float lds_seq_sum_n(const float *p, float s) {
    static_assert(N % 4 == 0, "whole float4s");
    const float4 *v = (const float4 *)p;
    float4 q[N / 4];
#pragma unroll
    for (int k = 0; k < N / 4; k++) q[k] = v[k];
#pragma unroll
    for (int k = 0; k < N / 4; k++) {
        s = s + q[k].x;
        s = s + q[k].y;
        s = s + q[k].z;
        s = s + q[k].w;
    }
    return s;
}

// Sequential fp32 sum of N LDS floats at p, in order, read B at a time: the
// reads of the next B values are issued before the additions of these, so
// the chain waits for the LDS only at its start.
template <int N, int B>
__device__ __forceinline__ float lds_seq_sum_pipe(const float *p, float s) {
    static_assert(B % 4 == 0 && N % B == 0, "whole float4s per batch");
    const float4 *v = (const float4 *)p;
    float4 q[2][B / 4];
#pragma unroll
    for (int k = 0; k < B / 4; k++) q[0][k] = v[k];
#pragma unroll
    for (int b = 0; b < N / B; b++) {
        if (b + 1 < N / B) {
#pragma unroll
            for (int k = 0; k < B / 4; k++) q[(b + 1) & 1][k] = v[(b + 1) * (B / 4) + k];
        }
#pragma unroll
        for (int k = 0; k < B / 4; k++) {
            s = s + q[b & 1][k].x;
            s = s + q[b & 1][k].y;
            s = s + q[b & 1][k].z;
            s = s + q[b & 1][k].w;
        }
    }
    return s;
}

// Sequential fp32 sum, in order, of the wavefront's 64 x 32 values, lane L
// holding values 32 L .. 32 L + 31 in v[0..31]: every lane adds its own 32
// values to its running sum, then the sums move one lane up (DPP wave_shr:1),
// so lane L starts from lane L - 1's total. Only lane L's additions count in
// round L; the sum of all 2048 values ends in lane 63. 2048 dependent
// additions with their operands in registers.
__device__ __forceinline__ float wave_seq_sum_2048(const float (&v)[32]) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) s = s + v[k];
    for (int L = 1; L < 64; L++) {
        s = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x138, 0xf, 0xf, false));
#pragma unroll
        for (int k = 0; k < 32; k++) s = s + v[k];
    }
    return s;
}

// Diagnostic: one thread of every workgroup (thread 0 unless named) records
// the 100 MHz real-time counter at the stage boundaries of a window of layers.
#define TRACE_BY(slot, who)                                                                \
    do {                                                                                   \
        if ((a.flags & MHIP_DECODE_TRACE) && tid == (who) && l >= MHIP_TRACE_L0 &&         \
            l < MHIP_TRACE_L0 + MHIP_TRACE_NL)                                             \
            ws->trace[l - MHIP_TRACE_L0][xcd + NX * rank][slot] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define TRACE(slot) TRACE_BY(slot, 0)
#define TRACE_CLK(slot)                                                                    \
    do {                                                                                   \
        if ((a.flags & MHIP_DECODE_TRACE) && tid == 0 && l >= MHIP_TRACE_L0 &&             \
            l < MHIP_TRACE_L0 + MHIP_TRACE_NL)                                             \
            ws->trace[l - MHIP_TRACE_L0][xcd + NX * rank][slot] = __builtin_amdgcn_s_memtime();  \
    } while (0)

// ---- the attention of a layer inside the model stack ------------------------------
//
// k_model_stack runs, for every layer, the attention of mhip_attention_layer
// (attn_layer.hip: the same arithmetic, forward.c:118-165) before the MoE,
// on x in LDS: every workgroup forms rmsnorm(x, attn_norm) and Q8 itself
// (four elements per thread), every wavefront gw = 8 (32 xcd + rank) + wave its q/k/v
// rows gw + 2048 j (the block-order sum passed lane to lane) and row gw of
// Wo; workgroups of rank < 4 run query head h = 8 rank + xcd (a key/value
// group's heads on one rank, its first head on XCD 0 appending the cache
// row). q/k/v, the heads' codes and scales and the new x meet through
// device-scope tagged words (AttnXWs), tagged like the MoE's words of the
// layer; every workgroup then holds the new x in LDS for the MoE.
constexpr int AT_NPRE = 32;                          // cache positions a head stages in LDS
constexpr int AT_RPW = (at::NROWS + NWG * NWAVE - 1) / (NWG * NWAVE);  // 3 q/k/v rows per wave
static_assert(at::D == D && at::NT == NT && D == NWG * NWAVE, "one Wo row per wavefront");
static_assert(at::NH == 4 * NX, "four heads per XCD");

// A pointer read from LDS, made wave-uniform (scalar registers).
template <class T> __device__ __forceinline__ T *uniform_ptr(T *p) {
    const uint64_t v = (uint64_t)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (T *)(((uint64_t)hi << 32) | lo);
}

// `before_x` runs once the Wo rows are published, before the new x is
// waited for: the caller's requests for the MoE that follows go there.
template <class F>
__device__ __forceinline__ void attn_stage(const DecodeArgs &a, Lds &sh, DecodeWs *ws, int tid,
                                           int lane, int wave, int xcd, int rank, int l,
                                           unsigned tag, F &&before_x) {
    // Values derived from the workgroup's place are recomputed in every
    // layer rather than held across the loop (the place is made opaque): the
    // registers they would hold are what the MoE stages need.
    asm volatile("" : "+s"(xcd), "+s"(rank), "+s"(wave));
    __shared__ at::HeadLds<AT_NPRE> hs;
    __shared__ alignas(16) int8_t attq[at::QD];
    __shared__ float atts[at::NBO];
    __shared__ mhip_attn_layer al_next;             // the next layer's tensors, read a layer ahead
    extern __shared__ __align__(16) float asc[];  // a head's scores, [pos + 1]
    constexpr int ALW = sizeof(mhip_attn_layer) / 4;
    static_assert(ALW <= NT && sizeof(mhip_attn_layer) % 4 == 0, "table row in words");
    // this layer's tensors, held in LDS: at layer 0 from the table, later
    // as read during the previous layer (the table row of layer l + 1 is
    // requested now and stored at the end of this stage)
    if (l == 0) {
        if (tid < ALW) ((unsigned *)&al_next)[tid] = ((const unsigned *)a.al)[tid];
        __syncthreads();
    }
    const mhip_attn_layer L = al_next;
    unsigned alw = 0;
    if (tid < ALW && l + 1 < a.L) alw = ((const unsigned *)(a.al + l + 1))[tid];
    const at::gptr<const float> attn_norm = at::glob(uniform_ptr(L.attn_norm));
    const at::gptr<const uint8_t> wqg = at::glob((const uint8_t *)uniform_ptr(L.wq));
    const at::gptr<const uint8_t> wkg = at::glob((const uint8_t *)uniform_ptr(L.wk));
    const at::gptr<const uint8_t> wvg = at::glob((const uint8_t *)uniform_ptr(L.wv));
    const at::gptr<const uint8_t> wog = at::glob((const uint8_t *)uniform_ptr(L.wo));
    const at::gptr<float> kcg = at::glob(uniform_ptr(L.kc)), vcg = at::glob(uniform_ptr(L.vc));
    AttnXWs *xw = a.xw;
    const int gw = (xcd * WPX + rank) * NWAVE + wave;
    const bool head = rank < at::NH / NX;
    const int h = rank * NX + xcd;
    // requests in the order they are needed: the norm weights of this
    // thread's elements tid + NT k, the weight rows, then a head's first
    // cache rows (copied into LDS)
    float anw[D / NT];
#pragma unroll
    for (int k = 0; k < D / NT; k++) anw[k] = attn_norm[tid + NT * k];
    at::Blk wr[AT_RPW];
#pragma unroll
    for (int j = 0; j < AT_RPW; j++) {
        const int r = min(gw + NWG * NWAVE * j, at::NROWS - 1);  // past the end: unused
        const at::gptr<const uint8_t> w = r < at::QD ? wqg + (size_t)r * at::NB * 36
                                          : r < at::QD + at::KVD
                                              ? wkg + (size_t)(r - at::QD) * at::NB * 36
                                              : wvg + (size_t)(r - at::QD - at::KVD) * at::NB * 36;
        wr[j] = at::load_blk(w + (size_t)lane * 36);
    }
    // This wavefront's Wo row is requested once its q/k/v rows are in (and,
    // in a head's workgroup, once the head is done): the q/k/v rows, on the
    // critical path, then do not share HBM with the Wo rows.
    const at::gptr<const uint8_t> wo = wog + (size_t)gw * at::NBO * 36;
    at::Blk wo0, wo1;
    at::HeadPre<AT_NPRE, true> hp;
    if (head)
        at::head_prefetch(hp, hs, h, a.pos, (at::gptr<const float>)kcg, (at::gptr<const float>)vcg,
                          at::glob(uniform_ptr(L.q_norm)), at::glob(uniform_ptr(L.k_norm)),
                          at::glob(a.rope), tid);
    TRACE(34);
    // the previous layer's MoE ends with every thread storing its own part
    // of x in LDS: all of it is there before wavefront 0 reads it below
    __syncthreads();
    TRACE(35);

    // rmsnorm(x, attn_norm) and Q8 (forward.c:123, quant.c:11-27) by every
    // thread over its elements i = tid + NT k (block i / 32 is 32 lanes of
    // one wavefront): the sum of squares in any order is within
    // (n + 64) 2^-52 S of the reference's sequential double sum (terms >= 0),
    // so when S -/+ that bound give the same fp32 scale it is the reference's;
    // otherwise thread 0 runs the sequential sum.
    {
        __shared__ double ssw[NWAVE];
        __shared__ float inv_seq;
        float xv[D / NT];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < D / NT; k++) {
            xv[k] = sh.x[tid + NT * k];
            ss = ss + (double)xv[k] * (double)xv[k];
        }
        ss = at::wave_sum63(ss);
        if (lane == 63) ssw[wave] = ss;
        __syncthreads();
        TRACE(36);
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) tot = tot + ssw[w];
        const double m = tot * ((double)(D + 64) * 0x1p-52);
        const float lo = (float)(1.0 / sqrt((tot + m) / D + (double)a.eps));
        const float hi = (float)(1.0 / sqrt((tot - m) / D + (double)a.eps));
        float inv = lo;
        if ((a.flags & MHIP_FORCE_SEQ_RMS) || lo != hi) {  // the same in every thread
            if (tid == 0) {
                double sq = 0.0;
                for (int i = 0; i < D; i++) sq = sq + (double)sh.x[i] * (double)sh.x[i];
                inv_seq = (float)(1.0 / sqrt(sq / D + (double)a.eps));
            }
            __syncthreads();
            inv = inv_seq;
        }
        TRACE(37);
#pragma unroll
        for (int k = 0; k < D / NT; k++) {
            const float v = (xv[k] * inv) * anw[k];
            // (a NaN counts as 0, as in the sequential max)
            const float am = at::max32(fmaxf(0.0f, fabsf(v)), lane);
            const float dsc = am / 127.0f;
            const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
            const int i = tid + NT * k;
            sh.xq[i] = (int8_t)roundf(v * qi);
            if ((lane & 31) == 0) sh.xs[i / 32] = dsc;
        }
    }
    __syncthreads();
    TRACE(25);

    // q/k/v rows (forward.c:124-126): lane b the term of block b, the
    // block-order sum passed lane to lane
    {
        const int4 xa = *(const int4 *)&sh.xq[32 * lane], xb = *(const int4 *)&sh.xq[32 * lane + 16];
        const float dx = sh.xs[lane];
        float t[AT_RPW], sv[AT_RPW];
#pragma unroll
        for (int j = 0; j < AT_RPW; j++) {
            t[j] = mhip_dev::block_term(mhip_dev::dot32_i8(wr[j].c0, wr[j].c1, xa, xb), wr[j].d, dx);
            sv[j] = 0.0f + t[j];
        }
        for (int k = 1; k < at::NB; k++) {
#pragma unroll
            for (int j = 0; j < AT_RPW; j++) sv[j] = at::shr1(sv[j]) + t[j];
        }
        if (lane == 63) {
#pragma unroll
            for (int j = 0; j < AT_RPW; j++) {
                const int r = gw + NWG * NWAVE * j;
                if (r < at::NROWS) put_tagged<false>(&xw->qkv[r], sv[j], tag);
            }
        }
    }
    TRACE_BY(26, 63);
    if (!head) {
        wo0 = at::load_blk(wo + (size_t)lane * 36);
        wo1 = at::load_blk(wo + (size_t)(lane + 64) * 36);
    }

    // query head h (forward.c:127-163)
    if (head) {
        const int g = h / at::GROUP;
        float v;
        if (tid < at::HD) {
            get_tagged<1, false>(ws, &xw->qkv[h * at::HD + tid], 0, tag, &v);
            hs.tq[tid] = v;
        } else if (tid < 2 * at::HD) {
            get_tagged<1, false>(ws, &xw->qkv[at::QD + g * at::HD + tid - at::HD], 0, tag, &v);
            hs.tk[tid - at::HD] = v;
        } else if (tid < 3 * at::HD) {
            get_tagged<1, false>(ws, &xw->qkv[at::QD + at::KVD + g * at::HD + tid - 2 * at::HD], 0,
                                 tag, &v);
            hs.tv[tid - 2 * at::HD] = v;
        }
        TRACE(27);
        at::head_run(hs, asc, hp, h, a.pos, kcg, vcg, a.eps, a.scale,
                     (a.flags & MHIP_FORCE_SEQ_RMS) != 0, sh.etab,
                     [=](int i) { TRACE(38 + i); });
        TRACE(28);
        if (tid < at::HD / 32) put_tagged<false>(&xw->atts[h * (at::HD / 32) + tid], hs.dsc[tid], tag);
        if (tid < at::HD / 4)
            put_tagged<false>(&xw->attq[h * (at::HD / 4) + tid],
                              __uint_as_float(((const unsigned *)hs.hq)[tid]), tag);
        wo0 = at::load_blk(wo + (size_t)lane * 36);
        wo1 = at::load_blk(wo + (size_t)(lane + 64) * 36);
    }

    // row gw of Wo over the heads' codes, plus the residual (forward.c:164-165)
    {
        float q2[2];
        get_tagged<2, false>(ws, &xw->attq[tid], NT, tag, q2);
        ((unsigned *)attq)[tid] = __float_as_uint(q2[0]);
        ((unsigned *)attq)[tid + NT] = __float_as_uint(q2[1]);
        if (tid < at::NBO) get_tagged<1, false>(ws, &xw->atts[tid], 0, tag, &atts[tid]);
        static_assert(at::QD / 4 == 2 * NT, "two code words per thread");
        __syncthreads();
        TRACE(29);
        const int4 *q0 = (const int4 *)&attq[32 * lane], *q1 = (const int4 *)&attq[32 * (lane + 64)];
        const float t0 = mhip_dev::block_term(mhip_dev::dot32_i8(wo0.c0, wo0.c1, q0[0], q0[1]), wo0.d,
                                              atts[lane]);
        const float t1 = mhip_dev::block_term(mhip_dev::dot32_i8(wo1.c0, wo1.c1, q1[0], q1[1]), wo1.d,
                                              atts[lane + 64]);
        // blocks 0..63 (t0 of lanes 0..63), then 64..127 (t1), in order
        float sv = 0.0f + t0;
        for (int k = 1; k < 64; k++) sv = at::ror1(sv) + t0;
        for (int k = 0; k < 64; k++) sv = at::ror1(sv) + t1;
        TRACE_BY(32, 63);
        if (lane == 63) put_tagged<false>(&xw->xa[gw], sh.x[gw] + sv, tag);
    }
    before_x();

    // the new x in every workgroup: workgroup `rank` of each XCD fetches
    // words 64 rank .. + 63 across the device and republishes them in its
    // XCD's L2, where every workgroup of the XCD reads all D of them (one
    // device-wide read of each word per XCD instead of one per workgroup)
    static_assert(WPX * 64 == D, "64 words per workgroup");
    if (wave == 0) {
        float v;
        get_tagged<1, false>(ws, &xw->xa[64 * rank + lane], 0, tag, &v);
        put_tagged<true>(&xw->xl[xcd][64 * rank + lane], v, tag);
    }
    {
        float xv[D / NT];
        get_tagged<D / NT, true>(ws, &xw->xl[xcd][tid], NT, tag, xv);
        TRACE(33);
        __syncthreads();  // every read of the old x is done
#pragma unroll
        for (int k = 0; k < D / NT; k++) sh.x[tid + NT * k] = xv[k];
        if (tid < ALW) ((unsigned *)&al_next)[tid] = alw;
        __syncthreads();
    }
    // every load of this stage has long arrived (the heads' values were
    // used, the other threads' loads are older than the exchanges above); a
    // wait the compiler sees keeps it from assuming any of them is still in
    // flight when the next layer reuses their registers
    __builtin_amdgcn_s_waitcnt(at::WAIT_VM0);
    TRACE(31);
}

// The kernels: one body (decode_body.inc) compiled twice.
__global__ __launch_bounds__(NT) void k_decode_stack(DecodeArgs a) {
#define DECODE_ATTN 0
#include "decode_body.inc"
#undef DECODE_ATTN
}
__global__ __launch_bounds__(NT) void k_model_stack(DecodeArgs a) {
#define DECODE_ATTN 1
#include "decode_body.inc"
#undef DECODE_ATTN
}

// Once per context (the device properties query is slow): 1 when every CU
// holds one workgroup of the kernel, 0 when not (c->decode_cus and
// c->decode_occ say why), -1 on a failed query.
int decode_device_fits(mhip_ctx *c) {
    if (!c->decode_checked) {
        hipDeviceProp_t prop;
        if (mhip::check(c, hipGetDeviceProperties(&prop, c->device), "hipGetDeviceProperties"))
            return -1;
        int occ = 0;
        if (mhip::check(c,
                        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_decode_stack, NT, 0),
                        "occupancy"))
            return -1;
        c->decode_cus = prop.multiProcessorCount;
        c->decode_occ = occ;
        c->decode_checked = prop.multiProcessorCount == NWG && occ >= 1 ? 1 : 2;
    }
    return c->decode_checked == 1 ? 1 : 0;
}

bool decode_shape_fits(const mhip_dims *s) {
    return s->dim == D && s->n_experts == E && s->expert_hidden == EH && s->n_active >= 1 &&
           s->n_active <= KMAX;
}

// ---- host side --------------------------------------------------------------------

// Argument checks shared by both entry points (no device call before they
// pass): 1 to launch, 0 for nothing to do (L = 0), -1 on an error. Exchange
// tags hold the layer in 8 bits, so one launch covers at most 256 layers.
int check_decode_args(mhip_ctx *c, const mhip_dims *s, int L) {
    if (mhip::check_dims(c, s)) return -1;
    if (L < 0 || L > MHIP_DECODE_MAX_LAYERS)
        return mhip::fail(c, "decode stack: L=%d outside [0, %d]", L, MHIP_DECODE_MAX_LAYERS);
    if (!decode_shape_fits(s))
        return mhip::fail(c, "decode stack: shape %d/%d/%d/%d is not the supported "
                             "2048/128/<=8/768", s->dim, s->n_experts, s->n_active,
                          s->expert_hidden);
    if (L == 0) return 0;
    if (mhip::use_device(c)) return -1;
    const int fits = decode_device_fits(c);
    if (fits < 0) return -1;
    if (!fits)
        return mhip::fail(c, "decode stack needs %d CUs with one %d-thread workgroup each "
                             "(device has %d CUs, occupancy %d)", NWG, NT, c->decode_cus,
                          c->decode_occ);
    return 1;
}

// The status words of the launch tagged `epoch`, copied to status[4]
// (status[3] = 0) for callers that read them later from device memory.
__global__ void k_decode_status_out(const DecodeWs *ws, unsigned epoch, int *status) {
    const int i = threadIdx.x;
    if (i < 3) {
        const tw v = __hip_atomic_load(&ws->status[i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        status[i] = (unsigned)(v >> 32) == epoch ? (int)(unsigned)v : 0;
    } else if (i == 3) {
        status[3] = 0;
    }
}

// One launch of the decode kernel on workspace ws, whose launches are
// counted by *epoch. Exchanged words and status words are tagged with the
// launch's epoch, so stale words of earlier launches never match, and the
// start counter grows by NWG per launch: nothing is cleared between launches.
// The workspace is cleared whole first (fill kernel, no memset) when `fresh`
// or when the epoch is about to leave its 24 bits. Queues no allocation.
// The model stack's part of a launch (k_model_stack): the attention of every
// layer before its MoE.
struct ModelPart {
    const mhip_attn_layer *al;
    AttnXWs *xw;
    const double *rope;
    int pos;
};

int launch_decode(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay, const void *d_table,
                  const float *d_router, const float *d_router_t, const float *d_norm,
                  const float *d_bias, float *d_x, int L, DecodeWs *ws, unsigned *epoch,
                  bool fresh, int *d_idx, float *d_w, int *d_status, int flags,
                  const ModelPart *mp = nullptr) {
    if (fresh || *epoch >= (1u << 24) - 1) {
        if (mhip_zero(c, ws, offsetof(DecodeWs, trace))) return -1;
        if (mp && mhip_zero(c, mp->xw, sizeof(AttnXWs))) return -1;
        *epoch = 0;
    }
    if ((flags & MHIP_DECODE_TRACE) && mhip_zero(c, ws->trace, sizeof(ws->trace))) return -1;
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
    a.epoch = ++*epoch;
    a.al = mp ? mp->al : nullptr;
    a.xw = mp ? mp->xw : nullptr;
    a.rope = mp ? mp->rope : nullptr;
    a.pos = mp ? mp->pos : 0;
    a.scale = 1.0f / sqrtf((float)at::HD);
    // An ordinary launch: one 512-thread workgroup fits each of the 256 CUs
    // (checked before), so on an otherwise idle device all of them are
    // resident at once. Should one not be, the start barrier times out and
    // the launch reports abort bit 2 instead of waiting for ever.
    int slot = mhip::stage_begin(c, MHIP_STAGE_DECODE);
    if (mp)  // a head's scores in dynamic LDS
        k_model_stack<<<NWG, NT, ((size_t)mp->pos + 1) * 4, c->stream>>>(a);
    else
        k_decode_stack<<<NWG, NT, 0, c->stream>>>(a);
    const hipError_t e = hipGetLastError();
    mhip::stage_end(c, slot);
    if (e != hipSuccess) {
        --*epoch;  // nothing arrived at the start counter
        return mhip::check(c, e, "decode stack launch");
    }
    if (d_status) {
        k_decode_status_out<<<1, 64, 0, c->stream>>>(ws, a.epoch, d_status);
        return mhip::check_launch(c, "decode status copy");
    }
    return 0;
}

// The dynamic-LDS limit of k_model_stack (a head's scores), set once per
// device.
int g_model_lds_set[MAX_DEVICES];
int model_lds_attr(mhip_ctx *c) {
    if (c->device < 0 || c->device >= MAX_DEVICES || g_model_lds_set[c->device]) return 0;
    if (mhip::check(c, hipFuncSetAttribute((const void *)k_model_stack,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           MHIP_MODEL_STACK_MAX_SEQ * 4),
                    "model stack LDS attribute"))
        return -1;
    g_model_lds_set[c->device] = 1;
    return 0;
}

}  // namespace

// Workspace of mhip_decode_stack_noalloc: a device-resident array of the
// library, one copy per GPU (each device holds its own instance at its own
// address until the process ends). Host code never uses this name as an
// address: the address of a device's copy comes from hipGetSymbolAddress,
// taken once per device at context set-up (decode_noalloc_setup).
static __device__ __align__(256) unsigned char scratch[STATIC_WS_BYTES];

namespace mhip {

int decode_noalloc_setup(mhip_ctx *c) {
    if (c->device < 0 || c->device >= MAX_DEVICES) return 0;  // the entry point then refuses
    StaticWs &st = g_static_ws[c->device];
    std::lock_guard<std::mutex> lock(st.mu);
    if (st.ptr) return 0;
    void *ptr = nullptr;
    if (check(c, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
              "hipGetSymbolAddress (decode workspace)"))
        return -1;
    if (!ptr || (uintptr_t)ptr % 256) return fail(c, "decode workspace symbol at %p", ptr);
    if (check(c, hipEventCreateWithFlags(&st.done, hipEventDisableTiming),
              "hipEventCreate (decode workspace)"))
        return -1;
    // cleared once here; afterwards the launches' epochs keep it consistent
    if (mhip_zero(c, ptr, STATIC_WS_BYTES) || mhip_sync(c)) {
        (void)hipEventDestroy(st.done);
        return -1;
    }
    st.last = nullptr;
    st.epoch = 0;
    st.ptr = ptr;
    return 0;
}

}  // namespace mhip

extern "C" {

size_t mhip_decode_ws_bytes(void) { return (sizeof(DecodeWs) + 255) / 256 * 256; }

int mhip_decode_supported(mhip_ctx *c, const mhip_dims *s) {
    if (mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    if (!decode_shape_fits(s)) return 0;
    return decode_device_fits(c);
}

int mhip_decode_stack(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                      const void *d_table, const float *d_router, const float *d_router_t,
                      const float *d_norm, const float *d_bias, float *d_x, int L, void *d_ws,
                      int *d_idx, float *d_w, int flags) {
    const int ok = check_decode_args(c, s, L);
    if (ok <= 0) return ok;
    if ((uintptr_t)d_ws % 256)
        return mhip::fail(c, "decode stack: workspace %p is not 256-byte aligned", d_ws);
    DecodeWs *ws = (DecodeWs *)d_ws;
    // A workspace this context has not used last starts from a cleared one.
    const int rc = launch_decode(c, s, lay, d_table, d_router, d_router_t, d_norm, d_bias, d_x,
                                 L, ws, &c->decode_epoch, ws != c->decode_ws, d_idx, d_w,
                                 nullptr, flags);
    if (rc == 0) c->decode_ws = ws;
    return rc;
}

int mhip_decode_stack_noalloc(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                              const void *d_table, const float *d_router,
                              const float *d_router_t, const float *d_norm, const float *d_bias,
                              float *d_x, int L, int *d_idx, float *d_w, int *d_status,
                              int flags) {
    const int ok = check_decode_args(c, s, L);
    if (ok <= 0) return ok;
    StaticWs *st = c->device < MAX_DEVICES ? &g_static_ws[c->device] : nullptr;
    if (!st) return mhip::fail(c, "no-alloc decode: device %d has no set-up workspace", c->device);
    // Calls on one device are serialized: the host side (the epoch, the
    // queueing) under the mutex, and the launches in stream order, a call
    // on another stream than the previous one waiting for that one's event.
    // Under stream capture the capturing caller orders its calls (an event
    // recorded outside the capture cannot be waited for inside it).
    std::lock_guard<std::mutex> lock(st->mu);
    if (!st->ptr)
        return mhip::fail(c, "no-alloc decode: device %d has no set-up workspace", c->device);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (mhip::check(c, hipStreamIsCapturing(c->stream, &cs), "hipStreamIsCapturing")) return -1;
    const bool captured = cs != hipStreamCaptureStatusNone;
    if (!captured && st->last && st->last != c->stream &&
        mhip::check(c, hipStreamWaitEvent(c->stream, st->done, 0), "hipStreamWaitEvent"))
        return -1;
    const int rc = launch_decode(c, s, lay, d_table, d_router, d_router_t, d_norm, d_bias, d_x,
                                 L, (DecodeWs *)st->ptr, &st->epoch, false, d_idx, d_w, d_status,
                                 flags);
    if (rc == 0 && !captured) {
        if (mhip::check(c, hipEventRecord(st->done, c->stream), "hipEventRecord")) return -1;
        st->last = c->stream;
    }
    return rc;
}

size_t mhip_model_stack_ws_bytes(void) { return mhip_decode_ws_bytes() + sizeof(AttnXWs); }

int mhip_model_stack_supported(mhip_ctx *c, const mhip_dims *s, const mhip_attn_dims *as,
                               int max_seq) {
    if (!as || mhip::check_dims(c, s) || mhip::use_device(c)) return -1;
    if (!decode_shape_fits(s) || s->n_active != NX) return 0;
    if (as->dim != D || as->n_heads != at::NH || as->n_kv_heads != at::NKV ||
        as->head_dim != at::HD)
        return 0;
    if (max_seq <= 0 || max_seq > MHIP_MODEL_STACK_MAX_SEQ) return 0;
    const int fits = decode_device_fits(c);
    if (fits <= 0) return fits;
    int occ = 0;
    if (model_lds_attr(c) ||
        mhip::check(c, hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_model_stack, NT,
                                                                     (size_t)max_seq * 4),
                    "occupancy"))
        return -1;
    return occ >= 1 ? 1 : 0;
}

int mhip_model_stack(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay,
                     const void *d_table, const float *d_router_dl, const float *d_router_t,
                     const float *d_norm, const float *d_bias, const mhip_attn_dims *as,
                     const mhip_attn_layer *d_al, const double *d_rope, int pos, int max_seq,
                     float *d_x, int L, void *d_ws, int *d_status, int flags) {
    const int ok = check_decode_args(c, s, L);
    if (ok <= 0) return ok;
    if (!as || !d_al || !d_rope || !d_status)
        return mhip::fail(c, "model stack: a null argument");
    if (s->n_active != NX || as->dim != D || as->n_heads != at::NH ||
        as->n_kv_heads != at::NKV || as->head_dim != at::HD)
        return mhip::fail(c, "model stack: shape not supported (top-%d of the MoE, dim 2048, "
                             "32/4 heads of 128)", NX);
    if (max_seq <= 0 || max_seq > MHIP_MODEL_STACK_MAX_SEQ || pos < 0 || pos >= max_seq)
        return mhip::fail(c, "model stack: pos=%d, max_seq=%d outside [0, %d]", pos, max_seq,
                          MHIP_MODEL_STACK_MAX_SEQ);
    if ((uintptr_t)d_ws % 256)
        return mhip::fail(c, "model stack: workspace %p is not 256-byte aligned", d_ws);
    if (model_lds_attr(c)) return -1;
    DecodeWs *ws = (DecodeWs *)d_ws;
    ModelPart mp;
    mp.al = d_al;
    mp.xw = (AttnXWs *)((uint8_t *)d_ws + mhip_decode_ws_bytes());
    mp.rope = d_rope;
    mp.pos = pos;
    // a forced abort of either half stops the whole launch
    const int f = (flags & MHIP_ATTN_FORCE_ABORT) ? (flags | MHIP_DECODE_FORCE_ABORT) : flags;
    const int rc = launch_decode(c, s, lay, d_table, d_router_dl, d_router_t, d_norm, d_bias, d_x,
                                 L, ws, &c->decode_epoch, ws != c->decode_ws, nullptr, nullptr,
                                 d_status, f & ~MHIP_ATTN_FORCE_ABORT, &mp);
    if (rc == 0) c->decode_ws = ws;
    return rc;
}

int mhip_decode_status(mhip_ctx *c, const void *d_ws, int status[4]) {
    const DecodeWs *ws = (const DecodeWs *)d_ws;
    tw st[3];
    if (mhip_d2h(c, st, ws->status, sizeof st)) return -1;
    for (int i = 0; i < 3; i++)
        status[i] = (d_ws == c->decode_ws && (unsigned)(st[i] >> 32) == c->decode_epoch)
                        ? (int)(unsigned)st[i] : 0;
    status[3] = 0;
    return 0;
}

int mhip_decode_trace(mhip_ctx *c, const void *d_ws, unsigned long long *out) {
    const DecodeWs *ws = (const DecodeWs *)d_ws;
    return mhip_d2h(c, out, ws->trace, sizeof(ws->trace));
}

}  // extern "C"
