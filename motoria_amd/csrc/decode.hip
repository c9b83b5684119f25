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
// rows and finish their h values without a workgroup barrier. Waves 4-7 hold
// the workgroup's down rows and the next layer's router rows in registers:
// they issue those loads during the gate/up pass and never wait for them at a
// synchronisation, so the h exchange overlaps the rest of the weight stream.
//
// Per layer, on every XCD:
//   A  x (8 KB) -> certified rmsnorm -> xn, Q8(xn) in LDS; 4 router logits per
//      workgroup (one per down wave) by a parallel sum with a rigorous bound
//      on the distance to the reference's sequential fp32 chain  [XCD sync]
//   B  all 128 logits -> ranks (LDS, 512 threads) -> top-K + certification
//      -> gate weights (if the ordering is not certified, the exact
//      sequential logits are computed and routing follows the reference bit
//      for bit)
//   C  gate/up rows of expert idx[k] + SwiGLU -> h (768 floats) [XCD sync]
//      (the down rows and the next layer's router rows are loaded meanwhile)
//   D  Q8(h) -> down rows -> the expert's output rows, published device-wide
//   E  combine x_r += w_j * out_j,r in top-K order for 64 rows [XCD sync]
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
constexpr int HROWS = EH / WPX;                 // 24 h rows per workgroup
constexpr int DROWS = D / WPX;                  // 64 down rows per workgroup
constexpr int LPW = E / WPX;                    // 4 logits per workgroup
constexpr int NGU = 4;                          // waves 0..3: gate/up
constexpr int NDN = NWAVE - NGU;                // waves 4..7: down + router rows
constexpr int GU_H = HROWS / NGU;               // 6 h rows per gate/up wave
constexpr int GU_R = 2 * GU_H;                  // its 12 weight rows
constexpr int DPK = DROWS * NBH / (NDN * 64);   // 6 (row, block) pairs per down thread
constexpr long SPIN = 1L << 18;

typedef int v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld_stream(const void *p) {
    const v4i v = __builtin_nontemporal_load((const v4i *)p);
    return make_int4(v.x, v.y, v.z, v.w);
}

static_assert(NB == 64, "one 32-block per lane");
static_assert(LPW == NDN, "one router row per down wave");
static_assert(GU_H * NGU == HROWS && DPK * NDN * 64 == DROWS * NBH, "tiling");
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
};

// The allocation-free entry point's workspace (the array `scratch` below):
// its size, and per device the address of that device's copy and the epoch
// of the last launch that used it (shared by every context of the device;
// calls that overlap on one GPU race, like two launches on one workspace).
constexpr size_t STATIC_WS_BYTES = (sizeof(DecodeWs) + 255) / 256 * 256;
constexpr int MAX_DEVICES = 64;
struct StaticWs {
    void *ptr;       // device address of this device's copy (0 until set up)
    unsigned epoch;  // launches since it was last cleared
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

// Sequential fp32 sum, in order, of the wavefront's 128 values, lane L
// holding value L in a and value 64 + L in b: each step adds a lane's value
// to the running sum of the lane before it (DPP wave_ror:1, lane 0 taking
// lane 63's), so step i's sum is correct in lane i % 64. The sum of all 128
// ends in lane 63.
__device__ __forceinline__ float wave_seq_sum_128(float a, float b) {
    float s = 0.0f + a;
    for (int i = 1; i < 64; i++)
        s = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x13C, 0xf, 0xf, false)) + a;
    for (int i = 0; i < 64; i++)
        s = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x13C, 0xf, 0xf, false)) + b;
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

__global__ __launch_bounds__(NT) void k_decode_stack(DecodeArgs a) {
    __shared__ Lds sh;
    DecodeWs *ws = a.ws;
    int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.K;
    const int need = K < E ? K + 1 : K;     // ranks certified: K and the first not taken
    const size_t layer_bytes = (size_t)E * a.lay.expert_bytes;
    const bool gu_wave = wave < NGU;

    // Start: every workgroup reads its XCD from the hardware and takes a
    // rank among that XCD's workgroups from the XCD's ticket counter of this
    // launch (the dispatcher deals the 256 workgroups to the 8 XCDs in turn,
    // 32 each, but which XCD receives the first one varies between launches
    // of different queues); then a device-wide barrier (the counter gains
    // NWG per launch; epochs count launches since the workspace was cleared).
    if (tid == 0) {
        const unsigned hx = xcc_id();
        unsigned rk = WPX;
        if (hx < NX)
            rk = __hip_atomic_fetch_add(&ws->xtick[a.epoch & 1][hx].n, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
        if (rk >= WPX) status_update(ws, ST_ABORT, a.epoch, false, 1);
        sh.role[0] = hx < NX ? (int)hx : 0;
        sh.role[1] = rk < WPX ? (int)rk : 0;
        if ((a.flags & MHIP_DECODE_FORCE_ABORT) && blockIdx.x == 0)
            status_update(ws, ST_ABORT, a.epoch, false, 4);
        __builtin_amdgcn_s_waitcnt(0);
        __hip_atomic_fetch_add(&ws->gstart[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_flag(ws, &ws->gstart[0], NWG * a.epoch, a.epoch);
        // every workgroup of this launch holds its ticket: the other parity's
        // counters start the next launch from zero
        if (blockIdx.x == 0)
            for (int k = 0; k < NX; k++)
                __hip_atomic_store(&ws->xtick[(a.epoch + 1) & 1][k].n, 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const int xcd = __builtin_amdgcn_readfirstlane(sh.role[0]);
    const int rank = __builtin_amdgcn_readfirstlane(sh.role[1]);
    // An XCD without a routed slot has nothing that another XCD reads.
    if (aborted(ws, a.epoch) || xcd >= K) return;

    // One register array serves both roles. A gate/up wave holds its GU_R
    // weight rows in wq0/wq1/wsc during stage C. A down wave holds its DPK
    // down (row, block) pairs in slots 0..DPK-1 from stage C to D, and the
    // router row of its logit (8 x 16 bytes per lane, as int bits) in the
    // slots above: wq0[DPK..GU_R), then wq1[DPK..). Sharing the registers
    // keeps the compiler from copying loads still in flight (which would wait
    // for them) where the two roles' code paths meet.
    constexpr int NR0 = GU_R - DPK;
    static_assert(2 * NR0 >= 8, "router row slots");
    int4 wq0[GU_R], wq1[GU_R];
    float wsc[GU_R];
    // In the decode layout, load k of the row (1 KB, contiguous) gives lane
    // L its elements 32 L + 4 k .. + 3.
#define LOAD_ROUTER(layer) LOAD_ROUTER_ROW((size_t)(layer) * E + rank * LPW + wave - NGU)
#define LOAD_ROUTER_ROW(row)                                                               \
    do {                                                                                   \
        const int4 *src_ = (const int4 *)(a.router + (size_t)(row) * D) + lane;            \
        _Pragma("unroll") for (int k_ = 0; k_ < NR0; k_++) wq0[DPK + k_] = src_[64 * k_];  \
        _Pragma("unroll") for (int k_ = 0; k_ < 8 - NR0; k_++) wq1[DPK + k_] = src_[64 * (NR0 + k_)]; \
    } while (0)
#define RROW(k)                                                                            \
    i4_as_f4((k) < NR0 ? wq0[DPK + ((k) < NR0 ? (k) : 0)] : wq1[DPK + ((k) < NR0 ? 0 : (k) - NR0)])
    // rmsnorm weights of the next layer at this thread's 4 positions.
    float wn[D / NT];
#define LOAD_NORM(layer)                                                                   \
    do {                                                                                   \
        _Pragma("unroll") for (int k_ = 0; k_ < D / NT; k_++)                              \
            wn[k_] = a.norm[(size_t)(layer) * D + tid + NT * k_];                          \
    } while (0)
    if (!gu_wave) LOAD_ROUTER(0);
    LOAD_NORM(0);
    for (int i = tid; i < D; i += NT) sh.x[i] = a.x[i];
    if (tid < E) sh.bias[tid] = a.bias ? a.bias[tid] : 0.0f;
    if (tid < 32) sh.etab[tid] = mia_expf_tab[tid];
    // no tag of this launch ((epoch << 8) | layer) has this value
    if (tid == 0) sh.invtag = (a.epoch + 1u) << 8;
    if (tid < NGU) sh.ptag[tid] = (a.epoch + 1u) << 8;

    for (int l = 0; l < a.L; l++) {
        // Per-thread addresses are recomputed in every layer rather than held
        // in registers across the loop (the thread index is made opaque).
        asm volatile("" : "+v"(tid));
        lane = tid & 63;
        const int dt = tid - NGU * 64;          // index among the down waves' threads
        const unsigned tag = (a.epoch << 8) | (unsigned)(l & 255);
        TRACE(0);
        TRACE_CLK(30);
        // ---- A: rmsnorm (certified), xn, Q8(xn), logits -----------------------------
        // Wavefront 0 computes the scale inv while the down waves form their
        // logits' products without it, from xt_i = fl(x_i * w_i) (w the norm
        // weight): p~_i = fl(W_ei * xt_i). The reference's product
        // p_i = fl(W_ei * fl(fl(x_i * inv) * w_i)) is inv * p~_i * (1 + eta_i)
        // with |eta_i| <= (1+u)^3 / (1-u)^2 - 1 < 5.0001 u (u = 2^-24, no
        // underflow), so once inv is known the sums of p~ scaled by inv bound
        // the reference's chain.
#pragma unroll
        for (int k = 0; k < D / NT; k++) {
            const int i = tid + NT * k;
            sh.xt[(i / 32) * XN_LD + i % 32] = sh.x[i] * wn[k];
        }
        __syncthreads();
        TRACE(14);
        // down waves, uniform in the wave: sum p~, sum_k |prefix_k|, sum |p~|
        double lgS = 0.0, lgA = 0.0, lgP = 0.0;
        if (gu_wave) {
            // partial sums of squares, one per gate/up wave; wavefront 0
            // adds them and brackets the scale. Any summation order is within
            // (n + log2 n) 2^-53 S of the reference's sequential double sum
            // (all terms >= 0); S -/+ m brackets it, and when both ends give
            // the same fp32 scale it is the reference's. Otherwise lane 0
            // runs the sequential sum.
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < D / (NGU * 64); k++) {
                const double v = (double)sh.x[tid + NGU * 64 * k];
                ss = ss + v * v;
            }
            ss = lane63_d(wave_scan_d(ss));
            if (lane == 0) {
                sh.part[wave] = ss;
                __hip_atomic_store(&sh.ptag[wave], tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            if (wave == 0) {
                long sp = 0;
                for (;;) {
                    const unsigned t = lane < NGU ? __hip_atomic_load(&sh.ptag[lane], __ATOMIC_ACQUIRE,
                                                                      __HIP_MEMORY_SCOPE_WORKGROUP)
                                                  : tag;
                    if (__ballot(t != tag) == 0) break;
                    __builtin_amdgcn_s_sleep(1);
                    if (++sp > SPIN) {
                        if (lane == 0) status_update(ws, ST_ABORT, a.epoch, false, 2);
                        break;
                    }
                }
                double S = 0.0;
                for (int k = 0; k < NGU; k++) S = S + sh.part[k];
                // lane 0 takes the lower end of the bracket, lane 1 the upper
                const double m = S * ((double)(D + 64) * 0x1p-52);
                const float end = (float)(1.0 / sqrt((lane == 1 ? S - m : S + m) / D + (double)a.eps));
                const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(end), 0));
                const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(end), 1));
                float iv = lo;
                if ((a.flags & MHIP_FORCE_SEQ_RMS) || lo != hi) {   // uniform in the wave
                    float sq_inv = 0.0f;
                    if (lane == 0) {
                        double sq = 0.0;
                        for (int i = 0; i < D; i++) sq = sq + (double)sh.x[i] * (double)sh.x[i];
                        sq_inv = (float)(1.0 / sqrt(sq / D + (double)a.eps));
                        if (xcd == 0 && rank == 0) status_update(ws, ST_RMS, a.epoch, true, 0);
                    }
                    iv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq_inv)));
                }
                if (lane == 0) {
                    sh.inv = iv;
                    sh.nanflag = 0;
                    __hip_atomic_store(&sh.invtag, tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        } else if (!gu_wave) {
            // This lane's 32 products, summed in four independent stretches
            // of 8; the prefix sums of the second pass restart each stretch
            // from its own offset, so no dependency chain is longer than 8
            // additions.
            const float4 *xv4 = (const float4 *)&sh.xt[lane * XN_LD];
            float pr[32];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 wv = RROW(k), xv = xv4[k];
                pr[4 * k + 0] = wv.x * xv.x;
                pr[4 * k + 1] = wv.y * xv.y;
                pr[4 * k + 2] = wv.z * xv.z;
                pr[4 * k + 3] = wv.w * xv.w;
            }
            // sum |p~| in fp32 (32 terms >= 0: within 32 u of the exact sum,
            // covered by the factor applied to lgP below)
            double cs[4];
            float ap = 0.0f;
#pragma unroll
            for (int m = 0; m < 4; m++) {
                cs[m] = 0.0;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    cs[m] = cs[m] + (double)pr[8 * m + j];
                    ap = ap + fabsf(pr[8 * m + j]);
                }
            }
            const double tot = (cs[0] + cs[1]) + (cs[2] + cs[3]);
            const double incl = wave_scan_d(tot);
            TRACE_BY(21, NGU * 64);
            double run[4], ab[4];
            run[0] = incl - tot;  // exclusive prefix of this lane
            run[1] = run[0] + cs[0];
            run[2] = run[1] + cs[1];
            run[3] = run[2] + cs[2];
#pragma unroll
            for (int m = 0; m < 4; m++) ab[m] = 0.0;
#pragma unroll
            for (int j = 0; j < 8; j++)
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    run[m] = run[m] + (double)pr[8 * m + j];
                    ab[m] = ab[m] + fabs(run[m]);
                }
            lgS = lane63_d(incl);
            lgA = lane63_d(wave_scan_d((ab[0] + ab[1]) + (ab[2] + ab[3])));
            lgP = lane63_d(wave_scan_d((double)ap)) * (1.0 + 0x1p-16);
            TRACE_BY(22, NGU * 64);
        }
        // every wave takes inv from wavefront 0 (LDS, release / acquire);
        // wavefront 0 never waits for another, so the wait ends
        {
            long sp = 0;
            while (__hip_atomic_load(&sh.invtag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != tag) {
                __builtin_amdgcn_s_sleep(1);
                if (++sp > SPIN) {
                    if (lane == 0) status_update(ws, ST_ABORT, a.epoch, false, 2);
                    break;
                }
            }
        }
        const float inv = sh.inv;
        TRACE(15);
        {
#pragma unroll
            for (int k = 0; k < D / NT; k++) {
                const int i = tid + NT * k;
                sh.xn[(i / 32) * XN_LD + i % 32] = (sh.x[i] * inv) * wn[k];
            }
        }
        if (!gu_wave && lane == 0) {
            // The logit S = inv * sum p~ (double) and its bound: the
            // reference's chain L over p is within u (1 + 2^-8) sum_k |S_k|
            // of the exact sum of p (S_k its prefix sums; the slack covers
            // the chain's own drift and the double sums), sum_k |S_k| <=
            // inv * lgA + D * Ep, and the exact sum of p is within
            // Ep = 5.0001 u inv lgP of inv * lgS. S goes out rounded to fp32
            // (|S - Sf| <= u |Sf|, 2^-52 |S| for the double product, 2^-100
            // for subnormal products); the bound is rounded upwards to fp32
            // by the (1 + 2^-22) factor.
            const int e = rank * LPW + wave - NGU;
            const double di = (double)inv;
            const double S = di * lgS;
            const float Sf = (float)S;
            const double Ep = 5.0001 * 0x1p-24 * di * lgP;
            const double B = 0x1p-24 * (1.0 + 0x1p-8) * (di * lgA + (double)D * Ep) + Ep +
                             0x1p-24 * fabs((double)Sf) + 0x1p-52 * fabs(S) + 0x1p-100;
            put_tagged<true>(&ws->lgs[xcd][e], Sf, tag);
            put_tagged<true>(&ws->lgb[xcd][e], (float)(B * (1.0 + 0x1p-22)), tag);
        }
        __syncthreads();
        TRACE_BY(20, NGU * 64);
        if (!gu_wave) {
            // Q8(xn) for stage C, while the logits travel (quant.c:11-27 per
            // element): four lanes per 32-block, eight elements each, the
            // block maximum over the quad by DPP (order-free).
            {
                const int blk = dt >> 2, sub = dt & 3;
                const float4 *src = (const float4 *)&sh.xn[blk * XN_LD + sub * 8];
                const float4 v0 = src[0], v1 = src[1];
                const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                float am = 0.0f;                                 // a NaN counts as 0
#pragma unroll
                for (int i = 0; i < 8; i++) am = fmaxf(am, fabsf(v[i]));
                am = fmaxf(am, dpp_keep_f<0xB1>(am));            // quad_perm [1,0,3,2]
                am = fmaxf(am, dpp_keep_f<0x4E>(am));            // quad_perm [2,3,0,1]
                const float d = am / 127.0f;
                const float qi = d != 0.0f ? 1.0f / d : 0.0f;
                union {
                    int8_t c[8];
                    int2 w;
                } q;
#pragma unroll
                for (int i = 0; i < 8; i++) q.c[i] = (int8_t)roundf(v[i] * qi);
                *(int2 *)&sh.xq[blk * 32 + sub * 8] = q.w;
                if (sub == 0) sh.xs[blk] = d;
            }
        }
        TRACE_BY(1, NGU * 64);
        TRACE(2);

        // ---- B: ranks, certification ------------------------------------------------
        if (tid < E) {
            float sb[2];
            get_tagged<2, true>(ws, &ws->lgs[xcd][tid], NX * E, tag, sb);
            const double S = (double)sb[0], B = (double)sb[1];
            const float bs = sh.bias[tid];
            const double c = S + (double)bs;
            // monotone 64-bit image of c with the low 7 bits replaced by
            // 127 - e: distinct keys, lower index first among (near-)equal
            // values; an order that differs from c's fails the gap test below
            uint64_t u = (uint64_t)__double_as_longlong(c);
            u = (u >> 63) ? ~u : (u | (1ull << 63));
            sh.key[tid] = ((u >> 7) << 7) | (uint64_t)(E - 1 - tid);
            sh.c[tid] = c;
            sh.lf[tid] = a.bias ? sb[0] + bs : sb[0];
            if (c != c) sh.nanflag = 1;
            const double bm = wave_max_d(B);
            if (lane == 0) sh.bpart[wave] = bm;
        }
        __syncthreads();
        TRACE(10);
        {
            // rank of expert e among the 32 keys of quarter q
            const int e = tid & (E - 1), q = tid >> 7;
            const uint64_t ke = sh.key[e];
            const ulonglong2 *kv = (const ulonglong2 *)&sh.key[q * 32];
            int rk = 0;
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const ulonglong2 v = kv[k];
                rk += (int)(v.x > ke) + (int)(v.y > ke);
            }
            sh.rk[q][e] = rk;
        }
        __syncthreads();
        if (tid < E) {
            const int rk = sh.rk[0][tid] + sh.rk[1][tid] + sh.rk[2][tid] + sh.rk[3][tid];
            if (rk < need) sh.order[rk] = tid;
        }
        __syncthreads();
        TRACE(11);
        if (wave == 0) {
            // Without NaN keys the ranks are a permutation, so order[0..need)
            // is set. The order is the reference's when every consecutive gap
            // exceeds twice the largest bound plus a margin for the fp32
            // roundings between the logit and the probability (logit + bias,
            // l - mx, expf, division). The gate weights are computed later,
            // while the XCD waits for h.
            // Under the exact router (MHIP_FORCE_EXACT_ROUTER) a certified
            // ranking is the reference's, so only the gate weights need the
            // exact chains: they run beside the gate/up stream (stage C)
            // unless MHIP_DECODE_CHAINS_FIRST asks for them before it.
            const bool exact = (a.flags & MHIP_FORCE_EXACT_ROUTER) != 0;
            bool ok = sh.nanflag == 0 && !(exact && (a.flags & MHIP_DECODE_CHAINS_FIRST));
            if (ok) {
                const double top = sh.c[sh.order[0]], bmax = fmax(sh.bpart[0], sh.bpart[1]);
                int bad = 0;
                if (lane >= 1 && lane < need) {
                    const double prev = sh.c[sh.order[lane - 1]], cw = sh.c[sh.order[lane]];
                    const double tau = 0x1p-19 * (2.0 + fabs(top) + fabs(prev));
                    bad = !(prev - cw > 2.0 * bmax + tau);
                }
                ok = __ballot(bad) == 0;
            }
            if (ok && lane < K) sh.idx[lane] = sh.order[lane];
            if (lane == 0) {
                sh.fallback = ok ? 0 : 1;
                sh.shadow_on = ok && exact ? 1 : 0;
            }
        }
        __syncthreads();
        if (sh.fallback) {
            // Exact logits, the reference's sequential chain: each down wave
            // computes one (products in registers, summed in order across
            // the lanes), then the XCD exchanges them.
            if (!gu_wave) {
                const float *xv = &sh.xn[lane * XN_LD];
                float pr[32];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 wv = RROW(k);
                    pr[4 * k + 0] = wv.x * xv[4 * k + 0];
                    pr[4 * k + 1] = wv.y * xv[4 * k + 1];
                    pr[4 * k + 2] = wv.z * xv[4 * k + 2];
                    pr[4 * k + 3] = wv.w * xv[4 * k + 3];
                }
                float sl = wave_seq_sum_2048(pr);
                const int e = rank * LPW + wave - NGU;
                if (a.bias) sl = sl + sh.bias[e];
                if (lane == 63) put_tagged<true>(&ws->lx[xcd][e], sl, tag);
            }
            if (tid < E) get_tagged<1, true>(ws, &ws->lx[xcd][tid], 0, tag, &sh.lf[tid]);
            __syncthreads();
            // forward.c:95-101: the first maximum, then the sequential sum.
            // With l[0] a NaN every comparison fails and the maximum stays
            // NaN; otherwise it is the largest non-NaN logit, which a
            // NaN-ignoring maximum finds in any order (equal maxima, +0 and
            // -0 among them, give the same exponentials).
            if (tid < E) {
                const double m = wave_max_d((double)sh.lf[tid]);
                if (lane == 0) sh.mxpart[tid >> 6] = (float)m;
            }
            __syncthreads();
            if (tid < E) {
                float mx = sh.mxpart[0];
#pragma unroll
                for (int q = 1; q < E / 64; q++) mx = fmaxf(mx, sh.mxpart[q]);
                if (sh.lf[0] != sh.lf[0]) mx = sh.lf[0];
                sh.p[tid] = mia_expf_glibc_tab(sh.lf[tid] - mx, sh.etab);
            }
            __syncthreads();
            if (tid == 0) sh.sum = lds_seq_sum_n<E>(sh.p, 0.0f);
            __syncthreads();
            if (tid < E) {
                const float pe = sh.p[tid] / sh.sum;
                sh.p[tid] = pe;
                if (pe != pe) sh.nanflag = 2;
            }
            if (tid < KMAX) sh.idx[tid] = 0;
            __syncthreads();
            if (sh.nanflag == 2) {
                // forward.c:104-114 literally (a NaN probability never wins a
                // comparison; the first untaken index stands in for it).
                if (tid == 0) {
                    for (int j = 0; j < K; j++) {
                        int best = -1;
                        for (int i = 0; i < E; i++) {
                            int taken = 0;
                            for (int t = 0; t < j; t++) taken |= sh.idx[t] == i;
                            if (!taken && (best < 0 || sh.p[i] > sh.p[best])) best = i;
                        }
                        sh.idx[j] = best;
                    }
                }
            } else if (tid < E) {
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
                // the K probabilities read first, then summed in rank order
                float pk[KMAX];
#pragma unroll
                for (int j = 0; j < KMAX; j++) pk[j] = j < K ? sh.p[sh.idx[j]] : 0.0f;
                float wsum = 0.0f;
#pragma unroll
                for (int j = 0; j < KMAX; j++)
                    if (j < K) wsum = wsum + pk[j];
#pragma unroll
                for (int j = 0; j < KMAX; j++)
                    if (j < K) sh.w[j] = a.norm_topk ? pk[j] / wsum : pk[j];
                if (xcd == 0 && rank == 0) status_update(ws, ST_ROUTER, a.epoch, true, 0);
            }
            __syncthreads();
        }
        TRACE(3);

        // ---- C: gate/up + SwiGLU for expert slot `xcd` -----------------------------
        const bool active = xcd < K;
        const int ex = min(max(sh.idx[active ? xcd : 0], 0), E - 1);
        const uint8_t *eb = a.table + (size_t)l * layer_bytes + (size_t)ex * a.lay.expert_bytes;
        // The next layer's rmsnorm weights are requested first: they arrive
        // before this wave's weight rows, so no later wait is held up by them
        // (the last layer reloads its own). Its router rows follow in stage D,
        // once this layer's rows are in.
        const int lnext = min(l + 1, a.L - 1);
        LOAD_NORM(lnext);
        if (gu_wave) {
            if (active) {
                // this wave's rows: gate h0..h0+GU_H-1, then up h0..h0+GU_H-1.
                // A row's 2 KB of codes arrive as two contiguous 1 KB loads:
                // lane l holds half (l & 1) of block l/2 and of block 32 + l/2;
                // the lane pair adds its two half dots, and lane l keeps
                // block blk = l/2 (l even) or 32 + l/2 (l odd).
                const int h0 = rank * HROWS + wave * GU_H;
                const int hf = lane & 1, bm = lane >> 1;
                const int blk = hf ? NB / 2 + bm : bm;
                const int4 xa = *(const int4 *)&sh.xq[bm * 32 + 16 * hf];
                const int4 xb = *(const int4 *)&sh.xq[(NB / 2 + bm) * 32 + 16 * hf];
                const float dx = sh.xs[blk];
#pragma unroll
                for (int r = 0; r < GU_R; r++) {
                    const int row = h0 + (r % GU_H);
                    const size_t qoff = (r < GU_H ? a.lay.gate_q : a.lay.up_q) + (size_t)row * D +
                                        (size_t)lane * 16;
                    const size_t soff = (r < GU_H ? a.lay.gate_s : a.lay.up_s);
                    const int4 *src = (const int4 *)(eb + qoff);
                    wq0[r] = ld_stream(src);
                    wq1[r] = ld_stream(src + 64);
                    wsc[r] = ((const float *)(eb + soff))[(size_t)row * NB + blk];
                }
                float *terms = &sh.scr[wave * GU_R * GU_LD];
#pragma unroll
                for (int r = 0; r < GU_R; r++) {
                    const int pa = dot16_i8(wq0[r], xa), pb = dot16_i8(wq1[r], xb);
                    const int other = __builtin_amdgcn_update_dpp(0, hf ? pa : pb, 0xB1, 0xf, 0xf, false);
                    terms[r * GU_LD + blk] =
                        mhip_dev::block_term((hf ? pb : pa) + other, wsc[r], dx);
                }
                TRACE(12);
                wave_lds_sync();
                if (lane < GU_R) sh.gu[wave][lane] = lds_seq_sum_n<NB>(&terms[lane * GU_LD], 0.0f);
                wave_lds_sync();
                TRACE(19);
                if (lane < GU_H) {
                    const float g = sh.gu[wave][lane], u = sh.gu[wave][GU_H + lane];
                    put_tagged<true>(&ws->h[xcd][h0 + lane],
                               (g / (1.0f + mia_expf_glibc_tab(-g, sh.etab))) * u, tag);
                }
                TRACE_BY(16, 64);
                TRACE_BY(17, 192);
            }
        } else {
            const bool shadow = sh.shadow_on != 0;
            if (shadow) {
                // The exact logit of this wave's expert (forward.c:173-176:
                // the reference's sequential chain) from its router row of
                // this layer, still in registers, before the loads that reuse
                // those registers: the HBM stream of the gate/up waves would
                // hold the loads' issue, and the chain behind them, for most
                // of this stage.
                const float *xv = &sh.xn[lane * XN_LD];
                float pr[32];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 wv = RROW(k);
                    pr[4 * k + 0] = wv.x * xv[4 * k + 0];
                    pr[4 * k + 1] = wv.y * xv[4 * k + 1];
                    pr[4 * k + 2] = wv.z * xv[4 * k + 2];
                    pr[4 * k + 3] = wv.w * xv[4 * k + 3];
                }
                float sl = wave_seq_sum_2048(pr);
                const int e = rank * LPW + wave - NGU;
                if (a.bias) sl = sl + sh.bias[e];
                if (lane == 63) put_tagged<true>(&ws->lx[xcd][e], sl, tag);
                TRACE_BY(23, NGU * 64);
            }
            // the down rows of this workgroup (used once h has arrived)
            if (wave == NGU && !sh.fallback && !shadow) {
                // The gate weights, before this wave's loads (a wave waiting
                // to issue a load runs nothing else, and the CU takes its
                // vector memory instructions in order). Softmax of the
                // parallel logits (forward.c:95-101 in shape; the weights
                // only need the 1e-3 tolerance); with renormalisation
                // (forward.c:178-181) the full sum cancels and only the
                // top K exponentials are needed.
                const float mx = sh.lf[sh.idx[0]];
                const float ek = mia_expf_glibc_tab(sh.lf[sh.idx[min(lane, K - 1)]] - mx, sh.etab);
                const float ej = lane < K ? ek : 0.0f;
                float den;
                if (a.norm_topk)
                    den = wave_sum_f(ej);
                else
                    den = wave_sum_f(mia_expf_glibc_tab(sh.lf[lane] - mx, sh.etab) +
                                     mia_expf_glibc_tab(sh.lf[lane + 64] - mx, sh.etab));
                if (lane < K) sh.w[lane] = ej / den;
                TRACE_BY(18, NGU * 64);
            }
#pragma unroll
            for (int k = 0; k < DPK; k++) {
                // The workgroup's 64 rows are one contiguous 48 KB run, read
                // as 16-byte pieces q = dt + 256 j (j < 12): the two halves of
                // block q/2 sit in a lane pair. Loads 2k, 2k + 1 go to
                // wq0[k], wq1[k]; the pair later keeps block P(2k + (dt & 1)).
                const int4 *run = (const int4 *)(eb + a.lay.down_q + (size_t)rank * DROWS * EH);
                wq0[k] = ld_stream(run + dt + NDN * 64 * (2 * k));
                wq1[k] = ld_stream(run + dt + NDN * 64 * (2 * k + 1));
                const int p = (dt >> 1) + (NDN * 32) * (2 * k + (dt & 1));
                wsc[k] = ((const float *)(eb + a.lay.down_s))[(size_t)rank * DROWS * NBH + p];
            }
        }
        TRACE(4);
        // ---- D: Q8(h) and down ------------------------------------------------------
        const int par = l & 1;
        if (active) {
            // h is polled by the gate/up waves, which have no loads in
            // flight: wave w takes h[192w, 192w + 192), i.e. six Q8 blocks,
            // two per register with one block per 32-lane half, and
            // quantizes them in place (quant.c:11-27 per element; the block
            // maximum is order-free).
            if (gu_wave) {
                constexpr int HPW = EH / (NGU * 64);
                float hv[HPW];
                get_tagged<HPW, true>(ws, &ws->h[xcd][wave * 64 * HPW + lane], 64, tag, hv);
#pragma unroll
                for (int k = 0; k < HPW; k++) {
                    const int i = wave * 64 * HPW + 64 * k + lane;
                    float am = fmaxf(0.0f, fabsf(hv[k]));   // a NaN counts as 0, as in the chain
                    am = fmaxf(am, dpp_keep_f<0x121>(am));  // row_ror 1, 2, 4, 8: 16-lane max
                    am = fmaxf(am, dpp_keep_f<0x122>(am));
                    am = fmaxf(am, dpp_keep_f<0x124>(am));
                    am = fmaxf(am, dpp_keep_f<0x128>(am));
                    am = fmaxf(am, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(am), 0x401f)));
                    const float d = am / 127.0f;
                    const float qi = d != 0.0f ? 1.0f / d : 0.0f;
                    sh.hq[i] = (int8_t)roundf(hv[k] * qi);
                    if ((lane & 31) == 0) sh.hsc[i / 32] = d;
                }
            }
            __syncthreads();
            TRACE(5);
            TRACE(13);
            float *dterm = sh.scr;
            if (!gu_wave) {
#pragma unroll
                for (int k = 0; k < DPK; k++) {
                    // blocks pa, pb = pa + 128 of the workgroup's rows (row
                    // p / 24, block p % 24); this lane keeps pa if even, pb if odd
                    const int hf = dt & 1;
                    const int pa = (dt >> 1) + (NDN * 32) * (2 * k), pb = pa + NDN * 32;
                    const int4 ha = *(const int4 *)&sh.hq[(pa % NBH) * 32 + 16 * hf];
                    const int4 hb = *(const int4 *)&sh.hq[(pb % NBH) * 32 + 16 * hf];
                    const int da = dot16_i8(wq0[k], ha), db = dot16_i8(wq1[k], hb);
                    const int other = __builtin_amdgcn_update_dpp(0, hf ? da : db, 0xB1, 0xf, 0xf, false);
                    const int p = hf ? pb : pa;
                    const int row = p / NBH, blk = p % NBH;
                    dterm[row * DN_LD + blk] = mhip_dev::block_term((hf ? db : da) + other, wsc[k],
                                                                    sh.hsc[blk]);
                }
                // the next layer's router rows, after this layer's stream:
                // they load while the expert outputs are exchanged. After the
                // last layer every wave reads router row 0 instead (the same
                // 8 KB, from the L2): the load is issued on every path, so
                // the compiler's wait counts stay exact and the expert
                // outputs' polls never wait for it.
                LOAD_ROUTER_ROW(l + 1 < a.L ? (size_t)lnext * E + rank * LPW + wave - NGU : 0);
            }
            __syncthreads();
            if (wave == 0)
                put_tagged<false>(&ws->out[par][xcd][rank * DROWS + lane],
                           lds_seq_sum_n<NBH>(&dterm[lane * DN_LD], 0.0f), tag);
        }
        TRACE(6);

        // ---- E: combine rows rank*64 .. +64 in top-K order ---------------------------
        if (sh.shadow_on && wave == 1) {
            // Under the exact router with a certified ranking: the XCD's 128
            // exact logits (the down waves' chains, long done) -> softmax
            // (forward.c:95-101: the first maximum as in the exact router
            // above, the sequential sum) -> the certified experts' weights
            // (forward.c:178-181), first needed by the combine below. Wave 1
            // computes them while the expert outputs are on their way (wave 0
            // fetches expert 1's rows).
            float lv[2];
            get_tagged<2, true>(ws, &ws->lx[xcd][lane], 64, tag, lv);
            float mx = (float)wave_max_d(fmax((double)lv[0], (double)lv[1]));
            const float l0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(lv[0])));
            if (l0 != l0) mx = l0;
            const float e0 = mia_expf_glibc_tab(lv[0] - mx, sh.etab);
            const float e1 = mia_expf_glibc_tab(lv[1] - mx, sh.etab);
            const float sum = __int_as_float(
                __builtin_amdgcn_readlane(__float_as_int(wave_seq_sum_128(e0, e1)), 63));
            const float p0 = e0 / sum, p1 = e1 / sum;
            // a NaN probability would rank differently in the reference
            // (forward.c:104-114): the launch reports it and the caller
            // reruns the layer per stage
            const bool nan = __ballot(p0 != p0 || p1 != p1) != 0;
            sh.p[lane] = p0;
            sh.p[lane + 64] = p1;
            wave_lds_sync();
            // lane j < K: the probability of rank j; their sum in rank order
            // (lane j adds its own to lane j - 1's running sum)
            const float pj = lane < K ? sh.p[sh.idx[lane]] : 0.0f;
            float wsum = 0.0f + pj;
            for (int j = 1; j < K; j++)
                wsum = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(wsum), 0x138, 0xf, 0xf, false)) + pj;
            wsum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsum), K - 1));
            if (lane < K) sh.w[lane] = a.norm_topk ? pj / wsum : pj;
            if (lane == 0) {
                if (nan) status_update(ws, ST_ABORT, a.epoch, false, 8);
                if (xcd == 0 && rank == 0) status_update(ws, ST_ROUTER, a.epoch, true, 0);
            }
            TRACE_BY(24, 64);
        }
        {
            // thread (j, r) fetches expert j's output row r; then one thread
            // per row adds them in top-K order
            const int j = tid / DROWS, r = tid % DROWS;
            if (sh.shadow_on && K > 1 && j < 2) {
                if (j == 0) {
                    float v2[2];
                    get_tagged<2, false>(ws, &ws->out[par][0][rank * DROWS + r], D, tag, v2);
                    sh.og[r] = v2[0];
                    sh.og[DROWS + r] = v2[1];
                }
            } else if (j < K) {
                get_tagged<1, false>(ws, &ws->out[par][j][rank * DROWS + r], 0, tag, &sh.og[j * DROWS + r]);
            }
        }
        __syncthreads();
        TRACE(7);
        if (xcd == 0 && rank == 0 && tid < K) {
            if (a.idx_out) a.idx_out[(size_t)l * K + tid] = sh.idx[tid];
            if (a.w_out) a.w_out[(size_t)l * K + tid] = sh.w[tid];
        }
        if (tid < DROWS) {
            const int r = rank * DROWS + tid;
            float v = sh.x[r];
            for (int j = 0; j < K; j++) v = v + sh.w[j] * sh.og[j * DROWS + tid];
            if (l + 1 < a.L) put_tagged<true>(&ws->x[xcd][r], v, tag);
            else if (xcd == 0) a.x[r] = v;
        }
        TRACE(8);
        if (l + 1 < a.L) {
            // the XCD's new residual stream; a row is written only after its
            // old value was read above, so no barrier is needed before this
            float xv[D / NT];
            get_tagged<D / NT, true>(ws, &ws->x[xcd][tid], NT, tag, xv);
#pragma unroll
            for (int k = 0; k < D / NT; k++) sh.x[tid + NT * k] = xv[k];
            TRACE(9);
        }
    }
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
int launch_decode(mhip_ctx *c, const mhip_dims *s, const mhip_layout *lay, const void *d_table,
                  const float *d_router, const float *d_router_t, const float *d_norm,
                  const float *d_bias, float *d_x, int L, DecodeWs *ws, unsigned *epoch,
                  bool fresh, int *d_idx, float *d_w, int *d_status, int flags) {
    if (fresh || *epoch >= (1u << 24) - 1) {
        if (mhip_zero(c, ws, offsetof(DecodeWs, trace))) return -1;
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
    // An ordinary launch: one 512-thread workgroup fits each of the 256 CUs
    // (checked before), so on an otherwise idle device all of them are
    // resident at once. Should one not be, the start barrier times out and
    // the launch reports abort bit 2 instead of waiting for ever.
    int slot = mhip::stage_begin(c, MHIP_STAGE_DECODE);
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
    if (st.ptr) return 0;
    void *ptr = nullptr;
    if (check(c, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
              "hipGetSymbolAddress (decode workspace)"))
        return -1;
    if (!ptr || (uintptr_t)ptr % 256) return fail(c, "decode workspace symbol at %p", ptr);
    // cleared once here; afterwards the launches' epochs keep it consistent
    if (mhip_zero(c, ptr, STATIC_WS_BYTES) || mhip_sync(c)) return -1;
    st.ptr = ptr;
    st.epoch = 0;
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
    if (!st || !st->ptr)
        return mhip::fail(c, "no-alloc decode: device %d has no set-up workspace", c->device);
    return launch_decode(c, s, lay, d_table, d_router, d_router_t, d_norm, d_bias, d_x, L,
                         (DecodeWs *)st->ptr, &st->epoch, false, d_idx, d_w, d_status, flags);
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
