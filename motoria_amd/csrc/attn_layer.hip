// The attention of one token for one layer in one launch (decode), on every
// CU: src/model/forward.c:118-165 of the reference with every value in its
// order -- the arithmetic of attention.hip's k_rmsnorm_q8_w, k_rows_q8 and
// k_attn_head, regrouped so that a layer costs one launch instead of four.
// Shape: the Qwen3-30B-A3B attention (dim 2048, 32 query and 4 key/value
// heads of 128).
//
//   P1 every workgroup: rmsnorm(x, attn_norm) and Q8(xn) (wavefront 0, lane
//      b owning 32-block b; the certified sum of squares)      forward.c:123
//   P2 every wavefront: its q/k/v rows (5120 rows over 2048 wavefronts),
//      lane b the term of block b, the block-order sum passed lane to lane
//                                                              forward.c:124-126
//   P3 workgroup h < 32: query head h -- norms, RoPE, the cache append (the
//      group's first head), scores, softmax, mix, Q8 of the head's output
//                                                              forward.c:127-163
//   P4 every wavefront: one row of Wo over the heads' codes, plus the
//      residual                                                forward.c:164-165
//
// Every weight row is requested at the start (45 dwords per lane), after
// what the norm and the heads need first, so the 21 MB of the layer's
// attention weights stream in while the norm runs. Workgroups meet only
// through tagged 64-bit words (value, launch tag) in a workspace, stored and
// polled at device scope (the producers of a word are on other XCDs). A wait
// that runs out (a workgroup not resident) marks the launch aborted and
// every later wait gives up at once; x is then left as it was and the caller
// reruns the layer through the per-stage kernels.
#include "mhip_internal.h"

namespace {

constexpr int D = 2048, NH = 32, NKV = 4, HD = 128;
constexpr int QD = NH * HD, KVD = NKV * HD, NROWS = QD + 2 * KVD;  // 4096, 512, 5120
constexpr int NB = D / 32, NBO = QD / 32;                            // 64, 128 blocks
constexpr int NWG = 256, NT = 512, NW = NT / 64;
constexpr int GW = NWG * NW;                  // 2048 wavefronts
constexpr int RPW = (NROWS + GW - 1) / GW;    // at most 3 q/k/v rows per wavefront
constexpr int GROUP = NH / NKV;
constexpr int NPRE = 64;                      // cache positions a head stages in LDS
constexpr int KPF = NPRE * HD / 4 / NT;       // float4 of those K (and V) rows per thread
constexpr int KLD = HD + 4;                   // K row stride in LDS (rows on distinct banks)
static_assert(KPF * 4 * NT == NPRE * HD, "whole staging rounds");
constexpr long SPIN = 1L << 18;
static_assert(D == GW, "one Wo row per wavefront");
static_assert(NB == 64 && NBO == 128, "one (two) block(s) per lane");

typedef unsigned long long tw;

struct AttnWs {
    unsigned abort_tag;                // the tag of a launch that gave up waiting
    alignas(256) tw qkv[NROWS];        // q, k, v
    alignas(256) tw attq[QD / 4];      // the heads' Q8 codes, four per word
    alignas(256) tw atts[QD / 32];     // their block scales
    // phase timestamps of every workgroup (diagnostic, MHIP_DECODE_TRACE)
    unsigned long long trace[NWG][MHIP_ATTN_TRACE_SLOTS];
};

struct AttnArgs {
    const uint8_t *wq, *wk, *wv, *wo;  // Q8_0 rows, 36-byte blocks
    const float *attn_norm, *q_norm, *k_norm;
    const double *rope;                // [max_seq][HD / 2] (cos, sin)
    float *kc, *vc;                    // this layer's cache, [max_seq][KVD]
    float *x;                          // [D], updated in place
    float *x_in, *x_out;               // copies of x before / after (or null)
    AttnWs *ws;
    int *status;                       // abort bits OR'ed in (or null)
    int pos, flags;
    float eps, scale;
    unsigned tag;                      // this launch
};

__device__ __forceinline__ unsigned ld_u(const unsigned *p) {
    return __hip_atomic_load((unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void give_up(const AttnArgs &a, int bit) {
    __hip_atomic_store(&a.ws->abort_tag, a.tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.status) __hip_atomic_fetch_or(a.status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void put_word(tw *p, unsigned v, unsigned tag) {
    __hip_atomic_store(p, ((tw)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The payload of *p once it carries this launch's tag; after SPIN rounds, or
// once the launch has given up, whatever is there.
__device__ __forceinline__ unsigned get_word(const AttnArgs &a, const tw *p) {
    tw v = __hip_atomic_load((tw *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    long s = 0;
    while ((unsigned)(v >> 32) != a.tag) {
        if (++s > SPIN || ((s & 255) == 0 && ld_u(&a.ws->abort_tag) == a.tag)) {
            give_up(a, 2);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        v = __hip_atomic_load((tw *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return (unsigned)v;
}

// One 36-byte block (scale, 32 codes) of a weight row as 9 dwords.
struct Blk {
    float d;
    int4 c0, c1;
};
__device__ __forceinline__ Blk load_blk(const uint8_t *p) {
    const unsigned *u = (const unsigned *)p;
    Blk b;
    b.d = __uint_as_float(u[0]);
    b.c0 = make_int4((int)u[1], (int)u[2], (int)u[3], (int)u[4]);
    b.c1 = make_int4((int)u[5], (int)u[6], (int)u[7], (int)u[8]);
    return b;
}

// DPP moves of the whole wavefront by one lane (lane 0 receives 0, resp.
// lane 63's value).
__device__ __forceinline__ float shr1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x138, 0xf, 0xf, false));
}
__device__ __forceinline__ float ror1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x13C, 0xf, 0xf, false));
}

// forward.c:75-81 over one head's row in LDS, by one wavefront: lane l
// squares elements 2l, 2l+1 in double (exact), a butterfly adds the 128
// squares in some order, and the bracket S -/+ (n + 64) 2^-52 S, which holds
// the reference's index-order sum as well, gives the scale when both ends
// round to the same float; otherwise lane 0 runs the index-order sum
// (head_inv_seq).
__device__ float head_inv_seq(const float *row, float eps);
__device__ __forceinline__ float head_inv_wave(const float *row, float eps, int lane, bool force_seq) {
    const float2 v = *(const float2 *)(row + 2 * lane);
    double ss = (double)v.x * (double)v.x + (double)v.y * (double)v.y;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss = ss + __shfl_xor(ss, o);
    ss = __shfl(ss, 0);
    const double m = ss * ((double)(HD + 64) * 0x1p-52);
    const float lo = (float)(1.0 / sqrt((ss + m) / HD + (double)eps));
    const float hi = (float)(1.0 / sqrt((ss - m) / HD + (double)eps));
    if (lo == hi && !force_seq) return lo;  // the same in every lane
    float r = 0.0f;
    if (lane == 0) r = head_inv_seq(row, eps);
    return __shfl(r, 0);
}
// The index-order sum itself (one lane).
__device__ float head_inv_seq(const float *row, float eps) {
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

struct Lds {
    alignas(16) int8_t xq[D];         // Q8(xn) codes
    alignas(16) int8_t attq[QD];      // the heads' codes
    float xs[NB];
    float atts[NBO];
    alignas(16) float tq[HD], tk[HD], tv[HD], qs[HD], ks[HD];
    alignas(16) float Ks[NPRE][KLD];  // the head's first cache rows
    alignas(16) float Vs[NPRE][HD];
    float red[NW];
    int8_t hq[HD];
    float inv_q, inv_k, sum;
    uint64_t etab[32];
};

// Diagnostic: thread `who` of every workgroup records the 100 MHz real-time
// counter at a phase boundary.
#define ATRACE(slot, who)                                                                   \
    do {                                                                                   \
        if ((a.flags & MHIP_DECODE_TRACE) && tid == (who))                                 \
            a.ws->trace[b][slot] = __builtin_amdgcn_s_memrealtime();                       \
    } while (0)

__global__ __launch_bounds__(NT) void k_attn_layer(AttnArgs a) {
    __shared__ Lds sh;
    extern __shared__ __align__(16) float sc[];  // scores, [pos + 1]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x, gw = b * NW + wave;
    ATRACE(0, 0);

    // Requests in the order they are needed (a CU serves its vector memory
    // requests in order): x and the norm weight (wavefront 0), the residual
    // of this wavefront's Wo row, a head's first cache rows, then the
    // weight rows -- rows gw + GW j of q/k/v (block `lane`) and row gw of Wo
    // (blocks lane, lane + 64) -- which stream in while the norm runs.
    float4 xv4[8], nv4[8];
    if (wave == 0) {
        const float4 *xr = (const float4 *)(a.x + 32 * lane);
        const float4 *nr = (const float4 *)(a.attn_norm + 32 * lane);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            xv4[k] = xr[k];
            nv4[k] = nr[k];
        }
    }
    const float xold = a.x[gw];
    const int npre = min(a.pos, NPRE);
    float4 kp[KPF], vp[KPF];
    // the RoPE angle and norm weights of element i = tid % 64 (threads < 64
    // rotate q, 64..127 k)
    float rw0 = 0.0f, rw1 = 0.0f;
    double rc = 0.0, rs = 0.0;
    if (b < NH && tid < HD) {
        const int i = tid % (HD / 2);
        const float *w = tid < HD / 2 ? a.q_norm : a.k_norm;
        rw0 = w[i];
        rw1 = w[i + HD / 2];
        const double *rp = a.rope + (size_t)a.pos * (HD / 2) * 2;
        rc = rp[2 * i];
        rs = rp[2 * i + 1];
    }
    if (b < NH) {
        const int g = b / GROUP;
#pragma unroll
        for (int j = 0; j < KPF; j++) {
            const int f = tid + NT * j, t = f / (HD / 4), c = f % (HD / 4);
            if (t < npre) {
                kp[j] = *(const float4 *)(a.kc + (size_t)t * KVD + (size_t)g * HD + 4 * c);
                vp[j] = *(const float4 *)(a.vc + (size_t)t * KVD + (size_t)g * HD + 4 * c);
            }
        }
    }
    // (a barrier keeps the other wavefronts' weight rows behind those requests)
    __syncthreads();
    Blk wr[RPW];
#pragma unroll
    for (int j = 0; j < RPW; j++) {
        const int r = min(gw + GW * j, NROWS - 1);  // past the end: a valid row, unused
        const uint8_t *w = r < QD ? a.wq + (size_t)r * NB * 36
                           : r < QD + KVD ? a.wk + (size_t)(r - QD) * NB * 36
                                          : a.wv + (size_t)(r - QD - KVD) * NB * 36;
        wr[j] = load_blk(w + (size_t)lane * 36);
    }
    // (and the q/k/v rows of every wavefront ahead of the Wo rows)
    __syncthreads();
    const uint8_t *wo = a.wo + (size_t)gw * NBO * 36;
    const Blk wo0 = load_blk(wo + (size_t)lane * 36), wo1 = load_blk(wo + (size_t)(lane + 64) * 36);
    // x's copy for a rerun: x is written back (in P4) only by a workgroup
    // whose waits all ended, and then every workgroup has started and read
    // its row and wavefront 0's part of x.
    if (lane == 63 && a.x_in) a.x_in[gw] = xold;
    if (tid < 32) sh.etab[tid] = mia_expf_tab[tid];
    ATRACE(1, 0);
    if (a.flags & MHIP_ATTN_FORCE_ABORT) {
        if (tid == 0) give_up(a, 4);
        return;
    }

    // ---- P1: rmsnorm + Q8(xn), wavefront 0 (k_rmsnorm_q8_w) ----------------------
    if (wave == 0) {
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 q = xv4[k];
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
        const double m = ss * ((double)(D + 64) * 0x1p-52);
        const float lo = (float)(1.0 / sqrt((ss + m) / D + (double)a.eps));
        const float hi = (float)(1.0 / sqrt((ss - m) / D + (double)a.eps));
        float inv = lo;
        if ((a.flags & MHIP_FORCE_SEQ_RMS) || lo != hi) {
            float r = 0.0f;
            if (lane == 0) {
                double sq = 0.0;
                for (int i = 0; i < D; i++) sq = sq + (double)a.x[i] * (double)a.x[i];
                r = (float)(1.0 / sqrt(sq / D + (double)a.eps));
            }
            inv = __shfl(r, 0);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 q = nv4[k];
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
        union {
            int8_t c[32];
            int4 q[2];
        } qc;
#pragma unroll
        for (int k = 0; k < 32; k++) qc.c[k] = (int8_t)roundf(v[k] * qi);
        *(int4 *)&sh.xq[32 * lane] = qc.q[0];
        *(int4 *)&sh.xq[32 * lane + 16] = qc.q[1];
        sh.xs[lane] = dsc;
    }
    __syncthreads();
    ATRACE(2, 0);

    // ---- P2: q/k/v rows (k_rows_q8), the block-order sum lane to lane -------------
    {
        const int4 xa = *(const int4 *)&sh.xq[32 * lane], xb = *(const int4 *)&sh.xq[32 * lane + 16];
        const float dx = sh.xs[lane];
        float t[RPW], s[RPW];
#pragma unroll
        for (int j = 0; j < RPW; j++) {
            t[j] = mhip_dev::block_term(mhip_dev::dot32_i8(wr[j].c0, wr[j].c1, xa, xb), wr[j].d, dx);
            s[j] = 0.0f + t[j];
        }
        for (int k = 1; k < NB; k++) {
#pragma unroll
            for (int j = 0; j < RPW; j++) s[j] = shr1(s[j]) + t[j];
        }
        if (lane == 63) {
#pragma unroll
            for (int j = 0; j < RPW; j++) {
                const int r = gw + GW * j;
                if (r < NROWS) put_word(&a.ws->qkv[r], __float_as_uint(s[j]), a.tag);
            }
        }
    }
    ATRACE(3, 63);

    // ---- P3: query head b (k_attn_head) --------------------------------------------
    if (b < NH) {
        const int h = b, g = h / GROUP, n = a.pos + 1;
        if (tid < HD) sh.tq[tid] = __uint_as_float(get_word(a, &a.ws->qkv[h * HD + tid]));
        else if (tid < 2 * HD) sh.tk[tid - HD] = __uint_as_float(get_word(a, &a.ws->qkv[QD + g * HD + tid - HD]));
        else if (tid < 3 * HD)
            sh.tv[tid - 2 * HD] = __uint_as_float(get_word(a, &a.ws->qkv[QD + KVD + g * HD + tid - 2 * HD]));
#pragma unroll
        for (int j = 0; j < KPF; j++) {
            const int f = tid + NT * j, t = f / (HD / 4), c = f % (HD / 4);
            if (t < npre) {
                *(float4 *)&sh.Ks[t][4 * c] = kp[j];
                *(float4 *)&sh.Vs[t][4 * c] = vp[j];
            }
        }
        __syncthreads();
        ATRACE(4, 0);
        if (wave < 2) {
            const float inv = head_inv_wave(wave == 0 ? sh.tq : sh.tk, a.eps, lane,
                                            (a.flags & MHIP_FORCE_SEQ_RMS) != 0);
            if (lane == 0) (wave == 0 ? sh.inv_q : sh.inv_k) = inv;
        }
        __syncthreads();
        if (tid < HD / 2) head_rope(sh.tq, sh.inv_q, rw0, rw1, rc, rs, sh.qs, tid);
        else if (tid < HD) head_rope(sh.tk, sh.inv_k, rw0, rw1, rc, rs, sh.ks, tid - HD / 2);
        __syncthreads();
        if (h % GROUP == 0 && tid < HD) {
            a.kc[(size_t)a.pos * KVD + (size_t)g * HD + tid] = sh.ks[tid];
            a.vc[(size_t)a.pos * KVD + (size_t)g * HD + tid] = sh.tv[tid];
        }
        // scores (forward.c:143-149): sequential fp32 dots, one position per
        // thread, the key row read 32 values ahead of the additions
        for (int t = tid; t < n; t += NT) {
            const float *kt = t == a.pos ? sh.ks
                              : t < npre ? &sh.Ks[t][0]
                                         : a.kc + (size_t)t * KVD + (size_t)g * HD;
            float dot = 0.0f;
            for (int i = 0; i < HD; i += 32) {
                float4 k4[8];
#pragma unroll
                for (int j = 0; j < 8; j++) k4[j] = *(const float4 *)(kt + i + 4 * j);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    dot = dot + sh.qs[i + 4 * j] * k4[j].x;
                    dot = dot + sh.qs[i + 4 * j + 1] * k4[j].y;
                    dot = dot + sh.qs[i + 4 * j + 2] * k4[j].z;
                    dot = dot + sh.qs[i + 4 * j + 3] * k4[j].w;
                }
            }
            sc[t] = dot * a.scale;
        }
        __syncthreads();
        // softmax (forward.c:150-156): the maximum (order-free), the restated
        // expf, the sequential sum, the division
        float mx = -__builtin_inff();
        for (int t = tid; t < n; t += NT) mx = fmaxf(mx, sc[t]);
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
        if (lane == 0) sh.red[wave] = mx;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; w++) mx = fmaxf(mx, sh.red[w]);
        for (int t = tid; t < n; t += NT) sc[t] = mia_expf_glibc_tab(sc[t] - mx, sh.etab);
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            for (int t = 0; t < n; t++) sum = sum + sc[t];
            sh.sum = sum;
        }
        __syncthreads();
        const float sum = sh.sum;
        for (int t = tid; t < n; t += NT) sc[t] = sc[t] / sum;
        __syncthreads();
        // mix (forward.c:157-162), then Q8 of the head's output (quant.c:11-27)
        if (tid < HD) {
            const float *vt = a.vc + (size_t)g * HD + tid;
            float o = 0.0f;
            int t = 0;
            for (; t < npre; t++) o = o + sc[t] * sh.Vs[t][tid];
            for (; t + 16 <= a.pos; t += 16) {
                float vv[16];
#pragma unroll
                for (int j = 0; j < 16; j++) vv[j] = vt[(size_t)(t + j) * KVD];
#pragma unroll
                for (int j = 0; j < 16; j++) o = o + sc[t + j] * vv[j];
            }
            for (; t < a.pos; t++) o = o + sc[t] * vt[(size_t)t * KVD];
            o = o + sc[a.pos] * sh.tv[tid];
            float am = fmaxf(0.0f, fabsf(o));
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) am = fmaxf(am, __shfl_xor(am, m, 32));
            const float d = am / 127.0f;
            const float qi = d != 0.0f ? 1.0f / d : 0.0f;
            sh.hq[tid] = (int8_t)roundf(o * qi);
            if ((lane & 31) == 0) put_word(&a.ws->atts[h * (HD / 32) + tid / 32], __float_as_uint(d), a.tag);
        }
        __syncthreads();
        if (tid < HD / 4) put_word(&a.ws->attq[h * (HD / 4) + tid], ((const unsigned *)sh.hq)[tid], a.tag);
        ATRACE(5, 0);
    }

    // ---- P4: Wo row gw over the heads' codes, plus the residual --------------------
    {
        for (int i = tid; i < QD / 4; i += NT) ((unsigned *)sh.attq)[i] = get_word(a, &a.ws->attq[i]);
        if (tid < NBO) sh.atts[tid] = __uint_as_float(get_word(a, &a.ws->atts[tid]));
        __syncthreads();
        ATRACE(6, 0);
        const int4 *q0 = (const int4 *)&sh.attq[32 * lane], *q1 = (const int4 *)&sh.attq[32 * (lane + 64)];
        const float t0 = mhip_dev::block_term(mhip_dev::dot32_i8(wo0.c0, wo0.c1, q0[0], q0[1]), wo0.d,
                                              sh.atts[lane]);
        const float t1 = mhip_dev::block_term(mhip_dev::dot32_i8(wo1.c0, wo1.c1, q1[0], q1[1]), wo1.d,
                                              sh.atts[lane + 64]);
        // blocks 0..63 (t0 of lanes 0..63), then 64..127 (t1), in order
        float s = 0.0f + t0;
        for (int k = 1; k < 64; k++) s = ror1(s) + t0;
        for (int k = 0; k < 64; k++) s = ror1(s) + t1;
        // an aborted launch leaves x as it was
        if (lane == 63 && ld_u(&a.ws->abort_tag) != a.tag) {
            const float xn = xold + s;
            a.x[gw] = xn;
            if (a.x_out) a.x_out[gw] = xn;
        }
        ATRACE(7, 63);
    }
}

int g_lds_set[64];  // per device ordinal: the dynamic-LDS attribute is set

}  // namespace

extern "C" {

size_t mhip_attention_layer_ws_bytes(void) { return (sizeof(AttnWs) + 255) / 256 * 256; }

int mhip_attention_layer_trace(mhip_ctx *c, const void *d_ws, unsigned long long *out) {
    return mhip_d2h(c, out, ((const AttnWs *)d_ws)->trace, sizeof(((AttnWs *)nullptr)->trace));
}

int mhip_attention_layer_supported(mhip_ctx *c, const mhip_attn_dims *s, int max_seq) {
    if (!s || mhip::use_device(c)) return -1;
    if (s->dim != D || s->n_heads != NH || s->n_kv_heads != NKV || s->head_dim != HD) return 0;
    if (max_seq <= 0 || sizeof(Lds) + (size_t)max_seq * 4 > 150 * 1024) return 0;
    hipDeviceProp_t prop;
    if (mhip::check(c, hipGetDeviceProperties(&prop, c->device), "hipGetDeviceProperties"))
        return -1;
    if (prop.multiProcessorCount != NWG) return 0;
    int occ = 0;
    if (mhip::check(c,
                    hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_attn_layer, NT,
                                                                 (size_t)max_seq * 4),
                    "occupancy"))
        return -1;
    return occ >= 1 ? 1 : 0;
}

int mhip_attention_layer(mhip_ctx *c, const mhip_attn_dims *s, const float *d_attn_norm,
                         const void *d_wq, const void *d_wk, const void *d_wv, const void *d_wo,
                         const float *d_q_norm, const float *d_k_norm, const double *d_rope,
                         float *d_kc, float *d_vc, int pos, int max_seq, float *d_x,
                         float *d_x_in, float *d_x_out, void *d_ws, int *d_status, int flags) {
    if (!s || s->dim != D || s->n_heads != NH || s->n_kv_heads != NKV || s->head_dim != HD)
        return mhip::fail(c, "attention layer: shape not supported (dim 2048, 32/4 heads of 128)");
    if (pos < 0 || pos >= max_seq)
        return mhip::fail(c, "attention layer: pos=%d outside [0, max_seq=%d)", pos, max_seq);
    if ((uintptr_t)d_ws % 256)
        return mhip::fail(c, "attention layer: workspace %p is not 256-byte aligned", d_ws);
    if (mhip::use_device(c)) return -1;
    const size_t dyn = (size_t)max_seq * 4;
    if (sizeof(Lds) + dyn > 150 * 1024)
        return mhip::fail(c, "attention layer: max_seq=%d needs too much LDS", max_seq);
    if (c->device >= 0 && c->device < 64 && !g_lds_set[c->device]) {
        if (mhip::check(c, hipFuncSetAttribute((const void *)k_attn_layer,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)(150 * 1024 - sizeof(Lds))),
                        "attention layer LDS attribute"))
            return -1;
        g_lds_set[c->device] = 1;
    }
    // A workspace this context has not used last starts cleared; so does one
    // whose tags would leave 24 bits.
    if (d_ws != c->attn_ws || c->attn_epoch >= (1u << 23)) {
        if (mhip_zero(c, d_ws, mhip_attention_layer_ws_bytes())) return -1;
        c->attn_epoch = 0;
        c->attn_ws = d_ws;
    }
    AttnArgs a;
    a.wq = (const uint8_t *)d_wq;
    a.wk = (const uint8_t *)d_wk;
    a.wv = (const uint8_t *)d_wv;
    a.wo = (const uint8_t *)d_wo;
    a.attn_norm = d_attn_norm;
    a.q_norm = d_q_norm;
    a.k_norm = d_k_norm;
    a.rope = d_rope;
    a.kc = d_kc;
    a.vc = d_vc;
    a.x = d_x;
    a.x_in = d_x_in;
    a.x_out = d_x_out;
    a.ws = (AttnWs *)d_ws;
    a.status = d_status;
    a.pos = pos;
    a.flags = flags;
    a.eps = s->norm_eps;
    a.scale = 1.0f / sqrtf((float)HD);
    a.tag = c->attn_epoch + 1;
    k_attn_layer<<<NWG, NT, dyn, c->stream>>>(a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return mhip::check(c, e, "attention layer launch");
    c->attn_epoch++;
    return 0;
}

}  // extern "C"
