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
#include "attn_common.h"

namespace {

using namespace mhip_attn;

constexpr int NWG = 256;
constexpr int GW = NWG * NW;                  // 2048 wavefronts
constexpr int RPW = (NROWS + GW - 1) / GW;    // at most 3 q/k/v rows per wavefront
constexpr long SPIN = 1L << 18;
constexpr int NPRE = 64;                      // cache positions a head stages in LDS
static_assert(D == GW, "one Wo row per wavefront");

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

struct Lds {
    alignas(16) int8_t xq[D];         // Q8(xn) codes
    alignas(16) int8_t attq[QD];      // the heads' codes
    float xs[NB];
    float atts[NBO];
    HeadLds<NPRE> head;               // the query head of workgroups 0..NH-1
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
    HeadPre<NPRE> hp;
    if (b < NH)
        head_prefetch(hp, sh.head, b, a.pos, glob((const float *)a.kc), glob((const float *)a.vc),
                      glob(a.q_norm), glob(a.k_norm), glob(a.rope), tid);
    // (a barrier keeps the other wavefronts' weight rows behind those requests)
    __syncthreads();
    Blk wr[RPW];
#pragma unroll
    for (int j = 0; j < RPW; j++) {
        const int r = min(gw + GW * j, NROWS - 1);  // past the end: a valid row, unused
        const uint8_t *w = r < QD ? a.wq + (size_t)r * NB * 36
                           : r < QD + KVD ? a.wk + (size_t)(r - QD) * NB * 36
                                          : a.wv + (size_t)(r - QD - KVD) * NB * 36;
        wr[j] = load_blk(glob(w + (size_t)lane * 36));
    }
    // (and the q/k/v rows of every wavefront ahead of the Wo rows)
    __syncthreads();
    // This wavefront's Wo row is requested once its q/k/v rows are out (in
    // a head's workgroup once the head is done): the q/k/v rows, on the
    // critical path, then do not share HBM with the Wo rows.
    const uint8_t *wo = a.wo + (size_t)gw * NBO * 36;
    Blk wo0, wo1;
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
    if (b >= NH) {
        wo0 = load_blk(glob(wo + (size_t)lane * 36));
        wo1 = load_blk(glob(wo + (size_t)(lane + 64) * 36));
    }

    // ---- P3: query head b (k_attn_head) --------------------------------------------
    if (b < NH) {
        const int h = b, g = h / GROUP;
        if (tid < HD) sh.head.tq[tid] = __uint_as_float(get_word(a, &a.ws->qkv[h * HD + tid]));
        else if (tid < 2 * HD)
            sh.head.tk[tid - HD] = __uint_as_float(get_word(a, &a.ws->qkv[QD + g * HD + tid - HD]));
        else if (tid < 3 * HD)
            sh.head.tv[tid - 2 * HD] =
                __uint_as_float(get_word(a, &a.ws->qkv[QD + KVD + g * HD + tid - 2 * HD]));
        ATRACE(4, 0);
        head_run(sh.head, sc, hp, h, a.pos, glob(a.kc), glob(a.vc), a.eps, a.scale,
                 (a.flags & MHIP_FORCE_SEQ_RMS) != 0, sh.etab);
        if (tid < HD / 32) put_word(&a.ws->atts[h * (HD / 32) + tid], __float_as_uint(sh.head.dsc[tid]), a.tag);
        if (tid < HD / 4) put_word(&a.ws->attq[h * (HD / 4) + tid], ((const unsigned *)sh.head.hq)[tid], a.tag);
        wo0 = load_blk(glob(wo + (size_t)lane * 36));
        wo1 = load_blk(glob(wo + (size_t)(lane + 64) * 36));
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
