// The token sampler on device logits: mia_sample of the reference
// (src/tokenizer/sampler.c:33-66) with the same picks.
//
//   greedy:  the first maximum (k_argmax_part / k_argmax_final; NaN never
//            wins except at index 0, as the reference's strict comparison)
//   else:    e_i = expf((l_i - l_best) / T)            (k_sample_exp)
//            sum = e_0 + e_1 + ... in index order       (k_chain_sum)
//            candidates p_i = e_i / sum >= cutoff as 64-bit keys
//            (descending p, ascending index), sorted    (k_sample_keys, rocPRIM)
//            the running sum of the sorted p up to top_p, r = u * cum, the
//            first candidate whose running sum exceeds r (k_sample_pick)
//
// The running sums are fp32 chains in a fixed order, as the reference adds
// them. They are computed exactly but not one addition at a time: while a
// running sum stays inside one binade every addition adds a whole number of
// that binade's ulps, so a workgroup turns 8192 additions at a time into an
// integer prefix sum and walks only the few additions that leave the binade
// (seq_scan). Everything else is parallel.
#include <rocprim/device/device_radix_sort.hpp>

#include "mhip_internal.h"

namespace {

constexpr int NT = 256;          // threads of every sampler kernel
constexpr int PARTS = 256;       // workgroups of the argmax's first pass
constexpr uint64_t NONE = ~0ull; // key of a dropped token

struct SampleState {
    int best;
    float sum;
    int token;
    int last;
    float cum;
};

struct Best {
    float v;
    int i;  // -1: no non-NaN value seen
};

// The better of two candidates from disjoint index ranges: the larger value,
// the lower index among equal values (+0 and -0 are equal).
__device__ __forceinline__ Best better(Best a, Best b) {
    if (b.i < 0) return a;
    if (a.i < 0) return b;
    if (b.v > a.v) return b;
    if (a.v > b.v) return a;
    return b.i < a.i ? b : a;
}

__device__ Best block_best(Best m, Best *sh) {
    const int tid = threadIdx.x;
    sh[tid] = m;
    __syncthreads();
    for (int o = NT / 2; o > 0; o >>= 1) {
        if (tid < o) sh[tid] = better(sh[tid], sh[tid + o]);
        __syncthreads();
    }
    return sh[0];
}

__global__ __launch_bounds__(NT) void k_argmax_part(const float *__restrict__ l, int n,
                                                    Best *__restrict__ part) {
    __shared__ Best sh[NT];
    Best m = {0.0f, -1};
    for (int i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT) {
        const float v = l[i];
        if (v == v && (m.i < 0 || v > m.v)) m = {v, i};  // indices rise: ties keep the first
    }
    m = block_best(m, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// sampler.c:34-37: best = 0, replaced by every later index whose value is
// strictly larger. With l[0] NaN nothing is larger; otherwise that is the
// first maximum of the non-NaN values.
__global__ __launch_bounds__(NT) void k_argmax_final(const float *__restrict__ l,
                                                     const Best *__restrict__ part, int nparts,
                                                     SampleState *st, int *token) {
    __shared__ Best sh[NT];
    Best m = {0.0f, -1};
    for (int p = threadIdx.x; p < nparts; p += NT) m = better(m, part[p]);
    m = block_best(m, sh);
    if (threadIdx.x == 0) {
        const float l0 = l[0];
        const int best = (l0 != l0 || m.i < 0) ? 0 : m.i;
        st->best = best;
        if (token) *token = best;
    }
}

// sampler.c:41-44, the exponentials (the sum is k_chain_sum's).
__global__ __launch_bounds__(NT) void k_sample_exp(const float *__restrict__ l, int n,
                                                   float temperature,
                                                   const SampleState *__restrict__ st,
                                                   float *__restrict__ e) {
    __shared__ uint64_t etab[32];
    if (threadIdx.x < 32) etab[threadIdx.x] = mia_expf_tab[threadIdx.x];
    __syncthreads();
    const float mx = l[st->best];
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < n) e[i] = mia_expf_glibc_tab((l[i] - mx) / temperature, etab);
}

// ---- exact running sums, 8192 additions at a time -------------------------------
//
// The chains s_0 = 0, s_{k+1} = fl(s_k + v_k) over v_k >= 0 (sampler.c:43,
// 55, 64). Let s lie on the grid of spacing u = 2^(P-23) below 2^(P+1):
// the binade [2^P, 2^(P+1)) for P >= -126, together with the subnormals for
// P = -126 (spacing 2^-149 below 2^-125). Then s = M u with an integer
// M < 2^24, and while s + v stays below 2^(P+1) - u/2 the rounded sum is
// u (M + n) with n the integer nearest to v / u: every value of the grid
// below 2^(P+1) is representable, and only an exact half (a tie, broken
// towards an even M + n) makes the result depend on M. So as long as
// M + n_0 + ... + n_j <= 2^24 - 1 (and no v_j / u is a tie), the chain's
// values are u times an integer prefix sum. The workgroup holds a window
// of SQ_W values (SQ_V consecutive per thread), forms every n_j and their
// prefix sums, and finds the first element at which the chain leaves the
// binade, meets a tie or a value that is not a finite v >= 0, or makes
// the caller's predicate true; that one addition is done in fp32 by its
// thread, the grid is taken from the new s, and the window goes on after
// it, first over its next SQ_SHORT values only (exits come in bursts while
// the sum is small; a short pass costs the waves that hold those values),
// then over the rest. Ties, exits from a binade (at most one per binade the
// sum passes through) and the stop are the only additions done one at a
// time. The prefix sums are fp32 sums of whole numbers: exact below 2^24,
// and at least 2^24 when the exact sum is, which is all the test needs (an
// n too large for the binade is entered as 2^25). A chain that becomes
// infinite, NaN or negative finishes one addition at a time on one lane.
constexpr int SQ_T = 1024, SQ_V = 8, SQ_W = SQ_T * SQ_V, SQ_SHORT = 1024;
constexpr float SQ_TOP = 16777216.0f;  // 2^24: a mantissa at or above it left the binade
constexpr int SQ_PF = 2;               // windows loaded ahead
constexpr size_t SQ_LDS = (size_t)(SQ_PF + 1) * SQ_W * sizeof(float);  // the window ring

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes from global memory straight into LDS at lds + 16 * lane.
__device__ __forceinline__ void sq_dma16(unsigned lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
enum { SQ_SUM = 0, SQ_GE = 1, SQ_GT = 2 };

template <int MODE>
__device__ __forceinline__ bool sq_pred(float s, float thr) {
    return MODE == SQ_GE ? s >= thr : MODE == SQ_GT ? thr < s : false;
}

// The grid of s >= 0 finite: P with s = M 2^(P-23), M an integer < 2^24.
__device__ __forceinline__ int sq_grid(float s) {
    return s >= 0x1p-126f ? ilogbf(s) : -126;
}

// Runs the chain over v[0 .. n) (16-byte aligned) on a workgroup of SQ_T
// threads, every thread calling. Returns the index of the first element
// after whose addition MODE's predicate holds (n if none) and leaves in *s
// the chain's value after that addition (after all n if none).
template <int MODE>
__device__ int seq_scan(const float *__restrict__ v, int n, float thr, float *s_out) {
    __shared__ float wtot[2][SQ_T / 64];
    __shared__ int wstop[2][SQ_T / 64];
    __shared__ float s1_sh[2];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int P = -126;
    float M = 0.0f;       // s = M 2^(P-23) = 0
    int lo = 0;           // the chain has added v[0 .. lo)
    int it = 0;           // parity of the LDS buffers
    float s = 0.0f;
    int stop = n;
    bool seq = false;     // the chain left the finite non-negative values
    const int nw = (n + SQ_W - 1) / SQ_W;
    // Windows stream into an LDS ring of SQ_PF + 1 windows, SQ_PF ahead,
    // straight from global memory (thread t's values land where it reads
    // them: load q of a wavefront puts lane l's 16 bytes at 16 l); every
    // load is a whole 16-byte vector at an in-range index (the last one
    // reaches up to 3 values past n: callers pad to a multiple of 4), and
    // values past n are zeroed when a window is taken.
    extern __shared__ __align__(16) float sq_ring[];
    const unsigned ring = (unsigned)(uintptr_t)sq_ring;
    const int nl = n > 4 ? (n - 1) & ~3 : 0;
    auto issue = [&](int w) {
        const int i0 = w * SQ_W + SQ_V * tid;
        const unsigned st = ring + (unsigned)(((w % (SQ_PF + 1)) * SQ_W + SQ_V * 64 * wave) * 4);
#pragma unroll
        for (int q = 0; q < SQ_V / 4; q++)
            sq_dma16(st + (unsigned)(q * 64 * 16), v + min(i0 + 4 * q, nl));
    };
    if (n > 0) {
#pragma unroll
        for (int q = 0; q < SQ_PF; q++) issue(q);
    }
    bool short_pass = false;
    for (int w = 0; w < nw && stop == n && !seq; w++) {
        // this wavefront's loads of window w are in (later ones may not be)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((SQ_PF - 1) * (SQ_V / 4)) : "memory");
        const int base = w * SQ_W + SQ_V * tid;
        float x[SQ_V];
        {
            const float4 *src = (const float4 *)(sq_ring + (w % (SQ_PF + 1)) * SQ_W + SQ_V * 64 * wave) + lane;
#pragma unroll
            for (int q = 0; q < SQ_V / 4; q++) {
                const float4 r = src[64 * q];
                x[4 * q] = base + 4 * q < n ? r.x : 0.0f;
                x[4 * q + 1] = base + 4 * q + 1 < n ? r.y : 0.0f;
                x[4 * q + 2] = base + 4 * q + 2 < n ? r.z : 0.0f;
                x[4 * q + 3] = base + 4 * q + 3 < n ? r.w : 0.0f;
            }
        }
        // window w + SQ_PF goes into the stage of window w - 1 (read before)
        issue(w + SQ_PF);
        const int wend = min(w * SQ_W + SQ_W, n);
        const int wbase = w * SQ_W + SQ_V * 64 * wave;  // this wavefront's values
        for (;;) {
            const int hi = short_pass ? min(lo + SQ_SHORT, wend) : wend;
            // a wavefront with none of [lo, hi) skips the element work
            const bool busy = wbase + SQ_V * 64 > lo && wbase < hi;
            const float lim = ldexpf(1.0f, P + 1);
            float L[SQ_V];
            bool sp[SQ_V];
            float run = 0.0f;
            if (busy) {
#pragma unroll
                for (int e = 0; e < SQ_V; e++) {
                    const int i = base + e;
                    const float xv = x[e];
                    float k = 0.0f;
                    bool special = false;
                    if (i >= lo && i < hi) {
                        if (!(xv >= 0.0f) || xv == __builtin_inff()) {
                            special = true;  // NaN, infinite or negative
                        } else if (xv >= lim) {
                            k = 2.0f * SQ_TOP;  // leaves the binade
                        } else {
                            const float t = ldexpf(xv, 23 - P);  // < 2^24, exact
                            k = rintf(t);
                            special = t - truncf(t) == 0.5f;  // a tie
                        }
                    }
                    sp[e] = special;
                    run = run + k;
                    L[e] = run;
                }
            }
            // exclusive prefix of the thread totals over the workgroup
            float incl = run;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const float y = __shfl_up(incl, o);
                if (lane >= o) incl = incl + y;
            }
            const float up = __shfl_up(incl, 1);
            const float exw = lane > 0 ? up : 0.0f;
            if (lane == 63) wtot[it][wave] = incl;
            __syncthreads();
            float before = 0.0f, total = 0.0f;
#pragma unroll
            for (int k = 0; k < SQ_T / 64; k++) {
                const float t = wtot[it][k];
                if (k < wave) before = before + t;
                total = total + t;
            }
            const float ex = M + (before + exw);
            // the first element that leaves the binade, is special or stops
            int first = SQ_V;
            if (busy) {
#pragma unroll
                for (int e = SQ_V - 1; e >= 0; e--) {
                    const float Me = ex + L[e];
                    bool st = sp[e] || Me >= SQ_TOP;
                    if (MODE != SQ_SUM && !st && base + e >= lo && base + e < hi)
                        st = sq_pred<MODE>(ldexpf(Me, P - 23), thr);
                    if (st) first = e;
                }
            }
            const unsigned long long b = __ballot(first < SQ_V);
            if (lane == (b ? __ffsll((long long)b) - 1 : 0))
                wstop[it][wave] = b ? SQ_V * tid + first : SQ_W;
            __syncthreads();
            int f = SQ_W;
#pragma unroll
            for (int k = 0; k < SQ_T / 64; k++) f = min(f, wstop[it][k]);
            it ^= 1;
            if (f == SQ_W) {  // [lo, hi) stays in the binade
                M = M + total;
                s = ldexpf(M, P - 23);
                lo = hi;
                short_pass = false;
                if (hi == wend) break;
                continue;
            }
            // element f: its thread adds it in fp32
            if (tid == f / SQ_V) {
                const int e = f % SQ_V;
                float Lp = 0.0f;
#pragma unroll
                for (int q = 0; q < SQ_V; q++)
                    if (q < e) Lp = L[q];
                float xe = x[0];
#pragma unroll
                for (int q = 1; q < SQ_V; q++)
                    if (q == e) xe = x[q];
                s1_sh[it ^ 1] = ldexpf(ex + Lp, P - 23) + xe;
            }
            __syncthreads();
            s = s1_sh[it ^ 1];
            const int fi = w * SQ_W + f;
            lo = fi + 1;
            short_pass = true;
            if (MODE != SQ_SUM && sq_pred<MODE>(s, thr)) {
                stop = fi;
                break;
            }
            if (!(s >= 0.0f) || s == __builtin_inff()) {
                seq = true;
                break;
            }
            P = sq_grid(s);
            M = ldexpf(s, 23 - P);
            if (lo == wend) break;
        }
    }
    if (seq) {  // the rest one addition at a time (NaN, infinite or negative sums)
        if (tid == 0) {
            int i = lo;
            for (; i < n; i++) {
                s = s + v[i];
                if (MODE != SQ_SUM && sq_pred<MODE>(s, thr)) break;
            }
            s1_sh[0] = s;
            wstop[0][0] = i;
        }
        __syncthreads();
        s = s1_sh[0];
        stop = MODE == SQ_SUM ? n : wstop[0][0];
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the loads past the end
    *s_out = s;
    return stop;
}

// sampler.c:43: sum = e_0 + e_1 + ... + e_{n-1} (fp32, index order).
__global__ __launch_bounds__(SQ_T) void k_chain_sum(const float *__restrict__ e, int n,
                                                    SampleState *st) {
    float s;
    seq_scan<SQ_SUM>(e, n, 0.0f, &s);
    if (threadIdx.x == 0) st->sum = s;
}

// sampler.c:46-51: p_i = e_i / sum; a candidate when p_i >= cutoff, as the
// key (0x7fffffff - bits(p)) << 32 | i: ascending keys are descending p, and
// ascending index among equal p (bits of p >= 0 order as p does).
__global__ __launch_bounds__(NT) void k_sample_keys(const float *__restrict__ e, int n,
                                                    float cutoff,
                                                    const SampleState *__restrict__ st,
                                                    uint64_t *__restrict__ keys) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i >= n) return;
    const float p = e[i] / st->sum;
    keys[i] = p >= cutoff
                  ? ((uint64_t)(0x7fffffffu - __float_as_uint(p)) << 32) | (uint32_t)i
                  : NONE;
}

__device__ __forceinline__ float key_p(uint64_t k) {
    return __uint_as_float(0x7fffffffu - (uint32_t)(k >> 32));
}

// The sorted keys as probabilities pf[] and token ids pi[]; the candidates
// are the keys before the first NONE: their count goes to st->last (as
// m - 1, the default last candidate).
__global__ __launch_bounds__(NT) void k_keys_split(const uint64_t *__restrict__ keys, int n,
                                                   float *__restrict__ pf, int *__restrict__ pi,
                                                   SampleState *st) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i >= n) return;
    const uint64_t k = keys[i];
    if (k == NONE) {
        if (i == 0) st->last = -1;
        return;
    }
    pf[i] = key_p(k);
    pi[i] = (int)(uint32_t)k;
    if (i + 1 == n || keys[i + 1] == NONE) st->last = i;
}

// sampler.c:53-66 on the m candidates (pf, pi; m - 1 in st->last): cum =
// p_0 + p_1 + ... until cum >= top_p (last = that candidate) or the
// candidates end; r = u * cum; the pick is the first candidate up to last
// whose running sum (the same additions from 0) exceeds r, else last.
__global__ __launch_bounds__(SQ_T) void k_sample_pick(const float *__restrict__ pf,
                                                      const int *__restrict__ pi, float top_p,
                                                      float u, SampleState *st, int *token) {
    const int m = st->last + 1;
    if (m == 0) {  // no candidate
        if (threadIdx.x == 0) *token = st->best;
        return;
    }
    float cum;
    const int j = seq_scan<SQ_GE>(pf, m, top_p, &cum);
    const int last = j < m ? j : m - 1;
    const float r = u * cum;
    float acc;
    const int k = seq_scan<SQ_GT>(pf, last + 1, r, &acc);
    if (threadIdx.x == 0) {
        st->cum = cum;
        st->last = last;
        *token = pi[k <= last ? k : last];
    }
}

template <int MODE>
__global__ __launch_bounds__(SQ_T) void k_chain(const float *__restrict__ v, int n, float thr,
                                                int *__restrict__ out) {
    float s;
    const int k = seq_scan<MODE>(v, n, thr, &s);
    if (threadIdx.x == 0) {
        out[0] = __float_as_int(s);
        out[1] = k;
    }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// The LDS ring of the running-sum kernels is above the default limit.
int sq_lds_attr(mhip_ctx *c) {
    const void *fns[] = {(const void *)k_chain_sum, (const void *)k_sample_pick,
                         (const void *)k_chain<SQ_SUM>, (const void *)k_chain<SQ_GE>,
                         (const void *)k_chain<SQ_GT>};
    for (const void *f : fns)
        if (mhip::check(c, hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)SQ_LDS),
                        "sampler LDS attribute"))
            return -1;
    return 0;
}

struct SampleScratch {
    SampleState *st;
    Best *part;
    float *e;
    uint64_t *kin, *kout;
    void *tmp;
    size_t tmp_bytes;
};

size_t sort_bytes(int n) {
    size_t b = 0;
    if (rocprim::radix_sort_keys(nullptr, b, (const uint64_t *)nullptr, (uint64_t *)nullptr,
                                 (unsigned)n, 0, 64) != hipSuccess)
        return 0;
    return b;
}

SampleScratch carve(int n, void *base) {
    uint8_t *p = (uint8_t *)base;
    SampleScratch s;
    s.st = (SampleState *)p;
    p += align256(sizeof(SampleState));
    s.part = (Best *)p;
    p += align256(sizeof(Best) * PARTS);
    s.e = (float *)p;
    p += align256((size_t)n * 4);
    s.kin = (uint64_t *)p;
    p += align256((size_t)n * 8);
    s.kout = (uint64_t *)p;
    p += align256((size_t)n * 8);
    s.tmp = p;
    s.tmp_bytes = sort_bytes(n);
    return s;
}

// sampler.c:20-25: xorshift64* (shifts 12, 25, 27; multiplier
// 2685821657736338717), its top 24 bits over 2^24.
float rand01(mhip_sampler *s) {
    uint64_t x = s->rng;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    s->rng = x;
    return (float)((x * 0x2545F4914F6CDD1DULL) >> 40) / 16777216.0f;
}

}  // namespace

extern "C" {

void mhip_sampler_init(mhip_sampler *s, float temperature, float top_p, int n, uint64_t seed) {
    s->temperature = temperature;
    s->top_p = (top_p > 0.0f && top_p <= 1.0f) ? top_p : 1.0f;
    s->n = n;
    s->rng = seed ? seed : 0x2545F4914F6CDD1DULL;
}

size_t mhip_sample_scratch_bytes(int n) {
    if (n < 1 || n > MHIP_SAMPLE_MAX_N) return 0;
    const size_t sb = sort_bytes(n);
    if (!sb) return 0;
    return align256(sizeof(SampleState)) + align256(sizeof(Best) * PARTS) +
           align256((size_t)n * 4) + 2 * align256((size_t)n * 8) + align256(sb);
}

int mhip_sample(mhip_ctx *c, mhip_sampler *s, const float *d_logits, void *d_scratch,
                int *d_token) {
    const int n = s ? s->n : 0;
    if (!s || n < 1 || n > MHIP_SAMPLE_MAX_N)
        return mhip::fail(c, "sampler: n=%d outside [1, %d]", n, MHIP_SAMPLE_MAX_N);
    if (!d_logits || !d_scratch || !d_token) return mhip::fail(c, "sampler: null pointer");
    if (mhip::use_device(c)) return -1;
    SampleScratch sc = carve(n, d_scratch);
    if (!sc.tmp_bytes) return mhip::fail(c, "sampler: sort workspace query failed");
    hipStream_t st = c->stream;
    const int greedy = s->temperature <= 0.0f;
    const unsigned parts = std::min<unsigned>(PARTS, mhip::blocks_for(n, NT));
    k_argmax_part<<<parts, NT, 0, st>>>(d_logits, n, sc.part);
    k_argmax_final<<<1, NT, 0, st>>>(d_logits, sc.part, parts, sc.st, greedy ? d_token : nullptr);
    if (greedy) return mhip::check_launch(c, "sampler (greedy)");
    // the host-side draw and cutoff, in the reference's order (sampler.c:47,63)
    const float u = rand01(s);
    const float cutoff = (1.0f - s->top_p) / (float)(n > 1 ? n - 1 : 1);
    const unsigned nb = mhip::blocks_for(n, NT);
    k_sample_exp<<<nb, NT, 0, st>>>(d_logits, n, s->temperature, sc.st, sc.e);
    if (sq_lds_attr(c)) return -1;
    k_chain_sum<<<1, SQ_T, SQ_LDS, st>>>(sc.e, n, sc.st);
    k_sample_keys<<<nb, NT, 0, st>>>(sc.e, n, cutoff, sc.st, sc.kin);
    if (mhip::check_launch(c, "sampler")) return -1;
    size_t tb = sc.tmp_bytes;
    if (mhip::check(c, rocprim::radix_sort_keys(sc.tmp, tb, sc.kin, sc.kout, (unsigned)n, 0, 64, st),
                    "sampler sort"))
        return -1;
    float *pf = (float *)sc.kin;  // the unsorted keys are dead after the sort
    int *pi = (int *)sc.kin + n;
    k_keys_split<<<nb, NT, 0, st>>>(sc.kout, n, pf, pi, sc.st);
    k_sample_pick<<<1, SQ_T, SQ_LDS, st>>>(pf, pi, s->top_p, u, sc.st, d_token);
    return mhip::check_launch(c, "sampler pick");
}

int mhip_chain_f32(mhip_ctx *c, const float *d_v, int n, int mode, float thr, int *d_out) {
    if (n < 0 || !d_out || (n > 0 && !d_v)) return mhip::fail(c, "chain: bad arguments (n=%d)", n);
    if ((uintptr_t)d_v % 16) return mhip::fail(c, "chain: d_v is not 16-byte aligned");
    if (mode != MHIP_CHAIN_SUM && mode != MHIP_CHAIN_GE && mode != MHIP_CHAIN_GT)
        return mhip::fail(c, "chain: mode %d", mode);
    if (mhip::use_device(c)) return -1;
    if (sq_lds_attr(c)) return -1;
    hipStream_t st = c->stream;
    if (mode == MHIP_CHAIN_SUM)
        k_chain<SQ_SUM><<<1, SQ_T, SQ_LDS, st>>>(d_v, n, thr, d_out);
    else if (mode == MHIP_CHAIN_GE)
        k_chain<SQ_GE><<<1, SQ_T, SQ_LDS, st>>>(d_v, n, thr, d_out);
    else
        k_chain<SQ_GT><<<1, SQ_T, SQ_LDS, st>>>(d_v, n, thr, d_out);
    return mhip::check_launch(c, "chain");
}

}  // extern "C"
