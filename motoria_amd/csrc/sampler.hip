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
// The two running sums are fp32 chains in a fixed order, as the reference
// adds them; one lane adds while the other waves of the workgroup stage
// the next chunk into LDS. Everything else is parallel.
#include <rocprim/device/device_radix_sort.hpp>

#include "mhip_internal.h"

namespace {

constexpr int NT = 256;          // threads of every sampler kernel
constexpr int PARTS = 256;       // workgroups of the argmax's first pass
constexpr int CH = 2048;         // chain chunk (values per LDS stage)
constexpr int MAXCH = 1024;      // chunks the pick records (n <= 2M)
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

// Copies values [base, base + CH) of src (those below n) into an LDS chunk,
// `nthr` threads numbered from 0.
template <typename V>
__device__ __forceinline__ void stage_chunk(V *dst, const V *__restrict__ src, int base, int n,
                                            int t, int nthr) {
    for (int j = t; j < CH; j += nthr)
        if (base + j < n) dst[j] = src[base + j];
}

// s + v[0] + v[1] + ... + v[len-1], one addition at a time.
__device__ __forceinline__ float chain_add(const float *v, int len, float s) {
    int j = 0;
    for (; j + 64 <= len; j += 64) {
        float4 q[16];
        const float4 *p = (const float4 *)(v + j);
#pragma unroll
        for (int k = 0; k < 16; k++) q[k] = p[k];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            s = s + q[k].x;
            s = s + q[k].y;
            s = s + q[k].z;
            s = s + q[k].w;
        }
    }
    for (; j < len; j++) s = s + v[j];
    return s;
}

// sampler.c:43: sum = e_0 + e_1 + ... + e_{n-1} (fp32, index order). Lane 0
// of wave 0 adds chunk c while waves 1-3 stage chunk c + 1.
__global__ __launch_bounds__(NT) void k_chain_sum(const float *__restrict__ e, int n,
                                                  SampleState *st) {
    __shared__ __align__(16) float buf[2][CH];
    const int tid = threadIdx.x;
    const int nch = (n + CH - 1) / CH;
    stage_chunk(buf[0], e, 0, n, tid, NT);
    __syncthreads();
    float s = 0.0f;
    for (int c = 0; c < nch; c++) {
        if (tid >= 64) {
            if (c + 1 < nch) stage_chunk(buf[(c + 1) & 1], e, (c + 1) * CH, n, tid - 64, NT - 64);
        } else if (tid == 0) {
            s = chain_add(buf[c & 1], min(CH, n - c * CH), s);
        }
        __syncthreads();
    }
    if (tid == 0) st->sum = s;
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

// Adds v[0], v[1], ... (at most len) to s one at a time and stops after the
// first addition that makes pred(s) true: returns that element's index (s
// then holds the sum through it), or len (s the sum of all). pred is
// monotone in s and every v >= 0, so a batch whose total leaves pred false
// holds no stopping point; only the batch where it turns true is walked
// element by element.
template <class P>
__device__ __forceinline__ int chain_until(const float *v, int len, float &s, P pred) {
    int j = 0;
    for (; j + 64 <= len; j += 64) {
        float4 q[16];
        const float4 *p = (const float4 *)(v + j);
#pragma unroll
        for (int k = 0; k < 16; k++) q[k] = p[k];
        float t = s;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            t = t + q[k].x;
            t = t + q[k].y;
            t = t + q[k].z;
            t = t + q[k].w;
        }
        if (pred(t)) {
            for (int k = 0; k < 64; k++) {
                s = s + v[j + k];
                if (pred(s)) return j + k;
            }
        }
        s = t;
    }
    for (; j < len; j++) {
        s = s + v[j];
        if (pred(s)) return j;
    }
    return len;
}

// sampler.c:53-66 on the m candidates (pf, pi; m - 1 in st->last). Pass 1
// (lane 0; waves 1-3 stage the next chunk): cum = p_0 + p_1 + ... until cum
// >= top_p (last = that candidate) or the candidates end, with the running
// sum at every chunk's end kept in LDS. r = u * cum. The pick is the first
// candidate whose running sum exceeds r: running sums never decrease, so it
// lies in the first chunk whose end value exceeds r, which pass 2 adds again
// from that chunk's starting value (the same additions, the same sums).
__global__ __launch_bounds__(NT) void k_sample_pick(const float *__restrict__ pf,
                                                    const int *__restrict__ pi, float top_p,
                                                    float u, SampleState *st, int *token) {
    __shared__ __align__(16) float buf[2][CH];
    __shared__ float cend[MAXCH];
    __shared__ int stop_sh, nch_used, pick_chunk, last_sh;
    __shared__ float r_sh;
    const int tid = threadIdx.x;
    const int m = st->last + 1;
    if (m == 0) {  // no candidate
        if (tid == 0) *token = st->best;
        return;
    }
    const int nch = (m + CH - 1) / CH;
    if (tid == 0) stop_sh = 0;
    stage_chunk(buf[0], pf, 0, m, tid, NT);
    __syncthreads();
    float cum = 0.0f;
    for (int c = 0; c < nch; c++) {
        if (tid >= 64) {
            if (c + 1 < nch) stage_chunk(buf[(c + 1) & 1], pf, (c + 1) * CH, m, tid - 64, NT - 64);
        } else if (tid == 0) {
            const int len = min(CH, m - c * CH);
            const int j = chain_until(buf[c & 1], len, cum, [=](float x) { return x >= top_p; });
            cend[c] = cum;
            if (j < len || c + 1 == nch) {
                stop_sh = 1;
                nch_used = c + 1;
                last_sh = j < len ? c * CH + j : m - 1;
            }
        }
        __syncthreads();
        if (stop_sh) break;
    }
    if (tid == 0) {
        const int last = last_sh;
        st->cum = cum;
        st->last = last;
        const float r = u * cum;
        r_sh = r;
        pick_chunk = -1;
        for (int c = 0; c < nch_used; c++)
            if (r < cend[c]) {
                pick_chunk = c;
                break;
            }
        if (pick_chunk < 0) *token = pi[last];
    }
    __syncthreads();
    const int pc = pick_chunk;
    if (pc < 0) return;
    stage_chunk(buf[0], pf, pc * CH, m, tid, NT);
    __syncthreads();
    if (tid == 0) {
        const float r = r_sh;
        const int last = last_sh;
        float acc = pc > 0 ? cend[pc - 1] : 0.0f;
        const int len = min(CH, last - pc * CH + 1);
        const int j = chain_until(buf[0], len, acc, [=](float x) { return r < x; });
        *token = j < len ? pi[pc * CH + j] : pi[last];
    }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

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
    k_chain_sum<<<1, NT, 0, st>>>(sc.e, n, sc.st);
    k_sample_keys<<<nb, NT, 0, st>>>(sc.e, n, cutoff, sc.st, sc.kin);
    if (mhip::check_launch(c, "sampler")) return -1;
    size_t tb = sc.tmp_bytes;
    if (mhip::check(c, rocprim::radix_sort_keys(sc.tmp, tb, sc.kin, sc.kout, (unsigned)n, 0, 64, st),
                    "sampler sort"))
        return -1;
    float *pf = (float *)sc.kin;  // the unsorted keys are dead after the sort
    int *pi = (int *)sc.kin + n;
    k_keys_split<<<nb, NT, 0, st>>>(sc.kout, n, pf, pi, sc.st);
    k_sample_pick<<<1, NT, 0, st>>>(pf, pi, s->top_p, u, sc.st, d_token);
    return mhip::check_launch(c, "sampler pick");
}

}  // extern "C"
