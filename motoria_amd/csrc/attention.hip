// Attention of one token (decode) for the Qwen3-MoE model on one MI355X:
// src/model/forward.c:118-165 of the reference, every value in the
// reference's operation order (bit-equal to its x86 build):
//
//   rmsnorm(x, attn_norm) -> Q8(xn)                       forward.c:123
//   q, k, v = Wq, Wk, Wv Q8(xn)   (k_rows_q8)             forward.c:124-126
//   per head: rmsnorm(q_h / k_h) and NeoX RoPE, then the
//   K and V rows appended to the cache (k_qk_rope)        forward.c:127-139
//   scores, softmax and the weighted sum of V per head
//   (k_attn_scores, k_attn_mix)                           forward.c:141-163
//   x += Wo Q8(att)   (k_quant_rows, k_rows_q8)           forward.c:164-165
//
// and the output head (forward.c:214-215) with the same row kernel. Weights
// stay in the .mia file's 36-byte Q8_0 blocks. RoPE's angles come from a
// table the host fills with its libm (the reference computes them in
// double with pow/cos/sin per call), so the rotations are the reference's.
#include "mhip_internal.h"

namespace {

constexpr int QK = mhip::QK;
constexpr int MAXNB = 256;  // blocks per row the row kernel holds (dims up to 8192)

// out[r] = (resid ? resid[r] : 0) + the reference's Q8 dot of weight row r
// (36-byte blocks) with the activation's codes xq[nb*32] and scales xs[nb]
// (src/tensor/matmul.c:19-28): one wavefront per row, lane b computes the
// block terms of blocks b, b + 64, ..., then lane 0 adds them in block order.
// Up to three matrices in one launch (rows of segment k: [r0[k], r0[k+1]),
// weights w[k], output out[k]); copy, when set, receives out[0] too.
struct RowSegs {
    const uint8_t *w[3];
    float *out[3];
    int r0[4];
};

__global__ __launch_bounds__(256) void k_rows_q8(RowSegs sg, int nb, const int8_t *__restrict__ xq,
                                                 const float *__restrict__ xs, const float *resid,
                                                 float *copy) {
    __shared__ float terms[4][MAXNB];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave;
    if (row >= sg.r0[3]) return;
    const int k = row >= sg.r0[1] ? (row >= sg.r0[2] ? 2 : 1) : 0;
    const int r = row - sg.r0[k];
    const uint8_t *wr = sg.w[k] + (size_t)r * nb * 36;
    for (int b = lane; b < nb; b += 64) {
        const uint32_t *blk = (const uint32_t *)(wr + (size_t)b * 36);
        const float dw = __uint_as_float(blk[0]);
        const int4 w0 = make_int4((int)blk[1], (int)blk[2], (int)blk[3], (int)blk[4]);
        const int4 w1 = make_int4((int)blk[5], (int)blk[6], (int)blk[7], (int)blk[8]);
        const int4 *xv = (const int4 *)(xq + (size_t)b * QK);
        terms[wave][b] = mhip_dev::block_term(mhip_dev::dot32_i8(w0, w1, xv[0], xv[1]), dw, xs[b]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) {
        float s = 0.0f;
        for (int b = 0; b < nb; b++) s = s + terms[wave][b];
        const float o = resid ? resid[r] + s : s;
        sg.out[k][r] = o;
        if (copy && k == 0) copy[r] = o;
    }
}

RowSegs one_seg(const void *w, float *out, int rows) {
    RowSegs g = {{(const uint8_t *)w, nullptr, nullptr}, {out, nullptr, nullptr}, {0, rows, rows, rows}};
    return g;
}

// Q8_0 of a row of n values into codes and scales (src/tensor/quant.c:11-27),
// one thread per 32-block.
__global__ __launch_bounds__(256) void k_quant_rows(const float *__restrict__ x, int nb,
                                                    int8_t *__restrict__ q,
                                                    float *__restrict__ s) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float *v = x + (size_t)b * QK;
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) {
        const float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    const float d = amax / 127.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < QK; i++) q[(size_t)b * QK + i] = (int8_t)roundf(v[i] * inv);
    s[b] = d;
}

// forward.c:127-139 and the cache append. Wavefront h < nh: query head h;
// nh <= h < nh + nkv: key head h - nh; then value heads, copied. A head's
// rmsnorm sums squares in double in index order (forward.c:75-81, one lane),
// then NeoX RoPE rotates element i with i + hd/2 by the angle of
// rope[pos][i] (cos, sin in double), each result rounded to float once.
__global__ __launch_bounds__(256) void k_qk_rope(float *__restrict__ q, const float *__restrict__ k,
                                                 const float *__restrict__ v,
                                                 const float *__restrict__ q_norm,
                                                 const float *__restrict__ k_norm,
                                                 const double *__restrict__ rope, int pos, int nh,
                                                 int nkv, int hd, float eps,
                                                 float *__restrict__ kc_row,
                                                 float *__restrict__ vc_row) {
    __shared__ float hv[4][256];
    __shared__ float inv_sh[4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = blockIdx.x * 4 + wave;
    if (h >= nh + 2 * nkv) return;
    if (h >= nh + nkv) {  // value head: the cache row as computed
        const int j = h - nh - nkv;
        for (int i = lane; i < hd; i += 64) vc_row[j * hd + i] = v[j * hd + i];
        return;
    }
    const bool isq = h < nh;
    const float *src = isq ? q + (size_t)h * hd : k + (size_t)(h - nh) * hd;
    const float *w = isq ? q_norm : k_norm;
    float *row = hv[wave];
    for (int i = lane; i < hd; i += 64) row[i] = src[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) {
        double ss = 0.0;
        for (int i = 0; i < hd; i++) ss = ss + (double)row[i] * (double)row[i];
        inv_sh[wave] = (float)(1.0 / sqrt(ss / hd + (double)eps));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float inv = inv_sh[wave];
    const int half = hd / 2;
    const double *rp = rope + (size_t)pos * half * 2;
    float *dst = isq ? q + (size_t)h * hd : kc_row + (size_t)(h - nh) * hd;
    for (int i = lane; i < half; i += 64) {
        const float x0 = (row[i] * inv) * w[i];
        const float x1 = (row[i + half] * inv) * w[i + half];
        const double c = rp[2 * i], s = rp[2 * i + 1];
        dst[i] = (float)((double)x0 * c - (double)x1 * s);
        dst[i + half] = (float)((double)x0 * s + (double)x1 * c);
    }
}

// forward.c:143-149: score[h][t] = (sequential fp32 dot of q_h and the
// cached k_t of its key head) * scale, one thread per (head, position).
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ q,
                                                     const float *__restrict__ kc, int n, int nh,
                                                     int group, int hd, int kvd, float scale,
                                                     float *__restrict__ scores, int ld) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nh * n) return;
    const int h = idx / n, t = idx % n;
    const float *qh = q + (size_t)h * hd;
    const float *kt = kc + (size_t)t * kvd + (size_t)(h / group) * hd;
    float dot = 0.0f;
    for (int i = 0; i < hd; i++) dot = dot + qh[i] * kt[i];
    scores[(size_t)h * ld + t] = dot * scale;
}

// forward.c:150-162 for head blockIdx.x: softmax of the n scores (first
// maximum, the restated glibc expf, sequential sum, division), then
// att[h][i] = sum over t of p_t * v_t[i] in position order, one thread per i.
__global__ __launch_bounds__(256) void k_attn_mix(float *__restrict__ scores, int ld, int n,
                                                  const float *__restrict__ vc, int group, int hd,
                                                  int kvd, float *__restrict__ att) {
    __shared__ float red[256];
    __shared__ float sum_sh;
    __shared__ uint64_t etab[32];
    const int h = blockIdx.x, tid = threadIdx.x;
    float *s = scores + (size_t)h * ld;
    if (tid < 32) etab[tid] = mia_expf_tab[tid];
    float mx = -__builtin_inff();
    for (int t = tid; t < n; t += 256) mx = fmaxf(mx, s[t]);
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    // the reference's running maximum picks the first maximum; every
    // maximum has the same value, and NaN scores stay NaN either way
    mx = red[0];
    for (int t = tid; t < n; t += 256) s[t] = mia_expf_glibc_tab(s[t] - mx, etab);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int t = 0; t < n; t++) sum = sum + s[t];
        sum_sh = sum;
    }
    __syncthreads();
    const float sum = sum_sh;
    for (int t = tid; t < n; t += 256) s[t] = s[t] / sum;
    __syncthreads();
    if (tid < hd) {
        const float *vt = vc + (size_t)(h / group) * hd + tid;
        float o = 0.0f;
        for (int t = 0; t < n; t++) o = o + s[t] * vt[(size_t)t * kvd];
        att[(size_t)h * hd + tid] = o;
    }
}

// One query head per workgroup, the whole of forward.c:127-163 for it:
// the head's rmsnorm and RoPE of q and of its key head's k (every head of a
// group recomputes that k; the group's first head appends k and v to the
// cache), the scores of positions 0..pos against the cache (position pos
// from the fresh k), softmax, the position-ordered mix, and Q8 of the
// head's att values (head_dim % 32 == 0: its blocks lie inside the head).
// The arithmetic of k_qk_rope, k_attn_scores, k_attn_mix and k_quant_rows,
// in the same order. LDS: q, k, the scores [max_seq] after them.
// forward.c:75-81 over one head's row in LDS (hd a multiple of 32): the
// sum of squares in double in index order, rows read 32 values ahead.
__device__ __forceinline__ float head_inv(const float *row, int hd, float eps) {
    double ss = 0.0;
    for (int i = 0; i < hd; i += 32) {
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
    return (float)(1.0 / sqrt(ss / hd + (double)eps));
}

// The head's normalized row, NeoX-rotated (forward.c:127-139): element i
// with i + hd/2 by the angle whose (cos, sin) are rp[2i], rp[2i+1].
__device__ __forceinline__ void head_rope(const float *row, float inv, const float *w,
                                          const double *rp, int hd, float *dst) {
    const int half = hd / 2;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float x0 = (row[i] * inv) * w[i];
        const float x1 = (row[i + half] * inv) * w[i + half];
        const double c = rp[2 * i], sn = rp[2 * i + 1];
        dst[i] = (float)((double)x0 * c - (double)x1 * sn);
        dst[i + half] = (float)((double)x0 * sn + (double)x1 * c);
    }
}

__global__ __launch_bounds__(256) void k_attn_head(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ q_norm, const float *__restrict__ k_norm,
    const double *__restrict__ rope, int pos, int nh, int nkv, int hd, float eps, float scale,
    float *__restrict__ kc, float *__restrict__ vc, int8_t *__restrict__ attq,
    float *__restrict__ atts) {
    extern __shared__ __align__(16) float lds[];
    __shared__ float red[256];
    __shared__ float inv_sh, inv2_sh, sum_sh;
    __shared__ uint64_t etab[32];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int group = nh / nkv, g = h / group, kvd = nkv * hd, n = pos + 1;
    float *qs = lds, *ks = lds + hd, *tq = lds + 2 * hd, *tk = lds + 3 * hd, *sc = lds + 4 * hd;
    if (tid < 32) etab[tid] = mia_expf_tab[tid];
    const double *rp = rope + (size_t)pos * (hd / 2) * 2;
    // the query head's and its key head's rows; their norms on two waves
    for (int i = tid; i < hd; i += blockDim.x) {
        tq[i] = q[(size_t)h * hd + i];
        tk[i] = k[(size_t)g * hd + i];
    }
    __syncthreads();
    if (tid == 0) inv_sh = head_inv(tq, hd, eps);
    if (tid == 64) inv2_sh = head_inv(tk, hd, eps);
    __syncthreads();
    head_rope(tq, inv_sh, q_norm, rp, hd, qs);
    head_rope(tk, inv2_sh, k_norm, rp, hd, ks);
    __syncthreads();
    if (h % group == 0)
        for (int i = tid; i < hd; i += blockDim.x) {
            kc[(size_t)pos * kvd + (size_t)g * hd + i] = ks[i];
            vc[(size_t)pos * kvd + (size_t)g * hd + i] = v[(size_t)g * hd + i];
        }
    // scores (forward.c:143-149): sequential fp32 dots, one position per
    // thread, the key row read 32 values ahead of the additions
    for (int t = tid; t < n; t += blockDim.x) {
        const float *kt = t == pos ? ks : kc + (size_t)t * kvd + (size_t)g * hd;
        float dot = 0.0f;
        for (int i = 0; i < hd; i += 32) {
            float4 k4[8];
#pragma unroll
            for (int j = 0; j < 8; j++) k4[j] = *(const float4 *)(kt + i + 4 * j);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                dot = dot + qs[i + 4 * j] * k4[j].x;
                dot = dot + qs[i + 4 * j + 1] * k4[j].y;
                dot = dot + qs[i + 4 * j + 2] * k4[j].z;
                dot = dot + qs[i + 4 * j + 3] * k4[j].w;
            }
        }
        sc[t] = dot * scale;
    }
    __syncthreads();
    // softmax (forward.c:150-156): the maximum (order-free), the restated
    // expf, the sequential sum, the division
    float mx = -__builtin_inff();
    for (int t = tid; t < n; t += blockDim.x) mx = fmaxf(mx, sc[t]);
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    mx = red[0];
    for (int t = tid; t < n; t += blockDim.x) sc[t] = mia_expf_glibc_tab(sc[t] - mx, etab);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int t = 0; t < n; t++) sum = sum + sc[t];
        sum_sh = sum;
    }
    __syncthreads();
    const float sum = sum_sh;
    for (int t = tid; t < n; t += blockDim.x) sc[t] = sc[t] / sum;
    __syncthreads();
    // mix (forward.c:157-162), then Q8 of the head's att (quant.c:11-27)
    float o = 0.0f;
    if (tid < hd) {
        // the value rows of 16 positions read before their additions
        const float *vt = vc + (size_t)g * hd + tid;
        int t = 0;
        for (; t + 16 <= pos; t += 16) {
            float vv[16];
#pragma unroll
            for (int j = 0; j < 16; j++) vv[j] = vt[(size_t)(t + j) * kvd];
#pragma unroll
            for (int j = 0; j < 16; j++) o = o + sc[t + j] * vv[j];
        }
        for (; t < pos; t++) o = o + sc[t] * vt[(size_t)t * kvd];
        o = o + sc[pos] * v[(size_t)g * hd + tid];
        // the block's maximum by a 32-lane butterfly (order-free; from 0,
        // a NaN never wins, as in the sequential loop)
        float am = fmaxf(0.0f, fabsf(o));
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) am = fmaxf(am, __shfl_xor(am, m, 32));
        const float d = am / 127.0f;
        const float qi = d != 0.0f ? 1.0f / d : 0.0f;
        attq[(size_t)h * hd + tid] = (int8_t)roundf(o * qi);
        if ((lane & 31) == 0) atts[((size_t)h * hd + tid) / QK] = d;
    }
}

// ---- the same for n consecutive tokens (a prompt) -----------------------------------
//
// Each token's values are the one-token path's: the row kernel below gives
// token t's output row r as k_rows_q8 does (the block terms added in block
// order), and the scores, softmax, mix and Q8 are k_qk_rope, k_attn_scores,
// k_attn_mix and k_quant_rows with a token index, token t at position pos + t
// reading the cache rows 0 .. pos + t, all of which (its own and the
// earlier tokens' of the batch among them) are appended before any score.

// out[k] + t * ld[k] + r = (resid ? resid[t * ld_r + r] : 0) + the Q8 dot of
// weight row r of segment k with token t's codes xq[t][nb*32] and scales
// xs[t][nb] (the block terms added in block order, as k_rows_q8 does), for
// the tokens 64 blockIdx.y .. + 63. Workgroup: RT_W wavefronts of RR rows
// each, lane i for token 64 blockIdx.y + i; the tokens' codes and scales and
// the rows' blocks are staged in LDS RT_BC blocks at a time.
constexpr int RT_W = 8, RT_BC = 16, RT_XLD = RT_BC * QK + 16;  // x row stride (bytes)

template <int RR>
__global__ __launch_bounds__(64 * RT_W) void k_rows_q8_t(RowSegs sg, int nb, int n,
                                                       const int8_t *__restrict__ xq,
                                                       const float *__restrict__ xs,
                                                       const float *resid, int ld_r) {
    constexpr int NR = RT_W * RR;  // rows of the workgroup
    __shared__ __align__(16) int8_t xq_l[64 * RT_XLD];
    __shared__ float xs_l[RT_BC][64];
    __shared__ __align__(16) int4 wq_l[NR][RT_BC][2];
    __shared__ float wd_l[NR][RT_BC];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.y * 64, nt = n - t0 < 64 ? n - t0 : 64;
    const int row0 = blockIdx.x * NR, nrows = sg.r0[3];
    float sum[RR];
#pragma unroll
    for (int j = 0; j < RR; j++) sum[j] = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += RT_BC) {
        const int nbc = nb - b0 < RT_BC ? nb - b0 : RT_BC;
        __syncthreads();
        for (int f = tid; f < nt * nbc * 2; f += 64 * RT_W) {
            const int tt = f / (nbc * 2), c = f % (nbc * 2);
            *(int4 *)&xq_l[tt * RT_XLD + c * 16] =
                *(const int4 *)(xq + ((size_t)(t0 + tt) * nb + b0) * QK + c * 16);
        }
        for (int f = tid; f < nt * nbc; f += 64 * RT_W) {
            const int tt = f / nbc, c = f % nbc;
            xs_l[c][tt] = xs[(size_t)(t0 + tt) * nb + b0 + c];
        }
        for (int f = tid; f < NR * nbc * 9; f += 64 * RT_W) {
            const int rr = f / (nbc * 9), c = f % (nbc * 9), b = c / 9, wd = c % 9;
            const int row = row0 + rr;
            if (row < nrows) {
                const int k = row >= sg.r0[1] ? (row >= sg.r0[2] ? 2 : 1) : 0;
                const uint32_t v = ((const uint32_t *)(sg.w[k] + ((size_t)(row - sg.r0[k]) * nb + b0 + b) * 36))[wd];
                if (wd == 0) wd_l[rr][b] = __uint_as_float(v);
                else ((uint32_t *)&wq_l[rr][b][0])[wd - 1] = v;
            }
        }
        __syncthreads();
        if (lane < nt) {
            for (int b = 0; b < nbc; b++) {
                const int4 *xv = (const int4 *)&xq_l[lane * RT_XLD + b * QK];
                const int4 x0 = xv[0], x1 = xv[1];
                const float dx = xs_l[b][lane];
#pragma unroll
                for (int j = 0; j < RR; j++) {
                    const int rr = wave * RR + j;
                    sum[j] = sum[j] + mhip_dev::block_term(
                                          mhip_dev::dot32_i8(wq_l[rr][b][0], wq_l[rr][b][1], x0, x1),
                                          wd_l[rr][b], dx);
                }
            }
        }
    }
    if (lane < nt) {
        const int t = t0 + lane;
#pragma unroll
        for (int j = 0; j < RR; j++) {
            const int row = row0 + wave * RR + j;
            if (row < nrows) {
                const int k = row >= sg.r0[1] ? (row >= sg.r0[2] ? 2 : 1) : 0;
                const int r = row - sg.r0[k], ld = sg.r0[k + 1] - sg.r0[k];
                sg.out[k][(size_t)t * ld + r] = resid ? resid[(size_t)t * ld_r + r] + sum[j] : sum[j];
            }
        }
    }
}

// ---- the batch's weight rows on the matrix cores --------------------------------------
//
// For a batch the rows are products of the row tile's weight codes with the
// tokens' codes: v_mfma_f32_16x16x32_f16 over one 32-code block multiplies
// Q8 codes held as fp16 integers and gives the exact int32 block dot (32
// products below 2^14 each, every partial sum an integer below 2^24), so
// the block term ((float)dot * d_w) * d_x and the sum in block order are the
// reference's (matmul.c:19-28). The weights are repacked once for this:
// codes as fp16 [R][nb*32], scales block-major [nb][R]; the tokens' codes
// are converted to fp16 [n][nb*32] per batch.
typedef _Float16 rh8 __attribute__((ext_vector_type(8)));
typedef float rf4 __attribute__((ext_vector_type(4)));
#ifndef RM_J
#define RM_J 2  // 16-token tiles per wavefront
#endif
constexpr int RM_R = 64, RM_T = 64 * RM_J;  // weight rows and tokens of a workgroup
constexpr int RM_MIN_N = 512;                // batches from which the rows run here

// Row r of a .mia Q8_0 matrix (36-byte blocks) into the packed form, one
// thread per block.
__global__ __launch_bounds__(256) void k_pack_rows_h(const uint8_t *__restrict__ w, int R, int nb,
                                                     _Float16 *__restrict__ qh,
                                                     float *__restrict__ sc) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)R * nb) return;
    const int r = (int)(q / nb), b = (int)(q % nb);
    const uint8_t *blk = w + q * 36;
    sc[(size_t)b * R + r] = *(const float *)blk;
    const int8_t *c = (const int8_t *)(blk + 4);
    _Float16 *o = qh + q * QK;
#pragma unroll
    for (int i = 0; i < QK; i++) o[i] = (_Float16)c[i];
}

// Q8 codes as fp16 integers (exact).
__global__ __launch_bounds__(256) void k_codes_h(const int8_t *__restrict__ q, size_t n,
                                                 _Float16 *__restrict__ o) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = (_Float16)q[i];
}

struct RowPack {
    const _Float16 *q[3];  // packed codes of segment k
    const float *s[3];     // its block-major scales
    float *out[3];
    int r0[4];             // rows of segment k: [r0[k], r0[k+1]), multiples of RM_R
};

// out[k][t * ld_k + r] = (resid ? resid[t * ld_r + r] : 0) + the Q8 dot of
// packed row r of segment k with token t (codes xh[t][nb*32], scales
// xs[t][nb]), for RM_R rows x RM_T tokens per workgroup: wavefront w takes
// tokens 16 RM_J w .. + 16 RM_J - 1 (RM_J 16-token tiles) against the 64
// rows (four 16-row tiles); lane l's results are rows 16 i + 4 (l / 16) + 0..3 of
// token 16 j + l % 16. The operands of block b + 1 are loaded while block
// b's products and terms are formed.
__global__ __launch_bounds__(256) void k_rows_mfma(RowPack sg, int nb, int n,
                                                   const _Float16 *__restrict__ xh,
                                                   const float *__restrict__ xs,
                                                   const float *resid, int ld_r) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, c = lane >> 4;
    const int row0 = blockIdx.x * RM_R;
    const int k = row0 >= sg.r0[1] ? (row0 >= sg.r0[2] ? 2 : 1) : 0;
    const int rl0 = row0 - sg.r0[k], R = sg.r0[k + 1] - sg.r0[k];
    const _Float16 *wq = sg.q[k];
    const float *ws = sg.s[k];
    const int t0 = blockIdx.y * RM_T + 16 * RM_J * wave;
    int tj[RM_J];
#pragma unroll
    for (int j = 0; j < RM_J; j++) tj[j] = min(t0 + 16 * j + l16, n - 1);
    rf4 acc[4][RM_J];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < RM_J; j++) acc[i][j] = (rf4){0.0f, 0.0f, 0.0f, 0.0f};
    struct Ops {
        rh8 a[4], x[RM_J];
        rf4 dw[4];
        float dx[RM_J];
    };
    auto load = [&](int b, Ops &o) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            o.a[i] = *(const rh8 *)(wq + ((size_t)(rl0 + 16 * i + l16) * nb + b) * QK + 8 * c);
#pragma unroll
        for (int j = 0; j < RM_J; j++)
            o.x[j] = *(const rh8 *)(xh + ((size_t)tj[j] * nb + b) * QK + 8 * c);
#pragma unroll
        for (int i = 0; i < 4; i++)
            o.dw[i] = *(const rf4 *)(ws + (size_t)b * R + rl0 + 16 * i + 4 * c);
#pragma unroll
        for (int j = 0; j < RM_J; j++) o.dx[j] = xs[(size_t)tj[j] * nb + b];
    };
    auto step = [&](const Ops &o) {
        const rf4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < RM_J; j++) {
                const rf4 blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.a[i], o.x[j], z, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float t = blk[r] * o.dw[i][r];
                    acc[i][j][r] = acc[i][j][r] + t * o.dx[j];  // (no contraction)
                }
            }
    };
    Ops o0, o1;
    load(0, o0);
    for (int b = 0; b < nb; b += 2) {
        if (b + 1 < nb) load(b + 1, o1);
        step(o0);
        if (b + 2 < nb) load(b + 2, o0);
        if (b + 1 < nb) step(o1);
    }
#pragma unroll
    for (int j = 0; j < RM_J; j++) {
        const int t = t0 + 16 * j + l16;
        if (t < n) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = rl0 + 16 * i + 4 * c + r;
                    const float v = acc[i][j][r];
                    sg.out[k][(size_t)t * R + row] = resid ? resid[(size_t)t * ld_r + row] + v : v;
                }
        }
    }
}

// k_qk_rope for token blockIdx.y at position pos + blockIdx.y: its q (in
// place), k and v rows at [t][qd], [t][kvd]; the cache rows at pos + t.
__global__ __launch_bounds__(256) void k_qk_rope_b(float *__restrict__ q,
                                                   const float *__restrict__ k,
                                                   const float *__restrict__ v,
                                                   const float *__restrict__ q_norm,
                                                   const float *__restrict__ k_norm,
                                                   const double *__restrict__ rope, int pos,
                                                   int nh, int nkv, int hd, float eps,
                                                   float *__restrict__ kc,
                                                   float *__restrict__ vc) {
    __shared__ float hv[4][256];
    __shared__ float inv_sh[4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = blockIdx.x * 4 + wave, t = blockIdx.y, p = pos + t;
    const int qd = nh * hd, kvd = nkv * hd;
    if (h >= nh + 2 * nkv) return;
    float *kc_row = kc + (size_t)p * kvd, *vc_row = vc + (size_t)p * kvd;
    if (h >= nh + nkv) {
        const int j = h - nh - nkv;
        for (int i = lane; i < hd; i += 64) vc_row[j * hd + i] = v[(size_t)t * kvd + j * hd + i];
        return;
    }
    const bool isq = h < nh;
    const float *src = isq ? q + (size_t)t * qd + (size_t)h * hd
                           : k + (size_t)t * kvd + (size_t)(h - nh) * hd;
    const float *w = isq ? q_norm : k_norm;
    float *row = hv[wave];
    for (int i = lane; i < hd; i += 64) row[i] = src[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) {
        double ss = 0.0;
        for (int i = 0; i < hd; i++) ss = ss + (double)row[i] * (double)row[i];
        inv_sh[wave] = (float)(1.0 / sqrt(ss / hd + (double)eps));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float inv = inv_sh[wave];
    const int half = hd / 2;
    const double *rp = rope + (size_t)p * half * 2;
    float *dst = isq ? q + (size_t)t * qd + (size_t)h * hd : kc_row + (size_t)(h - nh) * hd;
    for (int i = lane; i < half; i += 64) {
        const float x0 = (row[i] * inv) * w[i];
        const float x1 = (row[i + half] * inv) * w[i + half];
        const double c = rp[2 * i], sn = rp[2 * i + 1];
        dst[i] = (float)((double)x0 * c - (double)x1 * sn);
        dst[i + half] = (float)((double)x0 * sn + (double)x1 * c);
    }
}

// k_attn_scores for token blockIdx.y: scores[t][h][0 .. pos + t].
__global__ __launch_bounds__(256) void k_attn_scores_b(const float *__restrict__ q,
                                                       const float *__restrict__ kc, int pos,
                                                       int nh, int group, int hd, int kvd,
                                                       float scale, float *__restrict__ scores,
                                                       int ld) {
    const int t = blockIdx.y, np = pos + t + 1;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nh * np) return;
    const int h = idx / np, u = idx % np;
    const float *qh = q + (size_t)t * nh * hd + (size_t)h * hd;
    const float *kt = kc + (size_t)u * kvd + (size_t)(h / group) * hd;
    float dot = 0.0f;
    for (int i = 0; i < hd; i++) dot = dot + qh[i] * kt[i];
    scores[((size_t)t * nh + h) * ld + u] = dot * scale;
}

// k_attn_mix for head blockIdx.x of token blockIdx.y (positions 0 .. pos + t).
__global__ __launch_bounds__(256) void k_attn_mix_b(float *__restrict__ scores, int ld, int pos,
                                                    int nh, const float *__restrict__ vc,
                                                    int group, int hd, int kvd,
                                                    float *__restrict__ att) {
    __shared__ float red[256];
    __shared__ float sum_sh;
    __shared__ uint64_t etab[32];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, n = pos + t + 1;
    float *s = scores + ((size_t)t * nh + h) * ld;
    if (tid < 32) etab[tid] = mia_expf_tab[tid];
    float mx = -__builtin_inff();
    for (int u = tid; u < n; u += 256) mx = fmaxf(mx, s[u]);
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    mx = red[0];
    for (int u = tid; u < n; u += 256) s[u] = mia_expf_glibc_tab(s[u] - mx, etab);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int u = 0; u < n; u++) sum = sum + s[u];
        sum_sh = sum;
    }
    __syncthreads();
    const float sum = sum_sh;
    for (int u = tid; u < n; u += 256) s[u] = s[u] / sum;
    __syncthreads();
    if (tid < hd) {
        const float *vt = vc + (size_t)(h / group) * hd + tid;
        float o = 0.0f;
        for (int u = 0; u < n; u++) o = o + s[u] * vt[(size_t)u * kvd];
        att[(size_t)t * nh * hd + (size_t)h * hd + tid] = o;
    }
}

// k_attn_scores_b, k_attn_mix_b for key/value head blockIdx.x of token
// blockIdx.y and all `group` query heads that read it (head_dim AG_HD):
// the group shares each key and value row it loads. Scores: chunks of
// C = 256 / group positions, the chunk's key rows staged in LDS, thread
// (head tid / C, position tid % C) with its q row in registers. Softmax:
// wavefront w takes heads w, w + 4, ...; the sequential sums run on lanes
// 0 .. group - 1 of wavefront 0, one head each. Mix: thread (element
// tid % AG_HD, heads tid / AG_HD + 2 j), the value rows read 16 positions
// ahead of their additions. Scores (row stride sld, a multiple of 4) in
// LDS behind the key rows (SC_LDS) or at scores + ((t * nh + h) * sld).
constexpr int AG_HD = 128, AG_KLD = AG_HD + 4, AG_MAXG = 16;
constexpr size_t AG_LDS_MAX = 150 * 1024;
size_t ag_lds(int group, int sld, bool sc_lds) {
    return (size_t)(256 / group) * AG_KLD * 4 + (sc_lds ? (size_t)group * sld * 4 : 0);
}

template <bool SC_LDS>
__global__ __launch_bounds__(256) void k_attn_group_b(const float *__restrict__ q,
                                                      const float *__restrict__ kc,
                                                      const float *__restrict__ vc, int pos,
                                                      int nh, int group, int kvd, float scale,
                                                      float *__restrict__ scores, int sld,
                                                      float *__restrict__ att) {
    extern __shared__ __align__(16) float ag_sh[];
    __shared__ uint64_t etab[32];
    __shared__ float sum_sh[AG_MAXG];
    const int g = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = tid >> 6, np = pos + t + 1, C = 256 / group;
    float *kt = ag_sh;
    float *sc = SC_LDS ? ag_sh + (size_t)C * AG_KLD
                       : scores + ((size_t)t * nh + (size_t)g * group) * sld;
    if (tid < 32) etab[tid] = mia_expf_tab[tid];
    {
        const int hh = tid / C, c = tid % C;
        float4 qr[AG_HD / 4];
        const float4 *qh =
            (const float4 *)(q + (size_t)t * nh * AG_HD + (size_t)(g * group + hh) * AG_HD);
#pragma unroll
        for (int j = 0; j < AG_HD / 4; j++) qr[j] = qh[j];
        for (int u0 = 0; u0 < np; u0 += C) {
            const int nc = np - u0 < C ? np - u0 : C;
            __syncthreads();
            for (int f = tid; f < nc * (AG_HD / 4); f += 256) {
                const int row = f / (AG_HD / 4), c4 = f % (AG_HD / 4);
                *(float4 *)&kt[row * AG_KLD + 4 * c4] =
                    *(const float4 *)(kc + (size_t)(u0 + row) * kvd + (size_t)g * AG_HD + 4 * c4);
            }
            __syncthreads();
            if (c < nc) {
                const float4 *kr = (const float4 *)&kt[c * AG_KLD];
                float dot = 0.0f;
                for (int i = 0; i < AG_HD / 4; i += 8) {
                    float4 k4[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) k4[j] = kr[i + j];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        dot = dot + qr[i + j].x * k4[j].x;
                        dot = dot + qr[i + j].y * k4[j].y;
                        dot = dot + qr[i + j].z * k4[j].z;
                        dot = dot + qr[i + j].w * k4[j].w;
                    }
                }
                sc[(size_t)hh * sld + u0 + c] = dot * scale;
            }
        }
    }
    __syncthreads();
    for (int hh = wave; hh < group; hh += 4) {
        float *s = sc + (size_t)hh * sld;
        float mx = -__builtin_inff();
        for (int u = lane; u < np; u += 64) mx = fmaxf(mx, s[u]);
        // (fmaxf keeps the larger of a number and a NaN: any order gives this)
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
        for (int u = lane; u < np; u += 64) s[u] = mia_expf_glibc_tab(s[u] - mx, etab);
    }
    __syncthreads();
    if (tid < group) {
        const float *s = sc + (size_t)tid * sld;
        float sum = 0.0f;
        int u = 0;
        for (; u + 16 <= np; u += 16) {
            float4 b[4];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = *(const float4 *)(s + u + 4 * j);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sum = sum + b[j].x;
                sum = sum + b[j].y;
                sum = sum + b[j].z;
                sum = sum + b[j].w;
            }
        }
        for (; u < np; u++) sum = sum + s[u];
        sum_sh[tid] = sum;
    }
    __syncthreads();
    for (int hh = 0; hh < group; hh++) {
        float *s = sc + (size_t)hh * sld;
        const float sum = sum_sh[hh];
        for (int u = tid; u < np; u += 256) s[u] = s[u] / sum;
    }
    __syncthreads();
    {
        const int i = tid % AG_HD, r = tid / AG_HD;
        constexpr int NO = AG_MAXG / 2;
        float o[NO];
#pragma unroll
        for (int j = 0; j < NO; j++) o[j] = 0.0f;
        const float *vt = vc + (size_t)g * AG_HD + i;
        int u = 0;
        for (; u + 16 <= np; u += 16) {
            float vv[16];
#pragma unroll
            for (int j = 0; j < 16; j++) vv[j] = vt[(size_t)(u + j) * kvd];
#pragma unroll
            for (int jj = 0; jj < NO; jj++) {
                if (r + 2 * jj < group) {
                    const float4 *p4 = (const float4 *)(sc + (size_t)(r + 2 * jj) * sld + u);
#pragma unroll
                    for (int j4 = 0; j4 < 4; j4++) {
                        const float4 p = p4[j4];
                        o[jj] = o[jj] + p.x * vv[4 * j4];
                        o[jj] = o[jj] + p.y * vv[4 * j4 + 1];
                        o[jj] = o[jj] + p.z * vv[4 * j4 + 2];
                        o[jj] = o[jj] + p.w * vv[4 * j4 + 3];
                    }
                }
            }
        }
        for (; u < np; u++) {
            const float vu = vt[(size_t)u * kvd];
#pragma unroll
            for (int jj = 0; jj < NO; jj++)
                if (r + 2 * jj < group) o[jj] = o[jj] + sc[(size_t)(r + 2 * jj) * sld + u] * vu;
        }
#pragma unroll
        for (int jj = 0; jj < NO; jj++)
            if (r + 2 * jj < group)
                att[(size_t)t * nh * AG_HD + (size_t)(g * group + r + 2 * jj) * AG_HD + i] = o[jj];
    }
}

constexpr size_t HEAD_LDS_MAX = 150 * 1024;  // dynamic LDS of k_attn_head
size_t head_lds(int hd, int max_seq) { return ((size_t)4 * hd + (size_t)max_seq) * sizeof(float); }

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

struct AttnScratch {
    float *xn, *xs, *q, *k, *v, *att, *atts, *scores;
    int8_t *xq, *attq;
    int *status;
};

AttnScratch carve(const mhip_attn_dims *s, int max_seq, void *base) {
    const size_t d = s->dim, qd = (size_t)s->n_heads * s->head_dim,
                 kvd = (size_t)s->n_kv_heads * s->head_dim;
    uint8_t *p = (uint8_t *)base;
    auto take = [&](size_t bytes) {
        void *r = p;
        p += align256(bytes);
        return r;
    };
    AttnScratch a;
    a.xn = (float *)take(d * 4);
    a.xq = (int8_t *)take(d);
    a.xs = (float *)take(d / QK * 4);
    a.q = (float *)take(qd * 4);
    a.k = (float *)take(kvd * 4);
    a.v = (float *)take(kvd * 4);
    a.att = (float *)take(qd * 4);
    a.attq = (int8_t *)take(qd);
    a.atts = (float *)take(qd / QK * 4);
    a.scores = (float *)take((size_t)s->n_heads * max_seq * 4);
    a.status = (int *)take(16);
    return a;
}

int check_attn(mhip_ctx *c, const mhip_attn_dims *s, int max_seq) {
    if (!s) return mhip::fail(c, "null attention dims");
    const int qd = s->n_heads * s->head_dim;
    if (s->dim <= 0 || s->dim % QK || s->dim / QK > MAXNB || s->n_heads <= 0 ||
        s->n_kv_heads <= 0 || s->n_heads % s->n_kv_heads || s->head_dim <= 0 ||
        s->head_dim % 2 || s->head_dim > 256 || qd % QK || qd / QK > MAXNB)
        return mhip::fail(c, "attention shape dim=%d heads=%d/%d head_dim=%d not supported",
                          s->dim, s->n_heads, s->n_kv_heads, s->head_dim);
    if (max_seq <= 0) return mhip::fail(c, "max_seq=%d", max_seq);
    return 0;
}

}  // namespace

extern "C" {

size_t mhip_attention_scratch_bytes(const mhip_attn_dims *s, int max_seq) {
    const size_t d = s->dim, qd = (size_t)s->n_heads * s->head_dim,
                 kvd = (size_t)s->n_kv_heads * s->head_dim;
    return align256(d * 4) + align256(d) + align256(d / QK * 4) + align256(qd * 4) +
           2 * align256(kvd * 4) + align256(qd * 4) + align256(qd) + align256(qd / QK * 4) +
           align256((size_t)s->n_heads * max_seq * 4) + align256(16);
}

int mhip_attention(mhip_ctx *c, const mhip_attn_dims *s, const float *d_attn_norm,
                   const void *d_wq, const void *d_wk, const void *d_wv, const void *d_wo,
                   const float *d_q_norm, const float *d_k_norm, const double *d_rope,
                   float *d_kc, float *d_vc, int pos, int max_seq, float *d_x,
                   float *d_x_copy, void *d_scratch, int flags) {
    if (check_attn(c, s, max_seq)) return -1;
    if (pos < 0 || pos >= max_seq)
        return mhip::fail(c, "attention: pos=%d outside [0, max_seq=%d)", pos, max_seq);
    if (mhip::use_device(c)) return -1;
    const int d = s->dim, nh = s->n_heads, nkv = s->n_kv_heads, hd = s->head_dim;
    const int qd = nh * hd, kvd = nkv * hd, n = pos + 1;
    AttnScratch a = carve(s, max_seq, d_scratch);
    hipStream_t st = c->stream;
    mhip::launch_rmsnorm_q8(st, d_x, d_attn_norm, a.xn, a.xq, a.xs, 1, d, s->norm_eps,
                            (flags & MHIP_FORCE_SEQ_RMS) ? 1 : 0, a.status);
    const int nb = d / QK;
    RowSegs qkv = {{(const uint8_t *)d_wq, (const uint8_t *)d_wk, (const uint8_t *)d_wv},
                   {a.q, a.k, a.v},
                   {0, qd, qd + kvd, qd + 2 * kvd}};
    k_rows_q8<<<mhip::blocks_for(qd + 2 * kvd, 4), 256, 0, st>>>(qkv, nb, a.xq, a.xs, nullptr,
                                                                  nullptr);
    if (mhip::check_launch(c, "attention qkv")) return -1;
    const float scale = 1.0f / sqrtf((float)hd);
    const size_t hl = head_lds(hd, max_seq);
    if (hd % QK == 0 && hl <= HEAD_LDS_MAX) {
        static int lds_set[64];  // per device ordinal (contexts of one device share it)
        if (c->device >= 0 && c->device < 64 && !lds_set[c->device]) {
            if (mhip::check(c, hipFuncSetAttribute((const void *)k_attn_head,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)HEAD_LDS_MAX),
                            "attention LDS attribute"))
                return -1;
            lds_set[c->device] = 1;
        }
        k_attn_head<<<nh, 256, hl, st>>>(a.q, a.k, a.v, d_q_norm, d_k_norm, d_rope, pos, nh, nkv,
                                         hd, s->norm_eps, scale, d_kc, d_vc, a.attq, a.atts);
    } else {
        k_qk_rope<<<mhip::blocks_for(nh + 2 * nkv, 4), 256, 0, st>>>(
            a.q, a.k, a.v, d_q_norm, d_k_norm, d_rope, pos, nh, nkv, hd, s->norm_eps,
            d_kc + (size_t)pos * kvd, d_vc + (size_t)pos * kvd);
        k_attn_scores<<<mhip::blocks_for((size_t)nh * n, 256), 256, 0, st>>>(
            a.q, d_kc, n, nh, nh / nkv, hd, kvd, scale, a.scores, max_seq);
        k_attn_mix<<<nh, 256, 0, st>>>(a.scores, max_seq, n, d_vc, nh / nkv, hd, kvd, a.att);
        k_quant_rows<<<mhip::blocks_for(qd / QK, 256), 256, 0, st>>>(a.att, qd / QK, a.attq,
                                                                      a.atts);
    }
    k_rows_q8<<<mhip::blocks_for(d, 4), 256, 0, st>>>(one_seg(d_wo, d_x, d), qd / QK, a.attq,
                                                       a.atts, d_x, d_x_copy);
    return mhip::check_launch(c, "attention");
}

// Tokens per pass of the scores kept in device memory (contexts too long for
// LDS, other head shapes): the scratch holds this many tokens' scores.
constexpr int AB_SUB = 64;

size_t mhip_attention_batch_scratch_bytes(const mhip_attn_dims *s, int n, int max_seq) {
    if (!s || n <= 0 || max_seq <= 0) return 0;
    const size_t d = s->dim, qd = (size_t)s->n_heads * s->head_dim,
                 kvd = (size_t)s->n_kv_heads * s->head_dim, N = (size_t)n;
    return align256(N * d * 4) + align256(N * d) + align256(N * (d / QK) * 4) +
           align256(N * qd * 4) + 2 * align256(N * kvd * 4) + align256(N * qd * 4) +
           align256(N * qd) + align256(N * (qd / QK) * 4) + align256(N * d * 2) +
           align256(N * qd * 2) +
           align256((size_t)(n < AB_SUB ? n : AB_SUB) * s->n_heads * (size_t)((max_seq + 3) & ~3) * 4) +
           align256(16);
}

}  // extern "C"

namespace {

// The packed weights of one layer (mhip_attention_pack): fp16 codes of Q, K,
// V and O, then their block-major scales, each 256-byte aligned.
struct AttnPack {
    _Float16 *q[4];
    float *s[4];
};
AttnPack pack_carve(const mhip_attn_dims *s, void *base) {
    const size_t d = s->dim, qd = (size_t)s->n_heads * s->head_dim,
                 kvd = (size_t)s->n_kv_heads * s->head_dim;
    const size_t rows[4] = {qd, kvd, kvd, d}, cols[4] = {d, d, d, qd};
    AttnPack a;
    uint8_t *p = (uint8_t *)base;
    for (int m = 0; m < 4; m++) {
        a.q[m] = (_Float16 *)p;
        p += align256(rows[m] * cols[m] * 2);
    }
    for (int m = 0; m < 4; m++) {
        a.s[m] = (float *)p;
        p += align256(rows[m] * (cols[m] / QK) * 4);
    }
    return a;
}
bool pack_fits(const mhip_attn_dims *s) {
    const int qd = s->n_heads * s->head_dim, kvd = s->n_kv_heads * s->head_dim;
    return qd % RM_R == 0 && kvd % RM_R == 0 && s->dim % RM_R == 0;
}

}  // namespace

extern "C" {

size_t mhip_attention_pack_bytes(const mhip_attn_dims *s) {
    if (!s || s->dim <= 0 || s->n_heads <= 0 || s->n_kv_heads <= 0 || s->head_dim <= 0 ||
        !pack_fits(s))
        return 0;
    const size_t d = s->dim, qd = (size_t)s->n_heads * s->head_dim,
                 kvd = (size_t)s->n_kv_heads * s->head_dim;
    const size_t rows[4] = {qd, kvd, kvd, d}, cols[4] = {d, d, d, qd};
    size_t n = 0;
    for (int m = 0; m < 4; m++) n += align256(rows[m] * cols[m] * 2) + align256(rows[m] * (cols[m] / QK) * 4);
    return n;
}

int mhip_attention_pack(mhip_ctx *c, const mhip_attn_dims *s, const void *d_wq, const void *d_wk,
                        const void *d_wv, const void *d_wo, void *d_pack) {
    if (check_attn(c, s, 1)) return -1;
    if (!pack_fits(s))
        return mhip::fail(c, "attention pack: rows not multiples of %d", RM_R);
    if (mhip::use_device(c)) return -1;
    const int d = s->dim, qd = s->n_heads * s->head_dim, kvd = s->n_kv_heads * s->head_dim;
    const AttnPack a = pack_carve(s, d_pack);
    const void *w[4] = {d_wq, d_wk, d_wv, d_wo};
    const int rows[4] = {qd, kvd, kvd, d}, nbs[4] = {d / QK, d / QK, d / QK, qd / QK};
    for (int m = 0; m < 4; m++)
        k_pack_rows_h<<<mhip::blocks_for((size_t)rows[m] * nbs[m], 256), 256, 0, c->stream>>>(
            (const uint8_t *)w[m], rows[m], nbs[m], a.q[m], a.s[m]);
    return mhip::check_launch(c, "attention pack");
}

}  // extern "C"

namespace {

void rows_mfma(hipStream_t st, const AttnPack &a, int m0, int nseg, float *const *out,
               const int *r0, int nb, int n, const _Float16 *xh, const float *xs, const float *resid,
               int ld_r) {
    RowPack g = {{nullptr, nullptr, nullptr}, {nullptr, nullptr, nullptr}, {nullptr, nullptr, nullptr},
                 {r0[0], r0[1], r0[2], r0[3]}};
    for (int k = 0; k < nseg; k++) {
        g.q[k] = a.q[m0 + k];
        g.s[k] = a.s[m0 + k];
        g.out[k] = out[k];
    }
    k_rows_mfma<<<dim3((unsigned)(r0[3] / RM_R), (unsigned)((n + RM_T - 1) / RM_T)), 256, 0, st>>>(
        g, nb, n, xh, xs, resid, ld_r);
}

}  // namespace

extern "C" {

int mhip_attention_batch(mhip_ctx *c, const mhip_attn_dims *s, const float *d_attn_norm,
                         const void *d_wq, const void *d_wk, const void *d_wv, const void *d_wo,
                         const float *d_q_norm, const float *d_k_norm, const double *d_rope,
                         float *d_kc, float *d_vc, int pos, int n, int max_seq, float *d_x,
                         const void *d_pack, void *d_scratch, int flags) {
    if (check_attn(c, s, max_seq)) return -1;
    if (n <= 0 || pos < 0 || pos + n > max_seq)
        return mhip::fail(c, "attention batch: positions %d .. %d outside [0, max_seq=%d)", pos,
                          pos + n - 1, max_seq);
    if (mhip::use_device(c)) return -1;
    const int d = s->dim, nh = s->n_heads, nkv = s->n_kv_heads, hd = s->head_dim;
    const int qd = nh * hd, kvd = nkv * hd, nb = d / QK;
    // carve the batch scratch
    uint8_t *p = (uint8_t *)d_scratch;
    auto take = [&](size_t bytes) {
        void *r = p;
        p += align256(bytes);
        return r;
    };
    const size_t N = (size_t)n;
    float *xn = (float *)take(N * d * 4);
    int8_t *xq = (int8_t *)take(N * d);
    float *xs = (float *)take(N * nb * 4);
    float *q = (float *)take(N * qd * 4);
    float *k = (float *)take(N * kvd * 4);
    float *v = (float *)take(N * kvd * 4);
    float *att = (float *)take(N * qd * 4);
    int8_t *attq = (int8_t *)take(N * qd);
    float *atts = (float *)take(N * (qd / QK) * 4);
    _Float16 *xh = (_Float16 *)take(N * d * 2);
    _Float16 *atth = (_Float16 *)take(N * qd * 2);
    const int sld = (max_seq + 3) & ~3;  // row stride of the scores
    float *scores = (float *)take((size_t)(n < AB_SUB ? n : AB_SUB) * nh * (size_t)sld * 4);
    int *status = (int *)take(16);
    hipStream_t st = c->stream;
    static int lds_set[64];  // per device ordinal
    if (c->device >= 0 && c->device < 64 && !lds_set[c->device]) {
        if (mhip::check(c, hipFuncSetAttribute((const void *)k_attn_group_b<true>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)AG_LDS_MAX),
                        "attention LDS attribute") ||
            mhip::check(c, hipFuncSetAttribute((const void *)k_attn_group_b<false>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)AG_LDS_MAX),
                        "attention LDS attribute"))
            return -1;
        lds_set[c->device] = 1;
    }
    mhip::launch_rmsnorm_q8(st, d_x, d_attn_norm, xn, xq, xs, n, d, s->norm_eps,
                            (flags & MHIP_FORCE_SEQ_RMS) ? 1 : 0, status);
    RowSegs qkv = {{(const uint8_t *)d_wq, (const uint8_t *)d_wk, (const uint8_t *)d_wv},
                   {q, k, v},
                   {0, qd, qd + kvd, qd + 2 * kvd}};
    // the matrix cores from 512 tokens on, when the layer's weights are packed
    // (below that the vector rows measured as fast or faster)
    const bool mm = d_pack && pack_fits(s) && n >= RM_MIN_N;
    const AttnPack pk = mm ? pack_carve(s, (void *)d_pack) : AttnPack{};
    if (mm) {
        k_codes_h<<<mhip::blocks_for(N * d, 256), 256, 0, st>>>(xq, N * d, xh);
        float *outs[3] = {q, k, v};
        const int r0[4] = {0, qd, qd + kvd, qd + 2 * kvd};
        rows_mfma(st, pk, 0, 3, outs, r0, nb, n, xh, xs, nullptr, 0);
    } else {
        k_rows_q8_t<2><<<dim3(mhip::blocks_for(qd + 2 * kvd, 2 * RT_W), mhip::blocks_for(N, 64)),
                         64 * RT_W, 0, st>>>(qkv, nb, n, xq, xs, nullptr, 0);
    }
    if (mhip::check_launch(c, "attention batch qkv")) return -1;
    k_qk_rope_b<<<dim3(mhip::blocks_for(nh + 2 * nkv, 4), n), 256, 0, st>>>(
        q, k, v, d_q_norm, d_k_norm, d_rope, pos, nh, nkv, hd, s->norm_eps, d_kc, d_vc);
    const float scale = 1.0f / sqrtf((float)hd);
    const int group = nh / nkv;
    if (hd == AG_HD && group <= AG_MAXG && 256 % group == 0) {
        // the group's heads together; their scores in LDS while they fit
        const int sl = (pos + n + 3) & ~3;
        if (ag_lds(group, sl, true) <= AG_LDS_MAX)
            k_attn_group_b<true><<<dim3(nkv, n), 256, ag_lds(group, sl, true), st>>>(
                q, d_kc, d_vc, pos, nh, group, kvd, scale, nullptr, sl, att);
        else
            for (int t0 = 0; t0 < n; t0 += AB_SUB) {
                const int ns = n - t0 < AB_SUB ? n - t0 : AB_SUB;
                k_attn_group_b<false><<<dim3(nkv, ns), 256, ag_lds(group, sld, false), st>>>(
                    q + (size_t)t0 * qd, d_kc, d_vc, pos + t0, nh, group, kvd, scale, scores, sld,
                    att + (size_t)t0 * qd);
            }
    } else {
        for (int t0 = 0; t0 < n; t0 += AB_SUB) {
            const int ns = n - t0 < AB_SUB ? n - t0 : AB_SUB;
            k_attn_scores_b<<<dim3(mhip::blocks_for((size_t)nh * (pos + t0 + ns), 256), ns), 256, 0,
                              st>>>(q + (size_t)t0 * qd, d_kc, pos + t0, nh, group, hd, kvd, scale,
                                    scores, sld);
            k_attn_mix_b<<<dim3(nh, ns), 256, 0, st>>>(scores, sld, pos + t0, nh, d_vc, group, hd,
                                                       kvd, att + (size_t)t0 * qd);
        }
    }
    if (mhip::check_launch(c, "attention batch scores")) return -1;
    k_quant_rows<<<mhip::blocks_for(N * qd / QK, 256), 256, 0, st>>>(att, (int)(N * qd / QK),
                                                                      attq, atts);
    if (mm) {
        k_codes_h<<<mhip::blocks_for(N * qd, 256), 256, 0, st>>>(attq, N * qd, atth);
        float *outs[1] = {d_x};
        const int r0[4] = {0, d, d, d};
        rows_mfma(st, pk, 3, 1, outs, r0, qd / QK, n, atth, atts, d_x, d);
    } else {
        k_rows_q8_t<1><<<dim3(mhip::blocks_for(d, RT_W), mhip::blocks_for(N, 64)), 64 * RT_W, 0,
                         st>>>(one_seg(d_wo, d_x, d), qd / QK, n, attq, atts, d_x, d);
    }
    return mhip::check_launch(c, "attention batch");
}

int mhip_output_head(mhip_ctx *c, const mhip_attn_dims *s, const float *d_output_norm,
                     const void *d_output, int vocab, const float *d_x, float *d_logits,
                     void *d_scratch, int flags) {
    if (check_attn(c, s, 1)) return -1;
    if (vocab <= 0) return mhip::fail(c, "output head: vocab=%d", vocab);
    if (mhip::use_device(c)) return -1;
    AttnScratch a = carve(s, 1, d_scratch);
    const int d = s->dim;
    mhip::launch_rmsnorm_q8(c->stream, d_x, d_output_norm, a.xn, a.xq, a.xs, 1, d, s->norm_eps,
                            (flags & MHIP_FORCE_SEQ_RMS) ? 1 : 0, a.status);
    k_rows_q8<<<mhip::blocks_for(vocab, 4), 256, 0, c->stream>>>(
        one_seg(d_output, d_logits, vocab), d / QK, a.xq, a.xs, nullptr, nullptr);
    return mhip::check_launch(c, "output head");
}

}  // extern "C"
